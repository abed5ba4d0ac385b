// C++ caller of the runtime C-ABI, in the style of the reference's
// native/runtime_abi_test.cpp: the unchanged vector_add contract, then one int4
// projection through spaceslug_q4gemm checked against a double-precision loop.
// Build: g++ -std=c++17 -I<repo>/include runtime_abi_client.cpp
//            -L<repo>/spaceslug-main_amd/_lib -lspaceslug_runtime -Wl,-rpath,<that dir>
// Exit status: 0 when every call that ran passed (status 2 from the int4 call,
// "no HIP device", counts as passed only with --allow-no-device), 1 otherwise.
#include "runtime_abi.h"

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

namespace {

uint32_t lcg(uint32_t& s) {
    s = s * 1664525u + 1013904223u;
    return s;
}

}  // namespace

int main(int argc, char** argv) {
    const bool allow_no_device = argc > 1 && std::strcmp(argv[1], "--allow-no-device") == 0;
    float a[3] = {0.25f, 1.5f, -2.0f};
    float b[3] = {0.75f, 2.5f, 3.0f};
    float out[3] = {};
    if (spaceslug_vector_add(a, b, out, 3) != 0 || out[0] != 1.0f || out[1] != 4.0f || out[2] != 1.0f) return 1;
    std::puts("runtime_abi vector_add: PASS");

    const uint32_t m = 3, n = 40, k = 256, groups = k / 32;
    std::vector<float> x(m * k), scales(n * groups), y(m * n, 0.0f);
    std::vector<uint8_t> packed(n * k / 2, 0);
    std::vector<int> v(static_cast<size_t>(k) * n);
    uint32_t s = 0x5eedu;
    for (auto& e : x) e = static_cast<float>((lcg(s) >> 8) * (1.0 / 16777216.0) * 2.0 - 1.0);
    for (auto& e : scales) e = static_cast<float>(0.01 + 0.04 * ((lcg(s) >> 8) * (1.0 / 16777216.0)));
    for (uint32_t col = 0; col < n; ++col)
        for (uint32_t kk = 0; kk < k; ++kk) {
            const int val = static_cast<int>((lcg(s) >> 8) % 16u) - 8;
            v[static_cast<size_t>(kk) * n + col] = val;
            packed[col * (k / 2) + kk / 2] |= static_cast<uint8_t>((static_cast<unsigned>(val) & 0xFu) << ((kk & 1u) * 4u));
        }
    const int rc = spaceslug_q4gemm(x.data(), packed.data(), scales.data(), y.data(), m, n, k);
    if (rc == SPACESLUG_ERR_DEVICE && allow_no_device) {
        std::printf("runtime_abi q4gemm: no HIP device (%s)\n", spaceslug_last_error());
        return 0;
    }
    if (rc != SPACESLUG_OK) {
        std::printf("runtime_abi q4gemm: FAIL status %d (%s)\n", rc, spaceslug_last_error());
        return 1;
    }
    double worst = 0.0;
    for (uint32_t r = 0; r < m; ++r)
        for (uint32_t col = 0; col < n; ++col) {
            double ref = 0.0;
            for (uint32_t kk = 0; kk < k; ++kk)
                ref += static_cast<double>(x[r * k + kk]) *
                       (static_cast<double>(v[static_cast<size_t>(kk) * n + col]) * scales[col * groups + kk / 32]);
            const double rel = std::fabs(y[r * n + col] - ref) / std::fmax(1.0, std::fabs(ref));
            worst = std::fmax(worst, rel);
        }
    std::printf("runtime_abi q4gemm: %s (max rel %.3e)\n", worst <= 1e-5 ? "PASS" : "FAIL", worst);
    return worst <= 1e-5 ? 0 : 1;
}
