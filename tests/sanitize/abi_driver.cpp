// Drives the host side of the C-ABI (spaceslug-main_amd/csrc/runtime_abi.cpp) on a machine
// without a GPU, in a build whose host code carries -fsanitize=address,undefined: every entry
// point's argument validation (status 1), the no-device path of every compute entry point
// (status 2, also from several threads at once, which race on the first device query), the
// retained-chain rejections and the CPU-side entry points. Test infrastructure: built and run by
// tests/test_sanitize_cpu.py. Exits 0 when every check holds; the sanitizers abort on the first
// error they find.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "runtime_abi.h"

static int failures = 0;
#define CHECK(cond)                                                                 \
    do {                                                                            \
        if (!(cond)) {                                                              \
            std::fprintf(stderr, "check failed: %s (line %d): last error '%s'\n", #cond, __LINE__, \
                         spaceslug_last_error());                                   \
            ++failures;                                                             \
        }                                                                           \
    } while (0)

static bool error_has(const char* s) { return std::strstr(spaceslug_last_error(), s) != nullptr; }

// Stand-ins for device addresses: never dereferenced on the host (no device, validation only).
template <typename T>
static T* fake(uintptr_t a) { return reinterpret_cast<T*>(a); }

int main() {
    // CPU entry point kept from the reference (native/runtime_abi.cpp).
    const float l[3] = {1.0f, 2.0f, 3.0f}, r[3] = {0.5f, -2.0f, 4.0f};
    float o[3] = {};
    CHECK(spaceslug_vector_add(l, r, o, 3) == 0 && o[0] == 1.5f && o[1] == 0.0f && o[2] == 7.0f);
    CHECK(spaceslug_vector_add(nullptr, r, o, 3) == 1);
    CHECK(std::strlen(spaceslug_q4gemm_capability()) > 0);

    // Host-pointer q4gemm: validation, then the no-device path.
    const uint32_t m = 3, n = 8, k = 64;
    std::vector<float> x(m * k, 0.25f), y(m * n), s(n * (k / 32), 0.02f), la(k * 4, 0.01f), lb(4 * n, 0.01f);
    std::vector<uint8_t> w(n * k / 2, 0x71);
    CHECK(spaceslug_q4gemm(nullptr, w.data(), s.data(), y.data(), m, n, k) == 1);
    CHECK(spaceslug_q4gemm(x.data(), w.data(), s.data(), y.data(), m, n, 40) == 1 && error_has("k%32"));
    CHECK(spaceslug_q4gemm(x.data(), w.data(), s.data(), y.data(), 0, n, k) == 1);
    CHECK(spaceslug_q4gemm(x.data(), w.data(), s.data(), y.data(), m, n, k) == 2);
    CHECK(spaceslug_q4gemm_lora(x.data(), w.data(), s.data(), la.data(), lb.data(), y.data(), m, n, k, 0, 1.0f) == 1);
    CHECK(spaceslug_q4gemm_lora(x.data(), w.data(), s.data(), la.data(), lb.data(), y.data(), m, n, k,
                                SPACESLUG_Q4_MAX_LORA_RANK + 1, 1.0f) == 1);
    CHECK(spaceslug_q4gemm_lora(x.data(), w.data(), s.data(), nullptr, lb.data(), y.data(), m, n, k, 4, 1.0f) == 1);
    CHECK(spaceslug_q4gemm_lora(x.data(), w.data(), s.data(), la.data(), lb.data(), y.data(), m, n, k, 4, 8.0f) == 2);

    // Device-pointer entry points: alignment and shape checks before any device call.
    const float* dx = fake<const float>(0x100000);
    const uint8_t* dw = fake<const uint8_t>(0x200000);
    const float* ds = fake<const float>(0x300000);
    float* dy = fake<float>(0x400000);
    CHECK(spaceslug_q4gemm_device(fake<const float>(0x100004), dw, ds, dy, m, n, k, nullptr) == 1 &&
          error_has("misaligned"));
    CHECK(spaceslug_q4gemm_device(dx, fake<const uint8_t>(0x200008), ds, dy, m, n, k, nullptr) == 1);
    CHECK(spaceslug_q4gemm_device(dx, dw, ds, dy, m, n, 33, nullptr) == 1);
    CHECK(spaceslug_q4gemm_device(dx, dw, ds, dy, m, n, k, nullptr) == 2);
    CHECK(spaceslug_q4gemm_device_noalloc(dx, dw, ds, dy, m, n, k, nullptr) == 2);
    CHECK(spaceslug_q4gemm_device_noalloc(nullptr, dw, ds, dy, m, n, k, nullptr) == 1);
    CHECK(spaceslug_q4gemm_lora_device(dx, dw, ds, fake<const float>(0x500000), fake<const float>(0x600000), dy, m, n,
                                       k, 4, 8.0f, nullptr) == 2);
    CHECK(spaceslug_q4gemm_lora_device(dx, dw, ds, nullptr, fake<const float>(0x600000), dy, m, n, k, 4, 8.0f,
                                       nullptr) == 1);

    // The first device query from several threads at once: every one sees "no device".
    {
        std::vector<std::thread> threads;
        std::vector<int> rc(8, -1);
        for (int t = 0; t < 8; ++t)
            threads.emplace_back([&, t] { rc[t] = spaceslug_q4gemm_device(dx, dw, ds, dy, m, n, k, nullptr); });
        for (auto& th : threads) th.join();
        for (int v : rc) CHECK(v == 2);
    }

    // sgemm keeps the reference's shape contract (sgemm_api.cpp:31-38).
    std::vector<float> a(64 * 64, 1.0f), c(64 * 64);
    float err = -1.0f;
    CHECK(spaceslug_sgemm(a.data(), a.data(), c.data(), 63, 64, 32, &err) == 1);
    CHECK(spaceslug_sgemm(a.data(), a.data(), c.data(), 64, 64, 33, nullptr) == 1);
    CHECK(spaceslug_sgemm(a.data(), a.data(), c.data(), 64, 64, 32, &err) == 2);

    // Quantizer: non-finite weights are rejected before the device.
    std::vector<float> wf(n * k, 0.5f);
    std::vector<float> qs(n * (k / 32));
    std::vector<uint8_t> qp(n * k / 2);
    wf[5] = NAN;
    CHECK(spaceslug_q4_quantize(wf.data(), qp.data(), qs.data(), n, k) == 1 && error_has("non-finite"));
    wf[5] = 0.5f;
    CHECK(spaceslug_q4_quantize(wf.data(), qp.data(), qs.data(), n, 48) == 1);
    CHECK(spaceslug_q4_quantize(wf.data(), qp.data(), qs.data(), n, k) == 2);
    CHECK(spaceslug_q4_quantize_device(fake<const float>(0x100000), fake<uint8_t>(0x200004), fake<float>(0x300000), n,
                                       k, nullptr) == 1);

    // Weight handles.
    CHECK(spaceslug_q4_weight_create(nullptr, s.data(), n, k) == nullptr);
    CHECK(spaceslug_q4_weight_create(w.data(), s.data(), n, 40) == nullptr);
    CHECK(spaceslug_q4_weight_create(w.data(), s.data(), n, k) == nullptr);  // no device
    spaceslug_q4_weight_destroy(nullptr);
    CHECK(spaceslug_q4gemm_run(nullptr, x.data(), y.data(), m) == 1);

    // Retained chains: every step is validated before any device call.
    spaceslug_q4_step st[2];
    std::memset(st, 0, sizeof(st));
    for (auto& t : st) {
        t.d_x = dx;
        t.d_w_packed = dw;
        t.d_w_scales = ds;
        t.d_y = dy;
        t.m = m;
        t.n = n;
        t.k = k;
    }
    CHECK(spaceslug_q4_chain_create(nullptr, 1) == nullptr);
    CHECK(spaceslug_q4_chain_create(st, 0) == nullptr && error_has("at least one step"));
    st[1].k = 48;
    CHECK(spaceslug_q4_chain_create(st, 2) == nullptr && error_has("step 1"));
    st[1].k = k;
    st[0].d_lora_a = fake<const float>(0x500000);
    CHECK(spaceslug_q4_chain_create(st, 2) == nullptr && error_has("both factors"));
    st[0].d_lora_b = fake<const float>(0x600000);
    st[0].rank = SPACESLUG_Q4_MAX_LORA_RANK + 1;
    CHECK(spaceslug_q4_chain_create(st, 2) == nullptr && error_has("rank"));
    st[0].rank = 4;
    CHECK(spaceslug_q4_chain_create(st, 2) == nullptr);  // valid steps, no device
    CHECK(spaceslug_q4_chain_run(nullptr, nullptr) == 1);
    spaceslug_q4_chain_destroy(nullptr);

    // CQ4: the reference's early returns and the layouts it does not define.
    std::vector<uint16_t> cb(16, 0x3C00), ah(2 * 64, 0x3C00), ch(2 * 8), norms(8 * 2, 0x3C00);
    std::vector<uint8_t> idx(8 * 2 * 16, 0x21);
    spaceslug_cq4_matrix cm;
    std::memset(&cm, 0, sizeof(cm));
    cm.bits = 4;
    cm.K = 64;
    cm.N = 8;
    cm.group_size = 32;
    cm.num_groups = 2;
    cm.codebook = cb.data();
    cm.norms = norms.data();
    cm.packed_indices = idx.data();
    CHECK(spaceslug_cq4_matmul(nullptr, ah.data(), 2, ch.data()) == 1);
    cm.bits = 5;
    CHECK(spaceslug_cq4_matmul(&cm, ah.data(), 2, ch.data()) == 1);
    cm.bits = 4;
    cm.group_size = 24;
    cm.num_groups = 2;
    cm.K = 48;
    CHECK(spaceslug_cq4_matmul(&cm, ah.data(), 2, ch.data()) == 1);  // Hadamard group not a power of two
    cm.group_size = 32;
    cm.K = 64;
    CHECK(spaceslug_cq4_matmul(&cm, ah.data(), 2, ch.data()) == 2);  // valid, no device

    if (failures) {
        std::fprintf(stderr, "%d check(s) failed\n", failures);
        return 1;
    }
    std::printf("abi sanitizer driver: all checks passed\n");
    return 0;
}
