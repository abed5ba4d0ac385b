// C++ driver of the tiny forward's projections on the int4 path, through the
// C-ABI only: the reference's _execute_tiny_gpu_forward (python/spaceslug/
// backend.py:1707-1738) makes five spaceslug_sgemm calls that each re-stage
// their weights; here the weights are quantized once (spaceslug_q4_quantize),
// uploaded once, and the projections run as two retained chains:
//   chain 1: states [128][64] -> fused Q|K|V [128][192]          (one launch)
//   chain 2: context [128][64] -> output projection [128][64]
//            -> LM head, vocabulary padded to 320 [128][320]     (one graph launch)
// Causal attention between the chains is computed here on the host (it is not
// part of the int4 path). Every stage is checked against a double-precision loop
// over the dequantized int4 weights with the metric of test_q4gemm.cpp:378-383
// (|d| / max(1, |ref|) <= 1e-5).
// Build: g++ -std=c++17 -D__HIP_PLATFORM_AMD__ -I<repo>/include -I/opt/rocm/include tiny_projection_chain.cpp
//            -L<repo>/spaceslug-main_amd/_lib -lspaceslug_runtime -L/opt/rocm/lib -lamdhip64
//            -Wl,-rpath,<both dirs>
// Exit status 0 when every stage passed (or, with --allow-no-device, when no HIP device is present).
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "runtime_abi.h"

namespace {

constexpr uint32_t kRows = 128, kH = 64, kVocab = 259, kVocabPadded = 320, kTokens = 37;

uint32_t lcg(uint32_t& s) {
    s = s * 1664525u + 1013904223u;
    return s;
}

float normal(uint32_t& s) {
    const double u1 = ((lcg(s) >> 8) + 0.5) * (1.0 / 16777216.0);
    const double u2 = ((lcg(s) >> 8) + 0.5) * (1.0 / 16777216.0);
    return static_cast<float>(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
}

struct Q4 {
    uint32_t n = 0, k = 0;
    std::vector<uint8_t> packed;
    std::vector<float> scales;
    double dequant(uint32_t kk, uint32_t col) const {  // layout of include/runtime_abi.h
        const uint8_t b = packed[static_cast<size_t>(col) * (k / 2) + kk / 2];
        int v = (kk & 1) ? (b >> 4) : (b & 15);
        if (v >= 8) v -= 16;
        return v * static_cast<double>(scales[static_cast<size_t>(col) * (k / 32) + kk / 32]);
    }
};

// w is float[k][n]; returns its int4 form, or an empty Q4 when the call failed.
Q4 quantize(const std::vector<float>& w, uint32_t k, uint32_t n) {
    Q4 q;
    q.n = n;
    q.k = k;
    q.packed.resize(static_cast<size_t>(n) * k / 2);
    q.scales.resize(static_cast<size_t>(n) * k / 32);
    if (spaceslug_q4_quantize(w.data(), q.packed.data(), q.scales.data(), n, k) != SPACESLUG_OK) q.n = 0;
    return q;
}

std::vector<double> project(const std::vector<float>& x, uint32_t m, const Q4& w) {
    std::vector<double> y(static_cast<size_t>(m) * w.n, 0.0);
    for (uint32_t r = 0; r < m; ++r)
        for (uint32_t c = 0; c < w.n; ++c) {
            double a = 0.0;
            for (uint32_t kk = 0; kk < w.k; ++kk) a += static_cast<double>(x[static_cast<size_t>(r) * w.k + kk]) * w.dequant(kk, c);
            y[static_cast<size_t>(r) * w.n + c] = a;
        }
    return y;
}

bool close_enough(const char* what, const float* got, const std::vector<double>& want, size_t count) {
    double worst = 0.0;
    for (size_t i = 0; i < count; ++i) worst = std::max(worst, std::fabs(got[i] - want[i]) / std::max(1.0, std::fabs(want[i])));
    std::printf("%s: max rel %.3g %s\n", what, worst, worst <= 1e-5 ? "PASS" : "FAIL");
    return worst <= 1e-5;
}

struct Device {
    std::vector<void*> blocks;
    template <typename T>
    T* alloc(size_t count) {
        void* p = nullptr;
        if (hipMalloc(&p, count * sizeof(T)) != hipSuccess) return nullptr;
        blocks.push_back(p);
        return static_cast<T*>(p);
    }
    ~Device() {
        for (void* p : blocks) (void)hipFree(p);
    }
};

template <typename T>
bool upload(T* d, const std::vector<T>& h) {
    return hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice) == hipSuccess;
}

}  // namespace

int main(int argc, char** argv) {
    const bool allow_no_device = argc > 1 && std::strcmp(argv[1], "--allow-no-device") == 0;
    int devices = 0;
    if (hipGetDeviceCount(&devices) != hipSuccess || devices == 0) {
        std::puts(allow_no_device ? "no HIP device: skipped" : "no HIP device");
        return allow_no_device ? 0 : 1;
    }
    uint32_t seed = 0x7e57u;
    auto matrix = [&](uint32_t rows, uint32_t cols, float scale) {
        std::vector<float> m(static_cast<size_t>(rows) * cols);
        for (auto& e : m) e = scale * normal(seed);
        return m;
    };
    // fused Q|K|V weights [64][192], output [64][64], LM head [64][320] with columns >= 259 zero
    const std::vector<float> wqkv = matrix(kH, 3 * kH, 0.125f), wo = matrix(kH, kH, 0.125f);
    std::vector<float> wlm = matrix(kH, kVocabPadded, 0.125f);
    for (uint32_t r = 0; r < kH; ++r)
        for (uint32_t c = kVocab; c < kVocabPadded; ++c) wlm[static_cast<size_t>(r) * kVocabPadded + c] = 0.0f;
    const Q4 qkv = quantize(wqkv, kH, 3 * kH), out = quantize(wo, kH, kH), lm = quantize(wlm, kH, kVocabPadded);
    if (!qkv.n || !out.n || !lm.n) {
        std::printf("quantize failed: %s\n", spaceslug_last_error());
        return 1;
    }
    std::vector<float> states(static_cast<size_t>(kRows) * kH, 0.0f);
    for (size_t i = 0; i < static_cast<size_t>(kTokens) * kH; ++i) states[i] = normal(seed);

    Device dev;
    float* d_states = dev.alloc<float>(states.size());
    float* d_qkv = dev.alloc<float>(static_cast<size_t>(kRows) * 3 * kH);
    float* d_ctx = dev.alloc<float>(static_cast<size_t>(kRows) * kH);
    float* d_proj = dev.alloc<float>(static_cast<size_t>(kRows) * kH);
    float* d_logits = dev.alloc<float>(static_cast<size_t>(kRows) * kVocabPadded);
    uint8_t* d_wqkv = dev.alloc<uint8_t>(qkv.packed.size());
    float* d_sqkv = dev.alloc<float>(qkv.scales.size());
    uint8_t* d_wo = dev.alloc<uint8_t>(out.packed.size());
    float* d_so = dev.alloc<float>(out.scales.size());
    uint8_t* d_wlm = dev.alloc<uint8_t>(lm.packed.size());
    float* d_slm = dev.alloc<float>(lm.scales.size());
    if (dev.blocks.size() != 11 || !upload(d_states, states) || !upload(d_wqkv, qkv.packed) ||
        !upload(d_sqkv, qkv.scales) || !upload(d_wo, out.packed) || !upload(d_so, out.scales) ||
        !upload(d_wlm, lm.packed) || !upload(d_slm, lm.scales)) {
        std::puts("device allocation or upload failed");
        return 1;
    }

    const spaceslug_q4_step first[1] = {{d_states, d_wqkv, d_sqkv, d_qkv, kRows, 3 * kH, kH, nullptr, nullptr, 0, 0.0f}};
    const spaceslug_q4_step second[2] = {
        {d_ctx, d_wo, d_so, d_proj, kRows, kH, kH, nullptr, nullptr, 0, 0.0f},
        {d_proj, d_wlm, d_slm, d_logits, kRows, kVocabPadded, kH, nullptr, nullptr, 0, 0.0f},
    };
    spaceslug_q4_chain* c1 = spaceslug_q4_chain_create(first, 1);
    spaceslug_q4_chain* c2 = spaceslug_q4_chain_create(second, 2);
    bool ok = c1 && c2;
    if (!ok) std::printf("chain create failed: %s\n", spaceslug_last_error());

    std::vector<float> h_qkv(static_cast<size_t>(kRows) * 3 * kH), h_proj(static_cast<size_t>(kRows) * kH),
        h_logits(static_cast<size_t>(kRows) * kVocabPadded), ctx(static_cast<size_t>(kRows) * kH, 0.0f);
    if (ok) ok = spaceslug_q4_chain_run(c1, nullptr) == SPACESLUG_OK && hipDeviceSynchronize() == hipSuccess &&
                 hipMemcpy(h_qkv.data(), d_qkv, h_qkv.size() * 4, hipMemcpyDeviceToHost) == hipSuccess;
    if (ok) ok = close_enough("chain 1 (fused Q|K|V)", h_qkv.data(), project(states, kRows, qkv), h_qkv.size());
    if (ok) {  // causal softmax attention over the first kTokens rows, in double, on the host
        for (uint32_t i = 0; i < kTokens; ++i) {
            std::vector<double> p(i + 1);
            double mx = -INFINITY, sum = 0.0;
            for (uint32_t j = 0; j <= i; ++j) {
                double d = 0.0;
                for (uint32_t c = 0; c < kH; ++c)
                    d += static_cast<double>(h_qkv[static_cast<size_t>(i) * 3 * kH + c]) * h_qkv[static_cast<size_t>(j) * 3 * kH + kH + c];
                p[j] = d / std::sqrt(static_cast<double>(kH));
                mx = std::max(mx, p[j]);
            }
            for (auto& e : p) sum += (e = std::exp(e - mx));
            for (uint32_t c = 0; c < kH; ++c) {
                double a = 0.0;
                for (uint32_t j = 0; j <= i; ++j) a += p[j] / sum * h_qkv[static_cast<size_t>(j) * 3 * kH + 2 * kH + c];
                ctx[static_cast<size_t>(i) * kH + c] = static_cast<float>(a);
            }
        }
        ok = upload(d_ctx, ctx) && spaceslug_q4_chain_run(c2, nullptr) == SPACESLUG_OK &&
             hipDeviceSynchronize() == hipSuccess &&
             hipMemcpy(h_proj.data(), d_proj, h_proj.size() * 4, hipMemcpyDeviceToHost) == hipSuccess &&
             hipMemcpy(h_logits.data(), d_logits, h_logits.size() * 4, hipMemcpyDeviceToHost) == hipSuccess;
    }
    if (ok) ok = close_enough("chain 2 step 1 (output projection)", h_proj.data(), project(ctx, kRows, out), h_proj.size());
    if (ok) ok = close_enough("chain 2 step 2 (LM head)", h_logits.data(), project(h_proj, kRows, lm), h_logits.size());
    if (ok) {
        const float* last = h_logits.data() + static_cast<size_t>(kTokens - 1) * kVocabPadded;
        const size_t best = std::max_element(last, last + kVocab) - last;
        std::printf("last-token argmax over %u logits: %zu\n", kVocab, best);
    }
    spaceslug_q4_chain_destroy(c1);
    spaceslug_q4_chain_destroy(c2);
    std::puts(ok ? "tiny projection chain: PASS" : "tiny projection chain: FAIL");
    return ok ? 0 : 1;
}
