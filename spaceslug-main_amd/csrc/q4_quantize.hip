// fp32 -> int4 group-32 quantizer that writes the packed weight layout the
// GEMM/GEMV kernels read (q4gemm.comp:7-19: uint8[N][K/2], even k in the low
// nibble, two's-complement nibbles; float[N][K/32] scales).
//
// Rule, per column n and group g (32 consecutive k):
//   m     = the value of largest magnitude among w[32g .. 32g+31][n] (the first
//           one in k order when several share that magnitude);
//   scale = -m / 8                          (exact: a power-of-two division);
//   v_k   = clamp(rint(w_k / scale), -8, 7) (IEEE division, round to nearest
//           even), 0 for every k when scale == 0.
// The extreme value maps to -8 exactly; a value of the opposite sign and the
// same magnitude maps to +8 and is clamped to 7. A group holding a NaN or an
// infinity gets a NaN scale and zero nibbles (the host entry point rejects
// non-finite input before that).
//
// Mapping: a thread owns one (column, group); the 64 lanes of a wavefront hold
// 64 consecutive columns of one group, so every read of w[k][n0 .. n0+63] is
// one coalesced 256-byte row segment. Each thread writes its group's 16 packed
// bytes with one 128-bit store and its scale with one 32-bit store.
#include "q4_device.hpp"
#include "q4_kernels.hpp"

namespace spaceslug {
namespace {

__global__ __launch_bounds__(256) void q4_quantize_kernel(const float* __restrict__ w, u32x4* __restrict__ packed,
                                                          float* __restrict__ scales, int N, int K) {
    const int n = blockIdx.x * blockDim.x + threadIdx.x;
    const int g = blockIdx.y;
    if (n >= N) return;
    const int G = K >> 5;
    float v[32];
#pragma unroll
    for (int t = 0; t < 32; ++t) v[t] = w[static_cast<size_t>(g * 32 + t) * N + n];
    float m = v[0];
    bool finite = __builtin_isfinite(v[0]);
#pragma unroll
    for (int t = 1; t < 32; ++t) {
        m = fabsf(v[t]) > fabsf(m) ? v[t] : m;
        finite = finite && __builtin_isfinite(v[t]);
    }
    float scale = -m * 0.125f;
    uint32_t words[4] = {0u, 0u, 0u, 0u};
    if (!finite) {
        scale = __builtin_nanf("");
    } else if (scale == 0.0f) {
        scale = 0.0f;  // also turns -0 into +0
    } else {
#pragma unroll
        for (int t = 0; t < 32; ++t) {
            const float r = rintf(v[t] / scale);
            const int q = static_cast<int>(fminf(fmaxf(r, -8.0f), 7.0f));
            words[t >> 3] |= (static_cast<uint32_t>(q) & 0xFu) << (4 * (t & 7));
        }
    }
    packed[static_cast<size_t>(n) * G + g] = u32x4{words[0], words[1], words[2], words[3]};
    scales[static_cast<size_t>(n) * G + g] = scale;
}

}  // namespace

hipError_t launch_q4_quantize(const float* w, uint8_t* w_packed, float* w_scales, uint32_t n, uint32_t k,
                              hipStream_t stream) {
    const dim3 grid((n + 255) / 256, k / kGroup);
    hipLaunchKernelGGL(q4_quantize_kernel, grid, dim3(256), 0, stream, w, reinterpret_cast<u32x4*>(w_packed),
                       w_scales, static_cast<int>(n), static_cast<int>(k));
    return hipGetLastError();
}

}  // namespace spaceslug
