// Measurement probes for the decode GEMV's per-launch ceiling, built into their own
// library (libspaceslug_probes.so) and loaded only by the benchmark; nothing in the
// int4 runtime calls them.
//   - spaceslug_probe_empty: a kernel with no work on the GEMV's grid (256 workgroups of
//     256 threads at K = 4096, N = 14336), replayed back to back: the fixed cost of one
//     dependent launch (dispatch, wave launch, completion signal).
//   - spaceslug_probe_touch: the same grid, one 16-byte load per lane from a column run
//     of the GEMV's layout and one store per wavefront: the fixed cost of a launch that
//     reaches HBM once (first-load latency included).
//   - spaceslug_probe_read: a persistent streaming read (grid-stride, `unroll` 16-byte
//     loads per thread in flight, nontemporal like the GEMV's weight loads) whose best
//     rate over a few launch shapes is the HBM read rate a kernel can reach.
// The GEMV ceiling per launch is then touch + bytes / read rate.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void probe_empty_kernel(float* y, int flag) {
    if (flag < 0 && threadIdx.x == 0) y[blockIdx.x] = 1.0f;  // never taken: the host passes flag >= 0
}

// Wavefront w reads 16 bytes per lane at 16-byte unit w * stride + lane and stores their xor.
__global__ __launch_bounds__(256) void probe_touch_kernel(const u32x4* __restrict__ w, uint32_t* __restrict__ y,
                                                          size_t stride) {
    const int lane = threadIdx.x & 63;
    const size_t wave = static_cast<size_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const u32x4 v = __builtin_nontemporal_load(w + wave * stride + lane);
    const uint32_t s = v[0] ^ v[1] ^ v[2] ^ v[3];
    if (lane == 0) y[wave] = s;
}

template <int U>
__global__ __launch_bounds__(256) void probe_read_kernel(const u32x4* __restrict__ w, uint32_t* __restrict__ y,
                                                         size_t n16) {
    uint32_t s = 0;
    const size_t step = static_cast<size_t>(gridDim.x) * 256 * U;
    for (size_t base = static_cast<size_t>(blockIdx.x) * 256 * U + threadIdx.x; base < n16; base += step) {
        u32x4 v[U];
#pragma unroll
        for (int i = 0; i < U; ++i) {
            const size_t idx = base + static_cast<size_t>(i) * 256;
            v[i] = __builtin_nontemporal_load(w + (idx < n16 ? idx : n16 - 1));
        }
#pragma unroll
        for (int i = 0; i < U; ++i) s ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
    }
    y[static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x] = s;
}

}  // namespace

extern "C" {

// y: at least `blocks` floats (never written). Returns a hipError_t value.
int spaceslug_probe_empty(void* y, int blocks, void* stream) {
    if (blocks < 1) return static_cast<int>(hipErrorInvalidValue);
    hipLaunchKernelGGL(probe_empty_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<float*>(y), 0);
    return static_cast<int>(hipGetLastError());
}

// w: at least (4 * blocks - 1) * stride16 + 64 units of 16 bytes; y: 4 * blocks words.
int spaceslug_probe_touch(const void* w, size_t w_bytes, void* y, int blocks, size_t stride16, void* stream) {
    if (blocks < 1 || stride16 < 64) return static_cast<int>(hipErrorInvalidValue);
    const size_t need = ((static_cast<size_t>(blocks) * 4 - 1) * stride16 + 64) * 16;
    if (need > w_bytes) return static_cast<int>(hipErrorInvalidValue);
    hipLaunchKernelGGL(probe_touch_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const u32x4*>(w), static_cast<uint32_t*>(y),
                       stride16);
    return static_cast<int>(hipGetLastError());
}

// w: w_bytes (a multiple of 16, at least 16); y: 256 * blocks words; unroll 4, 8 or 16.
int spaceslug_probe_read(const void* w, size_t w_bytes, void* y, int blocks, int unroll, void* stream) {
    const size_t n16 = w_bytes / 16;
    if (blocks < 1 || n16 == 0 || w_bytes % 16) return static_cast<int>(hipErrorInvalidValue);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const u32x4* W = static_cast<const u32x4*>(w);
    uint32_t* Y = static_cast<uint32_t*>(y);
    const dim3 grid(static_cast<unsigned>(blocks));
    switch (unroll) {
        case 4: hipLaunchKernelGGL(probe_read_kernel<4>, grid, dim3(256), 0, st, W, Y, n16); break;
        case 8: hipLaunchKernelGGL(probe_read_kernel<8>, grid, dim3(256), 0, st, W, Y, n16); break;
        case 16: hipLaunchKernelGGL(probe_read_kernel<16>, grid, dim3(256), 0, st, W, Y, n16); break;
        default: return static_cast<int>(hipErrorInvalidValue);
    }
    return static_cast<int>(hipGetLastError());
}

}  // extern "C"
