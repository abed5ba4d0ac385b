// CQ4 codebook matmul on gfx950: C = transform(A) x decode(W), fp16 in and out,
// fp32 arithmetic. Semantics of cactus_quant_matmul (vulkan-runtime/src/cactus/
// cactus_x86.cpp:133-240, 384-397); the reference's GPU chain is three
// dispatches through two fp16 intermediates (transform_act -> dequant_w ->
// sgemm_f16_am, vulkan-runtime/tests/test_cq4.cpp:255-334). Here:
//   1. the activation transform writes the code-basis activations A' (scale and
//      left sign, a normalized Walsh-Hadamard transform per group, right sign and
//      permutation; a direct product with the rotation for the orthogonal mode):
//      in fp32 for the VALU GEMMs, or, for the MFMA GEMMs, each value as three
//      exact bf16 limbs;
//   2. one GEMM kernel decodes the packed indices on the fly (LSB-first bit
//      packing or 4-row interleaved panels), looks codebook values up in LDS and
//      sums products in fp32 over at most 32 values, folding each sum times its
//      group's norm in float64; the dequantized weight matrix is never
//      materialized, and C is rounded to fp16 once.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>
#include <utility>

#include "cq4_kernels.hpp"
#include "q4_device.hpp"

namespace spaceslug {
namespace {

template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}

// f(integral_constant<int, i>) for i = 0 .. N-1, unrolled at compile time.
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

__device__ __forceinline__ float half_bits_to_float(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }

__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));  // round to nearest even
}

// fp16 bits of a double, rounded to nearest even. Rounding to float first and then to fp16 gives the
// same result (24 >= 2 * 11 + 2 significant bits, so the first rounding cannot create a tie for the
// second); the empty asm keeps the compiler from fusing the two hardware conversions (v_cvt_f32_f64,
// v_cvt_f16_f32) into one from double, which it expands into about 40 integer instructions.
__device__ __forceinline__ uint16_t double_to_half_bits(double d) {
    float f = static_cast<float>(d);
    asm("" : "+v"(f));
    return float_to_half_bits(f);
}

// Per-element input scale reciprocal (cactus_x86.cpp:74-80).
__device__ __forceinline__ float input_recip(const Cq4View& w, uint32_t k) {
    if (w.input_scale_recip) return half_bits_to_float(w.input_scale_recip[k]);
    if (w.input_scale) return 1.0f / half_bits_to_float(w.input_scale[k]);
    return 1.0f;
}

// Stores the code-basis value x of (row, k): as fp32 into out[row][k], or, when xs is set
// (the MFMA path, K % 64 == 0), as its three exact bf16 limbs in the limb layout
// [M][K/64][3][64] that cq4_gemm_mfma_kernel copies to LDS.
__device__ __forceinline__ void store_code(float* out, uint16_t* xs, uint32_t K, size_t row, uint32_t k, float x) {
    if (xs == nullptr) {
        out[row * K + k] = x;
        return;
    }
    uint32_t b[3];
    split_bf16_limbs(x, b);
    uint16_t* d = xs + (row * (K >> 6) + (k >> 6)) * (3 * 64) + (k & 63);
    d[0] = static_cast<uint16_t>(b[0]);
    d[64] = static_cast<uint16_t>(b[1]);
    d[128] = static_cast<uint16_t>(b[2]);
}

// Hadamard basis: grid (num_groups, M), group_size / 2 threads; thread t owns
// elements t and t + gs/2 on load and store and butterfly t at every stage.
__global__ __launch_bounds__(128) void cq4_transform_hadamard_kernel(Cq4View w, const uint16_t* __restrict__ a,
                                                                     float* __restrict__ out, uint16_t* __restrict__ xs) {
    __shared__ float v[256];
    const uint32_t gs = w.group_size, half = gs >> 1;
    const uint32_t g = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
    const size_t row = static_cast<size_t>(m) * w.K + static_cast<size_t>(g) * gs;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const uint32_t k = t + e * half;
        const float sign = w.left_signs ? static_cast<float>(w.left_signs[k]) : 1.0f;
        v[k] = half_bits_to_float(a[row + k]) * input_recip(w, g * gs + k) * sign;
    }
    __syncthreads();
    for (uint32_t h = 1; h < gs; h <<= 1) {  // butterflies over strides 1, 2, 4, ... (cactus_x86.cpp:56-66)
        const uint32_t j = (t / h) * 2 * h + (t % h);  // each thread owns one disjoint pair per stage
        const float x = v[j], y = v[j + h];
        v[j] = x + y;
        v[j + h] = x - y;
        __syncthreads();
    }
    const float inv = 1.0f / sqrtf(static_cast<float>(gs));
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const uint32_t j = t + e * half;
        // an out-of-range entry is masked into the group (the host entry point rejects it)
        const uint32_t src = w.permutation ? (w.permutation[j] & (gs - 1)) : j;
        const float sign = w.right_signs ? static_cast<float>(w.right_signs[src]) : 1.0f;
        store_code(out, xs, w.K, m, g * gs + j, v[src] * inv * sign);
    }
}

// Hadamard basis for group sizes 64, 128 and 256 (E = gs / 64 elements per lane):
// one wavefront per (row, group), the group held in registers. Lane l holds
// elements l + 64 i, i < E; butterflies of stride 1..32 pair lanes l and l ^ h
// (__shfl_xor), strides 64 and 128 pair a lane's own elements, so no LDS and no
// barrier is involved. The right sign and permutation gather element src from
// lane src % 64. Same arithmetic, in the same order per element, as the LDS form
// above. Four wavefronts per workgroup cover four consecutive (row, group) pairs.
template <int E>
__global__ __launch_bounds__(256) void cq4_transform_hadamard_wave_kernel(Cq4View w, const uint16_t* __restrict__ a,
                                                                          float* __restrict__ out, uint16_t* __restrict__ xs,
                                                                          uint32_t pairs) {
    constexpr uint32_t gs = 64 * E;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t pair = blockIdx.x * 4 + (threadIdx.x >> 6);  // row * num_groups + group
    if (pair >= pairs) return;  // whole wavefronts only: no cross-lane exchange is cut short
    const uint32_t g = pair % w.num_groups;
    const size_t base = static_cast<size_t>(pair / w.num_groups) * w.K + static_cast<size_t>(g) * gs;
    // Every load of the wavefront is issued before any is used (one memory round trip): an
    // absent optional array is read from `a` instead (in bounds: its first K values) and the
    // value ignored, so only the permutation, when present, adds a branch.
    uint16_t ar[E], sr[E];
    int8_t ls[E], rs[E];
    uint32_t src[E];
    const uint16_t* srow = w.input_scale_recip ? w.input_scale_recip : (w.input_scale ? w.input_scale : a);
    const int8_t* lsp = w.left_signs ? w.left_signs : reinterpret_cast<const int8_t*>(a);
    const int8_t* rsp = w.right_signs ? w.right_signs : reinterpret_cast<const int8_t*>(a);
#pragma unroll
    for (int i = 0; i < E; ++i) {
        ar[i] = a[base + lane + 64 * i];
        sr[i] = srow[g * gs + lane + 64 * i];
        ls[i] = lsp[lane + 64 * i];
    }
    if (w.permutation) {
        // an out-of-range entry is masked into the group (the host entry point rejects it)
#pragma unroll
        for (int i = 0; i < E; ++i) src[i] = w.permutation[lane + 64 * i] & (gs - 1);
    } else {
#pragma unroll
        for (int i = 0; i < E; ++i) src[i] = lane + 64 * i;
    }
#pragma unroll
    for (int i = 0; i < E; ++i) rs[i] = rsp[src[i]];
    float v[E];
#pragma unroll
    for (int i = 0; i < E; ++i) {
        // input_recip's value: the reciprocal as given, or 1 / scale, or 1
        const float r = w.input_scale_recip ? half_bits_to_float(sr[i])
                                            : (w.input_scale ? 1.0f / half_bits_to_float(sr[i]) : 1.0f);
        const float sign = w.left_signs ? static_cast<float>(ls[i]) : 1.0f;
        v[i] = half_bits_to_float(ar[i]) * r * sign;
    }
    for (uint32_t h = 1; h < 64; h <<= 1) {  // strides 1 .. 32 across lanes
        const bool upper = (lane & h) != 0;
#pragma unroll
        for (int i = 0; i < E; ++i) {
            const float o = __shfl_xor(v[i], static_cast<int>(h));
            v[i] = upper ? o - v[i] : v[i] + o;
        }
    }
#pragma unroll
    for (int h = 1; h < E; h <<= 1)  // strides 64, 128 within the lane
#pragma unroll
        for (int i = 0; i < E; ++i)
            if ((i & h) == 0) {
                const float x = v[i], y = v[i + h];
                v[i] = x + y;
                v[i + h] = x - y;
            }
    const float inv = 1.0f / sqrtf(static_cast<float>(gs));
#pragma unroll
    for (int i = 0; i < E; ++i) {
        const uint32_t j = lane + 64 * i;
        float x = v[i];  // no permutation: element j is this lane's own
        if (w.permutation) {  // uniform
            x = 0.0f;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const float t = __shfl(v[e], static_cast<int>(src[i] & 63));
                x = (src[i] >> 6) == static_cast<uint32_t>(e) ? t : x;
            }
        }
        const float sign = w.right_signs ? static_cast<float>(rs[i]) : 1.0f;
        store_code(out, xs, w.K, pair / w.num_groups, g * gs + j, x * inv * sign);
    }
}

// Value of v in lane (this lane ^ MASK), MASK < 32, without LDS memory: DPP for masks 1 and 2
// (quad permutes) and 8 (rotate by 8 within each row of 16 lanes), ds_swizzle for 4 and 16.
template <int MASK>
__device__ __forceinline__ float lane_xor(float v) {
    const int x = __float_as_int(v);
    int r;
    if constexpr (MASK == 1)
        r = __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);  // quad_perm [1, 0, 3, 2]
    else if constexpr (MASK == 2)
        r = __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);  // quad_perm [2, 3, 0, 1]
    else if constexpr (MASK == 8)
        r = __builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false);  // row_ror:8
    else
        r = __builtin_amdgcn_ds_swizzle(x, 0x1F | (MASK << 10));  // bit mode: lane ^ MASK within 32
    return __int_as_float(r);
}

// Hadamard basis written straight as bf16 limbs for the MFMA GEMM (group size GS = 64, 128 or 256;
// activations and scales 16-byte aligned, signs 8-byte aligned): one wavefront per 512 consecutive
// values of a row, lane l holding values 8 l .. 8 l + 7, so every load and limb store is 16 bytes
// per lane. Butterflies of stride 1, 2 and 4 pair a lane's own values and strides 8 .. GS / 2 pair
// lane l with lane l ^ (stride / 8): the operations and their order are those of
// cq4_transform_hadamard_kernel (cactus_x86.cpp:56-66), so the values are identical. A group
// never straddles the end of a row (GS divides K and 512), so lanes past the end exchange only
// among themselves; they load nothing and store nothing. With a permutation the wavefront's
// values pass through LDS for the gather.
//
// With xcd_rows set (the GEMM's row tiles a multiple of 8), workgroup b works on the rows of 64-row
// tiles t with t % 8 == b % 8: workgroups run on XCD b % 8, and the GEMM reads row tile t on XCD
// t % 8, so each row's limbs are written through the L2 that later serves them.
template <int GS>
__global__ __launch_bounds__(256) void cq4_transform_hadamard_limbs_kernel(Cq4View w, const uint16_t* __restrict__ a,
                                                                           uint16_t* __restrict__ xs, uint32_t M,
                                                                           uint32_t chunks, bool xcd_rows) {
    __shared__ float gather[4][512];
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    uint32_t row, chunk;
    if (xcd_rows) {
        const uint32_t unit = (blockIdx.x / 8) * 4 + wv;  // within XCD lane blockIdx % 8
        const uint32_t lr = unit / chunks;
        row = (blockIdx.x % 8 + 8 * (lr / 64)) * 64 + lr % 64;
        chunk = unit - lr * chunks;
        if (row >= M) return;  // whole wavefronts
    } else {
        const uint32_t unit = blockIdx.x * 4 + wv;  // row * chunks + chunk
        if (unit >= M * chunks) return;             // whole wavefronts
        row = unit / chunks;
        chunk = unit - row * chunks;
    }
    const uint32_t K = w.K;
    const uint32_t k0 = chunk * 512 + 8 * lane;
    const bool live = k0 < K;
    const uint32_t j0 = k0 & (GS - 1);  // position of the lane's first value in its group
    u32x4 av = {0u, 0u, 0u, 0u}, sv = {0u, 0u, 0u, 0u};
    uint2 lv = {0u, 0u}, rv = {0u, 0u};
    u32x4 pv[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
    const uint16_t* sp = w.input_scale_recip ? w.input_scale_recip : w.input_scale;
    if (live) {
        av = *reinterpret_cast<const u32x4*>(a + static_cast<size_t>(row) * K + k0);
        if (sp) sv = *reinterpret_cast<const u32x4*>(sp + k0);
        if (w.left_signs) lv = *reinterpret_cast<const uint2*>(w.left_signs + j0);
        if (w.permutation) {
            pv[0] = *reinterpret_cast<const u32x4*>(w.permutation + j0);
            pv[1] = *reinterpret_cast<const u32x4*>(w.permutation + j0 + 4);
        } else if (w.right_signs) {
            rv = *reinterpret_cast<const uint2*>(w.right_signs + j0);
        }
    }
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint16_t ah = static_cast<uint16_t>(av[e >> 1] >> (16 * (e & 1)));
        const uint16_t sh = static_cast<uint16_t>(sv[e >> 1] >> (16 * (e & 1)));
        // input_recip's value: the reciprocal as given, or 1 / scale, or 1
        const float r = w.input_scale_recip ? half_bits_to_float(sh) : (w.input_scale ? 1.0f / half_bits_to_float(sh) : 1.0f);
        const int8_t ls = static_cast<int8_t>((e < 4 ? lv.x : lv.y) >> (8 * (e & 3)));
        const float sign = w.left_signs ? static_cast<float>(ls) : 1.0f;
        v[e] = half_bits_to_float(ah) * r * sign;
    }
#pragma unroll
    for (int h = 1; h < 8; h <<= 1)  // strides 1, 2, 4 within the lane
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if ((e & h) == 0) {
                const float x = v[e], y = v[e + h];
                v[e] = x + y;
                v[e + h] = x - y;
            }
    auto cross = [&](auto mask_c) {  // stride 8 mask: lane ^ mask holds the partner values
        constexpr int mask = decltype(mask_c)::value;
        const bool upper = (lane & mask) != 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float o = lane_xor<mask>(v[e]);
            v[e] = upper ? o - v[e] : v[e] + o;
        }
    };
    cross(std::integral_constant<int, 1>{});
    cross(std::integral_constant<int, 2>{});
    cross(std::integral_constant<int, 4>{});
    if constexpr (GS >= 128) cross(std::integral_constant<int, 8>{});
    if constexpr (GS >= 256) cross(std::integral_constant<int, 16>{});
    const float inv = 1.0f / sqrtf(static_cast<float>(GS));
    float x[8];
    int8_t rs[8];
    if (w.permutation) {  // uniform
        float* g = &gather[wv][0];
#pragma unroll
        for (int e = 0; e < 8; ++e) g[8 * lane + e] = v[e];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const uint32_t gbase = 8 * lane - j0;  // the group's first value in the wavefront's chunk
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            // an out-of-range entry is masked into the group (the host entry point rejects it)
            const uint32_t src = pv[e >> 2][e & 3] & (GS - 1);
            x[e] = g[gbase + src];
            rs[e] = (w.right_signs && live) ? w.right_signs[src] : int8_t{1};
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            x[e] = v[e];
            rs[e] = static_cast<int8_t>((e < 4 ? rv.x : rv.y) >> (8 * (e & 3)));
        }
    }
    uint32_t limb[3][8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float sign = w.right_signs ? static_cast<float>(rs[e]) : 1.0f;
        uint32_t b[3];
        split_bf16_limbs(x[e] * inv * sign, b);
#pragma unroll
        for (int li = 0; li < 3; ++li) limb[li][e] = b[li];
    }
    if (live) {
        uint16_t* d = xs + (static_cast<size_t>(row) * (K >> 6) + (k0 >> 6)) * (3 * 64) + (k0 & 63);
#pragma unroll
        for (int li = 0; li < 3; ++li) {
            u32x4 o;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = limb[li][2 * i] | (limb[li][2 * i + 1] << 16);
            *reinterpret_cast<u32x4*>(d + 64 * li) = o;
        }
    }
}

// Orthogonal basis: A_rot[m][i] = sum_k A[m][k] recip[k] R[k][i]; grid (ceil(K/256), M).
__global__ __launch_bounds__(256) void cq4_transform_orthogonal_kernel(Cq4View w, const uint16_t* __restrict__ a,
                                                                       float* __restrict__ out, uint16_t* __restrict__ xs) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x, m = blockIdx.y;
    if (i >= w.K) return;
    const uint16_t* arow = a + static_cast<size_t>(m) * w.K;
    float acc = 0.0f;
    for (uint32_t k = 0; k < w.K; ++k)
        acc = fmaf(half_bits_to_float(arow[k]) * input_recip(w, k), half_bits_to_float(w.rotation[static_cast<size_t>(k) * w.K + i]),
                   acc);
    store_code(out, xs, w.K, m, i, acc);
}

// Index k of a row's LSB-first group (cactus_x86.cpp:24-43), any bits in 1..4.
__device__ __forceinline__ uint32_t index_lsb(const uint8_t* p, uint32_t k, uint32_t bits) {
    const uint32_t bit = k * bits;
    uint32_t v = p[bit >> 3] >> (bit & 7);
    if ((bit & 7) + bits > 8) v |= static_cast<uint32_t>(p[(bit >> 3) + 1]) << (8 - (bit & 7));
    return v & ((1u << bits) - 1u);
}

// One thread per (column n, ROWS rows). Per group: 8 indices per 32-bit word of
// the row's packed group, codebook values from LDS, fp32 sums per row over at
// most 32 values, each folded as acc += norm(n, g) * sum in float64 (the error
// bound of the MFMA form above).
// LAYOUT 0: 4-bit LSB-first (nibble j of word c is k = 8c + j);
// LAYOUT 1: 4-bit interleaved panels (row r's word c is bytes 16c + 4r .. +3:
//           low nibble of byte b is k = 8c + b, high nibble k = 8c + 4 + b);
// LAYOUT 2: LSB-first of any width (element by element).
template <int ROWS, int LAYOUT>
__global__ __launch_bounds__(256) void cq4_gemm_kernel(Cq4View w, const float* __restrict__ ap, uint16_t* __restrict__ c,
                                                       uint32_t M, uint32_t gs, uint32_t ng) {
    __shared__ float lut[16];
    if (threadIdx.x < (1u << w.bits)) lut[threadIdx.x] = half_bits_to_float(w.codebook[threadIdx.x]);
    __syncthreads();
    const uint32_t n = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t m0 = blockIdx.y * ROWS;
    if (n >= w.N) return;
    const bool inter = LAYOUT == 1;
    const size_t pgb = (static_cast<size_t>(gs) * w.bits + 7) / 8;
    const float* arow[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) arow[r] = ap + static_cast<size_t>(min(m0 + r, M - 1)) * w.K;
    double acc[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) acc[r] = 0.0;
    for (uint32_t g = 0; g < ng; ++g) {
        const size_t ni = inter ? (static_cast<size_t>(n / 4) * ng + g) * 4 + (n & 3) : static_cast<size_t>(n) * ng + g;
        const double norm = static_cast<double>(half_bits_to_float(w.norms[ni]));
        float s[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; ++r) s[r] = 0.0f;
        auto fold = [&]() {
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                acc[r] = fma(norm, static_cast<double>(s[r]), acc[r]);
                s[r] = 0.0f;
            }
        };
        const uint32_t kg = g * gs;
        if constexpr (LAYOUT == 2) {
            const uint8_t* p = w.packed + (static_cast<size_t>(n) * ng + g) * pgb;
            for (uint32_t k = 0; k < gs; ++k) {
                const float cv = lut[index_lsb(p, k, w.bits)];
#pragma unroll
                for (int r = 0; r < ROWS; ++r) s[r] = fmaf(arow[r][kg + k], cv, s[r]);
                if ((k & 31) == 31) fold();
            }
        } else {
            const uint8_t* base = inter ? w.packed + (static_cast<size_t>(n / 4) * ng + g) * 4 * pgb + (n & 3) * 4
                                        : w.packed + (static_cast<size_t>(n) * ng + g) * pgb;
            const uint32_t stride = inter ? 16 : 4;  // bytes between consecutive 8-index words of the row
            for (uint32_t c8 = 0; c8 < gs / 8; ++c8) {
                const uint32_t word = *reinterpret_cast<const uint32_t*>(base + c8 * stride);
                float av[ROWS][8];
#pragma unroll
                for (int r = 0; r < ROWS; ++r) {
                    const f32x4_t lo = *reinterpret_cast<const f32x4_t*>(arow[r] + kg + 8 * c8);
                    const f32x4_t hi = *reinterpret_cast<const f32x4_t*>(arow[r] + kg + 8 * c8 + 4);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        av[r][q] = lo[q];
                        av[r][4 + q] = hi[q];
                    }
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    // nibble j holds k = 8c + j (LSB) or 8c + (j >> 1) + 4 (j & 1) (interleaved)
                    const int kk = inter ? (j >> 1) + 4 * (j & 1) : j;
                    const float cv = lut[(word >> (4 * j)) & 0xFu];
#pragma unroll
                    for (int r = 0; r < ROWS; ++r) s[r] = fmaf(av[r][kk], cv, s[r]);
                }
                if ((c8 & 3) == 3) fold();
            }
        }
        fold();  // the group's remainder (groups whose size is not a multiple of 32)
    }
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
        if (m0 + r < M) c[static_cast<size_t>(m0 + r) * w.N + n] = double_to_half_bits(acc[r]);
}

// Index word wi (8 indices, all in group wi / wpg) of column n, and the flat index of its norm.
// LSB-first: the column's group g is ng-major, its word cw at byte 4 cw; interleaved: row n & 3
// of panel n / 4, its word cw at byte 16 cw + 4 (n & 3).
template <bool INTER>
__device__ __forceinline__ uint32_t cq4_gemv_word(const Cq4View& w, uint32_t n, uint32_t wi, uint32_t wpg,
                                                  uint32_t ng, size_t& ni) {
    const uint32_t g = wi / wpg, cw = wi % wpg;
    const size_t pgb = static_cast<size_t>(wpg) * 4;  // bytes of one row's group
    if constexpr (INTER) {
        const size_t panel = static_cast<size_t>(n >> 2) * ng + g;
        ni = panel * 4 + (n & 3);
        return *reinterpret_cast<const uint32_t*>(w.packed + panel * 4 * pgb + (n & 3) * 4 + 16 * cw);
    } else {
        const size_t grp = static_cast<size_t>(n) * ng + g;
        ni = grp;
        return *reinterpret_cast<const uint32_t*>(w.packed + grp * pgb + 4 * cw);
    }
}

// One index word against ROWS activation rows: 8 codebook lookups, per row an fp32 sum of the
// 8 products, and acc[r] += norm * sum in float64.
template <int ROWS, bool INTER>
__device__ __forceinline__ void cq4_gemv_step(const float* lut, uint32_t word, uint16_t norm_bits,
                                              const float* const (&arow)[ROWS], uint32_t wi, double (&acc)[ROWS]) {
    float cv[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) cv[t] = lut[(word >> (4 * t)) & 0xFu];
    const double norm = static_cast<double>(half_bits_to_float(norm_bits));
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        const f32x4_t lo = *reinterpret_cast<const f32x4_t*>(arow[r] + 8 * wi);
        const f32x4_t hi = *reinterpret_cast<const f32x4_t*>(arow[r] + 8 * wi + 4);
        const float av[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        float sum = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            // nibble t holds k = 8 cw + t (LSB) or 8 cw + (t >> 1) + 4 (t & 1) (interleaved)
            const int kk = INTER ? (t >> 1) + 4 * (t & 1) : t;
            sum = fmaf(av[kk], cv[t], sum);
        }
        acc[r] = fma(norm, static_cast<double>(sum), acc[r]);
    }
}

// The 64 lane sums of each row reduced in float64 across the wavefront, rounded to fp16 once.
template <int ROWS>
__device__ __forceinline__ void cq4_gemv_store(double (&acc)[ROWS], uint16_t* c, uint32_t N, uint32_t M, uint32_t n,
                                               uint32_t lane) {
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) acc[r] += __shfl_xor(acc[r], off);
    if (lane == 0)
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
            if (static_cast<uint32_t>(r) < M) c[static_cast<size_t>(r) * N + n] = double_to_half_bits(acc[r]);
}

// Up to 4 rows with 4-bit indices in either layout and word-aligned groups
// (group size a multiple of 8): one wavefront per column, lane l taking the column's
// 32-bit index words l, l + 64, ... (8 values each, all in one group). Per word and
// row: 8 codebook lookups in LDS, an fp32 sum of 8 products, and norm * sum
// accumulated in float64; the 64 lane sums are reduced in float64 across the
// wavefront and rounded to fp16 once. At M = 1, N = 512 this keeps 512 wavefronts
// busy where one thread per column keeps 512 threads.
template <int ROWS, bool INTER>
__global__ __launch_bounds__(256) void cq4_gemv_kernel(Cq4View w, const float* __restrict__ ap,
                                                      uint16_t* __restrict__ c, uint32_t M, uint32_t gs, uint32_t ng) {
    __shared__ float lut[16];
    if (threadIdx.x < 16) lut[threadIdx.x] = half_bits_to_float(w.codebook[threadIdx.x]);
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t n = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= w.N) return;  // whole wavefronts, after the only barrier
    const uint32_t K = w.K, words = K >> 3, wpg = gs >> 3;
    const float* arow[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) arow[r] = ap + static_cast<size_t>(min(static_cast<uint32_t>(r), M - 1)) * K;
    double acc[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) acc[r] = 0.0;
    for (uint32_t wi = lane; wi < words; wi += 64) {
        size_t ni;
        const uint32_t word = cq4_gemv_word<INTER>(w, n, wi, wpg, ng, ni);
        cq4_gemv_step<ROWS, INTER>(lut, word, w.norms[ni], arow, wi, acc);
    }
    cq4_gemv_store<ROWS>(acc, c, w.N, M, n, lane);
}

// Rows x K values the fused GEMV transforms in LDS (two arrays of that many floats: 32 KiB).
constexpr uint32_t kCq4FusedMaxValues = 4096;

// The GEMV above with the Hadamard transform in the same launch (M <= 4, power-of-two group
// size <= 256, M * K <= kCq4FusedMaxValues): every workgroup transforms all M rows into LDS with
// the operations of cq4_transform_hadamard_kernel, in the same order (scale and left sign, the
// butterflies of strides 1 .. gs / 2, then the permuted, normalized, right-signed values), so
// its four wavefronts read exactly the values the two-launch form reads from memory, and run
// its columns. Each lane's first index word and norm are loaded before the transform, so their
// latency overlaps it; the call needs no workspace and one launch instead of two. Dynamic LDS:
// 2 * M * K floats.
template <int ROWS, bool INTER>
__global__ __launch_bounds__(256) void cq4_gemv_fused_kernel(Cq4View w, const uint16_t* __restrict__ a,
                                                            uint16_t* __restrict__ c, uint32_t M, uint32_t gs,
                                                            uint32_t ng) {
    extern __shared__ f32x4_t fused_lds[];
    __shared__ float lut[16];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t n = blockIdx.x * 4 + (tid >> 6);
    const uint32_t K = w.K, words = K >> 3, wpg = gs >> 3, total = M * K;
    float* xv = reinterpret_cast<float*>(fused_lds);  // scaled, signed, then transformed in place
    float* xa = xv + total;                            // code-basis activations, row-major
    if (tid < 16) lut[tid] = half_bits_to_float(w.codebook[tid]);
    const bool live = n < w.N;  // uniform per wavefront; every wavefront takes part in the transform
    uint32_t word0 = 0;
    uint16_t norm0 = 0;
    if (live && lane < words) {
        size_t ni;
        word0 = cq4_gemv_word<INTER>(w, n, lane, wpg, ng, ni);
        norm0 = w.norms[ni];
    }
    for (uint32_t e = tid; e < total; e += 256) {
        const uint32_t k = e % K;
        const float sign = w.left_signs ? static_cast<float>(w.left_signs[k % gs]) : 1.0f;
        xv[e] = half_bits_to_float(a[e]) * input_recip(w, k) * sign;
    }
    __syncthreads();
    for (uint32_t h = 1; h < gs; h <<= 1) {  // butterflies over strides 1, 2, 4, ... (cactus_x86.cpp:56-66)
        // butterfly t pairs j and j + h inside one block of 2h values, so never across a group
        for (uint32_t t = tid; t < total / 2; t += 256) {
            const uint32_t j = (t / h) * 2 * h + (t % h);
            const float x = xv[j], y = xv[j + h];
            xv[j] = x + y;
            xv[j + h] = x - y;
        }
        __syncthreads();
    }
    const float inv = 1.0f / sqrtf(static_cast<float>(gs));
    for (uint32_t e = tid; e < total; e += 256) {
        const uint32_t j = e % gs;  // K % gs == 0: the position inside the element's group
        const uint32_t src = w.permutation ? (w.permutation[j] & (gs - 1)) : j;
        const float sign = w.right_signs ? static_cast<float>(w.right_signs[src]) : 1.0f;
        xa[e] = xv[e - j + src] * inv * sign;
    }
    __syncthreads();
    if (!live) return;
    const float* arow[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) arow[r] = xa + min(static_cast<uint32_t>(r), M - 1) * K;
    double acc[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) acc[r] = 0.0;
    if (lane < words) cq4_gemv_step<ROWS, INTER>(lut, word0, norm0, arow, lane, acc);
    for (uint32_t wi = lane + 64; wi < words; wi += 64) {
        size_t ni;
        const uint32_t word = cq4_gemv_word<INTER>(w, n, wi, wpg, ng, ni);
        cq4_gemv_step<ROWS, INTER>(lut, word, w.norms[ni], arow, wi, acc);
    }
    cq4_gemv_store<ROWS>(acc, c, w.N, M, n, lane);
}

// MFMA form for 4-bit LSB-packed indices (the packing of cactus_x86.cpp:24-43 with
// bits = 4: column n's K/2 bytes are contiguous, index k in the low nibble of byte
// k/2 when k is even), a group size that is a multiple of 32, K % 64 == 0 and
// M >= 32. The weight bytes then have exactly the int4 GEMM's layout, and the int4
// wide kernel's design carries over: v_mfma_f32_16x16x32_bf16 on exact bf16 limbs.
//   - The transform stores each code-basis activation (an fp32 value) as three
//     bf16 limbs (split_bf16_limbs: b0 + b1 + b2 == A' for |A'| >= 2^-110, within
//     2^-133 below), laid out [M][K/64][3][64], so no fp32 copy of A' is written.
//   - A codebook value (fp16, 11 significant bits) is the sum of two bf16 limbs:
//     its top 8 significant bits and the remaining 3 (the fp16 exponent range lies
//     inside bf16's). The 16 entries sit in LDS as (high | low << 16) pairs.
//   - So every limb product is exact in fp32, and six MFMAs per 32-value sub-group
//     (3 activation limbs x 2 codebook limbs, smallest first) sum the sub-group's
//     products in fp32, as the fp32 MFMA form did with eight 16x16x4 MFMAs at
//     sixteen times the matrix-core cycles each.
// Lane (j, q) of a 16x16x32 MFMA holds A[row j][k = 8q .. 8q+7] and B[k = 8q ..
// 8q+7][column j], so its B operands are the 8 indices of word q of a sub-group.
// A workgroup owns a 64 x 64 tile (2 x 2 wavefronts of 32 x 32; 256 workgroups at
// M = N = 1024) and stages 64 values of K (two sub-groups) at a time through two
// LDS buffers, one barrier per stage: the activation limbs (3 x 64 rows x 64
// values) copied global -> LDS by global_load_lds_dwordx4 as full 128-byte rows,
// XOR-swizzled within 256-byte row pairs so MFMA-operand reads hit 16 bank groups;
// the weights decoded once per workgroup (each thread one 32-bit word per
// sub-group: 8 table lookups in LDS, 8 byte permutes) into both codebook limbs in
// the MFMA B layout. Each sub-group sum times its group's norm is accumulated in
// float64 (exact product); C is rounded to fp16 once. (The reference sums a whole
// group in fp32 before the norm, cactus_x86.cpp:214-226: over K = 1024 that leaves
// errors of ~1.5e-5 near zero outputs, beyond the fp16 rounding this path is held
// to; 32-value sums folded in float64 stay under 6.2e-6 in an emulation of
// 131,072 outputs.)
constexpr uint32_t kCq4MfmaMinRows = 32;
constexpr int kCq4Tile = 64;
constexpr int kCq4Limbs = 3;

struct Cq4MfmaStage {
    // activation limb li, 8-row block, lane slot: row r's 16-byte chunk c (k = 64 t + 8 c .. +7)
    // at u32x4 index (r >> 1) * 16 + 8 (r & 1) + (c ^ ((r >> 1) & 7)) of a[li]
    u32x4 a[kCq4Limbs][8][64];
    // sub-group u, codebook limb (0 high, 1 low), 16-column tile, lane (j, q): the limbs of the
    // codebook values of k = 64 t + 32 u + 8 q .. +7 of column 16 tile + j
    u32x4 b[2][2][4][64];
};

__global__ __launch_bounds__(256) void cq4_gemm_mfma_kernel(Cq4View w, const uint16_t* __restrict__ xs,
                                                           uint16_t* __restrict__ c, uint32_t M, uint32_t gs,
                                                           uint32_t ng, uint32_t tiles_m) {
    __shared__ Cq4MfmaStage stage[2];
    __shared__ uint32_t lut[16];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wid & 1, wn = wid >> 1;
    const int j = lane & 15, q = lane >> 4;
    const int K = static_cast<int>(w.K), N = static_cast<int>(w.N), Mi = static_cast<int>(M);
    const int T = K / 64;                       // stages (K % 64 == 0)
    const int spg = static_cast<int>(gs) >> 5;  // sub-groups per norm group
    const int mt0 = static_cast<int>(blockIdx.x % tiles_m) * kCq4Tile;
    const int nt0 = static_cast<int>(blockIdx.x / tiles_m) * kCq4Tile;
    const int m0 = mt0 + 32 * wm, n0 = nt0 + 32 * wn;
    if (tid < 16) {
        const float v = half_bits_to_float(w.codebook[tid]);
        const uint32_t hi = __float_as_uint(v) & 0xFFFF0000u;
        const float lo = v - __uint_as_float(hi);  // exact, at most 3 significant bits
        lut[tid] = (hi >> 16) | (__float_as_uint(lo) & 0xFFFF0000u);
    }

    // Activation-limb copies of this wavefront: 8-row blocks 2 wid and 2 wid + 1, three limbs each.
    const uint16_t* asrc[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int blk = 2 * wid + i;
        const int pair = 4 * blk + (lane >> 4);
        const int row_t = 2 * pair + ((lane >> 3) & 1);
        asrc[i] = xs + static_cast<size_t>(min(mt0 + row_t, Mi - 1)) * T * (kCq4Limbs * 64) +
                  8 * ((lane & 7) ^ (pair & 7));
    }
    // B: thread -> tile column bc, word bw of each sub-group's 16 bytes.
    const int bc = tid >> 2, bw = tid & 3;
    const uint32_t* bsrc =
        reinterpret_cast<const uint32_t*>(w.packed + static_cast<size_t>(min(nt0 + bc, N - 1)) * (K >> 1)) + bw;
    const int blane = (bc & 15) + 16 * bw;
    const uint16_t* nrm[2];
#pragma unroll
    for (int tn = 0; tn < 2; ++tn) nrm[tn] = w.norms + static_cast<size_t>(min(n0 + 16 * tn + j, N - 1)) * ng;

    auto issue_a = [&](int t, int st) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int li = 0; li < kCq4Limbs; ++li)  // 1 KiB = 8 rows of one limb
                __builtin_amdgcn_global_load_lds(asrc[i] + static_cast<size_t>(t) * (kCq4Limbs * 64) + li * 64,
                                                 &stage[st].a[li][2 * wid + i][0], 16, 0, 0);
    };
    auto load_b = [&](int t, uint32_t (&wd)[2]) {
#pragma unroll
        for (int u = 0; u < 2; ++u) wd[u] = bsrc[4 * (2 * t + u)];
    };
    auto write_b = [&](const uint32_t (&wd)[2], int st) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            uint32_t e[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) e[t] = lut[(wd[u] >> (4 * t)) & 0xFu];
            u32x4 hi, lo;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                hi[i] = __builtin_amdgcn_perm(e[2 * i + 1], e[2 * i], 0x05040100u);  // low halves
                lo[i] = __builtin_amdgcn_perm(e[2 * i + 1], e[2 * i], 0x07060302u);  // high halves
            }
            stage[st].b[u][0][bc >> 4][blane] = hi;
            stage[st].b[u][1][bc >> 4][blane] = lo;
        }
    };

    const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
    double acc[2][2][4];
#pragma unroll
    for (int tm = 0; tm < 2; ++tm)
#pragma unroll
        for (int tn = 0; tn < 2; ++tn)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[tm][tn][i] = 0.0;
    __syncthreads();  // the codebook is in LDS
    {
        issue_a(0, 0);
        uint32_t wd[2];
        load_b(0, wd);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        write_b(wd, 0);
    }
    __syncthreads();
    for (int t = 0; t < T; ++t) {
        const int st = t & 1;
        const bool more = t + 1 < T;  // uniform
        uint32_t wdn[2] = {};
        if (more) {
            issue_a(t + 1, st ^ 1);
            load_b(t + 1, wdn);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            bf16x8 bh[2], bl[2];
#pragma unroll
            for (int tn = 0; tn < 2; ++tn) {
                bh[tn] = __builtin_bit_cast(bf16x8, stage[st].b[u][0][wn * 2 + tn][lane]);
                bl[tn] = __builtin_bit_cast(bf16x8, stage[st].b[u][1][wn * 2 + tn][lane]);
            }
            f32x4_t P[2][2];
#pragma unroll
            for (int tm = 0; tm < 2; ++tm) {
                const int row_t = 32 * wm + 16 * tm + j;
                const int pr = row_t >> 1;
                const int idx = pr * 16 + 8 * (row_t & 1) + ((4 * u + q) ^ (pr & 7));
                bf16x8 av[kCq4Limbs];
#pragma unroll
                for (int li = 0; li < kCq4Limbs; ++li)
                    av[li] = __builtin_bit_cast(bf16x8, (&stage[st].a[li][0][0])[idx]);
#pragma unroll
                for (int tn = 0; tn < 2; ++tn) {
                    f32x4_t r = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[2], bl[tn], zero, 0, 0, 0);
                    r = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[1], bl[tn], r, 0, 0, 0);
                    r = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[2], bh[tn], r, 0, 0, 0);
                    r = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[0], bl[tn], r, 0, 0, 0);
                    r = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[1], bh[tn], r, 0, 0, 0);
                    P[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[0], bh[tn], r, 0, 0, 0);
                }
            }
            const int g = (2 * t + u) / spg;
#pragma unroll
            for (int tn = 0; tn < 2; ++tn) {
                const double nv = static_cast<double>(half_bits_to_float(nrm[tn][g]));
#pragma unroll
                for (int tm = 0; tm < 2; ++tm)
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[tm][tn][i] = fma(nv, static_cast<double>(P[tm][tn][i]), acc[tm][tn][i]);
            }
        }
        if (more) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            write_b(wdn, st ^ 1);
        }
        __syncthreads();
    }
#pragma unroll
    for (int tm = 0; tm < 2; ++tm)
#pragma unroll
        for (int tn = 0; tn < 2; ++tn) {
            const int col = n0 + 16 * tn + j;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = m0 + 16 * tm + 4 * q + i;
                if (row < Mi && col < N)
                    c[static_cast<size_t>(row) * N + col] = double_to_half_bits(acc[tm][tn][i]);
            }
        }
}

// Pipelined MFMA GEMM for 4-bit LSB-packed indices, taken when the tile's norms fit in LDS
// (ng <= 128, i.e. K <= 4096 at group size 32). The same 64 x 64 tiles, activation-limb
// layout, codebook limbs and float64 fold as cq4_gemm_mfma_kernel above, on
// v_mfma_f32_32x32x16_bf16 (32 matrix-core cycles) with a deeper copy pipeline:
//   - 8 wavefronts, two per SIMD: wavefront w owns the 32 x 32 output tile (rows 32 (w & 1),
//     columns 32 ((w >> 1) & 1)) for the sub-group (w >> 2) of every 64-value stage, so the
//     two wavefronts of a SIMD (w, w + 4) share a tile and split K between them. Per stage a
//     wavefront runs one chain of 12 MFMAs (3 activation limbs x 2 codebook limbs x 2 halves of
//     16 values, smallest products first; dependent 32x32x16 MFMAs issue back to back), and the
//     two halves of K are added in double at the end, through LDS, before the fp16 rounding.
//     On gfx950 a 32x32x16 MFMA leaves room for about 6 VALU instructions in the issue pipe it
//     shares with them (a 16x16x32 for about 2), so the previous stage's fold (16 conversions
//     and 16 float64 FMAs per wavefront) is laid between the chain's MFMAs;
//   - lane l of a 32x32x16 MFMA holds A[row l % 32][k = 8 (l / 32) .. +7] and B[k = 8 (l / 32)
//     .. +7][column l % 32], and result element v is row 8 (v / 4) + 4 (l / 32) + v % 4 of
//     column l % 32 (one column per lane, one norm per stage);
//   - every operand reaches LDS by global_load_lds: the activation limbs kCq4Stages stages deep
//     (wavefront w copies the 8-row block w of each limb, three 1 KiB copies per stage), the packed
//     indices by stage pairs (each thread copies the two words it decodes, one per stage, so it waits
//     only for its own wavefront's copies; a wavefront reads 8 columns x 32 contiguous bytes per
//     stage), the tile's norms (all groups) and the codebook once before the loop; the codebook
//     becomes two 256-entry tables (per byte of packed indices, the high or low bf16 limbs of its
//     two entries), so a word decodes with four byte extractions and eight table reads;
//   - iteration t copies stage t + 4 into slot t % 4 (its operands were read into registers in
//     iteration t - 1), and on even t the pair of stages t + 4, t + 5, then runs stage t's chain
//     with, between its MFMAs, stage t - 1's fold, the operand reads of stage t + 1 and the decode
//     of stage t + 2 into a double-buffered MFMA B layout (sub-group, codebook limb, 32-column
//     tile, half, slot), and passes one barrier. Past the last stage the copied stage is clamped,
//     so every wavefront issues the same copies per iteration and `s_waitcnt vmcnt(8)` leaves
//     exactly the two younger stages and one pair in flight. The loop issues no other
//     vector-memory instruction;
//   - the output tile is assembled in LDS and stored as 16-byte row pieces.
constexpr int kCq4Stages = 4;
constexpr int kCq4PipeWaves = 8;
constexpr uint32_t kCq4NormsMax = 128;  // norm groups per column held in LDS

struct Cq4PipeLds {
    // first, so that ds_read's 16-bit offset field reaches both tables from one address
    uint32_t lut[2][256];  // codebook limb (high, low), byte b: the limbs of entries b % 16 (low half) and b / 16
    u32x4 a[kCq4Stages][kCq4Limbs][8][64];   // as Cq4MfmaStage::a, per stage
    // stage-pair slot, wavefront w, stage of the pair, thread: the packed word the thread decodes
    uint32_t braw[2][kCq4PipeWaves][2][64];
    u32x4 b[2][2][2][2][2][64];              // stage parity, sub-group, codebook limb, 32-column tile, half, slot
    uint16_t norms[kCq4Tile * kCq4NormsMax + 128];  // tile column, group (fp16 bits), as in the array; copy slack
};
static_assert(sizeof(Cq4PipeLds) <= 160 * 1024, "LDS budget");


__global__ __launch_bounds__(64 * kCq4PipeWaves) void cq4_gemm_pipe_kernel(Cq4View w, const uint16_t* __restrict__ xs,
                                                                          uint16_t* __restrict__ c, uint32_t M,
                                                                          uint32_t gs, uint32_t ng, uint32_t tiles_m) {
    __shared__ Cq4PipeLds lds;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wid & 1, wn = (wid >> 1) & 1, ku = wid >> 2;
    const int col32 = lane & 31, half = lane >> 5;
    const int K = static_cast<int>(w.K), N = static_cast<int>(w.N), Mi = static_cast<int>(M);
    const int T = K / 64;
    const int spg = static_cast<int>(gs) >> 5;
    const int G = static_cast<int>(ng);
    const int mt0 = static_cast<int>(blockIdx.x % tiles_m) * kCq4Tile;
    const int nt0 = static_cast<int>(blockIdx.x / tiles_m) * kCq4Tile;

    // Activation-limb copy of this wavefront: 8-row block wid (row pairs 4 wid .. 4 wid + 3).
    const uint16_t* asrc;
    {
        const int pair = 4 * wid + (lane >> 4);
        const int row_t = 2 * pair + ((lane >> 3) & 1);
        asrc = xs + static_cast<size_t>(min(mt0 + row_t, Mi - 1)) * T * (kCq4Limbs * 64) + 8 * ((lane & 7) ^ (pair & 7));
    }
    // Packed-index word this thread decodes: sub-group bu, tile column bc, word bw.
    const int bc = 8 * wid + (lane >> 3), bu = (lane >> 2) & 1, bw = lane & 3;
    const int bdst = pipe_b_slot((bc & 31) + 32 * (bw & 1), bw >> 1, bu);
    // This thread copies the packed words it decodes (so it waits only for its own wavefront's
    // copies): per stage pair, words (lane % 8) of column bc for both stages, 32 contiguous bytes per
    // column and stage.
    const char* bsrc = reinterpret_cast<const char*>(w.packed) + static_cast<size_t>(min(nt0 + bc, N - 1)) * (K >> 1) +
                       4 * (lane & 7);
    // This lane's A operand: row 32 wm + (lane & 31), chunk 4 ku + 2 h + (lane >> 5) of a stage for
    // half h (the layout of Cq4MfmaStage::a).
    const int ar = 32 * wm + col32;
    const int apr = ar >> 1;
    const int aidx0 = apr * 16 + 8 * (ar & 1) + ((4 * ku + half) ^ (apr & 7));
    const int aidx1 = apr * 16 + 8 * (ar & 1) + ((4 * ku + 2 + half) ^ (apr & 7));
    const int bsrc0 = pipe_b_slot(lane, 0, ku), bsrc1 = pipe_b_slot(lane, 1, ku);

    // Stage t's activation limbs into stage slot st (past the last stage, t is clamped and st is not).
    auto issue = [&](int t, int st) {
#pragma unroll
        for (int li = 0; li < kCq4Limbs; ++li)
            __builtin_amdgcn_global_load_lds(asrc + static_cast<size_t>(t) * (kCq4Limbs * 64) + li * 64,
                                             &lds.a[st][li][wid][0], 16, 0, 0);
    };
    // Packed indices of stages 2 j and 2 j + 1 into slot `slot`, one copy per stage (each wavefront
    // reads 8 columns x 32 bytes). Past the end of a row (an odd stage count) the stage is clamped
    // to the last.
    auto issue_b = [&](int j, int slot) {
#pragma unroll
        for (int cc = 0; cc < 2; ++cc)
            __builtin_amdgcn_global_load_lds(bsrc + min(32 * (2 * j + cc), (K >> 1) - 32), &lds.braw[slot][wid][cc][0], 4,
                                             0, 0);
    };
    // Decode of stage t, in three steps laid into different MFMA windows: the packed word, its eight
    // codebook entries, then the high and low limbs written to the stage's B buffer.
    auto decode_word = [&](int t) { return lds.braw[(t >> 1) & 1][wid][t & 1][lane]; };
    auto decode_lookup = [&](uint32_t wd, u32x4& hi, u32x4& lo) {  // one table entry per byte (two values)
        // volatile: eight single reads straight into the two result vectors (paired reads of both
        // tables would need register moves, and a wait for them, before the writes)
        typedef __attribute__((address_space(3))) const volatile uint32_t lds_word;
        lds_word* lut = (lds_word*)(&lds.lut[0][0]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t b = (wd >> (8 * j)) & 0xFFu;
            hi[j] = lut[b];
            lo[j] = lut[256 + b];
        }
    };
    auto decode_write = [&](int t, const u32x4& hi, const u32x4& lo) {
        lds.b[t & 1][bu][0][bc >> 5][bw >> 1][bdst] = hi;
        lds.b[t & 1][bu][1][bc >> 5][bw >> 1][bdst] = lo;
    };
    auto decode = [&](int t) {
        u32x4 hi, lo;
        decode_lookup(decode_word(t), hi, lo);
        decode_write(t, hi, lo);
    };
    auto barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

    // The tile's norms (copied as they lie: 64 columns of G values, contiguous), the codebook, then
    // stages 0 .. 3 and pairs 0 and 1; stages 2 and 3 and pair 1 stay in flight while stages 0 and 1
    // are decoded and read: `s_waitcnt vmcnt(8)` below leaves exactly their 3 + 3 + 2 copies
    // outstanding, as each iteration's wait does.
    {
        const char* nsrc = reinterpret_cast<const char*>(w.norms) + static_cast<size_t>(nt0) * G * 2;
        const int units = kCq4Tile * G / 2;  // 4-byte units of the tile's norms
        const size_t last = static_cast<size_t>(N - nt0) * G * 2 - 4;  // the last whole unit in the array
        for (int b = wid; 64 * b < units; b += kCq4PipeWaves)  // uniform
            __builtin_amdgcn_global_load_lds(nsrc + min(static_cast<size_t>(4 * (64 * b + lane)), last),
                                             reinterpret_cast<char*>(lds.norms) + 256 * b, 4, 0, 0);
    }
    // The two codebook entries of this thread's table entry (byte tid % 256 of limb tid / 256). Loaded
    // through asm, which the compiler's wait insertion does not follow (it would otherwise wait for every
    // copy issued after them); the explicit vmcnt wait below covers them.
    uint32_t cb_lo, cb_hi;
    asm volatile("global_load_ushort %0, %1, off" : "=v"(cb_lo) : "v"(w.codebook + (tid & 15)) : "memory");
    asm volatile("global_load_ushort %0, %1, off" : "=v"(cb_hi) : "v"(w.codebook + ((tid >> 4) & 15)) : "memory");
    const int jmax = (T - 1) / 2;  // the last stage pair
    issue(0, 0);
    issue_b(0, 0);
    issue(min(1, T - 1), 1);
    issue(min(2, T - 1), 2);
    issue_b(min(1, jmax), 1);
    issue(min(3, T - 1), 3);
    // this wavefront's norms, codebook values, stages 0 and 1 and pair 0 are in; stages 2 and 3 (3
    // copies each) and pair 1 (2) may not be
    asm volatile("s_waitcnt vmcnt(8)" : "+v"(cb_lo), "+v"(cb_hi) :: "memory");  // the values are in from here
    {
        // The bf16 limbs of a codebook value are the high half of its fp32 form and the exact
        // remainder (at most 3 significant bits).
        auto limb = [&](uint16_t h) {
            const float v = half_bits_to_float(h);
            const uint32_t hi = __float_as_uint(v) & 0xFFFF0000u;
            return (tid >> 8) == 0 ? hi >> 16 : __float_as_uint(v - __uint_as_float(hi)) >> 16;
        };
        lds.lut[tid >> 8][tid & 255] = limb(static_cast<uint16_t>(cb_lo)) | (limb(static_cast<uint16_t>(cb_hi)) << 16);
    }
    barrier();  // norms and tables visible, every wavefront's stages 0 and 1 and pair 0 copied
    {
        u32x4 hi0, lo0, hi1, lo1;
        const uint32_t w0 = decode_word(0), w1 = decode_word(1);
        decode_lookup(w0, hi0, lo0);
        decode_lookup(w1, hi1, lo1);
        decode_write(0, hi0, lo0);
        decode_write(1, hi1, lo1);  // past the last stage: an unread buffer from a clamped copy
    }
    barrier();

    // MFMA operands of one stage in registers: activation limbs x halves, codebook limbs x halves.
    struct Operands {
        bf16x8 a[kCq4Limbs][2], b[2][2];
    };
    Operands ops[2];
    // Operand reads of stage t, in the order the chain uses them: limb 2, codebook low, limb 1,
    // codebook high, limb 0 (one pair per call, part 0 .. 4).
    auto read_part = [&](Operands& o, int t, int part) {
        const int sidx = t & (kCq4Stages - 1), par = t & 1;
        if (part == 0 || part == 2 || part == 4) {
            const int li = 2 - part / 2;
            o.a[li][0] = __builtin_bit_cast(bf16x8, (&lds.a[sidx][li][0][0])[aidx0]);
            o.a[li][1] = __builtin_bit_cast(bf16x8, (&lds.a[sidx][li][0][0])[aidx1]);
        } else {
            const int cl = part == 1 ? 1 : 0;
            o.b[cl][0] = __builtin_bit_cast(bf16x8, lds.b[par][ku][cl][wn][0][bsrc0]);
            o.b[cl][1] = __builtin_bit_cast(bf16x8, lds.b[par][ku][cl][wn][1][bsrc1]);
        }
    };
#pragma unroll
    for (int part = 0; part < 5; ++part) read_part(ops[0], 0, part);
    barrier();  // stage 0's slot is read before iteration 0 copies into it

    f32x16 zero16;
#pragma unroll
    for (int v = 0; v < 16; ++v) zero16[v] = 0.0f;
    double acc[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0;
    struct Stage {
        f32x16 p;
        double norm;
    };
    Stage st_buf[2];
    st_buf[1].p = zero16;  // iteration 0 folds these zeros
    st_buf[1].norm = 0.0;
    // fold operation f (0 .. 31) of a stage: per result a conversion, then (one result later) a
    // float64 FMA acc += norm * P
    double pd[2];
    auto fold_op = [&](const Stage& r, int f) {
        if (f == 0) {
            pd[0] = static_cast<double>(r.p[0]);
        } else if (f == 31) {
            acc[15] = fma(r.norm, pd[1], acc[15]);
        } else if (f & 1) {
            const int o = (f + 1) >> 1;  // 1 .. 15
            pd[o & 1] = static_cast<double>(r.p[o]);
        } else {
            const int o = (f - 2) >> 1;  // 0 .. 14
            acc[o] = fma(r.norm, pd[o & 1], acc[o]);
        }
    };

    // Iteration t: copies of stage t + 4 into slot t % 4 (stage t's operands are in registers) and on
    // even t of the pair t + 4, t + 5, then the 12-MFMA chain of stage t with, between its MFMAs, the
    // fold of stage t - 1, the operand reads of stage t + 1, stage t's norm, and the decode of stage
    // t + 2 (after `s_waitcnt vmcnt(8)`: this wavefront's copies of stage t + 2 and of its pair have
    // landed; stages t + 3 and t + 4 and the youngest pair may not have); then one barrier, after
    // which every wavefront's copies of stage t + 2 and its decode are visible and every read of
    // stage t + 1's slot is done.
    for (int t0 = 0; t0 < T; t0 += 2) {
        static_for<2>([&](auto uc) {
            constexpr int u = decltype(uc)::value;
            const int t = t0 + u;
            if (t < T) {  // uniform
                Stage& cur = st_buf[u];
                const Stage& old = st_buf[u ^ 1];
                const Operands& op = ops[u];
                Operands& nxt = ops[u ^ 1];
                issue(min(t + 4, T - 1), t & (kCq4Stages - 1));
                if constexpr (u == 0) issue_b(min(t / 2 + 2, jmax), (t / 2) & 1);  // t is even
                uint32_t wd = 0;
                u32x4 dhi, dlo;
                uint16_t nraw = 0;
                static_for<12>([&](auto ic) {
                    constexpr int i = decltype(ic)::value;
                    constexpr int pr = i >> 1, h = i & 1;
                    constexpr int li = (0x010212 >> (4 * pr)) & 0xF;  // 2, 1, 2, 0, 1, 0
                    constexpr int cl = (0x001011 >> (4 * pr)) & 0xF;  // 1, 1, 0, 1, 0, 0
                    cur.p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op.a[li][h], op.b[cl][h], i == 0 ? zero16 : cur.p,
                                                                    0, 0, 0);
                    __builtin_amdgcn_sched_barrier(0);  // the MFMA first: a wait below stalls only the rest
                    constexpr int f0 = i < 8 ? 3 * i : 24 + 2 * (i - 8);
                    constexpr int f1 = i < 8 ? f0 + 3 : f0 + 2;
                    static_for<f1 - f0>([&](auto fc) { fold_op(old, f0 + decltype(fc)::value); });
                    // LDS reads complete in issue order, so the decode's reads go first: its waits
                    // (for the packed word, then for the table entries) do not wait for the operand
                    // reads behind them.
                    if constexpr (i == 0) {
                        // this wavefront's copies of stage t + 2 and of its pair; after them come stages
                        // t + 3, t + 4 and one pair (3 + 3 + 2 copies)
                        asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
                        wd = decode_word(t + 2);
                        nraw = lds.norms[(32 * wn + col32) * G + (2 * t + ku) / spg];
                    }
                    if constexpr (i == 1) decode_lookup(wd, dhi, dlo);
                    if constexpr (i >= 2 && i < 7) read_part(nxt, t + 1, i - 2);  // past the last stage: unused
                    // the compiler waits for every LDS read before the writes; late, they are all in
                    if constexpr (i == 10) decode_write(t + 2, dhi, dlo);  // past the last stage: an unread buffer
                    if constexpr (i == 9) cur.norm = static_cast<double>(half_bits_to_float(nraw));
                    __builtin_amdgcn_sched_barrier(0);
                });
                barrier();
            }
        });
    }
    if (T & 1) {  // uniform: the last stage's products are in st_buf[(T - 1) % 2]
#pragma unroll
        for (int f = 0; f < 32; ++f) fold_op(st_buf[0], f);
    } else {
#pragma unroll
        for (int f = 0; f < 32; ++f) fold_op(st_buf[1], f);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the clamped copies past the last stage
    // The two halves of K of each tile, added in double: the wavefront of sub-group u finishes results
    // 8 u .. 8 u + 7 of its tile and hands the other eight to its partner through LDS. The fp16 tile
    // is then assembled in LDS and stored as one 16-byte row piece per thread.
    double* red = reinterpret_cast<double*>(&lds.a[0][0][0][0]);  // [4 tiles][16 results][64 lanes]
    uint16_t* tile = reinterpret_cast<uint16_t*>(&lds.b[0][0][0][0][0][0]);  // [64 rows][64 columns]
    auto hand_over = [&](auto mine_c) {
        constexpr int other = 8 - decltype(mine_c)::value;
#pragma unroll
        for (int v = 0; v < 8; ++v) red[((wid & 3) * 16 + other + v) * 64 + lane] = acc[other + v];
    };
    auto finish = [&](auto mine_c) {
        constexpr int mine = decltype(mine_c)::value;
#pragma unroll
        for (int v = mine; v < mine + 8; ++v) {
            const int row = 32 * wm + 8 * (v >> 2) + 4 * half + (v & 3);
            const double s = acc[v] + red[((wid & 3) * 16 + v) * 64 + lane];
            tile[row * kCq4Tile + 32 * wn + col32] = double_to_half_bits(s);
        }
    };
    __syncthreads();  // every wavefront is past its last read of lds.a and lds.b, and every copy has landed
    if (ku == 0)
        hand_over(std::integral_constant<int, 0>{});
    else
        hand_over(std::integral_constant<int, 8>{});
    __syncthreads();
    if (ku == 0)
        finish(std::integral_constant<int, 0>{});
    else
        finish(std::integral_constant<int, 8>{});
    __syncthreads();
    {
        const int rl = tid >> 3, c8 = 8 * (tid & 7);  // tile row, first of 8 columns
        const int row = mt0 + rl, col = nt0 + c8;
        const u32x4 v = *reinterpret_cast<const u32x4*>(&tile[rl * kCq4Tile + c8]);
        const bool vec = N % 8 == 0 && (reinterpret_cast<uintptr_t>(c) & 15) == 0;  // uniform
        if (row < Mi) {
            uint16_t* dst = c + static_cast<size_t>(row) * N + col;
            if (vec && col + 8 <= N) {
                *reinterpret_cast<u32x4*>(dst) = v;
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (col + e < N) dst[e] = static_cast<uint16_t>(v[e >> 1] >> (16 * (e & 1)));
            }
        }
    }
}

// A null pointer counts as aligned (the array is absent).
bool aligned(const void* p, uintptr_t bytes) { return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0; }

bool cq4_uses_mfma(const Cq4View& w, uint32_t m) {
    const bool orth = (w.flags & kCq4FlagOrthogonal) != 0;
    const uint32_t gs = orth ? w.K : w.group_size;
    const bool inter = (w.flags & kCq4FlagInterleaved4Row) != 0;
    return m >= kCq4MfmaMinRows && w.bits == 4 && !inter && gs % 32 == 0 && w.K % 64 == 0;
}

// Decode-sized Hadamard calls: transform and GEMV in one launch (cq4_gemv_fused_kernel).
bool cq4_gemv_fused(const Cq4View& w, uint32_t m) {
    const bool orth = (w.flags & kCq4FlagOrthogonal) != 0;
    const uint32_t gs = w.group_size;
    return !orth && m >= 1 && m <= 4 && w.bits == 4 && gs % 8 == 0 && gs <= 256 && (gs & (gs - 1)) == 0 &&
           static_cast<uint64_t>(m) * w.K <= kCq4FusedMaxValues;
}

template <int ROWS>
hipError_t launch_gemm(const Cq4View& w, const float* ap, uint16_t* c, uint32_t m, uint32_t gs, uint32_t ng,
                       hipStream_t stream) {
    const dim3 grid((w.N + 255) / 256, (m + ROWS - 1) / ROWS);
    const bool inter = (w.flags & kCq4FlagInterleaved4Row) != 0;
    if (inter)
        hipLaunchKernelGGL((cq4_gemm_kernel<ROWS, 1>), grid, dim3(256), 0, stream, w, ap, c, m, gs, ng);
    else if (w.bits == 4 && gs % 8 == 0)
        hipLaunchKernelGGL((cq4_gemm_kernel<ROWS, 0>), grid, dim3(256), 0, stream, w, ap, c, m, gs, ng);
    else
        hipLaunchKernelGGL((cq4_gemm_kernel<ROWS, 2>), grid, dim3(256), 0, stream, w, ap, c, m, gs, ng);
    return hipGetLastError();
}

}  // namespace

size_t cq4_workspace_bytes(const Cq4View& w, uint32_t m) {
    if (cq4_gemv_fused(w, m)) return 0;
    const size_t values = static_cast<size_t>(m) * w.K;  // K % 64 == 0 on the MFMA path: no padding
    return cq4_uses_mfma(w, m) ? values * 3 * sizeof(uint16_t) : values * sizeof(float);
}

hipError_t launch_cq4_matmul(const Cq4View& w, const uint16_t* a, uint32_t m, uint16_t* c, void* workspace,
                             hipStream_t stream) {
    // The transform writes the code-basis activations as fp32 rows, or, for the MFMA GEMM, directly as
    // their bf16 limbs.
    if (cq4_gemv_fused(w, m)) {
        const dim3 grid((w.N + 3) / 4);
        const size_t lds = 2 * sizeof(float) * m * w.K;
        const bool inter = (w.flags & kCq4FlagInterleaved4Row) != 0;
        const uint32_t gs = w.group_size, ng = w.num_groups;
        if (m == 1) {
            if (inter) hipLaunchKernelGGL((cq4_gemv_fused_kernel<1, true>), grid, dim3(256), lds, stream, w, a, c, m, gs, ng);
            else hipLaunchKernelGGL((cq4_gemv_fused_kernel<1, false>), grid, dim3(256), lds, stream, w, a, c, m, gs, ng);
        } else {
            if (inter) hipLaunchKernelGGL((cq4_gemv_fused_kernel<4, true>), grid, dim3(256), lds, stream, w, a, c, m, gs, ng);
            else hipLaunchKernelGGL((cq4_gemv_fused_kernel<4, false>), grid, dim3(256), lds, stream, w, a, c, m, gs, ng);
        }
        return hipGetLastError();
    }
    const bool mfma = cq4_uses_mfma(w, m);
    float* ap = mfma ? nullptr : static_cast<float*>(workspace);
    uint16_t* xs = mfma ? static_cast<uint16_t*>(workspace) : nullptr;
    const bool orth = (w.flags & kCq4FlagOrthogonal) != 0;
    const uint32_t gs = orth ? w.K : w.group_size, ng = orth ? 1 : w.num_groups;
    if (orth) {
        hipLaunchKernelGGL(cq4_transform_orthogonal_kernel, dim3((w.K + 255) / 256, m), dim3(256), 0, stream, w, a,
                           ap, xs);
    } else if (mfma && (w.group_size == 64 || w.group_size == 128 || w.group_size == 256) && aligned(a, 16) &&
               aligned(w.input_scale_recip, 16) && aligned(w.input_scale, 16) && aligned(w.left_signs, 8) &&
               aligned(w.right_signs, 8) && aligned(w.permutation, 16)) {
        const uint32_t chunks = (w.K + 511) / 512;
        const uint32_t tiles_m = (m + kCq4Tile - 1) / kCq4Tile;
        const bool xcd_rows = tiles_m % 8 == 0;  // the GEMM then reads row tile t on XCD t % 8
        // XCD lane x holds tiles_m / 8 row tiles of 64 rows (the last may be partial)
        const dim3 grid(xcd_rows ? 8 * ((tiles_m / 8 * kCq4Tile * chunks + 3) / 4) : (m * chunks + 3) / 4);
        if (w.group_size == 64)
            hipLaunchKernelGGL(cq4_transform_hadamard_limbs_kernel<64>, grid, dim3(256), 0, stream, w, a, xs, m, chunks,
                               xcd_rows);
        else if (w.group_size == 128)
            hipLaunchKernelGGL(cq4_transform_hadamard_limbs_kernel<128>, grid, dim3(256), 0, stream, w, a, xs, m, chunks,
                               xcd_rows);
        else
            hipLaunchKernelGGL(cq4_transform_hadamard_limbs_kernel<256>, grid, dim3(256), 0, stream, w, a, xs, m, chunks,
                               xcd_rows);
    } else if (w.group_size == 64 || w.group_size == 128 || w.group_size == 256) {
        const uint32_t pairs = m * w.num_groups;
        const dim3 grid((pairs + 3) / 4);
        if (w.group_size == 64)
            hipLaunchKernelGGL(cq4_transform_hadamard_wave_kernel<1>, grid, dim3(256), 0, stream, w, a, ap, xs, pairs);
        else if (w.group_size == 128)
            hipLaunchKernelGGL(cq4_transform_hadamard_wave_kernel<2>, grid, dim3(256), 0, stream, w, a, ap, xs, pairs);
        else
            hipLaunchKernelGGL(cq4_transform_hadamard_wave_kernel<4>, grid, dim3(256), 0, stream, w, a, ap, xs, pairs);
    } else {
        // group_size / 2 threads (one for a group of 1, whose transform is the identity)
        hipLaunchKernelGGL(cq4_transform_hadamard_kernel, dim3(w.num_groups, m), dim3(w.group_size > 1 ? w.group_size / 2 : 1),
                           0, stream, w, a, ap, xs);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const bool inter = (w.flags & kCq4FlagInterleaved4Row) != 0;
    if (mfma) {
        const uint32_t tiles_m = (m + kCq4Tile - 1) / kCq4Tile, tiles_n = (w.N + kCq4Tile - 1) / kCq4Tile;
        // the pipelined kernel copies the tile's norms in 4-byte units
        if (ng <= kCq4NormsMax && (static_cast<size_t>(w.N) * ng) % 2 == 0 && aligned(w.norms, 4))
            hipLaunchKernelGGL(cq4_gemm_pipe_kernel, dim3(tiles_m * tiles_n), dim3(64 * kCq4PipeWaves), 0, stream, w,
                               xs, c, m, gs, ng, tiles_m);
        else
            hipLaunchKernelGGL(cq4_gemm_mfma_kernel, dim3(tiles_m * tiles_n), dim3(256), 0, stream, w, xs, c, m, gs,
                               ng, tiles_m);
        return hipGetLastError();
    }
    if (m <= 4 && w.bits == 4 && gs % 8 == 0) {
        const dim3 grid((w.N + 3) / 4);
        if (m == 1) {
            if (inter) hipLaunchKernelGGL((cq4_gemv_kernel<1, true>), grid, dim3(256), 0, stream, w, ap, c, m, gs, ng);
            else hipLaunchKernelGGL((cq4_gemv_kernel<1, false>), grid, dim3(256), 0, stream, w, ap, c, m, gs, ng);
        } else {
            if (inter) hipLaunchKernelGGL((cq4_gemv_kernel<4, true>), grid, dim3(256), 0, stream, w, ap, c, m, gs, ng);
            else hipLaunchKernelGGL((cq4_gemv_kernel<4, false>), grid, dim3(256), 0, stream, w, ap, c, m, gs, ng);
        }
        return hipGetLastError();
    }
    return m >= 4 ? launch_gemm<4>(w, ap, c, m, gs, ng, stream) : launch_gemm<1>(w, ap, c, m, gs, ng, stream);
}

}  // namespace spaceslug
