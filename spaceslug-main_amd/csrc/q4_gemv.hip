// Decode GEMV for 1..4 rows: y[m][n] = sum_k x[m][k] * v(k, n) * s(n, k/32).
//
// HBM-bound: one pass over the packed weights and scales. Work mapping:
//   - a wavefront owns CPW consecutive columns; lane l owns the scale groups
//     g = l, l + 64, ... of each. A column's packed bytes are contiguous
//     (q4gemm.comp:13, byte n*(K/2) + k/2), so for one column the 64 lanes'
//     16-byte loads cover 1 KiB of contiguous memory: every weight load is a
//     fully coalesced 128-bit load, and a lane's 16 bytes are exactly one
//     32-value scale group. The lane's scale s(n, g) is one coalesced 32-bit
//     load (lanes hold consecutive groups of the column), so no LDS broadcast
//     is needed: each scale is read once, by the one lane that applies it;
//   - all weight and scale loads of the wavefront's columns for a K chunk are
//     issued before any arithmetic, so the whole wavefront's data is in flight
//     at once; the columns are then consumed in issue order as they land;
//   - x stays in registers for the whole chunk (the lane's own groups), read
//     straight from global memory (it is tiny and L1/L2 resident);
//   - nibbles are decoded in registers to v / 16 by v_cvt_off_f32_i4
//     (nibbles_signed_16th, exact), so a group partial is 2^-4 * sum x v with
//     no offset to cancel; it is scaled by s and accumulated per lane; the 64
//     lane partials of a column are summed with DPP row operations plus two
//     row broadcasts, and the factor 16 restored exactly at the end.
// K larger than one chunk (64 * SPC groups per lane pass) is walked in chunks.
// One row with K <= 4096 takes the software-pipelined integer kernel below
// (q4_gemv_pipe_kernel), which reads the weights in the same mapping.
#include "q4_device.hpp"
#include "q4_kernels.hpp"

namespace spaceslug {
namespace {

constexpr int kGemvThreads = 256;

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_src(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}

// Sum over the 64 lanes; every lane receives the total (readlane of lane 63).
__device__ __forceinline__ float wave_reduce_dpp(float v) {
    v += dpp_src<0xB1>(v);         // quad_perm [1,0,3,2]: pairs
    v += dpp_src<0x4E>(v);         // quad_perm [2,3,0,1]: quads
    v += dpp_src<0x141>(v);        // row_half_mirror: 8-lane halves
    v += dpp_src<0x140>(v);        // row_mirror: 16-lane rows
    v += dpp_src<0x142, 0xA>(v);   // row_bcast:15 into rows 1 and 3
    v += dpp_src<0x143, 0xC>(v);   // row_bcast:31 into rows 2 and 3 -> row 3 holds the total
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Loads of one K chunk for CPW columns: x first (coalesced, into xr), then every
// weight and scale word. Kept in one straight-line block so the memory counters,
// which retire loads in issue order, release x before any weight data.
template <int M, int SPC, int CPW>
struct ChunkLoads {
    static constexpr int kChunkF4 = 64 * SPC * 8;  // float4 of x per row and chunk
    static constexpr int kPerThread = kChunkF4 / kGemvThreads;
    static_assert(kChunkF4 % kGemvThreads == 0, "x chunk must split evenly over the workgroup");
    f32x4 xr[M][kPerThread];
    u32x4 wv[CPW][SPC];
    float sc[CPW][SPC];
};

template <int M, int SPC, int CPW>
__device__ __forceinline__ void issue_chunk(ChunkLoads<M, SPC, CPW>& L, const float* x,
                                            const u32x4* __restrict__ wq, const float* __restrict__ ws, int N,
                                            int K, int G, int col0, int g0, int lane) {
    using CL = ChunkLoads<M, SPC, CPW>;
    const int c4_begin = g0 * 8;
    const int c4_last = min(CL::kChunkF4, (K >> 2) - c4_begin) - 1;
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int i = 0; i < CL::kPerThread; ++i) {
            // slots past K repeat the last chunk; their groups get a zero scale
            const int c = min(static_cast<int>(threadIdx.x) + i * kGemvThreads, c4_last);
            L.xr[m][i] = reinterpret_cast<const f32x4*>(x + static_cast<size_t>(m) * K)[c4_begin + c];
        }
    // Compiler-only fence: no load moves across it, so x is issued before the weights
    // (x is deliberately not __restrict__, which would let its loads sink past it).
    asm volatile("" ::: "memory");
    // Column bases are wave-uniform (SGPR); the lane's offset is one unsigned 32-bit
    // byte offset, so each load is SGPR base + VGPR offset.
    uint32_t off16[SPC], off4[SPC];
#pragma unroll
    for (int s = 0; s < SPC; ++s) {
        const uint32_t g = static_cast<uint32_t>(min(g0 + 64 * s + lane, G - 1));
        off16[s] = g * 16u;
        off4[s] = g * 4u;
    }
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
        const size_t base = static_cast<size_t>(min(col0 + c, N - 1)) * G;
        const char* wcol = reinterpret_cast<const char*>(wq + base);
        const char* scol = reinterpret_cast<const char*>(ws + base);
#pragma unroll
        for (int s = 0; s < SPC; ++s) {
            L.wv[c][s] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wcol + off16[s]));
            L.sc[c][s] = __builtin_nontemporal_load(reinterpret_cast<const float*>(scol + off4[s]));
        }
    }
    asm volatile("" ::: "memory");
}

template <int M, int SPC, int CPW>
__device__ __forceinline__ void consume_chunk(ChunkLoads<M, SPC, CPW>& L, f32x4* xs, float (&acc)[CPW][M], int G,
                                              int g0, int lane) {
    using CL = ChunkLoads<M, SPC, CPW>;
    // x to LDS (chunk q of group g at slot g*8 + (q ^ (g & 7)): a wavefront's 128-bit
    // reads of 64 groups then hit 8 distinct 16-byte bank groups per 8 lanes).
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int i = 0; i < CL::kPerThread; ++i) {
            const int c = static_cast<int>(threadIdx.x) + i * kGemvThreads;
            const int g = c >> 3, q = c & 7;
            xs[m * CL::kChunkF4 + (g << 3) + (q ^ (g & 7))] = L.xr[m][i];
        }
    __syncthreads();
    float xv[M][SPC][32];
#pragma unroll
    for (int m = 0; m < M; ++m) {
#pragma unroll
        for (int s = 0; s < SPC; ++s) {
            const int gl = 64 * s + lane;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const f32x4 t = xs[m * CL::kChunkF4 + (gl << 3) + (q ^ (gl & 7))];
                xv[m][s][4 * q + 0] = t[0];
                xv[m][s][4 * q + 1] = t[1];
                xv[m][s][4 * q + 2] = t[2];
                xv[m][s][4 * q + 3] = t[3];
            }
        }
    }
    // Groups past K contribute through a zero scale: a select, not a branch, so no
    // branch splits the batch of outstanding loads.
#pragma unroll
    for (int c = 0; c < CPW; ++c)
#pragma unroll
        for (int s = 0; s < SPC; ++s) L.sc[c][s] = (g0 + 64 * s + lane < G) ? L.sc[c][s] : 0.0f;

    // Columns in issue order, each as soon as its loads have landed.
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
#pragma unroll
        for (int s = 0; s < SPC; ++s) {
            float f[32];
#pragma unroll
            for (int w = 0; w < 4; ++w) nibbles_signed_16th(L.wv[c][s][w], *reinterpret_cast<float(*)[8]>(&f[8 * w]));
#pragma unroll
            for (int m = 0; m < M; ++m) {
                float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    p0 = fmaf(xv[m][s][k], f[k], p0);
                    p1 = fmaf(xv[m][s][16 + k], f[16 + k], p1);
                }
                acc[c][m] = fmaf(L.sc[c][s], p0 + p1, acc[c][m]);
            }
        }
    }
}

// SINGLE: K fits one chunk (G <= 64 * SPC), straight-line code; otherwise K is
// walked chunk by chunk.
template <int M, int SPC, int CPW, bool SINGLE>
__global__ __launch_bounds__(kGemvThreads) void q4_gemv_kernel(const float* x,  // not restrict: see issue_chunk
                                                              const u32x4* __restrict__ wq,
                                                              const float* __restrict__ ws,
                                                              float* __restrict__ y, int N, int K) {
    using CL = ChunkLoads<M, SPC, CPW>;
    __shared__ f32x4 xs[M * CL::kChunkF4];
    const int lane = threadIdx.x & 63;
    // The wavefront index is uniform; readfirstlane keeps it and every column base
    // derived from it in SGPRs. Every wavefront takes part in the barriers;
    // past-the-end wavefronts work on a clamped column and store nothing.
    const int wave =
        __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x * (kGemvThreads >> 6) + (threadIdx.x >> 6)));
    const int col0 = wave * CPW;
    const int G = K >> 5;

    float acc[CPW][M];
#pragma unroll
    for (int c = 0; c < CPW; ++c)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[c][m] = 0.0f;

    if constexpr (SINGLE) {
        CL L;
        issue_chunk<M, SPC, CPW>(L, x, wq, ws, N, K, G, col0, 0, lane);
        consume_chunk<M, SPC, CPW>(L, xs, acc, G, 0, lane);
    } else {
        for (int g0 = 0; g0 < G; g0 += 64 * SPC) {
            CL L;
            issue_chunk<M, SPC, CPW>(L, x, wq, ws, N, K, G, col0, g0, lane);
            if (g0 > 0) __syncthreads();  // previous chunk's LDS reads are done
            consume_chunk<M, SPC, CPW>(L, xs, acc, G, g0, lane);
        }
    }
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
        const int col = col0 + c;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float total = wave_reduce_dpp(acc[c][m]);
            if (lane == 0 && col < N) y[static_cast<size_t>(m) * N + col] = total * kSixteenthsUnit;
        }
    }
}

// Software-pipelined single-row decode (M = 1, K <= 4096) in integer arithmetic.
//
// x is recoded once per workgroup. For each 32-value group g, with e_g the
// exponent for which max|x| < 2^e_g, X_k = rint(x_k * 2^(30 - e_g)) is an integer
// with |X_k| <= 2^30 that holds x_k to within 2^(e_g - 31), at most 2^-30 of the
// group's largest magnitude (finer than fp32's own rounding of a product of that
// magnitude, so a group holding an outlier loses nothing against float arithmetic).
// X_k is written as eight signed base-16 digits d_j in [-8, 7]: with
// Y = X + 0x88888888 (0 <= Y < 2^32), d_j = (hex digit j of Y) - 8, whose 4-bit two's
// complement is (hex digit j of Y) xor 8. Digit j of the eight values
// k = 8w .. 8w + 7 of a group is packed into one word, nibble t holding k = 8w + t:
// the layout of the packed weight words. v_dot8_i32_i4 (eight signed 4-bit
// products plus an int32 add) then takes a weight word and a digit word as they
// are, with no nibble decoding:
//   sum_k v_k X_k = 65536 H + L,  H = sum_{j=4..7} 16^(j-4) sum_k v_k d_kj,
//                                 L = sum_{j=0..3} 16^j     sum_k v_k d_kj,
// both evaluated by Horner steps (a shift by 4 between digits). Over one group
// |H|, |L| <= 32 * 8 * 34952 < 2^24, so both are exact in int32 and in float, and
// 65536 H + L is rounded once (one fma). The group partial
// (65536 H + L) * 2^(e_g - 30) * s(n, g) is accumulated in fp32 per lane.
// Cost per 32 nibbles: 32 v_dot8 + 6 shifts + 6 other VALU ops, against 68 for
// decoding to float (4 x (8 conversions + 1 shift + 8 fma)); the kernel is bound
// by its per-wavefront VALU time as much as by HBM, so this is what buys speed.
//
// Each wavefront owns cpb = D + (D + 1) * reps consecutive columns in D + 1
// register slots (column c in slot c % (D + 1)). Before computing column i it
// issues the loads of column i + D into the slot column i - 1 has released, so
// D columns stay in flight while a column computes (refilling a slot only after
// computing it leaves D - 1 in flight during that time: measured 8.0 against
// 7.5 us per launch at K = 4096, N = 14336).
constexpr int kXDigits = 8;               // signed base-16 digits per recoded x value
constexpr int kXFracBits = 30;            // |X| <= 2^30
constexpr uint32_t kXBias = 0x88888888u;  // 8 in each of the eight digit positions
constexpr int kBufferFlags = 0x00020000;   // buffer resource word 3: 32-bit data format
constexpr int kNontemporal = 2;            // buffer load cache policy: nt

// 8 x 8 transpose of 4-bit cells: on return nibble t of r[j] is what nibble j of
// r[t] held (16-bit and 8-bit blocks by byte permutes, then nibble swaps).
__device__ __forceinline__ void transpose_nibbles(uint32_t (&r)[8]) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint32_t a = r[t], b = r[t + 4];
        r[t] = __builtin_amdgcn_perm(b, a, 0x05040100u);      // bytes a0 a1 b0 b1
        r[t + 4] = __builtin_amdgcn_perm(b, a, 0x07060302u);  // bytes a2 a3 b2 b3
    }
#pragma unroll
    for (int t : {0, 1, 4, 5}) {
        const uint32_t a = r[t], b = r[t + 2];
        r[t] = __builtin_amdgcn_perm(b, a, 0x06020400u);      // bytes a0 b0 a2 b2
        r[t + 2] = __builtin_amdgcn_perm(b, a, 0x07030501u);  // bytes a1 b1 a3 b3
    }
#pragma unroll
    for (int t = 0; t < 8; t += 2) {
        const uint32_t a = r[t], b = r[t + 1];
        r[t] = (a & 0x0F0F0F0Fu) | ((b << 4) & 0xF0F0F0F0u);
        r[t + 1] = ((a >> 4) & 0x0F0F0F0Fu) | (b & 0xF0F0F0F0u);
    }
}

// Chunk swizzle of the recoded-x staging area (per group: 8 chunks of 16 bytes).
__device__ __forceinline__ int xds_swizzle(int group) { return (group >> 1) & 7; }

template <int SPC>
struct PipeSlot {
    u32x4 wv[SPC];
    float sc[SPC];
};

// The lane's recoded x: digit j of word w of group slot s at d[s][w * kXDigits + j],
// and the group's factor 2^(e_g - 30) (0 past K, NaN when the group holds a
// non-finite value, so that its outputs are NaN).
template <int SPC>
struct XDigits {
    uint32_t d[SPC][4 * kXDigits];
    float c[SPC];
};

// One column's weights and scales through buffer resources whose base is the
// column (scalar arithmetic only) and whose size is one column: the lane offsets
// are fixed for the whole kernel, and a lane whose group lies past K reads zeros
// (the buffer range check), so it contributes nothing without a per-column select.
// Weights and scales are read exactly once: nontemporal (aux 2) keeps them from
// displacing x and each other in the caches.
template <int SPC>
__device__ __forceinline__ void pipe_issue(PipeSlot<SPC>& slot, const u32x4* __restrict__ wq,
                                           const float* __restrict__ ws, int col, int N, int G,
                                           const uint32_t (&off16)[SPC], const uint32_t (&off4)[SPC]) {
    const size_t base = static_cast<size_t>(min(col, N - 1)) * G;
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<u32x4*>(wq + base), 0, G * 16, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(ws + base), 0, G * 4, kBufferFlags);
#pragma unroll
    for (int s = 0; s < SPC; ++s) {
        slot.wv[s] = __builtin_amdgcn_raw_buffer_load_b128(rw, off16[s], 0, kNontemporal);
        slot.sc[s] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, off4[s], 0, kNontemporal));
    }
}

// The lane's share of one column (not yet summed over the wavefront).
template <int SPC>
__device__ __forceinline__ float pipe_partial(const PipeSlot<SPC>& slot, const XDigits<SPC>& xd) {
    float acc = 0.0f;
#pragma unroll
    for (int s = 0; s < SPC; ++s) {
        int hi = 0;
#pragma unroll
        for (int j = kXDigits - 1; j >= 4; --j) {
            if (j < kXDigits - 1) hi *= 16;
#pragma unroll
            for (int w = 0; w < 4; ++w)
                hi = __builtin_amdgcn_sdot8(static_cast<int>(slot.wv[s][w]), static_cast<int>(xd.d[s][w * kXDigits + j]),
                                            hi, false);
        }
        int lo = 0;
#pragma unroll
        for (int j = 3; j >= 0; --j) {
            if (j < 3) lo *= 16;
#pragma unroll
            for (int w = 0; w < 4; ++w)
                lo = __builtin_amdgcn_sdot8(static_cast<int>(slot.wv[s][w]), static_cast<int>(xd.d[s][w * kXDigits + j]),
                                            lo, false);
        }
        const float p = fmaf(static_cast<float>(hi), 65536.0f, static_cast<float>(lo));
        acc = fmaf(slot.sc[s], p * xd.c[s], acc);
    }
    return acc;
}

// Columns col0 .. col0 + cpb - 1 of a row x holding an infinity or a NaN, in double
// with every term x * (v * s) formed as the double reference forms it (q4gemm_ref,
// test_q4gemm.cpp:102-119): such a row's outputs are all infinite or NaN, and IEEE
// arithmetic gives the reference's pattern (inf * 0 is NaN, opposite infinities give
// NaN) in any summation order. Lane l takes groups l, l + 64, ...; reached only for
// non-finite x, so it is written for clarity, not speed.
__device__ __forceinline__ void pipe_ieee_columns(const float* x, const uint32_t* __restrict__ wq,
                                               const float* __restrict__ ws, float* __restrict__ y, int N, int G,
                                               int col0, int cpb, int lane) {
    for (int i = 0; i < cpb && col0 + i < N; ++i) {
        const int col = col0 + i;
        double acc = 0.0;
        for (int g = lane; g < G; g += 64) {
            const double s = static_cast<double>(ws[static_cast<size_t>(col) * G + g]);
            for (int w = 0; w < 4; ++w) {
                const uint32_t word = wq[(static_cast<size_t>(col) * G + g) * 4 + w];
                for (int t = 0; t < 8; ++t) {
                    const int v = static_cast<int>(word << (28 - 4 * t)) >> 28;
                    acc += static_cast<double>(x[32 * g + 8 * w + t]) * (static_cast<double>(v) * s);
                }
            }
        }
        for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
        if (lane == 0) y[col] = static_cast<float>(acc);
    }
}

template <int SPC, int D>
__global__ __launch_bounds__(kGemvThreads) void q4_gemv_pipe_kernel(const float* x,  // not restrict: see issue_chunk
                                                                   const u32x4* __restrict__ wq,
                                                                   const float* __restrict__ ws,
                                                                   float* __restrict__ y, int N, int K, int reps) {
    constexpr int S = D + 1;           // register slots
    constexpr int kGroups = 64 * SPC;  // groups per lane pass: K <= 32 * kGroups
    static_assert(kGroups * 2 == kGemvThreads, "x is recoded by two threads per group");
    __shared__ __align__(16) uint32_t xds[kGroups * 4 * kXDigits];
    __shared__ float xcs[kGroups];
    const int lane = threadIdx.x & 63;
    const int wave =
        __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x * (kGemvThreads >> 6) + (threadIdx.x >> 6)));
    // Each wavefront streams one contiguous run of columns (a grid-strided
    // assignment, all wavefronts sweeping one band together, measured slower).
    const int cpb = D + S * reps;  // columns per wavefront (<= 64)
    const int col0 = wave * cpb;
    const int G = K >> 5;

    // x first (thread t recodes half t & 1, 16 values, of group t >> 1), then the
    // first D columns, all before any wait.
    const int rg = threadIdx.x >> 1, rh = threadIdx.x & 1;
    f32x4 xr[4];
    {
        const f32x4* src = reinterpret_cast<const f32x4*>(x + static_cast<size_t>(min(rg, G - 1)) * 32 + rh * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) xr[i] = src[i];
    }
    asm volatile("" ::: "memory");
    uint32_t off16[SPC], off4[SPC];
#pragma unroll
    for (int s = 0; s < SPC; ++s) {
        off16[s] = static_cast<uint32_t>(64 * s + lane) * 16u;  // past K: beyond the buffer, reads 0
        off4[s] = static_cast<uint32_t>(64 * s + lane) * 4u;
    }
    PipeSlot<SPC> slot[S];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        pipe_issue<SPC>(slot[d], wq, ws, col0 + d, N, G, off16, off4);
        // slot by slot, as in the steady state, so the loop's load counts line up
        __builtin_amdgcn_sched_barrier(0);
    }
    asm volatile("" ::: "memory");

    {
        float m = 0.0f, fin = 1.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                m = fmaxf(m, fabsf(xr[i][c]));  // maxNum: a NaN is caught by fin
                fin = __builtin_isfinite(xr[i][c]) ? fin : 0.0f;
            }
        m = fmaxf(m, dpp_src<0xB1>(m));  // the partner thread holds the group's other half
        fin = fminf(fin, dpp_src<0xB1>(fin));
        int e = 0;
        (void)frexpf(m, &e);  // m < 2^e (e = 0 for m = 0)
        const bool finite = fin > 0.5f;
        uint32_t r[2][8];
#pragma unroll
        for (int w = 0; w < 2; ++w)
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const float v = xr[(8 * w + t) >> 2][t & 3];
                const int X = finite ? static_cast<int>(rintf(ldexpf(v, kXFracBits - e))) : 0;
                r[w][t] = (static_cast<uint32_t>(X) + kXBias) ^ 0x88888888u;  // Y, each digit xor 8
            }
        // Group rg's 32 digit words as 8 16-byte chunks, chunk c at c ^ xds_swizzle(rg): a
        // wavefront's 128-bit reads (one group per lane, 128 bytes apart) then hit 16 distinct
        // 16-byte bank groups per 16 lanes instead of 2 (measured: 84% of the prologue's LDS cycles
        // were bank conflicts), and the writes 8 instead of 4 per 16 lanes.
        u32x4* xds4 = reinterpret_cast<u32x4*>(xds);
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            transpose_nibbles(r[w]);
#pragma unroll
            for (int h = 0; h < 2; ++h)
                xds4[rg * 8 + ((2 * (2 * rh + w) + h) ^ xds_swizzle(rg))] =
                    u32x4{r[w][4 * h], r[w][4 * h + 1], r[w][4 * h + 2], r[w][4 * h + 3]};
        }
        if (rh == 0)
            xcs[rg] = rg >= G ? 0.0f : (finite ? ldexpf(1.0f, e - kXFracBits) : __builtin_nanf(""));
    }
    __syncthreads();
    XDigits<SPC> xd;
#pragma unroll
    for (int s = 0; s < SPC; ++s) {
        const int gl = 64 * s + lane;
        const u32x4* src = reinterpret_cast<const u32x4*>(xds + gl * 4 * kXDigits);
#pragma unroll
        for (int q = 0; q < kXDigits; ++q) {
            const u32x4 t = src[q ^ xds_swizzle(gl)];
            xd.d[s][4 * q + 0] = t[0];
            xd.d[s][4 * q + 1] = t[1];
            xd.d[s][4 * q + 2] = t[2];
            xd.d[s][4 * q + 3] = t[3];
        }
        xd.c[s] = xcs[gl];
    }
    // The wavefront's lanes cover every group of x, so this test is the same in every
    // wavefront of the grid (uniform): with a non-finite x the integer form has nothing to
    // carry it, and the columns are taken by the IEEE path below instead.
    bool nonfinite = false;
#pragma unroll
    for (int s = 0; s < SPC; ++s) nonfinite = nonfinite || __builtin_isnan(xd.c[s]);
    if (__builtin_amdgcn_ballot_w64(nonfinite) != 0) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the prologue's column loads
        pipe_ieee_columns(x, reinterpret_cast<const uint32_t*>(wq), ws, y, N, G, col0, cpb, lane);
        return;
    }

    // Steady state, S columns per trip: issue column i + D into the free slot, then compute
    // column i (slot i % S). The sched barriers keep each column's arithmetic between its
    // own issue points: interleaved slots would make the wavefront wait for every
    // outstanding load first. (Reducing four columns at once with fewer instructions
    // measured slower: the wavefront then waits out one long dependent chain per four.)
    float result = 0.0f;
    for (int r = 0; r < reps; ++r) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int i = r * S + s;
            pipe_issue<SPC>(slot[(s + D) % S], wq, ws, col0 + i + D, N, G, off16, off4);
            __builtin_amdgcn_sched_barrier(0);
            const float t = wave_reduce_dpp(pipe_partial<SPC>(slot[s], xd));
            result = lane == i ? t : result;
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // The last D columns (slots 0 .. D-1, since reps * S is a multiple of S): no refills.
#pragma unroll
    for (int s = 0; s < D; ++s) {
        const int i = reps * S + s;
        const float t = wave_reduce_dpp(pipe_partial<SPC>(slot[s], xd));
        result = lane == i ? t : result;
    }
    // lane c holds column col0 + c: one coalesced store of the wavefront's run
    if (lane < cpb && col0 + lane < N) y[col0 + lane] = result;
}

template <int M, int SPC, int CPW>
hipError_t launch_rows(const float* x, const uint8_t* w_packed, const float* w_scales, float* y, uint32_t n,
                       uint32_t k, hipStream_t stream) {
    const size_t waves = (static_cast<size_t>(n) + CPW - 1) / CPW;
    const size_t blocks = (waves + kGemvThreads / 64 - 1) / (kGemvThreads / 64);
    const bool single = (k / kGroup) <= static_cast<uint32_t>(64 * SPC);
    // One row reaches this kernel only for K > 4096 (the pipelined kernel takes the rest),
    // so its single-chunk form is never instantiated.
    if constexpr (M > 1) {
        if (single) {
            hipLaunchKernelGGL((q4_gemv_kernel<M, SPC, CPW, true>), dim3(static_cast<unsigned>(blocks)),
                               dim3(kGemvThreads), 0, stream, x, reinterpret_cast<const u32x4*>(w_packed), w_scales, y,
                               static_cast<int>(n), static_cast<int>(k));
            return hipGetLastError();
        }
    }
    if (single) return hipErrorInvalidValue;
    hipLaunchKernelGGL((q4_gemv_kernel<M, SPC, CPW, false>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kGemvThreads), 0, stream, x, reinterpret_cast<const u32x4*>(w_packed), w_scales, y,
                       static_cast<int>(n), static_cast<int>(k));
    return hipGetLastError();
}

}  // namespace

// Single-row decode with K <= 4096: the pipelined kernel with D = 4 columns in flight
// per wavefront. Columns per wavefront: the fewest (cpb = 4 + 5 * reps, at most 64)
// whose workgroups of 4 wavefronts all fit on the CUs at once, so no workgroup waits
// for a second round. At K = 4096, N = 14336 that is 14 columns, 1024 wavefronts:
// 7.48 us per launch, against 7.9-8.1 us for D = 2..5 at 15-19 columns, 8.3 us for
// D = 1 and 9-10 us for all columns in flight at once; a grid 8% over one round
// (276 workgroups) took 11.9 us. 7 columns at D = 3 (two wavefronts per SIMD)
// measured the same within 1%.
static hipError_t launch_gemv_pipelined(const DeviceInfo& dev, const float* x, const uint8_t* w_packed,
                                 const float* w_scales, float* y, uint32_t n, uint32_t k, hipStream_t stream) {
    constexpr int D = 4, S = D + 1, kMaxReps = (64 - D) / S;
    const size_t waves_per_block = kGemvThreads / 64;
    const size_t slots = static_cast<size_t>(dev.cu_count) * waves_per_block;  // wavefronts in one round
    int reps = 0;
    while (reps < kMaxReps && (static_cast<size_t>(n) + D + S * reps - 1) / (D + S * reps) > slots) ++reps;
    const size_t cpb = D + S * reps;
    const size_t waves = (static_cast<size_t>(n) + cpb - 1) / cpb;
    const size_t blocks = (waves + waves_per_block - 1) / waves_per_block;
    hipLaunchKernelGGL((q4_gemv_pipe_kernel<2, D>), dim3(static_cast<unsigned>(blocks)), dim3(kGemvThreads), 0,
                       stream, x, reinterpret_cast<const u32x4*>(w_packed), w_scales, y, static_cast<int>(n),
                       static_cast<int>(k), reps);
    return hipGetLastError();
}

hipError_t launch_gemv(const DeviceInfo& dev, const float* x, const uint8_t* w_packed, const float* w_scales,
                       float* y, uint32_t m, uint32_t n, uint32_t k, hipStream_t stream) {
    switch (m) {
        case 1:
            if (k / kGroup <= 128) return launch_gemv_pipelined(dev, x, w_packed, w_scales, y, n, k, stream);
            return launch_rows<1, 2, 8>(x, w_packed, w_scales, y, n, k, stream);
        case 2: return launch_rows<2, 2, 4>(x, w_packed, w_scales, y, n, k, stream);
        case 3: return launch_rows<3, 1, 4>(x, w_packed, w_scales, y, n, k, stream);
        case 4: return launch_rows<4, 1, 4>(x, w_packed, w_scales, y, n, k, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace spaceslug
