// Decode GEMV: y[m][n] = sum_k x[m][k] * v(k, n) * s(n, k/32) for one row (K <= 32768) or two
// rows (2048 <= K <= 4096).
//
// HBM-bound: one pass over the packed weights and scales. Work mapping:
//   - a wavefront owns a run of consecutive columns; lane l owns the scale groups
//     g = l, l + 64 of each. A column's packed bytes are contiguous
//     (q4gemm.comp:13, byte n*(K/2) + k/2), so for one column the 64 lanes'
//     16-byte loads cover 1 KiB of contiguous memory: every weight load is a
//     fully coalesced 128-bit load, and a lane's 16 bytes are exactly one
//     32-value scale group. The lane's scale s(n, g) is one coalesced 32-bit
//     load (lanes hold consecutive groups of the column), so no LDS broadcast
//     is needed: each scale is read once, by the one lane that applies it;
//   - each group sum is formed exactly in integers (v_dot8_i32_i4 on x recoded
//     as signed hex digits, below) and the group partials are accumulated and
//     summed over the wavefront in double, so no fp32 rounding touches the sum.
// Up to K = 4096 one wavefront takes a whole column (lane l: groups l and l + 64) for one or two
// rows, each weight load serving both; above, K is split over the wavefronts of a workgroup
// (q4_gemv_split_kernel, one row). Every other shape up to 32 rows is the small-batch GEMM's
// (q4_small.hip), which forms its group sums the same exact way on the int8 matrix cores.
#include "q4_device.hpp"
#include "q4_kernels.hpp"

#include <algorithm>

namespace spaceslug {
namespace {

constexpr int kGemvThreads = 256;

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_src(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}

// The same DPP move of a double, one 32-bit half at a time (a row outside ROW_MASK reads 0).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ double dpp_src(double v) {
    const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(v), CTRL, ROW_MASK, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(v), CTRL, ROW_MASK, 0xF, false);
    return __hiloint2double(hi, lo);
}

// Sum over the 64 lanes in double; every lane receives the total (readlane of lane 63).
__device__ __forceinline__ double wave_reduce_dpp(double v) {
    v += dpp_src<0xB1>(v);         // quad_perm [1,0,3,2]: pairs
    v += dpp_src<0x4E>(v);         // quad_perm [2,3,0,1]: quads
    v += dpp_src<0x141>(v);        // row_half_mirror: 8-lane halves
    v += dpp_src<0x140>(v);        // row_mirror: 16-lane rows
    v += dpp_src<0x142, 0xA>(v);   // row_bcast:15 into rows 1 and 3
    v += dpp_src<0x143, 0xC>(v);   // row_bcast:31 into rows 2 and 3 -> row 3 holds the total
    const int lo = __builtin_amdgcn_readlane(__double2loint(v), 63);
    const int hi = __builtin_amdgcn_readlane(__double2hiint(v), 63);
    return __hiloint2double(hi, lo);
}

// Software-pipelined decode of MR rows (MR = 1 or 2, K <= 4096) in integer arithmetic.
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
// |H|, |L| <= 32 * 8 * 34952 < 2^24, so both are exact in int32, and 65536 H + L is
// exact in double. The group partial (65536 H + L) * 2^(e_g - 30) * s(n, g) is
// accumulated in double per lane and the 64 lane partials are summed in double
// (DPP), so the one rounding per group is double's: with fp32 accumulation the
// reference KAT's ranges (x in [-1, 1), scales in [0.5, 1.5)) measured 2.1e-5 at
// K = 1024 on outputs near zero, with double 6e-8 (the fp32 rounding of y itself).
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

// Recodes half rh (16 values, in xr) of group rg of x into its digit words in xds (layout and
// swizzle below) and, for rh == 0, writes the group's factor 2^(e_g - 30) to xcs[rg] (0 for
// rg >= G, NaN when the group holds a non-finite value). The thread holding the other half of
// the group is the partner lane (lane xor 1).
__device__ __forceinline__ void recode_x_half(const f32x4 (&xr)[4], int rg, int rh, int G, uint32_t* xds,
                                              float* xcs) {
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
    if (rh == 0) xcs[rg] = rg >= G ? 0.0f : (finite ? ldexpf(1.0f, e - kXFracBits) : __builtin_nanf(""));
}

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
    double cd[SPC];  // c as double
};

// One column's weights and scales through buffer resources whose base is the
// column (scalar arithmetic only) and whose size is one column: the lane offsets
// are fixed for the whole kernel, and a lane whose group lies past K reads zeros
// (the buffer range check), so it contributes nothing without a per-column select.
// Weights and scales are read exactly once: nontemporal (aux 2) keeps them from
// displacing x and each other in the caches.
// `groups` scale groups of a column from group index `base` (column * G + first group) on; with
// groups == 0 every load is out of range and reads zeros without touching memory.
template <int SPC>
__device__ __forceinline__ void pipe_issue_groups(PipeSlot<SPC>& slot, const u32x4* __restrict__ wq,
                                                  const float* __restrict__ ws, size_t base, int groups,
                                                  const uint32_t (&off16)[SPC], const uint32_t (&off4)[SPC]) {
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<u32x4*>(wq + base), 0, groups * 16, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(ws + base), 0, groups * 4, kBufferFlags);
#pragma unroll
    for (int s = 0; s < SPC; ++s) {
        slot.wv[s] = __builtin_amdgcn_raw_buffer_load_b128(rw, off16[s], 0, kNontemporal);
        slot.sc[s] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, off4[s], 0, kNontemporal));
    }
}

template <int SPC>
__device__ __forceinline__ void pipe_issue(PipeSlot<SPC>& slot, const u32x4* __restrict__ wq,
                                           const float* __restrict__ ws, int col, int N, int G,
                                           const uint32_t (&off16)[SPC], const uint32_t (&off4)[SPC]) {
    pipe_issue_groups<SPC>(slot, wq, ws, static_cast<size_t>(min(col, N - 1)) * G, G, off16, off4);
}

// The lane's share of one column (not yet summed over the wavefront).
template <int SPC>
__device__ __forceinline__ double pipe_partial(const PipeSlot<SPC>& slot, const XDigits<SPC>& xd) {
    double acc = 0.0;
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
        const double p = fma(static_cast<double>(hi), 65536.0, static_cast<double>(lo));
        acc = fma(p, static_cast<double>(slot.sc[s]) * xd.cd[s], acc);
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

template <int SPC, int D, int MR>
__global__ __launch_bounds__(kGemvThreads) void q4_gemv_pipe_kernel(const float* x,  // not restrict: x loads stay ahead of the weights
                                                                   const u32x4* __restrict__ wq,
                                                                   const float* __restrict__ ws,
                                                                   float* __restrict__ y, int N, int K, int reps) {
    constexpr int S = D + 1;                      // register slots
    constexpr int kGroups = 64 * SPC;             // groups per lane pass: K <= 32 * kGroups
    constexpr int kRecoded = kGemvThreads / 2;    // groups recoded (two threads per group)
    static_assert(kGroups <= kRecoded, "x is recoded by two threads per group");
    __shared__ __align__(16) uint32_t xds[MR][kRecoded * 4 * kXDigits];
    __shared__ float xcs[MR][kRecoded];
    const int lane = threadIdx.x & 63;
    const int wave =
        __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x * (kGemvThreads >> 6) + (threadIdx.x >> 6)));
    // Each wavefront streams one contiguous run of columns (a grid-strided
    // assignment, all wavefronts sweeping one band together, measured slower).
    const int cpb = D + S * reps;  // columns per wavefront (<= 64)
    const int col0 = wave * cpb;
    const int G = K >> 5;

    // x first (thread t recodes half t & 1, 16 values, of group t >> 1 of every row), then the
    // first D columns, all before any wait.
    const int rg = threadIdx.x >> 1, rh = threadIdx.x & 1;
    f32x4 xr[MR][4];
#pragma unroll
    for (int r = 0; r < MR; ++r) {
        const f32x4* src =
            reinterpret_cast<const f32x4*>(x + static_cast<size_t>(r) * K + static_cast<size_t>(min(rg, G - 1)) * 32 + rh * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) xr[r][i] = src[i];
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

#pragma unroll
    for (int r = 0; r < MR; ++r) recode_x_half(xr[r], rg, rh, G, xds[r], xcs[r]);
    __syncthreads();
    XDigits<SPC> xd[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int s = 0; s < SPC; ++s) {
            const int gl = 64 * s + lane;
            const u32x4* src = reinterpret_cast<const u32x4*>(xds[r] + gl * 4 * kXDigits);
#pragma unroll
            for (int q = 0; q < kXDigits; ++q) {
                const u32x4 t = src[q ^ xds_swizzle(gl)];
                xd[r].d[s][4 * q + 0] = t[0];
                xd[r].d[s][4 * q + 1] = t[1];
                xd[r].d[s][4 * q + 2] = t[2];
                xd[r].d[s][4 * q + 3] = t[3];
            }
            xd[r].c[s] = xcs[r][gl];
            xd[r].cd[s] = static_cast<double>(xd[r].c[s]);
        }
    // The wavefront's lanes cover every group of x, so this test is the same in every
    // wavefront of the grid (uniform): with a non-finite x the integer form has nothing to
    // carry it, and the columns of every row are taken by the IEEE path below instead.
    bool nonfinite = false;
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int s = 0; s < SPC; ++s) nonfinite = nonfinite || __builtin_isnan(xd[r].c[s]);
    if (__builtin_amdgcn_ballot_w64(nonfinite) != 0) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the prologue's column loads
        for (int r = 0; r < MR; ++r)
            pipe_ieee_columns(x + static_cast<size_t>(r) * K, reinterpret_cast<const uint32_t*>(wq), ws,
                              y + static_cast<size_t>(r) * N, N, G, col0, cpb, lane);
        return;
    }

    // Steady state, S columns per trip: issue column i + D into the free slot, then compute
    // column i (slot i % S) for every row. The sched barriers keep each column's arithmetic
    // between its own issue points: interleaved slots would make the wavefront wait for every
    // outstanding load first. (Reducing four columns at once with fewer instructions
    // measured slower: the wavefront then waits out one long dependent chain per four.)
    float result[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) result[r] = 0.0f;
    for (int rep = 0; rep < reps; ++rep) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int i = rep * S + s;
            pipe_issue<SPC>(slot[(s + D) % S], wq, ws, col0 + i + D, N, G, off16, off4);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int r = 0; r < MR; ++r) {
                const float t = static_cast<float>(wave_reduce_dpp(pipe_partial<SPC>(slot[s], xd[r])));
                result[r] = lane == i ? t : result[r];
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // The last D columns (slots 0 .. D-1, since reps * S is a multiple of S): no refills.
#pragma unroll
    for (int s = 0; s < D; ++s) {
        const int i = reps * S + s;
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            const float t = static_cast<float>(wave_reduce_dpp(pipe_partial<SPC>(slot[s], xd[r])));
            result[r] = lane == i ? t : result[r];
        }
    }
    // lane c holds column col0 + c: one coalesced store of the wavefront's run per row
    if (lane < cpb && col0 + lane < N)
#pragma unroll
        for (int r = 0; r < MR; ++r) y[static_cast<size_t>(r) * N + col0 + lane] = result[r];
}

// Unit i of a column set of the K-split kernel: column col0 + i, groups gb .. gb + gn - 1. A unit
// past the set (i >= cols) or past N loads nothing.
template <int SPC>
__device__ __forceinline__ void pipe_issue_unit(PipeSlot<SPC>& slot, const u32x4* __restrict__ wq,
                                                const float* __restrict__ ws, int i, int cols, int col0, int N,
                                                int G, int gb, int gn, const uint32_t (&off16)[SPC],
                                                const uint32_t (&off4)[SPC]) {
    const int col = col0 + i;
    const bool live = i < cols && col < N;
    pipe_issue_groups<SPC>(slot, wq, ws, static_cast<size_t>(min(col, N - 1)) * G + gb, live ? gn : 0, off16, off4);
}

// Decode of MR rows (one or two) with K > 32 * kGemvPipeMaxGroups: the kernel above with K split
// over the wavefronts of a workgroup. KZ wavefronts share a set of `cols` consecutive columns;
// wavefront z of a set takes groups [z G / KZ, (z + 1) G / KZ) (at most 64 * SPC, lane l holding
// the part's groups l, l + 64, ...) of every column of the set, so its loads of a column are
// still one contiguous run, each serving every row; a workgroup of THREADS / 64 wavefronts holds
// THREADS / (64 KZ) sets. The workgroup recodes all of x into LDS (two threads per group,
// THREADS / 2 groups per pass), each wavefront keeps the digits of its own groups in registers
// and streams the set's columns through the same pipeline, and the KZ wave-summed partials of a
// column are added in double through LDS, in part order (every term exact in double as before;
// one fp32 rounding of y). The pipeline runs D + S * reps units, at least `cols`: a unit past the
// set loads nothing and its arithmetic is skipped (a branch on a wavefront-uniform index).
//
// The recode of x is the same work in every workgroup (at K = 14336, N = 4096 it ends ~3 us after
// a wavefront starts, ~1.4 us of it waiting for x), so more wavefronts per SIMD shorten it: at
// one row, K = 14336, N = 4096, 64 weight copies, four wavefronts per column took 10.7 us per launch in
// workgroups of 256 threads, 9.6 in 512 and 9.6-9.7 in 1024 (D = 2); D = 6 at 256 threads 11.4;
// waiting for x before issuing the first units changed nothing.
template <int SPC, int D, int KZ, int THREADS, int MR>
__global__ __launch_bounds__(THREADS) void q4_gemv_split_kernel(const float* x,  // not restrict, as above
                                                               const u32x4* __restrict__ wq,
                                                               const float* __restrict__ ws,
                                                               float* __restrict__ y, int N, int K, int cols,
                                                               int reps) {
    constexpr int S = D + 1;
    constexpr int kWaves = THREADS >> 6;
    constexpr int kSets = kWaves / KZ;                        // column sets per workgroup
    constexpr int kMaxGroups = 64 * SPC * KZ;                 // G of the largest K (parts of 64 * SPC)
    constexpr int kPass = THREADS / 2;                        // groups recoded per pass
    constexpr int kPasses = (kMaxGroups + kPass - 1) / kPass;  // passes for the largest K
    static_assert(kWaves % KZ == 0 && kMaxGroups % 64 == 0, "whole sets per workgroup");
    __shared__ __align__(16) uint32_t xds[MR][kPasses * kPass * 4 * kXDigits];
    __shared__ float xcs[MR][kPasses * kPass];
    __shared__ double part[kWaves][MR][64];
    const int lane = threadIdx.x & 63;
    const int wb = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int z = wb % KZ;
    const int col0 = (static_cast<int>(blockIdx.x) * kSets + wb / KZ) * cols;
    const int G = K >> 5;
    const int gb = z * G / KZ;
    const int gn = (z + 1) * G / KZ - gb;

    // x first (every row's and pass's loads, groups past G clamped to the last), then the first D
    // units.
    const int rh = threadIdx.x & 1;
    f32x4 xr[MR][kPasses][4];
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int p = 0; p < kPasses; ++p) {
            const int rg = min(p * kPass + static_cast<int>(threadIdx.x >> 1), G - 1);
            const f32x4* src =
                reinterpret_cast<const f32x4*>(x + static_cast<size_t>(r) * K + static_cast<size_t>(rg) * 32 + rh * 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) xr[r][p][i] = src[i];
        }
    asm volatile("" ::: "memory");
    uint32_t off16[SPC], off4[SPC];
#pragma unroll
    for (int s = 0; s < SPC; ++s) {
        off16[s] = static_cast<uint32_t>(64 * s + lane) * 16u;  // past the part: beyond the buffer, reads 0
        off4[s] = static_cast<uint32_t>(64 * s + lane) * 4u;
    }
    PipeSlot<SPC> slot[S];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        pipe_issue_unit<SPC>(slot[d], wq, ws, d, cols, col0, N, G, gb, gn, off16, off4);
        __builtin_amdgcn_sched_barrier(0);
    }
    asm volatile("" ::: "memory");

#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int p = 0; p < kPasses; ++p)
            if (p * kPass < G)
                recode_x_half(xr[r][p], p * kPass + static_cast<int>(threadIdx.x >> 1), rh, G, xds[r], xcs[r]);
    __syncthreads();
    // Every wavefront scans all G group factors of every row, so the test is the same across the
    // workgroup.
    float fsum = 0.0f;  // NaN if any factor is (a sum, so that every read issues before the first test)
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int j = 0; j < kMaxGroups / 64; ++j) fsum += xcs[r][min(64 * j + lane, G - 1)];
    const bool nonfinite = __builtin_isnan(fsum);
    if (__builtin_amdgcn_ballot_w64(nonfinite) != 0) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the prologue's column loads
        if (z == 0)
            for (int r = 0; r < MR; ++r)
                pipe_ieee_columns(x + static_cast<size_t>(r) * K, reinterpret_cast<const uint32_t*>(wq), ws,
                                  y + static_cast<size_t>(r) * N, N, G, col0, cols, lane);
        return;
    }
    // The lane's groups gb + l and gb + 64 + l. Entries past the part (the next part's groups, or
    // past what the passes wrote) meet zero weights (outside the unit's buffer range), and their
    // factor is taken as 0, so they add nothing.
    XDigits<SPC> xd[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int s = 0; s < SPC; ++s) {
            const int gl = gb + 64 * s + lane;
            const u32x4* src = reinterpret_cast<const u32x4*>(xds[r] + gl * 4 * kXDigits);
#pragma unroll
            for (int q = 0; q < kXDigits; ++q) {
                const u32x4 t = src[q ^ xds_swizzle(gl)];
                xd[r].d[s][4 * q + 0] = t[0];
                xd[r].d[s][4 * q + 1] = t[1];
                xd[r].d[s][4 * q + 2] = t[2];
                xd[r].d[s][4 * q + 3] = t[3];
            }
            const float c = xcs[r][gl];
            xd[r].c[s] = 64 * s + lane < gn ? c : 0.0f;
            xd[r].cd[s] = static_cast<double>(xd[r].c[s]);
        }

    double result[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) result[r] = 0.0;
    for (int rep = 0; rep < reps; ++rep) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int i = rep * S + s;
            pipe_issue_unit<SPC>(slot[(s + D) % S], wq, ws, i + D, cols, col0, N, G, gb, gn, off16, off4);
            __builtin_amdgcn_sched_barrier(0);
            if (i < cols) {
#pragma unroll
                for (int r = 0; r < MR; ++r) {
                    const double t = wave_reduce_dpp(pipe_partial<SPC>(slot[s], xd[r]));
                    result[r] = lane == i ? t : result[r];
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int s = 0; s < D; ++s) {
        const int i = reps * S + s;
        if (i < cols) {
#pragma unroll
            for (int r = 0; r < MR; ++r) {
                const double t = wave_reduce_dpp(pipe_partial<SPC>(slot[s], xd[r]));
                result[r] = lane == i ? t : result[r];
            }
        }
    }
    // lane c of each wavefront holds its part of column col0 + c of every row
#pragma unroll
    for (int r = 0; r < MR; ++r) part[wb][r][lane] = result[r];
    __syncthreads();
    if (z == 0 && lane < cols && col0 + lane < N)
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            double t = part[wb][r][lane];
#pragma unroll
            for (int q = 1; q < KZ; ++q) t += part[wb + q][r][lane];
            y[static_cast<size_t>(r) * N + col0 + lane] = static_cast<float>(t);
        }
}

}  // namespace

// Decode of one or two rows with K <= 4096: the pipelined kernel with D = 4 columns in flight
// per wavefront (one lane slot per group up to K = 2048, two above). Columns per wavefront: the fewest (cpb = 4 + 5 * reps, at most 64)
// whose workgroups of 4 wavefronts all fit on the CUs at once, so no workgroup waits
// for a second round. At K = 4096, N = 14336 that is 14 columns, 1024 wavefronts:
// 7.48 us per launch, against 7.9-8.1 us for D = 2..5 at 15-19 columns, 8.3 us for
// D = 1 and 9-10 us for all columns in flight at once; a grid 8% over one round
// (276 workgroups) took 11.9 us. 7 columns at D = 3 (two wavefronts per SIMD)
// measured the same within 1%. Two rows share every weight load and double the arithmetic:
// 2 x 4096 -> 14336 takes 11.5 us against 14.8 for the small-batch GEMM (2 x 2048 -> 4096: 4.5
// against 5.7 us). One lane slot at K <= 2048 keeps half the lanes from computing on zeros:
// 1 x 2048 -> 14336 5.4 us against 6.8.
template <int MR>
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
    if (k / kGroup <= 64u)  // one group per lane: no idle second slot
        hipLaunchKernelGGL((q4_gemv_pipe_kernel<1, D, MR>), dim3(static_cast<unsigned>(blocks)), dim3(kGemvThreads), 0,
                           stream, x, reinterpret_cast<const u32x4*>(w_packed), w_scales, y, static_cast<int>(n),
                           static_cast<int>(k), reps);
    else
        hipLaunchKernelGGL((q4_gemv_pipe_kernel<2, D, MR>), dim3(static_cast<unsigned>(blocks)), dim3(kGemvThreads), 0,
                           stream, x, reinterpret_cast<const u32x4*>(w_packed), w_scales, y, static_cast<int>(n),
                           static_cast<int>(k), reps);
    return hipGetLastError();
}

// Single-row decode with 4096 < K <= 32768: the K-split kernel with KZ = ceil(G / 128) wavefronts
// per column up to K = 16384 and eight above (parts of 64..128 groups), in workgroups of four
// column sets (two for KZ = 2, whose smaller sets would leave the pipeline too short at N = 4096;
// one for KZ = 8): 256, 768, 1024 or 512 threads. Columns per set: the fewest whose workgroups all
// fit on the CUs at once (at most 64).
template <int D, int KZ, int THREADS, int MR = 1, int SPC = 2>
static hipError_t launch_gemv_split(const DeviceInfo& dev, const float* x, const uint8_t* w_packed,
                                    const float* w_scales, float* y, uint32_t n, uint32_t k, hipStream_t stream) {
    constexpr int S = D + 1;
    constexpr size_t kSets = (THREADS / 64) / KZ;
    const size_t slots = static_cast<size_t>(dev.cu_count) * kSets;  // column sets in one round
    const size_t cols = std::min<size_t>(64, std::max<size_t>(1, (n + slots - 1) / slots));
    const int reps = cols > static_cast<size_t>(D) ? static_cast<int>((cols - D + S - 1) / S) : 0;
    const size_t sets = (n + cols - 1) / cols;
    const size_t blocks = (sets + kSets - 1) / kSets;
    hipLaunchKernelGGL((q4_gemv_split_kernel<SPC, D, KZ, THREADS, MR>), dim3(static_cast<unsigned>(blocks)), dim3(THREADS), 0,
                       stream, x, reinterpret_cast<const u32x4*>(w_packed), w_scales, y, static_cast<int>(n),
                       static_cast<int>(k), static_cast<int>(cols), reps);
    return hipGetLastError();
}

hipError_t launch_gemv(const DeviceInfo& dev, const float* x, const uint8_t* w_packed, const float* w_scales,
                       float* y, uint32_t m, uint32_t n, uint32_t k, hipStream_t stream) {
    if (!gemv_takes(m, k)) return hipErrorInvalidValue;
    const uint32_t groups = k / kGroup;
    if (m == 2) {
        if (groups <= static_cast<uint32_t>(kGemvPipeMaxGroups))
            return launch_gemv_pipelined<2>(dev, x, w_packed, w_scales, y, n, k, stream);
        // Two rows' digits of two groups per lane take 128 registers, so the K-split forms run at
        // most two wavefronts per SIMD (up to K = 8192 two, against one in the one-row form:
        // 2 x 8192 -> 14336 20.4 against 22.4 us); between K = 8192 and 12288, where four parts of two
        // lane slots would leave a third of the lanes idle, six parts of one slot (3 per SIMD) instead:
        // 2 x 11008 -> 8192 20.8 against 23.8 us (one slot at K = 8192 or 14336 is slower: 11.3
        // against 10.0 and 17.1 against 15.4 us). Up to K = 4096 the one-wavefront kernel beats the
        // K-split one at two wavefronts per SIMD (2 x 4096 -> 14336: 11.5 against 12.3 us).
        if (groups <= 2u * kGemvPipeMaxGroups)
            return launch_gemv_split<4, 2, 512, 2>(dev, x, w_packed, w_scales, y, n, k, stream);
        if (groups <= 3u * kGemvPipeMaxGroups)
            return launch_gemv_split<3, 6, 768, 2, 1>(dev, x, w_packed, w_scales, y, n, k, stream);
        return launch_gemv_split<3, 4, 512, 2>(dev, x, w_packed, w_scales, y, n, k, stream);
    }
    if (groups <= static_cast<uint32_t>(kGemvPipeMaxGroups))
        return launch_gemv_pipelined<1>(dev, x, w_packed, w_scales, y, n, k, stream);
    if (groups <= 2u * kGemvPipeMaxGroups) return launch_gemv_split<4, 2, 256>(dev, x, w_packed, w_scales, y, n, k, stream);
    if (groups <= 3u * kGemvPipeMaxGroups) return launch_gemv_split<2, 3, 768>(dev, x, w_packed, w_scales, y, n, k, stream);
    if (groups <= 4u * kGemvPipeMaxGroups) return launch_gemv_split<2, 4, 1024>(dev, x, w_packed, w_scales, y, n, k, stream);
    return launch_gemv_split<4, 8, 512>(dev, x, w_packed, w_scales, y, n, k, stream);
}

}  // namespace spaceslug
