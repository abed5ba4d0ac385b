// MFMA int4 GEMM for 5+ rows (prefill, small-batch decode, LoRA projections).
// Three kernels: q4_gemm_wide_kernel for M > 32, q4_gemm_skinny_kernel for
// M <= 32 with K % 128 == 0 and q4_gemm_mfma_kernel (K-split) for the other
// M <= 32 shapes, each described at its definition.
//
// Replaces q4gemm.comp:61-175 (64x64 tile, LDS-staged dequantised B, 4x4 FMA
// micro-tile per thread) with a CDNA4 design on the matrix cores: the two
// small-M kernels on v_mfma_f32_16x16x4_f32, the wide kernel on
// v_mfma_f32_16x16x32_bf16 with x split exactly into three bf16 limbs.
// Common to all three:
//   - per 32-value scale group, lane (j = l%16, q = l/16) feeds the MFMA K slot
//     q with k = 8q .. 8q + 7, so its B operands for column j are the 8 nibbles
//     of ONE 32-bit word of the packed column (word q of the group's 16 bytes)
//     and its A operands are 8 consecutive values of row j. Weights are decoded
//     to v / 16 (v_cvt_off_f32_i4, exact; the factor 16 joins the scale);
//   - every product x * v / 16 is exact in fp32; the MFMA accumulates
//     P = sum x * v / 16 over one group in fp32 from zero, and the group is
//     folded as 16 s * P: straight into a float64 accumulator in the small-M
//     kernels, into an fp32 accumulator that is added into float64 every 8 groups
//     in the wide kernel. Scale application moves out of the inner loop, and the
//     long K sum is carried in double, which keeps the max relative error against
//     the double-precision reference well under 1e-5 at K = 4096;
//   - large grids are XCD-aware: workgroup ids are remapped so each of the 8
//     XCDs (one L2 each) walks a contiguous band of output tiles, sharing A
//     rows and weight columns within its L2;
//   - when the grid is too small to fill 256 CUs, K is split across
//     blockIdx.y and a second kernel sums the partials in a fixed order.
// LoRA: lora_t_kernel computes T = x * la on the MFMA as K-split partials,
// split_reduce_kernel sums them once into T (M x R), and the GEMM epilogue adds
// scale * T[rows] * lb[:, cols] with the same MFMA tile layout (r in the K
// slot) before the single store of y (summing the partials in every tile's
// epilogue instead cost 70 us of 280 at M=512, K=N=4096, r=16).
#include <algorithm>

#include "q4_device.hpp"
#include "q4_kernels.hpp"

namespace spaceslug {
namespace {

template <int WM, int WN, int WAVES_M, int WAVES_N>
struct TileShape {
    static constexpr int kWaves = WAVES_M * WAVES_N;
    static constexpr int kThreads = 64 * kWaves;
    static constexpr int kBM = 16 * WM * WAVES_M;
    static constexpr int kBN = 16 * WN * WAVES_N;
};

// Maps the linear workgroup id to (tile_n, tile_m) so that consecutive ids on
// one XCD (hardware dispatches workgroup i to XCD i % 8) cover a contiguous
// run of tiles, walked M-fastest inside column bands.
__device__ __forceinline__ void xcd_tile(int tiles_m, int tiles_n, int& tm, int& tn) {
    const int total = tiles_m * tiles_n;
    const int id = blockIdx.x;
    int lin = id;
    if (total >= 64 && (total & 7) == 0) {
        const int per_xcd = total >> 3;
        lin = (id & 7) * per_xcd + (id >> 3);
    }
    tm = lin % tiles_m;
    tn = lin / tiles_m;
}

// Operands of one 32-value group for a wavefront's WM x WN tiles.
template <int WM, int WN>
struct GroupOps {
    f32x4 alo[WM], ahi[WM];  // x[row j][8q .. 8q+7] of each M tile
    uint32_t bw[WN];         // packed word q of column j's group, each N tile
    float bs[WN];            // scale of column j's group, each N tile
};

template <int WM, int WN>
__device__ __forceinline__ void load_group(GroupOps<WM, WN>& o, const float* const (&arow)[WM],
                                           const uint32_t* const (&bcol)[WN], const float* const (&scol)[WN], int g) {
#pragma unroll
    for (int tm = 0; tm < WM; ++tm) {
        o.alo[tm] = *reinterpret_cast<const f32x4*>(arow[tm] + g * 32);
        o.ahi[tm] = *reinterpret_cast<const f32x4*>(arow[tm] + g * 32 + 4);
    }
#pragma unroll
    for (int tn = 0; tn < WN; ++tn) {
        o.bw[tn] = bcol[tn][g * 4];
        o.bs[tn] = scol[tn][g];
    }
}

// K-split kernel for the small-M shapes the skinny kernel does not take
// (M <= 32, K % 128 != 0): a wavefront owns a (16*WM) x (16*WN) output block,
// its A operands (two 128-bit loads of row j per group) and weight words go
// global -> VGPR, and PD groups are in flight behind the one being computed.
template <int WM, int WN, int WAVES_M, int WAVES_N, int PD>
// x, wq and ws are deliberately not __restrict__: as provably invariant loads
// the compiler would be free to re-issue the prefetched group's loads at their
// use (to save registers), which serialises them behind the compute.
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void q4_gemm_mfma_kernel(
    const float* x, const uint32_t* wq, const float* ws, float* __restrict__ out, int M, int N, int K, int tiles_m,
    int tiles_n, int groups_per_split, const float* __restrict__ tmat, const float* __restrict__ lb, int R,
    float lscale) {
    using Shape = TileShape<WM, WN, WAVES_M, WAVES_N>;
    const int lane = threadIdx.x & 63;
    const int wid = threadIdx.x >> 6;
    const int wm = wid % WAVES_M;
    const int wn = wid / WAVES_M;
    const int j = lane & 15;
    const int q = lane >> 4;
    const int G = K >> 5;

    int tile_m, tile_n;
    xcd_tile(tiles_m, tiles_n, tile_m, tile_n);
    const int m0 = tile_m * Shape::kBM + wm * 16 * WM;
    const int n0 = tile_n * Shape::kBN + wn * 16 * WN;
    const int g_begin = blockIdx.y * groups_per_split;
    const int g_end = min(G, g_begin + groups_per_split);

    const float* arow[WM];
#pragma unroll
    for (int tm = 0; tm < WM; ++tm) {
        const int row = min(m0 + 16 * tm + j, M - 1);
        arow[tm] = x + static_cast<size_t>(row) * K + 8 * q;
    }
    const uint32_t* bcol[WN];
    const float* scol[WN];
#pragma unroll
    for (int tn = 0; tn < WN; ++tn) {
        const int col = min(n0 + 16 * tn + j, N - 1);
        bcol[tn] = wq + static_cast<size_t>(col) * (K >> 3) + q;
        scol[tn] = ws + static_cast<size_t>(col) * G;
    }

    double acc[WM][WN][4];
#pragma unroll
    for (int tm = 0; tm < WM; ++tm)
#pragma unroll
        for (int tn = 0; tn < WN; ++tn)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[tm][tn][i] = 0.0;

    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    // One group: P = x * v over 32 K values on the MFMA from zero, then acc += s * P.
    auto do_group = [&](const GroupOps<WM, WN>& o) {
        f32x4 P[WM][WN];
        float bv[WN][8];
#pragma unroll
        for (int tn = 0; tn < WN; ++tn) nibbles_signed_16th_mfma(o.bw[tn], bv[tn]);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
#pragma unroll
            for (int tm = 0; tm < WM; ++tm) {
                const float av = t < 4 ? o.alo[tm][t & 3] : o.ahi[tm][t & 3];
#pragma unroll
                for (int tn = 0; tn < WN; ++tn)
                    P[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv[tn][t], t == 0 ? zero : P[tm][tn], 0, 0, 0);
            }
        }
#pragma unroll
        for (int tn = 0; tn < WN; ++tn) {
            const double sc = static_cast<double>(o.bs[tn]) * kSixteenthsUnit;
#pragma unroll
            for (int tm = 0; tm < WM; ++tm)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[tm][tn][i] = fma(sc, static_cast<double>(P[tm][tn][i]), acc[tm][tn][i]);
        }
    };
    if (g_begin < g_end) {
        // PD + 1 buffers used in rotation: while buffer s computes group g+s,
        // buffer (s+PD) % (PD+1) receives group g+s+PD, so PD groups are in flight
        // behind the one being computed. The rotation is unrolled, so no buffer
        // is copied (a register copy would wait for its loads). Loads past the
        // split are clamped to its last group and never accumulated.
        constexpr int NB = PD + 1;
        GroupOps<WM, WN> buf[NB];
#pragma unroll
        for (int p = 0; p < PD; ++p) {
            load_group<WM, WN>(buf[p], arow, bcol, scol, min(g_begin + p, g_end - 1));
            __builtin_amdgcn_sched_barrier(0);
        }
        for (int g = g_begin; g < g_end; g += NB) {
#pragma unroll
            for (int sl = 0; sl < NB; ++sl) {
                load_group<WM, WN>(buf[(sl + PD) % NB], arow, bcol, scol, min(g + sl + PD, g_end - 1));
                __builtin_amdgcn_sched_barrier(0);
                if (g + sl < g_end) do_group(buf[sl]);  // uniform across the workgroup
                // keep the next slot's loads and work below this point so each slot
                // waits only for its own loads
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

    if (lb != nullptr && blockIdx.y == 0) {
        // LoRA epilogue: + lscale * T[m0.., :R] * lb[:R, n0..] on the MFMA, r in the K slot
        // (T = x * la, M x R, summed by lora_t_reduce_kernel).
#pragma unroll
        for (int tm = 0; tm < WM; ++tm) {
            const int row = min(m0 + 16 * tm + j, M - 1);
#pragma unroll
            for (int tn = 0; tn < WN; ++tn) {
                const int col = min(n0 + 16 * tn + j, N - 1);
                f32x4 P = zero;
                for (int r0 = 0; r0 < R; r0 += 4) {
                    const int r = r0 + q;
                    const float av = r < R ? tmat[static_cast<size_t>(row) * R + r] : 0.0f;
                    const float bv = r < R ? lb[static_cast<size_t>(r) * N + col] : 0.0f;
                    P = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, P, 0, 0, 0);
                }
                const double s = static_cast<double>(lscale);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[tm][tn][i] = fma(s, static_cast<double>(P[i]), acc[tm][tn][i]);
            }
        }
    }

    float* dst = out + static_cast<size_t>(blockIdx.y) * M * N;
#pragma unroll
    for (int tm = 0; tm < WM; ++tm) {
#pragma unroll
        for (int tn = 0; tn < WN; ++tn) {
            const int col = n0 + 16 * tn + j;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = m0 + 16 * tm + 4 * q + i;
                if (row < M && col < N) dst[static_cast<size_t>(row) * N + col] = static_cast<float>(acc[tm][tn][i]);
            }
        }
    }
}

// Limbs per x value on the bf16 MFMA path.
constexpr int kLimbs = 3;

// x (fp32, M x K) -> x limbs (bf16, [M][KB][3][64] with KB = ceil(K / 64), rows
// zero-padded to KB * 64 values) for q4_gemm_wide_kernel. Each value is split by
// split_bf16_limbs (b0 + b1 + b2 == x for |x| >= 2^-110, within 2^-133 below), and a
// product of a limb with a bf16 weight v/16 is exact in fp32.
// One thread per 8 consecutive values of a row: two 16-byte loads, three
// 16-byte stores (one per limb), coalesced along the row.
__global__ __launch_bounds__(256) void split_x_kernel(const float* __restrict__ x, uint16_t* __restrict__ xs,
                                                      int M, int K, int KB) {
    const size_t idx = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    const size_t per_row = static_cast<size_t>(KB) * 8;
    if (idx >= static_cast<size_t>(M) * per_row) return;
    const int row = static_cast<int>(idx / per_row);
    const int c8 = static_cast<int>(idx % per_row);
    const int kb = c8 >> 3, c = c8 & 7;
    const int k0 = kb * 64 + c * 8;
    float v[8];
    if (k0 < K) {  // K % 32 == 0, so the 8 values are all inside the row or all past it
        const f32x4 lo = *reinterpret_cast<const f32x4*>(x + static_cast<size_t>(row) * K + k0);
        const f32x4 hi = *reinterpret_cast<const f32x4*>(x + static_cast<size_t>(row) * K + k0 + 4);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            v[t] = lo[t];
            v[t + 4] = hi[t];
        }
    } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) v[t] = 0.0f;
    }
    u32x4 limb[kLimbs];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        uint32_t lo[kLimbs], hi[kLimbs];
        split_bf16_limbs(v[2 * t], lo);
        split_bf16_limbs(v[2 * t + 1], hi);
#pragma unroll
        for (int li = 0; li < kLimbs; ++li) limb[li][t] = lo[li] | (hi[li] << 16);
    }
    uint16_t* dst = xs + (static_cast<size_t>(row) * KB + kb) * (kLimbs * 64) + c * 8;
#pragma unroll
    for (int li = 0; li < kLimbs; ++li) *reinterpret_cast<u32x4*>(dst + li * 64) = limb[li];
}

// Wide tile for M > 32 (prefill, LoRA projections): 128 x 128 outputs per
// workgroup, 2 x 2 wavefronts of 64 x 64 (4 x 4 MFMA tiles each), one wavefront
// per SIMD. The matrix instruction is v_mfma_f32_16x16x32_bf16, fed with x as
// three exact bf16 limbs (split_x_kernel) and the weights as bf16 v/16 (exact):
// every product is exact in fp32, each 32-value group's sum P = sum x * v/16 is
// accumulated in fp32 by three chained MFMAs (smallest limb first). The group is
// folded into an fp32 accumulator as acc32 += 16 s * P, and every 4 stages (8
// groups) acc32 is added into the float64 accumulator: one fp32 FMA per output and
// group instead of a convert and a float64 FMA, and 64 fewer live registers
// between flushes. Against the per-group float64 fold: 1.24 against 1.34 ms at
// M=2048, K=4096, N=14336 (same box); the measured max relative error stays
// under 1e-5 (an emulation of this order at 2.9e7 outputs: 4.1-4.8e-6 against
// 3.8-4.0e-6 for the per-group fold). One such MFMA (16 x 16 x 32) does the work of eight
// fp32 16x16x4 MFMAs at a sixteenth of their matrix-core cycles each, so three
// of them cost under a fifth of the fp32 form.
// Lane (j = l%16, q = l/16) of a 16x16x32 MFMA holds A[row j][k = 8q .. 8q+7] and
// B[k = 8q .. 8q+7][column j] (8 bf16 each), and result rows 4q .. 4q+3 of column
// j. Per stage of two groups (64 values of K) the workgroup fills one of two LDS
// buffers (64 KiB each):
//   - the x-limb tile (3 limbs x 128 rows x 64 values, 48 KiB), copied global ->
//     LDS by global_load_lds_dwordx4 (no VGPRs): per limb 16 copies of 8 full
//     128-byte rows, four rows' blocks per wavefront with the three limbs at
//     fixed offsets. Row chunks are XOR-swizzled so that the 16 rows a pass of
//     MFMA-operand reads touches fall on 16 distinct bank groups;
//   - the dequantised B tile (2 groups x 128 columns x 32 values as bf16 v/16,
//     16 KiB): each thread loads one group's 16 packed bytes of one column,
//     decodes them once for the whole workgroup and writes them in the MFMA B
//     layout, so every wavefront reads its B operands as linear 1 KiB runs.
// Stage s+1 is copied while stage s computes; one barrier per stage. An odd
// number of groups leaves the last stage's second group empty: its x limbs are
// zero padding, its weight loads are clamped into the column, and its MFMAs and
// fold are skipped (a wavefront-uniform branch). Against the same tile on
// v_mfma_f32_16x16x4_f32 with x staged as fp32 (the previous product kernel):
// 1.34 against 2.28-2.32 ms at M=2048, K=4096, N=14336 and 111 against 179 us at
// M=512, K=N=4096, same box, both with the per-group float64 fold.
struct WideLdsStage {
    // Limb li, 8-row copy block, lane slot: row r's 16-byte chunk c (k = 64 kb + 8 c .. +7)
    // at u32x4 index (r >> 1) * 16 + 8 * (r & 1) + (c ^ ((r >> 1) & 7)) of a[li].
    u32x4 a[kLimbs][16][64];
    // Group h of the stage, 16-column tile, lane (j, q): bf16 v/16 of k = 32 (2 kb + h) + 8 q .. +7
    // of tile column 16 * tile + j.
    u32x4 b[2][8][64];
};

__global__ __launch_bounds__(256) void q4_gemm_wide_kernel(const uint16_t* xs, const uint32_t* wq, const float* ws,
                                                          float* __restrict__ out, int M, int N, int K,
                                                          int tiles_m, int tiles_n, int stages_per_split,
                                                          const float* __restrict__ tmat,
                                                          const float* __restrict__ lb, int R, float lscale) {
    constexpr int WM = 4, WN = 4;
    __shared__ WideLdsStage stage[2];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wid & 1;
    const int wn = wid >> 1;
    const int j = lane & 15;
    const int q = lane >> 4;
    const int G = K >> 5;
    const int KB = (G + 1) >> 1;

    int tile_m, tile_n;
    xcd_tile(tiles_m, tiles_n, tile_m, tile_n);
    const int mt0 = tile_m * 128, nt0 = tile_n * 128;
    const int m0 = mt0 + wm * 64;
    const int n0 = nt0 + wn * 64;
    const int kb_begin = blockIdx.y * stages_per_split;
    const int kb_end = min(KB, kb_begin + stages_per_split);

    // x-limb copies of this wavefront: 8-row blocks 4 wid .. 4 wid + 3, three limbs each.
    const uint16_t* asrc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int blk = 4 * wid + i;
        const int pair = 4 * blk + (lane >> 4);  // row pair of this lane's 16 bytes
        const int row_t = 2 * pair + ((lane >> 3) & 1);
        const int c = (lane & 7) ^ (pair & 7);
        asrc[i] = xs + static_cast<size_t>(min(mt0 + row_t, M - 1)) * KB * (kLimbs * 64) + 8 * c;
    }
    // B: thread -> tile column bc, group bh of the stage (16 bytes = 4 packed words).
    const int bc = tid & 127, bh = tid >> 7;
    const u32x4* bsrc = reinterpret_cast<const u32x4*>(wq + static_cast<size_t>(min(nt0 + bc, N - 1)) * (K >> 3));
    // Scales of the lane's four MFMA columns, for the fold.
    const float* scol[WN];
#pragma unroll
    for (int tn = 0; tn < WN; ++tn) scol[tn] = ws + static_cast<size_t>(min(n0 + 16 * tn + j, N - 1)) * G;

    double acc[WM][WN][4];
    float acc32[WM][WN][4];
#pragma unroll
    for (int tm = 0; tm < WM; ++tm)
#pragma unroll
        for (int tn = 0; tn < WN; ++tn)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                acc[tm][tn][i] = 0.0;
                acc32[tm][tn][i] = 0.0f;
            }
    auto flush = [&]() {
#pragma unroll
        for (int tm = 0; tm < WM; ++tm)
#pragma unroll
            for (int tn = 0; tn < WN; ++tn)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    acc[tm][tn][i] += static_cast<double>(acc32[tm][tn][i]);
                    acc32[tm][tn][i] = 0.0f;
                }
    };

    auto issue_a = [&](int kb, int st) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int li = 0; li < kLimbs; ++li)  // 1 KiB = 8 rows of one limb
                __builtin_amdgcn_global_load_lds(asrc[i] + static_cast<size_t>(kb) * (kLimbs * 64) + li * 64,
                                                 &stage[st].a[li][4 * wid + i][0], 16, 0, 0);
    };
    auto load_b = [&](int kb) { return bsrc[min(2 * kb + bh, G - 1)]; };
    auto write_b = [&](u32x4 pk, int st) {
#pragma unroll
        for (int w = 0; w < 4; ++w) stage[st].b[bh][bc >> 4][(bc & 15) + 16 * w] = nibbles_bf16_16th(pk[w]);
    };
    auto load_s = [&](int kb, float (&s)[2][WN]) {
#pragma unroll
        for (int tn = 0; tn < WN; ++tn) {
            s[0][tn] = scol[tn][2 * kb];
            s[1][tn] = scol[tn][min(2 * kb + 1, G - 1)];
        }
    };

    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    auto fold = [&](const f32x4 (&P)[WM][WN], const float (&bsv)[WN]) {
#pragma unroll
        for (int tn = 0; tn < WN; ++tn) {
            const float sc = bsv[tn] * kSixteenthsUnit;
#pragma unroll
            for (int tm = 0; tm < WM; ++tm)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc32[tm][tn][i] = fmaf(sc, P[tm][tn][i], acc32[tm][tn][i]);
        }
    };
    auto mfma_group = [&](f32x4 (&P)[WM][WN], int st, int h) {
        bf16x8 bv[WN];
#pragma unroll
        for (int tn = 0; tn < WN; ++tn) bv[tn] = __builtin_bit_cast(bf16x8, stage[st].b[h][wn * 4 + tn][lane]);
#pragma unroll
        for (int tm = 0; tm < WM; ++tm) {
            const int row_t = wm * 64 + 16 * tm + j;
            const int p = row_t >> 1;
            const int idx = p * 16 + 8 * (row_t & 1) + ((4 * h + q) ^ (p & 7));
            bf16x8 av[kLimbs];
#pragma unroll
            for (int li = 0; li < kLimbs; ++li) av[li] = __builtin_bit_cast(bf16x8, (&stage[st].a[li][0][0])[idx]);
#pragma unroll
            for (int tn = 0; tn < WN; ++tn) {
                f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[2], bv[tn], zero, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[1], bv[tn], t, 0, 0, 0);
                P[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[0], bv[tn], t, 0, 0, 0);
            }
        }
    };
    if (kb_begin < kb_end) {
        float bs_cur[2][WN];
        f32x4 P[WM][WN];
        issue_a(kb_begin, 0);
        {
            const u32x4 pk = load_b(kb_begin);
            load_s(kb_begin, bs_cur);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            write_b(pk, 0);
        }
        __syncthreads();
        for (int kb = kb_begin; kb < kb_end; ++kb) {
            const int st = (kb - kb_begin) & 1;
            // The last stage copies its own stage again (in bounds, never read): no branch.
            const int kbn = min(kb + 1, kb_end - 1);
            issue_a(kbn, st ^ 1);
            const u32x4 pkn = load_b(kbn);
            float bsn[2][WN];
            load_s(kbn, bsn);
            const bool second = 2 * kb + 1 < G;
            mfma_group(P, st, 0);
            fold(P, bs_cur[0]);
            if (second) mfma_group(P, st, 1);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            write_b(pkn, st ^ 1);
            __syncthreads();
            if (second) fold(P, bs_cur[1]);  // P is in registers: the fold needs no LDS
            if (((kb - kb_begin) & 3) == 3) flush();
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int tn = 0; tn < WN; ++tn) bs_cur[h][tn] = bsn[h][tn];
        }
        flush();
    }

    if (lb != nullptr && blockIdx.y == 0) {
#pragma unroll
        for (int tm = 0; tm < WM; ++tm) {
            const int row = min(m0 + 16 * tm + j, M - 1);
#pragma unroll
            for (int tn = 0; tn < WN; ++tn) {
                const int col = min(n0 + 16 * tn + j, N - 1);
                f32x4 P = zero;
                for (int r0 = 0; r0 < R; r0 += 4) {
                    const int r = r0 + q;
                    const float av = r < R ? tmat[static_cast<size_t>(row) * R + r] : 0.0f;
                    const float bv = r < R ? lb[static_cast<size_t>(r) * N + col] : 0.0f;
                    P = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, P, 0, 0, 0);
                }
                const double s = static_cast<double>(lscale);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[tm][tn][i] = fma(s, static_cast<double>(P[i]), acc[tm][tn][i]);
            }
        }
    }

    float* dst = out + static_cast<size_t>(blockIdx.y) * M * N;
#pragma unroll
    for (int tm = 0; tm < WM; ++tm) {
#pragma unroll
        for (int tn = 0; tn < WN; ++tn) {
            const int col = n0 + 16 * tn + j;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = m0 + 16 * tm + 4 * q + i;
                if (row < M && col < N) dst[static_cast<size_t>(row) * N + col] = static_cast<float>(acc[tm][tn][i]);
            }
        }
    }
}

// LoRA pre-pass on the MFMA: tpart[s][m][r] = sum over the groups of split s of
// x[m][k] * la[k][r] (la is K x R row-major). One wavefront per 16 x 16 tile of
// (rows, ranks) and split; all of the split's operands are loaded before the
// first MFMA. Grid (ceil(M/16), ceil(R/16), t_splits).
constexpr int kLoraGroupsPerWave = 8;

__global__ __launch_bounds__(64) void lora_t_kernel(const float* __restrict__ x, const float* __restrict__ la,
                                                    float* __restrict__ tpart, int M, int K, int R) {
    const int lane = threadIdx.x & 63;
    const int j = lane & 15;
    const int q = lane >> 4;
    const int G = K >> 5;
    const int m0 = blockIdx.x * 16;
    const int r0 = blockIdx.y * 16;
    const int g_begin = blockIdx.z * kLoraGroupsPerWave;
    const int row = min(m0 + j, M - 1);
    const int r = r0 + j;
    const int rc = min(r, R - 1);
    const float* xr = x + static_cast<size_t>(row) * K + 8 * q;

    f32x4 a_lo[kLoraGroupsPerWave], a_hi[kLoraGroupsPerWave];
    float b[kLoraGroupsPerWave][8];
#pragma unroll
    for (int i = 0; i < kLoraGroupsPerWave; ++i) {
        const int g = min(g_begin + i, G - 1);
        a_lo[i] = *reinterpret_cast<const f32x4*>(xr + g * 32);
        a_hi[i] = *reinterpret_cast<const f32x4*>(xr + g * 32 + 4);
        const float* lr = la + static_cast<size_t>(g * 32 + 8 * q) * R + rc;
#pragma unroll
        for (int t = 0; t < 8; ++t) b[i][t] = lr[static_cast<size_t>(t) * R];
    }
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < kLoraGroupsPerWave; ++i) {
        if (g_begin + i < G) {  // uniform
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const float av = t < 4 ? a_lo[i][t & 3] : a_hi[i][t & 3];
                const float bv = r < R ? b[i][t] : 0.0f;
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc, 0, 0, 0);
            }
        }
    }
    float* dst = tpart + static_cast<size_t>(blockIdx.z) * M * R;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int rr = m0 + 4 * q + i;
        if (rr < M && r < R) dst[static_cast<size_t>(rr) * R + r] = acc[i];
    }
}

// Small-M GEMM (M <= 32, K % 128 == 0) with no K-split partials in memory: a
// workgroup owns one 16 x 16 output tile and its KW wavefronts split K between
// them; their float64 accumulators are summed through LDS in wavefront order
// (deterministic), and the LoRA term, if any, is added in double before the
// single store. Per wavefront, weights and scales move in units of 4 groups (a
// "quad"): lane (j, q) loads column j's 16 bytes of group 4*quad + q (one
// 128-bit load; the 4 lanes of a column read 64 contiguous bytes) and its
// scale, then a 4 x 4 transpose across the 16-lane rows (v_permlane*_swap)
// gives every lane word q of each of the 4 groups, the MFMA B layout. Two quads
// are in flight while one computes (statically named buffers E and O); the
// pipeline issues no load past the wavefront's last quad. KW is 16 when the
// tile grid has no more workgroups than the chip has CUs (16 wavefronts per CU
// from one tile), else 8. Above 8 rows x reaches the MFMA through LDS (below).
// Measured at M=16, K=N=4096: 10.9 us per call with x staged (12.5 us with x
// loaded directly, 14.2 us with 8 wavefronts), against 20.5 us for the split-K
// kernel plus its reduction.
constexpr int kSkinnyWavesFew = 16;
constexpr int kSkinnyWavesMany = 8;
// Rows up to which x goes global -> VGPR directly; taller tiles copy it through LDS.
constexpr int kSkinnyDirectMaxRows = 8;

// Per-quad operands of one wavefront: x for the quad's 4 groups (in registers
// straight from global memory, or copied through LDS first, below) and the
// weights and scales of its column.
struct QuadW {
    u32x4 bw;  // column j, group 4 * quad + q: its 16 packed bytes
    float bs;  // scale of column j, group 4 * quad + q
};

__device__ __forceinline__ void load_quad_w(QuadW& o, const u32x4* bq, const float* sq, int qi) {
    o.bw = __builtin_nontemporal_load(bq + 4 * qi);
    o.bs = __builtin_nontemporal_load(sq + 4 * qi);
}

// x[row j][32 g + 8 q .. +7] for the quad's 4 groups: two 128-bit loads per group, each
// instruction touching half of 16 rows' 128-byte lines.
__device__ __forceinline__ void load_quad_x(f32x4 (&alo)[4], f32x4 (&ahi)[4], const float* arow, int qi) {
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
        alo[gi] = *reinterpret_cast<const f32x4*>(arow + (4 * qi + gi) * 32);
        ahi[gi] = *reinterpret_cast<const f32x4*>(arow + (4 * qi + gi) * 32 + 4);
    }
}

__device__ __forceinline__ void mma_quad(const QuadW& o, const f32x4 (&alo)[4], const f32x4 (&ahi)[4],
                                         double (&acc)[4]) {
    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    const u32x4 bw = transpose_rows(o.bw);  // word q of each of the quad's groups
    const f32x4 bs = gather_rows(o.bs);     // the quad's 4 scales of column j
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
        float bv[8];
        nibbles_signed_16th_mfma(bw[gi], bv);
        f32x4 P;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float av = t < 4 ? alo[gi][t & 3] : ahi[gi][t & 3];
            P = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv[t], t == 0 ? zero : P, 0, 0, 0);
        }
        const double sc = static_cast<double>(bs[gi]) * kSixteenthsUnit;
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] = fma(sc, static_cast<double>(P[r]), acc[r]);
    }
}

// With kStageX, each wavefront copies its quad of x (16 rows x 128 floats, 8 KiB)
// global -> LDS by global_load_lds_dwordx4, two full 512-byte row runs per
// instruction, and reads its MFMA operands from there: the register-direct loads
// above touch twice the cache lines for the same bytes, which at 16 rows (x read
// whole by every CU) cost 13% of the kernel (M=16, K=N=4096: 12.5 -> 10.9 us).
// Row j's 16-byte chunk c (k = 4 c .. 4 c + 3 of the quad) sits at chunk c ^ j of
// the row, so a pass of 16 lanes reading one chunk of each row hits 16 distinct
// bank groups. The next quad's copy starts once this quad's operands are in
// registers. At M <= 8 the copy moves rows the tile does not use and the direct
// loads are faster (M=5: 9.9 against 10.7 us).
constexpr int kQuadXFloats = 16 * 128;

template <int KW, bool kStageX>
// x, wq and ws are not __restrict__ for the reason given at q4_gemm_mfma_kernel.
__global__ __launch_bounds__(64 * KW) void q4_gemm_skinny_kernel(const float* x, const uint32_t* wq, const float* ws,
                                                                float* __restrict__ y, int M, int N, int K,
                                                                int tiles_m, const float* __restrict__ tmat,
                                                                const float* __restrict__ lb, int R, float lscale) {
    // Per wavefront: its x unit (staged form), then 256 partial sums in double.
    constexpr int kRegionFloats = kStageX ? kQuadXFloats : 512;
    __shared__ f32x4 smem[KW * kRegionFloats / 4];
    const int lane = threadIdx.x & 63;
    const int wk = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int j = lane & 15;
    const int q = lane >> 4;
    const int G = K >> 5;
    const int Q = G >> 2;
    const int m0 = (blockIdx.x % tiles_m) * 16;
    const int n0 = (blockIdx.x / tiles_m) * 16;
    const int qpw = (Q + KW - 1) / KW;
    const int qb = wk * qpw;
    const int qe = min(Q, qb + qpw);
    const int col = min(n0 + j, N - 1);
    const u32x4* bq = reinterpret_cast<const u32x4*>(wq + static_cast<size_t>(col) * (K >> 3)) + q;
    const float* sq = ws + static_cast<size_t>(col) * G + q;
    const float* arow = x + static_cast<size_t>(min(m0 + j, M - 1)) * K + 8 * q;
    float* xs = reinterpret_cast<float*>(smem) + wk * kRegionFloats;

    // Staged copy: instruction i moves rows 2i and 2i+1; lane l fetches the chunk that
    // lands at position l & 31 of row 2i + (l >> 5).
    const float* xsrc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int r = 2 * i + (lane >> 5);
        xsrc[i] = x + static_cast<size_t>(min(m0 + r, M - 1)) * K + 4 * ((lane & 31) ^ r);
    }
    auto issue_x = [&](int qi) {
#pragma unroll
        for (int i = 0; i < 8; ++i) __builtin_amdgcn_global_load_lds(xsrc[i] + qi * 128, xs + i * 256, 16, 0, 0);
    };
    auto stage_start = [&](int qi) {
        if constexpr (kStageX) issue_x(qi);
    };
    // One quad: its x operands (staged: wait for the copy, read LDS, start the next copy
    // into the same bytes), then the MFMAs.
    auto step = [&](const QuadW& w, int qi, double (&acc)[4]) {
        f32x4 alo[4], ahi[4];
        if constexpr (kStageX) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
            for (int gi = 0; gi < 4; ++gi) {
                alo[gi] = *reinterpret_cast<const f32x4*>(xs + j * 128 + (((8 * gi + 2 * q) ^ j) << 2));
                ahi[gi] = *reinterpret_cast<const f32x4*>(xs + j * 128 + (((8 * gi + 2 * q + 1) ^ j) << 2));
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (qi + 1 < qe) issue_x(qi + 1);  // uniform
        } else {
            load_quad_x(alo, ahi, arow, qi);
        }
        mma_quad(w, alo, ahi, acc);
    };

    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    if (qb < qe) {  // every condition below is uniform per wavefront
        QuadW E, O;
        stage_start(qb);
        load_quad_w(E, bq, sq, qb);
        if (qb + 1 < qe) load_quad_w(O, bq, sq, qb + 1);
        for (int qi = qb; qi < qe; qi += 2) {
            step(E, qi, acc);
            if (qi + 2 < qe) load_quad_w(E, bq, sq, qi + 2);
            if (qi + 1 < qe) {
                step(O, qi + 1, acc);
                if (qi + 3 < qe) load_quad_w(O, bq, sq, qi + 3);
            }
        }
    }

    // Partial sums through the wavefront's own LDS region (no copy is in flight any
    // more), summed in wavefront order.
    double* red = reinterpret_cast<double*>(smem);
    constexpr int kRedStride = kRegionFloats / 2;  // doubles per wavefront region
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wk * kRedStride + (4 * q + r) * 16 + j] = acc[r];
    __syncthreads();
    for (int e = threadIdx.x; e < 256; e += 64 * KW) {
        const int rr = m0 + (e >> 4);
        const int cc = n0 + (e & 15);
        if (rr >= M || cc >= N) continue;
        double s = 0.0;
#pragma unroll
        for (int w = 0; w < KW; ++w) s += red[w * kRedStride + e];
        if (lb != nullptr) {
            double t = 0.0;
            for (int r = 0; r < R; ++r)
                t = fma(static_cast<double>(tmat[static_cast<size_t>(rr) * R + r]),
                        static_cast<double>(lb[static_cast<size_t>(r) * N + cc]), t);
            s = fma(static_cast<double>(lscale), t, s);
        }
        y[static_cast<size_t>(rr) * N + cc] = static_cast<float>(s);
    }
}

// y[i] = sum_s part[s][i], in ascending s, accumulated in double (K-split
// partials of the GEMM, and of the LoRA pre-pass T = x * la).
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* __restrict__ part,
                                                           float* __restrict__ y, size_t count,
                                                           int splits) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride) {
        double s = 0.0;
        int z = 0;
        // eight loads in flight per thread, summed in ascending z
        for (; z + 8 <= splits; z += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = part[static_cast<size_t>(z + u) * count + i];
#pragma unroll
            for (int u = 0; u < 8; ++u) s += static_cast<double>(v[u]);
        }
        for (; z < splits; ++z) s += static_cast<double>(part[static_cast<size_t>(z) * count + i]);
        y[i] = static_cast<float>(s);
    }
}

template <int WM, int WN, int WAVES_M, int WAVES_N, int PD>
hipError_t launch_mfma(const float* x, const uint8_t* w_packed, const float* w_scales, float* out,
                       uint32_t m, uint32_t n, uint32_t k, int splits, const float* tmat, const float* lb,
                       uint32_t rank, float lscale, hipStream_t stream) {
    using Shape = TileShape<WM, WN, WAVES_M, WAVES_N>;
    const int tiles_m = static_cast<int>((m + Shape::kBM - 1) / Shape::kBM);
    const int tiles_n = static_cast<int>((n + Shape::kBN - 1) / Shape::kBN);
    const int G = static_cast<int>(k / kGroup);
    const int gps = (G + splits - 1) / splits;
    hipLaunchKernelGGL((q4_gemm_mfma_kernel<WM, WN, WAVES_M, WAVES_N, PD>),
                       dim3(tiles_m * tiles_n, splits), dim3(Shape::kThreads), 0, stream, x,
                       reinterpret_cast<const uint32_t*>(w_packed), w_scales, out,
                       static_cast<int>(m), static_cast<int>(n), static_cast<int>(k), tiles_m,
                       tiles_n, gps, tmat, lb, static_cast<int>(rank), lscale);
    return hipGetLastError();
}

// Tile shape of q4_gemm_mfma_kernel (M <= 32 with K not a multiple of 128): one
// 16-row MFMA tile x 256 columns per workgroup (4 waves of 16 x 64), 2 groups in
// flight.
using SkinnyShape = TileShape<1, 4, 1, 4>;
constexpr int kSkinnyPD = 2;
// Wide tile of q4_gemm_wide_kernel: 128 x 128 outputs, 4 wavefronts.
constexpr int kWideTile = 128;
constexpr int kWideWaves = 4;

size_t align_up(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }


}  // namespace

size_t split_x_bf16_bytes(uint32_t m, uint32_t k) {
    return static_cast<size_t>(m) * ((k / kGroup + 1) / 2) * kLimbs * 64 * sizeof(uint16_t);
}

hipError_t launch_split_x_bf16(const float* x, uint16_t* xs, uint32_t m, uint32_t k, hipStream_t stream) {
    const int KB = static_cast<int>((k / kGroup + 1) / 2);
    const size_t chunks = static_cast<size_t>(m) * KB * 8;
    hipLaunchKernelGGL(split_x_kernel, dim3(static_cast<unsigned>((chunks + 255) / 256)), dim3(256), 0, stream, x, xs,
                       static_cast<int>(m), static_cast<int>(k), KB);
    return hipGetLastError();
}

Q4Plan plan_q4gemm(const DeviceInfo& dev, uint32_t m, uint32_t n, uint32_t k, uint32_t rank) {
    Q4Plan plan{Q4Plan::kGemv, 1, 0, 0};
    if (rank == 0 && m <= static_cast<uint32_t>(kGemvMaxRows)) {
        return plan;
    }
    const int groups = static_cast<int>(k / kGroup);
    size_t lora_bytes = 0;
    if (rank > 0) {
        plan.t_splits = (groups + kLoraGroupsPerWave - 1) / kLoraGroupsPerWave;
        lora_bytes += align_up(static_cast<size_t>(plan.t_splits) * m * rank * sizeof(float));  // T partials
        lora_bytes += align_up(static_cast<size_t>(m) * rank * sizeof(float));                  // T
    }
    if (m <= 32 && k % (4 * kGroup) == 0) {
        plan.kind = Q4Plan::kSkinny;  // K split inside the workgroup: no partials in memory
        plan.workspace_bytes = lora_bytes;
        return plan;
    }
    int bm, bn, waves_per_tile;
    if (m <= 32) {
        plan.kind = Q4Plan::kSkinnySplitK;
        bm = SkinnyShape::kBM;
        bn = SkinnyShape::kBN;
        waves_per_tile = SkinnyShape::kWaves;
    } else {
        plan.kind = Q4Plan::kWide;
        bm = kWideTile;
        bn = kWideTile;
        waves_per_tile = kWideWaves;
    }
    const size_t tiles = static_cast<size_t>((m + bm - 1) / bm) * ((n + bn - 1) / bn);
    const size_t waves = tiles * waves_per_tile;
    // Resident wavefronts per SIMD at these register counts: skinny 3 (2 targeted), wide 1.
    const size_t waves_per_simd = plan.kind == Q4Plan::kSkinnySplitK ? 2 : 1;
    const size_t target = 4 * waves_per_simd * static_cast<size_t>(dev.cu_count);
    const int min_groups = plan.kind == Q4Plan::kSkinnySplitK ? 8 : 4;
    int splits = 1;
    while (waves * splits * 2 <= target && groups / (splits * 2) >= min_groups) splits *= 2;
    // Re-derive so that no split is empty. The wide kernel splits whole stages of two groups.
    const int units = plan.kind == Q4Plan::kWide ? (groups + 1) / 2 : groups;
    const int per_split = (units + splits - 1) / splits;
    splits = (units + per_split - 1) / per_split;
    plan.splits = splits;
    size_t bytes = lora_bytes;
    if (plan.kind == Q4Plan::kWide) bytes += align_up(split_x_bf16_bytes(m, k));  // x limbs
    if (splits > 1) bytes += align_up(static_cast<size_t>(splits) * m * n * sizeof(float));
    plan.workspace_bytes = bytes;
    return plan;
}

hipError_t launch_q4gemm(const Q4Plan& plan, const DeviceInfo& dev, const float* x,
                         const uint8_t* w_packed, const float* w_scales, float* y, uint32_t m,
                         uint32_t n, uint32_t k, const float* la, const float* lb, uint32_t rank,
                         float lora_scale, void* workspace, hipStream_t stream) {
    if (plan.kind == Q4Plan::kGemv) return launch_gemv(dev, x, w_packed, w_scales, y, m, n, k, stream);

    char* wsp = static_cast<char*>(workspace);
    float* partial = nullptr;
    if (plan.splits > 1) {
        partial = reinterpret_cast<float*>(wsp);
        wsp += align_up(static_cast<size_t>(plan.splits) * m * n * sizeof(float));
    }
    float* tmat = nullptr;
    if (rank > 0) {
        float* tpart = reinterpret_cast<float*>(wsp);
        wsp += align_up(static_cast<size_t>(plan.t_splits) * m * rank * sizeof(float));
        tmat = reinterpret_cast<float*>(wsp);
        wsp += align_up(static_cast<size_t>(m) * rank * sizeof(float));
        hipLaunchKernelGGL(lora_t_kernel, dim3((m + 15) / 16, (rank + 15) / 16, plan.t_splits), dim3(64), 0, stream,
                           x, la, tpart, static_cast<int>(m), static_cast<int>(k), static_cast<int>(rank));
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const size_t tcount = static_cast<size_t>(m) * rank;
        const size_t tblocks = std::min((tcount + 255) / 256, static_cast<size_t>(dev.cu_count) * 8);
        hipLaunchKernelGGL(split_reduce_kernel, dim3(static_cast<unsigned>(tblocks)), dim3(256), 0, stream, tpart,
                           tmat, tcount, plan.t_splits);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    float* out = plan.splits > 1 ? partial : y;
    const float* lbp = rank ? lb : nullptr;
    hipError_t e;
    if (plan.kind == Q4Plan::kSkinny) {
        const int tiles_m = static_cast<int>((m + 15) / 16);
        const int tiles_n = static_cast<int>((n + 15) / 16);
        const uint32_t* wq = reinterpret_cast<const uint32_t*>(w_packed);
        const bool few = tiles_m * tiles_n <= dev.cu_count;
        const bool stage = m > kSkinnyDirectMaxRows;
        const int waves = few ? kSkinnyWavesFew : kSkinnyWavesMany;
        auto kernel = few ? (stage ? q4_gemm_skinny_kernel<kSkinnyWavesFew, true>
                                   : q4_gemm_skinny_kernel<kSkinnyWavesFew, false>)
                          : (stage ? q4_gemm_skinny_kernel<kSkinnyWavesMany, true>
                                   : q4_gemm_skinny_kernel<kSkinnyWavesMany, false>);
        hipLaunchKernelGGL(kernel, dim3(tiles_m * tiles_n), dim3(64 * waves), 0, stream, x, wq, w_scales, y,
                           static_cast<int>(m), static_cast<int>(n), static_cast<int>(k), tiles_m, tmat, lbp,
                           static_cast<int>(rank), lora_scale);
        return hipGetLastError();
    }
    if (plan.kind == Q4Plan::kSkinnySplitK) {
        e = launch_mfma<1, 4, 1, 4, kSkinnyPD>(x, w_packed, w_scales, out, m, n, k, plan.splits, tmat, lbp, rank,
                                               lora_scale, stream);
    } else {
        const int tiles_m = static_cast<int>((m + kWideTile - 1) / kWideTile);
        const int tiles_n = static_cast<int>((n + kWideTile - 1) / kWideTile);
        const int KB = static_cast<int>((k / kGroup + 1) / 2);
        const int stages_per_split = (KB + plan.splits - 1) / plan.splits;
        uint16_t* xs = reinterpret_cast<uint16_t*>(wsp);
        e = launch_split_x_bf16(x, xs, m, k, stream);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(q4_gemm_wide_kernel, dim3(tiles_m * tiles_n, plan.splits), dim3(64 * kWideWaves), 0,
                           stream, xs, reinterpret_cast<const uint32_t*>(w_packed), w_scales, out, static_cast<int>(m),
                           static_cast<int>(n), static_cast<int>(k), tiles_m, tiles_n, stages_per_split, tmat, lbp,
                           static_cast<int>(rank), lora_scale);
        e = hipGetLastError();
    }
    if (e != hipSuccess || plan.splits == 1) return e;
    const size_t count = static_cast<size_t>(m) * n;
    size_t blocks = (count + 255) / 256;
    const size_t cap = static_cast<size_t>(dev.cu_count) * 8;
    if (blocks > cap) blocks = cap;
    hipLaunchKernelGGL(split_reduce_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                       partial, y, count, plan.splits);
    return hipGetLastError();
}

}  // namespace spaceslug
