// MFMA int4 GEMM for more than 32 rows (prefill, LoRA projections, the reference's
// 1024^3 bench shape). Two kernels: q4_gemm_wide_kernel, and q4_gemm_mid_kernel for
// the shapes whose wide grid would need a K-split, each described at its definition.
// (Up to 32 rows the exact small-batch GEMM of q4_small.hip runs instead.)
//
// Replaces q4gemm.comp:61-175 (64x64 tile, LDS-staged dequantised B, 4x4 FMA
// micro-tile per thread) with a CDNA4 design on the matrix cores:
// v_mfma_f32_32x32x16_bf16 with x split exactly into three bf16 limbs. Common to both:
//   - per 32-value scale group, each lane feeds the MFMA K slots with 8
//     consecutive K values, so its B operands for one column are the 8 nibbles
//     of ONE 32-bit word of the packed column and its A operands are 8
//     consecutive values of one row. Weights are decoded to v / 16 (exact in
//     bf16; the factor 16 multiplies the float64 sums at the store);
//   - every product limb * v / 16 is exact in fp32; the MFMA accumulates
//     P = sum x * v / 16 over one group in fp32 from zero, and the group is
//     folded straight into a float64 accumulator as s * P. Scale application
//     moves out of the inner loop, the long K sum is carried in double, and the
//     fp32 roundings of each group's sum are the only error left;
//   - large grids are XCD-aware: workgroup ids are remapped so each of the 8
//     XCDs (one L2 each) walks a contiguous band of output tiles, sharing A
//     rows and weight columns within its L2;
//   - when the grid is too small to fill 256 CUs, the mid-size kernel's 64 x 64
//     tiles take the shape if they fill the CUs once, else K is split across
//     blockIdx.y and a second kernel sums the partials in a fixed order.
// LoRA: the preparation launch that splits x into limbs also computes T = x * la on
// the MFMA as a few K-split partials (one per 512 values of K), and the GEMM
// epilogue sums them (lora_t_values) and adds scale * T[rows] * lb[:, cols] with the
// same MFMA tile layout (r in the K slot) before the single store of y.
#include <algorithm>
#include <utility>

#include "q4_device.hpp"
#include "q4_kernels.hpp"
#include "q4_lora.hpp"

namespace spaceslug {
namespace {

// Calls f(std::integral_constant<int, I>{}) for I = 0 .. N-1 in order (compile-time indices, so
// register arrays indexed by I stay in registers).
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Limbs per x value on the bf16 MFMA path.
constexpr int kLimbs = 3;

// x (fp32, M x K) -> x limbs (bf16) for q4_gemm_wide_kernel, laid out the way its copies
// consume them: [ceil(M/16)][K/32][3][16][4][8] = (16-row block, group, limb, row of the block,
// 16-byte slot, value). Slot s of row r holds the row's values 8c .. 8c+7 of the group with
// c = s ^ ((r >> 2) & 3), the kernel's LDS chunk swizzle, so a wavefront copies one limb of one
// group of a 16-row block as one contiguous 1 KiB run (8 full cache lines). Rows >= M are zero.
// Each value is split by split_bf16_limbs (b0 + b1 + b2 == x for |x| >= 2^-110, within 2^-133
// below), and a product of a limb with a bf16 weight v/16 is exact in fp32.
// One thread per (block, group, row, slot): two 16-byte loads (4 threads read one row's 128
// bytes of the group), three 16-byte stores, each store instruction of a wavefront one 1 KiB run.
constexpr int kLimbBlockValues = 16 * 32;  // one limb of one group of a 16-row block (1 KiB)

__device__ __forceinline__ void split_x_block(const float* __restrict__ x, uint16_t* __restrict__ xs, int M, int K,
                                              int block) {
    const int G = K >> 5;
    const size_t idx = static_cast<size_t>(block) * 256 + threadIdx.x;
    const size_t unit = idx >> 6;  // (16-row block, group)
    if (unit >= static_cast<size_t>((M + 15) >> 4) * G) return;
    const int lane = static_cast<int>(idx & 63);
    const int rr = lane >> 2;
    const int c = (lane & 3) ^ ((rr >> 2) & 3);
    const int row = static_cast<int>(unit / G) * 16 + rr;
    const int g = static_cast<int>(unit % G);
    float v[8];
    if (row < M) {
        const float* src = x + static_cast<size_t>(row) * K + g * 32 + c * 8;
        const f32x4 lo = *reinterpret_cast<const f32x4*>(src);
        const f32x4 hi = *reinterpret_cast<const f32x4*>(src + 4);
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
    uint16_t* dst = xs + unit * (kLimbs * kLimbBlockValues) + lane * 8;
    // Nontemporal: the limbs are read back by the next launch, not by this one (at 512 x 4096 the
    // preparation launch measured 6.5 -> 5.8 us).
#pragma unroll
    for (int li = 0; li < kLimbs; ++li)
        __builtin_nontemporal_store(limb[li], reinterpret_cast<u32x4*>(dst + li * kLimbBlockValues));
}

// Wide tile for M > 32 (prefill, LoRA projections): 128 x 128 outputs per workgroup of 8
// wavefronts, two per SIMD, each wavefront 32 x 64 outputs (two 32 x 32 MFMA tiles). The
// matrix instruction is v_mfma_f32_32x32x16_bf16, fed with x as three exact bf16 limbs
// (split_x_block) and the weights as bf16 v/16 (exact): every product is exact in fp32, each
// 32-value group's sum P = sum x * v/16 is accumulated in fp32 by six chained MFMAs per tile
// (limb 2, 1, 0, smallest first, each over the group's two 16-value halves), and the group is
// folded into float64 as acc += s * P; the factor 16 multiplies the float64 sums once, at the
// store (exact). One fp32 rounding per MFMA is the whole error, and the two of limb 0 dominate
// it: 4.5e-6 emulated on the reference KAT against 4.3e-6 for one 32-value MFMA per limb.
// Why 32 x 32 x 16: a gfx950 SIMD executes VALU instructions under its MFMAs, from either of
// its wavefronts, but only about 2 per 16 x 16 x 32 MFMA (16 matrix-core cycles) against about
// 6 per 32 x 32 x 16 MFMA (32 cycles); the float64 fold costs 2 VALU instructions per output
// and group, the same number per matrix-core cycle for both shapes, so only this shape keeps
// the fold (66 instructions per group and wavefront) inside the shadow of its 12 MFMAs.
// Lane l of a 32x32x16 MFMA holds A[row l%32][k = 8(l/32) .. +7] and B[k = 8(l/32) .. +7]
// [column l%32] (8 bf16 each), and result element v is row 8(v/4) + 4(l/32) + v%4 of
// column l%32, so every result a lane holds is in one column and needs one scale. Every
// operand reaches LDS by global_load_lds (no VGPRs, no register waits):
//   - x limbs, one 32-value group per stage, kWideStages buffers (the stage being read into
//     registers and 3 in flight): 3 limbs x 128 rows x 32 values (24 KiB); wavefront w copies
//     rows 16w .. 16w+15 of each limb, one 1 KiB instruction per limb. Row r's 16-byte chunk c
//     (8 values) sits at chunk c ^ ((r >> 2) & 3) of the row's 64 bytes: gfx950 serves a 128-bit LDS read
//     16 lanes per cycle, the 4-lane chunks of a half-wavefront whose chunk index has even
//     parity (lanes 0-3, 12-15, 20-23, 24-27) in one cycle and odd parity in the other, and two
//     of those lanes conflict when their addresses agree modulo 256 bytes; an operand read
//     (32 rows, one chunk per half-wavefront) then touches 16 distinct 16-byte bank groups in
//     each cycle;
//   - packed weights and scales, four groups at a time (a "quad"): lane l of wavefront w copies
//     the 16 bytes of group 4Q + (l >> 4) of tile column 16w + (l & 15), and that group's scale.
//     A column's 4 lanes read 64 contiguous bytes, and the per-column scales (512 bytes apart in
//     [N][K/32]) cost 16 lines per instruction;
//   - one stage ahead of its use, each thread decodes one packed word of the stage's group (one
//     its own wavefront copied) into the MFMA B layout (bf16 v/16, 8 KiB per group: 32-column
//     tile, 16-value half, lane), so every wavefront reads its B operands as linear 1 KiB runs.
// Iteration s passes one workgroup barrier (publishing stage s + 1), copies stage s + 4 into the
// buffers stage s was read from, reads stage s + 1's operands into registers spread over the
// group's MFMAs, waits for stage s + 2 (s_waitcnt vmcnt with the exact count of copies issued
// after it: 3 per stage, 2 more on quad boundaries) and decodes it. Copies past the end of the K
// range are clamped to its last group (never computed), so the counts hold everywhere.
constexpr int kWideStages = 4;
constexpr int kWideWavesPerTile = 8;

struct WideLds {
    // byte b of packed weights -> the bf16 values v / 16 of its low and high nibbles (low and high
    // half); first, so that ds_read's 16-bit offset field reaches it from a byte-scaled address
    uint32_t lut[256];
    u32x4 a[kWideStages][kLimbs][128][4];  // stage, limb, tile row, swizzled 16-byte chunk
    u32x4 b[2][4][2][64];                  // stage parity, 32-column tile, 16-value half, lane
    u32x4 braw[2][8][64];                  // quad parity, wavefront, lane: 16 packed bytes as copied
    float s[2][8][64];                     // quad parity, wavefront, lane: one scale as copied
};

// Vector-memory instructions issue(t) adds per wavefront.
__host__ __device__ constexpr int wide_copies(int t) { return (t % 4 == 0) ? kLimbs + 2 : kLimbs; }
// Copies issued by stages first .. first + count - 1 (the s_waitcnt vmcnt immediate that leaves
// exactly those in flight).
__host__ __device__ constexpr int wide_inflight(int first, int count) {
    return count == 0 ? 0 : wide_copies(first) + wide_inflight(first + 1, count - 1);
}

// Tile order of the wide kernel: XCD-contiguous runs as in xcd_tile, over a linear order that
// walks bands of kWideBandRows tile rows, each band column by column with its rows fastest. The
// 32 CUs of an XCD then hold 2 tile rows x 16 tile columns at a time, whose operands per group
// (2 x 24 KiB of x limbs, 16 x 2.5 KiB of weights and scales) are a quarter of those of 16 tile
// rows x 2 columns: the x limbs of every row of the matrix, streamed from beyond the XCD's L2
// once per column pair.
constexpr int kWideBandRows = 2;
__device__ __forceinline__ void wide_tile(int tiles_m, int tiles_n, int& tm, int& tn) {
    const int total = tiles_m * tiles_n;
    const int id = blockIdx.x;
    int lin = id;
    if (total >= 64 && (total & 7) == 0) lin = (id & 7) * (total >> 3) + (id >> 3);
    const int band = lin / (kWideBandRows * tiles_n);
    const int within = lin - band * kWideBandRows * tiles_n;
    const int h = min(kWideBandRows, tiles_m - kWideBandRows * band);  // the last band may be shorter
    tn = within / h;
    tm = kWideBandRows * band + within % h;
}

__global__ __launch_bounds__(512) void q4_gemm_wide_kernel(const uint16_t* xs, const uint32_t* wq, const float* ws,
                                                          float* __restrict__ out, int M, int N, int K,
                                                          int tiles_m, int tiles_n, int groups_per_split,
                                                          const float* __restrict__ tpart, int t_splits,
                                                          const float* __restrict__ lb, int R, float lscale) {
    __shared__ WideLds lds;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wid & 3;   // rows 32 wm .. 32 wm + 31 of the tile
    const int wn = wid >> 2;  // columns 64 wn .. 64 wn + 63 of the tile
    const int col32 = lane & 31;
    const int half = lane >> 5;
    const int G = K >> 5;

    int tile_m, tile_n;
    wide_tile(tiles_m, tiles_n, tile_m, tile_n);
    const int mt0 = tile_m * 128, nt0 = tile_n * 128;
    const int m0 = mt0 + wm * 32;
    const int n0 = nt0 + wn * 64;
    const int g_begin = blockIdx.y * groups_per_split;
    const int g_end = min(G, g_begin + groups_per_split);
    const int n_groups = g_end - g_begin;

    // x-limb copy of this wavefront: the 16-row block of tile rows 16 wid .. 16 wid + 15, one
    // contiguous 1 KiB run per limb (split_x_block lays the rows out swizzled as the LDS reads
    // expect). Blocks past the last one (rows past M, never stored) re-read the last block. The
    // address is a uniform base advanced per stage in scalar registers plus lane * 16 bytes, and
    // each limb's offset is the instruction's immediate (added to both addresses).
    const int xblocks = (M + 15) >> 4;
    const char* abase = reinterpret_cast<const char*>(
        xs + static_cast<size_t>(min((mt0 >> 4) + wid, xblocks - 1)) * G * (kLimbs * kLimbBlockValues));
    const uint32_t aoff = static_cast<uint32_t>(lane) * 16;
    // Quad copies: tile column 16 wid + (lane & 15), group 4Q + (lane >> 4) of the quad.
    const int qcol = min(nt0 + 16 * wid + (lane & 15), N - 1);
    const u32x4* bsrc = reinterpret_cast<const u32x4*>(wq + static_cast<size_t>(qcol) * (K >> 3));
    const float* ssrc = ws + static_cast<size_t>(qcol) * G;
    const int qg = lane >> 4;

    // Copies of stage t of this split (clamped into it).
    auto issue = [&](int t) {
        const int g = g_begin + min(t, n_groups - 1);
        const char* src = abase + static_cast<size_t>(g) * (kLimbs * kLimbBlockValues * sizeof(uint16_t));
        static_for<kLimbs>([&](auto lc) {
            constexpr int li = decltype(lc)::value;
            constexpr int kLimbBytes = kLimbBlockValues * sizeof(uint16_t);
            char* dst = reinterpret_cast<char*>(&lds.a[t % kWideStages][li][16 * wid][0]) - li * kLimbBytes;
            __builtin_amdgcn_global_load_lds(src + aoff, dst, 16, li * kLimbBytes, 0);
        });
        if (t % 4 == 0) {  // uniform
            const int gq = g_begin + min(t + qg, n_groups - 1);
            const int qb = (t >> 2) & 1;
            __builtin_amdgcn_global_load_lds(bsrc + gq, &lds.braw[qb][wid][0], 16, 0, 0);
            __builtin_amdgcn_global_load_lds(ssrc + gq, &lds.s[qb][wid][0], 4, 0, 0);
        }
    };
    // Decode of stage t's group: lane (j = lane & 15, q = lane >> 4) of wavefront w turns word q
    // of tile column c = 16w + j (copied by this wavefront) into the B slot of 32-column tile
    // c >> 5, half q >> 1, lane (c & 31) + 32 (q & 1).
    const int dj = lane & 15, dq = lane >> 4;
    const int dslot = 16 * (wid & 1) + dj + 32 * (dq & 1);
    auto read_raw = [&](int t) {
        return reinterpret_cast<const uint32_t*>(&lds.braw[(t >> 2) & 1][wid][dj + 16 * (t & 3)])[dq];
    };
    auto write_b = [&](int t, uint32_t raw) { lds.b[t & 1][wid >> 1][dq >> 1][dslot] = nibbles_bf16_16th(raw); };
    // The same decode through the byte table: four table reads instead of 13 VALU instructions.
    auto lookup_b = [&](uint32_t raw, u32x4& v) {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = lds.lut[(raw >> (8 * j)) & 0xFFu];
    };
    auto store_b = [&](int t, const u32x4& v) { lds.b[t & 1][wid >> 1][dq >> 1][dslot] = v; };
    // The workgroup barrier without the fence __syncthreads() adds: that fence waits for every
    // outstanding copy (vmcnt(0)), including the stages still in flight. The copies a stage needs
    // are waited for explicitly before it; this wavefront's LDS reads and writes are waited for here.
    auto barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

    double acc[2][16];
#pragma unroll
    for (int tn = 0; tn < 2; ++tn)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[tn][v] = 0.0;

    f32x16 zero16;
#pragma unroll
    for (int v = 0; v < 16; ++v) zero16[v] = 0.0f;
    // Operands: A (limb, half) of limbs 2 and 1 for the group being computed, read one stage ahead
    // once the MFMAs that use each register have issued; limb 0's A and B (tile, half)
    // double-buffered, so every read of the next stage issues by window 9 and has landed when the
    // next group starts; a group's sums and scales.
    struct OpsB {
        bf16x8 b[2][2];
    };
    struct Sums {
        f32x16 p[2];
        float s[2];
    };
    const int arow = 32 * wm + col32;
    const int pch0 = (0 + half) ^ ((lane >> 2) & 3);
    const int pch1 = (2 + half) ^ ((lane >> 2) & 3);
    bf16x8 a[kLimbs][2];  // a[0] unused: limb 0 lives in a0
    bf16x8 a0[2][2];      // buffer, half
    auto lds_a = [&](int t, int li, int ks) {
        return __builtin_bit_cast(bf16x8, lds.a[t & 3][li][arow][ks ? pch1 : pch0]);
    };
    auto read_a = [&](int t, int li, int ks) { a[li][ks] = lds_a(t, li, ks); };
    auto read_a0 = [&](int buf, int t, int ks) { a0[buf][ks] = lds_a(t, 0, ks); };
    auto read_b = [&](OpsB& o, int t, int tn, int ks) {
        o.b[tn][ks] = __builtin_bit_cast(bf16x8, lds.b[t & 1][2 * wn + tn][ks][lane]);
    };
    const int sw = 4 * wn + ((lane >> 4) & 1);
    auto read_s = [&](Sums& r, int t, int tn) {
        r.s[tn] = lds.s[(t >> 2) & 1][sw + 2 * tn][(lane & 15) + 16 * (t & 3)];
    };
    // Window w's MFMA: limb 2 - w / 4, half (w / 2) & 1, tile w & 1 (two independent chains).
    auto mfma_w = [&](Sums& r, const OpsB& ob, int abuf, int w) {
        const int li = 2 - (w >> 2), ks = (w >> 1) & 1, tn = w & 1;
        const bf16x8 av = li == 0 ? a0[abuf][ks] : a[li][ks];
        r.p[tn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, ob.b[tn][ks], w < 2 ? zero16 : r.p[tn], 0, 0, 0);
    };
    // Fold operation f (0..65) of the previous group's sums: the two scales' conversions, then per
    // tile and result a conversion and a float64 FMA acc += s * P, software-pipelined by
    // kFoldDepth (the conversion of result o + kFoldDepth issues right after the FMA of result o,
    // so each FMA's operand was converted kFoldDepth - 1 operations earlier).
    constexpr int kFoldDepth = 4;
    double scd[2], pd[kFoldDepth];
    auto fold_op = [&](const Sums& r, int f) {
        if (f < 2) {
            scd[f] = static_cast<double>(r.s[f]);
            return;
        }
        const int tn = f >= 34 ? 1 : 0;
        const int e = f - 2 - 32 * tn;  // 0 .. 31
        auto cvt = [&](int o) { pd[o % kFoldDepth] = static_cast<double>(r.p[tn][o]); };
        auto fold = [&](int o) { acc[tn][o] = fma(scd[tn], pd[o % kFoldDepth], acc[tn][o]); };
        if (e < kFoldDepth) {
            cvt(e);
        } else if (e < 32 - kFoldDepth) {
            const int k = e - kFoldDepth;
            if (k & 1)
                cvt(kFoldDepth + (k >> 1));
            else
                fold(k >> 1);
        } else {
            fold(e - 16);
        }
    };
    auto fold_all = [&](const Sums& r) {
#pragma unroll
        for (int f = 0; f < 66; ++f) fold_op(r, f);
    };

    if (n_groups > 0) {
        // Iteration s computes group s from operand registers read during iteration s - 1 and
        // folds group s - 1's sums. Window 1 holds the barrier that publishes stage s + 1 (copied
        // and decoded during iteration s - 1; the barrier also waits for this wavefront's earlier
        // LDS reads, so once every wavefront passes it stage s's buffers have been read), then
        // copies stage s + 4 into stage s's buffers. Windows 2 - 8 read stage s + 1's operands,
        // each register once the MFMAs that use it have issued (limb 2 after window 3, limb 1
        // after window 7); stage s + 1's scales go straight into the sums slot they will be
        // folded with, whose scales were converted in window 0. Window 8 waits for stage s + 2's
        // copies (issued two iterations earlier) and window 11 decodes its word of it.
        OpsB ob[2];
        Sums sums[2];
#pragma unroll
        for (int tn = 0; tn < 2; ++tn) {  // iteration 0 folds these zeros
            sums[1].s[tn] = 0.0f;
            sums[1].p[tn] = zero16;
        }
        issue(0);
        issue(1);
        issue(2);
        issue(3);
        if (tid < 256) {  // the byte table, the same conversions as nibbles_bf16_16th
            const uint32_t lo = __float_as_uint(__builtin_amdgcn_cvt_off_f32_i4(tid));
            const uint32_t hi = __float_as_uint(__builtin_amdgcn_cvt_off_f32_i4(tid >> 4));
            lds.lut[tid] = (lo >> 16) | (hi & 0xFFFF0000u);
        }
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(wide_inflight(1, 3)) : "memory");
        write_b(0, read_raw(0));
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(wide_inflight(2, 2)) : "memory");
        write_b(1, read_raw(1));
        barrier();
#pragma unroll
        for (int li = 1; li < kLimbs; ++li) {
            read_a(0, li, 0);
            read_a(0, li, 1);
        }
        read_a0(0, 0, 0);
        read_a0(0, 0, 1);
#pragma unroll
        for (int tn = 0; tn < 2; ++tn) {
            read_b(ob[0], 0, tn, 0);
            read_b(ob[0], 0, tn, 1);
            read_s(sums[0], 0, tn);
        }
        for (int s0 = 0; s0 < n_groups; s0 += 4) {
            static_for<4>([&](auto uc) {
                constexpr int u = decltype(uc)::value;
                const int s = s0 + u;
                if (s < n_groups) {  // uniform across the workgroup
                    const OpsB& cb = ob[u & 1];
                    OpsB& nb = ob[(u + 1) & 1];
                    Sums& cur = sums[u & 1];
                    Sums& old = sums[(u + 1) & 1];
                    uint32_t raw = 0;
                    u32x4 dec;
                    static_for<12>([&](auto wc) {
                        constexpr int w = decltype(wc)::value;
                        constexpr int f0 = w < 6 ? 6 * w : 36 + 5 * (w - 6);
                        constexpr int f1 = w < 6 ? f0 + 6 : f0 + 5;
                        mfma_w(cur, cb, u & 1, w);
                        static_for<f1 - f0>([&](auto fc) { fold_op(old, f0 + decltype(fc)::value); });
                        if constexpr (w == 1) {
                            barrier();
                            issue(s + 4);
                        }
                        if constexpr (w == 2) {
                            read_b(nb, s + 1, 0, 0);
                            read_b(nb, s + 1, 0, 1);
                        }
                        if constexpr (w == 3) {
                            read_b(nb, s + 1, 1, 0);
                            read_b(nb, s + 1, 1, 1);
                            read_s(old, s + 1, 0);
                            read_s(old, s + 1, 1);
                        }
                        if constexpr (w == 4) {
                            read_a(s + 1, 2, 0);
                            read_a(s + 1, 2, 1);
                        }
                        if constexpr (w == 5) {
                            read_a0((u + 1) & 1, s + 1, 0);
                            read_a0((u + 1) & 1, s + 1, 1);
                        }
                        if constexpr (w == 8) {
                            read_a(s + 1, 1, 0);
                            read_a(s + 1, 1, 1);
                            // stage s + 2's copies are done once only those of stages s + 3, s + 4 are in flight
                            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(wide_inflight(u + 3, 2)) : "memory");
                            raw = read_raw(s + 2);
                        }
                        if constexpr (w == 9) lookup_b(raw, dec);
                        if constexpr (w == 11) store_b(s + 2, dec);
                        __builtin_amdgcn_sched_barrier(0);
                    });
                }
            });
        }
        if ((n_groups - 1) & 1)  // constant indices keep sums in registers
            fold_all(sums[1]);
        else
            fold_all(sums[0]);
        // the copies issued past the end still write LDS: let them land before the workgroup ends
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }

    // LoRA ranks of this K-split: split z of S adds ranks [R z / S, R (z + 1) / S) (all of them
    // without a split), so the splits share the term's loads and MFMAs.
    const int r_lo = R * static_cast<int>(blockIdx.y) / static_cast<int>(gridDim.y);
    const int nr = R * static_cast<int>(blockIdx.y + 1) / static_cast<int>(gridDim.y) - r_lo;
    if (lb != nullptr && nr > 0) {  // uniform
        // LoRA term on the fp32 MFMA (r in the K slot), added as (lscale / 16) * P since the sums
        // are multiplied by 16 at the store. The stage buffers are free now: the tile's 128 rows
        // of T (its partials summed) and 128 columns of lb, for this split's nr ranks, are loaded
        // there by the whole workgroup at once, rows padded to nr + 1 floats, then read as MFMA
        // operands.
        static_assert(sizeof(lds.a) >= sizeof(float) * (128 * (kMaxLoraRank + 1) + kMaxLoraRank * 128),
                      "the LoRA tiles fit in the stage buffers");
        const int RP = nr + 1;
        float* ts = reinterpret_cast<float*>(&lds.a[0][0][0][0]);  // [128][RP]
        float* bs = ts + 128 * RP;                                  // [nr][128]
        __syncthreads();  // every wavefront is past its last LDS read and copy
        // Four values of T and of lb per thread and pass, every load of a pass issued before the
        // first store (loads waited for one after another cost ~4.5 us per call at 512 x 4096 x
        // 4096, r = 16).
        constexpr int kNV = 4;
        for (int e0 = tid; e0 < 128 * nr; e0 += 512 * kNV) {
            float tv[kNV], bv[kNV];
#pragma unroll
            for (int v = 0; v < kNV; ++v) {
                const int e = e0 + 512 * v;
                bv[v] = lb[static_cast<size_t>(r_lo + min(e >> 7, nr - 1)) * N + min(nt0 + (e & 127), N - 1)];  // in bounds
            }
            lora_t_values<kNV>(tpart, t_splits, M, R, r_lo, nr, mt0, e0, 512, 128 * nr, tv);
#pragma unroll
            for (int v = 0; v < kNV; ++v) {
                const int e = e0 + 512 * v;
                if (e < 128 * nr) {
                    const int row = e / nr, r = e - row * nr;
                    ts[row * RP + r] = tv[v];
                    bs[e] = bv[v];
                }
            }
        }
        __syncthreads();
        const double s = static_cast<double>(lscale) * 0.0625;
        // Eight ranks per pass: every operand of the pass read (unconditionally, at a rank clamped
        // into range) before its MFMAs, which run the two 32-column tiles' chains interleaved; a
        // rank past nr enters as zeros.
        f32x16 P[2] = {zero16, zero16};
        for (int r8 = 0; r8 < nr; r8 += 8) {
            float av[4], bv[4][2];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int r = r8 + 2 * j + half, rc = min(r, nr - 1);
                const float a = ts[arow * RP + rc];
                av[j] = r < nr ? a : 0.0f;
#pragma unroll
                for (int tn = 0; tn < 2; ++tn) {
                    const float b = bs[rc * 128 + wn * 64 + 32 * tn + col32];
                    bv[j][tn] = r < nr ? b : 0.0f;
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int tn = 0; tn < 2; ++tn)
                    P[tn] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[j], bv[j][tn], P[tn], 0, 0, 0);
        }
#pragma unroll
        for (int tn = 0; tn < 2; ++tn)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[tn][v] = fma(s, static_cast<double>(P[tn][v]), acc[tn][v]);
    }

    float* dst = out + static_cast<size_t>(blockIdx.y) * M * N;
#pragma unroll
    for (int tn = 0; tn < 2; ++tn) {
        const int col = n0 + 32 * tn + col32;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int row = m0 + 8 * (v >> 2) + 4 * half + (v & 3);
            if (row < M && col < N) dst[static_cast<size_t>(row) * N + col] = static_cast<float>(acc[tn][v] * 16.0);
        }
    }
}

// Mid-size tiles for M > 32 when the 128 x 128 grid would leave CUs idle and need a K-split plus
// a reduction launch (the reference benchmark's M = N = K = 1024: 64 wide tiles): 64 x 64 outputs
// per workgroup of 8 wavefronts over the whole of K, no partials in memory. x comes as bf16 limbs
// laid out [M][K/64][3][64] (x_limb_rows_kernel), and the design is that of the pipelined CQ4
// kernel (cq4.hip) with one weight limb:
//   - wavefront w owns the 32 x 32 output tile (rows 32 (w & 1), columns 32 ((w >> 1) & 1)) for
//     the 32-value group (w >> 2) of every 64-value stage, so the two wavefronts of a SIMD split K
//     by groups; per stage a wavefront runs one chain of 6 v_mfma_f32_32x32x16_bf16 (limbs 2, 1, 0,
//     smallest first, each over the group's two 16-value halves: the order of the wide kernel) and
//     folds the previous stage's group sums into float64 between them (acc += s * P, 32 operations);
//     the two halves of K are added in double through LDS at the end, and the sums multiplied by
//     16 (the weights enter as v / 16) before the single fp32 store;
//   - every operand reaches LDS by global_load_lds: the x limbs four stages deep (wavefront w
//     copies the 8-row block w of each limb, rows paired and 16-byte chunks swizzled), the packed
//     weights by stage pairs (each thread copies the two words it decodes, one per stage), the
//     tile's scales (all groups) once before the loop;
//   - one stage ahead of its use each thread decodes its word (nibbles_bf16_16th) into the B
//     layout of pipe_b_slot, conflict-free for the writes and the MFMA reads;
//   - iteration t copies stage t + 4 into slot t % 4 and on even t the stage pair t + 4, t + 5,
//     then runs stage t's chain with, between its MFMAs, stage t - 1's fold, the operand reads of
//     stage t + 1 and the decode of stage t + 2, and passes one barrier. Past the last stage the
//     copied stage is clamped, so every wavefront issues the same copies per iteration and
//     `s_waitcnt vmcnt(8)` leaves exactly the two younger stages and one pair in flight.
constexpr int kMidTile = 64;
constexpr int kMidStages = 4;
constexpr int kMidWaves = 8;
constexpr int kMidGroupsMax = 128;  // scale groups per column held in LDS (K <= 4096)

struct MidLds {
    u32x4 a[kMidStages][kLimbs][8][64];      // stage, limb, 8-row block, 16-byte chunk (row pairs)
    uint32_t braw[2][kMidWaves][2][64];      // stage-pair slot, wavefront, stage of the pair, thread
    u32x4 b[2][2][2][2][64];                 // stage parity, group of the stage, 32-column tile, half, slot
    // the tile's scales as they lie in the array (column, group), one padding word after every 64:
    // value i at i + i / 64, so the 32 columns one read touches fall in distinct banks
    float s[kMidTile * kMidGroupsMax + kMidGroupsMax + 64];
};
static_assert(sizeof(MidLds) <= 160 * 1024, "LDS budget");

// x (fp32, M x K, K % 64 == 0) -> its bf16 limbs laid out [M][K/64][3][64] (row, 64-value stage,
// limb, value) for q4_gemm_mid_kernel: one thread per 8 values, two 16-byte loads and three 16-byte
// stores (8 consecutive threads write one limb's 128-byte run of a stage). With xcd_rows set (the
// GEMM's 64-row tiles a multiple of 8), workgroup b works on the rows of tiles t with t % 8 == b % 8:
// workgroups run on XCD b % 8 and the GEMM reads row tile t on XCD t % 8, so each row's limbs are
// written through the L2 that later serves them.
__global__ __launch_bounds__(256) void x_limb_rows_kernel(const float* __restrict__ x, uint16_t* __restrict__ xs,
                                                         int M, int K, bool xcd_rows) {
    const size_t per_row = static_cast<size_t>(K >> 3);
    size_t row, c;
    if (xcd_rows) {
        const size_t u = static_cast<size_t>(blockIdx.x / 8) * 256 + threadIdx.x;  // unit in XCD lane b % 8
        const size_t lr = u / per_row;                                             // row of that lane
        row = (blockIdx.x % 8 + 8 * (lr / kMidTile)) * kMidTile + lr % kMidTile;
        c = u - lr * per_row;
        if (row >= static_cast<size_t>(M)) return;
    } else {
        const size_t e = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;  // 8-value unit
        if (e >= static_cast<size_t>(M) * per_row) return;
        row = e / per_row;
        c = e % per_row;
    }
    const float* src = x + row * K + 8 * c;
    const f32x4 lo = *reinterpret_cast<const f32x4*>(src);
    const f32x4 hi = *reinterpret_cast<const f32x4*>(src + 4);
    u32x4 limb[kLimbs];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        uint32_t l0[kLimbs], l1[kLimbs];
        split_bf16_limbs(t < 2 ? lo[2 * t] : hi[2 * t - 4], l0);
        split_bf16_limbs(t < 2 ? lo[2 * t + 1] : hi[2 * t - 3], l1);
#pragma unroll
        for (int li = 0; li < kLimbs; ++li) limb[li][t] = l0[li] | (l1[li] << 16);
    }
    uint16_t* dst = xs + (row * (K >> 6) + (c >> 3)) * (kLimbs * 64) + 8 * (c & 7);
#pragma unroll
    for (int li = 0; li < kLimbs; ++li) *reinterpret_cast<u32x4*>(dst + li * 64) = limb[li];
}

// x limbs, wq and ws are deliberately not __restrict__: as provably invariant loads the compiler
// would be free to re-issue loads at their use (to save registers), serialising them behind compute.
__global__ __launch_bounds__(64 * kMidWaves) void q4_gemm_mid_kernel(const uint16_t* xs, const uint32_t* wq,
                                                                    const float* ws, float* __restrict__ y, int M,
                                                                    int N, int K, int tiles_m) {
    __shared__ MidLds lds;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wid & 1, wn = (wid >> 1) & 1, ku = wid >> 2;
    const int col32 = lane & 31, half = lane >> 5;
    const int T = K / 64;
    const int G = K / 32;
    const int mt0 = static_cast<int>(blockIdx.x % tiles_m) * kMidTile;
    const int nt0 = static_cast<int>(blockIdx.x / tiles_m) * kMidTile;

    // x-limb copy of this wavefront: 8-row block wid (row pairs 4 wid .. 4 wid + 3); lane l copies
    // chunk (l % 8) ^ (pair % 8) of its row, so that chunk c of a row sits at slot c ^ (pair % 8).
    const uint16_t* asrc;
    {
        const int pair = 4 * wid + (lane >> 4);
        const int row_t = 2 * pair + ((lane >> 3) & 1);
        asrc = xs + static_cast<size_t>(min(mt0 + row_t, M - 1)) * T * (kLimbs * 64) + 8 * ((lane & 7) ^ (pair & 7));
    }
    // Packed word this thread decodes: group bu of the stage, tile column bc, word bw of the group.
    const int bc = 8 * wid + (lane >> 3), bu = (lane >> 2) & 1, bw = lane & 3;
    const int bdst = pipe_b_slot((bc & 31) + 32 * (bw & 1), bw >> 1, bu);
    const char* bsrc = reinterpret_cast<const char*>(wq) + static_cast<size_t>(min(nt0 + bc, N - 1)) * (K >> 1) +
                       4 * (lane & 7);
    // This lane's A operand: row 32 wm + (lane & 31), chunk 4 ku + 2 h + (lane >> 5) of a stage for half h.
    const int ar = 32 * wm + col32;
    const int apr = ar >> 1;
    const int aidx0 = apr * 16 + 8 * (ar & 1) + ((4 * ku + half) ^ (apr & 7));
    const int aidx1 = apr * 16 + 8 * (ar & 1) + ((4 * ku + 2 + half) ^ (apr & 7));
    const int bsrc0 = pipe_b_slot(lane, 0, ku), bsrc1 = pipe_b_slot(lane, 1, ku);

    // Stage t's limbs into stage slot st (past the last stage, t is clamped and st is not).
    auto issue = [&](int t, int st) {
#pragma unroll
        for (int li = 0; li < kLimbs; ++li)
            __builtin_amdgcn_global_load_lds(asrc + static_cast<size_t>(t) * (kLimbs * 64) + li * 64,
                                             &lds.a[st][li][wid][0], 16, 0, 0);
    };
    // Packed weights of stages 2 j and 2 j + 1 into slot `slot`, one 4-byte copy per stage (clamped
    // to the last stage past the end of the column).
    auto issue_b = [&](int j, int slot) {
#pragma unroll
        for (int cc = 0; cc < 2; ++cc)
            __builtin_amdgcn_global_load_lds(bsrc + min(32 * (2 * j + cc), (K >> 1) - 32), &lds.braw[slot][wid][cc][0], 4,
                                             0, 0);
    };
    auto decode_word = [&](int t) { return lds.braw[(t >> 1) & 1][wid][t & 1][lane]; };
    // VALU decode (13 instructions per word): in this kernel, which waits on LDS more than it issues,
    // it measured faster than the wide kernel's byte table, whose reads land on random banks
    // (24.2 against 26.0-26.6 us per call at 1024^3).
    auto decode_lookup = [&](uint32_t wd, u32x4& v) { v = nibbles_bf16_16th(wd); };
    auto decode_write = [&](int t, const u32x4& v) { lds.b[t & 1][bu][bc >> 5][bw >> 1][bdst] = v; };
    auto barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

    // The tile's scales (64 columns of G values, contiguous in the array), then stages 0 .. 3 and
    // pairs 0 and 1; stages 2 and 3 and pair 1 stay in flight while stages 0 and 1 are decoded and
    // read: `s_waitcnt vmcnt(8)` leaves exactly their 3 + 3 + 2 copies outstanding.
    {
        const char* ssrc = reinterpret_cast<const char*>(ws) + static_cast<size_t>(nt0) * G * 4;
        const int units = kMidTile * G;  // 4-byte units
        const size_t last = static_cast<size_t>(N - nt0) * G * 4 - 4;
        for (int b = wid; 64 * b < units; b += kMidWaves)  // uniform
            __builtin_amdgcn_global_load_lds(ssrc + min(static_cast<size_t>(4 * (64 * b + lane)), last),
                                             reinterpret_cast<char*>(lds.s) + 260 * b, 4, 0, 0);
    }
    const int jmax = (T - 1) / 2;  // the last stage pair
    issue(0, 0);
    issue_b(0, 0);
    issue(min(1, T - 1), 1);
    issue(min(2, T - 1), 2);
    issue_b(min(1, jmax), 1);
    issue(min(3, T - 1), 3);
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    barrier();  // scales visible, every wavefront's stages 0 and 1 and pair 0 copied
    {
        u32x4 v0, v1;
        const uint32_t w0 = decode_word(0), w1 = decode_word(1);
        decode_lookup(w0, v0);
        decode_lookup(w1, v1);
        decode_write(0, v0);
        decode_write(1, v1);  // past the last stage: an unread buffer from a clamped copy
    }
    barrier();

    struct Operands {
        bf16x8 a[kLimbs][2], b[2];
    };
    Operands ops[2];
    // Operand reads of stage t in the order the chain uses them: limb 2, weights, limb 1, limb 0.
    auto read_part = [&](Operands& o, int t, int part) {
        const int sidx = t & (kMidStages - 1), par = t & 1;
        if (part == 1) {
            o.b[0] = __builtin_bit_cast(bf16x8, lds.b[par][ku][wn][0][bsrc0]);
            o.b[1] = __builtin_bit_cast(bf16x8, lds.b[par][ku][wn][1][bsrc1]);
        } else {
            const int li = part == 0 ? 2 : (part == 2 ? 1 : 0);
            o.a[li][0] = __builtin_bit_cast(bf16x8, (&lds.a[sidx][li][0][0])[aidx0]);
            o.a[li][1] = __builtin_bit_cast(bf16x8, (&lds.a[sidx][li][0][0])[aidx1]);
        }
    };
#pragma unroll
    for (int part = 0; part < 4; ++part) read_part(ops[0], 0, part);
    barrier();  // stage 0's slot is read before iteration 0 copies into it

    f32x16 zero16;
#pragma unroll
    for (int v = 0; v < 16; ++v) zero16[v] = 0.0f;
    double acc[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0;
    struct Stage {
        f32x16 p;
        double s;
    };
    Stage st_buf[2];
    st_buf[1].p = zero16;  // iteration 0 folds these zeros
    st_buf[1].s = 0.0;
    // fold operation f (0 .. 31) of a stage: per result a conversion, then (one result later) a
    // float64 FMA acc += s * P
    double pd[2];
    auto fold_op = [&](const Stage& r, int f) {
        if (f == 0) {
            pd[0] = static_cast<double>(r.p[0]);
        } else if (f == 31) {
            acc[15] = fma(r.s, pd[1], acc[15]);
        } else if (f & 1) {
            const int o = (f + 1) >> 1;  // 1 .. 15
            pd[o & 1] = static_cast<double>(r.p[o]);
        } else {
            const int o = (f - 2) >> 1;  // 0 .. 14
            acc[o] = fma(r.s, pd[o & 1], acc[o]);
        }
    };
    const int sbase = (32 * wn + col32) * G + ku;  // this lane's column, group ku of stage 0 (unpadded index)

    for (int t0 = 0; t0 < T; t0 += 2) {
        static_for<2>([&](auto uc) {
            constexpr int u = decltype(uc)::value;
            const int t = t0 + u;
            if (t < T) {  // uniform
                Stage& cur = st_buf[u];
                const Stage& old = st_buf[u ^ 1];
                const Operands& op = ops[u];
                Operands& nxt = ops[u ^ 1];
                issue(min(t + 4, T - 1), t & (kMidStages - 1));
                if constexpr (u == 0) issue_b(min(t / 2 + 2, jmax), (t / 2) & 1);  // t is even
                uint32_t wd = 0;
                u32x4 dec;
                float sraw = 0.0f;
                static_for<6>([&](auto ic) {
                    constexpr int i = decltype(ic)::value;
                    constexpr int li = 2 - (i >> 1), h = i & 1;
                    cur.p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op.a[li][h], op.b[h], i == 0 ? zero16 : cur.p, 0,
                                                                    0, 0);
                    __builtin_amdgcn_sched_barrier(0);  // the MFMA first: a wait below stalls only the rest
                    constexpr int f0 = i < 2 ? 6 * i : 12 + 5 * (i - 2);
                    constexpr int f1 = i < 2 ? f0 + 6 : f0 + 5;
                    static_for<f1 - f0>([&](auto fc) { fold_op(old, f0 + decltype(fc)::value); });
                    if constexpr (i == 0) {
                        // this wavefront's copies of stage t + 2 and of its pair; after them come stages
                        // t + 3, t + 4 and one pair (3 + 3 + 2 copies)
                        asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
                        wd = decode_word(t + 2);
                        const int si = sbase + 2 * t;
                        sraw = lds.s[si + (si >> 6)];
                    }
                    if constexpr (i == 1) decode_lookup(wd, dec);
                    if constexpr (i == 5) decode_write(t + 2, dec);  // past the last stage: an unread buffer
                    if constexpr (i >= 2) read_part(nxt, t + 1, i - 2);  // past the last stage: unused
                    if constexpr (i == 3) cur.s = static_cast<double>(sraw);
                    __builtin_amdgcn_sched_barrier(0);
                });
                barrier();
            }
        });
    }
    if (T & 1) {  // uniform: the last stage's sums are in st_buf[(T - 1) % 2]
#pragma unroll
        for (int f = 0; f < 32; ++f) fold_op(st_buf[0], f);
    } else {
#pragma unroll
        for (int f = 0; f < 32; ++f) fold_op(st_buf[1], f);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the clamped copies past the last stage
    // The two halves of K of each tile, added in double: the wavefront of group u finishes results
    // 8 u .. 8 u + 7 of its tile and hands the other eight to its partner through LDS; the fp32 tile
    // is then assembled in LDS and stored as 32-byte row pieces.
    double* red = reinterpret_cast<double*>(&lds.a[0][0][0][0]);  // [4 tiles][16 results][64 lanes]
    float* tile = reinterpret_cast<float*>(&lds.b[0][0][0][0][0]);  // [64 rows][64 columns]
    static_assert(sizeof(lds.b) >= sizeof(float) * kMidTile * kMidTile, "the output tile fits");
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
            tile[row * kMidTile + 32 * wn + col32] = static_cast<float>(s * 16.0);
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
        const f32x4 v0 = *reinterpret_cast<const f32x4*>(&tile[rl * kMidTile + c8]);
        const f32x4 v1 = *reinterpret_cast<const f32x4*>(&tile[rl * kMidTile + c8 + 4]);
        const bool vec = N % 4 == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;  // uniform
        if (row < M) {
            float* dst = y + static_cast<size_t>(row) * N + col;
            if (vec && col + 8 <= N) {
                *reinterpret_cast<f32x4*>(dst) = v0;
                *reinterpret_cast<f32x4*>(dst + 4) = v1;
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (col + e < N) dst[e] = e < 4 ? v0[e] : v1[e - 4];
            }
        }
    }
}

// One launch that prepares a call's GEMM: the first lora_blocks workgroups compute the LoRA T
// partials (lora_t_block, grid tiles_m_t x tiles_r x t_splits), the rest split x into bf16
// limbs (split_x_block; none when the GEMM reads fp32 x). Both only read x. The T workgroups
// come first because each runs a long dependent chain (all of its loads, then its MFMAs): started
// last, behind the many short split workgroups, they set the launch's end.
__global__ __launch_bounds__(256) void prep_kernel(const float* __restrict__ x, uint16_t* __restrict__ xs, int M,
                                                   int K, int lora_blocks, const float* __restrict__ la,
                                                   float* __restrict__ tpart, int R, int tiles_m_t, int tiles_r) {
    const int b = static_cast<int>(blockIdx.x);
    if (b >= lora_blocks) {
        split_x_block(x, xs, M, K, b - lora_blocks);
        return;
    }
    lora_t_block(x, la, tpart, M, K, R, b % tiles_m_t, (b / tiles_m_t) % tiles_r, b / (tiles_m_t * tiles_r));
}

// y[i] = sum_s part[s][i], in ascending s, accumulated in double (the K-split partials of the
// GEMM). With vec set (count % 4 == 0 and y 16-byte aligned) a thread takes four consecutive
// outputs with 16-byte loads and one 16-byte store, all of a pass's loads (up to four partial
// planes) issued before the first add: at two planes a thread waits for one round of loads per
// pass instead of one per output.
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* __restrict__ part,
                                                           float* __restrict__ y, size_t count,
                                                           int splits, bool vec) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    const size_t first = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (vec) {  // uniform
        const size_t quads = count >> 2;
        for (size_t q = first; q < quads; q += stride) {
            double s[4] = {0.0, 0.0, 0.0, 0.0};
            for (int z0 = 0; z0 < splits; z0 += 4) {
                f32x4 v[4];
#pragma unroll
                for (int u = 0; u < 4; ++u)  // a plane past the last re-reads the last (in bounds, not added)
                    v[u] = *reinterpret_cast<const f32x4*>(part + static_cast<size_t>(min(z0 + u, splits - 1)) * count +
                                                           4 * q);
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (z0 + u < splits)
#pragma unroll
                        for (int c = 0; c < 4; ++c) s[c] += static_cast<double>(v[u][c]);
            }
            *reinterpret_cast<f32x4*>(y + 4 * q) =
                f32x4{static_cast<float>(s[0]), static_cast<float>(s[1]), static_cast<float>(s[2]),
                      static_cast<float>(s[3])};
        }
        return;
    }
    for (size_t i = first; i < count; i += stride) {
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

// Wide tile of q4_gemm_wide_kernel: 128 x 128 outputs, 8 wavefronts.
constexpr int kWideTile = 128;

size_t align_up(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }


}  // namespace

size_t split_x_bf16_bytes(uint32_t m, uint32_t k) {
    return static_cast<size_t>((m + 15) / 16) * 16 * k * kLimbs * sizeof(uint16_t);
}

Q4Plan plan_q4gemm(const DeviceInfo& dev, uint32_t m, uint32_t n, uint32_t k, uint32_t rank) {
    Q4Plan plan{Q4Plan::kGemv, 1, 0, 0};
    if (rank == 0 && gemv_takes(m, k)) return plan;
    const int groups = static_cast<int>(k / kGroup);
    size_t lora_bytes = 0;
    if (rank > 0) {
        plan.t_splits = (groups + kLoraGroupsPerBlock - 1) / kLoraGroupsPerBlock;
        lora_bytes += align_up(static_cast<size_t>(plan.t_splits) * m * rank * sizeof(float));  // T partials
    }
    if (m <= 32) {
        plan.kind = Q4Plan::kDigits;
        plan.workspace_bytes = lora_bytes;  // the T partials of a LoRA call; none otherwise
        return plan;
    }
    plan.kind = Q4Plan::kWide;
    const size_t tiles = static_cast<size_t>((m + kWideTile - 1) / kWideTile) * ((n + kWideTile - 1) / kWideTile);
    const size_t waves = tiles * kWideWavesPerTile;
    // Resident wavefronts per SIMD: 2 (one workgroup of 8 per CU, bound by LDS).
    const size_t waves_per_simd = 2;
    const size_t target = 4 * waves_per_simd * static_cast<size_t>(dev.cu_count);
    const int min_groups = 4;
    int splits = 1;
    while (waves * splits * 2 <= target && groups / (splits * 2) >= min_groups) splits *= 2;
    // Re-derive so that no split is empty.
    const int per_split = (groups + splits - 1) / splits;
    splits = (groups + per_split - 1) / per_split;
    plan.splits = splits;
    const size_t mid_tiles = static_cast<size_t>((m + kMidTile - 1) / kMidTile) * ((n + kMidTile - 1) / kMidTile);
    if (splits > 1 && rank == 0 && k % 64 == 0 && groups <= kMidGroupsMax &&
        mid_tiles <= static_cast<size_t>(dev.cu_count)) {
        plan.kind = Q4Plan::kMid;  // whole K per 64 x 64 tile: no partials, no reduction launch
        plan.splits = 1;
        plan.workspace_bytes = align_up(static_cast<size_t>(m) * k * kLimbs * sizeof(uint16_t));  // x limbs
        return plan;
    }
    size_t bytes = lora_bytes + align_up(split_x_bf16_bytes(m, k));  // x limbs
    if (splits > 1) bytes += align_up(static_cast<size_t>(splits) * m * n * sizeof(float));
    plan.workspace_bytes = bytes;
    return plan;
}

hipError_t launch_q4gemm(const Q4Plan& plan, const DeviceInfo& dev, const float* x,
                         const uint8_t* w_packed, const float* w_scales, float* y, uint32_t m,
                         uint32_t n, uint32_t k, const float* la, const float* lb, uint32_t rank,
                         float lora_scale, void* workspace, hipStream_t stream) {
    if (plan.kind == Q4Plan::kGemv) return launch_gemv(dev, x, w_packed, w_scales, y, m, n, k, stream);
    if (plan.kind == Q4Plan::kDigits)
        return launch_q4gemm_small(dev, x, w_packed, w_scales, y, m, n, k, la, lb, rank, lora_scale, plan.t_splits,
                                   workspace, stream);
    if (plan.kind == Q4Plan::kMid) {
        uint16_t* xs = static_cast<uint16_t*>(workspace);
        const int tiles_m = static_cast<int>((m + kMidTile - 1) / kMidTile);
        const bool xcd_rows = tiles_m % 8 == 0;  // the GEMM then reads row tile t on XCD t % 8
        // XCD lane b % 8 holds tiles_m / 8 row tiles of 64 rows (the last may be partial)
        const size_t units = xcd_rows ? static_cast<size_t>(tiles_m / 8) * kMidTile * (k / 8) : static_cast<size_t>(m) * (k / 8);
        const size_t blocks = xcd_rows ? 8 * ((units + 255) / 256) : (units + 255) / 256;
        hipLaunchKernelGGL(x_limb_rows_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, x, xs,
                           static_cast<int>(m), static_cast<int>(k), xcd_rows);
        const hipError_t pe = hipGetLastError();
        if (pe != hipSuccess) return pe;
        const int tiles_n = static_cast<int>((n + kMidTile - 1) / kMidTile);
        hipLaunchKernelGGL(q4_gemm_mid_kernel, dim3(tiles_m * tiles_n), dim3(64 * kMidWaves), 0, stream, xs,
                           reinterpret_cast<const uint32_t*>(w_packed), w_scales, y, static_cast<int>(m),
                           static_cast<int>(n), static_cast<int>(k), tiles_m);
        return hipGetLastError();
    }

    char* wsp = static_cast<char*>(workspace);
    float* partial = nullptr;
    if (plan.splits > 1) {
        partial = reinterpret_cast<float*>(wsp);
        wsp += align_up(static_cast<size_t>(plan.splits) * m * n * sizeof(float));
    }
    float* tpart = nullptr;
    if (rank > 0) {
        tpart = reinterpret_cast<float*>(wsp);
        wsp += align_up(static_cast<size_t>(plan.t_splits) * m * rank * sizeof(float));
    }
    const int kk = static_cast<int>(k), mm = static_cast<int>(m), rr = static_cast<int>(rank);
    // One preparation launch: the bf16 limbs of x for the wide kernel and/or the LoRA T partials.
    uint16_t* xs = reinterpret_cast<uint16_t*>(wsp);
    {
        // split_x_block: 64 threads per (16-row block, group)
        const int split_blocks = static_cast<int>(((m + 15) / 16 * static_cast<size_t>(k / kGroup) * 64 + 255) / 256);
        const int tiles_m_t = static_cast<int>((m + 15) / 16), tiles_r = static_cast<int>((rank + 15) / 16);
        const int lora_blocks = rank ? tiles_m_t * tiles_r * plan.t_splits : 0;
        hipLaunchKernelGGL(prep_kernel, dim3(static_cast<unsigned>(split_blocks + lora_blocks)), dim3(256), 0, stream,
                           x, xs, mm, kk, lora_blocks, la, tpart, rr, tiles_m_t, tiles_r);
        const hipError_t pe = hipGetLastError();
        if (pe != hipSuccess) return pe;
    }
    float* out = plan.splits > 1 ? partial : y;
    const float* lbp = rank ? lb : nullptr;
    const int tiles_m = static_cast<int>((m + kWideTile - 1) / kWideTile);
    const int tiles_n = static_cast<int>((n + kWideTile - 1) / kWideTile);
    const int G = static_cast<int>(k / kGroup);
    const int groups_per_split = (G + plan.splits - 1) / plan.splits;
    hipLaunchKernelGGL(q4_gemm_wide_kernel, dim3(tiles_m * tiles_n, plan.splits),
                       dim3(64 * kWideWavesPerTile), 0, stream, xs, reinterpret_cast<const uint32_t*>(w_packed),
                       w_scales, out, mm, static_cast<int>(n), kk, tiles_m, tiles_n, groups_per_split, tpart,
                       plan.t_splits, lbp, rr, lora_scale);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || plan.splits == 1) return e;
    const size_t count = static_cast<size_t>(m) * n;
    // plane z starts z * count floats past the first: 16-byte aligned with the first when count % 4 == 0
    const bool vec = count % 4 == 0 && ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(partial)) & 15) == 0;
    size_t blocks = ((vec ? count / 4 : count) + 255) / 256;
    const size_t cap = static_cast<size_t>(dev.cu_count) * 8;
    if (blocks > cap) blocks = cap;
    hipLaunchKernelGGL(split_reduce_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                       partial, y, count, plan.splits, vec);
    return hipGetLastError();
}

}  // namespace spaceslug
