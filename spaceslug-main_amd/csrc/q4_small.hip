// Exact small-batch int4 GEMM: M <= 32 rows (and one row with K > 32768), any K % 32 == 0.
//
// Replaces q4gemm.comp:61-175 for decode-sized batches. Every 32-value group sum
// sum_k x[m][k] * v[k][n] is formed exactly, in integers, on the int8 matrix cores, in one
// launch with no device memory beyond the arguments (a LoRA call adds the T = x * la
// partials of a preparation launch):
//   - each wavefront recodes the groups of x it consumes, per row and 32-value group, in
//     31-bit fixed point: X = rint(x * 2^(30 - e)) with 2^(e-1) <= max|x| < 2^e over the
//     group (|X| <= 2^30; error at most 2^(e - 31), i.e. 2^-30 of the group's largest |x|), written as four
//     signed base-256 digits D_0..D_3 (X = sum_d 256^d D_d, each D_d in [-128, 127]: the bytes
//     of (X + 0x80808080) xor 0x80808080);
//   - v_mfma_i32_32x32x32_i8 takes one 32-value group per instruction: its 32 A rows are
//     (row, digit) pairs, 8 rows x 4 digits, and the B operand is the packed nibbles with
//     each nibble moved to the top of a byte, i.e. 16 v as int8 (two VALU ops per packed
//     word). Each result S_d = sum_k D_d * 16 v is an exact int32 (|S_d| <= 2^19);
//   - the group is folded into a float64 accumulator per output: C = 65536 (S_2 + 256 S_3)
//     + (S_0 + 256 S_1) is exact in double (|C| < 2^44) and y += C * s * 2^(e - 34) rounds
//     once per group in double. No fp32 rounding touches a group sum, so the error does not
//     grow with K the way an fp32 group sum's does.
// Work mapping: a workgroup owns 8 rows x 32 columns (one MFMA tile; lane l of the result
// holds column l % 32, rows 2i + l / 32 for i < 4) and its wavefronts split K; their float64
// accumulators are summed through LDS in wavefront order (deterministic). Per wavefront, x,
// packed weights and scales reach LDS by buffer loads to LDS in chunks of 4 groups, three
// chunks in flight; lane (row r, half h, quarter q) recodes 4 values of a group and writes
// the digits over the group's 1 KiB of staged x, in the layout the MFMA lanes read.
// Rows holding an infinity or a NaN are flagged while recoding and their outputs formed in
// IEEE double arithmetic over the non-finite terms, which is the double reference's result
// for such rows (test_q4gemm.cpp:102-119).
#include <type_traits>

#include "q4_device.hpp"
#include "q4_kernels.hpp"
#include "q4_lora.hpp"

namespace spaceslug {
namespace {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void* lds_ptr;

constexpr int kDigitRows = 8;        // rows of x per MFMA row block (x 4 digits = 32 A rows)
constexpr int kDigitCols = 32;       // columns per MFMA tile
constexpr int kDigitFracBits = 30;   // |X| <= 2^30
constexpr uint32_t kDigitBias = 0x80808080u;
constexpr int kChunk = 2;            // groups per staged chunk
constexpr int kXBytes = kChunk * kDigitRows * 128;  // x of a chunk: [group][row][32 floats] (2 KiB)
constexpr int kBBytes = kDigitCols * kChunk * 16;   // packed weights: [column][2 groups][16 B] (1 KiB)
constexpr int kSBytes = kDigitCols * kChunk * 4;    // scales: [column][2 groups] (256 B)
constexpr int kBOff = kXBytes, kSOff = kBOff + kBBytes;
constexpr int kStageBytes = kSOff + kSBytes;
constexpr int kStages = 3;           // chunks in flight per wavefront
constexpr int kBufferWord3 = 0x00020000;            // buffer resource word 3: 32-bit data format

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0,
                                             static_cast<int>(bytes < 0x7FFFFFFF ? bytes : 0x7FFFFFFF), kBufferWord3);
}

// A buffer load into LDS (each lane's BYTES bytes land at lds + lane * BYTES), written as
// assembly so the compiler neither counts it nor inserts waits for it: the kernel below issues
// only these in its main loop and waits for them itself, by exact vmcnt counts. (The compiler's
// own tracking of copies into LDS waits for all of them before any LDS read, which would stall
// every chunk behind the copies of the next.) The copy takes its LDS address from M0, which it
// saves and restores.
template <int BYTES>
__device__ __forceinline__ void copy_to_lds(__amdgpu_buffer_rsrc_t rsrc, uint32_t voffset, uint32_t soffset,
                                            unsigned char* lds) {
    // the LDS address and the scalar offset are wavefront-uniform; readfirstlane states it
    const uint32_t l = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(lds_ptr)lds);
    soffset = __builtin_amdgcn_readfirstlane(soffset);
    uint32_t saved;
    if constexpr (BYTES == 16)
        asm volatile(
            "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %4\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds\n\t"
            "s_nop 0\n\ts_mov_b32 m0, %0"
            : "=&s"(saved)
            : "v"(voffset), "s"(rsrc), "s"(soffset), "s"(l)
            : "memory");
    else
        asm volatile(
            "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %4\n\ts_nop 0\n\tbuffer_load_dword %1, %2, %3 offen lds\n\t"
            "s_nop 0\n\ts_mov_b32 m0, %0"
            : "=&s"(saved)
            : "v"(voffset), "s"(rsrc), "s"(soffset), "s"(l)
            : "memory");
}

// Byte selectors of a 4 x 4 byte transpose whose outputs come in the order s ^ r.
struct TransposeSel {
    uint32_t even, odd, lo, hi;
    __device__ explicit TransposeSel(int r)
        : even((r & 1) ? 0x07030501u : 0x06020400u), odd((r & 1) ? 0x06020400u : 0x07030501u),
          lo((r & 2) ? 0x07060302u : 0x05040100u), hi((r & 2) ? 0x05040100u : 0x07060302u) {}
};

// 4 x 4 byte transpose: byte i of o[s] = byte s ^ r of in[i]. With r = 0 the first level pairs
// bytes 0, 2 (even) and 1, 3 (odd) of a, b and of c, e, the second joins the low or high halves:
// o[0] = a0 b0 c0 e0, o[1] = a1 b1 c1 e1, ...; odd r swaps the first level's roles, r >= 2 the
// second's.
__device__ __forceinline__ void transpose_bytes(uint32_t a, uint32_t b, uint32_t c, uint32_t e,
                                                const TransposeSel& sel, uint32_t (&o)[4]) {
    const uint32_t t0 = __builtin_amdgcn_perm(b, a, sel.even);
    const uint32_t t1 = __builtin_amdgcn_perm(b, a, sel.odd);
    const uint32_t t2 = __builtin_amdgcn_perm(e, c, sel.even);
    const uint32_t t3 = __builtin_amdgcn_perm(e, c, sel.odd);
    o[0] = __builtin_amdgcn_perm(t2, t0, sel.lo);
    o[1] = __builtin_amdgcn_perm(t3, t1, sel.lo);
    o[2] = __builtin_amdgcn_perm(t2, t0, sel.hi);
    o[3] = __builtin_amdgcn_perm(t3, t1, sel.hi);
}

// K slot order shared by the A (digits) and B (weights) operands: in the 16 bytes a lane feeds
// for half h of a group, dword q byte i is k = 16 h + 8 (q >> 1) + 2 i + (q & 1). That is the
// order in which the weight decode below leaves the nibbles of packed words 2h and 2h + 1
// (dword 0: even k of word 2h, dword 1: odd k of word 2h, dwords 2, 3: the same of word 2h + 1).
__device__ __forceinline__ i32x4 weights_i8x16(uint32_t w0, uint32_t w1) {
    return i32x4{static_cast<int>((w0 << 4) & 0xF0F0F0F0u), static_cast<int>(w0 & 0xF0F0F0F0u),
                 static_cast<int>((w1 << 4) & 0xF0F0F0F0u), static_cast<int>(w1 & 0xF0F0F0F0u)};
}

// Exponent slot of local row ml within a group: [h = ml & 1][i = ml >> 1], so the lanes of
// result half h read their four rows 2 i + h as one 16-byte word.
__device__ __forceinline__ int exp_slot(int ml) { return (ml & 1) * 4 + (ml >> 1); }

// Nearest integer of v, halves rounded up (floor(v + 0.5) in one conversion, exact for every float);
// an infinity or a NaN converts to a clamped value without trapping. |v| <= 2^30 here.
__device__ __forceinline__ int round_half_up(float v) {
    int r;
    asm("v_cvt_rpi_i32_f32 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

// LoRA preparation launch of a small-batch call: the T partials only (lora_t_block).
__global__ __launch_bounds__(256) void small_lora_prep_kernel(const float* __restrict__ x, const float* __restrict__ la,
                                                              float* __restrict__ tpart, int M, int K, int R,
                                                              int tiles_m_t, int tiles_r) {
    const int b = static_cast<int>(blockIdx.x);
    lora_t_block(x, la, tpart, M, K, R, b % tiles_m_t, (b / tiles_m_t) % tiles_r, b / (tiles_m_t * tiles_r));
}

// Output of row m, column n of a row holding an infinity or a NaN: the IEEE double sum of its
// non-finite terms x * (v * s), formed as the reference forms each term. Every such row's outputs
// are infinite or NaN and finite terms cannot change that, so this is the reference's value.
// Written for clarity: it runs only for non-finite input.
__device__ float ieee_row_value(const float* x, const uint32_t* wq, const float* ws, int m, int n, int K) {
    const int G = K >> 5;
    double acc = 0.0;
    for (int k = 0; k < K; ++k) {
        const float xv = x[static_cast<size_t>(m) * K + k];
        if (__builtin_isfinite(xv)) continue;
        const int g = k >> 5;
        const double s = static_cast<double>(ws[static_cast<size_t>(n) * G + g]);
        const uint32_t word = wq[(static_cast<size_t>(n) * G + g) * 4 + ((k >> 3) & 3)];
        const int v = static_cast<int>(word << (28 - 4 * (k & 7))) >> 28;
        acc += static_cast<double>(xv) * (static_cast<double>(v) * s);
    }
    return static_cast<float>(acc);
}

// NI: output register pairs per lane in use (rows 2 i + h, i < NI): 1 for M <= 2, 2 for M <= 4,
// else 4. W: wavefronts per workgroup, splitting K. Every variant keeps four wavefronts per SIMD
// resident (at most 128 VGPRs and 40 KiB of LDS per wavefront), which hides the recoding's
// dependent chains.
template <int NI, int W>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(4))) void q4_gemm_small_kernel(const float* x, const uint32_t* wq, const float* ws,
                                                               float* __restrict__ y, int M, int N, int K, int RB,
                                                               int tiles_n, const float* __restrict__ tpart,
                                                               int t_splits, const float* __restrict__ lb, int R,
                                                               float lscale) {
    __shared__ __align__(16) unsigned char stages[kStages * W * kStageBytes];
    __shared__ __align__(16) int exps[W * kChunk * kDigitRows];
    __shared__ int rowmask;
    static_assert(W * NI * 64 * 8 <= W * kStageBytes, "epilogue partials fit stage 0");
    static_assert((kDigitRows + kDigitCols) * kMaxLoraRank * 4 <= W * kStageBytes, "LoRA staging fits stage 1");
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int c = lane & 31;  // result column of this lane
    const int h = lane >> 5;  // result half: rows 2i + h
    const int G = K >> 5;

    // Tile order: consecutive ids on one XCD (workgroup i runs on XCD i % 8) cover a contiguous
    // run of (row block, column tile) pairs, row block fastest, so the row blocks that share a
    // column tile share its weights in one L2.
    int lin = static_cast<int>(blockIdx.x);
    const int total = RB * tiles_n;
    if (total >= 64 && (total & 7) == 0) lin = (lin & 7) * (total >> 3) + (lin >> 3);
    const int rb = lin % RB;
    const int n0 = (lin / RB) * kDigitCols;
    const int m0 = rb * kDigitRows;
    if (threadIdx.x == 0) rowmask = 0;
    __syncthreads();

    // The workgroup's K range in chunks of kChunk groups, dealt to its wavefronts in turn (wave w
    // takes chunks w, w + W, ...): at any moment the wavefronts read neighbouring chunks, so each
    // column's weights are read as one run rather than W scattered pieces.
    const int nct = (G + kChunk - 1) / kChunk;
    const int nchunks = nct > w ? (nct - w + W - 1) / W : 0;
    auto chunk_group = [&](int j) { return (w + j * W) * kChunk; };

    // Every copy goes through a buffer resource with a uniform base: the lane's part is a fixed
    // 32-bit offset and the chunk's position a scalar offset, so issuing costs no vector ALU work,
    // and a read past a resource's end returns zeros (rows past M, columns past N).
    //   x: instruction gi moves group gi of the chunk for the block's 8 rows (lane i: row i / 8,
    //   16 bytes at i % 8), one 128-byte run per row.
    //   Weights: one instruction moves the tile's 32 columns, 32 bytes (the chunk's 2 groups)
    //   each; lane i takes column i / 2 and group slot (i % 2) ^ f(column), f(c) = (c >> 3) & 1,
    //   so that the MFMA-side reads (lane (c, h) reads group h of column c) hit 16 distinct
    //   16-byte bank groups per 16 lanes.
    //   Scales: one instruction moves the 2 scales of each column, lane i column i / 2.
    const __amdgpu_buffer_rsrc_t rx =
        make_rsrc(x + static_cast<size_t>(m0) * K, static_cast<size_t>(M - m0) * K * 4);
    // x placement: the 16-byte unit at slot q of row r's 128 bytes holds the row's unit
    // q ^ xsw(r), xsw(r) = (r >> 1) & 1, so that the recoding reads below (rows 0-3 and 4-7 in
    // the two halves of the wavefront, even or odd units per instruction) meet distinct banks.
    const uint32_t vx = static_cast<uint32_t>((lane >> 3) * K * 4 + ((lane & 7) ^ ((lane >> 4) & 1)) * 16);
    const int ci = lane >> 1;
    const int gs = lane & 1;
    const size_t left = static_cast<size_t>(N - n0) * G;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(wq + static_cast<size_t>(n0) * G * 4, left * 16);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(ws + static_cast<size_t>(n0) * G, left * 4);
    const uint32_t vw = static_cast<uint32_t>((ci * G + (gs ^ ((ci >> 3) & 1))) * 16);
    const uint32_t vs = static_cast<uint32_t>((ci * G + gs) * 4);
    const int bsw = (c >> 3) & 1;  // swizzle of this lane's column

    // A chunk's copies: x (kChunk of them), then weights and scales (2).
    static_assert(kChunk == 2, "copy counts and the partial chunk assume two groups per chunk");
    auto issue_x = [&](int cb, unsigned char* st) {
#pragma unroll
        for (int gi = 0; gi < kChunk; ++gi)
            copy_to_lds<16>(rx, vx, static_cast<uint32_t>((cb + gi) * 128), st + gi * 1024);
    };
    auto issue_ws = [&](int cb, unsigned char* st) {
        copy_to_lds<16>(rw, vw, static_cast<uint32_t>(cb * 16), st + kBOff);
        copy_to_lds<4>(rs, vs, static_cast<uint32_t>(cb * 4), st + kSOff);
    };

    // Recoding roles: lane (row rr = lane / 8, half rh = (lane / 4) % 2, quarter rq = lane % 4)
    // takes the 4 values of K-slot dword rq of half rh of its row, k = 16 rh + 8 (rq >> 1) +
    // (rq & 1) + 2 i, so its byte-transposed digits are exactly dword rq of the four A lanes
    // (row rr, digit d, half rh); the 8 lanes of a row hold its whole group.
    const int rr = lane >> 3, rh = (lane >> 2) & 1, rq = lane & 3;
    const int xq0 = 4 * rh + 2 * (rq >> 1), xsw = (rr >> 1) & 1;  // units xq0, xq0 + 1 of the row
    const int xoff0 = rr * 128 + (xq0 ^ xsw) * 16 + (rq & 1) * 4;
    const int xoff1 = rr * 128 + ((xq0 + 1) ^ xsw) * 16 + (rq & 1) * 4;
    // Digit writes: lane (row rr, half rh, quarter rq) writes digit d to dword rq of A lane
    // 32 rh + 4 rr + d. Its four writes go out in the order s ^ dr, dr = 2 rh + rr / 4, so that
    // each write instruction meets 64 distinct banks.
    const TransposeSel tsel(2 * rh + (rr >> 2));
    int wofs[4];
#pragma unroll
    for (int sl = 0; sl < 4; ++sl) wofs[sl] = ((32 * rh + 4 * rr + (sl ^ (2 * rh + (rr >> 2)))) * 4 + rq) * 4;
    int* xexp = exps + w * kChunk * kDigitRows;

    double acc[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) acc[i] = 0.0;

    // Recodes groups g0 .. g0 + NG - 1 of the chunk in stage st, in phases over the groups so that
    // their chains interleave: each group's digits are written over its x (a wavefront's LDS
    // operations run in order, so every lane's reads of a group precede the writes) and its
    // exponents (e - 34) go to xexp[group][exp_slot(row)]. Branch-free; a non-finite value only
    // raises mbrun, the lane's largest magnitude bits, which flags its row once the loop is done
    // (its digits and exponents are then never used).
    uint32_t mbrun = 0;
    auto recode = [&](const unsigned char* st, int g0, auto ng) {
        constexpr int NG = decltype(ng)::value;
        float vv[NG][4];
        uint32_t mb[NG];
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            const float* xs0 = reinterpret_cast<const float*>(st + (g0 + g) * 1024 + xoff0);
            const float* xs1 = reinterpret_cast<const float*>(st + (g0 + g) * 1024 + xoff1);
            vv[g][0] = xs0[0];
            vv[g][1] = xs0[2];
            vv[g][2] = xs1[0];
            vv[g][3] = xs1[2];
        }
        // largest magnitude as an integer maximum of the sign-cleared bits (every non-finite value,
        // 0x7F800000 and above, lands at the top); the row's 8 lanes combine theirs (quad pairs,
        // then the two quads)
#pragma unroll
        for (int g = 0; g < NG; ++g)
            mb[g] = max(max(__float_as_uint(vv[g][0]) & 0x7FFFFFFFu, __float_as_uint(vv[g][1]) & 0x7FFFFFFFu),
                        max(__float_as_uint(vv[g][2]) & 0x7FFFFFFFu, __float_as_uint(vv[g][3]) & 0x7FFFFFFFu));
#pragma unroll
        for (int g = 0; g < NG; ++g)
            mb[g] = max(mb[g], static_cast<uint32_t>(
                                   __builtin_amdgcn_update_dpp(0, static_cast<int>(mb[g]), 0xB1, 0xF, 0xF, false)));
#pragma unroll
        for (int g = 0; g < NG; ++g)
            mb[g] = max(mb[g], static_cast<uint32_t>(
                                   __builtin_amdgcn_update_dpp(0, static_cast<int>(mb[g]), 0x4E, 0xF, 0xF, false)));
#pragma unroll
        for (int g = 0; g < NG; ++g)
            mb[g] = max(mb[g], static_cast<uint32_t>(
                                   __builtin_amdgcn_update_dpp(0, static_cast<int>(mb[g]), 0x141, 0xF, 0xF, false)));
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            mbrun = max(mbrun, mb[g]);
            const int e = __builtin_amdgcn_frexp_expf(__uint_as_float(mb[g]));  // max < 2^e (0: all-zero group)
            const int sh = kDigitFracBits - e;
            uint32_t z[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                z[i] = (static_cast<uint32_t>(round_half_up(ldexpf(vv[g][i], sh))) + kDigitBias) ^ kDigitBias;
            uint32_t t[4];
            transpose_bytes(z[0], z[1], z[2], z[3], tsel, t);  // t[sl]: digit sl ^ dr of the 4 values
            unsigned char* xw = const_cast<unsigned char*>(st) + (g0 + g) * 1024;
#pragma unroll
            for (int sl = 0; sl < 4; ++sl) *reinterpret_cast<uint32_t*>(xw + wofs[sl]) = t[sl];
            xexp[(g0 + g) * 8 + exp_slot(rr)] = e - 34;  // the row's 8 lanes store the same value
        }
    };
    // A lane (row, digit, half) = lane 32 half + 4 row + digit reads its 16 bytes of group gi.
    auto digits = [&](const unsigned char* st, int gi) {
        return *reinterpret_cast<const i32x4*>(st + gi * 1024 + lane * 16);
    };

    auto fold = [&](const i32x16& r, float sf, const i32x4& e4) {
        const double sd = static_cast<double>(sf);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int lo = r[4 * i] + (r[4 * i + 1] << 8);
            const int hi = r[4 * i + 2] + (r[4 * i + 3] << 8);
            const double cg = fma(static_cast<double>(hi), 65536.0, static_cast<double>(lo));
            acc[i] = fma(cg, ldexp(sd, e4[i]), acc[i]);
        }
    };

    // Recodes the chunk at group cb (its groups in the K range) in stage st.
    auto recode_chunk = [&](int cb, const unsigned char* st) {
        if (G - cb >= kChunk)
            recode(st, 0, std::integral_constant<int, kChunk>{});
        else
            recode(st, 0, std::integral_constant<int, 1>{});
    };
    // The chunk's MFMAs and folds; the MFMA of group 1 is issued before group 0's fold.
    auto mfma_chunk = [&](int cb, const unsigned char* st) {
        const f32x2 s2 = *reinterpret_cast<const f32x2*>(st + kSOff + c * 8);
        // B operands: lane (c, 0) reads group 0, lane (c, 1) group 1, and the swaps leave lane
        // (c, h) with packed words 2h and 2h + 1 of both groups.
        const u32x4 wv = *reinterpret_cast<const u32x4*>(st + kBOff + 32 * c + 16 * (h ^ bsw));
        const auto x0 = __builtin_amdgcn_permlane32_swap(wv[0], wv[2], false, false);
        const auto x1 = __builtin_amdgcn_permlane32_swap(wv[1], wv[3], false, false);
        const i32x16 zero = {};
        const i32x4 a0 = digits(st, 0);
        const i32x4 e0 = *reinterpret_cast<const i32x4*>(xexp + h * 4);
        const i32x16 r0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, weights_i8x16(x0[0], x1[0]), zero, 0, 0, 0);
        if (G - cb >= kChunk) {
            const i32x4 a1 = digits(st, 1);
            const i32x4 e1 = *reinterpret_cast<const i32x4*>(xexp + 8 + h * 4);
            const i32x16 r1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, weights_i8x16(x0[1], x1[1]), zero, 0, 0, 0);
            fold(r0, s2[0], e0);
            fold(r1, s2[1], e1);
        } else {
            fold(r0, s2[0], e0);
        }
    };

    // Chunk j is staged in stage j % 3 of this wavefront and its copies are issued two chunks
    // ahead, so up to three chunks are in flight. Copies retire in issue order: leaving the copies
    // of the chunks issued after chunk j in flight is chunk j's wait. The loop is unrolled by the
    // stage count so that every LDS address is a fixed offset from the wavefront's stages.
    constexpr int kCopiesPerChunk = kChunk + 2;
    unsigned char* wst = stages + w * kStages * kStageBytes;
    auto issue = [&](int j, unsigned char* st) {
        issue_x(chunk_group(j), st);
        issue_ws(chunk_group(j), st);
    };
    auto step = [&](int j, unsigned char* st, unsigned char* st_ahead) {
        if (j + 2 < nchunks) {
            // the stage of chunk j + 2 last held chunk j - 1: its reads and digit writes are done
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            issue(j + 2, st_ahead);
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * kCopiesPerChunk) : "memory");
        } else if (j + 1 < nchunks) {
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kCopiesPerChunk) : "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        const int cb = chunk_group(j);
        recode_chunk(cb, st);
        mfma_chunk(cb, st);
    };
    if (nchunks > 0) issue(0, wst);
    if (nchunks > 1) issue(1, wst + kStageBytes);
    for (int j = 0; j < nchunks; j += kStages) {
        step(j, wst, wst + 2 * kStageBytes);
        if (j + 1 < nchunks) step(j + 1, wst + kStageBytes, wst);
        if (j + 2 < nchunks) step(j + 2, wst + 2 * kStageBytes, wst + kStageBytes);
    }

    if (mbrun >= 0x7F800000u) atomicOr(&rowmask, 1 << rr);  // rare: a row with an infinity or a NaN
    __syncthreads();  // every wavefront's K range is done: the stages are free
    double* red = reinterpret_cast<double*>(stages);
    float* lora_t_s = reinterpret_cast<float*>(stages + W * kStageBytes);  // [8 rows][R]
    float* lora_b_s = lora_t_s + kDigitRows * kMaxLoraRank;  // [R][32 columns]
#pragma unroll
    for (int i = 0; i < NI; ++i) red[(w * NI + i) * 64 + lane] = acc[i];
    if (lb != nullptr) {
        // T (8 rows) and lb (32 columns): every load of a pass issued before the first store.
        constexpr int kNV = 2;
        for (int e0 = static_cast<int>(threadIdx.x); e0 < R * kDigitCols; e0 += 64 * W * kNV) {
            float tv[kNV], bv[kNV];
#pragma unroll
            for (int v = 0; v < kNV; ++v) {
                const int e = e0 + 64 * W * v;
                bv[v] = lb[static_cast<size_t>(min(e >> 5, R - 1)) * N + min(n0 + (e & 31), N - 1)];  // in bounds
            }
            lora_t_values<kNV>(tpart, t_splits, M, R, 0, R, m0, e0, 64 * W, kDigitRows * R, tv);
#pragma unroll
            for (int v = 0; v < kNV; ++v) {
                const int e = e0 + 64 * W * v;
                if (e < kDigitRows * R) lora_t_s[e] = tv[v];
                if (e < R * kDigitCols) lora_b_s[e] = bv[v];
            }
        }
    }
    __syncthreads();
    const int t = static_cast<int>(threadIdx.x);
    if (t < kDigitRows * kDigitCols) {
        const int ml = t >> 5, cc = t & 31;
        const int m = m0 + ml, n = n0 + cc;
        if (m < M && n < N) {
            const int i = ml >> 1, hh = ml & 1;
            double s = 0.0;
            if (i < NI) {
#pragma unroll
                for (int v = 0; v < W; ++v) s += red[(v * NI + i) * 64 + cc + 32 * hh];
            }
            if ((rowmask >> ml) & 1) s = ieee_row_value(x, wq, ws, m, n, K);
            if (lb != nullptr) {
                double tb = 0.0;
#pragma unroll 8
                for (int r = 0; r < R; ++r)
                    tb = fma(static_cast<double>(lora_t_s[ml * R + r]), static_cast<double>(lora_b_s[r * 32 + cc]), tb);
                s = fma(static_cast<double>(lscale), tb, s);
            }
            y[static_cast<size_t>(m) * N + n] = static_cast<float>(s);
        }
    }
}

template <int NI, int W>
hipError_t launch_small_gemm(const float* x, const uint8_t* w_packed, const float* w_scales, float* y, int m, int n,
                             int k, int RB, int tiles_n, const float* tpart, int t_splits, const float* lb, int rank,
                             float lscale, hipStream_t stream) {
    hipLaunchKernelGGL((q4_gemm_small_kernel<NI, W>), dim3(static_cast<unsigned>(RB * tiles_n)), dim3(64 * W), 0,
                       stream, x, reinterpret_cast<const uint32_t*>(w_packed), w_scales, y, m, n, k, RB, tiles_n,
                       tpart, t_splits, lb, rank, lscale);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_q4gemm_small(const DeviceInfo& dev, const float* x, const uint8_t* w_packed, const float* w_scales,
                               float* y, uint32_t m, uint32_t n, uint32_t k, const float* la, const float* lb,
                               uint32_t rank, float lora_scale, int t_splits, void* workspace, hipStream_t stream) {
    const int M = static_cast<int>(m), N = static_cast<int>(n), K = static_cast<int>(k);
    const int RB = (M + kDigitRows - 1) / kDigitRows;
    const int R = static_cast<int>(rank);
    float* tpart = nullptr;
    if (rank) {
        tpart = static_cast<float*>(workspace);
        const int tiles_m_t = (M + 15) / 16, tiles_r = (R + 15) / 16;
        hipLaunchKernelGGL(small_lora_prep_kernel, dim3(static_cast<unsigned>(tiles_m_t * tiles_r * t_splits)),
                           dim3(256), 0, stream, x, la, tpart, M, K, R, tiles_m_t, tiles_r);
        const hipError_t pe = hipGetLastError();
        if (pe != hipSuccess) return pe;
    }
    const int tiles_n = (N + kDigitCols - 1) / kDigitCols;
    // Wavefronts per workgroup: 16 per CU in total, whether one, two or four workgroups share a CU.
    const int total = RB * tiles_n;
    const int W = total <= dev.cu_count ? 16 : total <= 2 * dev.cu_count ? 8 : 4;
    const int NI = M <= 2 ? 1 : M <= 4 ? 2 : 4;
    const float* lbp = rank ? lb : nullptr;
    auto go = [&](auto ni, auto wv) {
        return launch_small_gemm<decltype(ni)::value, decltype(wv)::value>(x, w_packed, w_scales, y, M, N, K, RB,
                                                                           tiles_n, tpart, t_splits, lbp, R,
                                                                           lora_scale, stream);
    };
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I4 = std::integral_constant<int, 4>;
    using W16 = std::integral_constant<int, 16>;
    using W8 = std::integral_constant<int, 8>;
    if (NI == 1) return W == 16 ? go(I1{}, W16{}) : W == 8 ? go(I1{}, W8{}) : go(I1{}, I4{});
    if (NI == 2) return W == 16 ? go(I2{}, W16{}) : W == 8 ? go(I2{}, W8{}) : go(I2{}, I4{});
    return W == 16 ? go(I4{}, W16{}) : W == 8 ? go(I4{}, W8{}) : go(I4{}, I4{});
}

}  // namespace spaceslug
