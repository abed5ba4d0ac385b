// Exact small-batch int4 GEMM: M <= 32 rows (and one row with K > 4096), any K % 32 == 0.
//
// Replaces q4gemm.comp:61-175 for decode-sized batches. Every 32-value group sum
// sum_k x[m][k] * v[k][n] is formed exactly, in integers, on the int8 matrix cores, in one
// launch with no device memory beyond the arguments (a LoRA call adds the T = x * la
// partials of a preparation launch):
//   - each wavefront recodes the groups of x it consumes, per row and 32-value group, in
//     31-bit fixed point: X = rint(x * 2^(30 - e)) with 2^(e-1) <= max|x| < 2^e over the
//     group (|X| <= 2^30; error at most 2^-31 of the group's largest |x|), written as four
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
// packed weights and scales reach LDS by buffer loads to LDS in chunks of 4 groups, two
// chunks in flight; lane (row r, half h, quarter q) recodes 4 values of a group and the
// digits reach the MFMA lanes through a 1 KiB LDS exchange.
// Rows holding an infinity or a NaN are flagged while recoding and their outputs formed in
// IEEE double arithmetic over the non-finite terms, which is the double reference's result
// for such rows (test_q4gemm.cpp:102-119).
#include <climits>

#include "q4_device.hpp"
#include "q4_kernels.hpp"
#include "q4_lora.hpp"

namespace spaceslug {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void* lds_ptr;

constexpr int kDigitRows = 8;        // rows of x per MFMA row block (x 4 digits = 32 A rows)
constexpr int kDigitCols = 32;       // columns per MFMA tile
constexpr int kDigitFracBits = 30;   // |X| <= 2^30
constexpr uint32_t kDigitBias = 0x80808080u;
constexpr int kExpNonFinite = INT_MIN;
constexpr int kChunk = 4;            // groups per staged chunk
constexpr int kXBytes = kChunk * kDigitRows * 128;  // x of a chunk: [group][row][32 floats] (4 KiB)
constexpr int kBBytes = kDigitCols * kChunk * 16;   // packed weights (2 KiB)
constexpr int kSBytes = kDigitCols * kChunk * 4;    // scales (512 B)
constexpr int kBOff = kXBytes, kSOff = kBOff + kBBytes;
constexpr int kStageBytes = kSOff + kSBytes;
constexpr int kXchgBytes = kChunk * 64 * 16;        // digit exchange of a chunk's groups
constexpr int kExpBytes = kChunk * kDigitRows * 4;  // exponents of a chunk's groups
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
    const uint32_t l = (uint32_t)(size_t)(lds_ptr)lds;  // the LDS address
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

// 4 x 4 byte transpose: byte i of o[d] = byte d of in[i].
__device__ __forceinline__ void transpose_bytes(uint32_t a, uint32_t b, uint32_t c, uint32_t e, uint32_t (&o)[4]) {
    const uint32_t t0 = __builtin_amdgcn_perm(b, a, 0x06020400u);  // a0 b0 a2 b2
    const uint32_t t1 = __builtin_amdgcn_perm(b, a, 0x07030501u);  // a1 b1 a3 b3
    const uint32_t t2 = __builtin_amdgcn_perm(e, c, 0x06020400u);  // c0 e0 c2 e2
    const uint32_t t3 = __builtin_amdgcn_perm(e, c, 0x07030501u);  // c1 e1 c3 e3
    o[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);              // a0 b0 c0 e0
    o[1] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);              // a1 b1 c1 e1
    o[2] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);              // a2 b2 c2 e2
    o[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);              // a3 b3 c3 e3
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
// else 4. W: wavefronts per workgroup, splitting K.
template <int NI, int W>
__global__ __launch_bounds__(64 * W) void q4_gemm_small_kernel(const float* x, const uint32_t* wq, const float* ws,
                                                               float* __restrict__ y, int M, int N, int K, int RB,
                                                               int tiles_n, const float* __restrict__ tpart,
                                                               int t_splits, const float* __restrict__ lb, int R,
                                                               float lscale) {
    __shared__ __align__(16) unsigned char stage0[W * kStageBytes];
    __shared__ __align__(16) unsigned char stage1[W * kStageBytes];
    __shared__ __align__(16) unsigned char xchg[W * (kXchgBytes + kExpBytes)];
    __shared__ int rowmask;
    static_assert(W * NI * 64 * 8 <= W * kStageBytes, "epilogue partials fit stage0");
    static_assert((kDigitRows + kDigitCols) * kMaxLoraRank * 4 <= W * kStageBytes, "LoRA staging fits stage1");
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

    // This wavefront's groups [gb, ge), in chunks of kChunk.
    const int gpw = (G + W - 1) / W;
    const int gb = min(G, w * gpw);
    const int ge = min(G, gb + gpw);
    const int nchunks = (ge - gb + kChunk - 1) / kChunk;

    // Every copy goes through a buffer resource with a uniform base: the lane's part is a fixed
    // 32-bit offset and the chunk's position a scalar offset, so issuing costs no vector ALU work,
    // and a read past a resource's end returns zeros (rows past M, columns past N).
    //   x: instruction gi moves group gi of the chunk for the block's 8 rows (lane i: row i / 8,
    //   16 bytes at i % 8), one 128-byte run per row.
    //   Weights: instruction p moves columns 16p .. 16p+15 of the tile, 64 bytes (the chunk's 4
    //   groups) each; lane i takes column 16p + i / 4 and group slot (i % 4) ^ f(column),
    //   f(c) = (c >> 2) & 3, so that the MFMA-side reads (lane (c, h) reads one group of column c)
    //   hit 16 distinct 16-byte bank groups per 16 lanes.
    //   Scales: instruction p moves the 4 scales of the same columns.
    const __amdgpu_buffer_rsrc_t rx =
        make_rsrc(x + static_cast<size_t>(m0) * K, static_cast<size_t>(M - m0) * K * 4);
    const uint32_t vx = static_cast<uint32_t>((lane >> 3) * K * 4 + (lane & 7) * 16);
    const int ci = lane >> 2;
    const int gs = lane & 3;
    __amdgpu_buffer_rsrc_t rw[2], rs[2];
    uint32_t vw[2], vs[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const int col0 = min(n0 + 16 * p, N);
        const size_t left = static_cast<size_t>(N - col0) * G;
        rw[p] = make_rsrc(wq + static_cast<size_t>(col0) * G * 4, left * 16);
        rs[p] = make_rsrc(ws + static_cast<size_t>(col0) * G, left * 4);
        vw[p] = static_cast<uint32_t>((ci * G + (gs ^ (((16 * p + ci) >> 2) & 3))) * 16);
        vs[p] = static_cast<uint32_t>((ci * G + gs) * 4);
    }
    const int fsw = (c >> 2) & 3;  // swizzle of this lane's column

    // The 8 copies of a chunk (counted by the waits below).
    constexpr int kCopiesPerChunk = kChunk + 2 + 2;
    auto issue = [&](int cb, unsigned char* st) {
#pragma unroll
        for (int gi = 0; gi < kChunk; ++gi)
            copy_to_lds<16>(rx, vx, static_cast<uint32_t>((cb + gi) * 128), st + gi * 1024);
#pragma unroll
        for (int p = 0; p < 2; ++p) copy_to_lds<16>(rw[p], vw[p], static_cast<uint32_t>(cb * 16), st + kBOff + p * 1024);
#pragma unroll
        for (int p = 0; p < 2; ++p) copy_to_lds<4>(rs[p], vs[p], static_cast<uint32_t>(cb * 4), st + kSOff + p * 256);
    };

    // Recoding roles: lane (row rr = lane / 8, half rh = (lane / 4) % 2, quarter rq = lane % 4)
    // takes the 4 values of K-slot dword rq of half rh of its row, k = 16 rh + 8 (rq >> 1) +
    // (rq & 1) + 2 i, so its byte-transposed digits are exactly dword rq of the four A lanes
    // (row rr, digit d, half rh); the 8 lanes of a row hold its whole group.
    const int rr = lane >> 3, rh = (lane >> 2) & 1, rq = lane & 3;
    const int xoff = rr * 128 + rh * 64 + (rq >> 1) * 32 + (rq & 1) * 4;
    unsigned char* xg = xchg + w * (kXchgBytes + kExpBytes);
    int* xexp = reinterpret_cast<int*>(xg + kXchgBytes);

    double acc[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) acc[i] = 0.0;

    // Recodes group gi of the chunk in stage st into exchange slot gi; the group's exponents
    // (e - 34, or INT_MIN with a non-finite value) go to xexp[gi][exp_slot(row)].
    auto recode = [&](const unsigned char* st, int gi) {
        const float* xs = reinterpret_cast<const float*>(st + gi * 1024 + xoff);
        const float v0 = xs[0], v1 = xs[2], v2 = xs[4], v3 = xs[6];
        // largest magnitude as an integer maximum of the sign-cleared bits: every non-finite value
        // (0x7F800000 and above) also lands at the top, so one compare detects it; the row's 8
        // lanes combine theirs (quad pairs, then the two quads)
        uint32_t mb = max(max(__float_as_uint(v0) & 0x7FFFFFFFu, __float_as_uint(v1) & 0x7FFFFFFFu),
                          max(__float_as_uint(v2) & 0x7FFFFFFFu, __float_as_uint(v3) & 0x7FFFFFFFu));
        mb = max(mb, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mb), 0xB1, 0xF, 0xF, false)));
        mb = max(mb, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mb), 0x4E, 0xF, 0xF, false)));
        mb = max(mb, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mb), 0x141, 0xF, 0xF, false)));
        const bool finite = mb < 0x7F800000u;
        int e = 0;
        (void)frexpf(__uint_as_float(mb), &e);  // max < 2^e (e = 0 for an all-zero group)
        const int sh = kDigitFracBits - e;
        uint32_t z[4];
        const float vv[4] = {v0, v1, v2, v3};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int X = finite ? static_cast<int>(rintf(ldexpf(vv[i], sh))) : 0;
            z[i] = (static_cast<uint32_t>(X) + kDigitBias) ^ kDigitBias;  // byte d = signed digit D_d
        }
        uint32_t t[4];
        transpose_bytes(z[0], z[1], z[2], z[3], t);  // t[d]: digit d of the 4 values = dword rq
        int* xw = reinterpret_cast<int*>(xg + gi * 1024);
#pragma unroll
        for (int d = 0; d < 4; ++d) xw[(32 * rh + 4 * rr + d) * 4 + rq] = static_cast<int>(t[d]);
        if ((lane & 7) == 0) xexp[gi * 8 + exp_slot(rr)] = finite ? e - 34 : kExpNonFinite;
        if (!finite) atomicOr(&rowmask, 1 << rr);  // rare: a row with an infinity or a NaN
    };
    // A lane (row, digit, half) = lane 32 half + 4 row + digit reads its 16 bytes of group gi.
    auto digits = [&](int gi) { return *reinterpret_cast<const i32x4*>(xg + gi * 1024 + lane * 16); };

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

    auto compute = [&](int cb, const unsigned char* st) {
        const f32x4 s4 = *reinterpret_cast<const f32x4*>(st + kSOff + c * 16);
        // B operands: lane (c, 0) reads group 2p, lane (c, 1) group 2p + 1, and the swaps leave
        // lane (c, h) with packed words 2h and 2h + 1 of both groups.
        i32x4 bq[kChunk];
#pragma unroll
        for (int p = 0; p < kChunk / 2; ++p) {
            const u32x4 wv = *reinterpret_cast<const u32x4*>(st + kBOff + 64 * c + 16 * ((2 * p + h) ^ fsw));
            const auto x0 = __builtin_amdgcn_permlane32_swap(wv[0], wv[2], false, false);
            const auto x1 = __builtin_amdgcn_permlane32_swap(wv[1], wv[3], false, false);
            bq[2 * p] = weights_i8x16(x0[0], x1[0]);
            bq[2 * p + 1] = weights_i8x16(x0[1], x1[1]);
        }
        const i32x16 zero = {};
        const int valid = ge - cb;  // groups of this chunk in the wavefront's range (uniform)
        if (valid >= kChunk) {
            // Full chunk, straight-line: the four groups are recoded back to back (independent
            // chains), then the MFMA of group g + 1 is issued before group g's fold.
#pragma unroll
            for (int g = 0; g < kChunk; ++g) recode(st, g);
            i32x4 a[kChunk], e4[kChunk];
#pragma unroll
            for (int g = 0; g < kChunk; ++g) {
                a[g] = digits(g);
                e4[g] = *reinterpret_cast<const i32x4*>(xexp + g * 8 + h * 4);
            }
            i32x16 r = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[0], bq[0], zero, 0, 0, 0);
#pragma unroll
            for (int g = 0; g < kChunk; ++g) {
                i32x16 rn;
                if (g + 1 < kChunk) rn = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[g + 1], bq[g + 1], zero, 0, 0, 0);
                fold(r, s4[g], e4[g]);
                if (g + 1 < kChunk) r = rn;
            }
        } else {
#pragma unroll
            for (int g = 0; g < kChunk; ++g) {
                if (g < valid) {
                    recode(st, g);
                    const i32x16 r = __builtin_amdgcn_mfma_i32_32x32x32_i8(digits(g), bq[g], zero, 0, 0, 0);
                    fold(r, s4[g], *reinterpret_cast<const i32x4*>(xexp + g * 8 + h * 4));
                }
            }
        }
    };

    // Two stages: chunk j in stage j % 2. Chunk j + 1's copies are issued before chunk j is
    // computed; copies retire in issue order, so leaving exactly those in flight is chunk j's wait.
    unsigned char* st0 = stage0 + w * kStageBytes;
    unsigned char* st1 = stage1 + w * kStageBytes;
    if (nchunks > 0) issue(gb, st0);
    for (int j = 0; j < nchunks; j += 2) {
        const int cb = gb + j * kChunk;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // stage 1's previous reads are done
        if (j + 1 < nchunks) {
            issue(cb + kChunk, st1);
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kCopiesPerChunk) : "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        compute(cb, st0);
        if (j + 1 >= nchunks) break;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // stage 0's reads are done
        if (j + 2 < nchunks) {
            issue(cb + 2 * kChunk, st0);
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kCopiesPerChunk) : "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        compute(cb + kChunk, st1);
    }

    __syncthreads();  // every wavefront's K range is done: the stages are free
    double* red = reinterpret_cast<double*>(stage0);
    float* lora_t_s = reinterpret_cast<float*>(stage1);  // [8 rows][R]
    float* lora_b_s = lora_t_s + kDigitRows * kMaxLoraRank;  // [R][32 columns]
#pragma unroll
    for (int i = 0; i < NI; ++i) red[(w * NI + i) * 64 + lane] = acc[i];
    if (lb != nullptr) {
        for (int e = static_cast<int>(threadIdx.x); e < kDigitRows * R; e += 64 * W)
            lora_t_s[e] = lora_t_value(tpart, t_splits, M, R, min(m0 + e / R, M - 1), e % R);
        for (int e = static_cast<int>(threadIdx.x); e < R * kDigitCols; e += 64 * W)
            lora_b_s[e] = lb[static_cast<size_t>(e >> 5) * N + min(n0 + (e & 31), N - 1)];
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
    const bool few = RB * tiles_n <= dev.cu_count;  // one round of workgroups: more wavefronts per tile
    const float* lbp = rank ? lb : nullptr;
    if (M <= 2)
        return few ? launch_small_gemm<1, 8>(x, w_packed, w_scales, y, M, N, K, RB, tiles_n, tpart, t_splits, lbp, R,
                                             lora_scale, stream)
                   : launch_small_gemm<1, 4>(x, w_packed, w_scales, y, M, N, K, RB, tiles_n, tpart, t_splits, lbp, R,
                                             lora_scale, stream);
    if (M <= 4)
        return few ? launch_small_gemm<2, 8>(x, w_packed, w_scales, y, M, N, K, RB, tiles_n, tpart, t_splits, lbp, R,
                                             lora_scale, stream)
                   : launch_small_gemm<2, 4>(x, w_packed, w_scales, y, M, N, K, RB, tiles_n, tpart, t_splits, lbp, R,
                                             lora_scale, stream);
    return few ? launch_small_gemm<4, 8>(x, w_packed, w_scales, y, M, N, K, RB, tiles_n, tpart, t_splits, lbp, R,
                                         lora_scale, stream)
               : launch_small_gemm<4, 4>(x, w_packed, w_scales, y, M, N, K, RB, tiles_n, tpart, t_splits, lbp, R,
                                         lora_scale, stream);
}

}  // namespace spaceslug
