// Exact small-batch int4 GEMM: M <= 32 rows (and one row with K > 4096), any K % 32 == 0.
//
// Replaces q4gemm.comp:61-175 for decode-sized batches. Every 32-value group sum
// sum_k x[m][k] * v[k][n] is formed exactly, in integers, on the int8 matrix cores:
//   - a preparation launch (digits_prep_kernel) writes each group of each row of x in
//     31-bit fixed point, X = rint(x * 2^(30 - e)) with 2^(e-1) <= max|x| < 2^e over the
//     group (|X| <= 2^30, error at most 2^-31 of the group's largest |x|), as four signed
//     base-256 digits D_0..D_3 (X = sum_d 256^d D_d, each D_d in [-128, 127]);
//   - the GEMM feeds v_mfma_i32_32x32x32_i8 with one 32-value group per instruction: the
//     32 A rows of a row block are (row, digit) pairs, 8 rows x 4 digits, and the B operand
//     is the packed nibbles with each nibble moved to the top of a byte, i.e. 16 v as int8
//     (two VALU ops per packed word, no table). Each result S_d = sum_k D_d * 16 v is an
//     exact int32 (|S_d| <= 2^19);
//   - the group is folded into a float64 accumulator per output: C = 65536 (S_2 + 256 S_3)
//     + (S_0 + 256 S_1) is exact in double (|C| < 2^44) and y += C * s * 2^(e - 34) rounds
//     once per group in double. No fp32 rounding touches a group sum, so the error does not
//     grow with K the way an fp32 group sum's does.
// A wavefront's output tile is 8 rows x 32 columns (lane l: column l % 32; rows 2i + l / 32
// for i < 4 in the MFMA result's register pairs); the workgroup's wavefronts split K and
// sum their float64 accumulators through LDS in wavefront order (deterministic). A wavefront
// issues the loads of 16 groups at once: their digits into VGPRs (each group's A operand is
// one contiguous 1 KiB run, laid out by the preparation launch in MFMA lane order), their
// packed weights, scales and exponents into LDS by buffer loads to LDS, whole column runs each.
// Rows holding an infinity or a NaN are flagged by the preparation (exponent INT_MIN) and
// their outputs are formed in IEEE double arithmetic over the non-finite terms, which is
// the double reference's result for such rows (test_q4gemm.cpp:102-119).
#include <climits>

#include "q4_device.hpp"
#include "q4_kernels.hpp"
#include "q4_lora.hpp"

namespace spaceslug {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int kDigitRows = 8;        // rows of x per MFMA row block (x 4 digits = 32 A rows)
constexpr int kDigitCols = 32;       // columns per MFMA tile
constexpr int kDigitFracBits = 30;   // |X| <= 2^30
constexpr uint32_t kDigitBias = 0x80808080u;
constexpr int kExpNonFinite = INT_MIN;
constexpr int kChunk = 4;            // groups per compute step (one LDS read of scales)
constexpr int kSuper = 4 * kChunk;   // groups a wavefront loads at once: digits into VGPRs, the rest into LDS
constexpr int kBBytes = kDigitCols * kSuper * 16;  // packed weights of a super-chunk (8 KiB)
constexpr int kSBytes = kDigitCols * kSuper * 4;   // scales (2 KiB)
constexpr int kEBytes = kSuper * kDigitRows * 4;   // exponents (512 B)
constexpr int kSOff = kBBytes, kEOff = kSOff + kSBytes;
constexpr int kWaveBytes = kEOff + kEBytes;        // LDS per wavefront
constexpr int kBufferWord3 = 0x00020000;           // buffer resource word 3: 32-bit data format

size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

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

// Exponent slot of local row ml within a (row block, group): [h = ml & 1][i = ml >> 1], so the
// lanes of half h read their four rows 2 i + h as one 16-byte word.
__device__ __forceinline__ int exp_slot(int ml) { return (ml & 1) * 4 + (ml >> 1); }

// One (row block, group) unit per 32 threads: thread (ml, h, p) recodes values 8p .. 8p+7 of half
// h of group g of row 8 rb + ml (its 4-thread quad holds the row's whole group). Units past
// RB * G return as a whole (a quad stays together).
__device__ __forceinline__ void digit_block(const float* __restrict__ x, u32x4* __restrict__ xd,
                                            int* __restrict__ xe, int M, int K, int RB, int b) {
    const int G = K >> 5;
    const int t = static_cast<int>(threadIdx.x);
    const int unit = b * 8 + (t >> 5);
    if (unit >= RB * G) return;
    const int rb = unit / G;
    const int g = unit - rb * G;
    const int ml = (t >> 2) & 7, h = (t >> 1) & 1, p = t & 1;
    const int m = rb * kDigitRows + ml;
    f32x4 v[2];
    if (m < M) {
        const f32x4* src = reinterpret_cast<const f32x4*>(x + static_cast<size_t>(m) * K + 32 * g + 16 * h + 8 * p);
        v[0] = src[0];
        v[1] = src[1];
    } else {
        v[0] = v[1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    // Largest magnitude as an integer maximum of the sign-cleared bits: every non-finite
    // value (0x7F800000 and above) also lands at the top, so one compare detects it.
    uint32_t mb = 0;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) mb = max(mb, __float_as_uint(v[i][c]) & 0x7FFFFFFFu);
    // the quad (lanes t ^ 1, t ^ 2) holds the group's other values
    mb = max(mb, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mb), 0xB1, 0xF, 0xF, false)));
    mb = max(mb, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mb), 0x4E, 0xF, 0xF, false)));
    const bool finite = mb < 0x7F800000u;
    int e = 0;
    (void)frexpf(__uint_as_float(mb), &e);  // max < 2^e (e = 0 for an all-zero group)
    const int sh = kDigitFracBits - e;
    uint32_t z[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int X = finite ? static_cast<int>(rintf(ldexpf(v[j >> 2][j & 3], sh))) : 0;
        z[j] = (static_cast<uint32_t>(X) + kDigitBias) ^ kDigitBias;  // byte d = signed digit D_d
    }
    // Values 8p + {0, 2, 4, 6} are dword q = 2p of the K slot order, 8p + {1, 3, 5, 7} dword 2p + 1.
    uint32_t lo[4], hi[4];
    transpose_bytes(z[0], z[2], z[4], z[6], lo);
    transpose_bytes(z[1], z[3], z[5], z[7], hi);
    // A operand lane of (row ml, digit d, half h): 32 h + 4 ml + d; this thread's dwords 2p, 2p + 1
    uint32_t* dst = reinterpret_cast<uint32_t*>(xd + (static_cast<size_t>(unit) * 64 + 32 * h + 4 * ml)) + 2 * p;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        *reinterpret_cast<u32x2*>(dst + 4 * d) = u32x2{lo[d], hi[d]};
    }
    if (h == 0 && p == 0)
        xe[static_cast<size_t>(unit) * 8 + exp_slot(ml)] = m >= M ? 0 : (finite ? e - 34 : kExpNonFinite);
}

// One launch that prepares a small-batch call: LoRA T partials first (long dependent chains, see
// lora_t_block), then the digit units.
__global__ __launch_bounds__(256) void digits_prep_kernel(const float* __restrict__ x, u32x4* __restrict__ xd,
                                                          int* __restrict__ xe, int M, int K, int RB, int lora_blocks,
                                                          const float* __restrict__ la, float* __restrict__ tpart,
                                                          int R, int tiles_m_t, int tiles_r) {
    const int b = static_cast<int>(blockIdx.x);
    if (b >= lora_blocks) {
        digit_block(x, xd, xe, M, K, RB, b - lora_blocks);
        return;
    }
    lora_t_block(x, la, tpart, M, K, R, b % tiles_m_t, (b / tiles_m_t) % tiles_r, b / (tiles_m_t * tiles_r));
}

// Output of row m, column n of a row holding an infinity or a NaN: the IEEE double sum of its
// non-finite terms x * (v * s), formed as the reference forms each term. Every such row's outputs
// are infinite or NaN and finite terms cannot change that, so this is the reference's value.
// Only flagged groups are visited. Written for clarity: it runs only for non-finite input.
__device__ float ieee_row_value(const float* x, const uint32_t* wq, const float* ws, const int* xe_rb, int slot,
                                int m, int n, int K) {
    const int G = K >> 5;
    double acc = 0.0;
    for (int g = 0; g < G; ++g) {
        if (xe_rb[g * 8 + slot] != kExpNonFinite) continue;
        const double s = static_cast<double>(ws[static_cast<size_t>(n) * G + g]);
        for (int w = 0; w < 4; ++w) {
            const uint32_t word = wq[(static_cast<size_t>(n) * G + g) * 4 + w];
            for (int t = 0; t < 8; ++t) {
                const float xv = x[static_cast<size_t>(m) * K + 32 * g + 8 * w + t];
                if (__builtin_isfinite(xv)) continue;
                const int v = static_cast<int>(word << (28 - 4 * t)) >> 28;
                acc += static_cast<double>(xv) * (static_cast<double>(v) * s);
            }
        }
    }
    return static_cast<float>(acc);
}

// NI: output register pairs per lane in use (rows 2 i + h, i < NI): 1 for M <= 2, 2 for M <= 4,
// else 4. W: wavefronts per workgroup, splitting K.
template <int NI, int W>
__global__ __launch_bounds__(64 * W) void q4_gemm_digits_kernel(
    const u32x4* xd, const int* __restrict__ xe, const float* x, const uint32_t* wq, const float* ws,
    float* __restrict__ y, int M, int N, int K, int RB, int tiles_n, const float* __restrict__ tpart, int t_splits,
    const float* __restrict__ lb, int R, float lscale) {
    constexpr int kEpilogueBytes = W * NI * 64 * 8;
    constexpr int kSmemBytes = W * kWaveBytes > kEpilogueBytes ? W * kWaveBytes : kEpilogueBytes;
    __shared__ __align__(16) unsigned char smem[kSmemBytes];
    __shared__ float lora_t_s[kDigitRows * kMaxLoraRank];
    __shared__ float lora_b_s[kMaxLoraRank * kDigitCols];
    __shared__ int rowmask;
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int c = lane & 31;
    const int h = lane >> 5;
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

    // This wavefront's groups [gb, ge), walked in super-chunks of kSuper groups.
    const int gpw = (G + W - 1) / W;
    const int gb = min(G, w * gpw);
    const int ge = min(G, gb + gpw);

    unsigned char* const st = smem + w * kWaveBytes;
    const size_t xdu = static_cast<size_t>(rb) * G;  // first (row block, group) unit of this row block

    // Every copy goes through a buffer resource whose base is uniform: the lane's part is a fixed
    // 32-bit offset and the super-chunk's position a scalar offset, so issuing costs no vector ALU
    // work, and a read past a resource's end returns zeros (columns past N, groups past K). Each
    // copy instruction moves whole runs of a column: gfx950's copies into LDS cost per 128-byte
    // line touched, not per byte.
    //   Weights: instruction p moves columns 4p .. 4p+3 of the tile, 256 bytes (the super-chunk's
    //   16 groups) each; lane i takes column 4p + i / 16 and group slot (i % 16) ^ (column % 16),
    //   so that the MFMA-side reads (lane (c, h) reads one group of column c, 256 bytes apart)
    //   hit 16 distinct 16-byte bank groups per 16 lanes.
    //   Scales: instruction p moves the 16 scales of columns 4p .. 4p+3 (64 bytes each).
    //   Exponents: instruction j moves those of groups 8j .. 8j+7 (256 contiguous bytes).
    const int col0 = min(n0, N);
    const size_t left = static_cast<size_t>(N - col0) * G;  // groups from the tile's first column
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(wq) + static_cast<size_t>(col0) * G * 4, 0,
        static_cast<int>(min(left * 16, size_t{0x7FFFFFFF})), kBufferWord3);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(ws) + static_cast<size_t>(col0) * G, 0, static_cast<int>(min(left * 4, size_t{0x7FFFFFFF})),
        kBufferWord3);
    const size_t units = static_cast<size_t>(RB) * G;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<u32x4*>(xd), 0, static_cast<int>(min(units * 1024, size_t{0x7FFFFFFF})), kBufferWord3);
    const __amdgpu_buffer_rsrc_t re = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int*>(xe), 0, static_cast<int>(min(units * 32, size_t{0x7FFFFFFF})), kBufferWord3);
    const int ci = lane >> 4;  // column within a copy instruction
    const int gs = lane & 15;  // group slot within a column's run
    uint32_t vw[8], vs[8];
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const int cc = 4 * p + ci;
        vw[p] = static_cast<uint32_t>((cc * G + (gs ^ (cc & 15))) * 16);
        vs[p] = static_cast<uint32_t>((cc * G + gs) * 4);
    }

    // A super-chunk: the digits of its 16 groups into VGPRs (each group one contiguous 1 KiB run in
    // MFMA lane order), its weights, scales and exponents into this wavefront's LDS.
    auto issue = [&](int sb, u32x4 (&a)[kSuper]) {
        typedef __attribute__((address_space(3))) void* lds_ptr;
#pragma unroll
        for (int gi = 0; gi < kSuper; ++gi)
            a[gi] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  ra, static_cast<uint32_t>(lane * 16),
                                                  static_cast<uint32_t>((xdu + sb + gi) * 1024), 0));
#pragma unroll
        for (int p = 0; p < 8; ++p)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr)(st + p * 1024), 16, vw[p],
                                                     static_cast<uint32_t>(sb * 16), 0, 0);
#pragma unroll
        for (int p = 0; p < 8; ++p)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(st + kSOff + p * 256), 4, vs[p],
                                                     static_cast<uint32_t>(sb * 4), 0, 0);
#pragma unroll
        for (int j = 0; j < 2; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(re, (lds_ptr)(st + kEOff + j * 256), 4,
                                                     static_cast<uint32_t>(lane * 4),
                                                     static_cast<uint32_t>((xdu + sb + 8 * j) * 32), 0, 0);
    };

    double acc[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) acc[i] = 0.0;

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
    // Groups 4q .. 4q+3 of the super-chunk starting at group sb.
    auto compute = [&](int sb, int q, const u32x4* a) {
        const int cb = sb + q * kChunk;
        const f32x4 s4 = *reinterpret_cast<const f32x4*>(st + kSOff + c * 64 + q * 16);
        const int* ex = reinterpret_cast<const int*>(st + kEOff);
        // B operands: lane (c, 0) reads group 2p, lane (c, 1) group 2p + 1, and the swaps leave
        // lane (c, h) with packed words 2h and 2h + 1 of both groups.
        i32x4 bq[kChunk];
#pragma unroll
        for (int p = 0; p < kChunk / 2; ++p) {
            const int g = q * kChunk + 2 * p + h;
            const u32x4 wv = *reinterpret_cast<const u32x4*>(st + 256 * c + 16 * (g ^ (c & 15)));
            const auto x0 = __builtin_amdgcn_permlane32_swap(wv[0], wv[2], false, false);
            const auto x1 = __builtin_amdgcn_permlane32_swap(wv[1], wv[3], false, false);
            bq[2 * p] = weights_i8x16(x0[0], x1[0]);
            bq[2 * p + 1] = weights_i8x16(x0[1], x1[1]);
        }
        i32x4 e4[kChunk];
#pragma unroll
        for (int g = 0; g < kChunk; ++g) e4[g] = *reinterpret_cast<const i32x4*>(ex + (q * kChunk + g) * 8 + h * 4);
        const i32x16 zero = {};
        const int valid = ge - cb;  // groups of this chunk in the wavefront's range (uniform)
        if (valid >= kChunk) {
            // Full chunk: the MFMA of group g + 1 is issued before group g's fold, so the fold
            // runs under the matrix core's latency.
            i32x16 r = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a[0]), bq[0], zero, 0, 0, 0);
#pragma unroll
            for (int g = 0; g < kChunk; ++g) {
                i32x16 rn;
                if (g + 1 < kChunk)
                    rn = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a[g + 1]), bq[g + 1], zero, 0,
                                                              0, 0);
                fold(r, s4[g], e4[g]);
                if (g + 1 < kChunk) r = rn;
            }
        } else {
#pragma unroll
            for (int g = 0; g < kChunk; ++g) {
                if (g < valid) {  // uniform
                    const i32x16 r =
                        __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a[g]), bq[g], zero, 0, 0, 0);
                    fold(r, s4[g], e4[g]);
                }
            }
        }
    };

    // A super-chunk's loads are issued at once, then one wait for all of them and its 16 groups'
    // MFMAs (the compiler waits for every copy into LDS before the first LDS read anyway). The
    // wavefronts sharing a SIMD overlap one another's waits.
    for (int sb = gb; sb < ge; sb += kSuper) {
        u32x4 a[kSuper];
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the previous super-chunk's LDS reads are done
        issue(sb, a);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (sb + q * kChunk < ge) compute(sb, q, a + q * kChunk);  // uniform
    }

    __syncthreads();  // every wavefront's K range is done: the staging area is free
    // Rows of this block holding a non-finite x (exponent INT_MIN in any group).
    {
        const int* xr = xe + xdu * 8;
        int mask = 0;
        for (int e = static_cast<int>(threadIdx.x); e < G * 8; e += 64 * W) {
            const int s = e & 7;
            if (xr[e] == kExpNonFinite) mask |= 1 << (2 * (s & 3) + (s >> 2));
        }
        if (mask) atomicOr(&rowmask, mask);
    }
    double* red = reinterpret_cast<double*>(smem);
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
            if ((rowmask >> ml) & 1) s = ieee_row_value(x, wq, ws, xe + xdu * 8, exp_slot(ml), m, n, K);
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
hipError_t launch_digits_gemm(const u32x4* xd, const int* xe, const float* x, const uint8_t* w_packed,
                              const float* w_scales, float* y, int m, int n, int k, int RB, int tiles_n,
                              const float* tpart, int t_splits, const float* lb, int rank, float lscale,
                              hipStream_t stream) {
    hipLaunchKernelGGL((q4_gemm_digits_kernel<NI, W>), dim3(static_cast<unsigned>(RB * tiles_n)), dim3(64 * W), 0,
                       stream, xd, xe, x, reinterpret_cast<const uint32_t*>(w_packed), w_scales, y, m, n, k, RB,
                       tiles_n, tpart, t_splits, lb, rank, lscale);
    return hipGetLastError();
}

}  // namespace

size_t digits_workspace_bytes(uint32_t m, uint32_t k) {
    const size_t units = static_cast<size_t>((m + kDigitRows - 1) / kDigitRows) * (k / kGroup);
    return align256(units * 64 * sizeof(u32x4)) + align256(units * kDigitRows * sizeof(int));
}

hipError_t launch_q4gemm_digits(const DeviceInfo& dev, const float* x, const uint8_t* w_packed, const float* w_scales,
                                float* y, uint32_t m, uint32_t n, uint32_t k, const float* la, const float* lb,
                                uint32_t rank, float lora_scale, int t_splits, void* workspace, hipStream_t stream) {
    const int M = static_cast<int>(m), N = static_cast<int>(n), K = static_cast<int>(k), G = K / kGroup;
    const int RB = (M + kDigitRows - 1) / kDigitRows;
    const size_t units = static_cast<size_t>(RB) * G;
    char* wsp = static_cast<char*>(workspace);
    u32x4* xd = reinterpret_cast<u32x4*>(wsp);
    wsp += align256(units * 64 * sizeof(u32x4));
    int* xe = reinterpret_cast<int*>(wsp);
    wsp += align256(units * kDigitRows * sizeof(int));
    float* tpart = rank ? reinterpret_cast<float*>(wsp) : nullptr;
    const int R = static_cast<int>(rank);
    const int tiles_m_t = (M + 15) / 16, tiles_r = (R + 15) / 16;
    const int lora_blocks = rank ? tiles_m_t * tiles_r * t_splits : 0;
    const int digit_blocks = static_cast<int>((units + 7) / 8);
    hipLaunchKernelGGL(digits_prep_kernel, dim3(static_cast<unsigned>(lora_blocks + digit_blocks)), dim3(256), 0,
                       stream, x, xd, xe, M, K, RB, lora_blocks, la, tpart, R, tiles_m_t, tiles_r);
    const hipError_t pe = hipGetLastError();
    if (pe != hipSuccess) return pe;
    const int tiles_n = (N + kDigitCols - 1) / kDigitCols;
    const bool few = RB * tiles_n <= dev.cu_count;  // one round of workgroups: more wavefronts per tile
    const float* lbp = rank ? lb : nullptr;
    if (M <= 2)
        return few ? launch_digits_gemm<1, 8>(xd, xe, x, w_packed, w_scales, y, M, N, K, RB, tiles_n, tpart, t_splits,
                                              lbp, R, lora_scale, stream)
                   : launch_digits_gemm<1, 4>(xd, xe, x, w_packed, w_scales, y, M, N, K, RB, tiles_n, tpart, t_splits,
                                              lbp, R, lora_scale, stream);
    if (M <= 4)
        return few ? launch_digits_gemm<2, 8>(xd, xe, x, w_packed, w_scales, y, M, N, K, RB, tiles_n, tpart, t_splits,
                                              lbp, R, lora_scale, stream)
                   : launch_digits_gemm<2, 4>(xd, xe, x, w_packed, w_scales, y, M, N, K, RB, tiles_n, tpart, t_splits,
                                              lbp, R, lora_scale, stream);
    return few ? launch_digits_gemm<4, 8>(xd, xe, x, w_packed, w_scales, y, M, N, K, RB, tiles_n, tpart, t_splits, lbp,
                                          R, lora_scale, stream)
               : launch_digits_gemm<4, 4>(xd, xe, x, w_packed, w_scales, y, M, N, K, RB, tiles_n, tpart, t_splits, lbp,
                                          R, lora_scale, stream);
}

}  // namespace spaceslug
