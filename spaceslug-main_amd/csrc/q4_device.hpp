// Device-side helpers shared by the gfx950 int4 kernels: nibble decoding and
// cross-lane reductions. Layout facts (q4gemm.comp:7-19): a packed byte holds
// k even in bits 0..3 and k odd in bits 4..7, so one little-endian 32-bit word
// holds 8 consecutive K values of one column, value t in bits 4t..4t+3, each a
// two's-complement nibble.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace spaceslug {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Signed value of nibble t (0..7) of w, as a float (exact): v_bfe_i32 + v_cvt_f32_i32.
__device__ __forceinline__ float nibble_signed(uint32_t w, int t) {
    return static_cast<float>(static_cast<int32_t>(w << (28 - 4 * t)) >> 28);
}

// v_cvt_off_f32_i4 reads bits 3..0 of its operand as a two's-complement value v
// and returns v / 16 exactly. The SDWA forms read byte 1, 2 or 3 of the operand
// in place, so a byte's low nibble needs no shift.
#define SPACESLUG_CVT_OFF_BYTE(SEL)                                                                      \
    __device__ __forceinline__ float cvt_off_##SEL(uint32_t w) {                                          \
        float r;                                                                                         \
        asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:" #SEL : "=v"(r) \
            : "v"(w));                                                                                   \
        return r;                                                                                        \
    }
SPACESLUG_CVT_OFF_BYTE(BYTE_1)
SPACESLUG_CVT_OFF_BYTE(BYTE_2)
SPACESLUG_CVT_OFF_BYTE(BYTE_3)
#undef SPACESLUG_CVT_OFF_BYTE

// Signed decode of all 8 nibbles of w: f[t] = v_t / 16 exactly, in 9 VALU ops
// (one shift for the odd nibbles, eight conversions). A sum of x * f times 16
// (exact) is the sum of x * v.
__device__ __forceinline__ void nibbles_signed_16th(uint32_t w, float (&f)[8]) {
    const uint32_t wo = w >> 4;
    f[0] = __builtin_amdgcn_cvt_off_f32_i4(static_cast<int>(w));
    f[1] = __builtin_amdgcn_cvt_off_f32_i4(static_cast<int>(wo));
    f[2] = cvt_off_BYTE_1(w);
    f[3] = cvt_off_BYTE_1(wo);
    f[4] = cvt_off_BYTE_2(w);
    f[5] = cvt_off_BYTE_2(wo);
    f[6] = cvt_off_BYTE_3(w);
    f[7] = cvt_off_BYTE_3(wo);
}

// The same values with compiler-visible instructions only (shifts plus the
// conversion builtin, about 13 VALU ops). Use this one where the results feed
// MFMA operands: the hazard recognizer does not see inside inline asm, and an
// asm write to a VGPR that an in-flight MFMA still reads as SrcB corrupts it.
__device__ __forceinline__ void nibbles_signed_16th_mfma(uint32_t w, float (&f)[8]) {
#pragma unroll
    for (int t = 0; t < 8; ++t) f[t] = __builtin_amdgcn_cvt_off_f32_i4(static_cast<int>(w >> (4 * t)));
}

// Scale that restores nibbles_signed_16th's values to the integers v.
constexpr float kSixteenthsUnit = 16.0f;

// Offset-binary decode of all 8 nibbles of w through the fp8 converter.
// u = v + 8 = nibble ^ 8 lies in [0, 15]; a byte holding u read as OCP e4m3
// (bias 7) is exactly u * 2^-9 (u < 8 is a subnormal m/8 * 2^-6, u >= 8 has
// exponent field 1 and mantissa u - 8: (1 + (u-8)/8) * 2^-6). So
// f[t] = (v_t + 8) * 2^-9 exactly. Two bit-ops place the even and the odd
// nibbles in separate bytes; each v_cvt_pk_f32_fp8 converts two bytes.
__device__ __forceinline__ void nibbles_offset_e4m3(uint32_t w, float (&f)[8]) {
    const uint32_t even = (w ^ 0x88888888u) & 0x0F0F0F0Fu;         // u0 u2 u4 u6
    const uint32_t odd = ((w >> 4) ^ 0x08080808u) & 0x0F0F0F0Fu;   // u1 u3 u5 u7
    const f32x2 e0 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(even), false);
    const f32x2 e1 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(even), true);
    const f32x2 o0 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(odd), false);
    const f32x2 o1 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(odd), true);
    f[0] = e0.x; f[1] = o0.x; f[2] = e0.y; f[3] = o0.y;
    f[4] = e1.x; f[5] = o1.x; f[6] = e1.y; f[7] = o1.y;
}

// (v + 8) * 2^-9 decoding scale: multiply a sum of x * f by this to get x * (v + 8).
constexpr float kE4m3OffsetUnit = 512.0f;

// Sum over the 64 lanes of a wavefront; every lane receives the total.
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

}  // namespace spaceslug
