// Device-side helpers shared by the gfx950 int4 kernels: vector types and
// nibble decoding. Layout facts (q4gemm.comp:7-19): a packed byte holds
// k even in bits 0..3 and k odd in bits 4..7, so one little-endian 32-bit word
// holds 8 consecutive K values of one column, value t in bits 4t..4t+3, each a
// two's-complement nibble.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace spaceslug {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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
// MFMA operands: a VALU result read by an MFMA as SrcB needs two wait states,
// and after an inline-asm write the compiler inserts only one (s_nop 0 instead
// of s_nop 1), which gave wrong products on gfx950.
__device__ __forceinline__ void nibbles_signed_16th_mfma(uint32_t w, float (&f)[8]) {
#pragma unroll
    for (int t = 0; t < 8; ++t) f[t] = __builtin_amdgcn_cvt_off_f32_i4(static_cast<int>(w >> (4 * t)));
}

// Scale that restores nibbles_signed_16th's values to the integers v.
constexpr float kSixteenthsUnit = 16.0f;

}  // namespace spaceslug
