// Internal launch interface between the C-ABI layer (runtime_abi.cpp) and the
// gfx950 kernels (q4_gemv.hip, q4_gemm.hip, sgemm.hip). Device pointers only;
// every function enqueues on `stream` and returns hipSuccess or the launch error.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace spaceslug {

// Scale group along K (q4gemm.comp:41,121): one fp32 scale per 32 K values.
constexpr int kGroup = 32;

// Largest LoRA rank of the fused epilogues (SPACESLUG_Q4_MAX_LORA_RANK in runtime_abi.h).
constexpr int kMaxLoraRank = 64;

// The decode GEMV takes one row with K <= 32 * kGemvSplitMaxGroups (one wavefront per column up to
// K = 32 * kGemvPipeMaxGroups, K split over a workgroup's wavefronts above); every other shape up to
// 32 rows goes to the small-batch GEMM, taller ones to the wide and mid-size kernels.
constexpr int kGemvPipeMaxGroups = 128;
constexpr int kGemvSplitMaxGroups = 1024;

// Shapes the decode GEMV takes: one row with K <= 32 * kGemvSplitMaxGroups, or two rows with
// 2048 <= K <= 16384 (one weight load serves both rows; below K = 2048 half of each wavefront's
// lanes would idle and the small-batch GEMM is as fast; above 16384 two rows' recoded x would not
// fit the LDS).
constexpr bool gemv_takes(uint32_t m, uint32_t k) {
    return (m == 1 && k / kGroup <= static_cast<uint32_t>(kGemvSplitMaxGroups)) ||
           (m == 2 && k >= 2048 && k / kGroup <= 4u * static_cast<uint32_t>(kGemvPipeMaxGroups));
}

// Launch shape chosen by plan_q4gemm for one call.
struct Q4Plan {
    // kGemv: decode GEMV (gemv_takes, no LoRA); kDigits: every other call up to 32 rows,
    // exact integer group sums on the int8 matrix cores (q4_small.hip); kWide: m > 32; kMid:
    // m > 32 without LoRA whose 128 x 128 grid would need a K-split while its 64 x 64 grid fits
    // the CUs once (k % 64 == 0, k <= 4096).
    enum Kind { kGemv, kDigits, kWide, kMid } kind;
    int splits;              // K-splits of the MFMA kernel (1 = write y directly)
    size_t workspace_bytes;  // device scratch the call needs (split partials, LoRA T partials and T, x limbs)
    int t_splits;            // K-splits of the LoRA pre-pass T = x * lora_a (0 without LoRA)
};

struct DeviceInfo {
    int cu_count;
    size_t max_lds_bytes;
};

// Decides the kernel and K-split for (m, n, k, rank). rank == 0 means no LoRA.
Q4Plan plan_q4gemm(const DeviceInfo& dev, uint32_t m, uint32_t n, uint32_t k, uint32_t rank);

// Decode GEMV for the shapes gemv_takes accepts (no device memory beyond its arguments).
hipError_t launch_gemv(const DeviceInfo& dev, const float* x, const uint8_t* w_packed,
                       const float* w_scales, float* y, uint32_t m, uint32_t n, uint32_t k,
                       hipStream_t stream);

// y = x * dequant(W) [+ scale * (x * la) * lb]. `workspace` must hold
// plan.workspace_bytes bytes (may be null when that is 0).
hipError_t launch_q4gemm(const Q4Plan& plan, const DeviceInfo& dev, const float* x,
                         const uint8_t* w_packed, const float* w_scales, float* y, uint32_t m,
                         uint32_t n, uint32_t k, const float* la, const float* lb, uint32_t rank,
                         float lora_scale, void* workspace, hipStream_t stream);

// Small-batch GEMM (kDigits, q4_small.hip): one launch, plus a preparation launch for the LoRA T
// partials; `workspace` holds t_splits * m * rank floats of them (unused without LoRA).
hipError_t launch_q4gemm_small(const DeviceInfo& dev, const float* x, const uint8_t* w_packed, const float* w_scales,
                               float* y, uint32_t m, uint32_t n, uint32_t k, const float* la, const float* lb,
                               uint32_t rank, float lora_scale, int t_splits, void* workspace, hipStream_t stream);

// Bytes of the wide int4 GEMM's x limbs for x (fp32, m x k, k % 32 == 0): three exact bf16 limbs
// per value in 16-row blocks (rows padded with zeros to a multiple of 16), written by the
// preparation launch of launch_q4gemm and part of plan.workspace_bytes.
size_t split_x_bf16_bytes(uint32_t m, uint32_t k);

// fp32 w[k][n] (row-major) -> packed int4 weights [n][k/2] and scales [n][k/32]; k % 32 == 0 and
// k / 32 <= 65535 (checked by the caller). Rule at q4_quantize.hip.
hipError_t launch_q4_quantize(const float* w, uint8_t* w_packed, float* w_scales, uint32_t n, uint32_t k,
                              hipStream_t stream);

// fp32 C = A * B, row-major, m % 64 == 0, n % 64 == 0, k % 32 == 0 (checked by the caller).
hipError_t launch_sgemm(const float* a, const float* b, float* c, uint32_t m, uint32_t n,
                        uint32_t k, hipStream_t stream);

}  // namespace spaceslug
