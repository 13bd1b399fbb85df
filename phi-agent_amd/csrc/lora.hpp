// Runtime LoRA correction kernels (fp32 fma chains in the reference's order).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace phi_dev {

// h [M, R] = x [M, ldx] (fp32 or bf16) . A [R, K]^T, fp32.
hipError_t launch_lora_down(hipStream_t stream, const void* x, bool x_bf16, int64_t ldx, const float* A, float* h,
                            int M, int K, int R);
// C [M, ldc] (fp32 or bf16) += h [M, R] . B [N, R]^T, in place.
hipError_t launch_lora_rank_add(hipStream_t stream, const float* h, const float* B, void* C, bool c_bf16, int64_t ldc,
                                int M, int N, int R);

}  // namespace phi_dev
