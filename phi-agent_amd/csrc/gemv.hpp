// Batched small-M int8 linear: parameters passed by value to the kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "i8_gemm.hpp"

namespace phi_dev {

constexpr int GEMV_MAX_ITEMS = 64;  // items per launch (kernel arguments: 64 x 40 bytes + the header, under 4 KB)

struct GemvBatch {
    const int8_t* q8;
    const float* s8;
    int M, N, K;
    int n_items;
    int bias_kind, c_kind;
    uint64_t sw_scalar_mask;
    const int8_t* W[GEMV_MAX_ITEMS];
    const float* sW[GEMV_MAX_ITEMS];
    const void* bias[GEMV_MAX_ITEMS];
    void* C[GEMV_MAX_ITEMS];
    int64_t ldc[GEMV_MAX_ITEMS];
};

hipError_t launch_gemv(hipStream_t stream, const GemvBatch& b);

hipError_t launch_gelu(hipStream_t stream, const void* x, int x_bf16, void* y, int y_bf16, int64_t n);

hipError_t launch_silu_gate(hipStream_t stream, const void* gx, int x_bf16, int64_t ldx, void* out, int y_bf16,
                            int64_t ldo, int64_t rows, int64_t cols);

}  // namespace phi_dev
