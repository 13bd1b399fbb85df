// Parameters of the grouped low-bit weight kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace phi_dev {

// Relative-scale storage types (RelDType, core/kernels/w4a8_expand.hpp:65-75).
enum WDType { W_F32 = 0, W_BF16 = 1, W_F16 = 2, W_E4M3 = 5, W_E5M2 = 6, W_U8_E4M3 = 7 };

struct W4a8Params {
    const uint8_t* codes;
    int64_t codes_row_bytes;
    const void* s_rel;
    int s_rel_dtype;
    int64_t srel_row_bytes;
    const float* s_channel;
    int sch_scalar;
    const float* codebook;
    const float* correction;
    int64_t rows, k, group;
    int layout;
};

hipError_t launch_w4a8_rows(hipStream_t stream, const W4a8Params& p, int8_t* out, float* s, bool lut);

// Load-time weight kernels (weights.hip).
enum DequantKind { DQ_F32 = 0, DQ_BF16 = 1, DQ_F16 = 2, DQ_I8 = 4, DQ_F8_E4M3 = 5, DQ_F8_E5M2 = 6, DQ_I4 = 8 };
hipError_t launch_dequant_rows(hipStream_t stream, const void* src, int kind, int64_t rows, int64_t cols, int64_t lds,
                               const float* row_scale, int scale_scalar, float* out, int64_t ldo);
// nvfp4 / mxfp4 rows row0 .. row0 + rows - 1: E2M1 codes (even column in the
// high nibble) times the (row, column / block) entry of the cuBLAS-tiled
// block-scale table (already fp32; null: 1) times the row's global scale.
struct Fp4Rows {
    const uint8_t* codes;
    int64_t codes_ld, row0, rows, k;
    const float* block_scale;
    int64_t scale_cols, block;
    const float* global;
    int global_scalar;
};
hipError_t launch_dequant_fp4_rows(hipStream_t stream, const Fp4Rows& p, float* out, int64_t ldo);
hipError_t launch_convrot_rows(hipStream_t stream, const float* x, int64_t ldx, float* y, int64_t ldy, int64_t rows,
                               int64_t K);
hipError_t launch_lora_fold(hipStream_t stream, float* w, int64_t ldw, int64_t rows, int64_t k, const float* A,
                            const float* B, int64_t rank, float scale);

}  // namespace phi_dev
