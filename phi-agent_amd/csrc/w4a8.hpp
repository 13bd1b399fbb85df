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

}  // namespace phi_dev
