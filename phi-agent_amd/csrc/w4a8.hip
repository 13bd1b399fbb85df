// Grouped low-bit weights (asym_w4a8_int8 nibble4, w6a8_int8 packed6) onto the
// int8 GEMM operand.
//
// Decode (core/host/quant.cpp:315-389, device core/kernels/w4a8_expand.cpp:99-257):
//   level = codebook ? codebook[code] : code - 8      (nibble4; low nibble = even col)
//         = code - 32                                 (packed6: k/2 low-nibble bytes,
//                                                      then k/4 bytes of top-2 bits)
//   v     = rint_clamp127(level * s_rel[row, col/group]) * s_channel[row] (+ corr[g][row])
// Requantise per row (core/host/quant.cpp:134-169, no rotation):
//   scale = amax > 1e-30 ? amax/127 : 1;  q = clamp(round_half_away(v * (1/scale)), +-127)
//
// expand: writes q [rows, k] and s [rows] -- the reference's expand pass.
// prepare: writes s [rows] and, per (row, group), the 16 codes the expand would
//   produce for nibbles 0..15 (lut [rows, groups, 16]), so a GEMM can turn packed
//   nibbles into the same int8 operand in registers (nibble4 only).
//
// One workgroup per row; each thread decodes 16 consecutive columns at a time.
// Pass 1 reduces the row amax, pass 2 decodes again and quantises.
#include "device_common.hpp"
#include "w4a8.hpp"

namespace phi_dev {

__device__ __forceinline__ float rel_at(const uint8_t* row, int dtype, int64_t g) {
    switch (dtype) {
        case W_F32: return ((const float*)row)[g];
        case W_F16: return f16_to_f32(((const uint16_t*)row)[g]);
        case W_BF16: return bf16_to_f32(((const uint16_t*)row)[g]);
        case W_E5M2: return e5m2_to_f32(row[g]);
        default: return e4m3_to_f32(row[g]);  // W_E4M3 and the byte-container spelling
    }
}

// The packer's int8 grid: nearest integer with ties to even, clamped to +-127.
__device__ __forceinline__ float grid8(float v) { return fminf(fmaxf(rintf(v), -127.0f), 127.0f); }

// Decode 16 consecutive columns starting at c0 (c0 % 16 == 0) of one row.
__device__ __forceinline__ void decode16(const W4a8Params& p, int64_t row, int64_t c0,
                                         const float* cb, float (&v)[16]) {
    const uint8_t* codes = p.codes + row * p.codes_row_bytes;
    const uint8_t* rel_row = (const uint8_t*)p.s_rel + row * p.srel_row_bytes;
    const float sch = p.s_channel ? (p.sch_scalar ? p.s_channel[0] : p.s_channel[row]) : 1.0f;
    int code[16];
    if (p.layout == 0) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t b = codes[c0 / 2 + j];
            code[2 * j] = (int)(b & 15u);
            code[2 * j + 1] = (int)(b >> 4);
        }
    } else {
        // Column i's top two bits sit in hi-plane byte i/4 at bit 2*(i & 3).
        const uint8_t* hi = codes + p.k / 2 + c0 / 4;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t b = codes[c0 / 2 + j];
            const uint32_t h = hi[j / 2];
            const int i0 = 2 * j, i1 = 2 * j + 1;
            code[i0] = (int)((b & 15u) | (((h >> (2 * (i0 & 3))) & 3u) << 4));
            code[i1] = (int)((b >> 4) | (((h >> (2 * (i1 & 3))) & 3u) << 4));
        }
    }
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int64_t col = c0 + i;
        const int64_t g = col / p.group;
        float level;
        if (p.layout == 0) level = cb ? cb[code[i]] : (float)(code[i] - 8);
        else level = (float)(code[i] - 32);
        const float rel = p.s_rel ? rel_at(rel_row, p.s_rel_dtype, g) : 1.0f;
        float val = grid8(level * rel) * sch;
        if (p.correction) val = val + p.correction[g * p.rows + row];
        v[i] = val;
    }
}

__device__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int tid = threadIdx.x;
    if ((tid & 63) == 0) red[tid >> 6] = v;
    __syncthreads();
    float m = red[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); w++) m = fmaxf(m, red[w]);
    return m;
}

template <bool LUT>
__global__ __launch_bounds__(256) void w4a8_rows_kernel(W4a8Params p, int8_t* __restrict__ out,
                                                        float* __restrict__ s) {
    __shared__ float cb[16];
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    if (tid < 16) cb[tid] = p.codebook ? p.codebook[tid] : 0.0f;
    __syncthreads();
    const float* cbp = p.codebook ? cb : nullptr;
    const int64_t chunks = p.k / 16;

    float amax = 0.0f;
    for (int64_t c = tid; c < chunks; c += blockDim.x) {
        float v[16];
        decode16(p, row, c * 16, cbp, v);
#pragma unroll
        for (int i = 0; i < 16; i++) amax = fmaxf(amax, fabsf(v[i]));
    }
    const float rmax = block_max(amax, red);
    const float scale = rmax > 1e-30f ? rmax / 127.0f : 1.0f;
    const float inv = 1.0f / scale;
    if (tid == 0) s[row] = scale;

    if (!LUT) {
        for (int64_t c = tid; c < chunks; c += blockDim.x) {
            float v[16];
            decode16(p, row, c * 16, cbp, v);
            uint32_t w[4];
#pragma unroll
            for (int i = 0; i < 4; i++)
                w[i] = pack4(quant_code(v[4 * i], inv, 127.0f, 0), quant_code(v[4 * i + 1], inv, 127.0f, 0),
                             quant_code(v[4 * i + 2], inv, 127.0f, 0), quant_code(v[4 * i + 3], inv, 127.0f, 0));
            *(uint4*)(out + row * p.k + c * 16) = make_uint4(w[0], w[1], w[2], w[3]);
        }
    } else {
        // One table per (row, group): the code each nibble value would expand to.
        const int64_t groups = p.k / p.group;
        const uint8_t* rel_row = (const uint8_t*)p.s_rel + row * p.srel_row_bytes;
        const float sch = p.s_channel ? (p.sch_scalar ? p.s_channel[0] : p.s_channel[row]) : 1.0f;
        for (int64_t g = tid; g < groups; g += blockDim.x) {
            const float rel = p.s_rel ? rel_at(rel_row, p.s_rel_dtype, g) : 1.0f;
            const float corr = p.correction ? p.correction[g * p.rows + row] : 0.0f;
            uint32_t w[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                int qv[4];
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const int code = 4 * i + t;
                    const float level = cbp ? cbp[code] : (float)(code - 8);
                    float val = grid8(level * rel) * sch;
                    if (p.correction) val = val + corr;
                    qv[t] = quant_code(val, inv, 127.0f, 0);
                }
                w[i] = pack4(qv[0], qv[1], qv[2], qv[3]);
            }
            *(uint4*)(out + (row * groups + g) * 16) = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
}

hipError_t launch_w4a8_rows(hipStream_t stream, const W4a8Params& p, int8_t* out, float* s, bool lut) {
    if (lut)
        hipLaunchKernelGGL(w4a8_rows_kernel<true>, dim3((unsigned)p.rows), dim3(256), 0, stream, p, out, s);
    else
        hipLaunchKernelGGL(w4a8_rows_kernel<false>, dim3((unsigned)p.rows), dim3(256), 0, stream, p, out, s);
    return hipGetLastError();
}

}  // namespace phi_dev
