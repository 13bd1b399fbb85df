// Load-time weight kernels: the steps the reference's loaders run on the host
// before a weight reaches the int8 GEMM, here on the device so a checkpoint
// goes from its file bytes to the GEMM operand without an fp32 round trip
// through host memory.
//
//   dequant_rows  a stored tensor's values in fp32 (SafeTensors::dequant_rows,
//                 core/host/st.cpp:601-700: int8 codes or a bare int4's signed
//                 nibbles times the row scale, fp8 codes times the row scale
//                 (dequant_fp8_row, core/host/quant.cpp:433-439),
//                 f16 / bf16 widened, fp32 copied)
//   dequant_fp4_rows  nvfp4 / mxfp4 rows (dequant_nvfp4_row,
//                 core/host/quant.cpp:390-431): E2M1 codes times their block's
//                 scale from the cuBLAS-tiled table times the global scale
//   convrot_rows  the 256-wide J-2R rotation of fp32 rows with no quantiser
//                 (convrot_forward, core/host/quant.cpp:66-100; its inverse is
//                 the same map, core/host/quant.hpp:63-65)
//   lora_fold     w[o][i] += (scale * B[o][r]) * A[r][i] for r ascending, rank
//                 entries of B that are 0 skipped (LoraSet::apply_rows_of,
//                 core/models/lora.cpp:182-201)
//   pack_k_tiled  an int8 row-major weight into the K-tiled operand layout of
//                 the persistent pipeline (k_tiled_offset); a pure re-layout
//   pack_banded   a W4 weight's codes and prepared tables into the band layout
//                 the 272 x 192 kernel's in-LDS expansion reads (bands of 192
//                 rows, one contiguous block a band and K-step or group); a
//                 pure re-layout
//
// The rotate + quantise that turns the result into int8 is quant_rotate, the
// same kernel the activations take: the reference's weight and activation
// quantisers are one function (quantize_impl_into, core/host/quant.cpp:134-169).
//
// All of this runs once per weight load and is bound by HBM at a few bytes per
// element; the kernels are plain and exact (-ffp-contract=off: every product
// and sum rounds on its own, as the reference's x86-64 host code does).
#include "device_common.hpp"
#include "i8_gemm.hpp"
#include "w4a8.hpp"

namespace phi_dev {

__global__ __launch_bounds__(256) void dequant_rows_kernel(const void* src, int kind, int64_t rows, int64_t cols,
                                                           int64_t lds, const float* row_scale, int scale_scalar,
                                                           float* out, int64_t ldo) {
    const int64_t total = rows * cols;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t r = i / cols, c = i - r * cols;
        const int64_t at = r * lds + c;
        float v;
        switch (kind) {
            case DQ_I8: v = (float)((const int8_t*)src)[at] * row_scale[scale_scalar ? 0 : r]; break;
            case DQ_I4: {
                const uint32_t b = ((const uint8_t*)src)[r * lds + (c >> 1)];
                const int nib = (int)((c & 1) ? b >> 4 : b & 15u);
                const float sc = row_scale ? row_scale[scale_scalar ? 0 : r] : 1.0f;
                v = (float)(nib >= 8 ? nib - 16 : nib) * sc;
                break;
            }
            case DQ_F8_E4M3:
            case DQ_F8_E5M2: {
                const uint32_t b = ((const uint8_t*)src)[at];
                const float d = kind == DQ_F8_E4M3 ? e4m3_to_f32(b) : e5m2_to_f32(b);
                v = d * (row_scale ? row_scale[scale_scalar ? 0 : r] : 1.0f);
                break;
            }
            case DQ_F16: v = f16_to_f32(((const uint16_t*)src)[at]); break;
            case DQ_BF16: v = bf16_to_f32(((const uint16_t*)src)[at]); break;
            default: v = ((const float*)src)[at]; break;
        }
        out[r * ldo + c] = v;
    }
}

// E2M1: sign, two exponent bits (bias 1), one mantissa bit; exponent 0 is the
// subnormal 0 / 0.5.  Magnitudes 0, .5, 1, 1.5, 2, 3, 4, 6.
__device__ __forceinline__ float e2m1_to_f32(uint32_t nib) {
    const uint32_t e = (nib >> 1) & 3u, m = nib & 1u;
    const float mag = e == 0u ? 0.5f * (float)m : (float)(2u + m) * __uint_as_float((e - 2u + 127u) << 23);
    return (nib & 8u) ? -mag : mag;
}

// The flat index of (row, block) in the cuBLAS "blocked" scale table: the
// [rows, blocks] table padded to (128 rows, 4 blocks) tiles, the tiles in
// row-tile-major order, and each 128 x 4 tile stored as 32 x (4 x 4) with the
// row's 32-row quarter inside the 16-byte group (core/host/quant.cpp:390-410).
__device__ __forceinline__ int64_t blocked_index(int64_t row, int64_t blk, int64_t nb_c) {
    const int64_t h = row & 127, chunk = (row >> 7) * nb_c + (blk >> 2);
    return chunk * 512 + (h & 31) * 16 + (h >> 5) * 4 + (blk & 3);
}

__global__ __launch_bounds__(256) void dequant_fp4_rows_kernel(Fp4Rows p, float* out, int64_t ldo) {
    const int64_t total = p.rows * p.k, nb_c = p.scale_cols >> 2;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t r = i / p.k, c = i - r * p.k;
        const uint32_t b = p.codes[r * p.codes_ld + (c >> 1)];
        const uint32_t nib = (c & 1) ? b & 15u : b >> 4;
        const float s = p.block_scale ? p.block_scale[blocked_index(p.row0 + r, c / p.block, nb_c)] : 1.0f;
        const float g = p.global ? p.global[p.global_scalar ? 0 : r] : 1.0f;
        out[r * ldo + c] = (e2m1_to_f32(nib) * s) * g;
    }
}

// One 256-element group per workgroup, one element per thread.  Stage d
// (stride 4^d) gives element j of each 4-tuple (((x0 + x1) + x2) + x3) - 2 x[3-j],
// the reference's butterfly in its operation order; the 1/16 is a final
// product, as in the reference.  x == y (same pitch) is allowed: a group is
// read whole into LDS before any of it is written.
__global__ __launch_bounds__(256) void convrot_rows_kernel(const float* x, int64_t ldx, float* y, int64_t ldy,
                                                           int64_t groups_per_row) {
    __shared__ float buf[256];
    const int t = threadIdx.x;
    const int64_t row = blockIdx.x / groups_per_row, g = blockIdx.x - row * groups_per_row;
    buf[t] = x[row * ldx + g * 256 + t];
    __syncthreads();
#pragma unroll
    for (int stride = 1; stride < 256; stride *= 4) {
        const int j = (t / stride) & 3, b = t - j * stride;
        const float x0 = buf[b], x1 = buf[b + stride], x2 = buf[b + 2 * stride], x3 = buf[b + 3 * stride];
        const float s = ((x0 + x1) + x2) + x3;
        const float mine = j == 0 ? x3 : j == 1 ? x2 : j == 2 ? x1 : x0;
        const float v = s - 2.0f * mine;
        __syncthreads();
        buf[t] = v;
        __syncthreads();
    }
    y[row * ldy + g * 256 + t] = buf[t] * (1.0f / 16.0f);
}

// One element per thread; the rank loop runs in one lane in the reference's
// order.  B is indexed from the factor's row0.
__global__ __launch_bounds__(256) void lora_fold_kernel(float* w, int64_t ldw, int64_t rows, int64_t k,
                                                        const float* A, const float* B, int64_t rank, float scale) {
    const int64_t total = rows * k;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t o = i / k, c = i - o * k;
        float acc = w[o * ldw + c];
        const float* brow = B + o * rank;
        for (int64_t r = 0; r < rank; r++) {
            const float br = brow[r];
            if (br == 0.0f) continue;
            const float s = scale * br;
            acc = acc + s * A[r * k + c];
        }
        w[o * ldw + c] = acc;
    }
}

// One 16-byte chunk a thread, read in row order (coalesced), written to its
// K-tiled slot.  src rows are 16-byte aligned; K % 64 == 0.
__global__ __launch_bounds__(256) void pack_k_tiled_kernel(const int8_t* __restrict__ src, int64_t ld, int64_t rows,
                                                           int64_t K, int8_t* __restrict__ dst) {
    const int64_t cpr = K >> 4, total = rows * cpr;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t r = i / cpr, c = (i - r * cpr) << 4;
        *(uint4*)(dst + k_tiled_offset(r, c, K, rows)) = *(const uint4*)(src + r * ld + c);
    }
}

// One 16-byte chunk of the band-packed W4 operand a thread (w4_banded_bytes):
// the code blocks (band b, K-step s: rows 192 b .. + 191, 32 bytes each),
// then the table blocks (band b, group g: 16 bytes a row); rows past N zero.
__global__ __launch_bounds__(256) void pack_banded_kernel(const uint8_t* __restrict__ codes, int64_t crb,
                                                          const int8_t* __restrict__ lut, int N, int K, int groups,
                                                          uint8_t* __restrict__ out, int64_t code_bytes,
                                                          int64_t total) {
    constexpr int TB = 192;
    const int KT = K / 64;
    for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 16; i < total; i += (int64_t)gridDim.x * 256 * 16) {
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (i < code_bytes) {
            const int64_t blk = i / (TB * 32);
            const int within = (int)(i - blk * (TB * 32)), b = (int)(blk / KT), st = (int)(blk - (int64_t)b * KT);
            const int64_t n = (int64_t)b * TB + within / 32;
            if (n < N) v = *(const uint4*)(codes + n * crb + st * 32 + (within & 31));
        } else {
            const int64_t t = i - code_bytes, blk = t / (TB * 16);
            const int within = (int)(t - blk * (TB * 16)), b = (int)(blk / groups), g = (int)(blk - (int64_t)b * groups);
            const int64_t n = (int64_t)b * TB + within / 16;
            if (n < N) v = *(const uint4*)(lut + (n * groups + g) * 16);
        }
        *(uint4*)(out + i) = v;
    }
}

static unsigned grid_for(int64_t n) {
    const int64_t b = (n + 255) / 256;
    return (unsigned)(b < 65536 ? (b > 0 ? b : 1) : 65536);
}

hipError_t launch_dequant_rows(hipStream_t stream, const void* src, int kind, int64_t rows, int64_t cols, int64_t lds,
                               const float* row_scale, int scale_scalar, float* out, int64_t ldo) {
    hipLaunchKernelGGL(dequant_rows_kernel, dim3(grid_for(rows * cols)), dim3(256), 0, stream, src, kind, rows, cols,
                       lds, row_scale, scale_scalar, out, ldo);
    return hipGetLastError();
}

hipError_t launch_dequant_fp4_rows(hipStream_t stream, const Fp4Rows& p, float* out, int64_t ldo) {
    hipLaunchKernelGGL(dequant_fp4_rows_kernel, dim3(grid_for(p.rows * p.k)), dim3(256), 0, stream, p, out, ldo);
    return hipGetLastError();
}

hipError_t launch_convrot_rows(hipStream_t stream, const float* x, int64_t ldx, float* y, int64_t ldy, int64_t rows,
                               int64_t K) {
    const int64_t gpr = K / 256;
    hipLaunchKernelGGL(convrot_rows_kernel, dim3((unsigned)(rows * gpr)), dim3(256), 0, stream, x, ldx, y, ldy, gpr);
    return hipGetLastError();
}

hipError_t launch_lora_fold(hipStream_t stream, float* w, int64_t ldw, int64_t rows, int64_t k, const float* A,
                            const float* B, int64_t rank, float scale) {
    hipLaunchKernelGGL(lora_fold_kernel, dim3(grid_for(rows * k)), dim3(256), 0, stream, w, ldw, rows, k, A, B, rank,
                       scale);
    return hipGetLastError();
}

hipError_t launch_w4_pack_banded(hipStream_t stream, const uint8_t* codes, int64_t crb, const int8_t* lut, int N,
                                 int K, int groups, uint8_t* out) {
    const int64_t bands = (N + 191) / 192, code_bytes = bands * (K / 64) * (192 * 32);
    const int64_t total = code_bytes + bands * groups * (192 * 16);
    hipLaunchKernelGGL(pack_banded_kernel, dim3(grid_for(total / 16)), dim3(256), 0, stream, codes, crb, lut, N, K,
                       groups, out, code_bytes, total);
    return hipGetLastError();
}

hipError_t launch_pack_k_tiled(hipStream_t stream, const int8_t* src, int64_t ld, int64_t rows, int64_t K,
                               int8_t* dst) {
    hipLaunchKernelGGL(pack_k_tiled_kernel, dim3(grid_for(rows * (K >> 4))), dim3(256), 0, stream, src, ld, rows, K,
                       dst);
    return hipGetLastError();
}

}  // namespace phi_dev
