// Small-M int8 linear (M <= 8) over a batch of weights that share one
// quantised activation block -- the adaLN modulation shape.  Bandwidth-bound:
// every weight byte is read exactly once, with 16-byte non-temporal loads.
//
//   acc[m, n] = sum_k q8[m, k] * W_i[n, k]        (v_dot4 int8, exact int32)
//   C_i[m, n] = fma((float)acc * s8[m], sW_i[n], bias_i[n])
// Same arithmetic contract as the GEMM (core/kernels/int8_gemm.cpp:588-620).
//
// Work split: a wave owns ROWS consecutive weight rows; lane l reads the
// 16-byte chunks l, l+64, l+128, ... of each row (a wave streams 1 KB of a row
// per step), keeps ROWS x M int32 partial sums, and the sums are reduced across
// the wave with xor-shuffles.  The item table travels by value in the kernel
// arguments, so the launch needs no device-side table.
#include "device_common.hpp"
#include "gemv.hpp"

namespace phi_dev {

// Weight rows per wave and waves per workgroup.  At config 4 (60 weights of
// 18432 x 3072) 16-wave workgroups stream 7.0 TB/s against 6.8 with 4 waves:
// 484 against 499 us a sweep at M = 1, 480 against 512 at M = 2 (rows per
// wave 2, 4 and 8 and waves 1-16 measured; 4 x 16 best for both).
constexpr int GEMV_ROWS = 4;
constexpr int GEMV_WAVES = 16;

template <int M>
__global__ __launch_bounds__(GEMV_WAVES * 64) void gemv_kernel(GemvBatch b) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rows_per_block = GEMV_ROWS * GEMV_WAVES;
    const int blocks_per_item = (b.N + rows_per_block - 1) / rows_per_block;
    const int item = blockIdx.x / blocks_per_item;
    const int n0 = (blockIdx.x - item * blocks_per_item) * rows_per_block + wave * GEMV_ROWS;
    if (n0 >= b.N) return;
    const int8_t* W = b.W[item];
    const int chunks = b.K >> 4;

    int acc[GEMV_ROWS][M];
#pragma unroll
    for (int r = 0; r < GEMV_ROWS; r++)
#pragma unroll
        for (int m = 0; m < M; m++) acc[r][m] = 0;

    for (int c = lane; c < chunks; c += 64) {
        v4i w[GEMV_ROWS];
#pragma unroll
        for (int r = 0; r < GEMV_ROWS; r++) {
            const int n = min(n0 + r, b.N - 1);
            w[r] = __builtin_nontemporal_load((const v4i*)(W + (int64_t)n * b.K) + c);
        }
#pragma unroll
        for (int m = 0; m < M; m++) {
            const v4i xv = *((const v4i*)(b.q8 + (int64_t)m * b.K) + c);
#pragma unroll
            for (int r = 0; r < GEMV_ROWS; r++) {
                int t = acc[r][m];
                t = __builtin_amdgcn_sdot4(xv.x, w[r].x, t, false);
                t = __builtin_amdgcn_sdot4(xv.y, w[r].y, t, false);
                t = __builtin_amdgcn_sdot4(xv.z, w[r].z, t, false);
                t = __builtin_amdgcn_sdot4(xv.w, w[r].w, t, false);
                acc[r][m] = t;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < GEMV_ROWS; r++)
#pragma unroll
        for (int m = 0; m < M; m++) {
            int t = acc[r][m];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) t += __shfl_xor(t, off, 64);
            acc[r][m] = t;
        }

    // Lane r*M + m writes output (m, n0 + r).
    if (lane < GEMV_ROWS * M) {
        const int r = lane / M, m = lane - (lane / M) * M;
        const int n = n0 + r;
        if (n < b.N) {
            int a = 0;
#pragma unroll
            for (int rr = 0; rr < GEMV_ROWS; rr++)
#pragma unroll
                for (int mm = 0; mm < M; mm++)
                    if (rr == r && mm == m) a = acc[rr][mm];
            const int64_t off = (int64_t)m * b.ldc[item] + n;
            if (b.c_kind == C_I32) {
                ((int32_t*)b.C[item])[off] = a;
            } else {
                const float sb = (b.sw_scalar_mask >> item) & 1ull ? b.sW[item][0] : b.sW[item][n];
                float bz = 0.0f;
                if (b.bias_kind == BIAS_F32) bz = ((const float*)b.bias[item])[n];
                else if (b.bias_kind == BIAS_BF16) bz = bf16_to_f32(((const uint16_t*)b.bias[item])[n]);
                const float v = fmaf((float)a * b.s8[m], sb, bz);
                if (b.c_kind == C_BF16) ((uint16_t*)b.C[item])[off] = (uint16_t)f32_to_bf16(v);
                else ((float*)b.C[item])[off] = v;
            }
        }
    }
}

hipError_t launch_gemv(hipStream_t stream, const GemvBatch& b) {
    const int rows_per_block = GEMV_ROWS * GEMV_WAVES;
    const unsigned blocks = (unsigned)(b.n_items * ((b.N + rows_per_block - 1) / rows_per_block));
    const dim3 grid(blocks), block(GEMV_WAVES * 64);
    switch (b.M) {
        case 1: hipLaunchKernelGGL(gemv_kernel<1>, grid, block, 0, stream, b); break;
        case 2: hipLaunchKernelGGL(gemv_kernel<2>, grid, block, 0, stream, b); break;
        case 3: hipLaunchKernelGGL(gemv_kernel<3>, grid, block, 0, stream, b); break;
        case 4: hipLaunchKernelGGL(gemv_kernel<4>, grid, block, 0, stream, b); break;
        case 5: hipLaunchKernelGGL(gemv_kernel<5>, grid, block, 0, stream, b); break;
        case 6: hipLaunchKernelGGL(gemv_kernel<6>, grid, block, 0, stream, b); break;
        case 7: hipLaunchKernelGGL(gemv_kernel<7>, grid, block, 0, stream, b); break;
        default: hipLaunchKernelGGL(gemv_kernel<8>, grid, block, 0, stream, b); break;
    }
    return hipGetLastError();
}

}  // namespace phi_dev
