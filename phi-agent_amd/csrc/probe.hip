// Ceiling probes for the benchmark (bench.py --config mfma_ceiling): what one
// MI355X sustains with no data movement around the MFMAs, and how fast a CU
// streams operands into LDS by buffer_load ... lds.  Measurement code only:
// built into lib/libphi_probe.so, which the product library does not link.
//
//   phi_probe_mfma  every wave issues v_mfma_i32_32x32x32_i8 back to back on
//                   16 independent 32 x 32 accumulators (the headline GEMM's
//                   wave tile), operands held in registers:
//                     mode 0  all-zero operands (no toggling: the clock ceiling)
//                     mode 1  one random A and B fragment per lane (static inputs)
//                     mode 2  8 A and 8 B random fragments used as the GEMM's
//                             wave uses a K-step's fragments (each 4 times),
//                             rotated by a cheap XOR every K-step so the
//                             operands change as they do when read from LDS
//   phi_probe_lds_dma  every wave streams 16 rows x 64 bytes per instruction
//                   from a window of global memory into LDS, 4 K-steps of the
//                   headline tile's A and B in flight, with no MFMAs.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void* lptr_t;
constexpr int kRsrcWord3 = 0x00020000;

template <int MODE>
__global__ __launch_bounds__(256) void mfma_probe(const int8_t* ops, int iters, int* sink) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v4i a[8], b[8];
#pragma unroll
    for (int f = 0; f < 8; f++) {
        if (MODE == 0) {
            a[f] = v4i{0, 0, 0, 0};
            b[f] = v4i{0, 0, 0, 0};
        } else {
            const int fa = MODE == 1 ? 0 : f;
            a[f] = *(const v4i*)(ops + ((wave * 16 + fa) * 64 + lane) * 16);
            b[f] = *(const v4i*)(ops + ((wave * 16 + 8 + fa) * 64 + lane) * 16);
        }
    }
    v16i acc[16];
#pragma unroll
    for (int q = 0; q < 16; q++) acc[q] = v16i{};
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
            for (int q = 0; q < 16; q++)
                acc[q] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b[(q >> 2) + 4 * s], a[(q & 3) + 4 * s], acc[q], 0, 0, 0);
        if (MODE == 2) {
            const int x = 0x5a3c96e1 * (it + 1) + lane;
#pragma unroll
            for (int f = 0; f < 8; f++) {
                a[f] ^= v4i{x, x >> 3, x >> 5, x >> 7};
                b[f] ^= v4i{x >> 1, x >> 2, x >> 4, x >> 6};
            }
        }
    }
    int t = 0;
#pragma unroll
    for (int q = 0; q < 16; q++)
#pragma unroll
        for (int r = 0; r < 16; r++) t += acc[q][r];
    if (t == 0x7fffffff) sink[blockIdx.x * 4 + wave] = t;  // keeps the MFMAs live
}

__global__ __launch_bounds__(256) void lds_dma_probe(const int8_t* src, int window, int iters, int* sink) {
    __shared__ __align__(16) int8_t st[4][4][8192];  // wave, stage, 8 loads of 1 KB
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & 3;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, window, kRsrcWord3);
    // lane l fetches row l / 4, chunk l % 4 of a 16-row x 64-byte piece at a
    // 3072-byte row pitch (the headline A and B rows).
    const int vo = (lane >> 2) * 3072 + (lane & 3) * 16;
    // Every load stays below window: a piece spans 16 rows at the pitch.
    // Each wave starts at its own share of the window, so a window much
    // larger than the MALL is read once, from HBM.
    const int span = window - (1 << 19);
    const int share = (int)(((long long)span / ((long long)gridDim.x * 4)) & ~63ll);
    const int base = (int)(((long long)blockIdx.x * 4 + wave) * share % span);
    for (int it = 0; it < iters; it++) {
        const int s = it & 3;
        const int off = (int)(((long long)base + (long long)it * 64) % span);
#pragma unroll
        for (int j = 0; j < 8; j++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lptr_t)(&st[wave][s][j * 1024]), 16, vo,
                                                     off + j * 16 * 3072, 0, 0);
        // Keep three later K-steps in flight, as the GEMM's pipeline does.
        __builtin_amdgcn_s_waitcnt((8 * 3 & 15) | (7 << 4) | (((8 * 3) >> 4) & 3) << 14);
    }
    __builtin_amdgcn_s_waitcnt(0 | (7 << 4));
    __syncthreads();
    if (st[wave][0][lane] == 127 && st[wave][1][lane] == -128 && lane == 0) sink[blockIdx.x] = 1;
}

}  // namespace

extern "C" {

int phi_probe_mfma(void* stream, const int8_t* ops, int mode, int iters, int* sink, int grid) {
    switch (mode) {
        case 0: hipLaunchKernelGGL(mfma_probe<0>, dim3(grid), dim3(256), 0, (hipStream_t)stream, ops, iters, sink); break;
        case 1: hipLaunchKernelGGL(mfma_probe<1>, dim3(grid), dim3(256), 0, (hipStream_t)stream, ops, iters, sink); break;
        default: hipLaunchKernelGGL(mfma_probe<2>, dim3(grid), dim3(256), 0, (hipStream_t)stream, ops, iters, sink); break;
    }
    return (int)hipGetLastError();
}

int phi_probe_lds_dma(void* stream, const int8_t* src, long long window, int iters, int* sink, int grid) {
    if (window < (1 << 20) || window > (1ll << 31) - 1) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(lds_dma_probe, dim3(grid), dim3(256), 0, (hipStream_t)stream, src, (int)window, iters, sink);
    return (int)hipGetLastError();
}

}  // extern "C"
