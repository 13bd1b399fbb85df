// The 272 x 192 persistent GEMM (i8_gemm_t272.hip) compiled a second time,
// into namespace phi_dev_t272trace, with its timeline hooks defined: one
// record of stamps per workgroup, each point in the shader clock (s_memtime,
// cycles) and the kernel's start and end also in the 100 MHz real-time
// clock.  Measurement tooling for bench.py (--config c1_up_t272_tiles /
// c1_down_t272_tiles / c2_t272_tiles); the product library does not contain
// it.
//
// The per-workgroup record (64 words):
//   [0]           kernel start, shader clock
//   [1 + 3 i + p] tile i < 16, point p (0 start, 1 K-loop end, 2 epilogue end), shader clock
//   [49]          kernel end, shader clock
//   [50]          the XCD the workgroup ran on
//   [51], [52]    kernel start and end, real-time clock
#include <hip/hip_runtime.h>
#include <stdint.h>

__shared__ unsigned long long phi_t272_lds[64];
__device__ unsigned long long* phi_t272_out;

#define PHI_T272_STAMP(tile, point) \
    if (threadIdx.x == 0 && (tile) < 16) phi_t272_lds[1 + 3 * (tile) + (point)] = __builtin_amdgcn_s_memtime();
#define PHI_T272_TRACE_BEGIN                                  \
    if (threadIdx.x < 64) phi_t272_lds[threadIdx.x] = 0;      \
    __syncthreads();                                          \
    if (threadIdx.x == 0) {                                   \
        phi_t272_lds[51] = __builtin_amdgcn_s_memrealtime();  \
        phi_t272_lds[0] = __builtin_amdgcn_s_memtime();       \
    }
#define PHI_T272_TRACE_END                                                        \
    __syncthreads();                                                              \
    if (threadIdx.x == 0) {                                                       \
        phi_t272_lds[49] = __builtin_amdgcn_s_memtime();                          \
        phi_t272_lds[52] = __builtin_amdgcn_s_memrealtime();                      \
        unsigned int xcc_;                                                        \
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc_));       \
        phi_t272_lds[50] = xcc_ & 15;                                             \
    }                                                                             \
    __syncthreads();                                                              \
    if (threadIdx.x < 64) phi_t272_out[blockIdx.x * 64 + threadIdx.x] = phi_t272_lds[threadIdx.x];

#define phi_dev phi_dev_t272trace
#include "i8_gemm_t272.hip"
#undef phi_dev

extern "C" {

// The traced GEMM: bf16 C [M, N] = fma((float)(A . B^T) * sA, sB[0], bf16
// bias) on K-tiled operands (kt = 1) or row-major ones of pitch K (kt = 0),
// one record of 64 words per workgroup into out (slots words).  0 on success,
// else the HIP error code.
int phi_probe_t272_trace(void* stream, const int8_t* A, const int8_t* B, const float* sA, const float* sB,
                         const void* bias, void* C, int M, int N, int K, unsigned long long* out, long long slots,
                         int kt) {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return (int)hipErrorInvalidDevice;
    phi_dev_t272trace::GemmParams p{};
    p.A = A;
    p.B = B;
    p.sA = sA;
    p.sB = sB;
    p.bias = bias;
    p.C = C;
    p.lda = K;
    p.ldb = K;
    p.ldc = N;
    p.M = M;
    p.N = N;
    p.K = K;
    p.sb_scalar = 1;
    p.bias_kind = bias ? phi_dev_t272trace::BIAS_BF16 : phi_dev_t272trace::BIAS_NONE;
    p.c_kind = phi_dev_t272trace::C_BF16;
    p.group_m = 4;
    p.kt = kt ? 1 : 0;
    if (M <= 0 || N <= 0 || !phi_dev_t272trace::t272_ok(p)) return (int)hipErrorInvalidValue;
    const long long tiles = phi_dev_t272trace::t272_tile_count(M, N);
    if ((tiles < cus ? tiles : cus) * 64 > slots) return (int)hipErrorInvalidValue;
    hipError_t e = hipMemcpyToSymbolAsync(HIP_SYMBOL(phi_t272_out), &out, sizeof(out), 0, hipMemcpyHostToDevice,
                                          (hipStream_t)stream);
    if (e != hipSuccess) return (int)e;
    return (int)phi_dev_t272trace::launch_i8_gemm_t272((hipStream_t)stream, p, cus);
}

// The traced W4A8 form (i8_gemm_t272w4_kernel): A K-tiled, B the packed codes
// [N, ldb] with the prepared table lut [N, K / group, 16], per-row scales sB,
// bf16 bias and output.
int phi_probe_t272w4_trace(void* stream, const int8_t* A, const uint8_t* codes, long long ldb, const int8_t* lut,
                           int group, const float* sA, const float* sB, const void* bias, void* C, int M, int N, int K,
                           unsigned long long* out, long long slots) {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return (int)hipErrorInvalidDevice;
    if (group <= 0 || (group & (group - 1)) != 0 || K % group != 0) return (int)hipErrorInvalidValue;
    phi_dev_t272trace::GemmParams p{};
    p.A = A;
    p.B = (const int8_t*)codes;
    p.sA = sA;
    p.sB = sB;
    p.bias = bias;
    p.C = C;
    p.lda = K;
    p.ldb = ldb;
    p.ldc = N;
    p.M = M;
    p.N = N;
    p.K = K;
    p.sb_scalar = 0;
    p.bias_kind = bias ? phi_dev_t272trace::BIAS_BF16 : phi_dev_t272trace::BIAS_NONE;
    p.c_kind = phi_dev_t272trace::C_BF16;
    p.group_m = 4;
    p.kt = 1;
    p.lut = lut;
    p.lut_groups = K / group;
    int gs = 0;
    while ((1 << gs) < group) gs++;
    p.group_shift = gs;
    if (M <= 0 || N <= 0 || !phi_dev_t272trace::t272w4_ok(p)) return (int)hipErrorInvalidValue;
    const long long tiles = phi_dev_t272trace::t272_tile_count(M, N);
    if ((tiles < cus ? tiles : cus) * 64 > slots) return (int)hipErrorInvalidValue;
    hipError_t e = hipMemcpyToSymbolAsync(HIP_SYMBOL(phi_t272_out), &out, sizeof(out), 0, hipMemcpyHostToDevice,
                                          (hipStream_t)stream);
    if (e != hipSuccess) return (int)e;
    return (int)phi_dev_t272trace::launch_i8_gemm_t272w4((hipStream_t)stream, p, cus);
}

}  // extern "C"
