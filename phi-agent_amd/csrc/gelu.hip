// GELU-tanh between the two MLP linears, fp32 arithmetic in the operation
// order of core/kernels/ops.cpp:83-89:
//   t = 0.7978845608028654 * (x + 0.044715 * x * x * x);  y = 0.5 * x * (1 + tanh(t))
// bf16 in/out are converted exactly / RNE.  tanhf is the device library's.
#include "device_common.hpp"
#include "gemv.hpp"

namespace phi_dev {

__device__ __forceinline__ float gelu_tanh(float a) {
    const float t = 0.7978845608028654f * (a + 0.044715f * a * a * a);
    return 0.5f * a * (1.0f + tanhf(t));
}

__global__ __launch_bounds__(256) void gelu_kernel(const void* __restrict__ x, int x_bf16,
                                                   void* __restrict__ y, int y_bf16, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float a = x_bf16 ? bf16_to_f32(((const uint16_t*)x)[i]) : ((const float*)x)[i];
        const float v = gelu_tanh(a);
        if (y_bf16) ((uint16_t*)y)[i] = (uint16_t)f32_to_bf16(v);
        else ((float*)y)[i] = v;
    }
}

hipError_t launch_gelu(hipStream_t stream, const void* x, int x_bf16, void* y, int y_bf16, int64_t n) {
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(gelu_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, x, x_bf16, y, y_bf16, n);
    return hipGetLastError();
}

}  // namespace phi_dev
