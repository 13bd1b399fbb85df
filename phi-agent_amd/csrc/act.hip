// Elementwise activations between the linears of an MLP:
//   GELU-tanh over [n]                       (core/kernels/ops.cpp:83-89, ElemOp::GeluTanh)
//   SiLU gate [rows, 2*cols] -> [rows, cols] (core/kernels/conv3d_causal.cpp:997-1013,
//                                             dispatch_silu_gate_fused core/kernels/h3_kernels.hpp:116-129)
//
// Both are HBM-bound (bf16: 2 B in, 2 B out per GELU element), so a lane
// moves 8 elements with 16-byte accesses; the maths is the per-element
// helpers of device_common.hpp, so the result does not depend on the
// vector width, and equals the fused quant_rotate pre-ops bit for bit.
#include "device_common.hpp"
#include "gemv.hpp"

namespace phi_dev {

// 8 consecutive elements of bf16 (one 16-B load) or fp32 (two) into fp32.
template <bool BF16>
__device__ __forceinline__ void load8(const void* p, int64_t i, float (&v)[8]) {
    if (BF16) {
        const uint4 a = *(const uint4*)((const uint16_t*)p + i);
        const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            v[2 * k] = bf16_to_f32(w[k] & 0xffffu);
            v[2 * k + 1] = bf16_to_f32(w[k] >> 16);
        }
    } else {
        const float4 a = *(const float4*)((const float*)p + i), b = *(const float4*)((const float*)p + i + 4);
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    }
}

template <bool BF16>
__device__ __forceinline__ void store8(void* p, int64_t i, const float (&v)[8]) {
    if (BF16) {
        *(uint4*)((uint16_t*)p + i) = make_uint4(f32x2_to_bf16x2(v[0], v[1]), f32x2_to_bf16x2(v[2], v[3]),
                                                 f32x2_to_bf16x2(v[4], v[5]), f32x2_to_bf16x2(v[6], v[7]));
    } else {
        *(float4*)((float*)p + i) = make_float4(v[0], v[1], v[2], v[3]);
        *(float4*)((float*)p + i + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
}

__device__ __forceinline__ float load1(const void* p, bool bf16, int64_t i) {
    return bf16 ? bf16_to_f32(((const uint16_t*)p)[i]) : ((const float*)p)[i];
}

__device__ __forceinline__ void store1(void* p, bool bf16, int64_t i, float v) {
    if (bf16) ((uint16_t*)p)[i] = (uint16_t)f32_to_bf16(v);
    else ((float*)p)[i] = v;
}

// One 8-element chunk per lane; n8 = n / 8 chunks (x and y 16-byte aligned).
// In place (x == y, same dtype) is allowed: a lane reads its chunk before
// writing it.
template <bool XB, bool YB>
__global__ __launch_bounds__(256) void gelu_vec_kernel(const void* x, void* y, int64_t n8) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= n8) return;
    float v[8];
    load8<XB>(x, 8 * c, v);
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = gelu_tanh(v[k]);
    store8<YB>(y, 8 * c, v);
}

// Elements [i0, n) one per lane: the tail after the vector chunks, or all of
// a misaligned tensor (grid-stride).
__global__ __launch_bounds__(256) void gelu_scalar_kernel(const void* x, int xb, void* y,
                                                          int yb, int64_t i0, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = i0 + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
        store1(y, yb, i, gelu_tanh(load1(x, xb, i)));
}

template <bool XB, bool YB>
static void launch_gelu_vec(hipStream_t stream, const void* x, void* y, int64_t n8) {
    hipLaunchKernelGGL((gelu_vec_kernel<XB, YB>), dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, stream, x, y, n8);
}

static unsigned scalar_blocks(int64_t n) {
    const int64_t b = (n + 255) / 256;
    return (unsigned)(b < 1 ? 1 : b > 65536 ? 65536 : b);
}

hipError_t launch_gelu(hipStream_t stream, const void* x, int x_bf16, void* y, int y_bf16, int64_t n) {
    const bool vec = ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % 16 == 0) && n / 8 < ((int64_t)1 << 31);
    const int64_t n8 = vec ? n / 8 : 0;
    if (n8 > 0) {
        if (x_bf16) y_bf16 ? launch_gelu_vec<true, true>(stream, x, y, n8) : launch_gelu_vec<true, false>(stream, x, y, n8);
        else y_bf16 ? launch_gelu_vec<false, true>(stream, x, y, n8) : launch_gelu_vec<false, false>(stream, x, y, n8);
    }
    if (8 * n8 < n)
        hipLaunchKernelGGL(gelu_scalar_kernel, dim3(scalar_blocks(n - 8 * n8)), dim3(256), 0, stream, x, x_bf16, y,
                           y_bf16, 8 * n8, n);
    return hipGetLastError();
}

// SiLU gate, cols % 8 == 0 and 16-byte aligned rows: one 8-column chunk per
// lane, the gate at gx[r][c], the value at gx[r][cols + c].
template <bool XB, bool YB>
__global__ __launch_bounds__(256) void silu_gate_vec_kernel(const void* __restrict__ gx, int64_t ldx,
                                                            void* __restrict__ out, int64_t ldo, int64_t rows,
                                                            int64_t cols) {
    const int64_t cpr = cols / 8;
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= rows * cpr) return;
    const int64_t r = c / cpr, k = 8 * (c - r * cpr);
    float g[8], v[8];
    load8<XB>(gx, r * ldx + k, g);
    load8<XB>(gx, r * ldx + cols + k, v);
#pragma unroll
    for (int j = 0; j < 8; j++) g[j] = silu_mul(g[j], v[j]);
    store8<YB>(out, r * ldo + k, g);
}

__global__ __launch_bounds__(256) void silu_gate_scalar_kernel(const void* __restrict__ gx, int xb, int64_t ldx,
                                                               void* __restrict__ out, int yb, int64_t ldo,
                                                               int64_t rows, int64_t cols) {
    const int64_t n = rows * cols, stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
        const int64_t r = i / cols, k = i - r * cols;
        store1(out, yb, r * ldo + k, silu_mul(load1(gx, xb, r * ldx + k), load1(gx, xb, r * ldx + cols + k)));
    }
}

template <bool XB, bool YB>
static void launch_silu_vec(hipStream_t stream, const void* gx, int64_t ldx, void* out, int64_t ldo, int64_t rows,
                            int64_t cols) {
    const int64_t chunks = rows * (cols / 8);
    hipLaunchKernelGGL((silu_gate_vec_kernel<XB, YB>), dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream,
                       gx, ldx, out, ldo, rows, cols);
}

hipError_t launch_silu_gate(hipStream_t stream, const void* gx, int x_bf16, int64_t ldx, void* out, int y_bf16,
                            int64_t ldo, int64_t rows, int64_t cols) {
    const int xe = x_bf16 ? 2 : 4, ye = y_bf16 ? 2 : 4;
    const bool vec = cols % 8 == 0 && (uintptr_t)gx % 16 == 0 && (uintptr_t)out % 16 == 0 && (ldx * xe) % 16 == 0 &&
                     (ldo * ye) % 16 == 0 && rows * (cols / 8) < ((int64_t)1 << 31);
    if (vec) {
        if (x_bf16) y_bf16 ? launch_silu_vec<true, true>(stream, gx, ldx, out, ldo, rows, cols)
                           : launch_silu_vec<true, false>(stream, gx, ldx, out, ldo, rows, cols);
        else y_bf16 ? launch_silu_vec<false, true>(stream, gx, ldx, out, ldo, rows, cols)
                    : launch_silu_vec<false, false>(stream, gx, ldx, out, ldo, rows, cols);
    } else {
        hipLaunchKernelGGL(silu_gate_scalar_kernel, dim3(scalar_blocks(rows * cols)), dim3(256), 0, stream, gx, x_bf16,
                           ldx, out, y_bf16, ldo, rows, cols);
    }
    return hipGetLastError();
}

}  // namespace phi_dev
