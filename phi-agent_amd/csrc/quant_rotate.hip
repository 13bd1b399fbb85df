// Rotate + quantise activations, one row (token) per workgroup, single pass.
//
// Maths (core/host/quant.cpp:109-169, device form core/kernels/int8_gemm.cpp:699-802):
//   per 256-group: y = H x with H = (J - 2R)^{(x)4} / 16, applied as four radix-4
//   passes over the base-4 digits of the in-group index (stride 1, 4, 16, 64);
//   each pass maps (x0,x1,x2,x3) to y[j] = (((x0+x1)+x2)+x3) - 2 x[3-j], then
//   every element is multiplied by 1/16;
//   amax = max |y| over the row; scale = amax > 1e-30 ? amax/qmax : 1;
//   q = clamp(round(y * (1/scale)), +-qmax), ties away from zero by default.
//
// Layout of the work.  A 16-lane team owns one 256-group.  In phase A lane l
// loads elements 16l..16l+15 (coalesced 64-B / 32-B runs), so digits 0 and 1
// of the index are in-lane and the first two passes run in registers.  The
// values go to LDS; in phase B lane l reads back the 16 elements whose low two
// digits equal l (a transpose through LDS), so digits 2 and 3 are in-lane and
// the last two passes also run in registers.  The rotated row stays in LDS
// (the reference reads the row from global memory twice instead), the row
// amax is reduced across the workgroup, and phase C quantises 16 contiguous
// elements per lane and writes them with one 16-byte store.
//
// LDS: a group's 256 floats sit as 16 slots of 20 floats (16 values + 4 pad,
// so the 16-B slot accesses of 8 lanes land on 8 distinct 4-bank windows), and
// groups are 336 floats apart (a 16-bank shift between the teams of a wave).
#include "device_common.hpp"

namespace phi_dev {

constexpr int QR_PITCH = 20;
constexpr int QR_GSTRIDE = 16 * QR_PITCH + 16;

// One radix-4 pass over 16 in-register values: the digit with stride `st`
// (1 or 4) varies, the other digit selects the quadruple.
template <int ST>
__device__ __forceinline__ void bfly16(float (&v)[16]) {
#pragma unroll
    for (int o = 0; o < 4; o++) {
        const int b = ST == 1 ? 4 * o : o;
        const float x0 = v[b], x1 = v[b + ST], x2 = v[b + 2 * ST], x3 = v[b + 3 * ST];
        const float sum = ((x0 + x1) + x2) + x3;
        v[b] = sum - 2.0f * x3;
        v[b + ST] = sum - 2.0f * x2;
        v[b + 2 * ST] = sum - 2.0f * x1;
        v[b + 3 * ST] = sum - 2.0f * x0;
    }
}

template <bool BF16_IN>
__global__ __launch_bounds__(1024) void quant_rotate_rows(const void* __restrict__ x, int64_t ldx,
                                                          int K, int8_t* __restrict__ q,
                                                          int64_t ldq, float* __restrict__ s,
                                                          float qmax, int half_even, int rotate) {
    extern __shared__ __align__(16) float lds[];
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const int nthreads = blockDim.x;
    const int team = tid >> 4, tl = tid & 15, nteams = nthreads >> 4;
    const int G = K >> 8;
    float* red = lds + G * QR_GSTRIDE;

    // ---- phase A: load, passes over digits 0 and 1, stage into LDS ----
    for (int g = team; g < G; g += nteams) {
        float v[16];
        const int64_t e0 = (int64_t)g * 256 + tl * 16;
        if (BF16_IN) {
            const uint4* src = (const uint4*)((const uint16_t*)x + (int64_t)row * ldx + e0);
            const uint4 a = src[0], b = src[1];
            const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                v[2 * i] = bf16_to_f32(w[i] & 0xffffu);
                v[2 * i + 1] = bf16_to_f32(w[i] >> 16);
            }
        } else {
            const float4* src = (const float4*)((const float*)x + (int64_t)row * ldx + e0);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 t = src[i];
                v[4 * i] = t.x;
                v[4 * i + 1] = t.y;
                v[4 * i + 2] = t.z;
                v[4 * i + 3] = t.w;
            }
        }
        if (rotate) {
            bfly16<1>(v);
            bfly16<4>(v);
        }
        float4* dst = (float4*)(lds + g * QR_GSTRIDE + tl * QR_PITCH);
#pragma unroll
        for (int i = 0; i < 4; i++) dst[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    }
    __syncthreads();

    // ---- phase B: transposed read, passes over digits 2 and 3, x 1/16, amax ----
    float amax = 0.0f;
    for (int g = team; g < G; g += nteams) {
        float* base = lds + g * QR_GSTRIDE + tl;
        float w[16];
#pragma unroll
        for (int j = 0; j < 16; j++) w[j] = base[j * QR_PITCH];
        if (rotate) {
            bfly16<1>(w);
            bfly16<4>(w);
#pragma unroll
            for (int j = 0; j < 16; j++) w[j] = w[j] * (1.0f / 16.0f);
#pragma unroll
            for (int j = 0; j < 16; j++) base[j * QR_PITCH] = w[j];
        }
#pragma unroll
        for (int j = 0; j < 16; j++) amax = fmaxf(amax, fabsf(w[j]));
    }
    amax = wave_max(amax);
    if ((tid & 63) == 0) red[tid >> 6] = amax;
    __syncthreads();
    float rmax = red[0];
    for (int w = 1; w < (nthreads >> 6); w++) rmax = fmaxf(rmax, red[w]);
    const float scale = rmax > 1e-30f ? rmax / qmax : 1.0f;
    const float inv = 1.0f / scale;

    // ---- phase C: quantise 16 contiguous elements per lane, 16-B store ----
    for (int g = team; g < G; g += nteams) {
        const float4* src = (const float4*)(lds + g * QR_GSTRIDE + tl * QR_PITCH);
        uint32_t packed[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 t = src[i];
            packed[i] = pack4(quant_code(t.x, inv, qmax, half_even), quant_code(t.y, inv, qmax, half_even),
                              quant_code(t.z, inv, qmax, half_even), quant_code(t.w, inv, qmax, half_even));
        }
        uint4* dst = (uint4*)(q + (int64_t)row * ldq + (int64_t)g * 256 + tl * 16);
        *dst = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    }
    if (tid == 0) s[row] = scale;
}

// Host-side launcher.  Validation is done by the C ABI layer.
hipError_t launch_quant_rotate(hipStream_t stream, const void* x, bool bf16_in, int64_t rows,
                               int64_t K, int64_t ldx, int8_t* q, int64_t ldq, float* s,
                               float qmax, int half_even, int rotate) {
    const int G = (int)(K / 256);
    int threads = ((16 * G + 63) / 64) * 64;
    if (threads > 1024) threads = 1024;
    const size_t lds_bytes = ((size_t)G * QR_GSTRIDE + 16) * sizeof(float);
    if (lds_bytes > 65536) {
        hipError_t e = hipFuncSetAttribute(bf16_in ? (const void*)quant_rotate_rows<true> : (const void*)quant_rotate_rows<false>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes);
        if (e != hipSuccess) return e;
    }
    if (bf16_in) {
        hipLaunchKernelGGL(quant_rotate_rows<true>, dim3((unsigned)rows), dim3(threads), lds_bytes,
                           stream, x, ldx, (int)K, q, ldq, s, qmax, half_even, rotate);
    } else {
        hipLaunchKernelGGL(quant_rotate_rows<false>, dim3((unsigned)rows), dim3(threads), lds_bytes,
                           stream, x, ldx, (int)K, q, ldq, s, qmax, half_even, rotate);
    }
    return hipGetLastError();
}

size_t quant_rotate_lds_bytes(int64_t K) { return ((size_t)(K / 256) * QR_GSTRIDE + 16) * sizeof(float); }

}  // namespace phi_dev
