// Device helpers shared by the gfx950 kernels of the quantized linear.
//
// Everything here is exact integer / IEEE arithmetic: the kernels are built
// with -ffp-contract=off, so a product is never fused into a following add
// unless the code says fmaf().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

namespace phi_dev {

// An integer tuning switch from the environment (the A/B switches the tests
// and the bench set between launches): its value when set and inside
// [lo, hi], else `dflt`.  Read at each launch, so a switch set between calls
// takes effect; a value out of range is ignored rather than passed to a kernel.
inline int env_switch(const char* name, int dflt, int lo, int hi) {
    const char* e = getenv(name);
    if (!e || !*e) return dflt;
    char* end = nullptr;
    const long v = strtol(e, &end, 10);
    return (*end == '\0' && v >= lo && v <= hi) ? (int)v : dflt;
}

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

// bf16 bits -> fp32, exact.
__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// fp32 -> bf16 bits, round to nearest even.  The reference's conversion is the
// integer carry rule (add 0x7fff plus the kept lsb, keep the top half;
// core/util/media_common.cpp:187-193), which is exactly round-to-nearest-even
// for every finite value; gfx950's v_cvt_pk_bf16_f32 (what a __bf16 cast
// lowers to) rounds the same way in one instruction.  The two differ only in
// NaN payloads, which the linear cannot produce from finite operands.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
    return __builtin_bit_cast(unsigned short, (__bf16)f);
}

// Two values in one v_cvt_pk_bf16_f32: lo in bits 0..15, hi in bits 16..31.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float lo, float hi) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

// IEEE binary16 -> fp32 (exact).
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)h);
}

// E4M3FN: bias 7, no infinity, S.1111.111 is NaN.
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
    const uint32_t s = (b >> 7) & 1u, e = (b >> 3) & 15u, m = b & 7u;
    float v;
    if (e == 15u && m == 7u) v = __uint_as_float(0x7fc00000u);
    else if (e == 0u) v = (float)m * 0x1p-9f;
    else v = (float)(8u + m) * __uint_as_float((e - 10u + 127u) << 23);
    return s ? -v : v;
}

// E5M2: bias 15, IEEE-shaped.
__device__ __forceinline__ float e5m2_to_f32(uint32_t b) {
    const uint32_t s = (b >> 7) & 1u, e = (b >> 2) & 31u, m = b & 3u;
    float v;
    if (e == 31u) v = m == 0u ? __uint_as_float(0x7f800000u) : __uint_as_float(0x7fc00000u);
    else if (e == 0u) v = (float)m * 0x1p-16f;
    else v = (float)(4u + m) * __uint_as_float((e - 17u + 127u) << 23);
    return s ? -v : v;
}

// Nearest integer to d, ties away from zero, exactly: d - trunc(d) is exact in
// fp32, so the tie test sees the true fraction.  Equal to the reference's
// (long)((double)d +- 0.5) for every fp32 d (core/host/quant.cpp:163-166).
__device__ __forceinline__ float round_half_away(float d) {
    const float t = truncf(d);
    const float frac = d - t;
    return fabsf(frac) >= 0.5f ? t + copysignf(1.0f, d) : t;
}

// v * inv onto the integer grid, clamped to +-qmax (qmax integral).
__device__ __forceinline__ int quant_code(float v, float inv, float qmax, int half_even) {
    const float d = v * inv;
    float r = half_even ? rintf(d) : round_half_away(d);
    r = fminf(fmaxf(r, -qmax), qmax);
    return (int)r;
}

// Four int codes -> one little-endian dword of int8.
__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return ((uint32_t)a & 0xffu) | (((uint32_t)b & 0xffu) << 8) | (((uint32_t)c & 0xffu) << 16) |
           ((uint32_t)d << 24);
}

// GELU, tanh form (core/kernels/ops.cpp:83-89):
//   t = 0.7978845608028654 * (x + 0.044715 * x^3);  y = 0.5 * x * (1 + tanh(t)),
// t with the one contraction NVRTC's default --fmad=true makes in it (the
// cube's last product fused into the add).  y is evaluated through the
// identity 0.5 (1 + tanh t) = 1 / (1 + e^(-2t)) as x * rcp(1 + exp2(-2 log2(e) t))
// on v_exp_f32 and v_rcp_f32 (1 ulp each): branch-free, about a quarter of
// the device library tanhf's instructions, and without the cancellation in
// 1 + tanh(t) for t << 0.  It stays within 3e-7 |x| of the reference's
// formula (2.3e-7 |x| measured over 4 M inputs; the GPU tests allow 4e-7);
// where that formula cancels to 0 (x < -9) this gives the tiny true value.  Every kernel that applies GELU calls this, so a fused form
// equals the standalone op bit for bit.
__device__ __forceinline__ float gelu_tanh(float a) {
    const float t = 0.7978845608028654f * fmaf(0.044715f * a * a, a, a);
    return a * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t * -2.8853900817779268f));
}

// The SiLU gate: silu(g) * v = (g / (1 + exp(-g))) * v, correctly rounded
// division (core/kernels/conv3d_causal.cpp:997-1013, OP_SILU_GATE
// core/kernels/ops.cpp:75).  expf is the device library's.
__device__ __forceinline__ float silu_mul(float g, float v) { return (g / (1.0f + expf(-g))) * v; }

// Wave-wide max over 64 lanes.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

}  // namespace phi_dev
