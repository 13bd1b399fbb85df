// The per-row scale of the rotate+quantise prologue and the factors its codes
// use: the reference's
//   scale = amax > 1e-30 ? amax / qmax : 1,   inv = 1 / scale
// (core/host/quant.cpp:134-169, device core/kernels/int8_gemm.cpp:747-801),
// both IEEE divisions, correctly rounded.
//
// The rotation's final 1/16 is applied to the amax and to inv instead of to
// every element.  max |w|/16 rounds to the max of the rounded |w|/16, so the
// amax and scale are exact.  When inv/16 is exact (inv >= 2^-122, i.e. amax
// below ~2^122 qmax), round(w * (inv/16)) = round((w/16) * inv) wherever w/16
// is exact, and where it is not (|w| < 2^-122) the code is 0 either way
// (|w| inv/16 < 1e-5).  Otherwise (fold false) each element is scaled by
// pre = 1/16 first.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace phi_dev {

struct QtScale {
    float scale, pre, post;
    bool fold;
};

__device__ __forceinline__ QtScale qt_scale(uint32_t amax, float qmax, int rotate) {
    const float sixteenth = rotate ? 1.0f / 16.0f : 1.0f;
    const float rmax = __uint_as_float(amax) * sixteenth;
    QtScale c;
    c.scale = rmax > 1e-30f ? rmax / qmax : 1.0f;
    const float inv = 1.0f / c.scale;
    c.fold = !rotate || inv >= 0x1p-122f;
    c.pre = c.fold ? 1.0f : sixteenth;
    c.post = c.fold ? inv * sixteenth : inv;
    return c;
}

// rmax / qmax for 2^-90 <= rmax < 2^122 and an integer qmax in [1, 127],
// from qrcp = 1/qmax rounded (the host's division): q0 = rmax qrcp, then one
// correction with the exact remainder fma(-q0, qmax, rmax).  Every value is
// normal there, so the result depends only on rmax's significand; it equals
// the IEEE quotient for all 2^23 significands and every such qmax (checked
// exhaustively on the CPU, tests/cpp/scale_exact.c, and on the GPU).
__device__ __forceinline__ float qt_div_qmax(float rmax, float qmax, float qrcp) {
    const float q0 = rmax * qrcp;
    return fmaf(fmaf(-q0, qmax, rmax), qrcp, q0);
}

// 1 / b for 2^-97 <= b <= 2^122, bb = b's bits: v_rcp_f32's estimate and
// two Newton steps y' = fma(fma(-b, y, 1), y, y).  From any estimate within
// 2 ulps of the rounded reciprocal this gives the rounded reciprocal for
// every significand but all ones (checked exhaustively on the CPU,
// tests/cpp/scale_exact.c, and on the GPU with v_rcp_f32 itself).  There
// 1/b = 2^-(e+1) (1 + 2^-24 + 2^-48 + ...), which rounds up to
// 2^-(e+1) (1 + 2^-23): b's biased exponent E gives the bits
// ((253 - E) << 23) | 1 directly.
__device__ __forceinline__ float qt_rcp_bits(float b, uint32_t bb) {
    const float y0 = __builtin_amdgcn_rcpf(b);
    const float y1 = fmaf(fmaf(-b, y0, 1.0f), y0, y0);
    const float y2 = fmaf(fmaf(-b, y1, 1.0f), y1, y1);
    return (bb & 0x7fffffu) == 0x7fffffu ? __uint_as_float(((253u - (bb >> 23)) << 23) | 1u) : y2;
}

// qt_rcp_bits for a wave-uniform b (the test on its bits runs on the scalar
// unit).
__device__ __forceinline__ float qt_rcp(float b) {
    return qt_rcp_bits(b, __builtin_amdgcn_readfirstlane(__float_as_uint(b)));
}

// qt_scale for a rotated row whose amax is finite and below 2^126 (rmax
// below 2^122, so inv >= 2^-122 and the 1/16 folds), with the divisions above
// where they are exact (rmax >= 2^-90, so scale >= 2^-97) and qt_scale's
// otherwise.  amax is wave-uniform.
__device__ __forceinline__ QtScale qt_scale_fast(uint32_t amax, float qmax, float qrcp) {
    // rmax >= 2^-90 is amax >= 2^-86, compared as the bits of a non-negative
    // float.
    if (__builtin_amdgcn_readfirstlane(amax) < 0x14800000u) return qt_scale(amax, qmax, 1);
    const float rmax = __uint_as_float(amax) * (1.0f / 16.0f);
    QtScale c;
    c.scale = qt_div_qmax(rmax, qmax, qrcp);
    c.fold = true;
    c.pre = 1.0f;
    c.post = qt_rcp(c.scale) * (1.0f / 16.0f);
    return c;
}

}  // namespace phi_dev
