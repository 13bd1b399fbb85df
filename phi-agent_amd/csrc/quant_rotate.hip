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
// An element-wise pre-op can run on every input element before the rotation,
// so the tensor between it and the linear never goes through memory: the
// adaLN modulation (QR_MOD), GELU-tanh (QR_GELU) or the SiLU gate over a
// [gate | value] row (QR_SILU_GATE).  They use the same per-element functions
// as the standalone kernels, so fused and unfused agree bit for bit where the
// unfused intermediate is fp32.
//
// LDS: a group's 256 floats sit as 16 slots of 20 floats (16 values + 4 pad,
// so the 16-B slot accesses of 8 lanes land on 8 distinct 4-bank windows), and
// groups are 336 floats apart (a 16-bank shift between the teams of a wave).
#include <cstdlib>

#include "device_common.hpp"
#include "i8_gemm.hpp"
#include "persist_common.hpp"
#include "qt_scale.hpp"

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

// Modulation before the rotation (the DiT's adaLN ModAdd, fused):
// v = fma(v, 1 + scale[col], shift[col]), the reference's `a * (1 + b) + c`
// (core/kernels/ops.cpp:82, ModAdd core/kernels/gpu_ops.hpp:29-35) as NVRTC's
// default --fmad=true contracts it.  scale or shift may be NULL (0).
__device__ __forceinline__ void modulate16(float (&v)[16], const float* __restrict__ sc, const float* __restrict__ sh,
                                           int64_t col) {
    float b[16], c[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 tb = sc ? *(const float4*)(sc + col + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 tc = sh ? *(const float4*)(sh + col + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
        b[4 * i] = tb.x, b[4 * i + 1] = tb.y, b[4 * i + 2] = tb.z, b[4 * i + 3] = tb.w;
        c[4 * i] = tc.x, c[4 * i + 1] = tc.y, c[4 * i + 2] = tc.z, c[4 * i + 3] = tc.w;
    }
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = fmaf(v[i], 1.0f + b[i], c[i]);
}

// 16 consecutive input elements at element offset off, as fp32.
template <bool BF16_IN>
__device__ __forceinline__ void load16(const void* __restrict__ x, int64_t off, float (&v)[16]) {
    if (BF16_IN) {
        const uint4* src = (const uint4*)((const uint16_t*)x + off);
        const uint4 a = src[0], b = src[1];
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            v[2 * i] = bf16_to_f32(w[i] & 0xffffu);
            v[2 * i + 1] = bf16_to_f32(w[i] >> 16);
        }
    } else {
        const float4* src = (const float4*)((const float*)x + off);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 t = src[i];
            v[4 * i] = t.x;
            v[4 * i + 1] = t.y;
            v[4 * i + 2] = t.z;
            v[4 * i + 3] = t.w;
        }
    }
}

template <bool BF16_IN>
__global__ __launch_bounds__(1024) void quant_rotate_rows(const void* __restrict__ x, int64_t ldx,
                                                          int K, int8_t* __restrict__ q,
                                                          int64_t ldq, float* __restrict__ s,
                                                          float qmax, int half_even, int rotate,
                                                          QrPre pre) {
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
        load16<BF16_IN>(x, (int64_t)row * ldx + e0, v);
        if (pre.op == QR_MOD) {
            modulate16(v, pre.sc, pre.sh, e0);
        } else if (pre.op == QR_GELU) {
#pragma unroll
            for (int i = 0; i < 16; i++) v[i] = gelu_tanh(v[i]);
        } else if (pre.op == QR_SILU_GATE) {
            float u[16];
            load16<BF16_IN>(x, (int64_t)row * ldx + pre.off2 + e0, u);
#pragma unroll
            for (int i = 0; i < 16; i++) v[i] = silu_mul(v[i], u[i]);
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

// ---------------------------------------------------------------------------
// Register-resident form, K <= 16384 (at most 64 groups).
//
// A wave works on 4R consecutive 256-groups of one row in R rounds of four,
// one 16-lane team per group, and keeps its rotated values in registers (16
// per lane per round) until the row amax is known.  WPR = ceil(G / 4R) waves
// cover a row (threadIdx.x) and a block holds RPB rows (threadIdx.y); only the
// amax crosses waves (one barrier, none when WPR is 1).  The two transposes
// of a round go through a 16x16 tile private to the team: a wave's LDS
// operations complete in issue order, so they need no barrier.
//
// Tile layout: row a holds group elements 16a..16a+15, and its 16-byte chunk c
// sits in chunk slot c ^ (a >> 2).  Row accesses (16 lanes x 16 B) and column
// accesses (one float per lane) are then free of bank conflicts; the four
// tiles of a wave are 272 floats apart, so the teams' column accesses use
// different banks.
//
// About fifteen VALU instructions an element against four bytes of HBM
// traffic (bf16 in, int8 out).  At one round a wave the prologue is bound by
// VALU issue (at 4352 x 3072 the VALU instructions fill 0.9 of the busy
// clocks, and the same loads and stores alone take 5.7 us against its
// 9.2 us); with more rounds a wave there are fewer waves, and it waits on
// memory instead.  Hence few instructions: one fma per butterfly output
// (exact as sum - 2x while 2x does not overflow), the final 1/16 folded into
// the scale, the amax as v_max3 over |.|, half-away rounding as add +
// truncate (pre_half_away) without the clamp on rows that cannot need it,
// the bytes packed by the conversions themselves (cvt_pack4), the row's
// address arithmetic on the scalar unit, and the scale's two divisions in
// nine instructions (qt_scale_fast).  R > 1 spreads the per-wave costs
// (addresses, scale divisions, reductions) over more elements.
constexpr int QT_TILE = 272;
constexpr int QT_WAVE = 4 * QT_TILE;
constexpr int QT_MAX_ROUNDS = 5;

// Orders one wave's LDS accesses across lanes for the compiler: the hardware
// already completes a wave's LDS operations in issue order, and a wavefront-
// scope fence emits no instruction, but it keeps the compiler from moving a
// load of another lane's slot above the store that fills it.
__device__ __forceinline__ void wave_lds_fence() { __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront"); }

// bfly16 with y = fma(-2, x[3-j], sum): bit-identical, one instruction fewer
// per output.
template <int ST>
__device__ __forceinline__ void bfly16f(float (&v)[16]) {
#pragma unroll
    for (int o = 0; o < 4; o++) {
        const int b = ST == 1 ? 4 * o : o;
        const float x0 = v[b], x1 = v[b + ST], x2 = v[b + 2 * ST], x3 = v[b + 3 * ST];
        const float sum = ((x0 + x1) + x2) + x3;
        v[b] = fmaf(-2.0f, x3, sum);
        v[b + ST] = fmaf(-2.0f, x2, sum);
        v[b + 2 * ST] = fmaf(-2.0f, x1, sum);
        v[b + 3 * ST] = fmaf(-2.0f, x0, sum);
    }
}

// bfly16f<4> that also returns (s0 + s1) + (s2 + s3) over its four quadruple
// sums.  That value is finite only if all 16 inputs are: an inf or NaN input
// makes its quadruple's sum inf or NaN (never finite).  With finite inputs the
// outputs fma(-2, x, sum) are finite or +-inf, never NaN.
__device__ __forceinline__ float bfly16f_last(float (&v)[16]) {
    float s[4];
#pragma unroll
    for (int o = 0; o < 4; o++) {
        const float x0 = v[o], x1 = v[o + 4], x2 = v[o + 8], x3 = v[o + 12];
        s[o] = ((x0 + x1) + x2) + x3;
        v[o] = fmaf(-2.0f, x3, s[o]);
        v[o + 4] = fmaf(-2.0f, x2, s[o]);
        v[o + 8] = fmaf(-2.0f, x1, s[o]);
        v[o + 12] = fmaf(-2.0f, x0, s[o]);
    }
    return (s[0] + s[1]) + (s[2] + s[3]);
}

// max(m, |a|, |b|) in one instruction (fmaxf would first canonicalise each
// operand separately).
__device__ __forceinline__ float max3_abs(float m, float a, float b) {
    float r;
    asm("v_max3_f32 %0, %1, |%2|, |%3|" : "=v"(r) : "v"(m), "v"(a), "v"(b));
    return r;
}

// Wave-wide max of non-negative floats, as their bit patterns (same order):
// four DPP steps leave each 16-lane row's max in all its lanes, then the four
// row maxima are read out.  The result is wave-uniform.
__device__ __forceinline__ uint32_t wave_max_bits(uint32_t u) {
    u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
    u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
    u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0x141, 0xF, 0xF, false));  // row_half_mirror
    u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0x140, 0xF, 0xF, false));  // row_mirror
    const uint32_t a = __builtin_amdgcn_readlane(u, 0), b = __builtin_amdgcn_readlane(u, 16);
    const uint32_t c = __builtin_amdgcn_readlane(u, 32), d = __builtin_amdgcn_readlane(u, 48);
    return max(max(a, b), max(c, d));
}

// For ties away from zero: min(|v| inv + (0.5 - 2^-25), qmax) with v's sign,
// whose truncation toward zero is the code.  For every non-negative fp32 d,
// floor(fl(d + (0.5 - 2^-25))) is d rounded half away from zero (checked over
// all fp32 d < 2^25; above that d is an integer and the addition returns d),
// and |v| * inv is |v * inv| exactly.  The clamp commutes with the truncation
// because qmax is an integer.  A NaN product (a NaN value, or inf * 0 in a
// row whose amax is inf) gives -qmax, as the reference's clamp
// fminf(fmaxf(d, -qmax), qmax) does (core/kernels/int8_gemm.cpp:779).
__device__ __forceinline__ float pre_half_away(float v, float inv, float qmax) {
    const float p = fabsf(v) * inv;
    return p != p ? -qmax : copysignf(fminf(p + 0.49999997f, qmax), v);
}

// fmaxf returns -qmax for a NaN product here.
__device__ __forceinline__ float pre_half_even(float v, float inv, float qmax) {
    return fminf(fmaxf(rintf(v * inv), -qmax), qmax);
}

// The fast path's codes: pre_half_away and pre_half_even without the clamp.
// They give the clamped codes whenever |v| inv < qmax + 1/2 and v inv is not
// NaN, which holds on every element of a row whose rotated values are all
// finite: there |v| <= amax, so |v| inv <= qmax (1 + 3 2^-24), and qmax is an
// integer in [1, 127] (checked by the C ABI).
__device__ __forceinline__ float pre_half_away_nc(float v, float inv) {
    return copysignf(fabsf(v) * inv + 0.49999997f, v);
}
__device__ __forceinline__ float pre_half_even_nc(float v, float inv) { return rintf(v * inv); }

// Four fp32 values truncated to int and packed little-endian into one dword:
// each conversion writes the low byte of its int32 result into its byte of
// the dword (SDWA dst_sel), the first clearing the others.  Callers pass
// values whose truncations fit int8.
__device__ __forceinline__ uint32_t cvt_pack4(float a, float b, float c, float d) {
    uint32_t r;
    asm("v_cvt_i32_f32_sdwa %0, %1 dst_sel:BYTE_0 dst_unused:UNUSED_PAD src0_sel:DWORD" : "=v"(r) : "v"(a));
    asm("v_cvt_i32_f32_sdwa %0, %1 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD" : "+v"(r) : "v"(b));
    asm("v_cvt_i32_f32_sdwa %0, %1 dst_sel:BYTE_2 dst_unused:UNUSED_PRESERVE src0_sel:DWORD" : "+v"(r) : "v"(c));
    asm("v_cvt_i32_f32_sdwa %0, %1 dst_sel:BYTE_3 dst_unused:UNUSED_PRESERVE src0_sel:DWORD" : "+v"(r) : "v"(d));
    return r;
}

template <int OP> constexpr int qt_ns = OP == QR_SILU_GATE ? 2 : 1;  // input sets (the SiLU gate has two)
template <bool BF16_IN> constexpr int qt_nw = BF16_IN ? 8 : 16;        // input dwords per lane and set

// One round's inputs: the lane's 16 elements of a group at element offset
// off of the row at xr, and for the SiLU gate the value operand's 16 at
// off + off2.
template <bool BF16_IN, int OP>
__device__ __forceinline__ void qt_load(const void* __restrict__ xr, int off, const QrPre& pre_op,
                                        uint32_t (&raw)[qt_ns<OP>][qt_nw<BF16_IN>]) {
#pragma unroll
    for (int h = 0; h < qt_ns<OP>; h++) {
        const int o = off + (h ? (int)pre_op.off2 : 0);
        const uint4* src = BF16_IN ? (const uint4*)((const uint16_t*)xr + o) : (const uint4*)((const float*)xr + o);
#pragma unroll
        for (int i = 0; i < qt_nw<BF16_IN> / 4; i++) {
            const uint4 t = src[i];
            raw[h][4 * i] = t.x;
            raw[h][4 * i + 1] = t.y;
            raw[h][4 * i + 2] = t.z;
            raw[h][4 * i + 3] = t.w;
        }
    }
}

// One round's rotation: the pre-op on the raw inputs, passes 1 and 4 in
// registers, the transpose through the team's tile, passes 16 and 64.  w[j]
// receives element 16 j + tl of the group (before the final 1/16).  SUB =
// false forms each butterfly output as fma(-2, x, sum), one rounding; SUB =
// true as sum - 2 x, the reference's mul and subtract.  The product 2x is
// exact unless it overflows (|x| >= 2^127), so the two agree on every group
// whose rotated values stay below 2^126: one radix-4 pass applied twice is
// 4 I, so each value inside the rotation is bounded by about the largest
// output of the pass after it.  For SUB = false the result is the last pass's
// check sum (bfly16f_last): finite only if every value entering that pass is.
template <bool BF16_IN, int OP, bool SUB>
__device__ __forceinline__ float qt_round(const uint32_t (&raw)[qt_ns<OP>][qt_nw<BF16_IN>], int64_t col0, int rotate,
                                          const QrPre& pre_op, float* T, float* trow, int tl, int sw,
                                          float (&w)[16]) {
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        if (BF16_IN) v[i] = __uint_as_float(i & 1 ? raw[0][i >> 1] & 0xffff0000u : raw[0][i >> 1] << 16);
        else v[i] = __uint_as_float(raw[0][i]);
    }
    if (OP == QR_MOD) modulate16(v, pre_op.sc, pre_op.sh, col0);
    if (OP == QR_GELU) {
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = gelu_tanh(v[i]);
    }
    if (OP == QR_SILU_GATE) {
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t u = raw[qt_ns<OP> - 1][BF16_IN ? i >> 1 : i];
            v[i] = silu_mul(v[i], __uint_as_float(BF16_IN ? (i & 1 ? u & 0xffff0000u : u << 16) : u));
        }
    }
    if (rotate) {
        if (SUB) {
            bfly16<1>(v);
            bfly16<4>(v);
        } else {
            bfly16f<1>(v);
            bfly16f<4>(v);
        }
    }
    // Row tl of the tile, then column tl: w[j] = element 16 j + tl.
#pragma unroll
    for (int c = 0; c < 4; c++)
        *(float4*)(trow + 4 * (c ^ sw)) = make_float4(v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3]);
    wave_lds_fence();
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float* col = T + 64 * k + 4 * (sw ^ k) + (tl & 3);
#pragma unroll
        for (int i = 0; i < 4; i++) w[4 * k + i] = col[16 * i];
    }
    wave_lds_fence();
    float f = 0.0f;
    if (rotate) {
        if (SUB) {
            bfly16<1>(w);
            bfly16<4>(w);
        } else {
            bfly16f<1>(w);
            f = bfly16f_last(w);
        }
    }
    return f;
}

// max |w[j]| over a round, as bits (NaN values are passed over, as the
// reference's `if (a > amax)` and fmaxf pass them over).
__device__ __forceinline__ uint32_t qt_amax16(const float (&w)[16]) {
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; j += 2) m = max3_abs(m, w[j], w[j + 1]);
    return __float_as_uint(m);
}

// One round's codes: column tl back into the tile, row tl out (16 contiguous
// elements), quantised and stored as one 16-byte write when live.  FAST
// leaves out the clamp (pre_half_away_nc).
template <bool HALF_EVEN, bool FAST>
__device__ __forceinline__ void qt_store(const float (&w)[16], float* T, float* trow, int tl, int sw,
                                         const QtScale& c, float qmax, int8_t* dst, bool live) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
        float* col = T + 64 * k + 4 * (sw ^ k) + (tl & 3);
#pragma unroll
        for (int i = 0; i < 4; i++) col[16 * i] = w[4 * k + i];
    }
    wave_lds_fence();
    uint32_t packed[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        float4 u = *(const float4*)(trow + 4 * (k ^ sw));
        // Wave-uniform and rare; never on a fast row (amax < 2^126 makes
        // inv >= 2^-122, so the 1/16 is folded).
        if (!FAST && !c.fold) u = make_float4(u.x * c.pre, u.y * c.pre, u.z * c.pre, u.w * c.pre);
        if (FAST) {
            if (HALF_EVEN)
                packed[k] = cvt_pack4(pre_half_even_nc(u.x, c.post), pre_half_even_nc(u.y, c.post),
                                      pre_half_even_nc(u.z, c.post), pre_half_even_nc(u.w, c.post));
            else
                packed[k] = cvt_pack4(pre_half_away_nc(u.x, c.post), pre_half_away_nc(u.y, c.post),
                                      pre_half_away_nc(u.z, c.post), pre_half_away_nc(u.w, c.post));
        } else {
            if (HALF_EVEN)
                packed[k] = cvt_pack4(pre_half_even(u.x, c.post, qmax), pre_half_even(u.y, c.post, qmax),
                                      pre_half_even(u.z, c.post, qmax), pre_half_even(u.w, c.post, qmax));
            else
                packed[k] = cvt_pack4(pre_half_away(u.x, c.post, qmax), pre_half_away(u.y, c.post, qmax),
                                      pre_half_away(u.z, c.post, qmax), pre_half_away(u.w, c.post, qmax));
        }
    }
    wave_lds_fence();
    if (live) *(uint4*)dst = make_uint4(packed[0], packed[1], packed[2], packed[3]);
}

// One row's work after its loads: the rotation of the wave's R rounds, the
// row amax across the row's waves (red: one word a wave of the block), the
// reference-form second pass for rows that need it, and the codes and scale.
template <bool BF16_IN, bool HALF_EVEN, int R, int OP>
__device__ __forceinline__ void qt_row(const uint32_t (&raw)[R][qt_ns<OP>][qt_nw<BF16_IN>],
                                       const void* __restrict__ xr, int row, int rows, int G,
                                       int8_t* __restrict__ q, int64_t ldq, float* __restrict__ s, float qmax,
                                       float qrcp, int rotate, const QrPre& pre_op, int qkt, uint32_t* red, float* T,
                                       float* trow,
                                       int lane, int wr, int wpr, int wave, int g0, int tl, int sw) {
    auto gcol = [&](int r) { return min(g0 + 4 * r, G - 1) * 256; };

    // First pass, on the inputs the caller loaded.
    float rot[R][16];
    uint32_t amax = 0;
    bool nonfinite = false;  // an inf or NaN among a live round's values
    {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float f = qt_round<BF16_IN, OP, false>(raw[r], gcol(r) + tl * 16, rotate, pre_op, T, trow, tl, sw, rot[r]);
            if (g0 + 4 * r < G) {
                amax = max(amax, qt_amax16(rot[r]));
                nonfinite |= !__builtin_isfinite(f);
            }
        }
    }

    // The lane's 16 bytes of group g land at qrow + g * gstep: row-major, or
    // K-tiled (256-row strips of h rows; the group's four 64-byte K-steps are
    // blocks h x 64 bytes apart; chunk tl & 3 of K-step tl >> 2 in slot
    // (tl & 3) ^ ((row >> 2) & 3)).
    int8_t* qrow;
    int64_t gstep;
    if (qkt) {
        const int64_t st = row >> 8, rr = row & 255, h = min(256, rows - (int)(st << 8));
        qrow = q + st * 256 * (int64_t)G * 256 + (tl >> 2) * h * 64 + rr * 64 + (((tl & 3) ^ ((rr >> 2) & 3)) * 16);
        gstep = 4 * h * 64;
    } else {
        qrow = q + (int64_t)row * ldq + tl * 16;
        gstep = 256;
    }

    // The row's amax (non-negative, so bit 31 is free) travels with a flag
    // for a non-finite value in bit 31.  A row is fast when its rotated
    // values are finite and below 2^126: the fma butterflies then give the
    // reference's values, and the codes need no clamp (pre_half_away_nc).
    // Other rows are rotated again in the reference's form, one round at a
    // time, and quantised with the clamp.  Where waves share barriers
    // (several waves a row), the whole block does so when any of its rows
    // needs it; a fast row gets the same values and codes that way.
    amax = wave_max_bits(amax);
    uint32_t flag = __builtin_amdgcn_ballot_w64(nonfinite) ? 0x80000000u : 0u;
    bool redo;
    if (wpr > 1) {
        // Lane l reads wave l's word (at most 16 waves a block; the lanes
        // past them repeat the last), then one reduction gives the row's
        // amax and flag, and one ballot whether any row of the block is slow.
        if (lane == 0) red[wave] = amax | flag;
        __syncthreads();
        const int nw = blockDim.y * wpr, first = __builtin_amdgcn_readfirstlane(threadIdx.y) * wpr;
        const uint32_t e = red[min(lane, nw - 1)];
        const bool mine = lane >= first && lane < first + wpr;
        amax = wave_max_bits(mine ? e & 0x7fffffffu : 0u);
        flag = __builtin_amdgcn_ballot_w64(mine && (e >> 31) != 0) ? 0x80000000u : 0u;
        redo = __builtin_amdgcn_ballot_w64((e >> 31) != 0 || (e & 0x7fffffffu) >= 0x7e800000u) != 0;
    } else {
        redo = (flag >> 31) != 0 || amax >= 0x7e800000u;
    }

    if (__builtin_amdgcn_readfirstlane(rotate && redo)) {
        // The inputs are loaded again each time: the opaque base keeps the
        // compiler from holding earlier loads live across the passes.
        uint32_t a2 = 0;
#pragma unroll 1
        for (int r = 0; r < R; r++) {
            const void* xo = xr;
            asm volatile("" : "+s"(xo));
            uint32_t raw[qt_ns<OP>][qt_nw<BF16_IN>];
            qt_load<BF16_IN, OP>(xo, tl * 16 + gcol(r), pre_op, raw);
            float w[16];
            qt_round<BF16_IN, OP, true>(raw, gcol(r) + tl * 16, rotate, pre_op, T, trow, tl, sw, w);
            if (g0 + 4 * r < G) a2 = max(a2, qt_amax16(w));
        }
        amax = wave_max_bits(a2);
        if (wpr > 1) {
            __syncthreads();  // every wave has read the first pass's entries
            if (lane == 0) red[wave] = amax;
            __syncthreads();
            for (int i = 0; i < wpr; i++) amax = max(amax, red[__builtin_amdgcn_readfirstlane(threadIdx.y) * wpr + i]);
        }
        const QtScale c = qt_scale(amax, qmax, rotate);
#pragma unroll 1
        for (int r = 0; r < R; r++) {
            const void* xo = xr;
            asm volatile("" : "+s"(xo));
            uint32_t raw[qt_ns<OP>][qt_nw<BF16_IN>];
            qt_load<BF16_IN, OP>(xo, tl * 16 + gcol(r), pre_op, raw);
            float w[16];
            qt_round<BF16_IN, OP, true>(raw, gcol(r) + tl * 16, rotate, pre_op, T, trow, tl, sw, w);
            qt_store<HALF_EVEN, false>(w, T, trow, tl, sw, c, qmax, qrow + (int64_t)(g0 + 4 * r) * gstep,
                                       row < rows && g0 + 4 * r < G);
        }
        if (wr == 0 && lane == 0 && row < rows) s[row] = c.scale;
    } else {
        // Here every row of the block is fast, or there is no rotation (then
        // nothing was checked, and the codes are clamped).
        if (__builtin_amdgcn_readfirstlane(rotate)) {
            const QtScale c = qt_scale_fast(amax, qmax, qrcp);
#pragma unroll
            for (int r = 0; r < R; r++)
                qt_store<HALF_EVEN, true>(rot[r], T, trow, tl, sw, c, qmax, qrow + (int64_t)(g0 + 4 * r) * gstep,
                                          row < rows && g0 + 4 * r < G);
            if (wr == 0 && lane == 0 && row < rows) s[row] = c.scale;
        } else {
            const QtScale c = qt_scale(amax, qmax, rotate);
#pragma unroll
            for (int r = 0; r < R; r++)
                qt_store<HALF_EVEN, false>(rot[r], T, trow, tl, sw, c, qmax, qrow + (int64_t)(g0 + 4 * r) * gstep,
                                           row < rows && g0 + 4 * r < G);
            if (wr == 0 && lane == 0 && row < rows) s[row] = c.scale;
        }
    }
}

// One block's share of a W4Expand job: item i (idx * threads + thread)
// turns 32 consecutive codes of one weight row into 32 int8, as
// w4_lut_expand_kernel's thread i does.
__device__ __forceinline__ void w4_expand_part(const W4Expand& ex, int idx) {
    const int nt = blockDim.x * blockDim.y;
    const int64_t per_row = ex.K / 32;
    const int64_t i = (int64_t)idx * nt + threadIdx.y * blockDim.x + threadIdx.x;
    if (i >= ex.N * per_row) return;
    const int64_t row = i / per_row, c32 = i - row * per_row;
    using persist::u32x4;
    const u32x4 c = *(const u32x4*)(ex.codes + row * ex.ldb + c32 * 16);
    const u32x4 t = ex.w4_signed ? persist::signed_nibble_table()
                                 : *(const u32x4*)(ex.lut + (row * ex.lut_groups + ((c32 * 32) >> ex.group_shift)) * 16);
    int8_t* o0 = ex.out + (ex.kt ? k_tiled_offset(row, c32 * 32, ex.K, ex.N) : row * ex.K + c32 * 32);
    int8_t* o1 = ex.out + (ex.kt ? k_tiled_offset(row, c32 * 32 + 16, ex.K, ex.N) : row * ex.K + c32 * 32 + 16);
    *(v4i*)o0 = persist::expand16b(c[0], c[1], t);
    *(v4i*)o1 = persist::expand16b(c[2], c[3], t);
}

template <bool BF16_IN, bool HALF_EVEN, int R, int OP>
__global__ __launch_bounds__(1024) void quant_rotate_tiles(const void* __restrict__ x, int64_t ldx, int rows,
                                                           int G, int8_t* __restrict__ q, int64_t ldq,
                                                           float* __restrict__ s, float qmax, float qrcp,
                                                           int rotate, QrPre pre_op, int qkt, int lg_run) {
    extern __shared__ __align__(16) float lds[];
    // The wave's index in its row and its row within the block are the same
    // for all its lanes; read as such, the row's address arithmetic runs on
    // the scalar unit instead of as 64-bit VALU work in every wave.
    const int lane = threadIdx.x & 63, wpr = blockDim.x >> 6;
    const int wr = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), ty = __builtin_amdgcn_readfirstlane(threadIdx.y);
    const int wave = ty * wpr + wr;
    // Blocks are dealt to the 8 XCDs in turn.  Each XCD takes runs of
    // 2^lg_run consecutive blocks' rows, so the rows that share the 128-byte
    // lines of the K-tiled codes (two rows a line) are written through one
    // L2.  The last partial set of runs keeps its order.
    int blk = blockIdx.x;
    unsigned nblk = gridDim.x;
    if (OP == QR_PLAIN && pre_op.ex.blocks) {
        // Beside a W4Expand job: groups of 16 blocks, 8 of the prologue then 8
        // of the expansion (each kind on all 8 XCDs), while both last; then
        // the rest of the longer one.
        const int nq = pre_op.ex.nq, ne = pre_op.ex.blocks, full = min(nq, ne) / 8;
        int kind, idx;
        if (blk < 16 * full) {
            kind = (blk >> 3) & 1;
            idx = 8 * (blk >> 4) + (blk & 7);
        } else {
            const int rest = blk - 16 * full, qrem = nq - 8 * full;
            kind = rest >= qrem;
            idx = 8 * full + (kind ? rest - qrem : rest);
        }
        if (kind) {
            w4_expand_part(pre_op.ex, idx);
            return;
        }
        blk = idx;
        nblk = (unsigned)nq;
    }
    {
        const int span = 8 << lg_run;
        if (blk < (int)(nblk & ~(unsigned)(span - 1))) {
            const int c = blk & (span - 1);
            blk += ((c & 7) << lg_run) + (c >> 3) - c;
        }
    }
    const int team = lane >> 4, tl = lane & 15, sw = tl >> 2;
    const int g0 = wr * 4 * R + team;  // round r works on group g0 + 4 r
    float* T = lds + wave * QT_WAVE + team * QT_TILE;
    float* trow = T + tl * 16;
    uint32_t* red = (uint32_t*)(lds + blockDim.y * wpr * QT_WAVE);

    // Lanes past the row's last group, or in a row past the last, read valid
    // data of another group and discard it.
    const int row = blk * blockDim.y + ty;
    const int64_t roff = (int64_t)min(row, rows - 1) * ldx;
    const void* xr = BF16_IN ? (const void*)((const uint16_t*)x + roff) : (const void*)((const float*)x + roff);
    uint32_t raw[R][qt_ns<OP>][qt_nw<BF16_IN>];
#pragma unroll
    for (int r = 0; r < R; r++) qt_load<BF16_IN, OP>(xr, tl * 16 + min(g0 + 4 * r, G - 1) * 256, pre_op, raw[r]);
    qt_row<BF16_IN, HALF_EVEN, R, OP>(raw, xr, row, rows, G, q, ldq, s, qmax, qrcp, rotate, pre_op, qkt, red, T, trow,
                                      lane, wr, wpr, wave, g0, tl, sw);
}

// Rounds per wave for G groups.  For a large problem R minimises the
// instructions per element: ~14.3 per element plus ~90 per wave and
// round-set spread over the 16 R elements a lane holds, times the share of
// lanes doing live work, with 10 % more for R >= 4 (at most five waves per
// SIMD).  A small one (under 2^17 groups, about two waves of waves on the
// chip) is bound by latency, and the most waves (R = 1) wins.
static int tile_rounds(int64_t rows, int G) {
    const int forced = env_switch("PHI_QR_ROUNDS", 0, 1, QT_MAX_ROUNDS);  // A/B switch: force R where it fits
    if (forced && (G + 4 * forced - 1) / (4 * forced) <= 16) return forced;
    if (rows * G < (1 << 17) && G <= 64) return 1;
    int best = 1;
    double best_cost = 1e30;
    for (int R = 1; R <= QT_MAX_ROUNDS; R++) {
        const int wpr = (G + 4 * R - 1) / (4 * R);
        if (wpr > 16) continue;
        const double cost = (double)(4 * R * wpr) / G * (14.3 + 90.0 / (16 * R)) * (R >= 4 ? 1.1 : 1.0);
        if (cost < best_cost - 1e-9) best = R, best_cost = cost;
    }
    return best;
}

template <bool BF16_IN, bool HALF_EVEN, int R, int OP>
static hipError_t launch_tiles_r(hipStream_t stream, const void* x, int64_t rows, int G, int64_t ldx, int8_t* q,
                                 int64_t ldq, float* s, float qmax, int rotate, const QrPre& pre, int qkt) {
    // Blocks of about four waves: against eight, 9.4 against 10.1 us at
    // 4352 x 3072, 28 against 30.5 at 4352 x 12288 and 92.5 against 97.4 at
    // 32760 x 5120 (one to sixteen waves measured).
    const int wpr = (G + 4 * R - 1) / (4 * R);
    const int rpb = wpr >= 4 ? 1 : 4 / wpr;
    const size_t lds = ((size_t)rpb * wpr * QT_WAVE + 16) * sizeof(float);
    static bool lds_set = false;  // one attribute call per instantiation and process
    if (!lds_set) {
        const hipError_t e = hipFuncSetAttribute((const void*)quant_rotate_tiles<BF16_IN, HALF_EVEN, R, OP>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)((16 * QT_WAVE + 16) * sizeof(float)));
        if (e != hipSuccess) return e;
        lds_set = true;
    }
    dim3 grid((unsigned)((rows + rpb - 1) / rpb)), block((unsigned)(64 * wpr), (unsigned)rpb);
    QrPre p2 = pre;
    if (OP == QR_PLAIN && pre.ex.on) {
        const int64_t items = pre.ex.N * (pre.ex.K / 32), nt = 64 * wpr * rpb;
        p2.ex.nq = (int)grid.x;
        p2.ex.blocks = (int)((items + nt - 1) / nt);
        grid.x += (unsigned)p2.ex.blocks;
    } else {
        p2.ex.blocks = 0;
    }
    // Runs of 8 blocks a XCD: config 1's prologue 11.0 -> 10.4 us, config 1
    // down's 32.3 -> 29.0 us (K-tiled codes; runs of 2 and 4 measured too).
    // A/B switch: log2 of the run length, 0..4 (the kernel shifts by it)
    const int lg_run = env_switch("PHI_QR_RUN", 3, 0, 4);
    hipLaunchKernelGGL((quant_rotate_tiles<BF16_IN, HALF_EVEN, R, OP>), grid, block, lds, stream, x, ldx, (int)rows,
                       G, q, ldq, s, qmax, 1.0f / qmax, rotate, p2, qkt, lg_run);
    return hipGetLastError();
}

// A pre-op keeps R at 1 or 2: the modulation holds per-round scale/shift
// registers and the SiLU gate a second set of loads, and GELU's VALU work
// per element dwarfs the per-wave costs a larger R spreads.
template <bool BF16_IN, bool HALF_EVEN, int OP>
static hipError_t launch_tiles_op(hipStream_t stream, const void* x, int64_t rows, int G, int64_t ldx, int8_t* q,
                                  int64_t ldq, float* s, float qmax, int rotate, const QrPre& pre, int qkt) {
    if (tile_rounds(rows, G) == 1)
        return launch_tiles_r<BF16_IN, HALF_EVEN, 1, OP>(stream, x, rows, G, ldx, q, ldq, s, qmax, rotate, pre, qkt);
    return launch_tiles_r<BF16_IN, HALF_EVEN, 2, OP>(stream, x, rows, G, ldx, q, ldq, s, qmax, rotate, pre, qkt);
}

template <bool BF16_IN, bool HALF_EVEN>
static hipError_t launch_tiles(hipStream_t stream, const void* x, int64_t rows, int G, int64_t ldx, int8_t* q,
                               int64_t ldq, float* s, float qmax, int rotate, const QrPre& pre, int qkt) {
    switch (pre.op) {
        case QR_MOD: return launch_tiles_op<BF16_IN, HALF_EVEN, QR_MOD>(stream, x, rows, G, ldx, q, ldq, s, qmax, rotate, pre, qkt);
        case QR_GELU: return launch_tiles_op<BF16_IN, HALF_EVEN, QR_GELU>(stream, x, rows, G, ldx, q, ldq, s, qmax, rotate, pre, qkt);
        case QR_SILU_GATE:
            return launch_tiles_op<BF16_IN, HALF_EVEN, QR_SILU_GATE>(stream, x, rows, G, ldx, q, ldq, s, qmax, rotate, pre, qkt);
        default: break;
    }
    switch (tile_rounds(rows, G)) {
        case 1: return launch_tiles_r<BF16_IN, HALF_EVEN, 1, QR_PLAIN>(stream, x, rows, G, ldx, q, ldq, s, qmax, rotate, pre, qkt);
        case 2: return launch_tiles_r<BF16_IN, HALF_EVEN, 2, QR_PLAIN>(stream, x, rows, G, ldx, q, ldq, s, qmax, rotate, pre, qkt);
        case 3: return launch_tiles_r<BF16_IN, HALF_EVEN, 3, QR_PLAIN>(stream, x, rows, G, ldx, q, ldq, s, qmax, rotate, pre, qkt);
        case 4: return launch_tiles_r<BF16_IN, HALF_EVEN, 4, QR_PLAIN>(stream, x, rows, G, ldx, q, ldq, s, qmax, rotate, pre, qkt);
        default: return launch_tiles_r<BF16_IN, HALF_EVEN, 5, QR_PLAIN>(stream, x, rows, G, ldx, q, ldq, s, qmax, rotate, pre, qkt);
    }
}

// Host-side launcher.  Validation is done by the C ABI layer.
hipError_t launch_quant_rotate(hipStream_t stream, const void* x, bool bf16_in, int64_t rows,
                               int64_t K, int64_t ldx, int8_t* q, int64_t ldq, float* s,
                               float qmax, int half_even, int rotate, const QrPre& pre, int qkt) {
    const int G = (int)(K / 256);
    if (rows == 0) return hipSuccess;
    if (qkt && G > 64) return hipErrorInvalidValue;  // the row kernel writes row-major q only
    // A W4Expand job rides only on the plain tiles kernel.
    if (pre.ex.on && (G > 64 || pre.op != QR_PLAIN)) return hipErrorInvalidValue;
    if (G <= 64) {
        if (bf16_in)
            return half_even ? launch_tiles<true, true>(stream, x, rows, G, ldx, q, ldq, s, qmax, rotate, pre, qkt)
                             : launch_tiles<true, false>(stream, x, rows, G, ldx, q, ldq, s, qmax, rotate, pre, qkt);
        return half_even ? launch_tiles<false, true>(stream, x, rows, G, ldx, q, ldq, s, qmax, rotate, pre, qkt)
                         : launch_tiles<false, false>(stream, x, rows, G, ldx, q, ldq, s, qmax, rotate, pre, qkt);
    }
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
                           stream, x, ldx, (int)K, q, ldq, s, qmax, half_even, rotate, pre);
    } else {
        hipLaunchKernelGGL(quant_rotate_rows<false>, dim3((unsigned)rows), dim3(threads), lds_bytes,
                           stream, x, ldx, (int)K, q, ldq, s, qmax, half_even, rotate, pre);
    }
    return hipGetLastError();
}

size_t quant_rotate_lds_bytes(int64_t K) { return ((size_t)(K / 256) * QR_GSTRIDE + 16) * sizeof(float); }

}  // namespace phi_dev
