/*
 * CPU oracle for the quantized-linear hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's host arithmetic, used as the
 * checker for the HIP kernels.  Built with -O2 -ffp-contract=off so every
 * float operation is rounded on its own, exactly as the reference's x86-64
 * build (g++ -O3, no -march, no fast-math: makefile:13) rounds it.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline may use it.
 */
#include "oracle.h"

#include <limits.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* scalar conversions                                                       */
/* ------------------------------------------------------------------------ */

static float bits_to_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static uint32_t f32_to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

/* IEEE binary16 -> binary32, exact (core/util/media_common.cpp:62-87). */
float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const int e = (h >> 10) & 0x1f;
    const uint32_t m = h & 0x3ff;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exactly representable in fp32 */
        const float v = ldexpf((float)m, -24);
        return sign ? -v : v;
    }
    if (e == 31) return bits_to_f32(sign | 0x7f800000u | (m << 13)); /* inf / nan */
    return bits_to_f32(sign | ((uint32_t)(e - 15 + 127) << 23) | (m << 13));
}

/* bf16 is the top half of an fp32 (media_common.cpp:116-121). */
float orc_bf16_to_f32(uint16_t h) { return bits_to_f32((uint32_t)h << 16); }

/* fp32 -> bf16, round to nearest even by the integer carry rule
 * (media_common.cpp:187-193): add 0x7fff plus the kept lsb, keep the top half. */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t b = f32_to_bits(f);
    b += 0x7fffu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}

/* E4M3FN: bias 7, no infinities, S.1111.111 is NaN (media_common.cpp:130-160). */
float orc_f8_e4m3_to_f32(uint8_t b) {
    const int s = b >> 7, e = (b >> 3) & 15, m = b & 7;
    float v;
    if (e == 15 && m == 7) v = NAN;
    else if (e == 0) v = ldexpf((float)m, -9);
    else v = ldexpf((float)(8 + m), e - 10);
    return s ? -v : v;
}

/* E5M2: bias 15, IEEE-shaped (media_common.cpp:130-160). */
float orc_f8_e5m2_to_f32(uint8_t b) {
    const int s = b >> 7, e = (b >> 2) & 31, m = b & 3;
    float v;
    if (e == 31) v = m == 0 ? INFINITY : NAN;
    else if (e == 0) v = ldexpf((float)m, -16);
    else v = ldexpf((float)(4 + m), e - 17);
    return s ? -v : v;
}

/* core/host/quant.cpp:285-299; a U8 scale table is E4M3 in a byte container. */
float orc_scale_at(const void* p, int dtype, int64_t i) {
    switch (dtype) {
        case ORC_F32: return ((const float*)p)[i];
        case ORC_F16: return orc_f16_to_f32(((const uint16_t*)p)[i]);
        case ORC_BF16: return orc_bf16_to_f32(((const uint16_t*)p)[i]);
        case ORC_F8_E4M3:
        case ORC_U8_E4M3: return orc_f8_e4m3_to_f32(((const uint8_t*)p)[i]);
        case ORC_F8_E5M2: return orc_f8_e5m2_to_f32(((const uint8_t*)p)[i]);
        default: return NAN;
    }
}

void orc_f32_to_bf16_n(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = orc_f32_to_bf16(x[i]);
}
void orc_bf16_to_f32_n(const uint16_t* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = orc_bf16_to_f32(x[i]);
}

/* ------------------------------------------------------------------------ */
/* A1: convrot                                                              */
/* ------------------------------------------------------------------------ */

/* One 256-group, in place.  H = H4^{(x)4}/16 with H4 = J - 2R: four radix-4
 * passes over the base-4 digits of the index, least significant first
 * (stride 1, 4, 16, 64).  Each pass maps (x0,x1,x2,x3) at one stride to
 * y[j] = (((x0 + x1) + x2) + x3) - 2*x[3-j]; afterwards every element is
 * multiplied by 1/16 (core/host/quant.cpp:109-131). */
static void convrot_group(float* o) {
    for (int stride = 1; stride < 256; stride *= 4) {
        for (int base = 0; base < 256; base += 4 * stride) {
            for (int off = 0; off < stride; off++) {
                float* p = o + base + off;
                const float x0 = p[0], x1 = p[stride], x2 = p[2 * stride], x3 = p[3 * stride];
                const float sum = ((x0 + x1) + x2) + x3;
                p[0] = sum - 2.0f * x3;
                p[stride] = sum - 2.0f * x2;
                p[2 * stride] = sum - 2.0f * x1;
                p[3 * stride] = sum - 2.0f * x0;
            }
        }
    }
    for (int i = 0; i < 256; i++) o[i] *= (1.0f / 16.0f);
}

void orc_convrot_rows(const float* x, float* out, int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; r++) {
        for (int64_t g = 0; g + 256 <= cols; g += 256) {
            float* o = out + r * cols + g;
            memcpy(o, x + r * cols + g, 256 * sizeof(float));
            convrot_group(o);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* A2: per-row quantiser                                                    */
/* ------------------------------------------------------------------------ */

/* The host rule: the fp32 product widened to double, pushed half a unit away
 * from zero and truncated (core/host/quant.cpp:163-166); or, with
 * ORC_ROUND_HALF_EVEN, the nearest integer with ties to even.  A NaN product
 * (a NaN element, or inf * 0 when the row's amax is inf) becomes the most
 * negative code: the device form clamps with fminf(fmaxf(d, -qmax), qmax),
 * which maps NaN to -qmax (core/kernels/int8_gemm.cpp:779), and the host
 * form's (long) cast of a NaN gives LONG_MIN on x86-64, clamped to -127
 * (core/host/quant.cpp:164-165).  Written out here instead of left to the
 * cast. */
static long round_code(float prod, int round_mode) {
    if (isnan(prod)) return LONG_MIN;
    const double d = (double)prod;
    if (round_mode == ORC_ROUND_HALF_EVEN) return (long)nearbyint(d);
    return (long)(d >= 0 ? d + 0.5 : d - 0.5);
}

/* The reference device kernel's form (core/kernels/int8_gemm.cpp:777-780): the
 * clamp first, in fp32 (NaN -> -qmax), then the half-unit push as an fp32 sum,
 * rounded to nearest even before floorf / ceilf see it. */
static long round_code_device(float prod, float qmax) {
    const float d = fminf(fmaxf(prod, -qmax), qmax);
    const float pushed = d >= 0.0f ? d + 0.5f : d - 0.5f;
    return (long)(d >= 0.0f ? floorf(pushed) : ceilf(pushed));
}

int64_t orc_round_forms_differ(float* out, int64_t cap) {
    int64_t found = 0;
    const uint32_t top = 0x43000000u; /* 128.0f */
    for (uint32_t sign = 0; sign <= 1; sign++) {
        for (uint32_t bits = 0; bits <= top; bits++) {
            const uint32_t b = bits | (sign << 31);
            float d;
            memcpy(&d, &b, 4);
            if (round_code(d, ORC_ROUND_HALF_AWAY) != round_code_device(d, 128.0f)) {
                if (found < cap) out[found] = d;
                found++;
            }
        }
    }
    return found;
}

int orc_quantize_rows(const void* x, int x_dtype, int64_t rows, int64_t cols, int64_t ldx,
                      int rotate, float qmax, int round_mode, int8_t* q, float* s) {
    if (rotate && cols % 256 != 0) return -1;
    float* row = (float*)malloc((size_t)(cols > 0 ? cols : 1) * sizeof(float));
    const long lim = (long)qmax;
    for (int64_t r = 0; r < rows; r++) {
        for (int64_t c = 0; c < cols; c++) {
            row[c] = x_dtype == ORC_BF16 ? orc_bf16_to_f32(((const uint16_t*)x)[r * ldx + c])
                                         : ((const float*)x)[r * ldx + c];
        }
        if (rotate)
            for (int64_t g = 0; g < cols; g += 256) convrot_group(row + g);
        float amax = 0.0f;
        for (int64_t c = 0; c < cols; c++) {
            const float a = fabsf(row[c]);
            if (a > amax) amax = a;
        }
        const float scale = amax > 1e-30f ? amax / qmax : 1.0f;
        const float inv = 1.0f / scale;
        s[r] = scale;
        for (int64_t c = 0; c < cols; c++) {
            long v = round_mode == ORC_ROUND_DEVICE_FLOOR ? round_code_device(row[c] * inv, qmax)
                                                           : round_code(row[c] * inv, round_mode);
            v = v < -lim ? -lim : (v > lim ? lim : v);
            q[r * cols + c] = (int8_t)v;
        }
    }
    free(row);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* A4 / A5: integer product and epilogue                                    */
/* ------------------------------------------------------------------------ */

void orc_gemm_i8_i32(const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb, int64_t M,
                     int64_t N, int64_t K, int32_t* acc) {
    for (int64_t m = 0; m < M; m++) {
        const int8_t* a = A + m * lda;
        for (int64_t n = 0; n < N; n++) {
            const int8_t* b = B + n * ldb;
            int32_t sum = 0;
            for (int64_t k = 0; k < K; k++) sum += (int32_t)a[k] * (int32_t)b[k];
            acc[m * N + n] = sum;
        }
    }
}

static float bias_at(const void* bias, int bias_dtype, int64_t n) {
    if (!bias || bias_dtype < 0) return 0.0f;
    if (bias_dtype == ORC_BF16) return orc_bf16_to_f32(((const uint16_t*)bias)[n]);
    return ((const float*)bias)[n];
}

void orc_epilogue(const int32_t* acc, int64_t M, int64_t N, const float* sa, const float* sb,
                  int sb_scalar, const void* bias, int bias_dtype, int fused, void* out,
                  int out_dtype) {
    for (int64_t m = 0; m < M; m++) {
        for (int64_t n = 0; n < N; n++) {
            const float t = (float)acc[m * N + n] * sa[m];
            const float w = sb_scalar ? sb[0] : sb[n];
            const float b = bias_at(bias, bias_dtype, n);
            const float v = fused ? fmaf(t, w, b) : (t * w) + b;
            if (out_dtype == ORC_BF16) ((uint16_t*)out)[m * N + n] = orc_f32_to_bf16(v);
            else ((float*)out)[m * N + n] = v;
        }
    }
}

int orc_q8_linear(const void* x, int x_dtype, int64_t M, int64_t K, const int8_t* W,
                  const float* sw, int sw_scalar, const void* bias, int bias_dtype, int64_t N,
                  int round_mode, void* out, int out_dtype, int8_t* q_out, float* s_out,
                  int32_t* acc_out) {
    int8_t* q = q_out ? q_out : (int8_t*)malloc((size_t)(M * K > 0 ? M * K : 1));
    float* s = s_out ? s_out : (float*)malloc((size_t)(M > 0 ? M : 1) * sizeof(float));
    int32_t* acc = acc_out ? acc_out : (int32_t*)malloc((size_t)(M * N > 0 ? M * N : 1) * 4);
    int rc = orc_quantize_rows(x, x_dtype, M, K, K, 1, 127.0f, round_mode, q, s);
    if (rc == 0) {
        orc_gemm_i8_i32(q, K, W, K, M, N, K, acc);
        orc_epilogue(acc, M, N, s, sw, sw_scalar, bias, bias_dtype, 1, out, out_dtype);
    }
    if (!q_out) free(q);
    if (!s_out) free(s);
    if (!acc_out) free(acc);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* A7: grouped 4/6-bit decode + per-row requantise                          */
/* ------------------------------------------------------------------------ */

/* The packer's grid: nearest integer, ties to even, clamped to +-127
 * (core/host/quant.cpp:315-321). */
static float int8_grid(float v) {
    double r = nearbyint((double)v);
    if (r < -127.0) r = -127.0;
    if (r > 127.0) r = 127.0;
    return (float)r;
}

/* core/host/quant.cpp:331-333 */
static float grouped_value(float level, float s_rel, float s_channel, float corr) {
    return int8_grid(level * s_rel) * s_channel + corr;
}

int orc_w4a8_expand(const uint8_t* codes, int64_t codes_row_bytes, const void* s_rel,
                    int s_rel_dtype, int64_t srel_row_bytes, const float* s_channel,
                    int sch_scalar, const float* codebook, const float* correction,
                    int64_t rows, int64_t k, int64_t group, int layout, int8_t* q, float* s,
                    float* values) {
    if (group <= 0 || k % group != 0) return -1;
    if (layout == 0 && group % 2 != 0) return -1;
    if (layout == 1 && (group % 4 != 0 || codebook)) return -1;
    float* v = (float*)malloc((size_t)k * sizeof(float));
    for (int64_t r = 0; r < rows; r++) {
        const uint8_t* c = codes + r * codes_row_bytes;
        const uint8_t* rel_row = (const uint8_t*)s_rel + r * srel_row_bytes;
        const float sch = s_channel ? (sch_scalar ? s_channel[0] : s_channel[r]) : 1.0f;
        for (int64_t col = 0; col < k; col++) {
            long code;
            float level;
            if (layout == 0) {
                /* low nibble = even column (quant.cpp:339-346) */
                const uint8_t b = c[col / 2];
                code = (col & 1) ? (b >> 4) & 15 : b & 15;
                level = codebook ? codebook[code] : (float)(code - 8);
            } else {
                /* two planes: k/2 low-nibble bytes, then k/4 top-two-bit bytes
                 * (quant.cpp:358-389) */
                const uint8_t lo = c[col / 2];
                const uint8_t hb = c[k / 2 + col / 4];
                const long nib = (col & 1) ? (lo >> 4) & 15 : lo & 15;
                code = nib | (long)(((hb >> (2 * (col & 3))) & 3) << 4);
                level = (float)(code - 32);
            }
            const int64_t g = col / group;
            const float rel = s_rel ? orc_scale_at(rel_row, s_rel_dtype, g) : 1.0f;
            const float corr = correction ? correction[g * rows + r] : 0.0f;
            v[col] = grouped_value(level, rel, sch, corr);
        }
        if (values) memcpy(values + r * k, v, (size_t)k * sizeof(float));
        /* quantize_weight_into with rotation off: per-row amax/127, half away */
        orc_quantize_rows(v, ORC_F32, 1, k, k, 0, 127.0f, ORC_ROUND_HALF_AWAY, q + r * k, s + r);
    }
    free(v);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* convrot_w4a4: signed int4 weights, absmax/7 activations                  */
/* ------------------------------------------------------------------------ */

/* quantize_convrot_w4a4 (core/host/quant.cpp:247-272): rotate each 256-group,
 * s = amax > 0 ? amax/7 : 1 per row, code = clamp(lround(v / s), +-7) (ties
 * away from zero, a true division), two codes a byte with column 2j in the low
 * nibble.  Returns 1 when cols is not a multiple of 256. */
int orc_quantize_convrot_w4a4(const float* w, int64_t rows, int64_t cols, uint8_t* packed, float* scales) {
    if (cols % 256 != 0) return 1;
    float* rot = (float*)malloc(sizeof(float) * (size_t)cols);
    for (int64_t r = 0; r < rows; r++) {
        orc_convrot_rows(w + r * cols, rot, 1, cols);
        float amax = 0.0f;
        for (int64_t c = 0; c < cols; c++) amax = fmaxf(amax, fabsf(rot[c]));
        const float s = amax > 0.0f ? amax / 7.0f : 1.0f;
        scales[r] = s;
        for (int64_t c = 0; c < cols; c += 2) {
            long lo = lroundf(rot[c] / s), hi = lroundf(rot[c + 1] / s);
            lo = lo < -7 ? -7 : (lo > 7 ? 7 : lo);
            hi = hi < -7 ? -7 : (hi > 7 ? 7 : hi);
            packed[r * (cols / 2) + c / 2] = (uint8_t)((lo & 0x0f) | ((hi & 0x0f) << 4));
        }
    }
    free(rot);
    return 0;
}

/* int4_gemm (core/kernels/h3_kernels.cpp:546-635): acc[m][n] = sum_k A[m][k] *
 * nib(B[n], k), nib the signed low (even k) or high (odd k) nibble of byte k/2,
 * then C = ((float)acc * sa[m]) * sb[n] in fp32, no bias. */
void orc_int4_gemm(const int8_t* a, int64_t lda, const uint8_t* b, int64_t ldb, const float* sa,
                   const float* sb, int64_t M, int64_t N, int64_t K, float* c, int64_t ldc) {
    int8_t* row = (int8_t*)malloc((size_t)K);
    for (int64_t n = 0; n < N; n++) {
        for (int64_t k = 0; k < K; k++) {
            int v = (b[n * ldb + k / 2] >> (4 * (k & 1))) & 0x0f;
            row[k] = (int8_t)(v >= 8 ? v - 16 : v);
        }
        for (int64_t m = 0; m < M; m++) {
            int32_t acc = 0;
            for (int64_t k = 0; k < K; k++) acc += (int32_t)a[m * lda + k] * row[k];
            c[m * ldc + n] = ((float)acc * sa[m]) * sb[n];
        }
    }
    free(row);
}

/* ------------------------------------------------------------------------ */
/* LoRA tail: out += (x A^T) B^T (core/models/model_common.cpp:1667-1700)   */
/* ------------------------------------------------------------------------ */

/* h[m][r] = fma chain over k ascending of x[m][k] * A[r][k] from 0, as
 * gemm_f16's `acc += av * bv` under NVRTC's --fmad=true
 * (core/kernels/gemm_f16.cpp:56-200, fp32 operands, no bias).  That kernel
 * walks whole 32-deep tiles with zero past K; the padding's only effect is
 * fma(0, 0, -0) = +0, applied once when K % 32 != 0. */
void orc_lora_down(const float* x, int64_t ldx, const float* a, float* h, int64_t M, int64_t K, int64_t R) {
    for (int64_t m = 0; m < M; m++)
        for (int64_t r = 0; r < R; r++) {
            float acc = 0.0f;
            for (int64_t k = 0; k < K; k++) acc = fmaf(x[m * ldx + k], a[r * K + k], acc);
            if (K % 32 != 0) acc = fmaf(0.0f, 0.0f, acc);
            h[m * R + r] = acc;
        }
}

/* c[m][n] = fma chain over r ascending of h[m][r] * b[n][r] from c[m][n]
 * (lora_rank_add, core/kernels/gemm_f16.cpp:237-308). */
void orc_lora_rank_add(const float* h, const float* b, float* c, int64_t ldc, int64_t M, int64_t N, int64_t R) {
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            float acc = c[m * ldc + n];
            for (int64_t r = 0; r < R; r++) acc = fmaf(h[m * R + r], b[n * R + r], acc);
            c[m * ldc + n] = acc;
        }
}

/* ------------------------------------------------------------------------ */
/* A9: GELU-tanh                                                            */
/* ------------------------------------------------------------------------ */

/* 0.5 x (1 + tanh(0.7978845608028654 (x + 0.044715 x^3))), fp32, the
 * operation order of core/kernels/ops.cpp:83-89, with the one contraction
 * NVRTC's default --fmad=true makes there: the cube's last product fused into
 * the add, fma(0.044715 x x, x, x). */
void orc_gelu_tanh(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        const float a = x[i];
        const float t = 0.7978845608028654f * fmaf(0.044715f * a * a, a, a);
        y[i] = 0.5f * a * (1.0f + tanhf(t));
    }
}

/* SiLU gate over gx [rows, 2 cols]: out[r][c] = (g / (1 + exp(-g))) * v with
 * g = gx[r][c], v = gx[r][cols + c] (core/kernels/conv3d_causal.cpp:997-1013;
 * OP_SILU_GATE core/kernels/ops.cpp:75).  No product feeds an add, so there is
 * nothing to contract. */
void orc_silu_gate(const float* gx, float* out, int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; r++)
        for (int64_t c = 0; c < cols; c++) {
            const float g = gx[r * 2 * cols + c], v = gx[r * 2 * cols + cols + c];
            out[r * cols + c] = (g / (1.0f + expf(-g))) * v;
        }
}

/* ---- fused neighbours: ModAdd and AddMul (core/kernels/ops.cpp:80-82) ---- */
void orc_mod_add(const float* a, const float* b, const float* c, float* y, int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; r++)
        for (int64_t k = 0; k < cols; k++) {
            const float one_b = 1.0f + (b ? b[k] : 0.0f);
            y[r * cols + k] = fmaf(a[r * cols + k], one_b, c ? c[k] : 0.0f);
        }
}

void orc_add_mul(const float* a, const float* b, const float* c, float* y, int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; r++)
        for (int64_t k = 0; k < cols; k++) y[r * cols + k] = fmaf(b[r * cols + k], c[k], a[r * cols + k]);
}

/* ------------------------------------------------------------------------ */
/* fp8 and nvfp4 / mxfp4 weights                                            */
/* ------------------------------------------------------------------------ */

/* core/host/quant.cpp:433-439 */
void orc_dequant_fp8_rows(const uint8_t* codes, int64_t ld, int64_t rows, int64_t k, int dtype, const float* scale,
                          float* out) {
    for (int64_t r = 0; r < rows; r++) {
        const float s = scale ? scale[r] : 1.0f;
        for (int64_t c = 0; c < k; c++) {
            const uint8_t b = codes[r * ld + c];
            out[r * k + c] = (dtype == ORC_F8_E5M2 ? orc_f8_e5m2_to_f32(b) : orc_f8_e4m3_to_f32(b)) * s;
        }
    }
}

/* E2M1 (core/util/media_common.cpp:179-185): magnitudes 0, .5, 1, 1.5, 2, 3,
 * 4, 6 by the low three bits, bit 3 the sign. */
static float e2m1(uint8_t nib) {
    static const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
    return (nib & 8) ? -mag[nib & 7] : mag[nib & 7];
}

/* core/host/quant.cpp:390-410: (row, block) in the cuBLAS tiled table. */
static int64_t tiled_index(int64_t row, int64_t blk, int64_t nb_c, int64_t cols) {
    const int64_t i_r = row / 128, h = row % 128, i_c = blk / 4, w = blk % 4, a = h / 32, b = h % 32;
    const int64_t flat = (i_r * nb_c + i_c) * 512 + b * 16 + a * 4 + w;
    return (flat / cols) * cols + flat % cols;
}

static size_t scale_bytes(int dtype) {
    switch (dtype) {
        case ORC_F32: return 4;
        case ORC_F16:
        case ORC_BF16: return 2;
        default: return 1;
    }
}

/* core/host/quant.cpp:412-431, with the row's global scale as
 * core/host/st.cpp:494-503 passes it. */
void orc_dequant_fp4_rows(const uint8_t* codes, int64_t ld, int64_t row0, int64_t rows, int64_t k,
                          const void* table, int table_dtype, int64_t table_rows, int64_t table_cols, int64_t block,
                          const float* global, float* out) {
    if (block <= 0) block = 16;
    const int64_t nb_c = table_cols > 0 ? table_cols / 4 : 0;
    const int have = table != NULL && nb_c > 0 && table_rows > 0;
    for (int64_t r = 0; r < rows; r++) {
        const uint8_t* row = codes + r * ld;
        const float g = global ? global[r] : 1.0f;
        for (int64_t c = 0; c < k; c++) {
            const uint8_t b = row[c / 2];
            const uint8_t nib = (uint8_t)((c & 1) ? (b & 0x0F) : (b >> 4));
            float s = 1.0f;
            if (have) {
                const int64_t i = tiled_index(row0 + r, c / block, nb_c, table_cols);
                s = orc_scale_at((const uint8_t*)table + (size_t)i * scale_bytes(table_dtype), table_dtype, 0);
            }
            out[r * k + c] = e2m1(nib) * s * g;
        }
    }
}
