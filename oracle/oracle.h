/*
 * CPU oracle for the quantized-linear hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the reference's CPU arithmetic for the
 * W8A8 / W4A8 linear.  It is the checker the GPU path is compared against:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The product library (phi-agent_amd/) never links or calls it.
 *
 * Every function names the reference file:line it restates (paths are
 * relative to the reference checkout's root).
 */
#ifndef PHI_ORACLE_H
#define PHI_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types understood by the scale / activation readers */
enum orc_dtype {
    ORC_F32 = 0,
    ORC_BF16 = 1,
    ORC_F16 = 2,
    ORC_I32 = 3,
    ORC_I8 = 4,
    ORC_F8_E4M3 = 5,
    ORC_F8_E5M2 = 6,
    ORC_U8_E4M3 = 7 /* an E4M3 table stored in a byte container */
};

/* HALF_AWAY: the host rule (core/host/quant.cpp:163-166), the library's contract.
 * HALF_EVEN: the documented alternative.
 * DEVICE_FLOOR: the reference's device kernel (core/kernels/int8_gemm.cpp:777-780):
 * clamp to +-qmax in fp32, then floorf(d + 0.5f) / ceilf(d - 0.5f) with fp32 sums,
 * which differs from HALF_AWAY exactly at d = +-(0.5 - 2^-25). */
enum orc_round { ORC_ROUND_HALF_AWAY = 0, ORC_ROUND_HALF_EVEN = 1, ORC_ROUND_DEVICE_FLOOR = 2 };

/* ---- scalar conversions (core/util/media_common.cpp:62-193) ---- */
float orc_f16_to_f32(uint16_t h);              /* media_common.cpp:62-87 */
float orc_bf16_to_f32(uint16_t h);             /* media_common.cpp:116-121 */
uint16_t orc_f32_to_bf16(float f);             /* media_common.cpp:187-193 */
float orc_f8_e4m3_to_f32(uint8_t b);           /* media_common.cpp:130-160 */
float orc_f8_e5m2_to_f32(uint8_t b);           /* media_common.cpp:130-160 */
float orc_scale_at(const void* p, int dtype, int64_t i); /* core/host/quant.cpp:285-299 */
void orc_f32_to_bf16_n(const float* x, uint16_t* y, int64_t n);
void orc_bf16_to_f32_n(const uint16_t* x, float* y, int64_t n);

/* ---- A1: 256-wide J-2R Hadamard per group (core/host/quant.cpp:66-131) ---- */
void orc_convrot_rows(const float* x, float* out, int64_t rows, int64_t cols);

/* ---- A2: per-row int8 quantiser (core/host/quant.cpp:134-169; qmax from
 *      core/kernels/int8_gemm.cpp:755) ----
 * x is f32 or bf16 [rows, ldx]; rotate selects the convrot pre-pass.
 * Returns 0, or -1 when cols is not a whole number of 256-groups. */
/* ---- fp8 and nvfp4 / mxfp4 weights (SafeTensors::dequant_rows, core/host/st.cpp:601-621, :465-503) ---- */
/* dequant_fp8_row (core/host/quant.cpp:433-439): out = f8(code) * scale[r]
 * (scale NULL: 1); dtype ORC_F8_E4M3 or ORC_F8_E5M2; codes [rows, ld]. */
void orc_dequant_fp8_rows(const uint8_t* codes, int64_t ld, int64_t rows, int64_t k, int dtype, const float* scale,
                          float* out);
/* dequant_nvfp4_row (core/host/quant.cpp:390-431) for weight rows row0 ..
 * row0 + rows - 1: out = e2m1(nibble) * table[tiled index of (row, c / block)]
 * * global[r]; the even column in the high nibble; the table read through
 * orc_scale_at with its dtype (NULL, or fewer than 4 columns: 1); global NULL: 1. */
void orc_dequant_fp4_rows(const uint8_t* codes, int64_t ld, int64_t row0, int64_t rows, int64_t k,
                          const void* table, int table_dtype, int64_t table_rows, int64_t table_cols, int64_t block,
                          const float* global, float* out);

/* Every fp32 d with |d| <= 128 whose HALF_AWAY and DEVICE_FLOOR codes differ:
 * returns how many, and stores the first `cap` of them in `out`. */
int64_t orc_round_forms_differ(float* out, int64_t cap);
int orc_quantize_rows(const void* x, int x_dtype, int64_t rows, int64_t cols, int64_t ldx,
                      int rotate, float qmax, int round_mode, int8_t* q, float* s);

/* ---- A4: int8 x int8 -> int32 (core/host/quant.cpp:223-236) ----
 * A [M, lda], B [N, ldb] (K contiguous), acc [M, N]. */
void orc_gemm_i8_i32(const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb, int64_t M,
                     int64_t N, int64_t K, int32_t* acc);

/* ---- A5: epilogue (core/kernels/int8_gemm.cpp:588-620; host :233) ----
 * out = fma((float)acc * sa[m], sb[n], bias[n])  -- bias 0 when absent.
 * fused=0 gives the separately-rounded (acc*sa)*sb + bias instead.
 * sb_scalar broadcasts sb[0]; bias_dtype is ORC_F32 or ORC_BF16 (or -1: none).
 * out_dtype ORC_F32 writes float, ORC_BF16 writes uint16 bf16 (RNE). */
void orc_epilogue(const int32_t* acc, int64_t M, int64_t N, const float* sa, const float* sb,
                  int sb_scalar, const void* bias, int bias_dtype, int fused, void* out,
                  int out_dtype);

/* ---- composite W8A8 linear: A1+A2 on x, A4, A5 ---- */
int orc_q8_linear(const void* x, int x_dtype, int64_t M, int64_t K, const int8_t* W,
                  const float* sw, int sw_scalar, const void* bias, int bias_dtype, int64_t N,
                  int round_mode, void* out, int out_dtype, int8_t* q_out, float* s_out,
                  int32_t* acc_out);

/* ---- A7: grouped 4/6-bit weight decode + per-row requantise ----
 * core/host/quant.cpp:315-389 (int8_grid, grouped_value, dequant_codebook_int4_row,
 * dequant_packed6_row) followed by quantize_weight_into without rotation
 * (core/host/st.cpp:1040-1048 turns rotation off for convrot files).
 * layout 0: nibble4 (asym_w4a8_int8), 1: packed6 (w6a8_int8).
 * s_channel: NULL, or [rows] (sch_scalar=0) or [1] (sch_scalar=1).
 * codebook: NULL or 16 floats.  correction: NULL or [groups][rows] fp32.
 * values (optional, [rows, k]) receives the decoded fp32 weights. */
int orc_w4a8_expand(const uint8_t* codes, int64_t codes_row_bytes, const void* s_rel,
                    int s_rel_dtype, int64_t srel_row_bytes, const float* s_channel,
                    int sch_scalar, const float* codebook, const float* correction,
                    int64_t rows, int64_t k, int64_t group, int layout, int8_t* q, float* s,
                    float* values);

/* ---- fused neighbours of the linear (core/kernels/ops.cpp:71-92, the opcode
 *      table; NVRTC compiles it with its default --fmad=true, which contracts
 *      each multiply-add below into one fma) ----
 * ModAdd (op 12, Row/Row modes, the adaLN modulation before a projection,
 * core/models/av_dit.cpp:1264):  y = fma(a, 1 + b[col], c[col])
 * AddMul (op 6, Flat/Row modes, the gated residual after a projection,
 * core/models/av_dit.cpp:1389):  y = fma(b, c[col], a)
 * b or c may be NULL (0).  a, b, y are [rows, cols]. */
void orc_mod_add(const float* a, const float* b, const float* c, float* y, int64_t rows, int64_t cols);
void orc_add_mul(const float* a, const float* b, const float* c, float* y, int64_t rows, int64_t cols);

/* ---- A9: GELU-tanh (core/kernels/ops.cpp:83-89) ---- */
int orc_quantize_convrot_w4a4(const float* w, int64_t rows, int64_t cols, uint8_t* packed, float* scales);
void orc_int4_gemm(const int8_t* a, int64_t lda, const uint8_t* b, int64_t ldb, const float* sa,
                   const float* sb, int64_t M, int64_t N, int64_t K, float* c, int64_t ldc);
void orc_lora_down(const float* x, int64_t ldx, const float* a, float* h, int64_t M, int64_t K, int64_t R);
void orc_lora_rank_add(const float* h, const float* b, float* c, int64_t ldc, int64_t M, int64_t N, int64_t R);
void orc_gelu_tanh(const float* x, float* y, int64_t n);
void orc_silu_gate(const float* gx, float* out, int64_t rows, int64_t cols);

#ifdef __cplusplus
}
#endif

#endif
