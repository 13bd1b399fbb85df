/*
 * phi_qlinear.h -- C ABI of the MI355X (gfx950) quantized-linear library.
 *
 * The library is the device half of Phi's int8 linear: the 256-wide convrot
 * rotation + per-token int8 quantiser, the int8 x int8 -> int32 GEMM with the
 * scale/bias epilogue, the grouped 4/6-bit weight decode, and the M<=8 GEMV.
 * Every entry point enqueues work on the caller's HIP stream and returns;
 * nothing synchronises and nothing allocates device memory: the caller owns
 * every buffer (the reference's GpuAlloc contract, core/runtime/sched.hpp:27-32,
 * and its VRAM accountant, core/runtime/vram_budget.hpp:42-264).
 *
 * Pointers are plain device addresses (the reference passes GpuBuffer* plus a
 * byte offset, core/runtime/compute.hpp:176-217: fold the offset in).
 * Sizes are int64_t.  Errors come back as a phi_status plus a thread-local
 * message from phi_hip_last_error(); the C++ shim turns them into MediaError
 * the way the reference's dispatchers throw (core/runtime/compute.cpp:552,
 * :665-668, core/kernels/w4a8_expand.cpp:264-281).
 */
#ifndef PHI_QLINEAR_H
#define PHI_QLINEAR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PHI_QLINEAR_ABI_VERSION 1

/* A hipStream_t (NULL = the default stream). */
typedef void* phi_stream_t;

typedef enum phi_status {
    PHI_OK = 0,
    PHI_ERR_ARG = 1,         /* null pointer, bad enum, negative size */
    PHI_ERR_SHAPE = 2,       /* shape contract violated (K % 256, K % group, ...) */
    PHI_ERR_ALIGN = 3,       /* a pointer or leading dimension breaks the alignment rule */
    PHI_ERR_WORKSPACE = 4,   /* workspace too small: see phi_hip_workspace_bytes */
    PHI_ERR_HIP = 5,         /* a HIP runtime call failed */
    PHI_ERR_DEVICE_LOST = 6, /* memory fault / illegal address: the device is unusable */
    PHI_ERR_UNSUPPORTED = 7  /* combination the library does not implement */
} phi_status;

/* Element types. */
typedef enum phi_dtype {
    PHI_F32 = 0,
    PHI_BF16 = 1,
    PHI_F16 = 2,
    PHI_I32 = 3,
    PHI_I8 = 4,
    PHI_F8_E4M3 = 5,
    PHI_F8_E5M2 = 6,
    PHI_U8_E4M3 = 7, /* an E4M3 table in a byte container (RelDType::U8_E4M3) */
    PHI_I4 = 8       /* two signed nibbles per byte, column 2j in the low nibble */
} phi_dtype;

/* Rounding of v * (1/scale) onto the integer grid. */
typedef enum phi_round {
    PHI_ROUND_HALF_AWAY = 0, /* the reference's rule (core/host/quant.cpp:163-166) */
    PHI_ROUND_HALF_EVEN = 1  /* documented alternative */
} phi_round;

/* Activation fused in front of phi_hip_quant_rotate_act. */
typedef enum phi_act {
    PHI_ACT_GELU_TANH = 1, /* ElemOp::GeluTanh (core/kernels/ops.cpp:83-89) */
    PHI_ACT_SILU_GATE = 2  /* silu_gate_fused (core/kernels/conv3d_causal.cpp:997-1013) */
} phi_act;

/* Message for the last failing call on this thread ("" after success). */
const char* phi_hip_last_error(void);
int phi_hip_abi_version(void);

/*
 * Rotate + quantise activations, per row (token).
 * Replaces dispatch_quant_convrot / QuantConvrotArgs
 * (core/runtime/compute.hpp:200-217, core/runtime/compute.cpp:663-684;
 * kernel core/kernels/int8_gemm.cpp:699-802; host maths core/host/quant.cpp:109-169).
 *
 *   x      [rows, ldx] of x_dtype (PHI_F32 or PHI_BF16); ldx >= K
 *   q      [rows, ldq] int8 out; ldq >= K
 *   s      [rows] fp32 out: scale = amax > 1e-30 ? amax / qmax : 1
 *   rotate 1: 256-wide J-2R Hadamard per group first (K % 256 == 0 required)
 *   qmax   127 for int8, 7 for the w4a4 tower (any integer value 1..127)
 * rows == 0 is a no-op (as in the reference).  K <= 32768 when rotate == 1.
 */
phi_status phi_hip_quant_rotate(phi_stream_t stream, const void* x, int x_dtype, int64_t rows,
                                int64_t K, int64_t ldx, int8_t* q, int64_t ldq, float* s,
                                float qmax, int round_mode, int rotate);

/*
 * phi_hip_quant_rotate with the DiT's adaLN modulation fused in front:
 * every element first becomes fma(x, 1 + mod_scale[k], mod_shift[k]) in fp32
 * (either vector may be NULL, meaning 0; both [K] fp32, 16-byte aligned).
 * Replaces dispatch_elem(ElemOp::ModAdd, Row, Row) followed by
 * dispatch_quant_convrot (core/models/av_dit.cpp:1264-1267; ModAdd
 * core/kernels/gpu_ops.hpp:29-35, maths core/kernels/ops.cpp:82 as NVRTC's
 * default --fmad=true contracts it), without the modulated tensor's round
 * trip through memory.
 */
phi_status phi_hip_quant_rotate_mod(phi_stream_t stream, const void* x, int x_dtype, int64_t rows,
                                    int64_t K, int64_t ldx, const float* mod_scale, const float* mod_shift,
                                    int8_t* q, int64_t ldq, float* s, float qmax, int round_mode,
                                    int rotate);

/*
 * phi_hip_quant_rotate with the MLP's activation fused in front, so the
 * activated tensor never goes through memory:
 *   PHI_ACT_GELU_TANH  x [rows, ldx >= K]: v = gelu_tanh(x[r][k]).  Replaces
 *     dispatch_elem(ElemOp::GeluTanh) followed by dispatch_quant_convrot
 *     (core/kernels/ops.cpp:83-89).
 *   PHI_ACT_SILU_GATE  x [rows, ldx >= 2K], gate then value halves:
 *     v = silu(x[r][k]) * x[r][K + k].  Replaces dispatch_silu_gate_fused
 *     (core/kernels/h3_kernels.hpp:116-129) followed by dispatch_quant_convrot.
 * The activation is computed in fp32 with the same functions as
 * phi_hip_gelu_tanh / phi_hip_silu_gate, so the codes and scales equal the
 * unfused pair's bit for bit when that pair's intermediate is fp32.
 */
phi_status phi_hip_quant_rotate_act(phi_stream_t stream, const void* x, int x_dtype, int64_t rows, int64_t K,
                                    int64_t ldx, int act, int8_t* q, int64_t ldq, float* s, float qmax,
                                    int round_mode, int rotate);

/*
 * int8 GEMM with the fused dequant epilogue:
 *   C[m,n] = fma((float)acc[m,n] * sA[m], sB[n], bias[n])   (bias = 0 when NULL)
 *   acc[m,n] = sum_k A[m,k] * B[n,k]   (int32, exact)
 * Replaces dispatch_int8_gemm / Int8GemmArgs (core/runtime/compute.hpp:176-198,
 * core/runtime/compute.cpp:551-661; kernel core/kernels/int8_gemm.cpp:466-621,
 * epilogue :588-620).
 *
 *   A [M, lda] int8, B [N, ldb] int8 (K contiguous: the checkpoint's [N,K]).
 *   sA [M] fp32; sB [N] fp32, or [1] when sb_scalar (per-tensor scale).
 *   bias: NULL, or [N] of bias_dtype (PHI_F32 / PHI_BF16).
 *   C [M, ldc] of c_dtype: PHI_F32 (reference), PHI_BF16 (RNE), or PHI_I32
 *     (raw accumulators; scales and bias are then ignored and may be NULL).
 *   Any K > 0 and any byte offset and pitch of A and B: K % 64 == 0 with
 *     16-byte aligned rows takes the MFMA pipelines; anything else the same
 *     MFMA tiles fed by byte-safe loads with the K tail zero-filled (the
 *     reference's dp4a fallback, core/runtime/compute.cpp:566-575).
 *   sA, sB, bias and C: naturally aligned (4 bytes; 2 for a bf16 bias or C).
 *   workspace: may be NULL when phi_hip_workspace_bytes() returns 0 (it
 *     does for every shape: the kernels keep all scratch in LDS).
 */
phi_status phi_hip_i8_gemm(phi_stream_t stream, const int8_t* A, int64_t lda, const int8_t* B,
                           int64_t ldb, const float* sA, const float* sB, int sb_scalar,
                           const void* bias, int bias_dtype, void* C, int c_dtype, int64_t ldc,
                           int64_t M, int64_t N, int64_t K, void* workspace, size_t ws_bytes);

/*
 * phi_hip_i8_gemm into a gated residual stream, in place:
 *   H[m,n] = fma(linear[m,n], gate[n], H[m,n]),  linear = fma((float)acc*sA, sB, bias)
 * H is fp32 [M, ldh] (16-byte aligned rows), gate fp32 [N].  Replaces
 * dispatch_int8_gemm into a scratch projection followed by
 * dispatch_elem(ElemOp::AddMul, Flat, Row) onto the residual
 * (core/models/av_dit.cpp:1382-1390, :1410-1412; maths core/kernels/ops.cpp:80
 * as NVRTC's default --fmad=true contracts it).  Needs K % 256 == 0 and
 * N % 4 == 0 (the persistent kernel); otherwise PHI_ERR_UNSUPPORTED.
 */
phi_status phi_hip_i8_gemm_residual(phi_stream_t stream, const int8_t* A, int64_t lda, const int8_t* B,
                                    int64_t ldb, const float* sA, const float* sB, int sb_scalar,
                                    const void* bias, int bias_dtype, const float* gate, float* H,
                                    int64_t ldh, int64_t M, int64_t N, int64_t K, void* workspace,
                                    size_t ws_bytes);

/* Workspace (bytes) phi_hip_i8_gemm / phi_hip_q8_linear need for this shape. */
size_t phi_hip_workspace_bytes(int64_t M, int64_t N, int64_t K);

/*
 * The fused W8A8 linear: rotate+quantise x into the caller's q8/s8 scratch,
 * then phi_hip_i8_gemm.  Replaces linear_gemm's int8 branch
 * (core/models/model_common.cpp:1384-1411), including its "activation
 * scratch" contract (q8 [M,K] int8, s8 [M] fp32 owned by the caller).
 */
phi_status phi_hip_q8_linear(phi_stream_t stream, const void* x, int x_dtype, int64_t ldx,
                             int64_t M, int64_t K, const int8_t* W, int64_t ldw, const float* sW,
                             int sw_scalar, const void* bias, int bias_dtype, int64_t N, void* C,
                             int c_dtype, int64_t ldc, int8_t* q8, float* s8, int round_mode,
                             void* workspace, size_t ws_bytes);

/*
 * The K-tiled operand layout: an int8 [rows, K] matrix (K % 256 == 0) in
 * strips of 256 rows (the last may hold fewer, h); within a strip, each
 * 64-byte K-step of all h rows is one contiguous h x 64-byte block, and the
 * 16-byte chunk c of row r sits in slot c ^ ((r >> 2) & 3) of the row's 64
 * bytes.  Byte (r, k) of the matrix is at
 *   256 K (r / 256) + h 64 (k / 64) + 64 (r % 256) + 16 (((k / 16) % 4) ^ ((r % 256 / 4) % 4)) + k % 16.
 * It is the persistent GEMM's LDS stage layout, so each operand load moves
 * 1 KB from one place instead of sixteen 64-byte row pieces.  It holds
 * rows x K bytes, as the row-major matrix does.  No counterpart in the
 * reference (its weights stay row-major, core/host/quant.cpp:223-236): these
 * entries serve callers that pack each weight once at load time.
 *
 * phi_hip_pack_k_tiled: src (row-major, pitch ld >= K, ld % 16 == 0, 16-byte
 * aligned) into dst (rows x K bytes, 16-byte aligned).  A pure re-layout.
 */
phi_status phi_hip_pack_k_tiled(phi_stream_t stream, const int8_t* src, int64_t ld, int64_t rows, int64_t K,
                                int8_t* dst);

/* phi_hip_quant_rotate (rotation on) writing q (rows x K bytes) K-tiled,
 * for callers that feed one quantised activation to several K-tiled GEMMs.
 * K % 256 == 0, K <= 16384. */
phi_status phi_hip_quant_rotate_kt(phi_stream_t stream, const void* x, int x_dtype, int64_t rows, int64_t K,
                                  int64_t ldx, int8_t* q, float* s, float qmax, int round_mode);

/* phi_hip_quant_rotate_mod and phi_hip_quant_rotate_act (rotation on) writing
 * q (rows x K bytes) K-tiled: the DiT block's modulation or the MLP's
 * activation fused in front of a K-tiled linear.  K % 256 == 0, K <= 16384. */
phi_status phi_hip_quant_rotate_mod_kt(phi_stream_t stream, const void* x, int x_dtype, int64_t rows, int64_t K,
                                      int64_t ldx, const float* mod_scale, const float* mod_shift, int8_t* q,
                                      float* s, float qmax, int round_mode);
phi_status phi_hip_quant_rotate_act_kt(phi_stream_t stream, const void* x, int x_dtype, int64_t rows, int64_t K,
                                      int64_t ldx, int act, int8_t* q, float* s, float qmax, int round_mode);

/* phi_hip_i8_gemm with A [M, K] and B [N, K] both K-tiled: the same result,
 * bit for bit, as phi_hip_i8_gemm on the row-major operands.  Needs
 * K % 256 == 0, whole 16-byte output pieces (N % 8 for bf16, N % 4 else) on
 * 16-byte aligned C rows; otherwise PHI_ERR_UNSUPPORTED. */
phi_status phi_hip_i8_gemm_kt(phi_stream_t stream, const int8_t* A, const int8_t* B, const float* sA, const float* sB,
                              int sb_scalar, const void* bias, int bias_dtype, void* C, int c_dtype, int64_t ldc,
                              int64_t M, int64_t N, int64_t K);

/* phi_hip_i8_gemm_residual with A and B K-tiled: H = fma(linear, gate[n], H)
 * in place on the fp32 residual stream H [M, ldh].  Same contract as
 * phi_hip_i8_gemm_kt (N % 4 == 0). */
phi_status phi_hip_i8_gemm_residual_kt(phi_stream_t stream, const int8_t* A, const int8_t* B, const float* sA,
                                       const float* sB, int sb_scalar, const void* bias, int bias_dtype,
                                       const float* gate, float* H, int64_t ldh, int64_t M, int64_t N, int64_t K);

/* The rows of an M x N persistent GEMM on the current device that run as
 * 256 x 256 tiles (a multiple of 256, or M); the rest run as 128 x 128 tiles
 * in the same launch.  The plan minimises the rounds of tiles over the
 * device's compute units.  0 for an empty problem. */
int64_t phi_hip_big_tile_rows(int64_t M, int64_t N);

/* The GEMM tuning table (replaces the reference's autotune store and tuned
 * dispatch, core/kernels/autotune.hpp:30-88: a stored launch configuration per
 * kernel, found by a sweep that checks every variant bit-identical).  Here a
 * plan per problem shape and operand layout for the persistent int8 GEMM that
 * phi_hip_i8_gemm / _kt, phi_hip_q8_linear / _kt and the gated residual run:
 *   big_rows  rows run as 256 x 256 tiles: a multiple of 256 up to M, or M;
 *             -1 leaves it to the library's cost model (phi_hip_big_tile_rows)
 *   group_m   tile rows per group of the XCD-aware tile order, 1..16; 0: 4
 *   split     1: the two tile sizes as two launches; 0: one launch
 *   tile      PHI_PLAN_TILE_SQUARE: the 256 x 256 / 128 x 128 plan above;
 *             PHI_PLAN_TILE_272: 272 x 192 tiles (K % 512 == 0 only; big_rows
 *             and split do not apply, group_m does); PHI_PLAN_TILE_AUTO (0):
 *             the library's cost model picks
 *   reserved  0
 * Every plan gives the same bits; only the time differs.  The table is
 * process-wide and thread-safe; the host layer's GemmTuneStore sweeps,
 * persists and loads it.  _set with plan NULL removes the shape's entry;
 * _get returns the plan a launch of that shape runs, the tile shape resolved
 * (tuned = 1 when it comes from the table).  PHI_GEMM_T272=0 / 1 in the
 * environment overrides the tile shape (an A/B switch). */
#define PHI_PLAN_TILE_AUTO 0
#define PHI_PLAN_TILE_SQUARE 1
#define PHI_PLAN_TILE_272 2
typedef struct phi_gemm_plan {
    int64_t big_rows;
    int32_t group_m;
    int32_t split;
    int32_t tile;
    int32_t reserved;
} phi_gemm_plan;
phi_status phi_hip_gemm_plan_set(int64_t M, int64_t N, int64_t K, int k_tiled, const phi_gemm_plan* plan);
phi_status phi_hip_gemm_plan_get(int64_t M, int64_t N, int64_t K, int k_tiled, phi_gemm_plan* plan, int* tuned);
int64_t phi_hip_gemm_plan_count(void);
void phi_hip_gemm_plan_clear(void);

/* phi_hip_q8_linear with the weight W K-tiled (phi_hip_pack_k_tiled at load
 * time): the prologue writes q8 (M x K bytes) K-tiled, then phi_hip_i8_gemm_kt.
 * C is bit-identical to phi_hip_q8_linear's; s8 is the same; q8 holds the same
 * bytes in the K-tiled layout.  Also needs K <= 16384. */
phi_status phi_hip_q8_linear_kt(phi_stream_t stream, const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K,
                                const int8_t* W, const float* sW, int sw_scalar, const void* bias, int bias_dtype,
                                int64_t N, void* C, int c_dtype, int64_t ldc, int8_t* q8, float* s8, int round_mode);

/* linear_gemm's int8 branch (core/models/model_common.cpp:1384-1411) for a
 * row-major weight, as phi_hip_q8_linear (same arguments, same C and s8, bit
 * for bit), with the activation scratch q8 written K-tiled where the
 * 272 x 192 plan takes the problem (K % 256 == 0, K <= 16384, 16-byte
 * aligned q8, W rows and C rows): the GEMM then reads A in K-tiled pieces
 * and only the weight's rows are gathered.  Elsewhere it is phi_hip_q8_linear
 * and q8 is row-major.  q8 is scratch either way: callers must not read it. */
phi_status phi_hip_q8_linear_kq(phi_stream_t stream, const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K,
                                const int8_t* W, int64_t ldw, const float* sW, int sw_scalar, const void* bias,
                                int bias_dtype, int64_t N, void* C, int c_dtype, int64_t ldc, int8_t* q8, float* s8,
                                int round_mode, void* workspace, size_t ws_bytes);

/* A grouped low-bit weight as the checkpoint stores it
 * (W4a8ExpandArgs, core/kernels/w4a8_expand.hpp:86-117). */
typedef struct phi_w4a8_weight {
    const uint8_t* codes;      /* [rows, codes_row_bytes] packed codes */
    int64_t codes_row_bytes;   /* >= k/2 (nibble4) or k/2 + k/4 (packed6) */
    const void* s_rel;         /* [rows, srel_row_bytes]: k/group relative scales */
    int s_rel_dtype;           /* PHI_F32/F16/BF16/F8_E4M3/F8_E5M2/U8_E4M3 */
    int64_t srel_row_bytes;
    const float* s_channel;    /* NULL (1.0), [rows], or [1] when sch_scalar */
    int sch_scalar;
    const float* codebook;     /* NULL (level = code - 8), or 16 fp32 levels */
    const float* correction;   /* NULL, or [k/group, rows] fp32 additive plane */
    int64_t rows;              /* N */
    int64_t k;                 /* K, a whole number of groups */
    int64_t group;             /* columns per relative scale */
    int layout;                /* 0: nibble4 (asym_w4a8_int8), 1: packed6 (w6a8_int8) */
} phi_w4a8_weight;

/*
 * Decode to the int8 GEMM operand: q [rows, k] int8 and s [rows] fp32, the
 * reference's device expand (core/kernels/w4a8_expand.cpp:151-258,
 * dispatch :263-303) and host decode+requantise (core/host/quant.cpp:315-389
 * then :134-169 without rotation).  A correction plane (host path only in the
 * reference, core/host/st.cpp:447-491) is supported.
 */
phi_status phi_hip_w4a8_expand(phi_stream_t stream, const phi_w4a8_weight* w, int8_t* q,
                               float* s);

/*
 * Load-time preparation for the in-register W4A8 GEMM: per (row, group) a
 * 16-entry int8 table lut[row][group][code] equal to the expanded code the
 * reference would produce for that nibble, and the per-row scale s [rows].
 * Nibble4 layout only.  No reference counterpart as an entry point: it is the
 * expand of phi_hip_w4a8_expand factored per (row, group), so the GEMM can
 * unpack nibbles in registers.
 */
phi_status phi_hip_w4a8_prepare(phi_stream_t stream, const phi_w4a8_weight* w, int8_t* lut,
                                float* s);

/*
 * W4A8 linear with nibbles unpacked through the prepared table.
 * Equal, bit for bit, to phi_hip_w4a8_expand followed by phi_hip_q8_linear.
 *   codes [N, codes_row_bytes] nibble4; lut [N, K/group, 16]; s_w [N].
 *   group % 64 == 0.
 *   workspace: optional, phi_hip_w4a8_workspace_bytes() bytes (16-byte
 *     aligned).  Given it, a call with many rows expands the codes once into
 *     it (int8 [N, K]) and runs the W8A8 GEMM; without it, or for few rows,
 *     the GEMM expands the codes tile by tile: for K % 1024 == 0 (K <= 16384)
 *     in LDS, once per workgroup, on the 272 x 192 pipeline, otherwise in
 *     registers.  Same bits on every path.
 *     The expand-once path and the LDS path (K <= 16384) keep the activation
 *     codes in the K-tiled layout (phi_hip_pack_k_tiled), so q8 then holds
 *     them K-tiled; s8 is the same on every path.
 */
phi_status phi_hip_w4a8_linear(phi_stream_t stream, const void* x, int x_dtype, int64_t ldx,
                               int64_t M, int64_t K, const uint8_t* codes,
                               int64_t codes_row_bytes, const int8_t* lut, int64_t group,
                               const float* s_w, const void* bias, int bias_dtype, int64_t N,
                               void* C, int c_dtype, int64_t ldc, int8_t* q8, float* s8,
                               int round_mode, void* workspace, size_t ws_bytes);

/* One weight of a batched GEMV. */
typedef struct phi_gemv_item {
    const int8_t* W;   /* [N, K] int8, rows 16-byte aligned */
    const float* sW;   /* [N] fp32, or [1] when sw_scalar */
    int sw_scalar;
    const void* bias;  /* NULL or [N] of the call's bias_dtype */
    void* C;           /* [M, ldc] of the call's c_dtype */
    int64_t ldc;
} phi_gemv_item;

/*
 * Small-M (M <= 8) linear over many weights that share one quantised
 * activation block: C_i = epilogue(q8 . W_i^T) for every item.  The
 * activations are quantised by the caller (phi_hip_quant_rotate) into
 * q8 [M, K] / s8 [M].  The adaLN modulation shape of the DiT blocks
 * (reference: host fp32, core/models/image_dit.cpp:1047-1072); same
 * arithmetic contract as phi_hip_i8_gemm.  items must be in host memory.
 */
phi_status phi_hip_i8_gemv_batched(phi_stream_t stream, const int8_t* q8, const float* s8,
                                   int64_t M, int64_t K, int64_t N, const phi_gemv_item* items,
                                   int n_items, int bias_dtype, int c_dtype, void* workspace,
                                   size_t ws_bytes);

/* The W4A8 weight packed for the in-LDS expansion (no counterpart in the
 * reference, whose loaders expand W4A8 to int8 at load time,
 * core/models/model_common.cpp:589-748): once per weight, codes (the nibble
 * layout, 16-byte aligned rows) and the table phi_hip_w4a8_prepare wrote are
 * laid out in bands of 192 rows, one contiguous block per band and K-step
 * (codes) or group (tables), so that the GEMM's loads read whole blocks
 * instead of gathering 32 code rows each.  phi_hip_w4a8_banded_bytes gives
 * the buffer's size (0 for a shape it cannot hold).
 * phi_hip_w4a8_linear_banded is phi_hip_w4a8_linear on it, with no
 * workspace: the same C and s8 bit for bit; q8 (M x K bytes) is written
 * K-tiled.  Needs K % 1024 == 0, K <= 16384, group a power of two >= 64, and
 * the phi_hip_q8_linear_kt rules for q8 and C. */
size_t phi_hip_w4a8_banded_bytes(int64_t rows, int64_t k, int64_t group);
phi_status phi_hip_w4a8_pack_banded(phi_stream_t stream, const uint8_t* codes, int64_t codes_row_bytes,
                                    const int8_t* lut, int64_t rows, int64_t k, int64_t group, void* banded);
phi_status phi_hip_w4a8_linear_banded(phi_stream_t stream, const void* x, int x_dtype, int64_t ldx, int64_t M,
                                      int64_t K, const void* banded, int64_t group, const float* s_w, const void* bias,
                                      int bias_dtype, int64_t N, void* C, int c_dtype, int64_t ldc, int8_t* q8,
                                      float* s8, int round_mode);

/* Workspace with which phi_hip_w4a8_linear expands the codes once per call
 * (N*K bytes; 0 when the shape keeps the in-register expansion).  No reference
 * counterpart: the reference expands at load time (dispatch_w4a8_expand). */
size_t phi_hip_w4a8_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group);

/*
 * int4 GEMM of the convrot_w4a4 family (the text encoder's weights):
 *   C[m, n] = ((float)acc * sA[m]) * sB[n],  acc = sum_k A[m, k] * w[n, k]
 * A [M, lda] int8 (activations rotated and quantised with qmax 7 by
 * phi_hip_quant_rotate); B [N, ldb] bytes of packed signed nibbles, column 2j in
 * the low nibble of byte j (w = code < 8 ? code : code - 16); sA [M], sB [N]
 * fp32; C [M, ldc] of c_dtype (PHI_F32 as the reference, PHI_BF16 RNE, or
 * PHI_I32 for the raw accumulators, which need no scales).  K % 512 == 0, as
 * the reference requires.  workspace: optional, phi_hip_i4_workspace_bytes()
 * bytes (the codes are then expanded once per call; same bits).
 * Replaces dispatch_int4_gemm / Int4GemmArgs (core/kernels/h3_kernels.hpp:90-107,
 * core/kernels/h3_kernels.cpp:546-662).
 */
phi_status phi_hip_i4_gemm(phi_stream_t stream, const int8_t* A, int64_t lda, const uint8_t* B, int64_t ldb,
                           const float* sA, const float* sB, void* C, int c_dtype, int64_t ldc, int64_t M,
                           int64_t N, int64_t K, void* workspace, size_t ws_bytes);

/* Workspace with which phi_hip_i4_gemm expands the codes once per call (N*K
 * bytes from 512 rows up; 0 otherwise).  No reference counterpart. */
size_t phi_hip_i4_workspace_bytes(int64_t M, int64_t N, int64_t K);

/*
 * Runtime LoRA correction of a linear's output, out += (x A^T) B^T, as the
 * reference's apply_lora_tail (core/models/model_common.cpp:1667-1700):
 *   x   [M, ldx >= K] of x_dtype (PHI_F32 as the reference, or PHI_BF16): the linear's input
 *   At  [R, K] fp32: the factors' A rows, stacked (LoraTail::at)
 *   Bt  [N, R] fp32: the factors' B columns, scaled (LoraTail::bt)
 *   out [M, ldo >= N] of out_dtype (PHI_F32 as the reference, or PHI_BF16), updated in place
 *   h   caller scratch of h_bytes >= M*R*4 (the [M, R] fp32 hidden form)
 * Both products are fp32 fma chains in the reference's order (k ascending from
 * 0 for h; r ascending from out's value for the update), so an fp32 out is
 * bit-exact.  M <= 0 or R <= 0 is a no-op (an inactive tail).  h must not
 * overlap x or out.
 */
phi_status phi_hip_lora_tail(phi_stream_t stream, const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K,
                             const float* At, const float* Bt, int64_t R, int64_t N, void* out, int out_dtype,
                             int64_t ldo, float* h, size_t h_bytes);

/* The tail's first product, h [M, R] = x . At^T in fp32 (replaces dispatch_gemm_f16
 * with fp32 operands and no bias, core/kernels/gemm_f16.cpp:56-200, as
 * apply_lora_tail uses it). */
phi_status phi_hip_lora_down(phi_stream_t stream, const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K,
                             const float* A, int64_t R, float* h);

/* The tail's update, C [M, ldc] += h [M, R] . B [N, R]^T, fp32 chain from C's
 * value (replaces dispatch_lora_rank_add / LoraRankAddArgs,
 * core/kernels/gpu_ops.hpp:190-196, kernel core/kernels/gemm_f16.cpp:237-308). */
phi_status phi_hip_lora_rank_add(phi_stream_t stream, const float* h, const float* B, void* C, int c_dtype,
                                 int64_t ldc, int64_t M, int64_t N, int64_t R);

/* Workspace for phi_hip_i8_gemv_batched (holds the item table on the device). */
size_t phi_hip_gemv_workspace_bytes(int n_items);

/* GELU-tanh over bf16 or fp32 [n] (core/kernels/ops.cpp:83-89), in place
 * allowed when the dtypes are equal; out_dtype PHI_BF16 rounds RNE. */
phi_status phi_hip_gelu_tanh(phi_stream_t stream, const void* x, int x_dtype, void* y,
                             int y_dtype, int64_t n);

/* SiLU gate: out[r][c] = silu(gx[r][c]) * gx[r][cols + c], gx [rows, ldx >= 2*cols],
 * out [rows, ldo >= cols], each f32 or bf16 (RNE), out not overlapping gx.
 * Replaces dispatch_silu_gate_fused (core/kernels/h3_kernels.hpp:116-129,
 * kernel core/kernels/conv3d_causal.cpp:997-1013). */
phi_status phi_hip_silu_gate(phi_stream_t stream, const void* gx, int x_dtype, int64_t rows, int64_t cols,
                             int64_t ldx, void* out, int out_dtype, int64_t ldo);

/*
 * Load-time weight steps, on the device.  The reference runs these on the
 * host while a loader turns a checkpoint tensor into the int8 GEMM operand;
 * here the host layer's loaders (load_quant_linear, load_quant3_linear,
 * upload_quant_linear_i8) chain them with phi_hip_quant_rotate, which is the
 * reference's weight quantiser as well (quantize_weight and
 * quantize_activation share quantize_impl_into, core/host/quant.cpp:134-195).
 */

/* The values of a stored tensor in fp32, as SafeTensors::dequant_rows
 * computes them (core/host/st.cpp:601-700): PHI_I8 codes, or PHI_I4 signed
 * nibbles (a bare packed int4), times their row's scale ((float)q * s;
 * row_scale [rows], or [1] when scale_scalar; NULL means 1 for PHI_I4),
 * PHI_F8_E4M3 / PHI_F8_E5M2 codes decoded and times the row scale (NULL
 * means 1; dequant_fp8_row, core/host/quant.cpp:433-439), PHI_F16 / PHI_BF16
 * widened exactly, PHI_F32 copied.  src [rows, lds] elements (bytes for
 * PHI_I4), out [rows, ldo] fp32. */
phi_status phi_hip_dequant_rows(phi_stream_t stream, const void* src, int src_dtype, int64_t rows, int64_t cols,
                                int64_t lds, const float* row_scale, int scale_scalar, float* out, int64_t ldo);

/* nvfp4 / mxfp4 weight rows in fp32 (replaces the host loop of
 * dequant_nvfp4_row, core/host/quant.cpp:390-431, as SafeTensors::dequant_rows
 * calls it, core/host/st.cpp:465-503): for rows row0 .. row0 + rows - 1 of the
 * weight, out[r][c] = (e2m1(code) * block_scale[i]) * global_scale[r], where
 * code is column c's nibble of codes + r * codes_ld (even columns in the HIGH
 * nibble) and i is (row0 + r, c / block)'s index in the cuBLAS-tiled table of
 * scale_rows x scale_cols entries (already decoded to fp32; NULL, or fewer
 * than 4 columns: 1).  global_scale: [rows], [1] when global_scalar, or NULL
 * (1).  block <= 0 means 16.  PHI_ERR_SHAPE when the table does not cover a
 * (row, block) the call reads. */
phi_status phi_hip_dequant_fp4_rows(phi_stream_t stream, const uint8_t* codes, int64_t codes_ld, int64_t row0,
                                    int64_t rows, int64_t k, const float* block_scale, int64_t scale_rows,
                                    int64_t scale_cols, int64_t block, const float* global_scale, int global_scalar,
                                    float* out, int64_t ldo);

/* The 256-wide J-2R rotation of fp32 rows alone, y = H x per group with the
 * reference's butterfly order and final 1/16 (convrot_forward,
 * core/host/quant.cpp:66-100; H is an involution, so this is also
 * convrot_inverse, core/host/quant.hpp:63-65).  K % 256 == 0; y == x (equal
 * pitches) runs in place. */
phi_status phi_hip_convrot_rows(phi_stream_t stream, const float* x, int64_t rows, int64_t K, int64_t ldx, float* y,
                                int64_t ldy);

/* Fold one LoRA factor into fp32 weight rows in place:
 *   w[o][i] += (scale * B[o][r]) * A[r][i]  for r = 0..rank-1, skipping B[o][r] == 0,
 * each product and sum rounded on its own (LoraSet::apply_rows_of,
 * core/models/lora.cpp:182-201).  w [rows, ldw]; A [rank, k]; B [rows, rank]:
 * the factor's B rows for these weight rows. */
phi_status phi_hip_lora_fold(phi_stream_t stream, float* w, int64_t ldw, int64_t rows, int64_t k, const float* A,
                             const float* B, int64_t rank, float scale);

/*
 * phi_hip_q8_linear without caller scratch, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments, arithmetic
 * and bits as phi_hip_q8_linear (it runs phi_hip_q8_linear_kq); its q8
 * (M x K bytes) / s8 [M] activation scratch is
 * a static device array of PHI_NOALLOC_SCRATCH_BYTES per GPU (held from the
 * library's load until the process ends), so M * K (rounded up to 256) + 4 M
 * must fit in it: larger calls return PHI_ERR_WORKSPACE.  Allocates nothing.
 * All calls on one GPU share that GPU's array: calls that overlap on one GPU
 * (other streams, other threads) race.
 */
#define PHI_NOALLOC_SCRATCH_BYTES (64ull << 20)
size_t phi_hip_noalloc_scratch_bytes(void);
phi_status phi_hip_q8_linear_noalloc(phi_stream_t stream, const void* x, int x_dtype, int64_t ldx, int64_t M,
                                     int64_t K, const int8_t* W, int64_t ldw, const float* sW, int sw_scalar,
                                     const void* bias, int bias_dtype, int64_t N, void* C, int c_dtype, int64_t ldc,
                                     int round_mode);

#ifdef __cplusplus
}
#endif

#endif /* PHI_QLINEAR_H */
