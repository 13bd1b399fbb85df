// Launch parameters shared by the int8 GEMM / GEMV kernels and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace phi_dev {

enum CKind { C_F32 = 0, C_BF16 = 1, C_I32 = 2 };
enum BiasKind { BIAS_NONE = 0, BIAS_F32 = 1, BIAS_BF16 = 2 };

struct GemmParams {
    const int8_t* A;
    const int8_t* B;
    const float* sA;
    const float* sB;
    const void* bias;
    void* C;
    int64_t lda, ldb, ldc;
    int M, N, K;
    int sb_scalar;
    int bias_kind;
    int c_kind;
    int group_m;  // tile-rows walked together inside one XCD's range
    // W4A8 operand (B = packed nibbles): per (row, group) 16-entry int8 table.
    const int8_t* lut;
    int64_t lut_groups;  // groups per row (K / group)
    int group_shift;     // log2(group)
    int c_vec;           // C rows allow 4-element vector stores (alignment and ldc % 4)
    int c_vec16;         // C rows allow 16-byte stores (16-byte aligned, row pitch a multiple of 16 bytes)
    int s_vec;           // sB and bias allow 4-element vector loads (16-byte / 8-byte aligned)
    int schedule;        // 256x256 kernel: 0 = eight waves, 64-deep K; 1 = four waves, 128-deep K
    // Persistent kernel, fp32 output: C = fma(linear, gate[n], C) in place (gated residual).
    const float* gate;
    // W4 operand of signed nibbles (convrot_w4a4): value = code < 8 ? code : code - 16,
    // from a constant table in registers; lut is not read.
    int w4_signed;
    // Persistent pipeline: A and B in the K-tiled layout (k_tiled_offset) instead
    // of row-major; lda / ldb are then K.
    int kt;
    // With kt, the 272 x 192 kernel only: B stays row-major (pitch ldb) while
    // A is K-tiled.  No other kernel reads it; it must be 0 for them.
    int b_rm;
    // The in-LDS W4 kernel only: B and lut point into one band-packed buffer
    // (w4_banded_bytes, the codes region then the tables region) instead of
    // the checkpoint's code rows and the [N, K / group, 16] table.
    int w4_banded;
};

// The K-tiled operand layout: rows in strips of 256 (the last strip may be
// shorter, h rows); within a strip, each 64-byte K-step of all h rows is one
// contiguous block of h x 64 bytes, and 16-byte chunk c of row r sits in slot
// c ^ ((r >> 2) & 3) of the row's 64 bytes -- the persistent pipeline's LDS
// stage layout, so a stage fills with contiguous 1 KB loads.  Byte offset of
// row r, column c (K columns, `rows` rows in all):
__host__ __device__ __forceinline__ int64_t k_tiled_offset(int64_t r, int64_t c, int64_t K, int64_t rows) {
    const int64_t s = r >> 8, rr = r & 255;
    const int64_t h = rows - (s << 8) < 256 ? rows - (s << 8) : 256;
    const int64_t k = c >> 6, chunk = (c >> 4) & 3, slot = chunk ^ ((rr >> 2) & 3);
    return s * 256 * K + k * h * 64 + rr * 64 + slot * 16 + (c & 15);
}

hipError_t launch_i8_gemm(hipStream_t stream, const GemmParams& p, int cfg);
hipError_t launch_w4a8_gemm(hipStream_t stream, const GemmParams& p, int cfg);
// Whether p's W4 operand (codes p.B, pitch p.ldb, tables p.lut) can be expanded
// into out (K-tiled with kt) by w4_lut_expand_kernel or a prologue's W4Expand.
bool w4_expand_ok(const GemmParams& p, const int8_t* out, bool kt);
// Any K > 0, operands at any byte offset and pitch (the K tail zero-filled).
hipError_t launch_i8_gemm_any(hipStream_t stream, const GemmParams& p, int cfg);
hipError_t launch_i8_gemm_256(hipStream_t stream, const GemmParams& p);
// Persistent kernel (K % 256 == 0): square tiles of 2 * wave_tile (128 -> 256 x 256,
// 64 -> 128 x 128), min(tiles, num_cus) workgroups.  w4: B is packed codes plus
// the per-(row, group) table (group a multiple of 128, code rows 16-byte aligned),
// or signed nibbles with p.w4_signed.
hipError_t launch_i8_gemm_persist(hipStream_t stream, const GemmParams& p, int num_cus, int wave_tile, bool w4);
// One launch of both tile sizes: pb's rows with 256 x 256 tiles, then ps's with
// 128 x 128 tiles (same K, B, sB, bias; the caller offsets A, sA and C).
hipError_t launch_i8_gemm_persist_mixed(hipStream_t stream, const GemmParams& pb, const GemmParams& ps, int num_cus,
                                        bool w4);
// The same contract without W4, on the four-stage 64-deep pipeline
// (i8_gemm_pipe.hip).
hipError_t launch_i8_gemm_pipe(hipStream_t stream, const GemmParams& p, int num_cus, int wave_tile);
hipError_t launch_i8_gemm_pipe_mixed(hipStream_t stream, const GemmParams& pb, const GemmParams& ps, int num_cus);
// Persistent kernel on 272 x 192 tiles (i8_gemm_t272.hip): K-tiled operands,
// row-major ones at 16-byte pitches and addresses, or (b_rm) A K-tiled and B
// row-major; K % 512 == 0, a gate only with fp32 output, rows x pitch below
// 2^31 for both operands (t272_ok).
bool t272_ok(const GemmParams& p);
int t272_tile_count(int64_t M, int64_t N);
hipError_t launch_i8_gemm_t272(hipStream_t stream, const GemmParams& p, int num_cus);
// The same tiles with B as W4 codes (p.B [N, ldb], p.lut, p.group_shift)
// expanded in LDS; K-tiled A, K % 1024 == 0 (t272w4_ok).
bool t272w4_ok(const GemmParams& p);
// Bytes of the band-packed W4 operand of an N x K weight (0 for a shape it
// cannot hold): bands of 192 rows, a 6144-byte code block a band and K-step,
// then a 3072-byte table block a band and group.
int64_t w4_banded_bytes(int64_t N, int64_t K, int64_t group);
// Packs codes [N, crb] (nibbles) and the prepared table lut [N, K / group, 16]
// into that layout (16-byte aligned sources, crb % 16 == 0).
hipError_t launch_w4_pack_banded(hipStream_t stream, const uint8_t* codes, int64_t crb, const int8_t* lut, int N,
                                 int K, int groups, uint8_t* out);
hipError_t launch_i8_gemm_t272w4(hipStream_t stream, const GemmParams& p, int num_cus);
// The W4 operand of p (codes, lut, group_shift, N, K) expanded to int8 [N, K] in out,
// row-major or (kt, K % 64 == 0) in the K-tiled layout.
hipError_t launch_w4_lut_expand(hipStream_t stream, const GemmParams& p, int8_t* out, bool kt = false);

// Element-wise operation applied to every input element before the rotation.
enum QrPreOp { QR_PLAIN = 0, QR_MOD = 1, QR_GELU = 2, QR_SILU_GATE = 3 };
// A 4-bit weight's expansion to int8 (w4_lut_expand_kernel's work) run as
// extra blocks of a plain prologue launch (the tiles kernel), so the
// memory-bound expansion overlaps the VALU-bound rotation.  `on` set by the
// caller after w4_expand_ok(); `blocks` and `nq` set by the launcher.
struct W4Expand {
    int on = 0;
    const uint8_t* codes = nullptr;
    int64_t ldb = 0;
    const int8_t* lut = nullptr;
    int64_t lut_groups = 0;
    int group_shift = 0, w4_signed = 0, kt = 0;
    int64_t N = 0, K = 0;
    int8_t* out = nullptr;
    int blocks = 0;  // expansion blocks in the launch
    int nq = 0;      // prologue blocks in the launch
};

struct QrPre {
    int op;             // QrPreOp
    const float* sc;    // QR_MOD: v = fma(v, 1 + sc[k], sh[k]); either may be NULL (0)
    const float* sh;
    int64_t off2;       // QR_SILU_GATE: v = silu(x[k]) * x[k + off2] (elements)
    W4Expand ex{};      // QR_PLAIN through the tiles kernel only
};
// q_kt: q is written in the K-tiled layout of `rows` rows (ldq unused; K <= 16384).
hipError_t launch_quant_rotate(hipStream_t stream, const void* x, bool bf16_in, int64_t rows,
                               int64_t K, int64_t ldx, int8_t* q, int64_t ldq, float* s,
                               float qmax, int half_even, int rotate, const QrPre& pre, int q_kt = 0);
// An int8 [rows, ld] row-major matrix into the K-tiled layout (16-byte aligned rows).
hipError_t launch_pack_k_tiled(hipStream_t stream, const int8_t* src, int64_t ld, int64_t rows, int64_t K, int8_t* dst);
size_t quant_rotate_lds_bytes(int64_t K);

}  // namespace phi_dev
