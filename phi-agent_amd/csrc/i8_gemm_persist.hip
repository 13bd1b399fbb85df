// Persistent int8 GEMM for gfx950: one workgroup per CU walks 256 x 256
// output tiles, and the next tile's first K-steps are loaded while the
// current tile finishes, so no tile starts on an empty pipeline.
//
//   acc[m,n] = sum_k A[m,k] * B[n,k]                  (exact int32)
//   C[m,n]   = fma((float)acc * sA[m], sB[n], bias[n])  -> bf16 (RNE) / fp32 / raw int32
//
// The product and epilogue are those of the reference's int8_gemm_tc
// (core/kernels/int8_gemm.cpp:466-621, epilogue :588-620) and host gemm_int8
// (core/host/quant.cpp:223-236).
//
// Design:
//   * Four waves (one per SIMD), each 128 x 128 outputs as 4 x 4 blocks of
//     v_mfma_i32_32x32x32_i8 with the 256 accumulators in AGPRs; 128-deep
//     K-steps in two 64 KB LDS stages (A and B 256 rows x 128 bytes each).
//   * Operands go global -> LDS by buffer_load ... lds (no staging
//     registers).  Each tile gets its own buffer resources, so rows past M or
//     N read as zero and need no clamping; lane offsets stay in VGPRs and the
//     per-load row offsets in SGPRs.  A load instruction moves eight whole
//     128-byte rows; chunk c of row r sits in slot c ^ ((r >> 1) & 7), so the
//     operand reads of 16 consecutive rows hit 16 distinct bank windows.
//   * One barrier per K-step, before its last quarter: every wave has then
//     finished with the stage the last quarter's loads overwrite, and the
//     next stage has landed.  Loads, LDS reads and MFMAs are interleaved
//     with sched_group_barrier.
//   * Cross-tile prefetch: the last two K-steps of a tile load the first two
//     of the workgroup's next tile, together with that tile's row scales,
//     column scales and bias (into one of two small LDS areas, by tile
//     parity).  The first MFMA of a tile starts from a zero accumulator.
//   * Epilogue: 32-row strips of the 128 x 128 wave tile are converted,
//     written to a 4 KB per-wave LDS area (swizzled) and read back so every
//     global store writes whole 128-byte rows (16 bytes a lane, 8 lanes a
//     row); stores past row M or column N are dropped by the buffer range
//     check or skipped.
//   * Tile order: workgroup ids are dealt round-robin to the 8 XCDs; each
//     XCD owns a contiguous run of tiles in every round, walked group_m
//     tile-rows at a time, so its concurrent tiles share A and B in its L2.
#include "device_common.hpp"
#include "i8_gemm.hpp"

namespace phi_dev {

namespace {

typedef __attribute__((address_space(3))) void* lptr_t;
typedef unsigned int u32x2 __attribute__((__vector_size__(2 * sizeof(unsigned int))));
typedef unsigned int u32x4 __attribute__((__vector_size__(4 * sizeof(unsigned int))));

// Raw buffer resource word 3 for gfx9-family: 32-bit data format, no swizzle.
constexpr int kRsrcWord3 = 0x00020000;

constexpr int BM = 256, BN = 256, BK = 128;
constexpr int STG = BM * BK;            // 32 KB per operand per stage
constexpr int DL = STG / 1024 / 4;      // 8 loads per operand per wave per K-step
constexpr int EBYTES = 3 * 1024;        // per parity: sa | sb | bias (4 waves x 256 B each)
constexpr int CHUNK = 4096;             // per-wave epilogue staging

constexpr int SG_MFMA = 0x008, SG_DSR = 0x100, SG_VMEM_R = 0x020;

// s_waitcnt vmcnt(0) lgkmcnt(0) (gfx9 encoding; expcnt untouched).
__device__ __forceinline__ void wait_all() { __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (0 << 8)); }
// s_waitcnt vmcnt(N) lgkmcnt(0).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt is six bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | (((N >> 4) & 3) << 14));
}

__device__ __forceinline__ int swz8(int row, int c) { return c ^ ((row >> 1) & 7); }

__device__ __forceinline__ int xcd_remap(int pid, int nblocks) {
    const int xcd = pid & 7, idx = pid >> 3;
    const int base = nblocks >> 3, rem = nblocks & 7;
    return xcd < rem ? xcd * (base + 1) + idx : rem * (base + 1) + (xcd - rem) * base + idx;
}

struct Shape {
    int tiles_m, tiles_n, ntiles, KT, group_m, G;
};

__device__ __forceinline__ void tile_mn(const Shape& s, int logical, int& tm, int& tn) {
    const int per_group = s.group_m * s.tiles_n;
    const int gid = logical / per_group;
    const int first_m = gid * s.group_m;
    const int gsz = min(s.tiles_m - first_m, s.group_m);
    const int in_group = logical - gid * per_group;
    tm = first_m + in_group % gsz;
    tn = in_group / gsz;
}

struct Frag {
    v4i a[4], b[4];
};

// Per-wave state.  The load cursor is the tile whose K-steps are being loaded
// (one ahead of the tile being multiplied near a tile's end).
struct Wv {
    int8_t* la[2];
    int8_t* lb[2];
    int8_t* le[2];
    int8_t* lc;
    __amdgpu_buffer_rsrc_t rA, rB;
    int cm0, cn0, ctile, ckt;
    int voA[2], voB[2];
    int wave, wm, wn, lane, lrow, lhalf;
    int oA[4], oB[4];
};

__device__ __forceinline__ void cursor_set(Wv& w, const GemmParams& p, const Shape& s, int t) {
    w.ctile = t;
    w.ckt = 0;
    int tm, tn;
    tile_mn(s, min(t, s.ntiles - 1), tm, tn);  // past the last tile: harmless reloads
    const int m0 = tm * BM, n0 = tn * BN;
    w.cm0 = m0;
    w.cn0 = n0;
    const int rows = min(BM, p.M - m0), cols = min(BN, p.N - n0);
    w.rA = __builtin_amdgcn_make_buffer_rsrc((void*)(p.A + (int64_t)m0 * p.lda), (short)0, rows * (int)p.lda, kRsrcWord3);
    w.rB = __builtin_amdgcn_make_buffer_rsrc((void*)(p.B + (int64_t)n0 * p.ldb), (short)0, cols * (int)p.ldb, kRsrcWord3);
}

// The cursor's next K-step into stage S: 8 A and 8 B loads per wave.
template <int S>
__device__ __forceinline__ void issue(Wv& w, const GemmParams& p, const Shape& s) {
    const int koff = min(w.ckt, s.KT - 1) * BK;
#pragma unroll
    for (int j = 0; j < DL; j++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(w.rA, (lptr_t)(w.la[S] + w.wave * (DL * 1024) + j * 1024), 16,
                                                 w.voA[j & 1], koff + (w.wave * 64 + j * 8) * (int)p.lda, 0, 0);
#pragma unroll
    for (int j = 0; j < DL; j++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(w.rB, (lptr_t)(w.lb[S] + w.wave * (DL * 1024) + j * 1024), 16,
                                                 w.voB[j & 1], koff + (w.wave * 64 + j * 8) * (int)p.ldb, 0, 0);
    w.ckt++;
}

// Epilogue operands of the cursor's tile into parity area PAR: wave w loads
// row scales 64w..64w+63, column scales / fp32 bias 64w..64w+63 and (waves
// 0-1) the bf16 bias words; past M or N they read as zero.
template <int PAR>
__device__ __forceinline__ void issue_epi(const Wv& w, const GemmParams& p) {
    const int rows = min(BM, p.M - w.cm0), cols = min(BN, p.N - w.cn0);
    const __amdgpu_buffer_rsrc_t rSA =
        __builtin_amdgcn_make_buffer_rsrc((void*)(p.sA ? p.sA + w.cm0 : (const float*)p.A), (short)0,
                                          p.sA ? rows * 4 : 0, kRsrcWord3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rSA, (lptr_t)(w.le[PAR] + w.wave * 256), 4, w.lane * 4, w.wave * 256, 0, 0);
    const bool sbs = p.sb_scalar != 0;
    const __amdgpu_buffer_rsrc_t rSB = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.sB ? (sbs ? p.sB : p.sB + w.cn0) : (const float*)p.A), (short)0, p.sB ? (sbs ? 4 : cols * 4) : 0,
        kRsrcWord3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rSB, (lptr_t)(w.le[PAR] + 1024 + w.wave * 256), 4, sbs ? 0 : w.lane * 4,
                                             sbs ? 0 : w.wave * 256, 0, 0);
    const int bsz = p.bias_kind == BIAS_F32 ? 4 : 2;
    const __amdgpu_buffer_rsrc_t rBZ = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.bias_kind != BIAS_NONE ? (const int8_t*)p.bias + (int64_t)w.cn0 * bsz : (const int8_t*)p.A), (short)0,
        p.bias_kind != BIAS_NONE ? cols * bsz : 0, kRsrcWord3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rBZ, (lptr_t)(w.le[PAR] + 2048 + w.wave * 256), 4, w.lane * 4,
                                             w.wave * 256, 0, 0);
}

template <int S, int Q>
__device__ __forceinline__ void frag(Frag& f, const Wv& w) {
    const int8_t* cA = w.la[S] + w.oA[Q];
    const int8_t* cB = w.lb[S] + w.oB[Q];
#pragma unroll
    for (int i = 0; i < 4; i++) f.a[i] = *(const v4i*)(cA + i * 32 * BK);
#pragma unroll
    for (int j = 0; j < 4; j++) f.b[j] = *(const v4i*)(cB + j * 32 * BK);
}

template <bool ZERO>
__device__ __forceinline__ void mma16(const Frag& f, v16i (&acc)[4][4]) {
#pragma unroll
    for (int q = 0; q < 16; q++) {
        const int j = q / 4, i = q % 4;
        if constexpr (ZERO) {
            const v16i z = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
            acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.b[j], f.a[i], z, 0, 0, 0);
        } else {
            acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.b[j], f.a[i], acc[j][i], 0, 0, 0);
        }
    }
}

// A quarter K-step: 16 MFMAs on cur, the eight fragment reads of quarter QN
// of stage SN into nxt; with LOADS the cursor's next K-step into stage S
// (EPI: plus the epilogue operands into parity PARE).  The first MFMA goes
// ahead of the reads because the compiler's wait for cur is a full
// lgkmcnt(0) that must not cover reads issued after it.
template <int S, int SN, int QN, bool ZERO, bool LOADS, bool EPI, int PARE>
__device__ __forceinline__ void quarter(const Frag& cur, Frag& nxt, v16i (&acc)[4][4], Wv& w, const GemmParams& p,
                                        const Shape& s) {
    mma16<ZERO>(cur, acc);
    if constexpr (LOADS) {
        issue<S>(w, p, s);
        if constexpr (EPI) issue_epi<PARE>(w, p);
    }
    frag<SN, QN>(nxt, w);
    __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
    if constexpr (LOADS) {
#pragma unroll
        for (int t = 0; t < 8; t++) {
            __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
            __builtin_amdgcn_sched_group_barrier(SG_VMEM_R, 1, 0);
            __builtin_amdgcn_sched_group_barrier(SG_DSR, 1, 0);
            __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
            __builtin_amdgcn_sched_group_barrier(SG_VMEM_R, 1, 0);
        }
    } else {
#pragma unroll
        for (int t = 0; t < 8; t++) {
            __builtin_amdgcn_sched_group_barrier(SG_DSR, 1, 0);
            __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 7, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
}

// One K-step on stage S.  With two stages the wait before the barrier covers
// every load in flight: the next stage's (issued one K-step earlier).
template <int S, bool Z, bool EPI, int PARE>
__device__ __forceinline__ void step(Frag& f0, v16i (&acc)[4][4], Wv& w, const GemmParams& p, const Shape& s) {
    Frag f1;
    quarter<S, S, 1, Z, false, false, 0>(f0, f1, acc, w, p, s);
    quarter<S, S, 2, false, false, false, 0>(f1, f0, acc, w, p, s);
    quarter<S, S, 3, false, false, false, 0>(f0, f1, acc, w, p, s);
    wait_all();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    quarter<S, S ^ 1, 0, false, true, EPI, PARE>(f1, f0, acc, w, p, s);
}

// The K-loop of one tile (operands in parity PAR): K-steps 0..KT-1, the last
// two loading the next tile's first two.  Needs KT even and >= 4.
template <int PAR>
__device__ __forceinline__ void tile_body(Frag& f0, v16i (&acc)[4][4], Wv& w, const GemmParams& p, const Shape& s) {
    step<0, true, false, 0>(f0, acc, w, p, s);
    step<1, false, false, 0>(f0, acc, w, p, s);
    for (int kt = 2; kt < s.KT - 2; kt += 2) {
        step<0, false, false, 0>(f0, acc, w, p, s);
        step<1, false, false, 0>(f0, acc, w, p, s);
    }
    cursor_set(w, p, s, w.ctile + s.G);  // every load of this tile is issued
    step<0, false, true, PAR ^ 1>(f0, acc, w, p, s);
    step<1, false, false, 0>(f0, acc, w, p, s);
}

// Scaled epilogue operands of this lane's four columns of group g in block j.
__device__ __forceinline__ void col_operands(const GemmParams& p, const int8_t* e, int ct, v4f& sb, v4f& bz) {
    if (p.sb_scalar) {
        const float v = *(const float*)(e + 1024);
        sb = v4f{v, v, v, v};
    } else {
        sb = *(const v4f*)(e + 1024 + ct * 4);
    }
    if (p.bias_kind == BIAS_F32) {
        bz = *(const v4f*)(e + 2048 + ct * 4);
    } else if (p.bias_kind == BIAS_BF16) {
        const uint2 h = *(const uint2*)(e + 2048 + ct * 2);
        bz = v4f{bf16_to_f32(h.x & 0xffffu), bf16_to_f32(h.x >> 16), bf16_to_f32(h.y & 0xffffu), bf16_to_f32(h.y >> 16)};
    } else {
        bz = v4f{0.f, 0.f, 0.f, 0.f};
    }
}

// Epilogue of tile t (operands in parity PAR).  Lane l holds row l % 32 of
// each A block and, in registers 4g..4g+3, columns 8g + 4(l/32) + 0..3 of each
// B block.  Each 32-row strip goes through the wave's LDS area (16-byte slots
// swizzled by row) and is stored as whole rows: bf16 in 32 x 64-column
// pieces (128 bytes a row), fp32 / int32 in 32 x 32-column pieces.
template <int PAR>
__device__ __forceinline__ void epilogue(v16i (&acc)[4][4], const GemmParams& p, const Shape& s, int t, const Wv& w) {
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) asm volatile("" : "+a"(acc[j][i]));
    int tm, tn;
    tile_mn(s, t, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int rows = min(BM, p.M - m0);
    const int esz = p.c_kind == C_BF16 ? 2 : 4;
    const int pitch = (int)p.ldc * esz;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (int8_t*)p.C + (int64_t)m0 * pitch, (short)0, rows * pitch, kRsrcWord3);
    const int8_t* e = w.le[PAR];
    int8_t* lc = w.lc;
    const int colw = n0 + w.wn * 128;  // first column of this wave
    float sa[4];
#pragma unroll
    for (int i = 0; i < 4; i++) sa[i] = *(const float*)(e + (w.wm * 128 + i * 32 + w.lrow) * 4);
    if (p.c_kind == C_BF16) {
#pragma unroll
        for (int jp = 0; jp < 2; jp++) {
            v4f sb[2][4], bz[2][4];
#pragma unroll
            for (int jj = 0; jj < 2; jj++)
#pragma unroll
                for (int g = 0; g < 4; g++)
                    col_operands(p, e, w.wn * 128 + (2 * jp + jj) * 32 + 8 * g + 4 * w.lhalf, sb[jj][g], bz[jj][g]);
#pragma unroll
            for (int i = 0; i < 4; i++) {
#pragma unroll
                for (int jj = 0; jj < 2; jj++) {
                    v16i blk = acc[2 * jp + jj][i];
                    asm volatile("" : "+v"(blk));
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        float v[4];
#pragma unroll
                        for (int q = 0; q < 4; q++)
                            v[q] = fmaf((float)blk[4 * g + q] * sa[i], sb[jj][g][q], bz[jj][g][q]);
                        const int slot = (jj * 4 + g) ^ (w.lrow & 7);
                        *(u32x2*)(lc + w.lrow * 128 + slot * 16 + w.lhalf * 8) =
                            u32x2{f32x2_to_bf16x2(v[0], v[1]), f32x2_to_bf16x2(v[2], v[3])};
                    }
                }
                // A wave's LDS accesses complete in order: these reads see its writes.
#pragma unroll
                for (int tt = 0; tt < 4; tt++) {
                    const int r = tt * 8 + (w.lane >> 3), sl = w.lane & 7;
                    const u32x4 v = *(const u32x4*)(lc + r * 128 + ((sl ^ (r & 7)) * 16));
                    const int col = colw + jp * 64 + sl * 8;
                    if (col < p.N)
                        __builtin_amdgcn_raw_buffer_store_b128(v, rs, (w.wm * 128 + i * 32 + r) * pitch + col * 2, 0, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        return;
    }
    // fp32 / int32: 32 x 32 pieces, one block at a time.
#pragma unroll
    for (int j = 0; j < 4; j++) {
        v4f sb[4], bz[4];
        if (p.c_kind == C_F32) {
#pragma unroll
            for (int g = 0; g < 4; g++) col_operands(p, e, w.wn * 128 + j * 32 + 8 * g + 4 * w.lhalf, sb[g], bz[g]);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v16i blk = acc[j][i];
            asm volatile("" : "+v"(blk));
#pragma unroll
            for (int g = 0; g < 4; g++) {
                u32x4 o;
                if (p.c_kind == C_F32) {
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        o[q] = __float_as_uint(fmaf((float)blk[4 * g + q] * sa[i], sb[g][q], bz[g][q]));
                } else {
#pragma unroll
                    for (int q = 0; q < 4; q++) o[q] = (unsigned)blk[4 * g + q];
                }
                const int slot = (2 * g + w.lhalf) ^ (w.lrow & 7);
                *(u32x4*)(lc + w.lrow * 128 + slot * 16) = o;
            }
#pragma unroll
            for (int tt = 0; tt < 4; tt++) {
                const int r = tt * 8 + (w.lane >> 3), sl = w.lane & 7;
                const u32x4 v = *(const u32x4*)(lc + r * 128 + ((sl ^ (r & 7)) * 16));
                const int col = colw + j * 32 + sl * 4;
                if (col < p.N)
                    __builtin_amdgcn_raw_buffer_store_b128(v, rs, (w.wm * 128 + i * 32 + r) * pitch + col * 4, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

}  // namespace

__global__ __launch_bounds__(256) void i8_gemm_persist_kernel(GemmParams p) {
    __shared__ __align__(16) int8_t a0[STG], a1[STG], b0[STG], b1[STG];
    __shared__ __align__(16) int8_t e0[EBYTES], e1[EBYTES];
    __shared__ __align__(16) int8_t cbuf[4 * CHUNK];
    Wv w;
    w.lane = threadIdx.x & 63;
    w.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    w.wm = w.wave >> 1;
    w.wn = w.wave & 1;
    w.lrow = w.lane & 31;
    w.lhalf = w.lane >> 5;
    Shape s;
    s.tiles_m = (p.M + BM - 1) / BM;
    s.tiles_n = (p.N + BN - 1) / BN;
    s.ntiles = s.tiles_m * s.tiles_n;
    s.KT = p.K / BK;
    s.group_m = p.group_m;
    s.G = gridDim.x;
    int t = xcd_remap(blockIdx.x, s.G);
    if (t >= s.ntiles) return;
    w.la[0] = a0;
    w.la[1] = a1;
    w.lb[0] = b0;
    w.lb[1] = b1;
    w.le[0] = e0;
    w.le[1] = e1;
    w.lc = cbuf + w.wave * CHUNK;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        w.oA[q] = (w.wm * 128 + w.lrow) * BK + swz8(w.lrow, 2 * q + w.lhalf) * 16;
        w.oB[q] = (w.wn * 128 + w.lrow) * BK + swz8(w.lrow, 2 * q + w.lhalf) * 16;
    }
    // A load instruction covers 8 rows; lane l fetches row l/8 and the chunk
    // whose swizzled slot is l % 8 (the swizzle depends on the row's parity
    // within the load's 16-row pair).
#pragma unroll
    for (int par = 0; par < 2; par++) {
        const int r = par * 8 + (w.lane >> 3);
        w.voA[par] = (w.lane >> 3) * (int)p.lda + swz8(r, w.lane & 7) * 16;
        w.voB[par] = (w.lane >> 3) * (int)p.ldb + swz8(r, w.lane & 7) * 16;
    }
    cursor_set(w, p, s, t);
    issue<0>(w, p, s);
    issue_epi<0>(w, p);
    issue<1>(w, p, s);
    wait_vm_lgkm0<2 * DL>();  // the first K-step (and the operands) have landed
    __builtin_amdgcn_s_barrier();
    Frag f0;
    frag<0, 0>(f0, w);
    v16i acc[4][4];
    tile_body<0>(f0, acc, w, p, s);
    for (;;) {
        epilogue<0>(acc, p, s, t, w);
        const int t1 = t + s.G;
        if (t1 >= s.ntiles) break;
        tile_body<1>(f0, acc, w, p, s);
        epilogue<1>(acc, p, s, t1, w);
        t = t1 + s.G;
        if (t >= s.ntiles) break;
        tile_body<0>(f0, acc, w, p, s);
    }
    // The reloads past the last tile still write LDS: let them land.
    wait_all();
}

hipError_t launch_i8_gemm_persist(hipStream_t stream, const GemmParams& p, int num_cus) {
    if (p.K % 256 != 0 || p.K < 512) return hipErrorInvalidValue;
    const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
    const int grid = tiles < num_cus ? tiles : num_cus;
    hipLaunchKernelGGL(i8_gemm_persist_kernel, dim3(grid), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace phi_dev
