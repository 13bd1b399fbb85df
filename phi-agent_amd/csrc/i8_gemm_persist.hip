// Persistent int8 GEMM for gfx950, two-stage form: one workgroup per CU walks
// square output tiles (256 x 256, or 128 x 128 for the rows a whole number of
// 256-row rounds does not cover), and the next tile's first K-steps are
// loaded while the current tile finishes, so no tile starts on an empty
// pipeline.  It runs B as packed 4-bit codes expanded in registers (W4A8 and
// int4); int8 B runs on the four-stage pipeline of i8_gemm_pipe.hip, with
// this kernel as its A/B counterpart.
//
//   acc[m,n] = sum_k A[m,k] * B[n,k]                  (exact int32)
//   C[m,n]   = fma((float)acc * sA[m], sB[n], bias[n])  -> bf16 (RNE) / fp32 / raw int32
//
// The product and epilogue are those of the reference's int8_gemm_tc
// (core/kernels/int8_gemm.cpp:466-621, epilogue :588-620) and host gemm_int8
// (core/host/quant.cpp:223-236).
//
// Design (WT = wave tile, 128 or 64; the workgroup tile is 2WT x 2WT):
//   * Four waves (one per SIMD), each WT x WT outputs as NB x NB blocks of
//     v_mfma_i32_32x32x32_i8 (NB = WT/32) with the accumulators in AGPRs;
//     128-deep K-steps in two LDS stages (A and B 2WT rows x 128 bytes each).
//   * Operands go global -> LDS by buffer_load ... lds (no staging
//     registers).  Each tile gets its own buffer resources, so rows past M or
//     N read as zero and need no clamping.  A load instruction moves eight
//     whole 128-byte rows; chunk c of row r sits in slot c ^ ((r >> 1) & 7),
//     so the operand reads of 16 consecutive rows hit 16 distinct bank
//     windows.
//   * One barrier per K-step, before its last quarter: every wave has then
//     finished with the stage the last quarter's loads overwrite, and the
//     next stage has landed.  Loads, LDS reads and MFMAs are interleaved
//     with sched_group_barrier.
//   * Cross-tile prefetch: the last K-step pair of a tile loads the first
//     pair of the workgroup's next tile, together with that tile's row
//     scales, column scales and bias (into one of two small LDS areas, by
//     tile parity).
//   * Epilogue: 32-row strips of the wave tile are converted, written to a
//     4 KB per-wave LDS area (swizzled) and read back so every global store
//     writes whole 128-byte rows (16 bytes a lane, 8 lanes a row); stores
//     past row M or column N are dropped by the buffer range check or
//     skipped.  Output stores are non-temporal.
//   * Tile order: workgroup ids are dealt round-robin to the 8 XCDs; each
//     XCD owns a contiguous run of tiles in every round, walked group_m
//     tile-rows at a time, so its concurrent tiles share A and B in its L2.
#include "device_common.hpp"
#include "i8_gemm.hpp"
#include "persist_common.hpp"

namespace phi_dev {

namespace {

using namespace persist;

constexpr int BK = 128;
#ifndef W4_Q1
#define W4_Q1 1
#endif

template <int WT>
struct Cfg {
    static constexpr int NB = WT / 32;         // MFMA blocks per wave dimension
    static constexpr int BM = 2 * WT;          // workgroup tile (square)
    static constexpr int STG = BM * BK;        // bytes per operand per stage
    static constexpr int DL = STG / 1024 / 4;  // loads per operand per wave per K-step
};

__device__ __forceinline__ int swz8(int row, int c) { return c ^ ((row >> 1) & 7); }

template <int WT>
struct Frag {
    v4i a[Cfg<WT>::NB], b[Cfg<WT>::NB];
};

// W4 operand: B is packed 4-bit codes (low nibble = even column) with a
// per-(row, group) 16-entry int8 table.  Each thread owns BM/256 of a B row
// per K-step: it loads that row's codes (64 bytes for a 256-row tile, 32 for
// 128) and the row's table for the K-step's group into registers one K-step
// ahead, and expands them into the int8 B stage between the next step's
// MFMAs, so the MFMA core is unchanged.
template <int WT>
struct W4Regs {
    static constexpr int C = Cfg<WT>::BM / 64;  // 16-byte code loads per thread per K-step
    u32x4 c[C];
    u32x4 t;
};

// Per-wave state.  The load cursor is the tile whose K-steps are being
// loaded: it moves to the workgroup's next tile during a tile's last K-step
// pair; after the last tile it reloads that tile's last pair (harmless).
struct Wv : EpiWave {
    int8_t* la[2];
    int8_t* lb[2];
    int8_t* le;                     // two epilogue-operand areas, one per tile parity
    __amdgpu_buffer_rsrc_t rA, rB;  // the load cursor's tile (W4: rB over the codes)
    __amdgpu_buffer_rsrc_t rL;      // W4: the cursor's tile's table rows
    int voA[2], voB[2];
    int w4row, w4half, vo4, voL;    // W4: this thread's B row, half, code and table offsets
    int oA[4], oB[4];
};

// Points the load cursor at logical tile t.
template <int WT, bool W4>
__device__ __forceinline__ void cursor_tile(Wv& w, const GemmParams& p, const Shape& s, int t) {
    constexpr int BM = Cfg<WT>::BM;
    int tm, tn;
    tile_mn(s, t, tm, tn);
    const int m0 = tm * BM, n0 = tn * BM;
    w.cm0 = m0;
    w.cn0 = n0;
    const int rows = min(BM, p.M - m0), cols = min(BM, p.N - n0);
    w.rA = __builtin_amdgcn_make_buffer_rsrc((void*)(p.A + (int64_t)m0 * p.lda), (short)0, rows * (int)p.lda, kRsrcWord3);
    w.rB = __builtin_amdgcn_make_buffer_rsrc((void*)(p.B + (int64_t)n0 * p.ldb), (short)0, cols * (int)p.ldb, kRsrcWord3);
    if constexpr (W4) {
        if (!p.w4_signed) {
            const int lrow = (int)p.lut_groups * 16;
            w.rL = __builtin_amdgcn_make_buffer_rsrc((void*)(p.lut + (int64_t)n0 * lrow), (short)0, cols * lrow,
                                                     kRsrcWord3);
        }
    }
}

// K-step kl of the cursor's tile into stage S: DL A loads per wave and DL B
// loads (W4: the thread's codes and table into r instead), with EPI plus the
// tile's epilogue operands into area le.
template <int WT, int S, bool EPI, bool W4, bool G>
__device__ __forceinline__ void issue(const Wv& w, const GemmParams& p, int kl, int8_t* le, W4Regs<WT>& r) {
    constexpr int DL = Cfg<WT>::DL;
    const int koff = kl * BK;
    // The LDS destinations (M0) come from bases made opaque here, one scalar
    // add per load: hoisted out of the loop, the 2 x 2 DL destinations would
    // hold as many SGPRs through it.
    int8_t* dA = opaque_lds(w.la[S] + w.wave * (DL * 1024));
#pragma unroll
    for (int j = 0; j < DL; j++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(w.rA, (lptr_t)(dA + j * 1024), 16, w.voA[j & 1],
                                                 koff + (w.wave * DL * 8 + j * 8) * (int)p.lda, 0, 0);
    if constexpr (W4) {
#pragma unroll
        for (int q = 0; q < W4Regs<WT>::C; q++)
            r.c[q] = __builtin_amdgcn_raw_buffer_load_b128(w.rB, w.vo4 + q * 16, kl * (BK / 2), 0);
        r.t = p.w4_signed ? signed_nibble_table()
                          : __builtin_amdgcn_raw_buffer_load_b128(w.rL, w.voL, ((kl * BK) >> p.group_shift) * 16, 0);
    } else {
        int8_t* dB = opaque_lds(w.lb[S] + w.wave * (DL * 1024));
#pragma unroll
        for (int j = 0; j < DL; j++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(w.rB, (lptr_t)(dB + j * 1024), 16, w.voB[j & 1],
                                                     koff + (w.wave * DL * 8 + j * 8) * (int)p.ldb, 0, 0);
    }
    if constexpr (EPI) issue_epi<WT, G>(w, p, le);
}

// W4: chunks [P0, P1) of the thread's 2C 16-column chunks of one K-step,
// expanded from r into the int8 B stage S at their swizzled slots.
template <int WT, int S, int P0, int P1>
__device__ __forceinline__ void expand(const W4Regs<WT>& r, const Wv& w) {
    constexpr int C = W4Regs<WT>::C;
    int8_t* dst = w.lb[S] + w.w4row * BK;
#pragma unroll
    for (int x = P0; x < P1; x++) {
        const int q = x / 2, h = x % 2;
        const int c = w.w4half * 2 * C + x;
        *(v4i*)(dst + swz8(w.w4row, c) * 16) = expand16b(r.c[q][2 * h], r.c[q][2 * h + 1], r.t);
    }
}

template <int WT, int S, int Q>
__device__ __forceinline__ void frag(Frag<WT>& f, const Wv& w) {
    constexpr int NB = Cfg<WT>::NB;
    const int8_t* cA = w.la[S] + w.oA[Q];
    const int8_t* cB = w.lb[S] + w.oB[Q];
#pragma unroll
    for (int i = 0; i < NB; i++) f.a[i] = *(const v4i*)(cA + i * 32 * BK);
#pragma unroll
    for (int j = 0; j < NB; j++) f.b[j] = *(const v4i*)(cB + j * 32 * BK);
}

template <int WT>
__device__ __forceinline__ void zero_acc(v16i (&acc)[Cfg<WT>::NB][Cfg<WT>::NB]) {
    constexpr int NB = Cfg<WT>::NB;
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
        for (int i = 0; i < NB; i++) acc[j][i] = v16i{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
}

// MFMAs Q0 .. Q1-1 of the NB x NB block (column block j = q / NB outer).
// Z: the tile's first MFMAs, which start the accumulators from an inline 0
// instead of reading them (no zeroing of 16 NB^2 AGPRs per tile).
template <int WT, int Q0 = 0, int Q1 = Cfg<WT>::NB * Cfg<WT>::NB, bool Z = false>
__device__ __forceinline__ void mma(const Frag<WT>& f, v16i (&acc)[Cfg<WT>::NB][Cfg<WT>::NB]) {
    constexpr int NB = Cfg<WT>::NB;
#pragma unroll
    for (int q = Q0; q < Q1; q++) {
        const int j = q / NB, i = q % NB;
        if constexpr (Z)
            acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.b[j], f.a[i], v16i{}, 0, 0, 0);
        else
            acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.b[j], f.a[i], acc[j][i], 0, 0, 0);
    }
}

// A quarter K-step: NB^2 MFMAs on cur, the 2 NB fragment reads of quarter QN
// of stage SN into nxt; with LOADS the cursor's K-step into stage S.  The
// first MFMA goes ahead of the reads because the compiler's wait for cur is
// a full lgkmcnt(0) that must not cover reads issued after it.
template <int WT, int S, int SN, int QN, bool LOADS, bool EPI, bool W4, bool G, int X0, int X1, bool Z = false>
__device__ __forceinline__ void quarter(const Frag<WT>& cur, Frag<WT>& nxt, v16i (&acc)[Cfg<WT>::NB][Cfg<WT>::NB],
                                        const Wv& w, const GemmParams& p, int kl, int8_t* le, W4Regs<WT>& r) {
    constexpr int NB = Cfg<WT>::NB, DL = Cfg<WT>::DL;
    mma<WT, 0, 1, Z>(cur, acc);
    if constexpr (LOADS) issue<WT, S, EPI, W4, G>(w, p, kl, le, r);
    frag<WT, SN, QN>(nxt, w);
    mma<WT, 1, NB * NB, Z>(cur, acc);
    if constexpr (X1 > X0) {
        // Chunks [X0, X1) of the previous step's codes into the other stage,
        // spread between the MFMAs (about 38 VALU ops and one LDS write each).
        expand<WT, S ^ 1, X0, X1>(r, w);
        constexpr int V = (38 * (X1 - X0) + NB * NB - 1) / (NB * NB);
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
#pragma unroll
        for (int t = 0; t < NB * NB; t++) {
            __builtin_amdgcn_sched_group_barrier(SG_DSR, 1, 0);
            __builtin_amdgcn_sched_group_barrier(SG_VALU, V, 0);
            __builtin_amdgcn_sched_group_barrier(SG_DSW, 1, 0);
            __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        return;
    }
    __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
    if constexpr (LOADS) {
        // Between the remaining MFMAs: the 2 DL loads and the 2 NB reads.
#pragma unroll
        for (int t = 0; t < 2 * NB; t++) {
            __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
            __builtin_amdgcn_sched_group_barrier(SG_VMEM_R, DL / NB / 2, 0);
            __builtin_amdgcn_sched_group_barrier(SG_DSR, 1, 0);
            if constexpr (NB / 2 > 1) __builtin_amdgcn_sched_group_barrier(SG_MFMA, NB / 2 - 1, 0);
            __builtin_amdgcn_sched_group_barrier(SG_VMEM_R, DL / NB / 2, 0);
        }
    } else {
#pragma unroll
        for (int t = 0; t < 2 * NB; t++) {
            __builtin_amdgcn_sched_group_barrier(SG_DSR, 1, 0);
            __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
        }
        if constexpr (NB * NB - 1 - 2 * NB > 0) __builtin_amdgcn_sched_group_barrier(SG_MFMA, NB * NB - 1 - 2 * NB, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
}

// One K-step on stage S.  With two stages the wait before the barrier covers
// every load in flight: the next stage's (issued one K-step earlier).  After
// the barrier every wave is done reading stage S, which the last quarter
// refills with K-step kl of the cursor's tile (EPI: epilogue operands into le).
// W4: the codes loaded by the previous step are expanded into stage S^1 over
// quarters 1-3, before the barrier that hands that stage to the next step.
// Z: the tile's first K-step (its first quarter starts the accumulators).
// VW: memory operations the wait before the barrier may leave in flight
// (the first K-step after an epilogue: that epilogue's stores, issued after
// the loads it waits for; memory operations complete in issue order).
template <int WT, int S, bool EPI, bool W4, bool G, bool Z = false, int VW = 0>
__device__ __forceinline__ void step(Frag<WT>& f0, v16i (&acc)[Cfg<WT>::NB][Cfg<WT>::NB], const Wv& w,
                                     const GemmParams& p, int kl, int8_t* le, W4Regs<WT>& r) {
    constexpr int X = W4 ? 2 * W4Regs<WT>::C : 0;  // chunks to expand, over quarters 1-3
    Frag<WT> f1;
    quarter<WT, S, S, 1, false, false, W4, G, 0, W4_Q1 * X / 3, Z>(f0, f1, acc, w, p, kl, le, r);
    quarter<WT, S, S, 2, false, false, W4, G, W4_Q1 * X / 3, W4_Q1 ? 2 * X / 3 : X / 2>(f1, f0, acc, w, p, kl, le, r);
    quarter<WT, S, S, 3, false, false, W4, G, W4_Q1 ? 2 * X / 3 : X / 2, X>(f0, f1, acc, w, p, kl, le, r);
    if constexpr (VW == 0) wait_all();
    else wait_vm_lgkm0<VW>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    quarter<WT, S, S ^ 1, 0, true, EPI, W4, G, 0, 0>(f1, f0, acc, w, p, kl, le, r);
}

}  // namespace

// The persistent loop over this workgroup's tiles of p, on LDS stages
// a0/a1/b0/b1 (STG bytes each), the epilogue-operand areas eall and the
// epilogue staging cbuf.  Returns at once when the workgroup has no tile.
template <int WT, bool W4, bool G>
__device__ __forceinline__ void persist_tiles(const GemmParams& p, int8_t* a0, int8_t* a1, int8_t* b0, int8_t* b1,
                                              int8_t* eall, int8_t* cbuf) {
    using C = Cfg<WT>;
    constexpr int NB = C::NB, DL = C::DL;
    Wv w;
    w.lane = threadIdx.x & 63;
    w.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & 3;  // bounded, so LDS offsets fold
    w.wm = w.wave >> 1;
    w.wn = w.wave & 1;
    w.lrow = w.lane & 31;
    w.lhalf = w.lane >> 5;
    Shape s;
    s.tiles_m = (p.M + C::BM - 1) / C::BM;
    s.tiles_n = (p.N + C::BM - 1) / C::BM;
    s.ntiles = s.tiles_m * s.tiles_n;
    s.KT = p.K / BK;
    s.group_m = p.group_m;
    s.G = gridDim.x;
    init_div(s);
    // Tiles r, r + G, ... of this workgroup (r after the XCD remap).
    const int r = xcd_remap(blockIdx.x, s.G);
    if (r >= s.ntiles) return;
    const int ntile = (s.ntiles - r - 1) / s.G + 1;
    w.la[0] = a0;
    w.la[1] = a1;
    w.lb[0] = opaque_lds(b0);
    w.lb[1] = w.lb[0] + (b1 - b0);
    w.le = eall;
    w.lc = cbuf + w.wave * CHUNK;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        w.oA[q] = (w.wm * WT + w.lrow) * BK + swz8(w.lrow, 2 * q + w.lhalf) * 16;
        w.oB[q] = (w.wn * WT + w.lrow) * BK + swz8(w.lrow, 2 * q + w.lhalf) * 16;
    }
    // A load instruction covers 8 rows; lane l fetches row l/8 and the chunk
    // whose swizzled slot is l % 8 (the swizzle depends on the row's parity
    // within the load's 16-row pair).
#pragma unroll
    for (int par = 0; par < 2; par++) {
        const int rr = par * 8 + (w.lane >> 3);
        w.voA[par] = (w.lane >> 3) * (int)p.lda + swz8(rr, w.lane & 7) * 16;
        w.voB[par] = (w.lane >> 3) * (int)p.ldb + swz8(rr, w.lane & 7) * 16;
    }
    if constexpr (W4) {
        constexpr int TPR = 256 / C::BM;  // threads per B row
        w.w4row = threadIdx.x / TPR;
        w.w4half = threadIdx.x % TPR;
        w.vo4 = w.w4row * (int)p.ldb + w.w4half * (BK / 2 / TPR);
        w.voL = w.w4row * (int)p.lut_groups * 16;
    }
    // The epilogue operands of the workgroup's i-th tile go to area i % 2,
    // loaded with its first K-step (during tile i-1's last pair), so at
    // least one barrier separates a tile's epilogue from the load into its
    // area for tile i+2.
    W4Regs<WT> w4r;
    cursor_tile<WT, W4>(w, p, s, r);
    issue<WT, 0, true, W4, G>(w, p, 0, w.le, w4r);
    if constexpr (W4) {
        wait_all();
        expand<WT, 0, 0, 2 * W4Regs<WT>::C>(w4r, w);
        issue<WT, 1, false, W4, G>(w, p, 1, w.le, w4r);
        wait_vm_lgkm0<DL + W4Regs<WT>::C + 1>();  // stage 0, its operands and its expansion are done
    } else {
        issue<WT, 1, false, W4, G>(w, p, 1, w.le, w4r);
        wait_vm_lgkm0<2 * DL>();  // the first K-step and its operands have landed
    }
    __builtin_amdgcn_s_barrier();
    Frag<WT> f0;
    frag<WT, 0, 0>(f0, w);
    v16i acc[NB][NB];
    for (int i = 0;;) {
        const int t = r + i * s.G;
        int8_t* le = w.le + (i & 1) * EBYTES;
        if (s.KT > 2) {
            // The first pair.  After an epilogue, its first wait leaves that
            // epilogue's stores in flight: 2 NB^2 a wave on the bf16 path, the
            // fewest of any output path (every store is issued, none skipped).
            if (i > 0) step<WT, 0, false, W4, G, true, 2 * NB * NB>(f0, acc, w, p, 2, le, w4r);
            else step<WT, 0, false, W4, G, true>(f0, acc, w, p, 2, le, w4r);
            step<WT, 1, false, W4, G>(f0, acc, w, p, 3, le, w4r);
        } else {
            zero_acc<WT>(acc);
        }
        for (int k = 2; k < s.KT - 2; k += 2) {
            step<WT, 0, false, W4, G>(f0, acc, w, p, k + 2, le, w4r);
            step<WT, 1, false, W4, G>(f0, acc, w, p, k + 3, le, w4r);
        }
        // The last pair: the cursor moves to the next tile, if any.
        int kn = s.KT - 2;
        int8_t* ln = le;
        if (i + 1 < ntile) {
            cursor_tile<WT, W4>(w, p, s, t + s.G);
            kn = 0;
            ln = w.le + ((i + 1) & 1) * EBYTES;
        }
        step<WT, 0, true, W4, G>(f0, acc, w, p, kn, ln, w4r);
        step<WT, 1, false, W4, G>(f0, acc, w, p, kn + 1, ln, w4r);
        {
            int tm, tn;
            tile_mn(s, t, tm, tn);
            epilogue<WT, G>(acc, p, tm * C::BM, tn * C::BM, w, le);
        }
        if (++i == ntile) break;
    }
    // The reloads past the last K-step still write LDS: let them land.
    wait_all();
}

template <int WT, bool W4, bool G>
__global__ __launch_bounds__(256) void i8_gemm_persist_kernel(GemmParams p) {
    constexpr int STG = Cfg<WT>::STG;
    __shared__ __align__(16) int8_t a0[STG], a1[STG], b0[STG], b1[STG];
    __shared__ __align__(16) int8_t eall[2 * EBYTES];
    __shared__ __align__(16) int8_t cbuf[4 * CHUNK];
    persist_tiles<WT, W4, G>(p, a0, a1, b0, b1, eall, cbuf);
}

// Both tile sizes in one launch: the workgroup's 256 x 256 tiles of pb, then
// its 128 x 128 tiles of ps (the rows below pb's), in the same LDS.  One
// launch instead of two saves a kernel boundary (about 6 us between dependent
// launches on one stream), and a workgroup starts its small tile as soon as
// its big ones are done.
template <bool W4, bool G>
__global__ __launch_bounds__(256) void i8_gemm_persist_mixed_kernel(GemmParams pb, GemmParams ps) {
    constexpr int STG = Cfg<128>::STG, STG2 = Cfg<64>::STG;
    static_assert(2 * STG2 <= STG, "the small tiles' stages fit in the big tiles' ones");
    __shared__ __align__(16) int8_t a0[STG], a1[STG], b0[STG], b1[STG];
    __shared__ __align__(16) int8_t eall[2 * EBYTES];
    __shared__ __align__(16) int8_t cbuf[4 * CHUNK];
    persist_tiles<128, W4, G>(pb, a0, a1, b0, b1, eall, cbuf);
    __syncthreads();  // every wave is done with the big tiles' LDS
    persist_tiles<64, W4, G>(ps, a0, a1, b0, b1, eall, cbuf);
}

// The W4 operand expanded once into an int8 [N, K] buffer (out, row pitch K):
// each thread turns 32 consecutive codes of one row (16 bytes, one table
// since group % 32 == 0) into 32 int8, the same bytes the in-register path
// writes to LDS.
__global__ __launch_bounds__(256) void w4_lut_expand_kernel(const uint8_t* __restrict__ codes, int64_t ldb,
                                                            const int8_t* __restrict__ lut, int64_t lut_groups,
                                                            int group_shift, int w4_signed, int64_t N, int64_t K,
                                                            int kt, int8_t* __restrict__ out) {
    const int64_t per_row = K / 32;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= N * per_row) return;
    const int64_t row = idx / per_row, c32 = idx - row * per_row;
    const u32x4 c = *(const u32x4*)(codes + row * ldb + c32 * 16);
    const u32x4 t = w4_signed ? signed_nibble_table()
                              : *(const u32x4*)(lut + (row * lut_groups + ((c32 * 32) >> group_shift)) * 16);
    // Row-major, or the K-tiled operand layout (k_tiled_offset).
    int8_t* o0 = out + (kt ? k_tiled_offset(row, c32 * 32, K, N) : row * K + c32 * 32);
    int8_t* o1 = out + (kt ? k_tiled_offset(row, c32 * 32 + 16, K, N) : row * K + c32 * 32 + 16);
    *(v4i*)o0 = expand16b(c[0], c[1], t);
    *(v4i*)o1 = expand16b(c[2], c[3], t);
}

bool w4_expand_ok(const GemmParams& p, const int8_t* out, bool kt) {
    return !(p.K % 32 != 0 || p.ldb % 16 != 0 || ((uintptr_t)p.B & 15) != 0 || ((uintptr_t)out & 15) != 0 ||
             (!p.w4_signed && (p.group_shift < 5 || !p.lut)) || (kt && p.K % 64 != 0));
}

hipError_t launch_w4_lut_expand(hipStream_t stream, const GemmParams& p, int8_t* out, bool kt) {
    if (!w4_expand_ok(p, out, kt)) return hipErrorInvalidValue;
    const int64_t threads = (int64_t)p.N * (p.K / 32);
    hipLaunchKernelGGL(w4_lut_expand_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream,
                       (const uint8_t*)p.B, p.ldb, p.lut, p.lut_groups, p.group_shift, p.w4_signed, (int64_t)p.N,
                       (int64_t)p.K, kt ? 1 : 0, out);
    return hipGetLastError();
}

hipError_t launch_i8_gemm_persist(hipStream_t stream, const GemmParams& p, int num_cus, int wave_tile, bool w4) {
    if (p.K % (2 * BK) != 0 || p.K < 2 * BK) return hipErrorInvalidValue;
    if (wave_tile != 128 && wave_tile != 64) return hipErrorInvalidValue;
    // W4: one table per K-step (group a multiple of 128), 16-byte code loads.
    if (w4 && (p.ldb % 16 != 0 || ((uintptr_t)p.B & 15) != 0 || (!p.w4_signed && (p.group_shift < 7 || !p.lut))))
        return hipErrorInvalidValue;
    const int bm = 2 * wave_tile;
    const int tiles = ((p.M + bm - 1) / bm) * ((p.N + bm - 1) / bm);
    const int grid = tiles < num_cus ? tiles : num_cus;
    // The gated residual (p.gate) is its own instantiation, so the plain
    // kernels carry none of its registers.
    if (w4 && p.gate) return hipErrorInvalidValue;
    if (wave_tile == 128) {
        if (w4) hipLaunchKernelGGL((i8_gemm_persist_kernel<128, true, false>), dim3(grid), dim3(256), 0, stream, p);
        else if (p.gate) hipLaunchKernelGGL((i8_gemm_persist_kernel<128, false, true>), dim3(grid), dim3(256), 0, stream, p);
        else hipLaunchKernelGGL((i8_gemm_persist_kernel<128, false, false>), dim3(grid), dim3(256), 0, stream, p);
    } else {
        if (w4) hipLaunchKernelGGL((i8_gemm_persist_kernel<64, true, false>), dim3(grid), dim3(256), 0, stream, p);
        else if (p.gate) hipLaunchKernelGGL((i8_gemm_persist_kernel<64, false, true>), dim3(grid), dim3(256), 0, stream, p);
        else hipLaunchKernelGGL((i8_gemm_persist_kernel<64, false, false>), dim3(grid), dim3(256), 0, stream, p);
    }
    return hipGetLastError();
}

hipError_t launch_i8_gemm_persist_mixed(hipStream_t stream, const GemmParams& pb, const GemmParams& ps, int num_cus,
                                        bool w4) {
    if (pb.K != ps.K || pb.K % (2 * BK) != 0 || pb.K < 2 * BK) return hipErrorInvalidValue;
    if (w4 && (pb.ldb % 16 != 0 || ((uintptr_t)pb.B & 15) != 0 || (!pb.w4_signed && (pb.group_shift < 7 || !pb.lut))))
        return hipErrorInvalidValue;
    if (w4 && pb.gate) return hipErrorInvalidValue;
    const int big = ((pb.M + 255) / 256) * ((pb.N + 255) / 256), small = ((ps.M + 127) / 128) * ((ps.N + 127) / 128);
    const int most = big > small ? big : small;
    const int grid = most < num_cus ? most : num_cus;
    if (w4) hipLaunchKernelGGL((i8_gemm_persist_mixed_kernel<true, false>), dim3(grid), dim3(256), 0, stream, pb, ps);
    else if (pb.gate) hipLaunchKernelGGL((i8_gemm_persist_mixed_kernel<false, true>), dim3(grid), dim3(256), 0, stream, pb, ps);
    else hipLaunchKernelGGL((i8_gemm_persist_mixed_kernel<false, false>), dim3(grid), dim3(256), 0, stream, pb, ps);
    return hipGetLastError();
}

}  // namespace phi_dev
