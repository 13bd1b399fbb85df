// Persistent int8 GEMM for gfx950 with a four-stage, 64-deep K pipeline:
// one workgroup per CU walks square output tiles (256 x 256, or 128 x 128 for
// the rows a whole number of 256-row rounds does not cover) as the
// two-stage kernel of i8_gemm_persist.hip does, with a different main loop.
//
//   acc[m,n] = sum_k A[m,k] * B[n,k]                  (exact int32)
//   C[m,n]   = fma((float)acc * sA[m], sB[n], bias[n])  -> bf16 (RNE) / fp32 / raw int32
//
// The product and epilogue are those of the reference's int8_gemm_tc
// (core/kernels/int8_gemm.cpp:466-621, epilogue :588-620) and host gemm_int8
// (core/host/quant.cpp:223-236).
//
// Why this loop.  A CU moves operands into LDS at about 57 bytes a clock;
// a 256 x 256 tile needs 64 KB of A and B per 128 K, against 64 MFMAs a wave
// (2048 clocks).  The two-stage kernel can refill a stage only after the
// barrier that ends its K-step, so each wave issues its 16 loads of a K-step
// in one quarter: the load queue backs up, and the MFMAs behind the loads in
// the wave's instruction stream wait for it.  Here:
//   * Four stages of 64 K (A and B 2WT rows x 64 bytes each: 128 KB for the
//     256 x 256 tile).  K-step k works on stage k % 4.
//   * A K-step is two quarters of NB^2 MFMAs.  Quarter 0 reads the second
//     half of the step's fragments and issues B's loads for K-step k + 3;
//     quarter 1 reads the first fragments of K-step k + 1 and issues A's
//     loads for K-step k + 4 into stage k % 4, which the barrier between the
//     quarters has released.  Loads are spread DL per quarter, and data is
//     loaded four to five quarters before it is read.
//   * Each load instruction moves 16 rows x 64 bytes.  64-byte row pieces
//     stream faster than whole 128-byte rows at a 3072-byte pitch (14 against
//     8 TB/s over a 48 MB operand, measured with the same instruction).
//   * One barrier per K-step, between its quarters, after a wait for the
//     wave's own loads of K-step k + 1 (the four later load groups may stay
//     in flight: memory operations complete in issue order).
//   * The A and B load cursors move to the workgroup's next tile on their
//     own K-steps (A at K-step KT - 4, B at KT - 3): a tile's first K-steps
//     are loaded while it finishes.  The next tile's epilogue operands are
//     loaded with A's first K-step.
//   * Chunk c (16 bytes) of row r sits in slot c ^ ((r >> 2) & 3) of the
//     row's 64 bytes: the 16-byte fragment reads of 16 consecutive rows hit
//     16 distinct bank windows.
//   * Fused tile transitions (bf16 output without a gate, K > 256): the
//     first half of the next tile's K-step 0 is issued inside the epilogue,
//     one MFMA per accumulator block as soon as the epilogue has read the
//     block out, so those MFMAs run beside the epilogue's conversion.
// The epilogue, the tile order and the epilogue-operand loads are those of
// persist_common.hpp.
#include "device_common.hpp"
#include "i8_gemm.hpp"
#include "persist_common.hpp"

// Tile-timeline hooks.  The library defines them empty.  The tracing build
// in probe.hip defines them to record the real-time clock per workgroup: at
// the kernel's start, at each tile's start, K-loop end and epilogue end, and
// between the two tile sizes.
#ifndef PHI_PIPE_STAMP
#define PHI_PIPE_STAMP(phase, tile, point)
#define PHI_PIPE_TRACE_BEGIN
#define PHI_PIPE_TRACE_END
#endif

namespace phi_dev {

namespace {

using namespace persist;

constexpr int PK = 64;   // K bytes per stage
constexpr int NSTG = 4;  // stages

template <int WT>
struct PCfg {
    static constexpr int NB = WT / 32;         // MFMA blocks per wave dimension
    static constexpr int BM = 2 * WT;          // workgroup tile (square)
    static constexpr int STG = BM * PK;        // bytes per operand per stage
    static constexpr int DL = STG / 1024 / 4;  // loads per operand per wave per K-step
    // Epilogue stores a wave issues on the bf16 path, the fewest of any
    // output path (every store is issued: none is branched around).
    static constexpr int NSTORE = 2 * NB * NB;
    // Memory operations a K-step's wait may leave in flight: the four load
    // groups issued after K-step k + 1's last one; in a tile's first two
    // K-steps also the previous tile's epilogue stores, issued between them.
    static constexpr int VWN = 4 * DL;
    static constexpr int VWR = 4 * DL + NSTORE;
    static_assert(VWR < 64, "vmcnt is six bits");
};

template <int WT>
struct Frag {
    v4i a[PCfg<WT>::NB], b[PCfg<WT>::NB];
};

// The next tile of the workgroup, if any (origins precomputed once a tile).
struct NextTile {
    int m0, n0;
    bool valid;
};

// Per-wave state.  Each operand has its own load cursor: a buffer resource
// over its tile's rows and the next K-step to load.
struct Pw : EpiWave {
    int8_t* la;  // A stage 0, stage s at la + s * STG (opaque, so fragment
    int8_t* lb;  // B stage 0  offsets stay immediates wherever the stages sit)
    int8_t* le;  // two epilogue-operand areas, one per tile parity
    __amdgpu_buffer_rsrc_t rA, rB;
    int voA, voB;  // per-lane global offset within a 16-row load
    int oA[2], oB[2];
    int kA, kB;
    // K-tiled operands: bytes from one K-step's block to the next (strip
    // height x 64), and the tile's offset within its 256-row strip's block.
    int kstA, kstB, hoA, hoB;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const int8_t* base, int64_t ld, int row0, int nrows) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)(base + (int64_t)row0 * ld), (short)0, nrows * (int)ld,
                                             kRsrcWord3);
}

// A K-tiled operand of `rows` rows and K columns (k_tiled_offset): the
// resource over the strip holding tile row row0, that strip's K-step stride,
// and the tile's offset within the strip's K-step block (128-row tiles sit in
// either half of a 256-row strip).
__device__ __forceinline__ void kt_cursor(const int8_t* base, int K, int row0, int rows, __amdgpu_buffer_rsrc_t& r,
                                          int& kst, int& ho) {
    const int s = row0 >> 8, h = min(256, rows - (s << 8));
    r = __builtin_amdgcn_make_buffer_rsrc((void*)(base + (int64_t)s * 256 * K), (short)0, h * K, kRsrcWord3);
    kst = h * 64;
    ho = (row0 & 255) * 64;
}

// DL loads of operand A's K-step w.kA into stage ST (16 rows each); then the
// cursor advances.
// KT: the operand is K-tiled, so the wave's 16-row pieces of the K-step are
// contiguous 1 KB blocks: each load fetches 1 KB from one place.
template <int WT, int ST, bool KT>
__device__ __forceinline__ void load_a(Pw& w, const GemmParams& p) {
    constexpr int DL = PCfg<WT>::DL, STG = PCfg<WT>::STG;
    int8_t* d = opaque_lds(w.la + ST * STG + w.wave * (DL * 1024));
    if constexpr (KT) {
        const int koff = w.kA * w.kstA + w.hoA;
#pragma unroll
        for (int j = 0; j < DL; j++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(w.rA, (lptr_t)(d + j * 1024), 16, w.voA,
                                                     koff + (w.wave * DL + j) * 1024, 0, 0);
    } else {
        const int koff = w.kA * PK;
#pragma unroll
        for (int j = 0; j < DL; j++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(w.rA, (lptr_t)(d + j * 1024), 16, w.voA,
                                                     koff + (w.wave * DL + j) * 16 * (int)p.lda, 0, 0);
    }
    w.kA++;
}

template <int WT, int ST, bool KT>
__device__ __forceinline__ void load_b(Pw& w, const GemmParams& p) {
    constexpr int DL = PCfg<WT>::DL, STG = PCfg<WT>::STG;
    int8_t* d = opaque_lds(w.lb + ST * STG + w.wave * (DL * 1024));
    if constexpr (KT) {
        const int koff = w.kB * w.kstB + w.hoB;
#pragma unroll
        for (int j = 0; j < DL; j++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(w.rB, (lptr_t)(d + j * 1024), 16, w.voB,
                                                     koff + (w.wave * DL + j) * 1024, 0, 0);
    } else {
        const int koff = w.kB * PK;
#pragma unroll
        for (int j = 0; j < DL; j++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(w.rB, (lptr_t)(d + j * 1024), 16, w.voB,
                                                     koff + (w.wave * DL + j) * 16 * (int)p.ldb, 0, 0);
    }
    w.kB++;
}

// Cursor switches at a tile's end: to the next tile's K-step 0, or, after
// the last tile, back to K-step 0 of the same tile (those loads land in
// released stages and are never read).
template <int WT, bool KT>
__device__ __forceinline__ void switch_a(Pw& w, const GemmParams& p, const NextTile& nt) {
    constexpr int BM = PCfg<WT>::BM;
    if (nt.valid) {
        if constexpr (KT) kt_cursor(p.A, p.K, nt.m0, p.M, w.rA, w.kstA, w.hoA);
        else w.rA = rows_rsrc(p.A, p.lda, nt.m0, min(BM, p.M - nt.m0));
        w.cm0 = nt.m0;
        w.cn0 = nt.n0;
    }
    w.kA = 0;
}

template <int WT, bool KT>
__device__ __forceinline__ void switch_b(Pw& w, const GemmParams& p, const NextTile& nt) {
    constexpr int BM = PCfg<WT>::BM;
    if (nt.valid) {
        if constexpr (KT) kt_cursor(p.B, p.K, nt.n0, p.N, w.rB, w.kstB, w.hoB);
        else w.rB = rows_rsrc(p.B, p.ldb, nt.n0, min(BM, p.N - nt.n0));
    }
    w.kB = 0;
}

template <int WT, int ST, int Q>
__device__ __forceinline__ void frag(Frag<WT>& f, const Pw& w) {
    constexpr int NB = PCfg<WT>::NB, STG = PCfg<WT>::STG;
    const int8_t* cA = w.la + ST * STG + w.oA[Q];
    const int8_t* cB = w.lb + ST * STG + w.oB[Q];
#pragma unroll
    for (int i = 0; i < NB; i++) f.a[i] = *(const v4i*)(cA + i * 32 * PK);
#pragma unroll
    for (int j = 0; j < NB; j++) f.b[j] = *(const v4i*)(cB + j * 32 * PK);
}

// MFMAs Q0 .. Q1-1 of the NB x NB block (column block j = q / NB outer).
// Z: the tile's first MFMAs, which start the accumulators from an inline 0.
template <int WT, int Q0, int Q1, bool Z>
__device__ __forceinline__ void mma(const Frag<WT>& f, v16i (&acc)[PCfg<WT>::NB][PCfg<WT>::NB]) {
    constexpr int NB = PCfg<WT>::NB;
#pragma unroll
    for (int q = Q0; q < Q1; q++) {
        const int j = q / NB, i = q % NB;
        if constexpr (Z)
            acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.b[j], f.a[i], v16i{}, 0, 0, 0);
        else
            acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.b[j], f.a[i], acc[j][i], 0, 0, 0);
    }
}

// Places a quarter's R fragment reads and V loads between the NB^2 - 1
// MFMAs after its first (slots 0 .. NB^2 - 2).  The reads are spread over all
// slots but the last, slot T taking those that bring the running total to
// (T + 1) / (NB^2 - 2) of R, so the next quarter's first MFMAs, which need
// them, have one MFMA of slack.  The loads are spread the same way over all
// slots; a 128 x 128 tile's two loads go to the first and the last slot.
// Spreading the reads keeps the four waves' fragment reads from meeting the
// stages' incoming DMA in bursts.  Measured at 4352 x 12288 x 3072 (clocks a
// K-step): the 256 x 256 tile's eight reads in the first eight slots 1206,
// spread as here 1092 (1024 of MFMA issue; twelve other placements
// 1092-1228); the 128 x 128 tile's four reads one, one and two a slot 392,
// two, two, none 382, with the loads moved as here 368 (256 of MFMA issue).
template <int NB, int R, int V, int T = 0>
__device__ __forceinline__ void sched_quarter() {
    constexpr int SLOTS = NB * NB - 1;
    if constexpr (T < SLOTS) {
        constexpr int r = T < SLOTS - 1 ? (T + 1) * R / (SLOTS - 1) - T * R / (SLOTS - 1) : 0;
        constexpr int v = NB == 2 && V == 2 ? (T == 0 || T == SLOTS - 1 ? 1 : 0) : (T + 1) * V / SLOTS - T * V / SLOTS;
        if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(SG_DSR, r, 0);
        if constexpr (v > 0) __builtin_amdgcn_sched_group_barrier(SG_VMEM_R, v, 0);
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
        sched_quarter<NB, R, V, T + 1>();
    }
}

// A quarter: NB^2 MFMAs on cur, the fragment reads of (stage SR, half QR)
// into nxt, and the loads issued by ld (V memory operations).  The first
// MFMA goes ahead of the reads: the wait the compiler puts before it covers
// cur's reads, which must not include reads issued after it.
template <int WT, int SR, int QR, int V, bool Z, typename Ld>
__device__ __forceinline__ void pquarter(const Frag<WT>& cur, Frag<WT>& nxt, v16i (&acc)[PCfg<WT>::NB][PCfg<WT>::NB],
                                         Pw& w, Ld&& ld) {
    constexpr int NB = PCfg<WT>::NB;
    mma<WT, 0, 1, Z>(cur, acc);
    ld();
    frag<WT, SR, QR>(nxt, w);
    mma<WT, 1, NB * NB, Z>(cur, acc);
    __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
    sched_quarter<NB, 2 * NB, V>();
    __builtin_amdgcn_sched_barrier(0);
}

// K-step k on stage S = k % 4.  f0 holds the step's first-half fragments on
// entry and the next step's on return.  Z: the tile's first K-step.  VW: the
// wait's allowance.  SWA / SWB: the A / B cursor moves to the next tile
// before its loads here (SWA also loads that tile's epilogue operands into
// area ln).
template <int WT, int S, bool Z, int VW, bool SWA, bool SWB, bool G, bool KT>
__device__ __forceinline__ void pstep(Frag<WT>& f0, v16i (&acc)[PCfg<WT>::NB][PCfg<WT>::NB], Pw& w,
                                      const GemmParams& p, const NextTile& nt, int8_t* ln) {
    constexpr int DL = PCfg<WT>::DL;
    constexpr int NE = G ? 4 : 3;  // epilogue-operand loads
    Frag<WT> f1;
    pquarter<WT, S, 1, DL, Z>(f0, f1, acc, w, [&] {
        if constexpr (SWB) switch_b<WT, KT>(w, p, nt);
        load_b<WT, (S + 3) % NSTG, KT>(w, p);
    });
    wait_vm_lgkm0<VW>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    pquarter<WT, (S + 1) % NSTG, 0, DL + (SWA ? NE : 0), false>(f1, f0, acc, w, [&] {
        if constexpr (SWA) {
            switch_a<WT, KT>(w, p, nt);
            issue_epi<WT, G>(w, p, ln);
        }
        load_a<WT, S, KT>(w, p);
    });
}

// The epilogue of the tile in acc (bf16 output, no gate) fused with the first
// half of the next tile's K-step 0.  f0 already holds that half's fragments
// (read from stage 0 during the last K-step, as for any tile).  As soon as the
// epilogue has read a block out of its accumulators, that block's first
// K-step-0 MFMA (an inline 0 as its input) is issued, and it runs beside the
// epilogue's conversion.  After the last tile the same code runs: stage 0
// then holds the last tile's own K-step 0 (the cursors' loads past the last
// K-step), and the MFMAs' results are dropped.
template <int WT>
__device__ __forceinline__ void epilogue_kstep0a(const Frag<WT>& f0, v16i (&acc)[PCfg<WT>::NB][PCfg<WT>::NB],
                                                 const Pw& w, const GemmParams& p, const NextTile& cur,
                                                 const int8_t* le) {
    epilogue<WT, false>(acc, p, cur.m0, cur.n0, w, le, [&](int j, int i) {
        acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f0.b[j], f0.a[i], v16i{}, 0, 0, 0);
    });
    __builtin_amdgcn_sched_barrier(0);
}

// The rest of the next tile's K-step 0, as pstep<0> runs it: B of K-step 3
// (stage 3 was released by the last K-step's barrier), the second-half
// fragments, the wait and barrier, and the second quarter (A of K-step 4 into
// stage 0, K-step 1's first fragments into f0).  The memory operations are
// those of the epilogue followed by pstep<0>'s, in the same order, so every
// wait counts as in the unfused loop.
template <int WT, bool KT>
__device__ __forceinline__ void kstep0b(Frag<WT>& f0, v16i (&acc)[PCfg<WT>::NB][PCfg<WT>::NB], Pw& w,
                                        const GemmParams& p) {
    load_b<WT, 3, KT>(w, p);
    Frag<WT> f1;
    frag<WT, 0, 1>(f1, w);
    wait_vm_lgkm0<PCfg<WT>::VWR>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    pquarter<WT, 1, 0, PCfg<WT>::DL, false>(f1, f0, acc, w, [&] { load_a<WT, 0, KT>(w, p); });
}

template <int WT>
__device__ __forceinline__ NextTile next_tile(const Shape& s, const GemmParams& p, int t, bool valid) {
    NextTile nt{0, 0, valid};
    if (valid) {
        int tm, tn;
        tile_mn(s, t, tm, tn);
        nt.m0 = tm * PCfg<WT>::BM;
        nt.n0 = tn * PCfg<WT>::BM;
    }
    return nt;
}

// The persistent loop over this workgroup's tiles of p, on four A stages at
// la and four B stages at lb (STG bytes each), the epilogue-operand areas
// eall and the epilogue staging cbuf.  K % 256 == 0.  Returns at once when
// the workgroup has no tile.
template <int WT, bool G, bool KT, bool F>
__device__ __forceinline__ void pipe_tiles(const GemmParams& p, int8_t* la, int8_t* lb, int8_t* eall, int8_t* cbuf) {
    using C = PCfg<WT>;
    constexpr int NB = C::NB, DL = C::DL, BM = C::BM;
    Pw w;
    w.lane = threadIdx.x & 63;
    w.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & 3;
    w.wm = w.wave >> 1;
    w.wn = w.wave & 1;
    w.lrow = w.lane & 31;
    w.lhalf = w.lane >> 5;
    Shape s;
    s.tiles_m = (p.M + BM - 1) / BM;
    s.tiles_n = (p.N + BM - 1) / BM;
    s.ntiles = s.tiles_m * s.tiles_n;
    s.KT = p.K / PK;
    s.group_m = p.group_m;
    s.G = gridDim.x;
    init_div(s);
    const int r = xcd_remap(blockIdx.x, s.G);
    if (r >= s.ntiles) return;
    const int ntile = (s.ntiles - r - 1) / s.G + 1;
    w.la = opaque_lds(la);
    w.lb = opaque_lds(lb);
    w.le = eall;
    w.lc = cbuf + w.wave * CHUNK;
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const int c = (2 * q + w.lhalf) ^ ((w.lrow >> 2) & 3);
        w.oA[q] = (w.wm * WT + w.lrow) * PK + c * 16;
        w.oB[q] = (w.wn * WT + w.lrow) * PK + c * 16;
    }
    // A load covers 16 rows: lane l writes row l / 4, slot l % 4, and fetches
    // the chunk that belongs in that slot (K-tiled: the slot's bytes as stored).
    if constexpr (KT) {
        w.voA = w.lane * 16;
        w.voB = w.lane * 16;
    } else {
        const int row = w.lane >> 2, c = (w.lane & 3) ^ ((row >> 2) & 3);
        w.voA = row * (int)p.lda + c * 16;
        w.voB = row * (int)p.ldb + c * 16;
    }
    // Prologue: the first tile's K-steps 0-2 and A of K-step 3, with its
    // epilogue operands; then NSTORE stores that land nowhere (offsets
    // outside a zero-length range), standing where a previous tile's
    // epilogue stores would stand, so every tile's first waits count alike.
    const NextTile first = next_tile<WT>(s, p, r, true);
    if constexpr (KT) {
        kt_cursor(p.A, p.K, first.m0, p.M, w.rA, w.kstA, w.hoA);
        kt_cursor(p.B, p.K, first.n0, p.N, w.rB, w.kstB, w.hoB);
    } else {
        w.rA = rows_rsrc(p.A, p.lda, first.m0, min(BM, p.M - first.m0));
        w.rB = rows_rsrc(p.B, p.ldb, first.n0, min(BM, p.N - first.n0));
    }
    w.cm0 = first.m0;
    w.cn0 = first.n0;
    w.kA = 0;
    w.kB = 0;
    load_a<WT, 0, KT>(w, p);
    issue_epi<WT, G>(w, p, w.le);
    load_b<WT, 0, KT>(w, p);
    load_a<WT, 1, KT>(w, p);
    load_b<WT, 1, KT>(w, p);
    load_a<WT, 2, KT>(w, p);
    load_b<WT, 2, KT>(w, p);
    load_a<WT, 3, KT>(w, p);
    __builtin_amdgcn_sched_barrier(0);
    {
        const __amdgpu_buffer_rsrc_t nowhere = __builtin_amdgcn_make_buffer_rsrc((void*)p.C, (short)0, 0, kRsrcWord3);
#pragma unroll
        for (int d = 0; d < C::NSTORE; d++)
            __builtin_amdgcn_raw_buffer_store_b32(0u, nowhere, w.lane * 4 + d * 256, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    wait_vm_lgkm0<5 * DL + C::NSTORE>();  // K-step 0 and the epilogue operands have landed
    __builtin_amdgcn_s_barrier();
    Frag<WT> f0;
    frag<WT, 0, 0>(f0, w);
    v16i acc[NB][NB];
    constexpr int VWR = C::VWR, VWN = C::VWN;
    if constexpr (F) {
        // Fused tile transitions (bf16 output, no gate, K > 256: the
        // launcher's condition).  K-step 0 of the first tile runs here; that
        // of every later tile inside the previous tile's epilogue
        // (epilogue_kstep0).  A separate loop: the accumulators are live
        // across its back edge, where the unfused loop's are dead.
        {
            const NextTile nt0 = next_tile<WT>(s, p, r + s.G, 1 < ntile);
            pstep<WT, 0, true, VWR, false, false, G, KT>(f0, acc, w, p, nt0, w.le + EBYTES);
        }
        NextTile cur = first;
        for (int i = 0;;) {
            const int t = r + i * s.G;
            int8_t* le = w.le + (i & 1) * EBYTES;
            int8_t* ln = w.le + ((i + 1) & 1) * EBYTES;
            const NextTile nt = next_tile<WT>(s, p, t + s.G, i + 1 < ntile);
            PHI_PIPE_STAMP(WT == 128 ? 0 : 1, i, 0);
            pstep<WT, 1, false, VWR, false, false, G, KT>(f0, acc, w, p, nt, ln);
            pstep<WT, 2, false, VWN, false, false, G, KT>(f0, acc, w, p, nt, ln);
            pstep<WT, 3, false, VWN, false, false, G, KT>(f0, acc, w, p, nt, ln);
            for (int k = 4; k < s.KT - 4; k += 4) {
                pstep<WT, 0, false, VWN, false, false, G, KT>(f0, acc, w, p, nt, ln);
                pstep<WT, 1, false, VWN, false, false, G, KT>(f0, acc, w, p, nt, ln);
                pstep<WT, 2, false, VWN, false, false, G, KT>(f0, acc, w, p, nt, ln);
                pstep<WT, 3, false, VWN, false, false, G, KT>(f0, acc, w, p, nt, ln);
            }
            pstep<WT, 0, false, VWN, true, false, G, KT>(f0, acc, w, p, nt, ln);
            pstep<WT, 1, false, VWN, false, true, G, KT>(f0, acc, w, p, nt, ln);
            pstep<WT, 2, false, VWN, false, false, G, KT>(f0, acc, w, p, nt, ln);
            pstep<WT, 3, false, VWN, false, false, G, KT>(f0, acc, w, p, nt, ln);
            PHI_PIPE_STAMP(WT == 128 ? 0 : 1, i, 1);
            epilogue_kstep0a<WT>(f0, acc, w, p, cur, le);
            PHI_PIPE_STAMP(WT == 128 ? 0 : 1, i, 2);
            if (++i == ntile) break;
            kstep0b<WT, KT>(f0, acc, w, p);
            cur = nt;
        }
    } else {
        NextTile cur = first;
        for (int i = 0;;) {
            const int t = r + i * s.G;
            int8_t* le = w.le + (i & 1) * EBYTES;
            int8_t* ln = w.le + ((i + 1) & 1) * EBYTES;
            const NextTile nt = next_tile<WT>(s, p, t + s.G, i + 1 < ntile);
            PHI_PIPE_STAMP(WT == 128 ? 0 : 1, i, 0);
            if (s.KT == 4) {
                pstep<WT, 0, true, VWR, true, false, G, KT>(f0, acc, w, p, nt, ln);
                pstep<WT, 1, false, VWR, false, true, G, KT>(f0, acc, w, p, nt, ln);
                pstep<WT, 2, false, VWN, false, false, G, KT>(f0, acc, w, p, nt, ln);
                pstep<WT, 3, false, VWN, false, false, G, KT>(f0, acc, w, p, nt, ln);
            } else {
                pstep<WT, 0, true, VWR, false, false, G, KT>(f0, acc, w, p, nt, ln);
                pstep<WT, 1, false, VWR, false, false, G, KT>(f0, acc, w, p, nt, ln);
                pstep<WT, 2, false, VWN, false, false, G, KT>(f0, acc, w, p, nt, ln);
                pstep<WT, 3, false, VWN, false, false, G, KT>(f0, acc, w, p, nt, ln);
                for (int k = 4; k < s.KT - 4; k += 4) {
                    pstep<WT, 0, false, VWN, false, false, G, KT>(f0, acc, w, p, nt, ln);
                    pstep<WT, 1, false, VWN, false, false, G, KT>(f0, acc, w, p, nt, ln);
                    pstep<WT, 2, false, VWN, false, false, G, KT>(f0, acc, w, p, nt, ln);
                    pstep<WT, 3, false, VWN, false, false, G, KT>(f0, acc, w, p, nt, ln);
                }
                pstep<WT, 0, false, VWN, true, false, G, KT>(f0, acc, w, p, nt, ln);
                pstep<WT, 1, false, VWN, false, true, G, KT>(f0, acc, w, p, nt, ln);
                pstep<WT, 2, false, VWN, false, false, G, KT>(f0, acc, w, p, nt, ln);
                pstep<WT, 3, false, VWN, false, false, G, KT>(f0, acc, w, p, nt, ln);
            }
            PHI_PIPE_STAMP(WT == 128 ? 0 : 1, i, 1);
            epilogue<WT, G>(acc, p, cur.m0, cur.n0, w, le);
            PHI_PIPE_STAMP(WT == 128 ? 0 : 1, i, 2);
            if (++i == ntile) break;
            cur = nt;
        }
    }
    // Loads past the last K-step (into released stages) and the epilogue's
    // stores are still in flight: let them land before the LDS is released.
    wait_all();
}

template <int WT, bool G, bool KT, bool F>
__global__ __launch_bounds__(256) void i8_gemm_pipe_kernel(GemmParams p) {
    constexpr int STG = PCfg<WT>::STG;
    __shared__ __align__(16) int8_t la[NSTG * STG], lb[NSTG * STG];
    __shared__ __align__(16) int8_t eall[2 * EBYTES];
    __shared__ __align__(16) int8_t cbuf[4 * CHUNK];
    PHI_PIPE_TRACE_BEGIN
    pipe_tiles<WT, G, KT, F>(p, la, lb, eall, cbuf);
    PHI_PIPE_TRACE_END
}

// Both tile sizes in one launch: the workgroup's 256 x 256 tiles of pb, then
// its 128 x 128 tiles of ps (the rows below pb's), in the same LDS.
template <bool G, bool KT, bool F>
__global__ __launch_bounds__(256) void i8_gemm_pipe_mixed_kernel(GemmParams pb, GemmParams ps) {
    constexpr int STG = PCfg<128>::STG;
    static_assert(PCfg<64>::STG <= STG, "the small tiles' stages fit in the big tiles' ones");
    __shared__ __align__(16) int8_t la[NSTG * STG], lb[NSTG * STG];
    __shared__ __align__(16) int8_t eall[2 * EBYTES];
    __shared__ __align__(16) int8_t cbuf[4 * CHUNK];
    PHI_PIPE_TRACE_BEGIN
    pipe_tiles<128, G, KT, F>(pb, la, lb, eall, cbuf);
    __syncthreads();  // every wave is done with the big tiles' LDS
    PHI_PIPE_STAMP(2, 0, 0);
    pipe_tiles<64, G, KT, F>(ps, la, lb, eall, cbuf);
    PHI_PIPE_TRACE_END
}

}  // namespace

// The fused tile transitions serve the bf16 output without a gate at K > 256.
static bool fuse_transitions(const GemmParams& p) { return !p.gate && p.c_kind == C_BF16 && p.K > NSTG * PK; }

template <int WT>
static void launch_pipe_wt(hipStream_t stream, const GemmParams& p, dim3 g3) {
    const dim3 b3(256);
    if (p.gate && p.kt) hipLaunchKernelGGL((i8_gemm_pipe_kernel<WT, true, true, false>), g3, b3, 0, stream, p);
    else if (p.gate) hipLaunchKernelGGL((i8_gemm_pipe_kernel<WT, true, false, false>), g3, b3, 0, stream, p);
    else if (fuse_transitions(p)) {
        if (p.kt) hipLaunchKernelGGL((i8_gemm_pipe_kernel<WT, false, true, true>), g3, b3, 0, stream, p);
        else hipLaunchKernelGGL((i8_gemm_pipe_kernel<WT, false, false, true>), g3, b3, 0, stream, p);
    } else if (p.kt) hipLaunchKernelGGL((i8_gemm_pipe_kernel<WT, false, true, false>), g3, b3, 0, stream, p);
    else hipLaunchKernelGGL((i8_gemm_pipe_kernel<WT, false, false, false>), g3, b3, 0, stream, p);
}

hipError_t launch_i8_gemm_pipe(hipStream_t stream, const GemmParams& p, int num_cus, int wave_tile) {
    if (p.K % (NSTG * PK) != 0 || p.K < NSTG * PK) return hipErrorInvalidValue;
    if (wave_tile != 128 && wave_tile != 64) return hipErrorInvalidValue;
    const int bm = 2 * wave_tile;
    const int tiles = ((p.M + bm - 1) / bm) * ((p.N + bm - 1) / bm);
    const int grid = tiles < num_cus ? tiles : num_cus;
    if (wave_tile == 128) launch_pipe_wt<128>(stream, p, dim3(grid));
    else launch_pipe_wt<64>(stream, p, dim3(grid));
    return hipGetLastError();
}

hipError_t launch_i8_gemm_pipe_mixed(hipStream_t stream, const GemmParams& pb, const GemmParams& ps, int num_cus) {
    if (pb.K != ps.K || pb.K % (NSTG * PK) != 0 || pb.K < NSTG * PK) return hipErrorInvalidValue;
    const int big = ((pb.M + 255) / 256) * ((pb.N + 255) / 256), small = ((ps.M + 127) / 128) * ((ps.N + 127) / 128);
    const int most = big > small ? big : small;
    const int grid = most < num_cus ? most : num_cus;
    if (pb.kt != ps.kt || (pb.gate != nullptr) != (ps.gate != nullptr) || pb.c_kind != ps.c_kind)
        return hipErrorInvalidValue;
    const dim3 g3(grid), b3(256);
    if (pb.gate && pb.kt) hipLaunchKernelGGL((i8_gemm_pipe_mixed_kernel<true, true, false>), g3, b3, 0, stream, pb, ps);
    else if (pb.gate) hipLaunchKernelGGL((i8_gemm_pipe_mixed_kernel<true, false, false>), g3, b3, 0, stream, pb, ps);
    else if (fuse_transitions(pb)) {
        if (pb.kt) hipLaunchKernelGGL((i8_gemm_pipe_mixed_kernel<false, true, true>), g3, b3, 0, stream, pb, ps);
        else hipLaunchKernelGGL((i8_gemm_pipe_mixed_kernel<false, false, true>), g3, b3, 0, stream, pb, ps);
    } else if (pb.kt) hipLaunchKernelGGL((i8_gemm_pipe_mixed_kernel<false, true, false>), g3, b3, 0, stream, pb, ps);
    else hipLaunchKernelGGL((i8_gemm_pipe_mixed_kernel<false, false, false>), g3, b3, 0, stream, pb, ps);
    return hipGetLastError();
}

}  // namespace phi_dev
