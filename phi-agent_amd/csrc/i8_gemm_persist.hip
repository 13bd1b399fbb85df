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

// Cache policy of the output stores: non-temporal.  The output is written
// once and never read back by this kernel; letting it allocate in L2 evicts
// the A and B strips the XCD's other tiles are still reading, and every CU
// finishing a tile at about the same time turns that into a write-back burst
// the next K-step's loads queue behind (measured: 17 % of the kernel time at
// 4352 x 12288 x 3072).
constexpr int kStoreNT = 2;

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

// The workgroup's work list.  Tiles [0, dp_tiles) are dealt whole, round
// by round: workgroup r (after the XCD remap) takes tiles r, r + G, ...
// The split phase covers the remaining sk_tiles tiles as U = sk_tiles * KT
// K-steps ("units"), cut into G contiguous ranges of whole unit pairs (KT is
// even, so a tile boundary is a pair boundary); range r is
// [2 * (r * (U/2) / G), 2 * ((r + 1) * (U/2) / G)).  A range starts or ends
// inside a tile at most once each, so a workgroup holds at most two partial
// tiles.
// The launcher guarantees U * G < 2^31, so all of this is 32-bit.
struct Plan {
    int G, r, KT, ntiles, dp_tiles, n_dp, n_sk, nseg;
    int U, s, e;  // split-phase units and this workgroup's range
    int sk_t0;    // first split-phase tile of the range
};

// One stretch of K-steps [kb, ke) of logical tile `tile`.
struct Seg {
    int tile, kb, ke;
};

__device__ __forceinline__ Seg seg_at(const Plan& P, int i) {
    Seg g;
    if (i < P.n_dp) {
        g.tile = i * P.G + P.r;
        g.kb = 0;
        g.ke = P.KT;
    } else {
        const int jt = P.sk_t0 + (i - P.n_dp);
        const int t0 = jt * P.KT;
        g.tile = P.dp_tiles + jt;
        g.kb = max(P.s, t0) - t0;
        g.ke = min(P.e, t0 + P.KT) - t0;
    }
    return g;
}

// The workgroup whose range holds split-phase unit u.
__device__ __forceinline__ int sk_owner(int u, const Plan& P) { return ((u / 2 + 1) * P.G - 1) / (P.U / 2); }

// Per-wave state.  The load cursor runs one K-step pair ahead of the
// multiply, so it enters a segment during the previous segment's last pair;
// after the last segment it reloads that segment's last pair (harmless).
struct Wv {
    int8_t* la[2];
    int8_t* lb[2];
    int8_t* le;   // two 3 KB epilogue-operand areas, one per segment parity
    int8_t* lc;
    __amdgpu_buffer_rsrc_t rA, rB;  // the load cursor's tile
    int cm0, cn0;
    int voA[2], voB[2];
    int wave, wm, wn, lane, lrow, lhalf;
    int oA[4], oB[4];
};

// Points the load cursor at logical tile t.
__device__ __forceinline__ void cursor_tile(Wv& w, const GemmParams& p, const Shape& s, int t) {
    int tm, tn;
    tile_mn(s, t, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    w.cm0 = m0;
    w.cn0 = n0;
    const int rows = min(BM, p.M - m0), cols = min(BN, p.N - n0);
    w.rA = __builtin_amdgcn_make_buffer_rsrc((void*)(p.A + (int64_t)m0 * p.lda), (short)0, rows * (int)p.lda, kRsrcWord3);
    w.rB = __builtin_amdgcn_make_buffer_rsrc((void*)(p.B + (int64_t)n0 * p.ldb), (short)0, cols * (int)p.ldb, kRsrcWord3);
}

// Epilogue operands of the cursor's tile into LDS area le: wave w loads row
// scales 64w..64w+63, column scales / fp32 bias 64w..64w+63 and (waves 0-1)
// the bf16 bias words; past M or N they read as zero.  Issued with the
// first K-step load of a segment.
__device__ __forceinline__ void issue_epi(const Wv& w, const GemmParams& p, int8_t* le) {
    const int rows = min(BM, p.M - w.cm0), cols = min(BN, p.N - w.cn0);
    const __amdgpu_buffer_rsrc_t rSA =
        __builtin_amdgcn_make_buffer_rsrc((void*)(p.sA ? p.sA + w.cm0 : (const float*)p.A), (short)0,
                                          p.sA ? rows * 4 : 0, kRsrcWord3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rSA, (lptr_t)(le + w.wave * 256), 4, w.lane * 4, w.wave * 256, 0, 0);
    const bool sbs = p.sb_scalar != 0;
    const __amdgpu_buffer_rsrc_t rSB = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.sB ? (sbs ? p.sB : p.sB + w.cn0) : (const float*)p.A), (short)0, p.sB ? (sbs ? 4 : cols * 4) : 0,
        kRsrcWord3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rSB, (lptr_t)(le + 1024 + w.wave * 256), 4, sbs ? 0 : w.lane * 4,
                                             sbs ? 0 : w.wave * 256, 0, 0);
    const int bsz = p.bias_kind == BIAS_F32 ? 4 : 2;
    const __amdgpu_buffer_rsrc_t rBZ = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.bias_kind != BIAS_NONE ? (const int8_t*)p.bias + (int64_t)w.cn0 * bsz : (const int8_t*)p.A), (short)0,
        p.bias_kind != BIAS_NONE ? cols * bsz : 0, kRsrcWord3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rBZ, (lptr_t)(le + 2048 + w.wave * 256), 4, w.lane * 4,
                                             w.wave * 256, 0, 0);
}

// K-step kl of the cursor's tile into stage S: 8 A and 8 B loads per wave,
// with EPI plus the tile's epilogue operands into area le.
template <int S, bool EPI>
__device__ __forceinline__ void issue(const Wv& w, const GemmParams& p, int kl, int8_t* le) {
    const int koff = kl * BK;
#pragma unroll
    for (int j = 0; j < DL; j++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(w.rA, (lptr_t)(w.la[S] + w.wave * (DL * 1024) + j * 1024), 16,
                                                 w.voA[j & 1], koff + (w.wave * 64 + j * 8) * (int)p.lda, 0, 0);
#pragma unroll
    for (int j = 0; j < DL; j++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(w.rB, (lptr_t)(w.lb[S] + w.wave * (DL * 1024) + j * 1024), 16,
                                                 w.voB[j & 1], koff + (w.wave * 64 + j * 8) * (int)p.ldb, 0, 0);
    if constexpr (EPI) issue_epi(w, p, le);
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

// Keeps the accumulators in their AGPRs across a region the register
// allocator would otherwise split them around.
__device__ __forceinline__ void pin_acc(v16i (&acc)[4][4]) {
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) asm volatile("" : "+a"(acc[j][i]));
}

__device__ __forceinline__ void zero_acc(v16i (&acc)[4][4]) {
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[j][i] = v16i{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
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
// of stage SN into nxt; with LOADS the cursor's K-step into stage S.  The
// first MFMA goes ahead of the reads because the compiler's wait for cur is
// a full lgkmcnt(0) that must not cover reads issued after it.
template <int S, int SN, int QN, bool ZERO, bool LOADS, bool EPI>
__device__ __forceinline__ void quarter(const Frag& cur, Frag& nxt, v16i (&acc)[4][4], const Wv& w,
                                        const GemmParams& p, int kl, int8_t* le) {
    mma16<ZERO>(cur, acc);
    if constexpr (LOADS) issue<S, EPI>(w, p, kl, le);
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
// every load in flight: the next stage's (issued one K-step earlier).  After
// the barrier every wave is done reading stage S, which the last quarter
// refills with K-step kl of the cursor's tile (epilogue operands into le).
template <int S, bool EPI>
__device__ __forceinline__ void step(Frag& f0, v16i (&acc)[4][4], const Wv& w, const GemmParams& p, int kl,
                                     int8_t* le) {
    Frag f1;
    quarter<S, S, 1, false, false, false>(f0, f1, acc, w, p, kl, le);
    quarter<S, S, 2, false, false, false>(f1, f0, acc, w, p, kl, le);
    quarter<S, S, 3, false, false, false>(f0, f1, acc, w, p, kl, le);
    wait_all();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    quarter<S, S ^ 1, 0, false, true, EPI>(f1, f0, acc, w, p, kl, le);
}

// Split-phase partial tiles.  Every split tile has exactly two shares (the
// launcher keeps each range at least a tile long): the tail, the tile's last
// K-steps, which its workgroup multiplies first in its range, and the head,
// the first K-steps, which another workgroup multiplies last in its range.
// The tail workgroup leaves its accumulators in its 256 KB slot and raises
// the tile's ready word; the head workgroup waits for the word (the tail is
// normally done long before), starts its accumulators from the slot instead
// of zero, and runs the epilogue.  Slot layout: wave, block (j, i), register
// quad g, lane -- 16 bytes a lane, so both sides move whole 1 KB rows per
// instruction in the accumulators' own layout.  Slots and ready words are
// shared across XCDs, whose L2s are not coherent with each other: every
// access is device-scope (sc1), which writes through and reads past the
// non-coherent caches.
constexpr int kDevScope = 16;  // sc1
constexpr int kReadyBase = 64;  // sk_cnt[0]: error count; ready words from here (one cache line apart)
constexpr int kSlotBytes = BM * BN * 4;

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

// Where an epilogue writes: the output tile, or (raw int32, device scope) a
// tail share's slot as a 256 x 256 row-major matrix.
struct Dst {
    __amdgpu_buffer_rsrc_t rs;  // the tile's rows
    int pitch;                  // bytes per row
    int n0, N;                  // first column; columns at or past N are dropped
    int kind;                   // C_BF16 / C_F32 / C_I32
    int dev;                    // device-scope stores (slots) instead of non-temporal ones
};

// Epilogue (operands in the LDS area e).  Lane l holds row l % 32 of
// each A block and, in registers 4g..4g+3, columns 8g + 4(l/32) + 0..3 of each
// B block.  Each 32-row strip goes through the wave's LDS area (16-byte slots
// swizzled by row) and is stored as whole rows: bf16 in 32 x 64-column
// pieces (128 bytes a row), fp32 / int32 in 32 x 32-column pieces.
__device__ __forceinline__ void epilogue(v16i (&acc)[4][4], const GemmParams& p, const Dst& d, const Wv& w,
                                         const int8_t* e) {
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) asm volatile("" : "+a"(acc[j][i]));
    const __amdgpu_buffer_rsrc_t rs = d.rs;
    const int pitch = d.pitch;
    int8_t* lc = w.lc;
    const int colw = d.n0 + w.wn * 128;  // first column of this wave
    float sa[4];
#pragma unroll
    for (int i = 0; i < 4; i++) sa[i] = *(const float*)(e + (w.wm * 128 + i * 32 + w.lrow) * 4);
    if (d.kind == C_BF16) {
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
                    if (col < d.N)
                        __builtin_amdgcn_raw_buffer_store_b128(v, rs, (w.wm * 128 + i * 32 + r) * pitch + col * 2, 0, kStoreNT);
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
        if (d.kind == C_F32) {
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
                if (d.kind == C_F32) {
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
                if (col < d.N) {
                    if (d.dev)
                        __builtin_amdgcn_raw_buffer_store_b128(v, rs, (w.wm * 128 + i * 32 + r) * pitch + col * 4, 0, kDevScope);
                    else
                        __builtin_amdgcn_raw_buffer_store_b128(v, rs, (w.wm * 128 + i * 32 + r) * pitch + col * 4, 0, kStoreNT);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// Head share of split tile jt: waits (bounded) for the tail's ready word and
// loads the tail's slot into the accumulators.  A wait that runs out counts
// in the workspace's error word and starts from zero instead (the tile is
// then wrong and the caller must clear the workspace before reusing it).
__device__ __forceinline__ void head_acquire(v16i (&acc)[4][4], const GemmParams& p, const Plan& P, const Wv& w,
                                             int jt, int* flag) {
    if (w.wave == 0 && w.lane == 0) {
        int ready = 0;
        for (int n = 0; n < p.sk_spin; n++) {
            ready = __hip_atomic_load(p.sk_cnt + kReadyBase + jt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (ready) break;
            __builtin_amdgcn_s_sleep(2);
        }
        if (!ready) __hip_atomic_fetch_add(p.sk_cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = ready;
    }
    __builtin_amdgcn_s_barrier();
    if (__builtin_amdgcn_readfirstlane(*flag) == 0) {
        zero_acc(acc);
        return;
    }
    const int q = sk_owner(jt * P.KT + P.KT - 1, P);  // the tail's workgroup
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.sk_part + (int64_t)q * kSlotBytes), (short)0, kSlotBytes, kRsrcWord3);
    // Element (row, col) of the slot is at (row * 256 + col) * 4; lane l holds
    // row wm*128 + 32i + l%32 and columns wn*128 + 32j + 8g + 4(l/32) + 0..3.
    const int base = ((w.wm * 128 + w.lrow) * BN + w.wn * 128 + 4 * w.lhalf) * 4;
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v16i blk;
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(
                    r, base + (i * 32 * BN + j * 32 + 8 * g) * 4, 0, kDevScope);
#pragma unroll
                for (int e = 0; e < 4; e++) blk[4 * g + e] = (int)v[e];
            }
            acc[j][i] = blk;
        }
}

}  // namespace

__global__ __launch_bounds__(256) void i8_gemm_persist_kernel(GemmParams p) {
    __shared__ __align__(16) int8_t a0[STG], a1[STG], b0[STG], b1[STG];
    __shared__ __align__(16) int8_t eall[2 * EBYTES];
    __shared__ __align__(16) int8_t cbuf[4 * CHUNK];
    __shared__ int flag;
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
    Plan P;
    P.G = gridDim.x;
    P.r = xcd_remap(blockIdx.x, P.G);
    P.KT = s.KT;
    P.ntiles = s.ntiles;
    P.dp_tiles = p.sk_tiles ? p.sk_dp_tiles : s.ntiles;
    P.n_dp = P.dp_tiles > P.r ? (P.dp_tiles - P.r - 1) / P.G + 1 : 0;
    P.U = p.sk_tiles * P.KT;
    P.s = 2 * (P.r * (P.U / 2) / P.G);
    P.e = 2 * ((P.r + 1) * (P.U / 2) / P.G);
    P.sk_t0 = P.s / P.KT;
    P.n_sk = P.e > P.s ? (P.e - 1) / P.KT - P.sk_t0 + 1 : 0;
    P.nseg = P.n_dp + P.n_sk;
    if (P.nseg == 0) return;
    w.la[0] = a0;
    w.la[1] = a1;
    w.lb[0] = b0;
    w.lb[1] = b1;
    w.le = eall;
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
    // Every segment holds at least one K-step pair.  The epilogue operands
    // of segment i go to area i % 2, loaded with its first K-step (during
    // segment i-1's last pair), so at least one barrier separates a
    // segment's epilogue from the load into its area for segment i+2.
    {
        const Seg g = seg_at(P, 0);
        cursor_tile(w, p, s, g.tile);
        issue<0, true>(w, p, g.kb, w.le);
        issue<1, false>(w, p, g.kb + 1, w.le);
    }
    wait_vm_lgkm0<2 * DL>();  // the first K-step and its operands have landed
    __builtin_amdgcn_s_barrier();
    Frag f0;
    frag<0, 0>(f0, w);
    v16i acc[4][4];
    for (int seg = 0;;) {
        const Seg g = seg_at(P, seg);
        const bool whole = g.kb == 0 && g.ke == P.KT;
        const int jt = g.tile - P.dp_tiles;  // split-phase tile index
        if (!whole && g.kb == 0) head_acquire(acc, p, P, w, jt, &flag);
        else zero_acc(acc);
        int8_t* le = w.le + (seg & 1) * EBYTES;
        for (int k = g.kb; k < g.ke - 2; k += 2) {
            step<0, false>(f0, acc, w, p, k + 2, le);
            step<1, false>(f0, acc, w, p, k + 3, le);
        }
        // The last pair: the cursor moves to the next segment, if any.
        int kn = g.ke - 2;
        int8_t* ln = le;
        if (seg + 1 < P.nseg) {
            const Seg h = seg_at(P, seg + 1);
            cursor_tile(w, p, s, h.tile);
            kn = h.kb;
            ln = w.le + ((seg + 1) & 1) * EBYTES;
        }
        step<0, true>(f0, acc, w, p, kn, ln);
        step<1, false>(f0, acc, w, p, kn + 1, ln);
        // A whole or head tile goes to C; a tail share goes to this
        // workgroup's slot as raw int32 and then raises the ready word.
        const bool tail = g.kb != 0;
        Dst d;
        if (!tail) {
            int tm, tn;
            tile_mn(s, g.tile, tm, tn);
            const int m0 = tm * BM;
            d.kind = p.c_kind;
            d.pitch = (int)p.ldc * (p.c_kind == C_BF16 ? 2 : 4);
            d.rs = __builtin_amdgcn_make_buffer_rsrc((int8_t*)p.C + (int64_t)m0 * d.pitch, (short)0,
                                                     min(BM, p.M - m0) * d.pitch, kRsrcWord3);
            d.n0 = tn * BN;
            d.N = p.N;
            d.dev = 0;
        } else {
            d.kind = C_I32;
            d.pitch = BN * 4;
            d.rs = __builtin_amdgcn_make_buffer_rsrc(p.sk_part + (int64_t)P.r * kSlotBytes, (short)0, kSlotBytes,
                                                     kRsrcWord3);
            d.n0 = 0;
            d.N = BN;
            d.dev = 1;
        }
        epilogue(acc, p, d, w, le);
        if (tail) {
            wait_all();  // every row of this wave's share has reached device scope
            __builtin_amdgcn_s_barrier();
            if (w.wave == 0 && w.lane == 0)
                __hip_atomic_store(p.sk_cnt + kReadyBase + jt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else if (!whole && w.wave == 0 && w.lane == 0) {
            __hip_atomic_store(p.sk_cnt + kReadyBase + jt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (++seg == P.nseg) break;
    }
    // The reloads past the last K-step still write LDS: let them land.
    wait_all();
}

hipError_t launch_i8_gemm_persist(hipStream_t stream, const GemmParams& p, int num_cus) {
    if (p.K % (2 * BK) != 0 || p.K < 4 * BK) return hipErrorInvalidValue;
    const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
    int grid = tiles < num_cus ? tiles : num_cus;
    if (p.sk_tiles) {
        // The split phase takes the whole device, and every range must be at
        // least a tile long (so a tile has at most two shares) and fewer than
        // two tiles (one ready word per tile fits the counter area).
        const int64_t units = (int64_t)p.sk_tiles * (p.K / BK);
        if (p.sk_dp_tiles % num_cus != 0 || p.sk_dp_tiles + p.sk_tiles != tiles || p.sk_tiles < num_cus ||
            p.sk_tiles >= 2 * num_cus || units * num_cus >= ((int64_t)1 << 31) ||
            (int64_t)(kReadyBase + p.sk_tiles) * 4 > (int64_t)kPersistCounterBytes || p.sk_spin < 0 || !p.sk_cnt ||
            !p.sk_part)
            return hipErrorInvalidValue;
        grid = num_cus;
    }
    hipLaunchKernelGGL(i8_gemm_persist_kernel, dim3(grid), dim3(256), 0, stream, p);
    return hipGetLastError();
}

size_t persist_workspace_bytes(int num_cus) {
    // The error word and ready words, then one tail slot per workgroup.
    return kPersistCounterBytes + (size_t)num_cus * kSlotBytes;
}

}  // namespace phi_dev
