// Persistent int8 GEMM for gfx950 on 272 x 192 output tiles (K-tiled
// operands, four-stage 64-deep K ring):
//
//   acc[m,n] = sum_k A[m,k] * B[n,k]                  (exact int32)
//   C[m,n]   = fma((float)acc * sA[m], sB[n], bias[n])  -> bf16 (RNE) / fp32 / raw int32,
//              or fp32 into a gated residual: C = fma(that, gate[n], C)
//
// The product and epilogue are those of the reference's int8_gemm_tc
// (core/kernels/int8_gemm.cpp:466-621, epilogue :588-620) and host gemm_int8
// (core/host/quant.cpp:223-236).
//
// Why this tile.  The DiT shapes have M = 4352 = 16 x 272 (4096 image + 256
// text tokens) and N a multiple of 3 x 1024.  Square 256 x 256 tiles leave
// the GPU's 256 CUs with partial rounds there: 204 tiles at 4352 x 3072 (52
// CUs idle for the whole kernel), 612 at 4352 x 9216 (a third round on 100
// CUs), and a 17th tile-row at 4352 x 12288 that needs a round of smaller,
// slower tiles.  A 272 x 192 tile (52224 outputs, 0.8 of a 256 x 256 one)
// gives exactly 256, 768 and 1024 tiles: whole rounds on every CU.
//
// Tile and waves.  The tile is 17 x 12 blocks of v_mfma_i32_16x16x64_i8
// (16 x 16 outputs, the whole 64-deep K-step in one instruction).  Four
// waves, one a SIMD, take 51 blocks each: wave (wm, wn) owns block columns
// 6 wn .. 6 wn + 5 and block rows 0-7 (wm = 0) or 9-16 (wm = 1), and shares
// block row 8 with its partner: wm = 0 takes its columns 0-2 there, wm = 1
// columns 3-5.  Every wave then issues 51 MFMAs and reads 15 fragments (9 of
// A, 6 of B) a K-step; a plain 2 x 2 split of the rows (144 / 128) would
// give 54 and 48 and hold the K-step at 54.  The accumulators are 204 AGPRs.
// The wave's half of the shared row makes wm a template parameter: each wave
// runs the loop of its half.
//
// The B fragment is the MFMA's first operand, so lane l holds output row
// l % 16 of a block and columns 4 (l / 16) .. + 3, as in the square kernels.
// Both fragments of a lane carry the same 16 K bytes (chunk l / 16 of the
// step's 64), so the product sums every k once whatever order the
// instruction pairs bytes in.
//
// The K ring.  Stage s holds A (272 rows x 64 bytes) then B (192 rows), 29
// KB; four stages.  K-step k runs on stage k % 4:
//   * wait for this wave's loads of K-step k + 1, then one barrier: K-step
//     k + 1 is in LDS for every wave, and every wave's reads of stage k % 4
//     (done during K-step k - 1) have completed;
//   * 51 MFMAs on the fragments read during K-step k - 1, with the 15 reads
//     of K-step k + 1's fragments and the loads of K-step k + 4 into stage
//     k % 4 placed between them.
// A K-step's 29 pieces of 16 rows x 64 bytes (contiguous 1 KB blocks in the
// K-tiled layout) are 4 whole A pieces, a quarter of the 17th and 3 B pieces
// per wave: eight load instructions for every wave, so the waits count alike
// on all of them.  The cursors move to the next tile for the loads of its
// K-step 0 (issued in K-step KT - 4, with the next tile's epilogue
// operands); after the last tile they point past the operands, whose range
// check returns zeros without touching memory.
//
// K direction.  A workgroup's odd tiles walk K downward.  With the tile
// order's groups of four tile rows, the 32 workgroups of an XCD keep the
// same eight B strips in every round at config 1 up, and the K-steps a round
// read last are the ones the XCD's L2 still holds when the next round
// starts: the L2 misses fall from 259 to 219 MB a call there.  The int32
// sums do not depend on the order.
//
// The epilogue converts one block row (16 rows x 96 or 48 columns) at a
// time, stages it in the wave's LDS area and stores whole 16-byte pieces.
#include "device_common.hpp"
#include "i8_gemm.hpp"
#include "persist_common.hpp"

// Tile-timeline hooks, empty in the library: a tracing build defines them to
// stamp the clocks per workgroup at the kernel's start, at each tile's start,
// K-loop end and epilogue end, and at the end.
#ifndef PHI_T272_STAMP
#define PHI_T272_STAMP(tile, point)
#define PHI_T272_TRACE_BEGIN
#define PHI_T272_TRACE_END
#endif

namespace phi_dev {

namespace {

using namespace persist;

// Output kinds: CKind's C_F32 / C_BF16 / C_I32, and the fp32 output into a
// gated residual stream, updated in place: C = fma(linear, gate[n], C), the
// reference's AddMul `a + b * c` (core/kernels/ops.cpp:80, after the
// projection at core/models/av_dit.cpp:1389) as NVRTC's --fmad=true
// contracts it.
constexpr int C_F32G = 3;
constexpr int TM = 272, TN = 192;      // output tile
constexpr int PK = 64, NSTG = 4;       // K bytes per stage, stages
constexpr int BOFF = TM * PK;          // B's offset within a stage
constexpr int STG = (TM + TN) * PK;    // 29696 bytes a stage
constexpr int NA = 5, NBL = 3;         // loads a wave issues per K-step: A (4 whole + a quarter), B
constexpr int NLD = NA + NBL;
constexpr int NE = 3;                  // epilogue-operand loads a wave issues per tile
// Epilogue operands of one tile (one area per tile parity): row scales
// (272 used of 320), column scales, bias (fp32 words or bf16 pairs), and
// the landing place of loads that fetch nothing.
constexpr int E_SA = 0, E_SB = 1280, E_BZ = 2048, E_PAD = 2816, EB = 3072;
// Epilogue staging: 16 rows of 12 16-byte pieces (6 blocks x 32 bytes of
// bf16, or 3 blocks x 64 bytes of fp32 / int32) at a pitch of 192 bytes, piece
// c of row r in slot (c + r / 4) % 12.  The read-back takes the pieces in row
// order, so 16 consecutive lanes read 16 consecutive slots of the 192-byte
// rows (distinct bank windows), and each store instruction writes rows of 192
// contiguous bytes; the rotation spreads a block's writes from 16 rows (whose
// pitch alone repeats every four rows) over every bank once.
constexpr int SP = 192, SBYTES = 16 * SP;
__device__ __forceinline__ int stage_slot(int r, int c) {
    const int x = c + (r >> 2);
    return x >= 12 ? x - 12 : x;
}
// Stores a wave issues in an epilogue: bf16 8 full block rows x 3 + the shared
// one 2; fp32 / int32 8 x 6 + 3.  Every one is issued (columns past N go to
// an offset the range check drops).
template <int CK>
struct Nst {
    static constexpr int v = CK == C_BF16 ? 8 * 3 + 2 : 8 * 6 + 3;
};
// Waits: this wave's memory operations issued after its loads of K-step
// k + 1 are those of K-steps k + 2 and k + 3 (2 NLD), plus the epilogue's
// stores in a tile's first three K-steps, plus the next tile's
// epilogue-operand loads (issued after K-step KT - 4's loads) in K-steps
// KT - 3 .. KT - 1.
constexpr int VW = 2 * NLD;

struct Frag {
    v4i a[9], b[6];
};

struct Acc {
    v4i f[8][6];  // the wave's full block rows
    v4i s[3];     // its half of the shared block row
};

struct Tw {
    int lane, wave, wn;
    int oF;          // this lane's byte offset within a 16-row piece (row l % 16, chunk l / 16, swizzled)
    int8_t* lds;     // stage 0 (opaque)
    int8_t* le;      // epilogue-operand areas
    int8_t* lc;      // this wave's staging area
    __amdgpu_buffer_rsrc_t rA, rB;
    // Running source offsets (this lane's byte of the piece included) and
    // K-step strides of the wave's pieces, in VGPRs: wave-uniform, but the
    // SGPRs cannot hold them beside the rest (they spilled there).
    int offA[NA], stA[NA], offB[NBL], stB[NBL];
    int cm0, cn0;    // the cursors' tile
};

// LDS slot of 16-byte chunk c of row r (r within a 16-row piece):
// c ^ ((r >> 1) & 3).  The fragment reads (row l % 16, chunk l / 16) of every
// 16-lane group then meet no bank conflict on gfx950, as measured; the K-tiled
// layout's own swizzle (c ^ ((r >> 2) & 3), the square kernels' LDS layout)
// costs two extra clocks on every one of these reads.  The DMA keeps its
// contiguous 1 KB sources: each lane fetches, from within the same 64-byte
// row, the chunk its LDS slot holds.
__device__ __forceinline__ int lds_slot(int r, int c) { return c ^ ((r >> 1) & 3); }
// Byte offset, within a 16-row piece of the K-tiled layout, of the bytes the
// DMA lane writing LDS piece byte q (a multiple of 4) fetches.
__device__ __forceinline__ int dma_src(int q) {
    const int r = q >> 6, slot = (q >> 4) & 3, c = slot ^ ((r >> 1) & 3);
    return r * 64 + 16 * (c ^ ((r >> 2) & 3)) + (q & 15);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t whole_rsrc(const void* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, bytes, kRsrcWord3);
}

// K-step 0 of the 16-row piece at row r of a K-tiled operand of `rows` rows:
// its byte offset and K-step stride.  A piece wholly past the operand reads
// from its end: the range check returns zeros (those rows only feed outputs
// the epilogue drops).
__device__ __forceinline__ void piece_at(int r, int rows, int K, int& off, int& st) {
    const bool in = r < rows;
    const int s = r >> 8, h = min(256, rows - (s << 8));
    off = in ? s * 256 * K + (r & 255) * PK : rows * K;
    st = in ? h * PK : 0;
}

// Row-major operand (row pitch ld bytes): the DMA lane writing byte q of the
// LDS piece at row r fetches row r + q / 64 at the chunk its slot holds, K-step
// 0, and steps 64 bytes a K-step.  A row past the operand points at its end
// with no step: the range check returns zeros (such rows only feed outputs
// the epilogue drops).
__device__ __forceinline__ void piece_rm(int r, int q, int rows, int ld, int& off, int& st) {
    const int rr = q >> 6, c = ((q >> 4) & 3) ^ ((rr >> 1) & 3), row = r + rr;
    const bool in = row < rows;
    off = in ? row * ld + 16 * c + (q & 15) : rows * ld;
    st = in ? PK : 0;
}

// The cursor of the piece at row r for the DMA lane writing its byte q.
__device__ __forceinline__ void piece_lane(const GemmParams& p, bool a, int r, int q, int& off, int& st) {
    const int rows = a ? p.M : p.N;
    if (p.kt && (a || !p.b_rm)) {
        piece_at(r, rows, p.K, off, st);
        off += dma_src(q);
    } else {
        piece_rm(r, q, rows, (int)(a ? p.lda : p.ldb), off, st);
    }
}

// Cursors onto the tile at (m0, n0), K-step 0; valid = false: onto nothing.
// rev: the tile walks K downward, from its last K-step (the cursors start
// there and step back); the int32 sums are the same in either order.
__device__ __forceinline__ void cursor_to(Tw& w, const GemmParams& p, int m0, int n0, bool valid, bool rev) {
#pragma unroll
    for (int j = 0; j < 4; j++)
        piece_lane(p, true, valid ? m0 + 16 * (w.wave + 4 * j) : p.M, w.lane * 16, w.offA[j], w.stA[j]);
    // this wave's quarter of the 17th piece
    piece_lane(p, true, valid ? m0 + 256 : p.M, 256 * w.wave + w.lane * 4, w.offA[4], w.stA[4]);
#pragma unroll
    for (int j = 0; j < NBL; j++)
        piece_lane(p, false, valid ? n0 + 16 * (w.wave + 4 * j) : p.N, w.lane * 16, w.offB[j], w.stB[j]);
    if (rev) {
        const int last = p.K / PK - 1;
#pragma unroll
        for (int j = 0; j < NA; j++) {
            w.offA[j] += last * w.stA[j];
            w.stA[j] = -w.stA[j];
        }
#pragma unroll
        for (int j = 0; j < NBL; j++) {
            w.offB[j] += last * w.stB[j];
            w.stB[j] = -w.stB[j];
        }
    }
#pragma unroll
    for (int j = 0; j < NA; j++) asm volatile("" : "+v"(w.offA[j]), "+v"(w.stA[j]));
#pragma unroll
    for (int j = 0; j < NBL; j++) asm volatile("" : "+v"(w.offB[j]), "+v"(w.stB[j]));
    if (valid) {
        w.cm0 = m0;
        w.cn0 = n0;
    }
}

// Load j (0-3 whole A pieces, 4 the quarter, 5-7 B pieces) of the cursors'
// K-step into the stage at d (this wave's first A piece) / dq (its quarter);
// the piece's cursor advances.
template <int J>
__device__ __forceinline__ void load1(Tw& w, int8_t* d, int8_t* dq) {
    if constexpr (J < 4) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(w.rA, (lptr_t)(d + 4096 * J), 16, w.offA[J], 0, 0, 0);
        w.offA[J] += w.stA[J];
    } else if constexpr (J == 4) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(w.rA, (lptr_t)dq, 4, w.offA[4], 0, 0, 0);
        w.offA[4] += w.stA[4];
    } else {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(w.rB, (lptr_t)(d + BOFF + 4096 * (J - 5)), 16, w.offB[J - 5], 0, 0,
                                                 0);
        w.offB[J - 5] += w.stB[J - 5];
    }
}

// The destinations are computed in the K-step from an opaque base: hoisted
// out of the loop, the 32 of the four stages would sit in SGPRs and spill.
template <int ST>
__device__ __forceinline__ int8_t* load_base(const Tw& w) {
    return opaque_lds(w.lds + ST * STG + 1024 * w.wave);
}
template <int ST>
__device__ __forceinline__ int8_t* quarter_base(const Tw& w) {
    return opaque_lds(w.lds + ST * STG + 16 * 1024 + 256 * w.wave);
}

// The cursors' whole K-step into stage ST (the prologue's loads).
template <int ST>
__device__ __forceinline__ void load_step(Tw& w) {
    int8_t* d = load_base<ST>(w);
    int8_t* dq = quarter_base<ST>(w);
    load1<0>(w, d, dq);
    load1<1>(w, d, dq);
    load1<2>(w, d, dq);
    load1<3>(w, d, dq);
    load1<4>(w, d, dq);
    load1<5>(w, d, dq);
    load1<6>(w, d, dq);
    load1<7>(w, d, dq);
}

// The epilogue operands of the cursors' tile into area le: twelve 256-byte
// slots (row scales 0-4, column scales 5-7, bias 8-10, nothing 11), three a
// wave, one dword a lane.  Past M or N, or with an operand absent (or the
// column scale a scalar, read in the epilogue instead), a slot's source range
// is short or empty and its words read as zero.
__device__ __forceinline__ void issue_epi(const Tw& w, const GemmParams& p, int8_t* le) {
    const int rows = min(TM, p.M - w.cm0), cols = min(TN, p.N - w.cn0);
    const int bsz = p.bias_kind == BIAS_F32 ? 4 : 2;
    const bool per_col = p.sB && !p.sb_scalar, has_bias = p.bias_kind != BIAS_NONE;
    const int8_t* sa = p.sA ? (const int8_t*)(p.sA + w.cm0) : p.A;
    const int8_t* sb = per_col ? (const int8_t*)(p.sB + w.cn0) : p.A;
    const int8_t* bz = has_bias ? (const int8_t*)p.bias + (int64_t)w.cn0 * bsz : p.A;
    const int na = p.sA ? rows * 4 : 0, nb = per_col ? cols * 4 : 0, nz = has_bias ? cols * bsz : 0;
#pragma unroll
    for (int q = 0; q < NE; q++) {
        // Selects on wave-uniform values: no branch inside the K-step's
        // scheduled block.
        const int s = 3 * w.wave + q;
        const bool isA = s < 5, isB = !isA && s < 8, isZ = !isA && !isB && s < 11;
        const int8_t* base = isA ? sa : isB ? sb : isZ ? bz : p.A;
        const int bytes = isA ? na : isB ? nb : isZ ? nz : 0;
        const int idx = isA ? s : isB ? s - 5 : isZ ? s - 8 : 0;
        const int dst = (isA ? E_SA : isB ? E_SB : isZ ? E_BZ : E_PAD) + 256 * idx;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(whole_rsrc(base, bytes), (lptr_t)(le + dst), 4, w.lane * 4, 256 * idx,
                                                 0, 0);
    }
}

// Fragments of stage ST: A block rows 8 WM .. 8 WM + 8, B block columns
// 6 wn .. 6 wn + 5.
// Fragment bases of stage ST for this lane: A block rows 8 WM .., B block
// columns 6 wn ...  The wave-uniform part is laundered through an SGPR in the
// K-step: otherwise the compiler hoists one address register per read (stage
// offsets past 64 KB do not fit the 16-bit ds_read offset), some 40 VGPRs.
template <int WM, int ST>
__device__ __forceinline__ const int8_t* frag_a(const Tw& w) {
    return opaque_lds(w.lds + ST * STG + 1024 * 8 * WM) + w.oF;
}
template <int WM, int ST>
__device__ __forceinline__ const int8_t* frag_b(const Tw& w) {
    return opaque_lds(w.lds + ST * STG + BOFF + 6144 * w.wn) + w.oF;
}

// Fragment read J: 0-8 the A block rows, 9-14 the B block columns.
template <int J>
__device__ __forceinline__ void read1(Frag& f, const int8_t* a, const int8_t* b) {
    if constexpr (J < 9) f.a[J] = *(const v4i*)(a + 1024 * J);
    else f.b[J - 9] = *(const v4i*)(b + 1024 * (J - 9));
}

template <int WM, int ST>
__device__ __forceinline__ void frag(Frag& f, const Tw& w) {
    const int8_t* a = frag_a<WM, ST>(w);
    const int8_t* b = frag_b<WM, ST>(w);
#pragma unroll
    for (int i = 0; i < 9; i++) f.a[i] = *(const v4i*)(a + 1024 * i);
#pragma unroll
    for (int c = 0; c < 6; c++) f.b[c] = *(const v4i*)(b + 1024 * c);
}

// MFMA q (0 .. 50) of the wave's K-step.  wm = 0: q < 48 is full row q / 6
// (A fragment q / 6), column q % 6; q >= 48 the shared row (A fragment 8),
// columns 0-2.  wm = 1: q < 3 the shared row (A fragment 0), columns 3-5;
// then full rows (A fragments 1-8).
// One MFMA with its accumulator tied in AGPRs (inline asm): the register
// allocator can then neither rotate the accumulators through spare AGPRs nor
// move them between iterations.  The compiler does not see the instruction,
// so its hazard tracking does not cover the accumulator's first VALU read
// after the last MFMA: mfma_drain() gives those wait states explicitly.
__device__ __forceinline__ void mfma_tied(v4i& acc, const v4i& b, const v4i& a) {
    asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(acc) : "v"(b), "v"(a));
}
__device__ __forceinline__ void mfma_first(v4i& acc, const v4i& b, const v4i& a) {
    asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, 0" : "=a"(acc) : "v"(b), "v"(a));
}
// Wait states after the last MFMA before any VALU instruction reads its
// accumulators: 18, more than the four-pass instruction's requirement.
__device__ __forceinline__ void mfma_drain() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 1" ::: "memory"); }

// Block of the wave's full block rows that MFMA q of a K-step updates.  The
// rows run in alternating column order, and the half row sits at the end
// (WM 0) or the start (WM 1) in the order that joins it: every change of
// A fragment keeps the B fragment of the MFMA before it, so the operands
// that switch from one MFMA to the next are fewer (the MFMA array's draw,
// and with it the board clock, follows how many operand bits toggle).
template <int WM, int Q>
struct Blk {
    static constexpr int q = WM == 0 ? Q : Q - 3, r = q / 6;
    static constexpr int c = ((r + WM) & 1) ? 5 - q % 6 : q % 6;
};

template <int WM, int Q, bool Z>
__device__ __forceinline__ void mma1t(const Frag& f, Acc& acc) {
    if constexpr (WM == 0 && Q >= 48) {
        constexpr int c = Q - 48;
        if constexpr (Z) mfma_first(acc.s[c], f.b[c], f.a[8]);
        else mfma_tied(acc.s[c], f.b[c], f.a[8]);
    } else if constexpr (WM == 1 && Q < 3) {
        if constexpr (Z) mfma_first(acc.s[Q], f.b[3 + Q], f.a[0]);
        else mfma_tied(acc.s[Q], f.b[3 + Q], f.a[0]);
    } else {
        constexpr int r = Blk<WM, Q>::r, c = Blk<WM, Q>::c;
        if constexpr (Z) mfma_first(acc.f[r][c], f.b[c], f.a[r + WM]);
        else mfma_tied(acc.f[r][c], f.b[c], f.a[r + WM]);
    }
}

template <int WM, int Q, bool Z>
__device__ __forceinline__ void mma1(const Frag& f, Acc& acc) {
    if constexpr (WM == 0 && Q >= 48) {
        constexpr int c = Q - 48;
        acc.s[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(f.b[c], f.a[8], Z ? v4i{} : acc.s[c], 0, 0, 0);
    } else if constexpr (WM == 1 && Q < 3) {
        acc.s[Q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(f.b[3 + Q], f.a[0], Z ? v4i{} : acc.s[Q], 0, 0, 0);
    } else {
        constexpr int r = Blk<WM, Q>::r, c = Blk<WM, Q>::c;
        acc.f[r][c] =
            __builtin_amdgcn_mfma_i32_16x16x64_i8(f.b[c], f.a[r + WM], Z ? v4i{} : acc.f[r][c], 0, 0, 0);
    }
}

struct NextTile {
    int m0, n0;
    bool valid, rev;  // rev: its K-loop walks K downward
};

// The K-step's instruction order, fixed: MFMA q, then the fragment read and
// the load that slot q carries, then a scheduling fence.  Reads of K-step
// k + 1's fragments go to slots 2, 4, .., 30, the loads of K-step k + 4 to
// slots 4, 10, .., 46, and (K-step KT - 4) the next tile's epilogue operands
// to slot 48.  Left to the scheduler, an interleave of the same instructions
// made the register allocator rotate the accumulators through spare AGPRs and
// VGPRs, with copies and s_nop waits in every K-step.
template <int Q>
struct Slot {
    static constexpr int read = Q >= 2 && Q <= 30 && Q % 2 == 0 ? (Q - 2) / 2 : -1;
    static constexpr int load = Q >= 4 && (Q - 4) % 6 == 0 && (Q - 4) / 6 < NLD ? (Q - 4) / 6 : -1;
};

struct StepPtrs {
    const int8_t *ra, *rb;  // fragment bases of the next K-step's stage
    int8_t *d, *dq;         // load destinations in this K-step's stage
    int8_t* ln;             // the next tile's epilogue-operand area
};

template <int WM, bool Z, bool SW, int Q>
__device__ __forceinline__ void kslots(const Frag& f, Frag& g, Acc& acc, Tw& w, const GemmParams& p,
                                       const StepPtrs& sp) {
    if constexpr (Q < 51) {
        mma1<WM, Q, Z>(f, acc);
        if constexpr (Slot<Q>::read >= 0) read1<Slot<Q>::read>(g, sp.ra, sp.rb);
        if constexpr (Slot<Q>::load >= 0) load1<Slot<Q>::load>(w, sp.d, sp.dq);
        if constexpr (SW && Q == 48) issue_epi(w, p, sp.ln);
        __builtin_amdgcn_sched_barrier(0);
        kslots<WM, Z, SW, Q + 1>(f, g, acc, w, p, sp);
    }
}

// K-step k on stage S = k % 4, on the fragments f; K-step k + 1's are read
// into g.  VWT: the wait's allowance.  Z: the tile's first K-step.  SW: the
// cursors move to the next tile first (K-step KT - 4), and that tile's
// epilogue operands are loaded into area ln after the K-step's loads.
template <int WM, int S, int VWT, bool Z, bool SW>
__device__ __forceinline__ void kstep(const Frag& f, Frag& g, Acc& acc, Tw& w, const GemmParams& p,
                                      const NextTile& nt, int8_t* ln) {
    if constexpr (SW) cursor_to(w, p, nt.m0, nt.n0, nt.valid, nt.rev);
    wait_vm_lgkm0<VWT>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    StepPtrs sp;
    sp.ra = frag_a<WM, (S + 1) % NSTG>(w);
    sp.rb = frag_b<WM, (S + 1) % NSTG>(w);
    sp.d = load_base<S>(w);
    sp.dq = quarter_base<S>(w);
    sp.ln = ln;
    kslots<WM, Z, SW, 0>(f, g, acc, w, p, sp);
}

// ---------------------------------------------------------------------------
// The W4 operand (asym_w4a8_int8): B is packed 4-bit codes [N, ldb] (low
// nibble = even column, as the checkpoint stores them) with the per-(row,
// group) 16-entry int8 table [N, K / group, 16] of the load-time prepare
// (w4a8.hip).  The int32 accumulators are those of expand-then-W8A8 exactly:
// every code becomes the int8 the expansion writes (the reference's
// w4a8_to_i8 then int8 GEMM, core/kernels/w4a8_expand.cpp:151-258).
//
// The codes and tables are DMA'd into LDS rings and expanded there, once per
// workgroup, into an int8 B area the MFMA fragments are read from:
//   * LDS: A stages 4 x 17 KB | code stages 4 x 6 KB (192 rows x 32 bytes) |
//     table stages 4 x 3 KB (192 rows x 16 bytes) | int8 B areas 2 x 12 KB,
//     128 KB.  A K-step's B bytes in LDS are half the int8 kernel's.
//   * K-step k: the loads of A of K-step k + 4 and of the codes and tables of
//     K-step k + 5; the expansion of K-step k + 2's codes (thread t: rows
//     t / 4 + 64 i, i < 3, 16 columns 16 (t % 4) ..; three 8-byte code reads,
//     three table reads, 12 v_perm-based lookups, six 8-byte writes) into
//     area k % 2; the fragment reads of K-step k + 1 (A from its stage, B
//     from area (k + 1) % 2, expanded during K-step k - 1).  The K-step's one
//     barrier orders all of it: its wait covers the loads of K-step k - 3
//     (A of k + 1, codes and tables of k + 2), and every wave's reads of the
//     stages and area it overwrites finished before it.
//   * Each wave issues 11 loads a K-step: its 5 A pieces, one whole 1 KB code
//     piece (32 rows) and two 256-byte quarters, and three 256-byte table
//     quarters (16 rows each).  The code pieces are gathered row by row from
//     the row-major codes (32 bytes a row and K-step); rows past N read past
//     the resource and come back zero.
// Expanding once per workgroup instead of once per wave that reads a B
// fragment halves the lookups (each B fragment is read by two waves), and the
// lookups are ~110 VALU instructions a wave a K-step beside its 51 MFMAs.
constexpr int W4_CS = TN * 32, W4_LS = TN * 16, W4_BS = TN * PK;  // code, table, int8 B stage bytes
constexpr int W4_C = NSTG * BOFF, W4_L = W4_C + NSTG * W4_CS, W4_B = W4_L + NSTG * W4_LS;
constexpr int W4_LDS = W4_B + 2 * W4_BS;  // 131072
constexpr int NC = 3, NTB = 3, NLD4 = NA + NC + NTB;  // loads a wave issues per K-step
constexpr int VW4 = 2 * NLD4;

// The code and table cursors: this lane's source byte of each of the wave's
// code and table pieces at K-step 0, the cursors' K-step, and the strides of
// the scalar offset: codes advance cstep bytes a K-step (32 on the
// checkpoint's rows, 6144 in the band layout), tables lstep bytes a group (16
// or 3072).
struct W4c {
    __amdgpu_buffer_rsrc_t rC, rL;
    int offC[NC], offL[NTB];
    int kc, cstep, lstep;
};

// The band layout (p.w4_banded, phi_hip_w4a8_pack_banded): B rows in bands of
// TN = 192; band b's 32 code bytes of every row for K-step s are one block of
// 6144 bytes at (b KT + s) 6144, row r at 32 r; after all code blocks, band
// b's tables of group g are one block of 3072 bytes at (b G + g) 3072, row r
// at 16 r.  Rows past N are zero.  A block is a stage's code or table area
// byte for byte, so every DMA a wave issues reads contiguous bytes; on the
// checkpoint's rows each one gathers 32 rows 3 KB apart (at config 2 that
// costs about 22 us of a 151 us step, measured with contiguous sources).
__device__ __forceinline__ int64_t w4_banded_code_bytes(int N, int K) {
    return (int64_t)((N + TN - 1) / TN) * (K / PK) * (TN * 32);
}

// Code and table cursors onto the tile with B rows n0 .., K-step 0; valid =
// false: onto nothing (every source past the resources).
__device__ __forceinline__ void w4_cursor_to(W4c& c, const Tw& w, const GemmParams& p, int n0, bool valid) {
    c.kc = 0;
    if (p.w4_banded) {
        const int KT = p.K / PK, G = (int)p.lut_groups, bands = (p.N + TN - 1) / TN;
        const int b = valid ? n0 / TN : bands;  // past the last band: past both resources
        const int cb = b * KT * (TN * 32), lb = b * G * (TN * 16);
        c.offC[0] = cb + 1024 * w.wave + 16 * w.lane;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int qi = 2 * w.wave + i;
            c.offC[1 + i] = cb + 4096 + 1024 * (qi >> 2) + 256 * (qi & 3) + 4 * w.lane;
        }
#pragma unroll
        for (int i = 0; i < NTB; i++) c.offL[i] = lb + 256 * (3 * w.wave + i) + 4 * w.lane;
        c.cstep = TN * 32;
        c.lstep = TN * 16;
#pragma unroll
        for (int i = 0; i < NC; i++) asm volatile("" : "+v"(c.offC[i]));
#pragma unroll
        for (int i = 0; i < NTB; i++) asm volatile("" : "+v"(c.offL[i]));
        return;
    }
    const int N = p.N, ldb = (int)p.ldb, g16 = (int)p.lut_groups * 16;
    const int base = valid ? n0 : N;
    c.cstep = 32;
    c.lstep = 16;
    {
        const int n = base + 32 * w.wave + (w.lane >> 1);  // whole piece w: rows 32 w .., 16 bytes a lane
        c.offC[0] = n < N ? n * ldb + 16 * (w.lane & 1) : N * ldb;
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int qi = 2 * w.wave + i;  // quarter qi of pieces 4-5: 8 rows, 4 bytes a lane
        const int n = base + 128 + 32 * (qi >> 2) + 8 * (qi & 3) + (w.lane >> 3);
        c.offC[1 + i] = n < N ? n * ldb + 4 * (w.lane & 7) : N * ldb;
    }
#pragma unroll
    for (int i = 0; i < NTB; i++) {
        const int n = base + 16 * (3 * w.wave + i) + (w.lane >> 2);  // table quarter: 16 rows, 4 bytes a lane
        c.offL[i] = n < N ? n * g16 + 4 * (w.lane & 3) : N * g16;
    }
#pragma unroll
    for (int i = 0; i < NC; i++) asm volatile("" : "+v"(c.offC[i]));
#pragma unroll
    for (int i = 0; i < NTB; i++) asm volatile("" : "+v"(c.offL[i]));
}

// W4 stage bases (opaque, computed in the K-step like the int8 ones).
template <int ST>
__device__ __forceinline__ int8_t* w4_a_base(const Tw& w) {
    return opaque_lds(w.lds + ST * BOFF + 1024 * w.wave);
}
template <int ST>
__device__ __forceinline__ int8_t* w4_a_quarter(const Tw& w) {
    return opaque_lds(w.lds + ST * BOFF + 16 * 1024 + 256 * w.wave);
}

// Load J of the code and table cursors' K-step: 0 the whole code piece, 1-2
// the code quarters, 3-5 the table quarters, into code stage CS / table
// stage CS.  The K-step advance rides in the scalar offset.
template <int CS, int J>
__device__ __forceinline__ void w4_load1(const W4c& c, const Tw& w, const GemmParams& p) {
    if constexpr (J == 0) {
        int8_t* d = opaque_lds(w.lds + W4_C + CS * W4_CS + 1024 * w.wave);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rC, (lptr_t)d, 16, c.offC[0], c.cstep * c.kc, 0, 0);
    } else if constexpr (J < 3) {
        const int qi = 2 * w.wave + (J - 1);
        int8_t* d = opaque_lds(w.lds + W4_C + CS * W4_CS + 4096 + 1024 * (qi >> 2) + 256 * (qi & 3));
        __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rC, (lptr_t)d, 4, c.offC[J], c.cstep * c.kc, 0, 0);
    } else {
        int8_t* d = opaque_lds(w.lds + W4_L + CS * W4_LS + 256 * (3 * w.wave + (J - 3)));
        const int goff = ((c.kc * PK) >> p.group_shift) * c.lstep;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rL, (lptr_t)d, 4, c.offL[J - 3], goff, 0, 0);
    }
}

// One expansion unit's state: 16 codes of one row, its table, a lookup's
// selection mask, and the even and odd columns' words of the current 8 codes.
struct W4u {
    u32x2 code;
    u32x4 tab;
    uint32_t m, ev, od;
    u32x2 lo;  // code word 0's 8 output bytes, written with word 1's as one 16-byte chunk
};

// Piece P (0 .. 10) of expansion unit U (thread t: row t / 4 + 64 U, columns
// 16 (t % 4) ..).  0: the reads.  Then for each code word h (8 codes): the
// even columns' lookup (mask, then the v_perm pair and select: lut4b split in
// two), the odd columns' (the same on the high nibbles), and the interleave
// of the two into 8 output bytes; word 1's piece writes both words' bytes
// into int8 area bo as one 16-byte chunk (two 8-byte writes a word took 63
// clocks more a K-step, 1623 against 1560).  No MFMA slot carries more than
// five VALU instructions, and a unit keeps eleven registers.
// This thread's byte offsets of unit 0 in a code stage, a table stage and an
// int8 B area (row t / 4, 16-byte chunk t % 4); unit u adds 64 u rows, an
// immediate offset.
struct W4o {
    int c, t, b;
};

__device__ __forceinline__ W4o w4_lane_offsets(const Tw& w) {
    const int t = 64 * w.wave + w.lane, r = t >> 2, ch = t & 3;
    W4o o;
    o.c = r * 32 + 8 * ch;
    o.t = r * 16;
    o.b = r * 64 + 16 * lds_slot(r & 15, ch);
    asm volatile("" : "+v"(o.c), "+v"(o.t), "+v"(o.b));
    return o;
}

template <int P>
__device__ __forceinline__ void w4_piece(W4u& u, int U, const W4o& lo4, const int8_t* cs, const int8_t* ls,
                                         int8_t* bo) {
    if constexpr (P == 0) {
        u.code = *(const u32x2*)(cs + lo4.c + 64 * 32 * U);
        u.tab = *(const u32x4*)(ls + lo4.t + 64 * 16 * U);
    } else {
        constexpr int h = (P - 1) / 5, k = (P - 1) % 5;  // code word, step within it
        const uint32_t x = u.code[h];
        if constexpr (k == 0 || k == 2) {
            // bit 3 of each code (bit 7 of the byte for the odd columns) picks
            // entries 8-15: selector 0x0d gives 0xff, 0x0c gives 0x00
            const uint32_t b = (k == 0 ? x >> 3 : x >> 7) & 0x01010101u;
            u.m = __builtin_amdgcn_perm(0u, 0u, b | 0x0c0c0c0cu);
        } else if constexpr (k == 1 || k == 3) {
            const uint32_t sel = (k == 1 ? x : x >> 4) & 0x07070707u;
            const uint32_t lo = __builtin_amdgcn_perm(u.tab[1], u.tab[0], sel);
            const uint32_t hi = __builtin_amdgcn_perm(u.tab[3], u.tab[2], sel);
            const uint32_t v = (hi & u.m) | (lo & ~u.m);
            if constexpr (k == 1) u.ev = v;
            else u.od = v;
        } else {
            // ev holds columns 0, 2, 4, 6 and od columns 1, 3, 5, 7: interleave.
            const u32x2 o = {__builtin_amdgcn_perm(u.od, u.ev, 0x05010400u),
                             __builtin_amdgcn_perm(u.od, u.ev, 0x07030602u)};
            if constexpr (h == 0) u.lo = o;
            else *(u32x4*)(bo + lo4.b + 64 * 64 * U) = u32x4{u.lo[0], u.lo[1], o[0], o[1]};
        }
    }
}

// The W4 K-step's fixed order: MFMA q, then what slot q carries.
//   slots 1-15:             the 15 fragment reads of K-step k + 1
//   slots 2, 6, .. 42:      the 11 loads (A 0-4, then codes and tables 0-5)
//   slots 0, 12, 24:        unit u's reads (piece 0), eight slots before
//   slots 8 + 12 u .. + 9:  its pieces 1-10
//   slot 48:                (K-step KT - 4) the next tile's epilogue operands
template <int Q>
struct Slot4 {
    static constexpr int read = Q >= 1 && Q <= 15 ? Q - 1 : -1;
    static constexpr int load = Q >= 2 && (Q - 2) % 4 == 0 && (Q - 2) / 4 < NLD4 ? (Q - 2) / 4 : -1;
    static constexpr int ureads = Q <= 24 && Q % 12 == 0 ? Q / 12 : -1;
    static constexpr int piece =  // 10 u + (p - 1)
        Q >= 8 && (Q - 8) / 12 < 3 && (Q - 8) % 12 < 10 ? 10 * ((Q - 8) / 12) + (Q - 8) % 12 : -1;
};

struct StepPtrs4 {
    const int8_t *ra, *rb;  // fragment bases of K-step k + 1 (A stage, int8 B area)
    int8_t *da, *dq;        // A load destinations in this K-step's stage
    const int8_t *cs, *ls;  // code and table stages of K-step k + 2
    int8_t* bo;             // int8 B area being written
    int8_t* ln;             // the next tile's epilogue-operand area
};

template <int WM, int CS, bool Z, bool SW, int Q>
__device__ __forceinline__ void kslots4(const Frag& f, Frag& g, Acc& acc, Tw& w, W4c& c, W4u (&u)[3],
                                        const W4o& lo4, const GemmParams& p, const StepPtrs4& sp) {
    if constexpr (Q < 51) {
        mma1t<WM, Q, Z>(f, acc);
        if constexpr (Slot4<Q>::ureads >= 0) {
            constexpr int U = Slot4<Q>::ureads;
            w4_piece<0>(u[U], U, lo4, sp.cs, sp.ls, sp.bo);
        }
        if constexpr (Slot4<Q>::read >= 0) read1<Slot4<Q>::read>(g, sp.ra, sp.rb);
        if constexpr (Slot4<Q>::load >= 0) {
            constexpr int L = Slot4<Q>::load;
            if constexpr (L < NA) load1<L>(w, sp.da, sp.dq);
            else w4_load1<CS, L - NA>(c, w, p);
        }
        if constexpr (Slot4<Q>::piece >= 0) {
            constexpr int U = Slot4<Q>::piece / 10, P = Slot4<Q>::piece % 10 + 1;
            w4_piece<P>(u[U], U, lo4, sp.cs, sp.ls, sp.bo);
        }
        if constexpr (SW && Q == 48) issue_epi(w, p, sp.ln);
        __builtin_amdgcn_sched_barrier(0);
        kslots4<WM, CS, Z, SW, Q + 1>(f, g, acc, w, c, u, lo4, p, sp);
    }
}

// W4 K-step k on A stage S = k % 4.  SWA: the A cursor moves to the next tile
// first (K-step KT - 4), with that tile's epilogue operands after the loads;
// SWC: the code and table cursors move to it first (K-step KT - 5).
template <int WM, int S, int VWT, bool Z, bool SWA, bool SWC>
__device__ __forceinline__ void kstep4(const Frag& f, Frag& g, Acc& acc, Tw& w, W4c& c, const W4o& lo4,
                                       const GemmParams& p, const NextTile& nt, int8_t* ln) {
    if constexpr (SWA) cursor_to(w, p, nt.m0, nt.n0, nt.valid, false);
    if constexpr (SWC) w4_cursor_to(c, w, p, nt.n0, nt.valid);
    wait_vm_lgkm0<VWT>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    StepPtrs4 sp;
    sp.ra = opaque_lds(w.lds + ((S + 1) % NSTG) * BOFF + 1024 * 8 * WM) + w.oF;
    sp.rb = opaque_lds(w.lds + W4_B + ((S + 1) % 2) * W4_BS + 6144 * w.wn) + w.oF;
    sp.da = w4_a_base<S>(w);
    sp.dq = w4_a_quarter<S>(w);
    sp.cs = opaque_lds(w.lds + W4_C + ((S + 2) % NSTG) * W4_CS);
    sp.ls = opaque_lds(w.lds + W4_L + ((S + 2) % NSTG) * W4_LS);
    sp.bo = opaque_lds(w.lds + W4_B + (S % 2) * W4_BS);
    sp.ln = ln;
    W4u u[3];
    kslots4<WM, (S + 1) % NSTG, Z, SWA, 0>(f, g, acc, w, c, u, lo4, p, sp);
    c.kc++;
}

// Column operands of this lane: columns 16 c + 4 (l / 16) .. + 3 of the
// wave's 96 (c = 0 .. 5).  The bias area holds bf16 pairs or fp32 words (zeros
// without a bias); both views are read and the uniform format selects.
struct ColOps {
    v4f sb[6], bz[6];
};

// Block row R (0 .. 8) of the wave's epilogue: tile block row 8 WM + R; the
// shared one (R = 8 for wm = 0, R = 0 for wm = 1) holds wave column blocks
// 3 WM .. 3 WM + 2.  fp32 / int32: convert three blocks (192 bytes a row),
// write the wave's staging rows, read them back as 16-byte pieces (piece x:
// row x / 12, piece x % 12 of the row) and store.
template <int WM, int CK, int R>
__device__ __forceinline__ void epi_row(Acc& acc, const ColOps& co, const GemmParams& p, const Tw& w,
                                        const int8_t* e, const __amdgpu_buffer_rsrc_t& rs,
                                        const __amdgpu_buffer_rsrc_t& rg, int pitch, int colw) {
    static_assert(CK != C_BF16, "bf16 takes the pipelined rows");
    constexpr bool gated = CK == C_F32G;
    constexpr bool shared = WM == 0 ? R == 8 : R == 0;
    constexpr int g = 8 * WM + R;          // block row in the tile
    constexpr int c0 = shared ? 3 * WM : 0;  // first wave column block
    constexpr int nb = shared ? 3 : 6;
    constexpr int fr = WM == 0 ? R : R - 1;  // full-row index (unused for the shared row)
    const int lr = w.lane & 15, lg = w.lane >> 4;
    int8_t* lc = w.lc;
    const float sa = CK != C_I32 ? *(const float*)(e + E_SA + (16 * g + lr) * 4) : 0.0f;
    // Gated: the residual pieces and the gate columns a group of three blocks
    // stores, fetched before its conversion so their latency overlaps it.
    u32x4 res[3], gts[3];
#pragma unroll
    for (int c = 0; c < nb; c++) {
        if constexpr (gated) {
            if (c % 3 == 0) {
#pragma unroll
                for (int t = 0; t < 3; t++) {
                    const int x = w.lane + 64 * t, rr = x / 12, ch = x - 12 * rr;
                    const int col = colw + 16 * (c0 + c) + 4 * ch;
                    res[t] = __builtin_amdgcn_raw_buffer_load_b128(
                        rs, col < p.N ? (16 * g + rr) * pitch + col * 4 : kDropOffset, 0, 0);
                    gts[t] = __builtin_amdgcn_raw_buffer_load_b128(rg, col * 4, 0, 0);
                }
            }
        }
        v4i blk;
        if constexpr (shared) blk = acc.s[c];
        else blk = acc.f[fr < 0 ? 0 : fr][c];
        asm volatile("" : "+v"(blk));
        u32x4 o;
        if constexpr (CK == C_F32 || gated) {
#pragma unroll
            for (int q = 0; q < 4; q++)
                o[q] = __float_as_uint(fmaf((float)blk[q] * sa, co.sb[c0 + c][q], co.bz[c0 + c][q]));
        } else {
#pragma unroll
            for (int q = 0; q < 4; q++) o[q] = (unsigned)blk[q];
        }
        *(u32x4*)(lc + lr * SP + stage_slot(lr, 4 * (c % 3) + lg) * 16) = o;
        if (c % 3 == 2) {
            const int cg = c - 2;
#pragma unroll
            for (int t = 0; t < 3; t++) {
                const int x = w.lane + 64 * t, rr = x / 12, ch = x - 12 * rr;
                u32x4 v = *(const u32x4*)(lc + rr * SP + stage_slot(rr, ch) * 16);
                if constexpr (gated) {
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        v[q] = __float_as_uint(
                            fmaf(__uint_as_float(v[q]), __uint_as_float(gts[t][q]), __uint_as_float(res[t][q])));
                }
                const int col = colw + 16 * (c0 + cg) + 4 * ch;
                const int off = col < p.N ? (16 * g + rr) * pitch + col * 4 : kDropOffset;
                __builtin_amdgcn_raw_buffer_store_b128(v, rs, off, 0, kStoreNT);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
}

// bf16, software-pipelined: block row R's read-back waits in registers while
// row R + 1 converts, and is stored after that conversion, so the LDS latency
// of the read-back (and of the row scales, all read at the start) hides
// behind VALU work instead of stalling each row.  The LDS runs a wave's
// operations in order, so row R + 1's staging writes cannot overtake row R's
// read-back of the same slots.
struct Pend {
    u32x4 v[3];
    int off[3];
};
constexpr int EG = 2;  // blocks converted together (measured: 2, 3, 4 and 6 alike within 4%)

template <int WM, int R>
__device__ __forceinline__ void epi_row_bf16(Acc& acc, const ColOps& co, const GemmParams& p, const Tw& w,
                                             float sa, Pend& pend, const __amdgpu_buffer_rsrc_t& rs, int pitch,
                                             int colw) {
    constexpr bool shared = WM == 0 ? R == 8 : R == 0;
    constexpr int g = 8 * WM + R;
    constexpr int c0 = shared ? 3 * WM : 0;
    constexpr int nb = shared ? 3 : 6;
    constexpr int fr = WM == 0 ? R : R - 1;
    // the previous row's store count: the shared row issues two
    constexpr int prev = R == 0 ? 0 : ((WM == 0 ? R - 1 == 8 : R - 1 == 0) ? 2 : 3);
    const int lr = w.lane & 15, lg = w.lane >> 4;
    int8_t* lc = w.lc;
    // EG blocks at a time: 4 EG independent conversions a step (one block's
    // four chains alone leave the VALU waiting on its own results: 7.3k
    // clocks an epilogue against 6.7k at c1 up).
#pragma unroll
    for (int c = 0; c < nb; c += EG) {
        const int nc = c + EG <= nb ? EG : nb - c;
        v4i blk[EG];
#pragma unroll
        for (int j = 0; j < EG; j++) {
            if (j < nc) {
                if constexpr (shared) blk[j] = acc.s[c + j];
                else blk[j] = acc.f[fr < 0 ? 0 : fr][c + j];
                asm volatile("" : "+v"(blk[j]));
            }
        }
        float v[EG][4];
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int j = 0; j < EG; j++)
                if (j < nc) v[j][q] = (float)blk[j][q] * sa;
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int j = 0; j < EG; j++)
                if (j < nc) v[j][q] = fmaf(v[j][q], co.sb[c0 + c + j][q], co.bz[c0 + c + j][q]);
#pragma unroll
        for (int j = 0; j < EG; j++)
            if (j < nc)
                *(u32x2*)(lc + lr * SP + stage_slot(lr, 2 * (c + j) + (lg >> 1)) * 16 + (lg & 1) * 8) =
                    u32x2{f32x2_to_bf16x2(v[j][0], v[j][1]), f32x2_to_bf16x2(v[j][2], v[j][3])};
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < prev; t++) __builtin_amdgcn_raw_buffer_store_b128(pend.v[t], rs, pend.off[t], 0, kStoreNT);
    __builtin_amdgcn_sched_barrier(0);
    // 16 rows x 2 nb pieces in row order (piece x: row x / (2 nb), piece
    // x % (2 nb) of the row): three stores a lane for a full row, two (the
    // second half empty) for the shared one.
#pragma unroll
    for (int t = 0; t < (shared ? 2 : 3); t++) {
        const int x = w.lane + 64 * t, rr = x / (2 * nb), ch = x - 2 * nb * rr;
        pend.v[t] = *(const u32x4*)(lc + (rr & 15) * SP + stage_slot(rr & 15, ch) * 16);
        const int col = colw + 16 * c0 + 8 * ch;
        pend.off[t] = col < p.N && rr < 16 ? (16 * g + rr) * pitch + col * 2 : kDropOffset;
    }
    __builtin_amdgcn_sched_barrier(0);
}

template <int WM, int R = 0>
__device__ __forceinline__ void epi_rows_bf16(Acc& acc, const ColOps& co, const GemmParams& p, const Tw& w,
                                              const float (&sa)[9], Pend& pend, const __amdgpu_buffer_rsrc_t& rs,
                                              int pitch, int colw) {
    if constexpr (R < 9) {
        epi_row_bf16<WM, R>(acc, co, p, w, sa[R], pend, rs, pitch, colw);
        epi_rows_bf16<WM, R + 1>(acc, co, p, w, sa, pend, rs, pitch, colw);
    } else {
        constexpr int last = WM == 0 ? 2 : 3;  // row 8 is the shared one for wm = 0
#pragma unroll
        for (int t = 0; t < last; t++) __builtin_amdgcn_raw_buffer_store_b128(pend.v[t], rs, pend.off[t], 0, kStoreNT);
    }
}

template <int WM, int CK, int R = 0>
__device__ __forceinline__ void epi_rows(Acc& acc, const ColOps& co, const GemmParams& p, const Tw& w,
                                         const int8_t* e, const __amdgpu_buffer_rsrc_t& rs,
                                         const __amdgpu_buffer_rsrc_t& rg, int pitch, int colw) {
    if constexpr (R < 9) {
        epi_row<WM, CK, R>(acc, co, p, w, e, rs, rg, pitch, colw);
        epi_rows<WM, CK, R + 1>(acc, co, p, w, e, rs, rg, pitch, colw);
    }
}

// Epilogue of the tile at (m0, n0) with operands in area e; s0 is the column
// scale when it is one scalar.
template <int WM, int CK>
__device__ __forceinline__ void epilogue(Acc& acc, const GemmParams& p, int m0, int n0, const Tw& w, const int8_t* e,
                                         float s0) {
#pragma unroll
    for (int r = 0; r < 8; r++)
#pragma unroll
        for (int c = 0; c < 6; c++) asm volatile("" : "+a"(acc.f[r][c]));
#pragma unroll
    for (int c = 0; c < 3; c++) asm volatile("" : "+a"(acc.s[c]));
    constexpr int esz = CK == C_BF16 ? 2 : 4;
    const int pitch = (int)p.ldc * esz;
    const __amdgpu_buffer_rsrc_t rs = whole_rsrc((int8_t*)p.C + (int64_t)m0 * pitch, min(TM, p.M - m0) * pitch);
    ColOps co;
    if constexpr (CK != C_I32) {
        // The formats are wave-uniform: a scalar branch runs one form (the
        // bias as bf16 pairs or fp32 words, the column scale as one scalar or
        // a row of columns), without converting and selecting both.
        const int lg = w.lane >> 4;
        if (p.bias_kind == BIAS_BF16) {
#pragma unroll
            for (int c = 0; c < 6; c++) {
                const u32x2 hz = *(const u32x2*)(e + E_BZ + (96 * w.wn + 16 * c + 4 * lg) * 2);
                co.bz[c] = v4f{__uint_as_float(hz[0] << 16), __uint_as_float(hz[0] & 0xffff0000u),
                               __uint_as_float(hz[1] << 16), __uint_as_float(hz[1] & 0xffff0000u)};
            }
        } else {
#pragma unroll
            for (int c = 0; c < 6; c++) co.bz[c] = *(const v4f*)(e + E_BZ + (96 * w.wn + 16 * c + 4 * lg) * 4);
        }
        if (p.sb_scalar) {
#pragma unroll
            for (int c = 0; c < 6; c++) co.sb[c] = v4f{s0, s0, s0, s0};
        } else {
#pragma unroll
            for (int c = 0; c < 6; c++) co.sb[c] = *(const v4f*)(e + E_SB + (96 * w.wn + 16 * c + 4 * lg) * 4);
        }
    }
    if constexpr (CK == C_BF16) {
        float sa[9];
        const int lr = w.lane & 15;
#pragma unroll
        for (int r = 0; r < 9; r++) sa[r] = *(const float*)(e + E_SA + (16 * (8 * WM + r) + lr) * 4);
        Pend pend;
        epi_rows_bf16<WM>(acc, co, p, w, sa, pend, rs, pitch, n0 + 96 * w.wn);
    } else {
        // The gate's columns (fp32 [N]); beyond N its loads read zeros.
        const __amdgpu_buffer_rsrc_t rg = whole_rsrc(CK == C_F32G ? (const void*)p.gate : (const void*)p.C,
                                                     CK == C_F32G ? p.N * 4 : 0);
        epi_rows<WM, CK>(acc, co, p, w, e, rs, rg, pitch, n0 + 96 * w.wn);
    }
}

template <int WM>
__device__ __forceinline__ NextTile next_tile(const Shape& s, int t, bool valid, bool rev) {
    NextTile nt{0, 0, valid, rev};
    if (valid) {
        int tm, tn;
        tile_mn(s, t, tm, tn);
        nt.m0 = tm * TM;
        nt.n0 = tn * TN;
    }
    return nt;
}

// The persistent loop of one wave (block-row half WM).  K % 512 == 0.
template <int WM, int CK>
__device__ __forceinline__ void t272_tiles(const GemmParams& p, int8_t* lds, int8_t* eall, int8_t* cbuf, int wave) {
    // bf16: the epilogue's stores stay in flight into the next tile, and its
    // first three waits count them.  fp32 / int32 issue 51 stores, more than
    // the wait counter holds beside the loads: the epilogue drains them.
    constexpr int NST = CK == C_BF16 ? Nst<CK>::v : 0;
    constexpr int VWR = VW + NST, VWE = VW + NE;
    static_assert(3 * NLD + NST < 64 && VWR < 64, "vmcnt is six bits");
    Tw w;
    w.lane = threadIdx.x & 63;
    w.wave = wave;
    w.wn = wave & 1;
    {
        const int lr = w.lane & 15;
        w.oF = lr * PK + lds_slot(lr, w.lane >> 4) * 16;
    }
    Shape s;
    s.tiles_m = (p.M + TM - 1) / TM;
    s.tiles_n = (p.N + TN - 1) / TN;
    s.ntiles = s.tiles_m * s.tiles_n;
    s.KT = p.K / PK;
    s.group_m = p.group_m;
    s.G = gridDim.x;
    init_div(s);
    const int r0 = xcd_remap(blockIdx.x, s.G);
    if (r0 >= s.ntiles) return;
    const int ntile = (s.ntiles - r0 - 1) / s.G + 1;
    const float s0 = p.sb_scalar && p.sB ? p.sB[0] : 0.0f;
    w.lds = opaque_lds(lds);
    w.le = eall;
    w.lc = cbuf + wave * SBYTES;
    w.rA = whole_rsrc(p.A, p.M * (int)p.lda);
    w.rB = whole_rsrc(p.B, p.N * (int)p.ldb);
    // Prologue: the epilogue operands and K-steps 0-3 of the first tile, then
    // NST stores that land nowhere, standing where a previous tile's epilogue
    // stores stand, so every tile's first waits count alike.
    const NextTile first = next_tile<WM>(s, r0, true, false);
    cursor_to(w, p, first.m0, first.n0, true, false);
    issue_epi(w, p, w.le);
    load_step<0>(w);
    load_step<1>(w);
    load_step<2>(w);
    load_step<3>(w);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NST > 0) {
        const __amdgpu_buffer_rsrc_t nowhere = whole_rsrc(p.C, 0);
#pragma unroll
        for (int d = 0; d < NST; d++) __builtin_amdgcn_raw_buffer_store_b32(0u, nowhere, w.lane * 4 + d * 256, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    wait_vm_lgkm0<3 * NLD + NST>();  // the epilogue operands and K-step 0 have landed
    __builtin_amdgcn_s_barrier();
    Frag f, g;
    frag<WM, 0>(f, w);
    Acc acc;
    NextTile cur = first;
    for (int i = 0;;) {
        const int t = r0 + i * s.G;
        int8_t* le = w.le + (i & 1) * EB;
        int8_t* ln = w.le + ((i + 1) & 1) * EB;
        // Odd tiles walk K downward: a workgroup's tiles in consecutive
        // rounds share their B strips (the XCD's tile order keeps its column
        // strips), and the K-steps a round read last are the ones its L2
        // still holds when the next round starts.
        const NextTile nt = next_tile<WM>(s, t + s.G, i + 1 < ntile, ((i + 1) & 1) != 0);
        PHI_T272_STAMP(i, 0);
        kstep<WM, 0, VWR, true, false>(f, g, acc, w, p, nt, ln);
        kstep<WM, 1, VWR, false, false>(g, f, acc, w, p, nt, ln);
        kstep<WM, 2, VWR, false, false>(f, g, acc, w, p, nt, ln);
        kstep<WM, 3, VW, false, false>(g, f, acc, w, p, nt, ln);
        for (int k = 4; k < s.KT - 4; k += 4) {
            kstep<WM, 0, VW, false, false>(f, g, acc, w, p, nt, ln);
            kstep<WM, 1, VW, false, false>(g, f, acc, w, p, nt, ln);
            kstep<WM, 2, VW, false, false>(f, g, acc, w, p, nt, ln);
            kstep<WM, 3, VW, false, false>(g, f, acc, w, p, nt, ln);
        }
        kstep<WM, 0, VW, false, true>(f, g, acc, w, p, nt, ln);
        kstep<WM, 1, VWE, false, false>(g, f, acc, w, p, nt, ln);
        kstep<WM, 2, VWE, false, false>(f, g, acc, w, p, nt, ln);
        kstep<WM, 3, VWE, false, false>(g, f, acc, w, p, nt, ln);
        PHI_T272_STAMP(i, 1);
        epilogue<WM, CK>(acc, p, cur.m0, cur.n0, w, le, s0);
        PHI_T272_STAMP(i, 2);
        if constexpr (NST == 0) wait_all();
        if (++i == ntile) break;
        cur = nt;
    }
    // Loads past the last K-step (zeros, into released stages) and the
    // epilogue's stores are still in flight: let them land before the LDS is
    // released.
    wait_all();
}

// The W4 persistent loop of one wave.  K % 1024 == 0 (the code cursor moves
// to the next tile at K-step KT - 5, which must fall after the tile's first
// four K-steps).
template <int WM, int CK>
__device__ __forceinline__ void t272w4_tiles(const GemmParams& p, int8_t* lds, int8_t* eall, int8_t* cbuf, int wave) {
    constexpr int NST = CK == C_BF16 ? Nst<CK>::v : 0;
    constexpr int VWR = VW4 + NST, VWE = VW4 + NE;
    static_assert(NST + 27 < 64 && VWR < 64, "vmcnt is six bits");
    Tw w;
    W4c c;
    w.lane = threadIdx.x & 63;
    w.wave = wave;
    w.wn = wave & 1;
    {
        const int lr = w.lane & 15;
        w.oF = lr * PK + lds_slot(lr, w.lane >> 4) * 16;
    }
    Shape s;
    s.tiles_m = (p.M + TM - 1) / TM;
    s.tiles_n = (p.N + TN - 1) / TN;
    s.ntiles = s.tiles_m * s.tiles_n;
    s.KT = p.K / PK;
    s.group_m = p.group_m;
    s.G = gridDim.x;
    init_div(s);
    const int r0 = xcd_remap(blockIdx.x, s.G);
    if (r0 >= s.ntiles) return;
    const int ntile = (s.ntiles - r0 - 1) / s.G + 1;
    const float s0 = p.sb_scalar && p.sB ? p.sB[0] : 0.0f;
    w.lds = opaque_lds(lds);
    w.le = eall;
    w.lc = cbuf + wave * SBYTES;
    w.rA = whole_rsrc(p.A, p.M * p.K);
    if (p.w4_banded) {
        const int64_t cb = w4_banded_code_bytes(p.N, p.K);
        c.rC = whole_rsrc(p.B, (int)cb);
        c.rL = whole_rsrc(p.lut, (int)((p.N + TN - 1) / TN * p.lut_groups * (TN * 16)));
    } else {
        c.rC = whole_rsrc(p.B, p.N * (int)p.ldb);
        c.rL = whole_rsrc(p.lut, p.N * (int)p.lut_groups * 16);
    }
    // Prologue: the epilogue operands; codes and tables of K-steps 0-3 and A
    // of K-steps 0-3 (in the order the K-steps would issue them); the
    // expansion of K-steps 0 and 1 once their codes have landed; then codes
    // and tables of K-step 4 into the stage K-step 0's codes left, and NST
    // stores that land nowhere, standing where a previous tile's epilogue
    // stores stand.  From there every K-step's wait counts as in the loop.
    const NextTile first = next_tile<WM>(s, r0, true, false);
    cursor_to(w, p, first.m0, first.n0, true, false);
    w4_cursor_to(c, w, p, first.n0, true);
    const W4o lo4 = w4_lane_offsets(w);
    issue_epi(w, p, w.le);
    {
#define PHI_W4_CODES(CS)                  \
    w4_load1<CS, 0>(c, w, p);             \
    w4_load1<CS, 1>(c, w, p);             \
    w4_load1<CS, 2>(c, w, p);             \
    w4_load1<CS, 3>(c, w, p);             \
    w4_load1<CS, 4>(c, w, p);             \
    w4_load1<CS, 5>(c, w, p);             \
    c.kc++;
#define PHI_W4_A(ST)                                                  \
    {                                                                 \
        int8_t* da = w4_a_base<ST>(w);                                \
        int8_t* dq = w4_a_quarter<ST>(w);                             \
        load1<0>(w, da, dq);                                          \
        load1<1>(w, da, dq);                                          \
        load1<2>(w, da, dq);                                          \
        load1<3>(w, da, dq);                                          \
        load1<4>(w, da, dq);                                          \
    }
        PHI_W4_CODES(0)
        PHI_W4_A(0)
        PHI_W4_CODES(1)
        PHI_W4_A(1)
        PHI_W4_CODES(2)
        PHI_W4_A(2)
        PHI_W4_CODES(3)
        PHI_W4_A(3)
    }
    __builtin_amdgcn_sched_barrier(0);
    wait_vm_lgkm0<2 * NLD4 + NA>();  // codes and tables of K-steps 0-1, A of K-step 0 have landed
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    {
        W4u u[3];
        const int8_t* cs0 = opaque_lds(w.lds + W4_C);
        const int8_t* ls0 = opaque_lds(w.lds + W4_L);
        int8_t* b0 = opaque_lds(w.lds + W4_B);
        const int8_t* cs1 = opaque_lds(w.lds + W4_C + W4_CS);
        const int8_t* ls1 = opaque_lds(w.lds + W4_L + W4_LS);
        int8_t* b1 = opaque_lds(w.lds + W4_B + W4_BS);
#pragma unroll
        for (int x = 0; x < 2; x++) {
#pragma unroll
            for (int U = 0; U < 3; U++) {
                const int8_t* cs = x ? cs1 : cs0;
                const int8_t* ls = x ? ls1 : ls0;
                int8_t* bo = x ? b1 : b0;
                w4_piece<0>(u[U], U, lo4, cs, ls, bo);
                w4_piece<1>(u[U], U, lo4, cs, ls, bo);
                w4_piece<2>(u[U], U, lo4, cs, ls, bo);
                w4_piece<3>(u[U], U, lo4, cs, ls, bo);
                w4_piece<4>(u[U], U, lo4, cs, ls, bo);
                w4_piece<5>(u[U], U, lo4, cs, ls, bo);
                w4_piece<6>(u[U], U, lo4, cs, ls, bo);
                w4_piece<7>(u[U], U, lo4, cs, ls, bo);
                w4_piece<8>(u[U], U, lo4, cs, ls, bo);
                w4_piece<9>(u[U], U, lo4, cs, ls, bo);
                w4_piece<10>(u[U], U, lo4, cs, ls, bo);
            }
        }
    }
    wait_vm_lgkm0<63>();  // this wave's expansion writes are done (lgkmcnt 0)
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    PHI_W4_CODES(0)
#undef PHI_W4_CODES
#undef PHI_W4_A
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NST > 0) {
        const __amdgpu_buffer_rsrc_t nowhere = whole_rsrc(p.C, 0);
#pragma unroll
        for (int d = 0; d < NST; d++) __builtin_amdgcn_raw_buffer_store_b32(0u, nowhere, w.lane * 4 + d * 256, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    Frag f, g;
    {
        const int8_t* a = opaque_lds(w.lds + 1024 * 8 * WM) + w.oF;
        const int8_t* b = opaque_lds(w.lds + W4_B + 6144 * w.wn) + w.oF;
#pragma unroll
        for (int i = 0; i < 9; i++) f.a[i] = *(const v4i*)(a + 1024 * i);
#pragma unroll
        for (int j = 0; j < 6; j++) f.b[j] = *(const v4i*)(b + 1024 * j);
    }
    Acc acc;
    NextTile cur = first;
    for (int i = 0;;) {
        const int t = r0 + i * s.G;
        int8_t* le = w.le + (i & 1) * EB;
        int8_t* ln = w.le + ((i + 1) & 1) * EB;
        const NextTile nt = next_tile<WM>(s, t + s.G, i + 1 < ntile, false);
        PHI_T272_STAMP(i, 0);
        kstep4<WM, 0, VWR, true, false, false>(f, g, acc, w, c, lo4, p, nt, ln);
        kstep4<WM, 1, VWR, false, false, false>(g, f, acc, w, c, lo4, p, nt, ln);
        kstep4<WM, 2, VWR, false, false, false>(f, g, acc, w, c, lo4, p, nt, ln);
        kstep4<WM, 3, VW4, false, false, false>(g, f, acc, w, c, lo4, p, nt, ln);
        for (int k = 4; k < s.KT - 8; k += 4) {
            kstep4<WM, 0, VW4, false, false, false>(f, g, acc, w, c, lo4, p, nt, ln);
            kstep4<WM, 1, VW4, false, false, false>(g, f, acc, w, c, lo4, p, nt, ln);
            kstep4<WM, 2, VW4, false, false, false>(f, g, acc, w, c, lo4, p, nt, ln);
            kstep4<WM, 3, VW4, false, false, false>(g, f, acc, w, c, lo4, p, nt, ln);
        }
        kstep4<WM, 0, VW4, false, false, false>(f, g, acc, w, c, lo4, p, nt, ln);
        kstep4<WM, 1, VW4, false, false, false>(g, f, acc, w, c, lo4, p, nt, ln);
        kstep4<WM, 2, VW4, false, false, false>(f, g, acc, w, c, lo4, p, nt, ln);
        kstep4<WM, 3, VW4, false, false, true>(g, f, acc, w, c, lo4, p, nt, ln);
        kstep4<WM, 0, VW4, false, true, false>(f, g, acc, w, c, lo4, p, nt, ln);
        kstep4<WM, 1, VWE, false, false, false>(g, f, acc, w, c, lo4, p, nt, ln);
        kstep4<WM, 2, VWE, false, false, false>(f, g, acc, w, c, lo4, p, nt, ln);
        kstep4<WM, 3, VWE, false, false, false>(g, f, acc, w, c, lo4, p, nt, ln);
        PHI_T272_STAMP(i, 1);
        mfma_drain();
        epilogue<WM, CK>(acc, p, cur.m0, cur.n0, w, le, s0);
        PHI_T272_STAMP(i, 2);
        if constexpr (NST == 0) wait_all();
        if (++i == ntile) break;
        cur = nt;
    }
    wait_all();
}

template <int CK>
__global__ __launch_bounds__(256) void i8_gemm_t272w4_kernel(GemmParams p) {
    __shared__ __align__(16) int8_t lds[W4_LDS];
    __shared__ __align__(16) int8_t eall[2 * EB];
    __shared__ __align__(16) int8_t cbuf[4 * SBYTES];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & 3;
    PHI_T272_TRACE_BEGIN
    if (wave < 2) t272w4_tiles<0, CK>(p, lds, eall, cbuf, wave);
    else t272w4_tiles<1, CK>(p, lds, eall, cbuf, wave);
    PHI_T272_TRACE_END
}

template <int CK>
__global__ __launch_bounds__(256) void i8_gemm_t272_kernel(GemmParams p) {
    __shared__ __align__(16) int8_t lds[NSTG * STG];
    __shared__ __align__(16) int8_t eall[2 * EB];
    __shared__ __align__(16) int8_t cbuf[4 * SBYTES];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & 3;
    PHI_T272_TRACE_BEGIN
    if (wave < 2) t272_tiles<0, CK>(p, lds, eall, cbuf, wave);
    else t272_tiles<1, CK>(p, lds, eall, cbuf, wave);
    PHI_T272_TRACE_END
}

}  // namespace

int t272_tile_count(int64_t M, int64_t N) { return (int)(((M + TM - 1) / TM) * ((N + TN - 1) / TN)); }

bool t272_ok(const GemmParams& p) {
    const int64_t esz = p.c_kind == C_BF16 ? 2 : 4;
    // Row-major operands: 16-byte lanes, and every source offset (rows x
    // pitch) within 32 bits.  K-tiled ones are packed with pitch K.  b_rm:
    // A K-tiled, B row-major.
    const bool kta = p.kt != 0, ktb = p.kt && !p.b_rm;
    const int64_t la = kta ? p.K : p.lda, lb = ktb ? p.K : p.ldb;
    const bool a_ok = kta || (p.lda >= p.K && p.lda % 16 == 0 && ((uintptr_t)p.A & 15) == 0);
    const bool b_ok = ktb || (p.ldb >= p.K && p.ldb % 16 == 0 && ((uintptr_t)p.B & 15) == 0);
    return a_ok && b_ok && (!p.b_rm || p.kt) && (!p.gate || p.c_kind == C_F32) && p.K % 512 == 0 &&
           (int64_t)p.M * la < ((int64_t)1 << 31) - (1 << 20) &&
           (int64_t)p.N * lb < ((int64_t)1 << 31) - (1 << 20) && (int64_t)TM * p.ldc * esz < ((int64_t)1 << 31) &&
           p.N % (16 / esz) == 0;
}

bool t272w4_ok(const GemmParams& p) {
    const int64_t esz = p.c_kind == C_BF16 ? 2 : 4;
    // The band layout: both regions' offsets within 31 bits, the tables
    // 16-byte aligned.  The checkpoint's rows: 16-byte code rows.
    const int64_t bands = (p.N + TN - 1) / TN;
    const bool src_ok = p.w4_banded ? bands * (p.K / 2) * TN + bands * p.lut_groups * TN * 16 < ((int64_t)1 << 31) &&
                                          ((uintptr_t)p.lut & 15) == 0
                                    : p.ldb >= p.K / 2 && p.ldb % 16 == 0 &&
                                          ((int64_t)p.N + 512) * p.ldb < ((int64_t)1 << 31) &&
                                          ((int64_t)p.N + 512) * p.lut_groups * 16 < ((int64_t)1 << 31);
    return p.kt && !p.gate && !p.w4_signed && p.lut && p.K % 1024 == 0 && p.group_shift >= 6 &&
           p.group_shift < 31 && (1ll << p.group_shift) <= p.K && p.lut_groups == (p.K >> p.group_shift) &&
           src_ok && ((uintptr_t)p.B & 15) == 0 &&
           (int64_t)p.M * p.K < ((int64_t)1 << 31) - (1 << 20) &&
           (int64_t)TM * p.ldc * esz < ((int64_t)1 << 31) && p.N % (16 / esz) == 0;
}

int64_t w4_banded_bytes(int64_t N, int64_t K, int64_t group) {
    if (N <= 0 || K <= 0 || K % PK != 0 || group <= 0 || K % group != 0) return 0;
    const int64_t bands = (N + TN - 1) / TN;
    return bands * (K / PK) * (TN * 32) + bands * (K / group) * (TN * 16);
}

hipError_t launch_i8_gemm_t272w4(hipStream_t stream, const GemmParams& p, int num_cus) {
    if (!t272w4_ok(p)) return hipErrorInvalidValue;
    const int tiles = t272_tile_count(p.M, p.N);
    const dim3 g3(tiles < num_cus ? tiles : num_cus), b3(256);
    if (p.c_kind == C_BF16) hipLaunchKernelGGL((i8_gemm_t272w4_kernel<C_BF16>), g3, b3, 0, stream, p);
    else if (p.c_kind == C_F32) hipLaunchKernelGGL((i8_gemm_t272w4_kernel<C_F32>), g3, b3, 0, stream, p);
    else hipLaunchKernelGGL((i8_gemm_t272w4_kernel<C_I32>), g3, b3, 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_i8_gemm_t272(hipStream_t stream, const GemmParams& p, int num_cus) {
    if (!t272_ok(p)) return hipErrorInvalidValue;
    const int tiles = t272_tile_count(p.M, p.N);
    const dim3 g3(tiles < num_cus ? tiles : num_cus), b3(256);
    if (p.c_kind == C_BF16) hipLaunchKernelGGL((i8_gemm_t272_kernel<C_BF16>), g3, b3, 0, stream, p);
    else if (p.c_kind == C_F32 && p.gate) hipLaunchKernelGGL((i8_gemm_t272_kernel<C_F32G>), g3, b3, 0, stream, p);
    else if (p.c_kind == C_F32) hipLaunchKernelGGL((i8_gemm_t272_kernel<C_F32>), g3, b3, 0, stream, p);
    else hipLaunchKernelGGL((i8_gemm_t272_kernel<C_I32>), g3, b3, 0, stream, p);
    return hipGetLastError();
}

}  // namespace phi_dev
