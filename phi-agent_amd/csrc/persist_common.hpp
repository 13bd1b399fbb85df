// Pieces shared by the persistent int8 GEMM kernels (i8_gemm_persist.hip,
// i8_gemm_pipe.hip, i8_gemm_t272.hip): buffer-resource and wait helpers, the
// XCD-aware tile order, the 4-bit code expansion through a per-(row, group)
// table, the epilogue-operand loads and the epilogue.
//
// The product and epilogue are those of the reference's int8_gemm_tc
// (core/kernels/int8_gemm.cpp:466-621, epilogue :588-620) and host gemm_int8
// (core/host/quant.cpp:223-236):
//   C[m,n] = fma((float)acc[m,n] * sA[m], sB[n], bias[n])  -> bf16 (RNE) / fp32 / raw int32
#pragma once

#include "device_common.hpp"
#include "i8_gemm.hpp"

namespace phi_dev {
namespace persist {

typedef __attribute__((address_space(3))) void* lptr_t;
typedef unsigned int u32x2 __attribute__((__vector_size__(2 * sizeof(unsigned int))));
typedef unsigned int u32x4 __attribute__((__vector_size__(4 * sizeof(unsigned int))));

// Raw buffer resource word 3 for gfx9-family: 32-bit data format, no swizzle.
constexpr int kRsrcWord3 = 0x00020000;


constexpr int EBYTES = 4 * 1024;  // per parity: sa | sb | bias | gate (4 waves x 256 B each)
constexpr int CHUNK = 4096 + 512;  // per-wave epilogue staging: 32 rows x 128 bytes, then fp32 bias

constexpr int SG_VALU = 0x002, SG_MFMA = 0x008, SG_VMEM_R = 0x020, SG_DSR = 0x100, SG_DSW = 0x200;

// Cache policy of the output stores: non-temporal.  The output is written
// once and never read back by this kernel; letting it allocate in L2 evicts
// the A and B strips the XCD's other tiles are still reading.
constexpr int kStoreNT = 2;

// Offset of a store that must not land (a column past N): beyond any tile
// buffer's range (those stay below 2^31 bytes), so the range check drops it.
// Every epilogue store is issued, none is branched around: the epilogue has
// no per-store blocks, and the number of memory operations it issues is
// fixed, which the first wait of the next tile counts on.
constexpr int kDropOffset = (int)0x80000000u;


// s_waitcnt vmcnt(0) lgkmcnt(0) (gfx9 encoding; expcnt untouched).
__device__ __forceinline__ void wait_all() { __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (0 << 8)); }
// s_waitcnt vmcnt(N) lgkmcnt(0).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt is six bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | (((N >> 4) & 3) << 14));
}


// An LDS pointer the compiler cannot fold into a constant address.  A ds_read
// takes a 16-bit immediate offset: when the B stages sit above 64 KB, a known
// base plus the block offset does not fit it, and each of a quarter's reads
// would get an address register of its own (32 for the 256 x 256 tile, live
// through the main loop).  With the base opaque, the stage and block offsets
// stay immediates on one register per quarter.
__device__ __forceinline__ int8_t* opaque_lds(int8_t* p) {
    typedef __attribute__((address_space(3))) int8_t lds_i8;
    uint32_t a = (uint32_t)(uintptr_t)(lds_i8*)p;
    asm volatile("" : "+s"(a));
    return (int8_t*)(lds_i8*)(uintptr_t)a;
}

__device__ __forceinline__ int xcd_remap(int pid, int nblocks) {
    const int xcd = pid & 7, idx = pid >> 3;
    const int base = nblocks >> 3, rem = nblocks & 7;
    return xcd < rem ? xcd * (base + 1) + idx : rem * (base + 1) + (xcd - rem) * base + idx;
}

// The lane and wave indices the epilogue and its operand loads use, the
// wave's epilogue staging area, and the load cursor's tile origin.
struct EpiWave {
    int8_t* lc;  // this wave's CHUNK bytes of epilogue staging (the bias copy at lc + 4096)
    int wave, wm, wn, lane, lrow, lhalf;
    int cm0, cn0;
};

struct Shape {
    int tiles_m, tiles_n, ntiles, KT, group_m, G;
    // Tile order divisors (group_m * tiles_n and group_m) and their
    // multipliers for udiv_inv, set by init_div.
    unsigned per_group, pg_mul, gm_mul;
};

// Multiplier for dividing by a loop-invariant d >= 1: ceil(2^32 / d), which
// is (2^32 - 1) / d + 1 for every d (0 for d = 1, handled in udiv_inv).
__device__ __forceinline__ unsigned inv_mul(unsigned d) { return 0xffffffffu / d + 1u; }

// n / d for n < 2^32 with m = inv_mul(d): the high word of n * m is n / d or
// one more (m exceeds 2^32 / d by less than 1, so n * m / 2^32 exceeds n / d
// by less than n / 2^32 < 1), and one comparison corrects it.  A handful of
// scalar instructions instead of the reciprocal sequence of a general
// division, which sits between every two tiles of the persistent loops.
__device__ __forceinline__ unsigned udiv_inv(unsigned n, unsigned d, unsigned m) {
    unsigned q = d == 1u ? n : __umulhi(n, m);
    return q * d > n ? q - 1u : q;
}

__device__ __forceinline__ void init_div(Shape& s) {
    s.per_group = (unsigned)(s.group_m * s.tiles_n);
    s.pg_mul = inv_mul(s.per_group);
    s.gm_mul = inv_mul((unsigned)s.group_m);
}

// Logical tile -> (tile row, tile column): groups of group_m tile rows, each
// walked down its rows first.
__device__ __forceinline__ void tile_mn(const Shape& s, int logical, int& tm, int& tn) {
    const int gid = (int)udiv_inv((unsigned)logical, s.per_group, s.pg_mul);
    const int first_m = gid * s.group_m;
    const int gsz = min(s.tiles_m - first_m, s.group_m);
    const int in_group = logical - gid * (int)s.per_group;
    // gsz is group_m except in a last, shorter group.
    const int q = gsz == s.group_m ? (int)udiv_inv((unsigned)in_group, (unsigned)gsz, s.gm_mul) : in_group / gsz;
    tm = first_m + (in_group - q * gsz);
    tn = q;
}


// Four codes (bytes of x, each 0..15) -> four int8 through the 16-byte table
// t: v_perm_b32 picks from entries 0..7 and 8..15 by the low three bits, and
// bit 3 chooses (selector bytes 0x0c / 0x0d give 0x00 / 0xff).
__device__ __forceinline__ uint32_t lut4b(uint32_t x, const u32x4& t) {
    const uint32_t sel = x & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(t[1], t[0], sel);
    const uint32_t hi = __builtin_amdgcn_perm(t[3], t[2], sel);
    const uint32_t m = __builtin_amdgcn_perm(0u, 0u, ((x >> 3) & 0x01010101u) | 0x0c0c0c0cu);
    return (hi & m) | (lo & ~m);
}

// The table of signed nibbles (convrot_w4a4): codes 0..7 are 0..7, 8..15 are -8..-1.
__device__ __forceinline__ u32x4 signed_nibble_table() { return u32x4{0x03020100u, 0x07060504u, 0xfbfaf9f8u, 0xfffefdfcu}; }

// 16 codes (8 bytes) -> 16 int8 operand bytes in column order.
__device__ __forceinline__ v4i expand16b(uint32_t c0, uint32_t c1, const u32x4& t) {
    const uint32_t e0 = lut4b(c0 & 0x0f0f0f0fu, t), o0 = lut4b((c0 >> 4) & 0x0f0f0f0fu, t);
    const uint32_t e1 = lut4b(c1 & 0x0f0f0f0fu, t), o1 = lut4b((c1 >> 4) & 0x0f0f0f0fu, t);
    // e holds columns 0,2,4,6 and o columns 1,3,5,7: interleave.
    v4i r;
    r.x = (int)__builtin_amdgcn_perm(o0, e0, 0x05010400u);
    r.y = (int)__builtin_amdgcn_perm(o0, e0, 0x07030602u);
    r.z = (int)__builtin_amdgcn_perm(o1, e1, 0x05010400u);
    r.w = (int)__builtin_amdgcn_perm(o1, e1, 0x07030602u);
    return r;
}

// Epilogue operands of the cursor's tile into LDS area le: wave w loads row
// scales 64w..64w+63, column scales / fp32 bias 64w..64w+63 and (waves 0-1)
// the bf16 bias words; past M or N (or the tile) they read as zero.
template <int WT, bool G>
__device__ __forceinline__ void issue_epi(const EpiWave& w, const GemmParams& p, int8_t* le) {
    constexpr int BM = 2 * WT;
    const int rows = min(BM, p.M - w.cm0), cols = min(BM, p.N - w.cn0);
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
    // G (the gated-residual instantiation): the gate, without a branch (a
    // branch here would split the tile's last K-step pair, whose loads and
    // MFMAs are scheduled as one block).
    if constexpr (G) {
        const __amdgpu_buffer_rsrc_t rG =
            __builtin_amdgcn_make_buffer_rsrc((void*)(p.gate + w.cn0), (short)0, cols * 4, kRsrcWord3);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rG, (lptr_t)(le + 3072 + w.wave * 256), 4, w.lane * 4,
                                                 w.wave * 256, 0, 0);
    }
}


// The bias of the wave's WT columns as fp32, written after the wave's
// staging rows: converted once a tile, one value a lane per 64 columns,
// instead of by each of the 32 lanes that use a column.  The bias area holds
// bf16 pairs or fp32 words, zeros without a bias (its loads fell outside a
// zero-length range); both views are read and the uniform format selects.
template <int WT>
__device__ __forceinline__ void bias_to_f32(const EpiWave& w, bool bf, const int8_t* e) {
#pragma unroll
    for (int c0 = 0; c0 < WT; c0 += 64) {
        const int c = c0 + w.lane, col = w.wn * WT + c;
        const float f = *(const float*)(e + 2048 + col * 4);
        const uint32_t h = *(const unsigned short*)(e + 2048 + col * 2);
        *(float*)(w.lc + 4096 + c * 4) = bf ? __uint_as_float(h << 16) : f;
    }
}

// Epilogue operands of this lane's four columns starting at wave column cw
// (tile column ct = the wave's first column + cw).  The column-scale area
// holds one float per column: a scalar scale was loaded into every slot.
__device__ __forceinline__ void col_operands(const EpiWave& w, const int8_t* e, int ct, int cw, v4f& sb, v4f& bz) {
    sb = *(const v4f*)(e + 1024 + ct * 4);
    bz = *(const v4f*)(w.lc + 4096 + cw * 4);
}

// Epilogue of the tile at (m0, n0) (operands in the LDS area e).  Lane l holds row
// l % 32 of each A block and, in registers 4g..4g+3, columns 8g + 4(l/32) +
// 0..3 of each B block.  Each 32-row strip goes through the wave's LDS area
// and is stored as whole rows: bf16 in 32 x 64-column pieces (128 bytes a
// row), fp32 / int32 in 32 x 32-column pieces.
//
// Staging layout: row r at r * 128; 16-byte chunk c of the row in slot
// c ^ ((r >> 1) & 7).  The 128-byte pitch puts even rows in banks 0-31 and
// odd rows in banks 32-63, and the slot swizzle spreads rows 2s and 2s + 1
// over the eight slots: a write of one chunk by 16 rows (fp32, 16 bytes a
// lane) touches every bank once.  The bf16 writes are 8 bytes a lane, 32
// rows at a time: their half of the slot is flipped for rows 16-31
// (lane half h goes to half h ^ (r >> 4)), so these too touch every bank
// once, and the reads of rows 16-31 swap the halves back.  The read-back (16
// lanes a clock: two rows, eight chunks each) is conflict-free as well.
//
// hook(j, i) runs on the bf16 path right after block (j, i) has been read
// out of its accumulators (the pipelined kernel issues the next tile's first
// MFMAs on that block there); the other paths never call it.
struct NoHook {
    __device__ __forceinline__ void operator()(int, int) const {}
};

template <int WT, bool G, typename Hook = NoHook>
__device__ __forceinline__ void epilogue(v16i (&acc)[WT / 32][WT / 32], const GemmParams& p, int m0, int n0,
                                         const EpiWave& w, const int8_t* e, Hook&& hook = Hook{}) {
    constexpr int NB = WT / 32, BM = 2 * WT;
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
        for (int i = 0; i < NB; i++) asm volatile("" : "+a"(acc[j][i]));
    const int esz = p.c_kind == C_BF16 ? 2 : 4;
    const int pitch = (int)p.ldc * esz;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (int8_t*)p.C + (int64_t)m0 * pitch, (short)0, min(BM, p.M - m0) * pitch, kRsrcWord3);
    int8_t* lc = w.lc;
    const int colw = n0 + w.wn * WT;  // first column of this wave
    float sa[NB];
#pragma unroll
    for (int i = 0; i < NB; i++) sa[i] = *(const float*)(e + (w.wm * WT + i * 32 + w.lrow) * 4);
    // A wave's LDS accesses complete in order: the operand reads below see
    // this copy.
    bias_to_f32<WT>(w, p.bias_kind == BIAS_BF16, e);
    if (p.c_kind == C_BF16) {
#pragma unroll
        for (int jp = 0; jp < NB / 2; jp++) {
            v4f sb[2][4], bz[2][4];
#pragma unroll
            for (int jj = 0; jj < 2; jj++)
#pragma unroll
                for (int g = 0; g < 4; g++)
                    col_operands(w, e, w.wn * WT + (2 * jp + jj) * 32 + 8 * g + 4 * w.lhalf,
                                 (2 * jp + jj) * 32 + 8 * g + 4 * w.lhalf, sb[jj][g], bz[jj][g]);
#pragma unroll
            for (int i = 0; i < NB; i++) {
#pragma unroll
                for (int jj = 0; jj < 2; jj++) {
                    v16i blk = acc[2 * jp + jj][i];
                    asm volatile("" : "+v"(blk));
                    hook(2 * jp + jj, i);
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        float v[4];
#pragma unroll
                        for (int q = 0; q < 4; q++)
                            v[q] = fmaf((float)blk[4 * g + q] * sa[i], sb[jj][g][q], bz[jj][g][q]);
                        const int slot = (jj * 4 + g) ^ ((w.lrow >> 1) & 7);
                        *(u32x2*)(lc + w.lrow * 128 + slot * 16 + (w.lhalf ^ (w.lrow >> 4)) * 8) =
                            u32x2{f32x2_to_bf16x2(v[0], v[1]), f32x2_to_bf16x2(v[2], v[3])};
                    }
                }
                // A wave's LDS accesses complete in order: these reads see its writes.
#pragma unroll
                for (int tt = 0; tt < 4; tt++) {
                    const int r = tt * 8 + (w.lane >> 3), sl = w.lane & 7;
                    const u32x4 h = *(const u32x4*)(lc + r * 128 + ((sl ^ ((r >> 1) & 7)) * 16));
                    const u32x4 v = tt < 2 ? h : u32x4{h[2], h[3], h[0], h[1]};  // rows 16-31: halves flipped
                    const int col = colw + jp * 64 + sl * 8;
                    const int off = col < p.N ? (w.wm * WT + i * 32 + r) * pitch + col * 2 : kDropOffset;
                    __builtin_amdgcn_raw_buffer_store_b128(v, rs, off, 0, kStoreNT);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        return;
    }
    // fp32 / int32: 32 x 32 pieces, one block at a time.  With a gate the
    // fp32 output is the residual stream, updated in place:
    // C = fma(v, gate[n], C), the reference's AddMul `a + b * c`
    // (core/kernels/ops.cpp:80, applied after the projection at
    // core/models/av_dit.cpp:1389) as NVRTC's default --fmad=true contracts it.
    constexpr bool gated = G;
#pragma unroll
    for (int j = 0; j < NB; j++) {
        v4f sb[4], bz[4];
        if (p.c_kind == C_F32) {
#pragma unroll
            for (int g = 0; g < 4; g++)
                col_operands(w, e, w.wn * WT + j * 32 + 8 * g + 4 * w.lhalf, j * 32 + 8 * g + 4 * w.lhalf, sb[g], bz[g]);
        }
#pragma unroll
        for (int i = 0; i < NB; i++) {
            // The residual rows this lane stores, fetched before the conversion
            // so their latency overlaps it.
            u32x4 res[4];
            if (gated) {
#pragma unroll
                for (int tt = 0; tt < 4; tt++) {
                    const int r = tt * 8 + (w.lane >> 3), col = colw + j * 32 + (w.lane & 7) * 4;
                    res[tt] = __builtin_amdgcn_raw_buffer_load_b128(rs, (w.wm * WT + i * 32 + r) * pitch + col * 4, 0, 0);
                }
            }
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
                const int slot = (2 * g + w.lhalf) ^ ((w.lrow >> 1) & 7);
                *(u32x4*)(lc + w.lrow * 128 + slot * 16) = o;
            }
#pragma unroll
            for (int tt = 0; tt < 4; tt++) {
                const int r = tt * 8 + (w.lane >> 3), sl = w.lane & 7;
                u32x4 v = *(const u32x4*)(lc + r * 128 + ((sl ^ ((r >> 1) & 7)) * 16));
                const int col = colw + j * 32 + sl * 4;
                if (gated) {
                    const v4f gt = *(const v4f*)(e + 3072 + (w.wn * WT + j * 32 + sl * 4) * 4);
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        v[q] = __float_as_uint(fmaf(__uint_as_float(v[q]), gt[q], __uint_as_float(res[tt][q])));
                }
                const int off = col < p.N ? (w.wm * WT + i * 32 + r) * pitch + col * 4 : kDropOffset;
                __builtin_amdgcn_raw_buffer_store_b128(v, rs, off, 0, kStoreNT);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

}  // namespace persist
}  // namespace phi_dev
