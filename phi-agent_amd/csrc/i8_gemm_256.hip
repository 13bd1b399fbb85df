// Large-tile int8 GEMM for gfx950: 256 x 256 output tiles, operands streamed
// global -> LDS by the direct-to-LDS loads (no staging registers).
//
//   acc[m,n] = sum_k A[m,k] * B[n,k]                  (exact int32)
//   C[m,n]   = fma((float)acc * sA[m], sB[n], bias[n])  -> fp32 / bf16 (RNE) / raw int32
//
// The product and epilogue are those of the reference's int8_gemm_tc
// (core/kernels/int8_gemm.cpp:466-621, epilogue :588-620) and host gemm_int8
// (core/host/quant.cpp:223-236).
//
// Two kernels share the tile order, the LDS loading and the epilogue maths:
//   * i8_gemm_w4_kernel (K % 128 == 0, the default): four waves of 128 x 128
//     (4 x 4 blocks of v_mfma_i32_32x32x32_i8, 256 accumulators in AGPRs) on
//     128-deep K-steps, two 64 KB LDS stages.  One wave per SIMD, so every
//     LDS read and load is threaded between MFMAs with sched_group_barrier;
//     the bf16 epilogue goes through LDS so global stores write whole rows.
//   * i8_gemm_256_kernel (any K % 64 == 0): eight waves of 128 x 64 on 64-deep
//     K-steps, three 32 KB stages, one barrier per K-step between its two MFMA
//     halves.
// Common design points:
//   * The B fragment is the MFMA's first operand, so a lane holds one output
//     row m and, per group of four registers, four consecutive columns n.
//   * Each LDS stage buffer is a separate __shared__ object so the compiler's
//     LDS-DMA wait tracking tells them apart.
//   * global_load_lds_dwordx4: a wave instruction fills 1 KB of LDS, lane l
//     writing bytes 16l..16l+15; rows are swizzled by choosing which global
//     chunk each lane fetches.  The LDS serves a 16-byte read for 16 lanes
//     (256 bytes) per clock, and the swizzles make the operand read of 16
//     consecutive rows cover all 16 bank windows.
//   * Tile order: the hardware deals workgroups round-robin to the 8 XCDs, so
//     the id is remapped to give each XCD a contiguous run of tiles, walked
//     group_m tile-rows at a time (concurrent tiles of one XCD share A rows and
//     B columns in that XCD's L2).
#include "device_common.hpp"
#include "i8_gemm.hpp"

namespace phi_dev {

namespace {

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int STAGE_BYTES = BM * BK;  // 16 KB per operand per stage

__shared__ __align__(16) int8_t lA0[STAGE_BYTES];
__shared__ __align__(16) int8_t lA1[STAGE_BYTES];
__shared__ __align__(16) int8_t lA2[STAGE_BYTES];
__shared__ __align__(16) int8_t lA3[STAGE_BYTES];
__shared__ __align__(16) int8_t lB0[STAGE_BYTES];
__shared__ __align__(16) int8_t lB1[STAGE_BYTES];
__shared__ __align__(16) int8_t lB2[STAGE_BYTES];
__shared__ __align__(16) int8_t lB3[STAGE_BYTES];

template <int S>
__device__ __forceinline__ int8_t* stA() { return S == 0 ? lA0 : S == 1 ? lA1 : S == 2 ? lA2 : lA3; }
template <int S>
__device__ __forceinline__ int8_t* stB() { return S == 0 ? lB0 : S == 1 ? lB1 : S == 2 ? lB2 : lB3; }

typedef __attribute__((address_space(1))) const void* gptr_t;
typedef __attribute__((address_space(3))) void* lptr_t;

__device__ __forceinline__ void dma16(const int8_t* g, int8_t* l) {
    __builtin_amdgcn_global_load_lds((gptr_t)g, (lptr_t)l, 16, 0, 0);
}

// s_waitcnt with vmcnt(n), lgkmcnt(0), expcnt untouched (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt is six bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | (((N >> 4) & 3) << 14));
}

__device__ __forceinline__ int swz(int row, int c) { return c ^ (((row >> 1) ^ (row >> 2)) & 3); }

// The hardware deals workgroup ids round-robin to the 8 XCDs (id % 8); give
// XCD x the contiguous run of logical ids [start_x, start_x + count_x).
__device__ __forceinline__ int xcd_remap(int pid, int nblocks) {
    const int xcd = pid & 7, idx = pid >> 3;
    const int base = nblocks >> 3, rem = nblocks & 7;
    return xcd < rem ? xcd * (base + 1) + idx : rem * (base + 1) + (xcd - rem) * base + idx;
}

// Logical tile id -> (tile_m, tile_n), walking group_m tile-rows at a time.
__device__ __forceinline__ void tile_of_logical(int logical, int tiles_m, int tiles_n, int group_m, int& tm,
                                                int& tn) {
    const int per_group = group_m * tiles_n;
    const int gid = logical / per_group;
    const int first_m = gid * group_m;
    const int gsz = min(tiles_m - first_m, group_m);
    const int in_group = logical - gid * per_group;
    tm = first_m + in_group % gsz;
    tn = in_group / gsz;
}

// Workgroup id -> (tile_m, tile_n): XCD remap, then grouped walk.
__device__ __forceinline__ void tile_of(int pid, int nblocks, int tiles_m, int tiles_n, int group_m,
                                        int& tm, int& tn) {
    tile_of_logical(xcd_remap(pid, nblocks), tiles_m, tiles_n, group_m, tm, tn);
}

template <int WM, int WN, int NST>
struct Cfg {
    static constexpr int NWAVE = WM * WN, NTHR = NWAVE * 64;
    static constexpr int WTM = BM / WM, WTN = BN / WN;      // wave tile
    static constexpr int TM = WTM / 32, TN = WTN / 32;      // MFMA blocks per wave
    static constexpr int NQ = TM * TN;                      // MFMAs per half K-step
    static constexpr int DMA = STAGE_BYTES / 1024 / NWAVE;  // wave loads per operand per K-step
    static constexpr int VM_PER_STEP = 2 * DMA;
    static_assert(DMA >= 1 && DMA * 1024 * NWAVE == STAGE_BYTES, "stage / wave mismatch");
    static_assert(NST >= 3 && NST <= 4, "three or four LDS stages");
};

template <class C>
struct Frag {
    v4i a[C::TM], b[C::TN];
};

template <class C>
struct Ctx {
    const int8_t* gA[C::DMA];
    const int8_t* gB[C::DMA];
    int dma_off;
    int oA[C::TM][2], oB[C::TN][2];
};

template <class C>
__device__ __forceinline__ void issue_loads(int8_t* sa, int8_t* sb, const Ctx<C>& x, int64_t koff) {
#pragma unroll
    for (int j = 0; j < C::DMA; j++) dma16(x.gA[j] + koff, sa + x.dma_off + j * 1024);
#pragma unroll
    for (int j = 0; j < C::DMA; j++) dma16(x.gB[j] + koff, sb + x.dma_off + j * 1024);
}

// Fragments of K half-step H from LDS stage S.
template <class C, int S, int H>
__device__ __forceinline__ void read_frag(Frag<C>& f, const Ctx<C>& x) {
    const int8_t* cA = stA<S>();
    const int8_t* cB = stB<S>();
#pragma unroll
    for (int i = 0; i < C::TM; i++) f.a[i] = *(const v4i*)(cA + x.oA[i][H]);
#pragma unroll
    for (int j = 0; j < C::TN; j++) f.b[j] = *(const v4i*)(cB + x.oB[j][H]);
}

// MFMAs number FIRST..LAST-1 of one half-step.
template <class C, int FIRST, int LAST>
__device__ __forceinline__ void mma(const Frag<C>& f, v16i (&acc)[C::TN][C::TM]) {
#pragma unroll
    for (int q = FIRST; q < LAST; q++) {
        const int j = q / C::TM, i = q % C::TM;
        acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.b[j], f.a[i], acc[j][i], 0, 0, 0);
    }
}

// One K-step on LDS stage S.  On entry f0 holds half-step 0 of this stage; on
// exit it holds half-step 0 of the next stage:
//   MFMA 1 of half 0 | read half 1 of S | rest of half 0 | wait (the next
//   K-step's loads landed, half 1 read) | barrier | loads of kt+NST into S
//   (every wave is done with S) | read half 0 of S+1 | MFMA half 1.
// The first MFMA goes ahead of the half-1 reads because the compiler's wait
// for f0 is a full lgkmcnt(0), which must not cover reads issued after it;
// sched_barrier(0) keeps the compiler from merging the phases.  Past the end of
// K the last tile is loaded again into a stage nobody reads, so every K-step
// has the same shape.
template <class C, int S, int NST>
__device__ __forceinline__ void kstep(int kt, int KT, const Ctx<C>& x, Frag<C>& f0,
                                      v16i (&acc)[C::TN][C::TM]) {
    Frag<C> f1;
    mma<C, 0, 1>(f0, acc);
    __builtin_amdgcn_sched_barrier(0);
    read_frag<C, S, 1>(f1, x);
    __builtin_amdgcn_sched_barrier(0);
    mma<C, 1, C::NQ>(f0, acc);
    __builtin_amdgcn_sched_barrier(0);
    wait_vm_lgkm0<C::VM_PER_STEP * (NST - 2)>();
    __builtin_amdgcn_s_barrier();
    issue_loads<C>(stA<S>(), stB<S>(), x, (int64_t)min(kt + NST, KT - 1) * BK);
    read_frag<C, (S + 1) % NST, 0>(f0, x);
    __builtin_amdgcn_sched_barrier(0);
    mma<C, 0, C::NQ>(f1, acc);
    __builtin_amdgcn_sched_barrier(0);
}

// Register-class pins (empty asm): the accumulators stay in AGPRs to the end
// of the K loop, and each 32x32 block moves to VGPRs only where the epilogue
// uses it -- otherwise the compiler copies all of them at once and spills.
__device__ __forceinline__ void pin_agpr(v16i& v) { asm volatile("" : "+a"(v)); }
__device__ __forceinline__ void pin_vgpr(v16i& v) { asm volatile("" : "+v"(v)); }

// Epilogue shared by the kernels: lane l holds row m = l % 32 of each A block
// and, in registers 4g..4g+3, columns 8g + 4(l/32) + 0..3 of each B block.
template <class C>
__device__ __forceinline__ void epilogue(const GemmParams& p, v16i (&acc)[C::TN][C::TM], int m0, int n0,
                                         int wm, int wn, int lrow, int lhalf) {
    if (p.c_kind == C_I32) {
#pragma unroll
        for (int i = 0; i < C::TM; i++) {
            const int m = m0 + wm * C::WTM + i * 32 + lrow;
            if (m >= p.M) continue;
#pragma unroll
            for (int j = 0; j < C::TN; j++) {
                v16i blk = acc[j][i];
                pin_vgpr(blk);
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const int nb = n0 + wn * C::WTN + j * 32 + 8 * g + 4 * lhalf;
                    int32_t* dst = (int32_t*)p.C + (int64_t)m * p.ldc + nb;
                    const v4i a = v4i{blk[4 * g], blk[4 * g + 1], blk[4 * g + 2], blk[4 * g + 3]};
                    if (p.c_vec && nb + 3 < p.N) {
                        *(v4i*)dst = a;
                    } else {
                        for (int t = 0; t < 4 && nb + t < p.N; t++) dst[t] = a[t];
                    }
                }
            }
            // One block at a time: keeps the compiler from pulling every
            // accumulator out of AGPRs at once.
            __builtin_amdgcn_sched_barrier(0);
        }
        return;
    }
    // Per B block: its column scales and bias (fetched once per lane), then
    // every A block's rows.
#pragma unroll
    for (int j = 0; j < C::TN; j++) {
        v4f sbv[4], bzv[4];
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int nb = n0 + wn * C::WTN + j * 32 + 8 * g + 4 * lhalf;
            if (p.sb_scalar) {
                const float v = p.sB[0];
                sbv[g] = v4f{v, v, v, v};
            } else if (p.s_vec && nb + 3 < p.N) {
                sbv[g] = *(const v4f*)(p.sB + nb);
            } else {
#pragma unroll
                for (int t = 0; t < 4; t++) sbv[g][t] = p.sB[min(nb + t, p.N - 1)];
            }
            if (p.bias_kind == BIAS_F32) {
                if (p.s_vec && nb + 3 < p.N) {
                    bzv[g] = *(const v4f*)((const float*)p.bias + nb);
                } else {
#pragma unroll
                    for (int t = 0; t < 4; t++) bzv[g][t] = ((const float*)p.bias)[min(nb + t, p.N - 1)];
                }
            } else if (p.bias_kind == BIAS_BF16) {
                if (p.s_vec && nb + 3 < p.N) {
                    const uint2 h = *(const uint2*)((const uint16_t*)p.bias + nb);
                    bzv[g] = v4f{bf16_to_f32(h.x & 0xffffu), bf16_to_f32(h.x >> 16), bf16_to_f32(h.y & 0xffffu),
                                 bf16_to_f32(h.y >> 16)};
                } else {
#pragma unroll
                    for (int t = 0; t < 4; t++)
                        bzv[g][t] = bf16_to_f32(((const uint16_t*)p.bias)[min(nb + t, p.N - 1)]);
                }
            } else {
                bzv[g] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
#pragma unroll
        for (int i = 0; i < C::TM; i++) {
            const int m = m0 + wm * C::WTM + i * 32 + lrow;
            if (m >= p.M) continue;
            const float sa = p.sA[m];
            v16i blk = acc[j][i];
            pin_vgpr(blk);
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int nb = n0 + wn * C::WTN + j * 32 + 8 * g + 4 * lhalf;
                float v[4];
#pragma unroll
                for (int t = 0; t < 4; t++) v[t] = fmaf((float)blk[4 * g + t] * sa, sbv[g][t], bzv[g][t]);
                const int64_t off = (int64_t)m * p.ldc + nb;
                if (p.c_kind == C_BF16) {
                    uint16_t* dst = (uint16_t*)p.C + off;
                    if (p.c_vec && nb + 3 < p.N) {
                        *(uint2*)dst = make_uint2(f32x2_to_bf16x2(v[0], v[1]), f32x2_to_bf16x2(v[2], v[3]));
                    } else {
                        for (int t = 0; t < 4 && nb + t < p.N; t++) dst[t] = (uint16_t)f32_to_bf16(v[t]);
                    }
                } else {
                    float* dst = (float*)p.C + off;
                    if (p.c_vec && nb + 3 < p.N) {
                        *(v4f*)dst = v4f{v[0], v[1], v[2], v[3]};
                    } else {
                        for (int t = 0; t < 4 && nb + t < p.N; t++) dst[t] = v[t];
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// Epilogue operands fetched ahead: the column scales and bias of this lane's
// columns and the row scales of its rows, issued before the K loop so their
// latency hides behind it (kernels with registers to spare).
template <class C>
struct EpiPre {
    v4f sb[C::TN][4], bz[C::TN][4];
    float sa[C::TM];
};

template <class C>
__device__ __forceinline__ void epi_prefetch(const GemmParams& p, EpiPre<C>& e, int m0, int n0, int wm, int wn,
                                             int lrow, int lhalf) {
    if (p.c_kind == C_I32) return;
#pragma unroll
    for (int i = 0; i < C::TM; i++) e.sa[i] = p.sA[min(m0 + wm * C::WTM + i * 32 + lrow, p.M - 1)];
#pragma unroll
    for (int j = 0; j < C::TN; j++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int nb = n0 + wn * C::WTN + j * 32 + 8 * g + 4 * lhalf;
            if (p.sb_scalar) {
                const float v = p.sB[0];
                e.sb[j][g] = v4f{v, v, v, v};
            } else if (p.s_vec && nb + 3 < p.N) {
                e.sb[j][g] = *(const v4f*)(p.sB + nb);
            } else {
#pragma unroll
                for (int t = 0; t < 4; t++) e.sb[j][g][t] = p.sB[min(nb + t, p.N - 1)];
            }
            if (p.bias_kind == BIAS_F32) {
                if (p.s_vec && nb + 3 < p.N) {
                    e.bz[j][g] = *(const v4f*)((const float*)p.bias + nb);
                } else {
#pragma unroll
                    for (int t = 0; t < 4; t++) e.bz[j][g][t] = ((const float*)p.bias)[min(nb + t, p.N - 1)];
                }
            } else if (p.bias_kind == BIAS_BF16) {
                if (p.s_vec && nb + 3 < p.N) {
                    const uint2 h = *(const uint2*)((const uint16_t*)p.bias + nb);
                    e.bz[j][g] = v4f{bf16_to_f32(h.x & 0xffffu), bf16_to_f32(h.x >> 16), bf16_to_f32(h.y & 0xffffu),
                                     bf16_to_f32(h.y >> 16)};
                } else {
#pragma unroll
                    for (int t = 0; t < 4; t++)
                        e.bz[j][g][t] = bf16_to_f32(((const uint16_t*)p.bias)[min(nb + t, p.N - 1)]);
                }
            } else {
                e.bz[j][g] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
}

// The scaled stores with prefetched operands (the int32 path is epilogue()'s).
template <class C>
__device__ __forceinline__ void epilogue_pre(const GemmParams& p, v16i (&acc)[C::TN][C::TM], const EpiPre<C>& e,
                                             int m0, int n0, int wm, int wn, int lrow, int lhalf) {
    if (p.c_kind == C_I32) {
        epilogue<C>(p, acc, m0, n0, wm, wn, lrow, lhalf);
        return;
    }
#pragma unroll
    for (int j = 0; j < C::TN; j++) {
#pragma unroll
        for (int i = 0; i < C::TM; i++) {
            const int m = m0 + wm * C::WTM + i * 32 + lrow;
            if (m >= p.M) continue;
            v16i blk = acc[j][i];
            pin_vgpr(blk);
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int nb = n0 + wn * C::WTN + j * 32 + 8 * g + 4 * lhalf;
                float v[4];
#pragma unroll
                for (int t = 0; t < 4; t++) v[t] = fmaf((float)blk[4 * g + t] * e.sa[i], e.sb[j][g][t], e.bz[j][g][t]);
                const int64_t off = (int64_t)m * p.ldc + nb;
                if (p.c_kind == C_BF16) {
                    uint16_t* dst = (uint16_t*)p.C + off;
                    if (p.c_vec && nb + 3 < p.N) {
                        *(uint2*)dst = make_uint2(f32x2_to_bf16x2(v[0], v[1]), f32x2_to_bf16x2(v[2], v[3]));
                    } else {
                        for (int t = 0; t < 4 && nb + t < p.N; t++) dst[t] = (uint16_t)f32_to_bf16(v[t]);
                    }
                } else {
                    float* dst = (float*)p.C + off;
                    if (p.c_vec && nb + 3 < p.N) {
                        *(v4f*)dst = v4f{v[0], v[1], v[2], v[3]};
                    } else {
                        for (int t = 0; t < 4 && nb + t < p.N; t++) dst[t] = v[t];
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

}  // namespace

template <int WM, int WN, int NST>
__global__ __launch_bounds__(WM* WN * 64) void i8_gemm_256_kernel(GemmParams p) {
    using C = Cfg<WM, WN, NST>;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + BN - 1) / BN;
    int tm, tn;
    tile_of(blockIdx.x, gridDim.x, tiles_m, tiles_n, p.group_m, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;

    // Direct-to-LDS sources: wave w fills 16*DMA consecutive rows of each
    // operand tile (DMA instructions of 16 rows); lane l fetches row l/4 of
    // its 16-row block and the chunk whose swizzled slot is l % 4.
    Ctx<C> x;
    x.dma_off = wave * (C::DMA * 1024);
#pragma unroll
    for (int j = 0; j < C::DMA; j++) {
        const int row = (wave * C::DMA + j) * 16 + (lane >> 2);
        const int chunk = swz(row, lane & 3);
        const int gm = min(m0 + row, p.M - 1);
        const int gn = min(n0 + row, p.N - 1);
        x.gA[j] = p.A + (int64_t)gm * p.lda + chunk * 16;
        x.gB[j] = p.B + (int64_t)gn * p.ldb + chunk * 16;
    }
    // Fragment read offsets; K half-step s reads chunk 2s + lane/32.
    const int lrow = lane & 31, lhalf = lane >> 5;
#pragma unroll
    for (int i = 0; i < C::TM; i++) {
        const int row = wm * C::WTM + i * 32 + lrow;
#pragma unroll
        for (int s = 0; s < 2; s++) x.oA[i][s] = row * BK + swz(row, 2 * s + lhalf) * 16;
    }
#pragma unroll
    for (int j = 0; j < C::TN; j++) {
        const int row = wn * C::WTN + j * 32 + lrow;
#pragma unroll
        for (int s = 0; s < 2; s++) x.oB[j][s] = row * BK + swz(row, 2 * s + lhalf) * 16;
    }

    v16i acc[C::TN][C::TM];
#pragma unroll
    for (int j = 0; j < C::TN; j++)
#pragma unroll
        for (int i = 0; i < C::TM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[j][i][r] = 0;

    const int KT = p.K / BK;
    // Prologue: K-steps 0..NST-1 in flight (clamped to the last K-step).
    issue_loads<C>(lA0, lB0, x, 0);
    issue_loads<C>(lA1, lB1, x, (int64_t)min(1, KT - 1) * BK);
    issue_loads<C>(lA2, lB2, x, (int64_t)min(2, KT - 1) * BK);
    if (NST == 4) issue_loads<C>(stA<3>(), stB<3>(), x, (int64_t)min(3, KT - 1) * BK);
    wait_vm_lgkm0<C::VM_PER_STEP * (NST - 1)>();
    __builtin_amdgcn_s_barrier();
    Frag<C> f0;
    read_frag<C, 0, 0>(f0, x);

    int kt = 0;
    for (; kt + NST <= KT; kt += NST) {
        kstep<C, 0, NST>(kt, KT, x, f0, acc);
        kstep<C, 1, NST>(kt + 1, KT, x, f0, acc);
        kstep<C, 2, NST>(kt + 2, KT, x, f0, acc);
        if (NST == 4) kstep<C, 3 % NST, NST>(kt + 3, KT, x, f0, acc);
    }
    if (kt < KT) kstep<C, 0, NST>(kt, KT, x, f0, acc);
    if (kt + 1 < KT) kstep<C, 1, NST>(kt + 1, KT, x, f0, acc);
    if (NST == 4 && kt + 2 < KT) kstep<C, 2, NST>(kt + 2, KT, x, f0, acc);
    // No load may still be writing LDS when the workgroup ends.
    wait_vm_lgkm0<0>();

    epilogue<C>(p, acc, m0, n0, wm, wn, lrow, lhalf);
}

// ---------------------------------------------------------------------------
// Four waves of 128 x 128 (4 x 4 MFMA blocks each) on 128-deep K-steps: half
// the LDS fragment reads per MFMA of the eight-wave form.  The 256
// accumulator registers live in AGPRs; LDS rows are 128 bytes (8 lanes fetch
// one whole 128-byte line per direct-to-LDS load); two stages of 64 KB.
namespace w4 {

constexpr int BK4 = 128;
constexpr int STG = BM * BK4;  // 32 KB per operand per stage
constexpr int DMA = STG / 1024 / 4;  // 8 eight-row loads per operand per wave

__shared__ __align__(16) int8_t tA0[STG];
__shared__ __align__(16) int8_t tA1[STG];
__shared__ __align__(16) int8_t tB0[STG];
__shared__ __align__(16) int8_t tB1[STG];

template <int S>
__device__ __forceinline__ int8_t* la() { return S == 0 ? tA0 : tA1; }
template <int S>
__device__ __forceinline__ int8_t* lb() { return S == 0 ? tB0 : tB1; }

// Chunk c (0..7) of row r sits in slot c ^ ((r >> 1) & 7): the operand read
// of 16 consecutive rows (row parity x slot) covers all 16 bank windows of a
// 256-byte LDS clock.  It depends on row bits 1..3 only, so the four 32-row A
// (or B) blocks of a wave share one offset register plus an immediate.
__device__ __forceinline__ int swz8(int row, int c) { return c ^ ((row >> 1) & 7); }

struct Frag4 {
    v4i a[4], b[4];
};

struct Ctx4 {
    const int8_t* gA[DMA];
    const int8_t* gB[DMA];
    int dma_off;
    int oA[4], oB[4];  // per quarter (32-deep K slice)
};

__device__ __forceinline__ void loads(int8_t* sa, int8_t* sb, const Ctx4& x, int64_t koff) {
#pragma unroll
    for (int j = 0; j < DMA; j++) dma16(x.gA[j] + koff, sa + x.dma_off + j * 1024);
#pragma unroll
    for (int j = 0; j < DMA; j++) dma16(x.gB[j] + koff, sb + x.dma_off + j * 1024);
}

template <int S, int Q>
__device__ __forceinline__ void frag(Frag4& f, const Ctx4& x) {
    const int8_t* cA = la<S>() + x.oA[Q];
    const int8_t* cB = lb<S>() + x.oB[Q];
#pragma unroll
    for (int i = 0; i < 4; i++) f.a[i] = *(const v4i*)(cA + i * 32 * BK4);
#pragma unroll
    for (int j = 0; j < 4; j++) f.b[j] = *(const v4i*)(cB + j * 32 * BK4);
}

template <int FIRST, int LAST>
__device__ __forceinline__ void mma4(const Frag4& f, v16i (&acc)[4][4]) {
#pragma unroll
    for (int q = FIRST; q < LAST; q++) {
        const int j = q / 4, i = q % 4;
        acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.b[j], f.a[i], acc[j][i], 0, 0, 0);
    }
}

// Scheduling groups (sched_group_barrier masks): MFMA, DS read, VMEM.
constexpr int SG_MFMA = 0x008, SG_DSR = 0x100, SG_VMEM = 0x020;

// MFMA quarter with the next quarter's eight fragment reads threaded between
// its MFMAs (one wave per SIMD: every issue slot outside the MFMA stream is an
// idle matrix pipe).  The first MFMA goes ahead of the reads because the
// compiler's wait for `cur` is a full lgkmcnt(0).
template <int S, int QN>
__device__ __forceinline__ void quarter(const Frag4& cur, Frag4& nxt, const Ctx4& x, v16i (&acc)[4][4]) {
    mma4<0, 16>(cur, acc);
    frag<S, QN>(nxt, x);
    __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
#pragma unroll
    for (int t = 0; t < 8; t++) {
        __builtin_amdgcn_sched_group_barrier(SG_DSR, 1, 0);
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(SG_MFMA, 7, 0);
    __builtin_amdgcn_sched_barrier(0);
}

// One 128-deep K-step on stage S; f0 holds quarter 0 on entry and quarter 0
// of the other stage on exit.  The barrier precedes the last quarter's MFMAs:
// every wave has read all of S and this wave's loads of the next K-step have
// landed; then the K-step two ahead is loaded into S (the last one again past
// the end of K, unread), its 16 loads and the next stage's first reads
// threaded between the last quarter's MFMAs.
template <int S>
__device__ __forceinline__ void step(int kt, int KT, const Ctx4& x, Frag4& f0, v16i (&acc)[4][4]) {
    Frag4 f1;
    quarter<S, 1>(f0, f1, x, acc);
    quarter<S, 2>(f1, f0, x, acc);
    quarter<S, 3>(f0, f1, x, acc);
    wait_vm_lgkm0<0>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    mma4<0, 16>(f1, acc);
    loads(la<S>(), lb<S>(), x, (int64_t)min(kt + 2, KT - 1) * BK4);
    frag<S ^ 1, 0>(f0, x);
#pragma unroll
    for (int t = 0; t < 8; t++) {
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
        __builtin_amdgcn_sched_group_barrier(SG_VMEM, 1, 0);
        __builtin_amdgcn_sched_group_barrier(SG_DSR, 1, 0);
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
        __builtin_amdgcn_sched_group_barrier(SG_VMEM, 1, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
}

struct Cfg4 {
    static constexpr int WTM = 128, WTN = 128, TM = 4, TN = 4;
};

// bf16 epilogue through LDS.  Each wave owns one 32 KB stage buffer (free once
// the K loop is done and every wave has passed the barrier) and writes its
// 128 x 128 bf16 block there row-major, 256 bytes a row, the 16-byte chunk q
// of row r at chunk q ^ (r & 15); it then reads whole rows back, 16 lanes per
// row, so each global store instruction writes four complete 256-byte rows
// (instead of 32 scattered 16-byte pieces straight from the MFMA layout).
__device__ __forceinline__ void epilogue_bf16_lds(const GemmParams& p, v16i (&acc)[4][4],
                                                  const EpiPre<Cfg4>& e, int8_t* lds, int m0, int n0,
                                                  int wm, int wn, int lane) {
    const int lrow = lane & 31, lhalf = lane >> 5;
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v16i blk = acc[j][i];
            pin_vgpr(blk);
            const int lr = i * 32 + lrow;
#pragma unroll
            for (int g = 0; g < 4; g++) {
                float v[4];
#pragma unroll
                for (int t = 0; t < 4; t++) v[t] = fmaf((float)blk[4 * g + t] * e.sa[i], e.sb[j][g][t], e.bz[j][g][t]);
                const int q = j * 4 + g;
                *(uint2*)(lds + lr * 256 + ((q ^ (lr & 15)) << 4) + lhalf * 8) =
                    make_uint2(f32x2_to_bf16x2(v[0], v[1]), f32x2_to_bf16x2(v[2], v[3]));
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // A wave's LDS accesses complete in order: its reads below see its writes.
    const int q = lane & 15;
    const int n = n0 + wn * 128 + q * 8;
#pragma unroll 4
    for (int t = 0; t < 32; t++) {
        const int lr = t * 4 + (lane >> 4);
        const int m = m0 + wm * 128 + lr;
        const uint4 w = *(const uint4*)(lds + lr * 256 + ((q ^ (lr & 15)) << 4));
        if (m >= p.M) continue;
        uint16_t* dst = (uint16_t*)p.C + (int64_t)m * p.ldc + n;
        if (n + 7 < p.N) {
            *(uint4*)dst = w;
        } else {
            const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
            for (int c = 0; c < 8 && n + c < p.N; c++) dst[c] = (uint16_t)(ww[c >> 1] >> (16 * (c & 1)));
        }
    }
}

}  // namespace w4

__global__ __launch_bounds__(256) void i8_gemm_w4_kernel(GemmParams p) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + BN - 1) / BN;
    int tm, tn;
    tile_of(blockIdx.x, gridDim.x, tiles_m, tiles_n, p.group_m, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;

    // Wave w fills rows 64w..64w+63 of each operand stage: eight loads of 8
    // rows; lane l fetches row l/8 and the chunk whose swizzled slot is l % 8.
    w4::Ctx4 x;
    x.dma_off = wave * (w4::DMA * 1024);
#pragma unroll
    for (int j = 0; j < w4::DMA; j++) {
        const int row = wave * 64 + j * 8 + (lane >> 3);
        const int chunk = w4::swz8(row, lane & 7);
        const int gm = min(m0 + row, p.M - 1);
        const int gn = min(n0 + row, p.N - 1);
        x.gA[j] = p.A + (int64_t)gm * p.lda + chunk * 16;
        x.gB[j] = p.B + (int64_t)gn * p.ldb + chunk * 16;
    }
    const int lrow = lane & 31, lhalf = lane >> 5;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        x.oA[q] = (wm * 128 + lrow) * w4::BK4 + w4::swz8(lrow, 2 * q + lhalf) * 16;
        x.oB[q] = (wn * 128 + lrow) * w4::BK4 + w4::swz8(lrow, 2 * q + lhalf) * 16;
    }

    v16i acc[4][4];
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[j][i][r] = 0;

    const int KT = p.K / w4::BK4;
    w4::loads(w4::tA0, w4::tB0, x, 0);
    w4::loads(w4::tA1, w4::tB1, x, (int64_t)min(1, KT - 1) * w4::BK4);
    wait_vm_lgkm0<2 * w4::DMA>();
    __builtin_amdgcn_s_barrier();
    w4::Frag4 f0;
    w4::frag<0, 0>(f0, x);
    int kt = 0;
    for (; kt + 2 <= KT; kt += 2) {
        w4::step<0>(kt, KT, x, f0, acc);
        w4::step<1>(kt + 1, KT, x, f0, acc);
    }
    if (kt < KT) w4::step<0>(kt, KT, x, f0, acc);
    wait_vm_lgkm0<0>();
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) pin_agpr(acc[j][i]);

    EpiPre<w4::Cfg4> epre;
    epi_prefetch<w4::Cfg4>(p, epre, m0, n0, wm, wn, lrow, lhalf);
    if (p.c_kind == C_BF16 && p.c_vec16) {
        __builtin_amdgcn_s_barrier();  // every wave is done with the stage buffers
        int8_t* lds = wave == 0 ? w4::tA0 : wave == 1 ? w4::tA1 : wave == 2 ? w4::tB0 : w4::tB1;
        w4::epilogue_bf16_lds(p, acc, epre, lds, m0, n0, wm, wn, lane);
    } else {
        epilogue_pre<w4::Cfg4>(p, acc, epre, m0, n0, wm, wn, lrow, lhalf);
    }
}

template <int WM, int WN, int NST>
static hipError_t launch_256(hipStream_t stream, const GemmParams& p) {
    const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
    hipLaunchKernelGGL((i8_gemm_256_kernel<WM, WN, NST>), dim3(tiles), dim3(WM * WN * 64), 0, stream, p);
    return hipGetLastError();
}

// schedule 0: eight 128x64 waves on 64-deep K-steps (any K % 64 == 0);
// schedule 1: four 128x128 waves on 128-deep K-steps (K % 128 == 0).
hipError_t launch_i8_gemm_256(hipStream_t stream, const GemmParams& p) {
    if (p.schedule == 1) {
        if (p.K % 128 != 0) return hipErrorInvalidValue;
        const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
        hipLaunchKernelGGL(i8_gemm_w4_kernel, dim3(tiles), dim3(256), 0, stream, p);
        return hipGetLastError();
    }
    return launch_256<2, 4, 3>(stream, p);
}

}  // namespace phi_dev
