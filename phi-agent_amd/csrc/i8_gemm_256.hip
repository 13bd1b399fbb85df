// Large-tile int8 GEMM for gfx950: 256 x 256 output tiles, 8 waves, operands
// streamed global -> LDS by the direct-to-LDS loads (no staging registers).
//
//   acc[m,n] = sum_k A[m,k] * B[n,k]                  (exact int32)
//   C[m,n]   = fma((float)acc * sA[m], sB[n], bias[n])  -> fp32 / bf16 (RNE) / raw int32
//
// The product and epilogue are those of the reference's int8_gemm_tc
// (core/kernels/int8_gemm.cpp:466-621, epilogue :588-620) and host gemm_int8
// (core/host/quant.cpp:223-236).
//
// Design:
//   * Workgroup tile 256 x 256, K-step 64 bytes, 512 threads = 8 waves laid out
//     2 (M) x 4 (N); each wave owns 128 x 64 outputs as 4 x 2 blocks of
//     v_mfma_i32_32x32x32_i8.  The B fragment is the instruction's first
//     operand, so a lane ends up holding one output row m and, per group of four
//     registers, four consecutive columns n -- the epilogue stores 8 or 16
//     contiguous bytes per lane.
//   * Three LDS stages of (A 16 KB + B 16 KB), each a separate __shared__ object
//     so the compiler's LDS-DMA wait tracking tells them apart.  One barrier
//     per K-step, between its two MFMA halves; loads run three K-steps ahead
//     and the wait before the barrier only retires the next K-step's loads
//     (vmcnt counts four loads per wave per K-step).
//   * Global -> LDS uses global_load_lds_dwordx4: a wave instruction fills 1 KB
//     of LDS, lane l writing bytes 16l..16l+15.  LDS rows are 64 bytes; the
//     16-byte chunk c of row r sits in slot c ^ (((r >> 1) ^ (r >> 2)) & 3),
//     realised by choosing which global chunk each lane fetches.  The LDS
//     serves a 16-byte read for 16 lanes (256 bytes) per clock; the operand
//     read of 16 consecutive rows then covers all 16 bank windows, and so do
//     any 8 consecutive rows.
//   * Tile order: the hardware deals workgroups round-robin to the 8 XCDs, so
//     the id is remapped to give each XCD a contiguous run of tiles, walked
//     group_m tile-rows at a time (concurrent tiles of one XCD share A rows and
//     B columns in that XCD's L2).
#include "device_common.hpp"
#include "i8_gemm.hpp"

namespace phi_dev {

namespace {

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int NTHR = 512;
constexpr int WAVES_N = 4;
constexpr int WTM = 128, WTN = 64;             // wave tile
constexpr int TM = WTM / 32, TN = WTN / 32;    // 4 x 2 MFMA blocks
constexpr int STAGE_BYTES = BM * BK;           // 16 KB per operand per stage
constexpr int DMA_PER_WAVE = 2;                // 1 KB wave loads per operand per K-step
constexpr int VM_PER_STEP = 2 * DMA_PER_WAVE;  // loads per wave per K-step

__shared__ __align__(16) int8_t lA0[STAGE_BYTES];
__shared__ __align__(16) int8_t lA1[STAGE_BYTES];
__shared__ __align__(16) int8_t lA2[STAGE_BYTES];
__shared__ __align__(16) int8_t lB0[STAGE_BYTES];
__shared__ __align__(16) int8_t lB1[STAGE_BYTES];
__shared__ __align__(16) int8_t lB2[STAGE_BYTES];

typedef __attribute__((address_space(1))) const void* gptr_t;
typedef __attribute__((address_space(3))) void* lptr_t;

__device__ __forceinline__ void dma16(const int8_t* g, int8_t* l) {
    __builtin_amdgcn_global_load_lds((gptr_t)g, (lptr_t)l, 16, 0, 0);
}

// s_waitcnt with vmcnt(n), lgkmcnt(0), expcnt untouched (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | (((N >> 4) & 3) << 14));
}

__device__ __forceinline__ int swz(int row, int c) { return c ^ (((row >> 1) ^ (row >> 2)) & 3); }

template <int S>
__device__ __forceinline__ int8_t* stA() { return S == 0 ? lA0 : S == 1 ? lA1 : lA2; }
template <int S>
__device__ __forceinline__ int8_t* stB() { return S == 0 ? lB0 : S == 1 ? lB1 : lB2; }

// Workgroup id -> (tile_m, tile_n): XCD remap, then grouped walk.
__device__ __forceinline__ void tile_of(int pid, int nblocks, int tiles_m, int tiles_n, int group_m,
                                        int& tm, int& tn) {
    const int xcd = pid & 7, idx = pid >> 3;
    const int base = nblocks >> 3, rem = nblocks & 7;
    const int logical = xcd < rem ? xcd * (base + 1) + idx : rem * (base + 1) + (xcd - rem) * base + idx;
    const int per_group = group_m * tiles_n;
    const int gid = logical / per_group;
    const int first_m = gid * group_m;
    const int gsz = min(tiles_m - first_m, group_m);
    const int in_group = logical - gid * per_group;
    tm = first_m + in_group % gsz;
    tn = in_group / gsz;
}

struct Frag {
    v4i a[TM], b[TN];
};

// Fragments of K half-step H (0 or 1) from LDS stage S.
template <int S, int H>
__device__ __forceinline__ void read_frag(Frag& f, const int (&oA)[TM][2], const int (&oB)[TN][2]) {
    const int8_t* cA = stA<S>();
    const int8_t* cB = stB<S>();
#pragma unroll
    for (int i = 0; i < TM; i++) f.a[i] = *(const v4i*)(cA + oA[i][H]);
#pragma unroll
    for (int j = 0; j < TN; j++) f.b[j] = *(const v4i*)(cB + oB[j][H]);
}

// MFMAs number FIRST..LAST-1 of one half-step (8 in all: 2 B blocks x 4 A blocks).
template <int FIRST, int LAST>
__device__ __forceinline__ void mma(const Frag& f, v16i (&acc)[TN][TM]) {
#pragma unroll
    for (int q = FIRST; q < LAST; q++) {
        const int j = q / TM, i = q % TM;
        acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.b[j], f.a[i], acc[j][i], 0, 0, 0);
    }
}

__device__ __forceinline__ void issue_loads(int8_t* sa, int8_t* sb, const int8_t* const (&gA)[DMA_PER_WAVE],
                                            const int8_t* const (&gB)[DMA_PER_WAVE], int64_t koff, int dma_off) {
#pragma unroll
    for (int j = 0; j < DMA_PER_WAVE; j++) dma16(gA[j] + koff, sa + dma_off + j * 1024);
#pragma unroll
    for (int j = 0; j < DMA_PER_WAVE; j++) dma16(gB[j] + koff, sb + dma_off + j * 1024);
}

// One K-step on LDS stage S.  On entry f0 holds half-step 0 of this stage; on
// exit it holds half-step 0 of the next stage.  The barrier sits between the
// two MFMA halves, so fragment reads always overlap MFMAs:
//   read half 1 of S | MFMA half 0 | wait (loads of kt+1 landed, half 1 read)
//   | barrier | loads of kt+3 into S (every wave is done with S)
//   | read half 0 of S+1 | MFMA half 1.
// Past the end of K the last tile is loaded again into a stage nobody reads,
// so every K-step has the same shape.
template <int S>
__device__ __forceinline__ void kstep(int kt, int KT, const int8_t* const (&gA)[DMA_PER_WAVE],
                                      const int8_t* const (&gB)[DMA_PER_WAVE], int dma_off,
                                      const int (&oA)[TM][2], const int (&oB)[TN][2], Frag& f0,
                                      v16i (&acc)[TN][TM]) {
    // sched_barrier(0) keeps the compiler from merging the phases (it would
    // otherwise reuse one register set and serialise reads and MFMAs).
    // The first MFMA goes ahead of the half-1 reads: the compiler's wait for
    // f0 is a full lgkmcnt(0), which must not cover reads issued after it.
    constexpr int NQ = TM * TN;
    Frag f1;
    mma<0, 1>(f0, acc);
    __builtin_amdgcn_sched_barrier(0);
    read_frag<S, 1>(f1, oA, oB);
    __builtin_amdgcn_sched_barrier(0);
    mma<1, NQ>(f0, acc);
    __builtin_amdgcn_sched_barrier(0);
    wait_vm_lgkm0<VM_PER_STEP>();
    __builtin_amdgcn_s_barrier();
    issue_loads(stA<S>(), stB<S>(), gA, gB, (int64_t)min(kt + 3, KT - 1) * BK, dma_off);
    read_frag<(S + 1) % 3, 0>(f0, oA, oB);
    __builtin_amdgcn_sched_barrier(0);
    mma<0, NQ>(f1, acc);
    __builtin_amdgcn_sched_barrier(0);
}

}  // namespace

__global__ __launch_bounds__(NTHR) void i8_gemm_256_kernel(GemmParams p) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + BN - 1) / BN;
    int tm, tn;
    tile_of(blockIdx.x, gridDim.x, tiles_m, tiles_n, p.group_m, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;

    // Direct-to-LDS sources: wave w fills rows 32w..32w+31 of each operand tile
    // (two 1 KB instructions of 16 rows); lane l fetches row 16j + l/4 and the
    // chunk whose swizzled slot is l % 4.
    const int dma_off = wave * (DMA_PER_WAVE * 1024);
    const int8_t* gA[DMA_PER_WAVE];
    const int8_t* gB[DMA_PER_WAVE];
#pragma unroll
    for (int j = 0; j < DMA_PER_WAVE; j++) {
        const int row = wave * 32 + j * 16 + (lane >> 2);
        const int chunk = swz(row, lane & 3);
        const int gm = min(m0 + row, p.M - 1);
        const int gn = min(n0 + row, p.N - 1);
        gA[j] = p.A + (int64_t)gm * p.lda + chunk * 16;
        gB[j] = p.B + (int64_t)gn * p.ldb + chunk * 16;
    }

    // Fragment read offsets; K half-step s reads chunk 2s + lane/32.
    const int lrow = lane & 31, lhalf = lane >> 5;
    int oA[TM][2], oB[TN][2];
#pragma unroll
    for (int i = 0; i < TM; i++) {
        const int row = wm * WTM + i * 32 + lrow;
#pragma unroll
        for (int s = 0; s < 2; s++) oA[i][s] = row * BK + swz(row, 2 * s + lhalf) * 16;
    }
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int row = wn * WTN + j * 32 + lrow;
#pragma unroll
        for (int s = 0; s < 2; s++) oB[j][s] = row * BK + swz(row, 2 * s + lhalf) * 16;
    }

    v16i acc[TN][TM];
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[j][i][r] = 0;

    const int KT = p.K / BK;
    // Prologue: K-steps 0, 1, 2 in flight (clamped to the last K-step).
    issue_loads(lA0, lB0, gA, gB, 0, dma_off);
    issue_loads(lA1, lB1, gA, gB, (int64_t)min(1, KT - 1) * BK, dma_off);
    issue_loads(lA2, lB2, gA, gB, (int64_t)min(2, KT - 1) * BK, dma_off);
    wait_vm_lgkm0<2 * VM_PER_STEP>();
    __builtin_amdgcn_s_barrier();
    Frag f0;
    read_frag<0, 0>(f0, oA, oB);

    int kt = 0;
    for (; kt + 3 <= KT; kt += 3) {
        kstep<0>(kt, KT, gA, gB, dma_off, oA, oB, f0, acc);
        kstep<1>(kt + 1, KT, gA, gB, dma_off, oA, oB, f0, acc);
        kstep<2>(kt + 2, KT, gA, gB, dma_off, oA, oB, f0, acc);
    }
    if (kt < KT) kstep<0>(kt, KT, gA, gB, dma_off, oA, oB, f0, acc);
    if (kt + 1 < KT) kstep<1>(kt + 1, KT, gA, gB, dma_off, oA, oB, f0, acc);
    // No load may still be writing LDS when the workgroup ends.
    wait_vm_lgkm0<0>();

    // ---- epilogue ----
    // Lane l holds row m = l % 32 of each A block and, in registers 4g..4g+3,
    // columns 8g + 4(l/32) + 0..3 of each B block.
    if (p.c_kind == C_I32) {
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int m = m0 + wm * WTM + i * 32 + lrow;
            if (m >= p.M) continue;
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const int nb = n0 + wn * WTN + j * 32 + 8 * g + 4 * lhalf;
                    int32_t* dst = (int32_t*)p.C + (int64_t)m * p.ldc + nb;
                    const v4i a = v4i{acc[j][i][4 * g], acc[j][i][4 * g + 1], acc[j][i][4 * g + 2], acc[j][i][4 * g + 3]};
                    if (p.c_vec && nb + 3 < p.N) {
                        *(v4i*)dst = a;
                    } else {
                        for (int t = 0; t < 4 && nb + t < p.N; t++) dst[t] = a[t];
                    }
                }
        }
        return;
    }
    // Column scales and bias for this lane's 32 columns, fetched once.
    v4f sbv[TN][4], bzv[TN][4];
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int nb = n0 + wn * WTN + j * 32 + 8 * g + 4 * lhalf;
            if (p.sb_scalar) {
                const float v = p.sB[0];
                sbv[j][g] = v4f{v, v, v, v};
            } else if (p.s_vec && nb + 3 < p.N) {
                sbv[j][g] = *(const v4f*)(p.sB + nb);
            } else {
#pragma unroll
                for (int t = 0; t < 4; t++) sbv[j][g][t] = p.sB[min(nb + t, p.N - 1)];
            }
            if (p.bias_kind == BIAS_F32) {
                if (p.s_vec && nb + 3 < p.N) {
                    bzv[j][g] = *(const v4f*)((const float*)p.bias + nb);
                } else {
#pragma unroll
                    for (int t = 0; t < 4; t++) bzv[j][g][t] = ((const float*)p.bias)[min(nb + t, p.N - 1)];
                }
            } else if (p.bias_kind == BIAS_BF16) {
                if (p.s_vec && nb + 3 < p.N) {
                    const uint2 h = *(const uint2*)((const uint16_t*)p.bias + nb);
                    bzv[j][g] = v4f{bf16_to_f32(h.x & 0xffffu), bf16_to_f32(h.x >> 16), bf16_to_f32(h.y & 0xffffu),
                                    bf16_to_f32(h.y >> 16)};
                } else {
#pragma unroll
                    for (int t = 0; t < 4; t++)
                        bzv[j][g][t] = bf16_to_f32(((const uint16_t*)p.bias)[min(nb + t, p.N - 1)]);
                }
            } else {
                bzv[j][g] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
#pragma unroll
    for (int i = 0; i < TM; i++) {
        const int m = m0 + wm * WTM + i * 32 + lrow;
        if (m >= p.M) continue;
        const float sa = p.sA[m];
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int nb = n0 + wn * WTN + j * 32 + 8 * g + 4 * lhalf;
                float v[4];
#pragma unroll
                for (int t = 0; t < 4; t++) v[t] = fmaf((float)acc[j][i][4 * g + t] * sa, sbv[j][g][t], bzv[j][g][t]);
                const int64_t off = (int64_t)m * p.ldc + nb;
                if (p.c_kind == C_BF16) {
                    uint16_t* dst = (uint16_t*)p.C + off;
                    if (p.c_vec && nb + 3 < p.N) {
                        *(uint2*)dst = make_uint2(f32_to_bf16(v[0]) | (f32_to_bf16(v[1]) << 16),
                                                  f32_to_bf16(v[2]) | (f32_to_bf16(v[3]) << 16));
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
    }
}

hipError_t launch_i8_gemm_256(hipStream_t stream, const GemmParams& p) {
    const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
    hipLaunchKernelGGL(i8_gemm_256_kernel, dim3(tiles), dim3(NTHR), 0, stream, p);
    return hipGetLastError();
}

}  // namespace phi_dev
