// The runtime LoRA correction of a linear, out += (x A^T) B^T, as the
// reference runs it (apply_lora_tail, core/models/model_common.cpp:1667-1700):
//
//   lora_down      h[m, r] = sum_k x[m, k] * A[r, k]          (dispatch_gemm_f16 with
//                  fp32 operands and no bias, core/kernels/gemm_f16.cpp:56-200)
//   lora_rank_add  out[m, n] += sum_r h[m, r] * B[n, r]       (dispatch_lora_rank_add,
//                  core/kernels/gemm_f16.cpp:237-308)
//
// Both are fp32 fma chains in a fixed order: the reference accumulates
// acc = fma(a, b, acc) (NVRTC's default --fmad=true) with k ascending from 0
// for h, and with r ascending from out's own value for the rank add.  Each
// output here runs the same chain in one lane, so the bits are the
// reference's; the tiling only decides which lane owns which outputs.
// lora_down pads K to its 32-deep tiles with zero products; the only effect
// of that padding is fma(0, 0, -0) = +0, reproduced by one extra fma when
// K % 32 != 0.
//
// The chains are VALU work (R fmas per output element of the rank add), so
// both kernels are sized for VALU issue: operands staged through LDS
// transposed (k- or r-major), read with 16-byte loads, many accumulators per
// lane.
#include <cstdlib>

#include "device_common.hpp"
#include "lora.hpp"

namespace phi_dev {

// ---- lora_down: h [M, R] = x [M, K] . A [R, K]^T -------------------------
// Main form (x rows 16-byte aligned, K % 64 == 0): a block owns 64 rows and
// 4 LD_TR ranks, a wave LD_TR of the ranks and a lane one row.  Each 64-k
// chunk of the rows' x and of the waves' A slices goes global -> registers ->
// LDS, double-buffered with one barrier a chunk, the next chunk's global
// loads in flight under the current chunk's fmas.  A lane reads its own row
// of x (68-float pitch: 16-byte aligned rows, conflict-free 16-byte reads and
// writes) and its wave's A values, which all the wave's lanes read at one
// address (a broadcast).  Earlier the A values came through the scalar cache;
// scalar loads complete out of order, so only a full wait covers them, and
// each 8-k step waited on a batch that missed the scalar cache.  LD_TR = 2
// by default (PHI_LORA_TR=1 or 4 as A/B switches).
constexpr int LD_KC = 64, LD_XP = LD_KC + 4;

// TR consecutive floats (a TR * 4-byte aligned address) to and from registers.
template <int TR>
__device__ __forceinline__ void load_tr(const float* __restrict__ p, float (&v)[TR]) {
    if constexpr (TR == 4) {
        const float4 t = *(const float4*)p;
        v[0] = t.x, v[1] = t.y, v[2] = t.z, v[3] = t.w;
    } else if constexpr (TR == 2) {
        const float2 t = *(const float2*)p;
        v[0] = t.x, v[1] = t.y;
    } else {
        v[0] = *p;
    }
}

template <int TR>
__device__ __forceinline__ void store_tr(float* p, const float (&v)[TR]) {
    if constexpr (TR == 4) *(float4*)p = make_float4(v[0], v[1], v[2], v[3]);
    else if constexpr (TR == 2) *(float2*)p = make_float2(v[0], v[1]);
    else *p = v[0];
}

// 64 rows x 64 k of x into registers: lane t holds row t / 4, k 16 (t % 4)..+15.
template <bool XB>
__device__ __forceinline__ void fetch_x_tile(const void* __restrict__ x, int64_t ldx, int m0, int M, int k0,
                                             float (&v)[16]) {
    const int row = threadIdx.x >> 2, kk = (threadIdx.x & 3) * 16;
    const int64_t off = (int64_t)min(m0 + row, M - 1) * ldx + k0 + kk;
    if (XB) {
        const uint4 a = *(const uint4*)((const uint16_t*)x + off), b = *(const uint4*)((const uint16_t*)x + off + 8);
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            v[2 * i] = bf16_to_f32(w[i] & 0xffffu);
            v[2 * i + 1] = bf16_to_f32(w[i] >> 16);
        }
    } else {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 t = *(const float4*)((const float*)x + off + 4 * q);
            v[4 * q] = t.x, v[4 * q + 1] = t.y, v[4 * q + 2] = t.z, v[4 * q + 3] = t.w;
        }
    }
}

template <bool XB, int LD_TR>
__global__ __launch_bounds__(256) void lora_down_rows_kernel(const void* __restrict__ x, int64_t ldx,
                                                             const float* __restrict__ A, float* __restrict__ h,
                                                             int M, int K, int R) {
    __shared__ __align__(16) float sx[2][64 * LD_XP];
    __shared__ __align__(16) float sa[2][4][LD_TR * LD_KC];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int m0 = blockIdx.x * 64;
    const int rb = (blockIdx.y * 4 + wave) * LD_TR;
    const bool live = rb < R;  // wave-uniform; a dead wave still stages x for the others
    // The wave's A slice of a chunk (LD_TR ranks x 64 k, rank-major): lane l
    // holds LD_TR consecutive k of rank l / LPR.  Ranks past R read rank R - 1.
    constexpr int LPR = LD_KC / LD_TR;
    const int at = lane / LPR, ak = (lane % LPR) * LD_TR;
    const float* arow = A + (int64_t)min(rb + at, R - 1) * K + ak;
    float acc[LD_TR];
#pragma unroll
    for (int t = 0; t < LD_TR; t++) acc[t] = 0.0f;
    float xt[16], ta[LD_TR];
    fetch_x_tile<XB>(x, ldx, m0, M, 0, xt);
    load_tr<LD_TR>(arow, ta);
    const int srow = threadIdx.x >> 2, skk = (threadIdx.x & 3) * 16;
    for (int k0 = 0, buf = 0; k0 < K; k0 += LD_KC, buf ^= 1) {
        float* st = sx[buf] + srow * LD_XP + skk;
#pragma unroll
        for (int q = 0; q < 4; q++) *(float4*)(st + 4 * q) = make_float4(xt[4 * q], xt[4 * q + 1], xt[4 * q + 2], xt[4 * q + 3]);
        store_tr<LD_TR>(&sa[buf][wave][at * LD_KC + ak], ta);
        __syncthreads();
        if (k0 + LD_KC < K) {
            fetch_x_tile<XB>(x, ldx, m0, M, k0 + LD_KC, xt);
            load_tr<LD_TR>(arow + k0 + LD_KC, ta);
        }
        if (live) {
            const float* xr = sx[buf] + lane * LD_XP;
            const float* as = sa[buf][wave];
#pragma unroll
            for (int kk = 0; kk < LD_KC; kk += 8) {
                const float4 x0 = *(const float4*)(xr + kk), x1 = *(const float4*)(xr + kk + 4);
                const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                float av[LD_TR][8];
#pragma unroll
                for (int t = 0; t < LD_TR; t++) {
                    const float4 a0 = *(const float4*)(as + t * LD_KC + kk), a1 = *(const float4*)(as + t * LD_KC + kk + 4);
                    av[t][0] = a0.x, av[t][1] = a0.y, av[t][2] = a0.z, av[t][3] = a0.w;
                    av[t][4] = a1.x, av[t][5] = a1.y, av[t][6] = a1.z, av[t][7] = a1.w;
                }
#pragma unroll
                for (int i = 0; i < 8; i++)
#pragma unroll
                    for (int t = 0; t < LD_TR; t++) acc[t] = fmaf(xv[i], av[t][i], acc[t]);
            }
        }
        // The buffer written next iteration was last read two iterations ago,
        // before this iteration's barrier: one barrier per chunk suffices.
    }
    const int m = m0 + lane;
    if (!live || m >= M) return;
    const bool pad = (K % 32) != 0;
#pragma unroll
    for (int t = 0; t < LD_TR; t++)
        if (rb + t < R) h[(int64_t)m * R + rb + t] = pad ? fmaf(0.0f, 0.0f, acc[t]) : acc[t];
}

// General form (any alignment and K): block of 32 rows x 32 ranks, 256 lanes
// of 2 x 2 outputs, K staged 64 deep through LDS, the next chunk's global
// loads issued before the current chunk's fmas.
constexpr int LD_BM = 32, LD_BR = 32, LD_BK = 64, LD_P = LD_BM + 4;

template <bool XB>
__device__ __forceinline__ void lora_down_fetch(const void* __restrict__ x, int64_t ldx, const float* __restrict__ A,
                                                int M, int K, int R, int m0, int r0, int k0, int tid, float (&vx)[8],
                                                float (&va)[8]) {
    const int row = tid >> 3, k = k0 + (tid & 7) * 8;
    const int m = m0 + row, r = r0 + row;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const bool in = m < M && k + i < K;
        if (XB) vx[i] = in ? bf16_to_f32(((const uint16_t*)x)[(int64_t)m * ldx + k + i]) : 0.0f;
        else vx[i] = in ? ((const float*)x)[(int64_t)m * ldx + k + i] : 0.0f;
        va[i] = (r < R && k + i < K) ? A[(int64_t)r * K + k + i] : 0.0f;
    }
}

template <bool XB>
__global__ __launch_bounds__(256) void lora_down_kernel(const void* __restrict__ x, int64_t ldx,
                                                        const float* __restrict__ A, float* __restrict__ h,
                                                        int M, int K, int R) {
    __shared__ __align__(16) float sx[LD_BK][LD_P];
    __shared__ __align__(16) float sa[LD_BK][LD_P];
    const int tid = threadIdx.x;
    const int m0 = blockIdx.x * LD_BM, r0 = blockIdx.y * LD_BR;
    const int tm = (tid & 15) * 2, tr = (tid >> 4) * 2;
    const int srow = tid >> 3, skk = (tid & 7) * 8;
    float acc[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};
    float vx[8], va[8];
    lora_down_fetch<XB>(x, ldx, A, M, K, R, m0, r0, 0, tid, vx, va);
    for (int k0 = 0; k0 < K; k0 += LD_BK) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            sx[skk + i][srow] = vx[i];
            sa[skk + i][srow] = va[i];
        }
        __syncthreads();
        if (k0 + LD_BK < K) lora_down_fetch<XB>(x, ldx, A, M, K, R, m0, r0, k0 + LD_BK, tid, vx, va);
        const int kn = min(LD_BK, K - k0);
        if (kn == LD_BK) {
#pragma unroll
            for (int kk = 0; kk < LD_BK; kk++) {
                const float2 xv = *(const float2*)&sx[kk][tm];
                const float2 av = *(const float2*)&sa[kk][tr];
                acc[0][0] = fmaf(xv.x, av.x, acc[0][0]);
                acc[0][1] = fmaf(xv.x, av.y, acc[0][1]);
                acc[1][0] = fmaf(xv.y, av.x, acc[1][0]);
                acc[1][1] = fmaf(xv.y, av.y, acc[1][1]);
            }
        } else {
            for (int kk = 0; kk < kn; kk++) {
                const float2 xv = *(const float2*)&sx[kk][tm];
                const float2 av = *(const float2*)&sa[kk][tr];
                acc[0][0] = fmaf(xv.x, av.x, acc[0][0]);
                acc[0][1] = fmaf(xv.x, av.y, acc[0][1]);
                acc[1][0] = fmaf(xv.y, av.x, acc[1][0]);
                acc[1][1] = fmaf(xv.y, av.y, acc[1][1]);
            }
        }
        __syncthreads();
    }
    const bool pad = (K % 32) != 0;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int m = m0 + tm + i, r = r0 + tr + j;
            if (m < M && r < R) h[(int64_t)m * R + r] = pad ? fmaf(0.0f, 0.0f, acc[i][j]) : acc[i][j];
        }
}

// ---- lora_rank_add: C [M, N] += h [M, R] . B [N, R]^T ---------------------
// Block: 128 x 128 outputs, 256 lanes of 8 x 8 (rows ty*8.., columns
// tx*4.. and 64 + tx*4..), R staged 32 deep, r-major with a 132-float pitch.
constexpr int RA_BM = 128, RA_BN = 128, RA_BR = 32, RA_P = 132;

// One rank of the update: acc[i][j] = fma(h[row i], b[col j], acc[i][j]).
__device__ __forceinline__ void rank_step(const float* __restrict__ hr, const float* __restrict__ br, int ty, int tx,
                                          float (&acc)[8][8]) {
    const float4 h0 = *(const float4*)&hr[ty * 8], h1 = *(const float4*)&hr[ty * 8 + 4];
    const float4 b0 = *(const float4*)&br[tx * 4], b1 = *(const float4*)&br[64 + tx * 4];
    const float hv[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
    const float bv[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) acc[i][j] = fmaf(hv[i], bv[j], acc[i][j]);
}

// VEC: C's rows are 16-byte (fp32) or 8-byte (bf16) aligned and N % 4 == 0,
// so each lane moves its four adjacent columns as one access.  Four waves a
// SIMD (at most 128 VGPRs; the LDS holds four blocks a CU): against three at
// the 134 the compiler picks unasked, 123.1 -> 110.9 us at 4352 x 12288 x 64,
// with 32 bytes of spill a lane outside the rank loop.
template <bool CB, bool VEC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4))) void lora_rank_add_kernel(const float* __restrict__ h, const float* __restrict__ B,
                                                            void* __restrict__ C, int64_t ldc, int M, int N, int R) {
    __shared__ __align__(16) float sh[RA_BR][RA_P];
    __shared__ __align__(16) float sb[RA_BR][RA_P];
    const int tid = threadIdx.x;
    const int m0 = blockIdx.y * RA_BM, n0 = blockIdx.x * RA_BN;
    const int ty = tid >> 4, tx = tid & 15;
    float acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int m = m0 + ty * 8 + i;
        if constexpr (VEC) {
#pragma unroll
            for (int g = 0; g < 2; g++) {
                const int n = n0 + g * 64 + tx * 4;
                float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                if (m < M && n < N) {
                    if (CB) {
                        const uint2 u = *(const uint2*)((const uint16_t*)C + (int64_t)m * ldc + n);
                        v[0] = bf16_to_f32(u.x & 0xffffu);
                        v[1] = bf16_to_f32(u.x >> 16);
                        v[2] = bf16_to_f32(u.y & 0xffffu);
                        v[3] = bf16_to_f32(u.y >> 16);
                    } else {
                        const float4 f = *(const float4*)((const float*)C + (int64_t)m * ldc + n);
                        v[0] = f.x;
                        v[1] = f.y;
                        v[2] = f.z;
                        v[3] = f.w;
                    }
                }
#pragma unroll
                for (int e = 0; e < 4; e++) acc[i][g * 4 + e] = v[e];
            }
            continue;
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int n = n0 + (j >> 2) * 64 + tx * 4 + (j & 3);
            float v = 0.0f;
            if (m < M && n < N) {
                if (CB) v = bf16_to_f32(((const uint16_t*)C)[(int64_t)m * ldc + n]);
                else v = ((const float*)C)[(int64_t)m * ldc + n];
            }
            acc[i][j] = v;
        }
    }
    // R % 4 == 0 with 16-byte aligned h and B: a lane's four ranks of a row
    // are one 16-byte load (r < R then covers r + 3).
    const bool r4 = (R & 3) == 0 && ((uintptr_t)h & 15) == 0 && ((uintptr_t)B & 15) == 0;
    for (int r0 = 0; r0 < R; r0 += RA_BR) {
        // 128 rows x 32 ranks of h and of B: lane t loads 4 consecutive ranks of
        // rows t/8 + 32 s and stores them rank-major.
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int row = (tid >> 3) + 32 * s, rr = (tid & 7) * 4, r = r0 + rr;
            const int m = m0 + row, n = n0 + row;
            if (r4) {
                const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                const float4 hv = (m < M && r < R) ? *(const float4*)&h[(int64_t)m * R + r] : z;
                const float4 bv = (n < N && r < R) ? *(const float4*)&B[(int64_t)n * R + r] : z;
                sh[rr][row] = hv.x, sh[rr + 1][row] = hv.y, sh[rr + 2][row] = hv.z, sh[rr + 3][row] = hv.w;
                sb[rr][row] = bv.x, sb[rr + 1][row] = bv.y, sb[rr + 2][row] = bv.z, sb[rr + 3][row] = bv.w;
                continue;
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sh[rr + i][row] = (m < M && r + i < R) ? h[(int64_t)m * R + r + i] : 0.0f;
                sb[rr + i][row] = (n < N && r + i < R) ? B[(int64_t)n * R + r + i] : 0.0f;
            }
        }
        __syncthreads();
        const int rn = min(RA_BR, R - r0);
        for (int r = 0; r < rn; r++) rank_step(sh[r], sb[r], ty, tx, acc);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int m = m0 + ty * 8 + i;
        if (m >= M) continue;
        if constexpr (VEC) {
#pragma unroll
            for (int g = 0; g < 2; g++) {
                const int n = n0 + g * 64 + tx * 4;
                if (n >= N) continue;
                const float* a = &acc[i][g * 4];
                if (CB)
                    *(uint2*)((uint16_t*)C + (int64_t)m * ldc + n) = make_uint2(f32x2_to_bf16x2(a[0], a[1]),
                                                                                f32x2_to_bf16x2(a[2], a[3]));
                else
                    *(float4*)((float*)C + (int64_t)m * ldc + n) = make_float4(a[0], a[1], a[2], a[3]);
            }
            continue;
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int n = n0 + (j >> 2) * 64 + tx * 4 + (j & 3);
            if (n >= N) continue;
            if (CB) ((uint16_t*)C)[(int64_t)m * ldc + n] = (uint16_t)f32_to_bf16(acc[i][j]);
            else ((float*)C)[(int64_t)m * ldc + n] = acc[i][j];
        }
    }
}

template <int TR>
static hipError_t launch_down_rows(hipStream_t stream, const void* x, bool x_bf16, int64_t ldx, const float* A,
                                   float* h, int M, int K, int R) {
    const dim3 grid((unsigned)((M + 63) / 64), (unsigned)((R + 4 * TR - 1) / (4 * TR)));
    if (x_bf16) hipLaunchKernelGGL((lora_down_rows_kernel<true, TR>), grid, dim3(256), 0, stream, x, ldx, A, h, M, K, R);
    else hipLaunchKernelGGL((lora_down_rows_kernel<false, TR>), grid, dim3(256), 0, stream, x, ldx, A, h, M, K, R);
    return hipGetLastError();
}

hipError_t launch_lora_down(hipStream_t stream, const void* x, bool x_bf16, int64_t ldx, const float* A, float* h,
                            int M, int K, int R) {
    const int esz = x_bf16 ? 2 : 4;
    if (K % LD_KC == 0 && (uintptr_t)x % 16 == 0 && (ldx * esz) % 16 == 0 && (uintptr_t)A % 16 == 0) {
        const int tr = env_switch("PHI_LORA_TR", 2, 1, 4);  // A/B switch: ranks per wave (1, 2 or 4)
        if (tr == 1) return launch_down_rows<1>(stream, x, x_bf16, ldx, A, h, M, K, R);
        if (tr == 2) return launch_down_rows<2>(stream, x, x_bf16, ldx, A, h, M, K, R);
        return launch_down_rows<4>(stream, x, x_bf16, ldx, A, h, M, K, R);
    }
    const dim3 grid((unsigned)((M + LD_BM - 1) / LD_BM), (unsigned)((R + LD_BR - 1) / LD_BR));
    if (x_bf16) hipLaunchKernelGGL(lora_down_kernel<true>, grid, dim3(256), 0, stream, x, ldx, A, h, M, K, R);
    else hipLaunchKernelGGL(lora_down_kernel<false>, grid, dim3(256), 0, stream, x, ldx, A, h, M, K, R);
    return hipGetLastError();
}

hipError_t launch_lora_rank_add(hipStream_t stream, const float* h, const float* B, void* C, bool c_bf16, int64_t ldc,
                                int M, int N, int R) {
    const dim3 grid((unsigned)((N + RA_BN - 1) / RA_BN), (unsigned)((M + RA_BM - 1) / RA_BM));
    const bool vec = N % 4 == 0 && ldc % 4 == 0 && (uintptr_t)C % (c_bf16 ? 8 : 16) == 0;
    if (c_bf16) {
        if (vec) hipLaunchKernelGGL((lora_rank_add_kernel<true, true>), grid, dim3(256), 0, stream, h, B, C, ldc, M, N, R);
        else hipLaunchKernelGGL((lora_rank_add_kernel<true, false>), grid, dim3(256), 0, stream, h, B, C, ldc, M, N, R);
    } else {
        if (vec) hipLaunchKernelGGL((lora_rank_add_kernel<false, true>), grid, dim3(256), 0, stream, h, B, C, ldc, M, N, R);
        else hipLaunchKernelGGL((lora_rank_add_kernel<false, false>), grid, dim3(256), 0, stream, h, B, C, ldc, M, N, R);
    }
    return hipGetLastError();
}

}  // namespace phi_dev
