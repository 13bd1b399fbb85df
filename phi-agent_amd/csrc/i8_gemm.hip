// int8 x int8 -> int32 GEMM on gfx950 MFMA, with the dequant epilogue fused
// into the store.
//
//   acc[m,n] = sum_k A[m,k] * B[n,k]                  (exact int32)
//   C[m,n]   = fma((float)acc * sA[m], sB[n], bias[n])  -> fp32 or bf16 (RNE)
//
// This is the product of the reference's int8_gemm_tc / int8_gemm_dp4a
// (core/kernels/int8_gemm.cpp:152-290, :466-621) and host gemm_int8
// (core/host/quant.cpp:223-236).  The epilogue is the reference kernel's
// `(float)acc * sa * sb + b` with the product-add fused the way NVRTC's
// default --fmad=true contracts it (:611-617); with no bias it equals the
// host's separately rounded (float)acc * sa * sb.
//
// Design (gfx950, wave64):
//   * v_mfma_i32_32x32x32_i8: a 32x32 int32 block per wave instruction, fed by
//     16 contiguous K-bytes per lane from each operand.  A and B both come in
//     K-contiguous ([M,K] and [N,K]), so both are read with the same per-lane
//     K-run and no repacking: the dot product is order-free in exact integers.
//   * Workgroup tile BM x BN x 64, waves arranged WM x WN, each wave a
//     (BM/WM) x (BN/WN) block of 32x32 MFMA tiles.
//   * Two LDS stages; the next K-tile is fetched into registers while the
//     current one is multiplied, then written to the idle stage: one barrier
//     per K-tile.
//   * LDS rows are 64 B (four 16-B chunks); chunk c of row r is stored at
//     chunk c ^ (((r >> 1) ^ (r >> 2)) & 3), so the 16-B operand reads of 16
//     consecutive rows (one LDS clock: 16 lanes x 16 B) hit 16 distinct bank
//     windows.
//   * Tile order: workgroup ids are dealt round-robin to the 8 XCDs; the id is
//     first remapped so each XCD owns a contiguous run of tiles, then the run
//     is walked GROUP_M tile-rows at a time so concurrently running tiles share
//     A rows and B columns in that XCD's L2.
#include "device_common.hpp"
#include "i8_gemm.hpp"

namespace phi_dev {

constexpr int GEMM_BK = 64;

__device__ __forceinline__ int swz(int row, int c) { return c ^ (((row >> 1) ^ (row >> 2)) & 3); }

// Four nibbles (bits 0..15 of `nib`, column i in bits 4i..4i+3) -> four int8
// through a 16-entry byte table held in `t` (entry c is byte c): v_perm_b32
// picks from entries 0..7 and 8..15 by the low three bits, bit 3 chooses.
__device__ __forceinline__ uint32_t lut4(uint32_t nib, const uint4& t) {
    uint32_t x = nib & 0xffffu;
    x = (x | (x << 8)) & 0x00ff00ffu;
    x = (x | (x << 4)) & 0x0f0f0f0fu;  // byte i = nibble i
    const uint32_t sel = x & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(t.y, t.x, sel);
    const uint32_t hi = __builtin_amdgcn_perm(t.w, t.z, sel);
    const uint32_t m = ((x >> 3) & 0x01010101u) * 0xffu;
    return (hi & m) | (lo & ~m);
}

// 16 columns of a packed nibble row (8 code bytes) -> 16 int8 operand bytes.
__device__ __forceinline__ v4i expand16(const uint2& c, const uint4& t) {
    v4i r;
    r.x = (int)lut4(c.x, t);
    r.y = (int)lut4(c.x >> 16, t);
    r.z = (int)lut4(c.y, t);
    r.w = (int)lut4(c.y >> 16, t);
    return r;
}

// 16 bytes of a row from byte k0 on, zero past K, from any address: one
// 16-byte load when the address is aligned and the chunk lies inside the row,
// byte loads otherwise (the ragged K tail, a row at an odd offset).
__device__ __forceinline__ v4i load16_any(const int8_t* row, int64_t k0, int K) {
    const int8_t* p = row + k0;
    if (k0 + 16 <= K && ((uintptr_t)p & 15) == 0) return *(const v4i*)p;
    uint32_t w[4];
#pragma unroll
    for (int d = 0; d < 4; d++) {
        uint32_t v = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int64_t k = k0 + 4 * d + b;
            v |= (k < K ? (uint32_t)(uint8_t)p[4 * d + b] : 0u) << (8 * b);
        }
        w[d] = v;
    }
    return v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
}

// Workgroup id -> (tile_m, tile_n).  XCD remap then grouped walk.
__device__ __forceinline__ void tile_coords(int pid, int nblocks, int tiles_m, int tiles_n,
                                            int group_m, int& tm, int& tn) {
    // Hardware deals ids round-robin over 8 XCDs: id -> xcd = id % 8.  Give xcd x
    // the contiguous range of logical ids [start_x, start_x + count_x).
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

// W4 = true: B is packed nibbles (row stride ldb bytes, K/2 used) plus the
// per-(row, group) table `lut` (with p.w4_signed, the constant table of signed
// nibbles instead); each staged 16-byte B chunk is expanded in
// registers before it is written to LDS, so the MFMA core is unchanged.
// ANY = true: any K > 0 and operands at any byte offset with any pitch (the
// service the reference's dp4a kernel gives, core/kernels/int8_gemm.cpp:
// 136-150): the last K-tile is zero-filled past K, which adds nothing to the
// exact integer sums.
template <int BM, int BN, int WM, int WN, bool W4, bool ANY = false>
__global__ __launch_bounds__(WM* WN * 64) void i8_gemm_kernel(GemmParams p) {
    constexpr int NT = WM * WN * 64;
    constexpr int WTM = BM / WM, WTN = BN / WN;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    constexpr int A_BYTES = BM * GEMM_BK, B_BYTES = BN * GEMM_BK;
    constexpr int CA = A_BYTES / 16 / NT, CB = B_BYTES / 16 / NT;
    static_assert(CA * NT * 16 == A_BYTES && CB * NT * 16 == B_BYTES, "tile/thread mismatch");

    __shared__ __align__(16) int8_t smem[2 * (A_BYTES + B_BYTES)];
    int8_t* sA = smem;
    int8_t* sB = smem + 2 * A_BYTES;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + BN - 1) / BN;
    int tm, tn;
    tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, p.group_m, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;

    // Global source rows for this thread's staging chunks (clamped into range:
    // a tail tile reads valid rows whose products are never stored).
    const int8_t* gA[CA];
    const int8_t* gB[CB];
    int lA[CA], lB[CB];
#pragma unroll
    for (int i = 0; i < CA; i++) {
        const int idx = tid + NT * i, row = idx >> 2, c = idx & 3;
        const int gm = min(m0 + row, p.M - 1);
        gA[i] = p.A + (int64_t)gm * p.lda + c * 16;
        lA[i] = row * GEMM_BK + swz(row, c) * 16;
    }
    const int8_t* gL[W4 ? CB : 1];
#pragma unroll
    for (int i = 0; i < CB; i++) {
        const int idx = tid + NT * i, row = idx >> 2, c = idx & 3;
        const int gn = min(n0 + row, p.N - 1);
        if (W4) {
            gB[i] = p.B + (int64_t)gn * p.ldb + c * 8;
            gL[i] = p.lut + (int64_t)gn * p.lut_groups * 16;
        } else {
            gB[i] = p.B + (int64_t)gn * p.ldb + c * 16;
        }
        lB[i] = row * GEMM_BK + swz(row, c) * 16;
    }

    v16i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;

    // Operand read offsets (per lane, per block), k-substep s adds chunk 2s.
    const int lrow = lane & 31, lhalf = lane >> 5;
    int oA[TM][2], oB[TN][2];
#pragma unroll
    for (int i = 0; i < TM; i++) {
        const int row = wm * WTM + i * 32 + lrow;
#pragma unroll
        for (int s = 0; s < 2; s++) oA[i][s] = row * GEMM_BK + swz(row, 2 * s + lhalf) * 16;
    }
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int row = wn * WTN + j * 32 + lrow;
#pragma unroll
        for (int s = 0; s < 2; s++) oB[j][s] = row * GEMM_BK + swz(row, 2 * s + lhalf) * 16;
    }

    v4i ra[CA], rb[CB];
    uint2 rc[W4 ? CB : 1];
    uint4 rl[W4 ? CB : 1];
    const int KT = ANY ? (p.K + GEMM_BK - 1) / GEMM_BK : p.K / GEMM_BK;

    // Fetch the K-tile at byte offset k into registers.
    auto fetch = [&](int64_t k) {
        if (ANY) {
            // gA / gB point at chunk c of their rows: the chunk's own K offset
            // is (tid + NT i) & 3 times 16, the same for every fetch.
#pragma unroll
            for (int i = 0; i < CA; i++) {
                const int c = ((tid + NT * i) & 3) * 16;
                ra[i] = load16_any(gA[i] - c, k + c, p.K);
            }
#pragma unroll
            for (int i = 0; i < CB; i++) {
                const int c = ((tid + NT * i) & 3) * 16;
                rb[i] = load16_any(gB[i] - c, k + c, p.K);
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < CA; i++) ra[i] = *(const v4i*)(gA[i] + k);
#pragma unroll
        for (int i = 0; i < CB; i++) {
            if (W4) {
                rc[i] = *(const uint2*)(gB[i] + (k >> 1));
                rl[i] = p.w4_signed ? make_uint4(0x03020100u, 0x07060504u, 0xfbfaf9f8u, 0xfffefdfcu)
                                    : *(const uint4*)(gL[i] + ((k >> p.group_shift) << 4));
            } else {
                rb[i] = *(const v4i*)(gB[i] + k);
            }
        }
    };
    // Write the fetched tile into LDS stage `st`.
    auto stage = [&](int st) {
        int8_t* dA = sA + st * A_BYTES;
        int8_t* dB = sB + st * B_BYTES;
#pragma unroll
        for (int i = 0; i < CA; i++) *(v4i*)(dA + lA[i]) = ra[i];
#pragma unroll
        for (int i = 0; i < CB; i++) *(v4i*)(dB + lB[i]) = W4 ? expand16(rc[i], rl[i]) : rb[i];
    };

    fetch(0);
    stage(0);
    __syncthreads();

    for (int kt = 0; kt < KT; kt++) {
        const int cur = kt & 1;
        const bool more = kt + 1 < KT;
        if (more) fetch((int64_t)(kt + 1) * GEMM_BK);
        const int8_t* cA = sA + cur * A_BYTES;
        const int8_t* cB = sB + cur * B_BYTES;
#pragma unroll
        for (int s = 0; s < 2; s++) {
            v4i fa[TM], fb[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) fa[i] = *(const v4i*)(cA + oA[i][s]);
#pragma unroll
            for (int j = 0; j < TN; j++) fb[j] = *(const v4i*)(cB + oB[j][s]);
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
        if (more) stage(cur ^ 1);
        __syncthreads();
    }

    // ---- epilogue ----
    // 32x32 block layout: lane l holds column l % 32 and, in register r, row
    // 8*(r/4) + 4*(l/32) + r%4.
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int n = n0 + wn * WTN + j * 32 + lrow;
        if (n >= p.N) continue;
        float sb = 0.0f, bz = 0.0f;
        if (p.c_kind != C_I32) {
            sb = p.sb_scalar ? p.sB[0] : p.sB[n];
            if (p.bias_kind == BIAS_F32) bz = ((const float*)p.bias)[n];
            else if (p.bias_kind == BIAS_BF16) bz = bf16_to_f32(((const uint16_t*)p.bias)[n]);
        }
#pragma unroll
        for (int i = 0; i < TM; i++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm * WTM + i * 32 + 8 * (r >> 2) + 4 * lhalf + (r & 3);
                if (m >= p.M) continue;
                const int a = acc[i][j][r];
                const int64_t off = (int64_t)m * p.ldc + n;
                if (p.c_kind == C_I32) {
                    ((int32_t*)p.C)[off] = a;
                } else {
                    const float t = (float)a * p.sA[m];
                    const float v = fmaf(t, sb, bz);
                    if (p.c_kind == C_BF16) ((uint16_t*)p.C)[off] = (uint16_t)f32_to_bf16(v);
                    else ((float*)p.C)[off] = v;
                }
            }
        }
    }
}

template <int BM, int BN, int WM, int WN, bool W4, bool ANY = false>
static hipError_t launch_cfg(hipStream_t stream, const GemmParams& p) {
    const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
    hipLaunchKernelGGL((i8_gemm_kernel<BM, BN, WM, WN, W4, ANY>), dim3(tiles), dim3(WM * WN * 64), 0, stream, p);
    return hipGetLastError();
}

// Tile configurations: 0 = 256x128 (default), 1 = 128x128.
hipError_t launch_i8_gemm(hipStream_t stream, const GemmParams& p, int cfg) {
    switch (cfg) {
        case 1: return launch_cfg<128, 128, 2, 2, false>(stream, p);
        default: return launch_cfg<256, 128, 2, 2, false>(stream, p);
    }
}

hipError_t launch_i8_gemm_any(hipStream_t stream, const GemmParams& p, int cfg) {
    switch (cfg) {
        case 1: return launch_cfg<128, 128, 2, 2, false, true>(stream, p);
        default: return launch_cfg<256, 128, 2, 2, false, true>(stream, p);
    }
}

hipError_t launch_w4a8_gemm(hipStream_t stream, const GemmParams& p, int cfg) {
    switch (cfg) {
        case 1: return launch_cfg<128, 128, 2, 2, true>(stream, p);
        default: return launch_cfg<256, 128, 2, 2, true>(stream, p);
    }
}

}  // namespace phi_dev
