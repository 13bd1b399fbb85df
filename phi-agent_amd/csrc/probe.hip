// Ceiling probes for the benchmark (bench.py --config mfma_ceiling): what one
// MI355X sustains with no data movement around the MFMAs, and how fast a CU
// streams operands into LDS by buffer_load ... lds.  Measurement code only:
// built into lib/libphi_probe.so, which the product library does not link.
//
//   phi_probe_mfma  every wave issues v_mfma_i32_32x32x32_i8 back to back on
//                   16 independent 32 x 32 accumulators (the headline GEMM's
//                   wave tile), operands held in registers:
//                     mode 0  all-zero operands (no toggling: the clock ceiling)
//                     mode 1  one random A and B fragment per lane (static inputs)
//                     mode 2  8 A and 8 B random fragments used as the GEMM's
//                             wave uses a K-step's fragments (each 4 times),
//                             rotated by a cheap XOR every K-step so the
//                             operands change as they do when read from LDS
//                     mode 3  mode 2 with the A fragments walked in snake
//                             order (one operand changes between MFMAs)
//                     mode 4  mode 2 with the two operands' roles swapped
//                     mode 5  mode 2's operands on v_mfma_i32_16x16x64_i8: the
//                             same 128 x 128 wave tile as 8 x 8 blocks of
//                             16 x 16, one MFMA a block per 64 K (the same
//                             operations per iteration)
//                     mode 6  mode 5 on all-zero operands
//   phi_probe_lds_dma  every wave streams 16 rows x 64 bytes per instruction
//                   from a window of global memory into LDS, 4 K-steps of the
//                   headline tile's A and B in flight, with no MFMAs.
//   phi_probe_mfma_valu  the mode-2 MFMA loop with V v_perm_b32 operations
//                   after every MFMA: the VALU work a wave can issue beside
//                   its MFMAs before they slow down.
//   phi_probe_prologue_stream  the rotate+quantise prologue's loads, stores
//                   and launch shape without its arithmetic (and, in mode 1,
//                   with its LDS round trips and barrier): the floor the
//                   prologue is measured against.
//   phi_probe_qt_scale  the prologue's exact scale divisions (qt_scale.hpp:
//                   rmax / qmax, and 1 / scale from v_rcp_f32) on each lane's
//                   own value, for the tests that hold them to IEEE division.
//   phi_probe_tile_trace  the persistent pipeline (i8_gemm_pipe.hip, compiled
//                   here a second time into namespace phi_dev_trace with its
//                   timeline hooks defined) with one record of stamps per
//                   workgroup, each point in both the real-time clock and
//                   the shader clock: kernel start, each tile's start, K-loop
//                   end and epilogue end, the switch between tile sizes, and
//                   the end.  The stamps go to LDS during the run and out to
//                   memory once, at the end.
#include <hip/hip_runtime.h>
#include <stdint.h>

// The per-workgroup record: words 0-63 hold the 100 MHz real-time clock,
// words 64-127 the shader clock (s_memtime, cycles) at the same points:
//   [3 i + p]       256 x 256 tile i < 8, point p (0 start, 1 K-loop end, 2 epilogue end)
//   [24] kernel start, [25] switch to 128 x 128 tiles, [50] kernel end
//   [26 + 3 i + p]  128 x 128 tile i < 8, point p
//   [60] the XCD the workgroup ran on
__shared__ unsigned long long phi_trace_lds[128];
__device__ unsigned long long* phi_trace_out;

#define PHI_TRACE_SLOT(k)                                               \
    do {                                                                \
        phi_trace_lds[k] = __builtin_amdgcn_s_memrealtime();             \
        phi_trace_lds[64 + (k)] = __builtin_amdgcn_s_memtime();          \
    } while (0)
#define PHI_PIPE_STAMP(phase, tile, point)                                                                  \
    if (threadIdx.x == 0 && (tile) < 8)                                                                     \
        PHI_TRACE_SLOT((phase) == 0 ? (tile) * 3 + (point) : (phase) == 1 ? 26 + (tile) * 3 + (point) : 25);
#define PHI_PIPE_TRACE_BEGIN                                                   \
    if (threadIdx.x < 128) phi_trace_lds[threadIdx.x] = 0;                    \
    __syncthreads();                                                           \
    if (threadIdx.x == 0) PHI_TRACE_SLOT(24);
#define PHI_PIPE_TRACE_END                                                            \
    __syncthreads();                                                                  \
    if (threadIdx.x == 0) {                                                           \
        PHI_TRACE_SLOT(50);                                                           \
        unsigned int xcc_;                                                            \
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc_));           \
        phi_trace_lds[60] = xcc_ & 15;                                                \
    }                                                                                 \
    __syncthreads();                                                                  \
    if (threadIdx.x < 128) phi_trace_out[blockIdx.x * 128 + threadIdx.x] = phi_trace_lds[threadIdx.x];

#define phi_dev phi_dev_trace
#include "i8_gemm_pipe.hip"
#undef phi_dev
#include "qt_scale.hpp"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void* lptr_t;
constexpr int kRsrcWord3 = 0x00020000;

// The 16 x 16 x 64 MFMA with its accumulator tied to one AGPR quad.  With
// the builtin, the register allocator moved the rotating-operand loop's
// accumulators between AGPRs (about 108 v_accvgpr moves an iteration): 2873
// TOPS on rotating operands, against 3544 with every accumulator in place.
__device__ __forceinline__ void mfma16_tied(v4i& c, const v4i& b, const v4i& a) {
    asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(c) : "v"(b), "v"(a));
}

// Modes 5 and 6: the 16 x 16 x 64 form, 64 accumulators of 4 registers.
template <int MODE>
__global__ __launch_bounds__(256) void mfma16_probe(const int8_t* ops, int iters, int* sink) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v4i a[8], b[8];
#pragma unroll
    for (int f = 0; f < 8; f++) {
        if (MODE == 6) {
            a[f] = v4i{0, 0, 0, 0};
            b[f] = v4i{0, 0, 0, 0};
        } else {
            a[f] = *(const v4i*)(ops + ((wave * 16 + f) * 64 + lane) * 16);
            b[f] = *(const v4i*)(ops + ((wave * 16 + 8 + f) * 64 + lane) * 16);
        }
    }
    v4i acc[64];
#pragma unroll
    for (int q = 0; q < 64; q++) acc[q] = v4i{};
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int q = 0; q < 64; q++)
            mfma16_tied(acc[q], b[q >> 3], a[q & 7]);
        if (MODE == 5) {
            const int x = 0x5a3c96e1 * (it + 1) + lane;
#pragma unroll
            for (int f = 0; f < 8; f++) {
                a[f] ^= v4i{x, x >> 3, x >> 5, x >> 7};
                b[f] ^= v4i{x >> 1, x >> 2, x >> 4, x >> 6};
            }
        }
    }
    int t = 0;
#pragma unroll
    for (int q = 0; q < 64; q++)
#pragma unroll
        for (int r = 0; r < 4; r++) t += acc[q][r];
    if (t == 0x7fffffff) sink[blockIdx.x * 4 + wave] = t;  // keeps the MFMAs live
}

template <int MODE>
__global__ __launch_bounds__(256) void mfma_probe(const int8_t* ops, int iters, int* sink) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v4i a[8], b[8];
#pragma unroll
    for (int f = 0; f < 8; f++) {
        if (MODE == 0) {
            a[f] = v4i{0, 0, 0, 0};
            b[f] = v4i{0, 0, 0, 0};
        } else {
            const int fa = MODE == 1 ? 0 : f;
            a[f] = *(const v4i*)(ops + ((wave * 16 + fa) * 64 + lane) * 16);
            b[f] = *(const v4i*)(ops + ((wave * 16 + 8 + fa) * 64 + lane) * 16);
        }
    }
    v16i acc[16];
#pragma unroll
    for (int q = 0; q < 16; q++) acc[q] = v16i{};
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const int jb = q >> 2, ia = MODE == 3 && (jb & 1) ? 3 - (q & 3) : q & 3;
                if (MODE == 4)
                    acc[q] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[ia + 4 * s], b[jb + 4 * s], acc[q], 0, 0, 0);
                else
                    acc[q] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b[jb + 4 * s], a[ia + 4 * s], acc[q], 0, 0, 0);
            }
        if (MODE >= 2) {
            const int x = 0x5a3c96e1 * (it + 1) + lane;
#pragma unroll
            for (int f = 0; f < 8; f++) {
                a[f] ^= v4i{x, x >> 3, x >> 5, x >> 7};
                b[f] ^= v4i{x >> 1, x >> 2, x >> 4, x >> 6};
            }
        }
    }
    int t = 0;
#pragma unroll
    for (int q = 0; q < 16; q++)
#pragma unroll
        for (int r = 0; r < 16; r++) t += acc[q][r];
    if (t == 0x7fffffff) sink[blockIdx.x * 4 + wave] = t;  // keeps the MFMAs live
}

// The GEMM's MFMA loop (mode 2 operands) with V independent VALU operations
// (v_perm_b32, the W4 table lookup's instruction) placed after every MFMA, in
// four chains: how much VALU work a wave can issue beside its MFMAs before
// they slow down.
template <int V>
__global__ __launch_bounds__(256) void mfma_valu_probe(const int8_t* ops, int iters, int* sink) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v4i a[8], b[8];
#pragma unroll
    for (int f = 0; f < 8; f++) {
        a[f] = *(const v4i*)(ops + ((wave * 16 + f) * 64 + lane) * 16);
        b[f] = *(const v4i*)(ops + ((wave * 16 + 8 + f) * 64 + lane) * 16);
    }
    v16i acc[16];
#pragma unroll
    for (int q = 0; q < 16; q++) acc[q] = v16i{};
    uint32_t c[4] = {(uint32_t)lane, (uint32_t)lane * 3u, (uint32_t)lane * 5u, (uint32_t)lane * 7u};
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
            for (int q = 0; q < 16; q++) {
                acc[q] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b[(q >> 2) + 4 * s], a[(q & 3) + 4 * s], acc[q], 0, 0, 0);
#pragma unroll
                for (int v = 0; v < V; v++)
                    c[v & 3] = __builtin_amdgcn_perm(c[v & 3], (uint32_t)b[(q + v) & 7][v & 3], 0x05010400u + v);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                if constexpr (V > 0) __builtin_amdgcn_sched_group_barrier(0x002, V, 0);
            }
        const int x = 0x5a3c96e1 * (it + 1) + lane;
#pragma unroll
        for (int f = 0; f < 8; f++) {
            a[f] ^= v4i{x, x >> 3, x >> 5, x >> 7};
            b[f] ^= v4i{x >> 1, x >> 2, x >> 4, x >> 6};
        }
    }
    int t = (int)(c[0] ^ c[1] ^ c[2] ^ c[3]);
#pragma unroll
    for (int q = 0; q < 16; q++)
#pragma unroll
        for (int r = 0; r < 16; r++) t += acc[q][r];
    if (t == 0x7fffffff) sink[blockIdx.x * 4 + wave] = t;
}

__global__ __launch_bounds__(256) void lds_dma_probe(const int8_t* src, int window, int iters, int* sink) {
    __shared__ __align__(16) int8_t st[4][4][8192];  // wave, stage, 8 loads of 1 KB
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & 3;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, window, kRsrcWord3);
    // lane l fetches row l / 4, chunk l % 4 of a 16-row x 64-byte piece at a
    // 3072-byte row pitch (the headline A and B rows).
    const int vo = (lane >> 2) * 3072 + (lane & 3) * 16;
    // Every load stays below window: a piece spans 16 rows at the pitch.
    // Each wave starts at its own share of the window, so a window much
    // larger than the MALL is read once, from HBM.
    const int span = window - (1 << 19);
    const int share = (int)(((long long)span / ((long long)gridDim.x * 4)) & ~63ll);
    const int base = (int)(((long long)blockIdx.x * 4 + wave) * share % span);
    for (int it = 0; it < iters; it++) {
        const int s = it & 3;
        const int off = (int)(((long long)base + (long long)it * 64) % span);
#pragma unroll
        for (int j = 0; j < 8; j++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lptr_t)(&st[wave][s][j * 1024]), 16, vo,
                                                     off + j * 16 * 3072, 0, 0);
        // Keep three later K-steps in flight, as the GEMM's pipeline does.
        __builtin_amdgcn_s_waitcnt((8 * 3 & 15) | (7 << 4) | (((8 * 3) >> 4) & 3) << 14);
    }
    __builtin_amdgcn_s_waitcnt(0 | (7 << 4));
    __syncthreads();
    if (st[wave][0][lane] == 127 && st[wave][1][lane] == -128 && lane == 0) sink[blockIdx.x] = 1;
}

// The rotate+quantise prologue's memory pattern without its arithmetic, on
// quant_rotate_tiles' launch shape at one round a wave: one row a block of
// ceil(G / 4) waves, a 16-lane team a 256-group.  Each lane loads its 16
// bf16 inputs (32 bytes), keeps their high bytes, and stores those 16 bytes
// where the codes go (K-tiled when kt, else row-major); lane 0 of the row's
// first wave stores one float.  MODE 1 adds the kernel's LDS traffic: the
// values as fp32 through the team's 16 x 16 tile and back (row write, column
// read, column write, row read) and the cross-wave exchange of one word a
// wave with its barrier.
// run > 0 remaps blocks so each XCD (blocks are dealt to the 8 XCDs in
// turn) takes runs of that many consecutive rows.
template <int MODE>
__global__ __launch_bounds__(1024) void prologue_stream_probe(const uint16_t* x, int rows, int G, int8_t* q,
                                                              float* s, int kt, int run) {
    extern __shared__ __align__(16) float plds[];
    const int lane = threadIdx.x & 63, wr = threadIdx.x >> 6, wpr = blockDim.x >> 6;
    int row = blockIdx.x;
    if (run > 0 && (int)blockIdx.x < (int)gridDim.x / (8 * run) * (8 * run)) {
        const int b = blockIdx.x, c = b % (8 * run);
        row = b - c + (c % 8) * run + c / 8;
    }
    const int team = lane >> 4, tl = lane & 15, sw = tl >> 2;
    const int g = wr * 4 + team;
    const uint4* src = (const uint4*)(x + (int64_t)row * G * 256 + (int64_t)min(g, G - 1) * 256 + tl * 16);
    const uint4 a = src[0], b = src[1];
    uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t packed[4];
    uint32_t word = w[0];
    if (MODE == 0) {
#pragma unroll
        for (int i = 0; i < 4; i++) packed[i] = __builtin_amdgcn_perm(w[2 * i + 1], w[2 * i], 0x07050301u);
    } else {
        float* T = plds + wr * 1088 + team * 272;
        float* trow = T + tl * 16;
        uint32_t* red = (uint32_t*)(plds + wpr * 1088);
        float v[16], c[16];
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = __uint_as_float(i & 1 ? w[i >> 1] & 0xffff0000u : w[i >> 1] << 16);
#pragma unroll
        for (int k = 0; k < 4; k++) *(float4*)(trow + 4 * (k ^ sw)) = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
        for (int k = 0; k < 4; k++)
#pragma unroll
            for (int i = 0; i < 4; i++) c[4 * k + i] = T[64 * k + 4 * (sw ^ k) + (tl & 3) + 16 * i];
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        if (lane == 0) red[wr] = __float_as_uint(c[0]);
        __syncthreads();
        for (int i = 0; i < wpr; i++) word ^= red[i];
#pragma unroll
        for (int k = 0; k < 4; k++)
#pragma unroll
            for (int i = 0; i < 4; i++) T[64 * k + 4 * (sw ^ k) + (tl & 3) + 16 * i] = c[4 * k + i];
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float4 u = *(const float4*)(trow + 4 * (k ^ sw));
            packed[k] = __builtin_amdgcn_perm(__float_as_uint(u.y), __float_as_uint(u.x), 0x07030703u) ^
                        __builtin_amdgcn_perm(__float_as_uint(u.w), __float_as_uint(u.z), 0x03070307u);
        }
    }
    int8_t* dst;
    if (kt) {
        const int64_t st = row >> 8, rr = row & 255, h = min(256, rows - (int)(st << 8));
        dst = q + st * 256 * (int64_t)G * 256 + (int64_t)g * 4 * h * 64 + (tl >> 2) * h * 64 + rr * 64 +
              (((tl & 3) ^ ((rr >> 2) & 3)) * 16);
    } else {
        dst = q + (int64_t)row * G * 256 + (int64_t)g * 256 + tl * 16;
    }
    if (g < G) *(uint4*)dst = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    if (wr == 0 && lane == 0) s[row] = __uint_as_float(word);
}

}  // namespace

// Mode 0: out = rmax / qmax by qt_div_qmax; mode 1: out = 1 / b by
// qt_rcp_bits, each lane on its own value.
__global__ __launch_bounds__(256) void qt_scale_probe(const float* in, int n, int mode, float qmax, float qrcp,
                                                      float* out) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float v = in[i];
    out[i] = mode == 0 ? phi_dev::qt_div_qmax(v, qmax, qrcp) : phi_dev::qt_rcp_bits(v, __float_as_uint(v));
}

extern "C" {

// The prologue's scale divisions over in[0, n) into out (see qt_scale_probe);
// qmax an integer in [1, 127] for mode 0.
int phi_probe_qt_scale(void* stream, const float* in, int n, int mode, float qmax, float* out) {
    if (n <= 0 || !in || !out || (mode != 0 && mode != 1)) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(qt_scale_probe, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, in, n,
                       mode, qmax, 1.0f / qmax, out);
    return (int)hipGetLastError();
}

// The prologue stream probe over x [rows, 256 G] bf16 into q (rows x 256 G
// bytes) and s [rows]; G <= 64; run as in prologue_stream_probe.
int phi_probe_prologue_stream(void* stream, const uint16_t* x, int rows, int G, int8_t* q, float* s, int mode, int kt,
                              int run) {
    if (rows <= 0 || G <= 0 || G > 64) return (int)hipErrorInvalidValue;
    const int wpr = (G + 3) / 4;
    const size_t lds = ((size_t)wpr * 1088 + 16) * sizeof(float);
    static bool lds_set = false;
    if (!lds_set) {
        const hipError_t e = hipFuncSetAttribute((const void*)prologue_stream_probe<1>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)((16 * 1088 + 16) * sizeof(float)));
        if (e != hipSuccess) return (int)e;
        lds_set = true;
    }
    if (mode == 0)
        hipLaunchKernelGGL(prologue_stream_probe<0>, dim3(rows), dim3(64 * wpr), 0, (hipStream_t)stream, x, rows, G, q,
                           s, kt, run);
    else
        hipLaunchKernelGGL(prologue_stream_probe<1>, dim3(rows), dim3(64 * wpr), lds, (hipStream_t)stream, x, rows, G,
                           q, s, kt, run);
    return (int)hipGetLastError();
}

int phi_probe_mfma(void* stream, const int8_t* ops, int mode, int iters, int* sink, int grid) {
    switch (mode) {
        case 0: hipLaunchKernelGGL(mfma_probe<0>, dim3(grid), dim3(256), 0, (hipStream_t)stream, ops, iters, sink); break;
        case 1: hipLaunchKernelGGL(mfma_probe<1>, dim3(grid), dim3(256), 0, (hipStream_t)stream, ops, iters, sink); break;
        case 3: hipLaunchKernelGGL(mfma_probe<3>, dim3(grid), dim3(256), 0, (hipStream_t)stream, ops, iters, sink); break;
        case 4: hipLaunchKernelGGL(mfma_probe<4>, dim3(grid), dim3(256), 0, (hipStream_t)stream, ops, iters, sink); break;
        case 5: hipLaunchKernelGGL(mfma16_probe<5>, dim3(grid), dim3(256), 0, (hipStream_t)stream, ops, iters, sink); break;
        case 6: hipLaunchKernelGGL(mfma16_probe<6>, dim3(grid), dim3(256), 0, (hipStream_t)stream, ops, iters, sink); break;
        default: hipLaunchKernelGGL(mfma_probe<2>, dim3(grid), dim3(256), 0, (hipStream_t)stream, ops, iters, sink); break;
    }
    return (int)hipGetLastError();
}

// V VALU operations after every MFMA (V in 0, 1, 2, 3, 4, 6, 8).
int phi_probe_mfma_valu(void* stream, const int8_t* ops, int v, int iters, int* sink, int grid) {
    hipStream_t st = (hipStream_t)stream;
    switch (v) {
        case 0: hipLaunchKernelGGL(mfma_valu_probe<0>, dim3(grid), dim3(256), 0, st, ops, iters, sink); break;
        case 1: hipLaunchKernelGGL(mfma_valu_probe<1>, dim3(grid), dim3(256), 0, st, ops, iters, sink); break;
        case 2: hipLaunchKernelGGL(mfma_valu_probe<2>, dim3(grid), dim3(256), 0, st, ops, iters, sink); break;
        case 3: hipLaunchKernelGGL(mfma_valu_probe<3>, dim3(grid), dim3(256), 0, st, ops, iters, sink); break;
        case 4: hipLaunchKernelGGL(mfma_valu_probe<4>, dim3(grid), dim3(256), 0, st, ops, iters, sink); break;
        case 6: hipLaunchKernelGGL(mfma_valu_probe<6>, dim3(grid), dim3(256), 0, st, ops, iters, sink); break;
        case 8: hipLaunchKernelGGL(mfma_valu_probe<8>, dim3(grid), dim3(256), 0, st, ops, iters, sink); break;
        default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

int phi_probe_lds_dma(void* stream, const int8_t* src, long long window, int iters, int* sink, int grid) {
    if (window < (1 << 20) || window > (1ll << 31) - 1) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(lds_dma_probe, dim3(grid), dim3(256), 0, (hipStream_t)stream, src, (int)window, iters, sink);
    return (int)hipGetLastError();
}

// The K-tiled (kt) or row-major pipeline over A [M, K], B [N, K] (bf16 out,
// fp32 row scales sA, one fp32 scale sB, bf16 bias): 256 x 256 tiles for the
// first big_rows rows (a multiple of 256), 128 x 128 tiles for the rest, in
// one launch, as the library's plan runs it.  out holds slots >= grid x 128
// words.
int phi_probe_tile_trace(void* stream, const int8_t* A, const int8_t* B, const float* sA, const float* sB,
                         const void* bias, void* C, int M, int N, int K, int big_rows, int kt,
                         unsigned long long* out, long long slots) {
    if (M <= 0 || N <= 0 || K % 256 != 0 || K <= 0 || big_rows < 0 || big_rows > M ||
        (big_rows % 256 != 0 && big_rows != M) || N % 8 != 0)
        return (int)hipErrorInvalidValue;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return (int)hipErrorInvalidDevice;
    const long long big = (long long)((big_rows + 255) / 256) * ((N + 255) / 256);
    const long long small = (long long)((M - big_rows + 127) / 128) * ((N + 127) / 128);
    const long long most = big > small ? big : small;
    if ((most < cus ? most : cus) * 128 > slots) return (int)hipErrorInvalidValue;
    hipError_t e = hipMemcpyToSymbolAsync(HIP_SYMBOL(phi_trace_out), &out, sizeof(out), 0, hipMemcpyHostToDevice,
                                          (hipStream_t)stream);
    if (e != hipSuccess) return (int)e;
    phi_dev_trace::GemmParams p{};
    p.A = A;
    p.B = B;
    p.sA = sA;
    p.sB = sB;
    p.bias = bias;
    p.C = C;
    p.lda = K;
    p.ldb = K;
    p.ldc = N;
    p.M = M;
    p.N = N;
    p.K = K;
    p.sb_scalar = 1;
    p.bias_kind = bias ? phi_dev_trace::BIAS_BF16 : phi_dev_trace::BIAS_NONE;
    p.c_kind = phi_dev_trace::C_BF16;
    p.group_m = 4;
    p.c_vec = 1;
    p.c_vec16 = 1;
    p.s_vec = 1;
    p.kt = kt ? 1 : 0;
    phi_dev_trace::GemmParams pb = p, ps = p;
    pb.M = big_rows;
    ps.M = M - big_rows;
    ps.A = A + (size_t)big_rows * K;
    ps.sA = sA + big_rows;
    ps.C = (int8_t*)C + (size_t)big_rows * N * 2;
    if (big_rows == M) return (int)phi_dev_trace::launch_i8_gemm_pipe((hipStream_t)stream, pb, cus, 128);
    if (big_rows == 0) return (int)phi_dev_trace::launch_i8_gemm_pipe((hipStream_t)stream, ps, cus, 64);
    return (int)phi_dev_trace::launch_i8_gemm_pipe_mixed((hipStream_t)stream, pb, ps, cus);
}

}  // extern "C"
