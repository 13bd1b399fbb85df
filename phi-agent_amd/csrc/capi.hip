// C ABI of the quantized-linear library: argument validation, dispatch to the
// gfx950 kernels, and the error contract.
//
// The reference's dispatchers throw MediaError on a contract violation
// (core/runtime/compute.cpp:552, :665-668; core/kernels/w4a8_expand.cpp:264-281)
// and mark the device lost on a memory fault (compute.cpp:461-467).  Here every
// entry point returns a phi_status and leaves a message for
// phi_hip_last_error(); a memory fault or illegal-address status from HIP is
// reported as PHI_ERR_DEVICE_LOST and stays sticky for the process.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <tuple>

#include "../../include/phi_qlinear.h"
#include "device_common.hpp"
#include "gemv.hpp"
#include "lora.hpp"
#include "i8_gemm.hpp"
#include "w4a8.hpp"

namespace {

thread_local std::string g_err;
std::atomic<bool> g_lost{false};

phi_status vfail(phi_status st, const char* fmt, va_list ap) {
    char buf[512];
    vsnprintf(buf, sizeof buf, fmt, ap);
    g_err = buf;
    return st;
}

phi_status fail(phi_status st, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vfail(st, fmt, ap);
    va_end(ap);
    return st;
}

phi_status ok() {
    g_err.clear();
    return PHI_OK;
}

bool is_fatal(hipError_t e) {
    return e == hipErrorIllegalAddress || e == hipErrorLaunchFailure || e == hipErrorECCNotCorrectable ||
           e == hipErrorAssert;
}

phi_status check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return ok();
    if (is_fatal(e)) {
        g_lost = true;
        return fail(PHI_ERR_DEVICE_LOST, "%s: device lost (%s)", what, hipGetErrorString(e));
    }
    return fail(PHI_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

int bias_kind_of(const void* bias, int bias_dtype, phi_status* st) {
    *st = PHI_OK;
    if (!bias) return phi_dev::BIAS_NONE;
    if (bias_dtype == PHI_F32) return phi_dev::BIAS_F32;
    if (bias_dtype == PHI_BF16) return phi_dev::BIAS_BF16;
    *st = PHI_ERR_ARG;
    return -1;
}

int c_kind_of(int c_dtype) {
    if (c_dtype == PHI_F32) return phi_dev::C_F32;
    if (c_dtype == PHI_BF16) return phi_dev::C_BF16;
    if (c_dtype == PHI_I32) return phi_dev::C_I32;
    return -1;
}

size_t c_elem_bytes(int c_dtype) { return c_dtype == PHI_BF16 ? 2 : 4; }

constexpr int64_t kMaxRotK = 24576;
// Rows from which phi_hip_w4a8_linear expands the codes into the workspace
// (when given one) rather than in registers per tile.
constexpr int64_t kW4ExpandMinRows = 512;  // rotated row held in LDS: 96 groups = 129 KB

// Shared validation of the GEMM operands (A [M,lda], B [N,ldb]).
phi_status check_gemm(const char* who, const int8_t* A, int64_t lda, const void* B, int64_t ldb,
                      int64_t M, int64_t N, int64_t K, const float* sA, const float* sB,
                      void* C, int c_dtype, int64_t ldc, bool w4, bool any_k = false) {
    if (M <= 0 || N <= 0 || K <= 0) return fail(PHI_ERR_SHAPE, "%s: empty problem (M=%lld N=%lld K=%lld)", who, (long long)M, (long long)N, (long long)K);
    if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return fail(PHI_ERR_SHAPE, "%s: dimension exceeds 2^31", who);
    if (!A || !B || !C) return fail(PHI_ERR_ARG, "%s: null operand", who);
    if (c_kind_of(c_dtype) < 0) return fail(PHI_ERR_ARG, "%s: bad output dtype %d", who, c_dtype);
    if (c_dtype != PHI_I32 && (!sA || !sB)) return fail(PHI_ERR_ARG, "%s: scales are required for a scaled output", who);
    if (!any_k && K % 64 != 0) return fail(PHI_ERR_SHAPE, "%s: K=%lld is not a multiple of 64", who, (long long)K);
    if (lda < K || ldc < N) return fail(PHI_ERR_SHAPE, "%s: leading dimension smaller than the row", who);
    if (!any_k && (!aligned(A, 16) || lda % 16 != 0)) return fail(PHI_ERR_ALIGN, "%s: A must be 16-byte aligned with lda %% 16 == 0", who);
    if (w4) {
        if (ldb < K / 2) return fail(PHI_ERR_SHAPE, "%s: a %lld-column nibble row needs %lld bytes, got %lld", who, (long long)K, (long long)(K / 2), (long long)ldb);
        if (!aligned(B, 8) || ldb % 8 != 0) return fail(PHI_ERR_ALIGN, "%s: codes must be 8-byte aligned with row bytes %% 8 == 0", who);
    } else {
        if (ldb < K) return fail(PHI_ERR_SHAPE, "%s: ldb < K", who);
        if (!any_k && (!aligned(B, 16) || ldb % 16 != 0)) return fail(PHI_ERR_ALIGN, "%s: B must be 16-byte aligned with ldb %% 16 == 0", who);
    }
    if (sA && !aligned(sA, 4)) return fail(PHI_ERR_ALIGN, "%s: sA is misaligned", who);
    if (sB && !aligned(sB, 4)) return fail(PHI_ERR_ALIGN, "%s: sB is misaligned", who);
    if (!aligned(C, c_elem_bytes(c_dtype))) return fail(PHI_ERR_ALIGN, "%s: C is misaligned", who);
    return PHI_OK;
}

int gemm_cfg_for(int64_t M, int64_t N) {
    // 256x128 tiles unless that leaves most of the 256 CUs idle.
    const int64_t big = ((M + 255) / 256) * ((N + 127) / 128);
    return big >= 256 ? 0 : 1;
}

// Kernel choice for the W8A8 GEMM.  PHI_GEMM_KERNEL forces one (an A/B
// switch for tests, like the reference's PHI_INT8_DP4A,
// core/runtime/compute.cpp:566-571):
//   tile128   the 256x128 / 128x128 register-staged kernel (small problems)
//   tile256   256x256, eight 128x64 waves, 64-deep K-steps
//   tile256w4 256x256, four 128x128 waves, 128-deep K-steps (needs K % 128 == 0)
//   persist   persistent kernel: 256x256 tiles for whole rounds, 128x128 for
//             the remaining rows (persist_ok)
//   persist256 / persist128  the persistent kernel with one tile size only
// Unset, every problem the persistent kernel accepts takes it; otherwise
// problems with enough 256x256 tiles to occupy the GPU take the four-wave
// kernel when K % 128 == 0 and the eight-wave one otherwise.
enum GemmKernel { GK_TILE128 = 0, GK_TILE256 = 1, GK_TILE256W4 = 2, GK_PERSIST = 3, GK_PERSIST256 = 4, GK_PERSIST128 = 5 };

// The persistent kernel's contract: 128-deep K-steps in pairs, whole 16-byte
// output pieces (8 bf16 or 4 fp32/int32 columns) on 16-byte aligned rows, and
// 32-bit byte offsets within a 256-row tile.
bool persist_ok(const void* C, int c_dtype, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc) {
    const int64_t esz = c_dtype == PHI_BF16 ? 2 : 4;
    if (K % 256 != 0) return false;
    if (N % (16 / esz) != 0) return false;
    if (!aligned(C, 16) || (ldc * esz) % 16 != 0) return false;
    const int64_t lim = (int64_t)1 << 23;  // 256 rows x pitch < 2^31
    return lda < lim && ldb < lim && ldc * esz < lim;
}

GemmKernel gemm_kernel_for(int64_t M, int64_t N, int64_t K, bool pok) {
    const char* e = getenv("PHI_GEMM_KERNEL");
    if (e && strcmp(e, "persist") == 0 && pok) return GK_PERSIST;
    if (e && strcmp(e, "persist256") == 0 && pok) return GK_PERSIST256;
    if (e && strcmp(e, "persist128") == 0 && pok) return GK_PERSIST128;
    if (e && strcmp(e, "tile256w4") == 0 && K % 128 == 0) return GK_TILE256W4;
    if (e && strcmp(e, "tile256") == 0) return GK_TILE256;
    if (e && strcmp(e, "tile128") == 0) return GK_TILE128;
    if (pok) return GK_PERSIST;
    const int64_t t256 = ((M + 255) / 256) * ((N + 255) / 256);
    if (t256 < 128) return GK_TILE128;
    return K % 128 == 0 ? GK_TILE256W4 : GK_TILE256;
}

// Compute units of the current device (one persistent workgroup each).
int num_cus() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// Rows of the problem the persistent kernel covers with 256 x 256 tiles; the
// rest (a multiple of 256 rows, from the bottom) get 128 x 128 tiles in a
// second launch.  A 256-tile round that leaves most CUs idle costs almost a
// full round (at 4352 x 12288 x 3072 the 48 tiles of the 17th tile-row took
// 41 of 183 us on 256 CUs), while 128 x 128 tiles spread the same rows over
// four times as many CUs.  The plan minimises
//   ceil(big tiles / CUs) + kSmallRound * ceil(small tiles / CUs)
// with kSmallRound the measured cost of a round of 128 x 128 tiles relative
// to a round of 256 x 256 ones at the same K.
constexpr double kSmallRound = 0.35;

int64_t big_tile_rows(int64_t M, int64_t N, int G) {
    const int64_t tm = (M + 255) / 256, tn = (N + 255) / 256, tn2 = (N + 127) / 128;
    int64_t best_r = tm;
    double best = (double)((tm * tn + G - 1) / G);
    for (int64_t r = tm - 1; r >= 0; r--) {
        const int64_t small = ((M - 256 * r + 127) / 128) * tn2;
        const double cost = (double)((r * tn + G - 1) / G) + kSmallRound * (double)((small + G - 1) / G);
        if (cost < best - 1e-9) {
            best = cost;
            best_r = r;
        }
    }
    return best_r * 256 < M ? best_r * 256 : M;
}

// The tuning table: a plan per (M, N, K, operand layout) for the int8-B
// persistent GEMM, set by the caller (a sweep's result, persisted by the host
// layer's GemmTuneStore).  Read on every such launch; the count lets the
// common case, an empty table, skip the lock.
struct PlanKey {
    int64_t M, N, K;
    int kt;
    bool operator<(const PlanKey& o) const { return std::tie(M, N, K, kt) < std::tie(o.M, o.N, o.K, o.kt); }
};
std::mutex g_plans_mu;
std::map<PlanKey, phi_gemm_plan> g_plans;
std::atomic<int64_t> g_plan_count{0};

bool tuned_plan(int64_t M, int64_t N, int64_t K, int kt, phi_gemm_plan* out) {
    if (g_plan_count.load(std::memory_order_acquire) == 0) return false;
    std::lock_guard<std::mutex> lk(g_plans_mu);
    const auto it = g_plans.find(PlanKey{M, N, K, kt ? 1 : 0});
    if (it == g_plans.end()) return false;
    *out = it->second;
    return true;
}

// Rounds of 256 x 256 tiles the square plan costs (big_tile_rows' measure).
double square_plan_cost(int64_t M, int64_t N, int G) {
    const int64_t rows = big_tile_rows(M, N, G);
    const int64_t big = (rows / 256 + (rows % 256 ? 1 : 0)) * ((N + 255) / 256);
    const int64_t small = ((M - rows + 127) / 128) * ((N + 127) / 128);
    return (double)((big + G - 1) / G) + kSmallRound * (double)((small + G - 1) / G);
}

// A round of 272 x 192 tiles against a round of 256 x 256 ones at the same K,
// measured.  In cycles it is the outputs' ratio, 52224 / 65536 = 0.80 (the
// traced builds: 905 against 1117 clocks a K-step, similar epilogues), but
// the 272 x 192 kernel's 16x16x64 MFMAs draw less power than the square
// kernel's 32x32x32 ones on random data, and the board runs it at a higher
// clock: config 3 attention took 635.0 us in 13 rounds against 671.9 us in
// 10 square ones (0.73 a round), its MLP 1657.8 us in 35 against 1773.1 us in
// 27 (0.72).  On row-major operands each DMA lane fetches 16 bytes of its own
// row, half a cache line a K-step, and that advantage is gone: 0.81 a round
// at config 1 up, 0.80 at config 3 attention (762.6 us in 13 rounds against
// 734.6 in 10), 0.90 at config 1 down's single round.
constexpr double kT272Round = 0.73, kT272RoundRowMajor = 0.80;
// K-tiled activations against a row-major weight (b_rm): only B's 192 rows a
// K-step are gathered row by row.
constexpr double kT272RoundMixed = 0.76;

// Whether the 272 x 192 kernel serves p: as the tuned plan's tile field says,
// else when its rounds cost less than the square plan's.  PHI_GEMM_T272=0 / 1
// turns it off / forces it where it applies (an A/B switch, above the table).
bool use_t272(const phi_dev::GemmParams& p, int G, int tile) {
    if (!phi_dev::t272_ok(p)) return false;
    const int e = phi_dev::env_switch("PHI_GEMM_T272", -1, 0, 1);
    if (e >= 0) return e == 1;
    if (tile != PHI_PLAN_TILE_AUTO) return tile == PHI_PLAN_TILE_272;
    const double t = (p.kt ? (p.b_rm ? kT272RoundMixed : kT272Round) : kT272RoundRowMajor) *
                     (double)((phi_dev::t272_tile_count(p.M, p.N) + G - 1) / G);
    return t < square_plan_cost(p.M, p.N, G) - 1e-9;
}

// The persistent kernel over the whole problem: 256 x 256 tiles for the rows
// big_tile_rows() gives it (or the tuning table's plan), then 128 x 128 tiles
// for the rest (A, sA, C and the output rows offset; B, sB and bias are shared);
// or, K-tiled, 272 x 192 tiles where those fill whole rounds better.
hipError_t launch_persist_plan(hipStream_t stream, const phi_dev::GemmParams& p0, GemmKernel gk, bool w4, int c_dtype,
                               int64_t ldc) {
    const int G = num_cus();
    const int64_t M = p0.M;
    phi_gemm_plan plan{};
    const bool tuned = gk == GK_PERSIST && !w4 && tuned_plan(M, p0.N, p0.K, p0.kt, &plan);
    phi_dev::GemmParams p = p0;
    if (tuned && plan.group_m > 0) p.group_m = plan.group_m;
    if (gk == GK_PERSIST && !w4 && use_t272(p0, G, tuned ? plan.tile : PHI_PLAN_TILE_AUTO))
        return phi_dev::launch_i8_gemm_t272(stream, p, G);
    // int8 B runs on the four-stage pipeline; PHI_GEMM_PIPE=0 selects the
    // two-stage kernel (an A/B switch).  W4 B (codes expanded in registers)
    // runs on the two-stage kernel.
    const char* pe = getenv("PHI_GEMM_PIPE");
    const bool pipe = p0.kt || (!w4 && !(pe && pe[0] == '0'));  // K-tiled operands: the pipeline only
    const int64_t rows = gk == GK_PERSIST ? (tuned && plan.big_rows >= 0 ? plan.big_rows : big_tile_rows(M, p.N, G))
                         : gk == GK_PERSIST256 ? M
                                               : 0;
    phi_dev::GemmParams q = p;
    q.M = (int)(M - rows);
    q.A = p.A + rows * p.lda;
    if (q.sA) q.sA = p.sA + rows;
    q.C = (int8_t*)p.C + rows * ldc * (int64_t)c_elem_bytes(c_dtype);
    if (rows > 0 && rows < M) {
        // Both tile sizes: one launch (PHI_GEMM_MIXED=0 splits it in two, an
        // A/B switch; so does a tuned plan's split).
        const char* e = getenv("PHI_GEMM_MIXED");
        if (!(e && e[0] == '0') && !(tuned && plan.split)) {
            phi_dev::GemmParams b = p;
            b.M = (int)rows;
            return pipe ? phi_dev::launch_i8_gemm_pipe_mixed(stream, b, q, G)
                        : phi_dev::launch_i8_gemm_persist_mixed(stream, b, q, G, w4);
        }
    }
    if (rows > 0) {
        phi_dev::GemmParams b = p;
        b.M = (int)rows;
        const hipError_t e = pipe ? phi_dev::launch_i8_gemm_pipe(stream, b, G, 128)
                                  : phi_dev::launch_i8_gemm_persist(stream, b, G, 128, w4);
        if (e != hipSuccess || rows == M) return e;
    }
    return pipe ? phi_dev::launch_i8_gemm_pipe(stream, q, G, 64) : phi_dev::launch_i8_gemm_persist(stream, q, G, 64, w4);
}

// Vector-store / vector-load eligibility of the epilogue operands.
void set_vec_flags(phi_dev::GemmParams& p, int c_dtype, int64_t ldc) {
    const size_t cal = c_dtype == PHI_BF16 ? 8 : 16;
    p.c_vec = aligned(p.C, cal) && ldc % 4 == 0;
    p.c_vec16 = aligned(p.C, 16) && (ldc * (int64_t)c_elem_bytes(c_dtype)) % 16 == 0;
    const bool sb_ok = p.sb_scalar || !p.sB || aligned(p.sB, 16);
    const bool b_ok = p.bias_kind == phi_dev::BIAS_NONE ||
                      aligned(p.bias, p.bias_kind == phi_dev::BIAS_BF16 ? 8 : 16);
    p.s_vec = sb_ok && b_ok;
}

}  // namespace

namespace phi_capi {

// The error contract for entry points defined in other files of the library.
phi_status fail(phi_status st, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vfail(st, fmt, ap);
    va_end(ap);
    return st;
}

bool device_lost() { return g_lost; }

}  // namespace phi_capi

extern "C" {

const char* phi_hip_last_error(void) { return g_err.c_str(); }

int phi_hip_abi_version(void) { return PHI_QLINEAR_ABI_VERSION; }

// The prologue's contract (rows > 0).
static phi_status quant_rotate_check(const char* who, const void* x, int x_dtype, int64_t rows, int64_t K, int64_t ldx,
                                     const phi_dev::QrPre& pre, int8_t* q, int64_t ldq, float* s, float qmax,
                                     int round_mode) {
    if (x_dtype != PHI_F32 && x_dtype != PHI_BF16) return fail(PHI_ERR_ARG, "%s: x dtype must be f32 or bf16", who);
    if (round_mode != PHI_ROUND_HALF_AWAY && round_mode != PHI_ROUND_HALF_EVEN) return fail(PHI_ERR_ARG, "%s: bad round mode", who);
    if (!x || !q || !s) return fail(PHI_ERR_ARG, "%s: null pointer", who);
    if (K <= 0 || K % 256 != 0)
        return fail(PHI_ERR_SHAPE, "quant_convrot: K=%lld is not a multiple of 256 (convrot group size)", (long long)K);
    if (K > kMaxRotK) return fail(PHI_ERR_UNSUPPORTED, "%s: K=%lld exceeds %lld", who, (long long)K, (long long)kMaxRotK);
    if (rows > INT32_MAX) return fail(PHI_ERR_SHAPE, "%s: rows exceeds 2^31", who);
    if (!(qmax >= 1.0f && qmax <= 127.0f) || qmax != (float)(int)qmax) return fail(PHI_ERR_ARG, "%s: qmax must be an integer in [1,127]", who);
    const int64_t xcols = pre.op == phi_dev::QR_SILU_GATE ? 2 * K : K;
    if (ldx < xcols || ldq < K)
        return fail(PHI_ERR_SHAPE, "%s: leading dimension smaller than %s", who,
                    pre.op == phi_dev::QR_SILU_GATE ? "2K (gate and value halves)" : "K");
    const size_t esz = x_dtype == PHI_BF16 ? 2 : 4;
    if (!aligned(x, 16) || (ldx * (int64_t)esz) % 16 != 0 || !aligned(q, 16) || ldq % 16 != 0 || !aligned(s, 4))
        return fail(PHI_ERR_ALIGN, "%s: x and q rows must be 16-byte aligned", who);
    if ((pre.sc && !aligned(pre.sc, 16)) || (pre.sh && !aligned(pre.sh, 16)))
        return fail(PHI_ERR_ALIGN, "%s: modulation vectors must be 16-byte aligned", who);
    return PHI_OK;
}

static phi_status quant_rotate_impl(const char* who, phi_stream_t stream, const void* x, int x_dtype, int64_t rows,
                                    int64_t K, int64_t ldx, const phi_dev::QrPre& pre, int8_t* q,
                                    int64_t ldq, float* s, float qmax, int round_mode, int rotate) {
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    if (rows < 0 || K < 0) return fail(PHI_ERR_SHAPE, "%s: negative size", who);
    if (rows == 0) return ok();
    const phi_status st = quant_rotate_check(who, x, x_dtype, rows, K, ldx, pre, q, ldq, s, qmax, round_mode);
    if (st != PHI_OK) return st;
    return check_hip(phi_dev::launch_quant_rotate((hipStream_t)stream, x, x_dtype == PHI_BF16, rows, K, ldx, q, ldq, s,
                                                  qmax, round_mode == PHI_ROUND_HALF_EVEN, rotate ? 1 : 0, pre),
                     who);
}

phi_status phi_hip_quant_rotate(phi_stream_t stream, const void* x, int x_dtype, int64_t rows,
                                int64_t K, int64_t ldx, int8_t* q, int64_t ldq, float* s,
                                float qmax, int round_mode, int rotate) {
    const phi_dev::QrPre pre = {phi_dev::QR_PLAIN, nullptr, nullptr, 0};
    return quant_rotate_impl("quant_rotate", stream, x, x_dtype, rows, K, ldx, pre, q, ldq, s, qmax, round_mode, rotate);
}

phi_status phi_hip_quant_rotate_mod(phi_stream_t stream, const void* x, int x_dtype, int64_t rows,
                                    int64_t K, int64_t ldx, const float* mod_scale, const float* mod_shift,
                                    int8_t* q, int64_t ldq, float* s, float qmax, int round_mode,
                                    int rotate) {
    const phi_dev::QrPre pre = {mod_scale || mod_shift ? phi_dev::QR_MOD : phi_dev::QR_PLAIN, mod_scale, mod_shift, 0};
    return quant_rotate_impl("quant_rotate_mod", stream, x, x_dtype, rows, K, ldx, pre, q, ldq, s, qmax, round_mode,
                             rotate);
}

phi_status phi_hip_quant_rotate_act(phi_stream_t stream, const void* x, int x_dtype, int64_t rows, int64_t K,
                                    int64_t ldx, int act, int8_t* q, int64_t ldq, float* s, float qmax,
                                    int round_mode, int rotate) {
    if (act != PHI_ACT_GELU_TANH && act != PHI_ACT_SILU_GATE)
        return fail(PHI_ERR_ARG, "quant_rotate_act: act must be PHI_ACT_GELU_TANH or PHI_ACT_SILU_GATE");
    const phi_dev::QrPre pre = {act == PHI_ACT_GELU_TANH ? phi_dev::QR_GELU : phi_dev::QR_SILU_GATE, nullptr, nullptr, K};
    return quant_rotate_impl("quant_rotate_act", stream, x, x_dtype, rows, K, ldx, pre, q, ldq, s, qmax, round_mode,
                             rotate);
}

size_t phi_hip_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    (void)M;
    (void)N;
    (void)K;
    return 0;
}

phi_status phi_hip_i8_gemm(phi_stream_t stream, const int8_t* A, int64_t lda, const int8_t* B,
                           int64_t ldb, const float* sA, const float* sB, int sb_scalar,
                           const void* bias, int bias_dtype, void* C, int c_dtype, int64_t ldc,
                           int64_t M, int64_t N, int64_t K, void* workspace, size_t ws_bytes) {
    static const char* who = "int8_gemm";
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    phi_status st = check_gemm(who, A, lda, B, ldb, M, N, K, sA, sB, C, c_dtype, ldc, false, true);
    if (st != PHI_OK) return st;
    (void)workspace;  // no kernel needs one (phi_hip_workspace_bytes is 0)
    (void)ws_bytes;
    const int bk = bias_kind_of(bias, bias_dtype, &st);
    if (st != PHI_OK) return fail(st, "%s: bias dtype must be f32 or bf16", who);
    if (bias && !aligned(bias, bk == phi_dev::BIAS_BF16 ? 2 : 4)) return fail(PHI_ERR_ALIGN, "%s: bias is misaligned", who);
    // The MFMA kernels stage 16-byte chunks of whole 64-deep K-tiles.  Any
    // other K, or an operand at an offset or pitch that is not a multiple of
    // 16 bytes, takes the same kernel in its any-K form (the reference routes
    // those to int8_gemm_dp4a, core/runtime/compute.cpp:566-575);
    // PHI_GEMM_KERNEL=any forces it (an A/B switch, like PHI_INT8_DP4A).
    const char* ek = getenv("PHI_GEMM_KERNEL");
    const bool staged_ok = K % 64 == 0 && aligned(A, 16) && lda % 16 == 0 && aligned(B, 16) && ldb % 16 == 0;
    phi_dev::GemmParams p{};
    p.A = A;
    p.B = B;
    p.sA = sA;
    p.sB = sB;
    p.bias = bias;
    p.C = C;
    p.lda = lda;
    p.ldb = ldb;
    p.ldc = ldc;
    p.M = (int)M;
    p.N = (int)N;
    p.K = (int)K;
    p.sb_scalar = sb_scalar ? 1 : 0;
    p.bias_kind = bk;
    p.c_kind = c_kind_of(c_dtype);
    p.group_m = 4;
    set_vec_flags(p, c_dtype, ldc);
    if (!staged_ok || (ek && strcmp(ek, "any") == 0))
        return check_hip(phi_dev::launch_i8_gemm_any((hipStream_t)stream, p, gemm_cfg_for(M, N)), who);
    const GemmKernel gk = gemm_kernel_for(M, N, K, persist_ok(C, c_dtype, N, K, lda, ldb, ldc));
    if (gk == GK_PERSIST || gk == GK_PERSIST256 || gk == GK_PERSIST128)
        return check_hip(launch_persist_plan((hipStream_t)stream, p, gk, false, c_dtype, ldc), who);
    if (gk != GK_TILE128) {
        p.schedule = gk == GK_TILE256W4 ? 1 : 0;
        return check_hip(phi_dev::launch_i8_gemm_256((hipStream_t)stream, p), who);
    }
    return check_hip(phi_dev::launch_i8_gemm((hipStream_t)stream, p, gemm_cfg_for(M, N)), who);
}

phi_status phi_hip_i8_gemm_residual(phi_stream_t stream, const int8_t* A, int64_t lda, const int8_t* B,
                                    int64_t ldb, const float* sA, const float* sB, int sb_scalar,
                                    const void* bias, int bias_dtype, const float* gate, float* H,
                                    int64_t ldh, int64_t M, int64_t N, int64_t K, void* workspace,
                                    size_t ws_bytes) {
    static const char* who = "int8_gemm_residual";
    (void)workspace;
    (void)ws_bytes;
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    phi_status st = check_gemm(who, A, lda, B, ldb, M, N, K, sA, sB, H, PHI_F32, ldh, false);
    if (st != PHI_OK) return st;
    if (!gate) return fail(PHI_ERR_ARG, "%s: null gate", who);
    if (!aligned(gate, 4)) return fail(PHI_ERR_ALIGN, "%s: gate must be 4-byte aligned", who);
    if (!persist_ok(H, PHI_F32, N, K, lda, ldb, ldh))
        return fail(PHI_ERR_UNSUPPORTED, "%s: needs K %% 256 == 0, N %% 4 == 0 and 16-byte aligned H rows", who);
    const int bk = bias_kind_of(bias, bias_dtype, &st);
    if (st != PHI_OK) return fail(st, "%s: bias dtype must be f32 or bf16", who);
    phi_dev::GemmParams p{};
    p.A = A;
    p.B = B;
    p.sA = sA;
    p.sB = sB;
    p.bias = bias;
    p.C = H;
    p.lda = lda;
    p.ldb = ldb;
    p.ldc = ldh;
    p.M = (int)M;
    p.N = (int)N;
    p.K = (int)K;
    p.sb_scalar = sb_scalar ? 1 : 0;
    p.bias_kind = bk;
    p.c_kind = phi_dev::C_F32;
    p.group_m = 4;
    p.gate = gate;
    set_vec_flags(p, PHI_F32, ldh);
    GemmKernel gk = GK_PERSIST;
    const char* e = getenv("PHI_GEMM_KERNEL");
    if (e && strcmp(e, "persist256") == 0) gk = GK_PERSIST256;
    if (e && strcmp(e, "persist128") == 0) gk = GK_PERSIST128;
    return check_hip(launch_persist_plan((hipStream_t)stream, p, gk, false, PHI_F32, ldh), who);
}

phi_status phi_hip_q8_linear(phi_stream_t stream, const void* x, int x_dtype, int64_t ldx,
                             int64_t M, int64_t K, const int8_t* W, int64_t ldw, const float* sW,
                             int sw_scalar, const void* bias, int bias_dtype, int64_t N, void* C,
                             int c_dtype, int64_t ldc, int8_t* q8, float* s8, int round_mode,
                             void* workspace, size_t ws_bytes) {
    static const char* who = "linear_gemm";
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    if (!q8 || !s8) return fail(PHI_ERR_ARG, "linear_gemm: the int8 path needs activation scratch");
    if (M <= 0) return fail(PHI_ERR_SHAPE, "%s: empty problem", who);
    phi_status st = check_gemm(who, q8, K, W, ldw, M, N, K, s8, sW, C, c_dtype, ldc, false);
    if (st != PHI_OK) return st;
    st = phi_hip_quant_rotate(stream, x, x_dtype, M, K, ldx, q8, K, s8, 127.0f, round_mode, 1);
    if (st != PHI_OK) return st;
    return phi_hip_i8_gemm(stream, q8, K, W, ldw, s8, sW, sw_scalar, bias, bias_dtype, C, c_dtype, ldc, M, N, K,
                           workspace, ws_bytes);
}

// The K-tiled operand contract: whole 256-deep K-steps (the pipeline's pairs
// of 64-deep stages, and whole rotation groups), 16-byte aligned bases, and
// strip offsets within 32 bits (256 x K < 2^31).
static phi_status check_kt(const char* who, const void* A, const void* B, int64_t K) {
    if (K % 256 != 0) return fail(PHI_ERR_SHAPE, "%s: K=%lld is not a multiple of 256", who, (long long)K);
    if (K >= ((int64_t)1 << 23)) return fail(PHI_ERR_SHAPE, "%s: K=%lld is too large for the K-tiled layout", who, (long long)K);
    if (!aligned(A, 16) || !aligned(B, 16)) return fail(PHI_ERR_ALIGN, "%s: K-tiled operands must be 16-byte aligned", who);
    return PHI_OK;
}

static phi_status i8_gemm_kt_impl(const char* who, phi_stream_t stream, const int8_t* A, const int8_t* B,
                                  const float* sA, const float* sB, int sb_scalar, const void* bias, int bias_dtype,
                                  void* C, int c_dtype, int64_t ldc, int64_t M, int64_t N, int64_t K,
                                  const float* gate = nullptr) {
    phi_status st = check_gemm(who, A, K, B, K, M, N, K, sA, sB, C, c_dtype, ldc, false);
    if (st != PHI_OK) return st;
    if ((st = check_kt(who, A, B, K)) != PHI_OK) return st;
    if (!persist_ok(C, c_dtype, N, K, K, K, ldc))
        return fail(PHI_ERR_UNSUPPORTED, "%s: needs whole 16-byte output pieces on 16-byte aligned C rows", who);
    const int bk = bias_kind_of(bias, bias_dtype, &st);
    if (st != PHI_OK) return fail(st, "%s: bias dtype must be f32 or bf16", who);
    if (bias && !aligned(bias, bk == phi_dev::BIAS_BF16 ? 2 : 4)) return fail(PHI_ERR_ALIGN, "%s: bias is misaligned", who);
    phi_dev::GemmParams p{};
    p.A = A;
    p.B = B;
    p.sA = sA;
    p.sB = sB;
    p.bias = bias;
    p.C = C;
    p.lda = K;
    p.ldb = K;
    p.ldc = ldc;
    p.M = (int)M;
    p.N = (int)N;
    p.K = (int)K;
    p.sb_scalar = sb_scalar ? 1 : 0;
    p.bias_kind = bk;
    p.c_kind = c_kind_of(c_dtype);
    p.group_m = 4;
    p.kt = 1;
    p.gate = gate;
    set_vec_flags(p, c_dtype, ldc);
    GemmKernel gk = GK_PERSIST;
    const char* e = getenv("PHI_GEMM_KERNEL");
    if (e && strcmp(e, "persist256") == 0) gk = GK_PERSIST256;
    if (e && strcmp(e, "persist128") == 0) gk = GK_PERSIST128;
    return check_hip(launch_persist_plan((hipStream_t)stream, p, gk, false, c_dtype, ldc), who);
}

phi_status phi_hip_gemm_plan_set(int64_t M, int64_t N, int64_t K, int k_tiled, const phi_gemm_plan* plan) {
    static const char* who = "gemm_plan_set";
    if (M <= 0 || N <= 0 || K <= 0) return fail(PHI_ERR_SHAPE, "%s: empty problem", who);
    const PlanKey key{M, N, K, k_tiled ? 1 : 0};
    std::lock_guard<std::mutex> lk(g_plans_mu);
    if (!plan) {
        g_plans.erase(key);
    } else {
        if (plan->big_rows < -1 || plan->big_rows > M || (plan->big_rows >= 0 && plan->big_rows % 256 != 0 &&
                                                          plan->big_rows != M))
            return fail(PHI_ERR_ARG, "%s: big_rows=%lld is not -1, a multiple of 256 up to M, or M=%lld", who,
                        (long long)plan->big_rows, (long long)M);
        if (plan->group_m < 0 || plan->group_m > 16)
            return fail(PHI_ERR_ARG, "%s: group_m=%d is not 0 (the default) or 1..16", who, (int)plan->group_m);
        if (plan->split != 0 && plan->split != 1) return fail(PHI_ERR_ARG, "%s: split must be 0 or 1", who);
        if (plan->tile < PHI_PLAN_TILE_AUTO || plan->tile > PHI_PLAN_TILE_272)
            return fail(PHI_ERR_ARG, "%s: tile=%d is not 0 (the cost model), 1 (square) or 2 (272 x 192)", who,
                        (int)plan->tile);
        if (plan->tile == PHI_PLAN_TILE_272 && K % 512 != 0)
            return fail(PHI_ERR_ARG, "%s: tile=2 (272 x 192) needs K %% 512 == 0 (K=%lld)", who, (long long)K);
        g_plans[key] = *plan;
    }
    g_plan_count.store((int64_t)g_plans.size(), std::memory_order_release);
    return ok();
}

phi_status phi_hip_gemm_plan_get(int64_t M, int64_t N, int64_t K, int k_tiled, phi_gemm_plan* plan, int* tuned) {
    static const char* who = "gemm_plan_get";
    if (M <= 0 || N <= 0 || K <= 0) return fail(PHI_ERR_SHAPE, "%s: empty problem", who);
    if (!plan) return fail(PHI_ERR_ARG, "%s: null plan", who);
    phi_gemm_plan p{-1, 0, 0, PHI_PLAN_TILE_AUTO, 0};
    const bool t = tuned_plan(M, N, K, k_tiled, &p);
    if (tuned) *tuned = t ? 1 : 0;
    const int G = num_cus();
    if (p.big_rows < 0) p.big_rows = big_tile_rows(M, N, G);
    if (p.group_m == 0) p.group_m = 4;
    // The tile shape a launch with bf16 output (ldc = N) resolves to.
    bool t272 = false;
    if (M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX) {
        phi_dev::GemmParams q{};
        q.M = (int)M;
        q.N = (int)N;
        q.K = (int)K;
        q.lda = K;
        q.ldb = K;
        q.ldc = N;
        q.c_kind = phi_dev::C_BF16;
        q.kt = k_tiled ? 1 : 0;
        t272 = use_t272(q, G, p.tile);
    }
    p.tile = t272 ? PHI_PLAN_TILE_272 : PHI_PLAN_TILE_SQUARE;
    p.reserved = 0;
    *plan = p;
    return ok();
}

int64_t phi_hip_gemm_plan_count(void) { return g_plan_count.load(std::memory_order_acquire); }

void phi_hip_gemm_plan_clear(void) {
    std::lock_guard<std::mutex> lk(g_plans_mu);
    g_plans.clear();
    g_plan_count.store(0, std::memory_order_release);
}

int64_t phi_hip_big_tile_rows(int64_t M, int64_t N) {
    if (M <= 0 || N <= 0 || M > INT32_MAX || N > INT32_MAX) return 0;
    return big_tile_rows(M, N, num_cus());
}

phi_status phi_hip_pack_k_tiled(phi_stream_t stream, const int8_t* src, int64_t ld, int64_t rows, int64_t K,
                                int8_t* dst) {
    static const char* who = "pack_k_tiled";
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    if (rows <= 0 || K <= 0) return fail(PHI_ERR_SHAPE, "%s: empty matrix (rows=%lld K=%lld)", who, (long long)rows, (long long)K);
    if (rows > INT32_MAX) return fail(PHI_ERR_SHAPE, "%s: rows exceeds 2^31", who);
    if (!src || !dst) return fail(PHI_ERR_ARG, "%s: null pointer", who);
    phi_status st = check_kt(who, src, dst, K);
    if (st != PHI_OK) return st;
    if (ld < K || ld % 16 != 0) return fail(PHI_ERR_ALIGN, "%s: ld must be >= K and a multiple of 16", who);
    return check_hip(phi_dev::launch_pack_k_tiled((hipStream_t)stream, src, ld, rows, K, dst), who);
}

static phi_status quant_rotate_kt_impl(const char* who, phi_stream_t stream, const void* x, int x_dtype, int64_t rows,
                                       int64_t K, int64_t ldx, const phi_dev::QrPre& pre, int8_t* q, float* s,
                                       float qmax, int round_mode) {
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    if (rows <= 0) return fail(PHI_ERR_SHAPE, "%s: empty problem (rows=%lld)", who, (long long)rows);
    phi_status st = quant_rotate_check(who, x, x_dtype, rows, K, ldx, pre, q, K, s, qmax, round_mode);
    if (st != PHI_OK) return st;
    if (K > 16384) return fail(PHI_ERR_UNSUPPORTED, "%s: K=%lld exceeds 16384 (K-tiled activations)", who, (long long)K);
    return check_hip(phi_dev::launch_quant_rotate((hipStream_t)stream, x, x_dtype == PHI_BF16, rows, K, ldx, q, K, s,
                                                  qmax, round_mode == PHI_ROUND_HALF_EVEN, 1, pre, 1),
                     who);
}

phi_status phi_hip_quant_rotate_kt(phi_stream_t stream, const void* x, int x_dtype, int64_t rows, int64_t K,
                                  int64_t ldx, int8_t* q, float* s, float qmax, int round_mode) {
    const phi_dev::QrPre pre{};
    return quant_rotate_kt_impl("quant_convrot_kt", stream, x, x_dtype, rows, K, ldx, pre, q, s, qmax, round_mode);
}

phi_status phi_hip_quant_rotate_mod_kt(phi_stream_t stream, const void* x, int x_dtype, int64_t rows, int64_t K,
                                      int64_t ldx, const float* mod_scale, const float* mod_shift, int8_t* q,
                                      float* s, float qmax, int round_mode) {
    const phi_dev::QrPre pre = {mod_scale || mod_shift ? phi_dev::QR_MOD : phi_dev::QR_PLAIN, mod_scale, mod_shift, 0};
    return quant_rotate_kt_impl("quant_rotate_mod_kt", stream, x, x_dtype, rows, K, ldx, pre, q, s, qmax, round_mode);
}

phi_status phi_hip_quant_rotate_act_kt(phi_stream_t stream, const void* x, int x_dtype, int64_t rows, int64_t K,
                                      int64_t ldx, int act, int8_t* q, float* s, float qmax, int round_mode) {
    if (act != PHI_ACT_GELU_TANH && act != PHI_ACT_SILU_GATE)
        return fail(PHI_ERR_ARG, "quant_rotate_act_kt: act must be PHI_ACT_GELU_TANH or PHI_ACT_SILU_GATE");
    const phi_dev::QrPre pre = {act == PHI_ACT_GELU_TANH ? phi_dev::QR_GELU : phi_dev::QR_SILU_GATE, nullptr, nullptr, K};
    return quant_rotate_kt_impl("quant_rotate_act_kt", stream, x, x_dtype, rows, K, ldx, pre, q, s, qmax, round_mode);
}

phi_status phi_hip_i8_gemm_kt(phi_stream_t stream, const int8_t* A, const int8_t* B, const float* sA, const float* sB,
                              int sb_scalar, const void* bias, int bias_dtype, void* C, int c_dtype, int64_t ldc,
                              int64_t M, int64_t N, int64_t K) {
    static const char* who = "int8_gemm_kt";
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    return i8_gemm_kt_impl(who, stream, A, B, sA, sB, sb_scalar, bias, bias_dtype, C, c_dtype, ldc, M, N, K);
}

phi_status phi_hip_i8_gemm_residual_kt(phi_stream_t stream, const int8_t* A, const int8_t* B, const float* sA,
                                       const float* sB, int sb_scalar, const void* bias, int bias_dtype,
                                       const float* gate, float* H, int64_t ldh, int64_t M, int64_t N, int64_t K) {
    static const char* who = "int8_gemm_residual_kt";
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    if (!gate) return fail(PHI_ERR_ARG, "%s: null gate", who);
    if (!aligned(gate, 4)) return fail(PHI_ERR_ALIGN, "%s: gate must be 4-byte aligned", who);
    return i8_gemm_kt_impl(who, stream, A, B, sA, sB, sb_scalar, bias, bias_dtype, H, PHI_F32, ldh, M, N, K, gate);
}

phi_status phi_hip_q8_linear_kt(phi_stream_t stream, const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K,
                                const int8_t* W, const float* sW, int sw_scalar, const void* bias, int bias_dtype,
                                int64_t N, void* C, int c_dtype, int64_t ldc, int8_t* q8, float* s8, int round_mode) {
    static const char* who = "linear_gemm_kt";
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    if (!q8 || !s8) return fail(PHI_ERR_ARG, "%s: the int8 path needs activation scratch", who);
    if (M <= 0) return fail(PHI_ERR_SHAPE, "%s: empty problem", who);
    phi_status st = check_gemm(who, q8, K, W, K, M, N, K, s8, sW, C, c_dtype, ldc, false);
    if (st != PHI_OK) return st;
    if ((st = check_kt(who, q8, W, K)) != PHI_OK) return st;
    if (K > 16384) return fail(PHI_ERR_UNSUPPORTED, "%s: K=%lld exceeds 16384 (K-tiled activations)", who, (long long)K);
    if (!persist_ok(C, c_dtype, N, K, K, K, ldc))
        return fail(PHI_ERR_UNSUPPORTED, "%s: needs whole 16-byte output pieces on 16-byte aligned C rows", who);
    st = phi_hip_quant_rotate_kt(stream, x, x_dtype, M, K, ldx, q8, s8, 127.0f, round_mode);
    if (st != PHI_OK) return st;
    return i8_gemm_kt_impl(who, stream, q8, W, s8, sW, sw_scalar, bias, bias_dtype, C, c_dtype, ldc, M, N, K);
}

// phi_hip_q8_linear with the activation scratch written K-tiled while the
// weight stays row-major: the 272 x 192 kernel reads A in K-tiled pieces and
// gathers B's rows.  Where that plan does not apply or does not pay (its
// rounds against the square plan's), the call is phi_hip_q8_linear itself.
phi_status phi_hip_q8_linear_kq(phi_stream_t stream, const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K,
                                const int8_t* W, int64_t ldw, const float* sW, int sw_scalar, const void* bias,
                                int bias_dtype, int64_t N, void* C, int c_dtype, int64_t ldc, int8_t* q8, float* s8,
                                int round_mode, void* workspace, size_t ws_bytes) {
    static const char* who = "linear_gemm";
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    if (!q8 || !s8) return fail(PHI_ERR_ARG, "linear_gemm: the int8 path needs activation scratch");
    if (M <= 0) return fail(PHI_ERR_SHAPE, "%s: empty problem", who);
    phi_status st = check_gemm(who, q8, K, W, ldw, M, N, K, s8, sW, C, c_dtype, ldc, false);
    if (st != PHI_OK) return st;
    const int bk = bias_kind_of(bias, bias_dtype, &st);
    if (st != PHI_OK) return fail(st, "%s: bias dtype must be f32 or bf16", who);
    bool mixed = K % 256 == 0 && K <= 16384 && aligned(q8, 16) && persist_ok(C, c_dtype, N, K, K, ldw, ldc) &&
                 !(bias && !aligned(bias, bk == phi_dev::BIAS_BF16 ? 2 : 4)) && !getenv("PHI_GEMM_KERNEL");
    phi_dev::GemmParams p{};
    if (mixed) {
        p.A = q8;
        p.B = W;
        p.sA = s8;
        p.sB = sW;
        p.bias = bias;
        p.C = C;
        p.lda = K;
        p.ldb = ldw;
        p.ldc = ldc;
        p.M = (int)M;
        p.N = (int)N;
        p.K = (int)K;
        p.sb_scalar = sw_scalar ? 1 : 0;
        p.bias_kind = bk;
        p.c_kind = c_kind_of(c_dtype);
        p.group_m = 4;
        p.kt = 1;
        p.b_rm = 1;
        set_vec_flags(p, c_dtype, ldc);
        mixed = use_t272(p, num_cus(), PHI_PLAN_TILE_AUTO);
    }
    if (!mixed)
        return phi_hip_q8_linear(stream, x, x_dtype, ldx, M, K, W, ldw, sW, sw_scalar, bias, bias_dtype, N, C, c_dtype,
                                 ldc, q8, s8, round_mode, workspace, ws_bytes);
    st = phi_hip_quant_rotate_kt(stream, x, x_dtype, M, K, ldx, q8, s8, 127.0f, round_mode);
    if (st != PHI_OK) return st;
    return check_hip(phi_dev::launch_i8_gemm_t272((hipStream_t)stream, p, num_cus()), who);
}

static phi_status check_w4a8(const char* who, const phi_w4a8_weight* w, bool lut) {
    if (!w) return fail(PHI_ERR_ARG, "%s: null weight descriptor", who);
    if (w->rows < 0 || w->k < 0) return fail(PHI_ERR_SHAPE, "%s: negative size", who);
    if (w->group <= 0 || w->k % w->group != 0)
        return fail(PHI_ERR_SHAPE, "w4a8_expand: K=%lld is not a multiple of group=%lld", (long long)w->k, (long long)w->group);
    if (w->layout != 0 && w->layout != 1) return fail(PHI_ERR_ARG, "%s: bad layout %d", who, w->layout);
    if (w->group % (w->layout == 0 ? 2 : 4) != 0)
        return fail(PHI_ERR_SHAPE, "w4a8_expand: group=%lld is not a whole number of code groups for this layout", (long long)w->group);
    if (w->k % 16 != 0) return fail(PHI_ERR_SHAPE, "%s: K=%lld is not a multiple of 16", who, (long long)w->k);
    const int64_t need = w->layout == 0 ? w->k / 2 : w->k / 2 + w->k / 4;
    if (w->codes_row_bytes < need)
        return fail(PHI_ERR_SHAPE, "w4a8_expand: a %lld-column row needs %lld packed bytes, got %lld", (long long)w->k, (long long)need, (long long)w->codes_row_bytes);
    if (!w->codes) return fail(PHI_ERR_ARG, "w4a8_expand: missing binding");
    if (w->codebook && w->layout != 0) return fail(PHI_ERR_ARG, "w4a8_expand: only the 4-bit family indexes a codebook");
    const int d = w->s_rel_dtype;
    if (w->s_rel && !(d == PHI_F32 || d == PHI_F16 || d == PHI_BF16 || d == PHI_F8_E4M3 || d == PHI_F8_E5M2 || d == PHI_U8_E4M3))
        return fail(PHI_ERR_ARG, "%s: unreadable relative-scale dtype %d", who, d);
    const int64_t rsz = d == PHI_F32 ? 4 : (d == PHI_F16 || d == PHI_BF16) ? 2 : 1;
    if (w->s_rel && w->srel_row_bytes < (w->k / w->group) * rsz) return fail(PHI_ERR_SHAPE, "%s: relative-scale row too short", who);
    if (lut && w->layout != 0) return fail(PHI_ERR_UNSUPPORTED, "%s: the in-register table is for the nibble layout only", who);
    if (w->rows > INT32_MAX || w->k > INT32_MAX) return fail(PHI_ERR_SHAPE, "%s: rows or K exceeds 2^31", who);
    return PHI_OK;
}

static phi_dev::W4a8Params w4a8_params(const phi_w4a8_weight* w) {
    phi_dev::W4a8Params p{};
    p.codes = w->codes;
    p.codes_row_bytes = w->codes_row_bytes;
    p.s_rel = w->s_rel;
    p.s_rel_dtype = w->s_rel_dtype;
    p.srel_row_bytes = w->srel_row_bytes;
    p.s_channel = w->s_channel;
    p.sch_scalar = w->sch_scalar;
    p.codebook = w->codebook;
    p.correction = w->correction;
    p.rows = w->rows;
    p.k = w->k;
    p.group = w->group;
    p.layout = w->layout;
    return p;
}

phi_status phi_hip_w4a8_expand(phi_stream_t stream, const phi_w4a8_weight* w, int8_t* q, float* s) {
    static const char* who = "w4a8_expand";
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    phi_status st = check_w4a8(who, w, false);
    if (st != PHI_OK) return st;
    if (w->rows == 0 || w->k == 0) return ok();
    if (!q || !s) return fail(PHI_ERR_ARG, "w4a8_expand: missing binding");
    if (!aligned(q, 16)) return fail(PHI_ERR_ALIGN, "%s: q must be 16-byte aligned", who);
    return check_hip(phi_dev::launch_w4a8_rows((hipStream_t)stream, w4a8_params(w), q, s, false), who);
}

phi_status phi_hip_w4a8_prepare(phi_stream_t stream, const phi_w4a8_weight* w, int8_t* lut, float* s) {
    static const char* who = "w4a8_prepare";
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    phi_status st = check_w4a8(who, w, true);
    if (st != PHI_OK) return st;
    if (w->rows == 0 || w->k == 0) return ok();
    if (!lut || !s) return fail(PHI_ERR_ARG, "%s: missing binding", who);
    if (!aligned(lut, 16)) return fail(PHI_ERR_ALIGN, "%s: lut must be 16-byte aligned", who);
    return check_hip(phi_dev::launch_w4a8_rows((hipStream_t)stream, w4a8_params(w), lut, s, true), who);
}

phi_status phi_hip_w4a8_linear(phi_stream_t stream, const void* x, int x_dtype, int64_t ldx,
                               int64_t M, int64_t K, const uint8_t* codes,
                               int64_t codes_row_bytes, const int8_t* lut, int64_t group,
                               const float* s_w, const void* bias, int bias_dtype, int64_t N,
                               void* C, int c_dtype, int64_t ldc, int8_t* q8, float* s8,
                               int round_mode, void* workspace, size_t ws_bytes) {
    static const char* who = "w4a8_linear";
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    if (!q8 || !s8) return fail(PHI_ERR_ARG, "%s: the int8 path needs activation scratch", who);
    if (!lut || !s_w) return fail(PHI_ERR_ARG, "%s: missing prepared table or row scales", who);
    phi_status st = check_gemm(who, q8, K, codes, codes_row_bytes, M, N, K, s8, s_w, C, c_dtype, ldc, true);
    if (st != PHI_OK) return st;
    if (group <= 0 || group % 64 != 0 || K % group != 0 || (group & (group - 1)) != 0)
        return fail(PHI_ERR_SHAPE, "%s: group=%lld must be a power of two, a multiple of 64 and divide K", who, (long long)group);
    if (!aligned(lut, 16)) return fail(PHI_ERR_ALIGN, "%s: lut must be 16-byte aligned", who);
    const int bk = bias_kind_of(bias, bias_dtype, &st);
    if (st != PHI_OK) return fail(st, "%s: bias dtype must be f32 or bf16", who);
    const char* e = getenv("PHI_GEMM_KERNEL");
    const bool force_staged = e && strcmp(e, "tile128") == 0;
    // With a workspace (phi_hip_w4a8_workspace_bytes), large M expands the
    // codes once into it and runs the W8A8 GEMM: one table lookup per weight
    // instead of one per weight per 256-row tile.  Both operands then take the
    // K-tiled layout (K <= 16384; PHI_GEMM_KT=0 keeps them row-major, an A/B
    // switch).
    const size_t need = phi_hip_w4a8_workspace_bytes(M, N, K, group);
    // The 272 x 192 pipeline expands the codes in LDS, with no workspace: on
    // K-tiled activations, K % 1024 == 0 (t272w4_ok).  PHI_W4_T272=1 / 0
    // prefers it to / keeps it from the expand-once path (an A/B switch);
    // without a workspace it is the in-register path wherever it applies.
    // A kernel forced by PHI_GEMM_KERNEL keeps its own path.
    const int w4t = phi_dev::env_switch("PHI_W4_T272", -1, 0, 1);
    if (!e && w4t != 0 && (w4t == 1 || !(need > 0 && workspace && ws_bytes >= need)) && K <= 16384 &&
        aligned(q8, 16) && aligned(codes, 16) && codes_row_bytes % 16 == 0 &&
        persist_ok(C, c_dtype, N, K, K, codes_row_bytes, ldc)) {
        phi_dev::GemmParams q{};
        q.A = q8;
        q.B = (const int8_t*)codes;
        q.sA = s8;
        q.sB = s_w;
        q.bias = bias;
        q.C = C;
        q.lda = K;
        q.ldb = codes_row_bytes;
        q.ldc = ldc;
        q.M = (int)M;
        q.N = (int)N;
        q.K = (int)K;
        q.sb_scalar = 0;
        q.bias_kind = bk;
        q.c_kind = c_kind_of(c_dtype);
        q.group_m = 4;
        q.lut = lut;
        q.lut_groups = K / group;
        int gs = 0;
        while ((1ll << gs) < group) gs++;
        q.group_shift = gs;
        q.kt = 1;
        set_vec_flags(q, c_dtype, ldc);
        if (phi_dev::t272w4_ok(q)) {
            st = phi_hip_quant_rotate_kt(stream, x, x_dtype, M, K, ldx, q8, s8, 127.0f, round_mode);
            if (st != PHI_OK) return st;
            return check_hip(phi_dev::launch_i8_gemm_t272w4((hipStream_t)stream, q, num_cus()), who);
        }
    }
    const bool expand = !force_staged && need > 0 && workspace && ws_bytes >= need && aligned(workspace, 16) &&
                        aligned(codes, 16) && codes_row_bytes % 16 == 0 && persist_ok(C, c_dtype, N, K, K, K, ldc);
    const char* ekt = getenv("PHI_GEMM_KT");
    const bool kt = expand && K <= 16384 && aligned(q8, 16) && !(ekt && ekt[0] == '0');
    phi_dev::GemmParams p{};
    p.A = q8;
    p.B = (const int8_t*)codes;
    p.sA = s8;
    p.sB = s_w;
    p.bias = bias;
    p.C = C;
    p.lda = K;
    p.ldb = codes_row_bytes;
    p.ldc = ldc;
    p.M = (int)M;
    p.N = (int)N;
    p.K = (int)K;
    p.sb_scalar = 0;
    p.bias_kind = bk;
    p.c_kind = c_kind_of(c_dtype);
    p.group_m = 4;
    p.lut = lut;
    p.lut_groups = K / group;
    int sh = 0;
    while ((1ll << sh) < group) sh++;
    p.group_shift = sh;
    // With K-tiled activations the expansion runs as extra blocks of the
    // prologue's launch, beside the rotation (PHI_W4_FUSE=0: two launches).
    const bool fuse = kt && phi_dev::w4_expand_ok(p, (const int8_t*)workspace, true) &&
                      phi_dev::env_switch("PHI_W4_FUSE", 1, 0, 1);
    phi_dev::QrPre pre{};
    if (fuse) {
        pre.ex.on = 1;
        pre.ex.codes = codes;
        pre.ex.ldb = codes_row_bytes;
        pre.ex.lut = lut;
        pre.ex.lut_groups = p.lut_groups;
        pre.ex.group_shift = p.group_shift;
        pre.ex.kt = 1;
        pre.ex.N = N;
        pre.ex.K = K;
        pre.ex.out = (int8_t*)workspace;
    }
    st = kt ? quant_rotate_kt_impl("quant_convrot_kt", stream, x, x_dtype, M, K, ldx, pre, q8, s8, 127.0f, round_mode)
            : phi_hip_quant_rotate(stream, x, x_dtype, M, K, ldx, q8, K, s8, 127.0f, round_mode, 1);
    if (st != PHI_OK) return st;
    if (expand) {
        if (!fuse) {
            st = check_hip(phi_dev::launch_w4_lut_expand((hipStream_t)stream, p, (int8_t*)workspace, kt), who);
            if (st != PHI_OK) return st;
        }
        phi_dev::GemmParams g = p;
        g.B = (const int8_t*)workspace;
        g.ldb = K;
        g.lut = nullptr;
        g.kt = kt ? 1 : 0;
        set_vec_flags(g, c_dtype, ldc);
        GemmKernel gk = GK_PERSIST;
        if (e && strcmp(e, "persist256") == 0) gk = GK_PERSIST256;
        if (e && strcmp(e, "persist128") == 0) gk = GK_PERSIST128;
        return check_hip(launch_persist_plan((hipStream_t)stream, g, gk, false, c_dtype, ldc), who);
    }
    // In registers: the persistent kernel takes whole 128-column groups and
    // 16-byte code rows; PHI_GEMM_KERNEL=tile128 forces the register-staged
    // kernel (A/B switch).
    if (!force_staged && group % 128 == 0 && aligned(codes, 16) && codes_row_bytes % 16 == 0 &&
        persist_ok(C, c_dtype, N, K, K, codes_row_bytes, ldc)) {
        set_vec_flags(p, c_dtype, ldc);
        GemmKernel gk = GK_PERSIST;
        if (e && strcmp(e, "persist256") == 0) gk = GK_PERSIST256;
        if (e && strcmp(e, "persist128") == 0) gk = GK_PERSIST128;
        return check_hip(launch_persist_plan((hipStream_t)stream, p, gk, true, c_dtype, ldc), who);
    }
    return check_hip(phi_dev::launch_w4a8_gemm((hipStream_t)stream, p, gemm_cfg_for(M, N)), who);
}

size_t phi_hip_w4a8_banded_bytes(int64_t rows, int64_t k, int64_t group) {
    if (rows <= 0 || rows > INT32_MAX || k <= 0 || k > INT32_MAX) return 0;
    return (size_t)phi_dev::w4_banded_bytes(rows, k, group);
}

phi_status phi_hip_w4a8_pack_banded(phi_stream_t stream, const uint8_t* codes, int64_t codes_row_bytes,
                                    const int8_t* lut, int64_t rows, int64_t k, int64_t group, void* banded) {
    static const char* who = "w4a8_pack_banded";
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    if (!codes || !lut || !banded) return fail(PHI_ERR_ARG, "%s: null operand", who);
    if (rows <= 0 || k <= 0 || rows > INT32_MAX || k > INT32_MAX) return fail(PHI_ERR_SHAPE, "%s: empty or oversized weight", who);
    if (k % 64 != 0 || group <= 0 || k % group != 0)
        return fail(PHI_ERR_SHAPE, "%s: K=%lld must be a multiple of 64 and of group=%lld", who, (long long)k, (long long)group);
    if (codes_row_bytes < k / 2) return fail(PHI_ERR_SHAPE, "%s: a %lld-column nibble row needs %lld bytes", who, (long long)k, (long long)(k / 2));
    if (!aligned(codes, 16) || codes_row_bytes % 16 != 0 || !aligned(lut, 16) || !aligned(banded, 16))
        return fail(PHI_ERR_ALIGN, "%s: codes rows, lut and the packed buffer must be 16-byte aligned", who);
    if (phi_hip_w4a8_banded_bytes(rows, k, group) == 0 ||
        phi_hip_w4a8_banded_bytes(rows, k, group) >= ((size_t)1 << 31))
        return fail(PHI_ERR_SHAPE, "%s: the packed weight must stay below 2 GiB", who);
    return check_hip(phi_dev::launch_w4_pack_banded((hipStream_t)stream, codes, codes_row_bytes, lut, (int)rows, (int)k,
                                                    (int)(k / group), (uint8_t*)banded),
                     who);
}

phi_status phi_hip_w4a8_linear_banded(phi_stream_t stream, const void* x, int x_dtype, int64_t ldx, int64_t M,
                                      int64_t K, const void* banded, int64_t group, const float* s_w, const void* bias,
                                      int bias_dtype, int64_t N, void* C, int c_dtype, int64_t ldc, int8_t* q8,
                                      float* s8, int round_mode) {
    static const char* who = "w4a8_linear_banded";
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    if (!q8 || !s8) return fail(PHI_ERR_ARG, "%s: the int8 path needs activation scratch", who);
    if (!banded || !s_w) return fail(PHI_ERR_ARG, "%s: missing packed weight or row scales", who);
    phi_status st = check_gemm(who, q8, K, banded, K / 2, M, N, K, s8, s_w, C, c_dtype, ldc, true);
    if (st != PHI_OK) return st;
    if (group <= 0 || group % 64 != 0 || K % group != 0 || (group & (group - 1)) != 0)
        return fail(PHI_ERR_SHAPE, "%s: group=%lld must be a power of two, a multiple of 64 and divide K", who, (long long)group);
    if (K % 1024 != 0 || K > 16384)
        return fail(PHI_ERR_UNSUPPORTED, "%s: needs K %% 1024 == 0 and K <= 16384 (K=%lld)", who, (long long)K);
    if (!aligned(q8, 16) || !aligned(banded, 16))
        return fail(PHI_ERR_ALIGN, "%s: q8 and the packed weight must be 16-byte aligned", who);
    if (!persist_ok(C, c_dtype, N, K, K, K, ldc))
        return fail(PHI_ERR_UNSUPPORTED, "%s: needs whole 16-byte output pieces on 16-byte aligned C rows", who);
    const int bk = bias_kind_of(bias, bias_dtype, &st);
    if (st != PHI_OK) return fail(st, "%s: bias dtype must be f32 or bf16", who);
    phi_dev::GemmParams q{};
    q.A = q8;
    q.B = (const int8_t*)banded;
    q.sA = s8;
    q.sB = s_w;
    q.bias = bias;
    q.C = C;
    q.lda = K;
    q.ldb = K / 2;
    q.ldc = ldc;
    q.M = (int)M;
    q.N = (int)N;
    q.K = (int)K;
    q.bias_kind = bk;
    q.c_kind = c_kind_of(c_dtype);
    q.group_m = 4;
    q.lut_groups = K / group;
    q.lut = (const int8_t*)banded + (((N + 191) / 192) * (K / 64) * (192 * 32));
    int gs = 0;
    while ((1ll << gs) < group) gs++;
    q.group_shift = gs;
    q.kt = 1;
    q.w4_banded = 1;
    set_vec_flags(q, c_dtype, ldc);
    if (!phi_dev::t272w4_ok(q)) return fail(PHI_ERR_UNSUPPORTED, "%s: shape outside the in-LDS kernel's limits", who);
    st = phi_hip_quant_rotate_kt(stream, x, x_dtype, M, K, ldx, q8, s8, 127.0f, round_mode);
    if (st != PHI_OK) return st;
    return check_hip(phi_dev::launch_i8_gemm_t272w4((hipStream_t)stream, q, num_cus()), who);
}

size_t phi_hip_w4a8_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group) {
    // The expand-then-W8A8 path pays off once enough rows share each weight.
    if (M < kW4ExpandMinRows || N <= 0 || K <= 0 || K % 256 != 0 || group <= 0 || group % 128 != 0) return 0;
    return (size_t)N * (size_t)K;
}

size_t phi_hip_i4_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    // As for W4A8: from kW4ExpandMinRows rows the codes are expanded once.
    if (M < kW4ExpandMinRows || N <= 0 || K <= 0 || K % 512 != 0) return 0;
    return (size_t)N * (size_t)K;
}

phi_status phi_hip_i4_gemm(phi_stream_t stream, const int8_t* A, int64_t lda, const uint8_t* B, int64_t ldb,
                           const float* sA, const float* sB, void* C, int c_dtype, int64_t ldc, int64_t M,
                           int64_t N, int64_t K, void* workspace, size_t ws_bytes) {
    static const char* who = "int4_gemm";
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    if (M <= 0 || N <= 0 || K <= 0) return fail(PHI_ERR_SHAPE, "int4_gemm: empty problem");
    if (K % 512 != 0) return fail(PHI_ERR_SHAPE, "int4_gemm: K=%lld is not a multiple of 512", (long long)K);
    phi_status st = check_gemm(who, A, lda, B, ldb, M, N, K, sA, sB, C, c_dtype, ldc, true);
    if (st != PHI_OK) return st;
    phi_dev::GemmParams p{};
    p.A = A;
    p.B = (const int8_t*)B;
    p.sA = sA;
    p.sB = sB;
    p.C = C;
    p.lda = lda;
    p.ldb = ldb;
    p.ldc = ldc;
    p.M = (int)M;
    p.N = (int)N;
    p.K = (int)K;
    p.bias_kind = phi_dev::BIAS_NONE;
    p.c_kind = c_kind_of(c_dtype);
    p.group_m = 4;
    p.w4_signed = 1;
    p.group_shift = 30;
    const char* e = getenv("PHI_GEMM_KERNEL");
    const bool force_staged = e && strcmp(e, "tile128") == 0;
    GemmKernel gk = GK_PERSIST;
    if (e && strcmp(e, "persist256") == 0) gk = GK_PERSIST256;
    if (e && strcmp(e, "persist128") == 0) gk = GK_PERSIST128;
    const bool codes16 = aligned(B, 16) && ldb % 16 == 0;
    const size_t need = phi_hip_i4_workspace_bytes(M, N, K);
    if (!force_staged && need > 0 && workspace && ws_bytes >= need && aligned(workspace, 16) && codes16 &&
        persist_ok(C, c_dtype, N, K, lda, K, ldc)) {
        st = check_hip(phi_dev::launch_w4_lut_expand((hipStream_t)stream, p, (int8_t*)workspace), who);
        if (st != PHI_OK) return st;
        phi_dev::GemmParams g = p;
        g.B = (const int8_t*)workspace;
        g.ldb = K;
        g.w4_signed = 0;
        set_vec_flags(g, c_dtype, ldc);
        return check_hip(launch_persist_plan((hipStream_t)stream, g, gk, false, c_dtype, ldc), who);
    }
    set_vec_flags(p, c_dtype, ldc);
    if (!force_staged && codes16 && persist_ok(C, c_dtype, N, K, lda, ldb, ldc))
        return check_hip(launch_persist_plan((hipStream_t)stream, p, gk, true, c_dtype, ldc), who);
    return check_hip(phi_dev::launch_w4a8_gemm((hipStream_t)stream, p, gemm_cfg_for(M, N)), who);
}

size_t phi_hip_gemv_workspace_bytes(int n_items) {
    (void)n_items;
    return 0;
}

phi_status phi_hip_i8_gemv_batched(phi_stream_t stream, const int8_t* q8, const float* s8,
                                   int64_t M, int64_t K, int64_t N, const phi_gemv_item* items,
                                   int n_items, int bias_dtype, int c_dtype, void* workspace,
                                   size_t ws_bytes) {
    static const char* who = "i8_gemv_batched";
    (void)workspace;
    (void)ws_bytes;
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    if (n_items < 0 || M < 0 || N < 0 || K < 0) return fail(PHI_ERR_SHAPE, "%s: negative size", who);
    if (n_items == 0 || M == 0 || N == 0) return ok();
    if (M > 8) return fail(PHI_ERR_SHAPE, "%s: M=%lld exceeds 8 (use the GEMM)", who, (long long)M);
    if (K <= 0 || K % 16 != 0) return fail(PHI_ERR_SHAPE, "%s: K=%lld is not a positive multiple of 16", who, (long long)K);
    if (N > INT32_MAX || K > INT32_MAX) return fail(PHI_ERR_SHAPE, "%s: dimension exceeds 2^31", who);
    if (!q8 || !s8 || !items) return fail(PHI_ERR_ARG, "%s: null pointer", who);
    if (!aligned(q8, 16)) return fail(PHI_ERR_ALIGN, "%s: q8 must be 16-byte aligned", who);
    const int ck = c_kind_of(c_dtype);
    if (ck < 0) return fail(PHI_ERR_ARG, "%s: bad output dtype %d", who, c_dtype);
    for (int i = 0; i < n_items; i++) {
        const phi_gemv_item& it = items[i];
        if (!it.W || !it.C || (ck != phi_dev::C_I32 && !it.sW)) return fail(PHI_ERR_ARG, "%s: item %d has a null pointer", who, i);
        if (!aligned(it.W, 16)) return fail(PHI_ERR_ALIGN, "%s: item %d weight must be 16-byte aligned", who, i);
        if (it.ldc < N) return fail(PHI_ERR_SHAPE, "%s: item %d ldc < N", who, i);
        if (it.bias && bias_dtype != PHI_F32 && bias_dtype != PHI_BF16) return fail(PHI_ERR_ARG, "%s: bias dtype must be f32 or bf16", who);
    }
    for (int i0 = 0; i0 < n_items; i0 += phi_dev::GEMV_MAX_ITEMS) {
        const int cnt = n_items - i0 < phi_dev::GEMV_MAX_ITEMS ? n_items - i0 : phi_dev::GEMV_MAX_ITEMS;
        phi_dev::GemvBatch b{};
        b.q8 = q8;
        b.s8 = s8;
        b.M = (int)M;
        b.N = (int)N;
        b.K = (int)K;
        b.n_items = cnt;
        b.c_kind = ck;
        // All items share the call's bias dtype; an item without bias reads none.
        b.bias_kind = phi_dev::BIAS_NONE;
        bool any_bias = false, all_bias = true;
        for (int j = 0; j < cnt; j++) {
            const phi_gemv_item& it = items[i0 + j];
            b.W[j] = it.W;
            b.sW[j] = it.sW;
            b.bias[j] = it.bias;
            b.C[j] = it.C;
            b.ldc[j] = it.ldc;
            if (it.sw_scalar) b.sw_scalar_mask |= 1ull << j;
            any_bias |= it.bias != nullptr;
            all_bias &= it.bias != nullptr;
        }
        if (any_bias && !all_bias) return fail(PHI_ERR_UNSUPPORTED, "%s: mixed biased and bias-free items in one call", who);
        if (any_bias) b.bias_kind = bias_dtype == PHI_BF16 ? phi_dev::BIAS_BF16 : phi_dev::BIAS_F32;
        phi_status st = check_hip(phi_dev::launch_gemv((hipStream_t)stream, b), who);
        if (st != PHI_OK) return st;
    }
    return ok();
}

phi_status phi_hip_lora_down(phi_stream_t stream, const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K,
                             const float* A, int64_t R, float* h) {
    static const char* who = "lora_down";
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    if (M <= 0 || R <= 0 || K <= 0) return fail(PHI_ERR_SHAPE, "%s: empty problem", who);
    if (M > INT32_MAX || R > INT32_MAX || K > INT32_MAX) return fail(PHI_ERR_SHAPE, "%s: dimension exceeds 2^31", who);
    if (!x || !A || !h) return fail(PHI_ERR_ARG, "%s: null pointer", who);
    if (x_dtype != PHI_F32 && x_dtype != PHI_BF16) return fail(PHI_ERR_ARG, "%s: x dtype must be f32 or bf16", who);
    if (ldx < K) return fail(PHI_ERR_SHAPE, "%s: ldx < K", who);
    if (!aligned(x, x_dtype == PHI_BF16 ? 2 : 4) || !aligned(A, 4) || !aligned(h, 4))
        return fail(PHI_ERR_ALIGN, "%s: misaligned operand", who);
    return check_hip(phi_dev::launch_lora_down((hipStream_t)stream, x, x_dtype == PHI_BF16, ldx, A, h, (int)M, (int)K,
                                               (int)R),
                     who);
}

phi_status phi_hip_lora_rank_add(phi_stream_t stream, const float* h, const float* B, void* C, int c_dtype,
                                 int64_t ldc, int64_t M, int64_t N, int64_t R) {
    static const char* who = "lora_rank_add";
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    if (M <= 0 || N <= 0 || R <= 0) return fail(PHI_ERR_SHAPE, "lora_rank_add: empty problem");
    if (M > INT32_MAX || N > INT32_MAX || R > INT32_MAX) return fail(PHI_ERR_SHAPE, "%s: dimension exceeds 2^31", who);
    if (!h || !B || !C) return fail(PHI_ERR_ARG, "%s: null pointer", who);
    if (c_dtype != PHI_F32 && c_dtype != PHI_BF16) return fail(PHI_ERR_ARG, "%s: C dtype must be f32 or bf16", who);
    if (ldc < N) return fail(PHI_ERR_SHAPE, "%s: ldc < N", who);
    if (!aligned(C, c_dtype == PHI_BF16 ? 2 : 4) || !aligned(h, 4) || !aligned(B, 4))
        return fail(PHI_ERR_ALIGN, "%s: misaligned operand", who);
    return check_hip(phi_dev::launch_lora_rank_add((hipStream_t)stream, h, B, C, c_dtype == PHI_BF16, ldc, (int)M,
                                                   (int)N, (int)R),
                     who);
}

phi_status phi_hip_lora_tail(phi_stream_t stream, const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K,
                             const float* At, const float* Bt, int64_t R, int64_t N, void* out, int out_dtype,
                             int64_t ldo, float* h, size_t h_bytes) {
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "lora_tail: device was lost earlier");
    if (M <= 0 || R <= 0) return ok();  // an inactive tail or no rows: nothing to add
    const uint64_t need = (uint64_t)M * (uint64_t)R * 4;
    if (h_bytes < need)
        return fail(PHI_ERR_WORKSPACE,
                    "LoRA correction: the hidden-form scratch is %llu bytes; a [%lld, %lld] fp32 one needs %llu",
                    (unsigned long long)h_bytes, (long long)M, (long long)R, (unsigned long long)need);
    phi_status st = phi_hip_lora_down(stream, x, x_dtype, ldx, M, K, At, R, h);
    if (st != PHI_OK) return st;
    return phi_hip_lora_rank_add(stream, h, Bt, out, out_dtype, ldo, M, N, R);
}

phi_status phi_hip_dequant_rows(phi_stream_t stream, const void* src, int src_dtype, int64_t rows, int64_t cols,
                                int64_t lds, const float* row_scale, int scale_scalar, float* out, int64_t ldo) {
    static const char* who = "dequant_rows";
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    if (rows < 0 || cols < 0) return fail(PHI_ERR_SHAPE, "%s: negative size", who);
    if (rows == 0 || cols == 0) return ok();
    if (!src || !out) return fail(PHI_ERR_ARG, "%s: null pointer", who);
    int kind;
    size_t esz;
    switch (src_dtype) {
        case PHI_I8: kind = phi_dev::DQ_I8, esz = 1; break;
        case PHI_I4: kind = phi_dev::DQ_I4, esz = 1; break;
        case PHI_F16: kind = phi_dev::DQ_F16, esz = 2; break;
        case PHI_BF16: kind = phi_dev::DQ_BF16, esz = 2; break;
        case PHI_F32: kind = phi_dev::DQ_F32, esz = 4; break;
        case PHI_F8_E4M3: kind = phi_dev::DQ_F8_E4M3, esz = 1; break;
        case PHI_F8_E5M2: kind = phi_dev::DQ_F8_E5M2, esz = 1; break;
        default: return fail(PHI_ERR_ARG, "%s: src dtype must be I8, I4, F8_E4M3, F8_E5M2, F16, BF16 or F32", who);
    }
    if (src_dtype == PHI_I8 && !row_scale) return fail(PHI_ERR_ARG, "%s: int8 codes need their row scales", who);
    const int64_t src_cols = src_dtype == PHI_I4 ? (cols + 1) / 2 : cols;
    if (lds < src_cols || ldo < cols) return fail(PHI_ERR_SHAPE, "%s: leading dimension smaller than the row", who);
    if (!aligned(src, esz) || !aligned(out, 4) || (row_scale && !aligned(row_scale, 4)))
        return fail(PHI_ERR_ALIGN, "%s: misaligned operand", who);
    return check_hip(phi_dev::launch_dequant_rows((hipStream_t)stream, src, kind, rows, cols, lds, row_scale,
                                                  scale_scalar ? 1 : 0, out, ldo),
                     who);
}

phi_status phi_hip_dequant_fp4_rows(phi_stream_t stream, const uint8_t* codes, int64_t codes_ld, int64_t row0,
                                    int64_t rows, int64_t k, const float* block_scale, int64_t scale_rows,
                                    int64_t scale_cols, int64_t block, const float* global_scale, int global_scalar,
                                    float* out, int64_t ldo) {
    static const char* who = "dequant_fp4_rows";
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    if (rows < 0 || k < 0 || row0 < 0) return fail(PHI_ERR_SHAPE, "%s: negative size", who);
    if (rows == 0 || k == 0) return ok();
    if (!codes || !out) return fail(PHI_ERR_ARG, "%s: null pointer", who);
    if (codes_ld < (k + 1) / 2 || ldo < k) return fail(PHI_ERR_SHAPE, "%s: leading dimension smaller than the row", who);
    if (block <= 0) block = 16;
    // The table is read only when it has a geometry; then every (row, block)
    // this call reads must fall inside it.
    const bool have = block_scale && scale_rows > 0 && scale_cols / 4 > 0;
    if (have) {
        const int64_t nb_c = scale_cols / 4, last_row = row0 + rows - 1, last_blk = (k - 1) / block;
        const int64_t last = ((last_row >> 7) * nb_c + (last_blk >> 2)) * 512 + 511;
        if (nb_c < (last_blk >> 2) + 1 || last >= scale_rows * scale_cols)
            return fail(PHI_ERR_SHAPE, "%s: the %lld x %lld block-scale table does not cover rows up to %lld and %lld "
                        "blocks of %lld", who, (long long)scale_rows, (long long)scale_cols, (long long)last_row,
                        (long long)(last_blk + 1), (long long)block);
    }
    if (!aligned(out, 4) || (have && !aligned(block_scale, 4)) || (global_scale && !aligned(global_scale, 4)))
        return fail(PHI_ERR_ALIGN, "%s: misaligned operand", who);
    phi_dev::Fp4Rows p{codes, codes_ld, row0, rows, k, have ? block_scale : nullptr, scale_cols, block,
                       global_scale, global_scalar ? 1 : 0};
    return check_hip(phi_dev::launch_dequant_fp4_rows((hipStream_t)stream, p, out, ldo), who);
}

phi_status phi_hip_convrot_rows(phi_stream_t stream, const float* x, int64_t rows, int64_t K, int64_t ldx, float* y,
                                int64_t ldy) {
    static const char* who = "convrot";
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    if (rows < 0 || K < 0) return fail(PHI_ERR_SHAPE, "%s: negative size", who);
    if (rows == 0 || K == 0) return ok();
    if (K % 256 != 0) return fail(PHI_ERR_SHAPE, "convrot: cols=%lld not a multiple of 256", (long long)K);
    if (!x || !y) return fail(PHI_ERR_ARG, "%s: null pointer", who);
    if (ldx < K || ldy < K) return fail(PHI_ERR_SHAPE, "%s: leading dimension smaller than the row", who);
    if (rows * (K / 256) > INT32_MAX) return fail(PHI_ERR_SHAPE, "%s: more than 2^31 groups", who);
    if (!aligned(x, 4) || !aligned(y, 4)) return fail(PHI_ERR_ALIGN, "%s: misaligned operand", who);
    const char* xb = (const char*)x;
    const char* yb = (const char*)y;
    const int64_t xe = ((rows - 1) * ldx + K) * 4, ye = ((rows - 1) * ldy + K) * 4;
    if (x != y && yb < xb + xe && xb < yb + ye) return fail(PHI_ERR_ARG, "%s: y overlaps x without being x", who);
    if (x == y && ldx != ldy) return fail(PHI_ERR_ARG, "%s: in place needs equal pitches", who);
    return check_hip(phi_dev::launch_convrot_rows((hipStream_t)stream, x, ldx, y, ldy, rows, K), who);
}

phi_status phi_hip_lora_fold(phi_stream_t stream, float* w, int64_t ldw, int64_t rows, int64_t k, const float* A,
                             const float* B, int64_t rank, float scale) {
    static const char* who = "lora_fold";
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    if (rows < 0 || k < 0 || rank < 0) return fail(PHI_ERR_SHAPE, "%s: negative size", who);
    if (rows == 0 || k == 0 || rank == 0) return ok();
    if (!w || !A || !B) return fail(PHI_ERR_ARG, "%s: null pointer", who);
    if (ldw < k) return fail(PHI_ERR_SHAPE, "%s: ldw < k", who);
    if (!aligned(w, 4) || !aligned(A, 4) || !aligned(B, 4)) return fail(PHI_ERR_ALIGN, "%s: misaligned operand", who);
    return check_hip(phi_dev::launch_lora_fold((hipStream_t)stream, w, ldw, rows, k, A, B, rank, scale), who);
}

phi_status phi_hip_gelu_tanh(phi_stream_t stream, const void* x, int x_dtype, void* y, int y_dtype, int64_t n) {
    static const char* who = "gelu_tanh";
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    if (n < 0) return fail(PHI_ERR_SHAPE, "%s: negative size", who);
    if (n == 0) return ok();
    if (!x || !y) return fail(PHI_ERR_ARG, "%s: null pointer", who);
    if ((x_dtype != PHI_F32 && x_dtype != PHI_BF16) || (y_dtype != PHI_F32 && y_dtype != PHI_BF16))
        return fail(PHI_ERR_ARG, "%s: dtypes must be f32 or bf16", who);
    if (x == y && x_dtype != y_dtype) return fail(PHI_ERR_ARG, "%s: in place needs equal dtypes", who);
    return check_hip(phi_dev::launch_gelu((hipStream_t)stream, x, x_dtype == PHI_BF16, y, y_dtype == PHI_BF16, n), who);
}

phi_status phi_hip_silu_gate(phi_stream_t stream, const void* gx, int x_dtype, int64_t rows, int64_t cols,
                             int64_t ldx, void* out, int out_dtype, int64_t ldo) {
    static const char* who = "silu_gate";
    if (g_lost) return fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    if (rows < 0 || cols < 0) return fail(PHI_ERR_SHAPE, "%s: negative size", who);
    if (rows == 0 || cols == 0) return ok();
    if (!gx || !out) return fail(PHI_ERR_ARG, "%s: null pointer", who);
    if ((x_dtype != PHI_F32 && x_dtype != PHI_BF16) || (out_dtype != PHI_F32 && out_dtype != PHI_BF16))
        return fail(PHI_ERR_ARG, "%s: dtypes must be f32 or bf16", who);
    if (ldx < 2 * cols || ldo < cols) return fail(PHI_ERR_SHAPE, "%s: ldx must be >= 2*cols and ldo >= cols", who);
    const int64_t xe = x_dtype == PHI_BF16 ? 2 : 4, ye = out_dtype == PHI_BF16 ? 2 : 4;
    const char* xb = (const char*)gx;
    const char* ob = (const char*)out;
    if (ob < xb + ((rows - 1) * ldx + 2 * cols) * xe && xb < ob + ((rows - 1) * ldo + cols) * ye)
        return fail(PHI_ERR_ARG, "%s: out must not overlap gx", who);
    return check_hip(phi_dev::launch_silu_gate((hipStream_t)stream, gx, x_dtype == PHI_BF16, ldx, out,
                                               out_dtype == PHI_BF16, ldo, rows, cols),
                     who);
}

}  // extern "C"
