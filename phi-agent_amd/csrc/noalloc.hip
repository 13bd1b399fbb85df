// The W8A8 linear for callers that cannot allocate (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc): the
// activation scratch of phi_hip_q8_linear / phi_hip_q8_linear_kq (q8, M x K
// int8 codes, and s8 [M] fp32) lives in a file-scope device array instead of
// caller buffers.
//
// `scratch` is a static device variable: every GPU the library runs on holds
// its own copy (kScratchBytes) from the code object's load until the process
// ends.  In host code its name is only a stand-in for the symbol, so the
// device address is looked up once per device with hipGetSymbolAddress, with
// that device current, and only that address is passed to the kernels.
//
// Every call on one GPU shares that GPU's array and leaves its contents
// behind.  Nothing in it has to start at zero: the prologue writes every q8
// byte and s8 entry the GEMM then reads.  Calls that overlap on one GPU (two
// streams, two threads) race on the array; a caller that needs concurrency
// uses phi_hip_q8_linear with its own scratch.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <cstdio>
#include <mutex>

#include "../../include/phi_qlinear.h"

namespace phi_capi {
phi_status fail(phi_status st, const char* fmt, ...);
bool device_lost();
}  // namespace phi_capi

namespace phi_noalloc {

constexpr size_t kScratchBytes = PHI_NOALLOC_SCRATCH_BYTES;

// The activation scratch, one copy per device.
__device__ __align__(256) uint8_t scratch[kScratchBytes];

}  // namespace phi_noalloc

namespace {

using phi_noalloc::kScratchBytes;
using phi_noalloc::scratch;
constexpr int kMaxDevices = 64;

std::mutex g_mu;
std::atomic<uintptr_t> g_ptr[kMaxDevices];

// The current device's copy of `scratch`, looked up on its first use on that
// device.  0 on failure, with the HIP status in *err.
uintptr_t scratch_on_current_device(int* dev_out, hipError_t* err) {
    int dev = -1;
    *err = hipGetDevice(&dev);
    if (*err != hipSuccess) return 0;
    *dev_out = dev;
    if (dev < 0 || dev >= kMaxDevices) {
        *err = hipErrorInvalidDevice;
        return 0;
    }
    uintptr_t p = g_ptr[dev].load(std::memory_order_acquire);
    if (p) return p;
    std::lock_guard<std::mutex> lock(g_mu);
    p = g_ptr[dev].load(std::memory_order_relaxed);
    if (p) return p;
    void* addr = nullptr;
    *err = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (*err != hipSuccess || !addr) {
        if (*err == hipSuccess) *err = hipErrorInvalidSymbol;
        return 0;
    }
    p = (uintptr_t)addr;
    g_ptr[dev].store(p, std::memory_order_release);
    return p;
}

}  // namespace

extern "C" {

size_t phi_hip_noalloc_scratch_bytes(void) { return kScratchBytes; }

phi_status phi_hip_q8_linear_noalloc(phi_stream_t stream, const void* x, int x_dtype, int64_t ldx, int64_t M,
                                     int64_t K, const int8_t* W, int64_t ldw, const float* sW, int sw_scalar,
                                     const void* bias, int bias_dtype, int64_t N, void* C, int c_dtype, int64_t ldc,
                                     int round_mode) {
    static const char* who = "q8_linear_noalloc";
    if (phi_capi::device_lost()) return phi_capi::fail(PHI_ERR_DEVICE_LOST, "%s: device was lost earlier", who);
    if (M <= 0 || N <= 0 || K <= 0)
        return phi_capi::fail(PHI_ERR_SHAPE, "%s: empty problem (M=%lld N=%lld K=%lld)", who, (long long)M,
                              (long long)N, (long long)K);
    // q8 at offset 0 with row pitch K, s8 at the next 256-byte boundary.
    uint64_t q_bytes = 0, need = 0;
    if (__builtin_mul_overflow((uint64_t)M, (uint64_t)K, &q_bytes) ||
        __builtin_add_overflow((q_bytes + 255) & ~(uint64_t)255, (uint64_t)M * 4, &need) || need > kScratchBytes)
        return phi_capi::fail(PHI_ERR_WORKSPACE,
                              "%s: M=%lld x K=%lld needs more activation scratch than the %llu-byte static scratch "
                              "(use phi_hip_q8_linear with caller scratch)",
                              who, (long long)M, (long long)K, (unsigned long long)kScratchBytes);
    const uint64_t s_off = (q_bytes + 255) & ~(uint64_t)255;
    int dev = -1;
    hipError_t e = hipSuccess;
    const uintptr_t base = scratch_on_current_device(&dev, &e);
    if (!base)
        return phi_capi::fail(PHI_ERR_HIP, "%s: the static scratch of device %d cannot be addressed (%s)", who, dev,
                              hipGetErrorString(e));
    // phi_hip_q8_linear_kq: the same C as phi_hip_q8_linear, with the codes
    // written K-tiled where the 272 x 192 plan takes the shape.
    return phi_hip_q8_linear_kq(stream, x, x_dtype, ldx, M, K, W, ldw, sW, sw_scalar, bias, bias_dtype, N, C,
                                c_dtype, ldc, (int8_t*)base, (float*)(base + s_off), round_mode, nullptr, 0);
}

}  // extern "C"
