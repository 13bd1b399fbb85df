// C++ host layer over the C ABI, keeping the reference's quantized-linear call
// surface so its callers (the DiT blocks' quant_gemm, the node graph) can drop
// it in:
//
//   QuantLinear / linear_gemm          core/models/model_common.hpp:37-49, :172-173
//   Int8GemmArgs / dispatch_int8_gemm  core/runtime/compute.hpp:176-198
//   QuantConvrotArgs / dispatch_quant_convrot  core/runtime/compute.hpp:200-217
//   W4a8ExpandArgs / dispatch_w4a8_expand      core/kernels/w4a8_expand.hpp:65-120
//   GpuBuffer / GpuAlloc               core/runtime/cuda_device.hpp:28-33, sched.hpp:27-32
//   MediaError                         core/util/media_common.hpp:28-30
//
// Buffers are caller-owned (base + byte offset), dispatches enqueue on the
// context's one stream and nothing synchronises until submit(), as in the
// reference (core/runtime/compute.cpp:434-490).  A failing call throws
// MediaError with the library's message; a device fault marks the context lost.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

namespace phi::media {

using i64 = int64_t;
using u8 = uint8_t;
using u32 = uint32_t;
using u64 = uint64_t;

struct MediaError : std::runtime_error {
    explicit MediaError(const std::string& what) : std::runtime_error(what) {}
};

enum class DType { Unknown, F32, F16, BF16, I8, U8, I4, F8_E4M3, F8_E5M2 };

// A device allocation: a plain address and its size.
struct GpuBuffer {
    uintptr_t base = 0;
    u64 bytes = 0;
};

struct GpuAlloc {
    GpuBuffer* res = nullptr;
    u64 off = 0;
    u64 bytes = 0;
    explicit operator bool() const { return res != nullptr; }
};

// One device, one stream.  begin()/submit() bracket a batch of dispatches;
// submit() is the fence.
class ComputeContext {
public:
    explicit ComputeContext(int device = 0);
    ~ComputeContext();
    ComputeContext(const ComputeContext&) = delete;
    ComputeContext& operator=(const ComputeContext&) = delete;

    void begin() {}
    void submit();
    bool lost() const { return lost_; }
    hipStream_t stream() const { return stream_; }
    int device() const { return device_; }

    GpuBuffer* create_device_buffer(u64 bytes);
    void release_buffer(GpuBuffer* b);
    void upload(GpuBuffer* dst, const void* src, u64 bytes, u64 dst_off = 0);
    void download(GpuBuffer* src, void* dst, u64 bytes, u64 src_off = 0);

    // Converts a library status into MediaError (and device-lost state).
    void check(int status, const char* what);

private:
    int device_ = 0;
    hipStream_t stream_ = nullptr;
    bool lost_ = false;
};

struct Int8GemmArgs {
    GpuBuffer* a = nullptr;  // [M,K] int8
    u64 a_offset = 0;
    GpuBuffer* b = nullptr;  // [N,K] int8
    u64 b_offset = 0;
    GpuBuffer* sa = nullptr;  // [M] fp32
    u64 sa_offset = 0;
    GpuBuffer* sb = nullptr;  // [N] fp32 (or [1] with sb_scalar)
    u64 sb_offset = 0;
    GpuBuffer* c = nullptr;  // [M,N] of c_dtype
    u64 c_offset = 0;
    GpuBuffer* bias = nullptr;  // optional [N] of bias_dtype
    u64 bias_offset = 0;
    i64 M = 0, N = 0, K = 0;
    // Extensions over the reference surface (defaults keep its behaviour).
    DType c_dtype = DType::F32;
    DType bias_dtype = DType::F32;
    bool sb_scalar = false;
};

void dispatch_int8_gemm(ComputeContext& ctx, const Int8GemmArgs& args);

struct QuantConvrotArgs {
    GpuBuffer* x = nullptr;  // [rows,K] fp32 (or bf16 with x_dtype)
    u64 x_offset = 0;
    GpuBuffer* q = nullptr;  // [rows,K] int8 out
    u64 q_offset = 0;
    GpuBuffer* s = nullptr;  // [rows] fp32 out
    u64 s_offset = 0;
    i64 rows = 0, K = 0;
    float qmax = 127.0f;
    DType x_dtype = DType::F32;
    bool round_half_even = false;
};

void dispatch_quant_convrot(ComputeContext& ctx, const QuantConvrotArgs& args);

enum class RelDType : int { F32 = 0, F16 = 1, BF16 = 2, F8_E4M3 = 3, F8_E5M2 = 4, U8_E4M3 = 5 };
enum class CodeLayout : int { Nibble4 = 0, Packed6 = 1 };

struct W4a8ExpandArgs {
    GpuBuffer* pool = nullptr;
    u64 codes_off = 0;
    u64 srel_off = 0;
    u64 sch_off = 0;
    u64 cb_off = 0;
    GpuBuffer* q = nullptr;
    u64 q_off = 0;
    GpuBuffer* s = nullptr;
    u64 s_off = 0;
    i64 rows = 0;
    i64 k = 0;
    i64 group = 0;
    i64 codes_row_bytes = 0;
    i64 srel_row_bytes = 0;
    RelDType rel_dtype = RelDType::F8_E4M3;
    CodeLayout layout = CodeLayout::Nibble4;
    bool has_channel_scale = false;
    bool has_codebook = false;
};

void dispatch_w4a8_expand(ComputeContext& ctx, const W4a8ExpandArgs& args);

// Elementwise ops (core/kernels/gpu_ops.hpp:14-48).  The opcode values are the
// reference's; this library serves the one that sits between the MLP's two
// linears (GeluTanh, flat) and refuses the others with MediaError.
enum class ElemOp {
    Add = 0, Mul = 1, SiluGate = 2, Tanh = 3, Silu = 4, Scale = 5, AddMul = 6, Copy = 7,
    Modulate = 8, Exp = 9, AddScale = 10, GeluTanh = 11, ModAdd = 12,
};
enum class ElemMode { Flat = 0, Row = 1, Col = 2, Scalar = 3 };

struct ElemArgs {
    ElemOp op = ElemOp::Add;
    GpuAlloc a, b, c, y;
    i64 rows = 1, cols = 1;
    ElemMode bMode = ElemMode::Flat;
    ElemMode cMode = ElemMode::Flat;
    float alpha = 0.0f;
    float beta = 0.0f;
};

void dispatch_elem(ComputeContext& ctx, const ElemArgs& a);

// out[r][c] = silu(gx[r][c]) * gx[r][cols + c], fp32 (core/kernels/h3_kernels.hpp:116-129).
void dispatch_silu_gate_fused(ComputeContext& ctx, const GpuAlloc& gx, const GpuAlloc& out, i64 rows, i64 cols);

// int4 GEMM of the convrot_w4a4 family (core/kernels/h3_kernels.hpp:90-107):
// C[M,N] fp32 = (A[M,K] int8 . B[N,K/2] signed nibbles) * sa[m] * sb[n].
struct Int4GemmArgs {
    GpuAlloc a;   // [M,K] int8 (rotated + quantised activations, qmax 7)
    GpuAlloc b;   // [N,K/2] packed int4, column 2j in the low nibble of byte j
    GpuAlloc sa;  // [M] fp32
    GpuAlloc sb;  // [N] fp32
    GpuAlloc c;   // [M,N] fp32
    i64 m = 0, n = 0, k = 0;
};

void dispatch_int4_gemm(ComputeContext& ctx, const Int4GemmArgs& a);

// C[m, n] += H[m, rank] . B^T (core/kernels/gpu_ops.hpp:190-196), fp32.
struct LoraRankAddArgs {
    GpuAlloc h, b, c;
    i64 m = 0, n = 0, rank = 0;
};
void dispatch_lora_rank_add(ComputeContext& ctx, const LoraRankAddArgs& a);

// The runtime LoRA correction of one linear (core/models/model_common.hpp:245-251).
struct LoraTail {
    bool active = false;
    i64 rank = 0;
    i64 n = 0, k = 0;
    GpuAlloc at;  // [rank, k] fp32: the factors' A rows, stacked
    GpuAlloc bt;  // [n, rank] fp32: the factors' B columns, scaled, stacked
};

// One linear weight in the int8 form the GEMM reads.
struct QuantLinear {
    GpuAlloc w;      // [n,k] int8
    GpuAlloc scale;  // [n] fp32
    GpuAlloc d;      // dense float storage (not served by this library)
    DType dtype = DType::Unknown;
    i64 n = 0, k = 0;
    bool dense() const { return dtype == DType::F16 || dtype == DType::BF16 || dtype == DType::F32; }
};

struct GpuCtx {
    ComputeContext* ctx = nullptr;
    bool ok() const { return ctx != nullptr; }
};

// rotate+quantise x into q8/s8, then the int8 GEMM; out is [m, n] fp32.
void linear_gemm(GpuCtx& g, const QuantLinear& w, const GpuAlloc& x, i64 m, i64 k,
                 const GpuAlloc& out, const GpuAlloc& q8, const GpuAlloc& s8);

// ---- loading weights from checkpoints (safetensors.hpp reads the files) ----

class SafeTensors;

// A bump allocator over one device buffer, as the reference's GpuArena hands
// out weight storage (core/runtime/sched.hpp:27-60): 256-byte aligned pieces,
// MediaError when full.  Owns the buffer.
class GpuArena {
public:
    GpuArena(ComputeContext& ctx, u64 bytes);
    ~GpuArena();
    GpuArena(const GpuArena&) = delete;
    GpuArena& operator=(const GpuArena&) = delete;
    GpuAlloc alloc(u64 bytes);
    u64 used() const { return used_; }
    u64 capacity() const { return buf_ ? buf_->bytes : 0; }

private:
    ComputeContext& ctx_;
    GpuBuffer* buf_ = nullptr;
    u64 used_ = 0;
};

// One linear from a checkpoint into the int8 form the GEMM reads
// (core/models/model_common.cpp:921-1010, without the dense and LoRA-folding
// branches): int8_tensorwise is uploaded verbatim with its weight_scale; the
// grouped families (asym_w4a8_int8, w6a8_int8) are uploaded as stored and
// expanded on the device (w4a8_plan_of / w4a8_pack_rows, :589-748).  Anything
// else throws MediaError naming the family.
QuantLinear load_quant_linear(GpuCtx& g, const SafeTensors& st, const std::string& base, GpuArena& into);

// convrot_w4a4 (signed int4, two per byte, one fp32 scale per row): the packed
// bytes verbatim for the int4 GEMM (core/models/model_common.cpp:1285-1340);
// k is the packed width K/2, as the reference's I4Upload records it.
struct I4Upload {
    GpuAlloc w, s;
    i64 n = 0, k = 0;
};
I4Upload upload_quant_linear_w4a4(GpuCtx& g, const SafeTensors& st, const std::string& base, GpuArena& arena);

// out [m, t.n] fp32 += (x [m, t.k] fp32 . at^T) . bt^T, with h the caller's
// [m, rank] fp32 scratch (core/models/model_common.cpp:1667-1700).
void apply_lora_tail(GpuCtx& g, const LoraTail& t, const GpuAlloc& x, i64 m, const GpuAlloc& out, const GpuAlloc& h);

}  // namespace phi::media
