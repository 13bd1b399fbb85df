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
#include <vector>

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
    // w holds the K-tiled operand layout (phi_hip_pack_k_tiled) rather than
    // row-major [n, k]; only linear_gemm reads such a weight.
    bool k_tiled = false;
    bool dense() const { return dtype == DType::F16 || dtype == DType::BF16 || dtype == DType::F32; }
};

class GpuArena;
class SafeTensors;
class LoraSet;

// What a model holds while it runs (core/models/model_common.hpp:51-63): the
// compute context and three bump arenas.  The weight arena is reset per layer,
// the activation arena per step, the keep arena holds long-lived buffers.  The
// reference's upload ring is not needed: uploads here are stream-ordered
// copies from the checkpoint's mapping.
struct GpuCtx {
    ComputeContext* ctx = nullptr;
    GpuArena* wa = nullptr;    // weights, reset per layer
    GpuArena* aa = nullptr;    // activations, reset per step
    GpuArena* keep = nullptr;  // long-lived buffers
    // load_quant_linear / load_quant3_linear store an int8 weight K-tiled where
    // the shape allows it (K % 256 == 0, K <= 16384, n % 4 == 0), so
    // linear_gemm runs the K-tiled prologue and GEMM (the same output, bit for
    // bit, about 8 % faster at the DiT shapes).  Off by default: a caller that
    // hands QuantLinear::w to dispatch_int8_gemm itself needs it row-major.
    bool k_tiled_weights = false;
    bool ok() const { return ctx && wa && aa; }

    GpuAlloc walloc(u64 bytes);
    GpuAlloc aalloc(u64 bytes);
    GpuAlloc kalloc(u64 bytes);
    // Bytes already in the form the kernels read, into an allocation.
    void upload_into(const GpuAlloc& a, const void* src, u64 bytes);

    void begin();      // a batch of dispatches (no-op: one stream)
    void submit();     // fence
    void new_layer();  // weight arena reset
    void end_layer();  // submit
    void new_step();   // activation arena reset
};

// rotate+quantise x into q8/s8, then the int8 GEMM; out is [m, n] fp32.  A
// K-tiled weight (QuantLinear::k_tiled) runs phi_hip_q8_linear_kt: q8 then
// holds the codes K-tiled, and out's rows must be 16-byte aligned.
void linear_gemm(GpuCtx& g, const QuantLinear& w, const GpuAlloc& x, i64 m, i64 k,
                 const GpuAlloc& out, const GpuAlloc& q8, const GpuAlloc& s8);

// ---- loading weights from checkpoints (safetensors.hpp reads the files) ----

// The process-wide VRAM accountant (core/runtime/vram_budget.hpp:42-264): the
// ledger every arena charges before it grows.  charge() throws MediaError when
// the ledger would pass the limit, before anything is allocated, so a plan that
// does not fit fails as a plain error, never as a half-committed device.
//   limit: PHI_VRAM_BUDGET_MB (MiB, at least 256, at most the device less a
//   256 MiB reserve) when set, else the device's memory less a reserve of one
//   sixteenth, kept within [384 MiB, 2 GiB].  set_limit() overrides both (0 goes
//   back to them).
class VramBudget {
public:
    static VramBudget& instance();
    void charge(u64 bytes, const char* tag = nullptr);
    void release(u64 bytes);
    u64 local() const;  // bytes charged and not released
    u64 peak() const;
    u64 limit() const;
    bool would_exceed(u64 bytes) const;
    void set_limit(u64 bytes);

private:
    VramBudget() = default;
    u64 derived_limit() const;
    struct State;
    State& state() const;
};
inline VramBudget& vram_budget() { return VramBudget::instance(); }

// A bump allocator over device memory chunks, as the reference's GpuArena
// (core/runtime/sched.hpp:40-100, sched.cpp:65-109): alloc() hands out aligned
// pieces (256 bytes by default) and adds a chunk when the current one is full,
// charging the VRAM accountant for it first; alloc(0) returns an empty
// GpuAlloc; a grow from a fully rewound arena (nothing live) first returns the
// old chunks, so a mark/rewind caller holds one chunk of the largest size it
// needed rather than the sum.  reset() invalidates every allocation and keeps
// the chunks; mark() / rewind_to() give back what was allocated after a mark.
// Owns its chunks and releases their charge with them.
class GpuArena {
public:
    struct Mark {
        size_t chunk = 0;
        u64 off = 0;
        u64 used = 0;
    };
    GpuArena() = default;
    // init(&ctx, bytes) with the first chunk allocated now.
    GpuArena(ComputeContext& ctx, u64 bytes);
    ~GpuArena();
    GpuArena(const GpuArena&) = delete;
    GpuArena& operator=(const GpuArena&) = delete;

    void init(ComputeContext* ctx, u64 chunk_bytes = 192ull << 20, const char* tag = "arena");
    // Size of future chunks (0 is ignored).
    void set_chunk_bytes(u64 chunk_bytes) {
        if (chunk_bytes) chunk_bytes_ = chunk_bytes;
    }
    u64 chunk_bytes() const { return chunk_bytes_; }
    // Returns every chunk to the device; only legal when nothing in the arena is live.
    void release_chunks();
    void destroy() { release_chunks(); }
    GpuAlloc alloc(u64 bytes, u64 align = 256);
    void reset();
    u64 used() const { return used_; }
    u64 capacity() const { return capacity_; }
    int chunks() const { return (int)chunks_.size(); }
    Mark mark() const { return Mark{cur_, cur_off_, used_}; }
    void rewind_to(const Mark& m);

private:
    GpuBuffer* grow(u64 bytes);
    ComputeContext* ctx_ = nullptr;
    const char* tag_ = "arena";
    u64 chunk_bytes_ = 192ull << 20;
    std::vector<GpuBuffer*> chunks_;
    size_t cur_ = 0;
    u64 cur_off_ = 0;
    u64 used_ = 0;
    u64 capacity_ = 0;
};

// LoRA factor files (core/models/lora.hpp:102-186): per adapted module a
// rank-r delta  W_eff = W + strength * (alpha / r) * B @ A  (A [r, k], B [n, r]).
// Keys in the diffusers / peft (lora_A / lora_B), kohya (lora_down / lora_up)
// and ComfyUI (display-name prefixes) conventions all normalise to the base
// weight's name without ".weight".  Files are applied in the order added.
inline constexpr int kMaxLoras = 2;
inline constexpr i64 kLoraRankBound = 256;
inline constexpr float kLoraStrengthDefault = 1.0f;

class LoraSet {
public:
    // Loads a safetensors LoRA and appends it; MediaError when it holds no
    // factor pair this loader can map.  strength scales the file's deltas.
    void add(const std::string& path, float strength = kLoraStrengthDefault);
    void clear() {
        adapters_.clear();
        paths_.clear();
    }
    bool empty() const { return paths_.empty(); }
    size_t size() const { return paths_.size(); }
    const std::vector<std::string>& paths() const { return paths_; }

    // One factor as stored: W_eff = W + scale * b @ a, a [rank, k], b [n, rank],
    // scale = strength * alpha / rank.
    struct Delta {
        i64 n = 0, k = 0, rank = 0;
        float scale = 1.0f;
        const float* a = nullptr;
        const float* b = nullptr;
    };
    // Every factor of `target` whose (n, k) is exactly the weight's, in file order.
    int deltas_for(const std::string& target, i64 n, i64 k, std::vector<Delta>* out) const;
    // Every factor of `target` with width k covering rows [row0, row0 + rows):
    // the factors apply_rows folds, in its order.
    int deltas_for_rows(const std::string& target, i64 row0, i64 rows, i64 k, std::vector<Delta>* out) const;
    // True if any factor could match `target`.
    bool touches(const std::string& target) const;
    // The folds on a host fp32 weight [n, k] (or its rows [row0, row0 + rows)):
    // w[o][i] += (scale * B[o][r]) * A[r][i], r ascending, B entries of 0 skipped.
    int apply(const std::string& target, float* w, i64 n, i64 k) const;
    int apply_rows(const std::string& target, float* w, i64 row0, i64 rows, i64 k) const;

private:
    // One adapted module of one file: the delta scale * up . down, with down
    // [rank, cols] and up [rows, rank] stored back to back in f32.
    struct Adapter {
        std::string module;
        i64 rows = 0, cols = 0, rank = 0;
        float scale = 1.0f;
        std::vector<float> f32;
        const float* down() const { return f32.data(); }
        const float* up() const { return f32.data() + (size_t)(rank * cols); }
        Delta delta() const { return Delta{rows, cols, rank, scale, down(), up()}; }
    };
    // The adapters whose module names `target`, in chain order.
    std::vector<const Adapter*> matching(const std::string& target) const;

    std::vector<Adapter> adapters_;  // file by file; within a file, modules in order of their first key
    std::vector<std::string> paths_;
};

// A LoRA tensor key -> the module it adapts (no ".weight"), or "" when the key
// is not a factor or alpha key.
std::string lora_normalize_target(const std::string& key, bool* is_a, bool* is_b);

// One linear from a checkpoint into the int8 form the GEMM reads
// (core/models/model_common.cpp:921-1090).  `into` null allocates from the
// context's weight arena.
//   int8_tensorwise: the codes verbatim with their weight_scale;
//   asym_w4a8_int8 / w6a8_int8: stored parts staged on the device and
//     expanded there (w4a8_plan_of / w4a8_pack_rows, :589-748);
//   another integer form (an int8 weight without a convrot sidecar, a bare I4):
//     decoded and requantised on the device with the reference's requant spec;
//   a LoRA in `lora` that touches the module is folded first: the weight is
//     decoded, rotated back to its original basis, the deltas added, then
//     rotated and quantised (int8_tensorwise sources).
// Dense float weights (f16 / bf16 / f32 / fp8 / nvfp4) belong to the dense GEMM
// and throw MediaError naming the precision.
QuantLinear load_quant_linear(GpuCtx& g, const SafeTensors& st, const std::string& base,
                              GpuArena* into = nullptr, const LoraSet* lora = nullptr);

// The fused q|k|v form (core/models/model_common.cpp:1414-1578): one [3N, K]
// int8 matrix whose rows are q then k then v, and the concatenated row scales.
// Three plain int8 weights are concatenated verbatim; otherwise each part is
// requantised into its rows (the grouped families through the device expand).
QuantLinear load_quant3_linear(GpuCtx& g, const SafeTensors& st, const std::string& base_q,
                               const std::string& base_k, const std::string& base_v,
                               GpuArena* into = nullptr, const LoraSet* lora = nullptr);

// The streaming int8 upload (core/models/model_common.cpp:1095-1283): a grouped
// family expanded on the device; an int8_tensorwise weight whose file declares
// convrot uploaded verbatim; anything else (f16 / bf16 / f32, int8 without a
// convrot sidecar) decoded and requantised on the device, rotated unless the
// file says it is stored rotated.  A LoRA that touches the module is folded.
struct I8Upload {
    GpuAlloc w, s;
    i64 n = 0, k = 0;
};
I8Upload upload_quant_linear_i8(GpuCtx& g, const SafeTensors& st, const std::string& base, GpuArena& arena,
                                const LoraSet* lora);

// convrot_w4a4 (signed int4, two per byte, one fp32 scale per row): the packed
// bytes verbatim for the int4 GEMM (core/models/model_common.cpp:1285-1340);
// k is the packed width K/2, as the reference's I4Upload records it.  A LoRA is
// not folded into int4 weights: it is applied by the runtime tail.
struct I4Upload {
    GpuAlloc w, s;
    i64 n = 0, k = 0;
};
I4Upload upload_quant_linear_w4a4(GpuCtx& g, const SafeTensors& st, const std::string& base, GpuArena& arena,
                                  const LoraSet* lora = nullptr);

// One module of a (possibly fused) projection: `base` corrects the output rows
// [row0, row0 + n) of the layer's weight (core/models/model_common.hpp:255-260).
struct LoraModule {
    std::string base;
    i64 row0 = 0;
    i64 n = 0;
    const LoraSet* lora = nullptr;
};

// The runtime correction's operands (core/models/model_common.cpp:1587-1652):
// every matching factor of every module stacked along the rank axis (A) and
// placed at its module's output rows with its scale folded in (B).  Inactive
// when no factor matches; MediaError past kLoraRankBound.
LoraTail load_lora_tail(GpuCtx& g, GpuArena& arena, const std::vector<LoraModule>& mods, i64 n, i64 k);
LoraTail load_lora_tail(GpuCtx& g, GpuArena& arena, const std::string& base, const LoraSet* lora, i64 n, i64 k);

// ---- the GEMM tuning table (core/kernels/autotune.hpp:30-88) ----
//
// One plan per (M, N, K, operand layout) for the persistent int8 GEMM:
// big_rows (rows run as 256 x 256 tiles), group_m (tile rows per group of the
// XCD-aware tile order), split (the two tile sizes as two launches) and tile
// (the square plan or 272 x 192 tiles, K % 512 == 0).  Every
// plan gives the same bits, so a sweep is free to pick the fastest; it checks
// that anyway.  The store persists as JSON and apply() hands its plans to the
// library, whose every launch of such a shape then runs the stored plan.
struct GemmTuneEntry {
    i64 M = 0, N = 0, K = 0;
    bool k_tiled = false;
    i64 big_rows = -1;  // -1: the library's cost model
    int group_m = 0;    // 0: 4
    bool split = false;
    int tile = 0;       // PHI_PLAN_TILE_*: 0 the cost model, 1 square, 2 272 x 192
    double measured_us = 0.0;
    double tops = 0.0;
};

class GemmTuneStore {
public:
    // The default file beside a data directory, as the reference keeps its table
    // (core/kernels/autotune.cpp:158-160).
    static std::string default_path(const std::string& base_dir);
    bool load(const std::string& path);        // false: unreadable or malformed (the store is unchanged)
    bool save(const std::string& path) const;  // written whole, then renamed into place
    void put(const GemmTuneEntry& e);          // replaces the entry of the same shape and layout
    const GemmTuneEntry* get(i64 M, i64 N, i64 K, bool k_tiled) const;
    // Every entry into the library's plan table (phi_hip_gemm_plan_set).
    void apply() const;
    size_t size() const { return items_.size(); }
    const std::vector<GemmTuneEntry>& items() const { return items_; }

private:
    std::vector<GemmTuneEntry> items_;
};

struct GemmTuneResult {
    bool ok = false;
    std::string error;
    GemmTuneEntry best;
    std::vector<GemmTuneEntry> tried;  // measured_us / tops filled
    int exact_matches = 0;             // candidates bit-identical to the default plan
    bool default_exact = false;        // the default plan's sampled rows equal a host integer GEMM
};

// Sweeps the candidate plans of an M x N x K int8 GEMM (bf16 output with a
// bias, row-major or K-tiled operands) on seeded random operands, `iters`
// timed launches each after one untimed, on the context's stream.  The
// default plan's int32 accumulators are checked on sampled rows against a
// host integer GEMM and every candidate's output against the default plan's,
// bit for bit.  Buffers are device allocations charged to the VRAM
// accountant, released on return.  The table is left as it was.
GemmTuneResult autotune_int8_gemm(ComputeContext& ctx, i64 M, i64 N, i64 K, int iters = 3, bool k_tiled = false);

// out [m, t.n] fp32 += (x [m, t.k] fp32 . at^T) . bt^T, with h the caller's
// [m, rank] fp32 scratch (core/models/model_common.cpp:1667-1700).
void apply_lora_tail(GpuCtx& g, const LoraTail& t, const GpuAlloc& x, i64 m, const GpuAlloc& out, const GpuAlloc& h);

}  // namespace phi::media
