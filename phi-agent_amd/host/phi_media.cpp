// C++ host layer: the reference's dispatch surface over the C ABI.
#include "phi_media.hpp"

#include "phi_qlinear.h"
#include "safetensors.hpp"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <map>
#include <mutex>
#include <optional>
#include <random>
#include <string_view>
#include <unordered_map>
#include <vector>

namespace phi::media {

namespace {

void* at(GpuBuffer* b, u64 off) { return b ? (void*)(b->base + off) : nullptr; }
const void* cat(GpuBuffer* b, u64 off) { return b ? (const void*)(b->base + off) : nullptr; }

int phi_dtype_of(DType t) {
    switch (t) {
        case DType::F32: return PHI_F32;
        case DType::BF16: return PHI_BF16;
        case DType::F16: return PHI_F16;
        case DType::F8_E4M3: return PHI_F8_E4M3;
        case DType::F8_E5M2: return PHI_F8_E5M2;
        default: return -1;
    }
}

int phi_rel_dtype(RelDType t) {
    switch (t) {
        case RelDType::F32: return PHI_F32;
        case RelDType::F16: return PHI_F16;
        case RelDType::BF16: return PHI_BF16;
        case RelDType::F8_E4M3: return PHI_F8_E4M3;
        case RelDType::F8_E5M2: return PHI_F8_E5M2;
        case RelDType::U8_E4M3: return PHI_U8_E4M3;
    }
    return -1;
}

}  // namespace

ComputeContext::ComputeContext(int device) : device_(device) {
    if (hipSetDevice(device) != hipSuccess) throw MediaError("hip: cannot select device " + std::to_string(device));
    if (hipStreamCreate(&stream_) != hipSuccess) throw MediaError("hip: stream creation failed");
}

ComputeContext::~ComputeContext() {
    if (stream_) (void)hipStreamDestroy(stream_);
}

void ComputeContext::check(int status, const char* what) {
    if (status == PHI_OK) return;
    if (status == PHI_ERR_DEVICE_LOST) lost_ = true;
    throw MediaError(std::string(what) + ": " + phi_hip_last_error());
}

void ComputeContext::submit() {
    const hipError_t e = hipStreamSynchronize(stream_);
    if (e != hipSuccess) {
        if (e == hipErrorIllegalAddress || e == hipErrorLaunchFailure) lost_ = true;
        throw MediaError(std::string("hip: stream sync failed: ") + hipGetErrorString(e));
    }
}

GpuBuffer* ComputeContext::create_device_buffer(u64 bytes) {
    void* p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) throw MediaError("hip: out of device memory");
    return new GpuBuffer{(uintptr_t)p, bytes};
}

void ComputeContext::release_buffer(GpuBuffer* b) {
    if (!b) return;
    (void)hipFree((void*)b->base);
    delete b;
}

void ComputeContext::upload(GpuBuffer* dst, const void* src, u64 bytes, u64 dst_off) {
    if (hipMemcpyAsync(at(dst, dst_off), src, bytes, hipMemcpyHostToDevice, stream_) != hipSuccess ||
        hipStreamSynchronize(stream_) != hipSuccess)
        throw MediaError("hip: upload failed");
}

void ComputeContext::download(GpuBuffer* src, void* dst, u64 bytes, u64 src_off) {
    if (hipMemcpyAsync(dst, cat(src, src_off), bytes, hipMemcpyDeviceToHost, stream_) != hipSuccess ||
        hipStreamSynchronize(stream_) != hipSuccess)
        throw MediaError("hip: download failed");
}

// core/runtime/compute.cpp:551-661
void dispatch_int8_gemm(ComputeContext& ctx, const Int8GemmArgs& a) {
    if (a.M <= 0 || a.N <= 0 || a.K <= 0) throw MediaError("int8_gemm: empty problem");
    const int cdt = a.c_dtype == DType::F32 ? PHI_F32 : (a.c_dtype == DType::BF16 ? PHI_BF16 : -1);
    if (cdt < 0) throw MediaError("int8_gemm: output must be F32 or BF16");
    ctx.check(phi_hip_i8_gemm(ctx.stream(), (const int8_t*)cat(a.a, a.a_offset), a.K,
                              (const int8_t*)cat(a.b, a.b_offset), a.K,
                              (const float*)cat(a.sa, a.sa_offset), (const float*)cat(a.sb, a.sb_offset),
                              a.sb_scalar ? 1 : 0, a.bias ? cat(a.bias, a.bias_offset) : nullptr,
                              phi_dtype_of(a.bias_dtype), at(a.c, a.c_offset), cdt, a.N, a.M, a.N, a.K,
                              nullptr, 0),
              "int8_gemm");
}

// core/runtime/compute.cpp:663-684
void dispatch_quant_convrot(ComputeContext& ctx, const QuantConvrotArgs& a) {
    if (a.rows <= 0) return;
    ctx.check(phi_hip_quant_rotate(ctx.stream(), cat(a.x, a.x_offset), phi_dtype_of(a.x_dtype), a.rows, a.K,
                                   a.K, (int8_t*)at(a.q, a.q_offset), a.K, (float*)at(a.s, a.s_offset), a.qmax,
                                   a.round_half_even ? PHI_ROUND_HALF_EVEN : PHI_ROUND_HALF_AWAY, 1),
              "quant_convrot");
}

// core/kernels/gpu_ops.cpp:14-47: the same opcode and size gates, GeluTanh served.
void dispatch_elem(ComputeContext& ctx, const ElemArgs& a) {
    if ((unsigned)a.op > 12u) throw MediaError("elem: unknown opcode " + std::to_string((int)a.op));
    const i64 n = a.rows * a.cols;
    if (n <= 0) throw MediaError("elem: empty");
    if (a.y.bytes && (u64)n * 4 > a.y.bytes) throw MediaError("elem: output buffer is too small");
    if (a.a.bytes && (u64)n * 4 > a.a.bytes)
        throw MediaError("elem: operand A is too small for " + std::to_string(n) + " elements");
    if (a.op != ElemOp::GeluTanh)
        throw MediaError("elem: opcode " + std::to_string((int)a.op) +
                         " is not served by the quantized-linear library (GeluTanh only)");
    ctx.check(phi_hip_gelu_tanh(ctx.stream(), cat(a.a.res, a.a.off), PHI_F32, at(a.y.res, a.y.off), PHI_F32, n),
              "elem");
}

// core/kernels/h3_kernels.cpp:466-482
void dispatch_silu_gate_fused(ComputeContext& ctx, const GpuAlloc& gx, const GpuAlloc& out, i64 rows, i64 cols) {
    if (rows <= 0 || cols <= 0) throw MediaError("silu_gate_fused: empty");
    if (gx.bytes && (u64)(rows * 2 * cols) * 4 > gx.bytes) throw MediaError("silu_gate_fused: gx is too small");
    if (out.bytes && (u64)(rows * cols) * 4 > out.bytes) throw MediaError("silu_gate_fused: out is too small");
    ctx.check(phi_hip_silu_gate(ctx.stream(), cat(gx.res, gx.off), PHI_F32, rows, cols, 2 * cols, at(out.res, out.off),
                                PHI_F32, cols),
              "silu_gate_fused");
}

// core/kernels/h3_kernels.cpp:637-662: the same contract (empty problem, K % 512).
void dispatch_int4_gemm(ComputeContext& ctx, const Int4GemmArgs& a) {
    ctx.check(phi_hip_i4_gemm(ctx.stream(), (const int8_t*)cat(a.a.res, a.a.off), a.k,
                              (const uint8_t*)cat(a.b.res, a.b.off), a.k / 2, (const float*)cat(a.sa.res, a.sa.off),
                              (const float*)cat(a.sb.res, a.sb.off), at(a.c.res, a.c.off), PHI_F32, a.n, a.m, a.n,
                              a.k, nullptr, 0),
              "int4_gemm");
}

// core/kernels/gpu_ops.cpp:505-522
void dispatch_lora_rank_add(ComputeContext& ctx, const LoraRankAddArgs& a) {
    if (a.m <= 0 || a.n <= 0 || a.rank <= 0) throw MediaError("lora_rank_add: empty problem");
    ctx.check(phi_hip_lora_rank_add(ctx.stream(), (const float*)cat(a.h.res, a.h.off), (const float*)cat(a.b.res, a.b.off),
                                    at(a.c.res, a.c.off), PHI_F32, a.n, a.m, a.n, a.rank),
              "lora_rank_add");
}

// core/models/model_common.cpp:1667-1700: the same scratch check, then both products.
void apply_lora_tail(GpuCtx& g, const LoraTail& t, const GpuAlloc& x, i64 m, const GpuAlloc& out, const GpuAlloc& h) {
    if (!t.active || m <= 0) return;
    const u64 need = (u64)m * (u64)t.rank * 4;
    if (h.bytes < need)
        throw MediaError("LoRA correction: the hidden-form scratch is " + std::to_string(h.bytes) + " bytes; a [" +
                         std::to_string(m) + ", " + std::to_string(t.rank) + "] fp32 one needs " + std::to_string(need));
    g.ctx->check(phi_hip_lora_tail(g.ctx->stream(), cat(x.res, x.off), PHI_F32, t.k, m, t.k,
                                   (const float*)cat(t.at.res, t.at.off), (const float*)cat(t.bt.res, t.bt.off), t.rank,
                                   t.n, at(out.res, out.off), PHI_F32, t.n, (float*)at(h.res, h.off), h.bytes),
                 "lora_tail");
}

// ---------------------------------------------------------------- GpuCtx

GpuAlloc GpuCtx::walloc(u64 bytes) {
    if (!wa) throw MediaError("GpuCtx: no weight arena");
    return wa->alloc(bytes);
}

GpuAlloc GpuCtx::aalloc(u64 bytes) {
    if (!aa) throw MediaError("GpuCtx: no activation arena");
    return aa->alloc(bytes);
}

GpuAlloc GpuCtx::kalloc(u64 bytes) {
    GpuArena* a = keep ? keep : aa;
    if (!a) throw MediaError("GpuCtx: no keep or activation arena");
    return a->alloc(bytes);
}

void GpuCtx::upload_into(const GpuAlloc& a, const void* src, u64 bytes) {
    if (!ctx) throw MediaError("GpuCtx: no compute context");
    if (bytes > a.bytes) throw MediaError("upload: " + std::to_string(bytes) + " bytes into a " + std::to_string(a.bytes) + "-byte allocation");
    ctx->upload(a.res, src, bytes, a.off);
}

void GpuCtx::begin() {
    if (ctx) ctx->begin();
}

void GpuCtx::submit() {
    if (ctx) ctx->submit();
}

void GpuCtx::new_layer() {
    begin();
    if (wa) wa->reset();
}

void GpuCtx::end_layer() { submit(); }

void GpuCtx::new_step() {
    if (aa) aa->reset();
}

// ---------------------------------------------------------------- VRAM accountant

struct VramBudget::State {
    mutable std::mutex m;
    u64 local = 0, peak = 0;
    u64 forced = 0;  // set_limit()
    mutable u64 derived = 0;
};

VramBudget& VramBudget::instance() {
    static VramBudget b;
    return b;
}

VramBudget::State& VramBudget::state() const {
    static State s;
    return s;
}

static std::string mib_text(u64 bytes) { return std::to_string((bytes + (1ull << 19)) >> 20) + " MiB"; }

u64 VramBudget::derived_limit() const {
    constexpr u64 kMiB = 1ull << 20, kMinReserve = 384 * kMiB, kMaxReserve = 2048 * kMiB, kEnvReserve = 256 * kMiB;
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) total_b = 0;
    const u64 total = total_b;
    if (const char* e = std::getenv("PHI_VRAM_BUDGET_MB")) {
        const long long mb = std::atoll(e);
        if (mb >= 256) {
            u64 want = (u64)mb * kMiB;
            if (total) want = std::min(want, total > kEnvReserve ? total - kEnvReserve : 0);
            return want;
        }
    }
    if (!total) return 0;  // no device answer: no ceiling of our own
    const u64 reserve = std::clamp(total / 16, kMinReserve, kMaxReserve);
    return total > reserve ? total - reserve : 0;
}

u64 VramBudget::limit() const {
    State& s = state();
    std::lock_guard<std::mutex> lk(s.m);
    if (s.forced) return s.forced;
    if (!s.derived) s.derived = derived_limit();
    return s.derived;
}

void VramBudget::set_limit(u64 bytes) {
    State& s = state();
    std::lock_guard<std::mutex> lk(s.m);
    s.forced = bytes;
    s.derived = 0;
}

bool VramBudget::would_exceed(u64 bytes) const {
    const u64 lim = limit();
    State& s = state();
    std::lock_guard<std::mutex> lk(s.m);
    return lim != 0 && (bytes > lim || s.local > lim - bytes);
}

void VramBudget::charge(u64 bytes, const char* tag) {
    if (bytes == 0) return;
    const u64 lim = limit();
    State& s = state();
    std::lock_guard<std::mutex> lk(s.m);
    if (lim != 0 && (bytes > lim || s.local > lim - bytes))
        throw MediaError("VRAM budget exceeded: requesting " + mib_text(bytes) + " for " + (tag ? tag : "allocation") +
                         " would take resident " + mib_text(s.local + bytes) + " past the limit " + mib_text(lim));
    s.local += bytes;
    s.peak = std::max(s.peak, s.local);
}

void VramBudget::release(u64 bytes) {
    State& s = state();
    std::lock_guard<std::mutex> lk(s.m);
    s.local = s.local > bytes ? s.local - bytes : 0;
}

u64 VramBudget::local() const {
    State& s = state();
    std::lock_guard<std::mutex> lk(s.m);
    return s.local;
}

u64 VramBudget::peak() const {
    State& s = state();
    std::lock_guard<std::mutex> lk(s.m);
    return s.peak;
}

// ---------------------------------------------------------------- GpuArena

GpuArena::GpuArena(ComputeContext& ctx, u64 bytes) {
    init(&ctx, bytes);
    chunks_.push_back(grow(bytes));
}

GpuArena::~GpuArena() { release_chunks(); }

void GpuArena::init(ComputeContext* ctx, u64 chunk_bytes, const char* tag) {
    ctx_ = ctx;
    if (chunk_bytes) chunk_bytes_ = chunk_bytes;
    if (tag) tag_ = tag;
}

// A new chunk, charged to the accountant before the device allocation; a
// refused charge allocates nothing.
GpuBuffer* GpuArena::grow(u64 bytes) {
    vram_budget().charge(bytes, tag_);
    GpuBuffer* b = nullptr;
    try {
        b = ctx_->create_device_buffer(bytes);
    } catch (...) {
        vram_budget().release(bytes);
        throw;
    }
    capacity_ += bytes;
    return b;
}

void GpuArena::release_chunks() {
    if (ctx_) {
        // Work still queued may read the chunks: let it finish first.
        (void)hipStreamSynchronize(ctx_->stream());
        for (GpuBuffer* b : chunks_) ctx_->release_buffer(b);
    }
    vram_budget().release(capacity_);
    chunks_.clear();
    cur_ = 0;
    cur_off_ = 0;
    used_ = 0;
    capacity_ = 0;
}

GpuAlloc GpuArena::alloc(u64 bytes, u64 align) {
    if (bytes == 0) return GpuAlloc{};
    if (!ctx_) throw MediaError("arena: not initialised");
    if (align == 0 || (align & (align - 1)) != 0) throw MediaError("arena: alignment must be a power of two");
    // The current chunk, then any later chunk (kept from before a reset) that
    // fits, then a new chunk.
    for (size_t c = cur_; c < chunks_.size(); c++) {
        const u64 start = c == cur_ ? cur_off_ : 0;
        const u64 off = (start + align - 1) & ~(align - 1);
        if (off + bytes <= chunks_[c]->bytes) {
            used_ += (off - (c == cur_ ? cur_off_ : 0)) + bytes;
            cur_ = c;
            cur_off_ = off + bytes;
            return GpuAlloc{chunks_[c], off, bytes};
        }
    }
    // Nothing live at a fully rewound arena: its chunks, each sized for some
    // earlier need, give way to one that fits this one.
    if (cur_ == 0 && cur_off_ == 0 && !chunks_.empty()) release_chunks();
    chunks_.push_back(grow(std::max(bytes, chunk_bytes_)));
    cur_ = chunks_.size() - 1;
    cur_off_ = bytes;
    used_ += bytes;
    return GpuAlloc{chunks_.back(), 0, bytes};
}

void GpuArena::reset() {
    cur_ = 0;
    cur_off_ = 0;
    used_ = 0;
}

void GpuArena::rewind_to(const Mark& m) {
    if (m.chunk > cur_ || (m.chunk == cur_ && m.off > cur_off_) || m.used > used_)
        throw MediaError("arena: rewind to a mark past the current position");
    cur_ = m.chunk;
    cur_off_ = m.off;
    used_ = m.used;
}

// ---------------------------------------------------------------- LoRA factor files
//
// Key grammar (the format notes of core/models/lora.hpp:1-45): a key names a
// module's down factor ("<module>.lora_A…" or "<module>.lora_down…"), its up
// factor (".lora_B…" / ".lora_up…") or its alpha ("<module>.alpha").  The module
// part then loses, in this order: every display prefix ComfyUI or kohya put in
// front of it, kohya's "lora_unet_" / "lora_te_" head (whose '_' stand for '.'),
// and a trailing ".weight".  Those spellings, the alpha defaults and the error
// texts are the file format's and the reference's (core/models/lora.cpp:20-84).

namespace {

enum class LoraRole { None, Down, Up, Alpha };

bool has_suffix(std::string_view s, std::string_view tail) {
    return s.size() >= tail.size() && s.substr(s.size() - tail.size()) == tail;
}

// True when `tail` is the last dotted components of `whole`
// ("attn.to_q" of "blocks.0.attn.to_q").
bool is_dotted_tail(std::string_view tail, std::string_view whole) {
    return whole.size() > tail.size() && whole[whole.size() - tail.size() - 1] == '.' && has_suffix(whole, tail);
}

// A factor names its module with or without the checkpoint's container prefix.
bool same_module(std::string_view factor, std::string_view weight) {
    return factor == weight || is_dotted_tail(factor, weight) || is_dotted_tail(weight, factor);
}

std::string canonical_module(std::string_view s) {
    static constexpr std::string_view kDisplay[] = {"model.diffusion_model.", "diffusion_model.", "model.", "unet.",
                                                    "transformer."};
    // A display prefix is peeled only when something follows it; the list is
    // searched afresh after every peel.
    for (;;) {
        const auto hit = std::find_if(std::begin(kDisplay), std::end(kDisplay), [&](std::string_view p) {
            return s.size() > p.size() && s.substr(0, p.size()) == p;
        });
        if (hit == std::end(kDisplay)) break;
        s.remove_prefix(hit->size());
    }
    std::string name(s);
    for (std::string_view head : {std::string_view("lora_unet_"), std::string_view("lora_te_")}) {
        if (name.compare(0, head.size(), head) != 0) continue;
        name.erase(0, head.size());
        std::replace(name.begin(), name.end(), '_', '.');
        break;
    }
    if (has_suffix(name, ".weight")) name.resize(name.size() - 7);
    return name;
}

// The role of a LoRA file's key and the module it belongs to ("" with None).
LoraRole classify_lora_key(const std::string& key, std::string* module) {
    module->clear();
    if (has_suffix(key, ".alpha")) {
        *module = canonical_module(std::string_view(key).substr(0, key.size() - 6));
        return LoraRole::Alpha;
    }
    static const struct {
        const char* tag;
        LoraRole role;
    } kTags[] = {{".lora_A", LoraRole::Down}, {".lora_down", LoraRole::Down}, {".lora_B", LoraRole::Up},
                 {".lora_up", LoraRole::Up}};
    for (const auto& tag : kTags) {
        const size_t at = key.find(tag.tag);
        if (at == std::string::npos) continue;
        *module = canonical_module(std::string_view(key).substr(0, at));
        return tag.role;
    }
    return LoraRole::None;
}

// The file-wide alpha: the first of the metadata spellings kohya and ComfyUI
// write ("ss_network_alpha", "lora_alpha", "network_alpha") that holds a
// positive number; 0 when none does.
float metadata_alpha(const std::map<std::string, std::string>& meta) {
    for (const char* key : {"ss_network_alpha", "lora_alpha", "network_alpha"}) {
        const auto it = meta.find(key);
        if (it == meta.end()) continue;
        const float v = (float)std::atof(it->second.c_str());
        if (v > 0) return v;
    }
    return 0.0f;
}

std::string file_name_of(const std::string& path) {
    const size_t cut = path.find_last_of("/\\");
    return cut == std::string::npos ? path : path.substr(cut + 1);
}

}  // namespace

std::string lora_normalize_target(const std::string& key, bool* is_a, bool* is_b) {
    std::string module;
    const LoraRole role = classify_lora_key(key, &module);
    if (is_a) *is_a = role == LoraRole::Down;
    if (is_b) *is_b = role == LoraRole::Up;
    return module;
}

// The semantics of core/models/lora.cpp:87-165: modules in the order of their
// first key; a module needs both factors, 2-D, with agreeing rank; its alpha is
// its own ".alpha" (the last one read), else the file's, else its rank; the
// file's strength multiplies the delta.
void LoraSet::add(const std::string& path, float strength) {
    if ((int)paths_.size() >= kMaxLoras)
        throw MediaError("LoRA: at most " + std::to_string(kMaxLoras) + " files may be chained");
    const SafeTensors st(path);
    const float file_alpha = metadata_alpha(st.metadata());

    struct ModuleKeys {
        std::string module;
        const StTensor* down = nullptr;
        const StTensor* up = nullptr;
        std::optional<float> alpha;
    };
    std::vector<ModuleKeys> modules;
    std::unordered_map<std::string, size_t> slot_of;
    std::string module;
    for (const std::string& key : st.names()) {
        const LoraRole role = classify_lora_key(key, &module);
        if (role == LoraRole::None || module.empty()) continue;
        const auto [slot, fresh] = slot_of.try_emplace(module, modules.size());
        if (fresh) modules.push_back(ModuleKeys{module, nullptr, nullptr, std::nullopt});
        ModuleKeys& keys = modules[slot->second];
        const StTensor& t = st.require(key);
        switch (role) {
            case LoraRole::Down: keys.down = &t; break;
            case LoraRole::Up: keys.up = &t; break;
            default:
                if (const std::vector<float> v = st.to_f32(t); !v.empty()) keys.alpha = v.front();
                break;
        }
    }

    const size_t before = adapters_.size();
    for (const ModuleKeys& keys : modules) {
        if (!keys.down || !keys.up || keys.down->shape.size() != 2 || keys.up->shape.size() != 2) continue;
        Adapter ad;
        ad.module = keys.module;
        ad.rank = keys.down->shape[0];
        ad.cols = keys.down->shape[1];
        ad.rows = keys.up->shape[0];
        if (keys.up->shape[1] != ad.rank || ad.rank <= 0 || ad.rows <= 0 || ad.cols <= 0) continue;
        const float alpha = keys.alpha ? *keys.alpha : file_alpha > 0 ? file_alpha : (float)ad.rank;
        ad.scale = strength * alpha / (float)ad.rank;
        std::vector<float> down = st.to_f32(*keys.down);
        const std::vector<float> up = st.to_f32(*keys.up);
        if ((i64)down.size() != ad.rank * ad.cols || (i64)up.size() != ad.rows * ad.rank) continue;
        ad.f32 = std::move(down);
        ad.f32.insert(ad.f32.end(), up.begin(), up.end());
        adapters_.push_back(std::move(ad));
    }
    if (adapters_.size() == before)
        throw MediaError("LoRA: " + file_name_of(path) + " holds no A/B factor pairs this engine can map");
    paths_.push_back(path);
}

std::vector<const LoraSet::Adapter*> LoraSet::matching(const std::string& target) const {
    std::vector<const Adapter*> hits;
    for (const Adapter& ad : adapters_)
        if (same_module(ad.module, target)) hits.push_back(&ad);
    return hits;
}

int LoraSet::deltas_for(const std::string& target, i64 n, i64 k, std::vector<Delta>* out) const {
    int count = 0;
    for (const Adapter* ad : matching(target)) {
        if (ad->rows != n || ad->cols != k) continue;  // a delta of another shape is never guessed onto this one
        if (out) out->push_back(ad->delta());
        count++;
    }
    return count;
}

int LoraSet::deltas_for_rows(const std::string& target, i64 row0, i64 rows, i64 k, std::vector<Delta>* out) const {
    if (rows <= 0 || k <= 0 || row0 < 0) return 0;
    int count = 0;
    for (const Adapter* ad : matching(target)) {
        if (ad->cols != k || row0 + rows > ad->rows) continue;  // the slice lies outside the delta
        if (out) out->push_back(ad->delta());
        count++;
    }
    return count;
}

bool LoraSet::touches(const std::string& target) const { return !matching(target).empty(); }

namespace {

// w[o][:] += (scale * up[row0 + o][r]) * down[r][:] as rank-one updates for
// r = 0, 1, …, rank-1, skipping the 0 entries of up.  Every element of w sees
// its terms in ascending r, the order that fixes the fp32 result
// (core/models/lora.cpp:182-201).
void rank1_updates(const LoraSet::Delta& d, float* w, i64 row0, i64 rows, i64 k) {
    for (i64 r = 0; r < d.rank; r++) {
        const float* down = d.a + r * k;
        for (i64 o = 0; o < rows; o++) {
            const float u = d.b[(row0 + o) * d.rank + r];
            if (u == 0.0f) continue;
            const float s = d.scale * u;
            float* wrow = w + o * k;
            for (i64 i = 0; i < k; i++) wrow[i] += s * down[i];
        }
    }
}

}  // namespace

int LoraSet::apply(const std::string& target, float* w, i64 n, i64 k) const {
    if (!w || n <= 0 || k <= 0) return 0;
    std::vector<Delta> ds;
    deltas_for(target, n, k, &ds);
    for (const Delta& d : ds) rank1_updates(d, w, 0, n, k);
    return (int)ds.size();
}

int LoraSet::apply_rows(const std::string& target, float* w, i64 row0, i64 rows, i64 k) const {
    if (!w) return 0;
    std::vector<Delta> ds;
    deltas_for_rows(target, row0, rows, k, &ds);
    for (const Delta& d : ds) rank1_updates(d, w, row0, rows, k);
    return (int)ds.size();
}

// The operands of core/models/model_common.cpp:1587-1652.  The matching factors
// sit side by side along the rank axis, module by module and in file order
// within a module; that order decides the correction's fp32 sums.
LoraTail load_lora_tail(GpuCtx& g, GpuArena& arena, const std::vector<LoraModule>& mods, i64 n, i64 k) {
    if (mods.empty() || n <= 0 || k <= 0) return LoraTail{};
    struct Slice {
        i64 out_row0;  // the module's first output row
        i64 col0;      // the factor's first rank column
        LoraSet::Delta d;
    };
    std::vector<Slice> slices;
    i64 width = 0;
    for (const LoraModule& m : mods) {
        if (!m.lora || m.n <= 0) continue;
        if (m.row0 < 0 || m.row0 + m.n > n)
            throw MediaError("LoRA correction: module " + m.base + " covers rows [" + std::to_string(m.row0) + ", " +
                             std::to_string(m.row0 + m.n) + ") of a " + std::to_string(n) + "-row weight");
        std::vector<LoraSet::Delta> ds;
        m.lora->deltas_for(m.base, m.n, k, &ds);
        for (const LoraSet::Delta& d : ds) {
            slices.push_back(Slice{m.row0, width, d});
            width += d.rank;
        }
    }
    if (width == 0) return LoraTail{};
    if (width > kLoraRankBound)
        throw MediaError("LoRA correction: the factors matching this module need a " + std::to_string(width) +
                         "-wide correction, past the " + std::to_string(kLoraRankBound) +
                         " the activation plans reserve (kLoraRankBound)");
    if (!g.ctx) throw MediaError("load_lora_tail: no compute context");

    // at [width, k]: each slice's down rows.  bt [n, width]: output row o of a
    // slice's module holds scale * up[o - out_row0][:] in the slice's columns and
    // zeros elsewhere, so bt . (at . x) is the sum of every factor's product.
    std::vector<float> at((size_t)(width * k)), bt((size_t)(n * width), 0.0f);
    for (const Slice& s : slices) {
        std::copy_n(s.d.a, (size_t)(s.d.rank * k), at.begin() + (std::ptrdiff_t)(s.col0 * k));
        for (i64 o = 0; o < s.d.n; o++) {
            const float* up = s.d.b + o * s.d.rank;
            std::transform(up, up + s.d.rank, bt.begin() + (std::ptrdiff_t)((s.out_row0 + o) * width + s.col0),
                           [scale = s.d.scale](float u) { return scale * u; });
        }
    }
    LoraTail tail;
    tail.at = arena.alloc((u64)at.size() * 4);
    tail.bt = arena.alloc((u64)bt.size() * 4);
    g.ctx->upload(tail.at.res, at.data(), at.size() * 4, tail.at.off);
    g.ctx->upload(tail.bt.res, bt.data(), bt.size() * 4, tail.bt.off);
    tail.rank = width;
    tail.n = n;
    tail.k = k;
    tail.active = true;
    return tail;
}

LoraTail load_lora_tail(GpuCtx& g, GpuArena& arena, const std::string& base, const LoraSet* lora, i64 n, i64 k) {
    if (!lora) return LoraTail{};
    return load_lora_tail(g, arena, {LoraModule{base, 0, n, lora}}, n, k);
}

namespace {

// Where the parts of a grouped weight (asym_w4a8_int8, w6a8_int8) live, for the
// device expand.  The family's rules are core/host/st.cpp:839-925 and the
// device path's own conditions core/models/model_common.cpp:605-680; unlike
// that path, a weight_correction plane is carried to the expand here.
struct GroupedParts {
    CodeLayout layout = CodeLayout::Nibble4;
    const StTensor* codes = nullptr;
    const StTensor* srel = nullptr;
    const StTensor* sch = nullptr;
    const StTensor* codebook = nullptr;
    const StTensor* correction = nullptr;
    i64 n = 0, k = 0, group = 0, srel_row_bytes = 0;
    RelDType rel_dtype = RelDType::F32;
};

std::optional<RelDType> rel_dtype_of(StDType d) {
    switch (d) {
        case StDType::F32: return RelDType::F32;
        case StDType::F16: return RelDType::F16;
        case StDType::BF16: return RelDType::BF16;
        case StDType::F8_E4M3: return RelDType::F8_E4M3;
        case StDType::F8_E5M2: return RelDType::F8_E5M2;
        case StDType::U8: return RelDType::U8_E4M3;  // an fp8 table in a byte container
        default: return std::nullopt;
    }
}

// Empty when `t` can be expanded on the device, with `out` filled; otherwise why not.
std::string grouped_parts_of(const SafeTensors& st, const StTensor& t, GroupedParts* out) {
    const SafeTensors::WeightLayout L = st.weight_layout(t.name);
    const bool six = L.spec.format == "w6a8_int8" || L.spec.format == "w6a8";
    if (!six && L.spec.format != "asym_w4a8_int8") return "the format is not a grouped int4 / int6 family";
    // Codes: a 2-D byte plane already in the rotated basis.
    if (t.shape.size() != 2 || (t.dtype != StDType::I8 && t.dtype != StDType::U8))
        return "codes are not a 2-D byte tensor";
    if (!L.spec.convrot) return "the weight is not convrot-rotated";
    // The relative-scale table and its element type.
    if (!L.rel_scale || L.rel_scale->shape.size() != 2) return "no 2-D weight_s_rel table";
    const std::optional<RelDType> rel = rel_dtype_of(L.rel_scale->dtype);
    if (!rel) return std::string("weight_s_rel dtype ") + st_dtype_name(L.rel_scale->dtype) + " is not decodable";
    // Geometry: whole groups of whole code bytes, and rows wide enough for K.
    GroupedParts p;
    p.n = t.shape[0];
    p.k = st.logical_cols(t);
    p.group = L.group;
    const i64 codes_per_unit = six ? 4 : 2;  // codes that fill whole bytes
    if (p.group <= 0 || p.group % codes_per_unit != 0 || p.k % p.group != 0)
        return "group " + std::to_string(p.group) + " does not divide K";
    const i64 row_need = six ? p.k / 2 + p.k / 4 : p.k / 2;  // six bits: a nibble plane, then a 2-bit plane
    if ((i64)t.row_bytes() < row_need) return "code rows are shorter than K needs";
    if (L.rel_scale->shape[0] != p.n || L.rel_scale->shape[1] != p.k / p.group)
        return "weight_s_rel is not [N, K/group]";
    // The optional tables.
    if (six && L.codebook) return "a six-bit weight with a codebook";
    if (L.codebook && !six && (L.codebook->dtype != StDType::F32 || L.codebook->numel != 16))
        return "the codebook is not 16 fp32 levels";
    if (L.row_scale) {
        const bool per_row_or_one = L.row_scale->numel == 1 || L.row_scale->numel == p.n;
        if (L.row_scale->dtype != StDType::F32 || !per_row_or_one) return "the channel scale is not fp32 [N] or [1]";
    }
    if (const StTensor* c = L.correction) {
        const bool fits = c->dtype == StDType::F32 && c->shape.size() == 2 && c->shape[0] == p.k / p.group &&
                          c->shape[1] == p.n;
        if (!fits) return "weight_correction is not fp32 [K/group, N]";
    }
    p.layout = six ? CodeLayout::Packed6 : CodeLayout::Nibble4;
    p.codes = &t;
    p.srel = L.rel_scale;
    p.sch = L.row_scale;
    p.codebook = six ? nullptr : L.codebook;
    p.correction = L.correction;
    p.srel_row_bytes = (i64)L.rel_scale->row_bytes();
    p.rel_dtype = *rel;
    *out = p;
    return "";
}

}  // namespace

namespace {

u64 up256(u64 v) { return (v + 255) & ~(u64)255; }

u64 checked_mul(u64 a, u64 b, const std::string& what) {
    u64 r = 0;
    if (__builtin_mul_overflow(a, b, &r)) throw MediaError(what + ": size overflows");
    return r;
}

// A device buffer for one load step; the stream is drained before it is freed.
struct Scratch {
    ComputeContext& ctx;
    GpuBuffer* b;
    u64 charged;
    Scratch(ComputeContext& c, u64 bytes) : ctx(c), b(nullptr), charged(bytes) {
        vram_budget().charge(bytes, "load scratch");
        try {
            b = c.create_device_buffer(bytes);
        } catch (...) {
            vram_budget().release(bytes);
            throw;
        }
    }
    ~Scratch() {
        (void)hipStreamSynchronize(ctx.stream());
        ctx.release_buffer(b);
        vram_budget().release(charged);
    }
    Scratch(const Scratch&) = delete;
    Scratch& operator=(const Scratch&) = delete;
    uintptr_t at(u64 off) const { return b->base + off; }
};

// The precision a weight carries on disk (weight_precision_of, core/host/st.cpp:954-983):
// the dense-float forms run the dense GEMM, not the int8 path.
const char* dense_precision(const SafeTensors& st, const StTensor& t) {
    switch (t.dtype) {
        case StDType::F16: return "f16";
        case StDType::BF16: return "bf16";
        case StDType::F32: return "f32";
        case StDType::F8_E4M3:
        case StDType::F8_E5M2: return "fp8";
        case StDType::I8:
        case StDType::U8: {
            const std::string& f = st.weight_layout(t.name).spec.format;
            return f == "nvfp4" || f == "mxfp4" ? "nvfp4" : nullptr;
        }
        default: return nullptr;
    }
}

// The spec a decoded weight is requantised with (requant_spec_for,
// core/host/st.cpp:1040-1048): convrot, unless the file says the stored
// matrix is already rotated.
bool requant_rotates(const SafeTensors& st, const std::string& base) {
    const StTensor* t = st.find(base + ".weight");
    if (!t) return true;
    const SafeTensors::WeightLayout L = st.weight_layout(t->name);
    return !(L.spec.valid && L.spec.convrot);
}

// What the device decodes: int8 codes times their row scale, fp8 codes times
// their optional row scale, f16 / bf16 / f32 widened, a bare packed int4 (two
// signed nibbles a byte) times its row scale, or nvfp4 / mxfp4 E2M1 codes times
// their block and global scales (SafeTensors::dequant_rows,
// core/host/st.cpp:601-700).
constexpr int kDecodeI4 = -2, kDecodeFp4 = -3;
struct Decodable {
    int dtype = -1;  // PHI_I8 / PHI_F8_E4M3 / PHI_F8_E5M2 / PHI_F16 / PHI_BF16 / PHI_F32, kDecodeI4, kDecodeFp4
    const StTensor* scale = nullptr;
};

Decodable decodable(const SafeTensors& st, const StTensor& t) {
    Decodable d;
    const SafeTensors::WeightLayout L = st.weight_layout(t.name);
    if ((t.dtype == StDType::I8 || t.dtype == StDType::U8) && (L.spec.format == "nvfp4" || L.spec.format == "mxfp4")) {
        d.dtype = kDecodeFp4;
        return d;
    }
    switch (t.dtype) {
        case StDType::F32: d.dtype = PHI_F32; break;
        case StDType::F16: d.dtype = PHI_F16; break;
        case StDType::BF16: d.dtype = PHI_BF16; break;
        case StDType::F8_E4M3:
        case StDType::F8_E5M2:
            d.dtype = t.dtype == StDType::F8_E4M3 ? PHI_F8_E4M3 : PHI_F8_E5M2;
            d.scale = L.row_scale;
            break;
        case StDType::I8:
            if (L.packed || L.rel_scale) return d;
            if (L.spec.valid && !L.known_family)
                throw MediaError("'" + t.name + "': the quantisation format \"" + L.spec.format +
                                 "\" is not one this engine can decode");
            d.dtype = PHI_I8;
            d.scale = st.find(t.name.substr(0, t.name.size() - 7) + ".weight_scale");
            if (!d.scale)
                throw MediaError("'" + t.name + "': an int8 weight without a scale table (or a packed format this "
                                 "engine does not know) cannot be read");
            break;
        case StDType::I4:
            if (L.packed) return d;
            d.dtype = kDecodeI4;
            d.scale = L.row_scale;
            break;
        default: break;
    }
    return d;
}

// Decode -> (rotate back) -> (fold LoRA deltas) -> rotate + quantise, for rows
// [0, n) of one stored weight, slab by slab, into q (+ row0 * k) and s (+ row0).
// `deltas(r0, rows)` returns the factors to fold into rows [r0, r0 + rows).
struct RequantPlan {
    bool unrotate = false;  // undo the stored convrot first (the fold's original basis)
    bool rotate = true;     // the quantiser's convrot
    std::function<std::vector<LoraSet::Delta>(i64, i64)> deltas;
};

void requant_rows_device(GpuCtx& g, const SafeTensors& st, const StTensor& t, i64 n, i64 k, const RequantPlan& plan,
                         int8_t* q, float* s) {
    ComputeContext& ctx = *g.ctx;
    const Decodable d = decodable(st, t);
    if (d.dtype == -1)
        throw MediaError("'" + t.name + "': " + st_dtype_name(t.dtype) + " is not a weight form this loader decodes");
    const bool i4 = d.dtype == kDecodeI4, fp4 = d.dtype == kDecodeFp4;
    const u64 src_row = i4 ? (u64)((k + 1) / 2) : t.row_bytes();
    if ((u64)n * src_row > t.nbytes) throw MediaError("'" + t.name + "' holds fewer rows than its shape says");
    if (fp4 && src_row < (u64)((k + 1) / 2)) throw MediaError("'" + t.name + "': fp4 code rows are shorter than K needs");
    const u64 slab = (u64)std::max<i64>(1, std::min<i64>(n, (64ll << 20) / std::max<i64>(k * 4, 1)));
    // Device copies: the row scales (host-decoded from their table), and every
    // LoRA factor's A and B once.
    std::vector<float> scales;
    if (d.scale) {
        scales.resize((size_t)n);
        for (i64 r = 0; r < n; r++) scales[(size_t)r] = st.row_scale_value(*d.scale, r);
    }
    // nvfp4 / mxfp4: the block table decoded to fp32 as stored (its tiled
    // layout kept), its geometry, and the global scale of every row.
    std::vector<float> blocks, globals;
    i64 blk_rows = 0, blk_cols = 0, block = 16;
    if (fp4) {
        const SafeTensors::WeightLayout L = st.weight_layout(t.name);
        block = L.group > 0 ? L.group : 16;
        if (const StTensor* b = L.rel_scale) {
            blk_rows = b->shape.empty() ? 1 : b->shape[0];
            blk_cols = b->shape.size() > 1 ? b->shape[1] : 0;
            blocks.resize((size_t)b->numel);
            for (i64 i = 0; i < b->numel; i++) blocks[(size_t)i] = st.row_scale_value(*b, i);
        }
        if (const StTensor* gs = L.global_scale) {
            globals.resize((size_t)n);
            for (i64 r = 0; r < n; r++) globals[(size_t)r] = st.row_scale_value(*gs, r);
        }
    }
    const u64 o_src = 0, o_f32 = up256(slab * src_row), o_sc = o_f32 + up256(slab * (u64)k * 4),
              o_blk = o_sc + up256((u64)n * 4 + 4), total = o_blk + up256((u64)blocks.size() * 4 + 4);
    Scratch work(ctx, total);
    if (!scales.empty()) ctx.upload(work.b, scales.data(), scales.size() * 4, o_sc);
    if (!globals.empty()) ctx.upload(work.b, globals.data(), globals.size() * 4, o_sc);
    if (!blocks.empty()) ctx.upload(work.b, blocks.data(), blocks.size() * 4, o_blk);
    float* f32 = (float*)work.at(o_f32);
    for (i64 r0 = 0; r0 < n; r0 += (i64)slab) {
        const i64 rows = std::min<i64>((i64)slab, n - r0);
        ctx.upload(work.b, t.data + (u64)r0 * src_row, (u64)rows * src_row, o_src);
        if (fp4) {
            ctx.check(phi_hip_dequant_fp4_rows(ctx.stream(), (const uint8_t*)work.at(o_src), (int64_t)src_row, r0, rows,
                                               k, blocks.empty() ? nullptr : (const float*)work.at(o_blk), blk_rows,
                                               blk_cols, block,
                                               globals.empty() ? nullptr : (const float*)work.at(o_sc) + r0, 0, f32, k),
                      "dequant_fp4_rows");
        } else {
            const bool sc = d.scale != nullptr;
            const bool sc1 = sc && d.scale->numel == 1;
            ctx.check(phi_hip_dequant_rows(ctx.stream(), (const void*)work.at(o_src), i4 ? PHI_I4 : d.dtype, rows, k,
                                           (int64_t)(i4 ? src_row : src_row / st_dtype_bytes(t.dtype)),
                                           sc ? (const float*)work.at(o_sc) + (sc1 ? 0 : r0) : nullptr, sc1 ? 1 : 0,
                                           f32, k),
                      "dequant_rows");
        }
        if (plan.unrotate) ctx.check(phi_hip_convrot_rows(ctx.stream(), f32, rows, k, k, f32, k), "convrot");
        if (plan.deltas) {
            for (const LoraSet::Delta& f : plan.deltas(r0, rows)) {
                const u64 ab = (u64)f.rank * (u64)f.k * 4, bb = (u64)rows * (u64)f.rank * 4;
                Scratch fac(ctx, up256(ab) + bb);
                ctx.upload(fac.b, f.a, ab, 0);
                ctx.upload(fac.b, f.b + r0 * f.rank, bb, up256(ab));
                ctx.check(phi_hip_lora_fold(ctx.stream(), f32, k, rows, k, (const float*)fac.at(0),
                                            (const float*)fac.at(up256(ab)), f.rank, f.scale),
                          "lora_fold");
                ctx.submit();
            }
        }
        ctx.check(phi_hip_quant_rotate(ctx.stream(), f32, PHI_F32, rows, k, k, q + r0 * k, k, s + r0, 127.0f,
                                       PHI_ROUND_HALF_AWAY, plan.rotate ? 1 : 0),
                  "quantize_weight");
        ctx.submit();
    }
}

// The stored parts of a grouped weight staged on the device and expanded into
// q [n, k] / s [n] (w4a8_pack_rows, core/models/model_common.cpp:680-748).
void expand_grouped(GpuCtx& g, const StTensor& t, const GroupedParts& parts, int8_t* q, float* s, const SafeTensors& st) {
    ComputeContext& ctx = *g.ctx;
    const i64 n = parts.n;
    const u64 cb = checked_mul((u64)n, t.row_bytes(), "w4a8 codes"), sb = parts.srel->nbytes, hb = parts.sch ? (u64)n * 4 : 0,
              kb = parts.codebook ? 64 : 0, rb = parts.correction ? parts.correction->nbytes : 0;
    const u64 o_codes = 0, o_srel = up256(cb), o_sch = o_srel + up256(sb), o_cb = o_sch + up256(hb),
              o_corr = o_cb + up256(kb), total = o_corr + up256(rb);
    Scratch stage(ctx, total);
    ctx.upload(stage.b, t.data, cb, o_codes);
    ctx.upload(stage.b, parts.srel->data, sb, o_srel);
    if (parts.sch) {
        std::vector<float> v((size_t)n);
        for (i64 r = 0; r < n; r++) v[(size_t)r] = st.row_scale_value(*parts.sch, r);  // a [1] table broadcasts
        ctx.upload(stage.b, v.data(), hb, o_sch);
    }
    if (parts.codebook) ctx.upload(stage.b, parts.codebook->data, kb, o_cb);
    if (parts.correction) ctx.upload(stage.b, parts.correction->data, rb, o_corr);
    phi_w4a8_weight w{};
    w.codes = (const uint8_t*)stage.at(o_codes);
    w.codes_row_bytes = (int64_t)t.row_bytes();
    w.s_rel = (const void*)stage.at(o_srel);
    w.s_rel_dtype = phi_rel_dtype(parts.rel_dtype);
    w.srel_row_bytes = parts.srel_row_bytes;
    w.s_channel = parts.sch ? (const float*)stage.at(o_sch) : nullptr;
    w.codebook = parts.codebook ? (const float*)stage.at(o_cb) : nullptr;
    w.correction = parts.correction ? (const float*)stage.at(o_corr) : nullptr;
    w.rows = n;
    w.k = parts.k;
    w.group = parts.group;
    w.layout = parts.layout == CodeLayout::Nibble4 ? 0 : 1;
    ctx.check(phi_hip_w4a8_expand(ctx.stream(), &w, q, s), "w4a8_expand");
    ctx.submit();
}

int8_t* dev_i8(const GpuAlloc& a, u64 off = 0) { return (int8_t*)(a.res->base + a.off + off); }
float* dev_f32(const GpuAlloc& a, u64 off = 0) { return (float*)(a.res->base + a.off + off); }

// Where a loader writes an int8 weight's rows: straight into the weight's
// allocation, or, for a K-tiled weight, into a charged load scratch that
// finish() packs into the allocation (phi_hip_pack_k_tiled) once every row is
// there.
class WeightRows {
public:
    WeightRows(GpuCtx& g, const GpuAlloc& w, i64 n, i64 k, bool k_tiled)
        : g_(g), w_(w), n_(n), k_(k) {
        if (k_tiled) staging_.emplace(*g.ctx, (u64)n * (u64)k);
    }
    int8_t* row(i64 r) const {
        return staging_ ? (int8_t*)staging_->at((u64)r * (u64)k_) : dev_i8(w_, (u64)r * (u64)k_);
    }
    void upload(i64 r, const void* src, u64 bytes) {
        if (staging_) g_.ctx->upload(staging_->b, src, bytes, (u64)r * (u64)k_);
        else g_.ctx->upload(w_.res, src, bytes, w_.off + (u64)r * (u64)k_);
    }
    // True when the weight ended up K-tiled.
    bool finish() {
        if (!staging_) return false;
        g_.ctx->check(phi_hip_pack_k_tiled(g_.ctx->stream(), row(0), k_, n_, k_, dev_i8(w_)), "pack_k_tiled");
        g_.ctx->submit();
        return true;
    }

private:
    GpuCtx& g_;
    GpuAlloc w_;
    i64 n_, k_;
    std::optional<Scratch> staging_;
};

// The shapes the K-tiled linear takes (phi_hip_q8_linear_kt with fp32 output).
bool k_tiled_shape(i64 n, i64 k) { return n > 0 && k > 0 && k % 256 == 0 && k <= 16384 && n % 4 == 0; }

// One plain int8 weight's scales, decoded from their table.
std::vector<float> weight_scales(const SafeTensors& st, const std::string& base, i64 n) {
    const StTensor& sc = st.require(base + ".weight_scale");
    if (sc.numel != n) throw MediaError("weight_scale length mismatch: " + base);
    std::vector<float> s((size_t)n);
    for (i64 r = 0; r < n; r++) s[(size_t)r] = st.row_scale_value(sc, r);
    return s;
}

}  // namespace

// core/models/model_common.cpp:921-1090
QuantLinear load_quant_linear(GpuCtx& g, const SafeTensors& st, const std::string& base, GpuArena* into,
                              const LoraSet* lora) {
    if (!g.ctx) throw MediaError("load_quant_linear: no compute context");
    auto alloc = [&](u64 bytes) { return into ? into->alloc(bytes) : g.walloc(bytes); };
    const StTensor& t = st.require(base + ".weight");
    if (t.shape.size() != 2) throw MediaError("load_quant_linear: '" + base + ".weight' is not a 2-D matrix");
    const i64 n = t.shape[0], k = st.logical_cols(t);
    const u64 nk = checked_mul((u64)n, (u64)k, "load_quant_linear: '" + base + "'");
    if (const char* prec = dense_precision(st, t))
        throw MediaError("load_quant_linear: '" + base + ".weight' is " + prec +
                         ": a dense float weight runs the dense GEMM, which the quantized-linear library does not "
                         "serve");
    const bool touched = lora && lora->touches(base);
    const bool kt = g.k_tiled_weights && k_tiled_shape(n, k);
    QuantLinear q;
    q.n = n;
    q.k = k;
    if (st.is_plain_int8(t) && !touched) {
        // Shipped int8 tensorwise: the codes verbatim, one fp32 scale per row.
        if (t.nbytes != nk) throw MediaError("load_quant_linear: '" + base + ".weight' is not [N, K] int8");
        const std::vector<float> s = weight_scales(st, base, n);
        q.w = alloc(nk);
        WeightRows rows(g, q.w, n, k, kt);
        rows.upload(0, t.data, t.nbytes);
        q.k_tiled = rows.finish();
        q.scale = alloc((u64)n * 4);
        g.ctx->upload(q.scale.res, s.data(), (u64)n * 4, q.scale.off);
        return q;
    }
    const SafeTensors::WeightLayout L = st.weight_layout(t.name);
    if (L.packed) {
        if (touched)
            throw MediaError("load_quant_linear: '" + base + "' (" + L.spec.format +
                             "): a LoRA is not folded into a grouped weight here; load the tail with load_lora_tail "
                             "and apply it with apply_lora_tail");
        GroupedParts parts;
        const std::string why = grouped_parts_of(st, t, &parts);
        if (!why.empty()) throw MediaError("load_quant_linear: '" + base + "' (" + L.spec.format + "): " + why);
        q.w = alloc(nk);
        q.scale = alloc((u64)n * 4);
        WeightRows rows(g, q.w, n, k, kt);
        expand_grouped(g, t, parts, rows.row(0), dev_f32(q.scale), st);
        q.k_tiled = rows.finish();
        return q;
    }
    if (L.spec.valid && L.spec.format == "convrot_w4a4")
        throw MediaError("load_quant_linear: '" + base + "' is convrot_w4a4: load it with upload_quant_linear_w4a4 "
                         "for the int4 GEMM");
    // Decode, (fold,) requantise.  A fold decodes into the original basis
    // (dequant_weight_f32 rotates a convrot weight back) and quantises with the
    // default spec, which rotates; otherwise the requant spec decides.
    const bool rotate = touched ? true : requant_rotates(st, base);
    if (rotate && k % 256 != 0)
        throw MediaError("'" + base + "' has K=" + std::to_string(k) +
                         ", not a multiple of the convrot group 256; load it on the bf16 path instead");
    RequantPlan plan;
    plan.rotate = rotate;
    if (touched) {
        plan.unrotate = L.spec.convrot;
        plan.deltas = [&](i64 r0, i64 rows) {
            std::vector<LoraSet::Delta> d;
            lora->deltas_for(base, n, k, &d);
            (void)r0;
            (void)rows;
            return d;
        };
    }
    q.w = alloc(nk);
    q.scale = alloc((u64)n * 4);
    WeightRows rows(g, q.w, n, k, kt);
    requant_rows_device(g, st, t, n, k, plan, rows.row(0), dev_f32(q.scale));
    q.k_tiled = rows.finish();
    return q;
}

// core/models/model_common.cpp:1414-1578
QuantLinear load_quant3_linear(GpuCtx& g, const SafeTensors& st, const std::string& base_q, const std::string& base_k,
                               const std::string& base_v, GpuArena* into, const LoraSet* lora) {
    if (!g.ctx) throw MediaError("load_quant3_linear: no compute context");
    auto alloc = [&](u64 bytes) { return into ? into->alloc(bytes) : g.walloc(bytes); };
    const std::string bases[3] = {base_q, base_k, base_v};
    const StTensor* ts[3] = {&st.require(base_q + ".weight"), &st.require(base_k + ".weight"),
                             &st.require(base_v + ".weight")};
    const i64 k = st.logical_cols(*ts[0]);
    for (int i = 0; i < 3; i++)
        if (ts[i]->shape.size() != 2 || st.logical_cols(*ts[i]) != k)
            throw MediaError("load_quant3_linear: shape mismatch at " + bases[i]);
    bool raw_int8 = true, touched = false, any_dense = false, all_dense = true;
    for (int i = 0; i < 3; i++) {
        raw_int8 = raw_int8 && st.is_plain_int8(*ts[i]);
        touched = touched || (lora && lora->touches(bases[i]));
        const bool d = dense_precision(st, *ts[i]) != nullptr;
        any_dense = any_dense || d;
        all_dense = all_dense && d;
    }
    if (any_dense) {
        if (!all_dense) throw MediaError("load_quant3_linear: q/k/v mix a float and a quantised precision");
        throw MediaError("load_quant3_linear: '" + base_q + "' is a dense float weight: the dense q|k|v GEMM is not "
                         "served by the quantized-linear library");
    }
    QuantLinear q;
    q.k = k;
    i64 rows_of[3], row0[3];
    i64 total = 0;
    for (int i = 0; i < 3; i++) {
        rows_of[i] = ts[i]->shape[0];
        row0[i] = total;
        total += rows_of[i];
    }
    q.n = total;
    const u64 nk = checked_mul((u64)q.n, (u64)k, "load_quant3_linear");
    const bool kt = g.k_tiled_weights && k_tiled_shape(q.n, k);
    if (raw_int8 && !touched) {
        // The raw int8 rows and scale vectors, concatenated.
        std::vector<float> scales;
        for (int i = 0; i < 3; i++) {
            const std::vector<float> s = weight_scales(st, bases[i], rows_of[i]);
            scales.insert(scales.end(), s.begin(), s.end());
            if (ts[i]->nbytes != (u64)rows_of[i] * (u64)k)
                throw MediaError("load_quant3_linear: '" + bases[i] + ".weight' is not [N, K] int8");
        }
        q.w = alloc(nk);
        WeightRows rows(g, q.w, q.n, k, kt);
        for (int i = 0; i < 3; i++) rows.upload(row0[i], ts[i]->data, ts[i]->nbytes);
        q.k_tiled = rows.finish();
        q.scale = alloc((u64)scales.size() * 4);
        g.ctx->upload(q.scale.res, scales.data(), scales.size() * 4, q.scale.off);
        return q;
    }
    // One requant spec for all three: base_q's (requant_spec_for(st, base_q)).
    const bool rotate = requant_rotates(st, base_q);
    if (rotate && k % 256 != 0)
        throw MediaError("load_quant3_linear: K=" + std::to_string(k) + " is not a multiple of the convrot group 256");
    q.w = alloc(nk);
    q.scale = alloc((u64)q.n * 4);
    WeightRows rows(g, q.w, q.n, k, kt);
    for (int i = 0; i < 3; i++) {
        const StTensor& t = *ts[i];
        const SafeTensors::WeightLayout L = st.weight_layout(t.name);
        int8_t* qi = rows.row(row0[i]);
        float* si = dev_f32(q.scale, (u64)row0[i] * 4);
        RequantPlan plan;
        plan.rotate = rotate;
        if (touched) {
            // The reference folds each part in its original basis (the decoded
            // part rotated back when its file declares convrot) and quantises the
            // stacked matrix with base_q's requant spec.
            if (L.packed)
                throw MediaError("load_quant3_linear: '" + bases[i] + "' (" + L.spec.format +
                                 "): a LoRA is not folded into a grouped weight here; use load_lora_tail");
            plan.unrotate = L.spec.convrot;
            const std::string b = bases[i];
            const i64 ni = rows_of[i];
            plan.deltas = [&lora, b, ni, k](i64, i64) {
                std::vector<LoraSet::Delta> d;
                lora->deltas_for(b, ni, k, &d);
                return d;
            };
            requant_rows_device(g, st, t, rows_of[i], k, plan, qi, si);
            continue;
        }
        if (L.packed) {
            // The grouped decode requantises without a rotation: the stored rows
            // are already in the rotated basis, which base_q's spec must agree with.
            if (rotate)
                throw MediaError("load_quant3_linear: '" + bases[i] + "' (" + L.spec.format +
                                 ") is stored rotated, but " + base_q + "'s spec asks for a rotation");
            GroupedParts parts;
            const std::string why = grouped_parts_of(st, t, &parts);
            if (!why.empty()) throw MediaError("load_quant3_linear: '" + bases[i] + "' (" + L.spec.format + "): " + why);
            expand_grouped(g, t, parts, qi, si, st);
            continue;
        }
        requant_rows_device(g, st, t, rows_of[i], k, plan, qi, si);
    }
    q.k_tiled = rows.finish();
    return q;
}

// core/models/model_common.cpp:1095-1283
I8Upload upload_quant_linear_i8(GpuCtx& g, const SafeTensors& st, const std::string& base, GpuArena& arena,
                                const LoraSet* lora) {
    if (!g.ctx) throw MediaError("upload_quant_linear_i8: no compute context");
    const StTensor& t = st.require(base + ".weight");
    if (t.shape.size() != 2) throw MediaError("upload_quant_linear_i8: '" + base + ".weight' is not a 2-D matrix");
    I8Upload out;
    out.n = t.shape[0];
    out.k = st.logical_cols(t);
    const u64 nk = checked_mul((u64)out.n, (u64)out.k, "upload_quant_linear_i8: '" + base + "'");
    const SafeTensors::WeightLayout L = st.weight_layout(t.name);
    // A grouped weight is expanded on the device whatever `lora` holds (the
    // reference never folds into a streamed weight: the tail corrects it).
    if (L.packed) {
        GroupedParts parts;
        if (grouped_parts_of(st, t, &parts).empty()) {
            out.w = arena.alloc(nk);
            out.s = arena.alloc((u64)out.n * 4);
            expand_grouped(g, t, parts, dev_i8(out.w), dev_f32(out.s), st);
            return out;
        }
    }
    const bool touched = lora && lora->touches(base);
    if (st.is_plain_int8(t) && L.spec.convrot && !touched) {
        const std::vector<float> s = weight_scales(st, base, out.n);
        out.w = arena.alloc(t.nbytes);
        g.ctx->upload(out.w.res, t.data, t.nbytes, out.w.off);
        out.s = arena.alloc((u64)s.size() * 4);
        g.ctx->upload(out.s.res, s.data(), s.size() * 4, out.s.off);
        return out;
    }
    const bool spec_rotates = requant_rotates(st, base);
    if (spec_rotates && out.k % 256 != 0)
        throw MediaError("'" + base + "' has K=" + std::to_string(out.k) +
                         ", not a multiple of the convrot group 256; load it on the bf16 path instead");
    RequantPlan plan;
    plan.rotate = spec_rotates;
    if (touched) {
        // Slab by slab: rotate a stored-rotated slab back, add the rows' deltas,
        // then quantise with the default spec (which rotates).
        if (out.k % 256 != 0)
            throw MediaError("'" + base + "' has K=" + std::to_string(out.k) + ", not a multiple of the convrot group 256");
        plan.unrotate = !spec_rotates;
        plan.rotate = true;
        plan.deltas = [&](i64 r0, i64 rows) {
            std::vector<LoraSet::Delta> d;
            lora->deltas_for_rows(base, r0, rows, out.k, &d);
            return d;
        };
    }
    out.w = arena.alloc(nk);
    out.s = arena.alloc((u64)out.n * 4);
    requant_rows_device(g, st, t, out.n, out.k, plan, dev_i8(out.w), dev_f32(out.s));
    return out;
}

// core/models/model_common.cpp:1285-1340 (the verbatim branch)
I4Upload upload_quant_linear_w4a4(GpuCtx& g, const SafeTensors& st, const std::string& base, GpuArena& arena,
                                  const LoraSet* lora) {
    if (!g.ctx) throw MediaError("upload_quant_linear_w4a4: no compute context");
    const StTensor& t = st.require(base + ".weight");
    if (t.shape.size() != 2)
        throw MediaError("upload_quant_linear_w4a4: '" + base + ".weight' is not a 2-D matrix");
    if (lora && lora->touches(base))
        throw MediaError("upload_quant_linear_w4a4: '" + base +
                         "': a LoRA is not folded into int4 weights here; use load_lora_tail / apply_lora_tail");
    const i64 packed_k = t.shape[1], logical_k = st.logical_cols(t);
    if (packed_k % 2 != 0 || packed_k % 256 != 0)
        throw MediaError("qwen3vl: " + base + " has a packed width of " + std::to_string(packed_k) +
                         ", not packable to convrot_w4a4");
    if (logical_k != packed_k * 2 || logical_k % 256 != 0)
        throw MediaError("qwen3vl: " + base + " has K=" + std::to_string(logical_k) +
                         ", not a convrot_w4a4 matrix (it must be twice the packed width)");
    if (st_dtype_bytes(t.dtype) != 1) throw MediaError("upload_quant_linear_w4a4: '" + base + ".weight' is not bytes");
    const StTensor& sc = st.require(base + ".weight_scale");
    I4Upload out;
    out.n = t.shape[0];
    out.k = packed_k;
    out.w = arena.alloc(checked_mul((u64)out.n, (u64)packed_k, "upload_quant_linear_w4a4"));
    g.ctx->upload(out.w.res, t.data, t.nbytes, out.w.off);
    std::vector<float> s((size_t)out.n);
    for (i64 r = 0; r < out.n; r++) s[(size_t)r] = st.row_scale_value(sc, r);
    out.s = arena.alloc((u64)out.n * 4);
    g.ctx->upload(out.s.res, s.data(), (u64)out.n * 4, out.s.off);
    return out;
}

// ---------------------------------------------------------------- GEMM tuning table

std::string GemmTuneStore::default_path(const std::string& base_dir) {
    return (base_dir.empty() ? std::string(".") : base_dir) + "/data/gemm_plans.json";
}

bool GemmTuneStore::load(const std::string& path) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) return false;
    std::string text;
    char buf[4096];
    for (size_t n; (n = fread(buf, 1, sizeof buf, f)) > 0;) text.append(buf, n);
    fclose(f);
    std::vector<std::map<std::string, double>> recs;
    if (!parse_number_records(text, "plans", &recs)) return false;
    std::vector<GemmTuneEntry> items;
    for (const auto& r : recs) {
        const auto num = [&](const char* k, double d) {
            const auto it = r.find(k);
            return it == r.end() ? d : it->second;
        };
        GemmTuneEntry e;
        e.M = (i64)num("M", 0);
        e.N = (i64)num("N", 0);
        e.K = (i64)num("K", 0);
        e.k_tiled = num("k_tiled", 0) != 0;
        e.big_rows = (i64)num("big_rows", -1);
        e.group_m = (int)num("group_m", 0);
        e.split = num("split", 0) != 0;
        e.tile = (int)num("tile", PHI_PLAN_TILE_AUTO);
        e.measured_us = num("us", 0);
        e.tops = num("tops", 0);
        if (e.M <= 0 || e.N <= 0 || e.K <= 0) return false;
        items.push_back(e);
    }
    items_.clear();
    for (const GemmTuneEntry& e : items) put(e);
    return true;
}

bool GemmTuneStore::save(const std::string& path) const {
    const std::string tmp = path + ".tmp";
    FILE* f = fopen(tmp.c_str(), "wb");
    if (!f) return false;
    bool ok = fprintf(f, "{\"version\": 1, \"plans\": [") > 0;
    for (size_t i = 0; i < items_.size(); i++) {
        const GemmTuneEntry& e = items_[i];
        ok = ok && fprintf(f,
                           "%s\n  {\"M\": %lld, \"N\": %lld, \"K\": %lld, \"k_tiled\": %d, \"big_rows\": %lld, "
                           "\"group_m\": %d, \"split\": %d, \"tile\": %d, \"us\": %.3f, \"tops\": %.1f}",
                           i ? "," : "", (long long)e.M, (long long)e.N, (long long)e.K, e.k_tiled ? 1 : 0,
                           (long long)e.big_rows, e.group_m, e.split ? 1 : 0, e.tile, e.measured_us, e.tops) > 0;
    }
    ok = ok && fprintf(f, "\n]}\n") > 0;
    ok = (fclose(f) == 0) && ok;
    return ok && std::rename(tmp.c_str(), path.c_str()) == 0;
}

void GemmTuneStore::put(const GemmTuneEntry& e) {
    for (GemmTuneEntry& x : items_)
        if (x.M == e.M && x.N == e.N && x.K == e.K && x.k_tiled == e.k_tiled) {
            x = e;
            return;
        }
    items_.push_back(e);
}

const GemmTuneEntry* GemmTuneStore::get(i64 M, i64 N, i64 K, bool k_tiled) const {
    for (const GemmTuneEntry& x : items_)
        if (x.M == M && x.N == N && x.K == K && x.k_tiled == k_tiled) return &x;
    return nullptr;
}

void GemmTuneStore::apply() const {
    for (const GemmTuneEntry& e : items_) {
        const phi_gemm_plan p{e.big_rows, e.group_m, e.split ? 1 : 0, e.tile, 0};
        if (phi_hip_gemm_plan_set(e.M, e.N, e.K, e.k_tiled ? 1 : 0, &p) != PHI_OK)
            throw MediaError(std::string("gemm tuning table: ") + phi_hip_last_error());
    }
}

namespace {

// A shape's table entry taken out for a sweep and put back afterwards.
struct PlanHold {
    i64 M, N, K;
    int kt;
    phi_gemm_plan saved{};
    int had = 0;
    PlanHold(i64 m, i64 n, i64 k, int t) : M(m), N(n), K(k), kt(t) {
        phi_hip_gemm_plan_get(M, N, K, kt, &saved, &had);
        phi_hip_gemm_plan_set(M, N, K, kt, nullptr);
    }
    ~PlanHold() { phi_hip_gemm_plan_set(M, N, K, kt, had ? &saved : nullptr); }
};

}  // namespace

// The sweep of core/kernels/autotune.cpp:264-334 over this library's plans.
GemmTuneResult autotune_int8_gemm(ComputeContext& ctx, i64 M, i64 N, i64 K, int iters, bool k_tiled) {
    GemmTuneResult r;
    try {
        if (M <= 0 || N <= 0 || K <= 0) throw MediaError("autotune: empty problem");
        if (K % 256 != 0 || N % 8 != 0)
            throw MediaError("autotune: the persistent GEMM's plans need K % 256 == 0 and N % 8 == 0");
        if (iters < 1) iters = 1;
        const int kt = k_tiled ? 1 : 0;
        PlanHold hold(M, N, K, kt);
        // Seeded operands: uniform int8 codes, scales in [0.002, 0.05), a bf16 bias.
        std::mt19937 rng(20261202u);
        std::uniform_int_distribution<int> code(-127, 127);
        std::uniform_real_distribution<float> scl(0.002f, 0.05f), bia(-0.05f, 0.05f);
        std::vector<int8_t> a((size_t)(M * K)), b((size_t)(N * K));
        std::vector<float> sa((size_t)M), sb((size_t)N);
        std::vector<uint16_t> bias((size_t)N);
        for (auto& v : a) v = (int8_t)code(rng);
        for (auto& v : b) v = (int8_t)code(rng);
        for (auto& v : sa) v = scl(rng);
        for (auto& v : sb) v = scl(rng);
        for (auto& v : bias) {
            const float f = bia(rng);
            uint32_t u;
            memcpy(&u, &f, 4);
            v = (uint16_t)(u >> 16);
        }
        const u64 ab = (u64)(M * K), bb = (u64)(N * K), cb = (u64)(M * N) * 2;
        const u64 o_a = 0, o_b = up256(ab), o_akt = o_b + up256(bb), o_bkt = o_akt + (kt ? up256(ab) : 0),
                  o_sa = o_bkt + (kt ? up256(bb) : 0), o_sb = o_sa + up256((u64)M * 4),
                  o_bias = o_sb + up256((u64)N * 4), o_c = o_bias + up256((u64)N * 2), o_c32 = o_c + up256(cb),
                  total = o_c32 + up256((u64)(M * N) * 4);
        Scratch buf(ctx, total);
        ctx.upload(buf.b, a.data(), ab, o_a);
        ctx.upload(buf.b, b.data(), bb, o_b);
        ctx.upload(buf.b, sa.data(), (u64)M * 4, o_sa);
        ctx.upload(buf.b, sb.data(), (u64)N * 4, o_sb);
        ctx.upload(buf.b, bias.data(), (u64)N * 2, o_bias);
        const int8_t* A = (const int8_t*)buf.at(o_a);
        const int8_t* B = (const int8_t*)buf.at(o_b);
        if (kt) {
            ctx.check(phi_hip_pack_k_tiled(ctx.stream(), A, K, M, K, (int8_t*)buf.at(o_akt)), "pack_k_tiled");
            ctx.check(phi_hip_pack_k_tiled(ctx.stream(), B, K, N, K, (int8_t*)buf.at(o_bkt)), "pack_k_tiled");
            A = (const int8_t*)buf.at(o_akt);
            B = (const int8_t*)buf.at(o_bkt);
        }
        auto gemm = [&](bool raw) {
            const float* sA = raw ? nullptr : (const float*)buf.at(o_sa);
            const float* sB = raw ? nullptr : (const float*)buf.at(o_sb);
            const void* bz = raw ? nullptr : (const void*)buf.at(o_bias);
            void* C = (void*)buf.at(raw ? o_c32 : o_c);
            const int cd = raw ? PHI_I32 : PHI_BF16;
            ctx.check(kt ? phi_hip_i8_gemm_kt(ctx.stream(), A, B, sA, sB, 0, bz, PHI_BF16, C, cd, N, M, N, K)
                         : phi_hip_i8_gemm(ctx.stream(), A, K, B, K, sA, sB, 0, bz, PHI_BF16, C, cd, N, M, N, K, nullptr,
                                           0),
                      "autotune gemm");
        };
        // The default plan: its accumulators on sampled rows against host
        // integer sums, and its bf16 output as every candidate's reference.
        gemm(true);
        gemm(false);
        ctx.submit();
        const i64 samples[] = {0, M / 3, M / 2, M - 1};
        std::vector<int32_t> row((size_t)N);
        r.default_exact = true;
        for (const i64 m : samples) {
            ctx.download(buf.b, row.data(), (u64)N * 4, o_c32 + (u64)(m * N) * 4);
            for (i64 n = 0; n < N; n++) {
                int64_t acc = 0;
                for (i64 k = 0; k < K; k++) acc += (int64_t)a[(size_t)(m * K + k)] * b[(size_t)(n * K + k)];
                if (acc != row[(size_t)n]) r.default_exact = false;
            }
        }
        std::vector<uint16_t> ref((size_t)(M * N)), got((size_t)(M * N));
        ctx.download(buf.b, ref.data(), cb, o_c);

        // Candidates: the square plan at the cost model's 256-row count and
        // its neighbours, all rows, group heights 2, 4, 8, and one or two
        // launches where both tile sizes run; with K % 512 == 0, also 272 x
        // 192 tiles at each group height.
        phi_gemm_plan def{};
        ctx.check(phi_hip_gemm_plan_get(M, N, K, kt, &def, nullptr), "gemm_plan_get");
        std::vector<i64> rows_opts{def.big_rows};
        for (const i64 v : {def.big_rows - 256, def.big_rows + 256, M})
            if (v >= 0 && v <= M && (v % 256 == 0 || v == M) &&
                std::find(rows_opts.begin(), rows_opts.end(), v) == rows_opts.end())
                rows_opts.push_back(v);
        hipEvent_t e0, e1;
        if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)
            throw MediaError("autotune: event creation failed");
        struct Events {
            hipEvent_t a, b;
            ~Events() {
                (void)hipEventDestroy(a);
                (void)hipEventDestroy(b);
            }
        } events{e0, e1};
        std::vector<phi_gemm_plan> cands;
        for (const i64 big : rows_opts)
            for (const int gm : {2, 4, 8})
                for (const int split : {0, 1})
                    if (!split || (big > 0 && big < M)) cands.push_back({big, gm, split, PHI_PLAN_TILE_SQUARE, 0});
        if (K % 512 == 0)
            for (const int gm : {2, 4, 8}) cands.push_back({def.big_rows, gm, 0, PHI_PLAN_TILE_272, 0});
        double best_us = 1e300;
        for (const phi_gemm_plan& p : cands) {
            ctx.check(phi_hip_gemm_plan_set(M, N, K, kt, &p), "gemm_plan_set");
            gemm(false);  // untimed
            if (hipEventRecord(e0, ctx.stream()) != hipSuccess) throw MediaError("autotune: event record");
            for (int i = 0; i < iters; i++) gemm(false);
            if (hipEventRecord(e1, ctx.stream()) != hipSuccess || hipEventSynchronize(e1) != hipSuccess)
                throw MediaError("autotune: event wait");
            float ms = 0.0f;
            (void)hipEventElapsedTime(&ms, e0, e1);
            GemmTuneEntry e;
            e.M = M, e.N = N, e.K = K, e.k_tiled = k_tiled;
            e.big_rows = p.big_rows, e.group_m = p.group_m, e.split = p.split != 0, e.tile = p.tile;
            e.measured_us = (double)ms * 1e3 / iters;
            e.tops = 2.0 * (double)M * (double)N * (double)K / (e.measured_us * 1e-6) / 1e12;
            ctx.download(buf.b, got.data(), cb, o_c);
            const bool exact = memcmp(got.data(), ref.data(), (size_t)cb) == 0;
            if (exact) r.exact_matches++;
            r.tried.push_back(e);
            if (exact && e.measured_us < best_us) {
                best_us = e.measured_us;
                r.best = e;
            }
        }
        if (best_us == 1e300) throw MediaError("autotune: no candidate reproduced the default plan's output");
        r.ok = r.default_exact;
        if (!r.default_exact) r.error = "autotune: the default plan's accumulators differ from the host integer GEMM";
    } catch (const std::exception& e) {
        r.ok = false;
        r.error = e.what();
    }
    return r;
}

// core/kernels/w4a8_expand.cpp:263-303
void dispatch_w4a8_expand(ComputeContext& ctx, const W4a8ExpandArgs& a) {
    if (a.rows <= 0 || a.k <= 0) return;
    if (!a.pool || !a.q || !a.s) throw MediaError("w4a8_expand: missing binding");
    phi_w4a8_weight w{};
    w.codes = (const uint8_t*)cat(a.pool, a.codes_off);
    w.codes_row_bytes = a.codes_row_bytes;
    w.s_rel = cat(a.pool, a.srel_off);
    w.s_rel_dtype = phi_rel_dtype(a.rel_dtype);
    w.srel_row_bytes = a.srel_row_bytes;
    w.s_channel = a.has_channel_scale ? (const float*)cat(a.pool, a.sch_off) : nullptr;
    w.sch_scalar = 0;
    w.codebook = a.has_codebook ? (const float*)cat(a.pool, a.cb_off) : nullptr;
    w.correction = nullptr;
    w.rows = a.rows;
    w.k = a.k;
    w.group = a.group;
    w.layout = a.layout == CodeLayout::Nibble4 ? 0 : 1;
    ctx.check(phi_hip_w4a8_expand(ctx.stream(), &w, (int8_t*)at(a.q, a.q_off), (float*)at(a.s, a.s_off)),
              "w4a8_expand");
}

// core/models/model_common.cpp:1363-1412 (int8 branch)
void linear_gemm(GpuCtx& g, const QuantLinear& w, const GpuAlloc& x, i64 m, i64 k, const GpuAlloc& out,
                 const GpuAlloc& q8, const GpuAlloc& s8) {
    if (w.k != k)
        throw MediaError("linear_gemm: K mismatch (weight " + std::to_string(w.k) + ", shape " + std::to_string(k) +
                         ")");
    if (w.dense()) throw MediaError("linear_gemm: dense float weights are not served by the int8 library");
    if (!w.w || !w.scale) throw MediaError("linear_gemm: the int8 weight is empty");
    if (!q8 || !s8) throw MediaError("linear_gemm: the int8 path needs activation scratch");
    if (!g.ctx) throw MediaError("linear_gemm: no compute context");
    const void* xp = cat(x.res, x.off);
    const float* sw = (const float*)cat(w.scale.res, w.scale.off);
    int8_t* qp = (int8_t*)at(q8.res, q8.off);
    float* sp = (float*)at(s8.res, s8.off);
    if (w.k_tiled) {
        // The prologue writes q8 K-tiled and the GEMM reads both operands that
        // way: the same fp32 output as the row-major weight's path below.
        if (x.bytes < (u64)m * (u64)k * 4 || out.bytes < (u64)m * (u64)w.n * 4 || q8.bytes < (u64)m * (u64)k ||
            s8.bytes < (u64)m * 4)
            throw MediaError("linear_gemm: a buffer is smaller than the [" + std::to_string(m) + ", " +
                             std::to_string(k) + "] x [" + std::to_string(w.n) + "] linear needs");
        g.ctx->check(phi_hip_q8_linear_kt(g.ctx->stream(), xp, PHI_F32, k, m, k, (const int8_t*)cat(w.w.res, w.w.off),
                                          sw, 0, nullptr, PHI_F32, w.n, at(out.res, out.off), PHI_F32, w.n, qp, sp,
                                          PHI_ROUND_HALF_AWAY),
                     "linear_gemm");
        return;
    }
    // A row-major weight: the reference's rotate+quantise (dispatch_quant_convrot)
    // then int8 GEMM (dispatch_int8_gemm), fused in one call that writes the
    // scratch q8 K-tiled where the 272 x 192 plan takes the shape; the output
    // is the same, bit for bit.
    g.ctx->check(phi_hip_q8_linear_kq(g.ctx->stream(), xp, PHI_F32, k, m, k, (const int8_t*)cat(w.w.res, w.w.off), k,
                                      sw, 0, nullptr, PHI_F32, w.n, at(out.res, out.off), PHI_F32, w.n, qp, sp,
                                      PHI_ROUND_HALF_AWAY, nullptr, 0),
                 "linear_gemm");
}

}  // namespace phi::media
