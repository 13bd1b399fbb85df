// C++ host layer: the reference's dispatch surface over the C ABI.
#include "phi_media.hpp"

#include "phi_qlinear.h"
#include "safetensors.hpp"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <map>
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

// ---------------------------------------------------------------- GpuArena

GpuArena::GpuArena(ComputeContext& ctx, u64 bytes) {
    init(&ctx, bytes);
    chunks_.push_back(ctx.create_device_buffer(bytes));
    capacity_ = bytes;
}

GpuArena::~GpuArena() { release_chunks(); }

void GpuArena::init(ComputeContext* ctx, u64 chunk_bytes) {
    ctx_ = ctx;
    if (chunk_bytes) chunk_bytes_ = chunk_bytes;
}

void GpuArena::release_chunks() {
    if (ctx_) {
        // Work still queued may read the chunks: let it finish first.
        (void)hipStreamSynchronize(ctx_->stream());
        for (GpuBuffer* b : chunks_) ctx_->release_buffer(b);
    }
    chunks_.clear();
    cur_ = 0;
    cur_off_ = 0;
    used_ = 0;
    capacity_ = 0;
}

GpuAlloc GpuArena::alloc(u64 bytes, u64 align) {
    if (!ctx_) throw MediaError("arena: not initialised");
    if (align == 0 || (align & (align - 1)) != 0) throw MediaError("arena: alignment must be a power of two");
    const u64 need = bytes ? bytes : 1;
    // The current chunk, then any later chunk (kept from before a reset) that
    // fits, then a new chunk.
    for (size_t c = cur_; c < chunks_.size(); c++) {
        const u64 start = c == cur_ ? cur_off_ : 0;
        const u64 off = (start + align - 1) & ~(align - 1);
        if (off + need <= chunks_[c]->bytes) {
            used_ += (off - (c == cur_ ? cur_off_ : 0)) + need;
            cur_ = c;
            cur_off_ = off + need;
            return GpuAlloc{chunks_[c], off, bytes};
        }
    }
    const u64 size = need > chunk_bytes_ ? need : chunk_bytes_;
    GpuBuffer* b = ctx_->create_device_buffer(size);
    chunks_.push_back(b);
    capacity_ += size;
    cur_ = chunks_.size() - 1;
    cur_off_ = need;
    used_ += need;
    return GpuAlloc{b, 0, bytes};
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

namespace {

bool ends_with_s(const std::string& s, const std::string& suf) {
    return s.size() >= suf.size() && s.compare(s.size() - suf.size(), suf.size(), suf) == 0;
}

// The display-name prefixes ComfyUI and kohya put before the module path, and
// kohya's lora_unet_ / lora_te_ forms where '_' stands for '.'.
std::string strip_display_prefix(std::string s) {
    static const char* prefixes[] = {"model.diffusion_model.", "diffusion_model.", "model.", "unet.", "transformer."};
    for (bool again = true; again;) {
        again = false;
        for (const char* p : prefixes) {
            const size_t n = strlen(p);
            if (s.size() > n && s.compare(0, n, p) == 0) {
                s.erase(0, n);
                again = true;
                break;
            }
        }
    }
    for (const char* p : {"lora_unet_", "lora_te_"}) {
        const size_t n = strlen(p);
        if (s.compare(0, n, p) == 0) {
            s.erase(0, n);
            for (char& c : s)
                if (c == '_') c = '.';
            break;
        }
    }
    if (ends_with_s(s, ".weight")) s.erase(s.size() - 7);
    return s;
}

// A factor names its module with or without the checkpoint's container prefix.
bool target_matches(const std::string& factor, const std::string& want) {
    return factor == want || ends_with_s(want, "." + factor) || ends_with_s(factor, "." + want);
}

}  // namespace

std::string lora_normalize_target(const std::string& key, bool* is_a, bool* is_b) {
    if (is_a) *is_a = false;
    if (is_b) *is_b = false;
    if (ends_with_s(key, ".alpha")) return strip_display_prefix(key.substr(0, key.size() - 6));
    for (const char* m : {".lora_A", ".lora_down"}) {
        const size_t p = key.find(m);
        if (p != std::string::npos) {
            if (is_a) *is_a = true;
            return strip_display_prefix(key.substr(0, p));
        }
    }
    for (const char* m : {".lora_B", ".lora_up"}) {
        const size_t p = key.find(m);
        if (p != std::string::npos) {
            if (is_b) *is_b = true;
            return strip_display_prefix(key.substr(0, p));
        }
    }
    return "";
}

// core/models/lora.cpp:86-181
void LoraSet::add(const std::string& path, float strength) {
    if ((int)files_.size() >= kMaxLoras)
        throw MediaError("LoRA: at most " + std::to_string(kMaxLoras) + " files may be chained");
    SafeTensors st(path);
    File file;
    file.path = path;
    file.strength = strength;
    // A file-wide alpha from the metadata; a per-module "<base>.alpha" overrides it.
    float file_alpha = 0.0f;
    for (const char* key : {"ss_network_alpha", "lora_alpha", "network_alpha"}) {
        const auto it = st.metadata().find(key);
        if (it == st.metadata().end()) continue;
        file_alpha = (float)std::atof(it->second.c_str());
        if (file_alpha > 0) break;
    }
    struct Pending {
        const StTensor* a = nullptr;
        const StTensor* b = nullptr;
        float alpha = 0.0f;
        bool has_alpha = false;
    };
    std::map<std::string, Pending> pending;
    std::vector<std::string> order;
    for (const std::string& name : st.names()) {
        const StTensor& t = st.require(name);
        bool is_a = false, is_b = false;
        const std::string target = lora_normalize_target(name, &is_a, &is_b);
        if (target.empty()) continue;
        auto it = pending.find(target);
        if (it == pending.end()) {
            order.push_back(target);
            it = pending.emplace(target, Pending{}).first;
        }
        Pending& p = it->second;
        if (is_a) {
            p.a = &t;
        } else if (is_b) {
            p.b = &t;
        } else if (ends_with_s(name, ".alpha")) {
            const std::vector<float> v = st.to_f32(t);
            if (!v.empty()) {
                p.alpha = v[0];
                p.has_alpha = true;
            }
        }
    }
    for (const std::string& target : order) {
        const Pending& p = pending[target];
        if (!p.a || !p.b || p.a->shape.size() != 2 || p.b->shape.size() != 2) continue;
        Factor f;
        f.target = target;
        f.rank = p.a->shape[0];
        f.k = p.a->shape[1];
        f.n = p.b->shape[0];
        if (p.b->shape[1] != f.rank || f.rank <= 0 || f.n <= 0 || f.k <= 0) continue;
        const float alpha = p.has_alpha ? p.alpha : (file_alpha > 0 ? file_alpha : (float)f.rank);
        f.scale = strength * alpha / (float)f.rank;
        f.A = st.to_f32(*p.a);
        f.B = st.to_f32(*p.b);
        if ((i64)f.A.size() != f.rank * f.k || (i64)f.B.size() != f.n * f.rank) continue;
        file.factors.push_back(std::move(f));
    }
    if (file.factors.empty()) {
        const size_t slash = path.find_last_of("/\\");
        throw MediaError("LoRA: " + (slash == std::string::npos ? path : path.substr(slash + 1)) +
                         " holds no A/B factor pairs this engine can map");
    }
    files_.push_back(std::move(file));
    paths_.push_back(path);
}

int LoraSet::deltas_for(const std::string& target, i64 n, i64 k, std::vector<Delta>* out) const {
    int found = 0;
    for (const File& file : files_)
        for (const Factor& f : file.factors) {
            if (!target_matches(f.target, target) || f.n != n || f.k != k) continue;
            if (out) out->push_back(Delta{f.n, f.k, f.rank, f.scale, f.A.data(), f.B.data()});
            found++;
        }
    return found;
}

int LoraSet::deltas_for_rows(const std::string& target, i64 row0, i64 rows, i64 k, std::vector<Delta>* out) const {
    int found = 0;
    if (rows <= 0 || k <= 0 || row0 < 0) return 0;
    for (const File& file : files_)
        for (const Factor& f : file.factors) {
            if (!target_matches(f.target, target) || f.k != k || row0 + rows > f.n) continue;
            if (out) out->push_back(Delta{f.n, f.k, f.rank, f.scale, f.A.data(), f.B.data()});
            found++;
        }
    return found;
}

bool LoraSet::touches(const std::string& target) const {
    for (const File& file : files_)
        for (const Factor& f : file.factors)
            if (target_matches(f.target, target)) return true;
    return false;
}

namespace {

// w[o][i] += (scale * B[row0 + o][r]) * A[r][i], r ascending, 0 entries of B skipped
// (core/models/lora.cpp:182-201).
void fold_rows_host(const LoraSet::Delta& d, float* w, i64 row0, i64 rows, i64 k) {
    for (i64 o = 0; o < rows; o++) {
        float* wrow = w + o * k;
        const float* brow = d.b + (row0 + o) * d.rank;
        for (i64 r = 0; r < d.rank; r++) {
            const float br = brow[r];
            if (br == 0.0f) continue;
            const float s = d.scale * br;
            const float* arow = d.a + r * k;
            for (i64 i = 0; i < k; i++) wrow[i] += s * arow[i];
        }
    }
}

}  // namespace

int LoraSet::apply(const std::string& target, float* w, i64 n, i64 k) const {
    if (!w || n <= 0 || k <= 0) return 0;
    std::vector<Delta> ds;
    deltas_for(target, n, k, &ds);
    for (const Delta& d : ds) fold_rows_host(d, w, 0, n, k);
    return (int)ds.size();
}

int LoraSet::apply_rows(const std::string& target, float* w, i64 row0, i64 rows, i64 k) const {
    if (!w) return 0;
    std::vector<Delta> ds;
    deltas_for_rows(target, row0, rows, k, &ds);
    for (const Delta& d : ds) fold_rows_host(d, w, row0, rows, k);
    return (int)ds.size();
}

// core/models/model_common.cpp:1587-1652
LoraTail load_lora_tail(GpuCtx& g, GpuArena& arena, const std::vector<LoraModule>& mods, i64 n, i64 k) {
    LoraTail t;
    if (mods.empty() || n <= 0 || k <= 0) return t;
    std::vector<std::pair<const LoraModule*, LoraSet::Delta>> found;
    i64 rank = 0;
    for (const LoraModule& m : mods) {
        if (!m.lora || m.n <= 0) continue;
        if (m.row0 < 0 || m.row0 + m.n > n)
            throw MediaError("LoRA correction: module " + m.base + " covers rows [" + std::to_string(m.row0) + ", " +
                             std::to_string(m.row0 + m.n) + ") of a " + std::to_string(n) + "-row weight");
        std::vector<LoraSet::Delta> d;
        m.lora->deltas_for(m.base, m.n, k, &d);
        for (const LoraSet::Delta& f : d) {
            found.push_back({&m, f});
            rank += f.rank;
        }
    }
    if (rank <= 0) return t;
    if (rank > kLoraRankBound)
        throw MediaError("LoRA correction: the factors matching this module need a " + std::to_string(rank) +
                         "-wide correction, past the " + std::to_string(kLoraRankBound) +
                         " the activation plans reserve (kLoraRankBound)");
    if (!g.ctx) throw MediaError("load_lora_tail: no compute context");
    // A stacked along the rank axis; B likewise, each factor's scale folded into
    // its own columns and its rows placed at its module's output rows.
    std::vector<float> a((size_t)rank * (size_t)k, 0.0f), b((size_t)n * (size_t)rank, 0.0f);
    i64 r0 = 0;
    for (const auto& [mod, f] : found) {
        memcpy(&a[(size_t)r0 * (size_t)k], f.a, (size_t)f.rank * (size_t)k * 4);
        for (i64 o = 0; o < f.n; o++) {
            float* brow = &b[(size_t)(mod->row0 + o) * (size_t)rank + (size_t)r0];
            const float* src = f.b + o * f.rank;
            for (i64 r = 0; r < f.rank; r++) brow[r] = f.scale * src[r];
        }
        r0 += f.rank;
    }
    t.at = arena.alloc((u64)a.size() * 4);
    t.bt = arena.alloc((u64)b.size() * 4);
    g.ctx->upload(t.at.res, a.data(), a.size() * 4, t.at.off);
    g.ctx->upload(t.bt.res, b.data(), b.size() * 4, t.bt.off);
    t.rank = rank;
    t.n = n;
    t.k = k;
    t.active = true;
    return t;
}

LoraTail load_lora_tail(GpuCtx& g, GpuArena& arena, const std::string& base, const LoraSet* lora, i64 n, i64 k) {
    if (!lora) return LoraTail{};
    return load_lora_tail(g, arena, {LoraModule{base, 0, n, lora}}, n, k);
}

namespace {

// The conditions of the reference's device-expand path (w4a8_plan_of,
// core/models/model_common.cpp:605-680), each checked rather than trusted.
struct W4a8Plan {
    CodeLayout layout = CodeLayout::Nibble4;
    const StTensor* codes = nullptr;
    const StTensor* srel = nullptr;
    const StTensor* sch = nullptr;
    const StTensor* codebook = nullptr;
    const StTensor* correction = nullptr;
    i64 n = 0, k = 0, group = 0, srel_row_bytes = 0;
    RelDType rel_dtype = RelDType::F32;
};

std::string w4a8_plan_of(const SafeTensors& st, const StTensor& t, W4a8Plan* out) {
    const SafeTensors::WeightLayout L = st.weight_layout(t.name);
    const std::string& f = L.spec.format;
    const bool six = f == "w6a8_int8" || f == "w6a8";
    if (t.shape.size() != 2 || (t.dtype != StDType::I8 && t.dtype != StDType::U8)) return "codes are not a 2-D byte tensor";
    if (!L.spec.convrot) return "the weight is not convrot-rotated";
    if (!L.rel_scale || L.rel_scale->shape.size() != 2) return "no 2-D weight_s_rel table";
    RelDType rdt;
    switch (L.rel_scale->dtype) {
        case StDType::F32: rdt = RelDType::F32; break;
        case StDType::F16: rdt = RelDType::F16; break;
        case StDType::BF16: rdt = RelDType::BF16; break;
        case StDType::F8_E4M3: rdt = RelDType::F8_E4M3; break;
        case StDType::F8_E5M2: rdt = RelDType::F8_E5M2; break;
        case StDType::U8: rdt = RelDType::U8_E4M3; break;
        default: return std::string("weight_s_rel dtype ") + st_dtype_name(L.rel_scale->dtype) + " is not decodable";
    }
    const i64 n = t.shape[0], k = st.logical_cols(t);
    const i64 group = L.group;
    const i64 per = six ? 4 : 2;
    if (group <= 0 || group % per != 0 || k % group != 0) return "group " + std::to_string(group) + " does not divide K";
    const i64 need = six ? (k / 2 + k / 4) : k / 2;
    if ((i64)t.row_bytes() < need) return "code rows are shorter than K needs";
    if (L.rel_scale->shape[0] != n || L.rel_scale->shape[1] != k / group) return "weight_s_rel is not [N, K/group]";
    if (six && L.codebook) return "a six-bit weight with a codebook";
    if (!six && L.codebook && (L.codebook->dtype != StDType::F32 || L.codebook->numel != 16))
        return "the codebook is not 16 fp32 levels";
    if (L.row_scale && (L.row_scale->dtype != StDType::F32 || (L.row_scale->numel != 1 && L.row_scale->numel != n)))
        return "the channel scale is not fp32 [N] or [1]";
    if (L.correction) {
        const i64 cg = L.correction->shape.empty() ? 0 : L.correction->shape[0];
        const i64 cn = L.correction->shape.size() > 1 ? L.correction->shape[1] : 0;
        if (L.correction->dtype != StDType::F32 || cg != k / group || cn != n)
            return "weight_correction is not fp32 [K/group, N]";
    }
    out->layout = six ? CodeLayout::Packed6 : CodeLayout::Nibble4;
    out->codes = &t;
    out->srel = L.rel_scale;
    out->sch = L.row_scale;
    out->codebook = six ? nullptr : L.codebook;
    out->correction = L.correction;
    out->n = n;
    out->k = k;
    out->group = group;
    out->srel_row_bytes = (i64)L.rel_scale->row_bytes();
    out->rel_dtype = rdt;
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
    Scratch(ComputeContext& c, u64 bytes) : ctx(c), b(c.create_device_buffer(bytes)) {}
    ~Scratch() {
        (void)hipStreamSynchronize(ctx.stream());
        ctx.release_buffer(b);
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

// What the device decodes: int8 codes times their row scale, f16 / bf16 / f32
// widened, or a bare packed int4 (two signed nibbles a byte) times its row scale
// (SafeTensors::dequant_rows, core/host/st.cpp:601-700).
struct Decodable {
    int dtype = -1;  // PHI_I8 / PHI_F16 / PHI_BF16 / PHI_F32, or -2 for I4
    const StTensor* scale = nullptr;
};

Decodable decodable(const SafeTensors& st, const StTensor& t) {
    Decodable d;
    const SafeTensors::WeightLayout L = st.weight_layout(t.name);
    switch (t.dtype) {
        case StDType::F32: d.dtype = PHI_F32; break;
        case StDType::F16: d.dtype = PHI_F16; break;
        case StDType::BF16: d.dtype = PHI_BF16; break;
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
            d.dtype = -2;
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
    const bool i4 = d.dtype == -2;
    const u64 src_row = i4 ? (u64)((k + 1) / 2) : t.row_bytes();
    if ((u64)n * src_row > t.nbytes) throw MediaError("'" + t.name + "' holds fewer rows than its shape says");
    const u64 slab = (u64)std::max<i64>(1, std::min<i64>(n, (64ll << 20) / std::max<i64>(k * 4, 1)));
    // Device copies: the row scales (host-decoded from their table), and every
    // LoRA factor's A and B once.
    std::vector<float> scales;
    if (d.scale) {
        scales.resize((size_t)n);
        for (i64 r = 0; r < n; r++) scales[(size_t)r] = st.row_scale_value(*d.scale, r);
    }
    const u64 o_src = 0, o_f32 = up256(slab * src_row), o_sc = o_f32 + up256(slab * (u64)k * 4),
              total = o_sc + up256((u64)n * 4 + 4);
    Scratch work(ctx, total);
    if (!scales.empty()) ctx.upload(work.b, scales.data(), scales.size() * 4, o_sc);
    float* f32 = (float*)work.at(o_f32);
    for (i64 r0 = 0; r0 < n; r0 += (i64)slab) {
        const i64 rows = std::min<i64>((i64)slab, n - r0);
        ctx.upload(work.b, t.data + (u64)r0 * src_row, (u64)rows * src_row, o_src);
        const bool sc = d.scale != nullptr;
        const bool sc1 = sc && d.scale->numel == 1;
        ctx.check(phi_hip_dequant_rows(ctx.stream(), (const void*)work.at(o_src), i4 ? PHI_I4 : d.dtype, rows, k,
                                       (int64_t)(i4 ? src_row : src_row / st_dtype_bytes(t.dtype)),
                                       sc ? (const float*)work.at(o_sc) + (sc1 ? 0 : r0) : nullptr, sc1 ? 1 : 0, f32,
                                       k),
                  "dequant_rows");
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
void expand_grouped(GpuCtx& g, const StTensor& t, const W4a8Plan& pl, int8_t* q, float* s, const SafeTensors& st) {
    ComputeContext& ctx = *g.ctx;
    const i64 n = pl.n;
    const u64 cb = checked_mul((u64)n, t.row_bytes(), "w4a8 codes"), sb = pl.srel->nbytes, hb = pl.sch ? (u64)n * 4 : 0,
              kb = pl.codebook ? 64 : 0, rb = pl.correction ? pl.correction->nbytes : 0;
    const u64 o_codes = 0, o_srel = up256(cb), o_sch = o_srel + up256(sb), o_cb = o_sch + up256(hb),
              o_corr = o_cb + up256(kb), total = o_corr + up256(rb);
    Scratch stage(ctx, total);
    ctx.upload(stage.b, t.data, cb, o_codes);
    ctx.upload(stage.b, pl.srel->data, sb, o_srel);
    if (pl.sch) {
        std::vector<float> v((size_t)n);
        for (i64 r = 0; r < n; r++) v[(size_t)r] = st.row_scale_value(*pl.sch, r);  // a [1] table broadcasts
        ctx.upload(stage.b, v.data(), hb, o_sch);
    }
    if (pl.codebook) ctx.upload(stage.b, pl.codebook->data, kb, o_cb);
    if (pl.correction) ctx.upload(stage.b, pl.correction->data, rb, o_corr);
    phi_w4a8_weight w{};
    w.codes = (const uint8_t*)stage.at(o_codes);
    w.codes_row_bytes = (int64_t)t.row_bytes();
    w.s_rel = (const void*)stage.at(o_srel);
    w.s_rel_dtype = phi_rel_dtype(pl.rel_dtype);
    w.srel_row_bytes = pl.srel_row_bytes;
    w.s_channel = pl.sch ? (const float*)stage.at(o_sch) : nullptr;
    w.codebook = pl.codebook ? (const float*)stage.at(o_cb) : nullptr;
    w.correction = pl.correction ? (const float*)stage.at(o_corr) : nullptr;
    w.rows = n;
    w.k = pl.k;
    w.group = pl.group;
    w.layout = pl.layout == CodeLayout::Nibble4 ? 0 : 1;
    ctx.check(phi_hip_w4a8_expand(ctx.stream(), &w, q, s), "w4a8_expand");
    ctx.submit();
}

int8_t* dev_i8(const GpuAlloc& a, u64 off = 0) { return (int8_t*)(a.res->base + a.off + off); }
float* dev_f32(const GpuAlloc& a, u64 off = 0) { return (float*)(a.res->base + a.off + off); }

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
    QuantLinear q;
    q.n = n;
    q.k = k;
    if (st.is_plain_int8(t) && !touched) {
        // Shipped int8 tensorwise: the codes verbatim, one fp32 scale per row.
        if (t.nbytes != nk) throw MediaError("load_quant_linear: '" + base + ".weight' is not [N, K] int8");
        const std::vector<float> s = weight_scales(st, base, n);
        q.w = alloc(nk);
        g.ctx->upload(q.w.res, t.data, t.nbytes, q.w.off);
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
        W4a8Plan pl;
        const std::string why = w4a8_plan_of(st, t, &pl);
        if (!why.empty()) throw MediaError("load_quant_linear: '" + base + "' (" + L.spec.format + "): " + why);
        q.w = alloc(nk);
        q.scale = alloc((u64)n * 4);
        expand_grouped(g, t, pl, dev_i8(q.w), dev_f32(q.scale), st);
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
    requant_rows_device(g, st, t, n, k, plan, dev_i8(q.w), dev_f32(q.scale));
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
        for (int i = 0; i < 3; i++)
            g.ctx->upload(q.w.res, ts[i]->data, ts[i]->nbytes, q.w.off + (u64)row0[i] * (u64)k);
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
    for (int i = 0; i < 3; i++) {
        const StTensor& t = *ts[i];
        const SafeTensors::WeightLayout L = st.weight_layout(t.name);
        int8_t* qi = dev_i8(q.w, (u64)row0[i] * (u64)k);
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
            W4a8Plan pl;
            const std::string why = w4a8_plan_of(st, t, &pl);
            if (!why.empty()) throw MediaError("load_quant3_linear: '" + bases[i] + "' (" + L.spec.format + "): " + why);
            expand_grouped(g, t, pl, qi, si, st);
            continue;
        }
        requant_rows_device(g, st, t, rows_of[i], k, plan, qi, si);
    }
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
        W4a8Plan pl;
        if (w4a8_plan_of(st, t, &pl).empty()) {
            out.w = arena.alloc(nk);
            out.s = arena.alloc((u64)out.n * 4);
            expand_grouped(g, t, pl, dev_i8(out.w), dev_f32(out.s), st);
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
    QuantConvrotArgs qa;
    qa.x = x.res;
    qa.x_offset = x.off;
    qa.q = q8.res;
    qa.q_offset = q8.off;
    qa.s = s8.res;
    qa.s_offset = s8.off;
    qa.rows = m;
    qa.K = k;
    dispatch_quant_convrot(*g.ctx, qa);

    Int8GemmArgs ga;
    ga.a = q8.res;
    ga.a_offset = q8.off;
    ga.b = w.w.res;
    ga.b_offset = w.w.off;
    ga.sa = s8.res;
    ga.sa_offset = s8.off;
    ga.sb = w.scale.res;
    ga.sb_offset = w.scale.off;
    ga.c = out.res;
    ga.c_offset = out.off;
    ga.M = m;
    ga.N = w.n;
    ga.K = k;
    dispatch_int8_gemm(*g.ctx, ga);
}

}  // namespace phi::media
