// C++ host layer: the reference's dispatch surface over the C ABI.
#include "phi_media.hpp"

#include "phi_qlinear.h"
#include "safetensors.hpp"

#include <cstring>
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

GpuArena::GpuArena(ComputeContext& ctx, u64 bytes) : ctx_(ctx) { buf_ = ctx_.create_device_buffer(bytes); }

GpuArena::~GpuArena() { ctx_.release_buffer(buf_); }

GpuAlloc GpuArena::alloc(u64 bytes) {
    const u64 off = (used_ + 255) & ~(u64)255;
    if (!buf_ || off + bytes > buf_->bytes)
        throw MediaError("arena: " + std::to_string(bytes) + " bytes do not fit (" + std::to_string(used_) + " of " +
                         std::to_string(capacity()) + " used)");
    used_ = off + bytes;
    return GpuAlloc{buf_, off, bytes};
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

// core/models/model_common.cpp:921-1010 (the int8 and device-expand branches)
QuantLinear load_quant_linear(GpuCtx& g, const SafeTensors& st, const std::string& base, GpuArena& into) {
    if (!g.ok()) throw MediaError("load_quant_linear: no compute context");
    const StTensor& t = st.require(base + ".weight");
    if (t.shape.size() != 2) throw MediaError("load_quant_linear: '" + base + ".weight' is not a 2-D matrix");
    const i64 n = t.shape[0], k = st.logical_cols(t);
    QuantLinear q;
    q.n = n;
    q.k = k;
    if (st.is_plain_int8(t)) {
        // Shipped int8 tensorwise: the codes verbatim, one fp32 scale per row.
        const StTensor& sc = st.require(base + ".weight_scale");
        if (sc.numel != n) throw MediaError("weight_scale length mismatch: " + base);
        if (t.nbytes != (u64)(n * k)) throw MediaError("load_quant_linear: '" + base + ".weight' is not [N, K] int8");
        q.w = into.alloc((u64)(n * k));
        g.ctx->upload(q.w.res, t.data, t.nbytes, q.w.off);
        std::vector<float> s((size_t)n);
        for (i64 r = 0; r < n; r++) s[(size_t)r] = st.row_scale_value(sc, r);
        q.scale = into.alloc((u64)n * 4);
        g.ctx->upload(q.scale.res, s.data(), (u64)n * 4, q.scale.off);
        return q;
    }
    const SafeTensors::WeightLayout L = st.weight_layout(t.name);
    if (L.packed) {
        W4a8Plan pl;
        const std::string why = w4a8_plan_of(st, t, &pl);
        if (!why.empty()) throw MediaError("load_quant_linear: '" + base + "' (" + L.spec.format + "): " + why);
        // Stage the stored parts on the device, 256-byte aligned, and expand.
        auto up256 = [](u64 v) { return (v + 255) & ~(u64)255; };
        const u64 cb = (u64)n * t.row_bytes(), sb = pl.srel->nbytes, hb = pl.sch ? (u64)n * 4 : 0,
                  kb = pl.codebook ? 64 : 0, rb = pl.correction ? pl.correction->nbytes : 0;
        const u64 o_codes = 0, o_srel = up256(cb), o_sch = o_srel + up256(sb), o_cb = o_sch + up256(hb),
                  o_corr = o_cb + up256(kb), total = o_corr + up256(rb);
        GpuBuffer* stage = g.ctx->create_device_buffer(total);
        try {
            g.ctx->upload(stage, t.data, cb, o_codes);
            g.ctx->upload(stage, pl.srel->data, sb, o_srel);
            if (pl.sch) {
                std::vector<float> v((size_t)n);
                for (i64 r = 0; r < n; r++) v[(size_t)r] = st.row_scale_value(*pl.sch, r);  // a [1] table broadcasts
                g.ctx->upload(stage, v.data(), hb, o_sch);
            }
            if (pl.codebook) g.ctx->upload(stage, pl.codebook->data, kb, o_cb);
            if (pl.correction) g.ctx->upload(stage, pl.correction->data, rb, o_corr);
            q.w = into.alloc((u64)(n * k));
            q.scale = into.alloc((u64)n * 4);
            phi_w4a8_weight w{};
            w.codes = (const uint8_t*)(stage->base + o_codes);
            w.codes_row_bytes = (int64_t)t.row_bytes();
            w.s_rel = (const void*)(stage->base + o_srel);
            w.s_rel_dtype = phi_rel_dtype(pl.rel_dtype);
            w.srel_row_bytes = pl.srel_row_bytes;
            w.s_channel = pl.sch ? (const float*)(stage->base + o_sch) : nullptr;
            w.codebook = pl.codebook ? (const float*)(stage->base + o_cb) : nullptr;
            w.correction = pl.correction ? (const float*)(stage->base + o_corr) : nullptr;
            w.rows = n;
            w.k = k;
            w.group = pl.group;
            w.layout = pl.layout == CodeLayout::Nibble4 ? 0 : 1;
            g.ctx->check(phi_hip_w4a8_expand(g.ctx->stream(), &w, (int8_t*)at(q.w.res, q.w.off),
                                             (float*)at(q.scale.res, q.scale.off)),
                         "w4a8_expand");
            g.ctx->submit();
        } catch (...) {
            g.ctx->release_buffer(stage);
            throw;
        }
        g.ctx->release_buffer(stage);
        return q;
    }
    if (L.spec.valid && L.spec.format == "convrot_w4a4")
        throw MediaError("load_quant_linear: '" + base + "' is convrot_w4a4: load it with upload_quant_linear_w4a4 "
                         "for the int4 GEMM");
    throw MediaError("load_quant_linear: '" + base + ".weight' is " + st_dtype_name(t.dtype) +
                     (L.spec.valid ? " (" + L.spec.format + ")" : std::string(" without a comfy_quant spec")) +
                     ": the quantized-linear library loads int8_tensorwise, asym_w4a8_int8 and w6a8_int8");
}

// core/models/model_common.cpp:1285-1340 (the verbatim, no-LoRA branch)
I4Upload upload_quant_linear_w4a4(GpuCtx& g, const SafeTensors& st, const std::string& base, GpuArena& arena) {
    if (!g.ok()) throw MediaError("upload_quant_linear_w4a4: no compute context");
    const StTensor& t = st.require(base + ".weight");
    if (t.shape.size() != 2)
        throw MediaError("upload_quant_linear_w4a4: '" + base + ".weight' is not a 2-D matrix");
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
    out.w = arena.alloc((u64)out.n * (u64)packed_k);
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
    if (!g.ok()) throw MediaError("linear_gemm: no compute context");
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
