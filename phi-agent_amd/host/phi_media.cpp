// C++ host layer: the reference's dispatch surface over the C ABI.
#include "phi_media.hpp"

#include "phi_qlinear.h"

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
