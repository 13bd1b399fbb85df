// Test program for the C++ host layer (phi-agent_amd/host/phi_media.hpp), the
// drop-in for the reference's dispatch surface.  It mirrors the reference's own
// in-binary gates (core/bench/media_bench.cpp:110-279: upload, dispatch,
// submit, download, compare with the host arithmetic), but every comparison
// here is bit-exact against the oracle (oracle/oracle.h).  Exit code 0 = pass.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "oracle.h"
#include "phi_media.hpp"

using namespace phi::media;

static int failures = 0;
#define CHECK(cond, ...)                       \
    do {                                       \
        if (!(cond)) {                         \
            printf("FAIL %s:%d ", __FILE__, __LINE__); \
            printf(__VA_ARGS__);               \
            printf("\n");                      \
            failures++;                        \
        }                                      \
    } while (0)

static void test_linear_gemm(ComputeContext& ctx) {
    const i64 m = 67, k = 1024, n = 320;
    std::mt19937 rng(7);
    std::normal_distribution<float> nd(0.0f, 2.0f);
    std::uniform_int_distribution<int> ud(-127, 127);
    std::uniform_real_distribution<float> us(0.001f, 0.01f);
    std::vector<float> x(m * k), sw(n);
    std::vector<int8_t> w(n * k);
    for (auto& v : x) v = nd(rng);
    for (auto& v : w) v = (int8_t)ud(rng);
    for (auto& v : sw) v = us(rng);

    // One arena-like buffer carved into sub-allocations, as GpuArena hands out.
    const u64 off_x = 0, off_w = off_x + m * k * 4, off_s = off_w + n * k, off_q8 = off_s + 4096,
              off_s8 = off_q8 + m * k, off_y = off_s8 + 4096;
    GpuBuffer* pool = ctx.create_device_buffer(off_y + m * n * 4);
    ctx.upload(pool, x.data(), m * k * 4, off_x);
    ctx.upload(pool, w.data(), n * k, off_w);
    ctx.upload(pool, sw.data(), n * 4, off_s);

    GpuCtx g;
    g.ctx = &ctx;
    QuantLinear ql;
    ql.w = GpuAlloc{pool, off_w, (u64)(n * k)};
    ql.scale = GpuAlloc{pool, off_s, (u64)(n * 4)};
    ql.n = n;
    ql.k = k;
    ctx.begin();
    linear_gemm(g, ql, GpuAlloc{pool, off_x, (u64)(m * k * 4)}, m, k, GpuAlloc{pool, off_y, (u64)(m * n * 4)},
                GpuAlloc{pool, off_q8, (u64)(m * k)}, GpuAlloc{pool, off_s8, (u64)(m * 4)});
    ctx.submit();

    std::vector<float> y(m * n), s8(m);
    std::vector<int8_t> q8(m * k);
    ctx.download(pool, y.data(), m * n * 4, off_y);
    ctx.download(pool, q8.data(), m * k, off_q8);
    ctx.download(pool, s8.data(), m * 4, off_s8);

    std::vector<float> yo(m * n), so(m);
    std::vector<int8_t> qo(m * k);
    orc_q8_linear(x.data(), ORC_F32, m, k, w.data(), sw.data(), 0, nullptr, -1, n, ORC_ROUND_HALF_AWAY,
                  yo.data(), ORC_F32, qo.data(), so.data(), nullptr);
    CHECK(memcmp(q8.data(), qo.data(), q8.size()) == 0, "linear_gemm: int8 activations differ");
    CHECK(memcmp(s8.data(), so.data(), s8.size() * 4) == 0, "linear_gemm: activation scales differ");
    CHECK(memcmp(y.data(), yo.data(), y.size() * 4) == 0, "linear_gemm: fp32 outputs differ");
    ctx.release_buffer(pool);
    printf("linear_gemm %lldx%lldx%lld: %s\n", (long long)m, (long long)n, (long long)k,
           failures ? "mismatch" : "bit-exact");
}

static void test_w4a8_expand(ComputeContext& ctx) {
    const i64 rows = 48, k = 512, group = 64, groups = k / group;
    std::mt19937 rng(3);
    std::uniform_int_distribution<int> ub(0, 255);
    std::uniform_real_distribution<float> ur(0.5f, 20.0f), uc(0.001f, 0.01f);
    std::vector<uint8_t> codes(rows * k / 2);
    for (auto& v : codes) v = (uint8_t)ub(rng);
    std::vector<uint16_t> srel(rows * groups);  // fp16 relative scales
    for (auto& v : srel) {
        const float f = ur(rng);
        uint32_t b;
        memcpy(&b, &f, 4);
        const int e = (int)((b >> 23) & 255) - 127 + 15;
        v = (uint16_t)((e << 10) | ((b >> 13) & 0x3ff));  // truncation onto fp16 (values are exact)
    }
    std::vector<float> sch(rows), cb(16);
    for (auto& v : sch) v = uc(rng);
    for (int i = 0; i < 16; i++) cb[i] = (float)(i - 8) * 0.75f + 0.125f;

    const u64 o_codes = 0, o_srel = 256 * ((codes.size() + 255) / 256),
              o_sch = o_srel + 256 * ((srel.size() * 2 + 255) / 256), o_cb = o_sch + 256 * ((rows * 4 + 255) / 256),
              o_q = o_cb + 256, o_s = o_q + rows * k;
    GpuBuffer* pool = ctx.create_device_buffer(o_s + rows * 4);
    ctx.upload(pool, codes.data(), codes.size(), o_codes);
    ctx.upload(pool, srel.data(), srel.size() * 2, o_srel);
    ctx.upload(pool, sch.data(), rows * 4, o_sch);
    ctx.upload(pool, cb.data(), 64, o_cb);
    W4a8ExpandArgs a;
    a.pool = pool;
    a.codes_off = o_codes;
    a.srel_off = o_srel;
    a.sch_off = o_sch;
    a.cb_off = o_cb;
    a.q = pool;
    a.q_off = o_q;
    a.s = pool;
    a.s_off = o_s;
    a.rows = rows;
    a.k = k;
    a.group = group;
    a.codes_row_bytes = k / 2;
    a.srel_row_bytes = groups * 2;
    a.rel_dtype = RelDType::F16;
    a.layout = CodeLayout::Nibble4;
    a.has_channel_scale = true;
    a.has_codebook = true;
    dispatch_w4a8_expand(ctx, a);
    ctx.submit();
    std::vector<int8_t> q(rows * k), qo(rows * k);
    std::vector<float> s(rows), so(rows);
    ctx.download(pool, q.data(), q.size(), o_q);
    ctx.download(pool, s.data(), rows * 4, o_s);
    orc_w4a8_expand(codes.data(), k / 2, srel.data(), ORC_F16, groups * 2, sch.data(), 0, cb.data(), nullptr, rows, k,
                    group, 0, qo.data(), so.data(), nullptr);
    const int before = failures;
    CHECK(memcmp(q.data(), qo.data(), q.size()) == 0, "w4a8_expand: codes differ");
    CHECK(memcmp(s.data(), so.data(), s.size() * 4) == 0, "w4a8_expand: row scales differ");
    ctx.release_buffer(pool);
    printf("w4a8_expand %lldx%lld (fp16 s_rel, codebook): %s\n", (long long)rows, (long long)k,
           failures == before ? "bit-exact" : "mismatch");
}

// dispatch_elem(GeluTanh) and dispatch_silu_gate_fused against the oracle.
// The device evaluates GELU's 0.5 (1 + tanh t) as 1 / (1 + e^(-2t)) and takes
// expf from its own library, so the bound is 4e-7 |x| (GELU) and 2e-6
// relative (SiLU gate) instead of bit equality.
static void test_activations(ComputeContext& ctx) {
    const i64 rows = 33, cols = 1000;
    std::mt19937 rng(11);
    std::normal_distribution<float> nd(0.0f, 3.0f);
    std::vector<float> gx(rows * 2 * cols);
    for (auto& v : gx) v = nd(rng);
    const u64 off_gx = 0, off_g = off_gx + gx.size() * 4, off_s = off_g + gx.size() * 4;
    GpuBuffer* pool = ctx.create_device_buffer(off_s + rows * cols * 4);
    ctx.upload(pool, gx.data(), gx.size() * 4, off_gx);
    ctx.begin();
    ElemArgs ea;
    ea.op = ElemOp::GeluTanh;
    ea.a = GpuAlloc{pool, off_gx, gx.size() * 4};
    ea.y = GpuAlloc{pool, off_g, gx.size() * 4};
    ea.rows = rows;
    ea.cols = 2 * cols;
    dispatch_elem(ctx, ea);
    dispatch_silu_gate_fused(ctx, GpuAlloc{pool, off_gx, gx.size() * 4}, GpuAlloc{pool, off_s, (u64)(rows * cols * 4)},
                             rows, cols);
    ctx.submit();
    std::vector<float> g(gx.size()), sg(rows * cols), go(gx.size()), so(rows * cols);
    ctx.download(pool, g.data(), g.size() * 4, off_g);
    ctx.download(pool, sg.data(), sg.size() * 4, off_s);
    orc_gelu_tanh(gx.data(), go.data(), (int64_t)gx.size());
    orc_silu_gate(gx.data(), so.data(), rows, cols);
    int bad = 0;
    for (size_t i = 0; i < g.size(); i++) bad += !(std::fabs(g[i] - go[i]) <= 4e-7f * std::fabs(gx[i]));
    CHECK(bad == 0, "elem GeluTanh: %d values off the oracle", bad);
    bad = 0;
    for (size_t i = 0; i < sg.size(); i++) bad += !(std::fabs(sg[i] - so[i]) <= 2e-6f * std::fabs(so[i]) + 1e-30f);
    CHECK(bad == 0, "silu_gate_fused: %d values off the oracle", bad);
    ctx.release_buffer(pool);

    bool threw = false;
    try {
        ElemArgs bad_op;
        bad_op.op = ElemOp::Exp;
        bad_op.rows = 1;
        bad_op.cols = 4;
        dispatch_elem(ctx, bad_op);
    } catch (const MediaError& e) {
        threw = strstr(e.what(), "not served") != nullptr;
    }
    CHECK(threw, "elem Exp must throw MediaError");
    threw = false;
    try {
        dispatch_silu_gate_fused(ctx, GpuAlloc{}, GpuAlloc{}, 0, 8);
    } catch (const MediaError& e) {
        threw = strstr(e.what(), "empty") != nullptr;
    }
    CHECK(threw, "silu_gate_fused rows=0 must throw MediaError");
    printf("activations: %s\n", failures ? "mismatch" : "within bounds");
}

// dispatch_int4_gemm (the text encoder's convrot_w4a4 linear) after
// dispatch_quant_convrot with qmax 7, against the oracle, bit for bit.
static void test_int4_gemm(ComputeContext& ctx) {
    const i64 m = 45, k = 1024, n = 200;
    std::mt19937 rng(13);
    std::normal_distribution<float> nd(0.0f, 1.5f);
    std::vector<float> x(m * k), w(n * k);
    for (auto& v : x) v = nd(rng);
    for (auto& v : w) v = nd(rng);
    std::vector<uint8_t> packed(n * k / 2);
    std::vector<float> sw(n);
    CHECK(orc_quantize_convrot_w4a4(w.data(), n, k, packed.data(), sw.data()) == 0, "w4a4 packer");
    const u64 off_x = 0, off_b = off_x + m * k * 4, off_sw = off_b + n * k / 2, off_q = off_sw + 4096,
              off_s = off_q + m * k, off_c = off_s + 4096;
    GpuBuffer* pool = ctx.create_device_buffer(off_c + m * n * 4);
    ctx.upload(pool, x.data(), m * k * 4, off_x);
    ctx.upload(pool, packed.data(), packed.size(), off_b);
    ctx.upload(pool, sw.data(), n * 4, off_sw);
    ctx.begin();
    QuantConvrotArgs qa;
    qa.x = pool;
    qa.x_offset = off_x;
    qa.q = pool;
    qa.q_offset = off_q;
    qa.s = pool;
    qa.s_offset = off_s;
    qa.rows = m;
    qa.K = k;
    qa.qmax = 7.0f;
    dispatch_quant_convrot(ctx, qa);
    Int4GemmArgs ga;
    ga.a = GpuAlloc{pool, off_q, (u64)(m * k)};
    ga.b = GpuAlloc{pool, off_b, (u64)(n * k / 2)};
    ga.sa = GpuAlloc{pool, off_s, (u64)(m * 4)};
    ga.sb = GpuAlloc{pool, off_sw, (u64)(n * 4)};
    ga.c = GpuAlloc{pool, off_c, (u64)(m * n * 4)};
    ga.m = m;
    ga.n = n;
    ga.k = k;
    dispatch_int4_gemm(ctx, ga);
    ctx.submit();
    std::vector<float> c(m * n), s(m), so(m), co(m * n);
    std::vector<int8_t> q(m * k), qo(m * k);
    ctx.download(pool, c.data(), c.size() * 4, off_c);
    ctx.download(pool, q.data(), q.size(), off_q);
    ctx.download(pool, s.data(), s.size() * 4, off_s);
    orc_quantize_rows(x.data(), ORC_F32, m, k, k, 1, 7.0f, ORC_ROUND_HALF_AWAY, qo.data(), so.data());
    orc_int4_gemm(qo.data(), k, packed.data(), k / 2, so.data(), sw.data(), m, n, k, co.data(), n);
    CHECK(memcmp(q.data(), qo.data(), q.size()) == 0, "int4: qmax-7 activations differ");
    CHECK(memcmp(s.data(), so.data(), s.size() * 4) == 0, "int4: activation scales differ");
    CHECK(memcmp(c.data(), co.data(), c.size() * 4) == 0, "int4: fp32 outputs differ");
    ctx.release_buffer(pool);
    bool threw = false;
    try {
        Int4GemmArgs bad;
        bad.m = 4;
        bad.n = 4;
        bad.k = 768;
        dispatch_int4_gemm(ctx, bad);
    } catch (const MediaError& e) {
        threw = strstr(e.what(), "not a multiple of 512") != nullptr;
    }
    CHECK(threw, "int4_gemm K=768 must throw MediaError");
    printf("int4_gemm %lldx%lldx%lld: %s\n", (long long)m, (long long)n, (long long)k,
           failures ? "mismatch" : "bit-exact");
}

// linear_gemm then apply_lora_tail (core/models/image_dit.cpp:955-960), bit for bit.
static void test_lora_tail(ComputeContext& ctx) {
    const i64 m = 50, k = 512, n = 96, rank = 12;
    std::mt19937 rng(17);
    std::normal_distribution<float> nd(0.0f, 1.0f);
    std::uniform_int_distribution<int> ud(-127, 127);
    std::vector<float> x(m * k), sw(n, 0.002f), a(rank * k), b(n * rank);
    std::vector<int8_t> w(n * k);
    for (auto& v : x) v = nd(rng);
    for (auto& v : w) v = (int8_t)ud(rng);
    for (auto& v : a) v = 0.05f * nd(rng);
    for (auto& v : b) v = 0.05f * nd(rng);
    const u64 off_x = 0, off_w = off_x + m * k * 4, off_s = off_w + n * k, off_a = off_s + 4096,
              off_b = off_a + rank * k * 4, off_q8 = off_b + n * rank * 4, off_s8 = off_q8 + m * k,
              off_h = off_s8 + 4096, off_y = off_h + m * rank * 4;
    GpuBuffer* pool = ctx.create_device_buffer(off_y + m * n * 4);
    ctx.upload(pool, x.data(), m * k * 4, off_x);
    ctx.upload(pool, w.data(), n * k, off_w);
    ctx.upload(pool, sw.data(), n * 4, off_s);
    ctx.upload(pool, a.data(), a.size() * 4, off_a);
    ctx.upload(pool, b.data(), b.size() * 4, off_b);
    GpuCtx g;
    g.ctx = &ctx;
    QuantLinear ql;
    ql.w = GpuAlloc{pool, off_w, (u64)(n * k)};
    ql.scale = GpuAlloc{pool, off_s, (u64)(n * 4)};
    ql.n = n;
    ql.k = k;
    LoraTail t;
    t.active = true;
    t.rank = rank;
    t.n = n;
    t.k = k;
    t.at = GpuAlloc{pool, off_a, (u64)(rank * k * 4)};
    t.bt = GpuAlloc{pool, off_b, (u64)(n * rank * 4)};
    const GpuAlloc xa{pool, off_x, (u64)(m * k * 4)}, ya{pool, off_y, (u64)(m * n * 4)};
    ctx.begin();
    linear_gemm(g, ql, xa, m, k, ya, GpuAlloc{pool, off_q8, (u64)(m * k)}, GpuAlloc{pool, off_s8, (u64)(m * 4)});
    apply_lora_tail(g, t, xa, m, ya, GpuAlloc{pool, off_h, (u64)(m * rank * 4)});
    ctx.submit();
    std::vector<float> y(m * n), yo(m * n), so(m), h(m * rank);
    std::vector<int8_t> qo(m * k);
    ctx.download(pool, y.data(), y.size() * 4, off_y);
    orc_q8_linear(x.data(), ORC_F32, m, k, w.data(), sw.data(), 0, nullptr, -1, n, ORC_ROUND_HALF_AWAY, yo.data(),
                  ORC_F32, qo.data(), so.data(), nullptr);
    orc_lora_down(x.data(), k, a.data(), h.data(), m, k, rank);
    orc_lora_rank_add(h.data(), b.data(), yo.data(), n, m, n, rank);
    CHECK(memcmp(y.data(), yo.data(), y.size() * 4) == 0, "lora tail: fp32 outputs differ");
    bool threw = false;
    try {
        apply_lora_tail(g, t, xa, m, ya, GpuAlloc{pool, off_h, (u64)(m * rank * 4 - 4)});
    } catch (const MediaError& e) {
        threw = strstr(e.what(), "hidden-form scratch") != nullptr;
    }
    CHECK(threw, "a short LoRA scratch must throw MediaError");
    ctx.release_buffer(pool);
    printf("lora tail %lldx%lldx%lld rank %lld: %s\n", (long long)m, (long long)n, (long long)k, (long long)rank,
           failures ? "mismatch" : "bit-exact");
}

static void test_errors(ComputeContext& ctx) {
    bool threw = false;
    try {
        QuantConvrotArgs qa;
        GpuBuffer dummy{0x1000, 0};
        qa.x = qa.q = qa.s = &dummy;
        qa.rows = 4;
        qa.K = 300;
        dispatch_quant_convrot(ctx, qa);
    } catch (const MediaError& e) {
        threw = strstr(e.what(), "not a multiple of 256") != nullptr;
    }
    CHECK(threw, "quant_convrot K=300 must throw MediaError");
    threw = false;
    try {
        Int8GemmArgs ga;
        dispatch_int8_gemm(ctx, ga);
    } catch (const MediaError& e) {
        threw = strstr(e.what(), "empty problem") != nullptr;
    }
    CHECK(threw, "int8_gemm M=0 must throw MediaError");
    threw = false;
    try {
        GpuCtx g;
        g.ctx = &ctx;
        QuantLinear ql;
        ql.k = 512;
        GpuAlloc none;
        linear_gemm(g, ql, none, 1, 256, none, none, none);
    } catch (const MediaError& e) {
        threw = strstr(e.what(), "K mismatch") != nullptr;
    }
    CHECK(threw, "linear_gemm K mismatch must throw MediaError");
    printf("error contract: %s\n", failures ? "mismatch" : "ok");
}

// dispatch_int8_gemm at K values the MFMA tiles do not divide and at byte
// offsets that are not multiples of 16 (the reference sends these to its dp4a
// kernel, core/runtime/compute.cpp:566-575): int32-exact accumulators and the
// reference's fp32 epilogue, bit for bit against the oracle.
static void test_any_k_gemm(ComputeContext& ctx) {
    std::mt19937 rng(11);
    std::uniform_int_distribution<int> ud(-127, 127);
    std::uniform_real_distribution<float> us(0.001f, 0.01f);
    std::normal_distribution<float> nd(0.0f, 0.02f);
    const i64 ks[] = {32, 96, 100, 3000, 64, 1};
    const u64 aoffs[] = {1, 3, 16, 7, 5, 0};
    const u64 boffs[] = {3, 0, 5, 1, 2, 9};
    int cases = 0;
    for (int t = 0; t < 6; t++) {
        const i64 m = 37 + 20 * t, n = 45 + 31 * t, k = ks[t];
        std::vector<int8_t> a(m * k), b(n * k);
        std::vector<float> sa(m), sb(n), bias(n);
        for (auto& v : a) v = (int8_t)ud(rng);
        for (auto& v : b) v = (int8_t)ud(rng);
        for (auto& v : sa) v = us(rng);
        for (auto& v : sb) v = us(rng);
        for (auto& v : bias) v = nd(rng);
        const u64 o_a = aoffs[t], o_b = (((o_a + m * k) + 255) & ~(u64)255) + boffs[t];
        const u64 o_sa = ((o_b + n * k) + 255) & ~(u64)255, o_sb = o_sa + ((m * 4 + 255) & ~(u64)255),
                  o_bias = o_sb + ((n * 4 + 255) & ~(u64)255), o_c = o_bias + ((n * 4 + 255) & ~(u64)255);
        GpuBuffer* pool = ctx.create_device_buffer(o_c + (u64)m * n * 4 + 256);
        ctx.upload(pool, a.data(), a.size(), o_a);
        ctx.upload(pool, b.data(), b.size(), o_b);
        ctx.upload(pool, sa.data(), sa.size() * 4, o_sa);
        ctx.upload(pool, sb.data(), sb.size() * 4, o_sb);
        ctx.upload(pool, bias.data(), bias.size() * 4, o_bias);
        for (int with_bias = 0; with_bias < 2; with_bias++) {
            Int8GemmArgs ga;
            ga.a = pool;
            ga.a_offset = o_a;
            ga.b = pool;
            ga.b_offset = o_b;
            ga.sa = pool;
            ga.sa_offset = o_sa;
            ga.sb = pool;
            ga.sb_offset = o_sb;
            ga.c = pool;
            ga.c_offset = o_c;
            if (with_bias) {
                ga.bias = pool;
                ga.bias_offset = o_bias;
            }
            ga.M = m;
            ga.N = n;
            ga.K = k;
            ctx.begin();
            dispatch_int8_gemm(ctx, ga);
            ctx.submit();
            std::vector<float> c(m * n), want(m * n);
            std::vector<int32_t> acc(m * n);
            ctx.download(pool, c.data(), c.size() * 4, o_c);
            orc_gemm_i8_i32(a.data(), k, b.data(), k, m, n, k, acc.data());
            orc_epilogue(acc.data(), m, n, sa.data(), sb.data(), 0, with_bias ? bias.data() : nullptr,
                         with_bias ? ORC_F32 : -1, 1, want.data(), ORC_F32);
            CHECK(memcmp(c.data(), want.data(), c.size() * 4) == 0,
                  "any-K gemm K=%lld a_off=%llu b_off=%llu bias=%d differs", (long long)k, (unsigned long long)o_a,
                  (unsigned long long)o_b, with_bias);
            cases++;
        }
        ctx.release_buffer(pool);
    }
    printf("any-K int8 gemm: %d cases %s\n", cases, failures ? "mismatch" : "bit-exact");
}

// GpuArena as the reference's (core/runtime/sched.hpp:40-100): aligned pieces,
// a new chunk when one is full, reset keeps the chunks, rewind to a mark; and
// GpuCtx's arenas.
static void test_arena(ComputeContext& ctx) {
    GpuArena a;
    a.init(&ctx, 1 << 20);
    const GpuAlloc p = a.alloc(100);
    const GpuAlloc q = a.alloc(1000, 1024);
    CHECK(p.off == 0 && q.res == p.res && q.off == 1024, "arena alignment: offsets %llu %llu",
          (unsigned long long)p.off, (unsigned long long)q.off);
    CHECK(a.chunks() == 1 && a.capacity() == (1u << 20), "arena: one chunk of the chunk size");
    const GpuArena::Mark m = a.mark();
    const GpuAlloc big = a.alloc(3u << 20);
    CHECK(a.chunks() == 2 && big.res != p.res && big.off == 0 && big.res->bytes >= (3u << 20),
          "arena: a request past the chunk size gets its own chunk");
    a.rewind_to(m);
    const GpuAlloc r = a.alloc(64);
    CHECK(r.res == p.res && r.off == 2048, "arena: rewind returns to the mark (off %llu)", (unsigned long long)r.off);
    a.reset();
    CHECK(a.used() == 0 && a.chunks() == 2, "arena: reset keeps the chunks");
    const GpuAlloc s2 = a.alloc(2u << 20);
    CHECK(s2.res == big.res && a.chunks() == 2, "arena: a reset arena reuses a later chunk that fits");
    GpuArena wa, aa;
    wa.init(&ctx, 1 << 16);
    aa.init(&ctx, 1 << 16);
    GpuCtx g;
    g.ctx = &ctx;
    CHECK(!g.ok(), "GpuCtx without arenas is not ok");
    g.wa = &wa;
    g.aa = &aa;
    CHECK(g.ok(), "GpuCtx with both arenas is ok");
    const GpuAlloc w1 = g.walloc(4096), a1 = g.aalloc(4096), k1 = g.kalloc(16);
    CHECK(w1.res != a1.res && k1.res == a1.res, "GpuCtx: weights and activations in their own arenas");
    const float v[4] = {1.f, 2.f, 3.f, 4.f};
    float back[4] = {};
    g.upload_into(w1, v, sizeof v);
    ctx.download(w1.res, back, sizeof back, w1.off);
    CHECK(memcmp(v, back, sizeof v) == 0, "GpuCtx::upload_into");
    g.new_layer();
    CHECK(wa.used() == 0 && aa.used() > 0, "new_layer resets the weight arena only");
    g.new_step();
    CHECK(aa.used() == 0, "new_step resets the activation arena");
    printf("arena and context: %s\n", failures ? "mismatch" : "ok");
}

// The ownership contract of core/runtime/sched.cpp:65-109 and
// core/runtime/vram_budget.cpp:345-420: alloc(0) is empty, every grow is
// charged before it allocates and a charge past the limit throws (the arena
// unchanged), a grow from a fully rewound arena returns the old chunks first,
// and a released arena gives its charge back.
static void test_arena_budget(ComputeContext& ctx) {
    constexpr u64 MiB = 1ull << 20;
    VramBudget& vb = vram_budget();
    const u64 base = vb.local();
    {
        GpuArena a;
        a.init(&ctx, 1 * MiB, "test arena");
        const GpuAlloc z = a.alloc(0);
        CHECK(!z && z.bytes == 0 && a.chunks() == 0 && vb.local() == base, "arena: alloc(0) is an empty GpuAlloc");
        const GpuAlloc p = a.alloc(4096);
        CHECK(p && a.chunks() == 1 && vb.local() == base + 1 * MiB, "arena: a grow charges its chunk (%llu)",
              (unsigned long long)(vb.local() - base));
        const GpuAlloc z2 = a.alloc(0);
        CHECK(!z2 && a.used() == 4096, "arena: alloc(0) leaves the arena as it was");

        // A limit 1.5 MiB above what is charged: the next 1 MiB chunk fits, the
        // one after is refused before anything is allocated.
        vb.set_limit(vb.local() + MiB + MiB / 2);
        const GpuAlloc q = a.alloc(MiB - 4096 + 1);  // does not fit the first chunk's rest
        CHECK(q && a.chunks() == 2, "arena: a grow within the limit");
        bool refused = false;
        const u64 charged = vb.local(), cap = a.capacity();
        try {
            (void)a.alloc(MiB);
        } catch (const MediaError& e) {
            refused = strstr(e.what(), "VRAM budget exceeded") && strstr(e.what(), "test arena");
        }
        CHECK(refused, "arena: a grow past the limit throws MediaError naming the arena");
        CHECK(vb.local() == charged && a.capacity() == cap && a.chunks() == 2,
              "arena: a refused grow allocates and charges nothing");
        vb.set_limit(0);

        // Fully rewound: the two chunks give way to one of the size asked for.
        a.reset();
        a.set_chunk_bytes(8 * MiB);
        const GpuAlloc big = a.alloc(5 * MiB);
        CHECK(big && a.chunks() == 1 && a.capacity() == 8 * MiB && vb.local() == base + 8 * MiB,
              "arena: a grow from a rewound arena releases the old chunks first (chunks %d, charged %llu)",
              a.chunks(), (unsigned long long)(vb.local() - base));
        // Not rewound: the live chunk stays.
        const GpuAlloc more = a.alloc(MiB);
        CHECK(more && more.res == big.res && a.chunks() == 1, "arena: a chunk with room is used");
        const GpuAlloc over = a.alloc(4 * MiB);
        CHECK(over && a.chunks() == 2 && vb.local() == base + 16 * MiB, "arena: a grow with live allocations keeps them");
    }
    CHECK(vb.local() == base, "arena: destruction releases the charge (%llu left)",
          (unsigned long long)(vb.local() - base));
    printf("arena budget: %s\n", failures ? "mismatch" : "ok");
}

int main() {
    try {
        ComputeContext ctx(0);
        test_errors(ctx);
        test_linear_gemm(ctx);
        test_w4a8_expand(ctx);
        test_activations(ctx);
        test_int4_gemm(ctx);
        test_lora_tail(ctx);
        test_any_k_gemm(ctx);
        test_arena(ctx);
        test_arena_budget(ctx);
    } catch (const std::exception& e) {
        printf("FAIL exception: %s\n", e.what());
        return 1;
    }
    printf("%s (%d failures)\n", failures ? "FAILED" : "PASSED", failures);
    return failures ? 1 : 0;
}
