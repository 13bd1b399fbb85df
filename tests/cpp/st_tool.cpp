// Test driver for the checkpoint readers of the C++ host layer
// (phi-agent_amd/host/safetensors.hpp, load_quant_linear,
// upload_quant_linear_w4a4).  The Python tests write safetensors files with
// known contents and compare what this prints or computes.
//
//   st_tool spec <json text>                       parse_quant_spec -> JSON line
//   st_tool probe <file> <base>                    layout of <base>.weight -> JSON line (no GPU)
//   st_tool linear <file> <base> <x.f32> <M> <out.f32> [<lora> <strength>]...
//        load_quant_linear, then linear_gemm of x [M, K] fp32 into out [M, N] fp32 (GPU)
//   st_tool linear_kt ...   the same with GpuCtx::k_tiled_weights set
//   st_tool int4 <file> <base> <x.f32> <M> <out.f32>
//        upload_quant_linear_w4a4, quant_convrot (qmax 7), int4 GEMM into out (GPU)
//   st_tool weights <how> <file> <out.bin> <base> [<base_k> <base_v>] [lora <path> <strength>]...
//        how = load (load_quant_linear), load3 (load_quant3_linear) or upload_i8
//        (upload_quant_linear_i8), with an optional LoraSet; writes n, k (int64)
//        then the int8 weight [n, k] and its fp32 scales [n] (GPU).  load_kt and
//        load3_kt set GpuCtx::k_tiled_weights and unpack the K-tiled weight.
//   st_tool tune <M> <N> <K> <iters> <k_tiled> <out.json>
//        autotune_int8_gemm, then the winner saved, loaded back and applied:
//        a JSON line with the sweep and the plan the library then runs (GPU)
//   st_tool lora_probe <target> <n> <k> lora <path> <strength>...
//        LoraSet::touches / deltas_for -> JSON line (no GPU)
//   st_tool tail <out.bin> <n> <k> <base>:<row0>:<rows>... lora <path> <strength>...
//        load_lora_tail over the modules; writes rank (int64), at [rank, k] and
//        bt [n, rank] fp32 (GPU)
// Exit code 0 on success; a MediaError prints "error: <message>" and exits 3.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "phi_media.hpp"
#include "phi_qlinear.h"
#include "safetensors.hpp"

using namespace phi::media;

static void print_spec(const QuantSpec& s, const char* tail) {
    printf("{\"valid\": %s, \"format\": \"%s\", \"convrot\": %s, \"convrot_groupsize\": %d, \"group_size\": %d}%s",
           s.valid ? "true" : "false", s.format.c_str(), s.convrot ? "true" : "false", s.convrot_groupsize,
           s.group_size, tail);
}

static std::vector<float> read_f32(const char* path, size_t n) {
    std::vector<float> v(n);
    FILE* f = fopen(path, "rb");
    if (!f || fread(v.data(), 4, n, f) != n) throw MediaError(std::string("cannot read ") + path);
    fclose(f);
    return v;
}

static void write_f32(const char* path, const std::vector<float>& v) {
    FILE* f = fopen(path, "wb");
    if (!f || fwrite(v.data(), 4, v.size(), f) != v.size()) throw MediaError(std::string("cannot write ") + path);
    fclose(f);
}

static void write_bytes(FILE* f, const void* p, size_t n) {
    if (fwrite(p, 1, n, f) != n) throw MediaError("short write");
}

// Splits trailing "lora <path> <strength>" triples off argv[from..argc).
static int lora_args(int argc, char** argv, int from, LoraSet& lora) {
    int end = argc;
    for (int i = from; i < argc; i++)
        if (std::string(argv[i]) == "lora") {
            if (end == argc) end = i;
            if (i + 2 >= argc) throw MediaError("lora needs <path> <strength>");
            lora.add(argv[i + 1], (float)atof(argv[i + 2]));
            i += 2;
        }
    return end;
}

// A K-tiled [rows, K] matrix back in row-major order (the layout's definition:
// 256-row strips of h rows, each 64-byte K-step of a strip one h x 64 block, the
// 16-byte chunk c of strip row r in slot c ^ ((r >> 2) & 3)).
static std::vector<int8_t> unpack_k_tiled(const std::vector<int8_t>& p, i64 rows, i64 K) {
    std::vector<int8_t> out(p.size());
    for (i64 r = 0; r < rows; r++) {
        const i64 strip = r / 256, rr = r % 256, h = std::min<i64>(256, rows - 256 * strip);
        for (i64 k = 0; k < K; k++) {
            const i64 slot = ((k / 16) % 4) ^ ((rr / 4) % 4);
            out[(size_t)(r * K + k)] = p[(size_t)(256 * K * strip + h * 64 * (k / 64) + 64 * rr + 16 * slot + k % 16)];
        }
    }
    return out;
}

static int weights(int argc, char** argv) {
    std::string how = argv[2];
    const bool want_kt = how.size() > 3 && how.compare(how.size() - 3, 3, "_kt") == 0;
    if (want_kt) how.resize(how.size() - 3);
    bool k_tiled = false;
    SafeTensors st(argv[3]);
    const char* out = argv[4];
    LoraSet lora;
    const int end = lora_args(argc, argv, 5, lora);
    const LoraSet* lp = lora.empty() ? nullptr : &lora;
    ComputeContext ctx(0);
    GpuArena wa, aa;
    wa.init(&ctx, 64ull << 20);
    aa.init(&ctx, 1 << 20);
    GpuCtx g;
    g.ctx = &ctx;
    g.wa = &wa;
    g.aa = &aa;
    g.k_tiled_weights = want_kt;
    GpuAlloc w, s;
    i64 n = 0, k = 0;
    if (how == "load" && end == 6) {
        const QuantLinear q = load_quant_linear(g, st, argv[5], nullptr, lp);
        w = q.w, s = q.scale, n = q.n, k = q.k, k_tiled = q.k_tiled;
    } else if (how == "load3" && end == 8) {
        const QuantLinear q = load_quant3_linear(g, st, argv[5], argv[6], argv[7], nullptr, lp);
        w = q.w, s = q.scale, n = q.n, k = q.k, k_tiled = q.k_tiled;
    } else if (how == "upload_i8" && end == 6) {
        const I8Upload u = upload_quant_linear_i8(g, st, argv[5], wa, lp);
        w = u.w, s = u.s, n = u.n, k = u.k;
    } else {
        fprintf(stderr, "st_tool weights: bad arguments\n");
        return 2;
    }
    ctx.submit();
    std::vector<int8_t> wq((size_t)(n * k));
    std::vector<float> sc((size_t)n);
    ctx.download(w.res, wq.data(), wq.size(), w.off);
    ctx.download(s.res, sc.data(), sc.size() * 4, s.off);
    if (k_tiled) wq = unpack_k_tiled(wq, n, k);
    FILE* f = fopen(out, "wb");
    if (!f) throw MediaError(std::string("cannot write ") + out);
    write_bytes(f, &n, 8);
    write_bytes(f, &k, 8);
    write_bytes(f, wq.data(), wq.size());
    write_bytes(f, sc.data(), sc.size() * 4);
    fclose(f);
    printf("{\"n\": %lld, \"k\": %lld, \"arena_used\": %llu, \"k_tiled\": %s}\n", (long long)n, (long long)k,
           (unsigned long long)wa.used(), k_tiled ? "true" : "false");
    return 0;
}

// autotune_int8_gemm, the winner stored and saved, the table cleared, the file
// loaded into a new store and applied: the plan the library then runs.
static int tune(char** argv) {
    const i64 M = atoll(argv[2]), N = atoll(argv[3]), K = atoll(argv[4]);
    const int iters = atoi(argv[5]);
    const bool kt = atoi(argv[6]) != 0;
    ComputeContext ctx(0);
    const GemmTuneResult r = autotune_int8_gemm(ctx, M, N, K, iters, kt);
    if (!r.ok) throw MediaError(r.error);
    GemmTuneStore store;
    store.put(r.best);
    if (!store.save(argv[7])) throw MediaError(std::string("cannot write ") + argv[7]);
    phi_hip_gemm_plan_clear();
    GemmTuneStore back;
    if (!back.load(argv[7])) throw MediaError(std::string("cannot read back ") + argv[7]);
    back.apply();
    phi_gemm_plan p{};
    int tuned = 0;
    if (phi_hip_gemm_plan_get(M, N, K, kt ? 1 : 0, &p, &tuned) != PHI_OK) throw MediaError(phi_hip_last_error());
    printf("{\"ok\": true, \"default_exact\": %s, \"exact\": %d, \"tried\": %zu, \"best_us\": %.3f, "
           "\"best\": [%lld, %d, %d, %d], \"applied\": [%lld, %d, %d, %d], \"tuned\": %d, \"entries\": %zu, "
           "\"us\": [",
           r.default_exact ? "true" : "false", r.exact_matches, r.tried.size(), r.best.measured_us,
           (long long)r.best.big_rows, r.best.group_m, r.best.split ? 1 : 0, r.best.tile, (long long)p.big_rows,
           (int)p.group_m, (int)p.split, (int)p.tile, tuned, back.size());
    for (size_t i = 0; i < r.tried.size(); i++) printf("%s%.3f", i ? ", " : "", r.tried[i].measured_us);
    printf("], \"tiles\": [");
    for (size_t i = 0; i < r.tried.size(); i++) printf("%s%d", i ? ", " : "", r.tried[i].tile);
    printf("]}\n");
    return 0;
}

static int tail(int argc, char** argv) {
    const char* out = argv[2];
    const i64 n = atoll(argv[3]), k = atoll(argv[4]);
    LoraSet lora;
    const int end = lora_args(argc, argv, 5, lora);
    std::vector<LoraModule> mods;
    for (int i = 5; i < end; i++) {
        const std::string spec = argv[i];
        const size_t a = spec.find(':'), b = spec.rfind(':');
        if (a == std::string::npos || a == b) throw MediaError("module spec is base:row0:rows");
        mods.push_back(LoraModule{spec.substr(0, a), atoll(spec.substr(a + 1, b - a - 1).c_str()),
                                  atoll(spec.substr(b + 1).c_str()), &lora});
    }
    ComputeContext ctx(0);
    GpuArena arena;
    arena.init(&ctx, 16ull << 20);
    GpuCtx g;
    g.ctx = &ctx;
    const LoraTail t = load_lora_tail(g, arena, mods, n, k);
    ctx.submit();
    FILE* f = fopen(out, "wb");
    if (!f) throw MediaError(std::string("cannot write ") + out);
    const i64 rank = t.active ? t.rank : 0;
    write_bytes(f, &rank, 8);
    if (rank > 0) {
        std::vector<float> at((size_t)(rank * k)), bt((size_t)(n * rank));
        ctx.download(t.at.res, at.data(), at.size() * 4, t.at.off);
        ctx.download(t.bt.res, bt.data(), bt.size() * 4, t.bt.off);
        write_bytes(f, at.data(), at.size() * 4);
        write_bytes(f, bt.data(), bt.size() * 4);
    }
    fclose(f);
    printf("{\"rank\": %lld, \"touches\": %s}\n", (long long)rank,
           mods.empty() ? "false" : (lora.touches(mods[0].base) ? "true" : "false"));
    return 0;
}

int main(int argc, char** argv) {
    if (argc < 3) {
        fprintf(stderr, "usage: st_tool spec|probe|linear|int4 ...\n");
        return 2;
    }
    const std::string op = argv[1];
    try {
        if (op == "spec") {
            const std::string text = argv[2];
            print_spec(parse_quant_spec(text.data(), text.size()), "\n");
            return 0;
        }
        if (op == "tune" && argc == 8) return tune(argv);
        if (op == "weights" && argc >= 6) return weights(argc, argv);
        if (op == "tail" && argc >= 6) return tail(argc, argv);
        if (op == "lora_probe" && argc >= 8) {
            LoraSet lora;
            lora_args(argc, argv, 5, lora);
            std::vector<LoraSet::Delta> d;
            lora.deltas_for(argv[2], atoll(argv[3]), atoll(argv[4]), &d);
            printf("{\"files\": %zu, \"touches\": %s, \"deltas\": [", lora.size(),
                   lora.touches(argv[2]) ? "true" : "false");
            for (size_t i = 0; i < d.size(); i++)
                printf("%s{\"rank\": %lld, \"scale\": %.9g, \"a0\": %.9g, \"b0\": %.9g}", i ? ", " : "",
                       (long long)d[i].rank, d[i].scale, d[i].a[0], d[i].b[0]);
            printf("]}\n");
            return 0;
        }
        if (argc < 4) return 2;
        SafeTensors st(argv[2]);
        const std::string base = argv[3];
        if (op == "probe") {
            const StTensor& t = st.require(base + ".weight");
            const SafeTensors::WeightLayout L = st.weight_layout(t.name);
            printf("{\"tensors\": %zu, \"dtype\": \"%s\", \"n\": %lld, \"k\": %lld, \"bits\": %d, \"group\": %lld, "
                   "\"packed\": %s, \"known\": %s, \"plain_int8\": %s, \"row_scale\": \"%s\", \"rel_scale\": \"%s\", "
                   "\"codebook\": %s, \"correction\": %s, \"global_scale\": \"%s\", \"row_scale0\": %.9g, \"spec\": ",
                   st.tensors().size(), st_dtype_name(t.dtype), (long long)(t.shape.empty() ? 0 : t.shape[0]),
                   (long long)st.logical_cols(t), L.bits, (long long)L.group, L.packed ? "true" : "false",
                   L.known_family ? "true" : "false", st.is_plain_int8(t) ? "true" : "false",
                   L.row_scale ? L.row_scale->name.c_str() : "", L.rel_scale ? L.rel_scale->name.c_str() : "",
                   L.codebook ? "true" : "false", L.correction ? "true" : "false",
                   L.global_scale ? L.global_scale->name.c_str() : "",
                   L.row_scale ? st.row_scale_value(*L.row_scale, 0) : 1.0);
            print_spec(L.spec, "}\n");
            fflush(stdout);
            return 0;
        }
        const bool linear_op = op == "linear" || op == "linear_kt";
        if ((linear_op && argc >= 7 && (argc - 7) % 2 == 0) || (op == "int4" && argc == 7)) {
            const i64 M = atoll(argv[5]);
            ComputeContext ctx(0);
            GpuCtx g;
            g.ctx = &ctx;
            g.k_tiled_weights = op == "linear_kt";
            bool k_tiled = false;
            const StTensor& t = st.require(base + ".weight");
            const i64 K = st.logical_cols(t), N = t.shape[0];
            std::vector<float> x = read_f32(argv[4], (size_t)(M * K)), y((size_t)(M * N));
            GpuArena arena(ctx, (u64)(N * K + N * 4 + 1024));
            GpuArena acts;
            acts.init(&ctx, 1 << 20);
            g.wa = &arena;
            g.aa = &acts;
            GpuBuffer* work = ctx.create_device_buffer((u64)(M * K * 4 + M * K + M * 4 + M * N * 4 + 4096));
            const u64 o_x = 0, o_q = (u64)M * K * 4, o_s = (o_q + M * K + 255) & ~(u64)255,
                      o_y = (o_s + M * 4 + 255) & ~(u64)255;
            ctx.upload(work, x.data(), x.size() * 4, o_x);
            if (linear_op) {
                LoraSet lora;
                for (int i = 7; i + 1 < argc; i += 2) lora.add(argv[i], (float)atof(argv[i + 1]));
                const QuantLinear ql = load_quant_linear(g, st, base, nullptr, lora.empty() ? nullptr : &lora);
                k_tiled = ql.k_tiled;
                linear_gemm(g, ql, GpuAlloc{work, o_x, (u64)M * K * 4}, M, K, GpuAlloc{work, o_y, (u64)M * N * 4},
                            GpuAlloc{work, o_q, (u64)M * K}, GpuAlloc{work, o_s, (u64)M * 4});
            } else {
                const I4Upload w = upload_quant_linear_w4a4(g, st, base, arena);
                QuantConvrotArgs qa;
                qa.x = work;
                qa.x_offset = o_x;
                qa.q = work;
                qa.q_offset = o_q;
                qa.s = work;
                qa.s_offset = o_s;
                qa.rows = M;
                qa.K = K;
                qa.qmax = 7.0f;
                dispatch_quant_convrot(ctx, qa);
                Int4GemmArgs ga;
                ga.a = GpuAlloc{work, o_q, (u64)M * K};
                ga.b = w.w;
                ga.sa = GpuAlloc{work, o_s, (u64)M * 4};
                ga.sb = w.s;
                ga.c = GpuAlloc{work, o_y, (u64)M * N * 4};
                ga.m = M;
                ga.n = N;
                ga.k = K;
                dispatch_int4_gemm(ctx, ga);
            }
            ctx.submit();
            ctx.download(work, y.data(), y.size() * 4, o_y);
            ctx.release_buffer(work);
            write_f32(argv[6], y);
            printf("{\"n\": %lld, \"k\": %lld, \"arena_used\": %llu, \"k_tiled\": %s}\n", (long long)N,
                   (long long)K, (unsigned long long)arena.used(), k_tiled ? "true" : "false");
            return 0;
        }
        fprintf(stderr, "st_tool: bad arguments for %s\n", op.c_str());
        return 2;
    } catch (const std::exception& e) {
        printf("error: %s\n", e.what());
        return 3;
    }
}
