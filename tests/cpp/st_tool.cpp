// Test driver for the checkpoint readers of the C++ host layer
// (phi-agent_amd/host/safetensors.hpp, load_quant_linear,
// upload_quant_linear_w4a4).  The Python tests write safetensors files with
// known contents and compare what this prints or computes.
//
//   st_tool spec <json text>                       parse_quant_spec -> JSON line
//   st_tool probe <file> <base>                    layout of <base>.weight -> JSON line (no GPU)
//   st_tool linear <file> <base> <x.f32> <M> <out.f32>
//        load_quant_linear, then linear_gemm of x [M, K] fp32 into out [M, N] fp32 (GPU)
//   st_tool int4 <file> <base> <x.f32> <M> <out.f32>
//        upload_quant_linear_w4a4, quant_convrot (qmax 7), int4 GEMM into out (GPU)
// Exit code 0 on success; a MediaError prints "error: <message>" and exits 3.
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "phi_media.hpp"
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
        if (argc < 4) return 2;
        SafeTensors st(argv[2]);
        const std::string base = argv[3];
        if (op == "probe") {
            const StTensor& t = st.require(base + ".weight");
            const SafeTensors::WeightLayout L = st.weight_layout(t.name);
            printf("{\"tensors\": %zu, \"dtype\": \"%s\", \"n\": %lld, \"k\": %lld, \"bits\": %d, \"group\": %lld, "
                   "\"packed\": %s, \"known\": %s, \"plain_int8\": %s, \"row_scale\": \"%s\", \"rel_scale\": \"%s\", "
                   "\"codebook\": %s, \"correction\": %s, \"row_scale0\": %.9g, \"spec\": ",
                   st.tensors().size(), st_dtype_name(t.dtype), (long long)(t.shape.empty() ? 0 : t.shape[0]),
                   (long long)st.logical_cols(t), L.bits, (long long)L.group, L.packed ? "true" : "false",
                   L.known_family ? "true" : "false", st.is_plain_int8(t) ? "true" : "false",
                   L.row_scale ? L.row_scale->name.c_str() : "", L.rel_scale ? L.rel_scale->name.c_str() : "",
                   L.codebook ? "true" : "false", L.correction ? "true" : "false",
                   L.row_scale ? st.row_scale_value(*L.row_scale, 0) : 1.0);
            print_spec(L.spec, "}\n");
            fflush(stdout);
            return 0;
        }
        if ((op == "linear" || op == "int4") && argc == 7) {
            const i64 M = atoll(argv[5]);
            ComputeContext ctx(0);
            GpuCtx g;
            g.ctx = &ctx;
            const StTensor& t = st.require(base + ".weight");
            const i64 K = st.logical_cols(t), N = t.shape[0];
            std::vector<float> x = read_f32(argv[4], (size_t)(M * K)), y((size_t)(M * N));
            GpuArena arena(ctx, (u64)(N * K + N * 4 + 1024));
            GpuBuffer* work = ctx.create_device_buffer((u64)(M * K * 4 + M * K + M * 4 + M * N * 4 + 4096));
            const u64 o_x = 0, o_q = (u64)M * K * 4, o_s = (o_q + M * K + 255) & ~(u64)255,
                      o_y = (o_s + M * 4 + 255) & ~(u64)255;
            ctx.upload(work, x.data(), x.size() * 4, o_x);
            if (op == "linear") {
                const QuantLinear ql = load_quant_linear(g, st, base, arena);
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
            printf("{\"n\": %lld, \"k\": %lld, \"arena_used\": %llu}\n", (long long)N, (long long)K,
                   (unsigned long long)arena.used());
            return 0;
        }
        fprintf(stderr, "st_tool: bad arguments for %s\n", op.c_str());
        return 2;
    } catch (const std::exception& e) {
        printf("error: %s\n", e.what());
        return 3;
    }
}
