// Driver around the reference's own CPU path -- TEST INFRASTRUCTURE ONLY.
//
// Linked (by oracle/Makefile) against the reference sources where they lie:
// core/host/quant.cpp, core/util/json.cpp and core/util/utf8.cpp.  The
// reference's core/util/media_common.cpp includes <windows.h> and cannot be
// built here, so its dtype helpers (f16/bf16/fp8 decoders) stay unresolved:
// the driver only ever passes fp32 scale tables, which never reach them.
//
// Usage (all arrays are raw little-endian files):
//   phiref convrot ROWS COLS x.f32 out.f32
//   phiref quant ROWS COLS ROTATE x.f32 q.i8 s.f32
//   phiref gemm M N K a.i8 sa.f32 b.i8 sb.f32 y.f32
//   phiref w4 ROWS K GROUP HAS_CB HAS_CORR codes.u8 srel.f32 sch.f32 cb.f32 corr.f32 out.f32
//   phiref w6 ROWS K GROUP HAS_CORR codes.u8 srel.f32 sch.f32 corr.f32 out.f32
//   phiref w4a4pack ROWS COLS w.f32 packed.u8 scales.f32   (quantize_convrot_w4a4, group 256)
//   phiref bench_q8 M N K ROWS_TIMED       (prints seconds for ROWS_TIMED rows)
//   phiref bench_q8_mt M N K ROWS_TIMED THREADS
//        the same rows spread over THREADS threads, one row per task from a
//        shared counter (the shape of core/kernels/parallel_for.hpp:44-65)
#include <atomic>
#include <chrono>
#include <thread>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "host/quant.hpp"

using namespace phi::media;

template <class T>
static std::vector<T> read_file(const char* path, size_t count) {
    std::vector<T> v(count);
    FILE* f = fopen(path, "rb");
    if (!f) {
        fprintf(stderr, "phiref: cannot open %s\n", path);
        exit(2);
    }
    if (count && fread(v.data(), sizeof(T), count, f) != count) {
        fprintf(stderr, "phiref: short read on %s\n", path);
        exit(2);
    }
    fclose(f);
    return v;
}

template <class T>
static void write_file(const char* path, const T* p, size_t count) {
    FILE* f = fopen(path, "wb");
    if (!f || (count && fwrite(p, sizeof(T), count, f) != count)) {
        fprintf(stderr, "phiref: cannot write %s\n", path);
        exit(2);
    }
    fclose(f);
}

static QuantSpec spec_of(bool rotate) {
    QuantSpec s;
    s.format = "int8_tensorwise";
    s.convrot = rotate;
    s.convrot_groupsize = 256;
    s.valid = true;
    return s;
}

int main(int argc, char** argv) {
    if (argc < 2) {
        fprintf(stderr, "phiref: missing op\n");
        return 2;
    }
    const std::string op = argv[1];
    try {
        if (op == "convrot" && argc == 6) {
            const i64 rows = atoll(argv[2]), cols = atoll(argv[3]);
            auto x = read_file<float>(argv[4], (size_t)(rows * cols));
            std::vector<float> y(x.size());
            convrot_forward(x.data(), y.data(), rows, cols, 256);
            write_file(argv[5], y.data(), y.size());
        } else if (op == "quant" && argc == 8) {
            const i64 rows = atoll(argv[2]), cols = atoll(argv[3]);
            const bool rot = atoi(argv[4]) != 0;
            auto x = read_file<float>(argv[5], (size_t)(rows * cols));
            QuantInt8 qa = quantize_activation(x.data(), rows, cols, spec_of(rot));
            write_file(argv[6], qa.q.data(), qa.q.size());
            write_file(argv[7], qa.scale.data(), qa.scale.size());
        } else if (op == "gemm" && argc == 10) {
            const i64 M = atoll(argv[2]), N = atoll(argv[3]), K = atoll(argv[4]);
            auto a = read_file<int8_t>(argv[5], (size_t)(M * K));
            auto sa = read_file<float>(argv[6], (size_t)M);
            auto b = read_file<int8_t>(argv[7], (size_t)(N * K));
            auto sb = read_file<float>(argv[8], (size_t)N);
            std::vector<float> y((size_t)(M * N));
            gemm_int8(a.data(), sa.data(), b.data(), sb.data(), M, N, K, y.data());
            write_file(argv[9], y.data(), y.size());
        } else if ((op == "w4" && argc == 13) || (op == "w6" && argc == 11)) {
            const bool six = op == "w6";
            const i64 rows = atoll(argv[2]), k = atoll(argv[3]), group = atoll(argv[4]);
            int ai = 5;
            const bool has_cb = six ? false : atoi(argv[ai++]) != 0;
            const bool has_corr = atoi(argv[ai++]) != 0;
            const i64 groups = k / group;
            const i64 row_bytes = six ? k / 2 + k / 4 : k / 2;
            auto codes = read_file<u8>(argv[ai++], (size_t)(rows * row_bytes));
            auto srel = read_file<float>(argv[ai++], (size_t)(rows * groups));
            auto sch = read_file<float>(argv[ai++], (size_t)rows);
            std::vector<float> cb;
            if (!six) {
                const char* p = argv[ai++];
                if (has_cb) cb = read_file<float>(p, 16);
            }
            std::vector<float> corr;
            {
                const char* p = argv[ai++];
                if (has_corr) corr = read_file<float>(p, (size_t)(groups * rows));
            }
            std::vector<float> out((size_t)(rows * k));
            std::vector<float> corr_row((size_t)groups);
            for (i64 r = 0; r < rows; r++) {
                if (has_corr)
                    for (i64 g = 0; g < groups; g++) corr_row[(size_t)g] = corr[(size_t)(g * rows + r)];
                if (six)
                    dequant_packed6_row(codes.data() + r * row_bytes, k, sch[(size_t)r],
                                        srel.data() + r * groups, DType::F32, group,
                                        has_corr ? corr_row.data() : nullptr, out.data() + r * k);
                else
                    dequant_codebook_int4_row(codes.data() + r * row_bytes, k,
                                              has_cb ? cb.data() : nullptr, sch[(size_t)r],
                                              srel.data() + r * groups, DType::F32, group,
                                              has_corr ? corr_row.data() : nullptr,
                                              out.data() + r * k);
            }
            write_file(argv[ai], out.data(), out.size());
        } else if (op == "w4a4pack" && argc == 7) {
            const i64 rows = atoll(argv[2]), cols = atoll(argv[3]);
            auto w = read_file<float>(argv[4], (size_t)(rows * cols));
            std::vector<u8> packed((size_t)(rows * cols / 2));
            std::vector<float> scales((size_t)rows);
            quantize_convrot_w4a4(w.data(), rows, cols, packed.data(), scales.data(), 256);
            write_file(argv[5], packed.data(), packed.size());
            write_file(argv[6], scales.data(), scales.size());
        } else if (op == "bench_q8" && argc == 6) {
            // The reference CPU linear on a bounded row sample: rotate+quantise
            // ROWS rows of x, then the naive int8 GEMM against all N rows of W.
            const i64 M = atoll(argv[2]), N = atoll(argv[3]), K = atoll(argv[4]);
            const i64 rows = std::min<i64>(M, atoll(argv[5]));
            std::mt19937 rng(0);
            std::normal_distribution<float> nd(0.0f, 1.0f);
            std::uniform_int_distribution<int> ud(-127, 127);
            std::vector<float> x((size_t)(rows * K));
            for (auto& v : x) v = nd(rng);
            std::vector<int8_t> w((size_t)(N * K));
            for (auto& v : w) v = (int8_t)ud(rng);
            std::vector<float> sw((size_t)N, 0.002f), y((size_t)(rows * N));
            const auto t0 = std::chrono::steady_clock::now();
            QuantInt8 qa = quantize_activation(x.data(), rows, K, spec_of(true));
            gemm_int8(qa.q.data(), qa.scale.data(), w.data(), sw.data(), rows, N, K, y.data());
            const auto t1 = std::chrono::steady_clock::now();
            double chk = 0;
            for (float v : y) chk += v;
            printf("%.6f %.6e\n", std::chrono::duration<double>(t1 - t0).count(), chk);
        } else if (op == "bench_q8_mt" && argc == 7) {
            const i64 M = atoll(argv[2]), N = atoll(argv[3]), K = atoll(argv[4]);
            const i64 rows = std::min<i64>(M, atoll(argv[5]));
            const int threads = std::max(1, atoi(argv[6]));
            std::mt19937 rng(0);
            std::normal_distribution<float> nd(0.0f, 1.0f);
            std::uniform_int_distribution<int> ud(-127, 127);
            std::vector<float> x((size_t)(rows * K));
            for (auto& v : x) v = nd(rng);
            std::vector<int8_t> w((size_t)(N * K));
            for (auto& v : w) v = (int8_t)ud(rng);
            std::vector<float> sw((size_t)N, 0.002f), y((size_t)(rows * N));
            std::atomic<i64> next{0};
            auto worker = [&] {
                for (;;) {
                    const i64 r = next.fetch_add(1, std::memory_order_relaxed);
                    if (r >= rows) break;
                    QuantInt8 qa = quantize_activation(x.data() + r * K, 1, K, spec_of(true));
                    gemm_int8(qa.q.data(), qa.scale.data(), w.data(), sw.data(), 1, N, K, y.data() + r * N);
                }
            };
            const auto t0 = std::chrono::steady_clock::now();
            std::vector<std::thread> pool;
            for (int t = 1; t < threads; t++) pool.emplace_back(worker);
            worker();
            for (auto& th : pool) th.join();
            const auto t1 = std::chrono::steady_clock::now();
            double chk = 0;
            for (float v : y) chk += v;
            printf("%.6f %.6e\n", std::chrono::duration<double>(t1 - t0).count(), chk);
        } else {
            fprintf(stderr, "phiref: bad arguments for %s\n", op.c_str());
            return 2;
        }
    } catch (const std::exception& e) {
        fprintf(stderr, "phiref: %s\n", e.what());
        return 3;
    }
    return 0;
}
