// spmm_vcsr.cpp -- benchmark driver with the reference's command line and CSV.
//
// Mirrors MuuSeoTia/VCSR_MC src/main.cpp (CLI :33-43, B fill :161-179, oracle :199-218,
// measure :239-308, VCSR loop :345-362, CSV :220) on top of libvcsrmc.so and libvcsrmc_bench.so:
//   vcsr_mc / vcsr_mc_fp32     through the drop-in C++ surface (include/vcsr_formats.hpp),
//                              with the reference's call sequence convert -> upload -> run
//   rocsparse / rocsparse_fp16 hipSPARSE SpMM (libvcsrmc_bench.so)
// --reorder rcm (main.cpp:182-183) runs the GPU column reordering through the drop-in
// include/reorder.hpp.  Additive: --gen K[:size] reads a seeded synthetic workload instead of
// --mtx (configs of include/vcsrmc_bench.h).
#include <getopt.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cerrno>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <functional>
#include <limits>
#include <numeric>
#include <random>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "csr.hpp"
#include "reorder.hpp"
#include "vcsr_formats.hpp"
#include "vcsrmc_bench.h"

namespace {

void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        std::fprintf(stderr, "HIP error in %s: %s\n", what, hipGetErrorString(e));
        std::exit(EXIT_FAILURE);
    }
}

// ---- Matrix Market coordinate files (semantics of include/mmio.hpp:19-75) ----------------
struct Triples {
    int M = 0, N = 0;
    std::vector<int> r, c;
    std::vector<float> v;
};

Triples read_mtx(const std::string& path) {
    std::ifstream in(path);
    if (!in) throw std::runtime_error("Failed to open MTX: " + path);
    std::string line;
    if (!std::getline(in, line)) throw std::runtime_error("Empty MTX file");
    std::istringstream banner(line);
    std::string magic, object, layout, field, sym;
    banner >> magic >> object >> layout >> field >> sym;
    if (magic != "%%MatrixMarket" || object != "matrix" || layout != "coordinate")
        throw std::runtime_error("Expected a Matrix Market coordinate matrix");
    if (field != "real" && field != "integer" && field != "pattern")
        throw std::runtime_error("Unsupported MTX field: " + field);
    if (sym != "general" && sym != "symmetric" && sym != "skew-symmetric")
        throw std::runtime_error("Unsupported MTX symmetry: " + sym);
    auto data_line = [&](std::string& out) {
        while (std::getline(in, out)) {
            const size_t k = out.find_first_not_of(" \t\r");
            if (k != std::string::npos && out[k] != '%') return true;
        }
        return false;
    };
    if (!data_line(line)) throw std::runtime_error("Missing MTX dimensions");
    long long m = 0, n = 0, cnt = 0;
    {
        std::istringstream d(line);
        if (!(d >> m >> n >> cnt) || m <= 0 || n <= 0 || m >= INT_MAX || n >= INT_MAX ||
            cnt < 0 || cnt > INT_MAX)
            throw std::runtime_error("Invalid or unsupported MTX dimensions/nnz");
    }
    if (sym != "general" && m != n) throw std::runtime_error("Symmetric MTX must be square");
    Triples t;
    t.M = (int)m;
    t.N = (int)n;
    auto push = [&](long long r, long long c, float v) {
        if (t.v.size() >= (size_t)INT_MAX)
            throw std::runtime_error("Expanded MTX exceeds 32-bit nnz limit");
        t.r.push_back((int)r);
        t.c.push_back((int)c);
        t.v.push_back(v);
    };
    for (long long i = 0; i < cnt; ++i) {
        if (!data_line(line)) throw std::runtime_error("Truncated MTX data");
        std::istringstream e(line);
        long long r, c;
        double val = 1.0;
        if (!(e >> r >> c) || (field != "pattern" && !(e >> val)))
            throw std::runtime_error("Bad MTX entry at index " + std::to_string(i));
        std::string extra;
        if (e >> extra) throw std::runtime_error("Extra fields in MTX entry");
        if (r < 1 || r > m || c < 1 || c > n)
            throw std::runtime_error("MTX row/column index out of range (expected one-based indices)");
        if (!std::isfinite(val) || std::fabs(val) > std::numeric_limits<float>::max())
            throw std::runtime_error("MTX value is not finite FP32");
        if (sym == "skew-symmetric" && r == c && val != 0)
            throw std::runtime_error("Skew-symmetric MTX diagonal must be zero");
        push(r - 1, c - 1, (float)val);
        if (sym != "general" && r != c) push(c - 1, r - 1, (float)(sym == "symmetric" ? val : -val));
    }
    if (data_line(line)) throw std::runtime_error("Extra entries after declared MTX nnz");
    return t;
}

// COO -> CSR with sorted columns; duplicates are rejected (include/csr.hpp:16-42).
CSR to_csr(const Triples& t) {
    CSR a;
    a.M = t.M;
    a.N = t.N;
    a.nnz = (int)t.v.size();
    a.row_ptr.assign((size_t)a.M + 1, 0);
    for (int r : t.r) a.row_ptr[(size_t)r + 1]++;
    for (int i = 0; i < a.M; ++i) a.row_ptr[i + 1] += a.row_ptr[i];
    std::vector<int> fill(a.row_ptr.begin(), a.row_ptr.end() - 1);
    std::vector<std::pair<int, float>> tmp(a.nnz);
    for (size_t i = 0; i < t.v.size(); ++i) tmp[fill[t.r[i]]++] = {t.c[i], t.v[i]};
    a.col.resize(a.nnz);
    a.val.resize(a.nnz);
    for (int r = 0; r < a.M; ++r) {
        auto b = tmp.begin() + a.row_ptr[r], e = tmp.begin() + a.row_ptr[r + 1];
        std::stable_sort(b, e, [](const auto& x, const auto& y) { return x.first < y.first; });
        for (auto it = b; it != e; ++it) {
            if (it != b && it->first == (it - 1)->first)
                throw std::runtime_error(
                    "Duplicate MTX coordinates are unsupported; coalesce them before benchmarking");
            a.col[it - tmp.begin()] = it->first;
            a.val[it - tmp.begin()] = it->second;
        }
    }
    return a;
}

CSR generated(const std::string& spec) {
    const size_t colon = spec.find(':');
    const int cfg = std::stoi(spec.substr(0, colon));
    const int size = colon == std::string::npos ? 0 : std::stoi(spec.substr(colon + 1));
    vcsrmc_matrix_t h = nullptr;
    if (vcsrmc_gen(cfg, size, 20260923ULL + (unsigned)cfg, &h) != 0)
        throw std::runtime_error("Unknown or failed --gen workload: " + spec);
    CSR a;
    long long nnz = 0;
    vcsrmc_gen_info(h, &a.M, &a.N, &nnz);
    a.nnz = (int)nnz;
    a.row_ptr.resize((size_t)a.M + 1);
    a.col.resize(a.nnz);
    a.val.resize(a.nnz);
    vcsrmc_gen_copy(h, a.row_ptr.data(), a.col.data(), a.val.data());
    vcsrmc_gen_free(h);
    return a;
}

int int_at_least(const char* s, long lo) {
    char* end = nullptr;
    errno = 0;
    const long v = std::strtol(s, &end, 10);
    if (errno || end == s || *end || v < lo || v > INT_MAX)
        throw std::runtime_error(std::string("Expected integer >= ") + std::to_string(lo) +
                                 ", got: " + s);
    return (int)v;
}

std::string quote(const std::string& s) {
    std::string o = "\"";
    for (char ch : s) { if (ch == '"') o += '"'; o += ch; }
    return o + '"';
}

void usage() {
    std::printf(
        "Usage: spmm_vcsr (--mtx file.mtx | --gen K[:size]) --O 128 [options]\n"
        "Algorithms: rocsparse, rocsparse_fp16, vcsr_mc (FP16 inputs, MFMA), vcsr_mc_fp32\n"
        "Options: --segw 16 --tileK 64 --repeat 10 --warmup 3 --stat mean|median\n"
        "         --reorder none|rcm --check cpu|rocsparse|none --csv --help\n"
        "         --bdist pattern|normal|uniform|wide   (B fill; random ones use a fixed seed)\n"
        "         --lenient   record a failed correctness check as FAIL instead of aborting\n"
        "         --gen K[:size]  seeded synthetic workload K = 1..5 instead of --mtx\n"
        "tileK must be one of 16, 32, 64, 128.\n");
}

int run(int argc, char** argv) {
    std::string mtx, gen, algo = "all", check = "rocsparse", reorder = "none", bdist = "pattern",
                                stat = "mean";
    int O = 128, segw = 16, tileK = 64, repeat = 10, warmup = 3;
    constexpr int bundle = 16;
    bool csv = false, lenient = false;
    static option opts[] = {
        {"mtx", required_argument, nullptr, 'm'},    {"gen", required_argument, nullptr, 'g'},
        {"O", required_argument, nullptr, 'o'},      {"segw", required_argument, nullptr, 's'},
        {"tileK", required_argument, nullptr, 't'},  {"repeat", required_argument, nullptr, 'r'},
        {"warmup", required_argument, nullptr, 'w'}, {"reorder", required_argument, nullptr, 'R'},
        {"algo", required_argument, nullptr, 'a'},   {"check", required_argument, nullptr, 'c'},
        {"csv", no_argument, nullptr, 'j'},          {"help", no_argument, nullptr, 'h'},
        {"bdist", required_argument, nullptr, 'D'},  {"lenient", no_argument, nullptr, 'L'},
        {"stat", required_argument, nullptr, 'S'},   {nullptr, 0, nullptr, 0}};
    int opt;
    while ((opt = getopt_long(argc, argv, "", opts, nullptr)) != -1) {
        switch (opt) {
            case 'm': mtx = optarg; break;
            case 'g': gen = optarg; break;
            case 'o': O = int_at_least(optarg, 1); break;
            case 's': segw = int_at_least(optarg, 1); break;
            case 't': tileK = int_at_least(optarg, 1); break;
            case 'r': repeat = int_at_least(optarg, 1); break;
            case 'w': warmup = int_at_least(optarg, 0); break;
            case 'R': reorder = optarg; break;
            case 'a': algo = optarg; break;
            case 'c': check = optarg; break;
            case 'D': bdist = optarg; break;
            case 'L': lenient = true; break;
            case 'S': stat = optarg; break;
            case 'j': csv = true; break;
            case 'h': usage(); return 0;
            default: usage(); return 2;
        }
    }
    const std::vector<std::string> known = {"all", "rocsparse", "rocsparse_fp16", "vcsr_mc",
                                            "vcsr_mc_fp32"};
    std::vector<std::string> want;
    for (size_t pos = 0;;) {
        const size_t comma = algo.find(',', pos);
        const std::string one = algo.substr(pos, comma == std::string::npos ? std::string::npos
                                                                              : comma - pos);
        if (one.empty() || std::find(known.begin(), known.end(), one) == known.end())
            throw std::runtime_error("Unknown algorithm: " + one);
        want.push_back(one);
        if (comma == std::string::npos) break;
        pos = comma + 1;
    }
    const bool all = std::find(want.begin(), want.end(), "all") != want.end();
    auto selected = [&](const char* n) {
        return all || std::find(want.begin(), want.end(), n) != want.end();
    };
    if (check != "cpu" && check != "rocsparse" && check != "none")
        throw std::runtime_error("Unknown reference: " + check);
    if ((mtx.empty() == gen.empty()) || optind != argc) { usage(); return 2; }
    if (reorder != "none" && reorder != "rcm")
        throw std::runtime_error("Unknown reordering: " + reorder);
    if (stat != "mean" && stat != "median")
        throw std::runtime_error("Unknown --stat: " + stat + " (mean|median)");
    if (tileK != 16 && tileK != 32 && tileK != 64 && tileK != 128)
        throw std::runtime_error("tileK must be one of 16, 32, 64, 128");

    CSR csr = mtx.empty() ? generated(gen) : to_csr(read_mtx(mtx));
    const std::string name = mtx.empty() ? "gen:" + gen : mtx;
    if ((size_t)csr.N * O > INT_MAX || (size_t)csr.M * O > INT_MAX || segw > INT_MAX - csr.N + 1 ||
        tileK > INT_MAX - O + 1)
        throw std::runtime_error("Dimensions exceed the kernels' 32-bit indexing limit");
    hipDeviceProp_t prop{};
    int dev = 0;
    hip_ok(hipGetDevice(&dev), "hipGetDevice");
    hip_ok(hipGetDeviceProperties(&prop, dev), "hipGetDeviceProperties");
    const size_t nB = (size_t)csr.N * O, nC = (size_t)csr.M * O;

    // B fill (src/main.cpp:161-179): the same generator and distributions, seed 20260923.
    std::vector<float> hB(nB);
    if (bdist == "pattern") {
        for (size_t i = 0; i < nB; ++i) hB[i] = float(int(i % 13) - 6) / 7.f;
    } else {
        std::mt19937_64 rng(20260923);
        if (bdist == "normal") {
            std::normal_distribution<float> d(0.f, 1.f);
            for (float& x : hB) x = d(rng);
        } else if (bdist == "uniform") {
            std::uniform_real_distribution<float> d(-1.f, 1.f);
            for (float& x : hB) x = d(rng);
        } else if (bdist == "wide") {
            std::uniform_real_distribution<float> e(-3.f, 3.f);
            std::bernoulli_distribution sgn(0.5);
            for (float& x : hB) x = (sgn(rng) ? -1.f : 1.f) * std::pow(10.f, e(rng));
        } else {
            throw std::runtime_error("Unknown --bdist: " + bdist + " (pattern|normal|uniform|wide)");
        }
    }

    // Relabelling A's columns and permuting B's rows to match leaves C = A B unchanged; done
    // once, before every algorithm and the reference result (src/main.cpp:180-183).
    if (reorder == "rcm" && csr.nnz) {
        const auto t0 = std::chrono::steady_clock::now();
        apply_column_permutation(csr, hB, O, rcm_column_order(csr));
        const double ms =
            std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        std::fprintf(stderr, "reorder rcm: %.1f ms (GPU ordering and relabelling, with copies)\n",
                     ms);
    }

    float *dB = nullptr, *dC = nullptr, *dval = nullptr;
    int *drp = nullptr, *dcol = nullptr;
    hip_ok(hipMalloc(&dB, std::max<size_t>(nB, 1) * 4), "hipMalloc");
    hip_ok(hipMalloc(&dC, std::max<size_t>(nC, 1) * 4), "hipMalloc");
    hip_ok(hipMalloc(&drp, ((size_t)csr.M + 1) * 4), "hipMalloc");
    hip_ok(hipMalloc(&dcol, std::max(csr.nnz, 1) * 4), "hipMalloc");
    hip_ok(hipMalloc(&dval, std::max(csr.nnz, 1) * 4), "hipMalloc");
    hip_ok(hipMemcpy(drp, csr.row_ptr.data(), ((size_t)csr.M + 1) * 4, hipMemcpyHostToDevice), "H2D");
    if (csr.nnz) {
        hip_ok(hipMemcpy(dcol, csr.col.data(), (size_t)csr.nnz * 4, hipMemcpyHostToDevice), "H2D");
        hip_ok(hipMemcpy(dval, csr.val.data(), (size_t)csr.nnz * 4, hipMemcpyHostToDevice), "H2D");
    }
    hip_ok(hipMemcpy(dB, hB.data(), nB * 4, hipMemcpyHostToDevice), "H2D");
    hipStream_t st;
    hip_ok(hipStreamCreate(&st), "hipStreamCreate");

    // Reference result (src/main.cpp:199-218).
    std::vector<double> ref;
    if (check != "none") ref.assign(nC, 0.0);
    if (check == "cpu") {
        for (int r = 0; r < csr.M; ++r)
            for (int p = csr.row_ptr[r]; p < csr.row_ptr[r + 1]; ++p)
                for (int k = 0; k < O; ++k)
                    ref[(size_t)r * O + k] += (double)csr.val[p] * hB[(size_t)csr.col[p] * O + k];
    } else if (check == "rocsparse" && csr.nnz) {
        hip_ok(hipMemset(dC, 0, nC * 4), "hipMemset");
        float ms = 0, setup = 0;
        if (vcsrmc_rocsparse_spmm(csr.M, csr.N, csr.nnz, drp, dcol, dval, 0, dB, 0, O, dC, 1.f, 0,
                                  st, &ms, &setup) != 0)
            throw std::runtime_error("hipSPARSE reference failed");
        std::vector<float> res(nC);
        hip_ok(hipMemcpy(res.data(), dC, nC * 4, hipMemcpyDeviceToHost), "D2H");
        ref.assign(res.begin(), res.end());
    }
    for (double v : ref)
        if (!std::isfinite(v)) throw std::runtime_error("Reference contains non-finite values");

    if (csv)
        std::printf("gpu,sm,mtx,O,segw,bundle,tileK,repeat,algo,ms,gflops,validation,rel_l2,"
                    "setup_ms,ms_mean,ms_median,convert_ms,upload_ms\n");
    else
        std::printf("Matrix: %d x %d, nnz=%d; O=%d segw=%d bundle=%d tileK=%d repeat=%d warmup=%d "
                    "reorder=%s; reference=%s\nKernel                Time (ms)      GFLOP/s   "
                    "Validation\n",
                    csr.M, csr.N, csr.nnz, O, segw, bundle, tileK, repeat, warmup, reorder.c_str(),
                    check.c_str());
    auto wall_ms = [](auto&& f) {
        const auto t0 = std::chrono::steady_clock::now();
        f();
        return std::chrono::duration<float, std::milli>(std::chrono::steady_clock::now() - t0)
            .count();
    };

    // measure (src/main.cpp:239-308)
    auto measure = [&](const char* kname, const std::function<void(float&)>& launch,
                       const float& setup_ms, float convert_ms = 0.f, float upload_ms = 0.f) {
        auto iterate = [&]() {
            hip_ok(hipMemsetAsync(dC, 0, nC * 4, st), "hipMemsetAsync");
            hip_ok(hipStreamSynchronize(st), "sync");
            float ms = 0;
            if (csr.nnz) launch(ms);
            hip_ok(hipGetLastError(), "launch");
            hip_ok(hipStreamSynchronize(st), "sync");
            if (!std::isfinite(ms) || ms < 0) throw std::runtime_error("Invalid kernel timing");
            return (double)ms;
        };
        for (int i = 0; i < warmup; ++i) iterate();
        std::vector<double> t(repeat);
        for (double& x : t) x = iterate();
        double rel = 0;
        bool failed = false;
        if (check != "none") {
            std::vector<float> res(nC);
            hip_ok(hipMemcpy(res.data(), dC, nC * 4, hipMemcpyDeviceToHost), "D2H");
            double e2 = 0, r2 = 0;
            bool nonfinite = false;
            for (size_t i = 0; i < nC; ++i) {
                if (!std::isfinite(res[i])) {
                    if (!lenient) throw std::runtime_error(std::string(kname) + ": non-finite output");
                    nonfinite = true;
                    break;
                }
                const double d = (double)res[i] - ref[i];
                e2 += d * d;
                r2 += ref[i] * ref[i];
            }
            const double err = std::sqrt(e2), norm = std::sqrt(r2);
            rel = norm > 0 ? err / norm : err;
            if (nonfinite) { rel = INFINITY; failed = true; }
            const std::string kn(kname);
            const bool half = kn == "vcsr_mc" || kn == "rocsparse_fp16";
            const double tol = (half ? 3e-3 : 1e-4) * norm + 1e-5 * std::sqrt((double)nC);
            if (!nonfinite && (err > tol || rel > (half ? 1e-1 : 1e-2))) {
                if (!lenient)
                    throw std::runtime_error(std::string(kname) +
                                             ": correctness check failed, rel_l2=" +
                                             std::to_string(rel));
                failed = true;
            }
        }
        const double mean = std::accumulate(t.begin(), t.end(), 0.0) / repeat;
        std::sort(t.begin(), t.end());
        const double median = repeat % 2 ? t[repeat / 2] : 0.5 * (t[repeat / 2 - 1] + t[repeat / 2]);
        const double ms = stat == "median" ? median : mean;
        const double gflops = ms > 0 ? 2.0 * csr.nnz * O / (ms * 1e6) : 0;
        const char* val = check == "none" ? "unchecked" : failed ? "FAIL" : "pass";
        if (csv)
            std::printf("%s,%d,%s,%d,%d,%d,%d,%d,%s,%.9g,%.9g,%s,%.9g,%.6g,%.9g,%.9g,%.6g,%.6g\n",
                        quote(prop.name).c_str(), prop.major * 10 + prop.minor, quote(name).c_str(),
                        O, segw, bundle, tileK, repeat, kname, ms, gflops, val, rel, setup_ms,
                        mean, median, convert_ms, upload_ms);
        else
            std::printf("%-20s %10.6f %12.2f   %s (rel_l2=%.3g, setup %.3f ms)\n", kname, ms, gflops,
                        val, rel, setup_ms);
        std::fflush(stdout);
    };

    if (selected("rocsparse")) {
        float setup = 0.f;
        measure("rocsparse", [&](float& ms) {
            if (vcsrmc_rocsparse_spmm(csr.M, csr.N, csr.nnz, drp, dcol, dval, 0, dB, 0, O, dC, 1.f,
                                      0, st, &ms, &setup) != 0)
                throw std::runtime_error("hipSPARSE SpMM failed");
        }, setup);
    }
    if (selected("rocsparse_fp16")) {
        // FP16 A (range-scaled) and B, FP32 compute and C; copies made outside the timing
        // (src/main.cpp:314-340).
        const float scale = half_scale(csr), inv = 1.f / scale;
        std::vector<_Float16> v16, b16;
        const float convert = wall_ms([&] {
            v16.resize(csr.nnz);
            b16.resize(nB);
            for (int i = 0; i < csr.nnz; ++i) v16[i] = (_Float16)(csr.val[i] * inv);
            for (size_t i = 0; i < nB; ++i) b16[i] = (_Float16)hB[i];
        });
        void *dv16 = nullptr, *db16 = nullptr;
        const float upload = wall_ms([&] {
            hip_ok(hipMalloc(&dv16, std::max(csr.nnz, 1) * 2), "hipMalloc");
            hip_ok(hipMalloc(&db16, std::max<size_t>(nB, 1) * 2), "hipMalloc");
            if (csr.nnz) hip_ok(hipMemcpy(dv16, v16.data(), (size_t)csr.nnz * 2, hipMemcpyHostToDevice), "H2D");
            hip_ok(hipMemcpy(db16, b16.data(), nB * 2, hipMemcpyHostToDevice), "H2D");
        });
        float lib = 0.f, setup = 0.f;
        measure("rocsparse_fp16", [&](float& ms) {
            if (vcsrmc_rocsparse_spmm(csr.M, csr.N, csr.nnz, drp, dcol, dv16, 1, db16, 1, O, dC,
                                      scale, 0, st, &ms, &lib) != 0)
                throw std::runtime_error("hipSPARSE FP16 SpMM failed");
            setup = convert + upload + lib;
        }, setup, convert, upload);
        hip_ok(hipFree(dv16), "hipFree");
        hip_ok(hipFree(db16), "hipFree");
    }
    // VCSR-MC through the drop-in surface (src/main.cpp:345-362).
    for (const bool fp32 : {false, true}) {
        const char* kname = fp32 ? "vcsr_mc_fp32" : "vcsr_mc";
        if (!selected(kname)) continue;
        if (segw != 16 && segw != 32 && segw != 48 && segw != 64) {
            std::fprintf(stderr, "Skipping %s: needs segw in {16,32,48,64}\n", kname);
            continue;
        }
        VCSRMC V;
        const float convert = wall_ms([&] { V = csr_to_vcsr_mc(csr, fp32, segw); });
        const float upload = wall_ms([&] { upload_vcsr_mc_device(V); });
        measure(kname, [&](float& ms) { run_vcsr_mc_spmm_gpu(V, dB, O, tileK, dC, st, ms); },
                convert + upload, convert, upload);
        destroy_vcsr_mc_device(st);
    }
    vcsrmc_rocsparse_release();
    hip_ok(hipStreamDestroy(st), "hipStreamDestroy");
    hip_ok(hipFree(dB), "hipFree");
    hip_ok(hipFree(dC), "hipFree");
    hip_ok(hipFree(drp), "hipFree");
    hip_ok(hipFree(dcol), "hipFree");
    hip_ok(hipFree(dval), "hipFree");
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        return run(argc, argv);
    } catch (const std::exception& e) {
        std::fprintf(stderr, "Error: %s\n", e.what());
        return 2;
    }
}
