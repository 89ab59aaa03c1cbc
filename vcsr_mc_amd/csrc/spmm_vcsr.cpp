// spmm_vcsr.cpp -- benchmark driver with the reference's command line, messages and CSV
// (MuuSeoTia/VCSR_MC src/main.cpp:33-372), over libvcsrmc.so and libvcsrmc_bench.so.
//
//   vcsr_mc / vcsr_mc_fp32     the drop-in C++ surface (include/vcsr_formats.hpp), called in the
//                              reference's sequence convert -> upload -> run -> destroy
//   rocsparse / rocsparse_fp16 hipSPARSE SpMM (libvcsrmc_bench.so)
// Input: a Matrix Market file through the drop-in reader (include/mmio.hpp, include/csr.hpp),
// or, additive, a seeded synthetic workload (--gen K[:size]).  --reorder rcm runs the GPU column
// reordering of include/reorder.hpp.  --dump-csr PATH (additive) writes the CSR as read and
// stops before any GPU call.
//
// The driver is organised as: options -> input matrix -> dense B -> device operands -> reference
// result -> for each selected kernel, the timing protocol, the validation and one report row.
#include <getopt.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cerrno>
#include <chrono>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "csr.hpp"
#include "cuda_check.hpp"
#include "mmio.hpp"
#include "reorder.hpp"
#include "vcsr_formats.hpp"
#include "vcsrmc_bench.h"

namespace {

using Clock = std::chrono::steady_clock;

double ms_since(Clock::time_point t0) {
    return std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
}

// ---- options ------------------------------------------------------------------------------
struct Options {
    std::string mtx, gen, dump_csr, write_mtx;
    std::string algo = "all", check = "rocsparse", reorder = "none", bdist = "pattern";
    std::string stat = "mean";
    int O = 128, segw = 16, tileK = 64, repeat = 10, warmup = 3;
    bool csv = false, lenient = false, help = false;
    std::vector<std::string> kernels;  // the --algo list, validated
};

// Decimal integer >= lo that fits an int, or the reference's error text.
int parse_int(const char* text, long lo) {
    errno = 0;
    char* end = nullptr;
    const long long v = std::strtoll(text, &end, 10);
    const bool whole = end != text && *end == '\0' && errno == 0;
    if (!whole || v < lo || v > INT_MAX)
        throw std::runtime_error("Expected integer >= " + std::to_string(lo) + ", got: " + text);
    return (int)v;
}

const char* const kKernelNames[] = {"all", "rocsparse", "rocsparse_fp16", "vcsr_mc",
                                    "vcsr_mc_fp32"};

std::vector<std::string> split_algorithms(const std::string& list) {
    std::vector<std::string> out;
    size_t b = 0;
    while (true) {
        size_t e = list.find(',', b);
        const std::string one = list.substr(b, e == std::string::npos ? std::string::npos : e - b);
        bool known = false;
        for (const char* k : kKernelNames) known |= one == k;
        if (!known) throw std::runtime_error("Unknown algorithm: " + one);
        out.push_back(one);
        if (e == std::string::npos) return out;
        b = e + 1;
    }
}

void print_usage() {
    std::printf(
        "Usage: spmm_vcsr (--mtx file.mtx | --gen K[:size]) --O 128 [options]\n"
        "Algorithms: rocsparse, rocsparse_fp16 (FP16 A and B, FP32 compute and C),\n"
        "            vcsr_mc (FP16 inputs, MFMA), vcsr_mc_fp32 (FP32 operands, FP32 MFMA)\n"
        "Options: --segw 16 --tileK 64 --repeat 10 --warmup 3 --stat mean|median\n"
        "         --reorder none|rcm --check cpu|rocsparse|none --csv --help\n"
        "         --bdist pattern|normal|uniform|wide   (B fill; random ones use a fixed seed)\n"
        "         --lenient   record a failed correctness check as FAIL instead of aborting\n"
        "         --gen K[:size]  seeded synthetic workload K = 1..5 instead of --mtx\n"
        "         --dump-csr PATH  write the CSR as read (PATH - = stdout) and stop\n"
        "         --write-mtx PATH write the input as a Matrix Market file and stop\n"
        "tileK must be one of 16, 32, 64, 128.\n");
}

// Returns false when the command line asks for usage with exit status 2.
bool parse_options(int argc, char** argv, Options& o) {
    enum { kMtx = 256, kGen, kO, kSegw, kTileK, kRepeat, kWarmup, kReorder, kAlgo, kCheck, kCsv,
           kHelp, kBdist, kLenient, kStat, kDump, kWriteMtx };
    static const option table[] = {
        {"mtx", required_argument, nullptr, kMtx},        {"gen", required_argument, nullptr, kGen},
        {"O", required_argument, nullptr, kO},            {"segw", required_argument, nullptr, kSegw},
        {"tileK", required_argument, nullptr, kTileK},    {"repeat", required_argument, nullptr, kRepeat},
        {"warmup", required_argument, nullptr, kWarmup},  {"reorder", required_argument, nullptr, kReorder},
        {"algo", required_argument, nullptr, kAlgo},      {"check", required_argument, nullptr, kCheck},
        {"csv", no_argument, nullptr, kCsv},              {"help", no_argument, nullptr, kHelp},
        {"bdist", required_argument, nullptr, kBdist},    {"lenient", no_argument, nullptr, kLenient},
        {"stat", required_argument, nullptr, kStat},      {"dump-csr", required_argument, nullptr, kDump},
        {"write-mtx", required_argument, nullptr, kWriteMtx}, {nullptr, 0, nullptr, 0}};
    for (int c; (c = getopt_long(argc, argv, "", table, nullptr)) != -1;) {
        switch (c) {
            case kMtx: o.mtx = optarg; break;
            case kGen: o.gen = optarg; break;
            case kO: o.O = parse_int(optarg, 1); break;
            case kSegw: o.segw = parse_int(optarg, 1); break;
            case kTileK: o.tileK = parse_int(optarg, 1); break;
            case kRepeat: o.repeat = parse_int(optarg, 1); break;
            case kWarmup: o.warmup = parse_int(optarg, 0); break;
            case kReorder: o.reorder = optarg; break;
            case kAlgo: o.algo = optarg; break;
            case kCheck: o.check = optarg; break;
            case kCsv: o.csv = true; break;
            case kHelp: o.help = true; return true;
            case kBdist: o.bdist = optarg; break;
            case kLenient: o.lenient = true; break;
            case kStat: o.stat = optarg; break;
            case kDump: o.dump_csr = optarg; break;
            case kWriteMtx: o.write_mtx = optarg; break;
            default: return false;
        }
    }
    o.kernels = split_algorithms(o.algo);
    if (o.check != "cpu" && o.check != "rocsparse" && o.check != "none")
        throw std::runtime_error("Unknown reference: " + o.check);
    if (o.mtx.empty() == o.gen.empty() || optind != argc) return false;
    if (o.reorder != "none" && o.reorder != "rcm")
        throw std::runtime_error("Unknown reordering: " + o.reorder);
    if (o.stat != "mean" && o.stat != "median")
        throw std::runtime_error("Unknown --stat: " + o.stat + " (mean|median)");
    if (o.tileK != 16 && o.tileK != 32 && o.tileK != 64 && o.tileK != 128)
        throw std::runtime_error("tileK must be one of 16, 32, 64, 128");
    return true;
}

bool wants(const Options& o, const char* name) {
    for (const std::string& k : o.kernels)
        if (k == "all" || k == name) return true;
    return false;
}

// ---- input ---------------------------------------------------------------------------------
CSR synthetic_csr(const std::string& spec) {
    const size_t colon = spec.find(':');
    const int config = parse_int(spec.substr(0, colon).c_str(), 1);
    const int size = colon == std::string::npos ? 0 : parse_int(spec.c_str() + colon + 1, 0);
    vcsrmc_matrix_t m = nullptr;
    if (vcsrmc_gen(config, size, 20260923ULL + (unsigned)config, &m) != 0)
        throw std::runtime_error("Unknown or failed --gen workload: " + spec);
    std::unique_ptr<vcsrmc_matrix_s, int (*)(vcsrmc_matrix_t)> guard(m, vcsrmc_gen_free);
    CSR a;
    long long nnz = 0;
    vcsrmc_gen_info(m, &a.M, &a.N, &nnz);
    a.nnz = (int)nnz;
    a.row_ptr.resize((size_t)a.M + 1);
    a.col.resize((size_t)a.nnz);
    a.val.resize((size_t)a.nnz);
    vcsrmc_gen_copy(m, a.row_ptr.data(), a.col.data(), a.val.data());
    return a;
}

// The CSR as text: "OK M N nnz", then row_ptr, col, and the values' bit patterns, one line each.
void dump_csr(const CSR& a, const std::string& path) {
    std::FILE* f = path == "-" ? stdout : std::fopen(path.c_str(), "w");
    if (!f) throw std::runtime_error("Cannot write " + path);
    std::fprintf(f, "OK %d %d %d\n", a.M, a.N, a.nnz);
    for (int x : a.row_ptr) std::fprintf(f, "%d ", x);
    std::fprintf(f, "\n");
    for (int x : a.col) std::fprintf(f, "%d ", x);
    std::fprintf(f, "\n");
    for (float v : a.val) {
        uint32_t u;
        std::memcpy(&u, &v, sizeof u);
        std::fprintf(f, "%08x ", u);
    }
    std::fprintf(f, "\n");
    if (f != stdout) std::fclose(f);
}

// The CSR as a general real Matrix Market file; 9 significant digits give back every float.
void write_mtx(const CSR& a, const std::string& path) {
    std::FILE* f = std::fopen(path.c_str(), "w");
    if (!f) throw std::runtime_error("Cannot write " + path);
    std::vector<char> buf(1 << 22);
    std::setvbuf(f, buf.data(), _IOFBF, buf.size());
    std::fprintf(f, "%%%%MatrixMarket matrix coordinate real general\n%d %d %d\n", a.M, a.N, a.nnz);
    for (int r = 0; r < a.M; ++r)
        for (int p = a.row_ptr[r]; p < a.row_ptr[r + 1]; ++p)
            std::fprintf(f, "%d %d %.9g\n", r + 1, a.col[p] + 1, (double)a.val[p]);
    if (std::fclose(f) != 0) throw std::runtime_error("Cannot write " + path);
}

// Dense B, row-major N x O (src/main.cpp:161-179): "pattern" cycles 13 values in [-6/7, 6/7];
// the random fills draw from one std::mt19937_64 seeded 20260923 in element order.
std::vector<float> make_b(size_t n, const std::string& dist) {
    std::vector<float> b(n);
    if (dist == "pattern") {
        for (size_t i = 0; i < n; ++i) b[i] = (float)((int)(i % 13) - 6) / 7.0f;
        return b;
    }
    std::mt19937_64 gen(20260923);
    if (dist == "normal") {
        std::normal_distribution<float> d(0.0f, 1.0f);
        std::generate(b.begin(), b.end(), [&] { return d(gen); });
    } else if (dist == "uniform") {
        std::uniform_real_distribution<float> d(-1.0f, 1.0f);
        std::generate(b.begin(), b.end(), [&] { return d(gen); });
    } else if (dist == "wide") {
        std::uniform_real_distribution<float> exponent(-3.0f, 3.0f);
        std::bernoulli_distribution negative(0.5);
        std::generate(b.begin(), b.end(), [&] {
            const float s = negative(gen) ? -1.0f : 1.0f;  // sign drawn before the magnitude
            return s * std::pow(10.0f, exponent(gen));
        });
    } else {
        throw std::runtime_error("Unknown --bdist: " + dist + " (pattern|normal|uniform|wide)");
    }
    return b;
}

// ---- device operands ------------------------------------------------------------------------
template <typename T>
class DeviceArray {
public:
    explicit DeviceArray(size_t n) : n_(n) { CUDA_CHECK(hipMalloc(&p_, std::max<size_t>(n, 1) * sizeof(T))); }
    DeviceArray(const DeviceArray&) = delete;
    DeviceArray& operator=(const DeviceArray&) = delete;
    ~DeviceArray() { (void)hipFree(p_); }
    T* get() const { return p_; }
    size_t size() const { return n_; }
    void upload(const T* h, size_t n) {
        if (n) CUDA_CHECK(hipMemcpy(p_, h, n * sizeof(T), hipMemcpyHostToDevice));
    }
    std::vector<T> download() const {
        std::vector<T> h(n_);
        if (n_) CUDA_CHECK(hipMemcpy(h.data(), p_, n_ * sizeof(T), hipMemcpyDeviceToHost));
        return h;
    }

private:
    T* p_ = nullptr;
    size_t n_;
};

struct Operands {
    const CSR& a;
    int O;
    hipStream_t stream = nullptr;
    DeviceArray<int> row_ptr, col;
    DeviceArray<float> val, B, C;
    Operands(const CSR& csr, const std::vector<float>& hB, int O_)
        : a(csr), O(O_), row_ptr((size_t)csr.M + 1), col((size_t)csr.nnz), val((size_t)csr.nnz),
          B(hB.size()), C((size_t)csr.M * O_) {
        row_ptr.upload(csr.row_ptr.data(), row_ptr.size());
        col.upload(csr.col.data(), col.size());
        val.upload(csr.val.data(), val.size());
        B.upload(hB.data(), hB.size());
        CUDA_CHECK(hipStreamCreate(&stream));
    }
    ~Operands() { (void)hipStreamDestroy(stream); }
};

// ---- kernels ---------------------------------------------------------------------------------
// One algorithm of the driver: launch() runs one SpMM into C (C zeroed before) and returns its
// event-timed milliseconds; setup / convert / upload are reported beside the timing.
struct Kernel {
    const char* name;
    bool half_inputs;  // FP16 operands: the looser validation bound
    double setup_ms = 0, convert_ms = 0, upload_ms = 0;
    Kernel(const char* n, bool h) : name(n), half_inputs(h) {}
    virtual ~Kernel() = default;
    virtual float launch(Operands& d) = 0;
};

struct RocsparseKernel : Kernel {
    RocsparseKernel() : Kernel("rocsparse", false) {}
    float launch(Operands& d) override {
        float ms = 0, setup = 0;
        if (vcsrmc_rocsparse_spmm(d.a.M, d.a.N, d.a.nnz, d.row_ptr.get(), d.col.get(),
                                  d.val.get(), 0, d.B.get(), 0, d.O, d.C.get(), 1.0f, 0, d.stream,
                                  &ms, &setup) != 0)
            throw std::runtime_error("hipSPARSE SpMM failed");
        setup_ms = setup;
        return ms;
    }
};

// FP16 A (divided by half_scale, undone through alpha) and FP16 B, FP32 compute and C; the
// copies are made once, outside the timing (src/main.cpp:314-340).
struct RocsparseFp16Kernel : Kernel {
    std::unique_ptr<DeviceArray<_Float16>> val16, b16;
    float scale = 1.0f;
    double lib_setup = 0;
    RocsparseFp16Kernel(const CSR& a, const std::vector<float>& hB) : Kernel("rocsparse_fp16", true) {
        scale = half_scale(a);
        const float inv = 1.0f / scale;
        std::vector<_Float16> v16, h16;
        auto t0 = Clock::now();
        v16.resize(a.val.size());
        h16.resize(hB.size());
        std::transform(a.val.begin(), a.val.end(), v16.begin(),
                       [inv](float v) { return (_Float16)(v * inv); });
        std::transform(hB.begin(), hB.end(), h16.begin(), [](float v) { return (_Float16)v; });
        convert_ms = ms_since(t0);
        t0 = Clock::now();
        val16 = std::make_unique<DeviceArray<_Float16>>(v16.size());
        b16 = std::make_unique<DeviceArray<_Float16>>(h16.size());
        val16->upload(v16.data(), v16.size());
        b16->upload(h16.data(), h16.size());
        upload_ms = ms_since(t0);
    }
    float launch(Operands& d) override {
        float ms = 0, setup = 0;
        if (vcsrmc_rocsparse_spmm(d.a.M, d.a.N, d.a.nnz, d.row_ptr.get(), d.col.get(),
                                  val16->get(), 1, b16->get(), 1, d.O, d.C.get(), scale, 0,
                                  d.stream, &ms, &setup) != 0)
            throw std::runtime_error("hipSPARSE FP16 SpMM failed");
        lib_setup = setup;
        setup_ms = convert_ms + upload_ms + lib_setup;
        return ms;
    }
};

// The drop-in surface, as the reference's driver calls it (src/main.cpp:356-361).
struct VcsrKernel : Kernel {
    VCSRMC V;
    int tileK;
    VcsrKernel(const CSR& a, bool fp32, int segw, int tileK_)
        : Kernel(fp32 ? "vcsr_mc_fp32" : "vcsr_mc", !fp32), tileK(tileK_) {
        auto t0 = Clock::now();
        V = csr_to_vcsr_mc(a, fp32, segw);
        convert_ms = ms_since(t0);
        t0 = Clock::now();
        upload_vcsr_mc_device(V);
        upload_ms = ms_since(t0);
        setup_ms = convert_ms + upload_ms;
    }
    ~VcsrKernel() override { destroy_vcsr_mc_device(nullptr); }
    float launch(Operands& d) override {
        float ms = 0;
        run_vcsr_mc_spmm_gpu(V, d.B.get(), d.O, tileK, d.C.get(), d.stream, ms);
        return ms;
    }
};

// ---- protocol, validation, report -----------------------------------------------------------
// `warmup` discarded launches, then `repeat` timed ones; C is zeroed and the stream drained
// before each (src/main.cpp:241-256).
std::vector<double> time_launches(Kernel& k, Operands& d, int warmup, int repeat) {
    std::vector<double> t;
    for (int i = 0; i < warmup + repeat; ++i) {
        CUDA_CHECK(hipMemsetAsync(d.C.get(), 0, d.C.size() * sizeof(float), d.stream));
        CUDA_CHECK(hipStreamSynchronize(d.stream));
        const float ms = d.a.nnz ? k.launch(d) : 0.0f;
        CUDA_CHECK(hipGetLastError());
        CUDA_CHECK(hipStreamSynchronize(d.stream));
        if (!(ms >= 0.0f) || std::isinf(ms)) throw std::runtime_error("Invalid kernel timing");
        if (i >= warmup) t.push_back(ms);
    }
    return t;
}

struct Outcome {
    double rel_l2 = 0;
    bool failed = false;
};

// Relative L2 error of C against the reference, and the reference's two-sided bound
// (src/main.cpp:257-291): error <= tol_rel * ||ref|| + 1e-5 sqrt(|C|) and rel_l2 <= cap, with
// (tol_rel, cap) = (3e-3, 1e-1) for FP16 inputs, (1e-4, 1e-2) otherwise.  A non-finite output,
// or a result outside the bound, aborts unless lenient (then FAIL).
Outcome validate(const Kernel& k, const std::vector<float>& got, const std::vector<double>& ref,
                 bool lenient) {
    Outcome v;
    double err2 = 0, ref2 = 0;
    for (size_t i = 0; i < got.size(); ++i) {
        if (!std::isfinite(got[i])) {
            if (!lenient) throw std::runtime_error(std::string(k.name) + ": non-finite output");
            v.rel_l2 = INFINITY;
            v.failed = true;
            return v;
        }
        const double e = (double)got[i] - ref[i];
        err2 += e * e;
        ref2 += ref[i] * ref[i];
    }
    const double err = std::sqrt(err2), norm = std::sqrt(ref2);
    v.rel_l2 = norm > 0 ? err / norm : err;
    const double tol_rel = k.half_inputs ? 3e-3 : 1e-4, cap = k.half_inputs ? 1e-1 : 1e-2;
    const double bound = tol_rel * norm + 1e-5 * std::sqrt((double)got.size());
    if (err > bound || v.rel_l2 > cap) {
        if (!lenient)
            throw std::runtime_error(std::string(k.name) + ": correctness check failed, rel_l2=" +
                                     std::to_string(v.rel_l2));
        v.failed = true;
    }
    return v;
}

std::string csv_field(const std::string& s) {
    std::string q = "\"";
    for (char ch : s) q += ch == '"' ? std::string("\"\"") : std::string(1, ch);
    return q + "\"";
}

struct Report {
    const Options& o;
    const CSR& a;
    std::string source, device;
    int sm = 0;

    void header() const {
        if (o.csv) {
            std::printf("gpu,sm,mtx,O,segw,bundle,tileK,repeat,algo,ms,gflops,validation,rel_l2,"
                        "setup_ms,ms_mean,ms_median,convert_ms,upload_ms\n");
            return;
        }
        std::printf("Matrix: %d x %d, nnz=%d; O=%d segw=%d bundle=%d tileK=%d repeat=%d warmup=%d "
                    "reorder=%s; reference=%s\n",
                    a.M, a.N, a.nnz, o.O, o.segw, 16, o.tileK, o.repeat, o.warmup,
                    o.reorder.c_str(), o.check.c_str());
        std::printf("Kernel                Time (ms)      GFLOP/s   Validation\n");
    }

    void row(const Kernel& k, std::vector<double> t, const Outcome& v) const {
        double sum = 0;
        for (double x : t) sum += x;
        const double mean = sum / (double)t.size();
        std::sort(t.begin(), t.end());
        const size_t h = t.size() / 2;
        const double median = t.size() % 2 ? t[h] : 0.5 * (t[h - 1] + t[h]);
        const double ms = o.stat == "median" ? median : mean;
        const double gflops = ms > 0 ? 2.0 * (double)a.nnz * o.O / (ms * 1e6) : 0.0;
        const char* outcome = o.check == "none" ? "unchecked" : v.failed ? "FAIL" : "pass";
        if (o.csv)
            std::printf("%s,%d,%s,%d,%d,%d,%d,%d,%s,%.9g,%.9g,%s,%.9g,%.6g,%.9g,%.9g,%.6g,%.6g\n",
                        csv_field(device).c_str(), sm, csv_field(source).c_str(), o.O, o.segw, 16,
                        o.tileK, o.repeat, k.name, ms, gflops, outcome, v.rel_l2, k.setup_ms, mean,
                        median, k.convert_ms, k.upload_ms);
        else
            std::printf("%-20s %10.6f %12.2f   %s (rel_l2=%.3g, setup %.3f ms)\n", k.name, ms,
                        gflops, outcome, v.rel_l2, k.setup_ms);
        std::fflush(stdout);
    }
};

// ---- the run --------------------------------------------------------------------------------
int run(int argc, char** argv) {
    Options o;
    if (!parse_options(argc, argv, o)) {
        print_usage();
        return 2;
    }
    if (o.help) {
        print_usage();
        return 0;
    }
    CSR a = o.mtx.empty() ? synthetic_csr(o.gen) : coo_to_csr(read_matrix_market_coo(o.mtx));
    if (!o.dump_csr.empty()) {
        dump_csr(a, o.dump_csr);
        return 0;
    }
    if (!o.write_mtx.empty()) {
        write_mtx(a, o.write_mtx);
        return 0;
    }
    // The kernels index B and C with 32-bit offsets.
    if ((size_t)a.N * o.O > INT_MAX || (size_t)a.M * o.O > INT_MAX ||
        o.segw > INT_MAX - a.N + 1 || o.tileK > INT_MAX - o.O + 1)
        throw std::runtime_error("Dimensions exceed the kernels' 32-bit indexing limit");
    std::vector<float> hB = make_b((size_t)a.N * o.O, o.bdist);
    int dev = 0;
    hipDeviceProp_t prop{};
    CUDA_CHECK(hipGetDevice(&dev));
    CUDA_CHECK(hipGetDeviceProperties(&prop, dev));

    // Relabelling A's columns and permuting B's rows to match leaves A.B unchanged; done once,
    // before every kernel and the reference result (src/main.cpp:180-183).
    if (o.reorder == "rcm" && a.nnz) {
        const auto t0 = Clock::now();
        apply_column_permutation(a, hB, o.O, rcm_column_order(a));
        std::fprintf(stderr, "reorder rcm: %.1f ms (GPU ordering and relabelling, with copies)\n",
                     ms_since(t0));
    }
    Operands d(a, hB, o.O);

    // Reference result, outside every timing (src/main.cpp:199-218).
    std::vector<double> ref;
    if (o.check == "cpu") {
        ref.assign((size_t)a.M * o.O, 0.0);
        for (int r = 0; r < a.M; ++r) {
            double* out = &ref[(size_t)r * o.O];
            for (int p = a.row_ptr[r]; p < a.row_ptr[r + 1]; ++p) {
                const double v = a.val[p];
                const float* brow = &hB[(size_t)a.col[p] * o.O];
                for (int k = 0; k < o.O; ++k) out[k] += v * brow[k];
            }
        }
    } else if (o.check == "rocsparse") {
        ref.assign((size_t)a.M * o.O, 0.0);
        if (a.nnz) {
            CUDA_CHECK(hipMemset(d.C.get(), 0, d.C.size() * sizeof(float)));
            RocsparseKernel().launch(d);
            CUDA_CHECK(hipStreamSynchronize(d.stream));
            const std::vector<float> c = d.C.download();
            std::copy(c.begin(), c.end(), ref.begin());
        }
    }
    if (std::any_of(ref.begin(), ref.end(), [](double x) { return !std::isfinite(x); }))
        throw std::runtime_error("Reference contains non-finite values");

    Report rep{o, a, o.mtx.empty() ? "gen:" + o.gen : o.mtx, prop.name, prop.major * 10 + prop.minor};
    rep.header();
    auto measure = [&](Kernel& k) {
        const std::vector<double> t = time_launches(k, d, o.warmup, o.repeat);
        const Outcome v = o.check == "none" ? Outcome{} : validate(k, d.C.download(), ref, o.lenient);
        rep.row(k, t, v);
    };
    if (wants(o, "rocsparse")) {
        RocsparseKernel k;
        measure(k);
    }
    if (wants(o, "rocsparse_fp16")) {
        RocsparseFp16Kernel k(a, hB);
        measure(k);
    }
    for (const bool fp32 : {false, true}) {
        const char* name = fp32 ? "vcsr_mc_fp32" : "vcsr_mc";
        if (!wants(o, name)) continue;
        if (o.segw != 16 && o.segw != 32 && o.segw != 48 && o.segw != 64) {
            std::fprintf(stderr, "Skipping %s: needs segw in {16,32,48,64}\n", name);
            continue;
        }
        VcsrKernel k(a, fp32, o.segw, o.tileK);
        measure(k);
    }
    vcsrmc_rocsparse_release();
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
