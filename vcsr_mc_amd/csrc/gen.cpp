// gen.cpp -- seeded synthetic matrices for the benchmark workloads (include/vcsrmc_bench.h).
//
// All randomness is std::mt19937_64 (whose output sequence the C++ standard fixes) with the
// distribution transforms written out here, since std::*_distribution is implementation
// defined.  Large draws are split into fixed blocks with their own engines, so results do not
// depend on the number of threads.
#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <new>
#include <random>
#include <stdexcept>
#include <vector>

#include "vcsrmc_bench.h"

struct vcsrmc_matrix_s {
    int M = 0, N = 0;
    std::vector<int> row_ptr, col;
    std::vector<float> val;
};

namespace {

using Engine = std::mt19937_64;

inline double uniform01(Engine& e) { return (double)(e() >> 11) * (1.0 / 9007199254740992.0); }
inline uint64_t uniform_int(Engine& e, uint64_t m) {  // [0, m)
    return (uint64_t)(((unsigned __int128)e() * m) >> 64);
}
inline float uniform_pm1(Engine& e) { return (float)(2.0 * uniform01(e) - 1.0); }
inline float normal01(Engine& e) {
    const double u1 = 1.0 - uniform01(e);  // (0, 1]
    const double u2 = uniform01(e);
    return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
}
int poisson(Engine& e, double lambda) {  // Knuth's product-of-uniforms method
    const double L = std::exp(-lambda);
    int k = 0;
    double p = 1.0;
    do {
        ++k;
        p *= uniform01(e);
    } while (p > L);
    return k - 1;
}

// Round to the nearest binary16 (ties to even) and back.
float round_f16(float x) {
    uint32_t f;
    std::memcpy(&f, &x, 4);
    const uint32_t bexp = (f >> 23) & 0xff;
    if (bexp == 0xff) return x;
    const int e = (int)bexp - 112;
    uint32_t out;
    if (e >= 31) {
        out = (f & 0x80000000u) | 0x7f800000u;
    } else if (e >= 1) {
        uint32_t r = f & ~0x1fffu;
        const uint32_t rem = f & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (f & 0x2000u))) r += 0x2000u;
        // an exponent carry past binary16's range becomes Inf
        if ((int)((r >> 23) & 0xff) - 112 >= 31) r = (f & 0x80000000u) | 0x7f800000u;
        out = r;
    } else {
        // subnormal binary16: quantum 2^-24
        const double q = std::ldexp(1.0, -24);
        const double v = std::nearbyint((double)x / q) * q;  // nearbyint: ties to even
        float y = (float)v;
        std::memcpy(&out, &y, 4);
        out |= f & 0x80000000u;
    }
    float y;
    std::memcpy(&y, &out, 4);
    return y;
}

// k distinct values of [0, n), sorted (Floyd's algorithm).
std::vector<int> floyd_sample(Engine& e, int n, int k) {
    std::vector<int> s;
    s.reserve(k);
    for (int j = n - k; j < n; ++j) {
        const int t = (int)uniform_int(e, (uint64_t)j + 1);
        if (std::find(s.begin(), s.end(), t) == s.end()) s.push_back(t);
        else s.push_back(j);
    }
    std::sort(s.begin(), s.end());
    return s;
}

Engine block_engine(uint64_t seed, uint64_t stream, uint64_t block) {
    std::seed_seq sq{(uint32_t)seed, (uint32_t)(seed >> 32), (uint32_t)stream, (uint32_t)block,
                     (uint32_t)(block >> 32)};
    return Engine(sq);
}

// CSR from (row, col) pairs: bucket by row, sort each row, drop duplicates.
void csr_from_pairs(vcsrmc_matrix_s& A, int M, int N, const std::vector<int>& r,
                    const std::vector<int>& c) {
    const long long E = (long long)r.size();
    std::vector<long long> cnt((size_t)M + 1, 0);
    for (long long i = 0; i < E; ++i) ++cnt[(size_t)r[i] + 1];
    for (int i = 0; i < M; ++i) cnt[i + 1] += cnt[i];
    std::vector<int> tmp((size_t)E);
    {
        std::vector<long long> fill(cnt.begin(), cnt.end() - 1);
        for (long long i = 0; i < E; ++i) tmp[fill[r[i]]++] = c[i];
    }
    std::vector<int> keep((size_t)M, 0);
#pragma omp parallel for schedule(dynamic, 1024)
    for (int i = 0; i < M; ++i) {
        auto b = tmp.begin() + cnt[i], e = tmp.begin() + cnt[i + 1];
        std::sort(b, e);
        keep[i] = (int)(std::unique(b, e) - b);
    }
    A.M = M;
    A.N = N;
    A.row_ptr.assign((size_t)M + 1, 0);
    for (int i = 0; i < M; ++i) A.row_ptr[i + 1] = A.row_ptr[i] + keep[i];
    A.col.resize((size_t)A.row_ptr[M]);
#pragma omp parallel for schedule(dynamic, 1024)
    for (int i = 0; i < M; ++i)
        std::copy(tmp.begin() + cnt[i], tmp.begin() + cnt[i] + keep[i], A.col.begin() + A.row_ptr[i]);
}

void fill_values(vcsrmc_matrix_s& A, uint64_t seed, int dist, bool f16) {
    const long long n = (long long)A.col.size();
    A.val.resize((size_t)n);
    const long long blk = 1 << 20;
    const long long nb = (n + blk - 1) / blk;
#pragma omp parallel for schedule(dynamic, 1)
    for (long long b = 0; b < nb; ++b) {
        Engine e = block_engine(seed, 7, (uint64_t)b);
        const long long end = std::min(n, (b + 1) * blk);
        for (long long i = b * blk; i < end; ++i) {
            float v = dist == 0 ? uniform_pm1(e) : normal01(e);
            A.val[i] = f16 ? round_f16(v) : v;
        }
    }
}

void gen_uniform(vcsrmc_matrix_s& A, int n, uint64_t seed) {
    Engine e = block_engine(seed, 1, 0);
    A.M = A.N = n;
    A.row_ptr.assign((size_t)n + 1, 0);
    for (int r = 0; r < n; ++r) {
        const int k = std::min(std::max(poisson(e, 16.0), 0), n);
        const std::vector<int> cols = floyd_sample(e, n, k);
        A.col.insert(A.col.end(), cols.begin(), cols.end());
        A.row_ptr[r + 1] = (int)A.col.size();
    }
    fill_values(A, seed, 0, false);
}

// Power-law graph: degrees Zipf(2.1) on [1, 1383], paired by the configuration model
// (shuffled stubs), self-loops and repeated pairs dropped, pattern symmetric.  The degree scale
// is calibrated so that the matrix holds about 368,000 * n / 36,692 nonzeros after the drops:
// the stub total aimed at is corrected by the ratio of the nonzeros it gave, a few times, and
// the closest matrix is kept (every attempt pairs with the same shuffle stream, so the result
// depends on the seed only).
void gen_powerlaw(vcsrmc_matrix_s& A, int n, uint64_t seed) {
    Engine e = block_engine(seed, 2, 0);
    const int dmax = 1383;
    const double alpha = 2.1;
    std::vector<double> cdf(dmax);
    double acc = 0.0;
    for (int k = 1; k <= dmax; ++k) { acc += std::pow((double)k, -alpha); cdf[k - 1] = acc; }
    std::vector<int> z((size_t)n);
    for (int i = 0; i < n; ++i) {
        const double u = uniform01(e) * acc;
        z[i] = (int)(std::upper_bound(cdf.begin(), cdf.end(), u) - cdf.begin()) + 1;
        if (z[i] > dmax) z[i] = dmax;
    }
    const Engine pairing = e;  // shuffle stream shared by every attempt
    const double goal = 368000.0 * (double)n / 36692.0;
    auto degree = [&](double s, int i) {
        return std::min<long long>(std::max<long long>(std::llround(s * z[i]), 1), dmax);
    };
    // Degree scale whose stub total first reaches `target` (bisection on a monotone sum).
    auto scale_for = [&](double target) {
        double lo = 0.0, hi = 1000.0;
        for (int it = 0; it < 100; ++it) {
            const double mid = 0.5 * (lo + hi);
            long long t = 0;
            for (int i = 0; i < n; ++i) t += degree(mid, i);
            if (t < target) lo = mid; else hi = mid;
        }
        return hi;
    };
    auto attempt = [&](double s, vcsrmc_matrix_s& out) {
        Engine sh = pairing;
        std::vector<int> stubs;
        for (int i = 0; i < n; ++i)
            for (long long j = degree(s, i); j > 0; --j) stubs.push_back(i);
        if (stubs.size() & 1) stubs.pop_back();
        for (size_t i = stubs.size(); i > 1; --i) std::swap(stubs[i - 1], stubs[uniform_int(sh, i)]);
        std::vector<int> r, c;
        for (size_t i = 0; i + 1 < stubs.size(); i += 2) {
            const int u = stubs[i], v = stubs[i + 1];
            if (u == v) continue;
            r.push_back(u); c.push_back(v);
            r.push_back(v); c.push_back(u);
        }
        csr_from_pairs(out, n, n, r, c);
        return (double)out.col.size();
    };
    double target = goal, best_gap = -1.0;
    for (int it = 0; it < 4; ++it) {
        vcsrmc_matrix_s T;
        const double got = attempt(scale_for(target), T);
        const double gap = std::fabs(got - goal);
        if (best_gap < 0.0 || gap < best_gap) {
            best_gap = gap;
            A = std::move(T);
        }
        if (got <= 0.0 || gap <= 1e-3 * goal) break;
        target *= goal / got;
    }
    fill_values(A, seed, 0, true);
}

void gen_stencil(vcsrmc_matrix_s& A, int g) {
    const long long n = (long long)g * g * g;
    if (n >= INT32_MAX) throw std::runtime_error("stencil too large");
    A.M = A.N = (int)n;
    A.row_ptr.assign((size_t)n + 1, 0);
    for (long long r = 0; r < n; ++r) {
        const int i = (int)(r / ((long long)g * g)), j = (int)((r / g) % g), k = (int)(r % g);
        int cnt = 0;
        for (int di = -1; di <= 1; ++di)
            for (int dj = -1; dj <= 1; ++dj)
                for (int dk = -1; dk <= 1; ++dk)
                    cnt += (unsigned)(i + di) < (unsigned)g && (unsigned)(j + dj) < (unsigned)g &&
                           (unsigned)(k + dk) < (unsigned)g;
        A.row_ptr[r + 1] = A.row_ptr[r] + cnt;
    }
    A.col.resize((size_t)A.row_ptr[n]);
    A.val.resize((size_t)A.row_ptr[n]);
#pragma omp parallel for schedule(static)
    for (long long r = 0; r < n; ++r) {
        const int i = (int)(r / ((long long)g * g)), j = (int)((r / g) % g), k = (int)(r % g);
        int p = A.row_ptr[r];
        for (int di = -1; di <= 1; ++di)
            for (int dj = -1; dj <= 1; ++dj)
                for (int dk = -1; dk <= 1; ++dk) {
                    if ((unsigned)(i + di) >= (unsigned)g || (unsigned)(j + dj) >= (unsigned)g ||
                        (unsigned)(k + dk) >= (unsigned)g)
                        continue;
                    A.col[p] = (int)(r + (long long)di * g * g + (long long)dj * g + dk);
                    A.val[p] = (di == 0 && dj == 0 && dk == 0) ? 26.0f : -1.0f;
                    ++p;
                }
    }
}

void gen_block(vcsrmc_matrix_s& A, int nb, uint64_t seed) {
    Engine e = block_engine(seed, 4, 0);
    const long long n = 32LL * nb;
    if (n >= INT32_MAX) throw std::runtime_error("block matrix too large");
    A.M = A.N = (int)n;
    const int per = std::min(4, nb);
    std::vector<std::vector<int>> bcols((size_t)nb);
    for (int b = 0; b < nb; ++b) bcols[b] = floyd_sample(e, nb, per);
    A.row_ptr.assign((size_t)n + 1, 0);
    for (long long r = 0; r < n; ++r) A.row_ptr[r + 1] = A.row_ptr[r] + 32 * per;
    A.col.resize((size_t)A.row_ptr[n]);
#pragma omp parallel for schedule(static)
    for (long long r = 0; r < n; ++r) {
        int p = A.row_ptr[r];
        for (int bc : bcols[r / 32])
            for (int j = 0; j < 32; ++j) A.col[p++] = 32 * bc + j;
    }
    fill_values(A, seed, 1, true);
}

void gen_rmat(vcsrmc_matrix_s& A, int scale, uint64_t seed) {
    if (scale < 1 || scale > 30) throw std::runtime_error("R-MAT scale out of range");
    const long long n = 1LL << scale;
    const long long E = 16 * n;
    const double a = 0.57, b = 0.19, c = 0.19;
    std::vector<int> r((size_t)E), cc((size_t)E);
    const int nblk = 256;
#pragma omp parallel for schedule(dynamic, 1)
    for (int blk = 0; blk < nblk; ++blk) {
        Engine e = block_engine(seed, 5, (uint64_t)blk);
        const long long b0 = E * blk / nblk, b1 = E * (blk + 1) / nblk;
        for (long long i = b0; i < b1; ++i) {
            long long row = 0, col = 0;
            for (int lvl = 0; lvl < scale; ++lvl) {
                const double u = uniform01(e);
                const int rb = u >= a + b;                      // quadrants c, d
                const int cb = (u >= a && u < a + b) || u >= a + b + c;  // quadrants b, d
                row = (row << 1) | rb;
                col = (col << 1) | cb;
            }
            r[i] = (int)row;
            cc[i] = (int)col;
        }
    }
    csr_from_pairs(A, (int)n, (int)n, r, cc);
    fill_values(A, seed, 0, true);
}

}  // namespace

extern "C" {

int vcsrmc_gen(int config, int size, unsigned long long seed, vcsrmc_matrix_t* out) {
    if (!out) return 1;
    *out = nullptr;
    try {
        auto* A = new vcsrmc_matrix_s();
        switch (config) {
            case 1: gen_uniform(*A, size > 0 ? size : 4096, seed); break;
            case 2: gen_powerlaw(*A, size > 0 ? size : 36692, seed); break;
            case 3: gen_stencil(*A, size > 0 ? size : 100); break;
            case 4: gen_block(*A, size > 0 ? size : 8192, seed); break;
            case 5: gen_rmat(*A, size > 0 ? size : 22, seed); break;
            default: delete A; return 1;
        }
        *out = A;
        return 0;
    } catch (...) {
        return 2;
    }
}

int vcsrmc_gen_info(vcsrmc_matrix_t m, int* M, int* N, long long* nnz) {
    if (!m) return 1;
    if (M) *M = m->M;
    if (N) *N = m->N;
    if (nnz) *nnz = (long long)m->col.size();
    return 0;
}

int vcsrmc_gen_copy(vcsrmc_matrix_t m, int* row_ptr, int* col, float* val) {
    if (!m) return 1;
    if (row_ptr) std::memcpy(row_ptr, m->row_ptr.data(), sizeof(int) * m->row_ptr.size());
    if (col && !m->col.empty()) std::memcpy(col, m->col.data(), sizeof(int) * m->col.size());
    if (val && !m->val.empty()) std::memcpy(val, m->val.data(), sizeof(float) * m->val.size());
    return 0;
}

int vcsrmc_gen_free(vcsrmc_matrix_t m) {
    delete m;
    return 0;
}

int vcsrmc_gen_dense(int dist, unsigned long long seed, int fp16_exact, float* out, long long n) {
    if (!out || n < 0 || (dist != 0 && dist != 1)) return 1;
    const long long blk = 1 << 20;
    const long long nb = (n + blk - 1) / blk;
#pragma omp parallel for schedule(dynamic, 1)
    for (long long b = 0; b < nb; ++b) {
        Engine e = block_engine(seed, 11, (uint64_t)b);
        const long long end = std::min(n, (b + 1) * blk);
        for (long long i = b * blk; i < end; ++i) {
            const float v = dist == 0 ? uniform_pm1(e) : normal01(e);
            out[i] = fp16_exact ? round_f16(v) : v;
        }
    }
    return 0;
}

}  // extern "C"
