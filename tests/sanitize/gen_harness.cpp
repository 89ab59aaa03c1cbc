// gen_harness.cpp -- runs the workload generators (vcsr_mc_amd/csrc/gen.cpp) at reduced sizes
// under AddressSanitizer and UndefinedBehaviorSanitizer (tests/test_host_sanitizers.py) and
// checks the CSR invariants of what they return.
#include <cstdio>
#include <vector>

#include "vcsrmc_bench.h"

static int check(int config, int size) {
    vcsrmc_matrix_t m = nullptr;
    if (vcsrmc_gen(config, size, 20260923ULL + config, &m) != 0) return 1;
    int M = 0, N = 0;
    long long nnz = 0;
    vcsrmc_gen_info(m, &M, &N, &nnz);
    std::vector<int> rp((size_t)M + 1), col((size_t)nnz);
    std::vector<float> val((size_t)nnz);
    vcsrmc_gen_copy(m, rp.data(), col.data(), val.data());
    vcsrmc_gen_free(m);
    if (rp[0] != 0 || rp[M] != nnz) return 2;
    for (int r = 0; r < M; ++r)
        for (int p = rp[r]; p < rp[r + 1]; ++p)
            if (col[p] < 0 || col[p] >= N || (p > rp[r] && col[p] <= col[p - 1])) return 3;
    std::printf("config %d size %d: %d x %d, %lld nonzeros\n", config, size, M, N, nnz);
    return 0;
}

int main() {
    const int sizes[][2] = {{1, 700}, {1, 3}, {2, 3000}, {2, 40}, {3, 9}, {3, 1},
                            {4, 40}, {4, 1}, {5, 11}, {5, 2}};
    for (const auto& s : sizes)
        if (int e = check(s[0], s[1])) {
            std::printf("FAILED config %d size %d: %d\n", s[0], s[1], e);
            return 1;
        }
    std::vector<float> d(1000);
    for (int dist = 0; dist < 2; ++dist)
        for (int exact = 0; exact < 2; ++exact)
            if (vcsrmc_gen_dense(dist, 7, exact, d.data(), (long long)d.size()) != 0) return 1;
    std::printf("ok\n");
    return 0;
}
