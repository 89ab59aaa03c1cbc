/* oracle_harness.c -- drives the oracle's C functions (oracle/vcsrmc_oracle.c, rcm_oracle.c) on
 * seeded random matrices under AddressSanitizer and UndefinedBehaviorSanitizer
 * (tests/test_host_sanitizers.py): format build and canonical order, both SpMM restatements,
 * the libstdc++ sort steps, RCM and the column relabelling. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "vcsrmc_oracle.h"

static unsigned long long s = 88172645463325252ull;
static unsigned rnd(void) {
    s ^= s << 13;
    s ^= s >> 7;
    s ^= s << 17;
    return (unsigned)(s >> 32);
}

/* Random CSR: rows sorted and distinct; some rows empty, a few heavy. */
static void make(int M, int N, int per_row, int **rp, int **col, float **val) {
    int *r = malloc(sizeof(int) * (M + 1));
    int cap = M * (per_row + 1) + 4 * N + 16;
    int *c = malloc(sizeof(int) * cap);
    char *seen = calloc(N, 1);
    r[0] = 0;
    int nnz = 0;
    for (int i = 0; i < M; ++i) {
        int k = (rnd() % 7 == 0) ? 0 : (int)(rnd() % (per_row + 1));
        if (i % 97 == 5) k = N / 2; /* a heavy row */
        if (k > N) k = N;
        int got = 0;
        while (got < k) {
            int j = (int)(rnd() % N);
            if (!seen[j]) { seen[j] = 1; ++got; }
        }
        for (int j = 0; j < N; ++j)
            if (seen[j]) { c[nnz++] = j; seen[j] = 0; }
        r[i + 1] = nnz;
    }
    float *v = malloc(sizeof(float) * (nnz ? nnz : 1));
    for (int p = 0; p < nnz; ++p) v[p] = (float)((int)(rnd() % 2001) - 1000) / 500.0f;
    free(seen);
    *rp = r; *col = c; *val = v;
}

int main(void) {
    const int shapes[][3] = {{1, 1, 1}, {17, 5, 3}, {300, 200, 9}, {129, 1000, 40}, {64, 33, 0}};
    for (int t = 0; t < (int)(sizeof shapes / sizeof shapes[0]); ++t) {
        const int M = shapes[t][0], N = shapes[t][1], O = 5;
        int *rp, *col;
        float *val;
        make(M, N, shapes[t][2], &rp, &col, &val);
        const int nnz = rp[M];
        float *B = malloc(sizeof(float) * N * O);
        for (int i = 0; i < N * O; ++i) B[i] = (float)((int)(rnd() % 201) - 100) / 64.0f;
        double *R1 = calloc((size_t)M * O, sizeof(double)), *R2 = calloc((size_t)M * O, sizeof(double));
        double *L1 = calloc(M, sizeof(double));
        for (int segw = 16; segw <= 64; segw += 16)
            for (int fp32 = 0; fp32 < 2; ++fp32) {
                orc_format f;
                if (orc_build(rp, col, val, M, N, segw, fp32, &f) != ORC_OK) return 1;
                if (orc_canonicalize(&f) != ORC_OK) return 2;
                orc_spmm_format(&f, B, O, R2);
                orc_free(&f);
            }
        orc_spmm_csr(rp, col, val, M, B, O, 1, orc_half_scale(val, nnz), R1, L1);
        memset(R1, 0, sizeof(double) * M * O);
        orc_cpu_spmm_f64(rp, col, val, M, B, O, R1);
        orc_cpu_spmm_f64_omp(rp, col, val, 0, M, B, O, R2, 3);
        int *pos = malloc(sizeof(int) * N);
        if (orc_rcm_order(rp, col, M, N, pos) != 0) return 3;
        float *Bo = malloc(sizeof(float) * N * O);
        if (orc_apply_column_permutation(rp, col, val, M, N, pos, B, O, Bo) != 0) return 4;
        int *a = malloc(sizeof(int) * N), *key = malloc(sizeof(int) * N);
        for (int i = 0; i < N; ++i) { a[i] = i; key[i] = (int)(rnd() % 5); }
        orc_std_sort_by_key(a, N, key);
        orc_heap_sort_by_key(a, N, key);
        printf("shape %d x %d: %d nonzeros\n", M, N, nnz);
        free(rp); free(col); free(val); free(B); free(R1); free(R2); free(L1); free(pos);
        free(Bo); free(a); free(key);
    }
    printf("ok\n");
    return 0;
}
