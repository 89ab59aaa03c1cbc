/*
 * vcsrmc_bench.h -- C ABI of libvcsrmc_bench.so: seeded synthetic matrices of the benchmark
 * workloads and the hipSPARSE comparison baseline.  Not part of the SpMM product; used by the
 * driver, the benchmark and the tests.
 */
#ifndef VCSRMC_BENCH_H
#define VCSRMC_BENCH_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Workloads.  `size` scales each one (0 = the full benchmark size):
 *   1 uniform   n x n, n = size (4096); nnz per row ~ Poisson(16) clipped to [0, n], distinct
 *               uniform columns (Floyd); values U[-1,1] FP32
 *   2 powerlaw  n x n, n = size (36692); symmetric pattern from a configuration model with
 *               degrees Zipf(2.1) on [1, 1383], scaled so that about 368000 * n / 36692
 *               nonzeros remain after self loops and duplicates are dropped (367,570 at the
 *               full size); values U[-1,1] rounded to FP16
 *   3 stencil   27-point stencil on a g^3 grid, g = size (100), natural order; diagonal 26,
 *               off-diagonals -1
 *   4 block     nb block rows of height 32, nb = size (8192), each with 4 distinct uniform
 *               block columns in [0, nb) holding dense 32 x 32 blocks; values N(0,1) rounded
 *               to FP16
 *   5 rmat      R-MAT of scale s = size (22), 16 * 2^s draws, (a,b,c,d) = (.57,.19,.19,.05),
 *               directed, duplicates merged; values U[-1,1] rounded to FP16
 * Every random draw comes from std::mt19937_64 with transforms written out in gen.cpp, so a
 * (config, size, seed) triple gives the same matrix on every machine. */
typedef struct vcsrmc_matrix_s *vcsrmc_matrix_t;

int vcsrmc_gen(int config, int size, unsigned long long seed, vcsrmc_matrix_t *out);
int vcsrmc_gen_info(vcsrmc_matrix_t m, int *M, int *N, long long *nnz);
/* Copies the CSR into caller buffers (row_ptr: M+1, col/val: nnz). */
int vcsrmc_gen_copy(vcsrmc_matrix_t m, int *row_ptr, int *col, float *val);
int vcsrmc_gen_free(vcsrmc_matrix_t m);

/* n dense values: dist 0 = U[-1,1], 1 = N(0,1); fp16_exact rounds each value to the nearest
 * binary16 (ties to even) and back. */
int vcsrmc_gen_dense(int dist, unsigned long long seed, int fp16_exact, float *out, long long n);

/* hipSPARSE SpMM (CSR, ALG_DEFAULT unless alg = 1..3 picks CSR_ALG1..3), C = alpha A.B with
 * beta = 0, row-major dense B (N x O) and C (M x O).  val_f16 / b_f16 select binary16 A values
 * and B (FP32 compute and C, as the reference's rocsparse_fp16, src/kernels.cu:139-206).
 * Descriptors, workspace and preprocess are built once per argument set (the four most recent
 * sets are kept) and timed into *setup_ms; *ms is the event-timed hipsparseSpMM call on
 * `stream`.  Sets are keyed by device addresses: call vcsrmc_rocsparse_release before reusing
 * freed addresses for other operands of the same sizes.  Returns 0, 2 (HIP error) or
 * 10 + a hipSPARSE status. */
int vcsrmc_rocsparse_spmm(int M, int N, int nnz, const int *d_row_ptr, const int *d_col,
                          const void *d_val, int val_f16, const void *d_B, int b_f16, int O,
                          float *d_C, float alpha, int alg, void *stream, float *ms,
                          float *setup_ms);
int vcsrmc_rocsparse_release(void);

#ifdef __cplusplus
}
#endif
#endif
