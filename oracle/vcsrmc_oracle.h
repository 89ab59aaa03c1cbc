/*
 * vcsrmc_oracle.h -- CPU restatement of the VCSR-MC SpMM path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library checks the product: only the test suite,
 * the smoke check and the CPU-baseline leg of the benchmark may load it.  The
 * product (libvcsrmc.so) never links, loads or calls it.
 *
 * Every function restates one piece of MuuSeoTia/VCSR_MC (paths are relative to
 * the reference repository):
 *   orc_half_scale        src/vcsr_mc.cu:14-22
 *   orc_f32_to_f16 / orc_f16_to_f32
 *                         the (_Float16) conversions of src/vcsr_mc.cu:195-196, 213
 *                         (IEEE-754 binary16, round to nearest even)
 *   orc_build             src/vcsr_mc.cu:25-123 with one change: rows of equal
 *                         count inside a segment are ordered by ascending row id
 *                         (the reference leaves that order to std::unordered_map
 *                         iteration plus an unstable std::sort, :59-66)
 *   orc_canonicalize      puts any format built by the reference rule into that
 *                         canonical tie order
 *   orc_spmm_csr          src/main.cpp:202-207 (r -> p -> k, double accumulation),
 *                         with the FP16 input model of src/vcsr_mc.cu:195-196, 213, 234
 *   orc_spmm_check        orc_spmm_csr row by row against a given C (the parity norm's
 *                         terms for every row, OpenMP over rows)
 *   orc_spmm_format       C = A.B read back from the format arrays
 *                         (the semantics of the kernels src/vcsr_mc.cu:144-329)
 *
 * How each function is pinned (tests/test_oracle.py):
 *   - orc_half_scale: closed form at amax = 0, 1, 6e-5, 60000, 1e5, inf, NaN.
 *   - orc_f32_to_f16: every float16 value, every rounding midpoint, overflow and
 *     subnormal boundaries against numpy.float16 (an independent RNE conversion).
 *   - orc_build: equal, after orc_canonicalize, to the reference's own
 *     csr_to_vcsr_mc compiled from its sources (oracle/_ref) and to the committed
 *     fixtures made by it; closed forms (diagonal, dense 32x32 blocks, < 16 rows,
 *     empty segments, N % segw != 0, nnz = 0); invariants (coverage, padding,
 *     seg_base + lcol = col, depth = max count, items partition the groups).
 *   - orc_spmm_csr: a dense numpy matmul in float64 of the same quantised inputs.
 *   - orc_spmm_format: equals orc_spmm_csr on the same matrix.
 *   - orc_spmm_check: its err, bound, ref_l1, sq_err and sq_ref equal |C - R|, rowL1, |R|,
 *     (C - R)^2 and R^2 summed in index order from orc_spmm_csr's R, bit for bit, in both modes,
 *     with and without C0, at 1 and several threads; a planted error in one element of C shows
 *     up in that row only.
 */
#ifndef VCSRMC_ORACLE_H
#define VCSRMC_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct orc_format {
    int M, N, segw, bundle, num_segments;
    int G;          /* number of groups                         */
    long long nval; /* |lcol| = |val| = group_ptr[G]             */
    int nitems;
    int *group_ptr, *group_depth, *group_seg_base, *group_rows, *lcol;
    float *val;
    int *item_gbeg, *item_gend;
    float scale;
    int fp32;
} orc_format;

/* Status codes. */
enum { ORC_OK = 0, ORC_BAD_SEGW = 1, ORC_BAD_CSR = 2, ORC_DUPLICATE = 3, ORC_NOMEM = 4,
       ORC_OVERFLOW = 5 };

float orc_half_scale(const float *val, long long nnz);
uint16_t orc_f32_to_f16(float x);
float orc_f16_to_f32(uint16_t h);
void orc_f32_to_f16_array(const float *x, uint16_t *out, long long n);
/* x -> float(f16(x)) elementwise */
void orc_round_f16_array(const float *x, float *out, long long n);

int orc_build(const int *row_ptr, const int *col, const float *val, int M, int N, int segw,
              int fp32, orc_format *out);
void orc_free(orc_format *f);
int orc_canonicalize(orc_format *f);

/* mode 0: FP32 inputs.  mode 1: FP16 model, a' = f16(f32(v * (1/scale))), b' = f16(b),
 * result scaled by `scale`.  R (M x O) and rowL1 (M, may be NULL) are overwritten:
 * R[r,k] = sum_p a'_p b'_{c_p,k} (times scale), rowL1[r] = sum_k sum_p |a'_p b'_{c_p,k}| (times scale). */
void orc_spmm_csr(const int *row_ptr, const int *col, const float *val, int M, const float *B,
                  int O, int mode, float scale, double *R, double *rowL1);
void orc_spmm_format(const orc_format *f, const float *B, int O, double *R);
/* The parity check of a whole product, rows split over `threads` OpenMP threads, without an
 * M x O result buffer: for every row r, the row of orc_spmm_csr (same arithmetic, so the same
 * doubles), then err[r] = sum_k |C[r,k] - (R[r,k] + C0[r,k])| and bound[r] = rowL1[r] +
 * sum_k |C0[r,k]| (C0 = C's values before a C += A.B launch; NULL = zero).  Optional (NULL = not
 * wanted), with want = R + C0: ref_l1[r] = sum_k |want[r,k]| (the stricter norm ||C_ref[r,:]||_1),
 * sq_err[r] = sum_k (C[r,k] - want[r,k])^2 and sq_ref[r] = sum_k want[r,k]^2, whose totals give
 * the reference driver's relative L2 error (src/main.cpp:262-275).  nb = the number of B elements
 * (mode 1 rounds B to binary16 once, in a buffer of that size).  Returns ORC_OK or ORC_NOMEM. */
int orc_spmm_check(const int *row_ptr, const int *col, const float *val, int M, const float *B,
                   long long nb, int O, int mode, float scale, const float *C, const float *C0,
                   int threads, double *err, double *bound, double *ref_l1, double *sq_err,
                   double *sq_ref);

/* The reference's CPU SpMM exactly as the driver runs it (main.cpp:202-207): plain FP32
 * inputs, double accumulation, r -> p -> k.  R must be zeroed by the caller (+=). */
void orc_cpu_spmm_f64(const int *row_ptr, const int *col, const float *val, int M,
                      const float *B, int O, double *R);
/* Same loop over rows [r0, r1) only (a bounded sample for timing). */
void orc_cpu_spmm_f64_rows(const int *row_ptr, const int *col, const float *val, int r0, int r1,
                           const float *B, int O, double *R);
/* Same loop with the rows split over `threads` OpenMP threads (rows are independent, so the
 * output is bit-identical to the single-thread loop). */
void orc_cpu_spmm_f64_omp(const int *row_ptr, const int *col, const float *val, int r0, int r1,
                          const float *B, int O, double *R, int threads);

/* Column reordering (rcm_oracle.c; include/reorder.hpp:17-108). */
/* std::sort(a, a + n, key[x] < key[y]) with the steps of GCC 11's libstdc++. */
void orc_std_sort_by_key(int *a, long long n, const int *key);
/* The heapsort step alone: std::partial_sort(a, a + n, a + n, key[x] < key[y]). */
void orc_heap_sort_by_key(int *a, long long n, const int *key);
/* rcm_column_order: position[N] = new position of each old column. */
int orc_rcm_order(const int *row_ptr, const int *col, int M, int N, int *position);
/* apply_column_permutation: relabels col in place and re-sorts each row (with val); if B and
 * B_out are non-NULL, B_out[position[r], :] = B[r, :] (N x O). */
int orc_apply_column_permutation(const int *row_ptr, int *col, float *val, int M, int N,
                                 const int *position, const float *B, int O, float *B_out);

#ifdef __cplusplus
}
#endif
#endif
