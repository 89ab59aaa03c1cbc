/*
 * vcsrmc_oracle.c -- CPU restatement of the VCSR-MC SpMM path (test infrastructure only;
 * the product never links it).  See vcsrmc_oracle.h for what each function follows and
 * how it is pinned.
 */
#include "vcsrmc_oracle.h"

#include <limits.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------------------------
 * FP16 range scale: src/vcsr_mc.cu:14-22.
 *  - The running maximum follows std::max(a, |v|) of the source, which keeps `a` when |v|
 *    is NaN.  (The reference binary is built with -ffast-math, CMakeLists.txt:24-27, whose
 *    vectorised max reduction treats NaN by lane position; NaN inputs are outside the
 *    bit-exact contract.)
 *  - `amax / 60000.0f` is evaluated as the reference binary evaluates it: -ffast-math turns
 *    the division by a constant into a multiplication by the float reciprocal
 *    fl(1/60000) = 1.66666669e-05f.  On finite inputs this matches the compiled reference
 *    bit for bit (pinned against oracle/_ref); IEEE division differs in the last bit for
 *    about one value in seven.
 * ------------------------------------------------------------------------------------- */
float orc_half_scale(const float *val, long long nnz) {
    const float headroom = 60000.0f;
    const float min_normal = 6.103515625e-05f;
    const volatile float one = 1.0f; /* keep the reciprocal a run-time float division */
    const float inv_headroom = one / headroom;
    float amax = 0.0f;
    for (long long i = 0; i < nnz; ++i) {
        const float a = fabsf(val[i]);
        if (amax < a) amax = a;
    }
    if (amax > headroom) return amax * inv_headroom;
    if (amax > 0.0f && amax < min_normal) return amax * inv_headroom;
    return 1.0f;
}

/* ---------------------------------------------------------------------------------------
 * IEEE binary32 -> binary16, round to nearest, ties to even (what a (_Float16) cast does).
 * ------------------------------------------------------------------------------------- */
uint16_t orc_f32_to_f16(float x) {
    uint32_t f;
    memcpy(&f, &x, sizeof f);
    const uint32_t sign = (f >> 16) & 0x8000u;
    const uint32_t bexp = (f >> 23) & 0xffu;
    const uint32_t mant = f & 0x7fffffu;
    if (bexp == 0xffu) /* Inf / NaN (NaN kept quiet) */
        return (uint16_t)(sign | 0x7c00u | (mant ? (0x200u | (mant >> 13)) : 0u));
    const int e = (int)bexp - 112; /* binary16 biased exponent */
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e >= 1) {
        uint32_t h = ((uint32_t)e << 10) | (mant >> 13);
        const uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h; /* may carry into Inf */
        return (uint16_t)(sign | h);
    }
    /* result is subnormal or zero: value = full * 2^(bexp-150), half ulp = 2^-24 */
    const int shift = 14 - e; /* = 126 - bexp */
    if (shift > 24 || bexp == 0) return (uint16_t)sign;
    const uint32_t full = mant | 0x800000u;
    uint32_t m = full >> shift;
    const uint32_t rem = full & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (m & 1u))) ++m; /* 0x400 becomes the min normal */
    return (uint16_t)(sign | m);
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t m = (uint32_t)h & 0x3ffu;
    uint32_t f;
    if (e == 0x1fu) {
        f = sign | 0x7f800000u | (m << 13);
    } else if (e != 0) {
        f = sign | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0) {
        f = sign;
    } else { /* subnormal: normalise */
        int ex = 113;
        while (!(m & 0x400u)) { m <<= 1; --ex; }
        f = sign | ((uint32_t)ex << 23) | ((m & 0x3ffu) << 13);
    }
    float x;
    memcpy(&x, &f, sizeof x);
    return x;
}

void orc_f32_to_f16_array(const float *x, uint16_t *out, long long n) {
    for (long long i = 0; i < n; ++i) out[i] = orc_f32_to_f16(x[i]);
}

void orc_round_f16_array(const float *x, float *out, long long n) {
    for (long long i = 0; i < n; ++i) out[i] = orc_f16_to_f32(orc_f32_to_f16(x[i]));
}

/* ---------------------------------------------------------------------------------------
 * Format construction: src/vcsr_mc.cu:25-123, canonical tie order.
 * ------------------------------------------------------------------------------------- */
typedef struct pair_s {
    int row;
    int count;
    long long first; /* index of the pair's first entry in the column-sorted entry buffer */
} pair_t;

typedef struct colidx_s { int col; int p; } colidx_t;
static int cmp_colidx(const void *a, const void *b) {
    const int x = ((const colidx_t *)a)->col, y = ((const colidx_t *)b)->col;
    return (x > y) - (x < y);
}

void orc_free(orc_format *f) {
    if (!f) return;
    free(f->group_ptr); free(f->group_depth); free(f->group_seg_base); free(f->group_rows);
    free(f->lcol); free(f->val); free(f->item_gbeg); free(f->item_gend);
    memset(f, 0, sizeof *f);
}

typedef struct item_s { int b, e; long long work; } item_t;

/* Stable order by work, descending (std::stable_sort at vcsr_mc.cu:120): merge sort. */
static void item_merge_sort(item_t *a, item_t *tmp, int n) {
    if (n < 2) return;
    const int h = n / 2;
    item_merge_sort(a, tmp, h);
    item_merge_sort(a + h, tmp, n - h);
    int i = 0, j = h, k = 0;
    while (i < h && j < n) tmp[k++] = (a[j].work > a[i].work) ? a[j++] : a[i++];
    while (i < h) tmp[k++] = a[i++];
    while (j < n) tmp[k++] = a[j++];
    memcpy(a, tmp, sizeof(item_t) * (size_t)n);
}

int orc_build(const int *row_ptr, const int *col, const float *val, int M, int N, int segw,
              int fp32, orc_format *out) {
    memset(out, 0, sizeof *out);
    if (segw != 16 && segw != 32 && segw != 48 && segw != 64) return ORC_BAD_SEGW;
    if (M < 0 || N < 0 || row_ptr[0] != 0) return ORC_BAD_CSR;
    for (int r = 0; r < M; ++r)
        if (row_ptr[r + 1] < row_ptr[r]) return ORC_BAD_CSR;
    const long long nnz = M ? row_ptr[M] : 0;
    for (long long p = 0; p < nnz; ++p)
        if (col[p] < 0 || col[p] >= N) return ORC_BAD_CSR;

    const int bundle = 16;
    out->M = M; out->N = N; out->segw = segw; out->bundle = bundle; out->fp32 = fp32 ? 1 : 0;
    out->scale = fp32 ? 1.0f : orc_half_scale(val, nnz);
    const float inv_scale = 1.0f / out->scale;
    const int S = (int)(((long long)N + segw - 1) / segw);
    out->num_segments = S;

    /* Entries of each row in ascending column order (vcsr_mc.cu:51-56 sorts each
     * (segment, row) bucket by local column; duplicates would leave that order open). */
    int *scol = (int *)malloc(sizeof(int) * (size_t)(nnz ? nnz : 1));
    float *sval = (float *)malloc(sizeof(float) * (size_t)(nnz ? nnz : 1));
    if (!scol || !sval) { free(scol); free(sval); return ORC_NOMEM; }
    for (int r = 0; r < M; ++r) {
        const int b = row_ptr[r], e = row_ptr[r + 1];
        int sorted = 1;
        for (int p = b + 1; p < e; ++p)
            if (col[p] <= col[p - 1]) { sorted = 0; break; }
        if (sorted) {
            for (int p = b; p < e; ++p) { scol[p] = col[p]; sval[p] = val[p]; }
            continue;
        }
        colidx_t *tmp = (colidx_t *)malloc(sizeof(colidx_t) * (size_t)(e - b));
        if (!tmp) { free(scol); free(sval); return ORC_NOMEM; }
        for (int p = b; p < e; ++p) { tmp[p - b].col = col[p]; tmp[p - b].p = p; }
        qsort(tmp, (size_t)(e - b), sizeof(colidx_t), cmp_colidx);
        for (int i = 0; i < e - b; ++i) {
            if (i > 0 && tmp[i].col == tmp[i - 1].col) {
                free(tmp); free(scol); free(sval); return ORC_DUPLICATE;
            }
            scol[b + i] = tmp[i].col; sval[b + i] = val[tmp[i].p];
        }
        free(tmp);
    }

    /* (segment, row) pairs, bucketed by segment; rows stay ascending inside a bucket. */
    long long *seg_n = (long long *)calloc((size_t)S + 1, sizeof(long long));
    if (!seg_n) { free(scol); free(sval); return ORC_NOMEM; }
    long long P = 0;
    for (int r = 0; r < M; ++r)
        for (int p = row_ptr[r]; p < row_ptr[r + 1]; ++p)
            if (p == row_ptr[r] || scol[p] / segw != scol[p - 1] / segw) { ++seg_n[scol[p] / segw + 1]; ++P; }
    for (int s = 0; s < S; ++s) seg_n[s + 1] += seg_n[s];
    pair_t *pairs = (pair_t *)malloc(sizeof(pair_t) * (size_t)(P ? P : 1));
    long long *fill = (long long *)malloc(sizeof(long long) * (size_t)(S ? S : 1));
    if (!pairs || !fill) { free(scol); free(sval); free(seg_n); free(pairs); free(fill); return ORC_NOMEM; }
    for (int s = 0; s < S; ++s) fill[s] = seg_n[s];
    for (int r = 0; r < M; ++r) {
        int p = row_ptr[r];
        while (p < row_ptr[r + 1]) {
            const int sid = scol[p] / segw;
            int q = p;
            while (q < row_ptr[r + 1] && scol[q] / segw == sid) ++q;
            pair_t *pr = &pairs[fill[sid]++];
            pr->row = r; pr->count = q - p; pr->first = p;
            p = q;
        }
    }

    /* Inside each segment: count descending, row ascending (stable counting sort). */
    pair_t *tmp = (pair_t *)malloc(sizeof(pair_t) * (size_t)(P ? P : 1));
    if (!tmp) { free(scol); free(sval); free(seg_n); free(pairs); free(fill); return ORC_NOMEM; }
    long long hist[65];
    for (int s = 0; s < S; ++s) {
        const long long b = seg_n[s], e = seg_n[s + 1];
        if (e - b < 2) continue;
        memset(hist, 0, sizeof hist);
        for (long long i = b; i < e; ++i) ++hist[segw - pairs[i].count + 1];
        for (int c = 0; c < 64; ++c) hist[c + 1] += hist[c];
        for (long long i = b; i < e; ++i) tmp[b + hist[segw - pairs[i].count]++] = pairs[i];
        memcpy(pairs + b, tmp + b, sizeof(pair_t) * (size_t)(e - b));
    }
    free(tmp);
    free(fill);

    /* Group sizes. */
    long long G = 0, nval = 0;
    for (int s = 0; s < S; ++s) {
        const long long n = seg_n[s + 1] - seg_n[s];
        for (long long i = 0; i < n; i += bundle) {
            ++G;
            nval += (long long)bundle * pairs[seg_n[s] + i].count;
        }
    }
    if (G >= INT_MAX || nval >= INT_MAX) {
        free(scol); free(sval); free(seg_n); free(pairs); return ORC_OVERFLOW;
    }
    out->G = (int)G;
    out->nval = nval;
    out->group_ptr = (int *)malloc(sizeof(int) * (size_t)(G + 1));
    out->group_depth = (int *)malloc(sizeof(int) * (size_t)(G ? G : 1));
    out->group_seg_base = (int *)malloc(sizeof(int) * (size_t)(G ? G : 1));
    out->group_rows = (int *)malloc(sizeof(int) * (size_t)(G ? 16 * G : 1));
    out->lcol = (int *)malloc(sizeof(int) * (size_t)(nval ? nval : 1));
    out->val = (float *)malloc(sizeof(float) * (size_t)(nval ? nval : 1));
    if (!out->group_ptr || !out->group_depth || !out->group_seg_base || !out->group_rows ||
        !out->lcol || !out->val) {
        free(scol); free(sval); free(seg_n); free(pairs); orc_free(out); return ORC_NOMEM;
    }
    long long g = 0, pos = 0;
    for (int s = 0; s < S; ++s) {
        const long long b = seg_n[s], n = seg_n[s + 1] - seg_n[s];
        for (long long i = 0; i < n; i += bundle) {
            const int depth = pairs[b + i].count;
            out->group_ptr[g] = (int)pos;
            out->group_depth[g] = depth;
            out->group_seg_base[g] = s * segw;
            for (int lane = 0; lane < bundle; ++lane)
                out->group_rows[16 * g + lane] = (i + lane < n) ? pairs[b + i + lane].row : -1;
            for (int d = 0; d < depth; ++d) {
                for (int lane = 0; lane < bundle; ++lane) {
                    int lc = -1;
                    float v = 0.0f;
                    if (i + lane < n) {
                        const pair_t *pr = &pairs[b + i + lane];
                        if (d < pr->count) {
                            lc = scol[pr->first + d] % segw;
                            v = sval[pr->first + d] * inv_scale;
                        }
                    }
                    out->lcol[pos] = lc;
                    out->val[pos] = v;
                    ++pos;
                }
            }
            ++g;
        }
    }
    out->group_ptr[G] = (int)pos;
    free(scol); free(sval); free(seg_n); free(pairs);

    /* Work items: vcsr_mc.cu:109-121. */
    const int chunk = (int)(G / 4096 < 1 ? 1 : (G / 4096 > 32 ? 32 : G / 4096));
    item_t *items = (item_t *)malloc(sizeof(item_t) * (size_t)(G ? G : 1));
    item_t *itmp = (item_t *)malloc(sizeof(item_t) * (size_t)(G ? G : 1));
    if (!items || !itmp) { free(items); free(itmp); orc_free(out); return ORC_NOMEM; }
    int ni = 0;
    for (int gb = 0; gb < (int)G;) {
        int e = gb;
        while (e < (int)G && e - gb < chunk && out->group_seg_base[e] == out->group_seg_base[gb]) ++e;
        items[ni].b = gb; items[ni].e = e;
        items[ni].work = (long long)out->group_ptr[e] - out->group_ptr[gb];
        ++ni;
        gb = e;
    }
    item_merge_sort(items, itmp, ni);
    out->nitems = ni;
    out->item_gbeg = (int *)malloc(sizeof(int) * (size_t)(ni ? ni : 1));
    out->item_gend = (int *)malloc(sizeof(int) * (size_t)(ni ? ni : 1));
    if (!out->item_gbeg || !out->item_gend) { free(items); free(itmp); orc_free(out); return ORC_NOMEM; }
    for (int i = 0; i < ni; ++i) { out->item_gbeg[i] = items[i].b; out->item_gend[i] = items[i].e; }
    free(items); free(itmp);
    return ORC_OK;
}

/* ---------------------------------------------------------------------------------------
 * Canonical tie order for a format built by the reference rule: inside each segment the
 * (count, row) sequence is non-increasing in count; rows of equal count are re-sorted by
 * ascending row id, carrying their entry columns.  Groups, depths, pointers and items are
 * unchanged by construction (depth is the count at a fixed rank).
 * ------------------------------------------------------------------------------------- */
typedef struct slot_s { int row; int count; int g; int lane; } slot_t;
static int cmp_slot(const void *a, const void *b) {
    const slot_t *x = (const slot_t *)a, *y = (const slot_t *)b;
    if (x->count != y->count) return (x->count < y->count) - (x->count > y->count);
    return (x->row > y->row) - (x->row < y->row);
}

int orc_canonicalize(orc_format *f) {
    const int G = f->G;
    int g0 = 0;
    while (g0 < G) {
        int g1 = g0 + 1;
        while (g1 < G && f->group_seg_base[g1] == f->group_seg_base[g0]) ++g1;
        const int nslot = 16 * (g1 - g0);
        slot_t *slots = (slot_t *)malloc(sizeof(slot_t) * (size_t)nslot);
        int ns = 0;
        long long ent = 0;
        for (int g = g0; g < g1; ++g) {
            for (int lane = 0; lane < 16; ++lane) {
                const int row = f->group_rows[16 * g + lane];
                if (row < 0) continue;
                int cnt = 0;
                while (cnt < f->group_depth[g] && f->lcol[f->group_ptr[g] + cnt * 16 + lane] >= 0) ++cnt;
                slots[ns].row = row; slots[ns].count = cnt; slots[ns].g = g; slots[ns].lane = lane;
                ent += cnt;
                ++ns;
            }
        }
        int *elc = (int *)malloc(sizeof(int) * (size_t)(ent ? ent : 1));
        float *ev = (float *)malloc(sizeof(float) * (size_t)(ent ? ent : 1));
        long long *eoff = (long long *)malloc(sizeof(long long) * (size_t)(ns ? ns : 1));
        if (!slots || !elc || !ev || !eoff) { free(slots); free(elc); free(ev); free(eoff); return ORC_NOMEM; }
        long long o = 0;
        for (int i = 0; i < ns; ++i) {
            eoff[i] = o;
            for (int d = 0; d < slots[i].count; ++d) {
                const long long idx = f->group_ptr[slots[i].g] + (long long)d * 16 + slots[i].lane;
                elc[o] = f->lcol[idx]; ev[o] = f->val[idx]; ++o;
            }
            slots[i].g = (int)i; /* remember original ordinal for the entry lookup */
        }
        qsort(slots, (size_t)ns, sizeof(slot_t), cmp_slot);
        for (int i = 0; i < nslot; ++i) {
            const int g = g0 + i / 16, lane = i % 16;
            const int depth = f->group_depth[g];
            if (i >= ns) {
                f->group_rows[16 * g + lane] = -1;
                for (int d = 0; d < depth; ++d) {
                    f->lcol[f->group_ptr[g] + d * 16 + lane] = -1;
                    f->val[f->group_ptr[g] + d * 16 + lane] = 0.0f;
                }
                continue;
            }
            const slot_t *s = &slots[i];
            f->group_rows[16 * g + lane] = s->row;
            for (int d = 0; d < depth; ++d) {
                const long long idx = f->group_ptr[g] + (long long)d * 16 + lane;
                if (d < s->count) { f->lcol[idx] = elc[eoff[s->g] + d]; f->val[idx] = ev[eoff[s->g] + d]; }
                else { f->lcol[idx] = -1; f->val[idx] = 0.0f; }
            }
        }
        free(slots); free(elc); free(ev); free(eoff);
        g0 = g1;
    }
    return ORC_OK;
}

/* ---------------------------------------------------------------------------------------
 * SpMM restatements.
 * ------------------------------------------------------------------------------------- */
static inline double q16(float x) { return (double)orc_f16_to_f32(orc_f32_to_f16(x)); }

/* One row of orc_spmm_csr: out[0..O) and the row's L1 norm of |a||b|.  Bq (mode 1) is B
 * already rounded to binary16 elementwise, or NULL to round each b as it is read; both give
 * the same doubles, q16 being a function of its argument. */
static void spmm_row(const int *row_ptr, const int *col, const float *val, int r, const float *B,
                     const float *Bq, int O, int mode, float inv, float scale, double *out,
                     double *rowL1) {
    for (int k = 0; k < O; ++k) out[k] = 0.0;
    double l1 = 0.0;
    for (int p = row_ptr[r]; p < row_ptr[r + 1]; ++p) {
        if (mode == 0) {
            const float *b = B + (size_t)col[p] * O;
            const double a = (double)val[p];
            for (int k = 0; k < O; ++k) {
                const double t = a * (double)b[k];
                out[k] += t;
                l1 += fabs(t);
            }
        } else if (Bq) {
            const float *b = Bq + (size_t)col[p] * O;
            const double a = q16(val[p] * inv);
            for (int k = 0; k < O; ++k) {
                const double t = a * (double)b[k];
                out[k] += t;
                l1 += fabs(t);
            }
        } else {
            const float *b = B + (size_t)col[p] * O;
            const double a = q16(val[p] * inv);
            for (int k = 0; k < O; ++k) {
                const double t = a * q16(b[k]);
                out[k] += t;
                l1 += fabs(t);
            }
        }
    }
    if (mode != 0) {
        for (int k = 0; k < O; ++k) out[k] *= (double)scale;
        l1 *= (double)scale;
    }
    *rowL1 = l1;
}

void orc_spmm_csr(const int *row_ptr, const int *col, const float *val, int M, const float *B,
                  int O, int mode, float scale, double *R, double *rowL1) {
    const float inv = 1.0f / scale;
    for (int r = 0; r < M; ++r) {
        double l1;
        spmm_row(row_ptr, col, val, r, B, NULL, O, mode, inv, scale, R + (size_t)r * O, &l1);
        if (rowL1) rowL1[r] = l1;
    }
}

int orc_spmm_check(const int *row_ptr, const int *col, const float *val, int M, const float *B,
                   long long nb, int O, int mode, float scale, const float *C, const float *C0,
                   int threads, double *err, double *bound, double *ref_l1, double *sq_err,
                   double *sq_ref) {
    const float inv = 1.0f / scale;
    float *Bq = NULL;
    if (mode != 0) {
        Bq = (float *)malloc(sizeof(float) * (size_t)(nb > 0 ? nb : 1));
        if (!Bq) return ORC_NOMEM;
#pragma omp parallel for schedule(static) num_threads(threads)
        for (long long i = 0; i < nb; ++i) Bq[i] = (float)q16(B[i]);
    }
    int status = ORC_OK;
#pragma omp parallel num_threads(threads)
    {
        double *out = (double *)malloc(sizeof(double) * (size_t)(O > 0 ? O : 1));
        if (!out) {
#pragma omp atomic write
            status = ORC_NOMEM;
        }
#pragma omp for schedule(dynamic, 256)
        for (int r = 0; r < M; ++r) {
            if (!out) continue;
            double l1;
            spmm_row(row_ptr, col, val, r, B, Bq, O, mode, inv, scale, out, &l1);
            const float *c = C + (size_t)r * O;
            const float *c0 = C0 ? C0 + (size_t)r * O : NULL;
            double e = 0.0, n0 = 0.0, rl1 = 0.0, se = 0.0, sr = 0.0;
            for (int k = 0; k < O; ++k) {
                double want = out[k];
                if (c0) {
                    want += (double)c0[k];
                    n0 += fabs((double)c0[k]);
                }
                const double d = (double)c[k] - want;
                e += fabs(d);
                rl1 += fabs(want);
                se += d * d;
                sr += want * want;
            }
            err[r] = e;
            bound[r] = l1 + n0;
            if (ref_l1) ref_l1[r] = rl1;
            if (sq_err) sq_err[r] = se;
            if (sq_ref) sq_ref[r] = sr;
        }
        free(out);
    }
    free(Bq);
    return status;
}

void orc_spmm_format(const orc_format *f, const float *B, int O, double *R) {
    memset(R, 0, sizeof(double) * (size_t)f->M * (size_t)O);
    for (int g = 0; g < f->G; ++g) {
        for (int lane = 0; lane < 16; ++lane) {
            const int row = f->group_rows[16 * g + lane];
            if (row < 0) continue;
            for (int d = 0; d < f->group_depth[g]; ++d) {
                const long long idx = f->group_ptr[g] + (long long)d * 16 + lane;
                const int lc = f->lcol[idx];
                if (lc < 0 || lc >= f->segw) continue;
                const int c = f->group_seg_base[g] + lc;
                const float *b = B + (size_t)c * O;
                double *out = R + (size_t)row * O;
                if (f->fp32) {
                    const double a = (double)f->val[idx];
                    for (int k = 0; k < O; ++k) out[k] += a * (double)b[k];
                } else {
                    const double a = q16(f->val[idx]);
                    for (int k = 0; k < O; ++k) out[k] += a * q16(b[k]);
                }
            }
        }
    }
    if (!f->fp32)
        for (size_t i = 0; i < (size_t)f->M * (size_t)O; ++i) R[i] *= (double)f->scale;
}

void orc_cpu_spmm_f64_rows(const int *row_ptr, const int *col, const float *val, int r0, int r1,
                           const float *B, int O, double *R) {
    for (int r = r0; r < r1; ++r)
        for (int p = row_ptr[r]; p < row_ptr[r + 1]; ++p)
            for (int k = 0; k < O; ++k)
                R[(size_t)r * O + k] += (double)val[p] * B[(size_t)col[p] * O + k];
}

void orc_cpu_spmm_f64(const int *row_ptr, const int *col, const float *val, int M,
                      const float *B, int O, double *R) {
    orc_cpu_spmm_f64_rows(row_ptr, col, val, 0, M, B, O, R);
}

void orc_cpu_spmm_f64_omp(const int *row_ptr, const int *col, const float *val, int r0, int r1,
                          const float *B, int O, double *R, int threads) {
#pragma omp parallel for schedule(dynamic, 64) num_threads(threads)
    for (int r = r0; r < r1; ++r)
        for (int p = row_ptr[r]; p < row_ptr[r + 1]; ++p)
            for (int k = 0; k < O; ++k)
                R[(size_t)r * O + k] += (double)val[p] * B[(size_t)col[p] * O + k];
}
