/*
 * rcm_oracle.c -- CPU restatement of the reference's column reordering
 * (include/reorder.hpp:17-108 of MuuSeoTia/VCSR_MC).
 *
 * TEST INFRASTRUCTURE ONLY (part of libvcsrmc_oracle.so; the product never loads it).
 *
 *   orc_std_sort_by_key   std::sort(first, last, [&](int a, int b) { return key[a] < key[b]; })
 *                         as GCC 11's libstdc++ carries it out (introsort: median-of-three
 *                         Hoare partitions above 16 elements, heapsort at depth 2*floor(lg n),
 *                         then one insertion-sort pass).  The reference sorts BFS children by
 *                         degree with this call (reorder.hpp:67-68), and equal degrees are
 *                         common, so the exact steps fix the tie order of the ordering.
 *   orc_rcm_order         rcm_column_order (reorder.hpp:17-77)
 *   orc_apply_column_permutation
 *                         apply_column_permutation (reorder.hpp:82-108)
 *
 *   orc_heap_sort_by_key  the heapsort step alone (std::partial_sort(a, a + n, a + n))
 *
 * Pinned by tests/test_oracle_rcm.py: orc_std_sort_by_key against the C++ std::sort of the
 * compiler here (oracle/_ref) on random inputs with many ties, on sizes around the 16-element
 * threshold and on adversarial inputs that force the heapsort fallback (with ties);
 * orc_heap_sort_by_key against std::partial_sort with ties; orc_rcm_order against the reference's rcm_column_order compiled from
 * its header (oracle/_ref) and the committed fixtures made by it; closed forms (a path
 * graph, a star, isolated columns, M > N rows that only add self-loops); the permutation
 * property and C = (A P)(P^T B) = A B.
 */
#include <stdlib.h>
#include <string.h>

#include "vcsrmc_oracle.h"

/* ---- std::sort steps (the comparator is key[x] < key[y] on int elements) ---------------- */
#define LESS_AT(i, j) (key[a[i]] < key[a[j]])

static void ss_swap(int *a, long i, long j) {
    const int t = a[i];
    a[i] = a[j];
    a[j] = t;
}

/* Shift a[pos] left past every element whose key is greater (no lower bound check: an
 * element with a key not greater than it sits somewhere to the left). */
static void ss_linear_insert(int *a, long pos, const int *key) {
    const int v = a[pos];
    while (key[v] < key[a[pos - 1]]) {
        a[pos] = a[pos - 1];
        --pos;
    }
    a[pos] = v;
}

static void ss_insertion(int *a, long lo, long hi, const int *key) {
    for (long i = lo + 1; i < hi; ++i) {
        if (LESS_AT(i, lo)) {
            const int v = a[i];
            memmove(a + lo + 1, a + lo, sizeof(int) * (size_t)(i - lo));
            a[lo] = v;
        } else {
            ss_linear_insert(a, i, key);
        }
    }
}

/* Sift the hole at `hole` of the heap a[base .. base+len) down to a leaf, then push `v` up. */
static void ss_sift(int *a, long base, long hole, long len, int v, const int *key) {
    const long top = hole;
    long child = hole;
    while (child < (len - 1) / 2) {
        child = 2 * child + 2;
        if (LESS_AT(base + child, base + child - 1)) --child;
        a[base + hole] = a[base + child];
        hole = child;
    }
    if ((len & 1) == 0 && child == (len - 2) / 2) {
        child = 2 * child + 2;
        a[base + hole] = a[base + child - 1];
        hole = child - 1;
    }
    long parent = (hole - 1) / 2;
    while (hole > top && key[a[base + parent]] < key[v]) {
        a[base + hole] = a[base + parent];
        hole = parent;
        parent = (hole - 1) / 2;
    }
    a[base + hole] = v;
}

static void ss_heapsort(int *a, long lo, long hi, const int *key) {
    const long len = hi - lo;
    if (len >= 2) {
        for (long parent = (len - 2) / 2;; --parent) {
            ss_sift(a, lo, parent, len, a[lo + parent], key);
            if (parent == 0) break;
        }
    }
    for (long end = hi - 1; end - lo > 0; --end) {
        const int v = a[end];
        a[end] = a[lo];
        ss_sift(a, lo, 0, end - lo, v, key);
    }
}

static void ss_median_to_first(int *a, long dst, long x, long y, long z, const int *key) {
    if (LESS_AT(x, y)) {
        if (LESS_AT(y, z)) ss_swap(a, dst, y);
        else if (LESS_AT(x, z)) ss_swap(a, dst, z);
        else ss_swap(a, dst, x);
    } else if (LESS_AT(x, z)) {
        ss_swap(a, dst, x);
    } else if (LESS_AT(y, z)) {
        ss_swap(a, dst, z);
    } else {
        ss_swap(a, dst, y);
    }
}

/* Hoare partition of a[lo .. hi) around the pivot a[piv] (no bounds checks: the pivot is a
 * median of three, so both scans stop inside the range). */
static long ss_partition(int *a, long lo, long hi, long piv, const int *key) {
    for (;;) {
        while (LESS_AT(lo, piv)) ++lo;
        --hi;
        while (LESS_AT(piv, hi)) --hi;
        if (!(lo < hi)) return lo;
        ss_swap(a, lo, hi);
        ++lo;
    }
}

static void ss_introsort(int *a, long lo, long hi, int depth, const int *key) {
    while (hi - lo > 16) {
        if (depth == 0) {
            ss_heapsort(a, lo, hi, key);
            return;
        }
        --depth;
        ss_median_to_first(a, lo, lo + 1, lo + (hi - lo) / 2, hi - 1, key);
        const long cut = ss_partition(a, lo + 1, hi, lo, key);
        ss_introsort(a, cut, hi, depth, key);
        hi = cut;
    }
}

void orc_heap_sort_by_key(int *a, long long n, const int *key) {
    if (n > 0) ss_heapsort(a, 0, (long)n, key);
}

void orc_std_sort_by_key(int *a, long long n, const int *key) {
    if (n <= 0) return;
    int lg = 0;
    while ((1LL << (lg + 1)) <= n) ++lg;
    ss_introsort(a, 0, (long)n, 2 * lg, key);
    if (n > 16) {
        ss_insertion(a, 0, 16, key);
        for (long i = 16; i < n; ++i) ss_linear_insert(a, i, key);
    } else {
        ss_insertion(a, 0, (long)n, key);
    }
}

/* ---- rcm_column_order (reorder.hpp:17-77) ---------------------------------------------- */
static int cmp_int(const void *x, const void *y) {
    const int a = *(const int *)x, b = *(const int *)y;
    return (a > b) - (a < b);
}

int orc_rcm_order(const int *row_ptr, const int *col, int M, int N, int *position) {
    if (N <= 0) return ORC_OK;
    /* Symmetrised pattern: nonzero (r, c) gives the edge r - c when r < N; a row r >= N only
     * marks c as its own neighbour (reorder.hpp:21-37). */
    long long *head = calloc((size_t)N + 1, sizeof(long long));
    int *deg = calloc((size_t)N, sizeof(int));
    if (!head || !deg) { free(head); free(deg); return ORC_NOMEM; }
    for (int r = 0; r < M; ++r)
        for (long long p = row_ptr[r]; p < row_ptr[r + 1]; ++p) {
            if (r < N) ++head[r + 1];
            ++head[col[p] + 1];
        }
    for (int i = 0; i < N; ++i) head[i + 1] += head[i];
    int *adj = malloc(sizeof(int) * (size_t)(head[N] ? head[N] : 1));
    long long *fill = malloc(sizeof(long long) * (size_t)N);
    if (!adj || !fill) { free(head); free(deg); free(adj); free(fill); return ORC_NOMEM; }
    memcpy(fill, head, sizeof(long long) * (size_t)N);
    for (int r = 0; r < M; ++r)
        for (long long p = row_ptr[r]; p < row_ptr[r + 1]; ++p) {
            const int c = col[p];
            if (r < N) adj[fill[r]++] = c;
            adj[fill[c]++] = r < N ? r : c;
        }
    /* Sorted distinct neighbours; the degree counts them (a self-loop included). */
    for (int i = 0; i < N; ++i) {
        int *b = adj + head[i];
        const long long len = head[i + 1] - head[i];
        qsort(b, (size_t)len, sizeof(int), cmp_int);
        int u = 0;
        for (long long k = 0; k < len; ++k)
            if (k == 0 || b[k] != b[k - 1]) b[u++] = b[k];
        deg[i] = u;
    }
    free(fill);

    /* Roots in ascending degree, ties by column id (a stable sort of 0..N-1): counting sort. */
    int *roots = malloc(sizeof(int) * (size_t)N);
    int *dcount = calloc((size_t)N + 2, sizeof(int));
    char *seen = calloc((size_t)N, 1);
    int *queue = malloc(sizeof(int) * (size_t)N);
    if (!roots || !dcount || !seen || !queue) {
        free(head); free(deg); free(adj); free(roots); free(dcount); free(seen); free(queue);
        return ORC_NOMEM;
    }
    for (int i = 0; i < N; ++i) ++dcount[deg[i] + 1];
    for (int d = 0; d <= N; ++d) dcount[d + 1] += dcount[d];
    for (int i = 0; i < N; ++i) roots[dcount[deg[i]]++] = i;

    /* Breadth-first search from each unseen root.  Every vertex enters the queue once, so the
     * queue array doubles as the visiting order; children of a vertex are its unseen
     * neighbours in ascending id, then std::sort by degree (reorder.hpp:52-71). */
    long long qtail = 0;
    for (int ri = 0; ri < N; ++ri) {
        const int root = roots[ri];
        if (seen[root]) continue;
        seen[root] = 1;
        long long qhead = qtail;
        queue[qtail++] = root;
        while (qhead < qtail) {
            const int v = queue[qhead++];
            const long long first = qtail;
            for (long long k = head[v]; k < head[v] + deg[v]; ++k) {
                const int u = adj[k];
                if (!seen[u]) {
                    seen[u] = 1;
                    queue[qtail++] = u;
                }
            }
            orc_std_sort_by_key(queue + first, qtail - first, deg);
        }
    }
    /* Reverse Cuthill-McKee: position[order[i]] = N - 1 - i (reorder.hpp:72-75). */
    for (int i = 0; i < N; ++i) position[queue[i]] = N - 1 - i;
    free(head); free(deg); free(adj); free(roots); free(dcount); free(seen); free(queue);
    return ORC_OK;
}

/* ---- apply_column_permutation (reorder.hpp:82-108) ------------------------------------- */
typedef struct { int c; float v; } colval_t;
static int cmp_colval(const void *x, const void *y) {
    const int a = ((const colval_t *)x)->c, b = ((const colval_t *)y)->c;
    return (a > b) - (a < b);
}

int orc_apply_column_permutation(const int *row_ptr, int *col, float *val, int M, int N,
                                 const int *position, const float *B, int O, float *B_out) {
    (void)N;
    int maxlen = 1;
    for (int r = 0; r < M; ++r)
        if (row_ptr[r + 1] - row_ptr[r] > maxlen) maxlen = row_ptr[r + 1] - row_ptr[r];
    colval_t *tmp = malloc(sizeof(colval_t) * (size_t)maxlen);
    if (!tmp) return ORC_NOMEM;
    for (int r = 0; r < M; ++r) {
        const int s = row_ptr[r], len = row_ptr[r + 1] - s;
        for (int i = 0; i < len; ++i) {
            tmp[i].c = position[col[s + i]];
            tmp[i].v = val[s + i];
        }
        /* New column ids of one row are distinct, so any sort gives the same order. */
        qsort(tmp, (size_t)len, sizeof(colval_t), cmp_colval);
        for (int i = 0; i < len; ++i) {
            col[s + i] = tmp[i].c;
            val[s + i] = tmp[i].v;
        }
    }
    free(tmp);
    if (B && B_out)
        for (int r = 0; r < N; ++r)
            memcpy(B_out + (size_t)position[r] * O, B + (size_t)r * O, sizeof(float) * (size_t)O);
    return ORC_OK;
}
