// reorder.hip -- reverse Cuthill-McKee column order and the column relabelling that goes with
// it, on the GPU (include/reorder.hpp:17-108 of MuuSeoTia/VCSR_MC).
//
// The reference walks the symmetrised pattern breadth-first with one host queue.  Here the
// same order is produced level by level, every connected component at once:
//   1. adjacency: the 2 nnz (vertex, neighbour) pairs of the symmetrised pattern, radix-sorted
//      and deduplicated; the degree counts distinct neighbours, a self-loop included
//      (reorder.hpp:21-42).
//   2. rank: vertices in ascending (degree, id) -- the reference's stable_sort of the roots
//      (reorder.hpp:47-50).
//   3. components: rounds of hooking (the parent of larger rank under the parent of smaller
//      rank, across every edge between two trees) and pointer jumping, until a round changes
//      nothing; each component ends up represented by its lowest-rank vertex, the root from
//      which the reference's loop (reorder.hpp:54-57) starts that component.
//   4. levels: level 0 holds every component's root in rank order.  A vertex of level L+1
//      belongs to the earliest level-L vertex adjacent to it (the one that pops it from the
//      reference's queue, reorder.hpp:63-66).  A level is ordered by that parent's index, then
//      inside one parent's children as the reference orders them: ascending id, then
//      std::sort by degree (reorder.hpp:67-69), whose steps (libstdc++ introsort) are carried
//      out exactly, since equal degrees make the result depend on them.  Levels of up to 8192
//      frontier edges run inside one work-group, many at a time (k_bfs_levels; groups above 64
//      elements partitioned by the work-group, pieces finished by one thread each); larger
//      levels take several kernels: claims, a radix sort by (parent index, id), and the group
//      sorts (large groups a partition step at a time by work-groups, pieces of up to 256
//      elements by one wave each in LDS, with wave-wide partition steps).
//   5. order: vertices sorted by (component rank, level, index in level) give the
//      Cuthill-McKee order; position = N - 1 - that index (reorder.hpp:72-76).
#include <algorithm>
#include <atomic>
#include <climits>
#include <cstdint>
#include <string>

#include "../../include/vcsrmc.h"
#include "internal.hpp"

namespace vcsrmc {
namespace {

using u64 = unsigned long long;

inline unsigned nblk(long long n) { return grid_for(n, 256); }

#define RLAUNCH(kernel, n, ...)                                                               \
    do {                                                                                      \
        if ((n) > 0) {                                                                        \
            hipLaunchKernelGGL(kernel, dim3(nblk(n)), dim3(256), 0, st, __VA_ARGS__);         \
            VCSRMC_HIP(hipGetLastError());                                                    \
        }                                                                                     \
    } while (0)

enum : int { kBadRowPtr = 1, kBadCol = 2, kBadPerm = 4, kDupCol = 8 };

__global__ void k_check_rp(const int* __restrict__ rp, int M, int nnz, int* __restrict__ err) {
    const long long r = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (r > M) return;
    const int a = rp[r];
    bool bad = a < 0 || a > nnz;
    if (r == 0) bad |= a != 0;
    if (r == M) bad |= a != nnz;
    if (r < M) bad |= rp[r + 1] < a;
    if (bad) atomicOr(err, kBadRowPtr);
}

__global__ void k_check_cols(const int* __restrict__ col, long long nnz, int N,
                             int* __restrict__ err) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nnz) return;
    const int c = col[i];
    if (c < 0 || c >= N) atomicOr(err, kBadCol);
}

void raise_if(const int* d_err, hipStream_t st) {
    const int e = read_scalar(d_err, st);
    if (e & kBadRowPtr) throw Error(VCSRMC_ERR_CSR, "row_ptr is not a monotone 0..nnz sequence");
    if (e & kBadCol) throw Error(VCSRMC_ERR_CSR, "column index out of range [0, N)");
    if (e & kBadPerm) throw Error(VCSRMC_ERR_ARG, "position is not a permutation of 0..N-1");
    if (e & kDupCol)
        throw Error(VCSRMC_ERR_UNSORTED, "a row holds the same column twice");
}

void check_csr(const int* rp, const int* col, int M, int N, int nnz, int* d_err, hipStream_t st) {
    VCSRMC_HIP(hipMemsetAsync(d_err, 0, sizeof(int), st));
    RLAUNCH(k_check_rp, (long long)M + 1, rp, M, nnz, d_err);
    RLAUNCH(k_check_cols, (long long)nnz, col, (long long)nnz, N, d_err);
    raise_if(d_err, st);
}

// ---- 1. adjacency ------------------------------------------------------------------------
// Nonzero (r, c) contributes r -> c and c -> r when r < N; a row r >= N has no vertex of its
// own and makes c its own neighbour (twice, merged by the deduplication).
__global__ void k_adj_pairs(const int* __restrict__ row_of, const int* __restrict__ col,
                            long long nnz, int N, int nb, u64* __restrict__ key) {
    const long long p = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= nnz) return;
    const int r = row_of[p], c = col[p];
    const bool own = r < N;
    key[2 * p] = own ? ((u64)r << nb | (u64)c) : ((u64)c << nb | (u64)c);
    key[2 * p + 1] = (u64)c << nb | (u64)(own ? r : c);
}

__global__ void k_unique_flags(const u64* __restrict__ key, long long n, int* __restrict__ flag) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) flag[i] = (i == 0 || key[i] != key[i - 1]) ? 1 : 0;
}

__global__ void k_unique_write(const u64* __restrict__ key, const int* __restrict__ flag,
                               const long long* __restrict__ pos, long long n, int nb,
                               int* __restrict__ adj_u, int* __restrict__ adj) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n || !flag[i]) return;
    const u64 k = key[i];
    const long long p = pos[i];
    adj_u[p] = (int)(k >> nb);
    adj[p] = (int)(k & ((1ull << nb) - 1));
}

// head[v] = first adjacency entry of vertex v (lower bound in the sorted adj_u), v in [0, N].
__global__ void k_heads(const int* __restrict__ adj_u, long long E, int N,
                        long long* __restrict__ head) {
    const long long v = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (v > N) return;
    long long lo = 0, hi = E;
    while (lo < hi) {
        const long long mid = (lo + hi) >> 1;
        if (adj_u[mid] < v) lo = mid + 1;
        else hi = mid;
    }
    head[v] = lo;
}

// ---- 2. rank -----------------------------------------------------------------------------
__global__ void k_rank_keys(const long long* __restrict__ head, int N, int nb,
                            u64* __restrict__ key, uint32_t* __restrict__ val) {
    const long long v = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (v >= N) return;
    key[v] = (u64)(head[v + 1] - head[v]) << nb | (u64)v;
    val[v] = (uint32_t)v;
}

__global__ void k_scatter_rank(const uint32_t* __restrict__ order, int N, int* __restrict__ rank) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < N) rank[order[i]] = (int)i;
}

// ---- 3. components -----------------------------------------------------------------------
// Rounds of hooking and pointer jumping over plain loads and stores.  A round hooks, for every
// edge whose ends have different parents, the parent of larger rank under the other one if it
// is still a root, then moves every vertex to its grandparent.  parent[] only ever points to a
// vertex of smaller rank, so the trees stay acyclic whatever order the stores land in.  A round
// that changes nothing leaves every tree a star (each vertex's parent is a root) and no edge
// between two trees, so parent[v] is then the root of v's component, its lowest-rank vertex:
// the vertex the reference's loop over roots in rank order starts the component from.
__global__ void k_cc_init(int* __restrict__ parent, int N) {
    const long long v = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (v < N) parent[v] = (int)v;
}

__global__ void k_cc_hook(const int* __restrict__ adj_u, const int* __restrict__ adj, long long E,
                          const int* __restrict__ rank, int* parent, int* __restrict__ changed) {
    const long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const int u = adj_u[e], w = adj[e];
    if (u >= w) return;  // each undirected edge once; self-loops join nothing
    int a = parent[u], b = parent[w];
    if (a == b) return;
    if (rank[a] > rank[b]) { const int t = a; a = b; b = t; }
    if (parent[b] == b) {
        parent[b] = a;
        *changed = 1;
    }
}

__global__ void k_cc_jump(int* parent, int N, int* __restrict__ changed) {
    const long long v = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (v >= N) return;
    const int p = parent[v], gp = parent[p];
    if (gp != p) {
        parent[v] = gp;
        *changed = 1;
    }
}

// ---- 4. levels ---------------------------------------------------------------------------
__global__ void k_root_flags(const uint32_t* __restrict__ order, const int* __restrict__ comp,
                             int N, int* __restrict__ flag) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < N) flag[i] = comp[order[i]] == (int)order[i] ? 1 : 0;
}

__global__ void k_root_list(const uint32_t* __restrict__ order, const int* __restrict__ flag,
                            const long long* __restrict__ pos, int N, int* __restrict__ front,
                            int* __restrict__ lev, int* __restrict__ seq) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N || !flag[i]) return;
    const int v = (int)order[i];
    const int p = (int)pos[i];
    front[p] = v;
    lev[v] = 0;
    seq[v] = p;
}

__global__ void k_front_degree(const int* __restrict__ front, int f,
                               const long long* __restrict__ head, long long* __restrict__ fdeg) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < f) {
        const int v = front[i];
        fdeg[i] = head[v + 1] - head[v];
    }
}

// One thread per (frontier vertex, neighbour) edge.  An unvisited neighbour keeps the smallest
// frontier index that reaches it; the thread that claims it first appends it to `next`
// (wave-aggregated counter).  The order of `next` is fixed afterwards by a sort.
__global__ void k_claim(const int* __restrict__ front, const long long* __restrict__ fofs, int f,
                        long long Ef, const long long* __restrict__ head,
                        const int* __restrict__ adj, const int* __restrict__ lev,
                        int* __restrict__ claim, int* __restrict__ next,
                        int* __restrict__ count) {
    const long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    bool first = false;
    int u = 0;
    if (e < Ef) {
        int lo = 0, hi = f;  // largest i with fofs[i] <= e
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (fofs[mid] <= e) lo = mid;
            else hi = mid;
        }
        const int v = front[lo];
        u = adj[head[v] + (e - fofs[lo])];
        if (lev[u] < 0) first = atomicMin(&claim[u], lo) == INT_MAX;
    }
    const u64 m = __ballot(first);
    if (m == 0) return;
    const int leader = __ffsll((long long)m) - 1;
    int base = 0;
    if (lane_id() == leader) base = atomicAdd(count, __popcll(m));
    base = __shfl(base, leader);
    if (first) {
        const u64 below = lane_id() ? (~0ull >> (64 - lane_id())) : 0ull;
        next[base + __popcll(m & below)] = u;
    }
}

__global__ void k_next_keys(const int* __restrict__ next, int n, const int* __restrict__ claim,
                            int nb, u64* __restrict__ key, uint32_t* __restrict__ val) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int u = next[i];
    key[i] = (u64)claim[u] << nb | (u64)u;
    val[i] = (uint32_t)u;
}

__global__ void k_group_flags(const u64* __restrict__ key, int n, int nb, int* __restrict__ flag) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) flag[i] = (i == 0 || (key[i] >> nb) != (key[i - 1] >> nb)) ? 1 : 0;
}

// Children in (parent, ascending id) order, packed as degree << 32 | id for the group sort.
__global__ void k_group_pack(const int* __restrict__ flag, const long long* __restrict__ pos,
                             const uint32_t* __restrict__ val, int n,
                             const long long* __restrict__ head, int* __restrict__ gstart,
                             u64* __restrict__ packed) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (flag[i]) gstart[pos[i]] = (int)i;
    const uint32_t u = val[i];
    packed[i] = (u64)(head[u + 1] - head[u]) << 32 | (u64)u;
}

// std::sort(first, last, [](a, b) { return degree[a] < degree[b]; }) with the steps of GCC 11's
// libstdc++ (introsort: median-of-three Hoare partitions while a range holds more than 16
// elements, heapsort once 2 floor(lg n) partition levels are used up, then one insertion pass).
// The scans carry bounds checks the library omits; they never fire, as the median-of-three
// pivot and the insertion pass's leftmost minimum stop every scan inside its range.
__device__ __forceinline__ uint32_t skey(u64 x) { return (uint32_t)(x >> 32); }

__device__ void ls_insert(u64* a, long long lo, long long pos) {
    const u64 v = a[pos];
    while (pos > lo && skey(v) < skey(a[pos - 1])) {
        a[pos] = a[pos - 1];
        --pos;
    }
    a[pos] = v;
}

__device__ void ls_sift(u64* a, long long base, long long hole, long long len, u64 v) {
    const long long top = hole;
    long long child = hole;
    while (child < (len - 1) / 2) {
        child = 2 * child + 2;
        if (skey(a[base + child]) < skey(a[base + child - 1])) --child;
        a[base + hole] = a[base + child];
        hole = child;
    }
    if ((len & 1) == 0 && child == (len - 2) / 2) {
        child = 2 * child + 2;
        a[base + hole] = a[base + child - 1];
        hole = child - 1;
    }
    long long parent = (hole - 1) / 2;
    while (hole > top && skey(a[base + parent]) < skey(v)) {
        a[base + hole] = a[base + parent];
        hole = parent;
        parent = (hole - 1) / 2;
    }
    a[base + hole] = v;
}

__device__ void ls_heapsort(u64* a, long long lo, long long hi) {
    const long long len = hi - lo;
    if (len >= 2)
        for (long long parent = (len - 2) / 2;; --parent) {
            ls_sift(a, lo, parent, len, a[lo + parent]);
            if (parent == 0) break;
        }
    for (long long end = hi - 1; end - lo > 0; --end) {
        const u64 v = a[end];
        a[end] = a[lo];
        ls_sift(a, lo, 0, end - lo, v);
    }
}

__device__ __forceinline__ void ls_swap(u64* a, long long i, long long j) {
    const u64 t = a[i];
    a[i] = a[j];
    a[j] = t;
}

__device__ void ls_median_to_first(u64* a, long long dst, long long x, long long y, long long z) {
    const uint32_t kx = skey(a[x]), ky = skey(a[y]), kz = skey(a[z]);
    if (kx < ky) {
        if (ky < kz) ls_swap(a, dst, y);
        else if (kx < kz) ls_swap(a, dst, z);
        else ls_swap(a, dst, x);
    } else if (kx < kz) {
        ls_swap(a, dst, x);
    } else if (ky < kz) {
        ls_swap(a, dst, z);
    } else {
        ls_swap(a, dst, y);
    }
}

// Every pass moves lo up and hi down by at least one, so at most (hi - lo) / 2 + 1 passes run;
// the loop states that bound.
__device__ long long ls_partition(u64* a, long long lo, long long hi, long long piv) {
    const uint32_t kp = skey(a[piv]);
    const long long end = hi;
    for (long long pass = (hi - lo) / 2 + 1; pass >= 0; --pass) {
        while (lo < end && skey(a[lo]) < kp) ++lo;
        --hi;
        while (hi > piv && kp < skey(a[hi])) --hi;
        if (!(lo < hi)) return lo;
        ls_swap(a, lo, hi);
        ++lo;
    }
    return lo;
}

struct SortRange {
    int lo, hi, depth;
};

// std::sort's introsort loop on a[lo, hi) from partition depth `depth`, then its insertion
// pass over the same range.  Ranges that the loop leaves untouched are independent, so any
// subrange the partitions produce can be finished on its own: the insertion pass never moves
// an element across a partition boundary (left part <= pivot <= right part, and it only moves
// past strictly greater keys).
__device__ void ls_sort_range(u64* a, int lo0, int hi0, int depth0) {
    if (hi0 - lo0 <= 1) return;
    SortRange stack[64];
    int sp = 0;
    stack[sp++] = {lo0, hi0, depth0};
    while (sp > 0) {
        const SortRange r = stack[--sp];
        long long lo = r.lo, hi = r.hi;
        int depth = r.depth;
        while (hi - lo > 16) {
            if (depth == 0) {
                ls_heapsort(a, lo, hi);
                break;
            }
            --depth;
            ls_median_to_first(a, lo, lo + 1, lo + (hi - lo) / 2, hi - 1);
            const long long cut = ls_partition(a, lo + 1, hi, lo);
            if (sp < 64) stack[sp++] = {(int)cut, (int)hi, depth};
            hi = cut;
        }
    }
    for (int i = lo0 + 1; i < hi0; ++i) ls_insert(a, lo0, i);
}

__device__ __forceinline__ int lg_floor(int n) {
    int lg = 0;
    while ((2ll << lg) <= n) ++lg;
    return lg;
}

// Ranges of at most this many elements are sorted by one thread; larger ones are partitioned by
// a work-group first.
constexpr int kSortSmall = 256;

// One job per child group: (begin, end, partition depth 2 floor(lg n)).
__global__ void k_group_jobs(const int* __restrict__ gstart, int ngroups, int n,
                             int4* __restrict__ big, int* __restrict__ nbig,
                             int4* __restrict__ small, int* __restrict__ nsmall) {
    const long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= ngroups) return;
    const int b = gstart[g], e = g + 1 < ngroups ? gstart[g + 1] : n;
    if (e - b <= 1) return;
    const int4 job = make_int4(b, e, 2 * lg_floor(e - b), 0);
    if (e - b > kSortSmall) big[atomicAdd(nbig, 1)] = job;
    else small[atomicAdd(nsmall, 1)] = job;
}

// One wave per piece of at most kSortSmall elements, in LDS.  The wave runs the library's
// introsort loop with wave-wide partition steps (wave_partition_lds) and marks the pieces it
// leaves (at most 16 elements, or depth exhausted); then each lane finishes the pieces it finds:
// the insertion pass, or a heapsort.  As in k_bfs_levels, every lane keeps its own identical
// copy of the range stack, so no branch taken by one lane alone steers the loop.
constexpr int kSmallSortWaves = 4;
constexpr unsigned char kPieceNone = 255, kPieceEnd = 254, kPieceHeap = 253;

__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One step of the introsort loop on s[lo, hi) (hi - lo > 16, depth > 0) by one wave: the
// computation of k_partition_pass on 64 lanes.  lpos and rpos hold the pair positions
// (K <= (hi - lo) / 2).  Returns the cut in every lane.
__device__ int wave_partition_lds(u64* s, int lo, int hi, int* lpos, int* rpos, int* lnext) {
    const int lane = threadIdx.x & 63;
    if (lane == 0) {
        ls_median_to_first(s, lo, lo + 1, lo + (hi - lo) / 2, hi - 1);
        *lnext = INT_MAX;
    }
    wave_lds_fence();
    const uint32_t kp = skey(s[lo]);
    const int first = lo + 1, n = hi - first;
    const int per = (n + 63) / 64;
    const int b0 = min(first + lane * per, hi), b1 = min(b0 + per, hi);
    int cge = 0, cle = 0;
    for (int p = b0; p < b1; ++p) {
        const uint32_t k = skey(s[p]);
        cge += !(k < kp);
        cle += !(kp < k);
    }
    const int ge_incl = wave_scan(cge, OpAdd{}, 0), le_all = wave_scan(cle, OpAdd{}, 0);
    const int ge_before = ge_incl - cge, le_before = le_all - cle;
    const int LE = __builtin_amdgcn_readlane(le_all, 63);
    int kc = 0;
    {
        int rank = ge_before, le_incl = le_before;
        for (int p = b0; p < b1; ++p) {
            const uint32_t k = skey(s[p]);
            le_incl += !(kp < k);
            if (!(k < kp)) {
                ++rank;
                kc += (LE - le_incl >= rank);
            }
        }
    }
    const int K = __builtin_amdgcn_readlane(wave_scan(kc, OpAdd{}, 0), 63);
    {
        int rank = ge_before, le_excl = le_before;
        for (int p = b0; p < b1; ++p) {
            const uint32_t k = skey(s[p]);
            if (!(k < kp)) {
                ++rank;
                if (rank <= K) lpos[rank - 1] = p;
                else if (rank == K + 1) *lnext = p;
            }
            if (!(kp < k)) {
                const int rr = LE - le_excl;
                if (rr <= K) rpos[rr - 1] = p;
                ++le_excl;
            }
        }
    }
    wave_lds_fence();
    for (int r = lane; r < K; r += 64) {
        const int x = lpos[r], y = rpos[r];
        const u64 ax = s[x], ay = s[y];
        s[x] = ay;
        s[y] = ax;
    }
    wave_lds_fence();
    return K == 0 ? *lnext : min(*lnext, rpos[K - 1]);
}

__global__ __launch_bounds__(64 * kSmallSortWaves) void k_small_sort(
    const int4* __restrict__ jobs, int njobs, u64* __restrict__ a) {
    __shared__ u64 piece[kSmallSortWaves][kSortSmall];
    __shared__ unsigned char marks[kSmallSortWaves][kSortSmall + 4];
    __shared__ int pairs[kSmallSortWaves][kSortSmall];  // lpos, then rpos
    __shared__ int lnext[kSmallSortWaves];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const long long j = (long long)blockIdx.x * kSmallSortWaves + w;
    if (j >= njobs) return;  // the same for every lane of the wave
    const int4 job = jobs[j];
    const int n = job.y - job.x;  // at most kSortSmall
    if (n <= 1) return;
    u64* s = piece[w];
    unsigned char* mark = marks[w];
    for (int i = lane; i < n; i += 64) s[i] = a[job.x + i];
    for (int i = lane; i < n; i += 64) mark[i] = kPieceNone;
    if (lane == 0) mark[n] = kPieceEnd;
    wave_lds_fence();
    int4 stk[64];  // depth <= 2 floor(lg n) < 63 for n < 2^31
    int sp = 1;
    stk[0] = make_int4(0, n, job.z, 0);
    while (sp > 0) {
        const int4 r = stk[sp - 1];
        if (r.y - r.x <= 16 || r.z == 0) {
            mark[r.x] = r.y - r.x > 16 ? kPieceHeap : (unsigned char)r.z;
            --sp;
        } else {
            const int cut = wave_partition_lds(s, r.x, r.y, pairs[w], pairs[w] + kSortSmall / 2,
                                               &lnext[w]);
            stk[sp - 1] = make_int4(cut, r.y, r.z - 1, 0);
            stk[sp] = make_int4(r.x, cut, r.z - 1, 0);
            ++sp;
        }
    }
    wave_lds_fence();
    for (int i = lane; i < n; i += 64) {
        const int m = mark[i];
        if (m <= kPieceHeap) {
            int e = i + 1;
            while (mark[e] == kPieceNone) ++e;
            if (m == kPieceHeap) ls_heapsort(s, i, e);
            else if (e - i > 1) ls_sort_range(s, i, e, m);
        }
    }
    wave_lds_fence();
    for (int i = lane; i < n; i += 64) a[job.x + i] = s[i];
}

// One step of the introsort loop on a large range, by a whole work-group, with the same result
// as the library's sequential step.  After the median of three is moved to a[lo], the Hoare
// scans over a[lo+1, hi) stop, from the left, at elements whose key is not below the pivot's
// (l_1 < l_2 < ...) and, from the right, at elements whose key is not above it
// (r_1 > r_2 > ...); the k-th swap exchanges a[l_k] and a[r_k] while l_k < r_k, so K = the
// number of left stops x with at least rank(x) right stops after x; the cut is l_1 when K = 0,
// else min(l_{K+1}, r_K).  Both parts continue with depth - 1; a range at depth 0 is heapsorted.
__global__ __launch_bounds__(256) void k_partition_pass(
    const int4* __restrict__ jobs, int4* __restrict__ next, int* __restrict__ nnext,
    int4* __restrict__ small, int* __restrict__ nsmall, u64* a, int* __restrict__ lpos,
    int* __restrict__ rpos) {
    __shared__ int wsum[4];
    __shared__ int sh_lnext;
    const int4 job = jobs[blockIdx.x];
    const int lo = job.x, hi = job.y, depth = job.z;
    const int t = threadIdx.x;
    if (depth == 0) {
        if (t == 0) ls_heapsort(a, lo, hi);  // sorted: the insertion pass would change nothing
        return;
    }
    if (t == 0) {
        ls_median_to_first(a, lo, lo + 1, lo + (hi - lo) / 2, hi - 1);
        sh_lnext = INT_MAX;
    }
    __syncthreads();
    const uint32_t kp = skey(a[lo]);
    const int first = lo + 1, n = hi - first;
    const int per = (n + 255) / 256;
    const int b0 = min(first + t * per, hi), b1 = min(b0 + per, hi);
    int cge = 0, cle = 0;
    for (int p = b0; p < b1; ++p) {
        const uint32_t k = skey(a[p]);
        cge += !(k < kp);
        cle += !(kp < k);
    }
    int GE, LE;
    const int ge_before = block_scan_256(cge, OpAdd{}, 0, wsum, GE) - cge;
    const int le_before = block_scan_256(cle, OpAdd{}, 0, wsum, LE) - cle;
    (void)GE;
    // K: left stops x (rank r) with LE - (right stops at or before x) >= r.
    int kc = 0;
    {
        int rank = ge_before, le_incl = le_before;
        for (int p = b0; p < b1; ++p) {
            const uint32_t k = skey(a[p]);
            le_incl += !(kp < k);
            if (!(k < kp)) {
                ++rank;
                kc += (LE - le_incl >= rank);
            }
        }
    }
    int K;
    block_scan_256(kc, OpAdd{}, 0, wsum, K);
    // Pair positions: lpos[lo + r - 1] = l_r, rpos[lo + r - 1] = r_r for r <= K; and l_{K+1}.
    {
        int rank = ge_before, le_excl = le_before;
        for (int p = b0; p < b1; ++p) {
            const uint32_t k = skey(a[p]);
            if (!(k < kp)) {
                ++rank;
                if (rank <= K) lpos[lo + rank - 1] = p;
                else if (rank == K + 1) sh_lnext = p;
            }
            if (!(kp < k)) {
                const int rr = LE - le_excl;  // right stops in [p, hi)
                if (rr <= K) rpos[lo + rr - 1] = p;
                ++le_excl;
            }
        }
    }
    __syncthreads();
    for (int r = t; r < K; r += 256) {
        const int x = lpos[lo + r], y = rpos[lo + r];
        const u64 ax = a[x], ay = a[y];
        a[x] = ay;
        a[y] = ax;
    }
    if (t == 0) {
        const int cut = K == 0 ? sh_lnext : min(sh_lnext, rpos[lo + K - 1]);
        const int d = depth - 1;
        const int4 left = make_int4(lo, cut, d, 0), right = make_int4(cut, hi, d, 0);
        if (cut - lo > kSortSmall) next[atomicAdd(nnext, 1)] = left;
        else small[atomicAdd(nsmall, 1)] = left;
        if (hi - cut > kSortSmall) next[atomicAdd(nnext, 1)] = right;
        else small[atomicAdd(nsmall, 1)] = right;
    }
}

__global__ void k_level_write(const u64* __restrict__ packed, int n, int level, int base,
                              int* __restrict__ front, int* __restrict__ lev,
                              int* __restrict__ seq) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int u = (int)(uint32_t)packed[i];
    front[i] = u;
    lev[u] = level;
    seq[u] = base + (int)i;
}

// ---- 4b. small levels in one work-group ---------------------------------------------------
// While a level has at most kBfsCap frontier vertices and frontier edges, one work-group runs
// level after level with no host round trip: each frontier edge claims its neighbour (atomic
// minimum of the frontier index, as k_claim), then an edge holds a child when its frontier
// vertex won the claim.  Frontier vertices are in level order and each adjacency list is in
// ascending id, so an exclusive scan over the edges places the children in (parent index,
// ascending id) order directly; each parent's children are then sorted by degree with
// std::sort's steps in LDS: groups of up to kBfsSortSmall by their parent's thread, larger ones
// (the children of hub vertices) partitioned by the whole work-group, a step at a time as
// k_partition_pass does, and the pieces finished by one thread each.  Thread t owns a contiguous run of up to
// kBfsPer vertices or edges, so each phase needs one block scan.  The work-group stops at the
// first level that does not fit (state.w = 0: the frontier is left in front[]) or when the walk
// ends (state.w = 1).  state = {frontier size, vertices placed, level, finished}.
constexpr int kBfsThreads = 1024;
constexpr int kBfsPer = 8;
constexpr int kBfsCap = kBfsThreads * kBfsPer;
constexpr int kBfsSortSmall = 64;
constexpr int kBfsMaxBig = kBfsCap / (kBfsSortSmall + 1) + 1;
// Marks of the piece starts during the work-group sort (one byte per child position): the
// partition depth a piece continues from, or one of these.
constexpr unsigned char kMarkNone = 255, kMarkGroupEnd = 254, kMarkHeap = 253;

template <int NW>
__device__ __forceinline__ int block_scan_int(int x, int* wsum /* LDS[NW] */, int& total) {
    const int t = threadIdx.x, w = t >> 6;
    const int incl = wave_scan(x, OpAdd{}, 0);
    if ((t & 63) == 63) wsum[w] = incl;
    __syncthreads();
    int before = 0, all = 0;
    for (int i = 0; i < NW; ++i) {
        const int s = wsum[i];
        if (i < w) before += s;
        all += s;
    }
    total = all;
    __syncthreads();
    return before + incl;
}

// One step of the introsort loop on a[lo, hi) (depth > 0) by the whole work-group, with the
// library's result: k_partition_pass's computation on an LDS range.  lpos and rpos hold the
// pair positions relative to the range (K <= (hi - lo) / 2, as the pairs are disjoint).
// Returns the cut (the same value in every thread).
template <int NW>
__device__ int block_partition_lds(u64* a, int lo, int hi, int* lpos, int* rpos, int* wsum,
                                   int* lnext) {
    const int t = threadIdx.x;
    if (t == 0) {
        ls_median_to_first(a, lo, lo + 1, lo + (hi - lo) / 2, hi - 1);
        *lnext = INT_MAX;
    }
    __syncthreads();
    const uint32_t kp = skey(a[lo]);
    const int first = lo + 1, n = hi - first;
    const int per = (n + kBfsThreads - 1) / kBfsThreads;
    const int b0 = min(first + t * per, hi), b1 = min(b0 + per, hi);
    int cge = 0, cle = 0;
    for (int p = b0; p < b1; ++p) {
        const uint32_t k = skey(a[p]);
        cge += !(k < kp);
        cle += !(kp < k);
    }
    int GE, LE;
    const int ge_before = block_scan_int<NW>(cge, wsum, GE) - cge;
    const int le_before = block_scan_int<NW>(cle, wsum, LE) - cle;
    int kc = 0;
    {
        int rank = ge_before, le_incl = le_before;
        for (int p = b0; p < b1; ++p) {
            const uint32_t k = skey(a[p]);
            le_incl += !(kp < k);
            if (!(k < kp)) {
                ++rank;
                kc += (LE - le_incl >= rank);
            }
        }
    }
    int K;
    block_scan_int<NW>(kc, wsum, K);
    {
        int rank = ge_before, le_excl = le_before;
        for (int p = b0; p < b1; ++p) {
            const uint32_t k = skey(a[p]);
            if (!(k < kp)) {
                ++rank;
                if (rank <= K) lpos[rank - 1] = p;
                else if (rank == K + 1) *lnext = p;
            }
            if (!(kp < k)) {
                const int rr = LE - le_excl;
                if (rr <= K) rpos[rr - 1] = p;
                ++le_excl;
            }
        }
    }
    __syncthreads();
    for (int r = t; r < K; r += kBfsThreads) {
        const int x = lpos[r], y = rpos[r];
        const u64 ax = a[x], ay = a[y];
        a[x] = ay;
        a[y] = ax;
    }
    const int cut = K == 0 ? *lnext : min(*lnext, rpos[K - 1]);
    __syncthreads();
    return cut;
}

// A walk of N vertices has at most N levels after the roots; the loop runs to `max_level` at
// most (N + 1, or lower when a test asks) and otherwise reports state.w = kBfsOverrun.
constexpr int kBfsOverrun = 2;

__global__ __launch_bounds__(kBfsThreads) void k_bfs_levels(
    int* __restrict__ front, const long long* __restrict__ head, const int* __restrict__ adj,
    int* __restrict__ lev, int* __restrict__ seq, int* claim, int N, long long max_level,
    int4* __restrict__ state) {
    constexpr int NW = kBfsThreads / 64;
    __shared__ int s_ofs[kBfsCap + 1];    // edge offset of each frontier vertex
    __shared__ int s_fx[kBfsCap + 1];     // the frontier; then children before each edge
    __shared__ u64 s_packed[kBfsCap];     // degree << 32 | id of the next level
    __shared__ int s_wsum[NW];
    __shared__ int2 s_big[kBfsMaxBig];  // child groups larger than kBfsSortSmall
    __shared__ int s_nbig, s_lnext;
    int* const s_front = s_fx;
    int* const s_ex = s_fx;
    unsigned char* const s_mark = reinterpret_cast<unsigned char*>(s_fx);  // during the sort
    const int t = threadIdx.x;
    const int4 s0 = *state;
    int f = s0.x, base = s0.y, level = s0.z;
    bool finished = false, moved = false, overrun = false;
    for (int i = t; i < f; i += kBfsThreads) s_front[i] = front[i];
    // `level` is the same in every thread: the bound ends the loop for all of them at once.
    for (;;) {
        __syncthreads();
        if (f == 0 || base >= N) {
            finished = true;
            break;
        }
        if (level > max_level) {
            overrun = true;
            break;
        }
        // edge offsets of the frontier vertices [v0, v1) of this thread
        const int pf = (f + kBfsThreads - 1) / kBfsThreads;
        const int v0 = min(t * pf, f), v1 = min(v0 + pf, f);
        int deg[kBfsPer];
        int dsum = 0;
#pragma unroll
        for (int i = 0; i < kBfsPer; ++i) {
            deg[i] = 0;
            if (v0 + i < v1) {
                const int v = s_front[v0 + i];
                deg[i] = (int)min(head[v + 1] - head[v], (long long)kBfsCap + 1);
                dsum += deg[i];
            }
        }
        int Ef;
        int ofs = block_scan_int<NW>(dsum, s_wsum, Ef) - dsum;
        if (Ef == 0) {
            finished = true;
            break;
        }
        if (Ef > kBfsCap) break;
#pragma unroll
        for (int i = 0; i < kBfsPer; ++i)
            if (v0 + i < v1) {
                s_ofs[v0 + i] = ofs;
                ofs += deg[i];
            }
        if (t == 0) s_ofs[f] = Ef;
        __syncthreads();
        // claims of the edges [e0, e1) of this thread
        const int pe = (Ef + kBfsThreads - 1) / kBfsThreads;
        const int e0 = min(t * pe, Ef), e1 = min(e0 + pe, Ef);
        int us[kBfsPer], los[kBfsPer];
        {
            int lo = 0, hi = f;  // largest lo with s_ofs[lo] <= e0
            while (hi - lo > 1) {
                const int mid = (lo + hi) >> 1;
                if (s_ofs[mid] <= e0) lo = mid;
                else hi = mid;
            }
#pragma unroll
            for (int i = 0; i < kBfsPer; ++i) {
                us[i] = -1;
                los[i] = 0;
                const int e = e0 + i;
                if (e < e1) {
                    while (s_ofs[lo + 1] <= e) ++lo;
                    const int v = s_front[lo];
                    const int u = adj[head[v] + (e - s_ofs[lo])];
                    if (lev[u] < 0) {
                        atomicMin(&claim[u], lo);
                        us[i] = u;
                        los[i] = lo;
                    }
                }
            }
        }
        __syncthreads();
        int child = 0, nchild = 0;
#pragma unroll
        for (int i = 0; i < kBfsPer; ++i) {
            const bool c = us[i] >= 0 && __hip_atomic_load(claim + us[i], __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT) == los[i];
            child |= (int)c << i;
            nchild += c;
        }
        int n;
        int pos = block_scan_int<NW>(nchild, s_wsum, n) - nchild;
#pragma unroll
        for (int i = 0; i < kBfsPer; ++i)
            if (e0 + i < e1) {
                s_ex[e0 + i] = pos;
                if ((child >> i) & 1) {
                    const int u = us[i];
                    s_packed[pos++] = (u64)(head[u + 1] - head[u]) << 32 | (u64)(uint32_t)u;
                }
            }
        if (t == 0) {
            s_ex[Ef] = n;
            s_nbig = 0;
        }
        __syncthreads();
        for (int lo = v0; lo < v1; ++lo) {
            const int b = s_ex[s_ofs[lo]], e = s_ex[s_ofs[lo + 1]];
            if (e - b > kBfsSortSmall) s_big[atomicAdd(&s_nbig, 1)] = make_int2(b, e);
            else if (e - b > 1) ls_sort_range(s_packed, b, e, 2 * lg_floor(e - b));
        }
        __syncthreads();
        const int nbig = s_nbig;
        if (nbig > 0) {
            // s_ex and s_ofs are free until the next level: s_mark over s_ex, the pair
            // positions over s_ofs.  Group ends are marked before any piece start, so a piece
            // starting where another group ends keeps its mark.
            for (int i = t; i <= n; i += kBfsThreads) s_mark[i] = kMarkNone;
            __syncthreads();
            for (int g = t; g < nbig; g += kBfsThreads) s_mark[s_big[g].y] = kMarkGroupEnd;
            // Every thread runs the same stack of ranges (lo, hi, depth) in its own registers:
            // its control flow depends only on values all threads share (the ranges and the
            // cuts), and no branch taken by one thread alone decides what the others do next
            // (with the stack in LDS and thread 0 alone updating it, the compiler moved that
            // update out of the loop for thread 0, and the other threads never saw it).
            for (int g = 0; g < nbig; ++g) {
                __syncthreads();
                const int2 gr = s_big[g];
                int4 stk[2 * 13 + 2];  // depth 2 floor(lg n) <= 26 for n <= kBfsCap
                int sp = 1;
                stk[0] = make_int4(gr.x, gr.y, 2 * lg_floor(gr.y - gr.x), 0);
                while (sp > 0) {
                    const int4 r = stk[sp - 1];
                    if (r.y - r.x <= kBfsSortSmall || r.z == 0) {
                        // a piece to finish after the loop, by the thread that finds its mark
                        s_mark[r.x] = r.y - r.x > kBfsSortSmall ? kMarkHeap : (unsigned char)r.z;
                        --sp;
                    } else {
                        const int cut = block_partition_lds<NW>(
                            s_packed, r.x, r.y, s_ofs, s_ofs + kBfsCap / 2, s_wsum, &s_lnext);
                        stk[sp - 1] = make_int4(cut, r.y, r.z - 1, 0);
                        stk[sp] = make_int4(r.x, cut, r.z - 1, 0);
                        ++sp;
                    }
                }
            }
            __syncthreads();
            for (int i = t; i < n; i += kBfsThreads) {
                const int m = s_mark[i];
                if (m <= kMarkHeap) {
                    int e = i + 1;
                    while (e < n && s_mark[e] == kMarkNone) ++e;  // the group's end is marked
                    if (m == kMarkHeap) ls_heapsort(s_packed, i, e);  // depth exhausted
                    else if (e - i > 1) ls_sort_range(s_packed, i, e, m);
                }
            }
        }
        __syncthreads();
        for (int i = t; i < n; i += kBfsThreads) {
            const int w = (int)(uint32_t)s_packed[i];
            s_front[i] = w;
            lev[w] = level;
            seq[w] = base + i;
        }
        base += n;
        f = n;
        ++level;
        moved = true;
    }
    if (moved)
        for (int i = t; i < f; i += kBfsThreads) front[i] = s_front[i];
    if (t == 0) *state = make_int4(f, base, level, overrun ? kBfsOverrun : finished ? 1 : 0);
}

// ---- 5. order ----------------------------------------------------------------------------
__global__ void k_order_keys(const int* __restrict__ comp, const int* __restrict__ rank,
                             const int* __restrict__ seq, int N, int nb, u64* __restrict__ key,
                             uint32_t* __restrict__ val) {
    const long long v = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (v >= N) return;
    key[v] = (u64)rank[comp[v]] << nb | (u64)seq[v];
    val[v] = (uint32_t)v;
}

__global__ void k_positions(const uint32_t* __restrict__ order, int N, int* __restrict__ position) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < N) position[order[i]] = N - 1 - (int)i;
}

// ---- relabelling -------------------------------------------------------------------------
__global__ void k_perm_check(const int* __restrict__ position, int N, int* __restrict__ seen,
                             int* __restrict__ err) {
    const long long v = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (v >= N) return;
    const int p = position[v];
    if (p < 0 || p >= N || atomicAdd(&seen[p], 1) != 0) atomicOr(err, kBadPerm);
}

__global__ void k_relabel_keys(const int* __restrict__ row_of, const int* __restrict__ col,
                               const int* __restrict__ position, long long nnz, int nb,
                               u64* __restrict__ key, uint32_t* __restrict__ val) {
    const long long p = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= nnz) return;
    key[p] = (u64)row_of[p] << nb | (u64)position[col[p]];
    val[p] = (uint32_t)p;
}

// Two equal sorted (row, new column) keys: a row holds a column twice.  Checked before
// anything is written, so a rejected call leaves the caller's CSR as it was.
__global__ void k_relabel_dups(const u64* __restrict__ key, long long nnz,
                               int* __restrict__ err) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i > 0 && i < nnz && key[i - 1] == key[i]) atomicOr(err, kDupCol);
}

__global__ void k_relabel_write(const u64* __restrict__ key, const uint32_t* __restrict__ src,
                                const float* __restrict__ vin, long long nnz, int nb,
                                int* __restrict__ col, float* __restrict__ vout) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nnz) return;
    col[i] = (int)(key[i] & ((1ull << nb) - 1));
    vout[i] = vin[src[i]];
}

// B_out[position[r], :] = B[r, :]; one thread per element, rows of O consecutive floats.
__global__ void k_permute_rows(const float* __restrict__ B, const int* __restrict__ position,
                               int N, int O, float* __restrict__ Bout) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)N * O) return;
    const long long r = i / O, k = i - r * O;
    Bout[(long long)position[r] * O + k] = B[i];
}

__global__ void k_mark_heads(const int* __restrict__ rp, int M, int* __restrict__ head) {
    const long long r = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= M) return;
    const int a = rp[r];
    if (a < rp[r + 1]) head[a] = (int)r;
}

// Row of every nonzero: each non-empty row marks its first slot, a running max fills the rest.
void row_of_nonzeros(const int* rp, int M, int nnz, int* row_of, hipStream_t st) {
    DevBuf<int> headmark(nnz);
    fill<int>(headmark.p, nnz, (int)0x80000000, st);
    RLAUNCH(k_mark_heads, M, rp, M, headmark.p);
    inclusive_max(headmark.p, row_of, nnz, st);
}

// Work lists of the child-group sort, sized for the largest level (a range never holds fewer
// than one element, so there are at most N ranges of each kind).
struct SortJobs {
    DevBuf<int4> big0, big1, small;
    DevBuf<int> lpos, rpos, counts;  // counts: {big0, big1, small}
    explicit SortJobs(int N)
        : big0(N), big1(N), small(N), lpos(N), rpos(N), counts(3) {}
};

// Each child group of one level sorted by degree with std::sort's steps: large ranges are
// partitioned a step at a time by work-groups until every piece holds at most kSortSmall
// elements (or reached heapsort), then one thread per piece finishes it.
void sort_groups(const int* gstart, int ngroups, int n, u64* packed, SortJobs& J, hipStream_t st) {
    VCSRMC_HIP(hipMemsetAsync(J.counts.p, 0, sizeof(int) * 3, st));
    RLAUNCH(k_group_jobs, ngroups, gstart, ngroups, n, J.big0.p, J.counts.p, J.small.p,
            J.counts.p + 2);
    int4* cur = J.big0.p;
    int4* nxt = J.big1.p;
    int* ccur = J.counts.p;
    int* cnxt = J.counts.p + 1;
    int counts[3];
    VCSRMC_HIP(hipMemcpyAsync(counts, J.counts.p, sizeof(counts), hipMemcpyDeviceToHost, st));
    VCSRMC_HIP(hipStreamSynchronize(st));
    int nbig = counts[0], nsmall = counts[2];
    const bool passes = nbig > 0;
    // Every pass lowers the depth of the ranges it keeps, which starts at 2 floor(lg n) < 63:
    // more passes than that means a broken partition step, reported instead of looping.
    int pass = 0;
    while (nbig > 0) {
        if (++pass > 64) throw Error(VCSRMC_ERR_STATE, "RCM child sort did not converge");
        VCSRMC_HIP(hipMemsetAsync(cnxt, 0, sizeof(int), st));
        hipLaunchKernelGGL(k_partition_pass, dim3(nbig), dim3(256), 0, st, cur, nxt, cnxt,
                           J.small.p, J.counts.p + 2, packed, J.lpos.p, J.rpos.p);
        VCSRMC_HIP(hipGetLastError());
        nbig = read_scalar(cnxt, st);
        std::swap(cur, nxt);
        std::swap(ccur, cnxt);
    }
    if (passes) nsmall = read_scalar(J.counts.p + 2, st);
    if (nsmall > 0) {
        hipLaunchKernelGGL(k_small_sort, dim3((unsigned)((nsmall + kSmallSortWaves - 1) /
                                                          kSmallSortWaves)),
                           dim3(64 * kSmallSortWaves), 0, st, J.small.p, nsmall, packed);
        VCSRMC_HIP(hipGetLastError());
    }
}

// Iteration limits of the ordering's loops; 0 selects the proven maxima (see rcm_order_device).
// Process-wide, read once by each ordering.
std::atomic<long long> g_max_level{0}, g_max_rounds{0};

}  // namespace

void set_rcm_limits(long long max_level, long long max_rounds) {
    g_max_level.store(max_level, std::memory_order_relaxed);
    g_max_rounds.store(max_rounds, std::memory_order_relaxed);
}

void rcm_order_device(const int* rp, const int* col, int M, int N, int nnz, int* position,
                      hipStream_t st) {
    if (M < 0 || N < 0 || nnz < 0) throw Error(VCSRMC_ERR_ARG, "negative matrix size");
    if (!rp || (nnz > 0 && !col) || (N > 0 && !position))
        throw Error(VCSRMC_ERR_ARG, "null pointer");
    if (2ll * nnz >= (1ll << 31))
        throw Error(VCSRMC_ERR_OVERFLOW, "rcm ordering handles fewer than 2^30 nonzeros");
    DevBuf<int> err(1);
    check_csr(rp, col, M, N, nnz, err.p, st);
    if (N == 0) return;

    const int nb = std::max(1, bits_for((u64)N));  // holds 0..N
    // 1. adjacency
    DevBuf<int> adj_u, adj;
    DevBuf<long long> head((size_t)N + 1);
    long long E = 0;
    {
        const long long P = 2ll * nnz;
        DevBuf<int> row_of(nnz);
        if (nnz) row_of_nonzeros(rp, M, nnz, row_of.p, st);
        DevBuf<u64> k1(P), k2(P);
        DevBuf<uint32_t> v1(P), v2(P);
        RLAUNCH(k_adj_pairs, nnz, row_of.p, col, (long long)nnz, N, nb, k1.p);
        row_of.release();
        u64 *ka = k1.p, *kb = k2.p;
        uint32_t *va = v1.p, *vb = v2.p;
        radix_sort_pairs<u64>(ka, va, kb, vb, P, 2 * nb, st);
        DevBuf<int> flag(P);
        DevBuf<long long> pos(P + 1);
        RLAUNCH(k_unique_flags, P, ka, P, flag.p);
        exclusive_sum<int, long long>(flag.p, pos.p, P, st);
        E = P ? read_scalar(pos.p + P, st) : 0;
        adj_u.alloc(E);
        adj.alloc(E);
        RLAUNCH(k_unique_write, P, ka, flag.p, pos.p, P, nb, adj_u.p, adj.p);
    }
    RLAUNCH(k_heads, (long long)N + 1, adj_u.p, E, N, head.p);

    // 2. rank
    DevBuf<uint32_t> order(N);
    DevBuf<int> rank(N);
    {
        DevBuf<u64> k1(N), k2(N);
        DevBuf<uint32_t> v2(N);
        RLAUNCH(k_rank_keys, N, head.p, N, nb, k1.p, order.p);
        u64 *ka = k1.p, *kb = k2.p;
        uint32_t *va = order.p, *vb = v2.p;
        radix_sort_pairs<u64>(ka, va, kb, vb, N, 2 * nb, st);
        if (va != order.p)
            VCSRMC_HIP(hipMemcpyAsync(order.p, va, sizeof(uint32_t) * (size_t)N,
                                      hipMemcpyDeviceToDevice, st));
        RLAUNCH(k_scatter_rank, N, order.p, N, rank.p);
    }

    // Proven maxima of the loops below.  Levels: every level but the last places at least one
    // vertex, so level <= N.  Component rounds: a round changes something or ends the loop;
    // between two rounds with a hook (each hook removes a tree, so at most N - 1 of them),
    // pointer jumping alone halves every depth, so after ceil(lg N) + 1 rounds all trees are
    // stars and the next round either hooks or changes nothing: at most
    // N (ceil(lg N) + 2) + 1 rounds.
    const long long lim_level = g_max_level.load(std::memory_order_relaxed);
    const long long lim_rounds = g_max_rounds.load(std::memory_order_relaxed);
    const long long max_level = lim_level > 0 ? lim_level : (long long)N + 1;
    const long long max_rounds =
        lim_rounds > 0 ? lim_rounds : (long long)N * (bits_for((u64)N) + 2) + 1;

    // 3. components
    DevBuf<int> comp(N);
    {
        DevBuf<int> changed(1);
        RLAUNCH(k_cc_init, N, comp.p, N);
        for (long long round = 0;; ++round) {
            if (round >= max_rounds)
                throw Error(VCSRMC_ERR_STATE, "rcm ordering: connected components did not settle "
                                              "within " + std::to_string(max_rounds) + " rounds");
            fill<int>(changed.p, 1, 0, st);
            RLAUNCH(k_cc_hook, E, adj_u.p, adj.p, E, rank.p, comp.p, changed.p);
            RLAUNCH(k_cc_jump, N, comp.p, N, changed.p);
            if (!read_scalar(changed.p, st)) break;
        }
    }
    adj_u.release();

    // 4. levels
    DevBuf<int> lev(N), seq(N), claim(N), front(N), next(N), count(1);
    fill<int>(lev.p, N, -1, st);
    fill<int>(claim.p, N, INT_MAX, st);
    int f = 0;
    {
        DevBuf<int> flag(N);
        DevBuf<long long> pos((size_t)N + 1);
        RLAUNCH(k_root_flags, N, order.p, comp.p, N, flag.p);
        exclusive_sum<int, long long>(flag.p, pos.p, N, st);
        f = (int)read_scalar(pos.p + N, st);
        RLAUNCH(k_root_list, N, order.p, flag.p, pos.p, N, front.p, lev.p, seq.p);
    }
    DevBuf<long long> fdeg(N), fofs((size_t)N + 1);
    DevBuf<u64> k1(N), k2(N);
    DevBuf<uint32_t> v1(N), v2(N);
    DevBuf<int> gflag(N), gstart(N);
    DevBuf<long long> gpos((size_t)N + 1);
    SortJobs jobs(N);
    DevBuf<int4> bfs_state(1);
    int base = f, level = 1;
    while (f > 0 && base < N) {
        if (f <= kBfsCap) {  // run levels inside one work-group while they are small
            const int4 s0 = make_int4(f, base, level, 0);
            VCSRMC_HIP(hipMemcpyAsync(bfs_state.p, &s0, sizeof(s0), hipMemcpyHostToDevice, st));
            hipLaunchKernelGGL(k_bfs_levels, dim3(1), dim3(kBfsThreads), 0, st, front.p, head.p,
                               adj.p, lev.p, seq.p, claim.p, N, max_level, bfs_state.p);
            VCSRMC_HIP(hipGetLastError());
            const int4 s1 = read_scalar(bfs_state.p, st);
            f = s1.x;
            base = s1.y;
            level = s1.z;
            if (s1.w || f == 0 || base >= N) break;  // finished, or overran max_level
        }
        if (level > max_level) break;
        // a level whose frontier or edge count exceeds one work-group
        RLAUNCH(k_front_degree, f, front.p, f, head.p, fdeg.p);
        exclusive_sum<long long, long long>(fdeg.p, fofs.p, f, st);
        const long long Ef = read_scalar(fofs.p + f, st);
        if (Ef == 0) break;
        VCSRMC_HIP(hipMemsetAsync(count.p, 0, sizeof(int), st));
        RLAUNCH(k_claim, Ef, front.p, fofs.p, f, Ef, head.p, adj.p, lev.p, claim.p, next.p,
                count.p);
        const int n = read_scalar(count.p, st);
        if (n == 0) break;
        const int cb = std::max(1, bits_for((u64)(f - 1)));
        RLAUNCH(k_next_keys, n, next.p, n, claim.p, nb, k1.p, v1.p);
        u64 *ka = k1.p, *kb = k2.p;
        uint32_t *va = v1.p, *vb = v2.p;
        radix_sort_pairs<u64>(ka, va, kb, vb, n, nb + cb, st);
        RLAUNCH(k_group_flags, n, ka, n, nb, gflag.p);
        exclusive_sum<int, long long>(gflag.p, gpos.p, n, st);
        const int ngroups = (int)read_scalar(gpos.p + n, st);
        u64* packed = kb;  // free half of the key double buffer
        RLAUNCH(k_group_pack, n, gflag.p, gpos.p, va, n, head.p, gstart.p, packed);
        sort_groups(gstart.p, ngroups, n, packed, jobs, st);
        RLAUNCH(k_level_write, n, packed, n, level, base, front.p, lev.p, seq.p);
        base += n;
        f = n;
        ++level;
    }
    if (level > max_level)
        throw Error(VCSRMC_ERR_STATE, "rcm ordering: the breadth-first walk passed " +
                                          std::to_string(max_level) + " levels");
    if (base != N) throw Error(VCSRMC_ERR_STATE, "rcm ordering left vertices unvisited");

    // 5. order
    {
        RLAUNCH(k_order_keys, N, comp.p, rank.p, seq.p, N, nb, k1.p, v1.p);
        u64 *ka = k1.p, *kb = k2.p;
        uint32_t *va = v1.p, *vb = v2.p;
        radix_sort_pairs<u64>(ka, va, kb, vb, N, 2 * nb, st);
        RLAUNCH(k_positions, N, va, N, position);
    }
    VCSRMC_HIP(hipStreamSynchronize(st));
}

void apply_column_permutation_device(const int* rp, int* col, float* val, int M, int N, int nnz,
                                     const int* position, const float* B, int O, float* B_out,
                                     hipStream_t st) {
    if (M < 0 || N < 0 || nnz < 0 || O < 0) throw Error(VCSRMC_ERR_ARG, "negative size");
    if (!rp || (nnz > 0 && (!col || !val)) || (N > 0 && !position))
        throw Error(VCSRMC_ERR_ARG, "null pointer");
    if ((B == nullptr) != (B_out == nullptr))
        throw Error(VCSRMC_ERR_ARG, "B and B_out must both be given or both be NULL");
    if (B && B == B_out) throw Error(VCSRMC_ERR_ARG, "B_out must not alias B");
    DevBuf<int> err(1);
    check_csr(rp, col, M, N, nnz, err.p, st);
    if (N > 0) {
        DevBuf<int> seen(N);
        VCSRMC_HIP(hipMemsetAsync(seen.p, 0, sizeof(int) * (size_t)N, st));
        RLAUNCH(k_perm_check, N, position, N, seen.p, err.p);
        raise_if(err.p, st);
    }
    if (nnz > 0) {
        const int nb = std::max(1, bits_for((u64)N));
        const int mb = std::max(1, bits_for((u64)M));
        DevBuf<int> row_of(nnz);
        row_of_nonzeros(rp, M, nnz, row_of.p, st);
        DevBuf<u64> k1(nnz), k2(nnz);
        DevBuf<uint32_t> v1(nnz), v2(nnz);
        RLAUNCH(k_relabel_keys, nnz, row_of.p, col, position, (long long)nnz, nb, k1.p, v1.p);
        row_of.release();
        u64 *ka = k1.p, *kb = k2.p;
        uint32_t *va = v1.p, *vb = v2.p;
        radix_sort_pairs<u64>(ka, va, kb, vb, nnz, nb + mb, st);
        RLAUNCH(k_relabel_dups, nnz, ka, (long long)nnz, err.p);
        raise_if(err.p, st);
        DevBuf<float> vcopy(nnz);
        VCSRMC_HIP(hipMemcpyAsync(vcopy.p, val, sizeof(float) * (size_t)nnz,
                                  hipMemcpyDeviceToDevice, st));
        RLAUNCH(k_relabel_write, nnz, ka, va, vcopy.p, (long long)nnz, nb, col, val);
    }
    if (B && N > 0 && O > 0)
        RLAUNCH(k_permute_rows, (long long)N * O, B, position, N, O, B_out);
    VCSRMC_HIP(hipStreamSynchronize(st));
}

}  // namespace vcsrmc
