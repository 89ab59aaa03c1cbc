// row_groups.hip -- a row order for the execution layout that puts rows sharing columns into the
// same 16-row panel.
//
// A panel's tiles are its distinct columns, 32 at a time, so a panel of rows that share columns
// has fewer tiles: fewer matrix-core steps, fewer B rows gathered, fuller tiles.  Natural order
// is often far from that: a 27-point stencil on a grid in natural order puts 16 consecutive x
// positions in a panel (a 16 x 1 x 1 strip, 162 distinct columns, 6 tiles), where a 4 x 2 x 2
// block of the same rows touches 96 (3 tiles).
//
// Method: multilevel heavy-edge matching on the row-column incidence.  Level k pairs clusters of
// up to 2^k rows, so four levels give groups of up to 16.  At each level every cluster scores
// the clusters it shares columns with (columns of more than `hub` rows are ignored: they link
// rows without telling them apart), keeps its best few, and clusters whose first choices are
// each other merge; a few rounds let clusters whose partner was taken try their next choice.
// The score is the number of shared columns; ties go to the pair whose first rows r < s satisfy
// floor(r / (s - r)) even, then to the nearer pair (the farther at the last level), then to a
// hash of the pair.  The parity rule makes chains of equally good partners pair up in phase
// (rows 0-1, 2-3, ... rather than a pairing that shifts from one chain to the next), which is
// what lets the next level merge the pairs into compact blocks; the distance rule keeps pairs
// near in the original order, except at the last level, where the farther of equally good
// partners makes a panel span more of the slowest direction of the natural order (z of a 3D
// grid: 2 x 2 x 4 blocks of a 27-point stencil, not 4 x 2 x 2; the same 96 columns): the B
// rows of a z-plane, reused by the panels one plane away long after one XCD's L2 has dropped
// them, are then fetched by 1.5 slabs of panels instead of 2.  Measured on gfx950 (kernel us,
// C += A.B / C = A.B): 27-point 100^3 FP32 444 / 347 -> 424 / 343, FP16 306 / 233 -> 308 /
// 225; 7-point 100^3 FP32 367 / 254 -> 354 / 253, FP16 268 / 194 -> 272 / 185; 7-point 60^3
// FP32 65.7 / 53.6 -> 60.7 / 48.1, FP16 48.3 / 29.8 -> 45.9 / 31.5; 2D 5-point grids unchanged.
// Finally the rows are ordered by their group's first row (rows in a group by index); rows
// without nonzeros go last, so they fill no panel.
//
// Every loop is bounded (levels, rounds, probes, insertions per cluster: a cluster whose
// candidates overflow its table keeps the ones it counted first), and the sorts are stable.
#include <algorithm>
#include <climits>

#include "internal.hpp"
#include "primitives.hpp"

namespace vcsrmc {
namespace {

typedef unsigned long long u64;

constexpr int kLevels = 4;            // 2^4 = kPanelRows rows per group
constexpr int kRounds = 8;            // proposal rounds per level
constexpr int kCand = 4;              // candidates kept per cluster and level
constexpr int kTable = 1024;          // LDS hash table slots per wave (one cluster)
constexpr int kProbes = 64;           // linear probes per insertion
constexpr int kMaxCols = 512;         // clusters with more (non-hub) columns take no partner
constexpr int kInsertsPerLane = 256;  // candidate insertions per lane and cluster

inline unsigned grid256(long long n) { return grid_for(n, 256); }

__device__ __forceinline__ unsigned mix32(unsigned x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

// keys[i] = col << shift | row for every triple.
__global__ void k_col_major_keys(const int* __restrict__ trow, const int* __restrict__ tcol,
                                 long long n, int shift, u64* __restrict__ key) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) key[i] = ((u64)tcol[i] << shift) | (u64)trow[i];
}

// ptr[v] = the first index of sorted `keys` whose key >> shift is >= v, for v in [0, count].
__global__ void k_lower_bounds(const u64* __restrict__ keys, long long n, int shift, int count,
                               int* __restrict__ ptr) {
    const long long v = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (v > count) return;
    long long lo = 0, hi = n;
    while (lo < hi) {
        const long long mid = (lo + hi) >> 1;
        if ((long long)(keys[mid] >> shift) < v) lo = mid + 1;
        else hi = mid;
    }
    ptr[v] = (int)lo;
}

// Level-0 cluster-column keys (row << cbits | col) of the triples whose column is not a hub.
__global__ void k_keep_flags(const int* __restrict__ tcol, const int* __restrict__ cptr,
                             long long n, int hub, int* __restrict__ keep) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int c = tcol[i];
    keep[i] = (cptr[c + 1] - cptr[c]) <= hub;
}

__global__ void k_keep_keys(const int* __restrict__ trow, const int* __restrict__ tcol,
                            const int* __restrict__ keep, const int* __restrict__ at, long long n,
                            int cbits, u64* __restrict__ key) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n && keep[i]) key[at[i]] = ((u64)trow[i] << cbits) | (u64)tcol[i];
}

// Column-major copy of cluster-column keys: (cluster << cbits | col) -> (col << clbits | cluster).
__global__ void k_transpose_keys(const u64* __restrict__ in, long long n, int cbits, int clbits,
                                 u64* __restrict__ out) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const u64 k = in[i];
    out[i] = ((k & ((1ull << cbits) - 1)) << clbits) | (k >> cbits);
}

// One wave per cluster a: counts, in an LDS hash table, how many of a's columns each other
// cluster b holds, then keeps the kCand best b with size(a) + size(b) <= maxsz (see the file
// comment for the order).  cand[a * kCand + i] = b, or -1.
__global__ __launch_bounds__(256) void k_score(const u64* __restrict__ crk,
                                               const int* __restrict__ cr_ptr,
                                               const u64* __restrict__ rck,
                                               const int* __restrict__ rc_ptr, int cbits,
                                               int clbits, const int* __restrict__ size,
                                               const int* __restrict__ cmin, int nc, int maxsz,
                                               bool far, int* __restrict__ cand) {
    __shared__ int tkey[4][kTable];
    __shared__ int tcnt[4][kTable];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const long long a = (long long)blockIdx.x * 4 + w;
    if (a >= nc) return;  // the whole wave
    int* K = tkey[w];
    int* Cn = tcnt[w];
    for (int i = lane; i < kTable; i += 64) {
        K[i] = -1;
        Cn[i] = 0;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int b0 = cr_ptr[a], b1 = cr_ptr[a + 1];
    const int sa = size[a];
    const bool active = (b1 - b0) <= kMaxCols && sa < maxsz;
    const u64 cmask = (1ull << cbits) - 1, lmask = (1ull << clbits) - 1;
    if (active) {
        int inserted = 0;
        for (int ci = b0 + lane; ci < b1 && inserted < kInsertsPerLane; ci += 64) {
            const int c = (int)(crk[ci] & cmask);
            const int r1 = rc_ptr[c + 1];
            for (int j = rc_ptr[c]; j < r1 && inserted < kInsertsPerLane; ++j) {
                const int b = (int)(rck[j] & lmask);
                if (b == (int)a) continue;
                ++inserted;
                unsigned h = mix32((unsigned)b) & (kTable - 1);
                for (int p = 0; p < kProbes; ++p) {
                    const int prev = atomicCAS(&K[h], -1, b);
                    if (prev == -1 || prev == b) {
                        atomicAdd(&Cn[h], 1);
                        break;
                    }
                    h = (h + 1) & (kTable - 1);
                }
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // Score keys of this lane's slots: shared columns, phase, nearness, hash.
    u64 score[kTable / 64];
    const int ma = cmin[a];
#pragma unroll
    for (int s = 0; s < kTable / 64; ++s) {
        const int slot = lane + 64 * s;
        const int b = K[slot];
        u64 key = 0;
        if (active && b >= 0 && sa + size[b] <= maxsz) {
            const int mb = cmin[b];
            const int lo = min(ma, mb), d = max(ma, mb) - lo;  // d >= 1: distinct first rows
            const u64 cnt = (u64)min(Cn[slot], 8191);
            const u64 phase = ((lo / d) & 1) == 0;
            const u64 near = far ? (u64)d : (u64)(0x7fffffff - d);
            const u64 tie = mix32((unsigned)min((int)a, b) * 0x9e3779b9u ^ (unsigned)max((int)a, b)) &
                            0x3ffffu;
            key = (cnt << 50) | (phase << 49) | (near << 18) | tie;
        }
        score[s] = key;
    }
    // kCand rounds of a wave-wide maximum; the winner's lane clears that slot.
    for (int r = 0; r < kCand; ++r) {
        u64 m = 0;
        int ms = -1;
#pragma unroll
        for (int s = 0; s < kTable / 64; ++s)
            if (score[s] > m) {
                m = score[s];
                ms = s;
            }
        u64 best = m;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const unsigned lo = __shfl_xor((unsigned)(best & 0xffffffffu), off);
            const unsigned hi = __shfl_xor((unsigned)(best >> 32), off);
            const u64 o = ((u64)hi << 32) | lo;
            best = o > best ? o : best;
        }
        int b = -1;
        if (best != 0 && m == best && ms >= 0) {
            // a lane holding the maximum; keys of two candidates tie only if their nearness,
            // phase and 18-bit pair hash all agree, and then the lowest lane's candidate is kept
            // and the other dropped
            b = K[lane + 64 * ms];
#pragma unroll
            for (int s = 0; s < kTable / 64; ++s)
                if (s == ms) score[s] = 0;
        }
        const unsigned long long own = __ballot(b >= 0);
        int chosen = -1;
        if (own) chosen = __shfl(b, (int)__builtin_ctzll(own));
        if (lane == 0) cand[a * kCand + r] = chosen;
    }
}

// A cluster still unmatched proposes to its first candidate that is unmatched too.
__global__ void k_propose(const int* __restrict__ cand, const int* __restrict__ mate, int nc,
                          int* __restrict__ prop) {
    const long long a = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (a >= nc) return;
    int p = -1;
    if (mate[a] < 0) {
        for (int i = 0; i < kCand; ++i) {
            const int b = cand[a * kCand + i];
            if (b >= 0 && mate[b] < 0) {
                p = b;
                break;
            }
        }
    }
    prop[a] = p;
}

// Mutual proposals match (each side records its own partner).
__global__ void k_accept(const int* __restrict__ prop, int nc, int* __restrict__ mate) {
    const long long a = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (a >= nc) return;
    const int b = prop[a];
    if (b >= 0 && prop[b] == (int)a) mate[a] = b;
}

// The merged cluster keeps the id rank of its smaller member.
__global__ void k_rep_flags(const int* __restrict__ mate, int nc, int* __restrict__ isrep) {
    const long long a = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (a < nc) isrep[a] = mate[a] < 0 || (int)a < mate[a];
}

__global__ void k_relabel(const int* __restrict__ mate, const int* __restrict__ nid,
                          const int* __restrict__ size, const int* __restrict__ cmin, int nc,
                          int* __restrict__ newcl, int* __restrict__ nsize,
                          int* __restrict__ ncmin) {
    const long long a = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (a >= nc) return;
    const int m = mate[a];
    const int rep = (m >= 0 && m < (int)a) ? m : (int)a;
    newcl[a] = nid[rep];
    if (rep == (int)a) {
        nsize[nid[a]] = size[a] + (m >= 0 ? size[m] : 0);
        ncmin[nid[a]] = m >= 0 ? min(cmin[a], cmin[m]) : cmin[a];
    }
}

__global__ void k_relabel_rows(const int* __restrict__ newcl, int M, int* __restrict__ rowcl) {
    const long long r = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (r < M) rowcl[r] = newcl[rowcl[r]];
}

__global__ void k_relabel_keys(const u64* __restrict__ in, long long n, int cbits,
                               const int* __restrict__ newcl, u64* __restrict__ out) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const u64 k = in[i];
    out[i] = ((u64)newcl[k >> cbits] << cbits) | (k & ((1ull << cbits) - 1));
}

__global__ void k_head_flags(const u64* __restrict__ k, long long n, int* __restrict__ head) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) head[i] = (i == 0) || k[i] != k[i - 1];
}

__global__ void k_compact_keys(const u64* __restrict__ in, const int* __restrict__ head,
                               const int* __restrict__ at, long long n, u64* __restrict__ out) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n && head[i]) out[at[i]] = in[i];
}

__global__ void k_init_clusters(int M, int* __restrict__ rowcl, int* __restrict__ size,
                                int* __restrict__ cmin) {
    const long long r = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= M) return;
    rowcl[r] = (int)r;
    size[r] = 1;
    cmin[r] = (int)r;
}

__global__ void k_has_nonzero(const int* __restrict__ trow, long long n,
                              unsigned char* __restrict__ has) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) has[trow[i]] = 1;
}

// Order key of row r: its group's first row (rows without nonzeros last), then r.
__global__ void k_order_keys(const int* __restrict__ rowcl, const int* __restrict__ cmin,
                             const unsigned char* __restrict__ has, int M, u64* __restrict__ key,
                             uint32_t* __restrict__ pay) {
    const long long r = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= M) return;
    const u64 first = has[r] ? (u64)cmin[rowcl[r]] : (u64)INT_MAX;
    key[r] = (first << 32) | (u64)r;
    pay[r] = (uint32_t)r;
}

__global__ void k_positions(const uint32_t* __restrict__ order, int M, int P,
                            int* __restrict__ rowpos, int* __restrict__ row_map) {
    const long long p = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= P) return;
    if (p < M) {
        const int r = (int)order[p];
        row_map[p] = r;
        rowpos[r] = (int)p;
    } else {
        row_map[p] = -1;
    }
}

void sort_keys(DevBuf<u64>& keys, DevBuf<u64>& alt, DevBuf<uint32_t>& pay,
               DevBuf<uint32_t>& pay_alt, long long n, int bits, hipStream_t st) {
    u64 *k = keys.p, *ka = alt.p;
    uint32_t *v = pay.p, *va = pay_alt.p;
    radix_sort_pairs<u64>(k, v, ka, va, n, bits, st);
    if (k != keys.p) {  // an odd number of passes: the result is in the alternate buffers
        std::swap(keys, alt);
        std::swap(pay, pay_alt);
    }
}

__global__ void k_flag_rows(const int* __restrict__ trow, long long n, int* __restrict__ flag) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) flag[trow[i]] = 1;
}

// Rows with nonzeros keep their order at positions 0..NE-1, the others follow in order.
__global__ void k_compact_positions(const int* __restrict__ flag, const int* __restrict__ rank,
                                    int M, int NE, int* __restrict__ rowpos,
                                    int* __restrict__ row_map) {
    const long long r = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= M) return;
    const int p = flag[r] ? rank[r] : NE + ((int)r - rank[r]);
    rowpos[r] = p;
    row_map[p] = (int)r;
}

}  // namespace

bool compact_rows(const int* trow, long long n, int M, hipStream_t st, DevBuf<int>& rowpos,
                  DevBuf<int>& row_map) {
    if (M < 1 || n < 1) return false;
    DevBuf<int> flag(M), rank((size_t)M + 1);
    fill<int>(flag.p, M, 0, st);
    hipLaunchKernelGGL(k_flag_rows, dim3(grid256(n)), dim3(256), 0, st, trow, n, flag.p);
    VCSRMC_HIP(hipGetLastError());
    exclusive_sum<int, int>(flag.p, rank.p, M, st);
    const int NE = read_scalar(rank.p + M, st);
    if (8LL * (M - NE) < M) return false;
    const int P = ((M + kPanelRows - 1) / kPanelRows) * kPanelRows;
    rowpos.alloc(M);
    row_map.alloc(P);
    fill<int>(row_map.p, P, -1, st);
    hipLaunchKernelGGL(k_compact_positions, dim3(grid256(M)), dim3(256), 0, st, flag.p, rank.p, M,
                       NE, rowpos.p, row_map.p);
    VCSRMC_HIP(hipGetLastError());
    return true;
}

bool group_rows(const int* trow, const int* tcol, long long n, int M, int N, hipStream_t st,
                DevBuf<int>& rowpos, DevBuf<int>& row_map) {
    if (M < 2 * kPanelRows || N < 1 || n < 1) return false;
    const int rbits = bits_for((unsigned long long)(M - 1));
    const int cbits = bits_for((unsigned long long)(N - 1));
    const int hub = (int)std::max<long long>(32, std::min<long long>(1024, 4 * n / N));

    // Column degrees from the column-major order of the triples.
    DevBuf<u64> keys(n), alt(n);
    DevBuf<uint32_t> pay(n), pay_alt(n);
    DevBuf<int> cptr((size_t)N + 1);
    hipLaunchKernelGGL(k_col_major_keys, dim3(grid256(n)), dim3(256), 0, st, trow, tcol, n, rbits,
                       keys.p);
    VCSRMC_HIP(hipGetLastError());
    sort_keys(keys, alt, pay, pay_alt, n, cbits + rbits, st);
    hipLaunchKernelGGL(k_lower_bounds, dim3(grid256((long long)N + 1)), dim3(256), 0, st, keys.p,
                       n, rbits, N, cptr.p);
    VCSRMC_HIP(hipGetLastError());

    // Level-0 cluster-column keys: the triples on columns of at most `hub` rows.
    long long np;
    {
        DevBuf<int> keep(n), at((size_t)n + 1);
        hipLaunchKernelGGL(k_keep_flags, dim3(grid256(n)), dim3(256), 0, st, tcol, cptr.p, n, hub,
                           keep.p);
        VCSRMC_HIP(hipGetLastError());
        exclusive_sum<int, int>(keep.p, at.p, n, st);
        np = read_scalar(at.p + n, st);
        hipLaunchKernelGGL(k_keep_keys, dim3(grid256(n)), dim3(256), 0, st, trow, tcol, keep.p,
                           at.p, n, cbits, keys.p);
        VCSRMC_HIP(hipGetLastError());
    }
    if (np == 0) return false;
    sort_keys(keys, alt, pay, pay_alt, np, rbits + cbits, st);

    int nc = M;
    DevBuf<int> rowcl(M), size(M), cmin(M);
    hipLaunchKernelGGL(k_init_clusters, dim3(grid256(M)), dim3(256), 0, st, M, rowcl.p, size.p,
                       cmin.p);
    VCSRMC_HIP(hipGetLastError());
    DevBuf<u64> rck(np), rca(np);
    for (int level = 0; level < kLevels; ++level) {
        const int clbits = bits_for((unsigned long long)(nc - 1));
        // cluster -> columns (keys, sorted) and column -> clusters
        DevBuf<int> cr_ptr((size_t)nc + 1), rc_ptr((size_t)N + 1);
        hipLaunchKernelGGL(k_lower_bounds, dim3(grid256((long long)nc + 1)), dim3(256), 0, st,
                           keys.p, np, cbits, nc, cr_ptr.p);
        VCSRMC_HIP(hipGetLastError());
        hipLaunchKernelGGL(k_transpose_keys, dim3(grid256(np)), dim3(256), 0, st, keys.p, np,
                           cbits, clbits, rck.p);
        VCSRMC_HIP(hipGetLastError());
        {
            u64 *k = rck.p, *ka = rca.p;
            uint32_t *v = pay.p, *va = pay_alt.p;
            radix_sort_pairs<u64>(k, v, ka, va, np, cbits + clbits, st);
            if (k != rck.p) std::swap(rck, rca);
        }
        hipLaunchKernelGGL(k_lower_bounds, dim3(grid256((long long)N + 1)), dim3(256), 0, st,
                           rck.p, np, clbits, N, rc_ptr.p);
        VCSRMC_HIP(hipGetLastError());

        const int maxsz = 2 << level;  // clusters of 2^level rows pair into 2^(level+1)
        DevBuf<int> cand((size_t)nc * kCand), mate(nc), prop(nc);
        hipLaunchKernelGGL(k_score, dim3(grid_for(nc, 4)), dim3(256), 0, st, keys.p, cr_ptr.p,
                           rck.p, rc_ptr.p, cbits, clbits, size.p, cmin.p, nc, maxsz,
                           level == kLevels - 1, cand.p);
        VCSRMC_HIP(hipGetLastError());
        fill<int>(mate.p, nc, -1, st);
        for (int round = 0; round < kRounds; ++round) {
            hipLaunchKernelGGL(k_propose, dim3(grid256(nc)), dim3(256), 0, st, cand.p, mate.p, nc,
                               prop.p);
            VCSRMC_HIP(hipGetLastError());
            hipLaunchKernelGGL(k_accept, dim3(grid256(nc)), dim3(256), 0, st, prop.p, nc, mate.p);
            VCSRMC_HIP(hipGetLastError());
        }
        DevBuf<int> isrep(nc), nid((size_t)nc + 1);
        hipLaunchKernelGGL(k_rep_flags, dim3(grid256(nc)), dim3(256), 0, st, mate.p, nc, isrep.p);
        VCSRMC_HIP(hipGetLastError());
        exclusive_sum<int, int>(isrep.p, nid.p, nc, st);
        const int nnc = read_scalar(nid.p + nc, st);
        if (nnc == nc) break;  // nothing merged at this level: none will at the next
        DevBuf<int> newcl(nc), nsize(nnc), ncmin(nnc);
        hipLaunchKernelGGL(k_relabel, dim3(grid256(nc)), dim3(256), 0, st, mate.p, nid.p, size.p,
                           cmin.p, nc, newcl.p, nsize.p, ncmin.p);
        VCSRMC_HIP(hipGetLastError());
        hipLaunchKernelGGL(k_relabel_rows, dim3(grid256(M)), dim3(256), 0, st, newcl.p, M,
                           rowcl.p);
        VCSRMC_HIP(hipGetLastError());
        size = std::move(nsize);
        cmin = std::move(ncmin);
        // the merged clusters' column sets: relabel, sort, drop repeats
        hipLaunchKernelGGL(k_relabel_keys, dim3(grid256(np)), dim3(256), 0, st, keys.p, np, cbits,
                           newcl.p, alt.p);
        VCSRMC_HIP(hipGetLastError());
        std::swap(keys, alt);
        const int nclbits = bits_for((unsigned long long)(nnc - 1));
        sort_keys(keys, alt, pay, pay_alt, np, nclbits + cbits, st);
        {
            DevBuf<int> head(np), at((size_t)np + 1);
            hipLaunchKernelGGL(k_head_flags, dim3(grid256(np)), dim3(256), 0, st, keys.p, np,
                               head.p);
            VCSRMC_HIP(hipGetLastError());
            exclusive_sum<int, int>(head.p, at.p, np, st);
            const long long nu = read_scalar(at.p + np, st);
            hipLaunchKernelGGL(k_compact_keys, dim3(grid256(np)), dim3(256), 0, st, keys.p, head.p,
                               at.p, np, alt.p);
            VCSRMC_HIP(hipGetLastError());
            std::swap(keys, alt);
            np = nu;
        }
        nc = nnc;
    }

    // Rows by group (first row of the group), rows without nonzeros last.
    const int P = ((M + kPanelRows - 1) / kPanelRows) * kPanelRows;
    DevBuf<unsigned char> has(M);
    fill<unsigned char>(has.p, M, 0, st);
    hipLaunchKernelGGL(k_has_nonzero, dim3(grid256(n)), dim3(256), 0, st, trow, n, has.p);
    VCSRMC_HIP(hipGetLastError());
    DevBuf<u64> okey(M), oalt(M);
    DevBuf<uint32_t> opay(M), opalt(M);
    hipLaunchKernelGGL(k_order_keys, dim3(grid256(M)), dim3(256), 0, st, rowcl.p, cmin.p, has.p,
                       M, okey.p, opay.p);
    VCSRMC_HIP(hipGetLastError());
    sort_keys(okey, oalt, opay, opalt, M, 64, st);
    rowpos.alloc(M);
    row_map.alloc(P);
    hipLaunchKernelGGL(k_positions, dim3(grid256(P)), dim3(256), 0, st, opay.p, M, P, rowpos.p,
                       row_map.p);
    VCSRMC_HIP(hipGetLastError());
    return true;
}

}  // namespace vcsrmc
