// format_build.hip -- the VCSR-MC format built on the GPU.
//
// Part 1 reproduces csr_to_vcsr_mc (MuuSeoTia/VCSR_MC src/vcsr_mc.cu:25-123) as a pipeline
// of scans, one stable radix sort and scatters:
//   1. validate row_ptr, expand the row id of every nonzero (max-scan of row heads)
//   2. flag the first nonzero of every (segment, row) run; exclusive scan -> pair index
//   3. pair keys (segment << 6 | segw - count); a stable radix sort orders each segment's
//      rows by count, descending, ties by ascending row (the reference's order of equal
//      counts is std::unordered_map iteration order, :59-66; here it is fixed)
//   4. bundles of 16 -> groups: depth, seg_base, rows; group_ptr = scan of 16*depth
//   5. depth-major, lane-minor scatter of lcol / val * (1/scale), padded with -1 / 0
//   6. work items: runs of <= chunk groups of one segment, stable sort by work, descending
// Part 2 derives the execution layout read by the multiply kernels (16-row panels cut into
// compacted 32-column tiles; see internal.hpp) from the same nonzeros.
#include <algorithm>
#include <atomic>
#include <climits>
#include <cmath>
#include <cstring>
#include <vector>

#include "../../include/vcsrmc.h"
#include "internal.hpp"

namespace vcsrmc {

// ------------------------------------------------------------------------------------------
// FP16 range scale.
// ------------------------------------------------------------------------------------------
float half_scale_from_amax(float amax) {
    // src/vcsr_mc.cu:14-22.  The reference binary is compiled with -ffast-math
    // (CMakeLists.txt:24-27), which evaluates `amax / 60000.0f` as amax * fl(1/60000); that
    // is reproduced here so the scale (and every val * (1/scale)) matches it bit for bit.
    const float headroom = 60000.0f;
    const float min_normal = 6.103515625e-05f;
    volatile float one = 1.0f;
    const float inv_headroom = one / headroom;
    if (amax > headroom) return amax * inv_headroom;
    if (amax > 0.0f && amax < min_normal) return amax * inv_headroom;
    return 1.0f;
}

__global__ __launch_bounds__(256) void k_absmax_bits(const float* __restrict__ v, long long n,
                                                     unsigned* __restrict__ out) {
    __shared__ int wsum[4];
    int m = 0;  // bit pattern of the largest finite-or-inf |v| seen (NaN skipped)
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x) {
        const unsigned b = __float_as_uint(v[i]) & 0x7fffffffu;
        if (b <= 0x7f800000u && (int)b > m) m = (int)b;
    }
    int total;
    block_scan_256(m, OpMax{}, 0, wsum, total);
    if (threadIdx.x == 0 && total > 0) atomicMax(out, (unsigned)total);
}

float device_absmax(const float* d_val, long long n, hipStream_t st) {
    DevBuf<unsigned> bits(1);
    VCSRMC_HIP(hipMemsetAsync(bits.p, 0, sizeof(unsigned), st));
    if (n > 0) {
        const unsigned grid = (unsigned)std::min<long long>(grid_for(n, 256), 4096);
        hipLaunchKernelGGL(k_absmax_bits, dim3(grid), dim3(256), 0, st, d_val, n, bits.p);
        VCSRMC_HIP(hipGetLastError());
    }
    const unsigned b = read_scalar(bits.p, st);
    float a;
    std::memcpy(&a, &b, sizeof a);
    return a;
}

// ------------------------------------------------------------------------------------------
// Part 1 kernels.
// ------------------------------------------------------------------------------------------
enum : int { kErrCsr = 1, kErrRange = 2, kErrUnsorted = 4, kErrFormat = 8, kErrDuplicate = 16 };

__global__ void k_check_row_ptr(const int* __restrict__ rp, int M, int nnz, int* __restrict__ err) {
    const long long r = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (r > M) return;
    const int a = rp[r];
    bool bad = a < 0 || a > nnz;
    if (r == 0) bad |= a != 0;
    if (r == M) bad |= a != nnz;
    if (r < M) bad |= rp[r + 1] < a;
    if (bad) atomicOr(err, kErrCsr);
}

__global__ void k_mark_row_heads(const int* __restrict__ rp, int M, int* __restrict__ head) {
    const long long r = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= M) return;
    const int a = rp[r];
    if (a < rp[r + 1]) head[a] = (int)r;
}

// Per nonzero: range / order checks and the (segment, row) run heads.
__global__ void k_pair_heads(const int* __restrict__ rp, const int* __restrict__ col,
                             const int* __restrict__ row_of, int nnz, int N, int segw,
                             int* __restrict__ head, int* __restrict__ err) {
    const long long p = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= nnz) return;
    const int r = row_of[p];
    const int c = col[p];
    int e = 0;
    if (c < 0 || c >= N) e |= kErrRange;
    const bool first = p == rp[r];
    int h = 1;
    if (!first) {
        const int prev = col[p - 1];
        if (prev >= c) e |= kErrUnsorted;
        h = (c / segw) != (prev / segw);
    }
    head[p] = h;
    if (e) atomicOr(err, e);
}

__global__ void k_emit_pairs(const int* __restrict__ head, const int* __restrict__ pidx,
                             const int* __restrict__ row_of, int nnz, int* __restrict__ pstart,
                             int* __restrict__ prow) {
    const long long p = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= nnz) return;
    if (head[p]) {
        const int q = pidx[p];
        pstart[q] = (int)p;
        prow[q] = row_of[p];
    }
}

template <typename K>
__global__ void k_pair_keys(const int* __restrict__ pstart, const int* __restrict__ col, int P,
                            int segw, K* __restrict__ key, uint32_t* __restrict__ pay) {
    const long long q = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= P) return;
    const int cnt = pstart[q + 1] - pstart[q];
    const int seg = col[pstart[q]] / segw;
    key[q] = ((K)seg << 6) | (K)(segw - cnt);
    pay[q] = (uint32_t)q;
}

// seg_start[s] = first sorted pair of segment s or later (s = 0..S; seg_start[S] = P): a lower
// bound over the sorted keys, one thread per segment.
template <typename K>
__global__ void k_seg_starts(const K* __restrict__ skey, int P, int S,
                             int* __restrict__ seg_start) {
    const long long s = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (s > S) return;
    const K want = (K)s << 6;
    int lo = 0, hi = P;
    while (lo < hi) {
        const int mid = (int)(((unsigned)lo + (unsigned)hi) >> 1);
        if (skey[mid] < want) lo = mid + 1;
        else hi = mid;
    }
    seg_start[s] = lo;
}

__global__ void k_groups_per_seg(const int* __restrict__ seg_start, int S,
                                 int* __restrict__ gnum) {
    const long long s = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (s < S) gnum[s] = (seg_start[s + 1] - seg_start[s] + 15) / 16;
}

template <typename K>
__global__ void k_group_heads(const K* __restrict__ skey, const int* __restrict__ seg_start,
                              const int* __restrict__ gbase, int P, int* __restrict__ ghead) {
    const long long s = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= P) return;
    const int seg = (int)(skey[s] >> 6);
    const int j = (int)s - seg_start[seg];
    if ((j & 15) == 0) ghead[gbase[seg] + (j >> 4)] = (int)s;
}

template <typename K>
__global__ void k_group_info(const K* __restrict__ skey, const uint32_t* __restrict__ spay,
                             const int* __restrict__ ghead, const int* __restrict__ seg_start,
                             const int* __restrict__ pstart, const int* __restrict__ prow, int G,
                             int segw, int* __restrict__ depth, int* __restrict__ seg_base,
                             int* __restrict__ rows, int* __restrict__ size16) {
    const long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= G) return;
    const int s = ghead[g];
    const int seg = (int)(skey[s] >> 6);
    const int end = seg_start[seg + 1];
    const uint32_t q = spay[s];
    const int d = pstart[q + 1] - pstart[q];
    depth[g] = d;
    seg_base[g] = seg * segw;
    size16[g] = 16 * d;
#pragma unroll
    for (int lane = 0; lane < 16; ++lane)
        rows[16 * g + lane] = (s + lane < end) ? prow[spay[s + lane]] : -1;
}

__global__ void k_to_int(const long long* __restrict__ a, int* __restrict__ b, long long n) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) b[i] = (int)a[i];
}

// One wave per group: 16 lanes per depth level, four levels per step.
template <typename K>
__global__ __launch_bounds__(256) void k_fill_group_entries(
    const K* __restrict__ skey, const uint32_t* __restrict__ spay, const int* __restrict__ ghead,
    const int* __restrict__ seg_start, const int* __restrict__ pstart,
    const int* __restrict__ group_ptr, const int* __restrict__ depth,
    const int* __restrict__ seg_base, const int* __restrict__ col, const float* __restrict__ v,
    int G, float inv_scale, int* __restrict__ lcol, float* __restrict__ val) {
    const long long g = ((long long)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (g >= G) return;
    const int lane = threadIdx.x & 63, l16 = lane & 15, dsub = lane >> 4;
    const int s = ghead[g];
    const int seg = (int)(skey[s] >> 6);
    const int end = seg_start[seg + 1];
    int cnt = 0, p0 = 0;
    if (s + l16 < end) {
        const uint32_t q = spay[s + l16];
        p0 = pstart[q];
        cnt = pstart[q + 1] - p0;
    }
    const int gp = group_ptr[g], dep = depth[g], base = seg_base[g];
    for (int d = dsub; d < dep; d += 4) {
        const long long idx = (long long)gp + (long long)d * 16 + l16;
        if (d < cnt) {
            lcol[idx] = col[p0 + d] - base;
            val[idx] = v[p0 + d] * inv_scale;
        } else {
            lcol[idx] = -1;
            val[idx] = 0.0f;
        }
    }
}

__global__ void k_items_per_seg(const int* __restrict__ gnum, int S, int chunk,
                                int* __restrict__ inum) {
    const long long s = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (s < S) inum[s] = (gnum[s] + chunk - 1) / chunk;
}

__global__ void k_make_items(const int* __restrict__ gbase, const int* __restrict__ ibase,
                             const int* __restrict__ group_ptr, int S, int chunk, int wmax,
                             int* __restrict__ ib, int* __restrict__ ie, uint32_t* __restrict__ ikey,
                             uint32_t* __restrict__ ipay) {
    const long long s = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= S) return;
    const int g0 = gbase[s], g1 = gbase[s + 1];
    int i = ibase[s];
    for (int gb = g0; gb < g1; gb += chunk, ++i) {
        const int ge = min(gb + chunk, g1);
        ib[i] = gb;
        ie[i] = ge;
        ikey[i] = (uint32_t)(wmax - (group_ptr[ge] - group_ptr[gb]));
        ipay[i] = (uint32_t)i;
    }
}

__global__ void k_gather_items(const uint32_t* __restrict__ spay, const int* __restrict__ ib,
                               const int* __restrict__ ie, int I, int* __restrict__ gbeg,
                               int* __restrict__ gend) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= I) return;
    gbeg[i] = ib[spay[i]];
    gend[i] = ie[spay[i]];
}

__global__ void k_scale_values(const float* __restrict__ v, float* __restrict__ out, long long n,
                               float inv_scale) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = v[i] * inv_scale;
}

// ------------------------------------------------------------------------------------------
// Part 2: execution layout from triples (row, col, value already divided by the scale).
// ------------------------------------------------------------------------------------------
// Rows are placed at positions (rowpos[row], or the row itself in natural order); a panel is 16
// consecutive positions.
template <typename K>
__global__ void k_panel_keys(const int* __restrict__ trow, const int* __restrict__ tcol,
                             const int* __restrict__ rowpos, long long n, int cbits,
                             K* __restrict__ key, uint32_t* __restrict__ pay) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int r = rowpos ? rowpos[trow[i]] : trow[i];
    key[i] = ((K)(r >> 4) << (cbits + 4)) | ((K)tcol[i] << 4) | (K)(r & 15);
    pay[i] = (uint32_t)i;
}

template <typename K>
__global__ void k_panel_heads(const K* __restrict__ skey, long long n, int cbits,
                              int* __restrict__ hdist, int* __restrict__ hpanel,
                              int* __restrict__ err) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const K k = skey[i];
    int hd = 1, hp = 1;
    if (i > 0) {
        const K prev = skey[i - 1];
        if (prev == k) atomicOr(err, kErrDuplicate);
        hd = (prev >> 4) != (k >> 4);
        hp = (prev >> (cbits + 4)) != (k >> (cbits + 4));
    }
    hdist[i] = hd;
    hpanel[i] = hp;
}

template <typename K>
__global__ void k_panel_starts(const K* __restrict__ skey, const int* __restrict__ hpanel,
                               const int* __restrict__ pin, long long n, int cbits,
                               int* __restrict__ pstart, int* __restrict__ ppanel) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (hpanel[i]) {
        const int j = pin[i] - 1;
        pstart[j] = (int)i;
        ppanel[j] = (int)(skey[i] >> (cbits + 4));
    }
}

__global__ void k_panel_chunks(const int* __restrict__ pstart, const int* __restrict__ dc, int NP,
                               int* __restrict__ nch) {
    const long long j = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= NP) return;
    const int ndist = dc[pstart[j + 1] - 1] - dc[pstart[j]] + 1;
    nch[j] = (ndist + kChunkCols - 1) / kChunkCols;
}

template <typename K, bool FP32>
__global__ void k_panel_entries(const K* __restrict__ skey, const uint32_t* __restrict__ spay,
                                const int* __restrict__ hdist, const int* __restrict__ dc,
                                const int* __restrict__ pin, const int* __restrict__ pstart,
                                const int* __restrict__ cbase, const int* __restrict__ tcol,
                                const float* __restrict__ tval, long long n,
                                uint32_t* __restrict__ entries, int* __restrict__ chunk_cols,
                                int* __restrict__ chunk_eptr, int* __restrict__ echunk) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int j = pin[i] - 1;
    const int lr = dc[i] - dc[pstart[j]];
    const int c = cbase[j] + lr / kChunkCols;
    const int k = lr % kChunkCols;
    const int r16 = (int)(skey[i] & 15);
    const uint32_t src = spay[i];
    echunk[i] = c;
    const float v = tval[src];
    if constexpr (FP32) {
        entries[2 * i] = (uint32_t)r16 | ((uint32_t)k << 4);
        entries[2 * i + 1] = __float_as_uint(v);
    } else {
        const _Float16 h = (_Float16)v;  // v_cvt_f16_f32, round to nearest even
        entries[i] = (uint32_t)__builtin_bit_cast(unsigned short, h) | ((uint32_t)r16 << 16) |
                     ((uint32_t)k << 20);
    }
    if (hdist[i]) {
        // FP32 formats keep a tile's columns in K-step order: lane group g of the kernel reads
        // columns 4 s + g (s = 0..7) as eight consecutive words.
        const int slot = FP32 ? (k & 3) * 8 + (k >> 2) : k;
        chunk_cols[(long long)c * kChunkCols + slot] = tcol[src];
        if (k == 0) chunk_eptr[c] = (int)i;
    }
}

// rflag[p] = 1 for every position whose row holds a nonzero (plain stores; every writer stores
// the same 1).
__global__ void k_row_flags(const int* __restrict__ trow, const int* __restrict__ rowpos,
                            long long n, unsigned char* __restrict__ rflag) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) rflag[rowpos ? rowpos[trow[i]] : trow[i]] = 1;
}

// pmask[j] = the non-empty rows of panel j, from its 16 row flags (one 16-byte load).
__global__ void k_panel_masks(const unsigned char* __restrict__ rflag,
                              const int* __restrict__ ppanel, int NP, int* __restrict__ pmask) {
    const long long j = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= NP) return;
    const uint4 w = *reinterpret_cast<const uint4*>(rflag + (long long)ppanel[j] * kPanelRows);
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
    int m = 0;
#pragma unroll
    for (int b = 0; b < 16; ++b) m |= ((words[b >> 2] >> (8 * (b & 3))) & 1u) << b;
    pmask[j] = m;
}

__global__ void k_dense_flags(const int* __restrict__ eptr, int NC, int dmin,
                              int* __restrict__ flag) {
    const long long c = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (c < NC) flag[c] = (eptr[c + 1] - eptr[c]) > dmin;
}

// Tiles holding more than this many nonzeros get a dense copy.  Every tile of a small FP32
// format does (each tile holds at least one nonzero): measured on gfx950 at O = 128, FP32
// formats of at most 256 panels ran 2-9% faster with all tiles dense (uniform 2048^2 / 4096^2,
// power-law 4000^2, 27-point stencil 16^3, R-MAT scale 12), while larger uniform and stencil
// formats ran 2-13% slower (uniform 8192^2 to 30,000^2, stencil 20^3 to 30^3: the copies' bytes
// outweigh the LDS round trip once the GPU holds more waves than it runs at once), and FP16
// formats gained or lost a few percent either way.
static int dense_min(bool fp32, int num_panels, int num_chunks) {
    return (fp32 && num_panels <= kSmallPanels && num_chunks <= kSmallTiles) ? 0 : kDenseMin;
}

__global__ void k_dense_index(const int* __restrict__ flag, const int* __restrict__ idx, int NC,
                              int* __restrict__ chunk_dense) {
    const long long c = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (c < NC) chunk_dense[c] = flag[c] ? idx[c] : -1;
}

template <bool FP32>
__global__ void k_dense_fill(const uint32_t* __restrict__ entries,
                             const int* __restrict__ echunk, const int* __restrict__ chunk_dense,
                             long long n, _Float16* __restrict__ a16, float* __restrict__ a32) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int d = chunk_dense[echunk[i]];
    if (d < 0) return;
    if constexpr (FP32) {
        const uint32_t w = entries[2 * i];
        const int r = w & 15, k = (w >> 4) & 31;
        a32[(long long)d * 512 + (k & 3) * 128 + r * 8 + (k >> 2)] = __uint_as_float(entries[2 * i + 1]);
    } else {
        const uint32_t w = entries[i];
        const int r = (w >> 16) & 15, k = (w >> 20) & 31;
        a16[(long long)d * 512 + r * 32 + k] = __builtin_bit_cast(_Float16, (unsigned short)(w & 0xffffu));
    }
}

// Row steps of FP32 panels (the layout is described with DeviceFormat).  rsmask[4c + g] = the
// columns k of tile c that row group g (rows 4g .. 4g + 3) holds, as a 32-bit set, and
// rscnt[g * NC + c] = their number; one thread per tile.
__global__ void k_row_step_masks(const int* __restrict__ eptr, const uint32_t* __restrict__ entries,
                                 int NC, uint32_t* __restrict__ rsmask, int* __restrict__ rscnt) {
    const long long c = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= NC) return;
    uint32_t m[4] = {0u, 0u, 0u, 0u};
    for (int e = eptr[c]; e < eptr[c + 1]; ++e) {
        const uint32_t w = entries[2 * (long long)e];
        m[(w & 15) >> 2] |= 1u << ((w >> 4) & 31);
    }
    for (int g = 0; g < 4; ++g) {
        rsmask[4 * c + g] = m[g];
        rscnt[g * (long long)NC + c] = __popc(m[g]);
    }
}

// nbat[j] = panel j's batches of 8 row steps (its busiest row group's columns, from the
// exclusive sums rspre[g * (NC + 1) + c] of rscnt over the tiles, / 8 rounded up) where it takes
// row steps, else 0: always (`all`), or when they are at most num / den per tile.  One thread
// per panel.
__global__ void k_row_step_batches(const int* __restrict__ cbase, const int* __restrict__ rspre,
                                   int NP, int NC, bool all, int num, int den,
                                   int* __restrict__ nbat) {
    const long long j = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= NP) return;
    const int c0 = cbase[j], c1 = cbase[j + 1];
    int steps = 0;
    for (int g = 0; g < 4; ++g) {
        const int* pre = rspre + g * ((long long)NC + 1);
        steps = max(steps, pre[c1] - pre[c0]);
    }
    const int nb = (steps + 7) / 8;
    nbat[j] = (all || (long long)nb * den <= (long long)num * (c1 - c0)) ? nb : 0;
}

// Writes the row steps of the panels that take them: entry (row 4g + x, tile column k of tile
// c in panel j) becomes step s = (row group g's columns in the panel's tiles before it) of batch
// rbase[j] + s / 8.  The slots were set to column -1 and value 0 before.  One thread per tile;
// its panel is the last j with cbase[j] <= c.
__global__ void k_row_step_fill(const int* __restrict__ cbase, const int* __restrict__ rbase,
                                const int* __restrict__ nbat, const uint32_t* __restrict__ rsmask,
                                const int* __restrict__ rspre, const int* __restrict__ eptr,
                                const uint32_t* __restrict__ entries,
                                const int* __restrict__ chunk_cols, int NP, int NC,
                                int* __restrict__ rs_cols, float* __restrict__ rs_vals) {
    const long long c = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= NC) return;
    int lo = 0, hi = NP - 1;  // cbase[0] = 0 <= c
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (cbase[mid] <= c) lo = mid;
        else hi = mid - 1;
    }
    const int j = lo;
    if (nbat[j] == 0) return;
    const long long b0 = rbase[j];
    const int c0 = cbase[j];
    for (int e = eptr[c]; e < eptr[c + 1]; ++e) {
        const uint32_t w = entries[2 * (long long)e];
        const int r = w & 15, k = (w >> 4) & 31, g = r >> 2, x = r & 3;
        const int* pre = rspre + g * ((long long)NC + 1);
        const int s = pre[c] - pre[c0] + __popc(rsmask[4 * c + g] & ((1u << k) - 1u));
        const long long b = b0 + s / 8;
        const int t = s & 7;
        // FP32 tiles keep their columns in K-step order: column k at slot (k & 3) * 8 + k / 4
        rs_cols[32 * b + 8 * g + t] = chunk_cols[c * kChunkCols + (k & 3) * 8 + (k >> 2)];
        rs_vals[128 * b + 32 * g + 8 * x + t] = __uint_as_float(entries[2 * (long long)e + 1]);
    }
}

__global__ void k_pick_work(const int* __restrict__ nbat, int NP, int* __restrict__ nch) {
    const long long j = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (j < NP && nbat[j] > 0) nch[j] = nbat[j];
}

// Units.  A panel with at most `light_max` tiles is one light unit (one wave); a larger panel
// is cut into heavy units of at most `heavy_tiles` tiles (the waves of a work-group share them).
// nsplit[j] = 1 for a panel cut into several units.
__global__ void k_units_per_panel(const int* __restrict__ nch, int NP, int light_max,
                                  int heavy_tiles, int* __restrict__ nu, int* __restrict__ nheavy,
                                  int* __restrict__ nsplit) {
    const long long j = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= NP) return;
    const bool heavy = nch[j] > light_max;
    const int n = heavy ? (nch[j] + heavy_tiles - 1) / heavy_tiles : 1;
    nu[j] = n;
    nheavy[j] = heavy ? n : 0;
    nsplit[j] = n > 1;
}

// Writes the units of panel j (in panel order) with their schedule keys: heavy units first,
// larger first; then light units in panel order (the stable sort keeps it), so that the
// contiguous range of light units an XCD walks holds neighbouring panels -- or, with
// `by_column`, light units ordered by their panel's smallest column (ties in panel order), so
// that panels reading the same B rows run close together on one XCD (see light_by_column).
// The first unit of a split panel also carries kUnitSplitFirst (it clears the panel's rows before
// an overwriting launch, see spmm_launch).
// A panel's work items are its tiles cbase[j] .. cbase[j + 1], or, where nbat[j] > 0, its
// row-step batches rbase[j] .. rbase[j] + nbat[j] (units flagged kUnitRowSteps); `nch` counts
// them either way.
__global__ void k_make_units(const int* __restrict__ cbase, const int* __restrict__ rbase,
                             const int* __restrict__ nbat, const int* __restrict__ ubase,
                             const int* __restrict__ ppanel, const int* __restrict__ pmask,
                             const int* __restrict__ nch, int NP, int light_max, int heavy_tiles,
                             const int* __restrict__ chunk_cols, bool by_column,
                             int4* __restrict__ units, uint32_t* __restrict__ key,
                             uint32_t* __restrict__ pay) {
    const long long j = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= NP) return;
    const bool rows = nbat != nullptr && nbat[j] > 0;
    const int c0 = rows ? rbase[j] : cbase[j], c1 = c0 + nch[j];
    const int u0 = ubase[j], nu = ubase[j + 1] - u0;
    const bool heavy = nch[j] > light_max;
    const int split = nu > 1 ? kUnitSplit : 0;
    const int kind = rows ? kUnitRowSteps : 0;
    const int step = heavy ? heavy_tiles : (c1 - c0);
    for (int u = 0; u < nu; ++u) {
        const int cb = c0 + u * step;
        const int ce = min(cb + step, c1);
        const int first = (split && u == 0) ? kUnitSplitFirst : 0;
        units[u0 + u] =
            make_int4(ppanel[j] * kPanelRows, cb, ce, (pmask[j] & 0xffff) | split | first | kind);
        // a panel's tile columns ascend, so slot 0 of its first tile is its smallest column
        const uint32_t light =
            by_column ? 0x80000000u | (uint32_t)chunk_cols[(long long)cbase[j] * kChunkCols]
                      : 1u << 16;
        key[u0 + u] = heavy ? (uint32_t)(0xffff - min(ce - cb, 0xffff)) : light;
        pay[u0 + u] = (uint32_t)(u0 + u);
    }
}

__global__ void k_gather_units(const int4* __restrict__ in, const uint32_t* __restrict__ perm,
                               int NU, int4* __restrict__ out) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < NU) out[i] = in[perm[i]];
}

// Tiles of light unit i (units sorted: heavy first).
__global__ void k_light_tiles(const int4* __restrict__ units, int NH, int NL, int* __restrict__ nt) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < NL) nt[i] = units[NH + i].z - units[NH + i].y;
}

// xcd_start[x] = first light unit of XCD x: the cut where the running tile count reaches
// x / 8 of the total (lower bound in the inclusive prefix `csum`).
__global__ void k_xcd_cuts(const long long* __restrict__ csum, int NL, int* __restrict__ cut) {
    const int x = threadIdx.x;
    if (x > 8) return;
    if (x == 0) { cut[0] = 0; return; }
    if (x == 8) { cut[8] = NL; return; }
    const long long total = csum[NL];
    const long long target = total * x / 8;
    int lo = 0, hi = NL;  // first i with csum[i] >= target (csum[i] = tiles of units < i)
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (csum[mid] < target) lo = mid + 1;
        else hi = mid;
    }
    cut[x] = lo;
}

static inline unsigned blocks(long long n) { return grid_for(n, 256); }

#define LAUNCH(kernel, n, ...)                                                                 \
    do {                                                                                       \
        if ((n) > 0) {                                                                         \
            hipLaunchKernelGGL(kernel, dim3(blocks(n)), dim3(256), 0, st, __VA_ARGS__);        \
            VCSRMC_HIP(hipGetLastError());                                                     \
        }                                                                                      \
    } while (0)

static void check_err(const int* d_err, hipStream_t st) {
    const int e = read_scalar(d_err, st);
    if (e & kErrCsr) throw Error(VCSRMC_ERR_CSR, "row_ptr is not a monotone 0..nnz sequence");
    if (e & kErrRange) throw Error(VCSRMC_ERR_CSR, "column index out of range [0, N)");
    if (e & kErrUnsorted)
        throw Error(VCSRMC_ERR_UNSORTED,
                    "columns of a row are not strictly increasing (unsorted or duplicate "
                    "coordinates)");
    if (e & kErrFormat) throw Error(VCSRMC_ERR_FORMAT, "format arrays are inconsistent");
    if (e & kErrDuplicate)
        throw Error(VCSRMC_ERR_FORMAT, "format holds the same (row, column) twice");
}

// Panels of at most this many tiles are light units (one wave each, four per work-group);
// larger panels become heavy units that the four waves of a work-group share and merge in LDS.
// With fewer than 2048 panels one wave per panel leaves most of the 1024 SIMDs idle, so every
// multi-tile panel is shared by a work-group; otherwise panels of up to 5 tiles stay on one
// wave (measured on gfx950: 5 to 12 tiles are equally good for the uniform, stencil, 32 x 32
// block and R-MAT matrices, within 0.5%; on the 36,692-row power-law matrix 5 is 2% faster
// than 6, 7 or 8 accumulating and 4% faster overwriting, and 4 is 7% slower accumulating; 16
// leaves R-MAT with long single-wave units).
static int light_tile_limit(int num_panels) { return num_panels >= kFewPanels ? 5 : 1; }

// Largest heavy unit.  Heavy units run first, larger first, each on the four waves of one
// work-group, while the GPU holds about 3072 waves (1024 SIMDs, three waves each); a unit of
// up to 1/1024 of all tiles gives each of its waves at most 3/4 of the average wave's share, so
// it ends before the launch does.  Smaller launches keep units of kHeavyTiles, which split the
// few large panels of a short launch across work-groups.  Every cut makes the panel's units
// merge in C through atomics.
static int heavy_tile_limit(int num_chunks) {
    return std::max(kHeavyTiles, std::min(num_chunks / 1024, 0xffff));
}

// Order of the light units.  Panel order keeps an XCD on neighbouring rows of C and of the
// format's arrays.  Where the rows of a panel share most of their columns (at least 4 nonzeros
// per distinct (panel, column) pair: blocks of 4 rows or more; grids have 1.4-2.7, random and
// graph matrices 1.0-1.2), a B row serves many nonzeros and re-reading it from beyond L2 is
// what costs, so light units are ordered by their panel's smallest column instead: panels whose
// blocks start at the same column follow each other.  Measured on gfx950 (kernel us, C += A.B /
// C = A.B): 32 x 32 blocks, 8192 block rows, O = 256, FP16 179 / 140 -> 178 / 132, FP32 284 /
// 234 -> 271 / 220; 32 x 32 blocks, 1024 block rows, 16 x 16 and 8 x 8 blocks -2.3 to -7.4%
// (median of 10 single launches); 4 x 4 blocks within 1%.  Applied everywhere it costs
// uniform random matrices 1-4% (300,000^2 with 3 per row +2.6% / +4.0%) and power-law ones up
// to 2.5%, and leaves grids, stencils and R-MAT within 1%.
static bool light_by_column(long long nnz, long long num_pairs) { return nnz >= 4 * num_pairs; }

template <typename K>
static void build_exec_layout_k(DeviceFormat& F, const int* trow, const int* tcol,
                                const float* tval, const int* rowpos, long long n,
                                hipStream_t st) {
    const int num_panels_all = (F.M + kPanelRows - 1) / kPanelRows;
    const int cbits = bits_for(F.N > 0 ? (unsigned long long)(F.N - 1) : 0ull);
    const int pbits = bits_for(num_panels_all > 0 ? (unsigned long long)(num_panels_all - 1) : 0ull);
    const int kbits = pbits + cbits + 4;

    DevBuf<K> k1(n), k2(n);
    DevBuf<uint32_t> v1(n), v2(n);
    LAUNCH((k_panel_keys<K>), n, trow, tcol, rowpos, n, cbits, k1.p, v1.p);
    K* kp = k1.p; K* ka = k2.p;
    uint32_t* vp = v1.p; uint32_t* va = v2.p;
    radix_sort_pairs<K>(kp, vp, ka, va, n, kbits, st);

    DevBuf<int> hdist(n), hpanel(n), dc(n), pin(n), err(1);
    VCSRMC_HIP(hipMemsetAsync(err.p, 0, sizeof(int), st));
    LAUNCH((k_panel_heads<K>), n, kp, n, cbits, hdist.p, hpanel.p, err.p);
    inclusive_sum<int, int>(hdist.p, dc.p, n, st);
    inclusive_sum<int, int>(hpanel.p, pin.p, n, st);
    check_err(err.p, st);
    const int NP = read_scalar(pin.p + (n - 1), st);
    F.num_pairs = read_scalar(dc.p + (n - 1), st);

    DevBuf<int> pstart(NP + 1), ppanel(NP), nch(NP), cbase(NP + 1), pmask(NP);
    LAUNCH((k_panel_starts<K>), n, kp, hpanel.p, pin.p, n, cbits, pstart.p, ppanel.p);
    fill<int>(pstart.p + NP, 1, (int)n, st);
    LAUNCH(k_panel_chunks, NP, pstart.p, dc.p, NP, nch.p);
    exclusive_sum<int, int>(nch.p, cbase.p, NP, st);
    const int NC = read_scalar(cbase.p + NP, st);
    {
        DevBuf<int> nmax(NP);
        inclusive_max(nch.p, nmax.p, NP, st);
        F.max_panel_tiles = read_scalar(nmax.p + (NP - 1), st);
    }

    F.chunk_eptr.alloc(NC + 1);
    F.chunk_cols.alloc((size_t)NC * kChunkCols);
    F.entries.alloc(F.fp32 ? 2 * n : n);
    fill<int>(F.chunk_cols.p, (long long)NC * kChunkCols, -1, st);
    fill<int>(F.chunk_eptr.p + NC, 1, (int)n, st);
    {
        DevBuf<unsigned char> rflag((size_t)num_panels_all * kPanelRows);
        fill<unsigned char>(rflag.p, (long long)num_panels_all * kPanelRows, 0, st);
        LAUNCH(k_row_flags, n, trow, rowpos, n, rflag.p);
        LAUNCH(k_panel_masks, NP, rflag.p, ppanel.p, NP, pmask.p);
    }
    DevBuf<int> echunk(n);
    if (F.fp32)
        LAUNCH((k_panel_entries<K, true>), n, kp, vp, hdist.p, dc.p, pin.p, pstart.p, cbase.p, tcol,
               tval, n, F.entries.p, F.chunk_cols.p, F.chunk_eptr.p, echunk.p);
    else
        LAUNCH((k_panel_entries<K, false>), n, kp, vp, hdist.p, dc.p, pin.p, pstart.p, cbase.p,
               tcol, tval, n, F.entries.p, F.chunk_cols.p, F.chunk_eptr.p, echunk.p);

    // dense copies of well-filled tiles
    {
        DevBuf<int> dflag(NC), didx(NC + 1);
        LAUNCH(k_dense_flags, NC, F.chunk_eptr.p, NC, dense_min(F.fp32, NP, NC), dflag.p);
        exclusive_sum<int, int>(dflag.p, didx.p, NC, st);
        const int ND = read_scalar(didx.p + NC, st);
        F.chunk_dense.alloc(NC);
        LAUNCH(k_dense_index, NC, dflag.p, didx.p, NC, F.chunk_dense.p);
        F.num_dense = ND;
        if (ND > 0) {
            if (F.fp32) {
                F.dense_a32.alloc((size_t)ND * 512);
                VCSRMC_HIP(hipMemsetAsync(F.dense_a32.p, 0, sizeof(float) * 512 * (size_t)ND, st));
                LAUNCH((k_dense_fill<true>), n, F.entries.p, echunk.p, F.chunk_dense.p, n,
                       (_Float16*)nullptr, F.dense_a32.p);
            } else {
                F.dense_a16.alloc((size_t)ND * 512);
                VCSRMC_HIP(hipMemsetAsync(F.dense_a16.p, 0, sizeof(_Float16) * 512 * (size_t)ND, st));
                LAUNCH((k_dense_fill<false>), n, F.entries.p, echunk.p, F.chunk_dense.p, n,
                       F.dense_a16.p, (float*)nullptr);
            }
        }
    }

    // row steps of FP32 panels whose rows rarely share a column; their units count batches
    DevBuf<int> nbat, rbase;
    int NB = 0;
    // (in the default mode only in formats whose launches take O tiles of 64 anyway: the
    // multiply kernel carries the row-step path only at that width)
    int rs_mode = F.fp32 ? fp32_row_steps() : 0;
    if (rs_mode == 1 && !fp32_narrow_o_tiles(n, NC, NP)) rs_mode = 0;
    if (rs_mode != 0) {
        DevBuf<uint32_t> rsmask((size_t)NC * 4);
        DevBuf<int> rscnt((size_t)NC * 4), rspre(((size_t)NC + 1) * 4);
        nbat.alloc(NP);
        rbase.alloc(NP + 1);
        LAUNCH(k_row_step_masks, NC, F.chunk_eptr.p, F.entries.p, NC, rsmask.p, rscnt.p);
        for (int g = 0; g < 4; ++g)
            exclusive_sum<int, int>(rscnt.p + (size_t)g * NC, rspre.p + (size_t)g * (NC + 1), NC,
                                    st);
        LAUNCH(k_row_step_batches, NP, cbase.p, rspre.p, NP, NC, rs_mode == 2, kRowStepRatioNum,
               kRowStepRatioDen, nbat.p);
        exclusive_sum<int, int>(nbat.p, rbase.p, NP, st);
        NB = read_scalar(rbase.p + NP, st);
        if (NB > 0) {
            F.rs_cols.alloc((size_t)NB * kChunkCols);
            F.rs_vals.alloc((size_t)NB * 128);
            fill<int>(F.rs_cols.p, (long long)NB * kChunkCols, -1, st);
            fill<float>(F.rs_vals.p, (long long)NB * 128, 0.0f, st);
            LAUNCH(k_row_step_fill, NC, cbase.p, rbase.p, nbat.p, rsmask.p, rspre.p,
                   F.chunk_eptr.p, F.entries.p, F.chunk_cols.p, NP, NC, F.rs_cols.p, F.rs_vals.p);
            // a panel's work items: its batches where it takes row steps, else its tiles
            LAUNCH(k_pick_work, NP, nbat.p, NP, nch.p);
        }
    }
    F.num_row_step_batches = NB;

    const int light_max = light_tile_limit(NP);
    const int heavy_tiles = heavy_tile_limit(NC);
    DevBuf<int> nu(NP), ubase(NP + 1), nheavy(NP), hbase(NP + 1), nsplit(NP), sbase(NP + 1);
    LAUNCH(k_units_per_panel, NP, nch.p, NP, light_max, heavy_tiles, nu.p, nheavy.p, nsplit.p);
    exclusive_sum<int, int>(nu.p, ubase.p, NP, st);
    exclusive_sum<int, int>(nheavy.p, hbase.p, NP, st);
    exclusive_sum<int, int>(nsplit.p, sbase.p, NP, st);
    const int NU = read_scalar(ubase.p + NP, st);
    const int NH = read_scalar(hbase.p + NP, st);
    const int NS = read_scalar(sbase.p + NP, st);
    {
        DevBuf<int4> raw(NU);
        DevBuf<uint32_t> k1(NU), k2(NU), v1(NU), v2(NU);
        const bool by_column = light_by_column(n, F.num_pairs);
        LAUNCH(k_make_units, NP, cbase.p, NB > 0 ? rbase.p : nullptr,
               NB > 0 ? nbat.p : nullptr, ubase.p, ppanel.p, pmask.p, nch.p, NP, light_max,
               heavy_tiles, F.chunk_cols.p, by_column, raw.p, k1.p, v1.p);
        uint32_t *kp2 = k1.p, *ka2 = k2.p, *vp2 = v1.p, *va2 = v2.p;
        radix_sort_pairs<uint32_t>(kp2, vp2, ka2, va2, NU, by_column ? 32 : 17, st);
        F.units.alloc(NU);
        LAUNCH(k_gather_units, NU, raw.p, vp2, NU, F.units.p);
    }
    // Light units are split into eight contiguous ranges of about equal tile count, one per XCD.
    {
        const int NL = NU - NH;
        DevBuf<int> nt(NL > 0 ? NL : 1), cut(9);
        DevBuf<long long> csum((size_t)NL + 1);
        LAUNCH(k_light_tiles, NL, F.units.p, NH, NL, nt.p);
        exclusive_sum<int, long long>(nt.p, csum.p, NL, st);
        hipLaunchKernelGGL(k_xcd_cuts, dim3(1), dim3(64), 0, st, csum.p, NL, cut.p);
        VCSRMC_HIP(hipGetLastError());
        VCSRMC_HIP(hipMemcpyAsync(F.xcd_start, cut.p, sizeof(int) * 9, hipMemcpyDeviceToHost, st));
        VCSRMC_HIP(hipStreamSynchronize(st));
    }
    F.num_panels = NP;
    F.num_chunks = NC;
    F.num_units = NU;
    F.num_heavy = NH;
    F.num_split_panels = NS;
    F.light_max = light_max;
    F.heavy_tiles = heavy_tiles;
}

static void build_layout_in_order(DeviceFormat& F, const int* trow, const int* tcol,
                                  const float* tval, const int* rowpos, long long n,
                                  hipStream_t st) {
    F.num_panels = F.num_chunks = F.num_units = F.num_dense = F.max_panel_tiles = 0;
    F.num_row_step_batches = 0;
    F.num_pairs = 0;
    if (n == 0) return;
    const int num_panels_all = (F.M + kPanelRows - 1) / kPanelRows;
    const int cbits = bits_for(F.N > 0 ? (unsigned long long)(F.N - 1) : 0ull);
    const int pbits = bits_for(num_panels_all > 0 ? (unsigned long long)(num_panels_all - 1) : 0ull);
    if (pbits + cbits + 4 <= 32)
        build_exec_layout_k<uint32_t>(F, trow, tcol, tval, rowpos, n, st);
    else
        build_exec_layout_k<unsigned long long>(F, trow, tcol, tval, rowpos, n, st);
}

// Moves the execution layout (not the format arrays) between two formats of the same matrix.
static void swap_layout(DeviceFormat& a, DeviceFormat& b) {
    std::swap(a.num_panels, b.num_panels);
    std::swap(a.num_chunks, b.num_chunks);
    std::swap(a.num_units, b.num_units);
    std::swap(a.num_heavy, b.num_heavy);
    std::swap(a.light_max, b.light_max);
    std::swap(a.heavy_tiles, b.heavy_tiles);
    std::swap(a.num_split_panels, b.num_split_panels);
    std::swap(a.max_panel_tiles, b.max_panel_tiles);
    std::swap(a.num_pairs, b.num_pairs);
    std::swap(a.xcd_start, b.xcd_start);
    std::swap(a.units, b.units);
    std::swap(a.row_map, b.row_map);
    std::swap(a.chunk_eptr, b.chunk_eptr);
    std::swap(a.chunk_cols, b.chunk_cols);
    std::swap(a.entries, b.entries);
    std::swap(a.num_dense, b.num_dense);
    std::swap(a.chunk_dense, b.chunk_dense);
    std::swap(a.dense_a16, b.dense_a16);
    std::swap(a.dense_a32, b.dense_a32);
    std::swap(a.num_row_step_batches, b.num_row_step_batches);
    std::swap(a.rs_cols, b.rs_cols);
    std::swap(a.rs_vals, b.rs_vals);
}

// 0 off, 1 when it pays (the default), 2 always; read once by each build.
static std::atomic<int> g_row_grouping{1};
void set_row_grouping(int mode) { g_row_grouping.store(mode, std::memory_order_relaxed); }
int row_grouping() { return g_row_grouping.load(std::memory_order_relaxed); }

// 0 tiles only, 1 row steps where they pay (the default), 2 always; read once by each build.
static std::atomic<int> g_fp32_row_steps{1};
void set_fp32_row_steps(int mode) { g_fp32_row_steps.store(mode, std::memory_order_relaxed); }
int fp32_row_steps() { return g_fp32_row_steps.load(std::memory_order_relaxed); }

// The execution layout's row order.  Mode 0: natural.  Otherwise, first, rows without nonzeros
// go after the others when they are at least an eighth of the rows (compact_rows; R-MAT scale
// 22, about 45% of its rows empty: panels 231,761 -> 125,559, kernel 2.60 -> 2.54 ms
// accumulating, scale 20 508 -> 488 us).  Then rows are grouped by shared columns
// (row_groups.hip), always in mode 2, and in mode 1 (the default) when the rows of a panel
// already share columns -- at least 1.3 nonzeros per distinct (panel, column) pair, as in grids
// and meshes in natural order (2D 5-point 1.6, 3D 7-point 1.37, 27-point 2.66) and not in
// uniform random, power-law or R-MAT matrices (1.01-1.23 at scales 16-22) -- and the tiles are
// not full (fewer than 256 nonzeros on average), keeping the grouped layout when it saves at
// least a tenth of the tiles.  Measured on gfx950, kernel us natural -> grouped (C += A.B /
// C = A.B): 27-point stencil FP32 20^3 7.97 / 7.49 -> 6.00 / 5.60, 60^3 126 / 109 -> 89 / 69,
// 100^3 564 / 510 -> 447 / 359 (tiles 365,224 -> 187,016, 4 x 2 x 2 blocks), FP16 100^3 337 /
// 300 -> 316 / 251; 2D 5-point 1000^2 FP32 312 / 234 -> 297 / 196 (tiles halved); 3D 7-point
// 100^3 FP32 390 / 328 -> 373 / 255; 27-point 16^3 (256 panels) within 2% either way.  Grouping
// the excluded classes anyway saved 1-7% of their tiles and ran from 6% faster to 13% slower.
static void build_exec_layout(DeviceFormat& F, const int* trow, const int* tcol, const float* tval,
                              long long n, hipStream_t st) {
    F.row_map.release();
    const int mode = row_grouping();
    DevBuf<int> cpos, cmap;
    const bool compact = mode != 0 && compact_rows(trow, n, F.M, st, cpos, cmap);
    build_layout_in_order(F, trow, tcol, tval, compact ? cpos.p : nullptr, n, st);
    if (compact) F.row_map = std::move(cmap);
    if (mode == 0 || F.num_chunks == 0) return;
    const long long NC = F.num_chunks;
    if (mode == 1) {
        if (!(10 * n >= 13 * F.num_pairs && n < 256 * NC)) return;
        // Grouping is an optimisation here: it is skipped, natural order kept, unless its buffers
        // (at most ~64 bytes per nonzero and per row, for the sorts and a second layout) fit
        // in half the free device memory.
        size_t free_b = 0, total_b = 0;
        if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) {
            (void)hipGetLastError();
            return;
        }
        if (64.0 * (double)n + 64.0 * (double)F.M > 0.5 * (double)free_b) return;
    }
    DevBuf<int> rowpos, row_map;
    if (!group_rows(trow, tcol, n, F.M, F.N, st, rowpos, row_map)) return;
    DeviceFormat G;
    G.M = F.M;
    G.N = F.N;
    G.fp32 = F.fp32;
    G.nnz = F.nnz;
    build_layout_in_order(G, trow, tcol, tval, rowpos.p, n, st);
    if (mode == 1 && 10LL * G.num_chunks > 9LL * NC) return;
    G.row_map = std::move(row_map);
    swap_layout(F, G);
}

// ------------------------------------------------------------------------------------------
// Part 1 driver.
// ------------------------------------------------------------------------------------------
template <typename K>
static void build_groups_k(DeviceFormat& F, const int* d_col, const float* d_val,
                           const int* pstart, const int* prow, int P, int S, float inv_scale,
                           hipStream_t st) {
    const int segw = F.segw;
    const int kbits = 6 + bits_for((unsigned long long)(S > 0 ? S - 1 : 0));
    DevBuf<K> k1(P), k2(P);
    DevBuf<uint32_t> v1(P), v2(P);
    DevBuf<int> seg_start(S + 1), gnum(S), gbase(S + 1);
    LAUNCH((k_pair_keys<K>), P, pstart, d_col, P, segw, k1.p, v1.p);
    K* kp = k1.p; K* ka = k2.p;
    uint32_t* vp = v1.p; uint32_t* va = v2.p;
    radix_sort_pairs<K>(kp, vp, ka, va, P, kbits, st);
    LAUNCH((k_seg_starts<K>), (long long)S + 1, kp, P, S, seg_start.p);
    LAUNCH(k_groups_per_seg, S, seg_start.p, S, gnum.p);
    exclusive_sum<int, int>(gnum.p, gbase.p, S, st);
    const int G = read_scalar(gbase.p + S, st);

    DevBuf<int> ghead(G), size16(G);
    DevBuf<long long> gp64(G + 1);
    F.group_depth.alloc(G);
    F.group_seg_base.alloc(G);
    F.group_rows.alloc((size_t)16 * G);
    F.group_ptr.alloc(G + 1);
    LAUNCH((k_group_heads<K>), P, kp, seg_start.p, gbase.p, P, ghead.p);
    LAUNCH((k_group_info<K>), G, kp, vp, ghead.p, seg_start.p, pstart, prow, G, segw,
           F.group_depth.p, F.group_seg_base.p, F.group_rows.p, size16.p);
    exclusive_sum<int, long long>(size16.p, gp64.p, G, st);
    const long long nval = read_scalar(gp64.p + G, st);
    if (nval > INT_MAX)
        throw Error(VCSRMC_ERR_OVERFLOW, "|val| of the format exceeds the int32 group_ptr");
    LAUNCH(k_to_int, (long long)G + 1, gp64.p, F.group_ptr.p, (long long)G + 1);
    F.lcol.alloc(nval);
    F.val.alloc(nval);
    if (G > 0) {
        hipLaunchKernelGGL((k_fill_group_entries<K>), dim3(grid_for((long long)G * 64, 256)),
                           dim3(256), 0, st, kp, vp, ghead.p, seg_start.p, pstart, F.group_ptr.p,
                           F.group_depth.p, F.group_seg_base.p, d_col, d_val, G, inv_scale,
                           F.lcol.p, F.val.p);
        VCSRMC_HIP(hipGetLastError());
    }

    // Work items (src/vcsr_mc.cu:109-121).
    const int chunk = std::max(1, std::min(32, G / 4096));
    DevBuf<int> inum(S), ibase(S + 1);
    LAUNCH(k_items_per_seg, S, gnum.p, S, chunk, inum.p);
    exclusive_sum<int, int>(inum.p, ibase.p, S, st);
    const int I = read_scalar(ibase.p + S, st);
    const int wmax = chunk * 16 * 64;  // work <= chunk groups x 16 lanes x depth <= 64
    DevBuf<int> ib(I), ie(I);
    DevBuf<uint32_t> ik1(I), ik2(I), ip1(I), ip2(I);
    LAUNCH(k_make_items, S, gbase.p, ibase.p, F.group_ptr.p, S, chunk, wmax, ib.p, ie.p, ik1.p,
           ip1.p);
    uint32_t *ikp = ik1.p, *ika = ik2.p, *ipp = ip1.p, *ipa = ip2.p;
    radix_sort_pairs<uint32_t>(ikp, ipp, ika, ipa, I, bits_for((unsigned long long)wmax), st);
    F.item_gbeg.alloc(I);
    F.item_gend.alloc(I);
    LAUNCH(k_gather_items, I, ipp, ib.p, ie.p, I, F.item_gbeg.p, F.item_gend.p);
    F.G = G;
    F.nval = nval;
    F.nitems = I;
}

void build_from_csr(DeviceFormat& F, const int* d_row_ptr, const int* d_col, const float* d_val,
                    int M, int N, int nnz, int segw, int fp32, hipStream_t st) {
    if (segw != 16 && segw != 32 && segw != 48 && segw != 64)
        throw Error(VCSRMC_ERR_SEGW, "vcsr_mc supports segw in {16, 32, 48, 64}");
    if (M < 0 || N < 0 || nnz < 0) throw Error(VCSRMC_ERR_ARG, "negative matrix size");
    if (!d_row_ptr || (nnz > 0 && (!d_col || !d_val)))
        throw Error(VCSRMC_ERR_ARG, "null CSR pointer");
    F.clear();
    F.M = M;
    F.N = N;
    F.segw = segw;
    F.bundle = 16;
    F.fp32 = fp32 ? 1 : 0;
    F.nnz = nnz;
    const int S = (int)(((long long)N + segw - 1) / segw);
    F.num_segments = S;

    DevBuf<int> err(1);
    VCSRMC_HIP(hipMemsetAsync(err.p, 0, sizeof(int), st));
    LAUNCH(k_check_row_ptr, (long long)M + 1, d_row_ptr, M, nnz, err.p);
    check_err(err.p, st);

    // Scale (src/vcsr_mc.cu:33-34).
    F.scale = F.fp32 ? 1.0f : half_scale_from_amax(device_absmax(d_val, nnz, st));
    const float inv_scale = 1.0f / F.scale;

    if (nnz == 0) {
        F.group_ptr.alloc(1);
        VCSRMC_HIP(hipMemsetAsync(F.group_ptr.p, 0, sizeof(int), st));
        VCSRMC_HIP(hipStreamSynchronize(st));
        F.ready = true;
        return;
    }

    // Row of every nonzero.
    DevBuf<int> row_of(nnz);
    {
        DevBuf<int> head(nnz);
        fill<int>(head.p, nnz, (int)0x80000000, st);
        LAUNCH(k_mark_row_heads, M, d_row_ptr, M, head.p);
        inclusive_max(head.p, row_of.p, nnz, st);
    }
    // (segment, row) runs.
    DevBuf<int> phead(nnz), pidx(nnz + 1);
    LAUNCH(k_pair_heads, nnz, d_row_ptr, d_col, row_of.p, nnz, N, segw, phead.p, err.p);
    check_err(err.p, st);
    exclusive_sum<int, int>(phead.p, pidx.p, nnz, st);
    const int P = read_scalar(pidx.p + nnz, st);
    DevBuf<int> pstart(P + 1), prow(P);
    LAUNCH(k_emit_pairs, nnz, phead.p, pidx.p, row_of.p, nnz, pstart.p, prow.p);
    fill<int>(pstart.p + P, 1, nnz, st);
    phead.release();
    pidx.release();

    if (6 + bits_for((unsigned long long)(S - 1)) <= 32)
        build_groups_k<uint32_t>(F, d_col, d_val, pstart.p, prow.p, P, S, inv_scale, st);
    else
        build_groups_k<unsigned long long>(F, d_col, d_val, pstart.p, prow.p, P, S, inv_scale,
                                           st);
    pstart.release();
    prow.release();

    // Execution layout from (row_of, col, val / scale).
    DevBuf<float> sval(nnz);
    LAUNCH(k_scale_values, nnz, d_val, sval.p, (long long)nnz, inv_scale);
    build_exec_layout(F, row_of.p, d_col, sval.p, nnz, st);
    VCSRMC_HIP(hipStreamSynchronize(st));
    F.ready = true;
}

// ------------------------------------------------------------------------------------------
// Upload of caller-held arrays.
// ------------------------------------------------------------------------------------------
__global__ void k_check_groups(const int* __restrict__ gp, const int* __restrict__ depth,
                               const int* __restrict__ seg_base, const int* __restrict__ rows,
                               int G, long long nval, int M, int N, int segw,
                               int* __restrict__ err) {
    const long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (g > G) return;
    bool bad = false;
    if (g == 0) bad |= gp[0] != 0;
    if (g == G) {
        bad |= (long long)gp[G] != nval;
    } else {
        const int d = depth[g];
        bad |= d < 0 || (long long)gp[g + 1] - gp[g] != 16LL * d;
        const int sb = seg_base[g];
        bad |= sb < 0 || sb >= N || sb % segw != 0;
        for (int l = 0; l < 16; ++l) {
            const int r = rows[16 * g + l];
            bad |= r < -1 || r >= M;
        }
    }
    if (bad) atomicOr(err, kErrFormat);
}

__global__ void k_expand_flags(const int* __restrict__ gp, const int* __restrict__ seg_base,
                               const int* __restrict__ rows, const int* __restrict__ lcol, int G,
                               long long nval, int N, int segw, int* __restrict__ flag,
                               int* __restrict__ err) {
    const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nval) return;
    // group of slot t: last g with gp[g] <= t
    int lo = 0, hi = G;  // gp[lo] <= t < gp[hi]
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if ((long long)gp[mid] <= t) lo = mid; else hi = mid;
    }
    const int lane = (int)((t - gp[lo]) & 15);
    const int lc = lcol[t];
    int f = 0;
    if (lc >= 0) {
        const int r = rows[16 * lo + lane];
        const long long c = (long long)seg_base[lo] + lc;
        if (lc >= segw || r < 0 || c >= N) atomicOr(err, kErrFormat);
        else f = 1;
    } else if (lc != -1) {
        atomicOr(err, kErrFormat);
    }
    flag[t] = f;
}

__global__ void k_expand_write(const int* __restrict__ gp, const int* __restrict__ seg_base,
                               const int* __restrict__ rows, const int* __restrict__ lcol,
                               const float* __restrict__ val, const int* __restrict__ flag,
                               const int* __restrict__ pos, int G, long long nval,
                               int* __restrict__ trow, int* __restrict__ tcol,
                               float* __restrict__ tval) {
    const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nval || !flag[t]) return;
    int lo = 0, hi = G;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if ((long long)gp[mid] <= t) lo = mid; else hi = mid;
    }
    const int lane = (int)((t - gp[lo]) & 15);
    const int i = pos[t];
    trow[i] = rows[16 * lo + lane];
    tcol[i] = seg_base[lo] + lcol[t];
    tval[i] = val[t];
}

template <typename T>
static void upload_array(DevBuf<T>& d, const T* h, long long n, hipStream_t st) {
    d.alloc(n > 0 ? n : 0);
    if (n > 0) {
        if (!h) throw Error(VCSRMC_ERR_ARG, "null format array");
        VCSRMC_HIP(hipMemcpyAsync(d.p, h, sizeof(T) * (size_t)n, hipMemcpyHostToDevice, st));
    }
}

void build_from_host(DeviceFormat& F, const HostArrays& H, hipStream_t st) {
    if (H.segw != 16 && H.segw != 32 && H.segw != 48 && H.segw != 64)
        throw Error(VCSRMC_ERR_SEGW, "vcsr_mc supports segw in {16, 32, 48, 64}");
    if (H.M < 0 || H.N < 0 || H.G < 0 || H.nval < 0 || H.nitems < 0 || H.nval > INT_MAX)
        throw Error(VCSRMC_ERR_ARG, "negative or oversized format size");
    if (H.bundle != 16) throw Error(VCSRMC_ERR_FORMAT, "bundle must be 16");
    if (H.nval != 16LL * (H.nval / 16)) throw Error(VCSRMC_ERR_FORMAT, "|val| is not 16 * depth");
    F.clear();
    F.M = H.M; F.N = H.N; F.segw = H.segw; F.bundle = H.bundle; F.num_segments = H.num_segments;
    F.G = H.G; F.nval = H.nval; F.nitems = H.nitems; F.scale = H.scale; F.fp32 = H.fp32 ? 1 : 0;
    upload_array(F.group_ptr, H.group_ptr, (long long)H.G + 1, st);
    upload_array(F.group_depth, H.group_depth, H.G, st);
    upload_array(F.group_seg_base, H.group_seg_base, H.G, st);
    upload_array(F.group_rows, H.group_rows, 16LL * H.G, st);
    upload_array(F.lcol, H.lcol, H.nval, st);
    upload_array(F.val, H.val, H.nval, st);
    upload_array(F.item_gbeg, H.item_gbeg, H.nitems, st);
    upload_array(F.item_gend, H.item_gend, H.nitems, st);

    DevBuf<int> err(1);
    VCSRMC_HIP(hipMemsetAsync(err.p, 0, sizeof(int), st));
    LAUNCH(k_check_groups, (long long)H.G + 1, F.group_ptr.p, F.group_depth.p,
           F.group_seg_base.p, F.group_rows.p, H.G, H.nval, H.M, H.N, H.segw, err.p);
    check_err(err.p, st);

    const long long nval = H.nval;
    DevBuf<int> flag(nval), pos(nval + 1);
    LAUNCH(k_expand_flags, nval, F.group_ptr.p, F.group_seg_base.p, F.group_rows.p, F.lcol.p,
           H.G, nval, H.N, H.segw, flag.p, err.p);
    check_err(err.p, st);
    exclusive_sum<int, int>(flag.p, pos.p, nval, st);
    const int n = nval ? read_scalar(pos.p + nval, st) : 0;
    F.nnz = n;
    DevBuf<int> trow(n), tcol(n);
    DevBuf<float> tval(n);
    LAUNCH(k_expand_write, nval, F.group_ptr.p, F.group_seg_base.p, F.group_rows.p, F.lcol.p,
           F.val.p, flag.p, pos.p, H.G, nval, trow.p, tcol.p, tval.p);
    build_exec_layout(F, trow.p, tcol.p, tval.p, n, st);
    VCSRMC_HIP(hipStreamSynchronize(st));
    F.ready = true;
}

}  // namespace vcsrmc
