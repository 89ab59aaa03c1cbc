// primitives.hpp -- device-wide scan, stable LSD radix sort and small utilities, written for
// gfx950 wave64: wave scans use DPP row shifts plus v_readlane carries; the radix scatter
// ranks keys with 8 wave ballots per round (a wave-level multisplit), so every pass is
// stable and deterministic.
#pragma once
#include <cstddef>
#include <cstdint>
#include <utility>

#include "hip_common.hpp"

namespace vcsrmc {

// ---- device memory owned for the duration of a scope ----------------------------------
template <typename T>
struct DevBuf {
    T* p = nullptr;
    size_t n = 0;
    DevBuf() = default;
    explicit DevBuf(size_t count) { alloc(count); }
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    DevBuf(DevBuf&& o) noexcept : p(o.p), n(o.n) { o.p = nullptr; o.n = 0; }
    DevBuf& operator=(DevBuf&& o) noexcept {
        if (this != &o) { release(); p = o.p; n = o.n; o.p = nullptr; o.n = 0; }
        return *this;
    }
    ~DevBuf() { release(); }
    // On failure the buffer stays empty (p null, n 0) and the runtime's error is cleared, so
    // a later launch does not report it.
    void alloc(size_t count) {
        release();
        if (!count) return;
        const hipError_t e = hipMalloc((void**)&p, count * sizeof(T));
        if (e != hipSuccess) {
            p = nullptr;
            (void)hipGetLastError();
            throw_hip(e, "hipMalloc", __FILE__, __LINE__);
        }
        n = count;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
    }
    T* take() { T* q = p; p = nullptr; n = 0; return q; }
};

constexpr int kScanThreads = 256;
constexpr int kScanItems = 8;
constexpr long long kScanTile = (long long)kScanThreads * kScanItems;

// Block-level inclusive scan of one value per thread (256 threads = 4 waves).
template <typename T, typename Op>
__device__ __forceinline__ T block_scan_256(T x, Op op, T identity, T* wsum /* LDS[4] */,
                                            T& block_total) {
    const int t = threadIdx.x, w = t >> 6;
    T incl = wave_scan(x, op, identity);
    if ((t & 63) == 63) wsum[w] = incl;
    __syncthreads();
    T wp = identity;
    for (int i = 0; i < w; ++i) wp = op(wp, wsum[i]);
    block_total = op(op(wsum[0], wsum[1]), op(wsum[2], wsum[3]));
    __syncthreads();
    return op(wp, incl);
}

template <typename TIn, typename TOut, typename Op>
__global__ __launch_bounds__(kScanThreads) void k_reduce_tile(const TIn* __restrict__ in,
                                                              TOut* __restrict__ partial,
                                                              long long n, Op op, TOut identity) {
    __shared__ TOut wsum[4];
    const long long base = (long long)blockIdx.x * kScanTile;
    TOut acc = identity;
    for (int j = 0; j < kScanItems; ++j) {
        const long long i = base + (long long)j * kScanThreads + threadIdx.x;
        if (i < n) acc = op(acc, (TOut)in[i]);
    }
    TOut total;
    block_scan_256(acc, op, identity, wsum, total);
    if (threadIdx.x == 0) partial[blockIdx.x] = total;
}

// EXCL: out[i] = in[0] + ... + in[i-1] (OpAdd only) and, when write_total, out[n] = total.
// Otherwise out[i] = op(in[0..i]).
template <typename TIn, typename TOut, typename Op, bool EXCL>
__global__ __launch_bounds__(kScanThreads) void k_scan_tile(const TIn* __restrict__ in,
                                                            TOut* __restrict__ out, long long n,
                                                            const TOut* __restrict__ prefix_incl,
                                                            Op op, TOut identity, int write_total) {
    __shared__ TOut wsum[4];
    const long long base = (long long)blockIdx.x * kScanTile;
    TOut running = (prefix_incl && blockIdx.x > 0) ? prefix_incl[blockIdx.x - 1] : identity;
    for (int j = 0; j < kScanItems; ++j) {
        const long long i = base + (long long)j * kScanThreads + threadIdx.x;
        const TOut x = i < n ? (TOut)in[i] : identity;
        TOut total;
        const TOut incl = block_scan_256(x, op, identity, wsum, total);
        if (i < n) {
            if constexpr (EXCL) out[i] = running + incl - x;
            else out[i] = op(running, incl);
        }
        running = op(running, total);
    }
    if (EXCL && write_total && blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) out[n] = running;
}

template <typename TIn, typename TOut, typename Op, bool EXCL>
void scan_impl(const TIn* in, TOut* out, long long n, Op op, TOut identity, int write_total,
               hipStream_t st) {
    if (n <= 0) {
        if (EXCL && write_total) VCSRMC_HIP(hipMemsetAsync(out, 0, sizeof(TOut), st));
        return;
    }
    const long long tiles = (n + kScanTile - 1) / kScanTile;
    if (tiles == 1) {
        hipLaunchKernelGGL((k_scan_tile<TIn, TOut, Op, EXCL>), dim3(1), dim3(kScanThreads), 0, st,
                           in, out, n, (const TOut*)nullptr, op, identity, write_total);
        VCSRMC_HIP(hipGetLastError());
        return;
    }
    DevBuf<TOut> partial(tiles), prefix(tiles);
    hipLaunchKernelGGL((k_reduce_tile<TIn, TOut, Op>), dim3((unsigned)tiles), dim3(kScanThreads), 0,
                       st, in, partial.p, n, op, identity);
    VCSRMC_HIP(hipGetLastError());
    scan_impl<TOut, TOut, Op, false>(partial.p, prefix.p, tiles, op, identity, 0, st);
    hipLaunchKernelGGL((k_scan_tile<TIn, TOut, Op, EXCL>), dim3((unsigned)tiles), dim3(kScanThreads),
                       0, st, in, out, n, (const TOut*)prefix.p, op, identity, write_total);
    VCSRMC_HIP(hipGetLastError());
}

// out[0..n]: exclusive prefix sums of in[0..n-1], out[n] = total.
template <typename TIn, typename TOut>
void exclusive_sum(const TIn* in, TOut* out, long long n, hipStream_t st) {
    scan_impl<TIn, TOut, OpAdd, true>(in, out, n, OpAdd{}, (TOut)0, 1, st);
}

template <typename TIn, typename TOut>
void inclusive_sum(const TIn* in, TOut* out, long long n, hipStream_t st) {
    scan_impl<TIn, TOut, OpAdd, false>(in, out, n, OpAdd{}, (TOut)0, 0, st);
}

inline void inclusive_max(const int* in, int* out, long long n, hipStream_t st) {
    scan_impl<int, int, OpMax, false>(in, out, n, OpMax{}, (int)0x80000000, 0, st);
}

// Copy one value back (synchronises the stream).
template <typename T>
T read_scalar(const T* dptr, hipStream_t st) {
    T v{};
    VCSRMC_HIP(hipMemcpyAsync(&v, dptr, sizeof(T), hipMemcpyDeviceToHost, st));
    VCSRMC_HIP(hipStreamSynchronize(st));
    return v;
}

// ---- stable LSD radix sort of (key, 32-bit payload) pairs ------------------------------
constexpr int kSortThreads = 256;
constexpr int kSortRounds = 16;
constexpr long long kSortTile = (long long)kSortThreads * kSortRounds;  // 4096 keys per tile

template <typename K>
__global__ __launch_bounds__(kSortThreads) void k_radix_hist(const K* __restrict__ keys, long long n,
                                                             int shift, int* __restrict__ hist,
                                                             int ntiles) {
    __shared__ int h[256];
    h[threadIdx.x] = 0;
    __syncthreads();
    const long long base = (long long)blockIdx.x * kSortTile;
    for (int r = 0; r < kSortRounds; ++r) {
        const long long i = base + (long long)r * kSortThreads + threadIdx.x;
        if (i < n) atomicAdd(&h[(int)((keys[i] >> shift) & 255u)], 1);
    }
    __syncthreads();
    hist[(long long)threadIdx.x * ntiles + blockIdx.x] = h[threadIdx.x];
}

// offsets: exclusive scan of the digit-major histogram.  Keys of one tile are ranked in
// index order: lane order inside a wave (ballot multisplit), wave order inside a round,
// round order inside the tile; tiles were ordered by the scan.
template <typename K>
__global__ __launch_bounds__(kSortThreads) void k_radix_scatter(
    const K* __restrict__ kin, const uint32_t* __restrict__ vin, K* __restrict__ kout,
    uint32_t* __restrict__ vout, long long n, int shift, const int* __restrict__ offsets,
    int ntiles) {
    __shared__ int run[256];
    __shared__ int wcnt[4][256];
    __shared__ int wofs[4][256];
    const int t = threadIdx.x, w = t >> 6, lane = t & 63;
    run[t] = offsets[(long long)t * ntiles + blockIdx.x];
    for (int i = 0; i < 4; ++i) wcnt[i][t] = 0;
    __syncthreads();
    const long long base = (long long)blockIdx.x * kSortTile;
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int r = 0; r < kSortRounds; ++r) {
        const long long i = base + (long long)r * kSortThreads + t;
        const bool valid = i < n;
        const K key = valid ? kin[i] : (K)0;
        const uint32_t val = valid ? vin[i] : 0u;
        const int d = valid ? (int)((key >> shift) & 255u) : 0;
        uint64_t peers = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const bool bit = (d >> b) & 1;
            const uint64_t m = __ballot(bit);
            peers &= bit ? m : ~m;
        }
        const int rank = __popcll(peers & lt);
        if (valid && rank == 0) wcnt[w][d] = __popcll(peers);
        __syncthreads();
        {
            int acc = run[t];
#pragma unroll
            for (int ww = 0; ww < 4; ++ww) {
                wofs[ww][t] = acc;
                acc += wcnt[ww][t];
                wcnt[ww][t] = 0;
            }
            run[t] = acc;
        }
        __syncthreads();
        if (valid) {
            const int dst = wofs[w][d] + rank;
            kout[dst] = key;
            vout[dst] = val;
        }
    }
}

// Sorts n pairs by the low `bits` bits of the key.  The sorted pairs end up in (k, v); the
// alternate buffers are scratch of the same size.  n must be below 2^31.
template <typename K>
void radix_sort_pairs(K*& k, uint32_t*& v, K*& k_alt, uint32_t*& v_alt, long long n, int bits,
                      hipStream_t st) {
    if (n <= 1 || bits <= 0) return;
    const int ntiles = (int)((n + kSortTile - 1) / kSortTile);
    DevBuf<int> hist((size_t)256 * ntiles), offs((size_t)256 * ntiles + 1);
    for (int shift = 0; shift < bits; shift += 8) {
        hipLaunchKernelGGL((k_radix_hist<K>), dim3(ntiles), dim3(kSortThreads), 0, st, k, n, shift,
                           hist.p, ntiles);
        VCSRMC_HIP(hipGetLastError());
        exclusive_sum<int, int>(hist.p, offs.p, (long long)256 * ntiles, st);
        hipLaunchKernelGGL((k_radix_scatter<K>), dim3(ntiles), dim3(kSortThreads), 0, st, k, v,
                           k_alt, v_alt, n, shift, offs.p, ntiles);
        VCSRMC_HIP(hipGetLastError());
        std::swap(k, k_alt);
        std::swap(v, v_alt);
    }
}

// ---- small kernels -----------------------------------------------------------------------
template <typename T>
__global__ void k_fill(T* __restrict__ p, long long n, T value) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = value;
}

template <typename T>
void fill(T* p, long long n, T value, hipStream_t st) {
    if (n <= 0) return;
    hipLaunchKernelGGL((k_fill<T>), dim3(grid_for(n, 256)), dim3(256), 0, st, p, n, value);
    VCSRMC_HIP(hipGetLastError());
}

__global__ void k_iota(uint32_t* __restrict__ p, long long n);
void iota(uint32_t* p, long long n, hipStream_t st);

}  // namespace vcsrmc
