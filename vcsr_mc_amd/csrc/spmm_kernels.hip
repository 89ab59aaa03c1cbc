// spmm_kernels.hip -- C += A.B for the VCSR-MC format on gfx950 MFMA.
//
// Work decomposition (atomic-free for all but split panels):
//   one 64-lane wave = one work unit = a run of compacted tiles of one 16-row panel,
//   for one tileK-wide slice of the output columns.  The wave keeps the 16 x tileK
//   accumulator tile in registers across all of its tiles and writes C once.
//
// Per 16 x 32 tile (32 distinct columns of the panel, any segments):
//   * B operand: lane (n = lane % 16, g = lane / 16) loads, for the 8 tile columns
//     k = 8g .. 8g+7, the contiguous VEC = tileK/16 output columns k0 + VEC n .. +VEC-1 of
//     that B row (one 128-bit load per row at tileK = 128, FP16 B); 16 lanes cover a
//     256-byte B row, so every load instruction reads four whole rows.  The VEC values are
//     then transposed in registers: MFMA q (q < VEC) takes the q-th value of each of the 8
//     rows, i.e. output column k0 + VEC n + q.  No LDS round trip for B.
//   * A operand: the tile's nonzeros (row, k, value) are scattered into a 16 x 32 LDS tile
//     that each lane then reads as its 8 contiguous K values (one 128-bit LDS read).
//   * FP16 format: v_mfma_f32_16x16x32_f16, FP32 accumulation.  FP32 format: eight K steps
//     of v_mfma_f32_16x16x4_f32.
//   The K order inside a tile is the same for A and B, so the contraction does not depend
//   on how the instruction maps lanes to K.
//
// Epilogue: lane (n, g) holds rows 4g..4g+3 at output columns k0 + VEC n .. + VEC-1, so each
// row is written as VEC contiguous floats per lane, 16 lanes per row: coalesced.  Rows that
// A does not touch are not written (the reference never touches them either).
#include "../../include/vcsrmc.h"
#include "internal.hpp"

namespace vcsrmc {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kApitch = 40;  // FP16 A tile row pitch in halves (80 B: conflict-free b128 reads)

// Map a linear work-group id to a unit so that each XCD (work-groups are dealt to the 8 XCDs
// round robin) walks a contiguous range of panels: neighbouring panels share B rows in L2.
__device__ __forceinline__ int unit_of_block(int bid, int num_units) {
    const int per = (num_units + 7) >> 3;
    return (bid & 7) * per + (bid >> 3);
}

// Raw B values of the 8 tile rows a lane feeds into the MFMA B operand, one vector of VEC
// consecutive output columns per row (kept in the storage type until use, so a prefetched load
// is never waited for early by a conversion).
template <int VEC, typename TB>
struct BRows {
    typedef TB vec_t __attribute__((ext_vector_type(VEC)));
    vec_t r[8];
};

// Zeros read in place of a B row by padding columns and by lanes past O.  Never written; not
// `const`, so that it lives in the global address space like B and the loads stay global loads
// (a constant-space operand would turn them into flat loads, which also count against the LDS
// wait counter).
__device__ __attribute__((aligned(16))) float kZeroRow[16];

// Every load is issued unconditionally (padding columns and lanes past O read kZeroRow): the
// number of loads in flight is then the same on every path, which lets the compiler wait for
// exactly the older loads it needs, and no select is needed after a load.
template <int VEC, typename TB, bool ALIGNED>
__device__ __forceinline__ void load_b_rows(const TB* __restrict__ B, const int (&cols)[8],
                                            long long O, int c0, BRows<VEC, TB>& R) {
    typedef typename BRows<VEC, TB>::vec_t vec_t;
    const bool lane_ok = c0 < O;
    const TB* zero = reinterpret_cast<const TB*>(kZeroRow);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int col = cols[i];
        const bool ok = col >= 0 && lane_ok;
        const TB* src = ok ? B + (long long)col * O + c0 : zero;
        if constexpr (ALIGNED && VEC * sizeof(TB) >= 4) {
            R.r[i] = *reinterpret_cast<const vec_t*>(src);
        } else {
            vec_t x;
#pragma unroll
            for (int q = 0; q < VEC; ++q) x[q] = (ok && c0 + q < O) ? src[q] : (TB)0;
            R.r[i] = x;
        }
    }
}

__device__ __forceinline__ void load_cols8(const int* __restrict__ chunk_cols, int c, int g,
                                           int (&cols)[8]) {
    const int4 lo = *reinterpret_cast<const int4*>(chunk_cols + (long long)c * kChunkCols + 8 * g);
    const int4 hi = *reinterpret_cast<const int4*>(chunk_cols + (long long)c * kChunkCols + 8 * g + 4);
    cols[0] = lo.x; cols[1] = lo.y; cols[2] = lo.z; cols[3] = lo.w;
    cols[4] = hi.x; cols[5] = hi.y; cols[6] = hi.z; cols[7] = hi.w;
}

__device__ __forceinline__ void scatter_a_f16(_Float16* As, uint32_t w) {
    As[((w >> 16) & 15) * kApitch + ((w >> 20) & 31)] =
        __builtin_bit_cast(_Float16, (unsigned short)(w & 0xffffu));
}

// Orders the LDS traffic of one wave (its private A tile): LDS instructions of a wave execute
// in issue order, so a wavefront-scope fence (no instruction, a compiler barrier) is enough.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Adds the unit's 16 x TK result into C.  W == 1: straight from the accumulators (lane (n, g)
// owns rows 4g..4g+3, columns k0 + VEC n .. + VEC - 1).  W > 1: every wave parks its partial
// tile in LDS, then the work-group sums the W partials and writes each row with consecutive
// threads on consecutive columns.  Split panels merge through atomics; other rows are a
// read-modify-write (C += A.B).  Rows outside the panel's row mask are never touched.
template <int TK, int W>
__device__ __forceinline__ void merge_into_c(const floatx4 (&acc)[TK / 16], float scale,
                                             const int4& U, int k0, int O, bool c4,
                                             float* __restrict__ C, float* P) {
    constexpr int VEC = TK / 16;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n = lane & 15, g = lane >> 4;
    const bool split = (U.w >> 16) & 1;
    const long long OL = O;
    if constexpr (W == 1) {
        const int c0 = k0 + VEC * n;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int rl = 4 * g + i;
            if (!((U.w >> rl) & 1)) continue;
            float* crow = C + (long long)(U.x + rl) * OL + c0;
            if (split) {
#pragma unroll
                for (int q = 0; q < VEC; ++q)
                    if (c0 + q < O) atomicAdd(crow + q, acc[q][i] * scale);
            } else if (VEC >= 4 && c4 && c0 + VEC <= O) {
#pragma unroll
                for (int h = 0; h < VEC; h += 4) {
                    floatx4 v = *reinterpret_cast<floatx4*>(crow + h);
#pragma unroll
                    for (int q = 0; q < 4; ++q) v[q] += acc[(h + q) % VEC][i] * scale;
                    *reinterpret_cast<floatx4*>(crow + h) = v;
                }
            } else {
#pragma unroll
                for (int q = 0; q < VEC; ++q)
                    if (c0 + q < O) crow[q] += acc[q][i] * scale;
            }
        }
    } else {
        float* Pw = P + wave * 16 * TK;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int q = 0; q < VEC; ++q) Pw[(4 * g + i) * TK + VEC * n + q] = acc[q][i];
        __syncthreads();
        for (int e = threadIdx.x * 4; e < 16 * TK; e += 64 * W * 4) {
            const int row = e / TK, col = e % TK;
            if (!((U.w >> row) & 1)) continue;
            floatx4 sum = *reinterpret_cast<const floatx4*>(P + e);
#pragma unroll
            for (int w = 1; w < W; ++w) {
                const floatx4 x = *reinterpret_cast<const floatx4*>(P + w * 16 * TK + e);
                sum += x;
            }
            const int cc = k0 + col;
            if (cc >= O) continue;
            float* crow = C + (long long)(U.x + row) * OL + cc;
            if (split) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (cc + j < O) atomicAdd(crow + j, sum[j] * scale);
            } else if (c4 && cc + 4 <= O) {
                floatx4 v = *reinterpret_cast<floatx4*>(crow);
                v += sum * scale;
                *reinterpret_cast<floatx4*>(crow) = v;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (cc + j < O) crow[j] += sum[j] * scale;
            }
        }
    }
}

// Per-tile metadata, wave-uniform: dense copy index (-1 if none) and the entry range.
struct TileMeta {
    int d, eb, ee;
};

__device__ __forceinline__ TileMeta tile_meta(int c, const int* __restrict__ chunk_dense,
                                              const int* __restrict__ chunk_eptr) {
    return TileMeta{chunk_dense[c], chunk_eptr[c], chunk_eptr[c + 1]};
}

// A sparse tile holds at most kDenseMin entries, three per lane.
static_assert(kDenseMin <= 3 * 64, "a sparse tile must fit three entries per lane");

// A state of an FP16 tile in four words per lane: the dense operand (8 halves), or this lane's
// entries eb + lane, eb + 64 + lane, eb + 128 + lane (addresses clamped into the tile, so the
// four loads are always issued; the scatter skips the ones past ee).
__device__ __forceinline__ uint4 load_a16(const TileMeta& m, int lane, int a_off,
                                          const uint32_t* __restrict__ entries,
                                          const _Float16* __restrict__ dense_a) {
    const uint32_t *p0, *p1, *p2, *p3;
    if (m.d >= 0) {
        const uint32_t* base =
            reinterpret_cast<const uint32_t*>(dense_a + (long long)m.d * 512 + a_off);
        p0 = base; p1 = base + 1; p2 = base + 2; p3 = base + 3;
    } else {
        const int last = m.ee - 1;
        p0 = entries + min(m.eb + lane, last);
        p1 = entries + min(m.eb + 64 + lane, last);
        p2 = entries + min(m.eb + 128 + lane, last);
        p3 = p2;
    }
    return uint4{*p0, *p1, *p2, *p3};
}

// Schedule of a 4-wave work-group.  Work-groups [0, H8) run the heavy units (H8 = num_heavy
// rounded up to a multiple of 8): the four waves share one unit's tiles.  The others run light
// units, one per wave, mapped so that each XCD walks a contiguous range of them (work-groups
// are dealt to the 8 XCDs round robin).  Returns false if this wave has nothing to do.
__device__ __forceinline__ bool schedule(int num_units, int num_heavy, int wave, int& u,
                                         bool& heavy) {
    const int h8 = (num_heavy + 7) & ~7;
    const int b = blockIdx.x;
    if (b < h8) {
        heavy = true;
        u = b;
        return b < num_heavy;
    }
    heavy = false;
    const int nlw = (num_units - num_heavy + kWaves - 1) / kWaves;
    const int j = unit_of_block(b - h8, nlw);
    u = num_heavy + j * kWaves + wave;
    return j < nlw && u < num_units;
}

// One FP16 tile: A operand (dense words, or the entries scattered into the wave's LDS tile),
// then VEC MFMAs against the B rows.
template <int VEC, typename TB>
__device__ __forceinline__ void mma_tile_f16(const TileMeta& m, const uint4& st, int lane,
                                             _Float16* Aw, _Float16* my_a, const BRows<VEC, TB>& R,
                                             floatx4 (&acc)[VEC]) {
    half8 a;
    if (m.d >= 0) {
        a = __builtin_bit_cast(half8, st);
    } else {
        *reinterpret_cast<half8*>(my_a) = half8{0, 0, 0, 0, 0, 0, 0, 0};
        wave_lds_sync();
        if (m.eb + lane < m.ee) scatter_a_f16(Aw, st.x);
        if (m.eb + 64 + lane < m.ee) scatter_a_f16(Aw, st.y);
        if (m.eb + 128 + lane < m.ee) scatter_a_f16(Aw, st.z);
        wave_lds_sync();
        a = *reinterpret_cast<const half8*>(my_a);
        wave_lds_sync();
    }
#pragma unroll
    for (int q = 0; q < VEC; ++q) {
        const half8 b = half8{(_Float16)R.r[0][q], (_Float16)R.r[1][q], (_Float16)R.r[2][q],
                              (_Float16)R.r[3][q], (_Float16)R.r[4][q], (_Float16)R.r[5][q],
                              (_Float16)R.r[6][q], (_Float16)R.r[7][q]};
        acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[q], 0, 0, 0);
    }
}

// FP16 tiles first, first + W, ... < end of one unit (wave-uniform indices), accumulated into
// acc.  While tile c is multiplied, the B rows and A state of the wave's next tile and the
// column indices of the tile after are in flight.  Three rules keep the prefetch effective
// (vector loads complete in issue order, and a wait names a count of younger loads):
//   * the loop is unrolled by two over fixed buffers A and B, so no register that a load is
//     still filling is ever copied (a copy would wait for the load);
//   * column indices are loaded before the B rows and A state they lead to, so waiting for
//     them does not wait for those;
//   * every iteration issues the same loads (column indices past the last tile are clamped).
template <int TK, typename TB, bool ALIGNED>
__device__ __forceinline__ void tiles_f16(int first, int end, int W, int lane, int n, int g,
                                          int c0, long long OL, const int* __restrict__ chunk_eptr,
                                          const int* __restrict__ chunk_cols,
                                          const int* __restrict__ chunk_dense,
                                          const uint32_t* __restrict__ entries,
                                          const _Float16* __restrict__ dense_a,
                                          const TB* __restrict__ B, _Float16* Aw,
                                          floatx4 (&acc)[TK / 16]) {
    constexpr int VEC = TK / 16;
    if (first >= end) return;
    const int a_off = n * 32 + 8 * g;  // this lane's A operand inside a dense tile
    _Float16* my_a = &Aw[n * kApitch + 8 * g];
    const int last = first + (end - 1 - first) / W * W;
    int c = first;
    BRows<VEC, TB> RA, RB;
    int colsA[8], colsB[8];
    TileMeta mA = tile_meta(c, chunk_dense, chunk_eptr);
    load_cols8(chunk_cols, c, g, colsA);
    const int c1 = min(c + W, last);
    load_cols8(chunk_cols, c1, g, colsB);
    TileMeta mB = tile_meta(c1, chunk_dense, chunk_eptr);
    load_b_rows<VEC, TB, ALIGNED>(B, colsA, OL, c0, RA);
    uint4 sA = load_a16(mA, lane, a_off, entries, dense_a);
    uint4 sB;
    // Invariant at the top: tile c in A (B rows, A state, metadata), the column indices and
    // metadata of tile c + W in B; at least three tiles c, c + W, c + 2 W remain.
    for (; c + W < last; c += 2 * W) {
        load_cols8(chunk_cols, c + 2 * W, g, colsA);
        const TileMeta mA2 = tile_meta(c + 2 * W, chunk_dense, chunk_eptr);
        load_b_rows<VEC, TB, ALIGNED>(B, colsB, OL, c0, RB);
        sB = load_a16(mB, lane, a_off, entries, dense_a);
        mma_tile_f16<VEC, TB>(mA, sA, lane, Aw, my_a, RA, acc);

        const int c3 = min(c + 3 * W, last);
        load_cols8(chunk_cols, c3, g, colsB);
        const TileMeta mB2 = tile_meta(c3, chunk_dense, chunk_eptr);
        load_b_rows<VEC, TB, ALIGNED>(B, colsA, OL, c0, RA);
        sA = load_a16(mA2, lane, a_off, entries, dense_a);
        mma_tile_f16<VEC, TB>(mB, sB, lane, Aw, my_a, RB, acc);
        mA = mA2;
        mB = mB2;
    }
    if (c < last) {  // two tiles left: c and c + W = last
        load_b_rows<VEC, TB, ALIGNED>(B, colsB, OL, c0, RB);
        sB = load_a16(mB, lane, a_off, entries, dense_a);
        mma_tile_f16<VEC, TB>(mA, sA, lane, Aw, my_a, RA, acc);
        mma_tile_f16<VEC, TB>(mB, sB, lane, Aw, my_a, RB, acc);
    } else {
        mma_tile_f16<VEC, TB>(mA, sA, lane, Aw, my_a, RA, acc);
    }
}

// Register budget: FP16 B with aligned rows fits three waves per SIMD without spilling; the
// FP32-B and unaligned variants hold more B data and are given two.
template <typename TB, bool ALIGNED>
constexpr int f16_min_waves() { return (sizeof(TB) == 2 && ALIGNED) ? 3 : 2; }

template <int TK, typename TB, bool ALIGNED>
__global__ __launch_bounds__(64 * kWaves, (f16_min_waves<TB, ALIGNED>())) void k_spmm_f16(
    const int4* __restrict__ units, int num_units, int num_heavy,
    const int* __restrict__ chunk_eptr, const int* __restrict__ chunk_cols,
    const int* __restrict__ chunk_dense, const uint32_t* __restrict__ entries,
    const _Float16* __restrict__ dense_a, const TB* __restrict__ B, int O, float scale, bool c4,
    float* __restrict__ C) {
    constexpr int VEC = TK / 16;
    __shared__ __attribute__((aligned(16))) _Float16 As[kWaves][16 * kApitch];
    __shared__ __attribute__((aligned(16))) float P[kWaves * 16 * TK];
    // The wave index is uniform across the wave: readfirstlane lets the compiler keep the unit
    // and tile indices in scalar registers and fetch tile metadata with scalar loads.
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    int u;
    bool heavy;
    if (!schedule(num_units, num_heavy, wave, u, heavy)) return;
    const int4 U = units[u];
    const int k0 = blockIdx.y * TK;
    const int c0 = k0 + VEC * n;
    floatx4 acc[VEC];
#pragma unroll
    for (int q = 0; q < VEC; ++q) acc[q] = floatx4{0.f, 0.f, 0.f, 0.f};
    tiles_f16<TK, TB, ALIGNED>(heavy ? U.y + wave : U.y, U.z, heavy ? kWaves : 1, lane, n, g, c0,
                               (long long)O, chunk_eptr, chunk_cols, chunk_dense, entries, dense_a,
                               B, As[wave], acc);
    if (heavy) merge_into_c<TK, kWaves>(acc, scale, U, k0, O, c4, C, P);
    else merge_into_c<TK, 1>(acc, scale, U, k0, O, c4, C, P);
}

// FP32 format: eight K steps of v_mfma_f32_16x16x4_f32 per tile; lane (n, g) feeds tile
// columns k = 4s + g (s = 0..7).  The A tile (LDS or dense copy) is K-step-major so a lane's 8
// values are contiguous: [(k & 3) * 128 + row * 8 + (k >> 2)].  B is fetched in half tiles
// (steps 0-3, then 4-7) so one half is in flight while the other is multiplied.
template <int VEC>
struct FRows {
    float v[4][VEC];
};

template <int VEC, bool ALIGNED>
__device__ __forceinline__ void load_b_half_f32(const float* __restrict__ B, const int* cols,
                                                long long O, int c0, FRows<VEC>& R) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int col = cols[s];
        const float* src = B + (long long)(col < 0 ? 0 : col) * O + c0;
        if constexpr (ALIGNED && VEC >= 4) {
            const bool ok = col >= 0 && c0 < O;
#pragma unroll
            for (int h = 0; h < VEC; h += 4) {
                floatx4 x = {0.f, 0.f, 0.f, 0.f};
                if (ok) x = *reinterpret_cast<const floatx4*>(src + h);
#pragma unroll
                for (int q = 0; q < 4; ++q) R.v[s][h + q] = x[q];
            }
        } else {
#pragma unroll
            for (int q = 0; q < VEC; ++q) R.v[s][q] = (col >= 0 && c0 + q < O) ? src[q] : 0.0f;
        }
    }
}

__device__ __forceinline__ void load_cols_steps(const int* __restrict__ chunk_cols, int c, int g,
                                                int (&cols)[8]) {
    const int* cc = chunk_cols + (long long)c * kChunkCols;
#pragma unroll
    for (int s = 0; s < 8; ++s) cols[s] = cc[4 * s + g];
}

template <int VEC>
__device__ __forceinline__ void mfma_half_f32(const float (&a)[8], int s0, const int (&cols)[8],
                                              const FRows<VEC>& R, floatx4 (&acc)[VEC]) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        if (__ballot(cols[s0 + s] >= 0) == 0) return;  // padding columns end a tile
#pragma unroll
        for (int q = 0; q < VEC; ++q)
            acc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s0 + s], R.v[s][q], acc[q], 0, 0, 0);
    }
}

// A state of an FP32 tile in 8 registers: the dense operand (8 floats), or the first two
// nonzeros of this lane (entry words, values) and the tile's entry range.
struct AState32 {
    uint4 x, y;
};

__device__ __forceinline__ AState32 load_a_state32(int d, int c, int lane, int a_off,
                                                   const int* __restrict__ chunk_eptr,
                                                   const uint32_t* __restrict__ entries,
                                                   const float* __restrict__ evals,
                                                   const float* __restrict__ dense_a) {
    AState32 s;
    if (d >= 0) {
        s.x = *reinterpret_cast<const uint4*>(dense_a + (long long)d * 512 + a_off);
        s.y = *reinterpret_cast<const uint4*>(dense_a + (long long)d * 512 + a_off + 4);
        return s;
    }
    const int eb = chunk_eptr[c], ee = chunk_eptr[c + 1];
    s.x = {0u, 0u, 0u, 0u};
    s.y = {(unsigned)eb, (unsigned)ee, 0u, 0u};
    if (eb + lane < ee) { s.x.x = entries[eb + lane]; s.x.z = __float_as_uint(evals[eb + lane]); }
    if (eb + 64 + lane < ee) {
        s.x.y = entries[eb + 64 + lane];
        s.x.w = __float_as_uint(evals[eb + 64 + lane]);
    }
    return s;
}

__device__ __forceinline__ void scatter_a_f32(float* At, uint32_t w, float v) {
    const int r = w & 15, k = (w >> 4) & 31;
    At[(k & 3) * 128 + r * 8 + (k >> 2)] = v;
}

template <int TK, bool ALIGNED>
__device__ __forceinline__ void tiles_f32(int first, int end, int W, int lane, int n, int g,
                                          int c0, long long OL, const int* __restrict__ chunk_eptr,
                                          const int* __restrict__ chunk_cols,
                                          const int* __restrict__ chunk_dense,
                                          const uint32_t* __restrict__ entries,
                                          const float* __restrict__ evals,
                                          const float* __restrict__ dense_a,
                                          const float* __restrict__ B, float* Aw,
                                          floatx4 (&acc)[TK / 16]) {
    constexpr int VEC = TK / 16;
    const int a_off = g * 128 + n * 8;
    float* my_a = &Aw[a_off];
    int c = first;
    if (c < end) {
        int cols[8], cols_next[8];
        FRows<VEC> R0, R1;
        load_cols_steps(chunk_cols, c, g, cols);
        load_b_half_f32<VEC, ALIGNED>(B, cols, OL, c0, R0);
        int d_next = -1;
        if (c + W < end) {
            load_cols_steps(chunk_cols, c + W, g, cols_next);
            d_next = chunk_dense[c + W];
        }
        int d = chunk_dense[c];
        AState32 cur = load_a_state32(d, c, lane, a_off, chunk_eptr, entries, evals, dense_a);
        for (; c < end; c += W) {
            const bool has1 = c + W < end;
            load_b_half_f32<VEC, ALIGNED>(B, cols + 4, OL, c0, R1);
            AState32 nxt = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
            if (has1) nxt = load_a_state32(d_next, c + W, lane, a_off, chunk_eptr, entries, evals,
                                           dense_a);
            floatx4 a_lo, a_hi;
            if (d >= 0) {
                a_lo = __builtin_bit_cast(floatx4, cur.x);
                a_hi = __builtin_bit_cast(floatx4, cur.y);
            } else {
                const int eb = (int)cur.y.x, ee = (int)cur.y.y;
                *reinterpret_cast<floatx4*>(my_a) = floatx4{0.f, 0.f, 0.f, 0.f};
                *reinterpret_cast<floatx4*>(my_a + 4) = floatx4{0.f, 0.f, 0.f, 0.f};
                wave_lds_sync();
                if (eb + lane < ee) scatter_a_f32(Aw, cur.x.x, __uint_as_float(cur.x.z));
                if (eb + 64 + lane < ee) scatter_a_f32(Aw, cur.x.y, __uint_as_float(cur.x.w));
                for (int e = eb + 128 + lane; e < ee; e += 64) scatter_a_f32(Aw, entries[e], evals[e]);
                wave_lds_sync();
                a_lo = *reinterpret_cast<const floatx4*>(my_a);
                a_hi = *reinterpret_cast<const floatx4*>(my_a + 4);
                wave_lds_sync();
            }
            const float a[8] = {a_lo[0], a_lo[1], a_lo[2], a_lo[3],
                                a_hi[0], a_hi[1], a_hi[2], a_hi[3]};
            mfma_half_f32<VEC>(a, 0, cols, R0, acc);
            int cols_after[8];
            int d_after = -1;
            if (has1) {
                load_b_half_f32<VEC, ALIGNED>(B, cols_next, OL, c0, R0);
                if (c + 2 * W < end) {
                    load_cols_steps(chunk_cols, c + 2 * W, g, cols_after);
                    d_after = chunk_dense[c + 2 * W];
                }
            }
            mfma_half_f32<VEC>(a, 4, cols, R1, acc);
            if (has1) {
#pragma unroll
                for (int i = 0; i < 8; ++i) { cols[i] = cols_next[i]; cols_next[i] = cols_after[i]; }
                d = d_next;
                d_next = d_after;
                cur = nxt;
            }
        }
    }
}

// Sparse FP32 panel on VALU: rows [r_first, r_first + r_count) of the panel, one row at a time
// from the CSR.  Lane l owns CPL consecutive output columns k0 + CPL l (CPL = 2 at tileK = 128),
// so every nonzero is one coalesced load of its B row slice plus CPL FMAs; the column index and
// value are wave-uniform (scalar loads).  The row is added to C once; rows outside the mask
// are skipped.
template <int TK, bool ALIGNED>
__device__ __forceinline__ void rows_f32_valu(const int4& U, int r_first, int r_count, int lane,
                                              int k0, int O, const int* __restrict__ rp,
                                              const int* __restrict__ col,
                                              const float* __restrict__ val,
                                              const float* __restrict__ B, float* __restrict__ C) {
    constexpr int CPL = TK >= 64 ? TK / 64 : 1;
    const int cc = k0 + CPL * lane;
    const bool active = (TK >= 64 || lane < TK) && cc < O;
    const long long OL = O;
    const bool vec = ALIGNED && CPL == 2 && cc + 1 < O;
    for (int rl = r_first; rl < r_first + r_count; ++rl) {
        if (!((U.w >> rl) & 1)) continue;
        const int r = U.x + rl;
        const int p0 = rp[r], p1 = rp[r + 1];
        float acc[CPL];
#pragma unroll
        for (int q = 0; q < CPL; ++q) acc[q] = 0.0f;
        auto fma_row = [&](int c, float v) {
            const float* src = B + (long long)c * OL + cc;
            if (vec) {
                const float2 b = *reinterpret_cast<const float2*>(src);
                acc[0] += v * b.x;
                acc[CPL - 1] += v * b.y;
            } else {
#pragma unroll
                for (int q = 0; q < CPL; ++q)
                    if (cc + q < O) acc[q] += v * src[q];
            }
        };
        int p = p0;
        if (active) {
            for (; p + 4 <= p1; p += 4) {
                const int ca = col[p], cb = col[p + 1], ccx = col[p + 2], cd = col[p + 3];
                const float va = val[p], vb = val[p + 1], vc = val[p + 2], vd = val[p + 3];
                fma_row(ca, va);
                fma_row(cb, vb);
                fma_row(ccx, vc);
                fma_row(cd, vd);
            }
            for (; p < p1; ++p) fma_row(col[p], val[p]);
            float* crow = C + (long long)r * OL + cc;
            if (vec) {
                float2 cv = *reinterpret_cast<float2*>(crow);
                cv.x += acc[0];
                cv.y += acc[CPL - 1];
                *reinterpret_cast<float2*>(crow) = cv;
            } else {
#pragma unroll
                for (int q = 0; q < CPL; ++q)
                    if (cc + q < O) crow[q] += acc[q];
            }
        }
    }
}

template <int TK, bool ALIGNED>
__global__ __launch_bounds__(64 * kWaves, 3) void k_spmm_f32(
    const int4* __restrict__ units, int num_units, int num_heavy,
    const int* __restrict__ chunk_eptr, const int* __restrict__ chunk_cols,
    const int* __restrict__ chunk_dense, const uint32_t* __restrict__ entries,
    const float* __restrict__ evals, const float* __restrict__ dense_a,
    const int* __restrict__ csr_rp, const int* __restrict__ csr_col,
    const float* __restrict__ csr_val, const float* __restrict__ B, int O, bool c4,
    float* __restrict__ C) {
    constexpr int VEC = TK / 16;
    __shared__ __attribute__((aligned(16))) float At[kWaves][4 * 16 * 8];
    __shared__ __attribute__((aligned(16))) float P[kWaves * 16 * TK];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    int u;
    bool heavy;
    if (!schedule(num_units, num_heavy, wave, u, heavy)) return;
    const int4 U = units[u];
    const int k0 = blockIdx.y * TK;
    if ((U.w >> 17) & 1) {  // sparse panel: VALU over its rows (a heavy one: 4 rows per wave)
        rows_f32_valu<TK, ALIGNED>(U, heavy ? 4 * wave : 0, heavy ? 4 : 16, lane, k0, O, csr_rp,
                                   csr_col, csr_val, B, C);
        return;
    }
    const int c0 = k0 + VEC * n;
    floatx4 acc[VEC];
#pragma unroll
    for (int q = 0; q < VEC; ++q) acc[q] = floatx4{0.f, 0.f, 0.f, 0.f};
    tiles_f32<TK, ALIGNED>(heavy ? U.y + wave : U.y, U.z, heavy ? kWaves : 1, lane, n, g, c0,
                           (long long)O, chunk_eptr, chunk_cols, chunk_dense, entries, evals,
                           dense_a, B, At[wave], acc);
    if (heavy) merge_into_c<TK, kWaves>(acc, 1.0f, U, k0, O, c4, C, P);
    else merge_into_c<TK, 1>(acc, 1.0f, U, k0, O, c4, C, P);
}

template <int TK>
static void launch_tk(const DeviceFormat& F, const void* dB, bool b_f16, int O, float* dC,
                      hipStream_t st) {
    constexpr int VEC = TK / 16;
    // Vector loads of B need O % VEC == 0 and a 16-byte aligned base.
    const bool aligned = (O % VEC) == 0 && ((uintptr_t)dB % 16) == 0;
    const bool c4 = (O % 4) == 0 && ((uintptr_t)dC % 16) == 0;
    const int h8 = (F.num_heavy + 7) & ~7;
    const int nlw = (F.num_units - F.num_heavy + kWaves - 1) / kWaves;
    const dim3 grid((unsigned)(h8 + 8 * ((nlw + 7) / 8)), (unsigned)((O + TK - 1) / TK));
    const dim3 block(64 * kWaves);
    const int NU = F.num_units, NH = F.num_heavy;
    if (F.fp32) {
        const float* B = static_cast<const float*>(dB);
        if (aligned)
            hipLaunchKernelGGL((k_spmm_f32<TK, true>), grid, block, 0, st, F.units.p, NU, NH,
                               F.chunk_eptr.p, F.chunk_cols.p, F.chunk_dense.p, F.entries.p,
                               F.evals.p, F.dense_a32.p, F.csr_rp.p, F.csr_col.p, F.csr_val.p, B,
                               O, c4, dC);
        else
            hipLaunchKernelGGL((k_spmm_f32<TK, false>), grid, block, 0, st, F.units.p, NU, NH,
                               F.chunk_eptr.p, F.chunk_cols.p, F.chunk_dense.p, F.entries.p,
                               F.evals.p, F.dense_a32.p, F.csr_rp.p, F.csr_col.p, F.csr_val.p, B,
                               O, c4, dC);
    } else if (b_f16) {
        const _Float16* B = static_cast<const _Float16*>(dB);
        if (aligned)
            hipLaunchKernelGGL((k_spmm_f16<TK, _Float16, true>), grid, block, 0, st, F.units.p, NU,
                               NH, F.chunk_eptr.p, F.chunk_cols.p, F.chunk_dense.p, F.entries.p,
                               F.dense_a16.p, B, O, F.scale, c4, dC);
        else
            hipLaunchKernelGGL((k_spmm_f16<TK, _Float16, false>), grid, block, 0, st, F.units.p, NU,
                               NH, F.chunk_eptr.p, F.chunk_cols.p, F.chunk_dense.p, F.entries.p,
                               F.dense_a16.p, B, O, F.scale, c4, dC);
    } else {
        const float* B = static_cast<const float*>(dB);
        if (aligned)
            hipLaunchKernelGGL((k_spmm_f16<TK, float, true>), grid, block, 0, st, F.units.p, NU,
                               NH, F.chunk_eptr.p, F.chunk_cols.p, F.chunk_dense.p, F.entries.p,
                               F.dense_a16.p, B, O, F.scale, c4, dC);
        else
            hipLaunchKernelGGL((k_spmm_f16<TK, float, false>), grid, block, 0, st, F.units.p, NU,
                               NH, F.chunk_eptr.p, F.chunk_cols.p, F.chunk_dense.p, F.entries.p,
                               F.dense_a16.p, B, O, F.scale, c4, dC);
    }
    VCSRMC_HIP(hipGetLastError());
}

void spmm_launch(const DeviceFormat& F, const void* dB, bool b_f16, int O, int tileK, float* dC,
                 hipStream_t st) {
    if (tileK != 16 && tileK != 32 && tileK != 64 && tileK != 128)
        throw Error(VCSRMC_ERR_TILEK, "vcsr_mc supports tileK in {16, 32, 64, 128}");
    if (!F.ready) throw Error(VCSRMC_ERR_STATE, "no format in this handle");
    if (O < 0) throw Error(VCSRMC_ERR_ARG, "O must be >= 0");
    if (F.fp32 && b_f16) throw Error(VCSRMC_ERR_ARG, "an FP32 format takes an FP32 B");
    if (F.num_units == 0 || O == 0) return;
    if (!dB || !dC) throw Error(VCSRMC_ERR_ARG, "null B or C");
    switch (tileK) {
        case 16: launch_tk<16>(F, dB, b_f16, O, dC, st); break;
        case 32: launch_tk<32>(F, dB, b_f16, O, dC, st); break;
        case 64: launch_tk<64>(F, dB, b_f16, O, dC, st); break;
        default: launch_tk<128>(F, dB, b_f16, O, dC, st); break;
    }
}

}  // namespace vcsrmc
