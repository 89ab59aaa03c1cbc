// spmm_kernels.hip -- C += A.B for the VCSR-MC format on gfx950 MFMA.
//
// Work decomposition (atomic-free for all but split panels):
//   a work unit is a run of compacted tiles of one 16-row panel (16 consecutive rows, or the
//   16 rows the layout's row map groups), for one tileK-wide slice of
//   the output columns.  A light unit is one 64-lane wave, which keeps the 16 x tileK
//   accumulator tile in registers across its tiles and writes C once; a heavy unit is shared by
//   the four waves of a work-group, which take its tiles round robin and sum their partial tiles
//   in LDS before writing C.  Panels cut into several heavy units (split) merge through atomics.
//   Work-groups are dealt to the 8 XCDs round robin; `schedule` maps each one to its units so
//   that an XCD walks neighbouring panels and, when there are several output slices, only its
//   slice of B.
//
// Per 16 x 32 tile (32 distinct columns of the panel, any segments):
//   * B operand: lane (n = lane % 16, g = lane / 16) loads, for the 8 tile columns
//     k = 8g .. 8g+7, the contiguous VEC = tileK/16 output columns k0 + VEC n .. +VEC-1 of
//     that B row (one 128-bit load per row at tileK = 128, FP16 B); 16 lanes cover a
//     256-byte B row, so every load instruction reads four whole rows.  The VEC values are
//     then transposed in registers: MFMA q (q < VEC) takes the q-th value of each of the 8
//     rows, i.e. output column k0 + VEC n + q.  No LDS round trip for B.
//   * A operand: a well-filled tile has a dense copy laid out in the order lanes read it (one
//     load per lane); otherwise the tile's nonzeros (row, k, value) are scattered into a
//     16 x 32 LDS tile that each lane then reads as its 8 contiguous K values.
//   * FP16 format: v_mfma_f32_16x16x32_f16, FP32 accumulation.  FP32 format: eight K steps
//     of v_mfma_f32_16x16x4_f32, in two halves.
//   The K order inside a tile is the same for A and B, so the contraction does not depend
//   on how the instruction maps lanes to K.
// FP32 panels whose rows rarely share a column run batches of 8 row steps instead of tiles
// (units flagged kUnitRowSteps): v_mfma_f32_4x4x1_16b_f32 with its 16 blocks as 4 row groups x
// 4 groups of output columns, each row group at its own column per step, a quarter of the
// cycles of a 16x16x4 step.  Lane group g loads the 8 step columns of row group g exactly as it
// loads 8 tile columns, and the accumulators end where the tile path leaves them.
//
// Epilogue: lane (n, g) holds rows 4g..4g+3 at output columns k0 + VEC n .. + VEC-1, so each
// row is written as VEC contiguous floats per lane, 16 lanes per row: coalesced.  Rows that
// A does not touch are not written (the reference never touches them either).
#include <vector>

#include "../../include/vcsrmc.h"
#include "internal.hpp"

namespace vcsrmc {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kApitch = 40;  // FP16 A tile row pitch in halves (80 B: conflict-free b128 reads)
// FP32 A tile in LDS: four K groups (k & 3) of 16 rows, each row the 8 values k >> 2 a lane
// reads with two 128-bit loads.  A row pitch of 12 floats (48 B) puts the 16 rows of a group on
// 16 distinct 16-byte bank windows (48 n mod 256 covers every multiple of 16), where a pitch of
// 8 made rows n and n + 8 collide.
constexpr int kApitch32 = 12;
constexpr int kAgroup32 = 16 * kApitch32;

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

// The C rows of a unit's 16 panel rows: U.x .. U.x + 15 for a layout in natural row order;
// for a layout with a row map (MAPPED), rmap[U.x + r], which lane r loads once per unit and
// row() reads across lanes -- so every lane of the wave executes row() together, outside
// branches that depend on the lane.  MAPPED is a kernel template parameter: with a run-time
// flag the natural-order kernels still paid for the cross-lane reads (power-law 36,692^2
// 15.0 -> 15.6 us).
template <bool MAPPED>
struct PanelRows {
    int base;  // U.x
    int mine;  // MAPPED: the C row of panel row (lane & 15)
    __device__ __forceinline__ long long row(int r) const {
        if constexpr (MAPPED) return (long long)__shfl(mine, r);
        else return (long long)(base + r);
    }
};

template <bool MAPPED>
__device__ __forceinline__ PanelRows<MAPPED> panel_rows(const int4& U,
                                                        const int* __restrict__ rmap) {
    PanelRows<MAPPED> p;
    p.base = U.x;
    if constexpr (MAPPED) p.mine = rmap[U.x + (threadIdx.x & 15)];
    else p.mine = 0;
    return p;
}

// C of a unit's output tile, read ahead of the merge (C += A.B needs it) so that its latency
// overlaps the tile loop.  W == 1 (light): just before the wave's last tile is multiplied; for a
// whole, aligned, unsplit tile (the staged merge below) lane l reads the float4s at l*4 + 256 j of
// the 16 x TK tile, row-major; otherwise lane (n, g) reads rows 4g..4g+3 at columns
// k0 + VEC n .. + VEC - 1 (VEC / 4 float4 per row).  W > 1 (heavy): thread t reads the float4 at
// t*4 + 256 W j of the tile when the unit starts.  The loads are always issued -- rows outside
// the mask, split panels, unaligned C, columns past O and overwriting launches read kZeroRow
// instead -- so their number is fixed and a wait for an older load never has to cover them.
template <int TK, int W>
struct CAhead {
    static constexpr int VEC = TK / 16;
    static constexpr int N = W == 1 ? TK / 16 : (16 * TK + 256 * W - 1) / (256 * W);
    floatx4 v[N > 0 ? N : 1];
};

// Sixteen bytes of C read ahead: an ordinary load, or (NT) a non-temporal one, which neither L2
// nor the last-level cache keeps.  Where C is larger than that cache can hold with B, ordinary
// reads of C only evict the B rows and layout that later units reuse; where it fits (power-law
// 36,692^2 at O = 128: 19 MB), back-to-back launches find C there.  Measured on gfx950, C += A.B
// back to back, ordinary -> non-temporal: 32 x 32 blocks, 262,144^2 at O = 256, FP16 180 ->
// 163 us, FP32 269 -> 254 us; 27-point stencil 100^3 FP32 426 -> 410 us; R-MAT scale 22 2.48
// -> 2.42 ms; power-law 15.9 -> 17.4 us.  (NT is a template parameter: the compiler merges a
// load whose kind a run-time flag selects into one ordinary load.)
template <bool NT>
__device__ __forceinline__ floatx4 load_c4(const float* p) {
    if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(p));
    else return *reinterpret_cast<const floatx4*>(p);
}

template <int TK, int W, bool NT = false, typename PR>
__device__ __forceinline__ void read_c_ahead(CAhead<TK, W>& ca, const int4& U,
                                             const PR& pr, int k0, int O, bool c4,
                                             bool accumulate, const float* __restrict__ C) {
    constexpr int VEC = TK / 16;
    constexpr int N = CAhead<TK, W>::N;
    const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    // Overwrite launches (C = A.B) read zeros instead of C; split panels merge through atomics.
    const bool ok = c4 && accumulate && !(U.w & kUnitSplit);
    const long long OL = O;
    if constexpr (W == 1) {
        if (c4 && !(U.w & kUnitSplit) && k0 + TK <= O) {
            // staged merge: lane-contiguous 16-byte pieces, as merge_into_c writes them back
#pragma unroll
            for (int j = 0; j < N; ++j) {
                const int e = lane * 4 + 256 * j;
                const int row = e / TK, col = e % TK;
                const long long cr = pr.row(row);
                const bool in = accumulate && ((U.w >> row) & 1);
                const float* src = in ? C + cr * OL + k0 + col : kZeroRow;
                ca.v[j] = load_c4<NT>(src);
            }
        } else if constexpr (VEC >= 4) {
            const int c0 = k0 + VEC * n;
            const bool lane_ok = ok && c0 + VEC <= O;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int rl = 4 * g + i;
                const long long cr = pr.row(rl);
                const bool in = lane_ok && ((U.w >> rl) & 1);
                const float* src = in ? C + cr * OL + c0 : kZeroRow;
#pragma unroll
                for (int h = 0; h < VEC / 4; ++h)
                    ca.v[i * (VEC / 4) + h] = load_c4<NT>(src + 4 * h);
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const int e = threadIdx.x * 4 + j * 256 * W;
            const int row = (e / TK) & 15, cc = k0 + e % TK;
            const long long cr = pr.row(row);
            const bool in = ok && e < 16 * TK && ((U.w >> row) & 1) && cc + 4 <= O;
            const float* src = in ? C + cr * OL + cc : kZeroRow;
            ca.v[j] = load_c4<NT>(src);
        }
    }
}

// Four floats of C: an ordinary store (ACC) or one that bypasses the caches (non-temporal), so
// that C does not evict the B rows other panels reuse.  Non-temporal stores are not combined in
// L2, so they are used where each store instruction covers whole lines (the staged merge).
// (ACC is a template parameter of the kernels: with a run-time flag the compiler merged the two
// stores into one ordinary store.)
template <bool ACC>
__device__ __forceinline__ void store_c4(float* p, const floatx4& v) {
    if constexpr (ACC) *reinterpret_cast<floatx4*>(p) = v;
    else __builtin_nontemporal_store(v, reinterpret_cast<floatx4*>(p));
}

// Parks a wave's 16 x TK tile row-major in P (row pitch TK floats): lane (n, g) holds rows
// 4g..4g+3 at columns VEC n .. VEC n + VEC - 1, written as 16-byte pieces.  The LDS serves 128
// bytes per cycle over 32 four-byte banks, so a ds_write_b128 runs 8 lanes at a time (measured
// on gfx950 with rocprofv3's SQ_LDS_BANK_CONFLICT: contiguous 16-byte pieces count no conflict,
// pieces 32 bytes apart one conflict cycle per cycle, a 32-bit access of 64 lanes on one bank 31
// per cycle).  At VEC = 8 the 8 lanes n = 0..7 of a row would write dword offsets 8n + 4h:
// lanes n and n + 4 on the same four banks.  Lanes with n & 4 therefore write their two pieces
// in the other order, and each 8-lane pass covers all 32 banks once; the layout, and so the
// contiguous reads of the merge, are unchanged.  (At VEC = 4 a pass is already conflict-free.)
template <int TK>
__device__ __forceinline__ void park_tile(float* Pw, const floatx4 (&acc)[TK / 16], float scale,
                                          int n, int g) {
    constexpr int VEC = TK / 16;
    if constexpr (VEC == 8) {
        const bool sw = (n & 4) != 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const floatx4 lo = floatx4{acc[0][i], acc[1][i], acc[2][i], acc[3][i]} * scale;
            const floatx4 hi = floatx4{acc[4][i], acc[5][i], acc[6][i], acc[7][i]} * scale;
            float* row = Pw + (4 * g + i) * TK + VEC * n;
            *reinterpret_cast<floatx4*>(row + (sw ? 4 : 0)) = sw ? hi : lo;
            *reinterpret_cast<floatx4*>(row + (sw ? 0 : 4)) = sw ? lo : hi;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int q = 0; q < VEC; ++q) Pw[(4 * g + i) * TK + VEC * n + q] = acc[q][i] * scale;
    }
}

// Adds the unit's 16 x TK result into C (ACC) or writes it (overwrite).  W == 1, staged merge
// (a whole, aligned tile of an unsplit panel): the wave parks its tile in its slice of P (lane
// (n, g) owns rows 4g..4g+3, columns k0 + VEC n .. + VEC - 1), reads it back with consecutive
// lanes on consecutive 16-byte pieces, adds the C read ahead in that order, and stores each run of
// 1 KB non-temporally.  From the accumulators, one store instruction covered every other 16
// bytes of a row at O tiles of 128, which non-temporal stores turned into 1.5x the C bytes.
// Measured on gfx950 against the register epilogue with ordinary stores: overwrite power-law
// 36,692^2 14.4 -> 12.8 us, 32 x 32 blocks 174 -> 140 us, 27-point stencil 543 -> 508 us, R-MAT
// scale 22 2.46 -> 2.38 ms; accumulate blocks 189 -> 178 us, stencil 584 -> 565 us, the others
// within 1%.  Other W == 1 tiles: straight from the accumulators.  W > 1: every wave parks its
// partial tile in LDS, then the work-group sums the W partials and writes each row with
// consecutive threads on consecutive columns.  Split panels merge through atomics; other rows
// are a read-modify-write (C += A.B) whose read came from read_c_ahead.  Rows outside the
// panel's row mask are never touched.
template <int TK, int W, bool ACC, typename PR>
__device__ __forceinline__ void merge_into_c(const floatx4 (&acc)[TK / 16], float scale,
                                             const int4& U, const PR& pr, int k0, int O,
                                             bool c4, float* __restrict__ C, float* P,
                                             const CAhead<TK, W>& ca) {
    constexpr int VEC = TK / 16;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n = lane & 15, g = lane >> 4;
    const bool split = U.w & kUnitSplit;
    const long long OL = O;
    if constexpr (W == 1) {
        if (!split && c4 && k0 + TK <= O) {  // staged merge
            park_tile<TK>(P + wave * 16 * TK, acc, scale, n, g);
            wave_lds_sync();
            const float* Pw = P + wave * 16 * TK;
#pragma unroll
            for (int j = 0; j < 16 * TK / 256; ++j) {
                const int e = lane * 4 + 256 * j;
                const int row = e / TK, col = e % TK;
                const long long cr = pr.row(row);
                floatx4 v = *reinterpret_cast<const floatx4*>(Pw + e);
                if constexpr (ACC) v += ca.v[j];
                if ((U.w >> row) & 1) store_c4<false>(C + cr * OL + k0 + col, v);
            }
            return;
        }
        const int c0 = k0 + VEC * n;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int rl = 4 * g + i;
            const long long cr = pr.row(rl);
            if (!((U.w >> rl) & 1)) continue;
            float* crow = C + cr * OL + c0;
            if (split) {
#pragma unroll
                for (int q = 0; q < VEC; ++q)
                    if (c0 + q < O) atomicAdd(crow + q, acc[q][i] * scale);
            } else if (VEC >= 4 && c4 && c0 + VEC <= O) {
#pragma unroll
                for (int h = 0; h < VEC; h += 4) {
                    floatx4 v = ca.v[(i * (VEC / 4) + h / 4) % CAhead<TK, W>::N];
#pragma unroll
                    for (int q = 0; q < 4; ++q) v[q] += acc[(h + q) % VEC][i] * scale;
                    store_c4<ACC>(crow + h, v);
                }
            } else {
#pragma unroll
                for (int q = 0; q < VEC; ++q)
                    if (c0 + q < O) crow[q] = (ACC ? crow[q] : 0.0f) + acc[q][i] * scale;
            }
        }
    } else {
        park_tile<TK>(P + wave * 16 * TK, acc, 1.0f, n, g);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < CAhead<TK, W>::N; ++j) {
            const int e = threadIdx.x * 4 + j * 256 * W;
            if (e >= 16 * TK) break;
            const int row = e / TK, col = e % TK;
            const long long cr = pr.row(row);
            if (!((U.w >> row) & 1)) continue;
            floatx4 sum = *reinterpret_cast<const floatx4*>(P + e);
#pragma unroll
            for (int w = 1; w < W; ++w) {
                const floatx4 x = *reinterpret_cast<const floatx4*>(P + w * 16 * TK + e);
                sum += x;
            }
            const int cc = k0 + col;
            if (cc >= O) continue;
            float* crow = C + cr * OL + cc;
            if (split) {
#pragma unroll
                for (int jj = 0; jj < 4; ++jj)
                    if (cc + jj < O) atomicAdd(crow + jj, sum[jj] * scale);
            } else if (c4 && cc + 4 <= O) {
                floatx4 v = ca.v[j];
                v += sum * scale;
                store_c4<ACC>(crow, v);
            } else {
#pragma unroll
                for (int jj = 0; jj < 4; ++jj)
                    if (cc + jj < O) crow[jj] = (ACC ? crow[jj] : 0.0f) + sum[jj] * scale;
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

// Schedule of a 4-wave work-group.  Work-groups are dealt to the 8 XCDs round robin (the grid's
// x extent is a multiple of 8, so work-group b runs on XCD b mod 8).  The O tiles of one launch
// row (blockIdx.y) go to G = 8 >> lgp groups of P = 1 << lgp XCDs: XCD x computes O tile x / P
// for row part x mod P, so each XCD's L2 holds only its slice of the B rows, and each B row
// slice is fetched by at most P XCDs.  Heavy work-groups come first (8 per P heavy units): the
// four waves share one unit's tiles.  The others run light units, one per wave; light
// work-group j takes the next four units of its row part, a range of units in panel order
// (neighbouring panels share B rows; panels of blocks: in the order of their first column)
// cut for equal tile counts.  Sets `ot`, the O tile within
// the launch row.  Returns false if this wave has nothing to do.
__device__ __forceinline__ bool schedule(int num_heavy, const XcdSplit& xs, int wave, int& u,
                                         bool& heavy, int& ot) {
    const int lgp = xs.lgp, parts = 1 << lgp;
    const int hwg = ((num_heavy + parts - 1) >> lgp) << 3;
    const int b = blockIdx.x, x = b & 7, r = x & (parts - 1);
    ot = x >> lgp;
    if (b < hwg) {
        heavy = true;
        u = ((b >> 3) << lgp) + r;
        return u < num_heavy;
    }
    heavy = false;
    const int j = b - hwg, G = 8 >> lgp;
    u = num_heavy + xs.start[r * G] + (j >> 3) * kWaves + wave;
    return u < num_heavy + xs.start[(r + 1) * G];
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
template <int TK, typename TB, bool ALIGNED, typename Pre>
__device__ __forceinline__ void tiles_f16(int first, int end, int W, int lane, int n, int g,
                                          int c0, long long OL, const int* __restrict__ chunk_eptr,
                                          const int* __restrict__ chunk_cols,
                                          const int* __restrict__ chunk_dense,
                                          const uint32_t* __restrict__ entries,
                                          const _Float16* __restrict__ dense_a,
                                          const TB* __restrict__ B, _Float16* Aw,
                                          floatx4 (&acc)[TK / 16], Pre&& pre) {
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
    // `pre` runs before the last multiply when a single tile is left and the other B buffer is
    // free (see read_c_ahead); with two tiles left, after them (holding both buffers and the C
    // values at once would spill registers).
    if (c < last) {  // two tiles left: c and c + W = last
        load_b_rows<VEC, TB, ALIGNED>(B, colsB, OL, c0, RB);
        sB = load_a16(mB, lane, a_off, entries, dense_a);
        mma_tile_f16<VEC, TB>(mA, sA, lane, Aw, my_a, RA, acc);
        mma_tile_f16<VEC, TB>(mB, sB, lane, Aw, my_a, RB, acc);
        pre();
    } else {
        pre();
        mma_tile_f16<VEC, TB>(mA, sA, lane, Aw, my_a, RA, acc);
    }
}

// Register budget: FP16 B with aligned rows fits three waves per SIMD without spilling; the
// FP32-B and unaligned variants hold more B data and are given two (at O tiles of 64 or less
// they still fit three: 139 VGPRs for FP32 B).
template <typename TB, bool ALIGNED>
constexpr int f16_min_waves() { return (sizeof(TB) == 2 && ALIGNED) ? 3 : 2; }

template <int TK, typename TB, bool ALIGNED, bool ACC, bool MAPPED, bool NTC>
__global__ __launch_bounds__(64 * kWaves, (f16_min_waves<TB, ALIGNED>())) void k_spmm_f16(
    const int4* __restrict__ units, const int* __restrict__ rmap, int num_heavy, XcdSplit xs,
    const int* __restrict__ chunk_eptr, const int* __restrict__ chunk_cols,
    const int* __restrict__ chunk_dense, const uint32_t* __restrict__ entries,
    const _Float16* __restrict__ dense_a, const TB* __restrict__ B, int O, int tiled_n,
    float scale, bool c4, float* __restrict__ C) {
    constexpr int VEC = TK / 16;
    __shared__ __attribute__((aligned(16))) _Float16 As[kWaves][16 * kApitch];
    __shared__ __attribute__((aligned(16))) float P[kWaves * 16 * TK];
    // The wave index is uniform across the wave: readfirstlane lets the compiler keep the unit
    // and tile indices in scalar registers and fetch tile metadata with scalar loads.
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    int u, ot;
    bool heavy;
    if (!schedule(num_heavy, xs, wave, u, heavy, ot)) return;
    const int4 U = units[u];
    const PanelRows<MAPPED> pr = panel_rows<MAPPED>(U, rmap);
    const int k0 = ((blockIdx.y << (3 - xs.lgp)) + ot) * TK;
    const int c0 = k0 + VEC * n;
    // B row-major (row stride O, this lane's columns from c0), or O-tile-major as the FP32-B
    // conversion writes it when every O tile is full (tiled_n = N: O tile k0 / TK is an N x TK
    // block of its own, so each XCD's gathered rows are whole 128-byte lines of contiguous
    // memory instead of every other half of the 256-byte rows).
    const TB* Bt = tiled_n > 0 ? B + (long long)(k0 / TK) * tiled_n * TK : B;
    const long long ldb = tiled_n > 0 ? TK : O;
    const int cb = tiled_n > 0 ? VEC * n : c0;
    floatx4 acc[VEC];
#pragma unroll
    for (int q = 0; q < VEC; ++q) acc[q] = floatx4{0.f, 0.f, 0.f, 0.f};
    // Heavy and light units take separate copies of the tile loop, so that the compiler's load
    // counting sees one fixed sequence of loads on each.
    if (heavy) {
        CAhead<TK, kWaves> ca;
        read_c_ahead<TK, kWaves, NTC>(ca, U, pr, k0, O, c4, ACC, C);
        tiles_f16<TK, TB, ALIGNED>(U.y + wave, U.z, kWaves, lane, n, g, cb, ldb,
                                   chunk_eptr, chunk_cols, chunk_dense, entries, dense_a, Bt,
                                   As[wave], acc, [] {});
        merge_into_c<TK, kWaves, ACC>(acc, scale, U, pr, k0, O, c4, C, P, ca);
    } else {
        CAhead<TK, 1> ca;
        tiles_f16<TK, TB, ALIGNED>(U.y, U.z, 1, lane, n, g, cb, ldb, chunk_eptr,
                                   chunk_cols, chunk_dense, entries, dense_a, Bt, As[wave], acc,
                                   [&] { read_c_ahead<TK, 1, NTC>(ca, U, pr, k0, O, c4, ACC, C); });
        merge_into_c<TK, 1, ACC>(acc, scale, U, pr, k0, O, c4, C, P, ca);
    }
}

// FP32 format: eight K steps of v_mfma_f32_16x16x4_f32 per tile; lane (n, g) feeds tile
// columns k = 4s + g (s = 0..7).  The A tile (LDS or dense copy) is K-step-major so a lane's 8
// values are contiguous: [(k & 3) * 128 + row * 8 + (k >> 2)].  B is fetched in half tiles
// (steps 0-3, then 4-7) so one half is in flight while the other is multiplied.
template <int VEC>
struct FRows {
    typedef float vec_t __attribute__((ext_vector_type(VEC)));
    vec_t r[4];
};

// Half a tile of B rows (K steps s0 .. s0 + 3 of the lane's column group): row s holds the VEC
// output columns c0 .. c0 + VEC - 1 of B row cols[s0 + s].  Loads are unconditional like
// load_b_rows (padding and lanes past O read kZeroRow).
template <int VEC, bool ALIGNED>
__device__ __forceinline__ void load_b_half_f32(const float* __restrict__ B, const int (&cols)[8],
                                                int s0, long long O, int c0, FRows<VEC>& R) {
    typedef typename FRows<VEC>::vec_t vec_t;
    const bool lane_ok = c0 < O;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int col = cols[s0 + s];
        const bool ok = col >= 0 && lane_ok;
        const float* src = ok ? B + (long long)col * O + c0 : kZeroRow;
        if constexpr (ALIGNED) {
            R.r[s] = *reinterpret_cast<const vec_t*>(src);
        } else {
            vec_t x;
#pragma unroll
            for (int q = 0; q < VEC; ++q) x[q] = (ok && c0 + q < O) ? src[q] : 0.0f;
            R.r[s] = x;
        }
    }
}

// K steps s0 .. s0 + 3 of one tile; steps whose four columns are all padding end the tile.
template <int VEC>
__device__ __forceinline__ void mfma_half_f32(const float (&a)[8], int s0, const int (&cols)[8],
                                              const FRows<VEC>& R, floatx4 (&acc)[VEC]) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        if (__ballot(cols[s0 + s] >= 0) == 0) return;
#pragma unroll
        for (int q = 0; q < VEC; ++q)
            acc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s0 + s], R.r[s][q], acc[q], 0, 0, 0);
    }
}

// Row steps s0 .. s0 + 3 of one batch on v_mfma_f32_4x4x1_16b_f32: block b = lane / 4 is row
// group g = b / 4 (rows 4g .. 4g + 3) and output columns c0 of lanes 4b .. 4b + 3; lane 4b + i
// gives A row i (a[s] = the value of row 4g + i at row group g's step-s column) and lane 4b + j
// B column j (R.r[s][q] = that column's B row at output column c0 + q), so register i of lane
// (n, g) accumulates row 4g + i at output column c0 + q -- where the 16x16x4 steps of a tile
// leave it, and the same epilogue applies.  Steps whose four columns are all padding end the
// batch.
template <int VEC>
__device__ __forceinline__ void mfma_half_rs(const float (&a)[8], int s0, const int (&cols)[8],
                                             const FRows<VEC>& R, floatx4 (&acc)[VEC]) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        if (__ballot(cols[s0 + s] >= 0) == 0) return;
#pragma unroll
        for (int q = 0; q < VEC; ++q)
            acc[q] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[s0 + s], R.r[s][q], acc[q], 0, 0, 0);
    }
}

// A state of an FP32 tile in eight words per lane, three loads either way: the dense operand
// (8 floats), or this lane's (entry, value) pairs eb + lane, eb + 64 + lane, eb + 128 + lane
// (clamped into the tile; the scatter skips the ones past ee).
struct AState32 {
    uint4 lo, hi;
};

__device__ __forceinline__ AState32 load_a32(const TileMeta& m, int lane, int a_off,
                                             const uint32_t* __restrict__ entries,
                                             const float* __restrict__ dense_a) {
    const uint32_t* p0;
    const uint32_t* p1;
    const uint32_t* p2;
    if (m.d >= 0) {
        p0 = reinterpret_cast<const uint32_t*>(dense_a + (long long)m.d * 512 + a_off);
        p1 = p0 + 4;
        p2 = p0 + 6;
    } else {
        const int last = m.ee - 1;
        p0 = entries + 2 * (long long)min(m.eb + lane, last);
        p1 = entries + 2 * (long long)min(m.eb + 64 + lane, last);
        p2 = entries + 2 * (long long)min(m.eb + 128 + lane, last);
    }
    AState32 s;
    if (m.d >= 0) {
        s.lo = *reinterpret_cast<const uint4*>(p0);
    } else {
        const uint2 e0 = *reinterpret_cast<const uint2*>(p0);
        s.lo = uint4{e0.x, e0.y, 0u, 0u};
    }
    const uint2 e1 = *reinterpret_cast<const uint2*>(p1);
    const uint2 e2 = *reinterpret_cast<const uint2*>(p2);
    if (m.d >= 0) {
        s.hi = uint4{e1.x, e1.y, e2.x, e2.y};
    } else {
        s.lo.z = e1.x;
        s.lo.w = e1.y;
        s.hi = uint4{e2.x, e2.y, 0u, 0u};
    }
    return s;
}

__device__ __forceinline__ void scatter_a_f32(float* At, uint32_t w, float v) {
    const int r = w & 15, k = (w >> 4) & 31;
    At[(k & 3) * kAgroup32 + r * kApitch32 + (k >> 2)] = v;
}

// This lane's 8 A values of a tile (K steps 0..7): the dense words, or the entries scattered
// into the wave's LDS tile and read back.
__device__ __forceinline__ void a_operand_f32(const TileMeta& m, const AState32& st, int lane,
                                              float* Aw, float* my_a, float (&a)[8]) {
    floatx4 lo, hi;
    if (m.d >= 0) {
        lo = __builtin_bit_cast(floatx4, st.lo);
        hi = __builtin_bit_cast(floatx4, st.hi);
    } else {
        *reinterpret_cast<floatx4*>(my_a) = floatx4{0.f, 0.f, 0.f, 0.f};
        *reinterpret_cast<floatx4*>(my_a + 4) = floatx4{0.f, 0.f, 0.f, 0.f};
        wave_lds_sync();
        if (m.eb + lane < m.ee) scatter_a_f32(Aw, st.lo.x, __uint_as_float(st.lo.y));
        if (m.eb + 64 + lane < m.ee) scatter_a_f32(Aw, st.lo.z, __uint_as_float(st.lo.w));
        if (m.eb + 128 + lane < m.ee) scatter_a_f32(Aw, st.hi.x, __uint_as_float(st.hi.y));
        wave_lds_sync();
        lo = *reinterpret_cast<const floatx4*>(my_a);
        hi = *reinterpret_cast<const floatx4*>(my_a + 4);
        wave_lds_sync();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a[i] = lo[i];
        a[4 + i] = hi[i];
    }
}

// FP32 tiles first, first + W, ... < end of one unit, in half tiles (K steps 0-3, then 4-7) so
// that one half is in flight while the other is multiplied.  Same rules as tiles_f16: the loop
// runs two tiles per iteration over fixed buffers (X: steps 0-3, Y: steps 4-7; tile sets A and
// B for the A state and column indices), column indices are issued before the loads they
// address, and every iteration issues the same loads.  Phases of one iteration (tiles c and
// d = c + W):
//   1. load Y (c);               multiply steps 0-3 of c (X)
//   2. load X (d), A state (d);  multiply steps 4-7 of c (Y); load columns of c + 2W
//   3. load Y (d);               multiply steps 0-3 of d (X)
//   4. load X (c + 2W), A state; multiply steps 4-7 of d (Y); load columns of c + 3W
//
// RS: the unit's work items are row-step batches instead (column slots in chunk_cols = rs_cols,
// A values in dense_a = rs_vals, 128 per batch, this lane's eight at 32 g + 8 (lane & 3)), with
// the same loads of columns and B rows and mfma_half_rs as the product.
template <int TK, bool ALIGNED, bool RS, typename Pre>
__device__ __forceinline__ void tiles_f32(int first, int end, int W, int lane, int n, int g,
                                          int c0, long long OL, const int* __restrict__ chunk_eptr,
                                          const int* __restrict__ chunk_cols,
                                          const int* __restrict__ chunk_dense,
                                          const uint32_t* __restrict__ entries,
                                          const float* __restrict__ dense_a,
                                          const float* __restrict__ B, float* Aw,
                                          floatx4 (&acc)[TK / 16], Pre&& pre) {
    constexpr int VEC = TK / 16;
    if (first >= end) return;
    const int a_off = g * 128 + n * 8;  // in a dense copy
    const int rs_off = g * 32 + (lane & 3) * 8;  // in a row-step batch
    float* my_a = &Aw[g * kAgroup32 + n * kApitch32];
    auto meta = [&](int c) {
        if constexpr (RS) return TileMeta{c, 0, 0};
        else return tile_meta(c, chunk_dense, chunk_eptr);
    };
    auto load_a = [&](const TileMeta& m) {
        if constexpr (RS) {
            const float* p = dense_a + (long long)m.d * 128 + rs_off;
            return AState32{*reinterpret_cast<const uint4*>(p),
                            *reinterpret_cast<const uint4*>(p + 4)};
        } else {
            return load_a32(m, lane, a_off, entries, dense_a);
        }
    };
    auto operand = [&](const TileMeta& m, const AState32& st, float (&a)[8]) {
        if constexpr (RS) {
            const floatx4 lo = __builtin_bit_cast(floatx4, st.lo);
            const floatx4 hi = __builtin_bit_cast(floatx4, st.hi);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                a[i] = lo[i];
                a[4 + i] = hi[i];
            }
        } else {
            a_operand_f32(m, st, lane, Aw, my_a, a);
        }
    };
    auto mma = [&](const float (&a)[8], int s0, const int (&cols)[8], const FRows<VEC>& R) {
        if constexpr (RS) mfma_half_rs<VEC>(a, s0, cols, R, acc);
        else mfma_half_f32<VEC>(a, s0, cols, R, acc);
    };
    const int last = first + (end - 1 - first) / W * W;
    int c = first;
    FRows<VEC> X, Y;
    int colsA[8], colsB[8];
    float a[8];
    TileMeta mA = meta(c);
    load_cols8(chunk_cols, c, g, colsA);
    const int c1 = min(c + W, last);
    load_cols8(chunk_cols, c1, g, colsB);
    TileMeta mB = meta(c1);
    load_b_half_f32<VEC, ALIGNED>(B, colsA, 0, OL, c0, X);
    AState32 sA = load_a(mA), sB;
    for (; c + W < last; c += 2 * W) {
        load_b_half_f32<VEC, ALIGNED>(B, colsA, 4, OL, c0, Y);
        operand(mA, sA, a);
        mma(a, 0, colsA, X);

        load_b_half_f32<VEC, ALIGNED>(B, colsB, 0, OL, c0, X);
        sB = load_a(mB);
        mma(a, 4, colsA, Y);
        load_cols8(chunk_cols, c + 2 * W, g, colsA);
        const TileMeta mA2 = meta(c + 2 * W);

        load_b_half_f32<VEC, ALIGNED>(B, colsB, 4, OL, c0, Y);
        operand(mB, sB, a);
        mma(a, 0, colsB, X);

        load_b_half_f32<VEC, ALIGNED>(B, colsA, 0, OL, c0, X);
        sA = load_a(mA2);
        mma(a, 4, colsB, Y);
        const int c3 = min(c + 3 * W, last);
        load_cols8(chunk_cols, c3, g, colsB);
        mB = meta(c3);
        mA = mA2;
    }
    load_b_half_f32<VEC, ALIGNED>(B, colsA, 4, OL, c0, Y);
    operand(mA, sA, a);
    mma(a, 0, colsA, X);
    // `pre` runs before the last half tile is multiplied, once X is free (see read_c_ahead).
    if (c < last) {  // two tiles left: c and c + W = last
        load_b_half_f32<VEC, ALIGNED>(B, colsB, 0, OL, c0, X);
        sB = load_a(mB);
        mma(a, 4, colsA, Y);
        load_b_half_f32<VEC, ALIGNED>(B, colsB, 4, OL, c0, Y);
        operand(mB, sB, a);
        mma(a, 0, colsB, X);
        pre();
        mma(a, 4, colsB, Y);
    } else {
        pre();
        mma(a, 4, colsA, Y);
    }
}

template <int TK, bool ALIGNED, bool ACC, bool MAPPED, bool NTC>
__global__ __launch_bounds__(64 * kWaves, 3) void k_spmm_f32(
    const int4* __restrict__ units, const int* __restrict__ rmap, int num_heavy, XcdSplit xs,
    const int* __restrict__ chunk_eptr, const int* __restrict__ chunk_cols,
    const int* __restrict__ chunk_dense, const uint32_t* __restrict__ entries,
    const float* __restrict__ dense_a, const int* __restrict__ rs_cols,
    const float* __restrict__ rs_vals, const float* __restrict__ B, int O, bool c4,
    float* __restrict__ C) {
    constexpr int VEC = TK / 16;
    __shared__ __attribute__((aligned(16))) float At[kWaves][4 * kAgroup32];
    __shared__ __attribute__((aligned(16))) float P[kWaves * 16 * TK];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    int u, ot;
    bool heavy;
    if (!schedule(num_heavy, xs, wave, u, heavy, ot)) return;
    const int4 U = units[u];
    const PanelRows<MAPPED> pr = panel_rows<MAPPED>(U, rmap);
    const int k0 = ((blockIdx.y << (3 - xs.lgp)) + ot) * TK;
    const int c0 = k0 + VEC * n;
    floatx4 acc[VEC];
#pragma unroll
    for (int q = 0; q < VEC; ++q) acc[q] = floatx4{0.f, 0.f, 0.f, 0.f};
    // The unit's work items, tiles or row-step batches (wave-uniform: U is a scalar load).  A
    // format with row steps always launches O tiles of at most 64 (o_tile_width): at 128 the
    // second path would make the kernel spill.
    const bool rs = TK <= 64 && (U.w & kUnitRowSteps);
    // Runs the unit's work items from `first` in strides of W, then `pre`.
    auto run = [&](int first, int W, auto&& pre) {
        if constexpr (TK <= 64) {
            if (rs) {
                tiles_f32<TK, ALIGNED, true>(first, U.z, W, lane, n, g, c0, (long long)O,
                                             chunk_eptr, rs_cols, chunk_dense, entries, rs_vals,
                                             B, At[wave], acc, pre);
                return;
            }
        }
        tiles_f32<TK, ALIGNED, false>(first, U.z, W, lane, n, g, c0, (long long)O, chunk_eptr,
                                      chunk_cols, chunk_dense, entries, dense_a, B, At[wave], acc,
                                      pre);
    };
    if (heavy) {
        CAhead<TK, kWaves> ca;
        read_c_ahead<TK, kWaves, NTC>(ca, U, pr, k0, O, c4, ACC, C);
        run(U.y + wave, kWaves, [] {});
        merge_into_c<TK, kWaves, ACC>(acc, 1.0f, U, pr, k0, O, c4, C, P, ca);
    } else {
        CAhead<TK, 1> ca;
        run(U.y, 1, [&] { read_c_ahead<TK, 1, NTC>(ca, U, pr, k0, O, c4, ACC, C); });
        merge_into_c<TK, 1, ACC>(acc, 1.0f, U, pr, k0, O, c4, C, P, ca);
    }
}

// NTC: C read ahead with non-temporal loads (accumulating launches whose C and B exceed the
// last-level cache, see load_c4); only the aligned variants take it.
template <int TK, bool ACC, bool MAPPED, bool NTC>
static void launch_tk_mode(const DeviceFormat& F, const void* dB, bool b_f16, bool b_tiled, int O,
                           float* dC, hipStream_t st) {
    constexpr int VEC = TK / 16;
    // Vector loads of B need O % VEC == 0 and a 16-byte aligned base.
    const bool aligned = (O % VEC) == 0 && ((uintptr_t)dB % 16) == 0;
    const bool c4 = (O % 4) == 0 && ((uintptr_t)dC % 16) == 0;
    // O tiles: G = the largest power of two <= 8 dividing their count go to separate XCD
    // groups; the rest are launch rows (blockIdx.y).
    const int otiles = (O + TK - 1) / TK;
    int G = 8;
    while (otiles % G) G >>= 1;
    XcdSplit xs;
    xs.lgp = G == 8 ? 0 : G == 4 ? 1 : G == 2 ? 2 : 3;
    const int parts = 1 << xs.lgp;
    for (int x = 0; x < 9; ++x) xs.start[x] = F.xcd_start[x];
    int per_xcd = 0;  // light work-groups per XCD
    for (int r = 0; r < parts; ++r)
        per_xcd = std::max(per_xcd,
                           (xs.start[(r + 1) * G] - xs.start[r * G] + kWaves - 1) / kWaves);
    const int hwg = 8 * ((F.num_heavy + parts - 1) / parts);
    const dim3 grid((unsigned)(hwg + 8 * per_xcd), (unsigned)(otiles / G));
    const dim3 block(64 * kWaves);
    const int NH = F.num_heavy;
    const int* rmap = F.row_map.n ? F.row_map.p : nullptr;
    const int4* U = F.units.p;
    const int *eptr = F.chunk_eptr.p, *cols = F.chunk_cols.p, *dense = F.chunk_dense.p;
    const uint32_t* ent = F.entries.p;
    if (F.fp32) {
        // row-step units exist only in kernels of O tiles up to 64 (o_tile_width keeps to that)
        if (TK > 64 && F.num_row_step_batches > 0)
            throw Error(VCSRMC_ERR_STATE, "row steps need O tiles of at most 64");
        const float* B = static_cast<const float*>(dB);
        const int* rsc = F.rs_cols.p;
        const float* rsv = F.rs_vals.p;
        if (aligned)
            hipLaunchKernelGGL((k_spmm_f32<TK, true, ACC, MAPPED, NTC>), grid, block, 0, st, U, rmap,
                               NH, xs, eptr, cols, dense, ent, F.dense_a32.p, rsc, rsv, B, O, c4,
                               dC);
        else
            hipLaunchKernelGGL((k_spmm_f32<TK, false, ACC, MAPPED, false>), grid, block, 0, st, U, rmap,
                               NH, xs, eptr, cols, dense, ent, F.dense_a32.p, rsc, rsv, B, O, c4,
                               dC);
    } else if (b_f16) {
        const _Float16* B = static_cast<const _Float16*>(dB);
        // O-tile-major B (written by the conversion pass) only with every O tile full
        if (b_tiled && (O % TK != 0 || !aligned))
            throw Error(VCSRMC_ERR_STATE, "O-tile-major B needs full, aligned O tiles");
        const int tiled_n = b_tiled ? F.N : 0;
        if (aligned)
            hipLaunchKernelGGL((k_spmm_f16<TK, _Float16, true, ACC, MAPPED, NTC>), grid, block, 0, st,
                               U, rmap, NH, xs, eptr, cols, dense, ent, F.dense_a16.p, B, O,
                               tiled_n, F.scale, c4, dC);
        else
            hipLaunchKernelGGL((k_spmm_f16<TK, _Float16, false, ACC, MAPPED, false>), grid, block, 0, st,
                               U, rmap, NH, xs, eptr, cols, dense, ent, F.dense_a16.p, B, O, 0,
                               F.scale, c4, dC);
    } else if constexpr (TK <= 64) {
        const float* B = static_cast<const float*>(dB);
        if (aligned)
            hipLaunchKernelGGL((k_spmm_f16<TK, float, true, ACC, MAPPED, NTC>), grid, block, 0, st, U,
                               rmap, NH, xs, eptr, cols, dense, ent, F.dense_a16.p, B, O, 0,
                               F.scale, c4, dC);
        else
            hipLaunchKernelGGL((k_spmm_f16<TK, float, false, ACC, MAPPED, false>), grid, block, 0, st, U,
                               rmap, NH, xs, eptr, cols, dense, ent, F.dense_a16.p, B, O, 0,
                               F.scale, c4, dC);
    } else {
        // o_tile_width never gives an FP16 format reading FP32 B an O tile of 128.
        throw Error(VCSRMC_ERR_STATE, "no O tile of 128 for FP32 B with an FP16 format");
    }
    VCSRMC_HIP(hipGetLastError());
}

template <int TK>
static void launch_tk(const DeviceFormat& F, const void* dB, bool b_f16, bool b_tiled, int O,
                      float* dC, bool accumulate, bool nt_c, hipStream_t st) {
    const bool mapped = F.row_map.n > 0;
    if (accumulate && nt_c) {
        if (mapped) launch_tk_mode<TK, true, true, true>(F, dB, b_f16, b_tiled, O, dC, st);
        else launch_tk_mode<TK, true, false, true>(F, dB, b_f16, b_tiled, O, dC, st);
    } else if (accumulate) {
        if (mapped) launch_tk_mode<TK, true, true, false>(F, dB, b_f16, b_tiled, O, dC, st);
        else launch_tk_mode<TK, true, false, false>(F, dB, b_f16, b_tiled, O, dC, st);
    } else {
        if (mapped) launch_tk_mode<TK, false, true, false>(F, dB, b_f16, b_tiled, O, dC, st);
        else launch_tk_mode<TK, false, false, false>(F, dB, b_f16, b_tiled, O, dC, st);
    }
}

// Before an overwriting launch (C = A.B), the rows of every split panel are set to zero: their
// units add into them through atomics.  One work-group per heavy unit; only a panel's first unit
// (kUnitSplitFirst) writes, its masked rows over columns [0, O).
__global__ __launch_bounds__(256) void k_zero_split_rows(const int4* __restrict__ units,
                                                         const int* __restrict__ rmap,
                                                         int num_heavy, int O,
                                                         float* __restrict__ C) {
    const int u = blockIdx.x;
    if (u >= num_heavy) return;
    const int4 U = units[u];
    if (!(U.w & kUnitSplitFirst)) return;
    const long long OL = O;
    for (int r = 0; r < kPanelRows; ++r) {
        if (!((U.w >> r) & 1)) continue;
        float* row = C + (long long)(rmap ? rmap[U.x + r] : U.x + r) * OL;
        for (int c = threadIdx.x; c < O; c += 256) row[c] = 0.0f;
    }
}

// B (n = rows x O floats) to binary16, round to nearest even -- the conversion the FP16 kernel
// applies to an FP32 operand, done once per call instead of once per gathered row.  tk = 0
// keeps B row-major; tk > 0 (O a multiple of tk, tk a multiple of 4) writes it O-tile-major:
// element (r, c) to ((c / tk) * rows + r) * tk + c % tk, four at a time within one tile row.
__global__ void k_b_to_half(const float* __restrict__ B, _Float16* __restrict__ out, long long n,
                            int O, int tk) {
    typedef _Float16 half4 __attribute__((ext_vector_type(4)));
    const long long i = ((long long)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i + 4 <= n) {
        const floatx4 v = *reinterpret_cast<const floatx4*>(B + i);
        const half4 h = half4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
        long long o = i;
        if (tk > 0) {
            const long long r = i / O, rows = n / O;
            const int c = (int)(i - r * O);
            o = ((long long)(c / tk) * rows + r) * tk + c % tk;
        }
        *reinterpret_cast<half4*>(out + o) = h;
    } else {
        for (long long j = i; j < n; ++j) out[j] = (_Float16)B[j];  // row-major only: O % 4 != 0
    }
}

// Width of the O tile a work-group covers.  tileK is the widest allowed (the results do not
// depend on it).  Narrower, where measured faster on gfx950:
//   * never wider than O needs (lanes past O would only multiply zeros);
//   * 64 instead of 128 for formats whose tiles hold few nonzeros (< 48 on average), if the
//     format is FP32 (each wave's chain of FP32 matrix-core steps halves: uniform 4096^2 8.1 ->
//     7.0 us, power-law 36,692^2 33.0 -> 30.2, R-MAT scale 22 5.91 -> 5.70 ms) or B is larger
//     than the 32 MB of L2 on the 8 XCDs (two O halves on separate XCD groups each fetch half of
//     every B row, over a union of fewer row ranges: FP16 R-MAT 3.05 -> 2.86 ms);
//   * 64 for FP32 formats with fewer than kFewPanels32 panels, where the launch at 128 holds
//     under three rounds of the ~3072 waves the GPU keeps resident, each wave a long FP32
//     chain (27-point stencil 18^3 8.22 -> 7.09 us, 30^3 26.6 -> 24.5, 40^3 30.3 -> 29.7;
//     32 x 32 blocks, 96 block rows 6.59 -> 5.97, 512 block rows 26.6 -> 24.7, 1024 block rows
//     24.0 -> 22.8; 4 x 4 blocks, 20,000 block rows 46.3 -> 43.7; a band of 33 per row,
//     50,000 rows 23.8 -> 22.6; an arrow matrix, 100,000 rows 45.6 -> 39.5 us; 2D 9-point
//     300^2 32.7 -> 31.8; 5-point 500^2 (15,625 panels) and 7-point 60^3 (13,500) within 1%);
//   * 64 for FP32 formats holding row steps (which only such formats take in the default mode):
//     the kernels carry the row-step path only up to that width;
//   * 64 for FP16 B above 4 MB with sparse tiles whose panels are alike (no panel more than three
//     times the average tile count, as in uniform random matrices; power-law and R-MAT
//     matrices have panels of hub rows 10x the average and keep 128): their B rows are used a
//     similar number of times from all over the matrix, so each XCD's L2 holds a larger share
//     of the half rows of its O half than of full rows (uniform random, 50,000^2 with 32 per row
//     53.7 -> 47.2 us, 20,000 x 100,000 22.0 -> 20.7, 100,000^2 with 16 per row 70.3 -> 68.3;
//     power-law, R-MAT, grids, bands and blocks unchanged);
//   * 64 for FP16 formats reading FP32 B rows: at 128 that kernel needs 222 VGPRs (two waves
//     per SIMD; three would spill), at 64 139 (three waves), which outweighs repeating the A
//     side (uniform 4096^2 7.9 -> 7.4 us, uniform 20,000^2 with 8 per row 17.9 -> 16.2,
//     power-law 36,692^2 24.5 -> 23.5, 27-point stencil 60^3 90.6 -> 83.1).
//   Otherwise fuller tiles keep 128, since every O tile repeats the A side of each tile
//   (27-point stencil 100^3 and 32 x 32 blocks at 8192 block rows: 2-14% slower at 64), as do
//   FP16 formats with a cache-resident FP16 B (power-law: 15.4 -> 17.4 us at 64).
static int o_tile_width(const DeviceFormat& F, bool b_f16, int O, int tileK) {
    int tk = tileK;
    while (tk > 16 && tk / 2 >= O) tk /= 2;
    if (tk == 128 && F.num_chunks > 0) {
        const bool sparse_tiles = F.nnz < (long long)kSparseTileNnz * F.num_chunks;
        const long long b_bytes = (long long)F.N * O * (b_f16 ? 2 : 4);
        if (F.fp32 && (fp32_narrow_o_tiles(F.nnz, F.num_chunks, F.num_panels) ||
                       F.num_row_step_batches > 0))
            tk = 64;
        else if (!F.fp32 && !b_f16) tk = 64;
        else if (sparse_tiles && b_bytes > (32LL << 20)) tk = 64;
        else if (sparse_tiles && b_bytes > (4LL << 20) &&
                 (long long)F.max_panel_tiles * F.num_panels <= 3LL * F.num_chunks)
            tk = 64;
    }
    return tk;
}

// FP16 format, FP32 B: the kernel rounds each gathered FP32 B row to binary16 as it loads it.
// Converting B once instead costs 6 bytes per element and a pass before the multiply, and saves
// 2 bytes per element on each gather from beyond the caches, so it pays only for B rows used
// many times (12 or more on average) that come from beyond the caches: B above 12 MB (three
// times one XCD's 4 MB L2, which each XCD fills with its own copies) with tiles of few nonzeros
// (< 48 on average: about one gathered row per nonzero), or B above the 256 MB last-level cache.
// Measured on gfx950 (reference protocol, 24 synthetic matrices and the benchmark workloads),
// direct -> converted: uniform random 100,000^2 with 16 per row 118 -> 83 us, 50,000^2 with 32
// per row 107 -> 62, power-law 30,000^2 with 20 per row 37 -> 31, 27-point stencil 100^3
// 572 -> 534; kept direct, where converting measured slower: 5-point grids 500^2 / 700^2
// 75 / 171 us (105 / 208 converted), 7-point 60^3 61 (88), 27-point 60^3 94 (117), uniform
// 300,000^2 with 3 per row 113 (129), uniform 4096^2 8.0 (11.9), power-law 36,692^2 24.9
// (25.7), R-MAT scale 17 51 (55).  Missed by the rule: R-MAT scale 15 (converted, 23 -> 26 us)
// and power-law 200,000^2 with 6 per row (direct, 98 against 92).  Same values either way:
// both round to nearest even.
static bool converts_b(const DeviceFormat& F, bool b_f16, bool b_aligned, int O) {
    const long long b32_bytes = (long long)F.N * O * 4;
    return !F.fp32 && !b_f16 && b_aligned && F.num_chunks > 0 && F.nnz >= 12LL * F.N &&
           ((F.nnz < (long long)kSparseTileNnz * F.num_chunks && b32_bytes > (12LL << 20)) ||
            b32_bytes > (256LL << 20));
}

SpmmPlan plan_spmm(const DeviceFormat& F, const void* dB, bool b_f16, int O, int tileK,
                   float* dC, bool accumulate, HalfScratch ext) {
    if (tileK != 16 && tileK != 32 && tileK != 64 && tileK != 128)
        throw Error(VCSRMC_ERR_TILEK, "vcsr_mc supports tileK in {16, 32, 64, 128}");
    if (!F.ready) throw Error(VCSRMC_ERR_STATE, "no format in this handle");
    if (O < 0) throw Error(VCSRMC_ERR_ARG, "O must be >= 0");
    if (F.fp32 && b_f16) throw Error(VCSRMC_ERR_ARG, "an FP32 format takes an FP32 B");
    SpmmPlan p;
    p.F = &F;
    if (F.num_units == 0 || O == 0) return p;  // nothing to launch
    if (!dB || !dC) throw Error(VCSRMC_ERR_ARG, "null B or C");
    p.dB = dB;
    p.b_f16 = b_f16;
    p.O = O;
    p.dC = dC;
    p.accumulate = accumulate;
    if (converts_b(F, b_f16, ((uintptr_t)dB % 16) == 0, O)) {
        const long long n = (long long)F.N * O;
        _Float16* half = ext.p;
        if (half) {
            if ((unsigned long long)n > ext.halves)
                throw Error(VCSRMC_ERR_SCRATCH,
                            "B of N x O = " + std::to_string(n) +
                                " values exceeds the static scratch of " +
                                std::to_string(ext.halves) + " binary16 values");
        } else {
            if (!F.b_half.p || (long long)F.b_half.n < n) F.b_half.alloc((size_t)n);
            half = F.b_half.p;
        }
        p.convert_to = half;
        p.convert_n = n;
        p.b_f16 = true;
    }
    p.zero_split = !accumulate && F.num_split_panels > 0;
    p.tk = o_tile_width(F, p.b_f16, O, tileK);
    // The conversion writes B O-tile-major where there are several O tiles, all full: each XCD
    // group then gathers whole, contiguous 128-byte lines of its tile instead of every other
    // half of 256-byte rows, which reach only half of an L2's sets (R-MAT scale 22, O tiles of
    // 64: 2.44 -> 2.29 ms; O tiles of 32: 4.78 -> 3.96 ms).  Same values either way.
    p.b_tiled = p.convert_to != nullptr && O > p.tk && O % p.tk == 0;
    // C read non-temporally where C and B together exceed the 256 MB last-level cache (load_c4)
    const long long c_bytes = (long long)F.M * O * 4;
    const long long b_bytes = (long long)F.N * O * (p.b_f16 ? 2 : 4);
    p.nt_c = accumulate && c_bytes + b_bytes > (256LL << 20);
    p.launch = true;
    return p;
}

void run_spmm(const SpmmPlan& p, hipStream_t st) {
    if (!p.launch) return;
    const DeviceFormat& F = *p.F;
    const void* dB = p.dB;
    if (p.convert_to) {
        hipLaunchKernelGGL(k_b_to_half, dim3(grid_for((p.convert_n + 3) / 4, 256)), dim3(256), 0,
                           st, static_cast<const float*>(p.dB), p.convert_to, p.convert_n, p.O,
                           p.b_tiled ? p.tk : 0);
        VCSRMC_HIP(hipGetLastError());
        dB = p.convert_to;
    }
    if (p.zero_split) {
        hipLaunchKernelGGL(k_zero_split_rows, dim3((unsigned)F.num_heavy), dim3(256), 0, st,
                           F.units.p, F.row_map.n ? F.row_map.p : nullptr, F.num_heavy, p.O, p.dC);
        VCSRMC_HIP(hipGetLastError());
    }
    switch (p.tk) {
        case 16: launch_tk<16>(F, dB, p.b_f16, p.b_tiled, p.O, p.dC, p.accumulate, p.nt_c, st); break;
        case 32: launch_tk<32>(F, dB, p.b_f16, p.b_tiled, p.O, p.dC, p.accumulate, p.nt_c, st); break;
        case 64: launch_tk<64>(F, dB, p.b_f16, p.b_tiled, p.O, p.dC, p.accumulate, p.nt_c, st); break;
        default: launch_tk<128>(F, dB, p.b_f16, p.b_tiled, p.O, p.dC, p.accumulate, p.nt_c, st); break;
    }
}

void spmm_launch(const DeviceFormat& F, const void* dB, bool b_f16, int O, int tileK, float* dC,
                 bool accumulate, hipStream_t st, HalfScratch ext) {
    run_spmm(plan_spmm(F, dB, b_f16, O, tileK, dC, accumulate, ext), st);
}

// ---- traffic floor of a launch ------------------------------------------------------------
// The row part (of the XCDs of one O group) that runs unit u, as `schedule` deals the units:
// heavy unit u to part u mod parts, light units by the ranges of xcd_start.
__device__ __forceinline__ int unit_part(int u, int num_heavy, const XcdSplit& xs) {
    const int parts = 1 << xs.lgp;
    if (u < num_heavy) return u & (parts - 1);
    const int j = u - num_heavy, G = 8 >> xs.lgp;
    int r = 0;
    while (r + 1 < parts && j >= xs.start[(r + 1) * G]) ++r;
    return r;
}

// One wave per unit: marks mark[part * N + column] for every column of the unit's tiles (or
// row-step batches) -- plain byte stores, every writer stores 1 -- and writes the bytes of the
// execution layout the unit reads once per O tile (unit 16 B, its row map 64 B; per tile the
// two entry offsets and the dense index 8 B, the column list 128 B, and the dense copy or the
// entries; per row-step batch its columns 128 B and the 512 B of values its lanes read) and the
// rows it writes (a split panel counted at its first unit).
__global__ __launch_bounds__(256) void k_floor_units(
    const int4* __restrict__ units, int num_units, int num_heavy, XcdSplit xs,
    const int* __restrict__ chunk_eptr, const int* __restrict__ chunk_cols,
    const int* __restrict__ chunk_dense, const int* __restrict__ rs_cols, int N, int fp32,
    int mapped, unsigned char* __restrict__ mark, long long* __restrict__ a_bytes,
    int* __restrict__ rows) {
    const int u = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (u >= num_units) return;
    const int lane = threadIdx.x & 63;
    const int4 U = units[u];
    unsigned char* m = mark + (long long)unit_part(u, num_heavy, xs) * N;
    const bool rs = U.w & kUnitRowSteps;
    const int* cols = rs ? rs_cols : chunk_cols;
    long long bytes = 16 + (mapped ? 64 : 0);
    for (int t = U.y; t < U.z; ++t) {
        if (lane < kChunkCols) {
            const int c = cols[(long long)kChunkCols * t + lane];
            if (c >= 0) m[c] = 1;
        }
        if (rs) {
            bytes += 128 + 512;
        } else {
            const int d = chunk_dense[t];
            bytes += 8 + 128 +
                     (d >= 0 ? 512LL * (fp32 ? 4 : 2)
                             : (long long)(chunk_eptr[t + 1] - chunk_eptr[t]) * (fp32 ? 8 : 4));
        }
    }
    if (lane == 0) {
        a_bytes[u] = bytes;
        const bool first = !(U.w & kUnitSplit) || (U.w & kUnitSplitFirst);
        rows[u] = first ? __popc(U.w & 0xffff) : 0;
    }
}

TrafficFloor traffic_floor(const DeviceFormat& F, bool b_f16, int O, int tileK, bool accumulate,
                           hipStream_t st) {
    if (tileK != 16 && tileK != 32 && tileK != 64 && tileK != 128)
        throw Error(VCSRMC_ERR_TILEK, "vcsr_mc supports tileK in {16, 32, 64, 128}");
    if (!F.ready) throw Error(VCSRMC_ERR_STATE, "no format in this handle");
    if (O < 0) throw Error(VCSRMC_ERR_ARG, "O must be >= 0");
    if (F.fp32 && b_f16) throw Error(VCSRMC_ERR_ARG, "an FP32 format takes an FP32 B");
    TrafficFloor t;
    if (F.num_units == 0 || O == 0) return t;
    // the launch's decisions for a 16-byte aligned B (plan_spmm)
    const bool convert = converts_b(F, b_f16, true, O);
    const bool bh = b_f16 || convert;
    t.o_tile_width = o_tile_width(F, bh, O, tileK);
    t.o_tiles = (O + t.o_tile_width - 1) / t.o_tile_width;
    int G = 8;
    while (t.o_tiles % G) G >>= 1;
    XcdSplit xs;
    xs.lgp = G == 8 ? 0 : G == 4 ? 1 : G == 2 ? 2 : 3;
    for (int x = 0; x < 9; ++x) xs.start[x] = F.xcd_start[x];
    t.row_parts = 1 << xs.lgp;
    const int parts = t.row_parts;
    DevBuf<unsigned char> mark((size_t)parts * F.N);
    DevBuf<long long> a_bytes((size_t)F.num_units);
    DevBuf<int> rows((size_t)F.num_units);
    VCSRMC_HIP(hipMemsetAsync(mark.p, 0, mark.n, st));
    hipLaunchKernelGGL(k_floor_units, dim3(grid_for(F.num_units, 4)), dim3(256), 0, st, F.units.p,
                       F.num_units, F.num_heavy, xs, F.chunk_eptr.p, F.chunk_cols.p,
                       F.chunk_dense.p, F.rs_cols.p, F.N, F.fp32, F.row_map.n > 0 ? 1 : 0,
                       mark.p, a_bytes.p, rows.p);
    VCSRMC_HIP(hipGetLastError());
    std::vector<unsigned char> hm(mark.n);
    std::vector<long long> ha((size_t)F.num_units);
    std::vector<int> hr((size_t)F.num_units);
    VCSRMC_HIP(hipMemcpyAsync(hm.data(), mark.p, mark.n, hipMemcpyDeviceToHost, st));
    VCSRMC_HIP(hipMemcpyAsync(ha.data(), a_bytes.p, sizeof(long long) * ha.size(),
                              hipMemcpyDeviceToHost, st));
    VCSRMC_HIP(hipMemcpyAsync(hr.data(), rows.p, sizeof(int) * hr.size(), hipMemcpyDeviceToHost,
                              st));
    VCSRMC_HIP(hipStreamSynchronize(st));
    const long long sb = bh ? 2 : 4;
    long long per_part = 0, once = 0;
    for (int c = 0; c < F.N; ++c) {
        bool any = false;
        for (int r = 0; r < parts; ++r) {
            const bool hit = hm[(size_t)r * F.N + c] != 0;
            per_part += hit;
            any = any || hit;
        }
        once += any;
    }
    long long a = 0, nrows = 0;
    for (size_t u = 0; u < ha.size(); ++u) {
        a += ha[u];
        nrows += hr[u];
    }
    t.b_bytes = per_part * O * sb;
    t.b_once_bytes = once * O * sb;
    t.a_bytes = a * t.o_tiles;
    t.c_bytes = nrows * O * 4LL * (accumulate ? 2 : 1);
    t.convert_bytes = convert ? (long long)F.N * O * 6 : 0;
    t.total = t.b_bytes + t.a_bytes + t.c_bytes + t.convert_bytes;
    return t;
}

}  // namespace vcsrmc
