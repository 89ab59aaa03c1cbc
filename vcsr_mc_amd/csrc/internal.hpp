// internal.hpp -- the device-resident VCSR-MC format and the functions that build and run it.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "primitives.hpp"

namespace vcsrmc {

// Chunk width of the execution layout: one MFMA K block (v_mfma_f32_16x16x32_f16), or eight
// K steps of v_mfma_f32_16x16x4_f32.
constexpr int kChunkCols = 32;
// Rows per panel = MFMA M.
constexpr int kPanelRows = 16;
// A tile holding more nonzeros than this (of 16 x 32) is also stored dense.
constexpr int kDenseMin = 192;
// An FP32 format of at most kSmallPanels non-empty panels and kSmallTiles tiles stores every tile
// dense (at most 8 MB of copies): such a launch is one short chain of dependent loads per wave,
// and a dense tile reaches the matrix cores without the round trip through LDS that scattering
// a tile's entries takes (format_build.hip, dense_min).
constexpr int kSmallPanels = 256;
constexpr int kSmallTiles = 4096;
// Fewest tiles a heavy unit may be cut to (shared by the kWaves waves of one work-group); large
// launches use larger units (format_build.hip, heavy_tile_limit).
constexpr int kHeavyTiles = 64;
// Flag bits of units[u].w above the 16-bit row mask.
constexpr int kUnitSplit = 1 << 16;       // the panel has several units (merge through atomics)
constexpr int kUnitSplitFirst = 1 << 17;  // ... and this is its first unit
constexpr int kUnitRowSteps = 1 << 18;    // the unit runs row-step batches, not tiles (FP32)
// Row steps of an FP32 panel, kept where a panel needs at most this many batches per tile
// (as numerator / denominator), in the default mode (format_build.hip, k_row_step_batches).
constexpr int kRowStepRatioNum = 3, kRowStepRatioDen = 2;
constexpr int kWaves = 4;

// Light-unit ranges per XCD, passed to the multiply kernels by value.
struct XcdSplit {
    int start[9];
    int lgp;  // log2 of the row parts per O group: the O tiles are dealt to 8 >> lgp XCD groups
};

// A format on one device.
//
// Boundary arrays (the reference's VCSRMC, include/vcsr_formats.hpp:14-21, built or uploaded
// bit for bit): group_ptr, group_depth, group_seg_base, group_rows, lcol, val, item_gbeg,
// item_gend.
//
// Execution layout (what the multiply kernels read), derived from the same matrix:
//   units[u]        = {pos0, chunk_begin, chunk_end, rowmask | flags}
//                     a run of chunks of one panel, the 16 row-order positions pos0 .. pos0 + 15
//                     (rows pos0 + r in natural order, row_map[pos0 + r] with a row map;
//                     rowmask bit r = that position holds a row with nonzeros); kUnitSplit =
//                     the panel has several units, whose partial sums meet in C through
//                     atomics, kUnitSplitFirst = the first of them; with kUnitRowSteps,
//                     chunk_begin .. chunk_end are row-step batches (below).  The first
//                     num_heavy units are heavy (one work-group each, larger first), the rest
//                     light (one wave each, four per work-group, in panel order, or in the
//                     order of the panels' first columns for blocks; XCD x runs the range
//                     starting at xcd_start[x], cut for equal tile counts).
//   chunk_eptr[c]   = first entry of chunk c (chunk_eptr[num_chunks] = nnz)
//   chunk_cols[32c+k] = column of the chunk's k-th distinct column, -1 past the end (FP32
//                   formats: slot (k & 3) * 8 + (k >> 2), the order the FP32 kernel's lanes read)
//   entries[e]      FP16 format: f16 value | row-in-panel << 16 | k << 20
//                   FP32 format: two words per entry, entries[2e] = row-in-panel | k << 4 and
//                   entries[2e+1] = the value's bits
//   row steps       (FP32 formats, panels whose rows rarely share a column): instead of tiles,
//                   a unit runs batches of 8 steps of v_mfma_f32_4x4x1_16b_f32, whose 16
//                   blocks are the panel's 4 row groups (rows 4g..4g+3) x 4 groups of output
//                   columns.  At each step every row group g takes its own next column: the
//                   row group's distinct columns in ascending order, one per step, padded with
//                   -1 after the last; a panel has as many steps as its busiest row group has
//                   columns, rounded up to 8.  rs_cols[32b + 8g + t] = the column of step t of
//                   batch b for row group g (the slots the tile path's lane group g reads), and
//                   rs_vals[128b + 32g + 8x + t] = the value of row 4g + x at that column (0 if
//                   the row does not hold it), so a lane reads its eight A values with two
//                   128-bit loads.  A panel takes row steps when its batches are at most
//                   kRowStepRatioNum / kRowStepRatioDen times its tiles: each step costs a
//                   quarter of the matrix-core cycles of a 16x16x4 K step and the same one B
//                   row load per lane.
//   chunk_dense[c]  -1, or the index of the tile's dense copy when more than kDenseMin of its
//                   512 slots are filled (every tile of a small FP32 format, kSmallPanels):
//                   dense_a16[512 d + 32 row + k] (FP16), or
//                   dense_a32[512 d + 128 (k & 3) + 8 row + (k >> 2)] (FP32) -- exactly the
//                   order in which MFMA lanes read their A operand, so a lane loads it directly
// Below this many 16-row panels a launch cannot fill the GPU's 1024 SIMDs with one wave per
// panel: every multi-tile panel is then shared by a work-group (format_build.hip), and FP32
// formats take O tiles of 64 (spmm_kernels.hip).
constexpr int kFewPanels = 2048;
// Tiles holding fewer nonzeros than this on average are sparse (about one gathered B row per
// nonzero); FP32 formats with sparse tiles, or with fewer than kFewPanels32 panels, take O
// tiles of 64 (spmm_kernels.hip, o_tile_width), and only such formats take row steps in the
// default mode (format_build.hip).
constexpr int kSparseTileNnz = 48;
constexpr int kFewPanels32 = 8192;
inline bool fp32_narrow_o_tiles(long long nnz, int num_chunks, int num_panels) {
    return nnz < (long long)kSparseTileNnz * num_chunks || num_panels < kFewPanels32;
}

struct DeviceFormat {
    int M = 0, N = 0, segw = 16, bundle = 16, num_segments = 0;
    int G = 0, nitems = 0;
    long long nval = 0, nnz = 0;
    float scale = 1.0f;
    int fp32 = 0;

    DevBuf<int> group_ptr, group_depth, group_seg_base, group_rows, lcol, item_gbeg, item_gend;
    DevBuf<float> val;

    int num_panels = 0, num_chunks = 0, num_units = 0, num_heavy = 0, light_max = 0;
    int heavy_tiles = 0;       // largest heavy unit, in tiles
    long long num_pairs = 0;   // distinct (panel, column) pairs: the tiles' filled columns
    int num_split_panels = 0;  // panels cut into several units
    int max_panel_tiles = 0;   // tiles of the largest panel
    // Light units [num_heavy + xcd_start[x], num_heavy + xcd_start[x + 1]) run on XCD x.
    int xcd_start[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
    DevBuf<int4> units;
    // Row map (empty: natural order).  The layout's panels are 16 consecutive positions of a row
    // order; row_map[p] = the row at position p (-1 past the last row).  Units, row masks and
    // the entries' row-in-panel refer to positions; the kernels write C row row_map[p].
    DevBuf<int> row_map;
    DevBuf<int> chunk_eptr, chunk_cols;
    DevBuf<uint32_t> entries;
    int num_dense = 0;
    DevBuf<int> chunk_dense;
    DevBuf<_Float16> dense_a16;
    DevBuf<float> dense_a32;
    int num_row_step_batches = 0;
    DevBuf<int> rs_cols;
    DevBuf<float> rs_vals;

    // FP32 B converted to binary16 for an FP16 format (spmm_launch), reused across calls.
    mutable DevBuf<_Float16> b_half;

    bool ready = false;
    void clear() { *this = DeviceFormat(); }
};

// FP16 range scale from the largest finite |value| (src/vcsr_mc.cu:14-22 as the reference
// binary evaluates it; see half_scale_from_amax).
float half_scale_from_amax(float amax);
float device_absmax(const float* d_val, long long n, hipStream_t st);

// A row order that groups rows sharing columns into 16-row panels (row_groups.hip), from the
// (row, col) of n nonzeros: rowpos[row] = position, row_map[position] = row (-1 past the last
// of M rows; M rounded up to 16 entries).  False when it found nothing to work with.
bool group_rows(const int* trow, const int* tcol, long long n, int M, int N, hipStream_t st,
                DevBuf<int>& rowpos, DevBuf<int>& row_map);
// The same maps for natural order with the rows that hold no nonzero moved after the others,
// when they are at least an eighth of the rows (false otherwise): panels then hold 16 rows
// with nonzeros instead of, on average, as many as the empty rows leave.
bool compact_rows(const int* trow, long long n, int M, hipStream_t st, DevBuf<int>& rowpos,
                  DevBuf<int>& row_map);
// Row order of the execution layout: 0 natural order, 1 empty rows moved last and rows grouped
// where that saves tiles (the default; format_build.hip, build_exec_layout), 2 always grouped.
// Read by later builds.
void set_row_grouping(int mode);
int row_grouping();
// Product of FP32 panels: 0 tiles only, 1 row steps where they take at most kRowStepRatioNum /
// kRowStepRatioDen batches per tile (the default), 2 row steps for every FP32 panel.  Read by
// later builds.
void set_fp32_row_steps(int mode);
int fp32_row_steps();

// GPU format pipeline from a device CSR (src/vcsr_mc.cu:25-123).
void build_from_csr(DeviceFormat& F, const int* d_row_ptr, const int* d_col, const float* d_val,
                    int M, int N, int nnz, int segw, int fp32, hipStream_t st);

// Format arrays given by the caller (host pointers, src/vcsr_mc.cu:332-349), validated on
// the device, then the execution layout is derived from them.
struct HostArrays {
    int M, N, segw, bundle, num_segments, G, nitems;
    long long nval;
    const int *group_ptr, *group_depth, *group_seg_base, *group_rows, *lcol;
    const float* val;
    const int *item_gbeg, *item_gend;
    float scale;
    int fp32;
};
void build_from_host(DeviceFormat& F, const HostArrays& H, hipStream_t st);

// C += A.B (src/vcsr_mc.cu:352-394 semantics).  b_f16: B is binary16 in HBM.
// Device memory a launch may use for the binary16 copy of an FP32 B (an FP16 format converts
// B once per call where that pays, see spmm_launch): `p` of `halves` elements, or p = null for
// the format's own buffer, allocated on first use.
struct HalfScratch {
    _Float16* p = nullptr;
    size_t halves = 0;
};

// accumulate: C += A.B; otherwise C = A.B on the rows A touches (other rows untouched).
void spmm_launch(const DeviceFormat& F, const void* dB, bool b_f16, int O, int tileK, float* dC,
                 bool accumulate, hipStream_t st, HalfScratch ext = HalfScratch());
// spmm_launch in two steps: plan_spmm checks the arguments and makes every host decision (O tile
// width, B conversion and its buffer, split-row clearing), run_spmm only enqueues the kernels,
// so a caller timing the launch with events brackets GPU work only (as the reference's
// run_vcsr_mc_spmm_gpu records its first event right before its launch, src/vcsr_mc.cu:381).
struct SpmmPlan {
    const DeviceFormat* F = nullptr;
    const void* dB = nullptr;
    float* dC = nullptr;
    int O = 0, tk = 128;
    bool b_f16 = false, accumulate = true, zero_split = false, launch = false;
    _Float16* convert_to = nullptr;  // FP32 B converted into this binary16 buffer first
    long long convert_n = 0;
    bool b_tiled = false;  // ... and laid out O-tile-major ([O tile][N][tk]; every O tile full)
    bool nt_c = false;     // C += A.B reads C non-temporally (C and B beyond the last-level cache)
};
SpmmPlan plan_spmm(const DeviceFormat& F, const void* dB, bool b_f16, int O, int tileK, float* dC,
                   bool accumulate, HalfScratch ext = HalfScratch());
void run_spmm(const SpmmPlan& p, hipStream_t st);

// The HBM bytes a launch cannot avoid under its schedule, if every XCD's L2 kept everything its
// work-groups touched for the whole launch: B, the distinct columns of each XCD row part's
// units, once per part; the execution layout each O tile reads; C written once per non-empty
// row (and read first when accumulating); the FP32-to-binary16 pass over B where the launch
// makes one (6 bytes per element).  The launch's own decisions for a 16-byte aligned B.
struct TrafficFloor {
    long long b_bytes = 0, b_once_bytes = 0, a_bytes = 0, c_bytes = 0, convert_bytes = 0,
              total = 0;
    int o_tile_width = 0, o_tiles = 0, row_parts = 0;
};
TrafficFloor traffic_floor(const DeviceFormat& F, bool b_f16, int O, int tileK, bool accumulate,
                           hipStream_t st);

// Reverse Cuthill-McKee order of the columns of a device CSR (include/reorder.hpp:17-77):
// position[old column] = new column.  Synchronises `st`.
void rcm_order_device(const int* rp, const int* col, int M, int N, int nnz, int* position,
                      hipStream_t st);
// Iteration limits of rcm_order_device's loops (BFS levels, component rounds); 0 restores the
// proven maxima.  Lowered only to test that an exhausted loop returns an error.
void set_rcm_limits(long long max_level, long long max_rounds);
// Column relabelling (include/reorder.hpp:82-108): col and val in place, rows re-sorted by new
// column; B_out[position[r], :] = B[r, :] when B is given.  Synchronises `st`.
void apply_column_permutation_device(const int* rp, int* col, float* val, int M, int N, int nnz,
                                     const int* position, const float* B, int O, float* B_out,
                                     hipStream_t st);

}  // namespace vcsrmc
