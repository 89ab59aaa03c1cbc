/*
 * vcsrmc.h -- C ABI of the MI355X (gfx950) VCSR-MC SpMM library, libvcsrmc.so.
 *
 * Plain pointers and sizes only.  Device pointers are HIP device memory of the current
 * device; `stream` is a hipStream_t passed as void* (NULL = the default stream).  Every entry
 * point returns a status code (VCSRMC_OK = 0); no exception or exit() crosses this boundary.
 * The C++ drop-in surface of the reference (include/vcsr_formats.hpp) is a thin layer over
 * these functions.
 *
 * Threads: a handle holds all of its format's state, so different handles may be used from
 * different host threads at the same time; one handle must not be used by two threads at once
 * (its FP16 copy of an FP32 B is allocated on first use).  State shared by all handles is the
 * row-grouping mode and the RCM limits (atomics, read once per call) and the per-device
 * scratch of vcsrmc_spmm_noalloc (see there).  The C++ drop-in keeps the reference's single
 * library-global format and is not re-entrant, like the reference (src/vcsr_mc.cu:126-131).
 *
 * Each entry point names the reference interface it replaces (MuuSeoTia/VCSR_MC,
 * path:line relative to that repository).
 */
#ifndef VCSRMC_H
#define VCSRMC_H

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define VCSRMC_OK 0
#define VCSRMC_ERR_ARG 1       /* null pointer, negative size, bad dtype/flag            */
#define VCSRMC_ERR_SEGW 2      /* segw not in {16,32,48,64}      (src/vcsr_mc.cu:26-27)   */
#define VCSRMC_ERR_TILEK 3     /* tileK not in {16,32,64,128}    (src/vcsr_mc.cu:385-388) */
#define VCSRMC_ERR_CSR 4       /* row_ptr not monotone / not 0..nnz, column out of range  */
#define VCSRMC_ERR_UNSORTED 5  /* columns of a row not strictly increasing: unsorted or a
                                  duplicate coordinate (include/csr.hpp:28-40)           */
#define VCSRMC_ERR_FORMAT 6    /* uploaded format arrays inconsistent                      */
#define VCSRMC_ERR_OVERFLOW 7  /* |val| or another size exceeds the int32 of the format   */
#define VCSRMC_ERR_HIP 8       /* HIP runtime error                                        */
#define VCSRMC_ERR_STATE 9     /* no format built or uploaded in this handle               */
#define VCSRMC_ERR_SCRATCH 10  /* input exceeds the static scratch of vcsrmc_spmm_noalloc  */

/* Element type of the dense B operand. */
#define VCSRMC_B_F32 0
#define VCSRMC_B_F16 1

typedef struct vcsrmc_format_s *vcsrmc_t;

typedef struct vcsrmc_info {
    int M, N, segw, bundle, num_segments;
    int num_groups;        /* G = group_depth.size()                 */
    long long nval;        /* |lcol| = |val| = group_ptr[G]          */
    int num_items;         /* item_gbeg.size()                       */
    float scale;           /* FP16 range scale (1 for FP32 formats)  */
    int fp32;              /* 1: vcsr_mc_fp32, 0: vcsr_mc            */
    long long nnz;
    int num_panels;        /* execution layout: non-empty 16-row panels */
    int num_chunks;        /* 32-column compacted tiles                 */
    int num_units;         /* kernel work units                         */
    int device;            /* HIP device the format lives on            */
    int num_dense;         /* tiles stored as dense 16 x 32 copies      */
    int row_grouped;       /* 1: the layout's panels follow a row map      */
    int num_heavy;         /* units shared by the four waves of a work-group */
    int num_split_panels;  /* panels cut into several heavy units (merged through atomics) */
    int num_row_step_batches; /* FP32: batches of 8 row steps (vcsrmc_set_fp32_row_steps) */
} vcsrmc_info;

/* Handle holding one device-resident format (the reference keeps one format in
 * namespace-static device pointers, src/vcsr_mc.cu:126-131; a handle removes that limit). */
int vcsrmc_create(vcsrmc_t *out);

/* Frees the device copies and the handle.  Replaces destroy_vcsr_mc_device
 * (include/vcsr_formats.hpp:26, src/vcsr_mc.cu:397-404). */
int vcsrmc_destroy(vcsrmc_t h);

/* FP16 range scale of the values of a device array (src/vcsr_mc.cu:14-22, evaluated as the
 * reference binary does: it is built with -ffast-math, CMakeLists.txt:24-27, so amax / 60000
 * is amax * fl(1/60000)).  Replaces half_scale (include/vcsr_formats.hpp:11). */
int vcsrmc_half_scale(const float *d_val, long long nnz, float *scale, void *stream);

/* Builds the format on the GPU from a device CSR (row_ptr[M+1], col[nnz] strictly increasing
 * inside each row, val[nnz]).  Replaces csr_to_vcsr_mc followed by upload_vcsr_mc_device
 * (include/vcsr_formats.hpp:22-23, src/vcsr_mc.cu:25-123, 332-349).  Synchronises `stream`. */
int vcsrmc_build_csr(vcsrmc_t h, const int *d_row_ptr, const int *d_col, const float *d_val,
                     int M, int N, int nnz, int fp32, int segw, void *stream);

/* Uploads format arrays held by the caller in host memory (the fields of the reference's
 * struct VCSRMC, include/vcsr_formats.hpp:14-21), validates them on the device and derives the
 * execution layout.  Replaces upload_vcsr_mc_device (include/vcsr_formats.hpp:23,
 * src/vcsr_mc.cu:332-349).  Synchronises `stream`. */
int vcsrmc_upload(vcsrmc_t h, int M, int N, int segw, int bundle, int num_segments,
                  int num_groups, long long nval, int num_items, const int *group_ptr,
                  const int *group_depth, const int *group_seg_base, const int *group_rows,
                  const int *lcol, const float *val, const int *item_gbeg, const int *item_gend,
                  float scale, int fp32, void *stream);

/* Sizes and scalar fields of the format in h. */
int vcsrmc_get_info(vcsrmc_t h, vcsrmc_info *out);

/* Copies the format arrays to caller-provided host buffers sized by vcsrmc_get_info
 * (group_ptr: G+1, group_depth/group_seg_base: G, group_rows: 16 G, lcol/val: nval,
 * item_gbeg/item_gend: num_items).  Any pointer may be NULL to skip that array.  This is the
 * output of csr_to_vcsr_mc (include/vcsr_formats.hpp:22). */
int vcsrmc_download(vcsrmc_t h, int *group_ptr, int *group_depth, int *group_seg_base,
                    int *group_rows, int *lcol, float *val, int *item_gbeg, int *item_gend);

/* C += A.B, C (M x O, row-major, ldc = O) and B (N x O, row-major, ldb = O) in device memory.
 * b_dtype = VCSRMC_B_F32 (the reference's `const float* dB`) or VCSRMC_B_F16 (B already in
 * binary16, converted once by the caller).  tileK in {16,32,64,128} is the widest
 * output-column tile of one work-group, as in the reference; the launcher takes a narrower one
 * where that measured faster, and the result does not depend on it:
 *   - never wider than O needs;
 *   - 64 instead of 128 for formats whose tiles hold few nonzeros (fewer than 48 on average)
 *     that are FP32 or whose B exceeds the GPU's 32 MB of L2;
 *   - 64 for FP32 formats of fewer than 8192 16-row panels, and for FP32 formats holding row
 *     steps (vcsrmc_set_fp32_row_steps);
 *   - 64 for FP16 B above 4 MB with sparse tiles and no panel of more than three times the
 *     average tile count (uniform random matrices);
 *   - 64 for an FP16 format reading FP32 B directly (at 128 that kernel holds too many
 *     registers for three waves per SIMD).
 * Rows of C that A does not touch are left as they are.  If ms is non-NULL the launch is
 * bracketed by two hipEvents on `stream`, the call waits for it and *ms is the elapsed time (the
 * reference's protocol); if ms is NULL the launch is asynchronous.  An FP16 format given FP32 B
 * rounds B to binary16 as the kernel loads it; where nnz >= 12 N and B exceeds 12 MB with tiles
 * averaging fewer than 48 nonzeros, or exceeds 256 MB, it converts B once per call instead,
 * into a buffer the handle keeps (N x O halves, allocated on first use and reallocated when a
 * later call needs more), so calls on one handle from several streams at once must not overlap.
 * Otherwise the launch allocates and clears nothing, so it can be captured in a HIP graph: make
 * the first FP32-B call, with the largest O, before capturing; a call with a larger O frees
 * that buffer, and graphs captured earlier must not be replayed after it
 * (vcsrmc_spmm_noalloc below never allocates).
 * Replaces run_vcsr_mc_spmm_gpu (include/vcsr_formats.hpp:24-25, src/vcsr_mc.cu:352-394). */
int vcsrmc_spmm(vcsrmc_t h, const void *dB, int b_dtype, int O, int tileK, float *dC,
                void *stream, float *ms);

/* Flags of vcsrmc_spmm_ex. */
#define VCSRMC_SPMM_OVERWRITE 1 /* C = A.B on the rows A touches, without reading C */

/* vcsrmc_spmm with flags; flags = 0 is vcsrmc_spmm (C += A.B).  VCSRMC_SPMM_OVERWRITE writes
 * C = A.B on every row that holds a nonzero of A and leaves the other rows as they are, so it
 * never reads C: it equals zeroing C and calling vcsrmc_spmm (the reference's measured protocol,
 * src/main.cpp:242-245), and saves the read of C.  Equal bit for bit on every row outside split
 * panels; where a 16-row panel of A is split across work-groups (panels of very many 32-column
 * tiles), its rows are first set to zero by a small kernel on `stream` and its work-groups add
 * into them with float atomics in no fixed order, so those rows agree within rounding (as two
 * runs of either call may).  No counterpart in the reference, whose kernels always
 * accumulate into C with atomicAdd (src/vcsr_mc.cu:228-234). */
int vcsrmc_spmm_ex(vcsrmc_t h, const void *dB, int b_dtype, int O, int tileK, float *dC,
                   int flags, void *stream, float *ms);

/* Bytes of the static device scratch of vcsrmc_spmm_noalloc, per GPU. */
#define VCSRMC_NOALLOC_SCRATCH_BYTES (64u << 20)

/* vcsrmc_spmm_ex that allocates nothing.  No counterpart in the reference: for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  The only device memory vcsrmc_spmm may allocate is the binary16 copy
 * of an FP32 B that an FP16 format converts once per call (N x O halves); here it lives in a
 * static device array of VCSRMC_NOALLOC_SCRATCH_BYTES per GPU, reserved when the library's
 * code is loaded on that GPU and held until the process ends.  A call whose conversion would
 * need more returns VCSRMC_ERR_SCRATCH before launching anything.  Every call on one GPU shares
 * that GPU's scratch, so calls that overlap on one GPU (several streams or threads) race; the
 * scratch keeps the last call's contents, and nothing in it needs to start at zero.  No timing
 * events: the launch is asynchronous on `stream`.  Same results as vcsrmc_spmm_ex under the
 * same arguments: bit for bit outside split panels, within rounding on their rows (float
 * atomics in no fixed order, see vcsrmc_spmm_ex). */
int vcsrmc_spmm_noalloc(vcsrmc_t h, const void *dB, int b_dtype, int O, int tileK, float *dC,
                        int flags, void *stream);

/* Reverse Cuthill-McKee order of the columns of a device CSR (row_ptr[M+1], col[nnz]; any
 * column order inside a row): d_position[N] receives the new position of every old column,
 * equal element for element to the reference's rcm_column_order, tie order included
 * (include/reorder.hpp:17-77).  Computed on the GPU; synchronises `stream`. */
int vcsrmc_rcm_order(const int *d_row_ptr, const int *d_col, int M, int N, int nnz,
                     int *d_position, void *stream);

/* Iteration limits of vcsrmc_rcm_order's loops: levels of the breadth-first walk and rounds of
 * the connected-component search.  0 (the default) keeps the proven maxima, N + 1 levels and
 * N (ceil(lg N) + 2) + 1 rounds, which a correct walk never reaches; a walk that would pass a
 * limit stops, with every kernel ended, and vcsrmc_rcm_order returns VCSRMC_ERR_STATE.  Lower
 * limits exist to test that path.  Process-wide; no counterpart in the reference. */
int vcsrmc_set_rcm_limits(long long max_levels, long long max_rounds);

/* Row order of the execution layout that later builds and uploads use (process-wide): 0 natural
 * order; 1 (the default) rows without nonzeros after the others when they are at least an
 * eighth of the rows, and rows grouped by shared columns into 16-row panels where the rows of a
 * panel already share columns (at least 1.3 nonzeros per distinct column of a panel: grids and
 * meshes), tiles are not full and grouping saves at least a tenth of the tiles; 2 always
 * grouped.  Only the execution layout changes: the format arrays, C's rows and the
 * product are the same (up to rounding: the sums of a row are formed in another order).
 * vcsrmc_info.row_grouped is 1 when a handle's layout has any row map.  No counterpart in the
 * reference. */
int vcsrmc_set_row_grouping(int mode);

/* Product of FP32 panels that later builds and uploads lay out (process-wide).  A tile step,
 * v_mfma_f32_16x16x4_f32, multiplies all 16 rows of a panel at 4 columns, however few of those
 * rows hold them; a row step, v_mfma_f32_4x4x1_16b_f32 with its blocks as 4 row groups x 4
 * groups of output columns, lets each group of 4 rows take its own next column, at a quarter of
 * the cycles, so a panel whose rows rarely share a column needs about as many row steps as tile
 * steps.  0: tile steps only; 1 (the default): row steps for every FP32 panel that needs at
 * most 3/2 as many batches of 8 row steps as it has tiles, in formats whose tiles average fewer
 * than 48 nonzeros or that have fewer than 8192 panels (those launch O tiles of 64 anyway);
 * 2: row steps for every FP32 panel.
 * The product is the same up to rounding (each row's sum is formed in another order).
 * vcsrmc_info.num_row_step_batches counts a format's batches.  No counterpart in the
 * reference. */
int vcsrmc_set_fp32_row_steps(int mode);

/* The row order of h's execution layout, for inspection: *length = the number of positions
 * (a multiple of 16; 0 when the layout keeps natural order, row r at position r), and, when
 * *length > 0 and row_of_position is not NULL, row_of_position[p] = the row at position p, or
 * -1 for padding past the last row (host buffer of `capacity` ints, at least *length; NULL:
 * only *length is set).  No counterpart in the reference. */
int vcsrmc_get_row_map(vcsrmc_t h, int *row_of_position, long long capacity, long long *length);

/* The work units of h's execution layout, for inspection: *num_units = their number and, when
 * units is not NULL, units[4u .. 4u+3] = {p0, first, end, mask | flags} of unit u (host buffer
 * of `capacity` ints, at least 4 * *num_units): the unit multiplies tiles (or, with flag bit 18,
 * batches of FP32 row steps) first .. end - 1 of the 16-row panel at row-order positions
 * p0 .. p0 + 15 (rows p0 + i, or row_of_position[p0 + i] of vcsrmc_get_row_map), bit i of the
 * low 16 bits set when position p0 + i holds a row with nonzeros; flag bit 16: the panel is
 * split into several units, which add into C through atomics; bit 17: this is its first unit.
 * The first vcsrmc_info.num_heavy units are shared by the four waves of a work-group; light
 * unit num_heavy + j runs on the XCD range x with xcd_start[x] <= j < xcd_start[x + 1]
 * (xcd_start: 9 ints, may be NULL).  No counterpart in the reference. */
int vcsrmc_get_units(vcsrmc_t h, int *units, long long capacity, long long *num_units,
                     int *xcd_start);

/* HBM bytes a launch of vcsrmc_spmm_ex with these arguments cannot avoid under its schedule,
 * if each XCD's L2 kept everything its work-groups touched for the whole launch (a floor for
 * measured traffic, not a prediction).  The launch deals row parts of the units to the XCDs of
 * each O group; B counts, per part, every distinct column of its units once, at O values of
 * the element type the kernel reads (binary16 where B is FP16 or converted first).  No
 * counterpart in the reference. */
typedef struct vcsrmc_traffic {
    long long b_bytes;       /* B: sum over row parts of (distinct columns) x O x element size */
    long long b_once_bytes;  /* B: every distinct column once for the whole GPU               */
    long long a_bytes;       /* execution layout a launch reads, once per O tile              */
    long long c_bytes;       /* C: non-empty rows x O x 4, x 2 when accumulating (read+write) */
    long long convert_bytes; /* FP32 B rounded to binary16 in a pass first: 6 B per element   */
    long long total;         /* b_bytes + a_bytes + c_bytes + convert_bytes                   */
    int o_tile_width;        /* output columns per work-group the launch takes                */
    int o_tiles;             /* ceil(O / o_tile_width)                                        */
    int row_parts;           /* row parts per O group (8 XCDs / O groups)                     */
} vcsrmc_traffic;
int vcsrmc_traffic_floor(vcsrmc_t h, int b_dtype, int O, int tileK, int flags,
                         vcsrmc_traffic *out, void *stream);

/* Relabels the columns of a device CSR in place, col[p] = position[col[p]], with every row
 * re-sorted by its new columns (values follow), and, when d_B is non-NULL, writes
 * d_B_out[position[r], :] = d_B[r, :] (N x O floats, d_B_out distinct from d_B), so that
 * C = (A P)(P^T B) = A B.  position must be a permutation of 0..N-1 and a row may not hold a
 * column twice.  Replaces apply_column_permutation (include/reorder.hpp:82-108); synchronises
 * `stream`. */
int vcsrmc_apply_column_permutation(const int *d_row_ptr, int *d_col, float *d_val, int M, int N,
                                    int nnz, const int *d_position, const float *d_B, int O,
                                    float *d_B_out, void *stream);

/* Text of a status code, and the detail message of the last failing call on this thread. */
const char *vcsrmc_status_string(int status);
const char *vcsrmc_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* VCSRMC_H */
