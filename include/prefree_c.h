/*
 * prefree_c.h — C ABI of the MI355X CSR SpMV library (libprefree.so).
 *
 * Plain pointers and sizes only.  Device pointers are HIP device memory on the
 * current device; `stream` is a hipStream_t passed as void* (NULL = the null
 * stream).  Every function returns a pf_status (0 = success) unless noted.
 *
 * Reference counterpart: the reference exposes exactly one entry point,
 *   void preFreeSpMV(valT*, int*, int*, valT*, valT*, int, int, int, double*, double*)
 *   (include/PreFree.h:3-5, defined at src/spmv_kernel/preFreeSpMV.cu:563-662),
 * which allocates, copies, pre-processes, times and computes in one call.
 * That call is kept as the C++ drop-in in include/PreFree.h.  The entries
 * below split it into the parts a caller that already holds device buffers
 * needs: analyse once (pf_plan_create, replacing the pre-pass launch at
 * preFreeSpMV.cu:599), then y = A·x many times (pf_plan_execute, replacing the
 * kernel launches at preFreeSpMV.cu:634-645).
 */
#ifndef PREFREE_C_H
#define PREFREE_C_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes --------------------------------------------------------- */
enum pf_status {
    PF_OK = 0,
    PF_ERR_INVALID = 1,     /* bad argument (negative size, NULL pointer, unknown enum) */
    PF_ERR_ALIGN = 2,       /* col / val not 16-byte aligned */
    PF_ERR_HIP = 3,         /* a HIP runtime call failed (see pf_last_error) */
    PF_ERR_NOMEM = 4,       /* device or host allocation failed */
    PF_ERR_UNSUPPORTED = 5, /* variant / tile combination not compiled in */
    PF_ERR_CSR = 6,         /* malformed CSR: row_ptr[0]!=0, decreasing, row_ptr[m]!=nnz, col out of range */
    PF_ERR_KERNEL = 7,      /* a kernel found an inconsistent tile (corrupted row_ptr after planning) */
    PF_ERR_IO = 8           /* a file could not be read or parsed (pf_mtx_last_error says why) */
};

/* ---- value types ----------------------------------------------------------- */
/* PF_F16: val, x and y hold IEEE binary16 values (2 bytes each); products and row sums are formed in
 * fp32 and each row sum is rounded to half once.  Every variant: FLAT (tiles 1024, 2048; hybrid plans in
 * dense mode without x halves; no band path), ADAPTIVE (its fp32 tiles), PREFREE (its tile-boundary rows' fp32 partials added in tile order by a
 * second kernel, where the reference adds half values with atomics). */
enum pf_dtype { PF_F64 = 0, PF_F32 = 1, PF_F16 = 2 };

/* ---- kernel variants (all compute y = A·x, y overwritten) ------------------
 * PF_AUTO      pick from row-length statistics (pf_select)
 * PF_PREFREE   the reference's algorithm: fixed 512-nnz tiles, per-tile first
 *              row found in-kernel (no pre-pass), thread / 4-lane / block
 *              reduction ladder, atomics on tile-boundary rows over a zeroed y
 *              (preFreeSpMV.cu:407-483, ladder "code 3")
 * PF_ADAPTIVE  CSR-adaptive row blocks found on the fly: tiles of the merged
 *              (row, nnz) key space, whole short rows per tile, long rows split
 *              across tiles and combined deterministically (no atomics)
 * PF_FLAT      flat fixed-nnz tiles: every row crossing a tile edge is split
 *              and combined deterministically (no atomics)                  */
enum pf_variant { PF_AUTO = 0, PF_PREFREE = 1, PF_ADAPTIVE = 2, PF_FLAT = 3 };

/* Row-length statistics of a CSR matrix (one pass over row_ptr). */
typedef struct pf_row_stats {
    long long m;
    long long nnz;
    long long max_row_len;
    long long min_row_len;
    long long n_empty_rows;
    long long n_decreasing;   /* rows with row_ptr[r+1] < row_ptr[r] (must be 0) */
    long long row_ptr_first;  /* row_ptr[0] (must be 0) */
    long long row_ptr_last;   /* row_ptr[m] (must be nnz) */
    long long n_bad_cols;     /* col[j] outside [0,n); -1 when columns were not checked */
    long long hist_log2[33];  /* [0]: empty rows; [k]: rows with 2^(k-1) <= len < 2^k */
    long long n_long_rows;    /* rows longer than 256 nnz (the longest a row-aligned tile takes) */
    long long max_short_row_len; /* longest row of at most 256 nnz */
    long long guess_dev;      /* largest |r - row_ptr[r] * m / nnz| over the rows, rounded up: how far a row
                                 lies from where the mean density puts it (sizes the row searches' first
                                 probe round) */
    long long line_q1_row_ptr;   /* row_ptr[m / 4] and row_ptr[3m / 4]: the line through (row_ptr[m / 4], m / 4) */
    long long line_q3_row_ptr;   /* and (row_ptr[3m / 4], 3m / 4) puts row_ptr values at rows */
    long long line_far_rows;     /* rows more than 28 rows from where that line puts their row_ptr (m when the
                                    line is undefined: m < 4 or row_ptr[m / 4] == row_ptr[3m / 4]) */
} pf_row_stats;

/* Launch configuration chosen for a matrix. */
typedef struct pf_plan_info {
    int variant;          /* resolved pf_variant (never PF_AUTO) */
    int dtype;            /* pf_dtype */
    int tile;             /* keys per tile (ADAPTIVE: rows+nnz, FLAT/PREFREE: nnz) */
    int long_row_min;     /* ADAPTIVE: rows longer than this are split across tiles */
    int guess_spread;     /* row search: spacing of the interpolated first probe round (the smallest power of
                             two, at most 64, whose 64 probes cover guess_dev; rows of at most 64 nnz), 0 = none */
    int needs_fixup;      /* 1 when split rows need the combine kernel */
    int run_tiles;        /* ADAPTIVE: consecutive tiles walked by one wave64 */
    int keep_cached;      /* ADAPTIVE: 1 = col/val read with ordinary loads (the matrix fits the
                             256 MB MALL and stays cached across calls), 0 = non-temporal loads */
    long long ntiles;     /* logical tiles */
    long long grid;       /* workgroups launched (tiles rounded up to a multiple of the XCD count) */
    size_t workspace_bytes;
    int row_aligned;      /* FLAT 1024/2048: 1 = each tile owns the rows starting in it (all rows hold at
                             most 256 nnz); no row is split and no combine kernel runs */
    int x_windows;        /* split-row FLAT 1024/2048: 1 = tiles dealt to XCDs by the eighth of x they
                             start in (chosen when rows span 4+ tiles and x exceeds one XCD's 4 MB L2) */
    long long chunk_nnz;  /* FLAT 1024/2048 without x windows: tiles dealt to the 8 XCDs in chunks of
                             consecutive tiles of about this many nnz (0 = one chunk per XCD) */
    int ladder;           /* PREFREE: the reduction ladder 1..5 (see pf_plan_set_ladder); 0 otherwise */
    int hybrid;           /* 1: the rows over 256 nnz are summed apart from the others, which go in row-aligned
                             tiles; chosen at planning (PF_AUTO or PF_FLAT with the default tile, columns given)
                             for split-row FLAT matrices of that shape (pf_plan_set_hybrid switches it).  Dense
                             mode: rows of at least a few thousand nnz with sorted columns ("dense rows") summed by
                             x windows staged in LDS, shared by 128 rows at a time.  Long mode (long_tiles > 0):
                             the long rows cut into tiles of 1024 nnz dealt to the XCDs by their first column. */
    long long dense_rows; /* hybrid plans: the rows summed apart (dense rows, or long rows in long mode) */
    int x_halves;         /* hybrid plans: 1 = the runs' tiles are processed once per half of x, by XCDs 0-3 and
                             4-7, so each XCD's random gathers fall in half of x (chosen when x is 4-24 MB) */
    int long_tiles;       /* hybrid plans in long mode: tiles of the long rows; 0 otherwise */
    double guess_a, guess_b; /* row-aligned FLAT tiles: when guess_a > 0, their row searches' first probe round
                                is centred on row guess_a * key + guess_b with a spacing of 1 (the line of
                                pf_row_stats, chosen when at most m / 256 rows lie over 28 rows from it); 0:
                                key * m / nnz with guess_spread */
    int band_w;              /* row-aligned FLAT plans, fp64 / fp32: > 0 when calls run the band kernel, which
                                keeps x[first row - band_w, last row + band_w) of each step of 4096 nnz in LDS
                                (85% or more of the columns lie within +-band_w of their row) and reads its steps
                                from the row map (searched by pfk_row_map on a first call and on every call of a
                                plan that remembers no rows); 0: the tiles' own kernel.  See pf_plan_set_band. */
} pf_plan_info;

typedef struct pf_plan pf_plan;

/* Version as 10000*major + 100*minor + patch. */
int pf_version(void);
const char *pf_status_string(int status);
/* Text of the last HIP error seen by this thread ("" if none). */
const char *pf_last_error(void);

/* Row statistics of a device CSR (synchronises `stream`).  d_col may be NULL;
 * otherwise col is range-checked against n (n_bad_cols). */
int pf_row_stats_compute(const int *d_row_ptr, const int *d_col, int m, int n, long long nnz,
                         pf_row_stats *out, void *stream);

/* Variant and tile selection from statistics (host only, no GPU call). */
int pf_select(const pf_row_stats *stats, int dtype, int variant, pf_plan_info *out);

/* Analyse a device CSR, choose a variant (PF_AUTO) or honour the requested
 * one, allocate the plan's workspace.  d_col may be NULL to skip the column
 * range check.  Synchronises `stream`.  The plan keeps no pointer to the
 * matrix; it is valid for any matrix with the same row_ptr. */
int pf_plan_create(pf_plan **plan, const int *d_row_ptr, const int *d_col, int m, int n, int nnz,
                   int dtype, int variant, void *stream);
/* Same, with an explicit tile size (0 = default) — used by the tuner. */
int pf_plan_create_tuned(pf_plan **plan, const int *d_row_ptr, const int *d_col, int m, int n,
                         int nnz, int dtype, int variant, int tile, void *stream);
int pf_plan_get_info(const pf_plan *plan, pf_plan_info *out);
/* Row-aligned FLAT plans of fp64 / fp32 matrices whose x exceeds one XCD's L2 (4 MB) and whose columns lie
 * within +-w of their row for 85% or more of the nnz (w a power of two from 64 to 16384 that fits the band
 * kernel's LDS ring): planning measures the band (pfk_band_stats) and, for matrices of under 4 nnz per row
 * on average, turns the band kernel on.  band 1 turns it on for any such plan, 0 off; PF_ERR_UNSUPPORTED for
 * a plan without a band.  Same y either way (bit for bit). */
int pf_plan_set_band(pf_plan *plan, int band);

/* Planning time of a plan made by pf_plan_create / pf_plan_create_tuned: plan_ms is the wall time of the
 * call (statistics, column check, selection, workspace, hybrid tables; the reference pays its pre-pass in
 * cdPre instead), plan_gpu_ms the event-timed GPU time of its kernels (-1 when events were unavailable;
 * 0 for plans made otherwise, e.g. by the tuner).  The rest of plan_ms is host work: allocation, copies,
 * synchronisation and the host's share of the hybrid tables. */
int pf_plan_get_timing(const pf_plan *plan, double *plan_ms, double *plan_gpu_ms);
/* Tuning: consecutive tiles per wave64 of the ADAPTIVE kernel (1..256). */
int pf_plan_set_run_tiles(pf_plan *plan, int run_tiles);
/* Tuning: cache policy of the ADAPTIVE col/val stream (1 = ordinary loads, 0 = non-temporal). */
int pf_plan_set_keep_cached(pf_plan *plan, int keep_cached);
/* FLAT 1024/2048 only: 1 = row-aligned tiles (chosen at planning when every
 * row holds at most 256 nnz), 0 = nnz tiles with split rows combined by a
 * second kernel.  Both give the same y. */
int pf_plan_set_row_aligned(pf_plan *plan, int row_aligned);
/* Split-row FLAT 1024/2048 only: 1 = the plan's first call records, with the row map, which eighth of x
 * each tile starts in, and later calls deal the tiles to the 8 XCDs by it (long rows then read one XCD's
 * share of x from its L2); 0 = tiles dealt by position.  Both give the same y. */
int pf_plan_set_x_windows(pf_plan *plan, int x_windows);
/* FLAT 1024/2048 only: nnz per chunk of consecutive tiles given to one XCD (0 = one chunk of an eighth
 * of the tiles per XCD).  Small chunks keep the eight XCDs streaming neighbouring addresses; large ones
 * keep more of a row's x neighbourhood in one XCD's L2.  All values give the same y. */
int pf_plan_set_chunk_nnz(pf_plan *plan, long long chunk_nnz);
/* PREFREE only: the per-tile reduction ladder, the reference tuner's TEST_CODE_VERSION
 * (scripts/profile_and_generate.py:109-235, ladders at src/spmv_kernel/preFreeSpMV.cu:440-559):
 *   1 thread per row always; 2 block for a single-row tile, else thread per row;
 *   3 (default, the reference's active ladder) thread per row above 32 rows, block for one row,
 *     else 4 lanes per row;
 *   4 as 3, but a tile of 2..32 rows whose longest row holds over 90% of their nnz sums it with 96
 *     threads and the other rows with one thread each (red_row_long_short_specialized);
 *   5 thread per row above 128 rows, block for one row, else groups of 128/rows lanes (2..32) per row.
 * The tile size (pf_plan_create_tuned: 512 or 1024 nnz) is the reference's P_NNZ 4 or 8. */
int pf_plan_set_ladder(pf_plan *plan, int ladder);
/* Plans that PF_AUTO made hybrid (pf_plan_info.hybrid): 0 = split-row FLAT tiles instead, 1 = back to
 * hybrid.  Both give y within rounding of each other (the dense rows' partial sums differ in order).  A hybrid
 * plan is built without the split-row workspace (pf_plan_info.workspace_bytes): the first switch to 0
 * allocates and initialises it on the default stream and synchronises that stream. */
int pf_plan_set_hybrid(pf_plan *plan, int hybrid);
/* Hybrid plans: 1 = run tiles per half of x (see pf_plan_info.x_halves), 0 = once each. */
int pf_plan_set_x_halves(pf_plan *plan, int x_halves);
/* FLAT 1024/2048: 1 (default) = the first call records each tile's first row and later calls read it;
 * 0 = every call searches row_ptr inside the tile kernel (no recorded map, tiles dealt to XCDs by
 * position).  Both give the same y.  The reference times its own row map as a separate pre-pass
 * (preFreeSpMV.cu:604-622); 0 measures what finding the rows costs when nothing is remembered. */
int pf_plan_set_remember_rows(pf_plan *plan, int remember);
int pf_plan_get_stats(const pf_plan *plan, pf_row_stats *out);

/* y = A·x on `stream` (asynchronous; no allocation, no synchronisation).
 * val/x/y are double* for PF_F64, float* for PF_F32 and IEEE binary16 (2 bytes
 * each) for PF_F16.  Calls that share one
 * plan must be ordered on one stream (the plan's workspace is reused). */
int pf_plan_execute(pf_plan *plan, const int *d_row_ptr, const int *d_col, const void *d_val,
                    const void *d_x, void *d_y, void *stream);
/* Reads and clears the plan's device error flag (synchronises `stream`);
 * returns PF_ERR_KERNEL if a kernel saw an inconsistent tile since the last check. */
int pf_plan_check(pf_plan *plan, void *stream);
int pf_plan_destroy(pf_plan *plan);

/* ---- tuning ------------------------------------------------------------------
 * pf_plan_autotune times every compiled configuration for the plan's dtype on
 * the caller's matrix and vectors (ADAPTIVE tiles x run lengths 1..16, FLAT
 * tiles and XCD chunks; PREFREE tiles x its five reduction ladders and the
 * ordinary-load cache policy when asked by `flags`), each as the best of two
 * batches of `reps` back-to-back SpMVs, and switches the plan to the fastest.
 * FLAT row groups (tiles 2..32) are candidates where no row exceeds 256 nnz.
 * When the plan's own call takes under 20 us launched one by one (bound by the
 * host's launch rate), every candidate is timed instead as one captured HIP
 * graph of max(reps, 20) calls on a stream of the tuner's own, so `stream`
 * must not be capturing.  The plan's own configuration (a hybrid plan
 * included) is the first candidate.  d_y holds A·x on return.  Synchronises
 * `stream`; allocates temporary plans and, for graphs, a stream and a graph.
 * The online counterpart of the reference tuner
 * (scripts/profile_and_generate.py:319-418), which compiled and timed each
 * candidate as a separate program. */
enum { PF_TUNE_PREFREE = 1, PF_TUNE_KEEP_CACHED = 2 };
typedef struct pf_tune_result {
    int variant, tile, run_tiles, keep_cached;
    int candidates;     /* configurations timed (including the plan's own) */
    double us;          /* microseconds per SpMV of the chosen configuration */
    double default_us;  /* of the configuration the plan had before tuning */
    long long chunk_nnz; /* FLAT 1024/2048: XCD chunk of the chosen configuration (see pf_plan_info) */
    int ladder;         /* PREFREE: the chosen reduction ladder 1..5; 0 otherwise */
    int hybrid;         /* 1 if the chosen configuration is the plan's own hybrid one */
} pf_tune_result;
int pf_plan_autotune(pf_plan *plan, const int *d_row_ptr, const int *d_col, const void *d_val, const void *d_x,
                     void *d_y, int reps, int flags, void *stream, pf_tune_result *result);

/* Table for PF_AUTO, as written by the offline tuner (prefree-public_amd/tune/autotune.py).
 * Text, one row per line ('#' starts a comment):
 *   <class> <nnz_upper | -1> <rows> <f64|f32|f16> <adaptive|flat|prefree|auto> <tile> <run_tiles | 0>
 *   <keep_cached> <ladder | 0> <hybrid 0|1>
 * (variant auto, tile 0: the matrices of that row keep PF_AUTO's built-in rules)
 * rows: the matrix's row-length class from its statistics — short (no row over 256 nnz, under 4 nnz
 * per row on average), regular (no row over 256 nnz), skewed (longer rows, under 16 nnz per row on
 * average), dense (longer rows, 16 or more on average) — or any.  The first row whose dtype and row
 * class match and whose bound exceeds the matrix's nnz decides (run 0: the built-in run rule; ladder
 * 0: the default ladder; hybrid 0: a FLAT plan stays split-row even with dense rows).  Rows of the
 * older form <class> <nnz_upper> <dtype> <variant> <tile> <run> <keep> match any row class.
 * NULL clears the table.  Without a call, the table named by $PREFREE_TUNING_TABLE is read once (an
 * empty value: none) or, when that is unset, tune/mi355x_tuning_table.txt beside the lib/ directory
 * of this library (the table measured on MI355X that ships with it).  Plans made before the call are
 * unaffected. */
int pf_set_tuning_table(const char *path);
/* Path of the table PF_AUTO consults ("" when none). */
const char *pf_tuning_table(void);

/* One-shot y = A·x: plan, execute, synchronise, destroy. */
int pf_spmv(const int *d_row_ptr, const int *d_col, const void *d_val, const void *d_x, void *d_y,
            int m, int n, int nnz, int dtype, int variant, void *stream);

/* No counterpart in the reference: pf_spmv for callers that cannot allocate device memory (tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments, result and errors as pf_spmv, but no
 * hipMalloc / hipFree and no allocating library call: the row statistics and the plan's workspace live in
 * a fixed 8 MiB device array of the library (PFK_SCRATCH_BYTES, one per device, kept until the process
 * ends).  Matrices whose workspace does not fit are refused with PF_ERR_UNSUPPORTED before any launch
 * (about 230M nnz for fp64 FLAT 2048-nnz tiles, 120M for 1024-nnz tiles; pf_last_error gives the bytes
 * needed).  It copies the row statistics to the host and synchronises `stream` twice, so it must not be
 * called on a stream that is capturing a HIP graph: a caller who captures makes a plan before the capture
 * (pf_plan_create) and captures pf_plan_execute.  Calls on one device from several host threads are
 * serialised by a per-device lock in this library, since they share the one array; each call has
 * finished with it when it returns. */
int pf_spmv_noalloc(const int *d_row_ptr, const int *d_col, const void *d_val, const void *d_x, void *d_y,
                    int m, int n, int nnz, int dtype, int variant, void *stream);

/* ---- synthetic matrices (the benchmark configurations) --------------------
 * cfg 1..5 = C1..C5: 1 uniform 4096^2 16/row, 2 5-point Laplacian 2048^2,
 * 3 power-law n=2M, 4 very sparse n=20M, 5 mixed dense rows n=1M.  Scaled-down
 * shapes for tests: `scale_n` > 0 replaces n (C2: grid side).  Generation is
 * deterministic in (cfg, seed, scale_n) and independent of the thread count.
 * vals: 0 = the configuration's values (U[-1,1], C2 stencil), 1 = initVec
 * known-answer values (v[i] = i % 15, include/common.h:126-133). */
int pf_synth_dims(int cfg, uint64_t seed, int scale_n, int *m, int *n, long long *nnz);
int pf_synth_csr(int cfg, uint64_t seed, int scale_n, int vals, int *row_ptr, int *col,
                 double *val_f64, float *val_f32);
int pf_synth_x(int cfg, uint64_t seed, int n, int vals, double *x_f64, float *x_f32);

/* ---- Matrix Market input (the reference harness's mmio_allinone,
 * utilities/mmio.cpp:1543-1713) ------------------------------------------------
 * Reads a coordinate-format file into newly malloc'ed host arrays (free each
 * with pf_host_free): 1-based indices made 0-based; entries kept in file order,
 * duplicates included; symmetric and hermitian files get every off-diagonal
 * entry mirrored right after it (skew-symmetric files are not mirrored, as in
 * the reference); pattern entries are 1.0, complex entries keep the real part.
 * Returns PF_ERR_IO with a reason in pf_mtx_last_error() for unreadable files. */
int pf_mtx_read(const char *path, int *m, int *n, int *nnz, int *is_symmetric, int **row_ptr, int **col,
                double **val);
const char *pf_mtx_last_error(void);
void pf_host_free(void *p);

/* ---- runtime helpers for hosts without HIP headers (thin wrappers) -------- */
int pf_device_malloc(void **ptr, size_t bytes);
int pf_device_free(void *ptr);
int pf_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream);
int pf_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream);
int pf_stream_synchronize(void *stream);

#ifdef __cplusplus
}
#endif
#endif
