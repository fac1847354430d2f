/*
 * prefree_kernels.h — thin extern "C" HIP layer (libprefree_kernels.so).
 *
 * The gfx950 kernels and the HIP runtime calls the C++ host layer needs.  Only
 * libprefree.so (host C++, g++) calls these; applications use prefree_c.h.
 * Every function returns 0 on success, or a pf_status code (prefree_c.h).
 *
 * Reference counterparts (wang-luhan/preFree-public):
 *   pfk_spmv_prefree      preFreeSpMV_kernel<4,128> launches, src/spmv_kernel/preFreeSpMV.cu:634-645,
 *                         with pre_start_rowPerTile (:3-28, launched :599) folded into the kernel
 *   pfk_spmv_adaptive     no counterpart: CSR-adaptive row blocks found on the fly
 *   pfk_spmv_flat         no counterpart launch: the flat nnz tiling of :407-428 without atomics
 *                         (tile 256: runs of tiles with carried row sums, combine included)
 *   pfk_spmv_fixup        no counterpart: replaces the cross-tile atomicAdd (:67,:91,:142)
 *   pfk_adaptive_owners   no counterpart: the per-pattern split-row table the combine kernel reads
 *   pfk_row_stats         test/statistic.cu:38-98 (per-tile statistics), reduced to row-length stats
 *   pfk_debug_*           expose in-kernel index computations for bit-exact tests
 *   pfk_malloc ... pfk_event_*  CUDA runtime calls of preFreeSpMV.cu:571-661 and CudaTimer
 *                         (include/common.h:66-124)
 */
#ifndef PREFREE_KERNELS_H
#define PREFREE_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Arguments of one SpMV launch.  val/x/y are double*, float* or IEEE binary16 by dtype. */
typedef struct pfk_spmv_args {
    const int *row_ptr;
    const int *col;
    const void *val;
    const void *x;
    void *y;
    int m;
    int n;
    int nnz;
    int tile;          /* keys (ADAPTIVE) or nnz (FLAT, PREFREE) per tile */
    int guess_spread;  /* 0 = plain 64-ary search */
    int run_tiles;     /* ADAPTIVE, FLAT 256: consecutive tiles per wave (0 = default 8) */
    int keep_cached;   /* ADAPTIVE: 1 = ordinary col/val loads (matrix fits the MALL), 0 = non-temporal */
    long long ntiles;
    void *head_slot;   /* [ntiles] partial of the split row entering a tile */
    void *tail_slot;   /* [ntiles] partial of the split row leaving a tile */
    int *owner_row;    /* [ntiles] row whose split starts in the tile, or -1 */
    int *err_flag;     /* [1] set non-zero by a kernel that finds an inconsistent tile */
    int *row_map;      /* FLAT 1024/2048: [2*(ntiles+1)] (first row, row_ptr there) of each tile, or NULL */
    int map_ready;     /* 1: row_map holds the rows an earlier call found; 0: search (and record them) */
    int row_aligned;   /* FLAT 1024/2048: 1 = each tile owns the rows starting in it (every row must hold
                          at most PFK_ALIGN_ROW_MAX nnz); no split rows, no pfk_spmv_fixup */
    int *sched;        /* split-row FLAT 1024/2048: x-window schedule of the tiles, [PFK_SCHED_INTS(ntiles,
                          sched_cap)] ints whose first 16 are zero before the call that records the row map;
                          NULL = tiles dealt to XCDs by position */
    long long sched_cap; /* tiles per XCD list: at least ceil(ntiles / 8) */
    long long chunk_nnz; /* FLAT 1024/2048 without a schedule: the tiles go to the 8 XCDs in chunks of
                            consecutive tiles of about chunk_nnz nnz, chunk i to XCD i % 8; 0 = one chunk
                            of ceil(ntiles / 8) tiles per XCD */
    int ladder;          /* PREFREE: reduction ladder 1..5, the reference tuner's TEST_CODE_VERSION
                            (scripts/profile_and_generate.py:109-235); 0 = 3, the active ladder of
                            preFreeSpMV.cu:466-483 */
    /* Bytes the caller allocated behind each workspace pointer.  Every entry point checks them before
     * any launch against what its kernels touch: head and tail ntiles slots of PFK_SLOT_BYTES(dtype),
     * owner ntiles ints (ADAPTIVE, split-row FLAT, the combine kernel, pfk_adaptive_owners), the row
     * map 8 * (ntiles + 1) bytes and the schedule PFK_SCHED_INTS(ntiles, sched_cap) ints when given;
     * a shortfall is PF_ERR_INVALID with nothing launched. */
    size_t head_bytes;
    size_t tail_bytes;
    size_t owner_bytes;
    size_t row_map_bytes;
    size_t sched_bytes;
    /* Hybrid plans (pfk_spmv_hybrid) only.  Dense rows (sorted columns) are summed by x windows of at most
     * PFK_DENSE_WINDOW(dtype) columns (pfk_dense_nwin, pfk_dense_width); the rows between them form runs, each cut into row-aligned
     * tiles of `tile` nnz (every run row holds at most PFK_ALIGN_ROW_MAX nnz).  ntiles counts the tiles
     * of all runs. */
    const int *dense_rows;   /* [n_dense] row indices, ascending */
    int n_dense;
    int n_win;               /* pfk_dense_nwin(n, dtype) */
    int n_runs;
    const int *runs;         /* [5 * (n_runs + 1)]: tile_begin[n_runs + 1] (the last = ntiles), then row_begin,
                                row_end, nnz_begin, nnz_end [n_runs + 1 each, the last unused] */
    int *run_map;            /* [8 * ntiles] ints: per tile (f, row_ptr[f], l, row_ptr[l], kb, B0, last, 0) */
    int *dense_seg;          /* [n_dense * (n_win + 1)] first nnz of each dense row in each window */
    void *dense_part;        /* [n_dense * n_win] window partial sums, PFK_SLOT_BYTES(dtype) each */
    size_t runs_bytes, run_map_bytes, dense_seg_bytes, dense_part_bytes;
    int x_halves;            /* 1: each run tile is processed twice, by XCDs 0-3 for the columns in the first half
                                of x and by XCDs 4-7 for the second, whose row sums go to half_part and are added
                                to y in that order (each XCD's random gathers then fall in half of x) */
    void *half_part;         /* [m] values of dtype */
    size_t half_part_bytes;
    /* Hybrid plans whose long rows (over PFK_ALIGN_ROW_MAX nnz) are not all dense with sorted columns: those
     * rows (dense_rows, n_dense of them) are cut into tiles of PFK_LONG_TILE nnz, each tile's partial sum
     * computed by one workgroup, and each row's partials added in tile order.  dense_seg, dense_part and
     * n_win are then unused. */
    int long_mode;           /* 1: long-row tiles instead of dense x windows */
    int n_long_tiles;
    const int *long_tiles;   /* [4 * n_long_tiles], in row order: (row index into dense_rows, first nnz loaded
                                (a multiple of 64), first nnz of the row in the tile, end) */
    const int *long_deal;    /* [n_long_tiles] tile indices in the order the 8 XCDs take them: by first column,
                                XCD k the k-th eighth */
    const int *long_row_tiles; /* [n_dense + 1] first tile of each long row; the last = n_long_tiles */
    void *long_part;         /* [n_long_tiles] partial sums, PFK_SLOT_BYTES(dtype) each */
    size_t long_tiles_bytes, long_deal_bytes, long_row_tiles_bytes, long_part_bytes;
    int ovf_cap;             /* row-aligned FLAT tiles (and hybrid runs): an upper bound on the length of any row
                                they hold; 0 = unknown.  When it is at most 64 and the rows are not in the
                                short-row mode (under 4 nnz per row on average), the last row's overflow past a
                                tile's nominal range is loaded with the range, and a tile whose overflow exceeds
                                the bound sets the error flag. */
    /* Hybrid: a second stream (non-blocking, default priority) and two events made with pfk_event_create_fence.
       When all three are set, the runs run on aux_stream alongside the dense-row (or long-row) kernels on the
       caller's stream, which waits for them before the combines.  NULL: one stream, in sequence. */
    void *aux_stream;
    void *ev_fork;
    void *ev_join;
    /* Row-aligned FLAT tiles that search rows: when guess_a > 0 the first probe round for key v is centred on
       row guess_a * v + guess_b, 64 rows apart by 1; else on v * m / nnz, guess_spread apart.  Any values give
       the same rows (a round that does not bracket the key is followed by wider ones). */
    double guess_a, guess_b;
    /* Hybrid plans with x halves (required then): [m] bytes, 1 for the rows summed apart (dense_rows), 0 for
       every other row, so that the halves' add (y += half_part over the runs' rows) and the combine of the rows
       summed apart are one launch (neither writes the other's rows).  A row summed apart whose byte is not 1 is
       left unwritten and sets the error flag; a run row marked 1 loses its second half's sum (not detected). */
    const unsigned char *row_apart;
    size_t row_apart_bytes;
    /* Row-aligned FLAT 1024/2048 plans whose row map is recorded (map_ready 1), fp64 / fp32: when band_w > 0
       the step runs the band kernel instead of the tiles' recorded-rows kernel: steps of PFK_BAND_STEP / tile
       tiles, each workgroup keeping x[first row - band_w, last row + band_w) of its step in an LDS ring of
       PFK_BAND_RING entries and gathering only the columns outside it from memory.  Any columns give the same
       sums (rows of at most 16 nnz in nnz order, bit-identical to the recorded-rows kernel); band_w only
       decides what stays in LDS.  0 < band_w <= PFK_BAND_RING / 2. */
    int band_w;
} pfk_spmv_args;

/* The band kernel: nnz per step (whole tiles of the row map), x entries of its LDS ring, and the band widths
 * its planning statistic counts (64 << i for i < PFK_BAND_WIDTHS). */
#define PFK_BAND_STEP 4096
#define PFK_BAND_RING 12288
#define PFK_BAND_WIDTHS 9

/* nnz per long-row tile of a hybrid plan in long mode. */
#define PFK_LONG_TILE 1024

/* Bytes of one split-row partial (head / tail slot): fp32 in the fp16 mode. */
#define PFK_SLOT_BYTES(dtype) ((dtype) == 0 ? 8 : 4)

/* Columns per x window of a hybrid plan's dense-row kernel, at most (64 KB of LDS fp64/fp32, 32 KB fp16). */
#define PFK_DENSE_WINDOW(dtype) ((dtype) == 0 ? 8192 : 16384)

/* x windows of a dense-mode hybrid plan: the fewest of at most PFK_DENSE_WINDOW(dtype) columns, rounded up to a
 * multiple of 8 so that each XCD takes as many windows as the others. */
static inline int pfk_dense_nwin(long long n, int dtype)
{
    const long long k = (n + PFK_DENSE_WINDOW(dtype) - 1) / PFK_DENSE_WINDOW(dtype);
    return (int)((k + 7) / 8 * 8);
}

/* Columns of each of those windows (the last may reach past n): n / n_win rounded up to a multiple of 64, so
 * every window starts on a 128-byte line of x.  At most PFK_DENSE_WINDOW(dtype) when n_win = pfk_dense_nwin. */
static inline int pfk_dense_width(long long n, int n_win)
{
    const long long c = n_win > 0 ? (n + n_win - 1) / n_win : 0;
    return (int)((c + 63) / 64 * 64);
}

/* y = A x for a hybrid plan (PF_F64 / PF_F32, and PF_F16 with 2048-nnz run tiles and no x halves): the runs' row-aligned tiles, the dense rows' window sums (or, in
 * long mode, the long-row tiles) and their combine, three or four launches.  map_ready 0: the call searches rows and segment bounds (and records them
 * when run_map / dense_seg are given); 1: it reads them. */
int pfk_spmv_hybrid(int dtype, const pfk_spmv_args *a, void *stream);
/* Planning scan of a hybrid plan: every row of at least dmin nnz as (row, row_ptr[row], row_ptr[row+1]) into
 * list[3 * cap] in no particular order; counters[0] = such rows (may exceed cap: then the list is partial),
 * counters[1] = listed rows whose columns decrease somewhere.  counters must be zero on entry. */
int pfk_dense_scan(const int *row_ptr, const int *col, int m, int dmin, int *list, int cap, int *counters,
                   void *stream);
/* out[i] = col[idx[i]] for i < count (planning of long-row tiles: each tile's first column); every idx must lie
 * in [0, nnz). */
int pfk_gather_cols(const int *col, long long nnz, const int *idx, int count, int *out, void *stream);
/* Hybrid planning, no counterpart in the reference: flags[rows[i]] = 1 for each of `count` rows (rows outside
 * [0, nflags) skipped); the other flags are left as they are (the caller zeroes them first). */
int pfk_mark_rows(const int *rows, int count, unsigned char *flags, long long nflags, void *stream);

/* Ints of an x-window schedule. */
#define PFK_SCHED_INTS(ntiles, cap) (16 + 8 * (cap) + (ntiles))

/* Longest row a row-aligned FLAT plan accepts. */
#define PFK_ALIGN_ROW_MAX 256

/* FLAT "tiles" 2, 4, 8, 16, 32: row groups, that many lanes per row and rows by index (k_vector: no tiles, no
 * search, no workspace; for small matrices of short rows). */
#define PFK_ROW_GROUP_TILE(t) ((t) == 2 || (t) == 4 || (t) == 8 || (t) == 16 || (t) == 32)

int pfk_spmv_adaptive(int dtype, const pfk_spmv_args *a, void *stream);
int pfk_spmv_flat(int dtype, const pfk_spmv_args *a, void *stream);
int pfk_spmv_fixup(int dtype, int merged_keys, const pfk_spmv_args *a, void *stream);
/* ADAPTIVE planning step: owner_row[t] = the row whose split starts in tile t, else -1, for every
 * tile (a function of row_ptr and the tiling only; pfk_spmv_adaptive no longer writes it). */
int pfk_adaptive_owners(int dtype, const pfk_spmv_args *a, void *stream);
/* PREFREE zeroes y and runs the reference kernel; fp64/fp32 add each tile-boundary row's partials to y with
 * atomics.  fp16 keeps them in fp32 instead, in head_slot / tail_slot (ntiles floats each: the partial of a
 * tile's first / last row), with each tile's row range in owner_row (2 ints per tile); a second kernel adds a
 * row's partials in tile order and stores it rounded to half once. */
int pfk_spmv_prefree(int dtype, const pfk_spmv_args *a, void *stream);
/* The row map of a row-aligned FLAT plan (tile 1024 or 2048 nnz, ntiles = ceil(nnz / tile)), searched afresh
 * from row_ptr: entry t of ntiles + 1 in a->row_map (room for (ntiles + 1) int2, row_map_bytes) is (f,
 * row_ptr[f]) with f the first row whose row_ptr is at or above t·tile (entry 0: row 0; entry ntiles: row m),
 * as the tiles kernel's search records it (guess_spread / guess_a / guess_b steer the search as there).  Band
 * plans run it before the band kernel on a first call and on every call that remembers no rows.  Replaces the
 * reference's pre-pass pre_start_rowPerTile (src/spmv_kernel/preFreeSpMV.cu:3-28) for these plans. */
int pfk_row_map(const pfk_spmv_args *a, void *stream);
/* Tile sizes compiled in for a variant: writes up to `cap` sizes, returns the count (at most
 * PFK_MAX_TILES, which a buffer of that length always holds). */
#define PFK_MAX_TILES 16
int pfk_supported_tiles(int variant, int dtype, int *tiles, int cap);
/* Long-row threshold the ADAPTIVE kernel uses for a tile size (-1 if unsupported). */
int pfk_adaptive_long_row_min(int dtype, int tile);
/* Wave64s of the ADAPTIVE kernel for (dtype, tile) resident on the current device at once
 * (occupancy per CU x CUs); sizes the tile runs so that one dispatch round covers the matrix. */
int pfk_adaptive_resident_waves(int dtype, int tile, long long *waves);
/* The same for the FLAT kernel of 256-nnz tiles (k_flow). */
int pfk_flow_resident_waves(int dtype, long long *waves);
/* Workgroups a FLAT 1024/2048 launch without a schedule uses for ntiles tiles and chunk_nnz. */
long long pfk_flat_grid(long long ntiles, int tile, long long chunk_nnz);

/* Row statistics.  d_out: PFK_STATS_WORDS unsigned long long (layout in prefree_kernels.hip; the first 46
 * are those of pf_row_stats, in its order of fields after m and nnz). */
#define PFK_STATS_WORDS 50
int pfk_row_stats(const int *row_ptr, const int *col, int m, int n, long long nnz,
                  unsigned long long *d_out, void *stream);
/* The planning scan: pfk_row_stats, and in the same launches every row over PFK_ALIGN_ROW_MAX nnz listed as
 * int4 (row, first nnz, end, 0) in `list` (the first `cap` of them, in no particular order; d_out[46] counts
 * them all), with the column descents col[j] > col[j+1] inside listed rows counted in d_out[47]; d_out[48]
 * is nonzero when that count is incomplete (a list over cap, or a range of col meeting too many listed
 * rows).  col is read once.  list: cap int4, 16-byte aligned. */
int pfk_plan_scan(const int *row_ptr, const int *col, int m, int n, long long nnz, unsigned long long *d_out,
                  void *list, int cap, void *stream);

/* Planning statistic of the band kernel, no counterpart in the reference, over a sample of the rows (every
 * PFK_BAND_SAMPLE-th block of 256 rows): out[i] = the sampled nnz whose column lies within +-(64 << i) of their
 * row (i < PFK_BAND_WIDTHS), out[PFK_BAND_WIDTHS] = the sampled nnz; PFK_BAND_WIDTHS + 1 unsigned long long,
 * zeroed by the call.  A thread per nnz of each sampled block, its row found by bisection of the block's row_ptr. */
#define PFK_BAND_SAMPLE 16
int pfk_band_stats(const int *row_ptr, const int *col, int m, unsigned long long *out, void *stream);

/* Tile descriptors of ADAPTIVE (merged=1) / FLAT (merged=0) for every tile:
 * d_out[8*t + 0..5] = first row, row count, first nnz, end nnz, head split, tail split. */
int pfk_debug_tile_desc(int dtype, int merged_keys, const pfk_spmv_args *a, int *d_out, void *stream);
/* PREFREE's in-kernel first row of every 512-nnz tile, d_out[0..ntiles] (ntiles+1 entries,
 * the last one = m), the map the reference pre-pass writes. */
int pfk_debug_prefree_rows(const int *row_ptr, int m, int nnz, int tile, int *d_out, void *stream);

/* Measurement only (bench.py --probe gather), no counterpart in the reference: the x gathers of an SpMV
 * alone.  One workgroup per 1024 indices streams them (16-byte non-temporal loads, as col is streamed) and
 * reads x[idx[j]] through a buffer resource over x[0, n) with cache policy bits `policy` (gfx950: 1 = sc0,
 * 2 = nt, 16 = sc1; 0, 1, 2, 3, 16, 17, 18 and 19 are compiled); an index outside [0, n) reads zero.
 * `out` receives 4 sums per 1024 indices: out_len values of dtype (PF_F64 / PF_F32) must hold
 * 4 * ceil(count / 1024) of them.  idx 16-byte aligned, 1 <= count < 2^31. */
int pfk_probe_gather(int dtype, const int *idx, long long count, const void *x, long long n, void *out,
                     long long out_len, int policy, void *stream);

/* No counterpart in the reference.  Device scratch for pf_spmv_noalloc, the entry point for callers that
 * cannot allocate (serving loops, harnesses that forbid hipMalloc): a file-scope __device__ array of
 * PFK_SCRATCH_BYTES bytes, 256-byte aligned, one copy per device, held until the process ends.  Writes the
 * current device's address of it (looked up once per device with hipGetSymbolAddress) and its size.
 * Every user on one device shares the same bytes. */
#define PFK_SCRATCH_BYTES (8u << 20)
int pfk_scratch(void **ptr, size_t *bytes);

/* Runtime wrappers. */
int pfk_malloc(void **p, size_t bytes);
int pfk_free(void *p);
int pfk_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream);
int pfk_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream);
int pfk_memcpy_d2d(void *dst, const void *src, size_t bytes, void *stream);
int pfk_fill_zero(void *p, size_t bytes, void *stream);  /* a fill kernel, not hipMemsetAsync */
int pfk_fill_u32(void *p, size_t nwords, unsigned value, void *stream);  /* fill kernel, 32-bit words */
int pfk_stream_create(void **s);
int pfk_stream_destroy(void *s);
int pfk_stream_sync(void *s);
int pfk_event_create(void **e);
int pfk_event_create_fence(void **e);  /* an event without timing, for ordering streams */
int pfk_event_destroy(void *e);
int pfk_event_record(void *e, void *s);
int pfk_event_sync(void *e);
int pfk_event_elapsed_ms(float *ms, void *start, void *stop);
/* A HIP graph of the work queued on `stream` (a non-null stream) between pfk_graph_begin and pfk_graph_end
 * (capture mode thread-local), instantiated into *exec; pfk_graph_end always ends the capture, and on failure
 * sets *exec to NULL.  pf_plan_autotune times launch-bound plans this way. */
int pfk_graph_begin(void *stream);
int pfk_graph_end(void *stream, void **exec);
int pfk_graph_launch(void *exec, void *stream);
int pfk_graph_destroy(void *exec);
int pfk_device_count(int *n);
int pfk_get_device(int *dev);  /* the calling thread's current device */
int pfk_device_name(char *buf, int len);
const char *pfk_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
