/*
 * oracle.h — CPU restatement of the reference CSR SpMV path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or the CPU baseline.  The product (prefree-public_amd/) never links it.
 *
 * Every function cites the reference file:line it restates
 * (wang-luhan/preFree-public).  How each one is pinned (closed forms, brute
 * force, library routines, invariants) is written next to it and exercised by
 * tests/test_oracle.py.
 */
#ifndef PREFREE_ORACLE_H
#define PREFREE_ORACLE_H

#ifdef __cplusplus
extern "C" {
#endif

/* y[i] += sum_j val[j]*x[col[j]] with a fresh accumulator per row, summed in
 * element order, product rounded before the add (built -ffp-contract=off).
 * Restates spmv_serial, test/test_cdspmv.cpp:4-20.
 * Pinned by: dense brute force, scipy.sparse on integer data (exact),
 * closed forms (identity, diagonal, Laplacian with constant x). */
void oracle_spmv_serial_f64(const double *val, const int *row_ptr, const int *col,
                            const double *x, double *y, int m);
void oracle_spmv_serial_f32(const float *val, const int *row_ptr, const int *col,
                            const float *x, float *y, int m);

/* Same arithmetic per row as the serial restatement, rows split over threads
 * in nnz-balanced contiguous chunks; bit-identical to the serial result.
 * The CPU baseline of bench.py.  nthreads <= 0 uses omp_get_max_threads(). */
void oracle_spmv_omp_f64(const double *val, const int *row_ptr, const int *col,
                         const double *x, double *y, int m, int nthreads);
void oracle_spmv_omp_f32(const float *val, const int *row_ptr, const int *col,
                         const float *x, float *y, int m, int nthreads);
int oracle_omp_max_threads(void);

/* Tile -> first row map of the reference pre-pass.  start_row has ntiles+1
 * entries and is zeroed first, as preFreeSpMV.cu:591-595 does.
 * Restates pre_start_rowPerTile, src/spmv_kernel/preFreeSpMV.cu:3-28.
 * Pinned by: closed form upper_bound(row_ptr, t*tile)-1 (numpy searchsorted). */
void oracle_pre_start_row(const int *row_ptr, int m, int tile, int *start_row, int ntiles);

/* Row range [start,end) reduced by tile b.  Restates preFreeSpMV.cu:429-438.
 * faithful_sentinel=1 keeps the reference's "start_row[b+1]==0 means m" rule
 * (:431), which is wrong when row 0 spans more than one tile;
 * faithful_sentinel=0 uses m only for the last tile. */
void oracle_tile_row_range(const int *row_ptr, int m, int tile, const int *start_row,
                           int ntiles, int b, int faithful_sentinel, int *start, int *end);

/* One legal execution of the reference kernel preFreeSpMV_kernel<4,128>
 * (preFreeSpMV.cu:407-483, reduction ladder "code 3") on the CPU: tiles run in
 * increasing order (decreasing with reverse_tiles=1; both are schedules the
 * GPU may produce), atomicAdd contributions land in that order, and every
 * in-tile reduction follows the reference's summation tree (red_row_thread
 * :71-98, red_row_vector<4> + warpReduceSum :100-150, red_row_block :30-69).
 * y must be zeroed by the caller (the reference memsets it, :644).
 * Pinned by: equals oracle_spmv_serial on integer (KAT) data for every input,
 * and bit-equal to it on rows reduced by the sequential thread path. */
void oracle_prefree_sim_f64(const double *val, const int *row_ptr, const int *col,
                            const double *x, double *y, int m, int nnz, int faithful_sentinel,
                            int reverse_tiles);
/* preFreeSpMV_kernel<p_nnz,128> with reduction ladder `code` (1..5, the tuner's
 * TEST_CODE_VERSION), p_nnz 4 or 8; plain / atomics (optional, m ints) count each
 * row's plain stores and atomic adds.  Returns -1 for an unknown code or p_nnz. */
int oracle_prefree_sim_code_f64(const double *val, const int *row_ptr, const int *col, const double *x, double *y,
                                int m, int nnz, int code, int p_nnz, int faithful_sentinel, int reverse_tiles,
                                int *plain, int *atomics);
/* calculate_vector_size<128> (preFreeSpMV.cu:394-405) for n rows, 0 for n <= 0. */
int oracle_prefree_vector_size(int n);

/* eQcheck, test/test_cdspmv.cpp:22-54 (fp64 branch): number of i with
 * |a-b|/max(|a|,|b|) > tol (a NaN comparison counts as a pass, as there). */
long long oracle_eqcheck_f64(const double *ref, const double *ours, int n, double tol);

/* Per-row error normalised by that row's sum_j |a_ij*x_j|.  Returns the max
 * over rows with a non-zero denominator; rows whose denominator is zero must
 * be exactly zero in both vectors, violations are counted in *zero_row_bad.
 * NaN or Inf in either vector counts as an infinite error. */
double oracle_rownorm_maxerr_f64(const double *val, const int *row_ptr, const int *col,
                                 const double *x, const double *yref, const double *y,
                                 int m, long long *zero_row_bad, int *worst_row);
double oracle_rownorm_maxerr_f32(const float *val, const int *row_ptr, const int *col,
                                 const float *x, const float *yref, const float *y,
                                 int m, long long *zero_row_bad, int *worst_row);

/* Byte models, test/test_cdspmv.cpp:305 ("effective": x and y once) and :306
 * ("gather": x counted per nonzero). */
long long oracle_bytes_effective(long long rows, long long cols, long long nnz, int val_bytes);
long long oracle_bytes_gather(long long rows, long long cols, long long nnz, int val_bytes);

/* initVec, include/common.h:126-133: v[i] = (valT)(float)(i % 15). */
void oracle_initvec_f64(double *v, long long n);
void oracle_initvec_f32(float *v, long long n);

#ifdef __cplusplus
}
#endif
#endif
