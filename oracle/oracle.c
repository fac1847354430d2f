/*
 * oracle.c — CPU restatement of the reference CSR SpMV path
 * (wang-luhan/preFree-public).  TEST INFRASTRUCTURE ONLY: loaded by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker or
 * the CPU baseline, never by the product.  Built with -ffp-contract=off so a
 * product is rounded before it is added, as in the reference build (no -O or
 * -march flags in its CMakeLists.txt, hence no FMA).
 */
#include "oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

/* ---- spmv_serial, test/test_cdspmv.cpp:4-20 ------------------------------ */

void oracle_spmv_serial_f64(const double *val, const int *row_ptr, const int *col,
                            const double *x, double *y, int m)
{
    for (int i = 0; i < m; i++) {
        double t = 0.0;
        const int p = row_ptr[i];
        const int len = row_ptr[i + 1] - p;
        for (int j = 0; j < len; j++) {
            const int c = col[j + p];
            t = t + val[j + p] * x[c];
        }
        y[i] = y[i] + t;
    }
}

void oracle_spmv_serial_f32(const float *val, const int *row_ptr, const int *col,
                            const float *x, float *y, int m)
{
    for (int i = 0; i < m; i++) {
        float t = 0.0f;
        const int p = row_ptr[i];
        const int len = row_ptr[i + 1] - p;
        for (int j = 0; j < len; j++) {
            const int c = col[j + p];
            t = t + val[j + p] * x[c];
        }
        y[i] = y[i] + t;
    }
}

/* First row r with row_ptr[r] >= target (lower bound over row_ptr[0..m]). */
static int first_row_at_or_after(const int *row_ptr, int m, long long target)
{
    int lo = 0, hi = m;
    while (lo < hi) {
        const int mid = lo + (hi - lo) / 2;
        if ((long long)row_ptr[mid] < target)
            lo = mid + 1;
        else
            hi = mid;
    }
    return lo;
}

int oracle_omp_max_threads(void) { return omp_get_max_threads(); }

#define ORACLE_OMP_BODY(T)                                                           \
    const long long nnz = row_ptr[m];                                                \
    if (nthreads <= 0)                                                               \
        nthreads = omp_get_max_threads();                                            \
    _Pragma("omp parallel num_threads(nthreads)")                                    \
    {                                                                                \
        const int tid = omp_get_thread_num();                                        \
        const int nt = omp_get_num_threads();                                        \
        const int r0 = tid == 0 ? 0 : first_row_at_or_after(row_ptr, m, nnz * tid / nt); \
        const int r1 = tid == nt - 1 ? m                                             \
                                     : first_row_at_or_after(row_ptr, m, nnz * (tid + 1) / nt); \
        for (int i = r0; i < r1; i++) {                                              \
            T t = (T)0;                                                              \
            const int p = row_ptr[i];                                                \
            const int len = row_ptr[i + 1] - p;                                      \
            for (int j = 0; j < len; j++)                                            \
                t = t + val[j + p] * x[col[j + p]];                                  \
            y[i] = y[i] + t;                                                         \
        }                                                                            \
    }

void oracle_spmv_omp_f64(const double *val, const int *row_ptr, const int *col,
                         const double *x, double *y, int m, int nthreads)
{
    ORACLE_OMP_BODY(double)
}

void oracle_spmv_omp_f32(const float *val, const int *row_ptr, const int *col,
                         const float *x, float *y, int m, int nthreads)
{
    ORACLE_OMP_BODY(float)
}

/* ---- pre_start_rowPerTile, src/spmv_kernel/preFreeSpMV.cu:3-28 ----------- */

void oracle_pre_start_row(const int *row_ptr, int m, int tile, int *start_row, int ntiles)
{
    memset(start_row, 0, sizeof(int) * (size_t)(ntiles + 1)); /* :591-595 */
    for (int r = 0; r < m; r++) {
        const int a = row_ptr[r];
        const int b = row_ptr[r + 1];
        if (a == b)
            continue;
        const int first = (a + tile - 1) / tile; /* divup, include/common.h:60-64 */
        const int last = (b - 1) / tile;
        for (int i = first; i <= last; ++i)
            start_row[i] = r;
    }
}

/* ---- tile row range, preFreeSpMV.cu:429-438 ------------------------------- */

void oracle_tile_row_range(const int *row_ptr, int m, int tile, const int *start_row,
                           int ntiles, int b, int faithful_sentinel, int *start, int *end)
{
    int s = start_row[b] < m ? start_row[b] : m;
    int e;
    if (faithful_sentinel) {
        e = start_row[b + 1] < m ? start_row[b + 1] : m;
        e = (e == 0) ? m : e;
    } else {
        e = (b + 1 >= ntiles) ? m : (start_row[b + 1] < m ? start_row[b + 1] : m);
    }
    if (row_ptr[e] % tile != 0 || e == s)
        e = (e + 1 < m) ? e + 1 : m;
    *start = s;
    *end = e;
}

/* ---- one execution of preFreeSpMV_kernel<4,128>, preFreeSpMV.cu:407-483 --- */

#define SIM_BLOCK 128
#define SIM_PNNZ 4
#define SIM_TILE (SIM_BLOCK * SIM_PNNZ)

/* warpReduceSum tree seen by lane 0 of a 32-lane warp (offsets 16..1),
 * preFreeSpMV.cu:49-53 and :100-114. */
static double warp32_lane0(const double *v)
{
    double u[16], w[8], x4[4], y2[2];
    for (int i = 0; i < 16; i++) u[i] = v[i] + v[i + 16];
    for (int i = 0; i < 8; i++) w[i] = u[i] + u[i + 8];
    for (int i = 0; i < 4; i++) x4[i] = w[i] + w[i + 4];
    for (int i = 0; i < 2; i++) y2[i] = x4[i] + x4[i + 2];
    return y2[0] + y2[1];
}

void oracle_prefree_sim_f64(const double *val, const int *row_ptr, const int *col,
                            const double *x, double *y, int m, int nnz, int faithful_sentinel,
                            int reverse_tiles)
{
    if (nnz <= 0 || m <= 0)
        return;
    const int G = (nnz + SIM_TILE - 1) / SIM_TILE;
    int *start_row = (int *)malloc(sizeof(int) * (size_t)(G + 1));
    oracle_pre_start_row(row_ptr, m, SIM_TILE, start_row, G);
    double s[SIM_TILE];
    const int last = row_ptr[m] - 1; /* :410 */
    for (int bi = 0; bi < G; bi++) {
        const int b = reverse_tiles ? G - 1 - bi : bi;
        const int base = b * SIM_TILE;
        for (int k = 0; k < SIM_TILE; k++) { /* :416-428 */
            int g = base + k;
            if (g > last) g = last;
            s[k] = val[g] * x[col[g]];
        }
        int start, end;
        oracle_tile_row_range(row_ptr, m, SIM_TILE, start_row, G, b, faithful_sentinel, &start, &end);
        const int n = end - start;
        if (n > SIM_BLOCK / 4) {
            /* red_row_thread, :71-98 */
            for (int r = start; r < end; r++) {
                int a = row_ptr[r] - base; if (a < 0) a = 0;
                int e = row_ptr[r + 1] - base; if (e > SIM_TILE) e = SIM_TILE;
                double sum = 0;
                for (int i = a; i < e; i++) sum += s[i];
                if (r == start || r == end - 1) y[r] += sum; else y[r] = sum;
            }
        } else if (n == 1) {
            /* red_row_block, :30-69 */
            const int r = start;
            int a = row_ptr[r] - base; if (a < 0) a = 0;
            int e = row_ptr[r + 1] - base; if (e > SIM_TILE) e = SIM_TILE;
            double th[SIM_BLOCK];
            for (int t = 0; t < SIM_BLOCK; t++) {
                double acc = 0;
                for (int j = a + t; j < e; j += SIM_BLOCK) acc += s[j];
                th[t] = acc;
            }
            double fin = 0;
            for (int w = 0; w < SIM_BLOCK / 32; w++) fin += warp32_lane0(th + 32 * w);
            y[r] += fin;
        } else if (n > 0) {
            /* red_row_vector<VECTOR_SIZE=4>, :116-150 */
            for (int r = start; r < end; r++) {
                int a = row_ptr[r] - base; if (a < 0) a = 0;
                int e = row_ptr[r + 1] - base; if (e > SIM_TILE) e = SIM_TILE;
                double l[4];
                for (int q = 0; q < 4; q++) {
                    double acc = 0;
                    for (int i = a + q; i < e; i += 4) acc += s[i];
                    l[q] = acc;
                }
                const double sum = (l[0] + l[2]) + (l[1] + l[3]);
                if (r == start || r == end - 1) y[r] += sum; else y[r] = sum;
            }
        }
    }
    free(start_row);
}

/* ---- eQcheck, test/test_cdspmv.cpp:22-54 ---------------------------------- */

long long oracle_eqcheck_f64(const double *ref, const double *ours, int n, double tol)
{
    long long bad = 0;
    for (int i = 0; i < n; i++) {
        const double a = ref[i], b = ours[i];
        if (fabs(a - b) / fmax(fabs(a), fabs(b)) > tol)
            bad++;
    }
    return bad;
}

/* ---- north-star per-row normalised error --------------------------------- */

#define ORACLE_ROWNORM_BODY(T)                                                     \
    double worst = 0.0;                                                            \
    long long zbad = 0;                                                            \
    int wrow = -1;                                                                 \
    for (int i = 0; i < m; i++) {                                                  \
        double den = 0.0;                                                          \
        for (int j = row_ptr[i]; j < row_ptr[i + 1]; j++)                          \
            den += fabs((double)val[j] * (double)x[col[j]]);                       \
        const double a = (double)yref[i], b = (double)y[i];                        \
        if (!isfinite(a) || !isfinite(b)) {                                        \
            worst = INFINITY; wrow = i; continue;                                  \
        }                                                                          \
        if (den == 0.0) {                                                          \
            if (a != 0.0 || b != 0.0) zbad++;                                      \
            continue;                                                              \
        }                                                                          \
        const double e = fabs(a - b) / den;                                        \
        if (e > worst) { worst = e; wrow = i; }                                    \
    }                                                                              \
    if (zero_row_bad) *zero_row_bad = zbad;                                        \
    if (worst_row) *worst_row = wrow;                                              \
    return worst;

double oracle_rownorm_maxerr_f64(const double *val, const int *row_ptr, const int *col,
                                 const double *x, const double *yref, const double *y,
                                 int m, long long *zero_row_bad, int *worst_row)
{
    ORACLE_ROWNORM_BODY(double)
}

double oracle_rownorm_maxerr_f32(const float *val, const int *row_ptr, const int *col,
                                 const float *x, const float *yref, const float *y,
                                 int m, long long *zero_row_bad, int *worst_row)
{
    ORACLE_ROWNORM_BODY(float)
}

/* ---- byte models, test/test_cdspmv.cpp:305-306 ---------------------------- */

long long oracle_bytes_effective(long long rows, long long cols, long long nnz, int val_bytes)
{
    return (nnz + cols + rows) * val_bytes + nnz * 4 + (rows + 1) * 4;
}

long long oracle_bytes_gather(long long rows, long long cols, long long nnz, int val_bytes)
{
    (void)cols;
    return (nnz + nnz + rows) * val_bytes + nnz * 4 + (rows + 1) * 4;
}

/* ---- initVec, include/common.h:126-133 ------------------------------------ */

void oracle_initvec_f64(double *v, long long n)
{
    for (long long i = 0; i < n; ++i)
        v[i] = (double)(float)(i % 15);
}

void oracle_initvec_f32(float *v, long long n)
{
    for (long long i = 0; i < n; ++i)
        v[i] = (float)(i % 15);
}
