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

/* ---- one execution of preFreeSpMV_kernel<P_NNZ,128>, preFreeSpMV.cu:407-561 --
 *
 * The reduction ladder is selected by `code`, the tuner's TEST_CODE_VERSION
 * (scripts/profile_and_generate.py:109-235): 1 = red_row_thread only (:440-446),
 * 2 = block / thread (:448-461), 3 = thread / block / vector<4> (:466-483, the
 * active ladder), 4 = as 3 with red_row_long_short_specialized<96> for
 * imbalanced tiles (:485-511 with :152-392), 5 = thread / block / vector<VS>
 * with VS from calculate_vector_size (:513-559, :394-405).  Every warp-level
 * tree is restated as lane 0 of a 32-lane warp sees it.  Tiles run one after
 * the other (reverse_tiles: last first), so atomicAdd becomes a plain += in
 * that order.  `plain` (optional, m ints) counts the rows' non-atomic stores
 * and `atomics` (optional) their atomic adds. */

#define SIM_BLOCK 128
#define SIM_TILE_MAX (SIM_BLOCK * 8)

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

/* warpReduceSum<VS> (:100-114) seen by lane 0 of a VS-lane group: offsets VS/2..1. */
static double group_lane0(double *v, int vs)
{
    for (int o = vs / 2; o >= 1; o /= 2)
        for (int i = 0; i < o; i++) v[i] = v[i] + v[i + o];
    return v[0];
}

typedef struct {
    const int *rp;
    const double *s;
    double *y;
    int *plain, *atomics;
    int base, tile, start, end;
} sim_tile;

static void sim_range(const sim_tile *t, int r, int *a, int *e)
{
    int lo = t->rp[r] - t->base; if (lo < 0) lo = 0;
    int hi = t->rp[r + 1] - t->base; if (hi > t->tile) hi = t->tile;
    *a = lo;
    *e = hi;
}

static void sim_put(const sim_tile *t, int r, double sum)
{
    if (r == t->start || r == t->end - 1) {
        t->y[r] += sum;                   /* atomicAdd */
        if (t->atomics) t->atomics[r]++;
    } else {
        t->y[r] = sum;
        if (t->plain) t->plain[r]++;
    }
}

/* red_row_thread, :71-98 */
static void sim_thread(const sim_tile *t)
{
    for (int r = t->start; r < t->end; r++) {
        int a, e;
        sim_range(t, r, &a, &e);
        double sum = 0;
        for (int i = a; i < e; i++) sum += t->s[i];
        sim_put(t, r, sum);
    }
}

/* red_row_block, :30-69 (always an atomicAdd) */
static void sim_block(const sim_tile *t)
{
    const int r = t->start;
    int a, e;
    sim_range(t, r, &a, &e);
    double th[SIM_BLOCK];
    for (int k = 0; k < SIM_BLOCK; k++) {
        double acc = 0;
        for (int j = a + k; j < e; j += SIM_BLOCK) acc += t->s[j];
        th[k] = acc;
    }
    double fin = 0;
    for (int w = 0; w < SIM_BLOCK / 32; w++) fin += warp32_lane0(th + 32 * w);
    t->y[r] += fin;
    if (t->atomics) t->atomics[r]++;
}

/* red_row_vector<VS>, :116-150 */
static void sim_vector(const sim_tile *t, int vs)
{
    for (int r = t->start; r < t->end; r++) {
        int a, e;
        sim_range(t, r, &a, &e);
        double l[32];
        for (int q = 0; q < vs; q++) {
            double acc = 0;
            for (int i = a + q; i < e; i += vs) acc += t->s[i];
            l[q] = acc;
        }
        sim_put(t, r, group_lane0(l, vs));
    }
}

/* is_imbalanced_warp, :342-373: the longest of the first 32 rows (whole row
 * lengths) holds more than 90% of their nnz, compared in float. */
static int sim_imbalanced(const sim_tile *t)
{
    const int n = t->end - t->start;
    long long total = 0;
    int mx = 0;
    for (int lane = 0; lane < 32; lane++) {
        int len = 0;
        if (lane < n) len = t->rp[t->start + lane + 1] - t->rp[t->start + lane];
        total += len;
        if (len > mx) mx = len;
    }
    const float dominance = 0.9f;
    return n > 1 && total > 0 && (float)mx > (float)(int)total * dominance;
}

/* red_row_long_short_specialized<96>, :152-340 (called with 2 <= n <= 32) */
static void sim_long_short(const sim_tile *t)
{
    const int n = t->end - t->start;
    /* phase 1: longest row by a shfl_down max-with-index tree; a lane past the
     * warp's end keeps its own value; a tie keeps the lane's own index */
    int len[32], idx[32];
    for (int lane = 0; lane < 32; lane++) {
        len[lane] = lane < n ? t->rp[t->start + lane + 1] - t->rp[t->start + lane] : -1;
        idx[lane] = lane;
    }
    for (int o = 16; o > 0; o >>= 1) {
        int nl[32], ni[32];
        for (int lane = 0; lane < 32; lane++) {
            const int src = lane + o < 32 ? lane + o : lane;
            nl[lane] = len[lane];
            ni[lane] = idx[lane];
            if (len[src] > len[lane]) { nl[lane] = len[src]; ni[lane] = idx[src]; }
        }
        memcpy(len, nl, sizeof len);
        memcpy(idx, ni, sizeof idx);
    }
    const int li = idx[0];
    double fin_sums[32];
    for (int i = 0; i < 32; i++) fin_sums[i] = 0.0;
    /* phase 2, team A: 96 threads stride the long row; one tree per 32-lane warp */
    double th[96];
    {
        int a, e;
        sim_range(t, t->start + li, &a, &e);
        for (int k = 0; k < 96; k++) {
            double acc = 0;
            for (int j = a + k; j < e; j += 96) acc += t->s[j];
            th[k] = acc;
        }
    }
    double wsum[3];
    for (int w = 0; w < 3; w++) wsum[w] = warp32_lane0(th + 32 * w);
    /* phase 2, team B: one thread per other row, short sums unrolled left to right */
    for (int i = 0; i < n; i++) {
        if (i == li) continue;
        int a, e;
        sim_range(t, t->start + i, &a, &e);
        const int l = e - a;
        const double *s = t->s;
        double sum = 0;
        switch (l) {
        case 1: sum = s[a]; break;
        case 2: sum = s[a] + s[a + 1]; break;
        case 3: sum = s[a] + s[a + 1] + s[a + 2]; break;
        case 4: sum = s[a] + s[a + 1] + s[a + 2] + s[a + 3]; break;
        case 0: break;
        default:
            for (int k = a; k < e; k++) sum += s[k];
            break;
        }
        fin_sums[i] = sum;
    }
    /* phase 3: the three warp sums through one more 32-lane tree */
    double v[32];
    for (int i = 0; i < 32; i++) v[i] = i < 3 ? wsum[i] : 0.0;
    fin_sums[li] = warp32_lane0(v);
    /* phase 4: rows whose sum is 0.0 are not written */
    for (int i = 0; i < n; i++) {
        if (fin_sums[i] == 0.0) continue;
        sim_put(t, t->start + i, fin_sums[i]);
    }
}

/* calculate_vector_size<128>, :394-405 */
static int sim_vector_size(int n)
{
    if (n >= SIM_BLOCK) return 2;
    const unsigned avg = (unsigned)SIM_BLOCK / (unsigned)n;
    unsigned p2 = 1;
    while (p2 * 2 <= avg) p2 *= 2;
    return p2 > 32 ? 32 : (p2 < 2 ? 2 : (int)p2);
}

int oracle_prefree_sim_code_f64(const double *val, const int *row_ptr, const int *col, const double *x, double *y,
                                int m, int nnz, int code, int p_nnz, int faithful_sentinel, int reverse_tiles,
                                int *plain, int *atomics)
{
    if (code < 1 || code > 5 || (p_nnz != 4 && p_nnz != 8))
        return -1;
    if (nnz <= 0 || m <= 0)
        return 0;
    const int T = SIM_BLOCK * p_nnz;
    const int G = (nnz + T - 1) / T;
    int *start_row = (int *)malloc(sizeof(int) * (size_t)(G + 1));
    oracle_pre_start_row(row_ptr, m, T, start_row, G);
    double s[SIM_TILE_MAX];
    const int last = row_ptr[m] - 1; /* :410 */
    for (int bi = 0; bi < G; bi++) {
        const int b = reverse_tiles ? G - 1 - bi : bi;
        const int base = b * T;
        for (int k = 0; k < T; k++) { /* :416-428 */
            int g = base + k;
            if (g > last) g = last;
            s[k] = val[g] * x[col[g]];
        }
        sim_tile t = {row_ptr, s, y, plain, atomics, base, T, 0, 0};
        oracle_tile_row_range(row_ptr, m, T, start_row, G, b, faithful_sentinel, &t.start, &t.end);
        const int n = t.end - t.start;
        switch (code) {
        case 1:
            sim_thread(&t);
            break;
        case 2:
            if (n == 1) sim_block(&t); else sim_thread(&t);
            break;
        case 3:
            if (n > SIM_BLOCK / 4) sim_thread(&t);
            else if (n == 1) sim_block(&t);
            else sim_vector(&t, 4);
            break;
        case 4:
            if (n > SIM_BLOCK / 4) sim_thread(&t);
            else if (n == 1) sim_block(&t);
            else if (sim_imbalanced(&t)) sim_long_short(&t);
            else sim_vector(&t, 4);
            break;
        case 5:
            if (n > SIM_BLOCK) sim_thread(&t);
            else if (n == 1) sim_block(&t);
            else if (n > 0) sim_vector(&t, sim_vector_size(n));
            break;
        }
    }
    free(start_row);
    return 0;
}

void oracle_prefree_sim_f64(const double *val, const int *row_ptr, const int *col,
                            const double *x, double *y, int m, int nnz, int faithful_sentinel,
                            int reverse_tiles)
{
    oracle_prefree_sim_code_f64(val, row_ptr, col, x, y, m, nnz, 3, 4, faithful_sentinel, reverse_tiles, NULL, NULL);
}

int oracle_prefree_vector_size(int n) { return n > 0 ? sim_vector_size(n) : 0; }

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
