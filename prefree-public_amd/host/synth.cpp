// synth.cpp — seeded generators of the five benchmark matrices C1..C5 and
// their x vectors (prefree_c.h: pf_synth_*).
//
// Every random draw comes from a SplitMix64 stream keyed by
// (seed, configuration, scale, purpose, row or column index), so the output
// does not depend on the number of OpenMP threads.  Columns are distinct and
// sorted within each row.  Shapes (n = rows = columns):
//   C1  n=4096, exactly 16 columns per row, uniform without replacement
//   C2  5-point Laplacian on a side x side grid (side=2048): 4 on the diagonal, -1 off it
//   C3  n=2,000,000, length min(200000, max(1, floor(u^(-1/1.1)))) (Pareto, density exponent 2.1)
//   C4  n=20,000,000, length Poisson(2.5); each column within +-4096 of the diagonal
//       with probability 0.9, else uniform over [0, n)
//   C5  n=1,000,000, 1000 seeded dense rows of U[50000, 500000] columns, the
//       rest U[8, 64] columns, all uniform without replacement
// With scale_n > 0 the same recipes run at n = scale_n (C2: side = scale_n;
// C5: n/1000 dense rows of U[n/20, n/2]).  Values are U[-1,1] (the C2 stencil
// for C2) or, with vals = 1, the reference's known-answer initVec values.
#include "prefree_c.h"

#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

namespace {

inline uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

struct Rng {
    uint64_t s;
    uint64_t next()
    {
        s += 0x9E3779B97F4A7C15ull;
        return mix64(s);
    }
    double u01() { return (double)(next() >> 11) * 0x1.0p-53; }  // [0, 1)
    double sym() { return 2.0 * u01() - 1.0; }                    // [-1, 1)
    long long below(long long n) { return (long long)(u01() * (double)n); }
    long long range(long long lo, long long hi) { return lo + below(hi - lo + 1); }  // [lo, hi]
};

enum Purpose : uint64_t { kLen = 1, kCols = 2, kVals = 3, kX = 4, kDense = 5 };

struct Spec {
    int cfg;
    uint64_t seed;
    int scale;
    long long n;     // rows = columns
    int side;        // C2 grid side
    int len_cap;     // C3 cap
    int dense_lo, dense_hi, n_dense;  // C5
};

Rng stream(const Spec &s, uint64_t purpose, uint64_t index)
{
    const uint64_t k = mix64(s.seed ^ mix64(((uint64_t)s.cfg << 40) ^ (uint64_t)(uint32_t)s.scale));
    return Rng{mix64(k ^ mix64(purpose * 0xD6E8FEB86659FD93ull + index))};
}

bool make_spec(int cfg, uint64_t seed, int scale_n, Spec &s)
{
    s = Spec{cfg, seed, scale_n, 0, 0, 0, 0, 0, 0};
    switch (cfg) {
    case 1: s.n = scale_n > 0 ? scale_n : 4096; return s.n >= 16;
    case 2:
        s.side = scale_n > 0 ? scale_n : 2048;
        s.n = (long long)s.side * s.side;
        return s.side >= 1 && s.n < (1ll << 31);
    case 3:
        s.n = scale_n > 0 ? scale_n : 2000000;
        s.len_cap = (int)std::min<long long>(200000, s.n);
        return s.n >= 1;
    case 4: s.n = scale_n > 0 ? scale_n : 20000000; return s.n >= 1;
    case 5:
        s.n = scale_n > 0 ? scale_n : 1000000;
        s.n_dense = (int)std::max<long long>(1, s.n / 1000);
        s.dense_lo = (int)std::max<long long>(1, s.n / 20);
        s.dense_hi = (int)std::max<long long>(s.dense_lo, s.n / 2);
        return s.n >= 64;
    }
    return false;
}

// Rows of C5 that are dense: n_dense distinct rows (Floyd's sampling), sorted.
std::vector<long long> dense_rows(const Spec &s)
{
    std::vector<long long> pick;
    if (s.cfg != 5) return pick;
    Rng r = stream(s, kDense, 0);
    std::vector<long long> chosen;
    chosen.reserve(s.n_dense);
    for (long long j = s.n - s.n_dense; j < s.n; ++j) {
        const long long t = r.range(0, j);
        if (std::find(chosen.begin(), chosen.end(), t) == chosen.end()) chosen.push_back(t);
        else chosen.push_back(j);
    }
    std::sort(chosen.begin(), chosen.end());
    return chosen;
}

long long row_length(const Spec &s, long long i, const std::vector<long long> &dense)
{
    switch (s.cfg) {
    case 1: return 16;
    case 2: {
        const long long r = i / s.side, c = i % s.side;
        return 1 + (r > 0) + (c > 0) + (c < s.side - 1) + (r < s.side - 1);
    }
    case 3: {
        Rng g = stream(s, kLen, (uint64_t)i);
        const double u = 1.0 - g.u01();  // (0, 1]
        const double L = std::floor(std::pow(u, -1.0 / 1.1));
        return (long long)std::min<double>((double)s.len_cap, std::max(1.0, L));
    }
    case 4: {
        Rng g = stream(s, kLen, (uint64_t)i);
        const double limit = std::exp(-2.5);
        long long k = 0;
        double p = g.u01();
        while (p > limit) {  // Knuth's product-of-uniforms Poisson sampler
            ++k;
            p *= g.u01();
        }
        return std::min<long long>(k, s.n);
    }
    case 5: {
        Rng g = stream(s, kLen, (uint64_t)i);
        if (std::binary_search(dense.begin(), dense.end(), i)) return g.range(s.dense_lo, s.dense_hi);
        return std::min<long long>(g.range(8, 64), s.n);
    }
    }
    return 0;
}

// L distinct sorted values drawn uniformly from [0, n).
void sample_distinct(Rng &g, long long n, long long L, int *out)
{
    if (L <= 0) return;
    if (L * 16 >= n) {  // selection sampling (Knuth's Algorithm S): one pass over [0, n)
        long long k = 0;
        for (long long c = 0; c < n && k < L; ++c)
            if ((double)(n - c) * g.u01() < (double)(L - k)) out[k++] = (int)c;
        return;
    }
    long long have = 0;
    while (have < L) {
        for (long long k = have; k < L; ++k) out[k] = (int)g.below(n);
        std::sort(out, out + L);
        have = std::unique(out, out + L) - out;
    }
}

// Columns of row i of C4: within +-4096 of i with probability 0.9, else uniform.
void sample_banded(Rng &g, long long n, long long i, long long L, int *out)
{
    const long long lo = std::max<long long>(0, i - 4096), hi = std::min<long long>(n - 1, i + 4096);
    long long have = 0;
    while (have < L) {
        for (long long k = have; k < L; ++k)
            out[k] = (int)(g.u01() < 0.9 ? g.range(lo, hi) : g.below(n));
        std::sort(out, out + L);
        have = std::unique(out, out + L) - out;
    }
}

void row_columns(const Spec &s, long long i, long long L, int *out)
{
    if (s.cfg == 2) {
        const long long c = i % s.side;
        int k = 0;
        if (i >= s.side) out[k++] = (int)(i - s.side);
        if (c > 0) out[k++] = (int)(i - 1);
        out[k++] = (int)i;
        if (c < s.side - 1) out[k++] = (int)(i + 1);
        if (i + s.side < s.n) out[k++] = (int)(i + s.side);
        return;
    }
    Rng g = stream(s, kCols, (uint64_t)i);
    if (s.cfg == 4) sample_banded(g, s.n, i, L, out);
    else sample_distinct(g, s.n, L, out);
}

}  // namespace

extern "C" {

int pf_synth_dims(int cfg, uint64_t seed, int scale_n, int *m, int *n, long long *nnz)
{
    Spec s;
    if (!m || !n || !nnz || !make_spec(cfg, seed, scale_n, s)) return PF_ERR_INVALID;
    const std::vector<long long> dense = dense_rows(s);
    long long total = 0;
#pragma omp parallel for reduction(+ : total) schedule(static)
    for (long long i = 0; i < s.n; ++i) total += row_length(s, i, dense);
    *m = (int)s.n;
    *n = (int)s.n;
    *nnz = total;
    return total < (1ll << 31) ? PF_OK : PF_ERR_UNSUPPORTED;
}

int pf_synth_csr(int cfg, uint64_t seed, int scale_n, int vals, int *row_ptr, int *col, double *val_f64,
                 float *val_f32)
{
    Spec s;
    if (!row_ptr || !make_spec(cfg, seed, scale_n, s) || (vals != 0 && vals != 1)) return PF_ERR_INVALID;
    const std::vector<long long> dense = dense_rows(s);
    const long long n = s.n;
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < n; ++i) row_ptr[i + 1] = (int)row_length(s, i, dense);
    row_ptr[0] = 0;
    long long acc = 0;
    for (long long i = 1; i <= n; ++i) {
        acc += row_ptr[i];
        if (acc >= (1ll << 31)) return PF_ERR_UNSUPPORTED;
        row_ptr[i] = (int)acc;
    }
    if (!col) return PF_OK;
#pragma omp parallel for schedule(dynamic, 256)
    for (long long i = 0; i < n; ++i) {
        const long long p = row_ptr[i], L = row_ptr[i + 1] - p;
        row_columns(s, i, L, col + p);
        if (vals == 1) {  // initVec over the whole value array, include/common.h:126-133
            for (long long j = p; j < p + L; ++j) {
                const double v = (double)(float)(j % 15);
                if (val_f64) val_f64[j] = v;
                if (val_f32) val_f32[j] = (float)v;
            }
        } else if (cfg == 2) {
            for (long long j = p; j < p + L; ++j) {
                const double v = col[j] == (int)i ? 4.0 : -1.0;
                if (val_f64) val_f64[j] = v;
                if (val_f32) val_f32[j] = (float)v;
            }
        } else {
            Rng g = stream(s, kVals, (uint64_t)i);
            for (long long j = p; j < p + L; ++j) {
                const double v = g.sym();
                if (val_f64) val_f64[j] = v;
                if (val_f32) val_f32[j] = (float)v;  // fp64 draw rounded to nearest
            }
        }
    }
    return PF_OK;
}

int pf_synth_x(int cfg, uint64_t seed, int n, int vals, double *x_f64, float *x_f32)
{
    if (n < 0 || cfg < 1 || cfg > 5 || (vals != 0 && vals != 1)) return PF_ERR_INVALID;
    Spec s{cfg, seed, 0, n, 0, 0, 0, 0, 0};
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < n; ++i) {
        double v;
        if (vals == 1) {
            v = (double)(float)(i % 15);
        } else {
            Rng g = stream(s, kX, (uint64_t)i);
            v = g.sym();
        }
        if (x_f64) x_f64[i] = v;
        if (x_f32) x_f32[i] = (float)v;
    }
    return PF_OK;
}

}  // extern "C"
