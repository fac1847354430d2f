// cdspmv.cpp — the benchmark harness of the reference (test/test_cdspmv.cpp:268-327)
// for MI355X: read a Matrix Market file, fill val and x with initVec values
// (v[i] = i % 15, include/common.h:126-133), run the drop-in preFreeSpMV
// (200 warm-up + 4000 timed SpMVs), check y against a sequential CPU SpMV
// (test_cdspmv.cpp:4-20) with the reference's relative test (eQcheck,
// test_cdspmv.cpp:22-54) and print the lines the reference's tuner parses
// ("our_perf: ... ms, our_pre: ... ms").
//
// The vendor comparison runs first, as in the reference (cuSPARSE there,
// test_cdspmv.cpp:155-267, 307): rocSPARSE's default algorithm, 200 warm-up
// and 4000 timed calls (PREFREE_ITERS overrides the count), printed as the
// "cusparse_perf: ... ms, cusparse_pre: ... ms" line the reference's tuner
// parses beside our_perf (scripts/profile_and_generate.py:293-303), followed
// by a "vendor:" line naming rocSPARSE; cusparse_pre is rocSPARSE's analysis
// stage.  fp64 and fp32; --no-vendor skips it.
//
// Differences, all deliberate: "m = .., n = .., nnz = .." is printed (the
// reference tuner looks for "nnz =" but the harness never printed it); the
// wall time of the whole preFreeSpMV call (allocation, host<->device copies,
// planning, warm-up and timed launches) is printed as our_total; a failed
// check exits with status 1 instead of printing "Success!" regardless.
//
// --f16 runs the reference's fp16 build (valT = half, include/common.h:43-46):
// values are IEEE binary16 (pf_half), the sequential check rounds every product
// and every sum to binary16 as the reference's half operators do, and the
// relative tolerance is the reference's 1e-1 (test_cdspmv.cpp:37-52).
//
// usage: cdspmv <matrix.mtx> [--f32|--f16] [--variant auto|prefree|adaptive|flat] [--no-check] [--no-vendor]
#include "PreFree.h"
#include "prefree_c.h"
#include "vendor_spmv.h"

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace {

// IEEE binary16 <-> float.  Every binary16 value is a float, so widening is
// exact; narrowing scales by a power of two (exact) and rounds the scaled
// significand with nearbyint, which rounds to nearest even in the default mode.
float widen(pf_half h)
{
    const int s = h.bits >> 15, e = (h.bits >> 10) & 31, f = h.bits & 1023;
    const float mag = e == 31 ? (f ? NAN : INFINITY)
                    : e == 0  ? std::ldexp((float)f, -24)
                              : std::ldexp((float)(f | 1024), e - 25);
    return s ? -mag : mag;
}

pf_half narrow(float v)
{
    const unsigned short sign = std::signbit(v) ? 0x8000 : 0;
    const float a = std::fabs(v);
    if (std::isnan(a)) return pf_half{0x7e00};
    if (std::isinf(a)) return pf_half{(unsigned short)(sign | 0x7c00)};
    if (a < 0x1p-14f) return pf_half{(unsigned short)(sign | (unsigned short)std::nearbyint(a * 0x1p24f))};
    int ex = 0;
    std::frexp(a, &ex);                         // a = g * 2^ex, g in [0.5, 1)
    int e = ex - 1;                             // a in [2^e, 2^(e+1))
    float q = std::nearbyint(std::ldexp(a, 10 - e));   // 11-bit significand, 1024..2048
    if (q == 2048.0f) q = 1024.0f, ++e;
    if (e > 15) return pf_half{(unsigned short)(sign | 0x7c00)};
    return pf_half{(unsigned short)(sign | ((e + 15) << 10) | ((int)q - 1024))};
}

double to_double(double v) { return v; }
double to_double(float v) { return v; }
double to_double(pf_half v) { return widen(v); }

template <typename T> T from_float(float v) { return (T)v; }
template <> pf_half from_float<pf_half>(float v) { return narrow(v); }

// One operation of the reference's sequential SpMV in type T.  For binary16
// the float result of a product or a sum of two binary16 values is rounded
// once more to binary16; float carries 24 bits >= 2*11+2, so the two
// roundings give the correctly rounded binary16 result of each operation.
double mul_add(double t, double a, double b) { return t + a * b; }
float mul_add(float t, float a, float b) { return t + a * b; }
pf_half mul_add(pf_half t, pf_half a, pf_half b)
{
    return narrow(widen(t) + widen(narrow(widen(a) * widen(b))));
}

template <typename T>
void init_vec(T *v, long long n)
{
    for (long long i = 0; i < n; ++i) v[i] = from_float<T>((float)(i % 15));
}

// The harness's reference y: one accumulator per row, products added in
// element order (test_cdspmv.cpp:4-20).
template <typename T>
void serial_spmv(const T *val, const int *rp, const int *col, const T *x, T *y, int m)
{
    for (int i = 0; i < m; ++i) {
        T t = from_float<T>(0.0f);
        for (int j = rp[i]; j < rp[i + 1]; ++j) t = mul_add(t, val[j], x[col[j]]);
        y[i] = t;                                  // y starts at zero: y[i] + t == t
    }
}

template <typename T>
int check(const T *ref, const T *ours, int n, double tol)
{
    int bad = 0;
    for (int i = 0; i < n; ++i) {
        const double a = to_double(ref[i]), b = to_double(ours[i]);
        const double den = std::fmax(std::fabs(a), std::fabs(b));
        const bool differ = std::isnan(a) != std::isnan(b) || (den > 0 && std::fabs(a - b) / den > tol);
        if (differ) {
            if (bad < 10)
                std::printf("Error at index (%d), res(%4.15f), our(%4.15f), please check your code!\n", i, a, b);
            ++bad;
        }
    }
    if (bad == 0)
        std::printf("Success! All values match within the tolerance for %d elements.\n", n);
    else
        std::printf("FAILED: %d of %d values differ by more than %g.\n", bad, n, tol);
    return bad;
}

// The vendor line: rocSPARSE for fp64 / fp32 (none for fp16).
struct Vendor {
    bool ran = false;
    double ms = 0, pre_ms = 0;
    std::string why;
};

template <typename T>
Vendor run_vendor(const T *val, const int *rp, const int *col, const T *x, int m, int n, int nnz)
{
    Vendor v;
    if constexpr (sizeof(T) == 2) {
        v.why = "no fp16 vendor SpMV in this harness";
    } else {
        std::vector<T> y((size_t)m);
        const char *it = std::getenv("PREFREE_ITERS");
        const int iters = (it && *it) ? std::atoi(it) : 4000;
        char why[256] = "";
        if (vendor_spmv(val, rp, col, x, y.data(), m, n, nnz, 200, iters, &v.ms, &v.pre_ms, why, sizeof why) == 0)
            v.ran = true;
        else
            v.why = why;
    }
    return v;
}

template <typename T>
int run(const char *path, int m, int n, int nnz, int *rp, int *col, bool do_check, bool do_vendor)
{
    std::vector<T> val((size_t)nnz), x((size_t)n), y((size_t)m, from_float<T>(0.0f)), ys((size_t)m, from_float<T>(0.0f));
    init_vec(val.data(), nnz);
    init_vec(x.data(), n);
    std::printf("INIT DONE\n");
    std::printf("m = %d, n = %d, nnz = %d\n", m, n, nnz);

    const Vendor vendor = do_vendor ? run_vendor(val.data(), rp, col, x.data(), m, n, nnz) : Vendor{};
    double cd_time = 0, cd_pre = 0;
    const auto t0 = std::chrono::steady_clock::now();
    preFreeSpMV(val.data(), rp, col, x.data(), y.data(), m, n, nnz, &cd_time, &cd_pre);
    const double total = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();

    const long long vb = sizeof(T);
    const long long data1 = ((long long)nnz + n + m) * vb + (long long)nnz * 4 + ((long long)m + 1) * 4;
    const long long data2 = (2LL * nnz + m) * vb + (long long)nnz * 4 + ((long long)m + 1) * 4;
    std::printf("our_perf:%8.4lf ms, our_pre:%8.4lf ms\n", cd_time, cd_pre);
    if (vendor.ran) {
        std::printf("cusparse_perf:%8.4lf ms, cusparse_pre:%8.4lf ms\n", vendor.ms, vendor.pre_ms);
        std::printf("vendor: rocSPARSE (rocsparse_v2_spmv, default algorithm) on this GPU; cusparse_pre is its "
                    "analysis stage\n");
    } else if (do_vendor) {
        std::printf("vendor: not run (%s)\n", vendor.why.c_str());
    }
    if (cd_time > 0)
        std::printf("our_gflops:%8.4lf, our_bandwidth1:%8.4lf GB/s, our_bandwidth2:%8.4lf GB/s\n",
                    2.0 * nnz / (cd_time * 1e6), data1 / (cd_time * 1e6), data2 / (cd_time * 1e6));
    std::printf("our_total:%8.4lf ms (one preFreeSpMV call: allocation, copies, planning, warm-up and timed SpMVs)\n",
                total);
    (void)path;
    if (!do_check) return 0;
    serial_spmv(val.data(), rp, col, x.data(), ys.data(), m);
    const double tol = sizeof(T) == 8 ? 1e-8 : sizeof(T) == 4 ? 1e-4 : 1e-1;
    return check(ys.data(), y.data(), m, tol) == 0 ? 0 : 1;
}

}  // namespace

int main(int argc, char **argv)
{
    const char *path = nullptr;
    bool f32 = false, f16 = false, do_check = true, do_vendor = true;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        if (a == "--f32") f32 = true, f16 = false;
        else if (a == "--f16") f16 = true, f32 = false;
        else if (a == "--no-check") do_check = false;
        else if (a == "--no-vendor") do_vendor = false;
        else if (a == "--variant" && i + 1 < argc) setenv("PREFREE_VARIANT", argv[++i], 1);
        else if (a == "-h" || a == "--help") path = nullptr, i = argc;
        else if (!path) path = argv[i];
    }
    if (!path) {
        std::printf("Run the code by './cdspmv matrix.mtx [--f32|--f16] [--variant auto|prefree|adaptive|flat] "
                    "[--no-check] [--no-vendor]'.\n");
        return 0;
    }
    std::printf("\n===%s===\n\n", path);
    int m = 0, n = 0, nnz = 0, sym = 0;
    int *rp = nullptr, *col = nullptr;
    double *val = nullptr;
    const int st = pf_mtx_read(path, &m, &n, &nnz, &sym, &rp, &col, &val);
    if (st != PF_OK) {
        std::fprintf(stderr, "cdspmv: cannot read %s: %s\n", path, pf_mtx_last_error());
        return 2;
    }
    const int rc = f16 ? run<pf_half>(path, m, n, nnz, rp, col, do_check, do_vendor)
                 : f32 ? run<float>(path, m, n, nnz, rp, col, do_check, do_vendor)
                       : run<double>(path, m, n, nnz, rp, col, do_check, do_vendor);
    pf_host_free(rp);
    pf_host_free(col);
    pf_host_free(val);
    return rc;
}
