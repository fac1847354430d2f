// dropin.cpp — the reference's one-call API, preFreeSpMV (include/PreFree.h),
// on top of the C ABI.  Restates the host orchestration of
// src/spmv_kernel/preFreeSpMV.cu:563-662: allocate, copy in, analyse, time 200
// warm-up + 4000 SpMVs with events on one stream, time the rows' search (the
// reference's pre-pass slot, cdPre), compute the checked y, copy out, free.
#include "PreFree.h"
#include "prefree_c.h"
#include "prefree_kernels.h"

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

namespace {

[[noreturn]] void die(const char *what, int status)
{
    std::fprintf(stderr, "PreFree error: %s failed: %s (%s)\n", what, pf_status_string(status), pf_last_error());
    std::exit(EXIT_FAILURE);
}

void check(int status, const char *what)
{
    if (status != PF_OK) die(what, status);
}

int env_int(const char *name, int dflt)
{
    const char *v = std::getenv(name);
    return (v && *v) ? std::atoi(v) : dflt;
}

int env_variant()
{
    const char *v = std::getenv("PREFREE_VARIANT");
    if (!v || !*v) return PF_AUTO;
    const std::string s(v);
    if (s == "prefree") return PF_PREFREE;
    if (s == "adaptive") return PF_ADAPTIVE;
    if (s == "flat") return PF_FLAT;
    if (s == "auto") return PF_AUTO;
    std::fprintf(stderr, "PreFree error: unknown PREFREE_VARIANT=%s\n", v);
    std::exit(EXIT_FAILURE);
}

template <typename T>
void run(T *csrVal, int *csrRowPtr, int *csrColInd, T *X_val, T *Y_val, int rowA, int colA, int nnzA,
         double *cdTime, double *cdPre)
{
    const int dtype = sizeof(T) == 8 ? PF_F64 : sizeof(T) == 4 ? PF_F32 : PF_F16;
    if (rowA < 0 || colA < 0 || nnzA < 0) die("argument check", PF_ERR_INVALID);
    void *stream = nullptr;
    check(pfk_stream_create(&stream), "stream create");

    void *d_y = nullptr, *d_x = nullptr, *d_val = nullptr, *d_col = nullptr, *d_rp = nullptr;
    // y in whole 4-byte words (fp16 with an odd row count), so that it can be zeroed word by word
    const size_t y_bytes = (sizeof(T) * (size_t)rowA + 3) & ~(size_t)3;
    check(pf_device_malloc(&d_y, y_bytes), "device allocation");
    check(pf_device_malloc(&d_x, sizeof(T) * (size_t)colA), "device allocation");
    check(pf_device_malloc(&d_val, sizeof(T) * (size_t)nnzA), "device allocation");
    check(pf_device_malloc(&d_col, sizeof(int) * (size_t)nnzA), "device allocation");
    check(pf_device_malloc(&d_rp, sizeof(int) * ((size_t)rowA + 1)), "device allocation");
    check(pf_memcpy_h2d(d_val, csrVal, sizeof(T) * (size_t)nnzA, stream), "copy val");
    check(pf_memcpy_h2d(d_col, csrColInd, sizeof(int) * (size_t)nnzA, stream), "copy col");
    check(pf_memcpy_h2d(d_rp, csrRowPtr, sizeof(int) * ((size_t)rowA + 1), stream), "copy row_ptr");
    check(pf_memcpy_h2d(d_x, X_val, sizeof(T) * (size_t)colA, stream), "copy x");
    check(pf_stream_synchronize(stream), "copy");

    // One-time analysis (row statistics + selection + workspace); its wall time
    // is printed with PREFREE_VERBOSE=1.
    const auto t0 = std::chrono::steady_clock::now();
    pf_plan *plan = nullptr;
    check(pf_plan_create_tuned(&plan, static_cast<int *>(d_rp), static_cast<int *>(d_col), rowA, colA, nnzA, dtype,
                               env_variant(), env_int("PREFREE_TILE", 0), stream),
          "plan");
    const auto t1 = std::chrono::steady_clock::now();
    const double plan_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();

    const int warm = env_int("PREFREE_WARMUP", 200), iters = env_int("PREFREE_ITERS", 4000);
    auto spmv = [&]() {
        check(pf_plan_execute(plan, static_cast<int *>(d_rp), static_cast<int *>(d_col), d_val, d_x, d_y, stream),
              "spmv");
    };
    void *e0 = nullptr, *e1 = nullptr;
    check(pfk_event_create(&e0), "event");
    check(pfk_event_create(&e1), "event");
    auto timed = [&](int n) {  // mean event-timed ms per SpMV over n back-to-back calls
        check(pfk_event_record(e0, stream), "event record");
        for (int i = 0; i < n; ++i) spmv();
        check(pfk_event_record(e1, stream), "event record");
        check(pfk_event_sync(e1), "event sync");
        float ms = 0.f;
        check(pfk_event_elapsed_ms(&ms, e0, e1), "event time");
        return n > 0 ? (double)ms / n : 0.0;
    };
    for (int i = 0; i < warm; ++i) spmv();
    check(pf_stream_synchronize(stream), "warm-up");
    *cdTime = timed(iters);

    // cdPre: what finding the tiles' rows costs per call.  The reference times
    // its separate pre-pass kernel (preFreeSpMV.cu:604-622); here the rows are
    // found inside the SpMV kernel, by its first call (later calls read what it
    // recorded), so cdPre is the mean time of calls that search on every call
    // minus cdTime.  Variants that always search report 0: their search is in cdTime.
    const int pre_iters = env_int("PREFREE_PRE_ITERS", iters / 10 > 20 ? iters / 10 : 20);
    check(pf_plan_set_remember_rows(plan, 0), "search mode");
    for (int i = 0; i < 5; ++i) spmv();
    const double search_ms = timed(pre_iters);
    check(pf_plan_set_remember_rows(plan, 1), "search mode");
    *cdPre = search_ms > *cdTime ? search_ms - *cdTime : 0.0;
    if (env_int("PREFREE_VERBOSE", 0))
        std::fprintf(stderr, "preFreeSpMV: plan %.3f ms, %.6f ms per SpMV, %.6f ms per SpMV searching rows\n", plan_ms,
                     *cdTime, search_ms);

    // The checked result: a fresh y, one SpMV (preFreeSpMV.cu:644-645).
    if (y_bytes) check(pfk_fill_zero(d_y, y_bytes, stream), "zero y");
    spmv();
    check(pf_plan_check(plan, stream), "spmv");
    check(pf_memcpy_d2h(Y_val, d_y, sizeof(T) * (size_t)rowA, stream), "copy y");
    check(pf_stream_synchronize(stream), "copy y");

    pfk_event_destroy(e0);
    pfk_event_destroy(e1);
    pf_plan_destroy(plan);
    pf_device_free(d_y);
    pf_device_free(d_x);
    pf_device_free(d_val);
    pf_device_free(d_col);
    pf_device_free(d_rp);
    pfk_stream_destroy(stream);
}

}  // namespace

void preFreeSpMV(double *csrVal, int *csrRowPtr, int *csrColInd, double *X_val, double *Y_val, int rowA, int colA,
                 int nnzA, double *cdTime, double *cdPre)
{
    run<double>(csrVal, csrRowPtr, csrColInd, X_val, Y_val, rowA, colA, nnzA, cdTime, cdPre);
}

void preFreeSpMV(float *csrVal, int *csrRowPtr, int *csrColInd, float *X_val, float *Y_val, int rowA, int colA,
                 int nnzA, double *cdTime, double *cdPre)
{
    run<float>(csrVal, csrRowPtr, csrColInd, X_val, Y_val, rowA, colA, nnzA, cdTime, cdPre);
}

void preFreeSpMV(pf_half *csrVal, int *csrRowPtr, int *csrColInd, pf_half *X_val, pf_half *Y_val, int rowA, int colA,
                 int nnzA, double *cdTime, double *cdPre)
{
    static_assert(sizeof(pf_half) == 2, "pf_half holds 16 bits");
    run<pf_half>(csrVal, csrRowPtr, csrColInd, X_val, Y_val, rowA, colA, nnzA, cdTime, cdPre);
}
