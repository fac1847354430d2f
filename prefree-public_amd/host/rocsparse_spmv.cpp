// rocsparse_spmv.cpp — the vendor comparison of the reference harness
// (test/test_cdspmv.cpp:155-267, cuSPARSE there) with rocSPARSE on MI355X:
// one rocsparse_spmv algorithm per process, timed on a benchmark matrix, its y
// checked against this library's y on the same inputs.
//
// rocSPARSE's version-2 SpMV (rocsparse/internal/generic/rocsparse_v2_spmv.h):
// an SpMV descriptor carries the algorithm, the analysis stage runs once per
// matrix and the compute stage repeats.  The earlier generic API documents
// that the analysis is kept per sparse-matrix descriptor and that the user
// buffer must outlive every call with it; this program therefore makes fresh
// descriptors for its one algorithm, keeps both stage buffers allocated until
// all descriptors are destroyed, and frees them last.
//
// usage: rocsparse_spmv <cfg 1-5> <adaptive|rowsplit|lrb|nnzsplit> [--iters N] [--scale N]
// prints one JSON line.
#include "prefree_c.h"

#include <hip/hip_runtime.h>
#include <rocsparse/rocsparse.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace {

[[noreturn]] void die(const char *what, long code)
{
    std::fprintf(stderr, "rocsparse_spmv: %s failed (%ld)\n", what, code);
    std::exit(1);
}

#define HIP_OK(x)                                      \
    do {                                               \
        hipError_t e_ = (x);                           \
        if (e_ != hipSuccess) die(#x, (long)e_);       \
    } while (0)
#define RS_OK(x)                                              \
    do {                                                      \
        rocsparse_status s_ = (x);                            \
        if (s_ != rocsparse_status_success) die(#x, (long)s_); \
    } while (0)
#define PF_OK_(x)                                      \
    do {                                               \
        int s_ = (x);                                  \
        if (s_ != PF_OK) die(#x, (long)s_);            \
    } while (0)

}  // namespace

int main(int argc, char **argv)
{
    if (argc < 3) {
        std::printf("usage: rocsparse_spmv <cfg 1-5> <adaptive|rowsplit|lrb|nnzsplit> [--iters N] [--scale N]\n");
        return 0;
    }
    const int cfg = std::atoi(argv[1]);
    const std::string name = argv[2];
    int iters = 200, scale = 0;
    for (int i = 3; i + 1 < argc; i += 2) {
        if (!std::strcmp(argv[i], "--iters")) iters = std::atoi(argv[i + 1]);
        else if (!std::strcmp(argv[i], "--scale")) scale = std::atoi(argv[i + 1]);
    }
    rocsparse_spmv_alg alg;
    if (name == "adaptive") alg = rocsparse_spmv_alg_csr_adaptive;
    else if (name == "rowsplit") alg = rocsparse_spmv_alg_csr_rowsplit;
    else if (name == "lrb") alg = rocsparse_spmv_alg_csr_lrb;
    else if (name == "nnzsplit") alg = rocsparse_spmv_alg_csr_nnzsplit;
    else die("unknown algorithm", 0);
    if (cfg < 1 || cfg > 5 || iters < 1) die("bad arguments", cfg);

    int m = 0, n = 0;
    long long nnz = 0;
    PF_OK_(pf_synth_dims(cfg, 1, scale, &m, &n, &nnz));
    std::vector<int> rp((size_t)m + 1), col((size_t)nnz);
    std::vector<double> val((size_t)nnz), x((size_t)n), y_rs((size_t)m), y_pf((size_t)m);
    PF_OK_(pf_synth_csr(cfg, 1, scale, 0, rp.data(), col.data(), val.data(), nullptr));
    PF_OK_(pf_synth_x(cfg, 1, n, 0, x.data(), nullptr));

    int *d_rp = nullptr, *d_col = nullptr;
    double *d_val = nullptr, *d_x = nullptr, *d_y = nullptr;
    HIP_OK(hipMalloc(&d_rp, sizeof(int) * ((size_t)m + 1)));
    HIP_OK(hipMalloc(&d_col, sizeof(int) * (size_t)nnz));
    HIP_OK(hipMalloc(&d_val, sizeof(double) * (size_t)nnz));
    HIP_OK(hipMalloc(&d_x, sizeof(double) * (size_t)n));
    HIP_OK(hipMalloc(&d_y, sizeof(double) * (size_t)m));
    HIP_OK(hipMemcpy(d_rp, rp.data(), sizeof(int) * ((size_t)m + 1), hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_col, col.data(), sizeof(int) * (size_t)nnz, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_val, val.data(), sizeof(double) * (size_t)nnz, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_x, x.data(), sizeof(double) * (size_t)n, hipMemcpyHostToDevice));

    // This library's y first (its own plan), for the cross-check.
    PF_OK_(pf_spmv(d_rp, d_col, d_val, d_x, d_y, m, n, (int)nnz, PF_F64, PF_AUTO, nullptr));
    HIP_OK(hipMemcpy(y_pf.data(), d_y, sizeof(double) * (size_t)m, hipMemcpyDeviceToHost));
    HIP_OK(hipMemset(d_y, 0, sizeof(double) * (size_t)m));

    hipEvent_t e0, e1;
    HIP_OK(hipEventCreate(&e0));
    HIP_OK(hipEventCreate(&e1));
    // This library timed the way rocSPARSE is timed below: the same launch loop
    // (back-to-back calls on the null stream from C++, events around them).
    float pf_ms = 0;
    {
        pf_plan *plan = nullptr;
        PF_OK_(pf_plan_create(&plan, d_rp, d_col, m, n, (int)nnz, PF_F64, PF_AUTO, nullptr));
        for (int i = 0; i < 10; ++i) PF_OK_(pf_plan_execute(plan, d_rp, d_col, d_val, d_x, d_y, nullptr));
        HIP_OK(hipEventRecord(e0, nullptr));
        for (int i = 0; i < iters; ++i) PF_OK_(pf_plan_execute(plan, d_rp, d_col, d_val, d_x, d_y, nullptr));
        HIP_OK(hipEventRecord(e1, nullptr));
        HIP_OK(hipEventSynchronize(e1));
        HIP_OK(hipEventElapsedTime(&pf_ms, e0, e1));
        pf_ms /= (float)iters;
        PF_OK_(pf_plan_check(plan, nullptr));
        PF_OK_(pf_plan_destroy(plan));
    }
    HIP_OK(hipMemset(d_y, 0, sizeof(double) * (size_t)m));

    rocsparse_handle h = nullptr;
    rocsparse_spmv_descr sd = nullptr;
    rocsparse_spmat_descr A = nullptr;
    rocsparse_dnvec_descr X = nullptr, Y = nullptr;
    RS_OK(rocsparse_create_handle(&h));
    RS_OK(rocsparse_create_csr_descr(&A, m, n, nnz, d_rp, d_col, d_val, rocsparse_indextype_i32,
                                     rocsparse_indextype_i32, rocsparse_index_base_zero, rocsparse_datatype_f64_r));
    RS_OK(rocsparse_create_dnvec_descr(&X, n, d_x, rocsparse_datatype_f64_r));
    RS_OK(rocsparse_create_dnvec_descr(&Y, m, d_y, rocsparse_datatype_f64_r));
    RS_OK(rocsparse_create_spmv_descr(&sd));
    const rocsparse_operation op = rocsparse_operation_none;
    const rocsparse_datatype f64 = rocsparse_datatype_f64_r;
    RS_OK(rocsparse_spmv_set_input(h, sd, rocsparse_spmv_input_alg, &alg, sizeof alg, nullptr));
    RS_OK(rocsparse_spmv_set_input(h, sd, rocsparse_spmv_input_operation, &op, sizeof op, nullptr));
    RS_OK(rocsparse_spmv_set_input(h, sd, rocsparse_spmv_input_scalar_datatype, &f64, sizeof f64, nullptr));
    RS_OK(rocsparse_spmv_set_input(h, sd, rocsparse_spmv_input_compute_datatype, &f64, sizeof f64, nullptr));
    const double alpha = 1.0, beta = 0.0;
    // Both buffers stay allocated until every descriptor is destroyed.
    size_t bytes_a = 0, bytes_c = 0;
    RS_OK(rocsparse_v2_spmv_buffer_size(h, sd, A, X, Y, rocsparse_v2_spmv_stage_analysis, &bytes_a, nullptr));
    void *buf_a = nullptr, *buf_c = nullptr;
    if (bytes_a == 0) bytes_a = 256;  // the size passed must be nonzero and at least the queried one
    HIP_OK(hipMalloc(&buf_a, bytes_a));
    HIP_OK(hipEventRecord(e0, nullptr));
    RS_OK(rocsparse_v2_spmv(h, sd, &alpha, A, X, &beta, Y, rocsparse_v2_spmv_stage_analysis, bytes_a, buf_a, nullptr));
    HIP_OK(hipEventRecord(e1, nullptr));
    HIP_OK(hipEventSynchronize(e1));
    float pre_ms = 0;
    HIP_OK(hipEventElapsedTime(&pre_ms, e0, e1));
    RS_OK(rocsparse_v2_spmv_buffer_size(h, sd, A, X, Y, rocsparse_v2_spmv_stage_compute, &bytes_c, nullptr));
    if (bytes_c == 0) bytes_c = 256;
    HIP_OK(hipMalloc(&buf_c, bytes_c));
    for (int i = 0; i < 10; ++i)
        RS_OK(rocsparse_v2_spmv(h, sd, &alpha, A, X, &beta, Y, rocsparse_v2_spmv_stage_compute, bytes_c, buf_c, nullptr));
    HIP_OK(hipEventRecord(e0, nullptr));
    for (int i = 0; i < iters; ++i)
        RS_OK(rocsparse_v2_spmv(h, sd, &alpha, A, X, &beta, Y, rocsparse_v2_spmv_stage_compute, bytes_c, buf_c, nullptr));
    HIP_OK(hipEventRecord(e1, nullptr));
    HIP_OK(hipEventSynchronize(e1));
    float ms = 0;
    HIP_OK(hipEventElapsedTime(&ms, e0, e1));
    ms /= (float)iters;
    HIP_OK(hipMemcpy(y_rs.data(), d_y, sizeof(double) * (size_t)m, hipMemcpyDeviceToHost));

    RS_OK(rocsparse_destroy_spmv_descr(sd));
    RS_OK(rocsparse_destroy_dnvec_descr(Y));
    RS_OK(rocsparse_destroy_dnvec_descr(X));
    RS_OK(rocsparse_destroy_spmat_descr(A));
    RS_OK(rocsparse_destroy_handle(h));
    HIP_OK(hipFree(buf_c));
    HIP_OK(hipFree(buf_a));
    const size_t bytes = bytes_a + bytes_c;

    // Row-wise agreement normalised by sum |a_ij x_j| of the row.
    double worst = 0;
    for (int i = 0; i < m; ++i) {
        double s = 0;
        for (int j = rp[(size_t)i]; j < rp[(size_t)i + 1]; ++j) s += std::fabs(val[(size_t)j] * x[(size_t)col[(size_t)j]]);
        const double d = std::fabs(y_rs[(size_t)i] - y_pf[(size_t)i]);
        const double e = s > 0 ? d / s : (d > 0 ? INFINITY : 0.0);
        if (!(e <= worst)) worst = e;
    }
    const double eff = (double)(nnz + m + n) * 8 + (double)nnz * 4 + ((double)m + 1) * 4;
    std::printf("{\"cfg\": \"C%d\", \"scale\": %d, \"rocsparse_alg\": \"%s\", \"us\": %.3f, \"gbps_effective\": %.1f, "
                "\"gflops\": %.2f, \"preprocess_ms\": %.3f, \"buffer_bytes\": %zu, \"max_rownorm_diff_vs_prefree\": %.3e, "
                "\"prefree_us\": %.3f}\n",
                cfg, scale, name.c_str(), ms * 1e3, eff / (ms * 1e6), 2.0 * nnz / (ms * 1e6), pre_ms, bytes, worst,
                pf_ms * 1e3);
    HIP_OK(hipEventDestroy(e0));
    HIP_OK(hipEventDestroy(e1));
    HIP_OK(hipFree(d_rp));
    HIP_OK(hipFree(d_col));
    HIP_OK(hipFree(d_val));
    HIP_OK(hipFree(d_x));
    HIP_OK(hipFree(d_y));
    return 0;
}
