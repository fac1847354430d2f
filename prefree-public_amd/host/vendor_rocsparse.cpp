// vendor_rocsparse.cpp — the vendor SpMV of the cdspmv harness: rocSPARSE on
// MI355X, timed the way the reference harness times cuSPARSE
// (test/test_cdspmv.cpp:155-267): device copies of the CSR matrix and x, the
// analysis stage timed as the preprocessing figure, 200 warm-up and 4000 timed
// compute calls on the null stream with events around them, y copied back.
// rocSPARSE's default algorithm, as the reference uses cuSPARSE's default.
// fp64 and fp32 only.
#include "vendor_spmv.h"

#include <hip/hip_runtime.h>
#include <rocsparse/rocsparse.h>

#include <cstdio>

namespace {

template <typename T> rocsparse_datatype rs_type();
template <> rocsparse_datatype rs_type<double>() { return rocsparse_datatype_f64_r; }
template <> rocsparse_datatype rs_type<float>() { return rocsparse_datatype_f32_r; }

#define V_HIP(x)                                                                  \
    do {                                                                          \
        hipError_t e_ = (x);                                                      \
        if (e_ != hipSuccess) {                                                   \
            std::snprintf(why, why_len, "%s: %s", #x, hipGetErrorString(e_));     \
            goto out;                                                             \
        }                                                                         \
    } while (0)
#define V_RS(x)                                                                   \
    do {                                                                          \
        rocsparse_status s_ = (x);                                                \
        if (s_ != rocsparse_status_success) {                                     \
            std::snprintf(why, why_len, "%s: status %d", #x, (int)s_);            \
            goto out;                                                             \
        }                                                                         \
    } while (0)

template <typename T>
int vendor(const T *val, const int *rp, const int *col, const T *x, T *y, int m, int n, int nnz, int warm,
           int iters, double *ms, double *pre_ms, char *why, int why_len)
{
    int rc = 1;
    int *d_rp = nullptr, *d_col = nullptr;
    T *d_val = nullptr, *d_x = nullptr, *d_y = nullptr;
    void *buf_a = nullptr, *buf_c = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    rocsparse_handle h = nullptr;
    rocsparse_spmv_descr sd = nullptr;
    rocsparse_spmat_descr A = nullptr;
    rocsparse_dnvec_descr X = nullptr, Y = nullptr;
    const rocsparse_spmv_alg alg = rocsparse_spmv_alg_default;
    const rocsparse_operation op = rocsparse_operation_none;
    const rocsparse_datatype dt = rs_type<T>();
    const T alpha = T(1), beta = T(0);
    size_t bytes_a = 0, bytes_c = 0;
    float t_pre = 0.f, t = 0.f;
    V_HIP(hipMalloc(&d_rp, sizeof(int) * ((size_t)m + 1)));
    V_HIP(hipMalloc(&d_col, sizeof(int) * ((size_t)nnz + 1)));
    V_HIP(hipMalloc(&d_val, sizeof(T) * ((size_t)nnz + 1)));
    V_HIP(hipMalloc(&d_x, sizeof(T) * ((size_t)n + 1)));
    V_HIP(hipMalloc(&d_y, sizeof(T) * ((size_t)m + 1)));
    V_HIP(hipMemcpy(d_rp, rp, sizeof(int) * ((size_t)m + 1), hipMemcpyHostToDevice));
    V_HIP(hipMemcpy(d_col, col, sizeof(int) * (size_t)nnz, hipMemcpyHostToDevice));
    V_HIP(hipMemcpy(d_val, val, sizeof(T) * (size_t)nnz, hipMemcpyHostToDevice));
    V_HIP(hipMemcpy(d_x, x, sizeof(T) * (size_t)n, hipMemcpyHostToDevice));
    V_HIP(hipMemset(d_y, 0, sizeof(T) * (size_t)m));
    V_HIP(hipEventCreate(&e0));
    V_HIP(hipEventCreate(&e1));
    V_RS(rocsparse_create_handle(&h));
    V_RS(rocsparse_create_csr_descr(&A, m, n, nnz, d_rp, d_col, d_val, rocsparse_indextype_i32,
                                    rocsparse_indextype_i32, rocsparse_index_base_zero, dt));
    V_RS(rocsparse_create_dnvec_descr(&X, n, d_x, dt));
    V_RS(rocsparse_create_dnvec_descr(&Y, m, d_y, dt));
    V_RS(rocsparse_create_spmv_descr(&sd));
    V_RS(rocsparse_spmv_set_input(h, sd, rocsparse_spmv_input_alg, &alg, sizeof alg, nullptr));
    V_RS(rocsparse_spmv_set_input(h, sd, rocsparse_spmv_input_operation, &op, sizeof op, nullptr));
    V_RS(rocsparse_spmv_set_input(h, sd, rocsparse_spmv_input_scalar_datatype, &dt, sizeof dt, nullptr));
    V_RS(rocsparse_spmv_set_input(h, sd, rocsparse_spmv_input_compute_datatype, &dt, sizeof dt, nullptr));
    // Both stage buffers stay allocated until every descriptor is destroyed (the analysis is kept per
    // descriptor and refers to its buffer).
    V_RS(rocsparse_v2_spmv_buffer_size(h, sd, A, X, Y, rocsparse_v2_spmv_stage_analysis, &bytes_a, nullptr));
    if (bytes_a == 0) bytes_a = 256;
    V_HIP(hipMalloc(&buf_a, bytes_a));
    V_HIP(hipEventRecord(e0, nullptr));
    V_RS(rocsparse_v2_spmv(h, sd, &alpha, A, X, &beta, Y, rocsparse_v2_spmv_stage_analysis, bytes_a, buf_a, nullptr));
    V_HIP(hipEventRecord(e1, nullptr));
    V_HIP(hipEventSynchronize(e1));
    V_HIP(hipEventElapsedTime(&t_pre, e0, e1));
    V_RS(rocsparse_v2_spmv_buffer_size(h, sd, A, X, Y, rocsparse_v2_spmv_stage_compute, &bytes_c, nullptr));
    if (bytes_c == 0) bytes_c = 256;
    V_HIP(hipMalloc(&buf_c, bytes_c));
    for (int i = 0; i < warm; ++i)
        V_RS(rocsparse_v2_spmv(h, sd, &alpha, A, X, &beta, Y, rocsparse_v2_spmv_stage_compute, bytes_c, buf_c, nullptr));
    V_HIP(hipDeviceSynchronize());
    V_HIP(hipEventRecord(e0, nullptr));
    for (int i = 0; i < iters; ++i)
        V_RS(rocsparse_v2_spmv(h, sd, &alpha, A, X, &beta, Y, rocsparse_v2_spmv_stage_compute, bytes_c, buf_c, nullptr));
    V_HIP(hipEventRecord(e1, nullptr));
    V_HIP(hipEventSynchronize(e1));
    V_HIP(hipEventElapsedTime(&t, e0, e1));
    V_HIP(hipMemcpy(y, d_y, sizeof(T) * (size_t)m, hipMemcpyDeviceToHost));
    *ms = iters > 0 ? (double)t / iters : 0.0;
    *pre_ms = t_pre;
    rc = 0;
out:
    if (sd) rocsparse_destroy_spmv_descr(sd);
    if (Y) rocsparse_destroy_dnvec_descr(Y);
    if (X) rocsparse_destroy_dnvec_descr(X);
    if (A) rocsparse_destroy_spmat_descr(A);
    if (h) rocsparse_destroy_handle(h);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipFree(buf_c);
    (void)hipFree(buf_a);
    (void)hipFree(d_y);
    (void)hipFree(d_x);
    (void)hipFree(d_val);
    (void)hipFree(d_col);
    (void)hipFree(d_rp);
    return rc;
}

}  // namespace

int vendor_spmv(const double *val, const int *rp, const int *col, const double *x, double *y, int m, int n, int nnz,
                int warm, int iters, double *ms, double *pre_ms, char *why, int why_len)
{
    return vendor(val, rp, col, x, y, m, n, nnz, warm, iters, ms, pre_ms, why, why_len);
}

int vendor_spmv(const float *val, const int *rp, const int *col, const float *x, float *y, int m, int n, int nnz,
                int warm, int iters, double *ms, double *pre_ms, char *why, int why_len)
{
    return vendor(val, rp, col, x, y, m, n, nnz, warm, iters, ms, pre_ms, why, why_len);
}
