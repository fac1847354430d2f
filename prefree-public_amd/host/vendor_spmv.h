// vendor_spmv.h — the vendor SpMV the cdspmv harness times beside preFreeSpMV
// (the reference harness's cusparse_spmv_all, test/test_cdspmv.cpp:155-267),
// here rocSPARSE's default algorithm (host/vendor_rocsparse.cpp).  Host
// buffers in and out; *ms = mean ms per compute call over `iters` after
// `warm`, *pre_ms = the analysis stage.  Returns 0, or 1 with a reason in why.
#ifndef PREFREE_VENDOR_SPMV_H
#define PREFREE_VENDOR_SPMV_H

int vendor_spmv(const double *val, const int *rp, const int *col, const double *x, double *y, int m, int n, int nnz,
                int warm, int iters, double *ms, double *pre_ms, char *why, int why_len);
int vendor_spmv(const float *val, const int *rp, const int *col, const float *x, float *y, int m, int n, int nnz,
                int warm, int iters, double *ms, double *pre_ms, char *why, int why_len);

#endif
