/*
 * PreFree.h — drop-in replacement for the reference's include/PreFree.h:3-5.
 *
 *   void preFreeSpMV(valT *csrVal, int *csrRowPtr, int *csrColInd,
 *                    valT *X_val, valT *Y_val, int rowA, int colA, int nnzA,
 *                    double *cdTime, double *cdPre);
 *
 * Same C++ linkage and argument meaning as the reference
 * (src/spmv_kernel/preFreeSpMV.cu:563-662): all pointers are host memory owned
 * by the caller; the call allocates device memory, copies the CSR matrix and
 * x, runs 200 warm-up and 4000 timed SpMVs, writes the mean kernel time per
 * SpMV in ms to *cdTime, computes Y_val = A·x (overwritten) and frees
 * everything.  Differences, all deliberate:
 *   - *cdPre is what finding the tiles' rows costs per SpMV in ms: there is
 *     no pre-pass kernel, the SpMV kernel's first call searches row_ptr and
 *     records the rows, later calls read them; cdPre is the event-timed mean of
 *     calls that search every time minus *cdTime (0 for variants that always
 *     search: PREFREE, ADAPTIVE);
 *   - exactly rowA+1 row_ptr entries are read (the reference copies rowA+2);
 *   - fatal errors print one line to stderr and exit(EXIT_FAILURE), as the
 *     reference's CUDA_CHECK_ERROR (include/common.h:49-58) does.
 * Environment knobs (all optional): PREFREE_VARIANT=auto|prefree|adaptive|flat,
 * PREFREE_TILE=<keys per tile>, PREFREE_WARMUP=<n> (200), PREFREE_ITERS=<n> (4000),
 * PREFREE_PRE_ITERS=<n> (ITERS/10, at least 20), PREFREE_VERBOSE=1 (planning time to stderr).
 *
 * valT is double (the reference's default -Dfp64 build).  Defining
 * PREFREE_VALT_FLOAT before including this header selects the float overload,
 * PREFREE_VALT_HALF the fp16 one: the reference's non-fp64 build stores half
 * values (include/common.h:43-46); pf_half holds the same 16 IEEE binary16
 * bits, so a half* converts with a reinterpret_cast.  The fp16 overload forms
 * products and row sums in fp32 and rounds each row sum to half once.
 */
#ifndef PREFREE_DROPIN_H
#define PREFREE_DROPIN_H

/* IEEE binary16 value, bit for bit. */
typedef struct pf_half {
    unsigned short bits;
} pf_half;

#ifndef valT
#if defined(PREFREE_VALT_FLOAT)
#define valT float
#elif defined(PREFREE_VALT_HALF)
#define valT pf_half
#else
#define valT double
#endif
#endif

void preFreeSpMV(double *csrVal, int *csrRowPtr, int *csrColInd, double *X_val, double *Y_val, int rowA, int colA,
                 int nnzA, double *cdTime, double *cdPre);
void preFreeSpMV(float *csrVal, int *csrRowPtr, int *csrColInd, float *X_val, float *Y_val, int rowA, int colA,
                 int nnzA, double *cdTime, double *cdPre);
void preFreeSpMV(pf_half *csrVal, int *csrRowPtr, int *csrColInd, pf_half *X_val, pf_half *Y_val, int rowA,
                 int colA, int nnzA, double *cdTime, double *cdPre);

#endif
