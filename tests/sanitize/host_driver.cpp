// host_driver.cpp — drives the host-only parts of the library that take
// untrusted input or do index arithmetic (Matrix Market reader, synthetic
// generators) for a build with -fsanitize=address,undefined.  Linked from the
// library's own sources (host/mtx.cpp, host/synth.cpp); no GPU, no HIP.
//
//   host_driver mtx <file>...   read each file; a readable one must give a valid
//                               CSR (row_ptr monotone from 0 to nnz, columns in
//                               [0, n)); an unreadable one a PF_ERR_IO status
//   host_driver synth           every configuration at scaled sizes, both value
//                               modes; checks the same invariants
// Prints one line per input and exits 0 when every check held; a sanitizer
// report aborts the process.
#include "prefree_c.h"

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

namespace {

int bad = 0;

bool csr_ok(const int *rp, const int *col, int m, int n, long long nnz)
{
    if (rp[0] != 0 || rp[m] != nnz) return false;
    for (int r = 0; r < m; ++r)
        if (rp[r + 1] < rp[r]) return false;
    for (long long j = 0; j < nnz; ++j)
        if (col[j] < 0 || col[j] >= n) return false;
    return true;
}

void one_mtx(const char *path)
{
    int m = 0, n = 0, nnz = 0, sym = 0, *rp = nullptr, *col = nullptr;
    double *val = nullptr;
    const int st = pf_mtx_read(path, &m, &n, &nnz, &sym, &rp, &col, &val);
    if (st == PF_OK) {
        const bool ok = csr_ok(rp, col, m, n, nnz);
        double sum = 0;
        for (int j = 0; j < nnz; ++j) sum += val[j];
        std::printf("%s: %d x %d, %d nnz%s, sum %g, %s\n", path, m, n, nnz, sym ? " (mirrored)" : "", sum,
                    ok ? "valid" : "INVALID CSR");
        if (!ok) ++bad;
    } else {
        std::printf("%s: status %d: %s\n", path, st, pf_mtx_last_error());
        if (st != PF_ERR_IO || rp || col || val) ++bad;
    }
    pf_host_free(rp);
    pf_host_free(col);
    pf_host_free(val);
}

void synth()
{
    const int scales[6] = {0, 0, 64, 20000, 100000, 20000};
    for (int cfg = 1; cfg <= 5; ++cfg) {
        for (int vals = 0; vals <= 1; ++vals) {
            int m = 0, n = 0;
            long long nnz = 0;
            if (pf_synth_dims(cfg, 3, scales[cfg], &m, &n, &nnz) != PF_OK) { ++bad; continue; }
            std::vector<int> rp((size_t)m + 1), col((size_t)nnz);
            std::vector<double> v64((size_t)nnz), x64((size_t)n);
            std::vector<float> v32((size_t)nnz), x32((size_t)n);
            const int a = pf_synth_csr(cfg, 3, scales[cfg], vals, rp.data(), col.data(), v64.data(), v32.data());
            const int b = pf_synth_x(cfg, 3, n, vals, x64.data(), x32.data());
            const bool ok = a == PF_OK && b == PF_OK && csr_ok(rp.data(), col.data(), m, n, nnz);
            std::printf("C%d vals %d: %d x %d, %lld nnz, %s\n", cfg, vals, m, n, nnz, ok ? "valid" : "INVALID");
            if (!ok) ++bad;
        }
    }
    int m = 0, n = 0;
    long long nnz = 0;
    if (pf_synth_dims(9, 1, 0, &m, &n, &nnz) == PF_OK) ++bad;  // unknown configuration refused
}

}  // namespace

int main(int argc, char **argv)
{
    if (argc >= 2 && std::strcmp(argv[1], "mtx") == 0) {
        for (int i = 2; i < argc; ++i) one_mtx(argv[i]);
    } else if (argc == 2 && std::strcmp(argv[1], "synth") == 0) {
        synth();
    } else {
        std::fprintf(stderr, "usage: host_driver mtx <file>... | host_driver synth\n");
        return 2;
    }
    std::printf("%s\n", bad ? "FAILED" : "ok");
    return bad ? 1 : 0;
}
