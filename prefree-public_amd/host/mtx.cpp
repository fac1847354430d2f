// mtx.cpp — Matrix Market (coordinate) reader with the reference harness's
// conventions (utilities/mmio.cpp:1543-1713, mmio_allinone, over the NIST
// mmio banner / size-line rules of mmio.cpp:246-465):
//   * banner "%%MatrixMarket matrix coordinate <field> <symmetry>", tokens
//     compared case-insensitively; field real | integer | pattern | complex
//     (pattern -> 1.0, complex -> real part), symmetry general | symmetric |
//     hermitian | skew-symmetric;
//   * comment lines start with '%'; the size line "M N NNZ" follows them;
//   * entries are 1-based and are kept in file order, duplicates included;
//   * symmetric and hermitian files mirror every off-diagonal entry (same
//     value) into the transposed position; skew-symmetric files are NOT
//     mirrored (the reference tests symmetric || hermitian only);
//   * row r of the CSR lists its entries in the order one pass over the file
//     meets them, an entry's mirror placed right after the entry itself.
// Unlike the reference, malformed input (bad banner, "array" format, entry
// indices out of range, short files) is reported instead of read past.
#include "prefree_c.h"

#include <algorithm>
#include <cctype>
#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace {

thread_local std::string g_mtx_err;

int mtx_fail(const std::string &msg)
{
    g_mtx_err = msg;
    return PF_ERR_IO;
}

std::string lower(std::string s)
{
    for (char &c : s) c = (char)std::tolower((unsigned char)c);
    return s;
}

struct Reader {
    FILE *f = nullptr;
    ~Reader()
    {
        if (f) std::fclose(f);
    }
    // Next line (without the newline); false at end of file.
    bool line(std::string &out)
    {
        out.clear();
        int c;
        bool any = false;
        while ((c = std::fgetc(f)) != EOF) {
            any = true;
            if (c == '\n') break;
            out.push_back((char)c);
        }
        if (!out.empty() && out.back() == '\r') out.pop_back();
        return any;
    }
};

bool blank(const std::string &s)
{
    for (char c : s)
        if (!std::isspace((unsigned char)c)) return false;
    return true;
}

}  // namespace

extern "C" {

const char *pf_mtx_last_error(void) { return g_mtx_err.c_str(); }

int pf_mtx_read(const char *path, int *m, int *n, int *nnz, int *is_symmetric, int **row_ptr, int **col,
                double **val)
{
    if (!path || !m || !n || !nnz || !is_symmetric || !row_ptr || !col || !val) {
        g_mtx_err = "pf_mtx_read: NULL argument";
        return PF_ERR_INVALID;
    }
    *row_ptr = nullptr;
    *col = nullptr;
    *val = nullptr;
    Reader r;
    r.f = std::fopen(path, "r");
    if (!r.f) return mtx_fail(std::string("cannot open ") + path + ": " + std::strerror(errno));

    std::string ln;
    if (!r.line(ln)) return mtx_fail("empty file");
    char tok[5][256];
    if (std::sscanf(ln.c_str(), "%255s %255s %255s %255s %255s", tok[0], tok[1], tok[2], tok[3], tok[4]) != 5)
        return mtx_fail("banner needs 5 fields: " + ln);
    if (std::strncmp(tok[0], "%%MatrixMarket", 14) != 0) return mtx_fail("no %%MatrixMarket banner");
    const std::string object = lower(tok[1]), format = lower(tok[2]), field = lower(tok[3]), sym = lower(tok[4]);
    if (object != "matrix") return mtx_fail("object '" + object + "' is not 'matrix'");
    if (format != "coordinate") return mtx_fail("format '" + format + "' is not 'coordinate'");
    enum { REAL, INTEGER, PATTERN, COMPLEX } kind;
    if (field == "real") kind = REAL;
    else if (field == "integer") kind = INTEGER;
    else if (field == "pattern") kind = PATTERN;
    else if (field == "complex") kind = COMPLEX;
    else return mtx_fail("unsupported field '" + field + "'");
    if (sym != "general" && sym != "symmetric" && sym != "hermitian" && sym != "skew-symmetric")
        return mtx_fail("unsupported symmetry '" + sym + "'");
    const bool mirror = sym == "symmetric" || sym == "hermitian";

    long long M = -1, N = -1, Z = -1;
    for (;;) {
        if (!r.line(ln)) return mtx_fail("missing size line");
        if (!ln.empty() && ln[0] == '%') continue;
        if (blank(ln)) continue;
        if (std::sscanf(ln.c_str(), "%lld %lld %lld", &M, &N, &Z) != 3) return mtx_fail("bad size line: " + ln);
        break;
    }
    if (M < 0 || N < 0 || Z < 0 || M > 0x7FFFFFFF - 1 || N > 0x7FFFFFFF || Z > 0x7FFFFFFF)
        return mtx_fail("size out of range");

    // The entry arrays grow as entries are read: a header's count alone (up to
    // 2^31 - 1) never decides an allocation.
    std::vector<int> ri, ci;
    std::vector<double> vi;
    const size_t first_reserve = (size_t)std::min<long long>(Z, 1 << 20);
    ri.reserve(first_reserve);
    ci.reserve(first_reserve);
    vi.reserve(first_reserve);
    long long got = 0;
    while (got < Z) {
        if (!r.line(ln)) return mtx_fail("file ends after " + std::to_string(got) + " of " + std::to_string(Z) + " entries");
        if (blank(ln) || ln[0] == '%') continue;
        long long i = 0, j = 0;
        double v = 1.0, im = 0.0;
        long long iv = 0;
        int k = 0;
        switch (kind) {
        case REAL: k = std::sscanf(ln.c_str(), "%lld %lld %lg", &i, &j, &v); break;
        case COMPLEX: k = std::sscanf(ln.c_str(), "%lld %lld %lg %lg", &i, &j, &v, &im); k = k == 4 ? 3 : 0; break;
        case INTEGER: k = std::sscanf(ln.c_str(), "%lld %lld %lld", &i, &j, &iv); v = (double)iv; break;
        case PATTERN: k = std::sscanf(ln.c_str(), "%lld %lld", &i, &j) == 2 ? 3 : 0; break;
        }
        if (k != 3) return mtx_fail("bad entry line: " + ln);
        if (i < 1 || i > M || j < 1 || j > N) return mtx_fail("entry index out of range: " + ln);
        if (mirror && j > M) return mtx_fail("symmetric entry outside a square matrix: " + ln);
        ri.push_back((int)(i - 1));
        ci.push_back((int)(j - 1));
        vi.push_back(v);
        ++got;
    }

    // Row counts, then one pass in file order placing each entry (and its mirror).
    std::vector<long long> start((size_t)M + 1, 0);
    for (long long e = 0; e < Z; ++e) {
        ++start[(size_t)ri[(size_t)e] + 1];
        if (mirror && ri[(size_t)e] != ci[(size_t)e]) ++start[(size_t)ci[(size_t)e] + 1];
    }
    for (long long k = 0; k < M; ++k) start[(size_t)k + 1] += start[(size_t)k];
    const long long total = start[(size_t)M];
    if (total > 0x7FFFFFFF) return mtx_fail("expanded nnz exceeds 2^31-1");

    int *rp = static_cast<int *>(std::malloc(sizeof(int) * (size_t)(M + 1)));
    int *cc = static_cast<int *>(std::malloc(sizeof(int) * (size_t)(total > 0 ? total : 1)));
    double *vv = static_cast<double *>(std::malloc(sizeof(double) * (size_t)(total > 0 ? total : 1)));
    if (!rp || !cc || !vv) {
        std::free(rp);
        std::free(cc);
        std::free(vv);
        g_mtx_err = "out of host memory";
        return PF_ERR_NOMEM;
    }
    for (long long k = 0; k <= M; ++k) rp[k] = (int)start[(size_t)k];
    std::vector<long long> fill(start.begin(), start.end() - 1);
    for (long long e = 0; e < Z; ++e) {
        const int a = ri[(size_t)e], b = ci[(size_t)e];
        long long o = fill[(size_t)a]++;
        cc[o] = b;
        vv[o] = vi[(size_t)e];
        if (mirror && a != b) {
            o = fill[(size_t)b]++;
            cc[o] = a;
            vv[o] = vi[(size_t)e];
        }
    }
    *m = (int)M;
    *n = (int)N;
    *nnz = (int)total;
    *is_symmetric = mirror ? 1 : 0;
    *row_ptr = rp;
    *col = cc;
    *val = vv;
    g_mtx_err.clear();
    return PF_OK;
}

void pf_host_free(void *p) { std::free(p); }

}  // extern "C"
