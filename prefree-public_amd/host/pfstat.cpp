// pfstat.cpp — tile statistics of a Matrix Market matrix, the counterpart of
// the reference's test/statistic.cu (analyzeMatrixTiles, :128-258).
//
// The reference maps 512/1024-nnz tiles to rows with its pre-pass and writes,
// per tile, the row span and the lengths of the rows' pieces inside the tile
// (stat/<name>.csv, same columns as here), then a summary.  This tool does the
// same for any of this library's tilings, with the maps computed by the
// kernels' own row search on the GPU (the descriptors the kernels use):
//   prefree   128*P_NNZ-nnz tiles, first row per tile as in preFreeSpMV.cu:3-28
//             (P_NNZ by the reference heuristic, statistic.cu:150, unless --tile);
//   adaptive  merged (row + nnz) key tiles of k_wave;
//   flat      nnz tiles of k_tiles.
// It also prints the row-length statistics and the configuration PF_AUTO picks.
// The reference's tile range rule (preFreeSpMV.cu:429-438) mistakes a start row
// of 0 for "unset" (a quirk its kernel inherits); the ranges here are exact.
//
// usage: pfstat <matrix.mtx> [--variant prefree|adaptive|flat] [--tile N] [--f32] [--out DIR]
#include "prefree_c.h"
#include "prefree_kernels.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iomanip>
#include <string>
#include <sys/stat.h>
#include <vector>

namespace {

struct TileStat {
    long long tile;
    int start_row, end_row;  // rows [start_row, end_row) hold the tile's nnz
    int max_len, min_len;
    double ratio, avg, var;
    int head, tail;          // split rows entering / leaving (adaptive, flat)
};

[[noreturn]] void die(const std::string &what, int st)
{
    std::fprintf(stderr, "pfstat: %s failed: %s (%s)\n", what.c_str(), pf_status_string(st), pf_last_error());
    std::exit(1);
}

void check(int st, const char *what)
{
    if (st != PF_OK) die(what, st);
}

std::string stem(const std::string &path)
{
    const size_t s = path.find_last_of("/\\");
    std::string f = s == std::string::npos ? path : path.substr(s + 1);
    const size_t d = f.find_last_of('.');
    return d == std::string::npos ? f : f.substr(0, d);
}

// Lengths of rows [r0, r1) restricted to the nnz range [a, b).
TileStat stats_of(long long tile, int r0, int r1, long long a, long long b, const std::vector<int> &rp)
{
    TileStat t{tile, r0, r1, 0, 0, 0.0, 0.0, 0.0, 0, 0};
    const int n = r1 - r0;
    if (n <= 0) return t;
    long long total = 0;
    int mx = 0, mn = 0x7FFFFFFF;
    for (int r = r0; r < r1; ++r) {
        const long long len = std::max(0LL, std::min<long long>(rp[r + 1], b) - std::max<long long>(rp[r], a));
        total += len;
        mx = std::max(mx, (int)len);
        mn = std::min(mn, (int)len);
    }
    t.max_len = mx;
    t.min_len = mn;
    t.ratio = mn > 0 ? (double)mx / mn : 0.0;
    t.avg = (double)total / n;
    double v = 0;
    for (int r = r0; r < r1; ++r) {
        const long long len = std::max(0LL, std::min<long long>(rp[r + 1], b) - std::max<long long>(rp[r], a));
        v += (len - t.avg) * (len - t.avg);
    }
    t.var = v / n;
    return t;
}

}  // namespace

int main(int argc, char **argv)
{
    const char *path = nullptr;
    std::string variant = "prefree", outdir = "stat";
    int tile = 0, dtype = PF_F64;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        if (a == "--variant" && i + 1 < argc) variant = argv[++i];
        else if (a == "--tile" && i + 1 < argc) tile = std::atoi(argv[++i]);
        else if (a == "--out" && i + 1 < argc) outdir = argv[++i];
        else if (a == "--f32") dtype = PF_F32;
        else if (!path && a[0] != '-') path = argv[i];
    }
    if (!path || (variant != "prefree" && variant != "adaptive" && variant != "flat")) {
        std::printf("usage: pfstat <matrix.mtx> [--variant prefree|adaptive|flat] [--tile N] [--f32] [--out DIR]\n");
        return path ? 2 : 0;
    }
    int m = 0, n = 0, nnz = 0, sym = 0;
    int *hrp = nullptr, *hcol = nullptr;
    double *hval = nullptr;
    if (pf_mtx_read(path, &m, &n, &nnz, &sym, &hrp, &hcol, &hval) != PF_OK) {
        std::fprintf(stderr, "pfstat: cannot read %s: %s\n", path, pf_mtx_last_error());
        return 2;
    }
    std::printf("matrix %s: %d x %d, nnz = %d, symmetric = %d\n", path, m, n, nnz, sym);
    std::vector<int> rp(hrp, hrp + m + 1);
    if (m == 0 || nnz == 0) {
        std::printf("empty matrix: no tiles\n");
        return 0;
    }

    void *d_rp = nullptr, *d_col = nullptr;
    check(pf_device_malloc(&d_rp, sizeof(int) * (size_t)(m + 1)), "device allocation");
    check(pf_device_malloc(&d_col, sizeof(int) * (size_t)nnz), "device allocation");
    check(pf_memcpy_h2d(d_rp, hrp, sizeof(int) * (size_t)(m + 1), nullptr), "copy");
    check(pf_memcpy_h2d(d_col, hcol, sizeof(int) * (size_t)nnz, nullptr), "copy");

    pf_row_stats rs;
    check(pf_row_stats_compute((const int *)d_rp, (const int *)d_col, m, n, nnz, &rs, nullptr), "row statistics");
    std::printf("rows: max %lld, min %lld, mean %.2f, empty %lld; log2 histogram:", rs.max_row_len, rs.min_row_len,
                (double)nnz / m, rs.n_empty_rows);
    for (int k = 0; k < 33; ++k)
        if (rs.hist_log2[k]) std::printf(" [%s%d]=%lld", k ? "<2^" : "=", k, rs.hist_log2[k]);
    std::printf("\n");
    pf_plan_info ai;
    if (pf_select(&rs, dtype, PF_AUTO, &ai) == PF_OK)
        std::printf("PF_AUTO: variant %s, tile %d, run %d, tiles %lld\n",
                    ai.variant == PF_ADAPTIVE ? "adaptive" : ai.variant == PF_FLAT ? "flat" : "prefree", ai.tile,
                    ai.run_tiles, ai.ntiles);

    std::vector<TileStat> out;
    int *d_out = nullptr, *d_err = nullptr;
    if (variant == "prefree") {
        // statistic.cu:150: P_NNZ 8 for large, not very dense matrices, else 4; tiles of 128 * P_NNZ nnz.
        if (tile <= 0) tile = (nnz > 16518948 && (float)nnz / (float)m < 500.f) ? 1024 : 512;
        const long long nt = ((long long)nnz + tile - 1) / tile;
        check(pf_device_malloc((void **)&d_out, sizeof(int) * (size_t)(nt + 1)), "device allocation");
        check(pfk_debug_prefree_rows((const int *)d_rp, m, nnz, tile, d_out, nullptr), "tile map");
        std::vector<int> start((size_t)nt + 1);
        check(pf_memcpy_d2h(start.data(), d_out, sizeof(int) * (size_t)(nt + 1), nullptr), "copy");
        for (long long b = 0; b < nt; ++b) {
            const long long a = b * tile, e = std::min<long long>(a + tile, nnz);
            // rows holding the tile's last nnz end the span
            const int last = (int)(std::upper_bound(rp.begin(), rp.end(), (int)(e - 1)) - rp.begin()) - 1;
            out.push_back(stats_of(b, start[(size_t)b], last + 1, a, e, rp));
        }
        std::printf("tiling: prefree, %d nnz per tile, %lld tiles\n", tile, nt);
    } else {
        const bool merged = variant == "adaptive";
        int tiles[PFK_MAX_TILES];
        const int ntl = pfk_supported_tiles(merged ? PF_ADAPTIVE : PF_FLAT, dtype, tiles, PFK_MAX_TILES);
        int largest = 0;  // the largest nnz tile; FLAT's 2..32 are row groups, which have no nnz tiles
        for (int i = 0; i < ntl; ++i)
            if (!(!merged && PFK_ROW_GROUP_TILE(tiles[i]))) largest = std::max(largest, tiles[i]);
        if (tile <= 0) tile = merged && ai.variant == PF_ADAPTIVE ? ai.tile : largest;
        if (!merged && PFK_ROW_GROUP_TILE(tile)) {
            std::fprintf(stderr, "pfstat: FLAT %d is a row group (%d lanes per row), not a tile of nnz\n", tile, tile);
            return 2;
        }
        const long long total = merged ? (long long)nnz + m : nnz;
        const long long nt = (total + tile - 1) / tile;
        check(pf_device_malloc((void **)&d_out, sizeof(int) * 8 * (size_t)nt), "device allocation");
        check(pf_device_malloc((void **)&d_err, 256), "device allocation");
        check(pfk_fill_zero(d_err, 256, nullptr), "fill");
        pfk_spmv_args a;
        std::memset(&a, 0, sizeof a);
        a.row_ptr = (const int *)d_rp;
        a.m = m;
        a.n = n;
        a.nnz = nnz;
        a.tile = tile;
        a.run_tiles = 1;
        a.ntiles = nt;
        a.err_flag = d_err;
        check(pfk_debug_tile_desc(dtype, merged ? 1 : 0, &a, d_out, nullptr), "tile descriptors");
        std::vector<int> d((size_t)nt * 8);
        check(pf_memcpy_d2h(d.data(), d_out, sizeof(int) * 8 * (size_t)nt, nullptr), "copy");
        for (long long t = 0; t < nt; ++t) {
            const int *q = &d[(size_t)t * 8];
            TileStat s = stats_of(t, q[0], q[0] + q[1], q[2], q[3], rp);
            s.head = q[4];
            s.tail = q[5];
            out.push_back(s);
        }
        std::printf("tiling: %s, %d %s per tile, %lld tiles\n", variant.c_str(), tile, merged ? "keys" : "nnz", nt);
    }

    mkdir(outdir.c_str(), 0755);
    const std::string csv = outdir + "/" + stem(path) + (variant == "prefree" ? "" : "_" + variant) + ".csv";
    std::ofstream f(csv);
    if (!f) {
        std::fprintf(stderr, "pfstat: cannot write %s\n", csv.c_str());
        return 1;
    }
    f << "tile_id,n_reduce_rows_num,row_length_ratio,max_row_length,min_row_length,avg_row_length,variance,"
         "start_row,end_row,head_split,tail_split\n";
    double s_rows = 0, s_max = 0, s_var = 0;
    for (const TileStat &t : out) {
        f << t.tile << ',' << (t.end_row - t.start_row) << ',' << std::fixed << std::setprecision(2) << t.ratio << ','
          << t.max_len << ',' << t.min_len << ',' << t.avg << ',' << t.var << ',' << t.start_row << ',' << t.end_row
          << ',' << t.head << ',' << t.tail << '\n';
        s_rows += t.end_row - t.start_row;
        s_max += t.max_len;
        s_var += t.var;
    }
    f.close();
    const double k = out.empty() ? 1.0 : (double)out.size();
    std::printf("wrote %s (%zu tiles)\n", csv.c_str(), out.size());
    std::printf("summary: mean rows per tile %.2f, mean max row piece %.2f, mean variance %.2f\n", s_rows / k,
                s_max / k, s_var / k);
    pf_device_free(d_out);
    if (d_err) pf_device_free(d_err);
    pf_device_free(d_rp);
    pf_device_free(d_col);
    pf_host_free(hrp);
    pf_host_free(hcol);
    pf_host_free(hval);
    return 0;
}
