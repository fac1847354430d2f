// capi.cpp — the public C ABI (include/prefree_c.h): row statistics, variant
// selection, plans and execution.  Host C++ only; every GPU action goes
// through the thin HIP layer of include/prefree_kernels.h.
#include "prefree_c.h"
#include "prefree_kernels.h"

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <dlfcn.h>
#include <fstream>
#include <chrono>
#include <mutex>
#include <set>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

thread_local std::string g_err;

int fail(int status, const std::string &msg)
{
    g_err = msg;
    return status;
}

int from_kernel_layer(int status, const char *what)
{
    if (status != PF_OK)
        g_err = std::string(what) + ": " + pfk_last_error();
    return status;
}

#define PF_TRY(call, what)                                   \
    do {                                                     \
        int st_ = (call);                                    \
        if (st_ != PF_OK) return from_kernel_layer(st_, what); \
    } while (0)

constexpr int kXcds = 8;

// FLAT tiles of 256 nnz are walked in runs by k_flow (rows carried between tiles).
constexpr int kFlowTile = 256;

// FLAT tiles of 1024 and 2048 nnz (k_flat) remember the rows their search found.
bool uses_row_map(int variant, int tile) { return variant == PF_FLAT && (tile == 1024 || tile == 2048); }

constexpr long long kXcdL2Bytes = 4LL << 20;  // MI355X: 4 MB of L2 per XCD
// AUTO's row groups: at most 2^18 rows whose values and columns fit the 256 MB MALL
constexpr long long kRowGroupRowsMax = 1LL << 18;
constexpr long long kRowGroupBytesMax = 256LL << 20;
constexpr long long kChipLanes = 256LL * 2048;  // lanes resident on the chip: 256 CUs x 32 waves x 64

// Tiles per XCD list of an x-window schedule: an even share plus 2% slack.
long long sched_cap(long long ntiles) { return (ntiles + kXcds - 1) / kXcds + ntiles / 400 + 1; }

int value_bytes(int dtype);

// Rows that span several tiles over an x larger than one XCD's L2: deal the
// split-row FLAT tiles to XCDs by the part of x they start in.
int x_windows_rule(const pf_row_stats &s, long long n, int dtype, int tile, int row_aligned)
{
    return (!row_aligned && s.max_row_len >= 4LL * tile && n * value_bytes(dtype) > kXcdL2Bytes) ? 1 : 0;
}

int value_bytes(int dtype) { return dtype == PF_F64 ? 8 : dtype == PF_F32 ? 4 : dtype == PF_F16 ? 2 : 0; }

// XCD chunks of FLAT 1024/2048 tiles.  The eight XCDs stream neighbouring
// chunks of 2^15 nnz rather than eight distant eighths of the matrix: C2
// (row-aligned, 1024-nnz tiles) 56.7 instead of 58.3 us per call in fp64,
// 32.6 instead of 33.7 in fp16, and C3 (split rows) 213.8 instead of 216.3.
// Matrices of very short rows (under 4 nnz on average, as C4: 2.5) keep one
// chunk per XCD: their x neighbourhood spans more rows than a chunk holds, and
// chunks of 2^15 nnz cost 1-2 us of 320 there (2^12: 354 us).
constexpr long long kChunkNnz = 1LL << 15;
long long chunk_rule(const pf_row_stats &s) { return s.nnz < 4LL * s.m ? 0 : kChunkNnz; }
// Bytes of one split-row partial sum (head / tail slot): fp32 in the fp16 mode.
int slot_bytes(int dtype) { return dtype == PF_F16 ? 4 : value_bytes(dtype); }

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int default_tile(int variant, int dtype)
{
    if (variant == PF_PREFREE) return 512;  // 128 threads x P_NNZ 4, preFreeSpMV.cu:583-587
    if (variant == PF_ADAPTIVE) return dtype == PF_F64 ? 512 : 440;
    return dtype == PF_F64 ? 1024 : 2048;  // FLAT: the measured best per value type on C2-C5 (fp16 as fp32)
}

// Wave64s of the ADAPTIVE kernel resident at once on an MI355X (256 CUs x 4
// SIMDs x the waves per SIMD the gfx950 build of each tile size reaches).
// Used when no device is queried (pf_select); plans ask the device.
long long nominal_resident_waves(int dtype, int tile)
{
    int per_simd = 4;
    if (tile == kFlowTile) per_simd = dtype == PF_F64 ? 7 : 8;
    else if (dtype == PF_F64) per_simd = tile == 188 ? 7 : tile == 238 ? 6 : tile == 494 ? 4 : 3;
    else per_simd = tile == 440 || tile == 494 ? 5 : 2;
    return 256LL * 4 * per_simd;
}

// The tiles of 494 / 238 keys hold only rows of at most 16 nnz (LMAX 16).
bool short_row_tile(int tile) { return tile == 494 || tile == 238; }

// Consecutive tiles per wave.  Short-row tiles: at most 3, so that several
// dispatch rounds keep the tiles in flight on an XCD close together in x
// (measured best on the banded and very sparse configurations).  Other tiles:
// enough that every resident wave gets one run, at most 16.
int choose_run(int tile, long long ntiles, long long resident)
{
    if (resident <= 0) return 8;
    long long r = (ntiles + resident - 1) / resident;
    const long long cap = short_row_tile(tile) ? 3 : 16;
    return (int)(r < 1 ? 1 : (r > cap ? cap : r));
}

// ---- tuning table (written by the offline tuner, prefree-public_amd/tune) ----
//
// One row per (size class, row-length class, value type): nnz below
// `nnz_upper` (-1: no bound) and the matrix's row-length class select
// (variant, tile, run_tiles, keep_cached, ladder, hybrid), or variant "auto"
// (tile 0): the built-in rules.  The row-length
// classes are the cuts of the built-in rules below: "short" (every row <= 256
// nnz, under 4 nnz per row on average), "regular" (every row <= 256 nnz),
// "skewed" (longer rows, under 16 nnz per row on average), "dense" (longer
// rows, 16 or more on average); "any" matches every matrix.  Loaded by
// pf_set_tuning_table, else from $PREFREE_TUNING_TABLE (an empty value: no
// table), else from tune/mi355x_tuning_table.txt beside this library's lib/
// directory; consulted by PF_AUTO before the built-in rules.  This replaces
// the reference tuner's generated size-class dispatch
// (templates/preFreeSpMV_template.cu.j2:845-1003).
enum RowClass { kRowsAny = -1, kRowsShort = 0, kRowsRegular, kRowsSkewed, kRowsDense };

int row_class(const pf_row_stats &s)
{
    if (s.max_row_len <= PFK_ALIGN_ROW_MAX) return s.nnz < 4LL * s.m ? kRowsShort : kRowsRegular;
    return s.nnz < 16LL * s.m ? kRowsSkewed : kRowsDense;
}

int parse_rows(const std::string &v)
{
    return v == "any" ? kRowsAny : v == "short" ? kRowsShort : v == "regular" ? kRowsRegular
         : v == "skewed" ? kRowsSkewed : v == "dense" ? kRowsDense : -2;
}

struct TableRow {
    std::string name;
    long long nnz_upper;
    int rows, dtype, variant, tile, run, keep, ladder, hybrid;
};

std::mutex g_table_mu;
std::vector<TableRow> g_table;
std::string g_table_path;
bool g_table_env_done = false;

int parse_dtype(const std::string &s)
{
    return s == "f64" ? PF_F64 : s == "f32" ? PF_F32 : s == "f16" ? PF_F16 : -1;
}
int parse_variant(const std::string &s)
{
    return s == "adaptive" ? PF_ADAPTIVE : s == "flat" ? PF_FLAT : s == "prefree" ? PF_PREFREE
         : s == "auto" ? PF_AUTO : -1;
}

// Rows: `class nnz_upper rows dtype variant tile run keep ladder hybrid`, or
// the older `class nnz_upper dtype variant tile run keep` (rows "any", the
// default ladder, hybrid allowed).
int load_table(const char *path, std::vector<TableRow> &out, std::string &why)
{
    std::ifstream f(path);
    if (!f) {
        why = std::string("cannot open tuning table ") + path;
        return PF_ERR_IO;
    }
    std::string line;
    int lineno = 0;
    out.clear();
    while (std::getline(f, line)) {
        ++lineno;
        const size_t hash = line.find('#');
        if (hash != std::string::npos) line.resize(hash);
        std::istringstream in(line);
        std::vector<std::string> w;
        for (std::string t; in >> t;) w.push_back(t);
        if (w.empty()) continue;  // blank or comment
        const auto bad = [&](const char *what) {
            why = std::string(path) + ":" + std::to_string(lineno) + ": " + what;
            return PF_ERR_IO;
        };
        if (w.size() != 7 && w.size() != 10)
            return bad("expected 'class nnz_upper rows dtype variant tile run keep ladder hybrid'");
        const bool v2 = w.size() == 10;
        const size_t o = v2 ? 1 : 0;
        TableRow r;
        r.name = w[0];
        r.rows = v2 ? parse_rows(w[2]) : kRowsAny;
        r.dtype = parse_dtype(w[2 + o]);
        r.variant = parse_variant(w[3 + o]);
        try {
            size_t used = 0;
            const auto num = [&](const std::string &t) {
                const long long v = std::stoll(t, &used);
                if (used != t.size()) throw std::invalid_argument(t);
                return v;
            };
            r.nnz_upper = num(w[1]);
            r.tile = (int)num(w[4 + o]);
            r.run = (int)num(w[5 + o]);
            r.keep = (int)num(w[6 + o]);
            r.ladder = v2 ? (int)num(w[8]) : 0;
            r.hybrid = v2 ? (int)num(w[9]) : 1;
        } catch (const std::exception &) {
            return bad("not a number");
        }
        if (r.rows < -1 || r.dtype < 0 || r.variant < 0 || (r.variant == PF_AUTO ? r.tile != 0 : r.tile <= 0) ||
            r.run < 0 || r.run > 256 || r.keep < 0 ||
            r.keep > 1 || r.ladder < 0 || r.ladder > 5 || (r.ladder != 0 && r.variant != PF_PREFREE) ||
            r.hybrid < 0 || r.hybrid > 1)
            return bad("bad value");
        out.push_back(r);
    }
    return PF_OK;
}

// tune/mi355x_tuning_table.txt beside the lib/ directory holding this library.
std::string default_table_path()
{
    Dl_info di;
    if (!dladdr(reinterpret_cast<void *>(&default_table_path), &di) || !di.dli_fname) return std::string();
    std::string lib(di.dli_fname);
    const size_t slash = lib.rfind('/');
    const std::string dir = slash == std::string::npos ? std::string(".") : lib.substr(0, slash);
    return dir + "/../tune/mi355x_tuning_table.txt";
}

// Loads the table once per process unless pf_set_tuning_table chose one.
// Caller holds g_table_mu.
void table_init_locked()
{
    if (g_table_env_done) return;
    g_table_env_done = true;
    const char *env = std::getenv("PREFREE_TUNING_TABLE");
    const std::string path = env ? std::string(env) : default_table_path();
    std::string why;
    if (!path.empty() && load_table(path.c_str(), g_table, why) == PF_OK) {
        g_table_path = path;
    } else {
        g_table.clear();
        g_table_path.clear();
    }
}

bool tile_supported(int variant, int dtype, int tile);

// Decision of PF_AUTO: variant and tile, plus the run length and cache
// policy when a tuning-table row fixes them (run 0 / keep -1: not fixed), the
// PREFREE ladder (0: the default) and whether FLAT may turn hybrid.
struct Choice {
    int variant = PF_ADAPTIVE, tile = 0, run = 0, keep = -1, ladder = 0;
    bool hybrid = true;
};

bool table_choice(const pf_row_stats &s, int dtype, Choice &c)
{
    std::lock_guard<std::mutex> lock(g_table_mu);
    table_init_locked();
    const int rc = row_class(s);
    for (const TableRow &r : g_table) {
        if (r.dtype != dtype || (r.nnz_upper >= 0 && s.nnz >= r.nnz_upper)) continue;
        if (r.rows != kRowsAny && r.rows != rc) continue;
        if (r.variant == PF_AUTO) return false;  // this class keeps the built-in rules
        if (!tile_supported(r.variant, dtype, r.tile)) continue;
        c.variant = r.variant;
        c.tile = r.tile;
        c.run = r.run;
        c.keep = r.keep;
        c.ladder = r.ladder;
        c.hybrid = r.hybrid != 0;
        return true;
    }
    return false;
}

// Lanes per row of a row-group plan (powers of two, 2..32): never more than the longest row needs for
// one pass; about half the mean row where the rows outnumber the chip's lanes (a lane's few loads in a row
// keep more in flight than idle lanes do), else as many as still fit the chip's resident lanes, up to four
// times the mean row or a quarter of the longest (more waves cost launch time where the rows are short).
// Measured on MI355X, graph-timed, uniform random columns, us per SpMV (fp64): 2048 rows of 2 nnz: 8 lanes
// 1.82 (2 lanes 2.19); 32768 x 2: 8 lanes 2.17 (16: 2.46); 131072 x 2: 4 lanes 3.27 (2: 3.65, 8: 3.80);
// 131072 x 8: 4 lanes 7.37 (16: 7.50); 131072 x 32: 16 lanes 24.8 (32: 25.6, 8: 27.1); 262144 x 2:
// 2 lanes 5.35 (4: 5.63).
int row_group_lanes(const pf_row_stats &s)
{
    int lat = 2;
    while (lat < 32 && lat < s.max_row_len) lat <<= 1;
    const double mean = (double)s.nnz / (double)s.m;
    int thr = 2;  // the power of two nearest half the mean row
    while (thr < 32 && 0.5 * mean >= thr * 1.4142135623730951) thr <<= 1;
    const double cap = std::max(4.0 * mean, s.max_row_len / 4.0);
    int fill = 2;
    while (fill < 32 && 2LL * fill * s.m <= kChipLanes && 2 * fill <= cap) fill <<= 1;
    return std::min(lat, std::max(thr, fill));
}

// PF_AUTO: a tuning-table row if one matches; else
//   * at most 2^18 rows, none longer than PFK_ALIGN_ROW_MAX, values and
//     columns within 256 MB (MALL-resident across calls): FLAT row groups,
//     row_group_lanes lanes per row (k_vector: no tiles, no workspace, one
//     launch; fp64 C1 1.9 us per SpMV in a graph against 3.5 for 1024-nnz
//     tiles; 131072 rows of 32 nnz 24.8 against 28.7; 262144 x 64 86 against
//     99; 262144 x 128, 403 MB, 239 against 192 for 2048-nnz tiles; 393216 x
//     8, 23.8 for 1024-nnz tiles against 24.3 for the best row groups);
//   * no row longer than PFK_ALIGN_ROW_MAX, or fp16 values (FLAT only): FLAT
//     (1024 nnz per tile for fp64, 2048 for fp32 / fp16 or for rows of under
//     4 nnz on average), row-aligned when the rows fit: one launch per call;
//   * a matrix too small to give half the resident waves a 512-key tile:
//     ADAPTIVE with the smallest tile (one wave per tile, launch-bound anyway);
//   * long rows carrying most of the nnz (mean >= 16, e.g. a few dense rows):
//     split-row FLAT with 2048-nnz tiles;
//   * otherwise split-row FLAT with 1024-nnz tiles.
// Split-row FLAT plans deal their tiles to XCDs by x window when rows span
// several tiles over an x larger than one XCD's L2 (x_windows_rule).
// (Measured on MI355X, us per call: C2 row-aligned FLAT 58.4 vs ADAPTIVE 75.0;
// C4 346 vs 400; C1 3.3 vs ADAPTIVE-188 4.5; C5 FLAT 2048 with x windows 1107 vs
// ADAPTIVE 1494, fp32 679 vs 882; C3 FLAT 1024 with x windows 210 vs 2048 219
// vs ADAPTIVE 230.)
Choice auto_choice(const pf_row_stats &s, int dtype)
{
    Choice c;
    if (table_choice(s, dtype, c)) return c;
    const long long m = s.m, nnz = s.nnz;
    c.variant = PF_FLAT;
    if (s.max_row_len <= PFK_ALIGN_ROW_MAX && m > 0 && m <= kRowGroupRowsMax &&
        nnz * (value_bytes(dtype) + 4) <= kRowGroupBytesMax) {
        c.tile = row_group_lanes(s);
        return c;
    }
    if (s.max_row_len <= PFK_ALIGN_ROW_MAX || dtype == PF_F16) {
        c.tile = default_tile(PF_FLAT, dtype);
        // Rows of under 4 nnz on average: a tile spends much of its time per
        // row, and 2048 nnz per workgroup keep twice the loads in flight
        // (C4 fp64: 333 instead of 347 us; C2, 5 nnz per row: 58.5 vs 59.3).
        if (nnz < 4 * m) c.tile = 2048;
        return c;
    }
    const int big = default_tile(PF_ADAPTIVE, dtype);
    if (dtype == PF_F64 && (nnz + m) / big < nominal_resident_waves(dtype, big) / 2) {
        c.variant = PF_ADAPTIVE;
        c.tile = 188;
        return c;
    }
    c.tile = nnz >= 16 * m ? 2048 : 1024;
    return c;
}

bool tile_supported(int variant, int dtype, int tile)
{
    int t[PFK_MAX_TILES];
    const int n = pfk_supported_tiles(variant, dtype, t, PFK_MAX_TILES);
    for (int i = 0; i < n; ++i)
        if (t[i] == tile) return true;
    return false;
}

// Workgroups launched: ADAPTIVE runs of run_tiles tiles, four waves per
// workgroup, runs dealt evenly to the XCDs; row groups ntiles workgroups; one
// tile per workgroup otherwise (FLAT 1024/2048: tiles padded to whole rounds
// of XCD chunks).
void set_grid(pf_plan_info &r)
{
    if (r.variant == PF_ADAPTIVE || (r.variant == PF_FLAT && r.tile == kFlowTile)) {
        const long long run = r.run_tiles > 0 ? r.run_tiles : 1;
        const long long nruns = (r.ntiles + run - 1) / run;
        const long long tx = (nruns + kXcds - 1) / kXcds;
        r.grid = ((tx + 3) / 4) * kXcds;
    } else if (uses_row_map(r.variant, r.tile)) {
        r.grid = pfk_flat_grid(r.ntiles, r.tile, r.chunk_nnz);
    } else if (r.variant == PF_FLAT && PFK_ROW_GROUP_TILE(r.tile)) {
        r.grid = r.ntiles;  // row groups: one workgroup per 256 lanes, by index
    } else {
        r.grid = ((r.ntiles + kXcds - 1) / kXcds) * kXcds;
    }
}

// A tuning-table row may fix the run length and cache policy of ADAPTIVE and
// the reduction ladder of PREFREE.
void apply_overrides(const Choice &c, pf_plan_info &info)
{
    if (info.variant == PF_PREFREE && c.ladder > 0) info.ladder = c.ladder;
    if (info.variant != PF_ADAPTIVE) return;
    if (c.run > 0) {
        info.run_tiles = c.run;
        set_grid(info);
    }
    if (c.keep >= 0) info.keep_cached = c.keep;
}

// Fills everything in `info` that follows from (stats, dtype, variant, tile).
int finish_info(const pf_row_stats &s, int dtype, int variant, int tile, pf_plan_info *info)
{
    if (!tile_supported(variant, dtype, tile))
        return fail(PF_ERR_UNSUPPORTED, "tile " + std::to_string(tile) + " not compiled for this variant/dtype");
    pf_plan_info r;
    std::memset(&r, 0, sizeof r);
    r.variant = variant;
    r.dtype = dtype;
    r.tile = tile;
    const long long m = s.m, nnz = s.nnz;
    // A regular matrix keeps row index and key position nearly proportional:
    // one interpolated probe round of 64 rows brackets the row when their
    // spacing covers the largest distance of a row from its guess (the row
    // search's answer lies within guess_dev + 2 rows of the guess).  The
    // smallest such spacing leaves the fewest rows to the closing round.
    const bool regular = s.max_row_len <= 64;
    int spread = 1;
    while (spread < 64 && 31LL * spread < s.guess_dev + 3) spread *= 2;
    r.guess_spread = regular ? spread : 0;
    // A matrix whose row_ptr is nearly a straight line away from its ends (C2: the first grid row's rows are a
    // nnz shorter than the rest, which shifts every later row 410 rows off the mean-density guess) puts almost
    // every row within 28 rows of the line through its quartile rows: row-aligned tiles then centre their
    // first probe round there, 1 row apart, and most searches end in that round.
    const long long q1 = m / 4, q3 = 3 * m / 4;
    if (regular && m >= 4 && s.line_q3_row_ptr > s.line_q1_row_ptr && s.line_far_rows * 256 <= m) {
        r.guess_a = (double)(q3 - q1) / ((double)s.line_q3_row_ptr - (double)s.line_q1_row_ptr);
        r.guess_b = (double)q1 - r.guess_a * (double)s.line_q1_row_ptr;
    }
    const long long vb = slot_bytes(dtype);
    if (variant == PF_ADAPTIVE) {
        r.long_row_min = pfk_adaptive_long_row_min(dtype, tile);
        const long long total = nnz + m;
        r.ntiles = total > 0 ? (total + tile - 1) / tile : 1;
        r.run_tiles = choose_run(tile, r.ntiles, nominal_resident_waves(dtype, tile));
        // Non-temporal col/val loads by default: they keep x in L2 and the MALL.
        // Ordinary loads (pf_plan_set_keep_cached) let a matrix that nearly fits the
        // 256 MB MALL survive between back-to-back calls: C2 72.5 instead of 74.8 us
        // per call, but 119 instead of 88 us when the caches start cold.
        r.keep_cached = 0;
        r.needs_fixup = s.max_row_len > r.long_row_min;
        r.workspace_bytes = (size_t)(r.ntiles * (2 * vb + 4) + 3 * 256);
    } else if (variant == PF_FLAT && PFK_ROW_GROUP_TILE(tile)) {  // row groups: `tile` lanes per row, by index
        r.long_row_min = 0;
        r.ntiles = std::max(1LL, (m * tile + 255) / 256);  // workgroups
        r.needs_fixup = 0;
        r.row_aligned = 1;  // no row is split
        r.workspace_bytes = 256;
    } else if (variant == PF_FLAT) {
        r.long_row_min = 0;
        r.ntiles = nnz > 0 ? (nnz + tile - 1) / tile : 1;
        r.needs_fixup = r.ntiles > 1;
        r.workspace_bytes = (size_t)(r.ntiles * (2 * vb + 4) + 3 * 256);
        if (uses_row_map(PF_FLAT, tile)) {
            r.workspace_bytes += (size_t)(r.ntiles + 1) * 8 + 256;
            r.workspace_bytes += (size_t)PFK_SCHED_INTS(r.ntiles, sched_cap(r.ntiles)) * 4 + 512;
            // Short rows only: each tile owns the rows starting in it, nothing
            // is split and a step is one launch.
            r.row_aligned = s.max_row_len <= PFK_ALIGN_ROW_MAX ? 1 : 0;
            if (r.row_aligned) r.needs_fixup = 0;
            r.x_windows = x_windows_rule(s, s.m, dtype, tile, r.row_aligned);  // n taken as m; plans use n
            r.chunk_nnz = chunk_rule(s);
        }
        if (tile == kFlowTile) {  // runs of tiles, rows carried across tile edges inside a run
            r.run_tiles = choose_run(tile, r.ntiles, nominal_resident_waves(dtype, tile));
            r.needs_fixup = r.ntiles > r.run_tiles;
        }
    } else if (variant == PF_PREFREE) {
        r.long_row_min = 0;
        r.ntiles = nnz > 0 ? (nnz + tile - 1) / tile : 1;
        r.needs_fixup = 0;
        r.workspace_bytes = 256;
        if (dtype == PF_F16)  // fp32 partials of each tile's boundary rows (head, tail) and its row range
            r.workspace_bytes += (size_t)(2 * ((r.ntiles * 4 + 255) & ~255LL) + ((r.ntiles * 8 + 255) & ~255LL));
        r.ladder = 3;  // the reference's active ladder, preFreeSpMV.cu:466-483
    } else {
        return fail(PF_ERR_INVALID, "unknown variant");
    }
    set_grid(r);
    *info = r;
    return PF_OK;
}

}  // namespace

struct pf_plan {
    int m = 0, n = 0, nnz = 0;
    double plan_ms = 0.0, plan_gpu_ms = 0.0;  // planning: wall time, and GPU time of its kernels (events)
    int band_avail = 0;                        // band width the band kernel may use (0: the plan has no band)
    pf_plan_info info{};
    pf_row_stats stats{};
    void *ws = nullptr;        // the error flag, and (ws_split == nullptr) the split-row arrays after it
    void *ws_split = nullptr;  // a hybrid plan's split-row arrays, allocated once pf_plan_set_hybrid(plan, 0) asks
    bool split_ready = true;   // the split-row arrays exist (a hybrid plan is built without them)
    void *head = nullptr;
    void *tail = nullptr;
    int *owner = nullptr;
    int *err = nullptr;
    int *row_map = nullptr;  // FLAT 1024/2048: tile -> (first row, row_ptr there), found by the first call
    bool map_ready = false;  // set once a call that records the map has been issued
    int *sched = nullptr;    // split-row FLAT 1024/2048: x-window schedule, recorded with the map
    long long sched_cap = 0;
    bool remember_rows = true;  // false: every call searches row_ptr (no row map, no schedule)
    // bytes of the workspace behind each array (passed to the kernel layer, which checks them)
    size_t head_bytes = 0, tail_bytes = 0, owner_bytes = 0, row_map_bytes = 0, sched_bytes = 0;
    // hybrid plans: dense rows by x windows, the rows between them in runs of row-aligned tiles
    bool hybrid = false;     // the hybrid path is in use (it can be switched off: the split-row layout stays)
    void *ws_hyb = nullptr;  // its tables: dense rows, runs, run tile map, segment bounds, partial sums
    int n_dense = 0, n_runs = 0, n_win = 0, run_tile = 0;
    long long run_tiles = 0, run_chunk = 0;
    int *dense_rows = nullptr, *runs = nullptr, *run_map = nullptr, *dense_seg = nullptr;
    void *dense_part = nullptr;
    size_t runs_bytes = 0, run_map_bytes = 0, dense_seg_bytes = 0, dense_part_bytes = 0;
    bool hyb_map_ready = false;
    bool x_halves = false;       // run tiles processed per half of x (see pfk_spmv_args.x_halves)
    void *half_part = nullptr;   // [m] second-half row sums
    size_t half_part_bytes = 0;
    unsigned char *row_apart = nullptr;  // [m] 1 for the rows summed apart (see pfk_spmv_args.row_apart)
    size_t row_apart_bytes = 0;
    // long mode: the long rows (dense_rows) cut into tiles of PFK_LONG_TILE nnz instead of x windows
    bool long_mode = false;
    int n_long_tiles = 0;
    int *long_tiles = nullptr, *long_deal = nullptr, *long_row_tiles = nullptr;
    void *long_part = nullptr;
    size_t long_tiles_bytes = 0, long_deal_bytes = 0, long_row_tiles_bytes = 0, long_part_bytes = 0;
    // the runs' stream beside the caller's, and the events that fork and join it (see pfk_spmv_args)
    void *aux_stream = nullptr, *ev_fork = nullptr, *ev_join = nullptr;
};

namespace {

// Launch configuration of a plan for a validated matrix with known statistics
// (host only, apart from occupancy queries): variant and tile (PF_AUTO
// resolved), run length, x windows, workspace size.
// `allow_hybrid` (optional) tells whether a FLAT plan of PF_AUTO may turn
// hybrid: always, unless a tuning-table row says otherwise.
int plan_info(const pf_row_stats &s, int n, int dtype, int variant, int tile, pf_plan_info *out,
              bool *allow_hybrid = nullptr)
{
    Choice c;
    if (allow_hybrid) *allow_hybrid = true;
    if (variant == PF_AUTO) {  // an explicit tile is kept only if the chosen variant has it
        c = auto_choice(s, dtype);
        if (allow_hybrid) *allow_hybrid = c.hybrid;
        variant = c.variant;
        if (tile <= 0 || !tile_supported(variant, dtype, tile)) tile = c.tile;
    }
    pf_plan_info info;
    const int st = finish_info(s, dtype, variant, tile > 0 ? tile : default_tile(variant, dtype), &info);
    if (st != PF_OK) return st;
    if (info.variant == PF_ADAPTIVE || (info.variant == PF_FLAT && info.tile == kFlowTile)) {
        long long resident = 0;
        const int rs = info.variant == PF_ADAPTIVE ? pfk_adaptive_resident_waves(dtype, info.tile, &resident)
                                                   : pfk_flow_resident_waves(dtype, &resident);
        if (rs == PF_OK && resident > 0) {
            info.run_tiles = choose_run(info.tile, info.ntiles, resident);
            if (info.variant == PF_FLAT) info.needs_fixup = info.ntiles > info.run_tiles;
            set_grid(info);
        }
    }
    if (c.tile == info.tile && c.variant == info.variant) apply_overrides(c, info);
    if (uses_row_map(info.variant, info.tile))
        info.x_windows = x_windows_rule(s, n, dtype, info.tile, info.row_aligned);
    *out = info;
    return PF_OK;
}

// Points the plan's arrays into its workspace `w` (info.workspace_bytes bytes,
// 256-byte aligned): error flag, head / tail slots, owners, row map, schedule.
// The split-row arrays of a workspace block of info.workspace_bytes (its first
// 256 bytes hold the error flag).
void plan_carve_split(pf_plan *p, void *w0)
{
    const pf_plan_info &info = p->info;
    char *w = static_cast<char *>(w0);
    const size_t total = info.workspace_bytes;
    if (info.variant == PF_FLAT && PFK_ROW_GROUP_TILE(info.tile)) {  // row groups: the error flag only
        p->split_ready = true;
        return;
    }
    if (info.variant != PF_PREFREE) {
        const size_t vb = (size_t)slot_bytes(info.dtype);
        const size_t slots = ((size_t)info.ntiles * vb + 255) & ~(size_t)255;
        const size_t owner_at = 256 + 2 * slots;
        p->head = w + 256;
        p->tail = w + 256 + slots;
        p->owner = reinterpret_cast<int *>(w + owner_at);
        p->head_bytes = p->tail_bytes = slots;
        p->owner_bytes = total - owner_at;
        if (uses_row_map(info.variant, info.tile)) {
            const size_t owners = ((size_t)info.ntiles * 4 + 255) & ~(size_t)255;
            const size_t map = ((size_t)(info.ntiles + 1) * 8 + 255) & ~(size_t)255;
            p->row_map = reinterpret_cast<int *>(w + owner_at + owners);
            p->sched = reinterpret_cast<int *>(w + owner_at + owners + map);
            p->sched_cap = sched_cap(info.ntiles);
            p->owner_bytes = owners;
            p->row_map_bytes = map;
            p->sched_bytes = total - (owner_at + owners + map);
        }
    } else if (info.dtype == PF_F16) {  // PREFREE fp16: boundary-row partials, then the tiles' row ranges
        const size_t slots = ((size_t)info.ntiles * 4 + 255) & ~(size_t)255;
        p->head = w + 256;
        p->tail = w + 256 + slots;
        p->owner = reinterpret_cast<int *>(w + 256 + 2 * slots);
        p->head_bytes = p->tail_bytes = slots;
        p->owner_bytes = total - (256 + 2 * slots);
    }
    p->split_ready = true;
}

void plan_carve(pf_plan *p, void *w0)
{
    p->ws = w0;
    p->err = static_cast<int *>(w0);
    plan_carve_split(p, w0);
}

// Fresh workspace state on `stream` (fill kernels, no memset): error flag
// clear, every owner slot "no split row" (a combine kernel never reads an
// unset slot), and ADAPTIVE's split-row owner table, which depends on
// row_ptr only.  Asynchronous.
int plan_init_split(pf_plan *p, const int *d_row_ptr, void *stream)
{
    const pf_plan_info &info = p->info;
    int rc = PF_OK;
    if (p->owner) rc = pfk_fill_u32(p->owner, (size_t)info.ntiles, 0xFFFFFFFFu, stream);
    if (rc == PF_OK && info.variant == PF_ADAPTIVE && info.needs_fixup) {
        pfk_spmv_args a;
        std::memset(&a, 0, sizeof a);
        a.row_ptr = d_row_ptr;
        a.m = p->m;
        a.n = p->n;
        a.nnz = p->nnz;
        a.tile = info.tile;
        a.guess_spread = info.guess_spread;
        a.run_tiles = info.run_tiles;
        a.ntiles = info.ntiles;
        a.owner_row = p->owner;
        a.owner_bytes = p->owner_bytes;
        a.err_flag = p->err;
        rc = pfk_adaptive_owners(info.dtype, &a, stream);
    }
    return rc;
}

int plan_init(pf_plan *p, const int *d_row_ptr, void *stream)
{
    const int rc = pfk_fill_zero(p->err, 256, stream);
    return rc == PF_OK ? plan_init_split(p, d_row_ptr, stream) : rc;
}

// The split-row arrays of a plan built without them (a hybrid plan), in a
// block of their own: the error flag stays where it is.  Synchronises the
// default stream.
int plan_add_split(pf_plan *p)
{
    if (p->split_ready) return PF_OK;
    void *w = nullptr;
    PF_TRY(pfk_malloc(&w, p->info.workspace_bytes), "split-row workspace");
    plan_carve_split(p, w);
    int rc = plan_init_split(p, nullptr, nullptr);  // FLAT: no row_ptr needed
    if (rc == PF_OK) rc = pfk_stream_sync(nullptr);
    if (rc != PF_OK) {
        pfk_free(w);
        p->head = p->tail = nullptr;
        p->owner = p->row_map = p->sched = nullptr;
        p->head_bytes = p->tail_bytes = p->owner_bytes = p->row_map_bytes = p->sched_bytes = 0;
        p->split_ready = false;
        return from_kernel_layer(rc, "split-row workspace");
    }
    p->ws_split = w;
    return PF_OK;
}

// Dense-row threshold of a hybrid plan: a power of two at least 4096 and at
// least 256 n / W, so that a dense row averages 256 or more nnz per x window.
long long dense_min(long long n, int dtype)
{
    const long long want = std::max(4096LL, (256LL * n + PFK_DENSE_WINDOW(dtype) - 1) / PFK_DENSE_WINDOW(dtype));
    long long t = 4096;
    while (t < want) t <<= 1;
    return t;
}

// Rows of at least 2^j nnz, from the log2 histogram (bucket k: 2^(k-1) <= len < 2^k).
long long rows_at_least_pow2(const pf_row_stats &s, int j)
{
    long long c = 0;
    for (int k = j + 1; k < 33; ++k) c += s.hist_log2[k];
    return c;
}

// A hybrid plan fits split-row FLAT matrices with some rows over 256 nnz and
// checked columns (the planning scan reads col) when those rows may all be
// dense (the histogram allows it) or x exceeds one XCD's L2 (long mode);
// try_hybrid decides.
// What the planning scan (pfk_plan_scan) found about the long rows: the list
// on the device (the first `cap` of them), how many there are, and whether
// the descents inside them were all counted (then `desc` is their number).
struct PlanScan {
    const int *list = nullptr;  // int4 (row, first nnz, end, 0) per long row, in no particular order
    long long cap = 0, listed = 0, desc = 0;
    bool checked = false;
    std::vector<int> host;  // the first host_n entries of the list, copied with the statistics
    long long host_n = 0;
    bool complete() const { return list && listed <= cap && checked; }
};

// Events around the GPU work of planning: their sum is the plan's GPU time.
struct PlanTimer {
    void *e[2] = {nullptr, nullptr};
    double gpu_ms = 0.0;
    bool ok = false;
    explicit PlanTimer() { ok = pfk_event_create(&e[0]) == PF_OK && pfk_event_create(&e[1]) == PF_OK; }
    ~PlanTimer() { pfk_event_destroy(e[0]); pfk_event_destroy(e[1]); }
    void start(void *stream) { if (ok) ok = pfk_event_record(e[0], stream) == PF_OK; }
    void stop(void *stream)  // after the work it times has been synchronised
    {
        float ms = 0.f;
        if (ok) ok = pfk_event_record(e[1], stream) == PF_OK && pfk_event_sync(e[1]) == PF_OK &&
                     pfk_event_elapsed_ms(&ms, e[0], e[1]) == PF_OK;
        if (ok) gpu_ms += ms;
    }
};

bool hybrid_candidate(const pf_row_stats &s, long long n, int dtype, const pf_plan_info &info, const int *d_col)
{
    if (!d_col || (dtype != PF_F64 && dtype != PF_F32 && dtype != PF_F16) || info.variant != PF_FLAT || info.row_aligned ||
        !uses_row_map(info.variant, info.tile) || s.n_long_rows < 1)
        return false;
    const long long t = dense_min(n, dtype);
    int j = 0;
    while ((1LL << j) < t) ++j;
    return rows_at_least_pow2(s, j) == s.n_long_rows || n * value_bytes(dtype) > kXcdL2Bytes;
}

// Adds the hybrid path to a split-row FLAT plan.  A planning scan lists the
// rows over 256 nnz and checks their columns.  When they are all dense rows
// (dense_min nnz or more) with sorted columns, they are summed by x windows
// (dense mode); otherwise, when they hold a tile (1024 nnz) or more on average
// and x exceeds one XCD's L2, they are cut into tiles dealt to the XCDs by
// their first column (long mode).  The rows between them are cut into runs of
// row-aligned tiles.  Leaves the plan as it is (split-row tiles) otherwise.
int try_hybrid(pf_plan *p, const int *d_row_ptr, const int *d_col, void *stream, const PlanScan *scan,
               PlanTimer *timer)
{
    const int dtype = p->info.dtype;
    const long long cap = p->stats.n_long_rows;
    std::vector<int> list((size_t)(3 * cap));
    int cnt[2] = {0, 0};
    int st = PF_OK;
    if (scan && scan->complete() && scan->listed == cap) {
        // the planning scan listed every long row and counted the descents inside them: no second pass over col
        std::vector<int> l4;
        if (cap <= scan->host_n) {  // copied with the statistics
            l4.assign(scan->host.begin(), scan->host.begin() + 4 * cap);
        } else {
            l4.resize((size_t)(4 * cap));
            st = pfk_memcpy_d2h(l4.data(), scan->list, l4.size() * sizeof(int), stream);
            if (st == PF_OK) st = pfk_stream_sync(stream);
            if (st != PF_OK) return from_kernel_layer(st, "long-row list");
        }
        for (long long k = 0; k < cap; ++k)
            for (int j = 0; j < 3; ++j) list[(size_t)(3 * k + j)] = l4[(size_t)(4 * k + j)];
        cnt[0] = (int)cap;
        cnt[1] = scan->desc > 0 ? 1 : 0;
    } else {
        int *tmp = nullptr;
        PF_TRY(pfk_malloc(reinterpret_cast<void **>(&tmp), (size_t)(2 + 3 * cap) * sizeof(int)),
               "long-row scan buffer");
        if (timer) timer->start(stream);
        st = pfk_fill_zero(tmp, 2 * sizeof(int), stream);
        if (st == PF_OK)
            st = pfk_dense_scan(d_row_ptr, d_col, p->m, PFK_ALIGN_ROW_MAX + 1, tmp + 2, (int)cap, tmp, stream);
        if (st == PF_OK) st = pfk_memcpy_d2h(cnt, tmp, sizeof cnt, stream);
        if (st == PF_OK) st = pfk_memcpy_d2h(list.data(), tmp + 2, list.size() * sizeof(int), stream);
        if (st == PF_OK) st = pfk_stream_sync(stream);
        if (st == PF_OK && timer) timer->stop(stream);
        pfk_free(tmp);
        if (st != PF_OK) return from_kernel_layer(st, "long-row scan");
    }
    if (cnt[0] != cap) return PF_OK;  // row_ptr and the statistics disagree: stay split-row

    // Long rows ascending, and the runs of rows between them.
    std::vector<int> order((size_t)cap);
    for (long long k = 0; k < cap; ++k) order[(size_t)k] = (int)k;
    std::sort(order.begin(), order.end(), [&](int x, int y) { return list[3 * (size_t)x] < list[3 * (size_t)y]; });
    const int nd = (int)cap, nruns = nd + 1, R = nruns + 1;
    std::vector<int> rows((size_t)nd), rb0((size_t)nd), rb1((size_t)nd), runs((size_t)5 * R, 0);
    long long short_rows = 0, short_nnz = 0, long_nnz = 0, shortest = INT32_MAX;
    for (int i = 0; i < nd; ++i) {
        rows[(size_t)i] = list[3 * (size_t)order[(size_t)i]];
        rb0[(size_t)i] = list[3 * (size_t)order[(size_t)i] + 1];
        rb1[(size_t)i] = list[3 * (size_t)order[(size_t)i] + 2];
        long_nnz += rb1[(size_t)i] - rb0[(size_t)i];
        shortest = std::min(shortest, (long long)(rb1[(size_t)i] - rb0[(size_t)i]));
    }
    const int nwin = pfk_dense_nwin(p->n, dtype);
    const long long xb = (long long)p->n * value_bytes(dtype);
    const bool dense = cnt[1] == 0 && shortest >= dense_min(p->n, dtype) &&
                       cap * (nwin + 1) <= (64LL << 20);  // segment table under 256 MB
    const bool lng = !dense && long_nnz >= (long long)PFK_LONG_TILE * cap && xb > kXcdL2Bytes;
    if (!dense && !lng) return PF_OK;
    for (int i = 0; i < nruns; ++i) {
        const int rb = i == 0 ? 0 : rows[(size_t)i - 1] + 1;
        const int re = i == nd ? p->m : rows[(size_t)i];
        const int nb = i == 0 ? 0 : rb1[(size_t)i - 1];
        const int ne = i == nd ? p->nnz : rb0[(size_t)i];
        runs[(size_t)R + i] = rb;
        runs[(size_t)2 * R + i] = re;
        runs[(size_t)3 * R + i] = nb;
        runs[(size_t)4 * R + i] = ne;
        short_rows += re - rb;
        short_nnz += ne - nb;
    }
    // Run tiles: the FLAT rule for the short rows alone.
    const int K = (dtype == PF_F64 && short_nnz >= 4 * short_rows) ? 1024 : 2048;
    long long tiles = 0;
    for (int i = 0; i < nruns; ++i) {
        runs[(size_t)i] = (int)tiles;
        const long long rr = runs[(size_t)2 * R + i] - runs[(size_t)R + i];
        // the kernel starts a run's tiles at its first nnz rounded down to 64 (whole lines per load)
        const long long nz = runs[(size_t)4 * R + i] - (runs[(size_t)3 * R + i] & ~63LL);
        tiles += rr > 0 ? std::max(1LL, (nz + K - 1) / K) : 0;
    }
    runs[(size_t)nruns] = (int)tiles;  // 0 when every row is long: only the long-row kernels run
    // Long mode: each long row in tiles of PFK_LONG_TILE nnz from its first nnz rounded down to 64.
    // host arrays copied to the device stay alive until the stream is synchronised below
    std::vector<int> lt, row_tiles((size_t)nd + 1, 0), first, fc, deal;
    if (lng) {
        for (int i = 0; i < nd; ++i) {
            row_tiles[(size_t)i] = (int)(lt.size() / 4);
            const long long s0 = rb0[(size_t)i] & ~63LL;
            for (long long st0 = s0; st0 < rb1[(size_t)i]; st0 += PFK_LONG_TILE) {
                const long long f = std::max<long long>(st0, rb0[(size_t)i]);
                lt.insert(lt.end(), {i, (int)st0, (int)f, (int)std::min<long long>(rb1[(size_t)i], st0 + PFK_LONG_TILE)});
                first.push_back((int)f);
            }
        }
        row_tiles[(size_t)nd] = (int)(lt.size() / 4);
    }
    const long long nlt = lng ? (long long)lt.size() / 4 : 0;
    auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
    const size_t b_rows = up((size_t)nd * 4), b_runs = up((size_t)5 * R * 4), b_map = up((size_t)tiles * 32),
                 b_seg = dense ? up((size_t)nd * (nwin + 1) * 4) : 0,
                 b_part = dense ? up((size_t)nd * nwin * slot_bytes(dtype)) : up((size_t)nlt * slot_bytes(dtype)),
                 b_lt = up((size_t)nlt * 16), b_deal = up((size_t)nlt * 4), b_rt = lng ? up(((size_t)nd + 1) * 4) : 0,
                 b_half = up((size_t)p->m * value_bytes(dtype)), b_apart = up((size_t)p->m);
    // a plan built without a workspace (a hybrid candidate) keeps its error flag at the head of the tables
    const size_t b_err = p->err ? 0 : 256;
    for (int i = 1; i < nd; ++i)  // ascending: a row listed twice would sit next to itself
        if (rows[(size_t)i] == rows[(size_t)i - 1])
            return fail(PF_ERR_KERNEL, "hybrid plan: the planning scan listed a row twice");
    void *w = nullptr;
    PF_TRY(pfk_malloc(&w, b_err + b_half + b_apart + b_rows + b_runs + b_map + b_seg + b_part + b_lt + b_deal + b_rt),
           "hybrid tables");
    char *c = static_cast<char *>(w);
    p->ws_hyb = w;
    // zeroed together below: the error flag, the second-half sums, the apart flags
    if (b_err) p->err = reinterpret_cast<int *>(c);
    c += b_err;
    p->half_part = c;
    p->half_part_bytes = b_half;
    c += b_half;
    p->row_apart = reinterpret_cast<unsigned char *>(c);
    p->row_apart_bytes = b_apart;
    c += b_apart;
    // dense_rows and runs adjacent: one copy
    p->dense_rows = reinterpret_cast<int *>(c);
    c += b_rows;
    p->runs = reinterpret_cast<int *>(c);
    c += b_runs;
    p->run_map = reinterpret_cast<int *>(c);
    c += b_map;
    p->dense_seg = dense ? reinterpret_cast<int *>(c) : nullptr;
    c += b_seg;
    void *part = c;
    c += b_part;
    p->long_tiles = lng ? reinterpret_cast<int *>(c) : nullptr;
    c += b_lt;
    p->long_deal = lng ? reinterpret_cast<int *>(c) : nullptr;
    c += b_deal;
    p->long_row_tiles = lng ? reinterpret_cast<int *>(c) : nullptr;
    c += b_rt;
    p->runs_bytes = b_runs;
    p->run_map_bytes = b_map;
    p->dense_seg_bytes = b_seg;
    p->dense_part = dense ? part : nullptr;
    p->dense_part_bytes = dense ? b_part : 0;
    p->long_mode = lng;
    p->n_long_tiles = (int)nlt;
    p->long_part = lng ? part : nullptr;
    p->long_part_bytes = lng ? b_part : 0;
    p->long_tiles_bytes = b_lt;
    p->long_deal_bytes = b_deal;
    p->long_row_tiles_bytes = b_rt;
    p->n_dense = nd;
    p->n_runs = nruns;
    p->n_win = dense ? nwin : 0;
    p->run_tile = K;
    p->run_tiles = tiles;
    p->run_chunk = short_nnz < 4 * short_rows ? 0 : kChunkNnz;
    // The runs' random x gathers fall in half of x per XCD when x exceeds one
    // XCD's 4 MB L2 but a half of it nearly fits (x up to 24 MB).
    // fp16 sums each row once in fp32 and rounds it once: the halves' two sums would be rounded apart
    p->x_halves = dtype != PF_F16 && xb > kXcdL2Bytes && xb <= 6 * kXcdL2Bytes;
    p->info.x_halves = p->x_halves ? 1 : 0;
    // the error flag clear; rows the runs never write (the long rows) keep a zero second-half sum; exactly one
    // byte set per row summed apart, 0 for every other row (the combine relies on it: the rows are distinct)
    st = pfk_fill_zero(w, b_err + b_half + b_apart, stream);
    std::vector<int> stage((b_rows + b_runs) / 4, 0);  // alive until the stream is synchronised below
    std::copy(rows.begin(), rows.end(), stage.begin());
    std::copy(runs.begin(), runs.end(), stage.begin() + b_rows / 4);
    if (st == PF_OK) st = pfk_memcpy_h2d(p->dense_rows, stage.data(), b_rows + b_runs, stream);
    if (st == PF_OK) st = pfk_mark_rows(p->dense_rows, nd, p->row_apart, p->m, stream);
    if (st == PF_OK && timer) timer->start(stream);
    if (st == PF_OK && lng) {
        // deal: the tiles ordered by their first column, XCD k taking the k-th eighth
        st = pfk_memcpy_h2d(p->long_tiles, lt.data(), lt.size() * 4, stream);
        if (st == PF_OK) st = pfk_memcpy_h2d(p->long_row_tiles, row_tiles.data(), row_tiles.size() * 4, stream);
        // first nnz of each tile into the deal slots, their columns into the partial slots (both overwritten below)
        int *d_first = p->long_deal, *d_cols = static_cast<int *>(part);
        if (st == PF_OK) st = pfk_memcpy_h2d(d_first, first.data(), first.size() * 4, stream);
        if (st == PF_OK) st = pfk_gather_cols(d_col, p->nnz, d_first, (int)nlt, d_cols, stream);
        fc.resize((size_t)nlt);
        deal.resize((size_t)nlt);
        if (st == PF_OK) st = pfk_memcpy_d2h(fc.data(), d_cols, fc.size() * 4, stream);
        if (st == PF_OK) st = pfk_stream_sync(stream);
        if (st == PF_OK) {
            for (long long t = 0; t < nlt; ++t) deal[(size_t)t] = (int)t;
            std::stable_sort(deal.begin(), deal.end(), [&](int x, int y) { return fc[(size_t)x] < fc[(size_t)y]; });
            st = pfk_memcpy_h2d(p->long_deal, deal.data(), deal.size() * 4, stream);
        }
    }
    if (st == PF_OK) st = pfk_stream_sync(stream);
    if (st == PF_OK && timer) timer->stop(stream);
    if (st != PF_OK) return from_kernel_layer(st, "hybrid tables");
    // a second stream only where the runs run beside the dense rows (x within one XCD's L2; creating a
    // stream costs milliseconds); without it the kernels run in sequence on the caller's stream
    if (!p->aux_stream && xb <= kXcdL2Bytes) {
        if (pfk_stream_create(&p->aux_stream) != PF_OK) p->aux_stream = nullptr;
        if (p->aux_stream && (pfk_event_create_fence(&p->ev_fork) != PF_OK ||
                              pfk_event_create_fence(&p->ev_join) != PF_OK)) {
            pfk_event_destroy(p->ev_fork);
            pfk_stream_destroy(p->aux_stream);
            p->aux_stream = p->ev_fork = p->ev_join = nullptr;
        }
    }
    p->hybrid = true;
    p->info.hybrid = 1;
    p->info.dense_rows = nd;
    p->info.long_tiles = (int)nlt;
    return PF_OK;
}

// The band kernel for a row-aligned plan: measures (on a sample of the rows)
// how many columns lie within +-w of their row (w = 64 << i) and keeps the
// smallest w that holds 85% of the nnz and, with two steps' rows, fits the
// kernel's LDS ring.  On by
// default for matrices of under 4 nnz per row on average (each row's x entry
// is then a large part of the stream, and the band's gathers cost most).
int try_band(pf_plan *p, const int *d_row_ptr, const int *d_col, void *stream, PlanTimer *timer)
{
    const pf_plan_info &in = p->info;
    const long long m = p->m, n = p->n, nnz = p->nnz;
    if (in.variant != PF_FLAT || !in.row_aligned || !uses_row_map(in.variant, in.tile) ||
        (in.dtype != PF_F64 && in.dtype != PF_F32) || n * value_bytes(in.dtype) <= kXcdL2Bytes ||
        nnz < 64LL * PFK_BAND_STEP || m < 1)
        return PF_OK;
    unsigned long long *d = nullptr;
    unsigned long long h[PFK_BAND_WIDTHS + 1];
    PF_TRY(pfk_malloc(reinterpret_cast<void **>(&d), sizeof h), "band statistic");
    if (timer) timer->start(stream);
    int st = pfk_band_stats(d_row_ptr, d_col, p->m, d, stream);
    if (st == PF_OK) st = pfk_memcpy_d2h(h, d, sizeof h, stream);
    if (st == PF_OK) st = pfk_stream_sync(stream);
    if (st == PF_OK && timer) timer->stop(stream);
    pfk_free(d);
    if (st != PF_OK) return from_kernel_layer(st, "band statistic");
    const long long rows_per_step = (PFK_BAND_STEP * m + nnz - 1) / nnz;
    for (int i = 0; i < PFK_BAND_WIDTHS; ++i) {
        const long long w = 64LL << i;
        if (2 * w + 2 * rows_per_step > PFK_BAND_RING) break;
        if ((double)h[i] >= 0.85 * (double)h[PFK_BAND_WIDTHS]) {  // of the sampled nnz
            p->band_avail = (int)w;
            break;
        }
    }
    p->info.band_w = (p->band_avail > 0 && nnz < 4 * m) ? p->band_avail : 0;
    return PF_OK;
}

// The plan for a validated matrix with known statistics (shared by plan
// creation and the tuner's candidates): workspace allocated and initialised.
// With columns given, PF_AUTO and PF_FLAT plans of the default tile also try
// the hybrid path.
int plan_build(const pf_row_stats &s, const int *d_row_ptr, int m, int n, int nnz, int dtype, int variant, int tile,
               void *stream, pf_plan **plan, const int *d_col = nullptr, const PlanScan *scan = nullptr,
               PlanTimer *timer = nullptr)
{
    bool allow_hybrid = true;
    pf_plan_info info;
    const int st = plan_info(s, n, dtype, variant, tile, &info, &allow_hybrid);
    const bool want_hybrid = (variant == PF_AUTO || variant == PF_FLAT) && tile <= 0 && allow_hybrid;
    if (st != PF_OK) return st;
    pf_plan *p = new pf_plan();
    p->m = m;
    p->n = n;
    p->nnz = nnz;
    p->info = info;
    p->stats = s;
    // A hybrid candidate starts with no workspace: a hybrid plan keeps its error flag with its own tables and
    // runs without the split-row arrays (C5: 7 MB, 0.3 ms to allocate), which come later if
    // pf_plan_set_hybrid(plan, 0) asks.
    const bool candidate = want_hybrid && hybrid_candidate(s, n, dtype, info, d_col);
    int rc = PF_OK;
    if (candidate) {
        p->split_ready = false;
    } else {
        void *w = nullptr;
        rc = pfk_malloc(&w, info.workspace_bytes);
        if (rc != PF_OK) {
            delete p;
            return from_kernel_layer(rc, "plan workspace");
        }
        plan_carve(p, w);
        if (timer) timer->start(stream);
        rc = plan_init(p, d_row_ptr, stream);
        if (rc == PF_OK) rc = pfk_stream_sync(stream);
        if (rc == PF_OK && timer) timer->stop(stream);
    }
    if (rc == PF_OK && d_col && !candidate) rc = try_band(p, d_row_ptr, d_col, stream, timer);
    if (rc == PF_OK && candidate) {
        rc = try_hybrid(p, d_row_ptr, d_col, stream, scan, timer);
        if (rc == PF_OK && !p->hybrid) {  // stays split-row: its workspace now
            void *full = nullptr;
            rc = pfk_malloc(&full, info.workspace_bytes);
            if (rc == PF_OK) {
                plan_carve(p, full);
                rc = plan_init(p, d_row_ptr, stream);
                if (rc == PF_OK) rc = pfk_stream_sync(stream);
            }
            if (rc != PF_OK) rc = from_kernel_layer(rc, "plan workspace");
        }
        if (rc != PF_OK) {
            pfk_free(p->ws_hyb);
            pfk_free(p->ws);
            delete p;
            return rc;
        }
    }
    if (rc != PF_OK) {
        pfk_free(p->ws);
        delete p;
        return from_kernel_layer(rc, "plan workspace init");
    }
    *plan = p;
    return PF_OK;
}

// Argument checks shared by plan creation and the no-allocation entry point.
int check_matrix_args(const int *d_row_ptr, const int *d_col, int m, int n, int nnz, int dtype, int variant)
{
    if (m < 0 || n < 0 || nnz < 0 || value_bytes(dtype) == 0 || variant < PF_AUTO || variant > PF_FLAT)
        return fail(PF_ERR_INVALID, "bad size, dtype or variant");
    if (m > 0 && !d_row_ptr) return fail(PF_ERR_INVALID, "row_ptr is NULL");
    if ((unsigned long long)nnz + (unsigned long long)m >= 0xFFFFFFFFull)
        return fail(PF_ERR_UNSUPPORTED, "nnz + m must stay below 2^32");
    // x and y are addressed through buffer resources with 32-bit byte offsets.
    if ((unsigned long long)n * (unsigned long long)value_bytes(dtype) >= 0xFFFFFFF0ull ||
        (unsigned long long)m * (unsigned long long)value_bytes(dtype) >= 0xFFFFFFF0ull)
        return fail(PF_ERR_UNSUPPORTED, "x and y must each stay below 4 GiB");
    if (d_col && !aligned16(d_col)) return fail(PF_ERR_ALIGN, "col not 16-byte aligned");
    if (nnz > 0 && m == 0) return fail(PF_ERR_CSR, "nnz > 0 with no rows");
    return PF_OK;
}

// Row statistics of a device CSR through a caller-supplied block of PFK_STATS_WORDS
// unsigned long long (synchronises `stream`).
void decode_stats(const unsigned long long *h, const int *d_col, int m, long long nnz, pf_row_stats *out);

int stats_via(unsigned long long *d, const int *d_row_ptr, const int *d_col, int m, int n, long long nnz,
              pf_row_stats *out, void *stream)
{
    unsigned long long h[PFK_STATS_WORDS];
    int st = pfk_row_stats(d_row_ptr, d_col, m, n, nnz, d, stream);
    if (st == PF_OK) st = pfk_memcpy_d2h(h, d, sizeof h, stream);
    if (st == PF_OK) st = pfk_stream_sync(stream);
    if (st != PF_OK) return from_kernel_layer(st, "row statistics");
    decode_stats(h, d_col, m, nnz, out);
    return PF_OK;
}

// pf_row_stats from the statistics block (the layout of prefree_kernels.hip).
void decode_stats(const unsigned long long *h, const int *d_col, int m, long long nnz, pf_row_stats *out)
{
    std::memset(out, 0, sizeof *out);
    out->m = m;
    out->nnz = nnz;
    out->max_row_len = (long long)h[0];
    out->min_row_len = m > 0 ? (long long)h[1] : 0;
    out->n_empty_rows = (long long)h[2];
    out->n_decreasing = (long long)h[3];
    out->row_ptr_first = (long long)h[4];
    out->row_ptr_last = (long long)h[5];
    out->n_bad_cols = (d_col && nnz > 0) ? (long long)h[6] : (nnz > 0 ? -1 : 0);
    for (int k = 0; k < 33; ++k) out->hist_log2[k] = (long long)h[7 + k];
    out->n_long_rows = (long long)h[40];
    out->max_short_row_len = (long long)h[41];
    out->guess_dev = (long long)h[42];
    out->line_q1_row_ptr = (long long)h[43];
    out->line_q3_row_ptr = (long long)h[44];
    out->line_far_rows = (long long)h[45];
}

int check_csr_stats(const pf_row_stats &s, int nnz)
{
    if (s.row_ptr_first != 0 || s.row_ptr_last != nnz || s.n_decreasing != 0 || s.n_bad_cols > 0)
        return fail(PF_ERR_CSR, "row_ptr[0]=" + std::to_string(s.row_ptr_first) + " row_ptr[m]=" +
                                    std::to_string(s.row_ptr_last) + " decreasing=" +
                                    std::to_string(s.n_decreasing) + " bad_cols=" + std::to_string(s.n_bad_cols));
    return PF_OK;
}

// Long rows the planning scan lists; a matrix with more of them scans again
// when it tries the hybrid path.
constexpr int kScanListCap = 8192;
constexpr int kScanHostList = 1024;  // list entries copied back with the statistics (one copy, one wait)

// Bytes of pf_spmv_noalloc's scratch taken by the row statistics block; the
// workspace starts after it, 256-byte aligned.
constexpr size_t kNoallocStatsBytes = 512;

// pf_spmv_noalloc's calls on one device share its one scratch array: a lock
// per device (the kernel layer keeps scratch for devices 0..63) serialises
// calls from several host threads.
constexpr int kNoallocDevices = 64;
std::mutex g_noalloc_mu[kNoallocDevices];

}  // namespace

extern "C" {

int pf_version(void) { return 100; }  // 0.1.0

const char *pf_status_string(int status)
{
    switch (status) {
    case PF_OK: return "success";
    case PF_ERR_INVALID: return "invalid argument";
    case PF_ERR_ALIGN: return "col/val pointer not 16-byte aligned";
    case PF_ERR_HIP: return "HIP runtime error";
    case PF_ERR_NOMEM: return "out of memory";
    case PF_ERR_UNSUPPORTED: return "unsupported variant/tile/dtype";
    case PF_ERR_CSR: return "malformed CSR matrix";
    case PF_ERR_KERNEL: return "kernel found an inconsistent tile";
    case PF_ERR_IO: return "file could not be read or parsed";
    }
    return "unknown status";
}

const char *pf_last_error(void) { return g_err.c_str(); }

int pf_row_stats_compute(const int *d_row_ptr, const int *d_col, int m, int n, long long nnz,
                         pf_row_stats *out, void *stream)
{
    if (!out || !d_row_ptr || m < 0 || n < 0 || nnz < 0)
        return fail(PF_ERR_INVALID, "pf_row_stats_compute: bad argument");
    unsigned long long *d = nullptr;
    PF_TRY(pfk_malloc(reinterpret_cast<void **>(&d), PFK_STATS_WORDS * sizeof(unsigned long long)), "stats buffer");
    const int st = stats_via(d, d_row_ptr, d_col, m, n, nnz, out, stream);
    pfk_free(d);
    return st;
}

int pf_select(const pf_row_stats *stats, int dtype, int variant, pf_plan_info *out)
{
    if (!stats || !out || value_bytes(dtype) == 0)
        return fail(PF_ERR_INVALID, "pf_select: bad argument");
    Choice c;
    if (variant == PF_AUTO) {
        c = auto_choice(*stats, dtype);
    } else {
        c.variant = variant;
        c.tile = default_tile(variant, dtype);
    }
    const int st = finish_info(*stats, dtype, c.variant, c.tile, out);
    if (st == PF_OK) apply_overrides(c, *out);
    return st;
}

// Once per device and process, before the first plan: create and destroy one non-blocking stream.  Measured
// on MI355X (ROCm 7.2): until a process has created a stream beside the null stream, C3's long-row kernel
// (k_long) takes 79 us per call instead of 66, with the same plan, buffers and L2 hit rate (C3 204.6 against
// 191.8 us per step; the other kernels within 1%).  The stream is not used; the cause lies in the HIP
// runtime's queue set-up and was not identified further (a synthetic kernel of the same shape shows nothing).
static void warm_queues()
{
    static std::mutex mu;
    static std::set<int> done;
    int dev = 0;
    if (pfk_get_device(&dev) != PF_OK) return;
    std::lock_guard<std::mutex> lock(mu);
    if (!done.insert(dev).second) return;
    void *s = nullptr;
    if (pfk_stream_create(&s) == PF_OK) pfk_stream_destroy(s);
}

int pf_plan_create_tuned(pf_plan **plan, const int *d_row_ptr, const int *d_col, int m, int n, int nnz,
                         int dtype, int variant, int tile, void *stream)
{
    if (!plan) return fail(PF_ERR_INVALID, "plan is NULL");
    *plan = nullptr;
    int st = check_matrix_args(d_row_ptr, d_col, m, n, nnz, dtype, variant);
    if (st != PF_OK) return st;
    warm_queues();  // one-time, outside the plan's own timing
    const auto t0 = std::chrono::steady_clock::now();
    pf_row_stats s;
    std::memset(&s, 0, sizeof s);
    s.m = m;
    s.nnz = nnz;
    PlanTimer timer;
    PlanScan scan;
    void *buf = nullptr;
    if (m > 0 && d_col) {
        // the planning scan: statistics, column check and the long rows (with the descents inside them) in one
        // pass over row_ptr and one over col
        const size_t stats_b = (PFK_STATS_WORDS * sizeof(unsigned long long) + 255) & ~(size_t)255;
        PF_TRY(pfk_malloc(&buf, stats_b + (size_t)kScanListCap * 16), "planning scan buffer");
        unsigned long long h[PFK_STATS_WORDS];
        auto *d = static_cast<unsigned long long *>(buf);
        int *list = reinterpret_cast<int *>(static_cast<char *>(buf) + stats_b);
        std::vector<unsigned long long> hb((stats_b + (size_t)kScanHostList * 16) / 8);
        timer.start(stream);
        st = pfk_plan_scan(d_row_ptr, d_col, m, n, nnz, d, list, kScanListCap, stream);
        if (st == PF_OK) st = pfk_memcpy_d2h(hb.data(), d, hb.size() * 8, stream);
        if (st == PF_OK) st = pfk_stream_sync(stream);
        if (st == PF_OK) timer.stop(stream);
        if (st != PF_OK) {
            pfk_free(buf);
            return from_kernel_layer(st, "planning scan");
        }
        std::memcpy(h, hb.data(), sizeof h);
        decode_stats(h, d_col, m, nnz, &s);
        scan.list = list;
        scan.cap = kScanListCap;
        scan.listed = (long long)h[46];
        scan.desc = (long long)h[47];
        scan.checked = h[48] == 0;
        scan.host_n = std::min<long long>(scan.listed, kScanHostList);
        const int *hl = reinterpret_cast<const int *>(reinterpret_cast<const char *>(hb.data()) + stats_b);
        scan.host.assign(hl, hl + 4 * scan.host_n);
    } else if (m > 0) {
        st = pf_row_stats_compute(d_row_ptr, d_col, m, n, nnz, &s, stream);
        if (st != PF_OK) return st;
    }
    if (m > 0) {
        st = check_csr_stats(s, nnz);
        if (st != PF_OK) {
            pfk_free(buf);
            return st;
        }
    }
    st = plan_build(s, d_row_ptr, m, n, nnz, dtype, variant, tile, stream, plan, d_col, &scan, &timer);
    pfk_free(buf);
    if (st == PF_OK) {
        (*plan)->plan_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        (*plan)->plan_gpu_ms = timer.ok ? timer.gpu_ms : -1.0;
    }
    return st;
}

int pf_plan_set_band(pf_plan *plan, int band)
{
    if (!plan || (band != 0 && band != 1)) return fail(PF_ERR_INVALID, "band must be 0 or 1");
    if (band && (plan->band_avail <= 0 || !plan->info.row_aligned))
        return fail(PF_ERR_UNSUPPORTED, "this plan has no band (row-aligned FLAT, fp64 / fp32, x over 4 MB, "
                                        "85% of the columns within a band that fits the LDS ring)");
    plan->info.band_w = band ? plan->band_avail : 0;
    return PF_OK;
}

int pf_plan_get_timing(const pf_plan *plan, double *plan_ms, double *plan_gpu_ms)
{
    if (!plan || !plan_ms || !plan_gpu_ms) return fail(PF_ERR_INVALID, "NULL plan or output");
    *plan_ms = plan->plan_ms;
    *plan_gpu_ms = plan->plan_gpu_ms;
    return PF_OK;
}

int pf_plan_create(pf_plan **plan, const int *d_row_ptr, const int *d_col, int m, int n, int nnz, int dtype,
                   int variant, void *stream)
{
    return pf_plan_create_tuned(plan, d_row_ptr, d_col, m, n, nnz, dtype, variant, 0, stream);
}

int pf_plan_get_info(const pf_plan *plan, pf_plan_info *out)
{
    if (!plan || !out) return fail(PF_ERR_INVALID, "NULL plan or output");
    *out = plan->info;
    return PF_OK;
}

int pf_plan_set_run_tiles(pf_plan *plan, int run_tiles)
{
    if (!plan || run_tiles < 1 || run_tiles > 256) return fail(PF_ERR_INVALID, "run_tiles must be in 1..256");
    plan->info.run_tiles = run_tiles;
    if (plan->info.variant == PF_FLAT && plan->info.tile == kFlowTile)
        plan->info.needs_fixup = plan->info.ntiles > run_tiles;
    set_grid(plan->info);
    return PF_OK;
}

int pf_plan_set_keep_cached(pf_plan *plan, int keep_cached)
{
    if (!plan || (keep_cached != 0 && keep_cached != 1)) return fail(PF_ERR_INVALID, "keep_cached must be 0 or 1");
    plan->info.keep_cached = keep_cached;
    return PF_OK;
}

int pf_plan_set_row_aligned(pf_plan *plan, int row_aligned)
{
    if (!plan || (row_aligned != 0 && row_aligned != 1)) return fail(PF_ERR_INVALID, "row_aligned must be 0 or 1");
    if (!uses_row_map(plan->info.variant, plan->info.tile))
        return fail(PF_ERR_UNSUPPORTED, "row-aligned tiles are FLAT 1024 or 2048");
    if (row_aligned && plan->stats.max_row_len > PFK_ALIGN_ROW_MAX)
        return fail(PF_ERR_INVALID, "a row holds more than " + std::to_string(PFK_ALIGN_ROW_MAX) + " nnz");
    plan->info.row_aligned = row_aligned;
    plan->info.needs_fixup = row_aligned ? 0 : (plan->info.ntiles > 1);
    if (row_aligned) plan->info.x_windows = 0;
    else plan->info.band_w = 0;  // the band kernel runs row-aligned steps only
    return PF_OK;
}

int pf_plan_set_x_windows(pf_plan *plan, int x_windows)
{
    if (!plan || (x_windows != 0 && x_windows != 1)) return fail(PF_ERR_INVALID, "x_windows must be 0 or 1");
    if (!uses_row_map(plan->info.variant, plan->info.tile) || (x_windows && plan->info.row_aligned))
        return fail(PF_ERR_UNSUPPORTED, "x-window schedules are for split-row FLAT 1024 or 2048 plans");
    if (x_windows && !plan->info.x_windows) plan->map_ready = false;  // the next call records the schedule
    plan->info.x_windows = x_windows;
    return PF_OK;
}

int pf_plan_set_chunk_nnz(pf_plan *plan, long long chunk_nnz)
{
    if (!plan || chunk_nnz < 0) return fail(PF_ERR_INVALID, "chunk_nnz must be 0 or positive");
    if (!uses_row_map(plan->info.variant, plan->info.tile))
        return fail(PF_ERR_UNSUPPORTED, "XCD chunks are for FLAT 1024 or 2048 plans");
    plan->info.chunk_nnz = chunk_nnz;
    set_grid(plan->info);
    return PF_OK;
}

int pf_plan_set_hybrid(pf_plan *plan, int hybrid)
{
    if (!plan || (hybrid != 0 && hybrid != 1)) return fail(PF_ERR_INVALID, "hybrid must be 0 or 1");
    if (hybrid && !plan->ws_hyb)
        return fail(PF_ERR_UNSUPPORTED, "this plan has no hybrid tables (its rows over 256 nnz are not summed apart)");
    if (!hybrid) {
        const int st = plan_add_split(plan);
        if (st != PF_OK) return st;
    }
    plan->hybrid = hybrid != 0;
    plan->info.hybrid = hybrid;
    plan->info.x_halves = hybrid ? (plan->x_halves ? 1 : 0) : plan->info.x_halves;
    plan->info.long_tiles = hybrid && plan->long_mode ? plan->n_long_tiles : 0;
    return PF_OK;
}

int pf_plan_set_x_halves(pf_plan *plan, int x_halves)
{
    if (!plan || (x_halves != 0 && x_halves != 1)) return fail(PF_ERR_INVALID, "x_halves must be 0 or 1");
    if (!plan->ws_hyb) return fail(PF_ERR_UNSUPPORTED, "x halves are for the runs of hybrid plans");
    if (x_halves && plan->info.dtype == PF_F16)
        return fail(PF_ERR_UNSUPPORTED, "fp16 rounds each row once: no x halves");
    plan->x_halves = x_halves != 0;
    plan->info.x_halves = x_halves;
    return PF_OK;
}

int pf_plan_set_ladder(pf_plan *plan, int ladder)
{
    if (!plan || ladder < 1 || ladder > 5) return fail(PF_ERR_INVALID, "ladder must be 1..5");
    if (plan->info.variant != PF_PREFREE) return fail(PF_ERR_UNSUPPORTED, "reduction ladders are for PREFREE plans");
    plan->info.ladder = ladder;
    return PF_OK;
}

int pf_plan_set_remember_rows(pf_plan *plan, int remember)
{
    if (!plan || (remember != 0 && remember != 1)) return fail(PF_ERR_INVALID, "remember must be 0 or 1");
    if (remember && !plan->remember_rows) {  // the next call records the map afresh
        plan->map_ready = false;
        plan->hyb_map_ready = false;
    }
    plan->remember_rows = remember != 0;
    return PF_OK;
}

int pf_plan_get_stats(const pf_plan *plan, pf_row_stats *out)
{
    if (!plan || !out) return fail(PF_ERR_INVALID, "NULL plan or output");
    *out = plan->stats;
    return PF_OK;
}

int pf_plan_execute(pf_plan *plan, const int *d_row_ptr, const int *d_col, const void *d_val, const void *d_x,
                    void *d_y, void *stream)
{
    if (!plan) return fail(PF_ERR_INVALID, "NULL plan");
    if (plan->m == 0) return PF_OK;
    if (!d_row_ptr || !d_y || (plan->nnz > 0 && (!d_col || !d_val || !d_x)))
        return fail(PF_ERR_INVALID, "NULL matrix or vector pointer");
    if (!aligned16(d_col) || !aligned16(d_val)) return fail(PF_ERR_ALIGN, "col/val not 16-byte aligned");
    pfk_spmv_args a{};
    a.row_ptr = d_row_ptr;
    a.col = d_col;
    a.val = d_val;
    a.x = d_x;
    a.y = d_y;
    a.m = plan->m;
    a.n = plan->n;
    a.nnz = plan->nnz;
    a.tile = plan->info.tile;
    a.guess_spread = plan->info.guess_spread;
    a.guess_a = plan->info.guess_a;
    a.guess_b = plan->info.guess_b;
    a.run_tiles = plan->info.run_tiles;
    a.keep_cached = plan->info.keep_cached;
    a.ntiles = plan->info.ntiles;
    a.head_slot = plan->head;
    a.tail_slot = plan->tail;
    a.owner_row = plan->owner;
    a.err_flag = plan->err;
    a.row_map = plan->remember_rows ? plan->row_map : nullptr;
    a.map_ready = (plan->remember_rows && plan->map_ready) ? 1 : 0;
    a.row_aligned = plan->info.row_aligned;
    a.sched = (plan->remember_rows && plan->info.x_windows && plan->sched) ? plan->sched : nullptr;
    a.sched_cap = plan->sched_cap;
    a.chunk_nnz = plan->info.chunk_nnz;
    a.ladder = plan->info.ladder;
    a.head_bytes = plan->head_bytes;
    a.tail_bytes = plan->tail_bytes;
    a.owner_bytes = plan->owner_bytes;
    a.row_map_bytes = plan->row_map_bytes;
    a.sched_bytes = plan->sched_bytes;
    // no row of a row-aligned tile is longer than this (longer rows take other plans), so the tile kernel can
    // load a tile's overflow with its nominal range
    a.ovf_cap = plan->info.row_aligned ? (int)std::min<long long>(PFK_ALIGN_ROW_MAX, plan->stats.max_row_len) : 0;
    a.band_w = a.row_map ? plan->info.band_w : 0;  // used once the row map is recorded; never without one
    const int dt = plan->info.dtype;
    if (plan->hybrid) {
        a.ntiles = plan->run_tiles;
        a.tile = plan->run_tile;
        a.row_aligned = 1;
        a.chunk_nnz = plan->run_chunk;
        a.row_map = nullptr;
        a.sched = nullptr;
        a.dense_rows = plan->dense_rows;
        a.n_dense = plan->n_dense;
        a.n_win = plan->n_win;
        a.n_runs = plan->n_runs;
        a.runs = plan->runs;
        a.runs_bytes = plan->runs_bytes;
        a.run_map = plan->remember_rows ? plan->run_map : nullptr;
        a.run_map_bytes = plan->run_map_bytes;
        a.dense_seg = plan->remember_rows ? plan->dense_seg : nullptr;
        a.dense_seg_bytes = plan->dense_seg_bytes;
        a.dense_part = plan->dense_part;
        a.dense_part_bytes = plan->dense_part_bytes;
        a.x_halves = plan->x_halves ? 1 : 0;
        a.half_part = plan->half_part;
        a.half_part_bytes = plan->half_part_bytes;
        a.row_apart = plan->row_apart;
        a.row_apart_bytes = plan->row_apart_bytes;
        a.long_mode = plan->long_mode ? 1 : 0;
        a.n_long_tiles = plan->n_long_tiles;
        a.long_tiles = plan->long_tiles;
        a.long_deal = plan->long_deal;
        a.long_row_tiles = plan->long_row_tiles;
        a.long_part = plan->long_part;
        a.long_tiles_bytes = plan->long_tiles_bytes;
        a.long_deal_bytes = plan->long_deal_bytes;
        a.long_row_tiles_bytes = plan->long_row_tiles_bytes;
        a.long_part_bytes = plan->long_part_bytes;
        // the runs beside the dense rows' kernel when x fits one XCD's L2 (C5 fp32: 561 -> 541 us per call);
        // over it, the two compete for the L2s and both slow down (C5 fp64: 839 -> 925 us), so one stream
        if (plan->aux_stream && (long long)plan->n * value_bytes(dt) <= kXcdL2Bytes) {
            a.aux_stream = plan->aux_stream;
            a.ev_fork = plan->ev_fork;
            a.ev_join = plan->ev_join;
        }
        a.map_ready = (plan->remember_rows && plan->hyb_map_ready) ? 1 : 0;
        a.ovf_cap = (int)std::min<long long>(PFK_ALIGN_ROW_MAX, plan->stats.max_short_row_len);  // the runs' rows
        PF_TRY(pfk_spmv_hybrid(dt, &a, stream), "hybrid kernels");
        if (plan->remember_rows) plan->hyb_map_ready = true;  // later calls read what this one recorded
        return PF_OK;
    }
    if (!plan->split_ready) return fail(PF_ERR_KERNEL, "plan has no split-row workspace");
    if (a.sched && !plan->map_ready)  // the recording call starts from empty lists
        PF_TRY(pfk_fill_zero(a.sched, 16 * sizeof(int), stream), "schedule reset");
    switch (plan->info.variant) {
    case PF_ADAPTIVE:
        PF_TRY(pfk_spmv_adaptive(dt, &a, stream), "adaptive kernel");
        if (plan->info.needs_fixup) PF_TRY(pfk_spmv_fixup(dt, 1, &a, stream), "split-row combine");
        return PF_OK;
    case PF_FLAT:
        // The band kernel reads its steps from the row map and does not search: a band plan's first call, and
        // every call of a plan that remembers no rows, searches the map afresh first (one wave per tile).
        if (plan->info.band_w > 0 && plan->info.row_aligned && plan->row_map &&
            (!plan->remember_rows || !plan->map_ready)) {
            a.row_map = plan->row_map;
            a.band_w = plan->info.band_w;
            PF_TRY(pfk_row_map(&a, stream), "row map");
            a.map_ready = 1;
        }
        PF_TRY(pfk_spmv_flat(dt, &a, stream), "flat kernel");  // tile 256 launches its own combine
        if (a.row_map && plan->remember_rows) plan->map_ready = true;  // later calls read the recorded rows
        if (plan->info.needs_fixup && plan->info.tile != kFlowTile)
            PF_TRY(pfk_spmv_fixup(dt, 0, &a, stream), "split-row combine");
        return PF_OK;
    case PF_PREFREE:
        PF_TRY(pfk_spmv_prefree(dt, &a, stream), "prefree kernel");
        return PF_OK;
    }
    return fail(PF_ERR_INVALID, "plan has an unknown variant");
}

int pf_plan_check(pf_plan *plan, void *stream)
{
    if (!plan) return fail(PF_ERR_INVALID, "NULL plan");
    int flag = 0;
    PF_TRY(pfk_memcpy_d2h(&flag, plan->err, sizeof flag, stream), "read error flag");
    PF_TRY(pfk_stream_sync(stream), "synchronise");
    if (flag) {
        PF_TRY(pfk_fill_zero(plan->err, 256, stream), "clear error flag");
        return fail(PF_ERR_KERNEL, "a tile found row_ptr inconsistent with the planned matrix");
    }
    return PF_OK;
}

int pf_plan_destroy(pf_plan *plan)
{
    if (!plan) return PF_OK;
    if (plan->aux_stream) {
        pfk_stream_sync(plan->aux_stream);
        pfk_event_destroy(plan->ev_fork);
        pfk_event_destroy(plan->ev_join);
        pfk_stream_destroy(plan->aux_stream);
    }
    int st = pfk_free(plan->ws);
    if (plan->ws_split) {
        const int st2 = pfk_free(plan->ws_split);
        if (st == PF_OK) st = st2;
    }
    if (plan->ws_hyb) {
        const int st2 = pfk_free(plan->ws_hyb);
        if (st == PF_OK) st = st2;
    }
    delete plan;
    return st == PF_OK ? PF_OK : from_kernel_layer(st, "free workspace");
}

int pf_spmv(const int *d_row_ptr, const int *d_col, const void *d_val, const void *d_x, void *d_y, int m, int n,
            int nnz, int dtype, int variant, void *stream)
{
    pf_plan *p = nullptr;
    int st = pf_plan_create(&p, d_row_ptr, d_col, m, n, nnz, dtype, variant, stream);
    if (st != PF_OK) return st;
    st = pf_plan_execute(p, d_row_ptr, d_col, d_val, d_x, d_y, stream);
    if (st == PF_OK) st = pf_plan_check(p, stream);
    const int st2 = pf_plan_destroy(p);
    return st != PF_OK ? st : st2;
}

int pf_spmv_noalloc(const int *d_row_ptr, const int *d_col, const void *d_val, const void *d_x, void *d_y, int m,
                    int n, int nnz, int dtype, int variant, void *stream)
{
    int st = check_matrix_args(d_row_ptr, d_col, m, n, nnz, dtype, variant);
    if (st != PF_OK) return st;
    if (m == 0) return PF_OK;
    if (!d_y || (nnz > 0 && (!d_col || !d_val || !d_x))) return fail(PF_ERR_INVALID, "NULL matrix or vector pointer");
    const size_t room = (size_t)PFK_SCRATCH_BYTES - kNoallocStatsBytes;
    if (variant != PF_AUTO) {  // an explicit variant's workspace follows from (m, nnz): refuse before any launch
        pf_row_stats g;
        std::memset(&g, 0, sizeof g);
        g.m = m;
        g.nnz = nnz;
        pf_plan_info guess;
        st = finish_info(g, dtype, variant, default_tile(variant, dtype), &guess);
        if (st != PF_OK) return st;
        if (guess.workspace_bytes > room)
            return fail(PF_ERR_UNSUPPORTED, "pf_spmv_noalloc: the workspace needs " +
                                                std::to_string(guess.workspace_bytes) + " bytes, the scratch holds " +
                                                std::to_string(room) + "; use pf_spmv");
    }
    void *scr = nullptr;
    size_t scr_bytes = 0;
    PF_TRY(pfk_scratch(&scr, &scr_bytes), "scratch");
    if (scr_bytes < kNoallocStatsBytes + 256) return fail(PF_ERR_UNSUPPORTED, "scratch too small");
    int dev = 0;
    PF_TRY(pfk_get_device(&dev), "current device");
    if (dev < 0 || dev >= kNoallocDevices) return fail(PF_ERR_UNSUPPORTED, "device index beyond the scratch table");
    std::lock_guard<std::mutex> scratch_lock(g_noalloc_mu[dev]);  // held until the stream is synchronised below
    pf_plan p;  // on the stack: no allocation of any kind
    p.m = m;
    p.n = n;
    p.nnz = nnz;
    st = stats_via(static_cast<unsigned long long *>(scr), d_row_ptr, d_col, m, n, nnz, &p.stats, stream);
    if (st != PF_OK) return st;
    st = check_csr_stats(p.stats, nnz);
    if (st != PF_OK) return st;
    st = plan_info(p.stats, n, dtype, variant, 0, &p.info);
    if (st != PF_OK) return st;
    if (p.info.workspace_bytes > scr_bytes - kNoallocStatsBytes)
        return fail(PF_ERR_UNSUPPORTED, "pf_spmv_noalloc: the workspace needs " + std::to_string(p.info.workspace_bytes) +
                                            " bytes, the scratch holds " +
                                            std::to_string(scr_bytes - kNoallocStatsBytes) + "; use pf_spmv");
    plan_carve(&p, static_cast<char *>(scr) + kNoallocStatsBytes);
    st = plan_init(&p, d_row_ptr, stream);
    if (st != PF_OK) return from_kernel_layer(st, "scratch workspace init");
    st = pf_plan_execute(&p, d_row_ptr, d_col, d_val, d_x, d_y, stream);
    if (st == PF_OK) st = pf_plan_check(&p, stream);  // synchronises: the scratch is free again on return
    return st;
}

int pf_set_tuning_table(const char *path)
{
    std::vector<TableRow> rows;
    if (path) {
        std::string why;
        const int st = load_table(path, rows, why);
        if (st != PF_OK) return fail(st, why);
    }
    std::lock_guard<std::mutex> lock(g_table_mu);
    g_table.swap(rows);
    g_table_path = path ? path : "";
    g_table_env_done = true;  // an explicit table (or none) overrides the environment and the default
    return PF_OK;
}

const char *pf_tuning_table(void)
{
    thread_local std::string path;
    std::lock_guard<std::mutex> lock(g_table_mu);
    table_init_locked();
    path = g_table_path;
    return path.c_str();
}

// An eager call under kGraphTimeUs is bound by the host's launch rate, which hides the kernels' differences
// (C1: about 3.9 us per call for every candidate launched one by one; in a graph, 1.96 us for 16-lane row groups
// and 3.60 for 1024-nnz tiles).  pf_plan_autotune then times every candidate as a captured graph.
constexpr double kGraphTimeUs = 20.0;

// Mean us per call of `reps` back-to-back calls on `stream`, the best of two batches, each batch launched
// call by call.
static int time_plan(pf_plan *p, const int *rp, const int *col, const void *val, const void *x, void *y, int reps,
                     void *stream, double *us)
{
    void *e0 = nullptr, *e1 = nullptr;
    PF_TRY(pfk_event_create(&e0), "event");
    int st = pfk_event_create(&e1);
    double best = 1e300;
    for (int trial = 0; st == PF_OK && trial < 2; ++trial) {
        for (int w = 0; st == PF_OK && w < 2; ++w) st = pf_plan_execute(p, rp, col, val, x, y, stream);
        if (st == PF_OK) st = pfk_event_record(e0, stream);
        for (int r = 0; st == PF_OK && r < reps; ++r) st = pf_plan_execute(p, rp, col, val, x, y, stream);
        if (st == PF_OK) st = pfk_event_record(e1, stream);
        if (st == PF_OK) st = pfk_event_sync(e1);
        float ms = 0;
        if (st == PF_OK) st = pfk_event_elapsed_ms(&ms, e0, e1);
        if (st == PF_OK) best = std::min(best, 1e3 * ms / reps);
    }
    pfk_event_destroy(e0);
    if (e1) pfk_event_destroy(e1);
    if (st != PF_OK) return from_kernel_layer(st, "autotune timing");
    *us = best;
    return PF_OK;
}

// The same as one captured HIP graph of at least 20 calls, on a stream of its own (after `stream` has
// drained), launched once untimed and then twice timed; the best of the two.
static int time_plan_graph(pf_plan *p, const int *rp, const int *col, const void *val, const void *x, void *y,
                           int reps, void *stream, double *us)
{
    const int n = std::max(reps, 20);
    void *s = nullptr, *e0 = nullptr, *e1 = nullptr, *g = nullptr;
    int kst = pfk_stream_sync(stream);  // kernel-layer status
    int pst = PF_OK;                    // this library's status (pf_plan_execute)
    if (kst == PF_OK) kst = pfk_stream_create(&s);
    if (kst == PF_OK) kst = pfk_event_create(&e0);
    if (kst == PF_OK) kst = pfk_event_create(&e1);
    if (kst == PF_OK) pst = pf_plan_execute(p, rp, col, val, x, y, s);  // the plan's own first-call work, eager
    if (kst == PF_OK && pst == PF_OK) {
        kst = pfk_graph_begin(s);
        if (kst == PF_OK) {
            for (int r = 0; pst == PF_OK && r < n; ++r) pst = pf_plan_execute(p, rp, col, val, x, y, s);
            kst = pfk_graph_end(s, &g);  // ends the capture whatever happened inside it
        }
    }
    double best = 1e300;
    if (kst == PF_OK && pst == PF_OK) kst = pfk_graph_launch(g, s);
    for (int trial = 0; kst == PF_OK && pst == PF_OK && trial < 2; ++trial) {
        kst = pfk_event_record(e0, s);
        if (kst == PF_OK) kst = pfk_graph_launch(g, s);
        if (kst == PF_OK) kst = pfk_event_record(e1, s);
        if (kst == PF_OK) kst = pfk_event_sync(e1);
        float ms = 0;
        if (kst == PF_OK) kst = pfk_event_elapsed_ms(&ms, e0, e1);
        if (kst == PF_OK) best = std::min(best, 1e3 * ms / n);
    }
    if (s) pfk_stream_sync(s);
    pfk_graph_destroy(g);
    pfk_event_destroy(e0);
    pfk_event_destroy(e1);
    pfk_stream_destroy(s);
    if (pst != PF_OK) return pst;
    if (kst != PF_OK) return from_kernel_layer(kst, "autotune graph timing");
    *us = best;
    return PF_OK;
}

int pf_plan_autotune(pf_plan *plan, const int *d_row_ptr, const int *d_col, const void *d_val, const void *d_x,
                     void *d_y, int reps, int flags, void *stream, pf_tune_result *result)
{
    if (!plan || reps < 1 || reps > 100000) return fail(PF_ERR_INVALID, "pf_plan_autotune: bad plan or reps");
    if (plan->m == 0 || plan->nnz == 0) {
        if (result) {
            std::memset(result, 0, sizeof *result);
            result->variant = plan->info.variant;
            result->tile = plan->info.tile;
            result->run_tiles = plan->info.run_tiles;
        }
        return PF_OK;
    }
    const int dtype = plan->info.dtype;
    double base_us = 0;
    int st = time_plan(plan, d_row_ptr, d_col, d_val, d_x, d_y, reps, stream, &base_us);
    if (st != PF_OK) return st;
    const bool graph = base_us < kGraphTimeUs;  // launch-bound: every candidate as a captured graph
    if (graph) {
        st = time_plan_graph(plan, d_row_ptr, d_col, d_val, d_x, d_y, reps, stream, &base_us);
        if (st != PF_OK) return st;
    }
    pf_tune_result best;
    std::memset(&best, 0, sizeof best);
    best.variant = plan->info.variant;
    best.tile = plan->info.tile;
    best.run_tiles = plan->info.run_tiles;
    best.keep_cached = plan->info.keep_cached;
    best.chunk_nnz = plan->info.chunk_nnz;
    best.ladder = plan->info.variant == PF_PREFREE ? plan->info.ladder : 0;
    best.hybrid = plan->info.hybrid;
    best.us = base_us;
    best.default_us = base_us;
    best.candidates = 1;
    pf_plan *best_plan = nullptr;

    static const int kRuns[] = {1, 2, 3, 4, 6, 8, 12, 16};
    static const long long kChunks[] = {-1, 0, 1LL << 13, 1LL << 15, 1LL << 17};  // -1: the plan's own rule
    const int variants[] = {PF_ADAPTIVE, PF_FLAT, PF_PREFREE};
    for (int variant : variants) {
        if (variant == PF_PREFREE && !(flags & PF_TUNE_PREFREE)) continue;
        int tiles[PFK_MAX_TILES];
        const int nt = pfk_supported_tiles(variant, dtype, tiles, PFK_MAX_TILES);
        for (int ti = 0; ti < nt; ++ti) {
            // row groups give one row `tile` lanes: timed only where no row is longer than a row-aligned tile
            if (variant == PF_FLAT && PFK_ROW_GROUP_TILE(tiles[ti]) && plan->stats.max_row_len > PFK_ALIGN_ROW_MAX)
                continue;
            pf_plan *cand = nullptr;
            st = plan_build(plan->stats, d_row_ptr, plan->m, plan->n, plan->nnz, dtype, variant, tiles[ti], stream,
                            &cand);
            if (st != PF_OK) {
                if (best_plan) pf_plan_destroy(best_plan);
                return st;
            }
            bool keep_cand = false;
            const bool walks_runs = variant == PF_ADAPTIVE || (variant == PF_FLAT && tiles[ti] == kFlowTile);
            const int nruns = walks_runs ? (int)(sizeof kRuns / sizeof kRuns[0]) : 1;
            const int nkeep = variant == PF_ADAPTIVE && (flags & PF_TUNE_KEEP_CACHED) ? 2 : 1;
            const bool chunked = uses_row_map(variant, tiles[ti]);
            const int nchunk = chunked ? (int)(sizeof kChunks / sizeof kChunks[0]) : 1;
            const long long rule_chunk = cand->info.chunk_nnz;
            // PREFREE: the reference tuner's code axis, its five reduction ladders
            // (scripts/profile_and_generate.py:109-235)
            const int nladder = variant == PF_PREFREE ? 5 : 1;
            int cand_run = cand->info.run_tiles, cand_keep = cand->info.keep_cached, cand_ladder = cand->info.ladder;
            long long cand_chunk = rule_chunk;
            double cand_us = 1e300;
            for (int li = 0; li < nladder; ++li) {
                for (int ri = 0; ri < nruns; ++ri) {
                    for (int k = 0; k < nkeep; ++k) {
                        for (int ci = 0; ci < nchunk; ++ci) {
                            if (ci > 0 && kChunks[ci] == rule_chunk) continue;  // timed as the rule's own
                            if (walks_runs) {
                                cand->info.run_tiles = kRuns[ri];
                                if (variant == PF_ADAPTIVE) cand->info.keep_cached = k;
                                else cand->info.needs_fixup = cand->info.ntiles > kRuns[ri];
                            }
                            if (chunked) cand->info.chunk_nnz = ci == 0 ? rule_chunk : kChunks[ci];
                            if (variant == PF_PREFREE) cand->info.ladder = li + 1;
                            set_grid(cand->info);
                            double us = 0;
                            st = graph ? time_plan_graph(cand, d_row_ptr, d_col, d_val, d_x, d_y, reps, stream, &us)
                                       : time_plan(cand, d_row_ptr, d_col, d_val, d_x, d_y, reps, stream, &us);
                            if (st != PF_OK) {
                                pf_plan_destroy(cand);
                                if (best_plan) pf_plan_destroy(best_plan);
                                return st;
                            }
                            ++best.candidates;
                            if (us < cand_us) {
                                cand_us = us;
                                cand_run = cand->info.run_tiles;
                                cand_keep = cand->info.keep_cached;
                                cand_chunk = cand->info.chunk_nnz;
                                cand_ladder = cand->info.ladder;
                            }
                        }
                    }
                }
            }
            if (cand_us < best.us) {
                cand->info.run_tiles = cand_run;
                cand->info.keep_cached = cand_keep;
                cand->info.chunk_nnz = cand_chunk;
                cand->info.ladder = cand_ladder;
                if (cand->info.variant == PF_FLAT && cand->info.tile == kFlowTile)
                    cand->info.needs_fixup = cand->info.ntiles > cand_run;
                set_grid(cand->info);
                best.variant = cand->info.variant;
                best.tile = cand->info.tile;
                best.run_tiles = cand->info.run_tiles;
                best.keep_cached = cand->info.keep_cached;
                best.chunk_nnz = cand->info.chunk_nnz;
                best.ladder = cand->info.variant == PF_PREFREE ? cand->info.ladder : 0;
                best.hybrid = 0;
                best.us = cand_us;
                if (best_plan) pf_plan_destroy(best_plan);
                best_plan = cand;
                keep_cand = true;
            }
            if (!keep_cand) pf_plan_destroy(cand);
        }
    }
    if (best_plan) {  // move the winner into the caller's plan
        std::swap(*plan, *best_plan);  // the same matrix: every field is the winner's
        pf_plan_destroy(best_plan);
    }
    // y = A x with the chosen configuration, so that the caller's y is defined.
    st = pf_plan_execute(plan, d_row_ptr, d_col, d_val, d_x, d_y, stream);
    if (st == PF_OK) st = pfk_stream_sync(stream) == PF_OK ? PF_OK : from_kernel_layer(PF_ERR_HIP, "autotune sync");
    if (st == PF_OK && result) *result = best;
    return st;
}

int pf_device_malloc(void **ptr, size_t bytes) { return from_kernel_layer(pfk_malloc(ptr, bytes), "device malloc"); }
int pf_device_free(void *ptr) { return from_kernel_layer(pfk_free(ptr), "device free"); }
int pf_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream)
{
    return from_kernel_layer(pfk_memcpy_h2d(dst, src, bytes, stream), "copy to device");
}
int pf_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream)
{
    return from_kernel_layer(pfk_memcpy_d2h(dst, src, bytes, stream), "copy to host");
}
int pf_stream_synchronize(void *stream) { return from_kernel_layer(pfk_stream_sync(stream), "synchronise"); }

}  // extern "C"
