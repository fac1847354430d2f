// prefree_kernels.hip — gfx950 CSR SpMV kernels and the thin extern "C" HIP
// layer declared in include/prefree_kernels.h.
//
// The kernels compute y = A·x (y overwritten).  None needs a pre-pass: every
// workgroup (or wave) finds its rows inside the SpMV kernel, by a wave search
// of row_ptr (device_common.hpp: wave_search_lt) or, from a plan's second call
// on, by reading the rows its first call found.
//
//  * k_rows<T, K, MODE, PRIO, RUNS, HALVES>  (PF_FLAT, K = 1024 / 2048 nnz;
//    the default when no row holds more than 256 nnz)  Tile t owns the rows
//    starting in its nnz range, whole: one launch per step, no split rows.
//    Its search mode splits the row search (row_probe_issue / _finish) so the
//    first probe round goes out ahead of the tile's loads.  RUNS: the runs of
//    short rows of a hybrid plan; HALVES: once per half of x.
//  * k_dense<T, MODE> + k_dense_sum  (hybrid plans, dense mode)  Dense rows by
//    x windows staged in LDS, a partial per (row, window), added in order.
//  * k_long<T> + k_long_sum  (hybrid plans, long mode)  Long rows cut into
//    1024-nnz tiles dealt to the XCDs by first column, partials added in order.
//  * k_combine<T, LONG>  (hybrid plans with x halves)  y = first half's row
//    sums + second half's over the runs' rows, and the dense or long rows'
//    combine, in one launch.
//  * k_flat<T, K, MODE>  (PF_FLAT 1024 / 2048, rows longer than 256 nnz)  The
//    same nnz tiles with rows cut at tile edges; k_fixup combines the pieces.
//    With the x-window schedule (sched_tile) tiles go to the XCDs by the part
//    of x they start in.
//  * k_flow<T>  (PF_FLAT 256)  A wave walks a run of 256-nnz tiles and carries
//    a row's partial sum across their edges.
//  * k_tiles<T, false, 4096>  (PF_FLAT 4096)  The first FLAT kernel: both tile
//    edges searched on every call.
//  * k_wave<T, K, LMAX, ...>  (PF_ADAPTIVE)  CSR-adaptive row blocks found on
//    the fly: tile t owns the keys [t*K, (t+1)*K) of the merged sequence in
//    which row r occupies keys row_ptr[r]+r .. row_ptr[r+1]+r, so a tile holds
//    at most K rows+nnz; rows longer than LMAX are cut at tile edges.  Each
//    wave64 walks a run of tiles with three in flight.
//  * k_prefree<T, P>  (PF_PREFREE)  The reference algorithm
//    (src/spmv_kernel/preFreeSpMV.cu:407-483): 128*P-nnz tiles, reduction
//    ladder "code 3", atomicAdd on tile-boundary rows over a zeroed y, its
//    first-row-per-tile map (the pre-pass, :3-28) searched inside the kernel.
//  * k_fixup<T, MERGE>  Split-row partials combined in tile order
//    (deterministic, no atomics).
//  * k_row_stats, k_col_check  Row statistics and the column range check, run
//    once at planning; k_tile_desc / k_prefree_rows  descriptors for tests.
//
// Shared data path of the FLAT tiles (one workgroup = 4 wave64s = one tile):
//   1. col / val of the tile's nnz range stream in as 16-byte non-temporal
//      loads before its rows are known; tiles go to the XCDs in chunks of
//      neighbouring tiles (xcd_tile);
//   2. x is gathered with ordinary loads, so it stays in L2 / MALL; products
//      go to LDS;
//   3. rows of <= 16 products are summed by one lane each in nnz order (the
//      order of the reference spmv_serial, test/test_cdspmv.cpp:4-20), rows of
//      <= 512 by a wave (DPP sum), longer ones by the whole workgroup;
//   4. k_rows stages the sums in LDS and writes them as 16-byte stores of
//      consecutive rows; k_flat writes each row's sum, or its head / tail
//      partial, directly.
#include "../../include/prefree_c.h"
#include "../../include/prefree_kernels.h"
#include "device_common.hpp"

#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

using namespace pfdev;

namespace {

constexpr int kBS = 256;               // workgroup size for k_tiles: 4 waves
constexpr int kWaves = kBS / kWave;
constexpr int kThreadMax = 16;         // rows up to this length: one lane each
constexpr int kWaveMax = 512;          // rows up to this length: one wave each

// Workgroup barrier for LDS traffic only.  __syncthreads() also orders global
// memory, which on gfx950 means waiting for every outstanding vector memory
// operation (loads in flight for the next tile, y stores not yet acknowledged);
// the tile kernels exchange data between threads only through LDS.
__device__ __forceinline__ void lds_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// fp16 mode: values, x and y stored as IEEE binary16; products and row sums
// are formed in fp32 (a product of two halves is exact in fp32) and each row
// sum is rounded to half once, when y is stored.
typedef _Float16 half_t;
template <typename T> struct AccOf { using type = T; };
template <> struct AccOf<half_t> { using type = float; };
template <typename T> using acc_t = typename AccOf<T>::type;

template <typename T>
struct Args {
    const int *__restrict__ rp;
    const int *__restrict__ col;
    const T *__restrict__ val;
    const T *__restrict__ x;
    T *__restrict__ y;
    int m;
    int n;
    int nnz;
    int guess_spread;
    double guess_a, guess_b;  // row-aligned tiles' row searches: the line row = guess_a * key + guess_b (a > 0)
    long long ntiles;
    long long g8;        // tiles per XCD, padded to whole chunks (grid = 8 * g8)
    long long xch;       // tiles per chunk (see xcd_tile)
    long long tx;        // k_stream: tiles per XCD
    long long tpw;       // k_stream: tiles per workgroup
    acc_t<T> *__restrict__ head;  // split-row partial sums (fp32 in the fp16 mode)
    acc_t<T> *__restrict__ tail;
    int *__restrict__ owner;
    int *__restrict__ err;
    int *__restrict__ sched;      // split-row FLAT x-window schedule (see k_flat), or null
    long long sched_cap;          // tiles per XCD list
    T *__restrict__ y2;           // x-halves runs: the second half's row sums (k_combine adds them to y)
    int ovf_cap;                  // row-aligned tiles: longest row (at most kAlignRowMax); 0 = unknown
};

// Long-row threshold of ADAPTIVE for tile size K (keys per wave tile).  A
// tile's nnz span is at most K + LMAX - 1 plus 3 for 16-byte alignment; the
// sizes are chosen so that it fits one (fp64) or two (fp32) 4-nnz vectors per
// lane of a wave64.
// The short-row tiles (238, 494) keep LMAX = 16 and are meant for matrices
// whose rows all fit one lane's sum: the span then fits 1 or 2 vectors.
constexpr int adaptive_lmax(int K) { return (K == 238 || K == 494) ? 16 : (K <= 440 ? 64 : K / 2 - 4); }

// ADAPTIVE tile sizes compiled in, per value type: X(type, dtype code, keys per tile).
#define PF_ADAPTIVE_TILES(X) \
    X(double, PF_F64, 188) X(double, PF_F64, 238) X(double, PF_F64, 494) X(double, PF_F64, 512) \
    X(float, PF_F32, 440) X(float, PF_F32, 494) X(float, PF_F32, 1024) \
    X(half_t, PF_F16, 440) X(half_t, PF_F16, 494) X(half_t, PF_F16, 1024)

// Logical tile of this workgroup.  Workgroups go to the XCDs round robin
// (XCD x = blockIdx % 8).  The tiles are cut into chunks of xch contiguous
// tiles, and in round r XCD x takes chunk 8r + x, so neighbouring rows (and
// their x entries) share an L2 while the eight XCDs stream neighbouring
// addresses.  With xch = g8 (one round) XCD x takes tiles [x*g8, (x+1)*g8).
// The grid is under 2^32 workgroups, so the arithmetic is 32-bit (a 64-bit
// divide is a software routine of about 200 instructions).
__device__ __forceinline__ long long xcd_tile(long long xch)
{
    const uint32_t b = blockIdx.x;
    const uint32_t q = b / kXcds;
    const uint32_t c = (uint32_t)xch;
    const uint32_t r = q / c;
    return (long long)r * (kXcds * (long long)c) + (long long)(b % kXcds) * c + (q - r * c);
}

// x-halves tiling (row-aligned runs of hybrid plans): every tile is processed
// twice, by a workgroup on XCDs 0-3 that gathers only the columns in the first
// half of x and one on XCDs 4-7 for the second half, so each XCD's random x
// gathers fall in half of x.  The tiles are chunked over the four XCDs of a
// half as xcd_tile chunks them over eight.
__device__ __forceinline__ long long xcd_tile_half(long long xch)
{
    const uint32_t b = blockIdx.x;
    const uint32_t q = b / kXcds;
    const uint32_t c = (uint32_t)xch;
    const uint32_t r = q / c;
    return (long long)r * ((kXcds / 2) * (long long)c) + (long long)((b % kXcds) & (kXcds / 2 - 1)) * c + (q - r * c);
}

// ---- 16-byte streaming loads through buffer resources ----------------------
//
// Every col / val / row_ptr load is a raw buffer load against a resource that
// spans exactly the bytes the workgroup may read.  The hardware range-checks
// each dword (a 16-byte load straddling the end returns the dwords inside and
// zeros for the rest, without touching memory beyond it), so the loads need no
// per-lane bounds branch and a lane past the end costs no traffic.

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int kRsrcWord3 = 0x00020000;  // gfx9 raw buffer resource, 32-bit elements
constexpr int kAuxNt = 2;               // cache policy bit 1: non-temporal (streamed once)
constexpr int kAuxDev = 16;             // cache policy bit 4 (sc1): device scope, written through to memory

// Callers pass wave-uniform base and size.  readfirstlane states that to the
// compiler, which otherwise may keep the descriptor in VGPRs and wrap every
// load in a loop over distinct descriptor values.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, long long bytes)
{
    const long long b = bytes < 0 ? 0 : (bytes > 0x40000000ll ? 0x40000000ll : bytes);
    const unsigned long long p = reinterpret_cast<unsigned long long>(base);
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)p);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(p >> 32));
    const int nb = __builtin_amdgcn_readfirstlane((int)b);
    void *u = reinterpret_cast<void *>(((unsigned long long)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(u, 0, nb, kRsrcWord3);
}

// Bytes of a val resource over `count` values starting at an even index.  The
// range check of a multi-dword load drops every dword that ends past the
// resource, so an fp16 range is rounded up to whole dwords: with val 16-byte
// aligned the extra two bytes share the last value's dword (never another
// page), and the lane slot they fill is never gathered or summed.
template <typename T>
__device__ __forceinline__ long long val_range_bytes(int count)
{
    return (((long long)count * (long long)sizeof(T)) + 3) & ~3ll;
}

// Scalar loads through a resource (x gathers, overflow values); an offset
// outside the resource reads zero.
constexpr uint32_t kOob = 0xFFFFFFF0u;  // byte offset beyond every resource

__device__ __forceinline__ double buf_load(__amdgpu_buffer_rsrc_t r, uint32_t off, double *)
{
    return __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
}

__device__ __forceinline__ float buf_load(__amdgpu_buffer_rsrc_t r, uint32_t off, float *)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}

__device__ __forceinline__ half_t buf_load(__amdgpu_buffer_rsrc_t r, uint32_t off, half_t *)
{
    return __builtin_bit_cast(half_t, __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0));
}


// A resource over a whole array addressed with 32-bit byte offsets (the plan
// guarantees it stays below 4 GiB).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc_full(const void *base, long long bytes)
{
    const long long b = bytes < 0 ? 0 : (bytes > (long long)kOob ? (long long)kOob : bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)(unsigned int)b, kRsrcWord3);
}

// col and val of the 4 consecutive nnz at 16-byte vector `vec` of a resource pair.
template <int AUX = kAuxNt>
__device__ __forceinline__ void load4(__amdgpu_buffer_rsrc_t rc, __amdgpu_buffer_rsrc_t rv, int vec, int (&c)[4],
                                      double (&v)[4])
{
    const u32x4 cc = __builtin_amdgcn_raw_buffer_load_b128(rc, vec * 16, 0, AUX);
    const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(rv, vec * 32, 0, AUX);
    const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(rv, vec * 32 + 16, 0, AUX);
    c[0] = (int)cc.x; c[1] = (int)cc.y; c[2] = (int)cc.z; c[3] = (int)cc.w;
    v[0] = __hiloint2double((int)v0.y, (int)v0.x);
    v[1] = __hiloint2double((int)v0.w, (int)v0.z);
    v[2] = __hiloint2double((int)v1.y, (int)v1.x);
    v[3] = __hiloint2double((int)v1.w, (int)v1.z);
}

template <int AUX = kAuxNt>
__device__ __forceinline__ void load4(__amdgpu_buffer_rsrc_t rc, __amdgpu_buffer_rsrc_t rv, int vec, int (&c)[4],
                                      float (&v)[4])
{
    const u32x4 cc = __builtin_amdgcn_raw_buffer_load_b128(rc, vec * 16, 0, AUX);
    const u32x4 vv = __builtin_amdgcn_raw_buffer_load_b128(rv, vec * 16, 0, AUX);
    c[0] = (int)cc.x; c[1] = (int)cc.y; c[2] = (int)cc.z; c[3] = (int)cc.w;
    v[0] = __int_as_float((int)vv.x); v[1] = __int_as_float((int)vv.y);
    v[2] = __int_as_float((int)vv.z); v[3] = __int_as_float((int)vv.w);
}

template <int AUX = kAuxNt>
__device__ __forceinline__ void load4(__amdgpu_buffer_rsrc_t rc, __amdgpu_buffer_rsrc_t rv, int vec, int (&c)[4],
                                      half_t (&v)[4])
{
    typedef unsigned int u32x2v __attribute__((ext_vector_type(2)));
    const u32x4 cc = __builtin_amdgcn_raw_buffer_load_b128(rc, vec * 16, 0, AUX);
    const u32x2v vv = __builtin_amdgcn_raw_buffer_load_b64(rv, vec * 8, 0, AUX);
    c[0] = (int)cc.x; c[1] = (int)cc.y; c[2] = (int)cc.z; c[3] = (int)cc.w;
    v[0] = __builtin_bit_cast(half_t, (unsigned short)(vv.x & 0xFFFFu));
    v[1] = __builtin_bit_cast(half_t, (unsigned short)(vv.x >> 16));
    v[2] = __builtin_bit_cast(half_t, (unsigned short)(vv.y & 0xFFFFu));
    v[3] = __builtin_bit_cast(half_t, (unsigned short)(vv.y >> 16));
}

// col and val of one nnz (element offset e of a resource pair): the wave-strided
// layout, in which a wave's load covers 64 consecutive nnz.
template <int AUX = kAuxNt>
__device__ __forceinline__ void load1(__amdgpu_buffer_rsrc_t rc, __amdgpu_buffer_rsrc_t rv, int e, int &c, double &v)
{
    c = (int)__builtin_amdgcn_raw_buffer_load_b32(rc, e * 4, 0, AUX);
    v = __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(rv, e * 8, 0, AUX));
}

template <int AUX = kAuxNt>
__device__ __forceinline__ void load1(__amdgpu_buffer_rsrc_t rc, __amdgpu_buffer_rsrc_t rv, int e, int &c, float &v)
{
    c = (int)__builtin_amdgcn_raw_buffer_load_b32(rc, e * 4, 0, AUX);
    v = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rv, e * 4, 0, AUX));
}

template <int AUX = kAuxNt>
__device__ __forceinline__ void load1(__amdgpu_buffer_rsrc_t rc, __amdgpu_buffer_rsrc_t rv, int e, int &c, half_t &v)
{
    c = (int)__builtin_amdgcn_raw_buffer_load_b32(rc, e * 4, 0, AUX);
    v = __builtin_bit_cast(half_t, __builtin_amdgcn_raw_buffer_load_b16(rv, e * 2, 0, AUX));
}

__device__ __forceinline__ void store4(double *s, const double (&p)[4])
{
    reinterpret_cast<f64x2 *>(s)[0] = f64x2{p[0], p[1]};
    reinterpret_cast<f64x2 *>(s)[1] = f64x2{p[2], p[3]};
}

__device__ __forceinline__ void store4(float *s, const float (&p)[4])
{
    reinterpret_cast<f32x4 *>(s)[0] = f32x4{p[0], p[1], p[2], p[3]};
}

// ---- tile descriptor of k_tiles -------------------------------------------

struct TileDesc {
    int lo_row;  // first local row (the split row entering the tile, if any)
    int nr;      // local rows
    int A, B;    // nnz range [A, B) reduced by the tile
    int head;    // local row 0 is a long row that started in an earlier tile
    int tail;    // local row nr-1 is a long row continuing into the next tile
};

// Keys of tile t: [kb, ke).  The last tile of FLAT also takes key nnz, the
// first index of trailing empty rows.
template <bool MERGE>
__device__ __forceinline__ void tile_keys(long long t, long long ntiles, int K, int m, int nnz,
                                          uint32_t &kb, uint32_t &ke, bool &last)
{
    const uint32_t total = MERGE ? (uint32_t)nnz + (uint32_t)m : (uint32_t)nnz;
    last = (t == ntiles - 1);
    kb = (uint32_t)((unsigned long long)t * (unsigned long long)K);
    ke = last ? (MERGE ? total : total + 1u) : kb + (uint32_t)K;
}

template <bool MERGE>
__device__ __forceinline__ long long key_guess(uint32_t v, int m, int nnz)
{
    const unsigned long long total = MERGE ? (unsigned long long)nnz + m : (unsigned long long)nnz;
    if (total == 0) return 0;
    return (long long)(((unsigned long long)v * (unsigned long long)m) / total);
}

// Waves 0 and 1 find the first row owned by this tile and by the next one.
// Writes s_rows[0] = f, s_rows[1] = l: the tile owns rows [f, l).
template <bool MERGE>
__device__ __forceinline__ void search_tile_rows(const int *__restrict__ rp, int m, int nnz, int spread,
                                                 uint32_t kb, uint32_t ke, bool last, int *s_rows)
{
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    if (wave == 0) {
        const int r = wave_search_lt<MERGE>(rp, m, kb, key_guess<MERGE>(kb, m, nnz), spread, lane);
        if (lane == 0) s_rows[0] = r + 1;
    } else if (wave == 1) {
        const int r = last ? m - 1 : wave_search_lt<MERGE>(rp, m, ke, key_guess<MERGE>(ke, m, nnz), spread, lane);
        if (lane == 0) s_rows[1] = r + 1;
    }
}

// Descriptor of a tile from its owned rows [f, l); run by one lane.
template <bool MERGE, int LMAX, int SPAN_MAX>
__device__ TileDesc make_desc(const int *__restrict__ rp, int m, int nnz, uint32_t kb, uint32_t ke,
                              int f, int l, int *err)
{
    TileDesc d{0, 0, 0, 0, 0, 0};
    const int h = f - 1;
    if (h >= 0) {
        const int ph = rp[h], qh = rp[h + 1];
        const long long jk = (long long)kb - (MERGE ? h : 0);  // nnz index holding key kb
        if (qh - ph > LMAX && jk < qh) {
            d.head = 1;
            d.A = (int)jk;
        }
    }
    d.lo_row = d.head ? h : f;
    if (f < l) {
        if (!d.head) d.A = rp[f];
        const int e = l - 1;
        const int pe = rp[e], qe = rp[e + 1];
        const long long jend = (long long)ke - (MERGE ? e : 0);
        if (qe - pe > LMAX && (long long)qe > jend) {
            d.B = (int)jend;
            d.tail = 1;
        } else {
            d.B = qe;
        }
    } else if (d.head) {
        const long long jend = (long long)ke - (MERGE ? h : 0);
        const int qh = rp[h + 1];
        d.B = (long long)qh < jend ? qh : (int)jend;
    } else {
        d.A = d.B = 0;
    }
    d.nr = l - d.lo_row;
    // Consistency: anything else means row_ptr changed after planning.
    const bool ok = d.lo_row >= 0 && d.nr >= 0 && (long long)d.lo_row + d.nr <= m && d.A >= 0 &&
                    d.A <= d.B && d.B <= nnz && d.B - (d.A & ~3) <= SPAN_MAX;
    if (!ok) {
        atomicOr(err, 1);
        d = TileDesc{0, 0, 0, 0, 0, 0};
    }
    return d;
}

// ---- k_tiles: ADAPTIVE (MERGE) and FLAT -----------------------------------

template <typename T, bool MERGE, int K, int LMAX>
struct TileShape {
    static constexpr int kSpanMax = K + LMAX + 2;            // B - (A & ~3)
    static constexpr int kVecMax = (kSpanMax + 3) / 4;
    static constexpr int kVPT = (kVecMax + kBS - 1) / kBS;   // 4-nnz vectors per lane
    static constexpr int kProd = kVPT * kBS * 4;             // LDS products
    static constexpr int kWaveCap = (K + LMAX) / (kThreadMax + 1) + 1;
    static constexpr int kBlockCap = (K + LMAX) / (kWaveMax + 1) + 1;
};

// ---- pieces shared by k_tiles and k_stream ---------------------------------

// Issue the 16-byte loads of the tile's col/val vectors (4 nnz each,
// lane-strided) for the nnz range [base, B); lanes past B read zeros.
template <typename T, int VPT>
__device__ __forceinline__ void issue_cv(const Args<T> &a, int base, int B, int nvec, int (&c)[VPT][4],
                                         T (&v)[VPT][4])
{
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(a.col + base, (long long)(B - base) * 4);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.val + base, (long long)(B - base) * (long long)sizeof(T));
#pragma unroll
    for (int k = 0; k < VPT; ++k)
        if (k * kBS < nvec)  // uniform: skip whole vector slots past the tile
            load4(rc, rv, (int)threadIdx.x + k * kBS, c[k], v[k]);
}

// Gather x (ordinary loads: x stays in L2 / MALL) through a resource over
// x[0, n): a column outside [0, n) reads zero instead of memory past x.  Lanes
// past the tile hold column 0 and gather x[0]; their products are masked later.
template <typename T, int VPT>
__device__ __forceinline__ void gather_x(const Args<T> &a, int nvec, const int (&c)[VPT][4], T (&xv)[VPT][4])
{
    const __amdgpu_buffer_rsrc_t rx = make_rsrc_full(a.x, (long long)a.n * (long long)sizeof(T));
#pragma unroll
    for (int k = 0; k < VPT; ++k)
        if (k * kBS < nvec)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                xv[k][j] = buf_load(rx, (uint32_t)c[k][j] * (uint32_t)sizeof(T), (T *)nullptr);
}

// val * x, rounded, into LDS (no contraction with the later sums).
template <typename T, int VPT>
__device__ __forceinline__ void products_to_lds(T *s_prod, int base, int nvec, int A, int B, const T (&v)[VPT][4],
                                                const T (&xv)[VPT][4])
{
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int vec = threadIdx.x + k * kBS;
        if (vec < nvec) {
            T p[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = base + 4 * vec + j;
                p[j] = (e >= A && e < B) ? v[k][j] * xv[k][j] : T(0);
            }
            store4(s_prod + 4 * vec, p);
        }
    }
}

template <typename T, int WCAP, int BCAP>
struct ReduceLds {
    int nw, nb;
    int wl[WCAP], wa[WCAP], wb[WCAP];
    int bl[BCAP], ba[BCAP], bb[BCAP];
    T red[kWaves];
};

// The row-aligned kernels' lists also keep the sums of the listed rows.
template <typename T, int WCAP, int BCAP>
struct RowsReduceLds : ReduceLds<T, WCAP, BCAP> {
    T ws[WCAP];
    T bs[BCAP];
};

// Row sums of a tile whose products sit in s_prod (index = nnz - base).
// bounds(i, ra, rb) gives row_ptr[r], row_ptr[r+1] of local row i; put(i, s)
// stores the sum.  Rows of <= kThreadMax products: one lane each, summed in
// nnz order; <= kWaveMax: one wave each (DPP sum); longer: the workgroup.
// Whole workgroup; L.nw / L.nb must be 0 on entry and are 0 again on exit.
template <typename T, int WCAP, int BCAP, typename Bounds, typename Put>
__device__ __forceinline__ void reduce_tile(const T *s_prod, ReduceLds<T, WCAP, BCAP> &L, int base, int A, int B,
                                            int nr, Bounds bounds, Put put)
{
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    for (int i = tid; i < nr; i += kBS) {
        int ra, rb;
        bounds(i, ra, rb);
        ra = max(ra, A);
        rb = min(rb, B);
        const int a0 = ra - base;
        const int len = rb - ra;
        if (len <= kThreadMax) {
            T s = T(0);
            for (int q = 0; q < len; ++q)
                s += s_prod[a0 + q];
            put(i, s);
        } else if (len <= kWaveMax) {
            const int j = atomicAdd(&L.nw, 1);
            if (j < WCAP) { L.wl[j] = i; L.wa[j] = a0; L.wb[j] = a0 + len; }
        } else {
            const int j = atomicAdd(&L.nb, 1);
            if (j < BCAP) { L.bl[j] = i; L.ba[j] = a0; L.bb[j] = a0 + len; }
        }
    }
    lds_sync();
    const int nw = min(L.nw, WCAP);
    for (int j = wave; j < nw; j += kWaves) {
        T s = T(0);
        for (int q = L.wa[j] + lane; q < L.wb[j]; q += kWave)
            s += s_prod[q];
        s = wave_sum(s);
        if (lane == 0)
            put(L.wl[j], s);
    }
    const int nb = min(L.nb, BCAP);
    for (int j = 0; j < nb; ++j) {
        T s = T(0);
        for (int q = L.ba[j] + tid; q < L.bb[j]; q += kBS)
            s += s_prod[q];
        s = wave_sum(s);
        if (lane == 0)
            L.red[wave] = s;
        lds_sync();
        if (tid == 0) {
            T tot = L.red[0];
#pragma unroll
            for (int w = 1; w < kWaves; ++w)
                tot += L.red[w];
            put(L.bl[j], tot);
        }
        lds_sync();
    }
    lds_sync();
    if (tid == 0) {
        L.nw = 0;
        L.nb = 0;
    }
}

// ---- k_tiles: one tile per workgroup (FLAT, and the reference for k_stream) --

template <typename T, bool MERGE, int K, int LMAX>
__global__ __launch_bounds__(kBS) void k_tiles(Args<T> a)
{
    using S = TileShape<T, MERGE, K, LMAX>;
    __shared__ __attribute__((aligned(16))) T s_prod[S::kProd];
    __shared__ int s_rows[2];
    __shared__ int s_desc[6];
    __shared__ ReduceLds<T, S::kWaveCap, S::kBlockCap> L;

    const int tid = threadIdx.x;
    const long long t = xcd_tile(a.xch);
    if (t >= a.ntiles)
        return;  // whole workgroup: padding of the XCD mapping

    uint32_t kb, ke;
    bool last;
    tile_keys<MERGE>(t, a.ntiles, K, a.m, a.nnz, kb, ke, last);
    int c[S::kVPT][4];
    T v[S::kVPT][4], xv[S::kVPT][4];
    if constexpr (!MERGE) {
        // FLAT: the nnz range [kb, min(ke, nnz)) is known before any row is
        // found, so the col/val stream starts first and the row search
        // overlaps its latency.
        const int A0 = (int)kb, B0 = (int)min(ke, (uint32_t)a.nnz);
        const int base0 = A0 & ~3;
        issue_cv(a, base0, B0, B0 > A0 ? (B0 - base0 + 3) >> 2 : 0, c, v);
    }
    search_tile_rows<MERGE>(a.rp, a.m, a.nnz, a.guess_spread, kb, ke, last, s_rows);
    lds_sync();
    if (tid == 0) {
        const TileDesc d = make_desc<MERGE, LMAX, S::kSpanMax>(a.rp, a.m, a.nnz, kb, ke, s_rows[0],
                                                                s_rows[1], a.err);
        s_desc[0] = d.lo_row; s_desc[1] = d.nr; s_desc[2] = d.A; s_desc[3] = d.B;
        s_desc[4] = d.head; s_desc[5] = d.tail;
        L.nw = 0;
        L.nb = 0;
        a.owner[t] = d.tail ? d.lo_row + d.nr - 1 : -1;
    }
    lds_sync();
    const int lo_row = s_desc[0], nr = s_desc[1], A = s_desc[2], B = s_desc[3];
    const int head = s_desc[4], tail = s_desc[5];
    const int base = A & ~3;
    const int nvec = B > A ? (B - base + 3) >> 2 : 0;

    if constexpr (MERGE) issue_cv(a, base, B, nvec, c, v);
    gather_x(a, nvec, c, xv);
    products_to_lds(s_prod, base, nvec, A, B, v, xv);
    lds_sync();

    const int *__restrict__ rp = a.rp;
    reduce_tile(
        s_prod, L, base, A, B, nr,
        [&](int i, int &ra, int &rb) { ra = rp[lo_row + i]; rb = rp[lo_row + i + 1]; },
        [&](int i, T s) {
            if (head && i == 0) a.head[t] = s;
            else if (tail && i == nr - 1) a.tail[t] = s;
            else a.y[lo_row + i] = s;
        });
}

// ---- k_wave: wave-granular persistent, software-pipelined ADAPTIVE kernel ----
//
// Every wave64 is an independent streaming agent: it walks a contiguous run of
// tiles (XCD x owns tiles [x*tx, (x+1)*tx), split evenly over the waves
// resident on it) with no workgroup barrier anywhere.  Only the first tile of
// a run searches row_ptr; every later tile starts at the row where the
// previous one stopped and finds its last row by a ballot over a block of
// row_ptr held in registers (lane i holds entries i, i+64, i+128).  Three
// tiles are in flight per wave: while the products of tile t are summed, the
// col/val stream of tile t+1 and the row_ptr block of tile t+2 are loading.
// LDS is wave-private scratch (products, row bounds, long-row list); LDS
// operations of one wave execute in order, so no barrier is needed.
//
// The loop body issues a fixed sequence of memory operations: every load and
// store is an unconditional buffer operation, lanes with nothing to do use an
// offset outside the resource (dropped by the hardware, no traffic).  The
// compiler can then count outstanding operations exactly and waits only for
// the data it consumes, so the next tiles' loads stay in flight.

#ifndef PF_STORE_AUX
#define PF_STORE_AUX 0
#endif
constexpr int kStoreAux = PF_STORE_AUX;  // cache policy of the y stores

__device__ __forceinline__ void buf_store(__amdgpu_buffer_rsrc_t r, uint32_t off, double v)
{
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, (int)off, 0, 0);
}

__device__ __forceinline__ void buf_store(__amdgpu_buffer_rsrc_t r, uint32_t off, float v)
{
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned int, v), r, (int)off, 0, 0);
}

__device__ __forceinline__ void buf_store(__amdgpu_buffer_rsrc_t r, uint32_t off, int v)
{
    __builtin_amdgcn_raw_buffer_store_b32((unsigned int)v, r, (int)off, 0, 0);
}

// 16 bytes of consecutive values; the hardware range check drops the dwords
// past the resource's end, so a lane straddling it writes only its in-range rows.
__device__ __forceinline__ void buf_store16(__amdgpu_buffer_rsrc_t r, uint32_t off, const double (&w)[2])
{
    const u32x4 v = {(unsigned)__double2loint(w[0]), (unsigned)__double2hiint(w[0]), (unsigned)__double2loint(w[1]),
                     (unsigned)__double2hiint(w[1])};
    __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)off, 0, kStoreAux);
}

__device__ __forceinline__ void buf_store16(__amdgpu_buffer_rsrc_t r, uint32_t off, const float (&w)[4])
{
    const u32x4 v = {__float_as_uint(w[0]), __float_as_uint(w[1]), __float_as_uint(w[2]), __float_as_uint(w[3])};
    __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)off, 0, kStoreAux);
}

__device__ __forceinline__ int rlane(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }

template <typename T, int K, int LMAX>
struct WaveShape {
    static constexpr int kSpanMax = K + LMAX + 2;              // B - (A & ~3) <= K + LMAX - 1 + 3
    static constexpr int kVecMax = (kSpanMax + 3) / 4;
    static constexpr int kVPT = (kVecMax + kWave - 1) / kWave; // 4-nnz vector slots per lane
    static constexpr int kProd = kVPT * kWave * 4;             // products per wave
    static constexpr int kRPL = 3;                             // row_ptr entries per lane per round
    static constexpr int kRB = kRPL * kWave;                   // entries per round
    static constexpr int kRpCap = K + 2;                       // rows + 2 of any tile
    static constexpr int kRounds = (kRpCap + kRB - 1) / kRB;
    static constexpr int kQ = (K + 1 + kWave - 1) / kWave;     // local-row slots per lane (<= K+1 rows)
    static constexpr int kListCap = (K + LMAX) / (kThreadMax + 1) + 1;
    static constexpr int kQS = (K + 1 + kWave * (16 / (int)sizeof(T)) - 1) / (kWave * (16 / (int)sizeof(T)));  // 16-byte y stores per lane
    static_assert(kProd >= K + 1, "row sums are staged in the product buffer");
};

constexpr int kWaveWG = 256;  // 4 independent waves per workgroup

struct WaveDesc {
    int f;       // first owned row; block entry j = row_ptr[f-1+j]
    int l;       // one past the last owned row
    int lo_row, nr, A, B, head, tail;
};

// Round `r0` of the row_ptr block of a tile whose owned rows start at f:
// entry j = row_ptr[f-1+j] for j in [r0*kRB, (r0+1)*kRB); 0 for j = 0 when
// f == 0 and past row m.  valid == false reads nothing.
template <int RPL>
__device__ __forceinline__ void rp_issue(const int *__restrict__ rp, int m, int f, bool valid, int r0, int (&rr)[RPL])
{
    const int b0 = f > 0 ? f - 1 : 0;
    const int shift = f - 1 - b0;  // -1 when f == 0: entry 0 addresses byte -4, out of range
    const __amdgpu_buffer_rsrc_t r = make_rsrc(rp + b0, valid ? (long long)(m + 1 - b0) * 4 : 0);
    const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int q = 0; q < RPL; ++q)
        rr[q] = (int)__builtin_amdgcn_raw_buffer_load_b32(r, (r0 * RPL * kWave + q * kWave + lane + shift) * 4, 0, 0);
}

// Entry j of a block round held in registers (j uniform, 0 <= j < kRB).
template <int RPL>
__device__ __forceinline__ int rp_entry(const int (&rr)[RPL], int j)
{
    int v = 0;
#pragma unroll
    for (int q = 0; q < RPL; ++q)
        if (j >= q * kWave && j < (q + 1) * kWave) v = rlane(rr[q], j - q * kWave);
    return v;
}

// Smallest block index j >= 1 in round r0 whose row reaches key ke (rows past
// m count as reaching it), or -1.
template <int RPL>
__device__ __forceinline__ int rp_find(const int (&rr)[RPL], int r0, int f, int m, uint32_t ke)
{
    const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int q = 0; q < RPL; ++q) {
        const int j = r0 * RPL * kWave + q * kWave + lane;
        const int row = f - 1 + j;
        const bool ge = j >= 1 && (row >= m || (uint32_t)rr[q] + (uint32_t)row >= ke);
        const uint64_t mask = __ballot(ge);
        if (mask) return r0 * RPL * kWave + q * kWave + __ffsll((long long)mask) - 1;
    }
    return -1;
}

// The tile descriptor of a tile with keys [kb, ke) whose owned rows start at
// f.  rr holds round 0 of its row_ptr block; a tile with more than kRB-1 rows
// scans further rounds with synchronous loads.  Wave-uniform result.
template <int RPL, int ROUNDS, int LMAX, int SPAN_MAX>
__device__ __forceinline__ WaveDesc wave_desc(const int *__restrict__ rp, int m, int nnz, int f, uint32_t kb,
                                              uint32_t ke, const int (&rr)[RPL], int &err)
{
    constexpr int RB = RPL * kWave;
    int js = rp_find(rr, 0, f, m, ke);
    int pe = 0, qe = 0;
    if (js >= 1) {
        pe = rp_entry(rr, js - 1);
        qe = js < RB ? rp_entry(rr, js) : 0;
    }
    if (js < 0 || js >= RB) {  // rare: the tile's last row lies beyond round 0
        int tmp[RPL];
        int prev = rp_entry(rr, RB - 1);
        int r = 1;
        if (js >= RB) r = 1;  // js == RB impossible (index < RB); kept for clarity
        for (js = -1; r < ROUNDS && js < 0; ++r) {
            rp_issue(rp, m, f, true, r, tmp);
            js = rp_find(tmp, r, f, m, ke);
            if (js >= 0) {
                const int jl = js - r * RB;
                pe = jl >= 1 ? rp_entry(tmp, jl - 1) : prev;
                qe = rp_entry(tmp, jl);
            } else {
                prev = rp_entry(tmp, RB - 1);
            }
        }
        if (js < 0) {  // more rows than keys: row_ptr changed after planning
            err = 1;
            js = 1;
            pe = qe = rp_entry(rr, 1);
        }
    }
    const int l = f - 1 + js;
    WaveDesc d{f, l, 0, 0, 0, 0, 0, 0};
    const int h = f - 1;
    const int ph = rp_entry(rr, 0), qh = rp_entry(rr, 1);
    if (h >= 0) {
        const long long jk = (long long)kb - h;
        if (qh - ph > LMAX && jk < qh) {
            d.head = 1;
            d.A = (int)jk;
        }
    }
    d.lo_row = d.head ? h : f;
    if (f < l) {
        if (!d.head) d.A = qh;
        const long long jend = (long long)ke - (l - 1);
        if (qe - pe > LMAX && (long long)qe > jend) {
            d.B = (int)jend;
            d.tail = 1;
        } else {
            d.B = qe;
        }
    } else if (d.head) {
        const long long jend = (long long)ke - h;
        d.B = (long long)qh < jend ? qh : (int)jend;
    }
    d.nr = l - d.lo_row;
    const bool ok = d.lo_row >= 0 && d.nr >= 0 && (long long)d.lo_row + d.nr <= m && d.A >= 0 && d.A <= d.B &&
                    d.B <= nnz && d.B - (d.A & ~3) <= SPAN_MAX;
    if (!ok) {
        err = 1;
        d.lo_row = f; d.nr = 0; d.A = 0; d.B = 0; d.head = 0; d.tail = 0;
    }
    return d;
}

// col/val of a tile (an empty descriptor reads nothing).
template <typename T, int VPT, int AUX>
__device__ __forceinline__ void wave_issue_cv(const Args<T> &a, const WaveDesc &d, int (&c)[VPT][4], T (&v)[VPT][4])
{
    const int base = d.A & ~3;
    const long long n = d.B > d.A ? d.B - base : 0;
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(a.col + base, n * 4);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.val + base, val_range_bytes<T>((int)n));
    const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int k = 0; k < VPT; ++k)
        load4<AUX>(rc, rv, lane + k * kWave, c[k], v[k]);
}

template <typename T, int VPT>
__device__ __forceinline__ void wave_gather(__amdgpu_buffer_rsrc_t rx, int nvec, const int (&c)[VPT][4],
                                            T (&xv)[VPT][4])
{
    const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const bool in = lane + k * kWave < nvec;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            xv[k][j] = buf_load(rx, in ? (uint32_t)c[k][j] * (uint32_t)sizeof(T) : kOob, (T *)nullptr);
    }
}

// Row bounds of a tile into the wave's LDS block: round 0 from registers,
// the rare rows beyond it straight from row_ptr.
template <int RPL, int CAP>
__device__ __forceinline__ void rp_to_lds(const int *__restrict__ rp, const WaveDesc &d, const int (&rr)[RPL], int *s_rpb)
{
    const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int q = 0; q < RPL; ++q)
        if (q * kWave + lane < CAP) s_rpb[q * kWave + lane] = rr[q];
    const int nent = d.l - d.f + 2;  // entries f-1 .. l
    if (nent > RPL * kWave)
        for (int j = RPL * kWave + lane; j < nent && j < CAP; j += kWave)
            s_rpb[j] = rp[d.f - 1 + j];
}

// DESC_ONLY: instead of computing y, write every tile's descriptor to dbg (8
// ints per tile; the index test of this exact code path) or, with dbg NULL,
// the owner of every tile (the row whose split starts in it, else -1) — the
// per-pattern table the combine kernel reads, built once at planning.
// Waves per SIMD the register allocation targets: 7 (72 VGPRs) for one
// 4-nnz vector per lane, fewer for larger tiles.
template <typename T, int K, int LMAX>
constexpr int wave_occupancy()
{
    constexpr int vpt = WaveShape<T, K, LMAX>::kVPT;
    return vpt == 1 ? (LMAX == 16 ? 6 : 7) : vpt == 2 ? 4 : vpt == 3 ? 3 : 2;
}

// NT: col/val loads non-temporal (a matrix larger than the MALL: keep x there);
// otherwise ordinary loads, so that a matrix that fits stays cached across calls.
template <typename T, int K, int LMAX, bool DESC_ONLY, bool NT = true, int WPE = wave_occupancy<T, K, LMAX>()>
__global__ __launch_bounds__(kWaveWG) __attribute__((amdgpu_waves_per_eu(WPE, 8))) void k_wave(Args<T> a, int *__restrict__ dbg)
{
    using S = WaveShape<T, K, LMAX>;
    using A = acc_t<T>;  // products and sums (fp32 in the fp16 mode)
    constexpr int VPT = S::kVPT, Q = S::kQ, RPL = S::kRPL, LCAP = S::kListCap, CAP = S::kRpCap;
    constexpr int NW = kWaveWG / kWave;
    __shared__ __attribute__((aligned(16))) A s_prod_all[NW][DESC_ONLY ? 4 : S::kProd];
    __shared__ int s_rpb_all[NW][2][DESC_ONLY ? 4 : CAP];
    __shared__ int s_la_all[NW][LCAP], s_lb_all[NW][LCAP];
    __shared__ A s_ls_all[NW][LCAP];
    // Row sums staged for the y stores: a buffer of their own when LDS allows
    // (one 4-nnz vector per lane), else the product buffer after the sums.
    constexpr bool YL = S::kVPT == 1 && !DESC_ONLY;
    __shared__ __attribute__((aligned(16))) A s_y_all[NW][YL ? K + 1 : 1];
    __shared__ int s_li_all[NW][YL ? LCAP : 1];

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    A *s_prod = s_prod_all[wave];
    int *s_la = s_la_all[wave];
    int *s_lb = s_lb_all[wave];
    A *s_ls = s_ls_all[wave];
    A *s_y = YL ? s_y_all[wave] : s_prod;
    int *s_li = s_li_all[wave];

    // Run of a.tpw consecutive tiles: XCD x owns runs [x*tx, (x+1)*tx), taken
    // in dispatch order, so the tiles in flight on an XCD form a narrow front
    // and their x entries stay in its L2.
    const long long xcd = blockIdx.x % kXcds;
    const long long wx = (blockIdx.x / kXcds) * NW + wave;  // run index inside its XCD
    if (wx >= a.tx)
        return;  // whole wave: no barrier in this kernel
    long long t = (xcd * a.tx + wx) * a.tpw;
    long long t_end = t + a.tpw;
    if (t_end > a.ntiles) t_end = a.ntiles;
    if (t >= t_end)
        return;

    const __amdgpu_buffer_rsrc_t rx = make_rsrc_full(a.x, (long long)a.n * (long long)sizeof(T));
    const __amdgpu_buffer_rsrc_t rhead = make_rsrc_full(a.head, a.ntiles * (long long)sizeof(A));
    const __amdgpu_buffer_rsrc_t rtail = make_rsrc_full(a.tail, a.ntiles * (long long)sizeof(A));
    int err = 0;

    uint32_t kb, ke;
    bool last;
    tile_keys<true>(t, a.ntiles, K, a.m, a.nnz, kb, ke, last);
    const int f0 = wave_search_lt<true>(a.rp, a.m, kb, key_guess<true>(kb, a.m, a.nnz), a.guess_spread, lane) + 1;
    int rr[RPL];
    rp_issue(a.rp, a.m, f0, true, 0, rr);
    WaveDesc d = wave_desc<RPL, S::kRounds, LMAX, S::kSpanMax>(a.rp, a.m, a.nnz, f0, kb, ke, rr, err);
    int buf = 0;
    if (!DESC_ONLY) rp_to_lds<RPL, CAP>(a.rp, d, rr, s_rpb_all[wave][0]);
    rp_issue(a.rp, a.m, d.l, t + 1 < t_end, 0, rr);
    int c[VPT][4];
    T v[VPT][4];
    constexpr int CV_AUX = NT ? kAuxNt : 0;
    if (!DESC_ONLY) wave_issue_cv<T, VPT, CV_AUX>(a, d, c, v);

    for (;;) {
        if (DESC_ONLY && lane == 0) {
            if (dbg) {
                int *o = dbg + 8 * t;
                o[0] = d.lo_row; o[1] = d.nr; o[2] = d.A; o[3] = d.B; o[4] = d.head; o[5] = d.tail;
                o[6] = d.f; o[7] = d.l;
            } else {
                a.owner[t] = d.tail ? d.lo_row + d.nr - 1 : -1;
            }
        }
        const int base = d.A & ~3;
        const int nvec = d.B > d.A ? (d.B - base + 3) >> 2 : 0;
        T xv[VPT][4], vt[VPT][4];
        if (!DESC_ONLY) {
            wave_gather(rx, nvec, c, xv);
#pragma unroll
            for (int k = 0; k < VPT; ++k)
#pragma unroll
                for (int j = 0; j < 4; ++j) vt[k][j] = v[k][j];
        }

        // Next tile: its row_ptr block was issued one iteration ago.
        const bool more = t + 1 < t_end;
        WaveDesc dn{d.l, d.l, d.l, 0, 0, 0, 0, 0};
        if (more) {
            uint32_t kbn, ken;
            bool lastn;
            tile_keys<true>(t + 1, a.ntiles, K, a.m, a.nnz, kbn, ken, lastn);
            dn = wave_desc<RPL, S::kRounds, LMAX, S::kSpanMax>(a.rp, a.m, a.nnz, d.l, kbn, ken, rr, err);
            if (!DESC_ONLY) rp_to_lds<RPL, CAP>(a.rp, dn, rr, s_rpb_all[wave][buf ^ 1]);
        }
        rp_issue(a.rp, a.m, dn.l, t + 2 < t_end, 0, rr);
        if (!DESC_ONLY) wave_issue_cv<T, VPT, CV_AUX>(a, dn, c, v);

        if (!DESC_ONLY) {
            const int *s_rpb = s_rpb_all[wave][buf];
            // Products of tile t (waits for its x gathers only).  Slots
            // outside [A, B) hold neighbours' products or zeros; no sum reads
            // them (every row range below is clamped to [A, B)).
#pragma unroll
            for (int k = 0; k < VPT; ++k) {
                const int vec = lane + k * kWave;
                A p[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) p[j] = A(vt[k][j]) * A(xv[k][j]);
                store4(s_prod + 4 * vec, p);
            }
            __builtin_amdgcn_wave_barrier();

            // Pass 1: rows of <= kThreadMax products, one lane each in nnz
            // order; longer rows are listed for pass 2.  The sums go to s_y
            // (YL) or are kept in registers until the products are consumed.
            const int jo = d.lo_row - (d.f - 1);  // block index of local row 0
            int tag[YL ? 1 : Q];
            A sq[YL ? 1 : Q];
            int nl = 0;
#pragma unroll
            for (int q = 0; q < Q; ++q) {
                const int i = lane + q * kWave;
                if (!YL) { tag[q] = -1; sq[q] = A(0); }
                if (q * kWave < d.nr) {
                    bool lng = false;
                    int a0 = 0, a1 = 0;
                    if (i < d.nr) {
                        a0 = max(s_rpb[jo + i], d.A) - base;
                        a1 = min(s_rpb[jo + i + 1], d.B) - base;
                        if (a1 - a0 <= kThreadMax) {
                            A s = A(0);
#pragma unroll 4
                            for (int p = a0; p < a1; ++p)
                                s += s_prod[p];
                            if (!YL) sq[q] = s;
                            if (YL) s_y[i] = s;
                        } else {
                            lng = true;
                        }
                    }
                    const uint64_t mask = __ballot(lng);
                    if (mask) {
                        const int pos = nl + (int)__builtin_amdgcn_mbcnt_hi(
                                                 (unsigned)(mask >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)mask, 0u));
                        if (lng && pos < LCAP) {
                            s_la[pos] = a0;
                            s_lb[pos] = a1;
                            if (YL) s_li[pos] = i; else tag[q] = pos;
                        }
                        nl += __popcll(mask);
                    }
                }
            }
            __builtin_amdgcn_wave_barrier();
            // Pass 2: one listed row at a time, all 64 lanes, DPP sum.
            nl = min(nl, LCAP);
            for (int j = 0; j < nl; ++j) {
                A s = A(0);
                const int e1 = s_lb[j];
                for (int p = s_la[j] + lane; p < e1; p += kWave)
                    s += s_prod[p];
                s = wave_sum(s);
                if (lane == 0) {
                    if (YL) s_y[s_li[j]] = s; else s_ls[j] = s;
                }
            }
            __builtin_amdgcn_wave_barrier();
            // Pass 3 (registers): every row sum into s_prod[local row].
            if (!YL) {
#pragma unroll
                for (int q = 0; q < Q; ++q) {
                    const int i = lane + q * kWave;
                    if (q * kWave < d.nr && i < d.nr)
                        s_y[i] = tag[q] >= 0 ? s_ls[tag[q]] : sq[q];
                }
                __builtin_amdgcn_wave_barrier();
            }
            // 16-byte stores of consecutive rows: a fixed number of store
            // instructions, the resource spanning exactly the rows this tile
            // owns (the split rows at its edges go to the head / tail slots).
            const int r0 = d.head;                 // first local row written to y
            const int nw = d.nr - d.head - d.tail; // rows written to y
            const __amdgpu_buffer_rsrc_t ryt =
                make_rsrc(a.y + (d.lo_row + r0), (long long)nw * (long long)sizeof(T));
            if constexpr (__is_same(T, half_t)) {
                // fp16: one 2-byte store per row (the range check drops whole dwords, so a 16-byte
                // store ending in a half-covered dword would lose the last row)
                for (int j = lane; j < nw; j += kWave)
                    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, T(s_y[r0 + j])), ryt,
                                                          j * 2, 0, kStoreAux);
            } else {
                constexpr int P = 16 / (int)sizeof(T);
#pragma unroll
                for (int q = 0; q < S::kQS; ++q) {
                    // Slot 0 always issues; later slots only when the tile has the
                    // rows (wave-uniform branch), so most tiles issue one store.
                    if (q == 0 || q * kWave * P < nw) {
                        const int j = (q * kWave + lane) * P;
                        T w[P];
#pragma unroll
                        for (int p = 0; p < P; ++p) w[p] = T(0);
                        if (j < nw) {
#pragma unroll
                            for (int p = 0; p < P; ++p) w[p] = T(s_y[r0 + j + p < K + 1 ? r0 + j + p : 0]);
                        }
                        buf_store16(ryt, j < nw ? (uint32_t)j * (uint32_t)sizeof(T) : kOob, w);
                    }
                }
            }
            // Partials of split rows (rare; owner[] is built once per pattern).
            const uint32_t tslot = (uint32_t)t * (uint32_t)sizeof(A);
            if (d.head) buf_store(rhead, lane == 0 ? tslot : kOob, s_y[0]);
            if (d.tail) buf_store(rtail, lane == 0 ? tslot : kOob, s_y[d.nr > 0 ? d.nr - 1 : 0]);
            __builtin_amdgcn_wave_barrier();
        }
        if (!more)
            break;
        ++t;
        d = dn;
        buf ^= 1;
    }
    if (err && lane == 0) atomicOr(a.err, 1);
}

// ---- x-window schedule of split-row FLAT tiles ------------------------------
//
// For matrices whose long rows sweep an x larger than one XCD's L2 (sorted
// columns: a row of 300k nnz touches every line of an 8 MB x), the tiles are
// dealt to XCDs by the part of x they start in rather than by position: tile t
// goes to list k = 8 * col[t*K] / n.  The first call of a plan (the one that
// searches rows) appends each tile to its list; later calls run workgroup
// (XCD k, slot s) on the s-th tile of list k, so the XCD's long-row tiles read
// one eighth of x, which its L2 holds.  Lists hold at most cap tiles; a tile
// finding its list full goes to an overflow list whose tiles fill the other
// XCDs' spare slots, so every XCD gets at most cap tiles whatever the columns.
// Every tile still runs exactly once with the same work, so y is unchanged.
// Layout (ints): [0, 8) list counts, [8] overflow count, [16, 16 + 8 cap) the
// lists, then the overflow list (ntiles).  The counts start at 0 before the
// recording call.
constexpr int kSchedHead = 16;

__device__ __forceinline__ void sched_record(int *sched, long long cap, long long t, int col0, int n)
{
    long long k = n > 0 ? ((long long)col0 * kXcds) / n : 0;
    k = k < 0 ? 0 : (k >= kXcds ? kXcds - 1 : k);
    const int pos = atomicAdd(&sched[k], 1);
    if (pos < cap) {
        sched[kSchedHead + k * cap + pos] = (int)t;
    } else {
        const int o = atomicAdd(&sched[kXcds], 1);
        sched[kSchedHead + kXcds * cap + o] = (int)t;
    }
}

// The tile of this workgroup under a recorded schedule, -1 for a spare slot.
__device__ __forceinline__ long long sched_tile(const int *__restrict__ sched, long long cap, long long ntiles)
{
    const int k = (int)(blockIdx.x % kXcds);
    const long long s = blockIdx.x / kXcds;
    long long before = 0, mine = 0;
#pragma unroll
    for (int i = 0; i < kXcds; ++i) {
        const long long ci = min((long long)sched[i], cap);
        if (i < k) before += cap - ci;
        if (i == k) mine = ci;
    }
    long long t = -1;
    if (s < mine) {
        t = sched[kSchedHead + k * cap + s];
    } else {
        const long long j = before + (s - mine);
        if (j < (long long)sched[kXcds]) t = sched[kSchedHead + kXcds * cap + j];
    }
    return t < ntiles ? t : -1;
}

// ---- k_flat: FLAT tiles with the row search remembered across calls ---------
//
// One workgroup (4 wave64s) per tile of K nnz, XCD-interleaved.  A FLAT tile's
// nnz range [kb, min(kb + K, nnz)) is known before any row is, so every wave
// starts streaming col/val at once (16-byte non-temporal loads, K/1024
// vectors per lane).  The tile's rows are [f, l): f = the first row starting
// at or after kb, l = the first at or after the next tile's start.
//   MODE kFlatSearch: waves 2 and 3 find f and l by a wave-cooperative search
//     of row_ptr and record (f, row_ptr[f]) in the plan's row map;
//   MODE kFlatMemo: the row map written by an earlier search is read instead
//     (one load), so later calls of a plan skip the search latency;
//   MODE kFlatDesc: search only, the descriptors written to dbg (index test).
// From f, l, row_ptr[f] and row_ptr[l] every lane derives the tile
// descriptor with no further memory access; the row bounds are staged in LDS
// while x is gathered.

constexpr int kFlatSearch = 0, kFlatMemo = 1, kFlatDesc = 2;
// Element layout of the FLAT tiles (k_flat, k_rows).  Wave-strided for fp64
// and fp32: element (k, j) of a lane is nnz 1024k + 256 wave + 64j + lane of
// the tile, loaded with one 4- or 8-byte load, so each of a wave's loads and x
// gathers covers 64 consecutive nnz.  On rows with sorted columns a gather then
// touches about a quarter of the x lines it touches when a lane holds 4
// consecutive nnz (a wave's gather spanning 256 nnz), and the L1 and L2
// process that many fewer lines: C5 1104 -> 1016 us, C2 55.2 -> 51.3, C4
// 311 -> 300.  fp16 keeps 4 consecutive nnz per lane (16-byte col loads, 8-byte
// val loads): its 2-byte val loads would cover only 128 bytes per wave
// (C2 fp16 34.2 instead of 32.0 us).
template <typename T>
constexpr bool strided_layout() { return sizeof(T) >= 4; }

// Offset in its tile of element (k, j) of this lane (k < K / 1024, j < 4).
template <typename T>
__device__ __forceinline__ int tile_elem(int k, int j)
{
    const int tid = (int)threadIdx.x;
    return strided_layout<T>() ? k * (4 * kBS) + (tid & ~(kWave - 1)) * 4 + j * kWave + (tid & (kWave - 1))
                               : 4 * (tid + k * kBS) + j;
}

template <typename T, int K>
struct FlatShape {
    static constexpr int kVPT = K / (4 * kBS);                   // 4-nnz vectors per lane
    static constexpr int kRpCap = K + 2;                         // row bounds staged in LDS
    static constexpr int kWaveCap = K / (kThreadMax + 1) + 1;
    static constexpr int kBlockCap = K / (kWaveMax + 1) + 1;
    static_assert(kVPT * 4 * kBS == K, "K must be a multiple of 1024");
};

template <typename T, int K, int MODE>
__global__ __launch_bounds__(kBS) void k_flat(Args<T> a, int *__restrict__ map, int *__restrict__ dbg)
{
    using S = FlatShape<T, K>;
    constexpr int VPT = S::kVPT;
    constexpr bool DESC = MODE == kFlatDesc;
    using P = acc_t<T>;
    __shared__ __attribute__((aligned(16))) P s_prod[DESC ? 4 : K];
    __shared__ int s_rp[DESC ? 4 : S::kRpCap];
    __shared__ int s_info[4];  // f, row_ptr[f], l, row_ptr[l]
    __shared__ ReduceLds<P, S::kWaveCap, S::kBlockCap> L;

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const long long t = (MODE == kFlatMemo && a.sched) ? sched_tile(a.sched, a.sched_cap, a.ntiles) : xcd_tile(a.xch);
    if (t < 0 || t >= a.ntiles)
        return;  // whole workgroup: padding of the XCD mapping, or a spare schedule slot
    const int m = a.m, nnz = a.nnz;
    const bool last = t == a.ntiles - 1;
    const int kb = (int)(t * K);
    const int B = last ? nnz : kb + K;                 // nnz range [kb, B)
    const uint32_t ke = last ? (uint32_t)nnz + 1u : (uint32_t)(kb + K);

    int c[VPT][4];
    T v[VPT][4];
    T xv[VPT][4];
    if (!DESC) {
        const __amdgpu_buffer_rsrc_t rc = make_rsrc(a.col + kb, (long long)(B - kb) * 4);
        const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.val + kb, val_range_bytes<T>(B - kb));
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
            if constexpr (strided_layout<T>()) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    load1(rc, rv, tile_elem<T>(k, j), c[k][j], v[k][j]);
            } else {
                load4(rc, rv, tid + k * kBS, c[k], v[k]);
            }
        }
        // The x gathers depend on col only: they are issued before the rows
        // are known and stay in flight across the row search (or the row map
        // read) and its barrier, which fences LDS only.  Slots past the tile
        // read nothing and are never summed.
        const __amdgpu_buffer_rsrc_t rx = make_rsrc_full(a.x, (long long)a.n * (long long)sizeof(T));
#pragma unroll
        for (int k = 0; k < VPT; ++k)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                xv[k][j] = buf_load(rx, tile_elem<T>(k, j) < B - kb ? (uint32_t)c[k][j] * (uint32_t)sizeof(T) : kOob,
                                    (T *)nullptr);
    }
    if (MODE == kFlatMemo) {
        if (tid == 0) {
            const int2 e0 = reinterpret_cast<const int2 *>(map)[t];
            const int2 e1 = reinterpret_cast<const int2 *>(map)[t + 1];
            s_info[0] = e0.x; s_info[1] = e0.y; s_info[2] = e1.x; s_info[3] = e1.y;
        }
    } else if (wave == 2) {  // f: first row with row_ptr >= kb
        if (MODE == kFlatSearch && a.sched && lane == 0)
            sched_record(a.sched, a.sched_cap, t, kb < nnz ? a.col[kb] : 0, a.n);
        int rpf = 0;
        const int f = kb == 0 ? (rpf = a.rp[0], 0)
                              : wave_search_lt_next(a.rp, m, (uint32_t)kb, key_guess<false>((uint32_t)kb, m, nnz),
                                                    a.guess_spread, lane, rpf) + 1;
        if (lane == 0) {
            s_info[0] = f; s_info[1] = rpf;
            if (MODE == kFlatSearch && map) reinterpret_cast<int2 *>(map)[t] = make_int2(f, rpf);
        }
    } else if (wave == 3) {  // l: first row with row_ptr >= ke (m for the last tile)
        int rpl = 0;
        const int l = last ? (rpl = a.rp[m], m)
                           : wave_search_lt_next(a.rp, m, ke, key_guess<false>(ke, m, nnz), a.guess_spread, lane,
                                                 rpl) + 1;
        if (lane == 0) {
            s_info[2] = l; s_info[3] = rpl;
            if (MODE == kFlatSearch && map && last) reinterpret_cast<int2 *>(map)[t + 1] = make_int2(l, rpl);
        }
    }
    if (tid == 0) { L.nw = 0; L.nb = 0; }
    lds_sync();

    // Descriptor (the FLAT case of make_desc, from the four values).
    const int f = s_info[0], rpf = s_info[1], l = s_info[2], rpl = s_info[3];
    const int head = (f > 0 && rpf > kb) ? 1 : 0;  // row f-1 started before kb and reaches into the tile
    int lo_row = head ? f - 1 : f;
    int nr = l - lo_row;
    int tail = (!last && f < l && rpl > (int)ke) ? 1 : 0;
    const bool ok = f >= 0 && l >= f && l <= m && lo_row >= 0 && rpf >= kb && rpf <= nnz && rpl <= nnz &&
                    (last || rpl >= (int)ke);
    if (!ok) {  // row_ptr (or the row map) changed after planning
        if (tid == 0) atomicOr(a.err, 1);
        lo_row = 0; nr = 0; tail = 0;
    }
    if (DESC) {
        if (tid == 0) {
            int *o = dbg + 8 * t;
            o[0] = lo_row; o[1] = nr;
            o[2] = nr > 0 ? kb : 0; o[3] = nr > 0 ? (f < l ? (tail ? (int)ke : rpl) : min(rpf, B)) : 0;
            o[4] = ok ? head : 0; o[5] = tail; o[6] = f; o[7] = l;
        }
        return;
    }

    // Row bounds into LDS (global row_ptr is read directly beyond kRpCap).
    for (int i = tid; i <= nr && i < S::kRpCap; i += kBS)
        s_rp[i] = a.rp[lo_row + i];
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        if constexpr (strided_layout<T>()) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                s_prod[tile_elem<T>(k, j)] = P(v[k][j]) * P(xv[k][j]);
        } else {
            P p[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                p[j] = P(v[k][j]) * P(xv[k][j]);
            store4(s_prod + 4 * (tid + k * kBS), p);
        }
    }
    lds_sync();

    const int *__restrict__ rp = a.rp;
    reduce_tile(
        s_prod, L, kb, kb, B, nr,
        [&](int i, int &ra, int &rb) {
            ra = i < S::kRpCap ? s_rp[i] : rp[lo_row + i];
            rb = i + 1 < S::kRpCap ? s_rp[i + 1] : rp[lo_row + i + 1];
        },
        [&](int i, P s) {
            if (head && i == 0) a.head[t] = s;
            else if (tail && i == nr - 1) a.tail[t] = s;
            else a.y[lo_row + i] = T(s);
        });
    if (tid == 0) a.owner[t] = tail ? lo_row + nr - 1 : -1;
}

// ---- k_rows: FLAT tiles that own whole rows --------------------------------
//
// For matrices whose rows all hold at most kAlignRowMax nnz (checked at
// planning).  Tile t owns the rows that start in its nnz range [kb, kb + K):
// rows [f, l), with f and l as in k_flat (the row map is the same).  No row is
// split, so a step is this one launch, with no head / tail partials and no
// combine kernel.  The tile's products are the nnz [row_ptr[f], row_ptr[l]),
// which start at or after kb and end before kb + K + kAlignRowMax:
//   * the nominal range [kb, kb + K) is streamed before the rows are known;
//     its nnz before row_ptr[f] belong to the previous tile's last row and
//     are not gathered;
//   * the overflow [kb + K, row_ptr[l]) of the tile's last row (fewer than
//     kAlignRowMax nnz, one per lane) is read once l is known.
//   MODE kFlatMemo: every wave reads (f, row_ptr[f]) of tiles t and t + 1 from
//     the row map itself (a uniform load, no barrier), so its row_ptr,
//     overflow and gather loads follow its col/val loads at once;
//   MODE kFlatSearch: waves 2 and 3 search and record the map, as in k_flat;
//   MODE kFlatDesc: descriptors only (index test).

constexpr int kAlignRowMax = PFK_ALIGN_ROW_MAX;

template <typename T, int K>
struct RowsShape {
    static constexpr int kVPT = K / (4 * kBS);                   // 4-nnz vectors per lane
    static constexpr int kProd = K + kAlignRowMax;               // products: nominal range + overflow
    static constexpr int kRpCap = K + 2;                         // row bounds staged in LDS
    static constexpr int kRpPer = (kRpCap + kBS - 1) / kBS;      // row_ptr loads per lane
    static constexpr int kWaveCap = kProd / (kThreadMax + 1) + 1;
    static constexpr int kBlockCap = kProd / (kWaveMax + 1) + 1;
    static_assert(kVPT * 4 * kBS == K, "K must be a multiple of 1024");
    static_assert(kAlignRowMax <= kBS, "one overflow nnz per lane");
};

// A row-aligned tile once its rows are known (see k_rows): rows [f0, f0 + nr),
// products of nnz [A, B), nov overflow nnz past kb + K, cnt row bounds staged.
struct RowsDesc {
    int kb, B0, f0, nr, nov, A, B, cnt;
    int clo, chi;  // x-halves: the columns this workgroup gathers, [clo, chi)
};

// The tile's loads after its col / val: the overflow col / val, the x gathers
// of the nominal range and of the overflow, and row_ptr[f0 .. f0 + cnt).  The
// gathers are issued by every lane (an out-of-range offset reads nothing), and
// so are the overflow loads except in the case below, so the compiler's wait
// counts in front of the gathers are exact.  The row_ptr loads skip whole
// waves past cnt.
//   EARLY_RP false: the row_ptr loads come last, where a wait for all of them
//     costs nothing.
//   EARLY_RP true (matrices of very short rows, where row_ptr is a third of
//     the stream): they are issued before the gathers, so their latency runs
//     alongside the col / val stream's; the wait in front of the gathers then
//     also covers some of them (the compiler cannot count loads a wave may
//     skip).  C4: 310.5 instead of 320.4 us (fp64), 224.3 instead of 227.9
//     (fp32); on C2 it costs 0.5-0.7 us in fp32 / fp16, hence the split.
//   preloaded: the overflow col / val (oc, ov) were loaded with the nominal
//     range, before the rows were known (see k_rows); only its gathers remain.
template <typename T, int K, bool EARLY_RP, bool HALVES = false>
__device__ __forceinline__ void rows_loads(const Args<T> &a, const RowsDesc &d, const int (&c)[RowsShape<T, K>::kVPT][4],
                                           T (&xv)[RowsShape<T, K>::kVPT][4], T &ov, T &xo,
                                           int (&rr)[RowsShape<T, K>::kRpPer], int &oc, bool preloaded)
{
    using S = RowsShape<T, K>;
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int ob = d.nov > 0 ? d.kb + K : 0;
    const __amdgpu_buffer_rsrc_t rco = make_rsrc(a.col + ob, (long long)d.nov * 4);
    const __amdgpu_buffer_rsrc_t rvo = make_rsrc(a.val + ob, (long long)d.nov * (long long)sizeof(T));
    // With one col vector per lane and the row_ptr loads last, a wave whose
    // lanes hold no overflow nnz skips the three overflow loads (C2 fp64:
    // 55.6 instead of 56.6 us): the wait before the gathers then also covers
    // the val loads issued right after col, which arrive with it.  With more
    // col vectors, or row_ptr loads ahead of the gathers, that wait would also
    // cover later vectors' loads or the row_ptr loads (C2 fp32 +0.4, fp16
    // +1.3, C4 fp64 +19 us), so every wave issues them.  ov, oc and xo are
    // read only by lanes below nov.
    constexpr bool kSkipOvf = S::kVPT == 1 && !EARLY_RP;
    const bool ovw = !kSkipOvf || wave * kWave < d.nov;  // wave-uniform
    if (!preloaded) {
        oc = -1;
        if (ovw) {
            oc = (int)__builtin_amdgcn_raw_buffer_load_b32(rco, tid * 4, 0, kAuxNt);
            ov = buf_load(rvo, (uint32_t)(tid * (int)sizeof(T)), (T *)nullptr);
        }
    }
    const __amdgpu_buffer_rsrc_t rrp = make_rsrc(a.rp + d.f0, (long long)d.cnt * 4);
    const auto rp_loads = [&] {
#pragma unroll
        for (int q = 0; q < S::kRpPer; ++q) {
            rr[q] = 0;
            if (q * kBS + wave * kWave < d.cnt)
                rr[q] = (int)__builtin_amdgcn_raw_buffer_load_b32(rrp, (tid + q * kBS) * 4, 0, 0);
        }
    };
    if constexpr (EARLY_RP) {
        rp_loads();
        __builtin_amdgcn_sched_barrier(0);  // keep them ahead of the gathers
    }
    const __amdgpu_buffer_rsrc_t rx = make_rsrc_full(a.x, (long long)a.n * (long long)sizeof(T));
#pragma unroll
    for (int k = 0; k < S::kVPT; ++k) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int g = d.kb + tile_elem<T>(k, j);
            const bool use = g >= d.A && g < d.B && g < d.B0 &&  // slots outside [A, B) are never read
                             (!HALVES || (c[k][j] >= d.clo && c[k][j] < d.chi));
            xv[k][j] = buf_load(rx, use ? (uint32_t)c[k][j] * (uint32_t)sizeof(T) : kOob, (T *)nullptr);
        }
    }
    if (ovw)
        xo = buf_load(rx, tid < d.nov && (!HALVES || (oc >= d.clo && oc < d.chi)) ? (uint32_t)oc * (uint32_t)sizeof(T)
                                                                                   : kOob, (T *)nullptr);
    if constexpr (!EARLY_RP) rp_loads();
}

// Products and row bounds of a row-aligned tile into LDS.
// x-halves: a column outside this workgroup's half gives the product 0 (not
// v * 0, which is NaN for an infinite v); its half's workgroup forms it.
template <typename T, int K, bool HALVES = false>
__device__ __forceinline__ void rows_stage(const RowsDesc &d, const int (&c)[RowsShape<T, K>::kVPT][4],
                                           const T (&v)[RowsShape<T, K>::kVPT][4],
                                           const T (&xv)[RowsShape<T, K>::kVPT][4], int oc, T ov, T xo,
                                           const int (&rr)[RowsShape<T, K>::kRpPer], acc_t<T> *s_prod, int *s_rp)
{
    using S = RowsShape<T, K>;
    using P = acc_t<T>;
    const int tid = threadIdx.x;
    const auto mine = [&](int col) { return !HALVES || (col >= d.clo && col < d.chi); };
#pragma unroll
    for (int k = 0; k < S::kVPT; ++k) {
        if constexpr (strided_layout<T>()) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                s_prod[tile_elem<T>(k, j)] = mine(c[k][j]) ? P(v[k][j]) * P(xv[k][j]) : P(0);
        } else {
            P p[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                p[j] = mine(c[k][j]) ? P(v[k][j]) * P(xv[k][j]) : P(0);
            store4(s_prod + 4 * (tid + k * kBS), p);
        }
    }
    if (tid < d.nov) s_prod[K + tid] = mine(oc) ? P(ov) * P(xo) : P(0);
#pragma unroll
    for (int q = 0; q < S::kRpPer; ++q)
        if (tid + q * kBS < d.cnt) s_rp[tid + q * kBS] = rr[q];
}

// fp64 / fp32 row sums of a row-aligned tile whose bounds fit LDS, written as
// 16-byte non-temporal stores of consecutive rows.  Rows of at most
// kThreadMax products are summed by one lane, in nnz order, into registers;
// longer rows are listed and summed by a wave (or the workgroup) into LDS
// slots.  Once every product has been read, the sums are written over the
// product buffer and stored from there, so the staging costs no LDS of its own
// (occupancy stays that of the product buffer).  The range check of the store
// resource, exactly the tile's rows, drops the dwords past the last row.
template <typename T, int K, int YAUX>
__device__ __forceinline__ void rows_sums_staged(const RowsDesc &d, T *s_prod, const int *s_rp,
                                                 RowsReduceLds<T, RowsShape<T, K>::kWaveCap,
                                                               RowsShape<T, K>::kBlockCap> &L,
                                                 __amdgpu_buffer_rsrc_t ry)
{
    using S = RowsShape<T, K>;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    T ys[S::kRpPer];
    bool mine[S::kRpPer];
#pragma unroll
    for (int q = 0; q < S::kRpPer; ++q) {
        ys[q] = T(0);
        mine[q] = false;
        const int i = tid + q * kBS;
        if (i < d.nr) {
            const int ra = max(s_rp[i], d.A);
            const int rb = min(s_rp[i + 1], d.B);
            const int a0 = ra - d.kb;
            const int len = rb - ra;
            if (len <= kThreadMax) {
                T acc = T(0);
                for (int j = 0; j < len; ++j)
                    acc += s_prod[a0 + j];
                ys[q] = acc;
                mine[q] = true;
            } else if (len <= kWaveMax) {
                const int j = atomicAdd(&L.nw, 1);
                if (j < S::kWaveCap) { L.wl[j] = i; L.wa[j] = a0; L.wb[j] = a0 + len; }
            } else {
                const int j = atomicAdd(&L.nb, 1);
                if (j < S::kBlockCap) { L.bl[j] = i; L.ba[j] = a0; L.bb[j] = a0 + len; }
            }
        }
    }
    lds_sync();
    const int nw = min(L.nw, S::kWaveCap);
    const int nb = min(L.nb, S::kBlockCap);
    for (int j = wave; j < nw; j += kWaves) {
        T acc = T(0);
        for (int q = L.wa[j] + lane; q < L.wb[j]; q += kWave)
            acc += s_prod[q];
        acc = wave_sum(acc);
        if (lane == 0) L.ws[j] = acc;
    }
    for (int j = 0; j < nb; ++j) {
        T acc = T(0);
        for (int q = L.ba[j] + tid; q < L.bb[j]; q += kBS)
            acc += s_prod[q];
        acc = wave_sum(acc);
        if (lane == 0) L.red[wave] = acc;
        lds_sync();
        if (tid == 0) {
            T tot = L.red[0];
#pragma unroll
            for (int w = 1; w < kWaves; ++w)
                tot += L.red[w];
            L.bs[j] = tot;
        }
        lds_sync();
    }
    lds_sync();  // every product has been read: the buffer takes the sums
    T *s_y = s_prod;
#pragma unroll
    for (int q = 0; q < S::kRpPer; ++q)
        if (mine[q]) s_y[tid + q * kBS] = ys[q];
    for (int j = tid; j < nw; j += kBS) s_y[L.wl[j]] = L.ws[j];
    for (int j = tid; j < nb; j += kBS) s_y[L.bl[j]] = L.bs[j];
    lds_sync();
    constexpr int kPer = 16 / (int)sizeof(T);
    const int n16 = (d.nr + kPer - 1) / kPer;
    for (int j = tid; j < n16; j += kBS)
        __builtin_amdgcn_raw_buffer_store_b128(*reinterpret_cast<const u32x4 *>(s_y + j * kPer), ry, j * 16, 0, YAUX);
}

// Row sums of a staged row-aligned tile into y.  Bounds come from LDS; a tile
// with more rows than LDS holds (long runs of empty rows) reads the rest from
// row_ptr in a separate branch, so the common path waits on LDS only and
// leaves the y stores and any loads already issued for the next tile in flight.
// YAUX is the cache policy of the y stores.
template <typename T, int K, int YAUX>
__device__ __forceinline__ void rows_reduce(const Args<T> &a, const RowsDesc &d, acc_t<T> *s_prod,
                                            const int *s_rp,
                                            RowsReduceLds<acc_t<T>, RowsShape<T, K>::kWaveCap, RowsShape<T, K>::kBlockCap> &L)
{
    using S = RowsShape<T, K>;
    using P = acc_t<T>;
    if (d.nr < S::kRpCap) {
        // y[f0 .. f0 + nr) through a resource over exactly those rows, written
        // with the policy YAUX, not through L2: y is not read again here, and
        // keeping it out of L2 leaves room for x (C4: 345 instead of 377 us per
        // call with 8-byte stores through L2).
        const __amdgpu_buffer_rsrc_t ry = make_rsrc(a.y + d.f0, (long long)d.nr * (long long)sizeof(T));
        const auto bounds = [&](int i, int &ra, int &rb) {
            ra = s_rp[i];
            rb = s_rp[i + 1];
        };
        if constexpr (sizeof(T) >= 4) {
            rows_sums_staged<T, K, YAUX>(d, s_prod, s_rp, L, ry);
        } else {
            // fp16: one 2-byte store per row.  The range check works on whole
            // dwords, so a 16-byte store ending in a half-covered dword would
            // drop the tile's last row.
            reduce_tile(s_prod, L, d.kb, d.A, d.B, d.nr, bounds, [&](int i, P s) {
                __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, T(s)), ry, i * 2, 0, YAUX);
            });
        }
    } else {  // more rows than LDS holds: any number, up to m
        const int *__restrict__ rp = a.rp + d.f0;
        T *__restrict__ y = a.y + d.f0;
        reduce_tile(
            s_prod, L, d.kb, d.A, d.B, d.nr,
            [&](int i, int &ra, int &rb) {
                ra = i < S::kRpCap ? s_rp[i] : rp[i];
                rb = i + 1 < S::kRpCap ? s_rp[i + 1] : rp[i + 1];
            },
            [&](int i, P s) { y[i] = T(s); });
    }
}

// Row search of a row-aligned tile (the row holding nnz v), in two parts so
// that the first probe round can be issued ahead of the tile's col / val
// loads: a wave's vector loads complete in issue order, so a probe issued
// after them would wait for them.  Once the bracket holds at most kClose
// rows, the closing round reads the row bounds after its start with one
// scalar load, which completes on a counter of its own.  Same result as
// wave_search_lt_next.
constexpr int kClose = 16;  // row bounds read by the closing round of a row search

struct RowProbe {
    int guess, spread;  // the probes: guess + (lane - 32) * spread
    int lo0, hi0;       // the bracket they refine: row_ptr[lo0] < v; hi0 == m or row_ptr[hi0] >= v
    int k;              // row_ptr of this lane's probe, when valid
    bool valid;         // the probe lies inside (lo0, hi0)
};

__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }

__device__ __forceinline__ RowProbe row_probe_at(const int *__restrict__ rp, int guess, int spread, int lo0, int hi0,
                                                 int lane)
{
    RowProbe p;
    p.guess = uni(guess);
    p.spread = uni(spread);
    p.lo0 = uni(lo0);
    p.hi0 = uni(hi0);
    const long long q = (long long)p.guess + (long long)(lane - 32) * p.spread;
    p.valid = p.spread > 0 && q > p.lo0 && q < p.hi0;
    p.k = p.valid ? rp[(int)q] : 0;
    return p;
}

// Whole matrix: around the row the matrix's mean density gives, `spread`
// from the plan (0: no probe round), or, when the plan fitted a line to
// row_ptr (ga > 0), around the row the line gives, 1 apart.  A hint: any
// value gives the same result.
__device__ __forceinline__ RowProbe row_probe_issue(const int *__restrict__ rp, int m, uint32_t v, int nnz,
                                                    int spread, double ga, double gb, int lane)
{
    const double g = ga > 0.0 ? ga * (double)v + gb : (nnz > 0 ? (double)v * ((double)m / (double)nnz) : 0.0);
    const double gc = fmin(fmax(g, 0.0), (double)(m > 0 ? m - 1 : 0));  // (NaN: 0)
    return row_probe_at(rp, (int)gc, ga > 0.0 ? 1 : spread, 0, m, lane);
}

// Inside a run of a hybrid plan, rows [r0, r1) holding nnz [n0, n1): the 256
// row_ptr entries around the row that linear interpolation over the run puts
// the key v at, four consecutive entries per lane (one 16-byte load each).  A
// key they bracket is found in this one round (row_window_finish); a run's
// rows deviate from the interpolation by a few rows (a random walk pinned at
// both ends: in C5's runs of about 1000 rows of 8-64 nnz its standard
// deviation is at most about 7 rows).  row_ptr[r0 - 1] (the dense or long row before the
// run) is below any key of the run's tiles, and row_ptr[r1] (the run's end)
// at or above it, so the search never leaves the run.
struct RowWindow {
    int base;      // entries [base, base + 256), base a multiple of 4
    int lo0, hi0;  // the bracket they refine: row_ptr[lo0] < v <= row_ptr[hi0]
    u32x4 k;       // row_ptr[base + 4 lane + j], 0 past row_ptr's m + 1 entries
};

__device__ __forceinline__ RowWindow row_window_run(const int *__restrict__ rp, int m, int r0, int r1, int n0,
                                                    int n1, uint32_t v, int lane)
{
    RowWindow w;
    const double f = n1 > n0 ? ((double)v - (double)n0) / ((double)n1 - (double)n0) : 0.0;
    const int g = r0 + (int)fmin(fmax(f * (double)(r1 - r0), 0.0), (double)max(r1 - r0, 0));
    w.base = uni(max(0, g - 4 * kWave / 2) & ~3);
    w.lo0 = uni(max(r0 - 1, 0));
    w.hi0 = uni(r1);
    const __amdgpu_buffer_rsrc_t rr =
        make_rsrc(rp + w.base, (long long)max(0, min(4 * kWave, m + 1 - w.base)) * 4);
    w.k = __builtin_amdgcn_raw_buffer_load_b128(rr, lane * 16, 0, 0);
    return w;
}

// Largest r in [0, m) with row_ptr[r] < v (v > 0), and row_ptr[r + 1] in
// next_key, from the first round's probe.  Whole wave active; wave-uniform
// (the bracket is kept in scalar registers).
__device__ __forceinline__ int row_probe_finish(const int *__restrict__ rp, int m, uint32_t v, const RowProbe &p,
                                                int lane, int &next_key)
{
    typedef const int __attribute__((address_space(4))) cint;
    // row_ptr + i through the constant address space: the compiler reads it with scalar loads at a uniform
    // address (row_ptr is read-only in every kernel)
    const auto srp = [&](int i) {
        const unsigned long long qa = reinterpret_cast<unsigned long long>(rp + i);
        // readfirstlane returns int: keep each half unsigned, so the low half is zero-extended
        const unsigned alo = __builtin_amdgcn_readfirstlane((unsigned)qa);
        const unsigned ahi = __builtin_amdgcn_readfirstlane((unsigned)(qa >> 32));
        return (const cint *)(((unsigned long long)ahi << 32) | (unsigned long long)alo);
    };
    // the probe's fields are uniform, but the compiler only knows that of values read from one lane
    const int g = uni(p.guess), spread = uni(p.spread);
    int lo = uni(p.lo0), hi = uni(p.hi0);  // row_ptr[lo] < v; hi == m or row_ptr[hi] >= v
    bool hi_probed = false;
    if (spread > 0) {
        const uint64_t okm = __ballot(p.valid && (uint32_t)p.k < v);
        const uint64_t badm = __ballot(p.valid && (uint32_t)p.k >= v);
        // both are positions of valid probes, inside (lo, hi)
        const int nlo = okm ? g + (63 - __clzll(okm) - 32) * spread : lo;
        const int nhi = badm ? g + (__ffsll((long long)badm) - 1 - 32) * spread : hi;
        if (nlo < nhi) { lo = nlo; hi = nhi; hi_probed = badm != 0; }
    }
    bool have = false;
    int key = 0;
    if (hi_probed && hi - lo == 1) {  // hi is a probe of the first round: its row_ptr is that lane's
        have = true;
        key = __builtin_amdgcn_readlane(p.k, (hi - g) / spread + 32);
    }
    while (hi - lo > 1) {
        if (hi - lo <= kClose && lo <= m - kClose) {
            // closing round: row_ptr[lo + 1 + i] for i < kClose (one 64-byte scalar load), all inside
            // row_ptr's m + 1 entries; the answer is lo plus the count of those inside the bracket below v
            const cint *q = srp(lo + 1);
            int kk[kClose];
#pragma unroll
            for (int i = 0; i < kClose; ++i) kk[i] = q[i];
            const int w = hi - lo - 1;
            int c = 0;
#pragma unroll
            for (int i = 0; i < kClose - 1; ++i) c += (i < w && (uint32_t)kk[i] < v) ? 1 : 0;
            int nk = kk[0];
#pragma unroll
            for (int i = 1; i < kClose; ++i) nk = i == c ? kk[i] : nk;
            next_key = nk;
            return lo + c;
        }
        const int step = (int)(((long long)hi - lo + 63) >> 6);
        const long long pp = (long long)lo + (long long)lane * step;
        const bool probe = lane > 0 && pp < hi;
        const int k = probe ? rp[(int)pp] : 0;
        const bool ok = probe && (uint32_t)k < v;
        const int c = __popcll(__ballot(ok));
        if (step == 1 && c + 1 < kWave && lo + c + 1 < hi) {
            have = true;
            key = __builtin_amdgcn_readlane(k, c + 1);
        }
        const int nlo = lo + c * step;  // a probe's position, below hi
        const long long nhi = (long long)nlo + step;
        hi = uni(nhi < hi ? (int)nhi : hi);
        lo = uni(nlo);
    }
    next_key = have ? key : *srp(lo + 1);
    return lo;
}

// Largest r in [lo0, hi0) with row_ptr[r] < v, and row_ptr[r + 1] in
// next_key, from a run tile's window.  The window's entries strictly inside
// (lo0, hi0) below v are a prefix of them (row_ptr is non-decreasing): when
// the entry after that prefix is also in the window, the two bracket v and
// the search ends here; otherwise row_probe_finish goes on from the bracket
// the window left.  Whole wave active; wave-uniform.
__device__ __forceinline__ int row_window_finish(const int *__restrict__ rp, int m, uint32_t v, const RowWindow &w,
                                                 int lane, int &next_key)
{
    const int base = uni(w.base), lo0 = uni(w.lo0), hi0 = uni(w.hi0);
    const int s = min(max(lo0 + 1 - base, 0), 4 * kWave);  // entries [s, e) of the window lie inside (lo0, hi0)
    const int e = min(max(hi0 - base, s), 4 * kWave);
    int c = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = 4 * lane + j;
        c += __popcll(__ballot(i >= s && i < e && w.k[j] < v));
    }
    const int nlo = c > 0 ? base + s + c - 1 : lo0;  // row_ptr[nlo] < v
    if (s + c < e && (c > 0 || s + base == lo0 + 1)) {  // row_ptr[nlo + 1] >= v is the window's entry s + c
        const int i = s + c;
        const unsigned k0 = __builtin_amdgcn_readlane(w.k[0], i >> 2), k1 = __builtin_amdgcn_readlane(w.k[1], i >> 2);
        const unsigned k2 = __builtin_amdgcn_readlane(w.k[2], i >> 2), k3 = __builtin_amdgcn_readlane(w.k[3], i >> 2);
        const int sel = i & 3;
        next_key = (int)(sel == 0 ? k0 : sel == 1 ? k1 : sel == 2 ? k2 : k3);
        return nlo;
    }
    const int nhi = s + c < e ? base + s + c : hi0;
    const RowProbe p{0, 0, nlo, nhi, 0, false};  // no first round: 64-ary rounds from (nlo, nhi)
    return row_probe_finish(rp, m, v, p, lane, next_key);
}

// Runs of a hybrid plan: the rows between two dense rows (or a matrix end), each
// cut into row-aligned tiles of its own; `runs` holds, with R = nruns + 1,
// tile_begin[R] then row_begin, row_end, nnz_begin, nnz_end [R each].
struct RunTable {
    const int *__restrict__ runs;
    int nruns;
};

// The run holding run tile t: the largest i < nruns with tile_begin[i] <= t.
// First 16 entries around where t falls if the runs held equal numbers of
// tiles, read with one scalar load (the table is small and shared by every
// workgroup, so it stays in the scalar cache); when those do not bracket t, a
// wave-cooperative search.  Every read stays inside the table.
__device__ __forceinline__ int run_of_tile(const RunTable &rt, long long t, long long ntiles, int lane)
{
    typedef const int __attribute__((address_space(4))) cint;
    const int nr = rt.nruns;
    if (nr >= 16 && ntiles > 0) {
        const long long gl = t * nr / ntiles - 8;
        const int g = uni((int)min(max(gl, 0LL), (long long)(nr - 16)));  // entries [g, g + 16) of [0, nr)
        const unsigned long long qa = reinterpret_cast<unsigned long long>(rt.runs + g);
        const unsigned alo = __builtin_amdgcn_readfirstlane((unsigned)qa);  // each half unsigned (zero-extended)
        const unsigned ahi = __builtin_amdgcn_readfirstlane((unsigned)(qa >> 32));
        const cint *q = (const cint *)(((unsigned long long)ahi << 32) | (unsigned long long)alo);
        int kk[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) kk[i] = q[i];
        int c = 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) c += (long long)kk[i] <= t ? 1 : 0;
        // the entries at or below t are a prefix; t is bracketed when the first is one and the last is not
        // (or the window ends the table, whose end tile_begin[nr] is above every tile)
        if (c > 0 && (c < 16 || g + 16 == nr)) return g + c - 1;
    }
    long long lo = 0, hi = nr;  // tile_begin[lo] <= t < tile_begin[hi] (tile_begin[nruns] = total)
    while (hi - lo > 1) {
        const long long step = (hi - lo + 63) >> 6;
        const long long p = lo + (long long)lane * step;
        const bool ok = lane > 0 && p < hi && (long long)rt.runs[p] <= t;
        lo += (long long)__popcll(__ballot(ok)) * step;
        hi = (lo + step < hi) ? lo + step : hi;
    }
    return (int)lo;
}

template <typename T, int K, int MODE, bool PRIO = false, bool RUNS = false, bool HALVES = false>
__global__ __launch_bounds__(kBS) void k_rows(Args<T> a, int *__restrict__ map, int *__restrict__ dbg,
                                              RunTable rt = RunTable{nullptr, 0})
{
    using S = RowsShape<T, K>;
    constexpr int VPT = S::kVPT;
    constexpr bool DESC = MODE == kFlatDesc;
    __shared__ __attribute__((aligned(16))) acc_t<T> s_prod[DESC ? 4 : S::kProd];
    __shared__ int s_rp[DESC ? 4 : S::kRpCap];
    __shared__ int s_info[4];  // f, row_ptr[f], l, row_ptr[l] (search modes)
    __shared__ RowsReduceLds<acc_t<T>, S::kWaveCap, S::kBlockCap> L;

    // PRIO (chosen at launch for matrices of very short rows, under 4 nnz on
    // average): raised wave priority while the tile's loads are issued, so a
    // workgroup that has just started gets its memory streams going ahead of
    // the long per-row phase of older workgroups on the CU (C4: 320 instead of
    // 332 us per call), and the row_ptr loads issued before the gathers (see
    // rows_loads).  With longer rows the priority delays the older
    // workgroups' stores instead (C2: 60.2 instead of 58.1 us), and even
    // untaken it changes the code, hence a separate instantiation.
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const long long t = HALVES ? xcd_tile_half(a.xch) : xcd_tile(a.xch);
    if (t >= a.ntiles)
        return;  // whole workgroup: padding of the XCD mapping
    const int m = a.m, nnz = a.nnz;
    // Tile t's nominal nnz range [kb, B0); its rows end at row `lend` with
    // row_ptr `nend` when it is the last tile (of the matrix, or of its run).
    bool last = t == a.ntiles - 1;
    int kb = (int)(t * K);
    int B0 = last ? nnz : kb + K;
    int lend = m, nend = nnz;
    int run_r0 = 0, run_n0 = 0, run_n1 = 0;  // RUNS search: the run's first row, its nnz range
    int f = 0, rpf = 0, l = 0, rpl = 0;
    if constexpr (RUNS) {
        if (MODE == kFlatMemo) {  // recorded by the call that searched: (f, rpf, l, rpl), (kb, B0, last)
            const int4 *mp = reinterpret_cast<const int4 *>(map);
            const int4 e0 = mp[2 * t], e1 = mp[2 * t + 1];
            f = e0.x; rpf = e0.y; l = e0.z; rpl = e0.w;
            kb = e1.x; B0 = e1.y; last = e1.z != 0;
            lend = l; nend = rpl;
        } else {
            const int i = run_of_tile(rt, t, a.ntiles, lane);
            const int R = rt.nruns + 1;
            // tiles from the run's first nnz rounded down to 64, so every 64-lane load covers whole lines of
            // col and val; the nnz before the run's first row belong to the dense row before it and are
            // neither gathered nor summed (they precede row_ptr[f])
            const int nb = rt.runs[3 * R + i] & ~(kWave - 1), ne = rt.runs[4 * R + i];
            kb = nb + (int)(t - rt.runs[i]) * K;
            last = ne - kb <= K;
            B0 = last ? ne : kb + K;
            lend = rt.runs[2 * R + i];
            run_r0 = rt.runs[R + i];
            run_n0 = rt.runs[3 * R + i];
            run_n1 = ne;
            nend = ne;
        }
    }
    if constexpr (RUNS) {  // keep every load of the tile inside [0, nnz) and rows inside [0, m] whatever the tables hold
        kb = min(max(kb, 0), nnz);
        B0 = min(max(B0, kb), min(nnz, kb + K));
        lend = min(max(lend, 0), m);
        run_r0 = min(max(run_r0, 0), lend);
    }
    const uint32_t ke = last ? (uint32_t)nend + 1u : (uint32_t)(kb + K);

    if (!RUNS && MODE == kFlatMemo) {
        const int2 *mp = reinterpret_cast<const int2 *>(map);
        const int2 e0 = mp[t], e1 = mp[t + 1];
        f = e0.x; rpf = e0.y; l = e1.x; rpl = e1.y;
    }
    // Search modes: waves 2 and 3 issue the first probe round of their row
    // searches (f, l) ahead of the tile's col / val loads.
    RowProbe probe{0, 0, 0, m, 0, false};
    RowWindow window{0, 0, m, u32x4{0u, 0u, 0u, 0u}};
    if (MODE != kFlatMemo && ((wave == 2 && kb != 0) || (wave == 3 && !last))) {
        const uint32_t key = wave == 2 ? (uint32_t)kb : ke;
        if constexpr (RUNS)
            window = row_window_run(a.rp, m, run_r0, lend, run_n0, run_n1, key, lane);
        else
            probe = row_probe_issue(a.rp, m, key, nnz, a.guess_spread, a.guess_a, a.guess_b, lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    int c[VPT][4];
    T v[VPT][4];
    // The overflow of the tile's last row past kb + K is shorter than the
    // longest row (ovf_cap, from the plan's statistics): when that is known
    // and at most a wave, wave 0 loads its col / val here with the nominal
    // range, before the rows are known, so its gathers need not wait for a
    // load issued after the row search (C5's runs: 835 instead of 842 us per
    // step, C2 50.7 instead of 51.1).  Longer caps cost more than they save
    // (C3's runs, rows up to 256: 210 instead of 206 us, the cap re-read by
    // every tile), and so does the short-row mode, whose loads are ordered
    // for the row_ptr stream (C4: 307 instead of 299 us).
    const bool pre = !PRIO && a.ovf_cap > 0 && a.ovf_cap <= kWave;
    const int ocap = (pre && !last) ? max(0, min(a.ovf_cap, nnz - (kb + K))) : 0;
    int oc = -1;
    T ov = T(0);
    if (!DESC) {
        const __amdgpu_buffer_rsrc_t rc = make_rsrc(a.col + kb, (long long)(B0 - kb) * 4);
        const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.val + kb, val_range_bytes<T>(B0 - kb));
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
            if constexpr (strided_layout<T>()) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    load1(rc, rv, tile_elem<T>(k, j), c[k][j], v[k][j]);
            } else {
                load4(rc, rv, tid + k * kBS, c[k], v[k]);
            }
        }
        if (wave == 0 && ocap > 0) {  // wave-uniform
            const int ob = ocap > 0 ? kb + K : 0;
            const __amdgpu_buffer_rsrc_t rco = make_rsrc(a.col + ob, (long long)ocap * 4);
            const __amdgpu_buffer_rsrc_t rvo = make_rsrc(a.val + ob, val_range_bytes<T>(ocap));
            oc = (int)__builtin_amdgcn_raw_buffer_load_b32(rco, tid * 4, 0, kAuxNt);
            ov = buf_load(rvo, (uint32_t)(tid * (int)sizeof(T)), (T *)nullptr);
        }
    }
    if (MODE != kFlatMemo) {
        if (wave == 2) {  // f: first row with row_ptr >= kb
            int r = 0;
            const int ff = kb == 0 ? (r = a.rp[0], 0)
                                   : (RUNS ? row_window_finish(a.rp, m, (uint32_t)kb, window, lane, r)
                                           : row_probe_finish(a.rp, m, (uint32_t)kb, probe, lane, r)) + 1;
            if (lane == 0) {
                s_info[0] = ff; s_info[1] = r;
                if (!RUNS && MODE == kFlatSearch && map) reinterpret_cast<int2 *>(map)[t] = make_int2(ff, r);
            }
        } else if (wave == 3) {  // l: first row with row_ptr >= ke (the run's or matrix's end for a last tile)
            int r = 0;
            const int ll = last ? (r = a.rp[lend], lend)
                                : (RUNS ? row_window_finish(a.rp, m, ke, window, lane, r)
                                        : row_probe_finish(a.rp, m, ke, probe, lane, r)) + 1;
            if (lane == 0) {
                s_info[2] = ll; s_info[3] = r;
                if (!RUNS && MODE == kFlatSearch && map && last) reinterpret_cast<int2 *>(map)[t + 1] = make_int2(ll, r);
            }
        }
        lds_sync();
        f = s_info[0]; rpf = s_info[1]; l = s_info[2]; rpl = s_info[3];
        if (RUNS && MODE == kFlatSearch && map && tid == 0 && (!HALVES || blockIdx.x % kXcds < kXcds / 2)) {
            int4 *mp = reinterpret_cast<int4 *>(map);
            mp[2 * t] = make_int4(f, rpf, l, rpl);
            mp[2 * t + 1] = make_int4(kb, B0, last ? 1 : 0, 0);
        }
    }
    if (tid == 0) { L.nw = 0; L.nb = 0; }

    // The tile's rows [f, l) and nnz [rpf, rpl); everything read below is
    // bounded by these checks even if row_ptr changed after planning.
    const int ovf = last ? 0 : rpl - (int)ke;  // nnz of the last row past the nominal range
    const bool ok = f >= 0 && l >= f && l <= m && kb >= 0 && B0 >= kb && B0 <= nnz && rpf >= kb && rpf <= rpl &&
                    rpl <= nnz &&
                    (last ? (l == lend && rpl == nend && rpl == B0)
                          : (ovf >= 0 && ovf < kAlignRowMax && (!pre || ovf <= ocap)));
    if (!ok && tid == 0) atomicOr(a.err, 1);
    const int f0 = ok ? f : 0;
    const int nr = ok ? l - f : 0;
    const int nov = ok ? ovf : 0;
    const int A = ok ? rpf : kb, B = ok ? rpl : kb;
    if (DESC) {
        if (tid == 0) {
            int *o = dbg + 8 * t;
            o[0] = f0; o[1] = nr; o[2] = A; o[3] = B;
            o[4] = 0; o[5] = 0; o[6] = f; o[7] = l;
        }
        return;
    }

    const bool second = HALVES && blockIdx.x % kXcds >= kXcds / 2;  // the second half of x, rows into y2
    const int hx = (a.n + 1) / 2;
    const RowsDesc d{kb, B0, f0, nr, nov, A, B, min(nr + 1, S::kRpCap), second ? hx : 0, second ? a.n : hx};
    T xv[VPT][4], xo;
    int rr[S::kRpPer];
    rows_loads<T, K, PRIO, HALVES>(a, d, c, xv, ov, xo, rr, oc, pre);
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
    rows_stage<T, K, HALVES>(d, c, v, xv, oc, ov, xo, rr, s_prod, s_rp);
    lds_sync();
    if (second) a.y = a.y2;

    // y stores: device scope (written through to memory) in general, C2:
    // 55.25 instead of 55.6 us (fp64), 36.0 instead of 36.5 (fp32), 31.9
    // instead of 32.55 (fp16); non-temporal in the short-row mode, where y is
    // a sixth of the bytes and device scope took C4 from 320 to 357 us.
    rows_reduce<T, K, PRIO ? kAuxNt : kAuxDev>(a, d, s_prod, s_rp, L);
}

// ---- k_band: row-aligned steps with the x band staged in an LDS ring -------
//
// For row-aligned plans whose columns lie mostly within +-w of their own row
// (a banded matrix with outliers: C4's columns within +-4096 of the diagonal,
// 10% anywhere).  In k_rows every tile gathers its band from L1 / L2, one
// cache-line request per gather lane, and those requests bound the kernel.
// Here one workgroup of 1024 threads per CU walks a contiguous range of steps
// (about PFK_BAND_STEP nnz of whole rows each: `group` tiles of the plan's
// recorded row map) and keeps x[f - w, l + w) of its current step (rows
// [f, l)) in an LDS ring, x[c] at slot c mod PFK_BAND_RING.  Consecutive steps
// share most of their band, so between steps only the entries the next step
// adds are loaded (about as many as its rows): each band entry of x is read
// about once per workgroup, and a gather inside the window is an LDS read.
// Columns outside the window are gathered from memory.  Three steps are in
// flight: the col / val stream of step s + 2, the outside gathers, ring
// entries and row bounds of step s + 1, and the products and row sums of step
// s.  Every load is issued by every lane (a lane with nothing to read uses an
// offset the range check turns into zeros), so the compiler's wait counts
// stay exact across the pipeline.  Rows of at most kThreadMax nnz are summed
// by one lane in nnz order (bit-identical to spmv_serial), longer rows (at
// most PFK_ALIGN_ROW_MAX) by a wave.  The map is the plan's recorded one, or
// one k_row_map searched just before (a first call, or a plan that remembers
// no rows).
constexpr int kBandBS = 1024;
constexpr int kBandWaves = kBandBS / kWave;
constexpr int kBandPer = 5;                         // elements per thread: a step and its last row's overflow
constexpr int kBandSlots = kBandPer * kBandBS;
constexpr int kBandRing = PFK_BAND_RING;            // x entries in the ring
constexpr int kBandRp = 2 * kBandBS;                // row bounds staged per step (rows + 1)
constexpr int kBandExt = 2 * kBandBS;               // ring entries prefetched per step
constexpr int kBandList = kBandSlots / (kThreadMax + 1) + 1;  // rows longer than kThreadMax in a step, at most
static_assert(kBandSlots >= PFK_BAND_STEP + PFK_ALIGN_ROW_MAX, "a step's products fit its slots");

struct BandArgs {
    const int2 *__restrict__ map;  // the plan's row map: (first row, row_ptr there) of each tile, ntiles + 1
    int w;                         // band half width (columns)
    int group;                     // tiles of the map per step
    int nsteps;
    int per;                       // steps per workgroup
};

// A step: rows [f, l), nnz [A, B), and the window [lo, hi) of x the ring holds
// while it is processed.  Windows only move forward and span at most
// kBandRing entries, so the ring holds any window, and a window keeps the
// entries it shares with the one before.
struct BandStep {
    int f, l, A, B, lo, hi;
};

// Step s from the row map (s outside [begin, end): an empty step).  A map
// entry that does not describe whole rows of at most kBandSlots nnz sets the
// error flag and makes the step empty.
__device__ __forceinline__ BandStep band_step(const BandArgs &b, long long ntiles, int s, int begin, int end, int m,
                                              int nnz, int *err)
{
    BandStep d{0, 0, 0, 0, 0, 0};
    if (s < begin || s >= end)
        return d;
    const long long t0 = (long long)s * b.group;
    const long long t1 = min(t0 + b.group, ntiles);
    // scalar loads (through the constant address space, at wave-uniform addresses): they complete on a
    // counter of their own, so reading the map does not wait for the vector loads in flight
    typedef const int __attribute__((address_space(4))) cint;
    const auto smap = [&](long long t) {
        const unsigned long long q = reinterpret_cast<unsigned long long>(b.map + t);
        const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)q);  // each half unsigned (zero-extended)
        const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(q >> 32));
        const cint *e = (const cint *)(((unsigned long long)hi << 32) | (unsigned long long)lo);
        return make_int2(e[0], e[1]);
    };
    const int2 e0 = smap(t0), e1 = smap(t1);
    const bool ok = e0.x >= 0 && e0.x <= e1.x && e1.x <= m && e0.y >= 0 && e0.y <= e1.y && e1.y <= nnz &&
                    e1.y - e0.y <= kBandSlots;
    if (!ok) {
        if (threadIdx.x == 0) atomicOr(err, 1);
        return d;
    }
    d.f = e0.x;
    d.l = e1.x;
    d.A = e0.y;
    d.B = e1.y;
    return d;
}

// The window of step d after step p: x[f - w, l + w) clipped to [0, n), never
// behind p's window, and at most kBandRing entries (the lowest dropped).
__device__ __forceinline__ void band_window(BandStep &d, const BandStep &p, int n, int w)
{
    if (d.l == d.f) {  // no rows: keep the window
        d.lo = p.lo;
        d.hi = p.hi;
        return;
    }
    const long long hi = max(min((long long)d.l + w, (long long)n), (long long)p.hi);
    long long lo = max((long long)d.f - w, (long long)p.lo);
    lo = min(max(lo, 0LL), hi);
    lo = max(lo, hi - kBandRing);
    d.lo = (int)lo;
    d.hi = (int)hi;
}

template <typename T>
__device__ __forceinline__ void band_load_cv(const Args<T> &a, const BandStep &d, int (&c)[kBandPer],
                                             T (&v)[kBandPer])
{
    const int nq = d.B - d.A;
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(a.col + d.A, (long long)nq * 4);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.val + d.A, (long long)nq * (long long)sizeof(T));
#pragma unroll
    for (int k = 0; k < kBandPer; ++k) {
        const int q = k * kBandBS + (int)threadIdx.x;
        // col and val non-temporal, which most likely leaves more of the MALL to x for the outside gathers
        // (C4 269.1 -> 260.6 us with val so loaded, fp32 209.7 -> 203.4; row_ptr so loaded too: 263.2, 209.4)
        static_assert(sizeof(T) == 8 || sizeof(T) == 4, "fp64 / fp32");
        c[k] = (int)__builtin_amdgcn_raw_buffer_load_b32(rc, q * 4, 0, kAuxNt);
        if constexpr (sizeof(T) == 8)
            v[k] = __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b64(rv, q * 8, 0, kAuxNt));
        else
            v[k] = __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b32(rv, q * 4, 0, kAuxNt));
    }
}

// Inside step d's window: an LDS read; otherwise a gather from memory.
__device__ __forceinline__ bool band_in(int c, const BandStep &d)
{
    return (unsigned)(c - d.lo) < (unsigned)(d.hi - d.lo);
}

template <typename T>
__device__ __forceinline__ void band_gather_out(const Args<T> &a, const BandStep &d, const int (&c)[kBandPer],
                                                T (&xo)[kBandPer])
{
    const int nq = d.B - d.A;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc_full(a.x, (long long)a.n * (long long)sizeof(T));
#pragma unroll
    for (int k = 0; k < kBandPer; ++k) {
        const int q = k * kBandBS + (int)threadIdx.x;
        const bool g = q < nq && !band_in(c[k], d);
        xo[k] = buf_load(rx, g ? (uint32_t)c[k] * (uint32_t)sizeof(T) : kOob, (T *)nullptr);
    }
}

// y[i] of a step through a resource over its rows, non-temporal (y is not read again).
__device__ __forceinline__ void band_store(__amdgpu_buffer_rsrc_t r, int i, double v)
{
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, i * 8, 0, kAuxNt);
}

__device__ __forceinline__ void band_store(__amdgpu_buffer_rsrc_t r, int i, float v)
{
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned int, v), r, i * 4, 0, kAuxNt);
}

template <typename T>
__device__ __forceinline__ void band_row_bounds(const Args<T> &a, const BandStep &d, int (&rr)[2])
{
    const __amdgpu_buffer_rsrc_t r = make_rsrc(a.rp + d.f, (long long)min(d.l - d.f + 1, kBandRp) * 4);
    rr[0] = (int)__builtin_amdgcn_raw_buffer_load_b32(r, (int)threadIdx.x * 4, 0, 0);
    rr[1] = (int)__builtin_amdgcn_raw_buffer_load_b32(r, ((int)threadIdx.x + kBandBS) * 4, 0, 0);
}

// One step's registers in the pipeline: its descriptor, col / val, the
// outside gathers, the ring entries it adds ([e, e + ne), the first kBandExt
// of them prefetched) and its first kBandRp row bounds.  Three stages rotate
// by name (the loop is unrolled three times), so no register holding a load
// in flight is ever copied, which would wait for the load.
template <typename T>
struct BandStage {
    BandStep d;
    int c[kBandPer];
    T v[kBandPer];
    T xo[kBandPer];
    T xe[2];
    int e, ne;
    int rr[2];
};

// Step s + 2 into nn (col / val), step s + 1 in nx (outside gathers, ring
// entries, row bounds), and, with PROCESS, step s in cu summed.  The two
// iterations before a workgroup's first step run without PROCESS, so the
// pipeline fills with the loads in the order of every later iteration.
template <bool PROCESS, typename T>
__device__ __forceinline__ void band_iter(const Args<T> &a, const BandArgs &b, int s, int s0, int s1, T *s_ring,
                                          acc_t<T> *s_prod, int *s_rp, int *s_list, int &s_nlist,
                                          BandStage<T> &cu, BandStage<T> &nx, BandStage<T> &nn)
{
    using P = acc_t<T>;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int n = a.n;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc_full(a.x, (long long)n * (long long)sizeof(T));
    // ---- step s + 2: col / val
    nn.d = band_step(b, a.ntiles, s + 2, s0, s1, a.m, a.nnz, a.err);
    band_window(nn.d, nx.d, n, b.w);
    band_load_cv(a, nn.d, nn.c, nn.v);
    // the loads keep this order in every iteration (step s + 2's stream first), so the counted waits for
    // each step's loads are the same on every path into the loop
    __builtin_amdgcn_sched_barrier(0);
    // ---- step s + 1: outside gathers, the ring entries it adds, its row bounds
    band_gather_out(a, nx.d, nx.c, nx.xo);
    nx.e = max(cu.d.hi, nx.d.lo);
    nx.ne = nx.d.hi - nx.e;
    {
        const __amdgpu_buffer_rsrc_t re = make_rsrc(a.x + nx.e, (long long)min(nx.ne, kBandExt) * (long long)sizeof(T));
        nx.xe[0] = buf_load(re, (uint32_t)(tid * (int)sizeof(T)), (T *)nullptr);
        nx.xe[1] = buf_load(re, (uint32_t)((tid + kBandBS) * (int)sizeof(T)), (T *)nullptr);
    }
    band_row_bounds(a, nx.d, nx.rr);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (!PROCESS)
        return;

    // ---- step s: the ring entries it adds and its row bounds into LDS (every
    // read of the previous step's entries and bounds ended at its last barrier)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int i = j * kBandBS + tid;
        if (i < cu.ne) s_ring[(unsigned)(cu.e + i) % (unsigned)kBandRing] = cu.xe[j];
        s_rp[i] = cu.rr[j];
    }
    for (int c = cu.e + kBandExt + tid; c < cu.e + cu.ne; c += kBandBS)  // a window that moves further (rare)
        s_ring[(unsigned)c % (unsigned)kBandRing] = buf_load(rx, (uint32_t)c * (uint32_t)sizeof(T), (T *)nullptr);
    lds_sync();
    if (tid == 0) s_nlist = 0;  // every wave read the previous step's count before the barrier above
    // products: inside the window from the ring, outside from the gathers
    const BandStep d = cu.d;
    const int nq = d.B - d.A;
#pragma unroll
    for (int k = 0; k < kBandPer; ++k) {
        const int q = k * kBandBS + tid;
        // both values read, then one chosen (a choice between the two addresses would put xo in memory)
        const T xr = s_ring[(unsigned)cu.c[k] % (unsigned)kBandRing];
        const T xv = band_in(cu.c[k], d) ? xr : cu.xo[k];
        if (q < nq) s_prod[q] = P(cu.v[k]) * P(xv);
    }
    lds_sync();
    // row sums of rows [f, l): bounds from LDS, or from row_ptr past kBandRp - 1 rows
    const int nr = d.l - d.f;
    const __amdgpu_buffer_rsrc_t ry = make_rsrc(a.y + d.f, (long long)nr * (long long)sizeof(T));
    bool bad = false;
    const auto row = [&](int i, int ra, int rb) {
        ra -= d.A;
        rb -= d.A;
        if (ra < 0 || rb < ra || rb > nq) {  // row_ptr changed after planning: stay inside the step
            bad = true;
            ra = min(max(ra, 0), nq);
            rb = min(max(rb, ra), nq);
        }
        if (rb - ra <= kThreadMax) {
            P acc = P(0);
            for (int j = ra; j < rb; ++j)
                acc += s_prod[j];
            band_store(ry, i, T(acc));
        } else {
            // disjoint rows of over kThreadMax products: at most kBandList of them (more only with a row_ptr
            // changed after planning, whose rows were clamped above and are reported)
            const int k = atomicAdd(&s_nlist, 1);
            if (k < kBandList) {
                s_list[3 * k] = i;
                s_list[3 * k + 1] = ra;
                s_list[3 * k + 2] = rb;
            } else {
                bad = true;
            }
        }
    };
    const int nfast = min(nr, kBandRp - 1);
    for (int i = tid; i < nfast; i += kBandBS)  // bounds from LDS
        row(i, s_rp[i], s_rp[i + 1]);
    for (int i = nfast + tid; i < nr; i += kBandBS)  // a step of more rows (empty ones): bounds from row_ptr
        row(i, a.rp[d.f + i], a.rp[d.f + i + 1]);
    if (bad) atomicOr(a.err, 1);
    lds_sync();
    const int nl = min(s_nlist, kBandList);
    for (int k = wave; k < nl; k += kBandWaves) {
        const int i = s_list[3 * k], ra = s_list[3 * k + 1], rb = s_list[3 * k + 2];
        P acc = P(0);
        for (int j = ra + lane; j < rb; j += kWave)
            acc += s_prod[j];
        acc = wave_sum(acc);
        if (lane == 0) band_store(ry, i, T(acc));
    }
}

template <typename T>
__global__ __launch_bounds__(kBandBS) void k_band(Args<T> a, BandArgs b)
{
    __shared__ __attribute__((aligned(16))) T s_ring[kBandRing];
    __shared__ __attribute__((aligned(16))) acc_t<T> s_prod[kBandSlots];
    __shared__ int s_rp[kBandRp];
    __shared__ int s_list[3 * kBandList];
    __shared__ int s_nlist;
    const int s0 = (int)blockIdx.x * b.per;
    const int s1 = min(b.nsteps, s0 + b.per);
    if (s0 >= s1)
        return;  // whole workgroup
    // The pipeline fills with two iterations that only load (steps s0 and s0 + 1; the steps before s0 are
    // empty, with an empty window, so step s0 brings its whole window into the ring).  Steps past s1 are
    // empty too (no loads, no rows), so every trip of the loop runs three.
    BandStage<T> X{}, Y{}, Z{};
    band_iter<false>(a, b, s0 - 2, s0, s1, s_ring, s_prod, s_rp, s_list, s_nlist, Y, Z, X);
    band_iter<false>(a, b, s0 - 1, s0, s1, s_ring, s_prod, s_rp, s_list, s_nlist, Z, X, Y);
    for (int s = s0; s < s1; s += 3) {
        band_iter<true>(a, b, s, s0, s1, s_ring, s_prod, s_rp, s_list, s_nlist, X, Y, Z);
        band_iter<true>(a, b, s + 1, s0, s1, s_ring, s_prod, s_rp, s_list, s_nlist, Y, Z, X);
        band_iter<true>(a, b, s + 2, s0, s1, s_ring, s_prod, s_rp, s_list, s_nlist, Z, X, Y);
    }
}

// Planning statistic of the band kernel: out[i] = the nnz whose column lies
// within +-(64 << i) of their row, i < PFK_BAND_WIDTHS.  A thread per row
// (row-aligned plans: rows of at most PFK_ALIGN_ROW_MAX nnz).
// A sample: the rows of every PFK_BAND_SAMPLE-th block of kBS rows, spread over
// the whole matrix; out[PFK_BAND_WIDTHS] counts the sampled nnz.  The count
// only chooses w (the band kernel gives the same sums for any w), so a sample
// serves.  A workgroup per sampled block at a time: the block's row_ptr in
// LDS, then a thread per nnz (coalesced col loads, its row found by bisection
// in LDS), the counts reduced over the wave and the workgroup before a few
// global atomics per workgroup (at most kBandStatsWg workgroups).
constexpr int kBandStatsWg = 512;

__global__ __launch_bounds__(kBS) void k_band_stats(const int *__restrict__ rp, const int *__restrict__ col, int m,
                                                    unsigned long long *__restrict__ out)
{
    __shared__ int s_rp[kBS + 1];
    __shared__ unsigned int s_c[PFK_BAND_WIDTHS + 1];
    const int tid = threadIdx.x;
    if (tid <= PFK_BAND_WIDTHS) s_c[tid] = 0;
    unsigned int cnt[PFK_BAND_WIDTHS + 1];
#pragma unroll
    for (int i = 0; i <= PFK_BAND_WIDTHS; ++i) cnt[i] = 0;
    const long long nblk = ((long long)m + kBS - 1) / kBS;
    const long long nsamp = (nblk + PFK_BAND_SAMPLE - 1) / PFK_BAND_SAMPLE;
    for (long long sb = blockIdx.x; sb < nsamp; sb += gridDim.x) {  // workgroup-uniform
        const long long r0 = sb * PFK_BAND_SAMPLE * kBS;
        const int nr = (int)min((long long)kBS, (long long)m - r0);
        for (int i = tid; i <= nr; i += kBS) s_rp[i] = rp[r0 + i];  // row_ptr[r0, r0 + nr]
        __syncthreads();
        const int A = s_rp[0], B = s_rp[nr];
        for (int j = A + tid; j < B; j += kBS) {
            const int c = col[j];
            int lo = 0, hi = nr;  // s_rp[lo] <= j < s_rp[hi]: lo ends as the row of nnz j
            while (hi - lo > 1) {
                const int mid = (lo + hi) >> 1;
                if (s_rp[mid] <= j) lo = mid; else hi = mid;
            }
            const long long d = llabs((long long)c - (r0 + lo));
            cnt[PFK_BAND_WIDTHS] += 1u;
#pragma unroll
            for (int i = 0; i < PFK_BAND_WIDTHS; ++i) cnt[i] += d <= (64ll << i) ? 1u : 0u;
        }
        __syncthreads();  // s_rp is rewritten by the next block
    }
    const auto add = [](unsigned int x, unsigned int y) { return x + y; };
#pragma unroll
    for (int i = 0; i <= PFK_BAND_WIDTHS; ++i) {
        const unsigned int c = wave_reduce_u32(cnt[i], add);
        if ((tid & (kWave - 1)) == 0 && c) atomicAdd(&s_c[i], c);
    }
    __syncthreads();
    if (tid <= PFK_BAND_WIDTHS && s_c[tid]) atomicAdd(out + tid, (unsigned long long)s_c[tid]);
}

// ---- k_dense: dense rows by x windows staged in LDS (hybrid plans) -----------
//
// A dense row (at least the plan's dense_min nnz, columns sorted) sweeps all of
// x.  Summed tile by tile, each of its tiles drags its whole x span from L2
// into a CU's L1 for a few nnz per line.  Here a workgroup stages one window
// of win consecutive x entries (at most W, 64 KB) in LDS and sums, for each of
// at most G dense rows, the segment of the row whose columns fall in the
// window: x is read once per group of rows instead of once per row.  The
// windows are a multiple of 8 (pfk_dense_nwin) and the groups as even as they
// can be, and workgroup (window w, group g) is dealt so that each XCD takes a
// contiguous eighth of the windows (its x entries stay in its L2): every XCD
// does the same work.  Each (row, window) partial sum goes to part[row][w];
// k_dense_sum adds them up.  Segment bounds: MODE kFlatSearch finds them by a
// per-lane search of each row's columns and records them in seg; kFlatMemo
// reads them.  C5 (1000 rows of 50k-500k nnz, 280M nnz): 558 us against 742 us for
// the same rows in split-row tiles with the x-window schedule.  16 loads in
// flight per lane and 128 rows per workgroup were the best of U = 4-16 and
// G = 64-256 (C5 fp64 whole step 896-1015 us, fp32 598-942).

#ifndef PF_DENSE_G
#define PF_DENSE_G 128
#endif
#ifndef PF_DENSE_U
#define PF_DENSE_U 16
#endif
template <typename T>
struct DenseShape {
    // x window: 64 KB of LDS, at most 16384 columns (fp16 windows of 32768 columns halve the workgroups: one per
    // CU on C5, 640 us for k_dense against 470 for fp32)
    static constexpr int kW = sizeof(T) == 8 ? 8192 : 16384;
    static constexpr int kG = PF_DENSE_G;              // dense rows per workgroup
    static constexpr int kU = PF_DENSE_U;              // loads in flight per lane
    static_assert(kW == PFK_DENSE_WINDOW(sizeof(T) == 8 ? PF_F64 : sizeof(T) == 4 ? PF_F32 : PF_F16),
                  "window of the C ABI");
};

struct DenseArgs {
    const int *__restrict__ rows;  // dense rows, ascending
    int nd;
    int nwin;
    int ngroups;
    int win;                       // columns per window (at most kW), window w = [w win, (w + 1) win)
    int gsz;                       // dense rows per group (at most kG): the groups are as even as they can be
    int *__restrict__ seg;         // [nd][nwin + 1] first nnz of each window (recorded / read)
    void *__restrict__ part;       // [nd][nwin] partial sums (accumulation type)
};

// The segments of a wave's rows in window w, lane k holding [ms, me) of row
// i0 + kWaves k (k < nk; read by the recorded-bounds call, one load per lane,
// or found by the call that searches), streamed as one sequence of batches of
// U loads per lane, double buffered: the next batch (of the same row or the
// next one) is in flight while the current one is summed, so neither a row
// change nor a row's last partial batch leaves the wave without loads in
// flight.  Both calls sum through here, so they give the same sums bit for bit.
template <typename T>
__device__ __forceinline__ void dense_rows_stream(const Args<T> &a, const DenseArgs &d, const T *sx, int w, int c0,
                                                  int i0, int nk, int ms, int me)
{
    using P = acc_t<T>;
    // fp16: 4 consecutive nnz per lane and load (16-byte col, 8-byte val loads); a 2-byte val load per lane
    // would cover one line per wave (C5 fp16 670 us against 503 for split-row tiles)
    constexpr int V = sizeof(T) == 2 ? 4 : 1;
    constexpr int W = DenseShape<T>::kW, U = DenseShape<T>::kU / V;
    constexpr int B = kWave * U * V;  // nnz per batch
    const int lane = threadIdx.x & (kWave - 1);
    if (lane < nk && me == ms) static_cast<P *>(d.part)[(long long)(i0 + kWaves * lane) * d.nwin + w] = P(0);
    const uint64_t todo = __ballot(lane < nk && me > ms);
    int cA[U][V], cB[U][V];
    T vA[U][V], vB[U][V];
    P acc = P(0);
    // Batches start at the segment's first nnz rounded down to a multiple of 64,
    // so every 64-lane load covers whole 128-byte lines of col and val (a
    // segment starts anywhere; unaligned, a load touched one line more); the
    // lanes before the segment's start read the row's earlier nnz and add nothing.
    const int ma = ms & ~(kWave - 1);
    const auto issue = [&](int k, int j, int (&c)[U][V], T (&v)[U][V]) {
        const int s = __builtin_amdgcn_readlane(ma, k), e = __builtin_amdgcn_readlane(me, k);
        const __amdgpu_buffer_rsrc_t rc = make_rsrc(a.col + s, (long long)(e - s) * 4);
        const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.val + s, val_range_bytes<T>(e - s));
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if constexpr (V == 1)
                load1(rc, rv, j + u * kWave + lane, c[u][0], v[u][0]);
            else
                load4(rc, rv, j / 4 + u * kWave + lane, c[u], v[u]);
        }
    };
    const auto consume = [&](int k, int j, const int (&c)[U][V], const T (&v)[U][V]) {
        const int base = __builtin_amdgcn_readlane(ma, k);
        const int lead = __builtin_amdgcn_readlane(ms, k) - base;
        const int len = __builtin_amdgcn_readlane(me, k) - base;
#pragma unroll
        for (int u = 0; u < U; ++u) {  // no product for slots outside the segment (x may hold inf or NaN)
#pragma unroll
            for (int e = 0; e < V; ++e) {
                const T xv = sx[(c[u][e] - c0) & (W - 1)];  // the mask keeps every LDS read inside the window
                const int q = V == 1 ? j + u * kWave + lane : j + 4 * (u * kWave + lane) + e;
                if (q >= lead && q < len)
                    acc += P(v[u][e]) * P(xv);
            }
        }
        if (j + B >= len) {  // the row's last batch
            acc = wave_sum(acc);
            if (lane == 0) static_cast<P *>(d.part)[(long long)(i0 + kWaves * k) * d.nwin + w] = acc;
            acc = P(0);
        }
    };
    const auto advance = [&](int &k, int &j) {  // the batch after (k, j); false at the end
        const int len = __builtin_amdgcn_readlane(me, k) - __builtin_amdgcn_readlane(ma, k);
        j += B;
        if (j < len) return true;
        const uint64_t rest = todo & ~((2ull << k) - 1ull);
        if (!rest) return false;
        k = __ffsll((long long)rest) - 1;
        j = 0;
        return true;
    };
    if (!todo) return;
    int k = __ffsll((long long)todo) - 1, j = 0;
    issue(k, j, cA, vA);
    for (;;) {
        int k2 = k, j2 = j;
        bool more = advance(k2, j2);
        if (more) issue(k2, j2, cB, vB);
        consume(k, j, cA, vA);
        if (!more) break;
        k = k2;
        j = j2;
        more = advance(k2, j2);
        if (more) issue(k2, j2, cA, vA);
        consume(k, j, cB, vB);
        if (!more) break;
        k = k2;
        j = j2;
    }
}

// The recorded-bounds call: lane k reads the bounds of row i0 + kWaves k.
template <typename T>
__device__ __forceinline__ void dense_rows_recorded(const Args<T> &a, const DenseArgs &d, const T *sx, int w,
                                                    int c0, int i0, int nk)
{
    const int lane = threadIdx.x & (kWave - 1);
    const int nnz = a.nnz;
    int ms = 0, me = 0;
    if (lane < nk) {
        const int *sg = d.seg + (long long)(i0 + kWaves * lane) * (d.nwin + 1) + w;
        ms = min(max(sg[0], 0), nnz);
        me = min(max(sg[1], ms), nnz);
    }
    dense_rows_stream<T>(a, d, sx, w, c0, i0, nk, ms, me);
}

// One lane's lower_bound(v) over col[a, b) (sorted): a first round of 8
// probes `sp` apart around `guess`, then 8-ary rounds inside the bracket.
// Every probe lies in [a, b), and the loop ends for any data (each round
// leaves at most an eighth of the bracket).
__device__ __forceinline__ int lane_lower_bound(const int *__restrict__ col, int a, int b, int v, int guess, int sp)
{
    int lo = a - 1, hi = b;  // col[lo] < v, col[hi] >= v, both virtual at the ends
    {
        int k[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const long long p = (long long)guess + (long long)(i - 4) * sp;
            k[i] = (p >= a && p < b) ? col[(int)p] : 0;
        }
        int nlo = lo, nhi = hi;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const long long p = (long long)guess + (long long)(i - 4) * sp;
            if (p >= a && p < b) {
                if (k[i] < v) nlo = max(nlo, (int)p);
                else nhi = min(nhi, (int)p);
            }
        }
        if (nlo < nhi) { lo = nlo; hi = nhi; }  // (columns out of order: keep the whole row)
    }
    while (hi - lo > 1) {
        const int step = (hi - lo + 7) >> 3;
        int k[7];
#pragma unroll
        for (int i = 1; i < 8; ++i) {
            const int p = lo + i * step;
            k[i - 1] = p < hi ? col[p] : 0;
        }
        int c = 0;
#pragma unroll
        for (int i = 1; i < 8; ++i)
            c += (lo + i * step < hi && k[i - 1] < v) ? 1 : 0;
        const int nlo = lo + c * step;
        hi = min(nlo + step, hi);
        lo = nlo;
    }
    return hi;
}

// The call that searches (kFlatSearch): lane k finds the segment of row
// i0 + kWaves k in window w itself, the 32 rows side by side (a row's place
// for column c guessed as c * len / n past its start, the rows' columns being
// spread over [0, n)), records it when the plan keeps bounds, and the wave
// sums the segments exactly as the recorded-bounds call does.
template <typename T>
__device__ __forceinline__ void dense_rows_searched(const Args<T> &a, const DenseArgs &d, const T *sx, int w,
                                                    int c0, int i0, int nk)
{
    const int W = d.win;
    const int lane = threadIdx.x & (kWave - 1);
    const int nnz = a.nnz;
    int ms = 0, me = 0;
    if (lane < nk) {
        const int i = i0 + kWaves * lane;
        const int r = d.rows[i];
        if (r < 0 || r >= a.m) {  // a table entry that is not a row: an empty segment, reported
            atomicOr(a.err, 1);
        } else {
            const int a0 = min(max(a.rp[r], 0), nnz);
            const int a1 = min(max(a.rp[r + 1], a0), nnz);
            const int len = a1 - a0;
            const int sp = (int)max(1.0, ceil(sqrt((double)len) / 4.0));
            const auto guess = [&](int v) {
                const double place = a.n > 0 ? (double)v * ((double)len / (double)a.n) : 0.0;
                return a0 + (int)fmin(fmax(place, 0.0), (double)max(len - 1, 0));
            };
            const int ce = (int)min((long long)c0 + W, (long long)a.n);  // the window's end, at most n
            ms = lane_lower_bound(a.col, a0, a1, c0, guess(c0), sp);
            me = lane_lower_bound(a.col, a0, a1, ce, guess(ce), sp);
            if (d.seg) {
                int *sg = d.seg + (long long)i * (d.nwin + 1);
                sg[w] = ms;
                if (w == d.nwin - 1) sg[d.nwin] = me;
            }
        }
    }
    dense_rows_stream<T>(a, d, sx, w, c0, i0, nk, ms, me);
}

template <typename T, int MODE>
__global__ __launch_bounds__(kBS) void k_dense(Args<T> a, DenseArgs d)
{
    constexpr int W = DenseShape<T>::kW, G = DenseShape<T>::kG;
    __shared__ __attribute__((aligned(16))) T sx[W];
    const int tid = threadIdx.x, wave = tid / kWave;
    const int xcd = blockIdx.x % kXcds, q = blockIdx.x / kXcds;
    const int wper = (d.nwin + kXcds - 1) / kXcds;
    const int w = xcd * wper + q % wper, g = q / wper;
    if (w >= d.nwin || g >= d.ngroups)
        return;
    const int c0 = (int)min((long long)w * d.win, (long long)a.n);  // a window past n holds no column
    const int i_end = min(d.nd, (g + 1) * d.gsz);
    {  // the window x[c0, c0 + win) into LDS, 16 bytes per lane and load; zeros past n
        const long long have = max(0LL, min((long long)d.win, (long long)a.n - c0));
        // fp16: whole dwords (the range check drops a half-covered one; the extra entry is past n, never read)
        const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + (have > 0 ? c0 : 0), val_range_bytes<T>((int)have));
        constexpr int kPer = 16 / (int)sizeof(T);
        const int nv = min(d.win, W) / kPer;
#pragma unroll 4
        for (int i = tid; i < nv; i += kBS)
            *reinterpret_cast<u32x4 *>(sx + i * kPer) = __builtin_amdgcn_raw_buffer_load_b128(rx, i * 16, 0, 0);
    }
    lds_sync();
    static_assert(G / kWaves <= kWave, "one lane per row of a wave");
    const int i0 = g * d.gsz + wave;
    const int nk = i0 < i_end ? (i_end - i0 + kWaves - 1) / kWaves : 0;
    if constexpr (MODE == kFlatMemo)
        dense_rows_recorded<T>(a, d, sx, w, c0, i0, nk);
    else
        dense_rows_searched<T>(a, d, sx, w, c0, i0, nk);
}

// y of each dense row from its window partial sums: one wave per row, lane j
// adding windows j, j + 64, ... in order, then the wave's DPP tree (a fixed
// order: deterministic).  One thread per row walking 123 windows took 34 us
// on C5; a wave per row takes a few.
template <typename T>
__device__ __forceinline__ void dense_sum_row(const Args<T> &a, const DenseArgs &d, int i, int lane)
{
    using P = acc_t<T>;
    if (i >= d.nd)
        return;  // whole wave
    const int r = d.rows[i];
    if (r < 0 || r >= a.m)
        return;  // whole wave
    const P *pp = static_cast<const P *>(d.part) + (long long)i * d.nwin;
    P sum = P(0);
    for (int w = lane; w < d.nwin; w += kWave)
        sum += pp[w];
    sum = wave_sum(sum);
    if (lane == 0) a.y[r] = T(sum);
}

template <typename T>
__global__ __launch_bounds__(kBS) void k_dense_sum(Args<T> a, DenseArgs d)
{
    dense_sum_row<T>(a, d, blockIdx.x * kWaves + (int)threadIdx.x / kWave, threadIdx.x & (kWave - 1));
}

// Planning scan of a hybrid plan: every row of at least `dmin` nnz goes to the
// list as (row, row_ptr[row], row_ptr[row + 1]) (in no particular order; the
// host sorts it), and counters[1] counts the decreasing column pairs inside
// the listed rows (a hybrid plan needs sorted columns).
__global__ __launch_bounds__(kBS) void k_dense_scan(const int *__restrict__ rp, int m, int dmin, int *__restrict__ list,
                                                    int cap, int *__restrict__ counters)
{
    for (long long r = (long long)blockIdx.x * kBS + threadIdx.x; r < m; r += (long long)gridDim.x * kBS) {
        const int a0 = rp[r], a1 = rp[r + 1];
        if (a1 - a0 >= dmin) {
            const int k = atomicAdd(counters, 1);
            if (k < cap) {
                list[3 * k] = (int)r;
                list[3 * k + 1] = a0;
                list[3 * k + 2] = a1;
            }
        }
    }
}

__global__ __launch_bounds__(kBS) void k_dense_sorted(const int *__restrict__ col, const int *__restrict__ list,
                                                      int cap, int *__restrict__ counters)
{
    const int nk = min(cap, counters[0]);
    int bad = 0;
    for (int k = blockIdx.y; k < nk; k += gridDim.y) {
        const int a0 = list[3 * k + 1], a1 = list[3 * k + 2];
        for (long long j = a0 + (long long)blockIdx.x * kBS + threadIdx.x; j + 1 < a1; j += (long long)gridDim.x * kBS)
            bad += col[j] > col[j + 1];
    }
    if (__ballot(bad != 0) && (threadIdx.x & (kWave - 1)) == 0)
        atomicAdd(counters + 1, 1);
}

// ---- k_long: long rows of a hybrid plan in long mode -------------------------
//
// A matrix whose long rows (over PFK_ALIGN_ROW_MAX nnz) are not all dense rows
// with sorted columns (a power-law matrix, C3) keeps its short rows in the
// row-aligned runs and cuts each long row into tiles of kLongTile nnz.  One
// workgroup sums one tile: each lane its 4 elements of the wave-strided
// layout in order, then the wave's DPP tree, then the 4 waves in order, one
// partial per tile; k_long_sum adds a row's partials in tile order, so the
// result is deterministic.  The host deals the tiles to the 8 XCDs by their
// first column, XCD k taking the k-th eighth: with sorted columns each XCD
// then gathers from about an eighth of x, which stays in its L2.  A tile's
// loads start at a multiple of 64 nnz (whole lines); its slots before the
// row's first nnz or past its end add nothing.
constexpr int kLongTile = PFK_LONG_TILE;
static_assert(kLongTile == 4 * kBS, "one 4-element group of the wave-strided layout per lane");

struct LongArgs {
    const int4 *__restrict__ tiles;  // (row index, first nnz loaded, first nnz of the row, end)
    const int *__restrict__ deal;
    const int *__restrict__ row_tiles;
    const int *__restrict__ rows;
    int nrows, ntiles;
    void *__restrict__ part;
};

template <typename T>
__global__ __launch_bounds__(kBS) void k_long(Args<T> a, LongArgs L)
{
    using P = acc_t<T>;
    __shared__ P s_red[kWaves];
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int per = (L.ntiles + kXcds - 1) / kXcds;
    const int q = (int)(blockIdx.x / kXcds);
    const int slot = (int)(blockIdx.x % kXcds) * per + q;
    if (q >= per || slot >= L.ntiles)
        return;  // whole workgroup: padding of the XCD deal
    const int t = L.deal[slot];
    if (t < 0 || t >= L.ntiles) {  // a deal entry that is not a tile: skip it, report it (whole workgroup)
        if (tid == 0) atomicOr(a.err, 1);
        return;
    }
    const int4 d = L.tiles[t];
    const int nnz = a.nnz;
    const int s = min(max(d.y, 0), nnz);                // first nnz loaded
    const int e = min(max(d.w, s), min(nnz, s + kLongTile));
    const int lo = min(max(d.z, s), e) - s;             // slots before lo belong to the row before
    const int len = e - s;
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(a.col + s, (long long)len * 4);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.val + s, (long long)len * (long long)sizeof(T));
    const __amdgpu_buffer_rsrc_t rx = make_rsrc_full(a.x, (long long)a.n * (long long)sizeof(T));
    int c[4];
    T v[4], xv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        load1(rc, rv, tile_elem<T>(0, j), c[j], v[j]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int qj = tile_elem<T>(0, j);
        xv[j] = buf_load(rx, qj >= lo && qj < len ? (uint32_t)c[j] * (uint32_t)sizeof(T) : kOob, (T *)nullptr);
    }
    P acc = P(0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // no product for slots outside the row (x may hold inf or NaN)
        const int qj = tile_elem<T>(0, j);
        if (qj >= lo && qj < len)
            acc += P(v[j]) * P(xv[j]);
    }
    acc = wave_sum(acc);
    if (lane == 0) s_red[wave] = acc;
    lds_sync();
    if (tid == 0) {
        P tot = s_red[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w)
            tot += s_red[w];
        static_cast<P *>(L.part)[t] = tot;
    }
}

// y of each long row from its tiles' partials: one wave per row, lane j adding
// tiles j, j + 64, ... in order, then the wave's DPP tree (a fixed order).
template <typename T>
__device__ __forceinline__ void long_sum_row(const Args<T> &a, const LongArgs &L, int i, int lane)
{
    using P = acc_t<T>;
    if (i >= L.nrows)
        return;  // whole wave
    const int r = L.rows[i];
    if (r < 0 || r >= a.m) {  // a table entry that is not a row (whole wave)
        if (lane == 0) atomicOr(a.err, 1);
        return;
    }
    const int b0 = min(max(L.row_tiles[i], 0), L.ntiles);
    const int b1 = min(max(L.row_tiles[i + 1], b0), L.ntiles);
    const P *pp = static_cast<const P *>(L.part);
    P sum = P(0);
    for (int t = b0 + lane; t < b1; t += kWave)
        sum += pp[t];
    sum = wave_sum(sum);
    if (lane == 0) a.y[r] = T(sum);
}

template <typename T>
__global__ __launch_bounds__(kBS) void k_long_sum(Args<T> a, LongArgs L)
{
    long_sum_row<T>(a, L, blockIdx.x * kWaves + (int)threadIdx.x / kWave, threadIdx.x & (kWave - 1));
}

// Hybrid plans with x halves: y = (first half's row sum) + (second half's),
// in that order.  The first hblocks workgroups form y = y + y2 over the rows
// not summed apart (apart[r] == 0), and the others combine the rows summed
// apart, one wave per row, as k_dense_sum (LONG false) or k_long_sum (LONG
// true) do; neither part writes the other's rows, so one launch does both.
// A row summed apart whose apart byte is not 1 would be written by both parts:
// the combining wave skips it and sets the error flag.
template <typename T, bool LONG>
__global__ __launch_bounds__(kBS) void k_combine(Args<T> a, DenseArgs d, LongArgs L,
                                                 const unsigned char *__restrict__ apart, int hblocks)
{
    if ((int)blockIdx.x < hblocks) {
        for (long long r = (long long)blockIdx.x * kBS + threadIdx.x; r < a.m; r += (long long)hblocks * kBS)
            if (!apart[r]) a.y[r] = T(acc_t<T>(a.y[r]) + acc_t<T>(a.y2[r]));
        return;
    }
    const int i = ((int)blockIdx.x - hblocks) * kWaves + (int)threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    if (i >= (LONG ? L.nrows : d.nd))
        return;  // whole wave
    const int r = LONG ? L.rows[i] : d.rows[i];
    if (r >= 0 && r < a.m && apart[r] != 1) {  // whole wave
        if (lane == 0) atomicOr(a.err, 1);
        return;
    }
    if constexpr (LONG)
        long_sum_row<T>(a, L, i, lane);
    else
        dense_sum_row<T>(a, d, i, lane);
}

// flags[rows[i]] = 1 for every listed row inside the flags (planning).
__global__ __launch_bounds__(kBS) void k_mark_rows(const int *__restrict__ rows, int count,
                                                   unsigned char *__restrict__ flags, long long nflags)
{
    for (long long i = (long long)blockIdx.x * kBS + threadIdx.x; i < count; i += (long long)gridDim.x * kBS) {
        const int r = rows[i];
        if (r >= 0 && r < nflags) flags[r] = 1;
    }
}

// Planning of long-row tiles: out[i] = col[idx[i]] (-1 for an index outside [0, nnz)).
__global__ __launch_bounds__(kBS) void k_gather_cols(const int *__restrict__ col, long long nnz,
                                                     const int *__restrict__ idx, int count, int *__restrict__ out)
{
    for (long long i = (long long)blockIdx.x * kBS + threadIdx.x; i < count; i += (long long)gridDim.x * kBS) {
        const int k = idx[i];
        out[i] = k >= 0 && k < nnz ? col[k] : -1;
    }
}

// ---- k_flow: FLAT tiles of 256 nnz with carried row sums ------------------
//
// Every wave64 walks a run of consecutive 256-nnz tiles (one 4-nnz vector per
// lane).  A row that crosses a tile edge carries its partial sum in a register
// into the next tile, continuing the sum in nnz order (rows of <= 16 nnz stay
// bit-identical to the serial sum); only rows crossing a run edge leave
// partials in head / tail slots for k_fixup (runs of R tiles = R*256 nnz).
// Rows belong to the tile holding their first nnz (empty rows: the tile
// holding nnz row_ptr[r]; trailing empty rows: the last tile).  Only a run's
// first tile searches row_ptr; later tiles scan forward from the previous end.
// Pipelining as in k_wave: while tile t is reduced, col/val of t+1 and the
// row_ptr block of t+1 are in flight.

constexpr int kFlowT = 256;                            // nnz per tile
constexpr int kFlowRB = 3 * kWave;                     // row_ptr entries per block
constexpr int kFlowLC = kFlowT / (kThreadMax + 1) + 2; // long pieces per tile

// Row r's piece goes to y[r]; kFlowCarry: the row continuing into the next tile.
constexpr int kFlowCarry = -1;

template <typename T>
__global__ __launch_bounds__(kWaveWG) void k_flow(Args<T> a)
{
    constexpr int NW = kWaveWG / kWave;
    __shared__ __attribute__((aligned(16))) T s_prod_all[NW][kFlowT];
    __shared__ int s_rp_all[NW][kFlowRB];
    __shared__ int s_la_all[NW][kFlowLC], s_lb_all[NW][kFlowLC], s_ld_all[NW][kFlowLC];
    __shared__ T s_cout_all[NW][1];

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    T *s_prod = s_prod_all[wave];
    int *s_rp = s_rp_all[wave];
    int *s_la = s_la_all[wave], *s_lb = s_lb_all[wave], *s_ld = s_ld_all[wave];
    T *s_cout = s_cout_all[wave];

    const long long xcd = blockIdx.x % kXcds;
    const long long wx = (blockIdx.x / kXcds) * NW + wave;  // run index inside its XCD
    if (wx >= a.tx)
        return;
    const long long u = xcd * a.tx + wx;  // run
    const long long t_begin = u * a.tpw;
    long long t_end = t_begin + a.tpw;
    if (t_end > a.ntiles) t_end = a.ntiles;
    if (t_begin >= t_end)
        return;

    const int m = a.m, nnz = a.nnz;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc_full(a.x, (long long)a.n * (long long)sizeof(T));
    const __amdgpu_buffer_rsrc_t ry = make_rsrc_full(a.y, (long long)m * (long long)sizeof(T));
    const __amdgpu_buffer_rsrc_t rrp = make_rsrc_full(a.rp, ((long long)m + 1) * 4);
    const __amdgpu_buffer_rsrc_t rhead = make_rsrc_full(a.head, a.ntiles * (long long)sizeof(T));
    const __amdgpu_buffer_rsrc_t rtail = make_rsrc_full(a.tail, a.ntiles * (long long)sizeof(T));
    const __amdgpu_buffer_rsrc_t rowner = make_rsrc_full(a.owner, a.ntiles * 4);

    // row_ptr block: lane holds entries F + lane + 64 q (entries past m read 0 and are never used).
    auto load_block = [&](int F, int (&rr)[3]) {
#pragma unroll
        for (int q = 0; q < 3; ++q)
            rr[q] = (int)__builtin_amdgcn_raw_buffer_load_b32(rrp, (F + q * kWave + lane) * 4, 0, 0);
    };
    // col/val of tile t (16-byte loads; lanes past the tile read zeros).
    int c[4];
    T v[4];
    auto issue_cv = [&](long long t) {
        const int A = (int)(t * kFlowT);
        const int B = min(A + kFlowT, nnz);
        const __amdgpu_buffer_rsrc_t rc = make_rsrc(a.col + A, (long long)(B - A) * 4);
        const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.val + A, (long long)(B - A) * (long long)sizeof(T));
        load4(rc, rv, lane, c, v);
    };

    // First row of the run's first tile: rows [0, F) start before its nnz A0.
    const int A0 = (int)(t_begin * kFlowT);
    int F = wave_search_lt<false>(a.rp, m, (uint32_t)A0, key_guess<false>((uint32_t)A0, m, nnz), a.guess_spread,
                                  lane) + 1;
    int rr[3];
    load_block(F, rr);
    issue_cv(t_begin);
    // A row started before A0 and ending after it continues into the run.
    int c_row = -1;
    bool c_in_run = false;
    T c_sum = T(0);
    {
        const int rpF = rlane(rr[0], 0);
        if (F > 0 && rpF > A0) c_row = F - 1;
    }

    for (long long t = t_begin;; ++t) {
        const int A = (int)(t * kFlowT);
        const int B = min(A + kFlowT, nnz);
        const bool last = t == a.ntiles - 1;
        const int len_t = B - A;

        // Rows starting in this tile: [F, Fn).
#pragma unroll
        for (int q = 0; q < 3; ++q) s_rp[q * kWave + lane] = rr[q];
        int Fn;
        if (last) {
            Fn = m;
        } else {
            int j = -1;
#pragma unroll
            for (int q = 2; q >= 0; --q) {
                const int idx = q * kWave + lane;
                const uint64_t mask = __ballot(F + idx > m || rr[q] >= B);
                if (mask) j = q * kWave + __ffsll((long long)mask) - 1;
            }
            Fn = j >= 0 ? F + j
                        : wave_search_lt<false>(a.rp, m, (uint32_t)B, key_guess<false>((uint32_t)B, m, nnz), 0, lane) + 1;
        }
        const int nr = Fn - F;
        const int rpF = rlane(rr[0], 0);  // row_ptr[F] (== nnz when F == m)

        // x gathers of this tile, then the next tile's loads.
        T xv[4];
        T vt[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const bool in = lane * 4 + j < len_t;
            xv[j] = buf_load(rx, in ? (uint32_t)c[j] * (uint32_t)sizeof(T) : kOob, (T *)nullptr);
            vt[j] = v[j];
        }
        const bool more = t + 1 < t_end;
        if (more) {
            load_block(Fn, rr);
            issue_cv(t + 1);
        }
        {
            T p[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) p[j] = vt[j] * xv[j];
            store4(s_prod + 4 * lane, p);
        }
        __builtin_amdgcn_wave_barrier();

        int nl = 0;
        // The row carried in from the previous tile: piece [A, min(row_ptr[F], B)).
        if (c_row >= 0) {
            const int cend = min(rpF, B);
            const int clen = cend - A;
            if (clen <= kThreadMax) {
                T s = c_sum;
                for (int q = 0; q < clen; ++q) s += s_prod[q];
                c_sum = s;  // every lane computes the same sum (uniform loop)
            } else {
                T s = T(0);
                for (int q = lane; q < clen; q += kWave) s += s_prod[q];
                c_sum = c_sum + wave_sum(s);
            }
            if (rpF <= B) {  // the row ends in this tile
                if (c_in_run) buf_store(ry, lane == 0 ? (uint32_t)c_row * (uint32_t)sizeof(T) : kOob, c_sum);
                else buf_store(rhead, lane == 0 ? (uint32_t)u * (uint32_t)sizeof(T) : kOob, c_sum);
                c_row = -1;
            }
        }
        // Rows starting here, one lane each; pieces of more than 16 products are listed.
        const int rpFn = nr < kFlowRB ? s_rp[nr] : a.rp[Fn];  // row_ptr[Fn]: end of the last row starting here
        const bool cont = nr > 0 && !last && rpFn > B;
        for (int q0 = 0; q0 < nr; q0 += kWave) {
            const int i = q0 + lane;
            const bool valid = i < nr;
            int ra = 0, rbf = 0;
            if (valid) {
                ra = i < kFlowRB ? s_rp[i] : a.rp[F + i];
                rbf = i + 1 < kFlowRB ? s_rp[i + 1] : a.rp[F + i + 1];
            }
            const int rb = min(rbf, B);
            const int len = rb - ra;
            const bool is_cont = cont && i == nr - 1;
            T s = T(0);
            bool lng = false;
            if (valid) {
                if (len <= kThreadMax) {
                    for (int q = ra - A; q < rb - A; ++q) s += s_prod[q];
                    if (is_cont) s_cout[0] = s;
                } else {
                    lng = true;
                }
            }
            const uint64_t mask = __ballot(lng);
            if (mask) {
                const int pos = nl + (int)__builtin_amdgcn_mbcnt_hi((unsigned)(mask >> 32),
                                                                     __builtin_amdgcn_mbcnt_lo((unsigned)mask, 0u));
                if (lng && pos < kFlowLC) {
                    s_la[pos] = ra - A;
                    s_lb[pos] = rb - A;
                    s_ld[pos] = is_cont ? kFlowCarry : F + i;
                }
                nl += __popcll(mask);
            }
            buf_store(ry, valid && !lng && !is_cont ? (uint32_t)(F + i) * (uint32_t)sizeof(T) : kOob, s);
        }
        __builtin_amdgcn_wave_barrier();
        if (nl > kFlowLC) {
            nl = kFlowLC;  // cannot happen: at most 256/17 pieces exceed 16 products
            atomicOr(a.err, 1);
        }
        for (int j = 0; j < nl; ++j) {
            T s = T(0);
            const int e1 = s_lb[j];
            for (int q = s_la[j] + lane; q < e1; q += kWave) s += s_prod[q];
            s = wave_sum(s);
            const int dst = s_ld[j];
            if (dst == kFlowCarry) {
                if (lane == 0) s_cout[0] = s;
            } else {
                buf_store(ry, lane == 0 ? (uint32_t)dst * (uint32_t)sizeof(T) : kOob, s);
            }
        }
        __builtin_amdgcn_wave_barrier();
        if (cont) {  // the last row starting here continues into the next tile
            c_row = F + nr - 1;
            c_sum = s_cout[0];
            c_in_run = true;
        }
        if (!more)
            break;
        F = Fn;
    }
    // Run end: the row leaving the run (if any) and its partial.
    const uint32_t uslot = (uint32_t)u * (uint32_t)sizeof(T);
    const bool leaving = c_row >= 0;
    buf_store(rtail, lane == 0 && leaving && c_in_run ? uslot : kOob, c_sum);
    buf_store(rhead, lane == 0 && leaving && !c_in_run ? uslot : kOob, c_sum);
    buf_store(rowner, lane == 0 ? (uint32_t)u * 4u : kOob, leaving && c_in_run ? c_row : -1);
}

// Debug: the descriptor every tile of k_tiles computes.
template <bool MERGE, int K, int LMAX, int SPAN_MAX>
__global__ __launch_bounds__(kBS) void k_tile_desc(Args<double> a, int *__restrict__ out)
{
    __shared__ int s_rows[2];
    const long long t = xcd_tile(a.xch);
    if (t >= a.ntiles)
        return;
    uint32_t kb, ke;
    bool last;
    tile_keys<MERGE>(t, a.ntiles, K, a.m, a.nnz, kb, ke, last);
    search_tile_rows<MERGE>(a.rp, a.m, a.nnz, a.guess_spread, kb, ke, last, s_rows);
    __syncthreads();
    if (threadIdx.x == 0) {
        const TileDesc d = make_desc<MERGE, LMAX, SPAN_MAX>(a.rp, a.m, a.nnz, kb, ke, s_rows[0],
                                                            s_rows[1], a.err);
        int *o = out + 8 * t;
        o[0] = d.lo_row; o[1] = d.nr; o[2] = d.A; o[3] = d.B; o[4] = d.head; o[5] = d.tail;
        o[6] = s_rows[0]; o[7] = s_rows[1];
    }
}

// ---- k_fixup: combine the partials of split rows in tile order -------------

// One thread per tile: a split row that ends within kFixSerial tiles of the
// tile where it starts is summed by that thread, head slots in tile order; a
// longer one is listed and summed by a wave (lane-strided partials, DPP sum).
// Both orders are fixed functions of the tiling, so y is reproducible.
constexpr int kFixSerial = 16;

template <typename T, bool MERGE>
__global__ __launch_bounds__(kBS) void k_fixup(Args<T> a, int K)
{
    __shared__ int s_list[kBS];
    __shared__ int s_n;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    if (tid == 0) s_n = 0;
    __syncthreads();
    const long long t0 = (long long)blockIdx.x * kBS;
    const long long t = t0 + tid;
    int r = t < a.ntiles ? a.owner[t] : -1;
    if (r >= a.m) {  // an owner outside the matrix: report, never dereference
        atomicOr(a.err, 1);
        r = -1;
    }
    if (r >= 0) {
        const long long last_key = (long long)a.rp[r + 1] - 1 + (MERGE ? r : 0);
        long long tb = last_key / K;  // last tile holding a piece of row r
        if (tb >= a.ntiles) { atomicOr(a.err, 1); tb = a.ntiles - 1; }
        if (tb - t <= kFixSerial) {
            acc_t<T> s = 0;
            for (long long u = t + 1; u <= tb; ++u)
                s += a.head[u];
            a.y[r] = T(a.tail[t] + s);
        } else {
            s_list[atomicAdd(&s_n, 1)] = tid;
        }
    }
    __syncthreads();
    const int n = s_n;
    for (int j = wave; j < n; j += kWaves) {
        const long long tl = t0 + s_list[j];
        const int rl = a.owner[tl];  // validated above (listed only when 0 <= rl < m)
        long long tb = ((long long)a.rp[rl + 1] - 1 + (MERGE ? rl : 0)) / K;
        if (tb >= a.ntiles) tb = a.ntiles - 1;
        acc_t<T> s = 0;
        for (long long u = tl + 1 + lane; u <= tb; u += kWave)
            s += a.head[u];
        s = wave_sum(s);
        if (lane == 0)
            a.y[rl] = T(a.tail[tl] + s);
    }
}

// ---- k_row_map: a row-aligned plan's row map, searched afresh --------------
//
// Entry t (0 <= t <= ntiles) of a row-aligned plan's row map is (f, row_ptr[f])
// with f the first row whose row_ptr is at or above v = t * K (entry 0: row 0;
// entry ntiles: row m), what k_rows's search records.  The band kernel reads
// its steps from the map and cannot search: a band plan's first call, and
// every call of one that remembers no rows, runs this kernel before it.
// A group of kMapLanes lanes per entry, so that every entry's search is in
// flight at once (C4: 24,416 entries, 6,104 waves): the first round probes
// kMapLanes rows around the plan's interpolated guess, 4 x guess_spread apart
// (the span k_rows's 64 probes cover), each later round kMapLanes rows evenly
// inside the bracket left, which it cuts about 17-fold.  The bracket
// (lo, hi] always holds the answer: row_ptr[lo] < v <= row_ptr[hi], lo = -1
// standing for "below every row"; probes are non-decreasing in the lane, so
// the lanes whose row_ptr lies below v are the group's lowest.
constexpr int kMapLanes = 16;

__global__ __launch_bounds__(kBS) void k_row_map(const int *__restrict__ rp, int m, int nnz, int K, long long ntiles,
                                                 int spread, double ga, double gb, int2 *__restrict__ map)
{
    const long long t = ((long long)blockIdx.x * kBS + threadIdx.x) / kMapLanes;
    const int lane = (int)(threadIdx.x & (kWave - 1));
    const int q = lane & (kMapLanes - 1);
    const int base = lane - q;  // the group's first lane in the wave
    const bool search = t > 0 && t < ntiles;  // whole groups
    const uint32_t v = search ? (uint32_t)(t * K) : 0u;
    int lo = -1, hi = m;
    int khi = (t <= ntiles) ? rp[m] : 0;  // row_ptr[hi], issued beside the first round
    // first round: around the guess
    const double g = ga > 0.0 ? ga * (double)v + gb : (nnz > 0 ? (double)v * ((double)m / (double)nnz) : 0.0);
    const long long gc = (long long)fmin(fmax(g, 0.0), (double)m);  // (NaN: 0)
    const long long step0 = 4LL * max(spread, 1);
    int p = (int)min(max(gc + (long long)(q - kMapLanes / 2) * step0, 0LL), (long long)m);
    int k = search ? rp[p] : 0;
    for (;;) {
        const unsigned below = (unsigned)(__ballot(search && k < (int)v) >> base) & ((1u << kMapLanes) - 1);
        const int nb = __popc(below);  // probes below v: lanes 0 .. nb - 1 of the group
        const int plo = __shfl(p, base + max(nb - 1, 0));
        const int phi = __shfl(p, base + min(nb, kMapLanes - 1));
        const int khn = __shfl(k, base + min(nb, kMapLanes - 1));
        if (search) {
            if (nb > 0) lo = max(lo, plo);
            if (nb < kMapLanes && phi < hi) { hi = phi; khi = khn; }
        }
        if (!__ballot(search && hi - lo > 1))
            break;
        // kMapLanes probes evenly inside (lo, hi), the last at most hi - 1
        const int step = hi - lo > 1 ? (hi - lo + kMapLanes) / (kMapLanes + 1) : 1;
        p = search && hi - lo > 1 ? (int)min((long long)lo + (long long)(q + 1) * step, (long long)hi - 1) : max(lo, 0);
        k = search && hi - lo > 1 ? rp[p] : 0;
    }
    if (q == 0 && t <= ntiles) {
        if (t == 0)
            map[0] = make_int2(0, rp[0]);
        else
            map[t] = search ? make_int2(hi, khi) : make_int2(m, khi);
    }
}

// ---- k_vector: row groups (FLAT "tiles" 2..32) — small matrices -----------
//
// For a matrix small enough that its SpMV is a few dependent memory round trips
// (C1: 65k nnz), the tiles' machinery (row map, LDS staging, per-row sums from
// LDS) is latency on the critical path.  Here row g belongs to the g-th group
// of L lanes (256 / L rows per workgroup, by index: no tiles, no search): lane
// q sums products a + q, a + q + L, ... of its row in order, the group's DPP /
// swizzle tree adds the L lane sums, and the group's first lane stores y.
// Every index is clamped to the matrix: a row_ptr changed after planning reads
// in bounds.  C1 in a HIP graph: 1.85 us per SpMV with L = 16 against 3.50 for
// 1024-nnz tiles (2.49 in a launch loop against 2.73 for rocSPARSE's row split).
template <typename T, int L>
__global__ __launch_bounds__(kBS) void k_vector(Args<T> a)
{
    using P = acc_t<T>;
    static_assert(L >= 2 && L <= 32 && (L & (L - 1)) == 0, "a power of two group inside a 32-lane half");
    const long long g = ((long long)blockIdx.x * kBS + threadIdx.x) / L;
    const int q = threadIdx.x & (L - 1);
    if (g >= a.m)
        return;  // whole groups (L divides the workgroup), so every group below is whole
    const int nnz = a.nnz;
    const int r0 = min(max(a.rp[g], 0), nnz);
    const int r1 = min(max(a.rp[g + 1], r0), nnz);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc_full(a.x, (long long)a.n * (long long)sizeof(T));
    P s = P(0);
    for (int j = r0 + q; j < r1; j += L)
        s += P(a.val[j]) * P(buf_load(rx, (uint32_t)a.col[j] * (uint32_t)sizeof(T), (T *)nullptr));
    s = group_sum<L>(s);
    if (q == 0) a.y[g] = T(s);
}

// ---- k_prefree: the reference kernel's algorithm on wave64 -----------------

constexpr int kPfBS = 128;  // preFreeSpMV.cu:583

// Lane 0 of each 32-lane half receives the tree sum that warpReduceSum over a
// 32-lane warp (offsets 16,8,4,2,1) gives, preFreeSpMV.cu:49-53.
template <typename T>
__device__ __forceinline__ T half_wave_tree(T v)
{
    v += swizzle<swizzle_xor_pattern<16>()>(v);
    v += swizzle<swizzle_xor_pattern<8>()>(v);
    v += swizzle<swizzle_xor_pattern<4>()>(v);
    v += swizzle<swizzle_xor_pattern<2>()>(v);
    v += swizzle<swizzle_xor_pattern<1>()>(v);
    return v;
}

template <typename T>
__device__ __forceinline__ void atomic_add(T *p, T v) { atomicAdd(p, v); }

// Sum over the aligned groups of V lanes of each 32-lane half, as lane 0 of a
// group sees the reference's warpReduceSum<V> (__shfl_down_sync offsets V/2 ..
// 1, preFreeSpMV.cu:100-114): an xor tree from the largest offset down gives
// lane 0 the same additions in the same order.
template <int V, typename T>
__device__ __forceinline__ T group_tree32(T v)
{
    if constexpr (V >= 32) v += swizzle<swizzle_xor_pattern<16>()>(v);
    if constexpr (V >= 16) v += swizzle<swizzle_xor_pattern<8>()>(v);
    if constexpr (V >= 8) v += swizzle<swizzle_xor_pattern<4>()>(v);
    if constexpr (V >= 4) v += dpp<kDppXor2>(v);
    if constexpr (V >= 2) v += dpp<kDppXor1>(v);
    return v;
}

// One tile of the reference algorithm: products in LDS, rows [start, end).
// Products and sums in acc_t<T> (fp32 in the fp16 mode).
template <typename T, int TT>
struct PfTile {
    using A = acc_t<T>;
    const A *s;
    const int *__restrict__ rp;
    T *__restrict__ y;
    int first, start, end;
    A *__restrict__ head;  // fp16: the partial of row start, of row end - 1 (tail), slot `tile`
    A *__restrict__ tail;
    long long tile;

    __device__ __forceinline__ void range(int r, int &lo, int &hi) const
    {
        lo = max(0, rp[r] - first);
        hi = min(TT, rp[r + 1] - first);
    }
    // A tile-boundary row's partial sum: atomicAdd to y (preFreeSpMV.cu:92-96,
    // :139-146); fp16 keeps it in fp32 for k_prefree_join, which adds a row's
    // partials in tile order and rounds to half once.
    __device__ __forceinline__ void shared(int r, A v) const
    {
        if constexpr (__is_same(T, half_t))
            (r == start ? head : tail)[tile] = v;
        else
            atomic_add(y + r, v);
    }
    // Interior rows are stored.
    __device__ __forceinline__ void put(int r, A v) const
    {
        if (r == start || r == end - 1)
            shared(r, v);
        else
            y[r] = T(v);
    }
};

// red_row_thread (preFreeSpMV.cu:71-98): one thread per row, in nnz order.
template <typename T, int TT>
__device__ __forceinline__ void pf_red_thread(const PfTile<T, TT> &t)
{
    for (int r = t.start + (int)threadIdx.x; r < t.end; r += kPfBS) {
        int lo, hi;
        t.range(r, lo, hi);
        acc_t<T> sum = 0;
        for (int i = lo; i < hi; ++i)
            sum += t.s[i];
        t.put(r, sum);
    }
}

// red_row_block (:30-69): strided lane sums, a 32-lane tree per half wave,
// then the four half-wave results summed in order by thread 0.
template <typename T, int TT>
__device__ __forceinline__ void pf_red_block(const PfTile<T, TT> &t, acc_t<T> *s_warp)
{
    const int tid = threadIdx.x;
    int lo, hi;
    t.range(t.start, lo, hi);
    acc_t<T> v = 0;
    for (int j = lo + tid; j < hi; j += kPfBS)
        v += t.s[j];
    v = half_wave_tree(v);
    if ((tid & 31) == 0)
        s_warp[tid >> 5] = v;
    __syncthreads();
    if (tid == 0) {
        acc_t<T> fin = 0;
#pragma unroll
        for (int w = 0; w < kPfBS / 32; ++w)
            fin += s_warp[w];
        t.shared(t.start, fin);
    }
}

// red_row_vector<VS> (:116-150): groups of VS lanes per row, lane 0 of the
// group ends with warpReduceSum<VS>'s tree.
template <int VS, typename T, int TT>
__device__ __forceinline__ void pf_red_vector(const PfTile<T, TT> &t)
{
    const int g = threadIdx.x / VS, q = threadIdx.x % VS;
    for (int r = t.start + g; r < t.end; r += kPfBS / VS) {
        int lo, hi;
        t.range(r, lo, hi);
        acc_t<T> v = 0;
        for (int i = lo + q; i < hi; i += VS)
            v += t.s[i];
        v = group_tree32<VS>(v);
        if (q == 0)
            t.put(r, v);
    }
}

// is_imbalanced_warp (:342-373): among the first 32 rows of the range, the
// longest (whole row length) holds more than 90% of their nnz, compared in
// float as there.  Integer sums and maxima are exact in any order.
template <typename T, int TT>
__device__ __forceinline__ bool pf_imbalanced(const PfTile<T, TT> &t, int *s_flag)
{
    const int tid = threadIdx.x;
    const int n = t.end - t.start;
    if (tid < 32) {
        const int len = tid < n ? t.rp[t.start + tid + 1] - t.rp[t.start + tid] : 0;
        int tot = len, mx = len;
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) {
            tot += __shfl_down(tot, o, 32);
            mx = max(mx, __shfl_down(mx, o, 32));
        }
        if (tid == 0) {
            const float dominance = 0.9f;
            *s_flag = (n > 1 && tot > 0 && (float)mx > (float)tot * dominance) ? 1 : 0;
        }
    }
    __syncthreads();
    return *s_flag != 0;
}

// red_row_long_short_specialized<96> (:152-340), for 2 <= n <= 32 rows: the
// longest row (a shfl_down max-with-index tree over whole row lengths; a tie
// keeps the lane's own index) is summed by threads 0..95 in stride 96 with a
// 32-lane tree per warp and one more tree over the three warp sums; threads
// 96..127 sum the other rows one each, left to right.  Rows whose sum is 0.0
// are not written (:326; y is zeroed before the launch).
template <typename T, int TT>
__device__ __forceinline__ void pf_red_long_short(const PfTile<T, TT> &t, acc_t<T> *s_final, acc_t<T> *s_warp,
                                                  int *s_li)
{
    using A = acc_t<T>;
    constexpr int kLong = 96;
    const int tid = threadIdx.x;
    const int n = t.end - t.start;
    if (tid < 32) {
        int len = -1;
        if (tid < n) {
            len = t.rp[t.start + tid + 1] - t.rp[t.start + tid];
            s_final[tid] = A(0);
        }
        int ml = len, mi = tid;
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) {
            const int rl = __shfl_down(ml, o, 32);
            const int ri = __shfl_down(mi, o, 32);
            if (rl > ml) { ml = rl; mi = ri; }
        }
        if (tid == 0) *s_li = mi;
    }
    __syncthreads();
    const int li = *s_li;
    if (tid < kLong) {
        int lo, hi;
        t.range(t.start + li, lo, hi);
        A v = A(0);
        for (int j = lo + tid; j < hi; j += kLong)
            v += t.s[j];
        v = half_wave_tree(v);
        if ((tid & 31) == 0)
            s_warp[tid >> 5] = v;
    } else {
        for (int i = tid - kLong; i < n; i += kPfBS - kLong) {
            if (i == li)
                continue;
            int lo, hi;
            t.range(t.start + i, lo, hi);
            const A *sp = t.s + lo;
            A sum = A(0);
            switch (hi - lo) {  // left to right, as the unrolled cases of :293-313
            case 0: break;
            case 1: sum = sp[0]; break;
            case 2: sum = sp[0] + sp[1]; break;
            case 3: sum = sp[0] + sp[1] + sp[2]; break;
            case 4: sum = sp[0] + sp[1] + sp[2] + sp[3]; break;
            default:
                for (int k = lo; k < hi; ++k)
                    sum += t.s[k];
                break;
            }
            s_final[i] = sum;
        }
    }
    __syncthreads();
    if (tid < 32) {
        A v = tid < kLong / 32 ? s_warp[tid] : A(0);
        v = half_wave_tree(v);
        if (tid == 0)
            s_final[li] = v;
    }
    __syncthreads();
    if (tid < n) {
        const A fs = s_final[tid];
        if (fs != A(0))
            t.put(t.start + tid, fs);
    }
}

// calculate_vector_size<128> (:394-405).
__device__ __forceinline__ int pf_vector_size(int n)
{
    if (n >= kPfBS)
        return 2;
    const unsigned avg = (unsigned)kPfBS / (unsigned)n;
    const unsigned p2 = 1u << (31 - __clz((int)avg));
    return (int)min(32u, max(2u, p2));
}

// The reference kernel preFreeSpMV_kernel<P, 128> (:407-561) with reduction
// ladder CODE, the tuner's TEST_CODE_VERSION (scripts/profile_and_generate.py:
// 109-235): 1 thread per row always (:440-446); 2 block for a single row, else
// thread (:448-461); 3 thread above 32 rows, block for one, else vector<4>
// (:466-483, the active ladder); 4 as 3 with the long/short split for
// imbalanced tiles (:485-511); 5 thread above 128 rows, block for one, else
// vector<calculate_vector_size> (:513-559).  The tile's first row (the
// pre-pass map, :3-28) is searched in the kernel.
template <typename T, int P, int CODE>
__global__ __launch_bounds__(kPfBS) void k_prefree(Args<T> a)
{
    using A = acc_t<T>;
    constexpr int TT = kPfBS * P;  // 512 nnz for P = 4 (preFreeSpMV.cu:587), 1024 for P = 8
    constexpr int VPT = P / 4;     // 4-nnz vectors per lane
    constexpr bool F16 = __is_same(T, half_t);
    __shared__ __attribute__((aligned(16))) A s_prod[TT];
    __shared__ int s_rows[2];
    __shared__ A s_warp[kPfBS / 32];
    __shared__ A s_final[32];
    __shared__ int s_flag, s_li;

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const long long b = xcd_tile(a.xch);
    if (b >= a.ntiles)
        return;
    const int m = a.m;
    if (F16 && tid == 0) {  // a boundary row this tile leaves unwritten adds zero (ordered by the barrier below)
        a.head[b] = A(0);
        a.tail[b] = A(0);
    }

    // First row of this tile and of the next one (the pre-pass map, :3-28).
    const uint32_t first = (uint32_t)(b * TT);
    if (wave == 0) {
        const int r = wave_search_lt<false>(a.rp, m, first + 1u, key_guess<false>(first, m, a.nnz),
                                            a.guess_spread, lane);
        if (lane == 0) s_rows[0] = r;
    } else {
        const bool last = b + 1 >= a.ntiles;
        const int r = last ? m
                           : wave_search_lt<false>(a.rp, m, first + TT + 1u,
                                                   key_guess<false>(first + TT, m, a.nnz), a.guess_spread, lane);
        if (lane == 0) s_rows[1] = r;
    }

    // Product stage (:416-428): 16-byte buffer loads of this tile's nnz and x
    // through a range-checked resource; positions past nnz give zero products.
    const int tile_nnz = min(TT, a.nnz - (int)first);
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(a.col + first, (long long)tile_nnz * 4);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.val + first, val_range_bytes<T>(tile_nnz));
    const __amdgpu_buffer_rsrc_t rx = make_rsrc_full(a.x, (long long)a.n * (long long)sizeof(T));
    int c[VPT][4];
    T v[VPT][4];
#pragma unroll
    for (int k = 0; k < VPT; ++k)
        load4(rc, rv, tid + k * kPfBS, c[k], v[k]);
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int off = 4 * (tid + k * kPfBS);
        A p[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            p[j] = A(v[k][j]) * A(buf_load(rx, off + j < tile_nnz ? (uint32_t)c[k][j] * (uint32_t)sizeof(T) : kOob,
                                           (T *)nullptr));
        store4(s_prod + off, p);
    }
    __syncthreads();

    // Row range (:429-438); the last tile ends at m.
    const int start = min(s_rows[0], m);
    int end = min(s_rows[1], m);
    if (a.rp[end] % TT != 0 || end == start)
        end = min(end + 1, m);
    const int nrows = end - start;
    const PfTile<T, TT> t{s_prod, a.rp, a.y, (int)first, start, end, a.head, a.tail, b};
    if (F16 && tid == 0) {  // the row range, for k_prefree_join
        a.owner[2 * b] = start;
        a.owner[2 * b + 1] = end;
    }

    if constexpr (CODE == 1) {
        pf_red_thread(t);
    } else if constexpr (CODE == 2) {
        if (nrows == 1) pf_red_block(t, s_warp);
        else pf_red_thread(t);
    } else if constexpr (CODE == 3) {
        if (nrows > kPfBS / 4) pf_red_thread(t);
        else if (nrows == 1) pf_red_block(t, s_warp);
        else pf_red_vector<4>(t);
    } else if constexpr (CODE == 4) {
        if (nrows > kPfBS / 4) pf_red_thread(t);
        else if (nrows == 1) pf_red_block(t, s_warp);
        else if (pf_imbalanced(t, &s_flag)) pf_red_long_short(t, s_final, s_warp, &s_li);
        else pf_red_vector<4>(t);
    } else {
        static_assert(CODE == 5, "ladder codes 1..5");
        if (nrows > kPfBS) {
            pf_red_thread(t);
        } else if (nrows == 1) {
            pf_red_block(t, s_warp);
        } else if (nrows > 0) {
            switch (pf_vector_size(nrows)) {
            case 32: pf_red_vector<32>(t); break;
            case 16: pf_red_vector<16>(t); break;
            case 8: pf_red_vector<8>(t); break;
            case 4: pf_red_vector<4>(t); break;
            default: pf_red_vector<2>(t); break;
            }
        }
    }
}

// fp16: the tile-boundary rows of k_prefree<half_t>.  One wave per tile b; a
// row shared by tiles b, b+1, ... (its partials in their head or tail slots) is
// summed by the wave of the first of them, 64 tiles per round (a DPP tree per
// round, the rounds in tile order), in fp32, and stored to y rounded to half
// once.  ranges[b] = (start, end) of tile b's rows.
__global__ __launch_bounds__(kBS) void k_prefree_join(const int *__restrict__ ranges, const float *__restrict__ head,
                                                      const float *__restrict__ tail, long long ntiles,
                                                      half_t *__restrict__ y)
{
    const int lane = threadIdx.x & (kWave - 1);
    const long long b = (long long)blockIdx.x * (kBS / kWave) + threadIdx.x / kWave;
    if (b >= ntiles)
        return;  // whole wave
    const int s0 = ranges[2 * b], e0 = ranges[2 * b + 1];
    const int sp = b > 0 ? ranges[2 * b - 2] : -1, ep = b > 0 ? ranges[2 * b - 1] : -1;
    if (e0 <= s0)
        return;
    for (int which = 0; which < 2; ++which) {
        const int r = which == 0 ? s0 : e0 - 1;
        if (which == 1 && r == s0)
            break;  // a single row: one partial
        if (b > 0 && ep > sp && (r == sp || r == ep - 1))
            continue;  // an earlier tile's wave sums it
        float acc = 0.f;
        for (long long t0 = b; t0 < ntiles; t0 += kWave) {
            const long long t = t0 + lane;
            bool mem = false;
            float v = 0.f;
            if (t < ntiles) {
                const int st = ranges[2 * t], et = ranges[2 * t + 1];
                mem = et > st && (r == st || r == et - 1);
                if (mem) v = r == st ? head[t] : tail[t];
            }
            const uint64_t mm = __ballot(mem);
            const int run = mm == ~0ull ? kWave : __ffsll((long long)~mm) - 1;  // the tiles sharing r from t0 on
            acc += wave_sum(lane < run ? v : 0.f);
            if (run < kWave)
                break;
        }
        if (lane == 0) y[r] = (half_t)acc;
    }
}

// Debug: the first row of every tile as k_prefree finds it; out[ntiles] = m.
__global__ __launch_bounds__(kWave) void k_prefree_rows(const int *__restrict__ rp, int m, int nnz, int tile,
                                                        long long ntiles, int spread, int *__restrict__ out)
{
    const long long b = blockIdx.x;
    const int lane = threadIdx.x;
    if (b > ntiles)
        return;
    int r = m;
    if (b < ntiles) {
        const uint32_t first = (uint32_t)(b * tile);
        r = wave_search_lt<false>(rp, m, first + 1u, key_guess<false>(first, m, nnz), spread, lane);
    }
    if (lane == 0)
        out[b] = r;
}

// ---- gather probe: the x-gather ceiling (measurement only, not an SpMV path) --
//
// One workgroup per 1024 indices, as a 1024-nnz FLAT tile: each lane streams
// 4 indices with one 16-byte non-temporal load (the way col is streamed) and
// gathers x at them through a resource over x with cache policy AUX; each
// wave stores one sum, so the gathers cannot be dropped and the stores cost
// next to nothing.  Run over a matrix's own column indices, it gives the time
// the x gathers of its SpMV take with nothing else in flight.

constexpr int kProbeTile = 1024;

template <int AUX>
__device__ __forceinline__ double probe_load(__amdgpu_buffer_rsrc_t r, uint32_t off, double *)
{
    return __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, AUX));
}

template <int AUX>
__device__ __forceinline__ float probe_load(__amdgpu_buffer_rsrc_t r, uint32_t off, float *)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, AUX));
}

template <typename T, int AUX>
__global__ __launch_bounds__(kBS) void k_probe_gather(const int *__restrict__ idx, long long count,
                                                      const T *__restrict__ x, long long n, T *__restrict__ out)
{
    const long long t = blockIdx.x;
    const long long kb = t * kProbeTile;
    const long long rest = count - kb;
    const int len = (int)(rest < kProbeTile ? rest : kProbeTile);
    const __amdgpu_buffer_rsrc_t ri = make_rsrc(idx + kb, (long long)len * 4);
    const u32x4 cc = __builtin_amdgcn_raw_buffer_load_b128(ri, (int)threadIdx.x * 16, 0, kAuxNt);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc_full(x, n * (long long)sizeof(T));
    const int base = 4 * (int)threadIdx.x;
    const unsigned c[4] = {cc.x, cc.y, cc.z, cc.w};
    T s = T(0);
#pragma unroll
    for (int j = 0; j < 4; ++j)
        s += probe_load<AUX>(rx, base + j < len ? c[j] * (uint32_t)sizeof(T) : kOob, (T *)nullptr);
    s = wave_sum(s);
    if ((threadIdx.x & (kWave - 1)) == 0) out[t * kWaves + threadIdx.x / kWave] = s;
}

// ---- statistics, fills -----------------------------------------------------

// Layout of the statistics block (unsigned long long):
enum StatSlot {
    kStMax = 0, kStMin = 1, kStEmpty = 2, kStDec = 3, kStFirst = 4, kStLast = 5, kStBadCol = 6,
    kStHist = 7, kStOverAlign = 40, kStMaxShort = 41, kStGuessDev = 42, kStLineQ1 = 43, kStLineQ3 = 44,
    kStLineFar = 45,
    // planning scan only (pfk_plan_scan): long rows appended to its list, column descents found inside them,
    // and a flag set when the descents could not all be checked
    kStLongListed = 46, kStLongDesc = 47, kStLongUnchecked = 48, kStCount = 49
};
static_assert(kStCount <= PFK_STATS_WORDS, "statistics block of the C ABI");

__global__ void k_stats_init(unsigned long long *out)
{
    const int i = threadIdx.x;
    if (i < kStCount)
        out[i] = (i == kStMin) ? ~0ull : 0ull;
}

// Row statistics; with a list (the planning scan), every row over
// PFK_ALIGN_ROW_MAX nnz is also appended to it as (row, first nnz, end, 0),
// the first `cap` of them (out[kStLongListed] counts them all).
constexpr int kStatsBS = 1024;  // k_row_stats: workgroups of 16 waves
constexpr int kStatsRows = 8;   // rows per group: row_ptr[r0, r0 + 8] as two 16-byte loads and one 4-byte load
constexpr int kStatsGroups = 1; // groups per lane and pass (4, with their loads in flight together: C4 56 -> 87 us)
constexpr int kStatsBins = 8;   // histogram bins a lane counts in registers (rows of under 128 nnz)

// Each workgroup takes a contiguous range of rows; its lanes read row_ptr in
// groups of kStatsRows rows, kStatsGroups groups per pass (the workgroup's
// passes are uniform, so it can synchronise inside them).  Every statistic is
// reduced over the wave before it meets LDS, and over the workgroup before it
// meets memory.  The long rows of a pass are listed with one global atomic per
// workgroup pass (the list's counter is the one address every workgroup meets).
__global__ __launch_bounds__(kStatsBS) void k_row_stats(const int *__restrict__ rp, int m,
                                                        unsigned long long *__restrict__ out,
                                                        int4 *__restrict__ list, int cap)
{
    constexpr int kWaves = kStatsBS / kWave;
    __shared__ unsigned int s_hist[33];
    __shared__ unsigned int s_max, s_min, s_empty, s_dec, s_over, s_short, s_dev, s_far;
    __shared__ unsigned int s_wsum[kWaves];
    __shared__ unsigned long long s_lbase;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    if (tid < 33) s_hist[tid] = 0;
    if (tid == 0) {
        s_max = 0; s_min = 0xFFFFFFFFu; s_empty = 0; s_dec = 0; s_over = 0; s_short = 0; s_dev = 0; s_far = 0;
    }
    __syncthreads();
    unsigned int lmax = 0, lmin = 0xFFFFFFFFu, lempty = 0, ldec = 0, lover = 0, lshort = 0, lfar = 0;
    unsigned int hc[kStatsBins];
#pragma unroll
    for (int i = 0; i < kStatsBins; ++i) hc[i] = 0;
    // distance in rows between row r and where the matrix's mean density puts row_ptr[r] (the row
    // searches' first guess), largest over the rows; 0 when row_ptr[m] is not positive
    const int total = rp[m];
    const double per_nnz = total > 0 ? (double)m / (double)total : 0.0;
    double ldev = 0.0;
    // rows more than 28 rows from the line through (row_ptr[m / 4], m / 4) and (row_ptr[3m / 4], 3m / 4), the
    // row-aligned tiles' alternative first guess (every row counts when the line is undefined)
    const int q1 = m / 4, q3 = (int)(3LL * m / 4);
    const int p1 = m >= 4 ? rp[q1] : 0, p3 = m >= 4 ? rp[q3] : 0;
    const bool line = m >= 4 && p3 > p1;
    const double la = line ? (double)(q3 - q1) / ((double)p3 - (double)p1) : 0.0;
    const double lb = line ? (double)q1 - la * (double)p1 : 0.0;
    const long long per = (((long long)m + gridDim.x - 1) / gridDim.x + kStatsRows - 1) / kStatsRows * kStatsRows;
    const long long rb = min((long long)m, (long long)blockIdx.x * per);
    const long long re = min((long long)m, rb + per);
    // row_ptr[rb, re]: entries past it read zeros (only for rows past re, which are skipped)
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(rp + rb, re > rb ? (re - rb + 1) * 4 : 0);
    const int ng = (int)((re - rb + kStatsRows - 1) / kStatsRows);
    for (int gb = 0; gb < ng; gb += kStatsGroups * kStatsBS) {  // the same passes for every thread
        u32x4 v0[kStatsGroups], v1[kStatsGroups];
        int v8[kStatsGroups];
#pragma unroll
        for (int q = 0; q < kStatsGroups; ++q) {  // groups past the range read zeros (and are skipped)
            const int g = gb + tid + q * kStatsBS;
            v0[q] = __builtin_amdgcn_raw_buffer_load_b128(rr, g * 32, 0, kAuxNt);
            v1[q] = __builtin_amdgcn_raw_buffer_load_b128(rr, g * 32 + 16, 0, kAuxNt);
            v8[q] = (int)__builtin_amdgcn_raw_buffer_load_b32(rr, g * 32 + 32, 0, 0);
        }
        unsigned int nlong = 0;  // this lane's rows over PFK_ALIGN_ROW_MAX in this pass
#pragma unroll
        for (int q = 0; q < kStatsGroups; ++q) {
            const int g = gb + tid + q * kStatsBS;
            const int e[kStatsRows + 1] = {(int)v0[q].x, (int)v0[q].y, (int)v0[q].z, (int)v0[q].w,
                                           (int)v1[q].x, (int)v1[q].y, (int)v1[q].z, (int)v1[q].w, v8[q]};
            const double rd0 = (double)(rb + (long long)g * kStatsRows);  // exact: rows are below 2^31
#pragma unroll
            for (int i = 0; i < kStatsRows; ++i) {
                const long long r = rb + (long long)g * kStatsRows + i;
                if (r < re) {
                    const double rd = rd0 + (double)i;
                    if (total > 0) ldev = fmax(ldev, fabs(rd - (double)e[i] * per_nnz));
                    lfar += !line || fabs(rd - (la * (double)e[i] + lb)) > 28.0;
                    int len = e[i + 1] - e[i];
                    if (len < 0) { ++ldec; len = 0; }
                    const unsigned int u = (unsigned int)len;
                    lmax = max(lmax, u);
                    lmin = min(lmin, u);
                    lempty += (u == 0);
                    nlong += (u > (unsigned)PFK_ALIGN_ROW_MAX);
                    if (u <= (unsigned)PFK_ALIGN_ROW_MAX) lshort = max(lshort, u);
                    const int bin = u == 0 ? 0 : 32 - __clz(u);
                    if (bin < kStatsBins) {
#pragma unroll
                        for (int k = 0; k < kStatsBins; ++k) hc[k] += bin == k ? 1u : 0u;
                    } else {
                        atomicAdd(&s_hist[bin], 1u);  // rows of 128 nnz or more
                    }
                }
            }
        }
        lover += nlong;
        if (list && __syncthreads_or(nlong > 0)) {
            // this pass's long rows: an exclusive scan of the lanes' counts over the workgroup, one global atomic
            unsigned int incl = nlong;
#pragma unroll
            for (int o = 1; o < kWave; o <<= 1) {
                const unsigned int t = (unsigned int)__shfl_up((int)incl, o);
                incl += lane >= o ? t : 0u;
            }
            if (lane == kWave - 1) s_wsum[wave] = incl;
            __syncthreads();
            if (tid == 0) {
                unsigned int run = 0;
                for (int w = 0; w < kWaves; ++w) {
                    const unsigned int c = s_wsum[w];
                    s_wsum[w] = run;
                    run += c;
                }
                s_lbase = atomicAdd(out + kStLongListed, (unsigned long long)run);
            }
            __syncthreads();
            unsigned long long k = s_lbase + s_wsum[wave] + (incl - nlong);
#pragma unroll
            for (int q = 0; q < kStatsGroups; ++q) {
                const int g = gb + tid + q * kStatsBS;
                const int e[kStatsRows + 1] = {(int)v0[q].x, (int)v0[q].y, (int)v0[q].z, (int)v0[q].w,
                                               (int)v1[q].x, (int)v1[q].y, (int)v1[q].z, (int)v1[q].w, v8[q]};
#pragma unroll
                for (int i = 0; i < kStatsRows; ++i) {
                    const long long r = rb + (long long)g * kStatsRows + i;
                    const int len = e[i + 1] - e[i];
                    if (r < re && len > PFK_ALIGN_ROW_MAX) {
                        if (k < (unsigned long long)cap) list[k] = make_int4((int)r, e[i], e[i + 1], 0);
                        ++k;
                    }
                }
            }
            __syncthreads();  // s_wsum and s_lbase are read before the next pass writes them
        }
    }
    const auto add = [](unsigned int x, unsigned int y) { return x + y; };
    const auto mx = [](unsigned int x, unsigned int y) { return max(x, y); };
    const auto mn = [](unsigned int x, unsigned int y) { return min(x, y); };
#pragma unroll
    for (int k = 0; k < kStatsBins; ++k) {
        const unsigned int c = wave_reduce_u32(hc[k], add);
        if (lane == 0 && c) atomicAdd(&s_hist[k], c);
    }
    lmax = wave_reduce_u32(lmax, mx);
    lmin = wave_reduce_u32(lmin, mn);
    lempty = wave_reduce_u32(lempty, add);
    ldec = wave_reduce_u32(ldec, add);
    lover = wave_reduce_u32(lover, add);
    lshort = wave_reduce_u32(lshort, mx);
    lfar = wave_reduce_u32(lfar, add);
    const unsigned int udev = wave_reduce_u32((unsigned int)fmin(ceil(ldev), 4294967295.0), mx);
    if (lane == 0) {
        atomicMax(&s_max, lmax);
        atomicMin(&s_min, lmin);
        atomicAdd(&s_empty, lempty);
        atomicAdd(&s_dec, ldec);
        atomicAdd(&s_over, lover);
        atomicMax(&s_short, lshort);
        atomicMax(&s_dev, udev);
        atomicAdd(&s_far, lfar);
    }
    __syncthreads();
    if (tid < 33 && s_hist[tid]) atomicAdd(out + kStHist + tid, (unsigned long long)s_hist[tid]);
    if (tid == 0) {
        atomicMax(out + kStMax, (unsigned long long)s_max);
        atomicMin(out + kStMin, (unsigned long long)s_min);
        if (s_empty) atomicAdd(out + kStEmpty, (unsigned long long)s_empty);
        if (s_dec) atomicAdd(out + kStDec, (unsigned long long)s_dec);
        if (s_over) atomicAdd(out + kStOverAlign, (unsigned long long)s_over);
        atomicMax(out + kStMaxShort, (unsigned long long)s_short);
        atomicMax(out + kStGuessDev, (unsigned long long)s_dev);
        if (s_far) atomicAdd(out + kStLineFar, (unsigned long long)s_far);
        if (blockIdx.x == 0) {
            out[kStFirst] = (unsigned long long)(long long)rp[0];
            out[kStLast] = (unsigned long long)(long long)rp[m];
            out[kStLineQ1] = (unsigned long long)(long long)p1;
            out[kStLineQ3] = (unsigned long long)(long long)p3;
        }
    }
}

// Column range check, col streamed once as 16-byte loads, each workgroup over
// a contiguous range of nnz.  With a list (the planning scan, after
// k_row_stats filled it), it also counts the descents col[j] > col[j + 1]
// with j and j + 1 inside one listed long row (a hybrid plan's dense rows need
// sorted columns), so planning reads col once.  A workgroup whose range meets
// more listed rows than it holds, or a list that overflowed, sets
// out[kStLongUnchecked] instead of counting.
constexpr int kColRowsCap = 256;  // listed rows one workgroup's range may meet

__global__ __launch_bounds__(kBS) void k_col_check(const int *__restrict__ col, long long nnz, int n,
                                                   unsigned long long *__restrict__ out, const int4 *__restrict__ list,
                                                   int cap)
{
    __shared__ int s_nrows, s_over;
    __shared__ int2 s_rows[kColRowsCap];  // nnz ranges [first, end) of the listed rows this range meets
    __shared__ int2 s_sorted[kColRowsCap];  // the same, by first nnz (disjoint ranges: distinct firsts)
    const int tid = threadIdx.x;
    const long long per = ((nnz + gridDim.x - 1) / gridDim.x + 1023) & ~1023ll;  // whole vectors per lane
    const long long j0 = (long long)blockIdx.x * per;
    const long long j1 = min(nnz, j0 + per);
    if (j0 >= nnz)
        return;  // whole workgroup
    if (tid == 0) { s_nrows = 0; s_over = 0; }
    __syncthreads();
    if (list) {
        const unsigned long long listed = out[kStLongListed];
        const int nl = (int)min(listed, (unsigned long long)cap);
        if (listed > (unsigned long long)cap && blockIdx.x == 0 && tid == 0) atomicOr(out + kStLongUnchecked, 1ull);
        for (int i = tid; i < nl; i += kBS) {
            const int4 e = list[i];
            if ((long long)e.y < j1 && (long long)e.z > j0) {
                const int k = atomicAdd(&s_nrows, 1);
                if (k < kColRowsCap) s_rows[k] = make_int2(e.y, e.z);
                else s_over = 1;
            }
        }
        __syncthreads();
        if (s_over && tid == 0) atomicOr(out + kStLongUnchecked, 1ull);
        const int nr = s_over ? 0 : min(s_nrows, kColRowsCap);
        for (int t = tid; t < nr; t += kBS) {  // rank sort: a descent then finds its row by bisection
            const int2 me = s_rows[t];
            int rank = 0;
            for (int k = 0; k < nr; ++k) rank += s_rows[k].x < me.x ? 1 : 0;
            s_sorted[rank] = me;
        }
        __syncthreads();
    }
    const int nrows = s_over ? 0 : min(s_nrows, kColRowsCap);
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(col + j0, (j1 - j0) * 4);
    // the entry after the range, for the descent at its last position (zero past nnz: unused there)
    const __amdgpu_buffer_rsrc_t rn = make_rsrc(col + j0, min(nnz - j0, j1 - j0 + 1) * 4);
    unsigned int bad = 0, desc = 0;
    const int nvec = (int)((j1 - j0 + 3) / 4);
    const int lane = tid & (kWave - 1);
    for (int v0 = tid; v0 < nvec; v0 += 4 * kBS) {
        u32x4 c[4];
        int nx[4] = {0, 0, 0, 0};
#pragma unroll
        for (int u = 0; u < 4; ++u)  // four loads in flight per lane; vectors past the range read zeros
            c[u] = __builtin_amdgcn_raw_buffer_load_b128(rc, (v0 + u * kBS) * 16, 0, kAuxNt);
        if (nrows > 0) {  // workgroup-uniform
            // The entry after a lane's vector is the next lane's first (taken below with a lane shift)
            // unless the lane is the wave's last or its vector ends the range: those read it here.
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const long long je = j0 + 4ll * (v0 + u * kBS) + 4;
                if (lane == kWave - 1 || je >= j1)
                    nx[u] = (int)__builtin_amdgcn_raw_buffer_load_b32(rn, (v0 + u * kBS) * 16 + 16, 0, 0);
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const long long jb = j0 + 4ll * (v0 + u * kBS);
            const int e[4] = {(int)c[u].x, (int)c[u].y, (int)c[u].z, (int)c[u].w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
                bad += (jb + i < j1 && (e[i] < 0 || e[i] >= n)) ? 1u : 0u;
            // lane + 1 holds vector v0 + u * kBS + 1, and is active whenever jb + 4 < j1 (that vector is in range)
            const int next = nrows > 0 ? __shfl_down(e[0], 1) : 0;
            if (nrows > 0 && jb < j1) {  // descents inside listed rows (rare: sorted rows have none)
                const int nxu = (lane == kWave - 1 || jb + 4 >= j1) ? nx[u] : next;
                const int f[5] = {e[0], e[1], e[2], e[3], nxu};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const long long j = jb + i;
                    if (j + 1 < nnz && j + 1 <= j1 && j < j1 && f[i] > f[i + 1]) {
                        int lo = 0, hi = nrows;  // the last listed row starting at or before j
                        while (hi - lo > 1) {
                            const int mid = (lo + hi) >> 1;
                            if ((long long)s_sorted[mid].x <= j) lo = mid; else hi = mid;
                        }
                        desc += (s_sorted[lo].x <= j && j + 1 < s_sorted[lo].y) ? 1u : 0u;
                    }
                }
            }
        }
    }
    if (__ballot(bad != 0)) {
        for (int o = 32; o > 0; o >>= 1)
            bad += __shfl_down(bad, o);
        if ((tid & (kWave - 1)) == 0 && bad)
            atomicAdd(out + kStBadCol, (unsigned long long)bad);
    }
    if (__ballot(desc != 0)) {
        for (int o = 32; o > 0; o >>= 1)
            desc += __shfl_down(desc, o);
        if ((tid & (kWave - 1)) == 0 && desc)
            atomicAdd(out + kStLongDesc, (unsigned long long)desc);
    }
}

__global__ __launch_bounds__(kBS) void k_fill_u32(uint32_t *__restrict__ p, size_t nwords, uint32_t value)
{
    for (size_t i = (size_t)blockIdx.x * kBS + threadIdx.x; i < nwords; i += (size_t)gridDim.x * kBS)
        p[i] = value;
}

__global__ __launch_bounds__(kBS) void k_fill_zero(uint32_t *__restrict__ p, size_t nwords)
{
    for (size_t i = (size_t)blockIdx.x * kBS + threadIdx.x; i < nwords; i += (size_t)gridDim.x * kBS)
        p[i] = 0u;
}

__global__ __launch_bounds__(kBS) void k_fill_zero16(unsigned short *__restrict__ p, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * kBS + threadIdx.x; i < n; i += (size_t)gridDim.x * kBS)
        p[i] = 0;
}

// ---- scratch of the no-allocation entry point --------------------------------
//
// pf_spmv_noalloc takes its row statistics and plan workspace from this array
// instead of allocating.  Each device holds its own copy, at its own address,
// for the life of the process.  In host code `scratch` only names the symbol:
// kernels get the address pfk_scratch looks up with hipGetSymbolAddress.
}  // namespace

static __device__ __align__(256) unsigned char scratch[PFK_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// ---- host side of the thin layer -------------------------------------------

thread_local char g_err[256] = "";

int hip_fail(hipError_t e, const char *what)
{
    snprintf(g_err, sizeof g_err, "%s: %s", what, hipGetErrorString(e));
    return PF_ERR_HIP;
}

#define PFK_HIP(call)                                            \
    do {                                                         \
        hipError_t e_ = (call);                                  \
        if (e_ != hipSuccess) return hip_fail(e_, #call);        \
    } while (0)

#define PFK_LAUNCHED(what)                                       \
    do {                                                         \
        hipError_t e_ = hipGetLastError();                       \
        if (e_ != hipSuccess) return hip_fail(e_, what);         \
    } while (0)

#define PFK_TRY(expr)                                            \
    do {                                                         \
        const int rc_ = (expr);                                  \
        if (rc_ != PF_OK) return rc_;                            \
    } while (0)

inline hipStream_t S(void *s) { return reinterpret_cast<hipStream_t>(s); }

inline unsigned grid_for(long long work, long long per_block, long long cap)
{
    long long g = (work + per_block - 1) / per_block;
    if (g > cap) g = cap;
    return (unsigned)(g < 1 ? 1 : g);
}

// XCD chunks (see xcd_tile) for tiles of tile_nnz: chunks of about chunk_nnz
// nnz, or one chunk of ceil(ntiles / 8) tiles per XCD when chunk_nnz is 0.
// The rounds are balanced: every XCD gets the same number of chunks, of
// ceil(g / rounds) tiles, so the last round does not fall on a few XCDs.
void chunk_shape(long long ntiles, long long tile_nnz, long long chunk_nnz, long long &xch, long long &g8,
                 int nx = kXcds)
{
    const long long g = (ntiles + nx - 1) / nx;
    long long target = chunk_nnz > 0 ? chunk_nnz / tile_nnz : g;
    if (target < 1) target = 1;
    const long long rounds = (g + target - 1) / target;
    xch = (g + rounds - 1) / rounds;
    g8 = rounds * xch;
}

template <typename T>
Args<T> make_args(const pfk_spmv_args *a)
{
    Args<T> r;
    r.rp = a->row_ptr;
    r.col = a->col;
    r.val = static_cast<const T *>(a->val);
    r.x = static_cast<const T *>(a->x);
    r.y = static_cast<T *>(a->y);
    r.m = a->m;
    r.n = a->n;
    r.nnz = a->nnz;
    r.guess_spread = a->guess_spread;
    r.guess_a = a->guess_a > 0.0 ? a->guess_a : 0.0;  // (false for NaN)
    r.guess_b = r.guess_a > 0.0 ? a->guess_b : 0.0;
    r.ntiles = a->ntiles;
    r.g8 = (a->ntiles + kXcds - 1) / kXcds;
    r.xch = r.g8;
    r.tx = r.g8;
    r.tpw = 1;
    r.head = static_cast<acc_t<T> *>(a->head_slot);
    r.tail = static_cast<acc_t<T> *>(a->tail_slot);
    r.owner = a->owner_row;
    r.err = a->err_flag;
    r.sched = a->sched;
    r.sched_cap = a->sched_cap;
    r.y2 = static_cast<T *>(a->half_part);
    r.ovf_cap = a->ovf_cap;
    return r;
}

// A workspace buffer of `have` bytes where `need` are touched.
bool room(const void *p, size_t have, long long need, const char *what)
{
    if (need <= 0) return true;
    if (p && have >= (size_t)need) return true;
    snprintf(g_err, sizeof g_err, "%s: %zu bytes given, %lld needed", what, p ? have : (size_t)0, need);
    return false;
}

// The workspace a launch touches, against the sizes the caller declared.
// split: head / tail / owner slots are written or read (every tiling but the
// row-aligned FLAT and PREFREE ones).
bool ws_ok(int dtype, const pfk_spmv_args *a, bool split)
{
    const long long nt = a->ntiles;
    if (split && !(room(a->head_slot, a->head_bytes, nt * PFK_SLOT_BYTES(dtype), "head slots") &&
                   room(a->tail_slot, a->tail_bytes, nt * PFK_SLOT_BYTES(dtype), "tail slots") &&
                   room(a->owner_row, a->owner_bytes, nt * 4, "owner slots")))
        return false;
    if (a->row_map && !room(a->row_map, a->row_map_bytes, (nt + 1) * 8, "row map"))
        return false;
    if (a->sched) {
        if (a->sched_cap < (nt + kXcds - 1) / kXcds) {
            snprintf(g_err, sizeof g_err, "schedule lists of %lld tiles for %lld tiles", a->sched_cap, nt);
            return false;
        }
        if (!room(a->sched, a->sched_bytes, (long long)PFK_SCHED_INTS(nt, a->sched_cap) * 4, "x-window schedule"))
            return false;
    }
    return true;
}

bool args_ok(const pfk_spmv_args *a, bool need_ws)
{
    if (!a || !a->row_ptr || !a->y || a->m < 0 || a->n < 0 || a->nnz < 0 || a->ntiles < 1 || !a->err_flag)
        return false;
    if (a->nnz > 0 && (!a->col || !a->val || !a->x))
        return false;
    if ((unsigned long long)a->nnz + (unsigned long long)a->m >= 0xFFFFFFFFull)
        return false;
    if (need_ws && (!a->head_slot || !a->tail_slot || !a->owner_row))
        return false;
    if (((uintptr_t)a->col & 15) || ((uintptr_t)a->val & 15))
        return false;
    return true;
}

template <typename T, bool MERGE, int K, int LMAX>
int launch_tiles(const pfk_spmv_args *a, void *stream)
{
    Args<T> r = make_args<T>(a);
    const long long grid = r.g8 * kXcds;
    hipLaunchKernelGGL((k_tiles<T, MERGE, K, LMAX>), dim3((unsigned)grid), dim3(kBS), 0, S(stream), r);
    PFK_LAUNCHED("k_tiles");
    return PF_OK;
}

int device_cus()
{
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev] && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus[dev] = 256;
    return cus[dev];
}

// Runs of `run` consecutive tiles, one run per wave, 4 waves per workgroup;
// XCD x takes runs [x*tx, (x+1)*tx).
template <typename T>
void wave_grid(Args<T> &r, int run, long long &grid)
{
    constexpr long long NW = kWaveWG / kWave;
    const long long nruns = (r.ntiles + run - 1) / run;
    r.tpw = run;
    r.tx = (nruns + kXcds - 1) / kXcds;
    grid = ((r.tx + NW - 1) / NW) * kXcds;
}

template <typename T, int K, int LMAX, bool DESC_ONLY, bool NT = true>
int launch_stream(const pfk_spmv_args *a, int *dbg, void *stream)
{
    Args<T> r = make_args<T>(a);
    long long grid = 0;
    wave_grid<T>(r, a->run_tiles > 0 ? a->run_tiles : 8, grid);
    hipLaunchKernelGGL((k_wave<T, K, LMAX, DESC_ONLY, NT>), dim3((unsigned)grid), dim3(kWaveWG), 0, S(stream), r, dbg);
    PFK_LAUNCHED("k_wave");
    return PF_OK;
}

// Wave64s of k_wave<T, K> resident on the whole device at once.
template <typename T, int K>
int wave_residency(long long *waves)
{
    int per_cu = 0;
    PFK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &per_cu, reinterpret_cast<const void *>(&k_wave<T, K, adaptive_lmax(K), false>), kWaveWG, 0));
    *waves = (long long)per_cu * (kWaveWG / kWave) * device_cus();
    return PF_OK;
}

template <typename T>

int dispatch_adaptive(const pfk_spmv_args *a, void *stream)
{
#define PF_DISPATCH(TT, DT, KK) \
    if (std::is_same<T, TT>::value && a->tile == KK)                                                      \
        return a->keep_cached ? launch_stream<TT, KK, adaptive_lmax(KK), false, false>(a, nullptr, stream) \
                              : launch_stream<TT, KK, adaptive_lmax(KK), false, true>(a, nullptr, stream);
    PF_ADAPTIVE_TILES(PF_DISPATCH)
#undef PF_DISPATCH
    snprintf(g_err, sizeof g_err, "tile %d not compiled for this value type", a->tile);
    return PF_ERR_UNSUPPORTED;
}

// k_flow over runs of run_tiles tiles, then the combine of rows crossing run
// edges (k_fixup over runs: "tile" = one run of run_tiles * 256 nnz).
template <typename T>
int launch_flow(const pfk_spmv_args *a, void *stream)
{
    Args<T> r = make_args<T>(a);
    const long long run = a->run_tiles > 0 ? a->run_tiles : 8;
    const long long nruns = (r.ntiles + run - 1) / run;
    r.tpw = run;
    r.tx = (nruns + kXcds - 1) / kXcds;
    const long long grid = ((r.tx + 3) / 4) * kXcds;
    hipLaunchKernelGGL((k_flow<T>), dim3((unsigned)grid), dim3(kWaveWG), 0, S(stream), r);
    PFK_LAUNCHED("k_flow");
    if (nruns > 1) {
        Args<T> f = r;
        f.ntiles = nruns;
        const unsigned fgrid = (unsigned)((nruns + kBS - 1) / kBS);
        hipLaunchKernelGGL((k_fixup<T, false>), dim3(fgrid), dim3(kBS), 0, S(stream), f, (int)(run * kFlowT));
        PFK_LAUNCHED("k_fixup");
    }
    return PF_OK;
}

// The band kernel over a recorded row map: one workgroup per CU, each over a
// contiguous range of steps of PFK_BAND_STEP / K tiles.
template <typename T, int K>
int launch_band(const pfk_spmv_args *a, void *stream)
{
    static_assert(PFK_BAND_STEP % K == 0, "whole tiles per step");
    Args<T> r = make_args<T>(a);
    BandArgs b;
    b.map = reinterpret_cast<const int2 *>(a->row_map);
    b.w = a->band_w;
    b.group = PFK_BAND_STEP / K;
    const long long nsteps = (a->ntiles + b.group - 1) / b.group;
    const long long wgs = std::min<long long>(nsteps, std::max(1, device_cus()));
    b.per = (int)((nsteps + wgs - 1) / wgs);
    b.nsteps = (int)nsteps;
    const long long grid = (nsteps + b.per - 1) / b.per;
    hipLaunchKernelGGL((k_band<T>), dim3((unsigned)grid), dim3(kBandBS), 0, S(stream), r, b);
    PFK_LAUNCHED("k_band");
    return PF_OK;
}

// k_flat (split rows) or k_rows (row-aligned tiles): search (and record the
// row map when the plan has one) or, once the map is recorded, read it (or run
// the band kernel over it).
template <typename T, int K>
int launch_flat(const pfk_spmv_args *a, int *dbg, void *stream)
{
    Args<T> r = make_args<T>(a);
    chunk_shape(r.ntiles, K, a->chunk_nnz, r.xch, r.g8);
    const long long grid = r.g8 * kXcds;
    if constexpr (!__is_same(T, half_t)) {
        if (a->row_aligned && !dbg && a->row_map && a->map_ready && a->band_w > 0) return launch_band<T, K>(a, stream);
    }
    if (a->row_aligned) {
        if (dbg)
            hipLaunchKernelGGL((k_rows<T, K, kFlatDesc>), dim3((unsigned)grid), dim3(kBS), 0, S(stream), r, nullptr,
                               dbg);
        else if (a->row_map && a->map_ready && (long long)a->nnz < 4LL * a->m)  // very short rows
            hipLaunchKernelGGL((k_rows<T, K, kFlatMemo, true>), dim3((unsigned)grid), dim3(kBS), 0, S(stream), r,
                               a->row_map, nullptr);
        else if (a->row_map && a->map_ready)
            hipLaunchKernelGGL((k_rows<T, K, kFlatMemo>), dim3((unsigned)grid), dim3(kBS), 0, S(stream), r,
                               a->row_map, nullptr);
        else
            hipLaunchKernelGGL((k_rows<T, K, kFlatSearch>), dim3((unsigned)grid), dim3(kBS), 0, S(stream), r,
                               a->row_map, nullptr);
        PFK_LAUNCHED("k_rows");
        return PF_OK;
    }
    if (dbg)
        hipLaunchKernelGGL((k_flat<T, K, kFlatDesc>), dim3((unsigned)grid), dim3(kBS), 0, S(stream), r, nullptr, dbg);
    else if (a->row_map && a->map_ready)
        hipLaunchKernelGGL((k_flat<T, K, kFlatMemo>), dim3((unsigned)(a->sched ? a->sched_cap * kXcds : grid)),
                           dim3(kBS), 0, S(stream), r, a->row_map, nullptr);
    else
        hipLaunchKernelGGL((k_flat<T, K, kFlatSearch>), dim3((unsigned)grid), dim3(kBS), 0, S(stream), r,
                           a->row_map, nullptr);
    PFK_LAUNCHED("k_flat");
    return PF_OK;
}

// Row groups (FLAT tiles 2..32): L = tile lanes per row, m * L threads.
template <typename T>
int launch_vector(const pfk_spmv_args *a, void *stream)
{
    const Args<T> r = make_args<T>(a);
    const long long grid = ((long long)a->m * a->tile + kBS - 1) / kBS;
    if (grid < 1 || grid > 0x7FFFFFFFLL) {
        snprintf(g_err, sizeof g_err, "row groups: %lld workgroups", grid);
        return PF_ERR_UNSUPPORTED;
    }
    switch (a->tile) {
    case 2: hipLaunchKernelGGL((k_vector<T, 2>), dim3((unsigned)grid), dim3(kBS), 0, S(stream), r); break;
    case 4: hipLaunchKernelGGL((k_vector<T, 4>), dim3((unsigned)grid), dim3(kBS), 0, S(stream), r); break;
    case 8: hipLaunchKernelGGL((k_vector<T, 8>), dim3((unsigned)grid), dim3(kBS), 0, S(stream), r); break;
    case 16: hipLaunchKernelGGL((k_vector<T, 16>), dim3((unsigned)grid), dim3(kBS), 0, S(stream), r); break;
    case 32: hipLaunchKernelGGL((k_vector<T, 32>), dim3((unsigned)grid), dim3(kBS), 0, S(stream), r); break;
    default: return PF_ERR_INVALID;
    }
    PFK_LAUNCHED("k_vector");
    return PF_OK;
}

template <typename T>
int dispatch_flat(const pfk_spmv_args *a, void *stream)
{
    if (a->row_aligned && a->tile != 1024 && a->tile != 2048) {
        snprintf(g_err, sizeof g_err, "row-aligned FLAT tiles are 1024 or 2048 nnz, not %d", a->tile);
        return PF_ERR_INVALID;
    }
    if constexpr (__is_same(T, half_t)) {  // fp16: the 1024 / 2048 kernels only
        switch (a->tile) {
        case 1024: return launch_flat<T, 1024>(a, nullptr, stream);
        case 2048: return launch_flat<T, 2048>(a, nullptr, stream);
        }
    } else {
        if (a->tile == kFlowT) return launch_flow<T>(a, stream);
        switch (a->tile) {
        case 1024: return launch_flat<T, 1024>(a, nullptr, stream);
        case 2048: return launch_flat<T, 2048>(a, nullptr, stream);
        case 4096: return launch_tiles<T, false, 4096, 0>(a, stream);
        }
    }
    snprintf(g_err, sizeof g_err, "tile %d not compiled for this value type", a->tile);
    return PF_ERR_UNSUPPORTED;
}

template <int K>
int launch_flat_desc(const pfk_spmv_args *a, int *out, void *stream)
{
    Args<double> r = make_args<double>(a);
    const long long grid = r.g8 * kXcds;
    hipLaunchKernelGGL((k_tile_desc<false, K, 0, K + 2>), dim3((unsigned)grid), dim3(kBS), 0, S(stream), r, out);
    PFK_LAUNCHED("k_tile_desc");
    return PF_OK;
}

template <typename T, int P>
int launch_prefree(const pfk_spmv_args *a, void *stream)
{
    Args<T> r = make_args<T>(a);
    const dim3 grid((unsigned)(((a->ntiles + kXcds - 1) / kXcds) * kXcds));
    switch (a->ladder == 0 ? 3 : a->ladder) {
    case 1: hipLaunchKernelGGL((k_prefree<T, P, 1>), grid, dim3(kPfBS), 0, S(stream), r); break;
    case 2: hipLaunchKernelGGL((k_prefree<T, P, 2>), grid, dim3(kPfBS), 0, S(stream), r); break;
    case 3: hipLaunchKernelGGL((k_prefree<T, P, 3>), grid, dim3(kPfBS), 0, S(stream), r); break;
    case 4: hipLaunchKernelGGL((k_prefree<T, P, 4>), grid, dim3(kPfBS), 0, S(stream), r); break;
    case 5: hipLaunchKernelGGL((k_prefree<T, P, 5>), grid, dim3(kPfBS), 0, S(stream), r); break;
    default: return PF_ERR_INVALID;
    }
    PFK_LAUNCHED("k_prefree");
    if constexpr (__is_same(T, half_t)) {
        hipLaunchKernelGGL(k_prefree_join, dim3((unsigned)((a->ntiles + 3) / 4)), dim3(kBS), 0, S(stream),
                           static_cast<const int *>(a->owner_row), static_cast<const float *>(a->head_slot),
                           static_cast<const float *>(a->tail_slot), a->ntiles, static_cast<half_t *>(a->y));
        PFK_LAUNCHED("k_prefree_join");
    }
    return PF_OK;
}

// A hybrid plan's call: run tiles (k_rows over the run table), the dense rows'
// window sums (k_dense), their combine (k_dense_sum).
template <typename T, int K>
int launch_hybrid(const pfk_spmv_args *a, void *stream)
{
    Args<T> r = make_args<T>(a);
    const bool halves = a->x_halves && a->half_part;
    if (r.ntiles > 0) chunk_shape(r.ntiles, K, a->chunk_nnz, r.xch, r.g8, halves ? kXcds / 2 : kXcds);
    const RunTable rt{a->runs, a->n_runs};
    const bool memo = a->map_ready && a->run_map && (a->long_mode || a->dense_seg);
    const bool prio = (long long)a->nnz < 4LL * a->m;
    const dim3 rgrid((unsigned)(r.g8 * kXcds));
    // Two streams: the runs (bound by the address units and L2 hits) on the
    // second, the dense rows' stream of col / val (bound by HBM) on the
    // caller's; they share no output until the combines, which run on the
    // caller's stream after it waits for the runs.
    const bool fork = a->aux_stream && a->ev_fork && a->ev_join && a->ntiles > 0;
    void *rs = stream;
    if (fork) {
        PFK_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(a->ev_fork), S(stream)));
        PFK_HIP(hipStreamWaitEvent(S(a->aux_stream), reinterpret_cast<hipEvent_t>(a->ev_fork), 0));
        rs = a->aux_stream;
    }
    const auto join = [&]() -> int {
        if (!fork) return PF_OK;
        PFK_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(a->ev_join), S(a->aux_stream)));
        PFK_HIP(hipStreamWaitEvent(S(stream), reinterpret_cast<hipEvent_t>(a->ev_join), 0));
        return PF_OK;
    };
    if (a->ntiles == 0)  // every row is dense
        ;
    else if (halves && memo)
        hipLaunchKernelGGL((k_rows<T, K, kFlatMemo, false, true, true>), rgrid, dim3(kBS), 0, S(rs), r, a->run_map, nullptr, rt);
    else if (halves)
        hipLaunchKernelGGL((k_rows<T, K, kFlatSearch, false, true, true>), rgrid, dim3(kBS), 0, S(rs), r, a->run_map, nullptr, rt);
    else if (memo && prio)
        hipLaunchKernelGGL((k_rows<T, K, kFlatMemo, true, true>), rgrid, dim3(kBS), 0, S(rs), r, a->run_map, nullptr, rt);
    else if (memo)
        hipLaunchKernelGGL((k_rows<T, K, kFlatMemo, false, true>), rgrid, dim3(kBS), 0, S(rs), r, a->run_map, nullptr, rt);
    else
        hipLaunchKernelGGL((k_rows<T, K, kFlatSearch, false, true>), rgrid, dim3(kBS), 0, S(rs), r, a->run_map, nullptr, rt);
    if (a->ntiles > 0) PFK_LAUNCHED("k_rows (runs)");
    // With x halves, y = first half + second half over the runs' rows joins the
    // combine of the rows summed apart (one launch at the end)
    const bool fuse = a->ntiles > 0 && halves;
    const int hblocks = fuse ? (int)grid_for(a->m, kBS, 8192) : 0;
    const unsigned sblocks = (unsigned)((a->n_dense + kWaves - 1) / kWaves);
    if (a->long_mode) {
        const LongArgs L{reinterpret_cast<const int4 *>(a->long_tiles), a->long_deal, a->long_row_tiles,
                         a->dense_rows, a->n_dense, a->n_long_tiles, a->long_part};
        const unsigned lgrid = (unsigned)(kXcds * ((a->n_long_tiles + kXcds - 1) / kXcds));
        hipLaunchKernelGGL((k_long<T>), dim3(lgrid), dim3(kBS), 0, S(stream), r, L);
        PFK_LAUNCHED("k_long");
        if (fork) PFK_TRY(join());
        if (fuse) {
            hipLaunchKernelGGL((k_combine<T, true>), dim3((unsigned)hblocks + sblocks), dim3(kBS), 0, S(stream), r,
                               DenseArgs{}, L, a->row_apart, hblocks);
            PFK_LAUNCHED("k_combine");
            return PF_OK;
        }
        hipLaunchKernelGGL((k_long_sum<T>), dim3(sblocks), dim3(kBS), 0, S(stream), r, L);
        PFK_LAUNCHED("k_long_sum");
        return PF_OK;
    }
    const int ngroups = (a->n_dense + DenseShape<T>::kG - 1) / DenseShape<T>::kG;
    const int gsz = ngroups > 0 ? (a->n_dense + ngroups - 1) / ngroups : 0;
    const DenseArgs d{a->dense_rows, a->n_dense, a->n_win, ngroups, pfk_dense_width(a->n, a->n_win), gsz,
                      a->dense_seg, a->dense_part};
    const unsigned dgrid = (unsigned)(kXcds * ((a->n_win + kXcds - 1) / kXcds) * ngroups);
    if (memo)
        hipLaunchKernelGGL((k_dense<T, kFlatMemo>), dim3(dgrid), dim3(kBS), 0, S(stream), r, d);
    else
        hipLaunchKernelGGL((k_dense<T, kFlatSearch>), dim3(dgrid), dim3(kBS), 0, S(stream), r, d);
    PFK_LAUNCHED("k_dense");
    if (fork) PFK_TRY(join());
    if (fuse) {
        hipLaunchKernelGGL((k_combine<T, false>), dim3((unsigned)hblocks + sblocks), dim3(kBS), 0, S(stream), r, d,
                           LongArgs{}, a->row_apart, hblocks);
        PFK_LAUNCHED("k_combine");
        return PF_OK;
    }
    hipLaunchKernelGGL((k_dense_sum<T>), dim3(sblocks), dim3(kBS), 0, S(stream), r, d);
    PFK_LAUNCHED("k_dense_sum");
    return PF_OK;
}

// Row statistics, and with a list the planning scan's long rows and descents.
int launch_stats(const int *row_ptr, const int *col, int m, int n, long long nnz, unsigned long long *d_out,
                 int4 *list, int cap, void *stream)
{
    if (!row_ptr || !d_out || m < 0 || nnz < 0 || cap < 0) return PF_ERR_INVALID;
    hipLaunchKernelGGL(k_stats_init, dim3(1), dim3(64), 0, S(stream), d_out);
    PFK_LAUNCHED("k_stats_init");
    if (m > 0) {
        // a workgroup per CU (fewer for small m), each row range within a buffer resource's reach
        const long long rows_wg = (long long)kStatsBS * kStatsRows * kStatsGroups;  // rows of one pass
        long long grid = std::min<long long>(((long long)m + rows_wg - 1) / rows_wg, std::max(1, device_cus()));
        grid = std::max<long long>(grid, ((long long)m + (1ll << 26) - 1) >> 26);
        hipLaunchKernelGGL(k_row_stats, dim3((unsigned)grid), dim3(kStatsBS), 0, S(stream), row_ptr, m, d_out, list,
                           cap);
        PFK_LAUNCHED("k_row_stats");
    }
    if (col && nnz > 0) {
        // about 16 vectors of 4 nnz per lane and workgroup, at most 4096 workgroups
        const unsigned grid = grid_for((nnz + 15) / 16, kBS * 4, 4096);
        hipLaunchKernelGGL(k_col_check, dim3(grid), dim3(kBS), 0, S(stream), col, nnz, n, d_out, list, cap);
        PFK_LAUNCHED("k_col_check");
    }
    return PF_OK;
}

}  // namespace

extern "C" {

int pfk_spmv_adaptive(int dtype, const pfk_spmv_args *a, void *stream)
{
    if (a && a->m == 0 && a->nnz == 0) return PF_OK;
    if (!args_ok(a, true) || !ws_ok(dtype, a, true)) return PF_ERR_INVALID;
    return dtype == PF_F64 ? dispatch_adaptive<double>(a, stream)
         : dtype == PF_F32 ? dispatch_adaptive<float>(a, stream)
         : dtype == PF_F16 ? dispatch_adaptive<half_t>(a, stream) : PF_ERR_INVALID;
}

int pfk_spmv_flat(int dtype, const pfk_spmv_args *a, void *stream)
{
    if (!a) return PF_ERR_INVALID;
    if (a->m == 0 && a->nnz == 0) return PF_OK;
    if (PFK_ROW_GROUP_TILE(a->tile)) {  // row groups: no workspace, no tiles
        if (!args_ok(a, false) || a->band_w != 0 || a->row_map || a->sched) return PF_ERR_INVALID;
        return dtype == PF_F64 ? launch_vector<double>(a, stream)
             : dtype == PF_F32 ? launch_vector<float>(a, stream)
             : dtype == PF_F16 ? launch_vector<half_t>(a, stream) : PF_ERR_INVALID;
    }
    if (!args_ok(a, !a->row_aligned) || !ws_ok(dtype, a, !a->row_aligned)) return PF_ERR_INVALID;
    if (a->band_w < 0 || a->band_w > PFK_BAND_RING / 2 ||
        (a->band_w > 0 && (dtype == PF_F16 || !a->row_aligned || !a->row_map))) {
        snprintf(g_err, sizeof g_err, "band width %d: 0..%d, for row-aligned fp64 / fp32 plans with a row map",
                 a->band_w, PFK_BAND_RING / 2);
        return PF_ERR_INVALID;
    }
    return dtype == PF_F64 ? dispatch_flat<double>(a, stream)
         : dtype == PF_F32 ? dispatch_flat<float>(a, stream)
         : dtype == PF_F16 ? dispatch_flat<half_t>(a, stream) : PF_ERR_INVALID;
}

int pfk_spmv_hybrid(int dtype, const pfk_spmv_args *a, void *stream)
{
    if (!a) return PF_ERR_INVALID;
    if (dtype != PF_F64 && dtype != PF_F32 && dtype != PF_F16) return PF_ERR_INVALID;
    if (dtype == PF_F16 && (a->x_halves || a->tile != 2048)) {  // fp16: one rounding per row, so no halves
        snprintf(g_err, sizeof g_err, "fp16 hybrid plans: 2048-nnz run tiles, no x halves");
        return PF_ERR_UNSUPPORTED;
    }
    if (a->m == 0 && a->nnz == 0) return PF_OK;
    pfk_spmv_args v = *a;  // a hybrid plan may have no run tiles (every row dense)
    v.ntiles = a->ntiles > 0 ? a->ntiles : 1;
    if (a->ntiles < 0 || !args_ok(&v, false) || a->n_dense < 1 || a->n_runs < 1 || !a->dense_rows || !a->runs ||
        (a->long_mode ? (!a->long_tiles || !a->long_deal || !a->long_row_tiles || !a->long_part ||
                         a->n_long_tiles < 1)
                      : !a->dense_part) ||
        (a->tile != 1024 && a->tile != 2048)) {
        snprintf(g_err, sizeof g_err, "hybrid call: missing tables or tile %d", a->tile);
        return PF_ERR_INVALID;
    }
    if (!a->long_mode && (a->n_win != pfk_dense_nwin(a->n, dtype) || a->n_win < 1 ||
                          pfk_dense_width(a->n, a->n_win) > PFK_DENSE_WINDOW(dtype))) {
        snprintf(g_err, sizeof g_err, "hybrid call: %d x windows for n = %d", a->n_win, a->n);
        return PF_ERR_INVALID;
    }
    const long long nd = a->n_dense, nw = a->n_win, nl = a->n_long_tiles;
    if (!room(a->runs, a->runs_bytes, 5LL * (a->n_runs + 1) * 4, "run table") ||
        (!a->long_mode && !room(a->dense_part, a->dense_part_bytes, nd * nw * PFK_SLOT_BYTES(dtype),
                                "dense partial sums")) ||
        (a->long_mode && (!room(a->long_tiles, a->long_tiles_bytes, nl * 16, "long-row tiles") ||
                          !room(a->long_deal, a->long_deal_bytes, nl * 4, "long-row tile deal") ||
                          !room(a->long_row_tiles, a->long_row_tiles_bytes, (nd + 1) * 4, "long-row tile index") ||
                          !room(a->long_part, a->long_part_bytes, nl * PFK_SLOT_BYTES(dtype),
                                "long-row partial sums"))) ||
        (a->run_map && !room(a->run_map, a->run_map_bytes, a->ntiles * 32, "run tile map")) ||
        (!a->long_mode && a->dense_seg &&
         !room(a->dense_seg, a->dense_seg_bytes, nd * (nw + 1) * 4, "dense segment bounds")) ||
        (a->x_halves && !room(a->half_part, a->half_part_bytes, (long long)a->m * (dtype == PF_F64 ? 8 : 4),
                              "x-halves row sums")) ||
        (a->x_halves && !room(a->row_apart, a->row_apart_bytes, (long long)a->m, "rows summed apart")))
        return PF_ERR_INVALID;
    if (dtype == PF_F64) return a->tile == 1024 ? launch_hybrid<double, 1024>(a, stream) : launch_hybrid<double, 2048>(a, stream);
    if (dtype == PF_F16) return launch_hybrid<half_t, 2048>(a, stream);
    return a->tile == 1024 ? launch_hybrid<float, 1024>(a, stream) : launch_hybrid<float, 2048>(a, stream);
}

int pfk_dense_scan(const int *row_ptr, const int *col, int m, int dmin, int *list, int cap, int *counters, void *stream)
{
    if (!row_ptr || !col || !list || !counters || m < 1 || dmin < 1 || cap < 1) return PF_ERR_INVALID;
    hipLaunchKernelGGL(k_dense_scan, dim3(grid_for(m, kBS, 2048)), dim3(kBS), 0, S(stream), row_ptr, m, dmin, list,
                       cap, counters);
    PFK_LAUNCHED("k_dense_scan");
    hipLaunchKernelGGL(k_dense_sorted, dim3(64, (unsigned)std::min(cap, 4096)), dim3(kBS), 0, S(stream), col, list,
                       cap, counters);
    PFK_LAUNCHED("k_dense_sorted");
    return PF_OK;
}

int pfk_mark_rows(const int *rows, int count, unsigned char *flags, long long nflags, void *stream)
{
    if (!rows || !flags || count < 0 || nflags < 0) return PF_ERR_INVALID;
    if (count == 0) return PF_OK;
    hipLaunchKernelGGL(k_mark_rows, dim3(grid_for(count, kBS, 1024)), dim3(kBS), 0, S(stream), rows, count, flags,
                       nflags);
    PFK_LAUNCHED("k_mark_rows");
    return PF_OK;
}

int pfk_gather_cols(const int *col, long long nnz, const int *idx, int count, int *out, void *stream)
{
    if (!col || !idx || !out || count < 0 || nnz < 0) return PF_ERR_INVALID;
    if (count == 0) return PF_OK;
    hipLaunchKernelGGL(k_gather_cols, dim3(grid_for(count, kBS, 1024)), dim3(kBS), 0, S(stream), col, nnz, idx, count,
                       out);
    PFK_LAUNCHED("k_gather_cols");
    return PF_OK;
}

long long pfk_flat_grid(long long ntiles, int tile, long long chunk_nnz)
{
    if (ntiles < 1 || tile < 1) return 0;
    long long xch = 0, g8 = 0;
    chunk_shape(ntiles, tile, chunk_nnz, xch, g8);
    return g8 * kXcds;
}

int pfk_flow_resident_waves(int dtype, long long *waves)
{
    if (!waves) return PF_ERR_INVALID;
    int per_cu = 0;
    if (dtype == PF_F64)
        PFK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(&k_flow<double>),
                                                              kWaveWG, 0));
    else if (dtype == PF_F32)
        PFK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(&k_flow<float>),
                                                              kWaveWG, 0));
    else
        return PF_ERR_INVALID;
    *waves = (long long)per_cu * (kWaveWG / kWave) * device_cus();
    return PF_OK;
}

int pfk_adaptive_resident_waves(int dtype, int tile, long long *waves)
{
    if (!waves) return PF_ERR_INVALID;
    *waves = 0;
#define PF_RESIDENCY(TT, DT, KK) \
    if (dtype == DT && tile == KK) return wave_residency<TT, KK>(waves);
    PF_ADAPTIVE_TILES(PF_RESIDENCY)
#undef PF_RESIDENCY
    snprintf(g_err, sizeof g_err, "tile %d not compiled for this value type", tile);
    return PF_ERR_UNSUPPORTED;
}

int pfk_adaptive_owners(int dtype, const pfk_spmv_args *a, void *stream)
{
    if (!a || !a->row_ptr || !a->owner_row || !a->err_flag || a->m <= 0 || a->ntiles < 1) return PF_ERR_INVALID;
    if (!room(a->owner_row, a->owner_bytes, a->ntiles * 4, "owner slots")) return PF_ERR_INVALID;
    // The descriptors depend on (K, LMAX) only; the double instantiation serves both value types.
#define PF_OWNERS(TT, DT, KK) \
    if (dtype == DT && a->tile == KK) return launch_stream<double, KK, adaptive_lmax(KK), true>(a, nullptr, stream);
    PF_ADAPTIVE_TILES(PF_OWNERS)
#undef PF_OWNERS
    snprintf(g_err, sizeof g_err, "tile %d not compiled for this value type", a->tile);
    return PF_ERR_UNSUPPORTED;
}

int pfk_spmv_fixup(int dtype, int merged_keys, const pfk_spmv_args *a, void *stream)
{
    if (a && a->m == 0 && a->nnz == 0) return PF_OK;
    if (!args_ok(a, true) || a->tile <= 0 || !ws_ok(dtype, a, true)) return PF_ERR_INVALID;
    const unsigned grid = (unsigned)((a->ntiles + kBS - 1) / kBS);
    if (dtype == PF_F64) {
        Args<double> r = make_args<double>(a);
        if (merged_keys) hipLaunchKernelGGL((k_fixup<double, true>), dim3(grid), dim3(kBS), 0, S(stream), r, a->tile);
        else hipLaunchKernelGGL((k_fixup<double, false>), dim3(grid), dim3(kBS), 0, S(stream), r, a->tile);
    } else if (dtype == PF_F32) {
        Args<float> r = make_args<float>(a);
        if (merged_keys) hipLaunchKernelGGL((k_fixup<float, true>), dim3(grid), dim3(kBS), 0, S(stream), r, a->tile);
        else hipLaunchKernelGGL((k_fixup<float, false>), dim3(grid), dim3(kBS), 0, S(stream), r, a->tile);
    } else if (dtype == PF_F16) {
        Args<half_t> r = make_args<half_t>(a);
        if (merged_keys) hipLaunchKernelGGL((k_fixup<half_t, true>), dim3(grid), dim3(kBS), 0, S(stream), r, a->tile);
        else hipLaunchKernelGGL((k_fixup<half_t, false>), dim3(grid), dim3(kBS), 0, S(stream), r, a->tile);
    } else {
        return PF_ERR_INVALID;
    }
    PFK_LAUNCHED("k_fixup");
    return PF_OK;
}

int pfk_spmv_prefree(int dtype, const pfk_spmv_args *a, void *stream)
{
    if (dtype != PF_F64 && dtype != PF_F32 && dtype != PF_F16) return PF_ERR_INVALID;  // before y is sized from it
    if (a && a->m == 0 && a->nnz == 0) return PF_OK;
    if (!args_ok(a, dtype == PF_F16)) return PF_ERR_INVALID;
    // fp16: fp32 partials of the tile-boundary rows (head, tail) and each tile's row range (owner_row, 2 ints)
    if (dtype == PF_F16 && !(room(a->head_slot, a->head_bytes, a->ntiles * 4, "head slots") &&
                             room(a->tail_slot, a->tail_bytes, a->ntiles * 4, "tail slots") &&
                             room(a->owner_row, a->owner_bytes, a->ntiles * 8, "row ranges")))
        return PF_ERR_INVALID;
    if (a->ladder < 0 || a->ladder > 5) {
        snprintf(g_err, sizeof g_err, "reduction ladder %d: the reference has codes 1..5", a->ladder);
        return PF_ERR_INVALID;
    }
    if (a->tile != 512 && a->tile != 1024) return PF_ERR_UNSUPPORTED;
    // the reference memsets y, preFreeSpMV.cu:644
    int st = PF_OK;
    if (dtype == PF_F16) {
        hipLaunchKernelGGL(k_fill_zero16, dim3(grid_for(a->m, kBS, 8192)), dim3(kBS), 0, S(stream),
                           static_cast<unsigned short *>(a->y), (size_t)a->m);
        PFK_LAUNCHED("k_fill_zero16");
    } else {
        st = pfk_fill_zero(a->y, (size_t)a->m * (dtype == PF_F64 ? 8 : 4), stream);
    }
    if (st != PF_OK || a->nnz == 0) return st;
    if (dtype == PF_F64) return a->tile == 512 ? launch_prefree<double, 4>(a, stream) : launch_prefree<double, 8>(a, stream);
    if (dtype == PF_F16) return a->tile == 512 ? launch_prefree<half_t, 4>(a, stream) : launch_prefree<half_t, 8>(a, stream);
    return a->tile == 512 ? launch_prefree<float, 4>(a, stream) : launch_prefree<float, 8>(a, stream);
}

int pfk_supported_tiles(int variant, int dtype, int *tiles, int cap)
{
    static const int ad64[] = {188, 238, 494, 512};  // k_wave: keys per wave tile
    static const int ad32[] = {440, 494, 1024};
    // nnz per tile: k_flow, k_flat, k_flat, k_tiles; 2..32: lanes per row of the row groups (k_vector)
    static const int fl64[] = {256, 1024, 2048, 4096, 2, 4, 8, 16, 32};
    static const int fl32[] = {256, 1024, 2048, 4096, 2, 4, 8, 16, 32};
    static const int fl16[] = {1024, 2048, 2, 4, 8, 16, 32};  // fp16: k_flat / k_rows and the row groups
    static const int pf_tiles[] = {512, 1024};   // k_prefree: 128 x P_NNZ
    const int *src;
    int n;
    if (variant == PF_PREFREE) { src = pf_tiles; n = 2; }
    else if (variant == PF_ADAPTIVE && dtype == PF_F64) { src = ad64; n = 4; }
    else if (variant == PF_ADAPTIVE && (dtype == PF_F32 || dtype == PF_F16)) { src = ad32; n = 3; }  // fp16 as fp32
    else if (variant == PF_FLAT && dtype == PF_F64) { src = fl64; n = 9; }
    else if (variant == PF_FLAT && dtype == PF_F32) { src = fl32; n = 9; }
    else if (variant == PF_FLAT && dtype == PF_F16) { src = fl16; n = 7; }
    else return 0;
    for (int i = 0; i < n && i < cap; ++i) tiles[i] = src[i];
    return n;
}

int pfk_adaptive_long_row_min(int dtype, int tile)
{
    int t[PFK_MAX_TILES];
    const int n = pfk_supported_tiles(PF_ADAPTIVE, dtype, t, PFK_MAX_TILES);
    for (int i = 0; i < n; ++i)
        if (t[i] == tile) return adaptive_lmax(tile);
    return -1;
}

int pfk_row_stats(const int *row_ptr, const int *col, int m, int n, long long nnz,
                  unsigned long long *d_out, void *stream)
{
    return launch_stats(row_ptr, col, m, n, nnz, d_out, nullptr, 0, stream);
}

int pfk_row_map(const pfk_spmv_args *a, void *stream)
{
    if (!a || !a->row_ptr || !a->row_map || a->m <= 0 || a->nnz <= 0 || !a->row_aligned ||
        (a->tile != 1024 && a->tile != 2048)) {
        snprintf(g_err, sizeof g_err, "pfk_row_map: a row-aligned FLAT plan of 1024 or 2048 nnz per tile");
        return PF_ERR_INVALID;
    }
    const long long nt = a->ntiles;
    if (nt != ((long long)a->nnz + a->tile - 1) / a->tile) {
        snprintf(g_err, sizeof g_err, "pfk_row_map: %lld tiles for %d nnz of %d per tile", nt, a->nnz, a->tile);
        return PF_ERR_INVALID;
    }
    if (!room(a->row_map, a->row_map_bytes, (nt + 1) * 8, "row map")) return PF_ERR_INVALID;
    const long long per_wg = kBS / kMapLanes;
    hipLaunchKernelGGL(k_row_map, dim3((unsigned)((nt + 1 + per_wg - 1) / per_wg)), dim3(kBS), 0, S(stream),
                       a->row_ptr, a->m, (int)a->nnz, a->tile, nt, a->guess_spread, a->guess_a, a->guess_b,
                       reinterpret_cast<int2 *>(a->row_map));
    PFK_LAUNCHED("k_row_map");
    return PF_OK;
}

int pfk_band_stats(const int *row_ptr, const int *col, int m, unsigned long long *out, void *stream)
{
    if (!row_ptr || !out || m < 0 || (m > 0 && !col)) return PF_ERR_INVALID;
    hipLaunchKernelGGL(k_fill_zero, dim3(1), dim3(kBS), 0, S(stream), reinterpret_cast<uint32_t *>(out),
                       (size_t)(2 * (PFK_BAND_WIDTHS + 1)));
    PFK_LAUNCHED("k_fill_zero");
    if (m > 0) {
        const long long blocks = (m + kBS - 1) / kBS;
        hipLaunchKernelGGL(k_band_stats, dim3(grid_for(blocks, PFK_BAND_SAMPLE, kBandStatsWg)), dim3(kBS), 0,
                           S(stream), row_ptr, col, m, out);
        PFK_LAUNCHED("k_band_stats");
    }
    return PF_OK;
}

int pfk_plan_scan(const int *row_ptr, const int *col, int m, int n, long long nnz, unsigned long long *d_out,
                  void *list, int cap, void *stream)
{
    if (!col && nnz > 0) return PF_ERR_INVALID;
    if (cap > 0 && !list) return PF_ERR_INVALID;
    return launch_stats(row_ptr, col, m, n, nnz, d_out, static_cast<int4 *>(list), cap, stream);
}

int pfk_debug_tile_desc(int dtype, int merged_keys, const pfk_spmv_args *a, int *d_out, void *stream)
{
    (void)dtype;
    if (!a || !a->row_ptr || !d_out || !a->err_flag || a->m <= 0 || a->ntiles < 1) return PF_ERR_INVALID;
    if (merged_keys) {  // the descriptors of the k_wave code path itself (independent of the value type)
        switch (a->tile) {
        case 188: return launch_stream<double, 188, adaptive_lmax(188), true>(a, d_out, stream);
        case 238: return launch_stream<double, 238, adaptive_lmax(238), true>(a, d_out, stream);
        case 440: return launch_stream<double, 440, adaptive_lmax(440), true>(a, d_out, stream);
        case 494: return launch_stream<double, 494, adaptive_lmax(494), true>(a, d_out, stream);
        case 512: return launch_stream<double, 512, adaptive_lmax(512), true>(a, d_out, stream);
        case 1024: return launch_stream<double, 1024, adaptive_lmax(1024), true>(a, d_out, stream);
        }
    } else {
        switch (a->tile) {  // the descriptors of the kernel each FLAT tile size runs
        case 1024: return launch_flat<double, 1024>(a, d_out, stream);
        case 2048: return launch_flat<double, 2048>(a, d_out, stream);
        case 4096: return launch_flat_desc<4096>(a, d_out, stream);
        }
    }
    return PF_ERR_UNSUPPORTED;
}

int pfk_probe_gather(int dtype, const int *idx, long long count, const void *x, long long n, void *out,
                     long long out_len, int policy, void *stream)
{
    if (!idx || !x || !out || count < 1 || count > 0x7FFFFFFFll || n < 1 || ((uintptr_t)idx & 15))
        return PF_ERR_INVALID;
    const long long vb = dtype == PF_F64 ? 8 : dtype == PF_F32 ? 4 : 0;
    if (!vb || n * vb >= (long long)kOob) return PF_ERR_INVALID;
    const long long tiles = (count + kProbeTile - 1) / kProbeTile;
    if (out_len < tiles * kWaves) {
        snprintf(g_err, sizeof g_err, "probe output holds %lld values, %lld needed", out_len, tiles * kWaves);
        return PF_ERR_INVALID;
    }
#define PF_PROBE(AUX)                                                                                          \
    case AUX:                                                                                                  \
        if (dtype == PF_F64)                                                                                   \
            hipLaunchKernelGGL((k_probe_gather<double, AUX>), dim3((unsigned)tiles), dim3(kBS), 0, S(stream), idx, \
                               count, static_cast<const double *>(x), n, static_cast<double *>(out));          \
        else                                                                                                   \
            hipLaunchKernelGGL((k_probe_gather<float, AUX>), dim3((unsigned)tiles), dim3(kBS), 0, S(stream), idx,  \
                               count, static_cast<const float *>(x), n, static_cast<float *>(out));            \
        break;
    switch (policy) {
    PF_PROBE(0) PF_PROBE(1) PF_PROBE(2) PF_PROBE(3) PF_PROBE(16) PF_PROBE(17) PF_PROBE(18) PF_PROBE(19)
    default:
        snprintf(g_err, sizeof g_err, "cache policy %d not compiled into the gather probe", policy);
        return PF_ERR_UNSUPPORTED;
    }
#undef PF_PROBE
    PFK_LAUNCHED("k_probe_gather");
    return PF_OK;
}

int pfk_debug_prefree_rows(const int *row_ptr, int m, int nnz, int tile, int *d_out, void *stream)
{
    if (!row_ptr || !d_out || m <= 0 || nnz <= 0 || tile <= 0) return PF_ERR_INVALID;
    const long long ntiles = ((long long)nnz + tile - 1) / tile;
    hipLaunchKernelGGL(k_prefree_rows, dim3((unsigned)(ntiles + 1)), dim3(kWave), 0, S(stream), row_ptr, m, nnz,
                       tile, ntiles, 0, d_out);
    PFK_LAUNCHED("k_prefree_rows");
    return PF_OK;
}

int pfk_malloc(void **p, size_t bytes)
{
    if (!p) return PF_ERR_INVALID;
    *p = nullptr;
    if (bytes == 0) return PF_OK;
    const hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) { hip_fail(e, "hipMalloc"); return PF_ERR_NOMEM; }
    return PF_OK;
}

int pfk_free(void *p)
{
    if (p) PFK_HIP(hipFree(p));
    return PF_OK;
}

int pfk_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream)
{
    if (bytes) PFK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, S(stream)));
    return PF_OK;
}

int pfk_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream)
{
    if (bytes) PFK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, S(stream)));
    return PF_OK;
}

int pfk_memcpy_d2d(void *dst, const void *src, size_t bytes, void *stream)
{
    if (bytes) PFK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, S(stream)));
    return PF_OK;
}

int pfk_fill_zero(void *p, size_t bytes, void *stream)
{
    if (!p || (bytes & 3)) return PF_ERR_INVALID;
    const size_t words = bytes / 4;
    if (!words) return PF_OK;
    const unsigned grid = grid_for((long long)words, kBS, 8192);
    hipLaunchKernelGGL(k_fill_zero, dim3(grid), dim3(kBS), 0, S(stream), static_cast<uint32_t *>(p), words);
    PFK_LAUNCHED("k_fill_zero");
    return PF_OK;
}

int pfk_fill_u32(void *p, size_t nwords, unsigned value, void *stream)
{
    if (!p) return PF_ERR_INVALID;
    if (!nwords) return PF_OK;
    const unsigned grid = grid_for((long long)nwords, kBS, 8192);
    hipLaunchKernelGGL(k_fill_u32, dim3(grid), dim3(kBS), 0, S(stream), static_cast<uint32_t *>(p), nwords,
                       (uint32_t)value);
    PFK_LAUNCHED("k_fill_u32");
    return PF_OK;
}

int pfk_stream_create(void **s)
{
    hipStream_t h;
    PFK_HIP(hipStreamCreateWithFlags(&h, hipStreamNonBlocking));
    *s = h;
    return PF_OK;
}

int pfk_stream_destroy(void *s) { if (s) PFK_HIP(hipStreamDestroy(S(s))); return PF_OK; }
int pfk_stream_sync(void *s) { PFK_HIP(hipStreamSynchronize(S(s))); return PF_OK; }

int pfk_event_create(void **e)
{
    hipEvent_t h;
    PFK_HIP(hipEventCreate(&h));
    *e = h;
    return PF_OK;
}

int pfk_event_create_fence(void **e)
{
    hipEvent_t h;
    PFK_HIP(hipEventCreateWithFlags(&h, hipEventDisableTiming));
    *e = h;
    return PF_OK;
}

int pfk_event_destroy(void *e) { if (e) PFK_HIP(hipEventDestroy(reinterpret_cast<hipEvent_t>(e))); return PF_OK; }
int pfk_event_record(void *e, void *s) { PFK_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(e), S(s))); return PF_OK; }
int pfk_event_sync(void *e) { PFK_HIP(hipEventSynchronize(reinterpret_cast<hipEvent_t>(e))); return PF_OK; }

int pfk_event_elapsed_ms(float *ms, void *start, void *stop)
{
    PFK_HIP(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start), reinterpret_cast<hipEvent_t>(stop)));
    return PF_OK;
}

int pfk_graph_begin(void *stream)
{
    if (!stream) {
        snprintf(g_err, sizeof g_err, "pfk_graph_begin: the null stream cannot be captured");
        return PF_ERR_INVALID;
    }
    PFK_HIP(hipStreamBeginCapture(S(stream), hipStreamCaptureModeThreadLocal));
    return PF_OK;
}

int pfk_graph_end(void *stream, void **exec)
{
    if (!exec) return PF_ERR_INVALID;
    *exec = nullptr;
    hipGraph_t g = nullptr;
    PFK_HIP(hipStreamEndCapture(S(stream), &g));
    hipGraphExec_t x = nullptr;
    const hipError_t e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);  // the executable graph keeps its own copy
    if (e != hipSuccess) {
        snprintf(g_err, sizeof g_err, "hipGraphInstantiate: %s", hipGetErrorString(e));
        return PF_ERR_HIP;
    }
    *exec = x;
    return PF_OK;
}

int pfk_graph_launch(void *exec, void *stream)
{
    PFK_HIP(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(exec), S(stream)));
    return PF_OK;
}

int pfk_graph_destroy(void *exec)
{
    if (exec) PFK_HIP(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(exec)));
    return PF_OK;
}

int pfk_device_count(int *n) { PFK_HIP(hipGetDeviceCount(n)); return PF_OK; }

int pfk_get_device(int *dev) { PFK_HIP(hipGetDevice(dev)); return PF_OK; }

int pfk_device_name(char *buf, int len)
{
    int dev = 0;
    PFK_HIP(hipGetDevice(&dev));
    hipDeviceProp_t p;
    PFK_HIP(hipGetDeviceProperties(&p, dev));
    snprintf(buf, (size_t)len, "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
    return PF_OK;
}

int pfk_scratch(void **ptr, size_t *bytes)
{
    if (!ptr || !bytes) return PF_ERR_INVALID;
    *ptr = nullptr;
    *bytes = 0;
    int dev = 0;
    PFK_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) {
        snprintf(g_err, sizeof g_err, "device %d: scratch is kept for devices 0..%d", dev, kMaxDevices - 1);
        return PF_ERR_UNSUPPORTED;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {  // once per device, with that device current
        void *p = nullptr;
        PFK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) {
            snprintf(g_err, sizeof g_err, "hipGetSymbolAddress(scratch) gave a null address");
            return PF_ERR_HIP;
        }
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    *bytes = PFK_SCRATCH_BYTES;
    return PF_OK;
}

const char *pfk_last_error(void) { return g_err; }

}  // extern "C"
