// prefree_kernels.hip — gfx950 CSR SpMV kernels and the thin extern "C" HIP
// layer declared in include/prefree_kernels.h.
//
// Three kernel families compute y = A·x (y overwritten):
//
//  * k_tiles<MERGE=true>   (PF_ADAPTIVE)  CSR-adaptive row blocks found on the fly.
//    Tile t owns the keys [t*K, (t+1)*K) of the merged sequence in which row r
//    occupies keys row_ptr[r]+r .. row_ptr[r+1]+r (its nnz, then one key for
//    its end), so a tile holds at most K rows+nnz whatever the row lengths.
//    A row whose first key lies in the tile is reduced there whole, unless it
//    is longer than LMAX; such long rows are cut at tile edges and their
//    partials combined by k_fixup in tile order (deterministic, no atomics).
//  * k_tiles<MERGE=false>  (PF_FLAT)  the same machinery on plain nnz tiles
//    with LMAX = 0: every row crossing a tile edge is cut and combined.
//  * k_prefree             (PF_PREFREE)  the reference algorithm
//    (src/spmv_kernel/preFreeSpMV.cu:407-483): 128*P-nnz tiles, reduction
//    ladder "code 3", atomicAdd on tile-boundary rows over a zeroed y.  Its
//    first-row-per-tile map (the pre-pass pre_start_rowPerTile, :3-28) is
//    computed inside the kernel by a wave-cooperative search of row_ptr.
//
// No kernel needs a pre-pass: every workgroup finds its rows by searching
// row_ptr (device_common.hpp: wave_search_lt).
//
// Data path of k_tiles (one workgroup = 4 wave64s = one tile):
//   1. waves 0 and 1 search row_ptr for the rows at the two tile edges;
//   2. col / val of the tile's nnz range stream in as 16-byte non-temporal
//      loads (dwordx4: 4 col, 2 fp64 or 4 fp32 values per lane), x is gathered
//      with ordinary loads so it stays in L2 / MALL; products go to LDS;
//   3. rows of <= 16 products are summed by one lane each in nnz order
//      (the exact order of the reference spmv_serial, test/test_cdspmv.cpp:4-20),
//      rows of <= 512 by a wave (DPP sum), longer ones by the whole workgroup.
#include "../../include/prefree_c.h"
#include "../../include/prefree_kernels.h"
#include "device_common.hpp"

#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

using namespace pfdev;

namespace {

constexpr int kBS = 256;               // workgroup size for k_tiles: 4 waves
constexpr int kWaves = kBS / kWave;
constexpr int kThreadMax = 16;         // rows up to this length: one lane each
constexpr int kWaveMax = 512;          // rows up to this length: one wave each

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
    long long ntiles;
    long long g8;        // tiles per XCD (ceil(ntiles / 8))
    T *__restrict__ head;
    T *__restrict__ tail;
    int *__restrict__ owner;
    int *__restrict__ err;
};

// Long-row threshold of ADAPTIVE for tile size K: keeps a tile's nnz span
// (at most K + LMAX - 1, plus 3 for 16-byte alignment) within 1.5 K.
constexpr int adaptive_lmax(int K) { return K / 2 - 4; }

// Logical tile of this workgroup: XCD x (= blockIdx % 8) takes the contiguous
// tiles [x*g8, (x+1)*g8), so neighbouring rows (and their x entries) share an L2.
__device__ __forceinline__ long long xcd_tile(long long g8)
{
    const long long b = blockIdx.x;
    return (b % kXcds) * g8 + b / kXcds;
}

// ---- 16-byte streaming loads of 4 consecutive nnz -------------------------

__device__ __forceinline__ void load4(const int *__restrict__ col, const double *__restrict__ val,
                                      int e0, int nnz, int (&c)[4], double (&v)[4])
{
    if (e0 + 4 <= nnz) {
        const i32x4 cc = __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(col + e0));
        const f64x2 v0 = __builtin_nontemporal_load(reinterpret_cast<const f64x2 *>(val + e0));
        const f64x2 v1 = __builtin_nontemporal_load(reinterpret_cast<const f64x2 *>(val + e0 + 2));
        c[0] = cc.x; c[1] = cc.y; c[2] = cc.z; c[3] = cc.w;
        v[0] = v0.x; v[1] = v0.y; v[2] = v1.x; v[3] = v1.y;
    } else {  // the last vector of the matrix
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const bool in = e0 + j < nnz;
            c[j] = in ? col[e0 + j] : 0;
            v[j] = in ? val[e0 + j] : 0.0;
        }
    }
}

__device__ __forceinline__ void load4(const int *__restrict__ col, const float *__restrict__ val,
                                      int e0, int nnz, int (&c)[4], float (&v)[4])
{
    if (e0 + 4 <= nnz) {
        const i32x4 cc = __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(col + e0));
        const f32x4 vv = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(val + e0));
        c[0] = cc.x; c[1] = cc.y; c[2] = cc.z; c[3] = cc.w;
        v[0] = vv.x; v[1] = vv.y; v[2] = vv.z; v[3] = vv.w;
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const bool in = e0 + j < nnz;
            c[j] = in ? col[e0 + j] : 0;
            v[j] = in ? val[e0 + j] : 0.0f;
        }
    }
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

template <typename T, bool MERGE, int K, int LMAX>
__global__ __launch_bounds__(kBS) void k_tiles(Args<T> a)
{
    using S = TileShape<T, MERGE, K, LMAX>;
    __shared__ __attribute__((aligned(16))) T s_prod[S::kProd];
    __shared__ int s_rows[2];
    __shared__ int s_desc[6];
    __shared__ int s_nw, s_nb;
    __shared__ int s_wl[S::kWaveCap], s_wa[S::kWaveCap], s_wb[S::kWaveCap];
    __shared__ int s_bl[S::kBlockCap], s_ba[S::kBlockCap], s_bb[S::kBlockCap];
    __shared__ T s_red[kWaves];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const long long t = xcd_tile(a.g8);
    if (t >= a.ntiles)
        return;  // whole workgroup: padding of the XCD mapping

    uint32_t kb, ke;
    bool last;
    tile_keys<MERGE>(t, a.ntiles, K, a.m, a.nnz, kb, ke, last);
    search_tile_rows<MERGE>(a.rp, a.m, a.nnz, a.guess_spread, kb, ke, last, s_rows);
    __syncthreads();
    if (tid == 0) {
        const TileDesc d = make_desc<MERGE, LMAX, S::kSpanMax>(a.rp, a.m, a.nnz, kb, ke, s_rows[0],
                                                                s_rows[1], a.err);
        s_desc[0] = d.lo_row; s_desc[1] = d.nr; s_desc[2] = d.A; s_desc[3] = d.B;
        s_desc[4] = d.head; s_desc[5] = d.tail;
        s_nw = 0;
        s_nb = 0;
        a.owner[t] = d.tail ? d.lo_row + d.nr - 1 : -1;
    }
    __syncthreads();
    const int lo_row = s_desc[0], nr = s_desc[1], A = s_desc[2], B = s_desc[3];
    const int head = s_desc[4], tail = s_desc[5];
    const int base = A & ~3;
    const int nvec = B > A ? (B - base + 3) >> 2 : 0;

    // Stream col/val (16-byte non-temporal loads), gather x, products -> LDS.
    int c[S::kVPT][4];
    T v[S::kVPT][4];
#pragma unroll
    for (int k = 0; k < S::kVPT; ++k) {
        const int vec = tid + k * kBS;
        if (vec < nvec)
            load4(a.col, a.val, base + 4 * vec, a.nnz, c[k], v[k]);
    }
#pragma unroll
    for (int k = 0; k < S::kVPT; ++k) {
        const int vec = tid + k * kBS;
        if (vec < nvec) {
            T p[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = base + 4 * vec + j;
                p[j] = (e >= A && e < B) ? v[k][j] * a.x[c[k][j]] : T(0);
            }
            store4(s_prod + 4 * vec, p);
        }
    }
    __syncthreads();

    auto put = [&](int i, T s) {
        if (head && i == 0)
            a.head[t] = s;
        else if (tail && i == nr - 1)
            a.tail[t] = s;
        else
            a.y[lo_row + i] = s;
    };

    // Rows of <= kThreadMax products: one lane each, sequential in nnz order.
    for (int i = tid; i < nr; i += kBS) {
        const int r = lo_row + i;
        const int ra = max(a.rp[r], A);
        const int rb = min(a.rp[r + 1], B);
        const int a0 = ra - base;
        const int len = rb - ra;
        if (len <= kThreadMax) {
            T s = T(0);
            for (int q = 0; q < len; ++q)
                s += s_prod[a0 + q];
            put(i, s);
        } else if (len <= kWaveMax) {
            const int j = atomicAdd(&s_nw, 1);
            if (j < S::kWaveCap) { s_wl[j] = i; s_wa[j] = a0; s_wb[j] = a0 + len; }
        } else {
            const int j = atomicAdd(&s_nb, 1);
            if (j < S::kBlockCap) { s_bl[j] = i; s_ba[j] = a0; s_bb[j] = a0 + len; }
        }
    }
    __syncthreads();

    // Rows of <= kWaveMax products: one wave each.
    const int nw = min(s_nw, S::kWaveCap);
    for (int j = wave; j < nw; j += kWaves) {
        T s = T(0);
        for (int q = s_wa[j] + lane; q < s_wb[j]; q += kWave)
            s += s_prod[q];
        s = wave_sum(s);
        if (lane == 0)
            put(s_wl[j], s);
    }

    // Longer rows: the whole workgroup.
    const int nb = min(s_nb, S::kBlockCap);
    for (int j = 0; j < nb; ++j) {
        T s = T(0);
        for (int q = s_ba[j] + tid; q < s_bb[j]; q += kBS)
            s += s_prod[q];
        s = wave_sum(s);
        if (lane == 0)
            s_red[wave] = s;
        __syncthreads();
        if (tid == 0) {
            T tot = s_red[0];
#pragma unroll
            for (int w = 1; w < kWaves; ++w)
                tot += s_red[w];
            put(s_bl[j], tot);
        }
        __syncthreads();
    }
}

// Debug: the descriptor every tile of k_tiles computes.
template <bool MERGE, int K, int LMAX, int SPAN_MAX>
__global__ __launch_bounds__(kBS) void k_tile_desc(Args<double> a, int *__restrict__ out)
{
    __shared__ int s_rows[2];
    const long long t = xcd_tile(a.g8);
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
    if (t0 + tid < a.ntiles && a.owner[t0 + tid] >= 0)
        s_list[atomicAdd(&s_n, 1)] = tid;
    __syncthreads();
    const int n = s_n;
    for (int j = wave; j < n; j += kWaves) {
        const long long t = t0 + s_list[j];
        const int r = a.owner[t];
        const long long last_key = (long long)a.rp[r + 1] - 1 + (MERGE ? r : 0);
        const long long tb = last_key / K;  // last tile holding a piece of row r
        T s = T(0);
        for (long long u = t + 1 + lane; u <= tb; u += kWave)
            s += a.head[u];
        s = wave_sum(s);
        if (lane == 0)
            a.y[r] = a.tail[t] + s;
    }
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

template <typename T, int P>
__global__ __launch_bounds__(kPfBS) void k_prefree(Args<T> a)
{
    constexpr int TT = kPfBS * P;  // 512 nnz for P = 4 (preFreeSpMV.cu:587)
    constexpr int VPT = P / 4;     // 4-nnz vectors per lane
    __shared__ __attribute__((aligned(16))) T s_prod[TT];
    __shared__ int s_rows[2];
    __shared__ T s_warp[kPfBS / 32];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const long long b = xcd_tile(a.g8);
    if (b >= a.ntiles)
        return;
    const int m = a.m;

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

    // Product stage (:416-428), 16-byte loads.
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int off = 4 * (tid + k * kPfBS);
        const int e0 = (int)first + off;
        T p[4] = {T(0), T(0), T(0), T(0)};
        if (e0 < a.nnz) {
            int c[4];
            T v[4];
            load4(a.col, a.val, e0, a.nnz, c, v);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                p[j] = (e0 + j < a.nnz) ? v[j] * a.x[c[j]] : T(0);
        }
        store4(s_prod + off, p);
    }
    __syncthreads();

    // Row range (:429-438); the last tile ends at m.
    const int start = min(s_rows[0], m);
    int end = min(s_rows[1], m);
    if (a.rp[end] % TT != 0 || end == start)
        end = min(end + 1, m);
    const int nrows = end - start;

    auto range = [&](int r, int &lo, int &hi) {
        lo = max(0, a.rp[r] - (int)first);
        hi = min(TT, a.rp[r + 1] - (int)first);
    };
    auto put = [&](int r, T s) {
        if (r == start || r == end - 1)
            atomic_add(a.y + r, s);
        else
            a.y[r] = s;
    };

    if (nrows > kPfBS / 4) {
        // red_row_thread (:71-98)
        for (int r = start + tid; r < end; r += kPfBS) {
            int lo, hi;
            range(r, lo, hi);
            T s = T(0);
            for (int i = lo; i < hi; ++i)
                s += s_prod[i];
            put(r, s);
        }
    } else if (nrows == 1) {
        // red_row_block (:30-69): strided lane sums, a 32-lane tree per half
        // wave, then the four half-wave results summed in order.
        int lo, hi;
        range(start, lo, hi);
        T s = T(0);
        for (int j = lo + tid; j < hi; j += kPfBS)
            s += s_prod[j];
        s = half_wave_tree(s);
        if ((lane & 31) == 0)
            s_warp[tid >> 5] = s;
        __syncthreads();
        if (tid == 0) {
            T fin = T(0);
#pragma unroll
            for (int w = 0; w < kPfBS / 32; ++w)
                fin += s_warp[w];
            atomic_add(a.y + start, fin);
        }
    } else {
        // red_row_vector<4> (:116-150): 4 lanes per row; lane 0 of the group
        // ends with (l0 + l2) + (l1 + l3) as warpReduceSum<4> gives.
        const int g = tid >> 2, q = tid & 3;
        for (int r = start + g; r < end; r += kPfBS / 4) {
            int lo, hi;
            range(r, lo, hi);
            T s = T(0);
            for (int i = lo + q; i < hi; i += 4)
                s += s_prod[i];
            s += dpp<kDppXor2>(s);
            s += dpp<kDppXor1>(s);
            if (q == 0)
                put(r, s);
        }
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

// ---- statistics, fills -----------------------------------------------------

// Layout of the statistics block (unsigned long long):
enum StatSlot {
    kStMax = 0, kStMin = 1, kStEmpty = 2, kStDec = 3, kStFirst = 4, kStLast = 5, kStBadCol = 6,
    kStHist = 7, kStCount = 44
};

__global__ void k_stats_init(unsigned long long *out)
{
    const int i = threadIdx.x;
    if (i < kStCount)
        out[i] = (i == kStMin) ? ~0ull : 0ull;
}

__global__ __launch_bounds__(kBS) void k_row_stats(const int *__restrict__ rp, int m,
                                                   unsigned long long *__restrict__ out)
{
    __shared__ unsigned int s_hist[33];
    __shared__ unsigned int s_max, s_min, s_empty, s_dec;
    const int tid = threadIdx.x;
    if (tid < 33) s_hist[tid] = 0;
    if (tid == 0) { s_max = 0; s_min = 0xFFFFFFFFu; s_empty = 0; s_dec = 0; }
    __syncthreads();
    unsigned int lmax = 0, lmin = 0xFFFFFFFFu, lempty = 0, ldec = 0;
    for (long long r = (long long)blockIdx.x * kBS + tid; r < m; r += (long long)gridDim.x * kBS) {
        int len = rp[r + 1] - rp[r];
        if (len < 0) { ++ldec; len = 0; }
        const unsigned int u = (unsigned int)len;
        lmax = max(lmax, u);
        lmin = min(lmin, u);
        lempty += (u == 0);
        atomicAdd(&s_hist[u == 0 ? 0 : 32 - __clz(u)], 1u);
    }
    atomicMax(&s_max, lmax);
    atomicMin(&s_min, lmin);
    atomicAdd(&s_empty, lempty);
    atomicAdd(&s_dec, ldec);
    __syncthreads();
    if (tid < 33 && s_hist[tid]) atomicAdd(out + kStHist + tid, (unsigned long long)s_hist[tid]);
    if (tid == 0) {
        atomicMax(out + kStMax, (unsigned long long)s_max);
        atomicMin(out + kStMin, (unsigned long long)s_min);
        atomicAdd(out + kStEmpty, (unsigned long long)s_empty);
        atomicAdd(out + kStDec, (unsigned long long)s_dec);
        if (blockIdx.x == 0) {
            out[kStFirst] = (unsigned long long)(long long)rp[0];
            out[kStLast] = (unsigned long long)(long long)rp[m];
        }
    }
}

__global__ __launch_bounds__(kBS) void k_col_check(const int *__restrict__ col, long long nnz, int n,
                                                   unsigned long long *__restrict__ out)
{
    unsigned int bad = 0;
    for (long long j = (long long)blockIdx.x * kBS + threadIdx.x; j < nnz; j += (long long)gridDim.x * kBS) {
        const int c = __builtin_nontemporal_load(col + j);
        bad += (c < 0 || c >= n);
    }
    if (__ballot(bad != 0)) {
        for (int o = 32; o > 0; o >>= 1)
            bad += __shfl_down(bad, o);
        if ((threadIdx.x & (kWave - 1)) == 0 && bad)
            atomicAdd(out + kStBadCol, (unsigned long long)bad);
    }
}

__global__ __launch_bounds__(kBS) void k_fill_zero(uint32_t *__restrict__ p, size_t nwords)
{
    for (size_t i = (size_t)blockIdx.x * kBS + threadIdx.x; i < nwords; i += (size_t)gridDim.x * kBS)
        p[i] = 0u;
}

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

inline hipStream_t S(void *s) { return reinterpret_cast<hipStream_t>(s); }

inline unsigned grid_for(long long work, long long per_block, long long cap)
{
    long long g = (work + per_block - 1) / per_block;
    if (g > cap) g = cap;
    return (unsigned)(g < 1 ? 1 : g);
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
    r.ntiles = a->ntiles;
    r.g8 = (a->ntiles + kXcds - 1) / kXcds;
    r.head = static_cast<T *>(a->head_slot);
    r.tail = static_cast<T *>(a->tail_slot);
    r.owner = a->owner_row;
    r.err = a->err_flag;
    return r;
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

template <typename T, bool MERGE>
int dispatch_tiles(const pfk_spmv_args *a, void *stream)
{
    if constexpr (sizeof(T) == 8) {
        switch (a->tile) {
        case 1024: return launch_tiles<T, MERGE, 1024, MERGE ? adaptive_lmax(1024) : 0>(a, stream);
        case 2048: return launch_tiles<T, MERGE, 2048, MERGE ? adaptive_lmax(2048) : 0>(a, stream);
        case 4096: return launch_tiles<T, MERGE, 4096, MERGE ? adaptive_lmax(4096) : 0>(a, stream);
        }
    } else {
        switch (a->tile) {
        case 2048: return launch_tiles<T, MERGE, 2048, MERGE ? adaptive_lmax(2048) : 0>(a, stream);
        case 4096: return launch_tiles<T, MERGE, 4096, MERGE ? adaptive_lmax(4096) : 0>(a, stream);
        }
    }
    snprintf(g_err, sizeof g_err, "tile %d not compiled for this value type", a->tile);
    return PF_ERR_UNSUPPORTED;
}

template <bool MERGE, int K>
int launch_desc(const pfk_spmv_args *a, int *out, void *stream)
{
    constexpr int LMAX = MERGE ? adaptive_lmax(K) : 0;
    Args<double> r = make_args<double>(a);
    const long long grid = r.g8 * kXcds;
    hipLaunchKernelGGL((k_tile_desc<MERGE, K, LMAX, K + LMAX + 2>), dim3((unsigned)grid), dim3(kBS), 0,
                       S(stream), r, out);
    PFK_LAUNCHED("k_tile_desc");
    return PF_OK;
}

}  // namespace

extern "C" {

int pfk_spmv_adaptive(int dtype, const pfk_spmv_args *a, void *stream)
{
    if (a && a->m == 0 && a->nnz == 0) return PF_OK;
    if (!args_ok(a, true)) return PF_ERR_INVALID;
    return dtype == PF_F64 ? dispatch_tiles<double, true>(a, stream)
         : dtype == PF_F32 ? dispatch_tiles<float, true>(a, stream) : PF_ERR_INVALID;
}

int pfk_spmv_flat(int dtype, const pfk_spmv_args *a, void *stream)
{
    if (a && a->m == 0 && a->nnz == 0) return PF_OK;
    if (!args_ok(a, true)) return PF_ERR_INVALID;
    return dtype == PF_F64 ? dispatch_tiles<double, false>(a, stream)
         : dtype == PF_F32 ? dispatch_tiles<float, false>(a, stream) : PF_ERR_INVALID;
}

int pfk_spmv_fixup(int dtype, int merged_keys, const pfk_spmv_args *a, void *stream)
{
    if (a && a->m == 0 && a->nnz == 0) return PF_OK;
    if (!args_ok(a, true) || a->tile <= 0) return PF_ERR_INVALID;
    const unsigned grid = (unsigned)((a->ntiles + kBS - 1) / kBS);
    if (dtype == PF_F64) {
        Args<double> r = make_args<double>(a);
        if (merged_keys) hipLaunchKernelGGL((k_fixup<double, true>), dim3(grid), dim3(kBS), 0, S(stream), r, a->tile);
        else hipLaunchKernelGGL((k_fixup<double, false>), dim3(grid), dim3(kBS), 0, S(stream), r, a->tile);
    } else if (dtype == PF_F32) {
        Args<float> r = make_args<float>(a);
        if (merged_keys) hipLaunchKernelGGL((k_fixup<float, true>), dim3(grid), dim3(kBS), 0, S(stream), r, a->tile);
        else hipLaunchKernelGGL((k_fixup<float, false>), dim3(grid), dim3(kBS), 0, S(stream), r, a->tile);
    } else {
        return PF_ERR_INVALID;
    }
    PFK_LAUNCHED("k_fixup");
    return PF_OK;
}

int pfk_spmv_prefree(int dtype, const pfk_spmv_args *a, void *stream)
{
    if (a && a->m == 0 && a->nnz == 0) return PF_OK;
    if (!args_ok(a, false)) return PF_ERR_INVALID;
    const size_t ybytes = (size_t)a->m * (dtype == PF_F64 ? 8 : 4);
    int st = pfk_fill_zero(a->y, ybytes, stream);  // the reference memsets y, preFreeSpMV.cu:644
    if (st != PF_OK || a->nnz == 0) return st;
    const long long grid = ((a->ntiles + kXcds - 1) / kXcds) * kXcds;
    if (dtype == PF_F64) {
        Args<double> r = make_args<double>(a);
        if (a->tile == 512) hipLaunchKernelGGL((k_prefree<double, 4>), dim3((unsigned)grid), dim3(kPfBS), 0, S(stream), r);
        else if (a->tile == 1024) hipLaunchKernelGGL((k_prefree<double, 8>), dim3((unsigned)grid), dim3(kPfBS), 0, S(stream), r);
        else return PF_ERR_UNSUPPORTED;
    } else if (dtype == PF_F32) {
        Args<float> r = make_args<float>(a);
        if (a->tile == 512) hipLaunchKernelGGL((k_prefree<float, 4>), dim3((unsigned)grid), dim3(kPfBS), 0, S(stream), r);
        else if (a->tile == 1024) hipLaunchKernelGGL((k_prefree<float, 8>), dim3((unsigned)grid), dim3(kPfBS), 0, S(stream), r);
        else return PF_ERR_UNSUPPORTED;
    } else {
        return PF_ERR_INVALID;
    }
    PFK_LAUNCHED("k_prefree");
    return PF_OK;
}

int pfk_supported_tiles(int variant, int dtype, int *tiles, int cap)
{
    static const int f64_tiles[] = {1024, 2048, 4096};
    static const int f32_tiles[] = {2048, 4096};
    static const int pf_tiles[] = {512, 1024};
    const int *src;
    int n;
    if (variant == PF_PREFREE) { src = pf_tiles; n = 2; }
    else if (variant == PF_ADAPTIVE || variant == PF_FLAT) {
        if (dtype == PF_F64) { src = f64_tiles; n = 3; }
        else if (dtype == PF_F32) { src = f32_tiles; n = 2; }
        else return 0;
    } else return 0;
    for (int i = 0; i < n && i < cap; ++i) tiles[i] = src[i];
    return n;
}

int pfk_adaptive_long_row_min(int dtype, int tile)
{
    int t[4];
    const int n = pfk_supported_tiles(PF_ADAPTIVE, dtype, t, 4);
    for (int i = 0; i < n; ++i)
        if (t[i] == tile) return adaptive_lmax(tile);
    return -1;
}

int pfk_row_stats(const int *row_ptr, const int *col, int m, int n, long long nnz,
                  unsigned long long *d_out, void *stream)
{
    if (!row_ptr || !d_out || m < 0 || nnz < 0) return PF_ERR_INVALID;
    hipLaunchKernelGGL(k_stats_init, dim3(1), dim3(64), 0, S(stream), d_out);
    PFK_LAUNCHED("k_stats_init");
    if (m > 0) {
        const unsigned grid = grid_for(m, kBS, 2048);
        hipLaunchKernelGGL(k_row_stats, dim3(grid), dim3(kBS), 0, S(stream), row_ptr, m, d_out);
        PFK_LAUNCHED("k_row_stats");
    }
    if (col && nnz > 0) {
        const unsigned grid = grid_for(nnz, kBS, 4096);
        hipLaunchKernelGGL(k_col_check, dim3(grid), dim3(kBS), 0, S(stream), col, nnz, n, d_out);
        PFK_LAUNCHED("k_col_check");
    }
    return PF_OK;
}

int pfk_debug_tile_desc(int dtype, int merged_keys, const pfk_spmv_args *a, int *d_out, void *stream)
{
    (void)dtype;
    if (!a || !a->row_ptr || !d_out || !a->err_flag || a->m <= 0 || a->ntiles < 1) return PF_ERR_INVALID;
    switch (a->tile) {
    case 1024: return merged_keys ? launch_desc<true, 1024>(a, d_out, stream) : launch_desc<false, 1024>(a, d_out, stream);
    case 2048: return merged_keys ? launch_desc<true, 2048>(a, d_out, stream) : launch_desc<false, 2048>(a, d_out, stream);
    case 4096: return merged_keys ? launch_desc<true, 4096>(a, d_out, stream) : launch_desc<false, 4096>(a, d_out, stream);
    }
    return PF_ERR_UNSUPPORTED;
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

int pfk_event_destroy(void *e) { if (e) PFK_HIP(hipEventDestroy(reinterpret_cast<hipEvent_t>(e))); return PF_OK; }
int pfk_event_record(void *e, void *s) { PFK_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(e), S(s))); return PF_OK; }
int pfk_event_sync(void *e) { PFK_HIP(hipEventSynchronize(reinterpret_cast<hipEvent_t>(e))); return PF_OK; }

int pfk_event_elapsed_ms(float *ms, void *start, void *stop)
{
    PFK_HIP(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start), reinterpret_cast<hipEvent_t>(stop)));
    return PF_OK;
}

int pfk_device_count(int *n) { PFK_HIP(hipGetDeviceCount(n)); return PF_OK; }

int pfk_device_name(char *buf, int len)
{
    int dev = 0;
    PFK_HIP(hipGetDevice(&dev));
    hipDeviceProp_t p;
    PFK_HIP(hipGetDeviceProperties(&p, dev));
    snprintf(buf, (size_t)len, "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
    return PF_OK;
}

const char *pfk_last_error(void) { return g_err; }

}  // extern "C"
