// device_common.hpp — wave64 building blocks for the gfx950 CSR SpMV kernels.
//
// Cross-lane sums use DPP (quad_perm, row_half_mirror, row_mirror: fused into
// the VALU op) inside 16-lane rows and ds_swizzle across the two 16-lane rows
// of each 32-lane half; the two halves are joined with v_readlane.  No
// warp-32 shuffles anywhere.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pfdev {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef double f64x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kXcds = 8;  // MI355X: 8 XCDs, workgroups dispatched round-robin over them

// DPP controls, GFX9 encoding.
constexpr int kDppXor1 = 0xB1;        // quad_perm:[1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm:[2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // row_half_mirror: lane i <- lane 7-i in each 8-lane half-row
constexpr int kDppMirror = 0x140;     // row_mirror: lane i <- lane 15-i in each 16-lane row

// ds_swizzle bit mode: lane = ((lane & 0x1F) ^ xor) inside each 32-lane half.
template <int XOR>
constexpr int swizzle_xor_pattern() { return 0x1F | (XOR << 10); }

template <int CTRL, typename T>
__device__ __forceinline__ T dpp(T v)
{
    return __builtin_amdgcn_update_dpp(T(0), v, CTRL, 0xF, 0xF, false);
}

template <int PATTERN>
__device__ __forceinline__ double swizzle(double v)
{
    const int lo = __builtin_amdgcn_ds_swizzle(__double2loint(v), PATTERN);
    const int hi = __builtin_amdgcn_ds_swizzle(__double2hiint(v), PATTERN);
    return __hiloint2double(hi, lo);
}

template <int PATTERN>
__device__ __forceinline__ float swizzle(float v)
{
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), PATTERN));
}

__device__ __forceinline__ double readlane(double v, int lane)
{
    const int lo = __builtin_amdgcn_readlane(__double2loint(v), lane);
    const int hi = __builtin_amdgcn_readlane(__double2hiint(v), lane);
    return __hiloint2double(hi, lo);
}

__device__ __forceinline__ float readlane(float v, int lane)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Sum over all 64 lanes; every lane receives the same (deterministic) value.
// Must be called with the whole wave active.
template <typename T>
__device__ __forceinline__ T wave_sum(T v)
{
    v += dpp<kDppXor1>(v);
    v += dpp<kDppXor2>(v);
    v += dpp<kDppHalfMirror>(v);
    v += dpp<kDppMirror>(v);
    v += swizzle<swizzle_xor_pattern<16>()>(v);
    return readlane(v, 0) + readlane(v, 32);
}

// Sum over aligned groups of V lanes (V = 2, 4, 8, 16, 32); every lane of a
// group receives the group sum.  All lanes of each group must be active.
template <int V, typename T>
__device__ __forceinline__ T group_sum(T v)
{
    static_assert(V == 2 || V == 4 || V == 8 || V == 16 || V == 32, "group size");
    v += dpp<kDppXor1>(v);
    if constexpr (V >= 4) v += dpp<kDppXor2>(v);
    if constexpr (V >= 8) v += dpp<kDppHalfMirror>(v);
    if constexpr (V >= 16) v += dpp<kDppMirror>(v);
    if constexpr (V >= 32) v += swizzle<swizzle_xor_pattern<16>()>(v);
    return v;
}

// Reduction of a 32-bit value over all 64 lanes by an associative, commutative
// op (sum, max, min); every lane receives the result.  Whole wave active.
template <typename Op>
__device__ __forceinline__ unsigned int wave_reduce_u32(unsigned int v, Op op)
{
    v = op(v, dpp<kDppXor1>(v));
    v = op(v, dpp<kDppXor2>(v));
    v = op(v, dpp<kDppHalfMirror>(v));
    v = op(v, dpp<kDppMirror>(v));
    v = op(v, (unsigned int)__builtin_amdgcn_ds_swizzle((int)v, swizzle_xor_pattern<16>()));
    return op((unsigned int)__builtin_amdgcn_readlane((int)v, 0), (unsigned int)__builtin_amdgcn_readlane((int)v, 32));
}

// Key of row r: its first nnz index, plus r itself when tiles cut the merged
// (row, nnz) sequence.  Strictly increasing in r for MERGE, non-decreasing otherwise.
template <bool MERGE>
__device__ __forceinline__ uint32_t row_key(const int *__restrict__ rp, int r)
{
    return (uint32_t)rp[r] + (MERGE ? (uint32_t)r : 0u);
}

// Largest r in [0, m) with key(r) < v, or -1 when v == 0 (key(0) = row_ptr[0] = 0).
// Wave-cooperative 64-ary search: each round probes 64 evenly spaced rows and
// keeps the bracket, so m = 20M rows takes 5 rounds of dependent loads.  With
// spread > 0 a first round probes `guess + (lane-32)*spread`, which brackets
// the answer in one round for regular matrices.  Call with the whole wave
// active; the result is wave-uniform.  Every probe stays inside [0, m).
template <bool MERGE>
__device__ int wave_search_lt(const int *__restrict__ rp, int m, uint32_t v, long long guess,
                              int spread, int lane)
{
    if (v == 0)
        return -1;
    long long lo = 0, hi = m;  // key(lo) < v; hi == m or key(hi) >= v
    if (spread > 0) {
        const long long p = guess + (long long)(lane - 32) * spread;
        const bool valid = p > lo && p < hi;
        const uint32_t k = valid ? row_key<MERGE>(rp, (int)p) : 0u;
        const uint64_t okm = __ballot(valid && k < v);
        const uint64_t badm = __ballot(valid && k >= v);
        long long nlo = lo, nhi = hi;
        if (okm) nlo = guess + (long long)(63 - __clzll(okm) - 32) * spread;
        if (badm) nhi = guess + (long long)(__ffsll((long long)badm) - 1 - 32) * spread;
        if (nlo < nhi) { lo = nlo; hi = nhi; }
    }
    while (hi - lo > 1) {
        const long long step = (hi - lo + 63) >> 6;
        const long long p = lo + (long long)lane * step;
        const bool ok = lane > 0 && p < hi && row_key<MERGE>(rp, (int)p) < v;
        const int c = __popcll(__ballot(ok));
        lo += (long long)c * step;
        hi = (lo + step < hi) ? lo + step : hi;
    }
    return (int)lo;
}

// wave_search_lt for row_ptr itself (keys = row_ptr[r]), also returning
// row_ptr[result + 1]: the final round of the search probes that entry in
// most cases, and a lane's probe is read back instead of loaded again; only
// otherwise is it loaded.  Same preconditions; v > 0 and result + 1 <= m.
__device__ __forceinline__ int wave_search_lt_next(const int *__restrict__ rp, int m, uint32_t v, long long guess,
                                                   int spread, int lane, int &next_key)
{
    long long lo = 0, hi = m;
    if (spread > 0) {
        const long long p = guess + (long long)(lane - 32) * spread;
        const bool valid = p > lo && p < hi;
        const uint32_t k = valid ? (uint32_t)rp[(int)p] : 0u;
        const uint64_t okm = __ballot(valid && k < v);
        const uint64_t badm = __ballot(valid && k >= v);
        long long nlo = lo, nhi = hi;
        if (okm) nlo = guess + (long long)(63 - __clzll(okm) - 32) * spread;
        if (badm) nhi = guess + (long long)(__ffsll((long long)badm) - 1 - 32) * spread;
        if (nlo < nhi) { lo = nlo; hi = nhi; }
    }
    bool have = false;
    int key = 0;
    while (hi - lo > 1) {
        const long long step = (hi - lo + 63) >> 6;
        const long long p = lo + (long long)lane * step;
        const bool probe = lane > 0 && p < hi;
        const int k = probe ? rp[(int)p] : 0;
        const bool ok = probe && (uint32_t)k < v;
        const int c = __popcll(__ballot(ok));
        // lo + (c + 1) * step is the first probe at or past v, if it was made
        if (step == 1 && c + 1 < kWave && lo + c + 1 < hi) {
            have = true;
            key = __builtin_amdgcn_readlane(k, c + 1);
        }
        lo += (long long)c * step;
        hi = (lo + step < hi) ? lo + step : hi;
    }
    next_key = have ? key : rp[(int)lo + 1];
    return (int)lo;
}

}  // namespace pfdev
