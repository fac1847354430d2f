"""Helpers shared by the GPU tests: device copies and one SpMV through the C ABI."""
from __future__ import annotations

import numpy as np
import torch

import oracle
import prefree_amd as pf

DEV = "cuda:0"
# Per-row error normalised by sum_j |a_ij x_j|.  fp16: one rounding of the row sum to binary16
# (2^-11 = 4.9e-4 relative; in the subnormal range below 2^-14 an absolute 2^-25, allowed for
# separately as F16_ABS) plus fp32 accumulation, against fp64 on the same fp16 data.
TOL = {"f64": 1e-12, "f32": 1e-5, "f16": 1e-3}
F16_ABS = 2.0 ** -24
NP = {"f64": np.float64, "f32": np.float32, "f16": np.float16}
TORCH = {"f64": torch.float64, "f32": torch.float32, "f16": torch.float16}


def dev(a, min_len=4):
    a = np.ascontiguousarray(a)
    if a.size < min_len:  # keep a real allocation behind empty arrays
        a = np.concatenate([a, np.zeros(min_len - a.size, dtype=a.dtype)])
    return torch.from_numpy(a).to(DEV)


def gpu_spmv(rp, col, val, x, variant="auto", tile=0, dtype="f64", fill=float("nan"), repeat=2, row_aligned=None,
             x_windows=None, chunk_nnz=None, ladder=None, x_halves=None):
    """y = A·x on the GPU through pf_plan_create / pf_plan_execute; returns (y, plan info).

    The plan executes `repeat` times, y refilled with `fill` before each call,
    and the last call's y is returned.  A plan's first call may differ in
    kind from later ones (FLAT records the rows its search found and later
    calls read them), so the first and the last y must agree bit for bit
    (up to atomic ordering for the reference's PREFREE algorithm).
    row_aligned (FLAT 1024/2048): force row-aligned (1) or split-row (0) tiles; x_windows (split-row
    FLAT): force the x-window schedule on (1) or off (0); chunk_nnz (FLAT 1024/2048): the XCD chunk;
    ladder (PREFREE): the reduction ladder 1..5; x_halves (hybrid plans): run tiles per half of x."""
    m, n, nnz = len(rp) - 1, len(x), len(col)
    d_rp, d_col, d_val, d_x = dev(rp), dev(col), dev(val), dev(x)
    y = torch.full((max(m, 1),), fill, dtype=TORCH[dtype], device=DEV)
    stream = torch.cuda.current_stream()
    first = None
    with pf.Plan(d_rp, d_col, m, n, nnz, dtype, variant, tile, stream=stream) as p:
        if row_aligned is not None:
            p.set_row_aligned(row_aligned)
        if x_windows is not None:
            p.set_x_windows(x_windows)
        if chunk_nnz is not None:
            p.set_chunk_nnz(chunk_nnz)
        if ladder is not None:
            p.set_ladder(ladder)
        if x_halves is not None:
            p.set_x_halves(x_halves)
        for k in range(repeat):
            y.fill_(fill)
            p.execute(d_rp, d_col, d_val, d_x, y, stream=stream)
            if k == 0:
                torch.cuda.synchronize()
                first = y[:m].cpu().numpy()
        torch.cuda.synchronize()
        p.check(stream=stream)
        info = p.info.as_dict()
    out = y[:m].cpu().numpy()
    if info["variant_name"] != "prefree":
        assert np.array_equal(first, out, equal_nan=True), "first and repeated calls of one plan differ"
    return out, info


def kat_exact_possible(rp, dtype):
    """initVec values are integers <= 14; row sums stay exact below 2^53 (f64) / 2^24 (f32).  fp16 sums are
    formed in fp32 and rounded once: exact below 2^24, and any sum of 65520 or more (nonnegative terms, so
    every partial sum too) gives infinity either way, so fp16 always matches the rounded exact sum."""
    if dtype == "f16":
        return True
    longest = int(np.max(np.diff(rp))) if len(rp) > 1 else 0
    return longest * 196 < (2 ** 53 if dtype == "f64" else 2 ** 24)


def assert_parity(rp, col, val, x, y, dtype, exact=False, what=""):
    """exact: bit equality with the oracle in `dtype`.  Otherwise the normalised
    per-row error against the oracle; for f32 the oracle is evaluated in f64 on
    the same f32 data, because a sequential f32 sum of a row with 10^4-10^5
    terms is itself off by more than 1e-5 of sum_j |a_ij x_j|."""
    if dtype == "f16":
        ref = oracle.spmv_f16_rounded(rp, col, val, x)
        if exact:
            bad = np.flatnonzero(ref.view(np.uint16) != np.asarray(y, dtype=np.float16).view(np.uint16))
            assert bad.size == 0, f"{what}: {bad.size} rows differ, first {bad[:5]} ref {ref[bad[:3]]} got {y[bad[:3]]}"
            return 0.0
        v64, x64 = val.astype(np.float64), x.astype(np.float64)
        ref64 = oracle.spmv_serial(rp, col, v64, x64)
        den = oracle.spmv_serial(rp, col, np.abs(v64), np.abs(x64))      # sum_j |a_ij x_j|
        dev_ = np.abs(np.asarray(y, dtype=np.float64) - ref64)
        zero_bad = int(np.count_nonzero((den == 0) & (np.asarray(y, dtype=np.float64) != 0)))
        assert zero_bad == 0, f"{what}: {zero_bad} empty-denominator rows not exactly zero"
        bad = np.flatnonzero(~(dev_ <= TOL[dtype] * den + F16_ABS))
        assert bad.size == 0, (f"{what}: {bad.size} rows beyond {TOL[dtype]} * sum|a x| + 2^-24, first {bad[:5]} "
                               f"got {y[bad[:3]]} fp64 {ref64[bad[:3]]}")
        nz = den > 0
        return float((np.maximum(dev_[nz] - F16_ABS, 0) / den[nz]).max()) if nz.any() else 0.0
    ref = oracle.spmv_serial(rp, col, val, x)
    if exact:
        bad = np.flatnonzero(ref != y)
        assert bad.size == 0, f"{what}: {bad.size} rows differ, first {bad[:5]} ref {ref[bad[:3]]} got {y[bad[:3]]}"
        return 0.0
    if dtype == "f32":
        v64, x64 = val.astype(np.float64), x.astype(np.float64)
        err, zero_bad, worst = oracle.rownorm_maxerr(rp, col, v64, x64, oracle.spmv_serial(rp, col, v64, x64),
                                                     y.astype(np.float64))
    else:
        err, zero_bad, worst = oracle.rownorm_maxerr(rp, col, val, x, ref, y)
    assert zero_bad == 0, f"{what}: {zero_bad} empty-denominator rows not exactly zero"
    assert err <= TOL[dtype], f"{what}: normalised error {err:.3e} at row {worst} (tol {TOL[dtype]})"
    return err
