"""GPU parity at the benchmark's full sizes (C2-C5, the matrices bench.py measures).

At these sizes the checks are the ones that do not depend on size:
  * known-answer inputs (the reference's initVec values on val and x,
    include/common.h:126-133): every product is an integer <= 196 and every
    row sum is exact in the value type (below 2^53 in fp64; C2 and C4 rows stay
    below 2^24 in fp32), so y must equal the oracle bit for bit whatever the
    summation order;
  * U[-1,1] values: per row |y - y_ref| <= tol * sum_j |a_ij x_j| against the
    oracle (1e-12 fp64, 1e-5 fp32 with the oracle in fp64), empty rows exactly 0.
The oracle is the row-parallel C restatement of spmv_serial
(test/test_cdspmv.cpp:4-20), bit-identical to the serial loop.  y starts as
NaN, so every row must be written.  Each case prints its size before the GPU
step.
"""
import numpy as np
import pytest

import oracle
import prefree_amd as pf
from gpu_util import NP, TOL, gpu_spmv

pytestmark = pytest.mark.gpu

FULL = [(2, "f64"), (3, "f64"), (4, "f64"), (4, "f32"), (5, "f64")]


@pytest.mark.parametrize("cfg,dtype", FULL, ids=[f"C{c}-{d}" for c, d in FULL])
def test_full_size_known_answer_and_random(cfg, dtype):
    rp, col, kv = pf.synth_csr(cfg, seed=1, vals=1, dtypes=(dtype,))
    m, nnz = len(rp) - 1, len(col)
    kx = pf.synth_x(cfg, m, seed=1, vals=1, dtypes=(dtype,))[dtype]
    print(f"C{cfg} {dtype}: m={m} nnz={nnz}", flush=True)

    y, info = gpu_spmv(rp, col, kv[dtype], kx, "auto", dtype=dtype)
    ref = oracle.spmv_omp(rp, col, kv[dtype], kx)
    bad = np.flatnonzero(ref != y)
    assert bad.size == 0, f"C{cfg} {dtype} {info['variant_name']}: {bad.size} rows differ, first {bad[:5]}"
    del kv

    rng = np.random.default_rng(cfg)
    val = rng.uniform(-1, 1, nnz).astype(NP[dtype])
    x = rng.uniform(-1, 1, m).astype(NP[dtype])
    y, info = gpu_spmv(rp, col, val, x, "auto", dtype=dtype)
    v64, x64 = val.astype(np.float64, copy=False), x.astype(np.float64, copy=False)
    ref = oracle.spmv_omp(rp, col, v64, x64)
    err, zero_bad, worst = oracle.rownorm_maxerr(rp, col, v64, x64, ref, y.astype(np.float64))
    assert zero_bad == 0, f"C{cfg} {dtype}: {zero_bad} empty rows not exactly zero"
    assert err <= TOL[dtype], f"C{cfg} {dtype} {info['variant_name']}: row {worst} error {err:.3e}"
    print(f"C{cfg} {dtype} {info['variant_name']} {info['tile']}: known answer exact, U[-1,1] max error {err:.2e}",
          flush=True)


OTHER = [(5, "prefree", 0, 3), (5, "prefree", 1024, 4), (4, "prefree", 0, 3), (2, "adaptive", 0, 0),
         (5, "flat", 2048, 0)]


@pytest.mark.parametrize("cfg,variant,tile,ladder", OTHER,
                         ids=[f"C{c}-{v}-{t}-{l}" for c, v, t, l in OTHER])
def test_full_size_other_tilings(cfg, variant, tile, ladder):
    """The reference algorithm at full size, atomics on every tile-boundary row over C5's dense rows
    included, the ADAPTIVE tiling on C2, and C5 in split-row FLAT tiles (a plan whose dense rows are not
    made hybrid): known-answer inputs bit-exact, U[-1,1] within the tolerance."""
    rp, col, kv = pf.synth_csr(cfg, seed=1, vals=1, dtypes=("f64",))
    m, nnz = len(rp) - 1, len(col)
    kx = pf.synth_x(cfg, m, seed=1, vals=1, dtypes=("f64",))["f64"]
    print(f"C{cfg} {variant} tile {tile} ladder {ladder}: m={m} nnz={nnz}", flush=True)
    kw = {"ladder": ladder} if ladder else {}
    y, info = gpu_spmv(rp, col, kv["f64"], kx, variant, tile, **kw)
    assert info["variant_name"] == variant and not info["hybrid"]
    if ladder:
        assert info["ladder"] == ladder
    ref = oracle.spmv_omp(rp, col, kv["f64"], kx)
    bad = np.flatnonzero(ref != y)
    assert bad.size == 0, f"C{cfg} {variant}: {bad.size} rows differ, first {bad[:5]}"
    del kv
    rng = np.random.default_rng(cfg + 10)
    val = rng.uniform(-1, 1, nnz)
    x = rng.uniform(-1, 1, m)
    y, info = gpu_spmv(rp, col, val, x, variant, tile, **kw)
    ref = oracle.spmv_omp(rp, col, val, x)
    err, zero_bad, worst = oracle.rownorm_maxerr(rp, col, val, x, ref, y)
    assert zero_bad == 0 and err <= TOL["f64"], f"C{cfg} {variant}: row {worst} error {err:.3e}"
    print(f"C{cfg} {variant} {info['tile']}: known answer exact, U[-1,1] max error {err:.2e}", flush=True)
