"""FLAT row groups (k_vector: FLAT "tiles" 2..32 are lanes per row) on the GPU, against the oracle.

Every edge case of csr_cases (empty rows, empty rows at both ends, one row, rows longer than the lanes and
than 256 nnz, duplicate and unsorted columns, rectangular x) and scaled C1, C2 and C4, for every lane count
and every value type, y NaN-prefilled before each call:

* initVec values bit for bit against spmv_serial (fp16: against the once-rounded exact sum): the products
  and partial sums are small integers, exact in any order;
* U[-1,1] values within the tolerance of assert_parity;
* the plan is one launch with no split-row workspace (row_aligned 1, needs_fixup 0, one workgroup per 256
  lanes) and the same y on its first and later calls.
"""
import numpy as np
import pytest

import oracle
import prefree_amd as pf
from csr_cases import edge_cases
from gpu_util import NP, assert_parity, gpu_spmv, kat_exact_possible

pytestmark = pytest.mark.gpu

LANES = [2, 4, 8, 16, 32]


def _cases():
    out = list(edge_cases())
    for cfg, scale in ((1, 0), (2, 200), (4, 300000)):
        rp, col, _ = pf.synth_csr(cfg, seed=3, scale_n=scale, dtypes=())
        out.append((f"C{cfg}", rp, col, len(rp) - 1))
    return out


CASES = _cases()


@pytest.mark.parametrize("dtype", ["f64", "f32", "f16"])
@pytest.mark.parametrize("lanes", LANES)
def test_row_groups_match_oracle(lanes, dtype):
    assert lanes in pf.supported_tiles("flat", dtype)
    for name, rp, col, n in CASES:
        m = len(rp) - 1
        if m == 0:
            continue
        what = f"{name} lanes={lanes} {dtype}"
        print(what, flush=True)
        kv, kx = oracle.initvec(len(col), NP[dtype]), oracle.initvec(n, NP[dtype])
        y, info = gpu_spmv(rp, col, kv, kx, "flat", tile=lanes, dtype=dtype)
        assert (info["tile"], info["row_aligned"], info["needs_fixup"]) == (lanes, 1, 0), what
        assert info["ntiles"] == max(1, -(-m * lanes // 256)), what
        assert_parity(rp, col, kv, kx, y, dtype, exact=kat_exact_possible(rp, dtype), what=what + " kat")
        rng = np.random.default_rng(lanes * 31 + len(col))
        uv = rng.uniform(-1, 1, len(col)).astype(NP[dtype])
        ux = rng.uniform(-1, 1, n).astype(NP[dtype])
        y, _ = gpu_spmv(rp, col, uv, ux, "flat", tile=lanes, dtype=dtype)
        assert_parity(rp, col, uv, ux, y, dtype, what=what + " random")


def test_auto_takes_row_groups_for_small_short_rows():
    """AUTO's rule on real plans: C1 takes 16 lanes, C2 at 512^2 (262,144 rows of 5) takes 2; one row more
    than 2^18 takes row-aligned tiles."""
    for cfg, scale, lanes in ((1, 0, 16), (2, 512, 2)):
        rp, col, v = pf.synth_csr(cfg, seed=1, scale_n=scale)
        x = pf.synth_x(cfg, len(rp) - 1, seed=1)["f64"]
        y, info = gpu_spmv(rp, col, v["f64"], x, "auto")
        assert (info["variant_name"], info["tile"]) == ("flat", lanes), (cfg, info)
        assert_parity(rp, col, v["f64"], x, y, "f64", what=f"C{cfg} auto")
    m = (1 << 18) + 1
    rp = np.arange(m + 1, dtype=np.int32) * 3
    col = (np.arange(3 * m, dtype=np.int64) * 7919 % m).astype(np.int32)
    y, info = gpu_spmv(rp, col, oracle.initvec(len(col)), oracle.initvec(m), "auto")
    assert info["tile"] in (1024, 2048) and info["row_aligned"] == 1, info


def test_row_groups_at_the_rule_bounds():
    """2^18 rows of up to 256 nnz: fp32 values and columns within 256 MB take row groups (half the mean row of
    48: 32 lanes), the same pattern at 128 nnz per row in fp64 (403 MB) takes tiles; both against the oracle."""
    rng = np.random.default_rng(17)
    m = 1 << 18
    for dtype, lam, want_groups in (("f32", 48.0, True), ("f64", 128.0, False)):
        lens = np.minimum(rng.poisson(lam, m), 256)
        rp = np.zeros(m + 1, dtype=np.int64)
        np.cumsum(lens, out=rp[1:])
        rp = rp.astype(np.int32)
        col = rng.integers(0, m, int(rp[-1])).astype(np.int32)
        val = oracle.initvec(len(col), NP[dtype])
        x = oracle.initvec(m, NP[dtype])
        print(f"bounds {dtype} nnz={len(col)}", flush=True)
        y, info = gpu_spmv(rp, col, val, x, "auto", dtype=dtype)
        groups = info["variant_name"] == "flat" and info["tile"] <= 32
        assert groups == want_groups, (dtype, info)
        if want_groups:
            assert info["tile"] == 32, info
        assert_parity(rp, col, val, x, y, dtype, exact=kat_exact_possible(rp, dtype), what=f"bounds {dtype}")
