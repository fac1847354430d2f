"""GPU parity of the reference algorithm's five reduction ladders (PF_PREFREE).

Ladder codes 1..5 (src/spmv_kernel/preFreeSpMV.cu:440-559, the tuner's
TEST_CODE_VERSION, scripts/profile_and_generate.py:109-235) at P_NNZ 4 and 8
(512- and 1024-nnz tiles), through the C ABI (pf_plan_set_ladder):

* known-answer values (initVec): bit-exact against the serial oracle;
* U[-1,1] values: within 1e-12 (f64) / 1e-5 (f32) of it, per row normalised
  by sum |a_ij x_j|;
* f64 U[-1,1]: every row the reference stores plainly (not by atomicAdd) is
  bit-identical to the oracle's simulation of the same ladder
  (oracle.prefree_sim), which restates each warp-level tree; only the
  boundary rows' atomic order may differ.
"""
import numpy as np
import pytest

import oracle
import prefree_amd as pf
from csr_cases import csr_from_lengths, edge_cases
from gpu_util import NP, assert_parity, gpu_spmv, kat_exact_possible

pytestmark = pytest.mark.gpu

CASES = edge_cases()
LADDERS = [(code, tile) for code in (1, 2, 3, 4, 5) for tile in (512, 1024)]
IDS = [f"code{c}-tile{t}" for c, t in LADDERS]


def _check_against_sim(rp, col, val, x, y, code, tile, what):
    ysim, plain, _ = oracle.prefree_sim(rp, col, val, x, code=code, p_nnz=tile // 128, counts=True)
    rows = np.flatnonzero(plain > 0)
    bad = rows[y[rows] != ysim[rows]]
    assert bad.size == 0, f"{what}: {bad.size} plainly stored rows differ from the simulation, first {bad[:5]}"
    return rows.size


@pytest.mark.parametrize("code,tile", LADDERS, ids=IDS)
@pytest.mark.parametrize("dtype", ["f64", "f32"])
def test_ladder_edge_cases(code, tile, dtype):
    rng = np.random.default_rng(code * 100 + tile)
    for name, rp, col, n in CASES:
        kv, kx = oracle.initvec(len(col), NP[dtype]), oracle.initvec(n, NP[dtype])
        y, info = gpu_spmv(rp, col, kv, kx, "prefree", tile, dtype=dtype, ladder=code)
        assert info["ladder"] == code and info["tile"] == tile
        assert_parity(rp, col, kv, kx, y, dtype, exact=kat_exact_possible(rp, dtype), what=f"{name}/kat")
        val = rng.uniform(-1, 1, len(col)).astype(NP[dtype])
        x = rng.uniform(-1, 1, n).astype(NP[dtype])
        y, _ = gpu_spmv(rp, col, val, x, "prefree", tile, dtype=dtype, ladder=code)
        assert_parity(rp, col, val, x, y, dtype, what=f"{name}/random")
        if dtype == "f64":
            _check_against_sim(rp, col, val, x, y, code, tile, name)


SCALED = [(1, 0), (2, 300), (3, 60000), (4, 400000), (5, 40000)]


@pytest.mark.parametrize("code,tile", LADDERS, ids=IDS)
@pytest.mark.parametrize("cfg,scale", SCALED, ids=[f"C{c}" for c, _ in SCALED])
def test_ladder_scaled_configs(cfg, scale, code, tile):
    rp, col, v = pf.synth_csr(cfg, seed=13, scale_n=scale, dtypes=("f64",))
    x = pf.synth_x(cfg, len(rp) - 1, seed=13)["f64"]
    y, _ = gpu_spmv(rp, col, v["f64"], x, "prefree", tile, ladder=code)
    assert_parity(rp, col, v["f64"], x, y, "f64", what=f"C{cfg}/code{code}")
    plain_rows = _check_against_sim(rp, col, v["f64"], x, y, code, tile, f"C{cfg}/code{code}")
    assert plain_rows > 0 or cfg == 5
    kv, kx = oracle.initvec(len(col)), oracle.initvec(len(x))
    ky, _ = gpu_spmv(rp, col, kv, kx, "prefree", tile, ladder=code)
    assert_parity(rp, col, kv, kx, ky, "f64", exact=kat_exact_possible(rp, "f64"), what=f"C{cfg}/code{code}/kat")


@pytest.mark.parametrize("tile", [512, 1024])
def test_ladder4_long_short_tiles(tile):
    # Tiles of 2..32 rows dominated by one long row (> 90% of their nnz) take the
    # long/short split of ladder 4; some of their rows sum to exactly zero and are skipped.
    rng = np.random.default_rng(tile)
    lengths = []
    for _ in range(300):
        k = int(rng.integers(1, 8))
        lengths += [int(v) for v in rng.integers(1, 6, size=k)] + [int(rng.integers(tile - 40, tile - 10))]
    rp, col = csr_from_lengths(lengths, 5000, rng)
    val = rng.uniform(-1, 1, len(col))
    x = rng.uniform(-1, 1, 5000)
    for r in range(0, len(lengths), 7):  # plant exact zero sums
        a, b = rp[r], rp[r + 1]
        if b - a == 2:
            val[a], val[a + 1] = 1.0, -1.0
            x[col[a]] = x[col[a + 1]] = 0.5
    y, _ = gpu_spmv(rp, col, val, x, "prefree", tile, ladder=4)
    assert_parity(rp, col, val, x, y, "f64", what="long_short")
    assert _check_against_sim(rp, col, val, x, y, 4, tile, "long_short") > 100


def test_ladder_setter_rejects():
    import torch
    rp, col = csr_from_lengths([3, 3, 3], 4, np.random.default_rng(0))
    d_rp, d_col = torch.from_numpy(rp).cuda(), torch.from_numpy(col).cuda()
    with pf.Plan(d_rp, d_col, 3, 4, 9, "f64", "prefree") as p:
        for bad in (0, 6):
            with pytest.raises(pf.PrefreeError):
                p.set_ladder(bad)
    with pf.Plan(d_rp, d_col, 3, 4, 9, "f64", "flat") as p:
        with pytest.raises(pf.PrefreeError):
            p.set_ladder(3)
