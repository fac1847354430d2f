"""The band kernel (k_band) on the GPU, through the C ABI.

Row-aligned FLAT plans of matrices whose columns lie mostly within +-w of their row keep each step's band of
x in an LDS ring (pf_plan_set_band; on by default for matrices of under 4 nnz per row).  The band kernel reads
its steps from the plan's row map: the plan's first call searches the map afresh (k_row_map, one wave per tile)
and later calls read it; a plan that remembers no rows searches it on every call.  Checked against the CPU
oracle and against the tiles' own kernel on the same plan:

* known-answer values bit for bit; U[-1,1] values within 1e-12 (fp64) / 1e-5 (fp32) of sum |a_ij x_j|;
* the band kernel's y equals the tiles' kernel's y bit for bit (both sum each row in nnz order);
* scaled C4 and C2, banded matrices with outliers, bands wider and narrower than the columns' spread,
  steps of very many empty rows (windows that jump), rectangular x, fp64 and fp32;
* graph replays of a band plan equal its eager calls;
* pf_plan_set_band is refused for a plan without a band;
* the row-map search (pfk_row_map) gives, for every tile t, the first row whose row_ptr is at or above t·tile
  (numpy's searchsorted, side "left"), with its row_ptr, whatever the search's guess parameters.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
import prefree_amd as pf
from gpu_util import NP, TORCH, assert_parity, dev

pytestmark = pytest.mark.gpu


def _banded(m, lam, w, outliers, seed, n=None):
    """m rows of Poisson(lam) nnz; columns within +-w of the row, a share `outliers` anywhere; sorted per row."""
    rng = np.random.default_rng(seed)
    n = n or m
    lengths = rng.poisson(lam, size=m)
    rp = np.zeros(m + 1, dtype=np.int64)
    np.cumsum(lengths, out=rp[1:])
    row = np.repeat(np.arange(m, dtype=np.int64), lengths)
    lo, hi = np.maximum(0, row - w), np.minimum(n - 1, row + w)
    near = lo + (rng.random(len(row)) * (hi - lo + 1)).astype(np.int64)
    col = np.where(rng.random(len(row)) < outliers, rng.integers(0, n, len(row)), near)
    col = col[np.lexsort((col, row))]
    return rp.astype(np.int32), col.astype(np.int32), n


def _cases():
    out = []
    rp, col, _ = pf.synth_csr(4, seed=3, scale_n=1500000, dtypes=())
    out.append(("C4", rp, col, len(rp) - 1))
    rp, col, _ = pf.synth_csr(2, seed=3, scale_n=1100, dtypes=())
    out.append(("C2", rp, col, len(rp) - 1))
    out.append(("banded_w1024_o12",) + _banded(1200000, 1.0, 1024, 0.12, seed=1))
    out.append(("banded_w64",) + _banded(1200000, 1.5, 64, 0.0, seed=2))
    out.append(("banded_w1024_dense",) + _banded(1100000, 2.0, 1024, 0.1, seed=3))
    out.append(("wide_x",) + _banded(700000, 3.0, 2048, 0.05, seed=4, n=2100000))
    rng = np.random.default_rng(9)
    m = 3000000
    lengths = np.where(rng.random(m) < 0.05, rng.integers(1, 40, m), 0)
    lengths[:1000] = 30  # a dense start, then long runs of empty rows
    rp = np.zeros(m + 1, dtype=np.int64)
    np.cumsum(lengths, out=rp[1:])
    row = np.repeat(np.arange(m, dtype=np.int64), lengths)
    col = np.clip(row + rng.integers(-1500, 1501, len(row)), 0, m - 1)
    col = col[np.lexsort((col, row))]
    out.append(("empty_runs", rp.astype(np.int32), col.astype(np.int32), m))
    return out


CASES = _cases()


def _run(rp, col, val, x, dtype, band, repeat=3):
    m, n, nnz = len(rp) - 1, len(x), len(col)
    d_rp, d_col, d_val, d_x = dev(rp), dev(col), dev(val), dev(x)
    y = torch.full((m,), float("nan"), dtype=TORCH[dtype], device="cuda:0")
    outs = []
    with pf.Plan(d_rp, d_col, m, n, nnz, dtype, "flat") as p:
        info = p.info.as_dict()
        if band is not None:
            p.set_band(band)
        for _ in range(repeat):
            y.fill_(float("nan"))
            p.execute(d_rp, d_col, d_val, d_x, y)
            torch.cuda.synchronize()
            outs.append(y.cpu().numpy())
        p.check()
        info_after = p.info.as_dict()
    return outs, info, info_after


@pytest.mark.parametrize("dtype", ["f64", "f32"])
@pytest.mark.parametrize("case", range(len(CASES)), ids=[c[0] for c in CASES])
def test_band_parity(case, dtype):
    name, rp, col, n = CASES[case]
    assert int(np.diff(rp).max()) <= 256
    rng = np.random.default_rng(case)
    for kat in (True, False):
        if kat:
            val, x = oracle.initvec(len(col), NP[dtype]), oracle.initvec(n, NP[dtype])
        else:
            val = rng.uniform(-1, 1, len(col)).astype(NP[dtype])
            x = rng.uniform(-1, 1, n).astype(NP[dtype])
        outs, info, after = _run(rp, col, val, x, dtype, True)
        assert info["row_aligned"] == 1 and after["band_w"] > 0, (name, info, after)
        for y in outs[1:]:  # the band kernel's calls: the same as the first, searching call of the tiles' kernel
            assert np.array_equal(y, outs[0]), name
        assert_parity(rp, col, val, x, outs[-1], dtype, exact=kat, what=f"{name}/{dtype}/kat={kat}")
        tiles, _, _ = _run(rp, col, val, x, dtype, False, repeat=2)
        assert np.array_equal(outs[-1], tiles[-1]), f"{name}: band and tiles kernels differ"


def test_band_default_rule():
    name, rp, col, n = CASES[0]  # C4: under 4 nnz per row, band on by default
    d_rp, d_col = dev(rp), dev(col)
    with pf.Plan(d_rp, d_col, len(rp) - 1, n, len(col), "f64", "auto") as p:
        assert p.info.band_w == 4096, p.info.as_dict()
    name, rp, col, n = CASES[1]  # C2: 5 nnz per row, off by default (the plan has a band to switch on)
    d_rp, d_col = dev(rp), dev(col)
    with pf.Plan(d_rp, d_col, len(rp) - 1, n, len(col), "f64", "auto") as p:
        assert p.info.band_w == 0
        p.set_band(True)
        assert p.info.band_w > 0
    torch.cuda.synchronize()


def test_band_plan_searching_every_call():
    """A band plan told to search its rows on every call (pf_plan_set_remember_rows(plan, 0)) searches its row
    map afresh before each band kernel, with the remembering plan's y; switching back records the map again."""
    name, rp, col, n = CASES[0]
    m = len(rp) - 1
    val, x = oracle.initvec(len(col)), oracle.initvec(n)
    d_rp, d_col, d_val, d_x = dev(rp), dev(col), dev(val), dev(x)
    y = torch.full((m,), float("nan"), dtype=torch.float64, device="cuda:0")
    outs = []
    with pf.Plan(d_rp, d_col, m, n, len(col), "f64", "auto") as p:
        assert p.info.band_w > 0
        for remember in (True, False, False, True, True):
            p.set_remember_rows(remember)
            y.fill_(float("nan"))
            p.execute(d_rp, d_col, d_val, d_x, y)
            torch.cuda.synchronize()
            outs.append(y.cpu().numpy())
        p.check()
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])
    assert_parity(rp, col, val, x, outs[0], "f64", exact=True, what=name)


def test_band_refused_without_band():
    rp, col, _ = pf.synth_csr(2, seed=3, scale_n=300, dtypes=())  # x of 720 KB: no band
    with pf.Plan(dev(rp), dev(col), len(rp) - 1, len(rp) - 1, len(col), "f64", "auto") as p:
        with pytest.raises(pf.PrefreeError) as e:
            p.set_band(True)
        assert e.value.status == 5
    torch.cuda.synchronize()


def test_band_graph_replays():
    name, rp, col, n = CASES[0]
    m = len(rp) - 1
    val, x = oracle.initvec(len(col)), oracle.initvec(n)
    d_rp, d_col, d_val, d_x = dev(rp), dev(col), dev(val), dev(x)
    y = torch.full((m,), float("nan"), dtype=torch.float64, device="cuda:0")
    s = torch.cuda.Stream()
    with pf.Plan(d_rp, d_col, m, n, len(col), "f64", "auto", stream=s) as p:
        assert p.info.band_w > 0
        with torch.cuda.stream(s):
            p.execute(d_rp, d_col, d_val, d_x, y, stream=s)  # the first call records the map
            p.execute(d_rp, d_col, d_val, d_x, y, stream=s)
        s.synchronize()
        eager = y.cpu().numpy()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            p.execute(d_rp, d_col, d_val, d_x, y, stream=torch.cuda.current_stream())
        for _ in range(3):
            y.fill_(float("nan"))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(y.cpu().numpy(), eager)
        p.check(stream=s)
    assert np.array_equal(eager, oracle.spmv_serial(rp, col, val, x))


def _band_stats_np(rp, col):
    """pfk_band_stats restated: over the rows of every BAND_SAMPLE-th block of 256 rows, the nnz within
    +-(64 << i) of their row, and the sampled nnz."""
    m = len(rp) - 1
    blk = np.arange(m) // 256
    rows = np.flatnonzero(blk % pf.BAND_SAMPLE == 0)
    lens = np.diff(rp.astype(np.int64))[rows]
    row = np.repeat(rows.astype(np.int64), lens)
    idx = np.concatenate([np.arange(rp[r], rp[r + 1]) for r in rows]) if len(row) else np.zeros(0, np.int64)
    d = np.abs(col[idx].astype(np.int64) - row)
    return [int((d <= (64 << i)).sum()) for i in range(pf.BAND_WIDTHS)] + [len(row)]


@pytest.mark.parametrize("case", ["C2", "banded_w64", "empty_runs"])
def test_band_stats_sample(case):
    """The planning statistic equals its restatement over the same sample of rows."""
    _, rp, col, n = [c for c in CASES if c[0] == case][0]
    out = torch.zeros(pf.BAND_WIDTHS + 1, dtype=torch.int64, device="cuda")
    pf.band_stats(dev(rp), dev(col), len(rp) - 1, out)
    torch.cuda.synchronize()
    assert out.cpu().tolist() == _band_stats_np(rp, col), case


def _row_map_cases():
    rng = np.random.default_rng(77)
    out = []
    lens = rng.poisson(2.5, 300000)
    lens[rng.random(300000) < 0.3] = 0
    out.append(("poisson_empty", lens))
    out.append(("exact_256", np.full(8192, 256)))                      # every tile boundary a row start
    lens = rng.integers(0, 9, 200000)
    lens[50000:150000] = 0                                             # 100k empty rows in one stretch
    out.append(("empty_stretch", lens))
    out.append(("one_tile", rng.integers(0, 4, 300)))                  # nnz under a tile
    out.append(("multiple", np.full(4096, 4)))                         # nnz a multiple of both tiles
    lens = rng.integers(0, 3, 400000)
    lens[-1000:] = 200                                                 # a dense tail
    out.append(("dense_tail", lens))
    return out


@pytest.mark.parametrize("name,lens", _row_map_cases(), ids=[c[0] for c in _row_map_cases()])
@pytest.mark.parametrize("tile", [1024, 2048])
def test_row_map_search(name, lens, tile):
    rp = np.zeros(len(lens) + 1, dtype=np.int64)
    np.cumsum(lens, out=rp[1:])
    m, nnz = len(lens), int(rp[-1])
    nt = -(-nnz // tile)
    f = [0] + [int(np.searchsorted(rp, t * tile, side="left")) for t in range(1, nt)] + [m]
    want = np.array([(r, rp[r]) for r in f], dtype=np.int64)
    d_rp = dev(rp.astype(np.int32))
    out = torch.full((2 * (nt + 1),), -7, dtype=torch.int32, device="cuda:0")
    K = pf.klib()
    guesses = [(0, 0.0, 0.0), (16, 0.0, 0.0), (1, m / nnz, 3.0), (4, 1e-3, -5.0)]
    for spread, ga, gb in guesses:
        out.fill_(-7)
        a = pf.SpmvArgs(row_ptr=d_rp.data_ptr(), m=m, nnz=nnz, tile=tile, ntiles=nt, row_aligned=1,
                        row_map=out.data_ptr(), row_map_bytes=8 * (nt + 1), guess_spread=spread, guess_a=ga,
                        guess_b=gb)
        print(f"row map {name} tile={tile} m={m} nnz={nnz} guess=({spread}, {ga}, {gb})", flush=True)
        assert K.pfk_row_map(ctypes.byref(a), None) == 0, K.pfk_last_error()
        torch.cuda.synchronize()
        got = out.cpu().numpy().astype(np.int64).reshape(-1, 2)
        bad = np.nonzero((got != want).any(axis=1))[0]
        assert bad.size == 0, (name, tile, spread, ga, gb, bad[:5], got[bad[:5]], want[bad[:5]])


def test_row_map_refuses_bad_args():
    K = pf.klib()
    fake = 0x10000  # never dereferenced: refused on the host
    a = pf.SpmvArgs(row_ptr=fake, m=100, nnz=5000, tile=1024, ntiles=5, row_aligned=1, row_map=fake,
                    row_map_bytes=8 * 5)
    assert K.pfk_row_map(ctypes.byref(a), None) == 1 and b"row map" in K.pfk_last_error()
    a.row_map_bytes = 8 * 6
    a.ntiles = 4
    assert K.pfk_row_map(ctypes.byref(a), None) == 1  # ntiles is not ceil(nnz / tile)
    a.ntiles, a.tile = 5, 512
    assert K.pfk_row_map(ctypes.byref(a), None) == 1
