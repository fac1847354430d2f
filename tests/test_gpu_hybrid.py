"""Hybrid plans on the GPU: dense rows by x windows, the rows between them in runs of row-aligned tiles.

PF_AUTO makes a split-row FLAT plan hybrid when every row longer than 256 nnz
is dense (at least the plan's threshold, 4096 nnz or more) and those rows'
columns are sorted.  Checked through the C ABI against the CPU oracle:
known-answer values bit for bit, U[-1,1] values within 1e-12 (f64) / 1e-5
(f32) / the fp16 bound per row normalised by sum |a_ij x_j| (fp16: dense mode,
no x halves, each row rounded once), the first call (which searches rows
and window bounds and records them) and later calls (which read them)
bit-identical, the split-row path of the same plan within tolerance, and
edge shapes: dense first and last rows, adjacent dense rows, empty rows and
empty runs between them, rectangular matrices, duplicate columns.
"""
import numpy as np
import pytest
import torch

import oracle
import prefree_amd as pf
from csr_cases import csr_from_lengths
from gpu_util import NP, TORCH, assert_parity, dev, gpu_spmv, kat_exact_possible

pytestmark = pytest.mark.gpu


def _lengths(pattern, rng, dense_len=(9000, 30000), short=(0, 60)):
    out = []
    for p in pattern:
        if p in ("D", "L"):  # a dense row, or a long row in the long-mode shapes
            out.append(int(rng.integers(*dense_len)))
        elif p == "E":
            out.append(0)
        else:
            out += [int(v) for v in rng.integers(short[0], short[1] + 1, size=int(p))]
    return out


SHAPES = {
    "dense_first_and_last": "D 300 D 500 D",
    "adjacent_dense": "40 D D D 200 D D 10",
    "empty_runs": "E E D E D E E E D 100 D E",
    "only_dense": "D D D",
    "single_dense_middle": "1000 D 1000",
    "many_short_runs": " ".join(["D 3"] * 60),
    "uneven_runs": "5000 D " + " ".join(["D 2"] * 40),
}


def _case(name, n=60000, seed=3):
    rng = np.random.default_rng(seed)
    lengths = _lengths(SHAPES[name].split(), rng)
    rp, col = csr_from_lengths(lengths, n, rng)
    return rp, col, n


@pytest.mark.parametrize("dtype", ["f64", "f32", "f16"])
@pytest.mark.parametrize("name", sorted(SHAPES))
def test_hybrid_shapes(name, dtype):
    rp, col, n = _case(name)
    rng = np.random.default_rng(1)
    kv, kx = oracle.initvec(len(col), NP[dtype]), oracle.initvec(n, NP[dtype])
    y, info = gpu_spmv(rp, col, kv, kx, "flat", dtype=dtype)
    assert info["hybrid"] == 1 and info["dense_rows"] == int(np.sum(np.diff(rp) > 256)), info
    assert info["x_halves"] == 0 or dtype != "f16"  # fp16 rounds each row once: no halves
    # fp16: the dense rows' KAT sums overflow binary16; the once-rounded model gives the same infinities
    assert_parity(rp, col, kv, kx, y, dtype, exact=kat_exact_possible(rp, dtype), what=f"{name}/kat")
    val = rng.uniform(-1, 1, len(col)).astype(NP[dtype])
    x = rng.uniform(-1, 1, n).astype(NP[dtype])
    y, _ = gpu_spmv(rp, col, val, x, "flat", dtype=dtype)
    assert_parity(rp, col, val, x, y, dtype, what=f"{name}/random")


@pytest.mark.parametrize("dtype", ["f64", "f32", "f16"])
def test_hybrid_scaled_c5(dtype):
    rp, col, v = pf.synth_csr(5, seed=9, scale_n=200000, dtypes=(dtype,))
    x = pf.synth_x(5, len(rp) - 1, seed=9, dtypes=(dtype,))[dtype]
    y, info = gpu_spmv(rp, col, v[dtype], x, "auto", dtype=dtype)
    assert info["hybrid"] == 1 and info["dense_rows"] == 200
    assert_parity(rp, col, v[dtype], x, y, dtype, what="C5/200000")
    kv, kx = oracle.initvec(len(col), NP[dtype]), oracle.initvec(len(x), NP[dtype])
    ky, _ = gpu_spmv(rp, col, kv, kx, "auto", dtype=dtype)
    assert_parity(rp, col, kv, kx, ky, dtype, exact=kat_exact_possible(rp, dtype), what="C5/200000/kat")


def test_hybrid_f16_refuses_x_halves():
    rp, col, n = _case("single_dense_middle")
    with pf.Plan(dev(rp), dev(col), len(rp) - 1, n, len(col), "f16", "flat") as p:
        assert p.info.hybrid == 1
        with pytest.raises(pf.PrefreeError) as e:
            p.set_x_halves(True)
        assert e.value.status == 5
    torch.cuda.synchronize()


def test_hybrid_rectangular_and_duplicates():
    rng = np.random.default_rng(7)
    lengths = _lengths("500 D 20 D 800".split(), rng)
    # n = 100000 columns for 1.3k rows: several x windows; duplicate (non-decreasing) columns in dense rows
    rp, col = csr_from_lengths(lengths, 100000, rng, distinct=False)
    for r in np.flatnonzero(np.diff(rp) > 256):
        assert np.all(np.diff(col[rp[r]:rp[r + 1]]) >= 0)
    val, x = oracle.initvec(len(col)), oracle.initvec(100000)
    y, info = gpu_spmv(rp, col, val, x, "flat")
    assert info["hybrid"] == 1
    assert_parity(rp, col, val, x, y, "f64", exact=True, what="rectangular")


def test_hybrid_refused_for_unsorted_or_medium_rows():
    rng = np.random.default_rng(8)
    lengths = _lengths("300 D 300 D".split(), rng)
    rp, col = csr_from_lengths(lengths, 50000, rng, sorted_cols=False)
    val, x = oracle.initvec(len(col)), oracle.initvec(50000)
    y, info = gpu_spmv(rp, col, val, x, "flat")
    assert info["hybrid"] == 0  # unsorted columns in the dense rows: split-row tiles
    assert_parity(rp, col, val, x, y, "f64", exact=True, what="unsorted")
    rp2, col2 = csr_from_lengths(lengths + [700], 50000, rng)  # a 700-nnz row is long but not dense
    val2 = oracle.initvec(len(col2))
    y2, info2 = gpu_spmv(rp2, col2, val2, x, "flat")
    assert info2["hybrid"] == 0
    assert_parity(rp2, col2, val2, x, y2, "f64", exact=True, what="medium row")


def test_hybrid_switch_and_search_modes():
    rp, col, n = _case("adjacent_dense", seed=11)
    rng = np.random.default_rng(12)
    val = rng.uniform(-1, 1, len(col))
    x = rng.uniform(-1, 1, n)
    d_rp, d_col, d_val, d_x = dev(rp), dev(col), dev(val), dev(x)
    m = len(rp) - 1
    y = torch.empty(m, dtype=torch.float64, device="cuda")
    outs = {}
    with pf.Plan(d_rp, d_col, m, n, len(col), "f64", "flat") as p:
        assert p.info.hybrid == 1
        for label, setup in (("first", None), ("memo", None), ("split", lambda: p.set_hybrid(False)),
                             ("back", lambda: p.set_hybrid(True)), ("search", lambda: p.set_remember_rows(False)),
                             ("rerecord", lambda: p.set_remember_rows(True)), ("memo2", None)):
            if setup:
                setup()
            y.fill_(float("nan"))
            p.execute(d_rp, d_col, d_val, d_x, y)
            p.check()
            outs[label] = y.cpu().numpy()
    for label in ("memo", "back", "search", "rerecord", "memo2"):
        assert np.array_equal(outs[label], outs["first"]), label
    assert_parity(rp, col, val, x, outs["first"], "f64", what="hybrid")
    assert_parity(rp, col, val, x, outs["split"], "f64", what="split-row")
    with pf.Plan(d_rp, d_col, m, n, len(col), "f64", "flat", 2048) as p:  # explicit tile: never hybrid
        assert p.info.hybrid == 0
        with pytest.raises(pf.PrefreeError):
            p.set_hybrid(True)


def test_hybrid_special_values():
    # NaN and infinities in x and val propagate exactly as in the serial sum (integer values otherwise),
    # including x entries next to a segment's end, whose products must not be formed.
    rp, col, n = _case("dense_first_and_last", seed=5)
    rng = np.random.default_rng(6)
    val, x = oracle.initvec(len(col)), oracle.initvec(n)
    for arr in (val, x):
        idx = rng.choice(len(arr), size=max(1, len(arr) // 700), replace=False)
        arr[idx] = rng.choice([np.nan, np.inf, -np.inf], size=len(idx))
    y, info = gpu_spmv(rp, col, val, x, "flat")
    assert info["hybrid"] == 1
    ref = oracle.spmv_serial(rp, col, val, x)
    assert np.array_equal(np.isnan(y), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(y[ok], ref[ok])


@pytest.mark.parametrize("dtype", ["f64", "f32"])
@pytest.mark.parametrize("name", sorted(SHAPES))
def test_hybrid_x_halves(name, dtype):
    # Run tiles processed once per half of x (XCDs 0-3 and 4-7), the halves' row sums added in order.
    rp, col, n = _case(name, seed=21)
    rng = np.random.default_rng(22)
    kv, kx = oracle.initvec(len(col), NP[dtype]), oracle.initvec(n, NP[dtype])
    y, info = gpu_spmv(rp, col, kv, kx, "flat", dtype=dtype, x_halves=True)
    assert info["hybrid"] == 1 and info["x_halves"] == 1
    assert_parity(rp, col, kv, kx, y, dtype, exact=kat_exact_possible(rp, dtype), what=f"{name}/halves/kat")
    val = rng.uniform(-1, 1, len(col)).astype(NP[dtype])
    x = rng.uniform(-1, 1, n).astype(NP[dtype])
    y, _ = gpu_spmv(rp, col, val, x, "flat", dtype=dtype, x_halves=True)
    assert_parity(rp, col, val, x, y, dtype, what=f"{name}/halves/random")


def test_hybrid_x_halves_special_values():
    # A column outside a workgroup's half must not multiply its value (inf * 0 would be NaN).
    rp, col, n = _case("many_short_runs", seed=23)
    rng = np.random.default_rng(24)
    val, x = oracle.initvec(len(col)), oracle.initvec(n)
    for arr in (val, x):
        idx = rng.choice(len(arr), size=max(1, len(arr) // 500), replace=False)
        arr[idx] = rng.choice([np.nan, np.inf, -np.inf], size=len(idx))
    y, info = gpu_spmv(rp, col, val, x, "flat", x_halves=True)
    assert info["x_halves"] == 1
    ref = oracle.spmv_serial(rp, col, val, x)
    assert np.array_equal(np.isnan(y), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(y[ok], ref[ok])


def test_full_c5_plan_choice():
    # C5 as bench.py measures it: hybrid with x halves (x = 8 MB), and the same y as the split-row plan
    # within rounding.
    rp, col, v = pf.synth_csr(5, seed=1, dtypes=("f64",))
    x = pf.synth_x(5, len(rp) - 1, seed=1)["f64"]
    y, info = gpu_spmv(rp, col, v["f64"], x, "auto")
    assert info["hybrid"] == 1 and info["x_halves"] == 1 and info["dense_rows"] == 1000
    assert_parity(rp, col, v["f64"], x, y, "f64", what="C5 hybrid")


# ---- long mode: long rows that are not all dense, cut into tiles dealt to the XCDs by their first column ----

LONG_SHAPES = {
    "long_mix": "200 L 300 L L 50 L 10",
    "long_first_and_last": "L 500 L 700 L",
    "only_long": "L L L L",
    "long_with_empty_runs": "E E L E L E E 80 L",
}


def _long_case(name, dtype, seed=31, sorted_cols=True):
    # x over one XCD's 4 MB L2 (long mode needs it); long rows of 300-6000 nnz (about 3000 on average,
    # so each holds a 1024-nnz tile or more on average), short rows of 0-60 nnz
    rng = np.random.default_rng(seed)
    n = 600000 if dtype == "f64" else 1100000
    lengths = _lengths(LONG_SHAPES[name].split(), rng, dense_len=(300, 6000))
    rp, col = csr_from_lengths(lengths, n, rng, sorted_cols=sorted_cols)
    return rp, col, n


@pytest.mark.parametrize("dtype", ["f64", "f32"])
@pytest.mark.parametrize("name", sorted(LONG_SHAPES))
def test_hybrid_long_mode_shapes(name, dtype):
    rp, col, n = _long_case(name, dtype)
    lens = np.diff(rp)
    rng = np.random.default_rng(2)
    kv, kx = oracle.initvec(len(col), NP[dtype]), oracle.initvec(n, NP[dtype])
    y, info = gpu_spmv(rp, col, kv, kx, "flat", dtype=dtype)
    n_long = int(np.sum(lens > 256))
    want_tiles = int(sum(-(-(rp[r + 1] - (rp[r] & ~63)) // 1024) for r in np.flatnonzero(lens > 256)))
    assert info["hybrid"] == 1 and info["dense_rows"] == n_long and info["long_tiles"] == want_tiles, info
    assert info["x_halves"] == 1
    assert_parity(rp, col, kv, kx, y, dtype, exact=kat_exact_possible(rp, dtype), what=f"{name}/kat")
    val = rng.uniform(-1, 1, len(col)).astype(NP[dtype])
    x = rng.uniform(-1, 1, n).astype(NP[dtype])
    y, _ = gpu_spmv(rp, col, val, x, "flat", dtype=dtype)
    assert_parity(rp, col, val, x, y, dtype, what=f"{name}/random")
    y, info = gpu_spmv(rp, col, val, x, "flat", dtype=dtype, x_halves=False)
    assert info["x_halves"] == 0
    assert_parity(rp, col, val, x, y, dtype, what=f"{name}/random/no halves")


def test_hybrid_long_mode_unsorted_columns():
    # long mode needs no sorted columns (only the XCD deal's locality does)
    rp, col, n = _long_case("long_mix", "f64", seed=33, sorted_cols=False)
    val, x = oracle.initvec(len(col)), oracle.initvec(n)
    y, info = gpu_spmv(rp, col, val, x, "flat")
    assert info["hybrid"] == 1 and info["long_tiles"] > 0
    assert_parity(rp, col, val, x, y, "f64", exact=True, what="long/unsorted")


def test_hybrid_long_mode_switch_and_search():
    rp, col, n = _long_case("long_mix", "f64", seed=35)
    rng = np.random.default_rng(36)
    val = rng.uniform(-1, 1, len(col))
    x = rng.uniform(-1, 1, n)
    d_rp, d_col, d_val, d_x = dev(rp), dev(col), dev(val), dev(x)
    m = len(rp) - 1
    y = torch.empty(m, dtype=torch.float64, device="cuda")
    outs = {}
    with pf.Plan(d_rp, d_col, m, n, len(col), "f64", "flat") as p:
        assert p.info.hybrid == 1 and p.info.long_tiles > 0
        for label, setup in (("first", None), ("memo", None), ("split", lambda: p.set_hybrid(False)),
                             ("back", lambda: p.set_hybrid(True)), ("search", lambda: p.set_remember_rows(False)),
                             ("memo2", lambda: p.set_remember_rows(True))):
            if setup:
                setup()
            y.fill_(float("nan"))
            p.execute(d_rp, d_col, d_val, d_x, y)
            p.check()
            outs[label] = y.cpu().numpy()
        assert p.info.long_tiles > 0
    for label in ("memo", "back", "search", "memo2"):
        assert np.array_equal(outs[label], outs["first"]), label
    assert_parity(rp, col, val, x, outs["first"], "f64", what="long hybrid")
    assert_parity(rp, col, val, x, outs["split"], "f64", what="long split-row")


def test_hybrid_long_mode_special_values():
    rp, col, n = _long_case("long_first_and_last", "f64", seed=37)
    rng = np.random.default_rng(38)
    val, x = oracle.initvec(len(col)), oracle.initvec(n)
    for arr in (val, x):
        idx = rng.choice(len(arr), size=max(1, len(arr) // 700), replace=False)
        arr[idx] = rng.choice([np.nan, np.inf, -np.inf], size=len(idx))
    y, info = gpu_spmv(rp, col, val, x, "flat")
    assert info["long_tiles"] > 0
    ref = oracle.spmv_serial(rp, col, val, x)
    assert np.array_equal(np.isnan(y), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(y[ok], ref[ok])


def test_hybrid_long_mode_refused_below_a_tile_per_row():
    # long rows of 257-600 nnz (under a 1024-nnz tile on average): the plan stays split-row
    rng = np.random.default_rng(39)
    lengths = _lengths("200 L 300 L L 50 L".split(), rng, dense_len=(257, 600))
    rp, col = csr_from_lengths(lengths, 600000, rng)
    val, x = oracle.initvec(len(col)), oracle.initvec(600000)
    y, info = gpu_spmv(rp, col, val, x, "flat")
    assert info["hybrid"] == 0
    assert_parity(rp, col, val, x, y, "f64", exact=True, what="short long rows")


def test_full_c3_plan_choice():
    # C3 as bench.py measures it: long mode (4442 long rows, most far below a dense row) with x halves
    rp, col, v = pf.synth_csr(3, seed=1, dtypes=("f64",))
    x = pf.synth_x(3, len(rp) - 1, seed=1)["f64"]
    y, info = gpu_spmv(rp, col, v["f64"], x, "auto")
    assert info["hybrid"] == 1 and info["x_halves"] == 1 and info["long_tiles"] > 0
    assert info["dense_rows"] == int(np.sum(np.diff(rp) > 256))
    assert_parity(rp, col, v["f64"], x, y, "f64", what="C3 long mode")


@pytest.mark.parametrize("kind", ["dense", "dense-halves", "long"])
def test_hybrid_graph_replays_match_eager(kind):
    # A hybrid plan whose x fits one XCD's L2 (the dense shapes here) runs its runs on a second stream beside
    # the dense rows' kernel, forked from and joined back to the caller's stream with events; the long shape
    # (x 4.8 MB) uses one stream.  Captured into a HIP graph on the plan's stream, every replay gives the eager
    # y bit for bit, with eager calls and synchronisation between the replays.
    if kind == "long":
        rp, col, n = _long_case("long_mix", "f64")
    else:
        rp, col, n = _case("many_short_runs", seed=41)
    rng = np.random.default_rng(42)
    m = len(rp) - 1
    val = rng.uniform(-1, 1, len(col))
    x = rng.uniform(-1, 1, n)
    d_rp, d_col, d_val, d_x = dev(rp), dev(col), dev(val), dev(x)
    y = torch.full((m,), float("nan"), dtype=torch.float64, device="cuda")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        plan = pf.Plan(d_rp, d_col, m, n, len(col), "f64", "flat", stream=s)
        assert plan.info.hybrid == 1
        if kind == "dense-halves":
            plan.set_x_halves(1)
        assert plan.info.x_halves == (0 if kind == "dense" else 1)
        plan.execute(d_rp, d_col, d_val, d_x, y, stream=s)     # first call: searches and records
        s.synchronize()
        eager = y.clone()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for _ in range(3):
                plan.execute(d_rp, d_col, d_val, d_x, y, stream=s)
        for rep in range(3):
            y.fill_(float("nan"))
            g.replay()
            s.synchronize()
            assert torch.equal(y, eager), f"replay {rep} differs from the eager result"
            y.fill_(0.0)
            plan.execute(d_rp, d_col, d_val, d_x, y, stream=s)
            s.synchronize()
            assert torch.equal(y, eager)
        plan.check(stream=s)
        plan.close()
    assert_parity(rp, col, val, x, eager.cpu().numpy(), "f64", what=f"{kind}/graph")


@pytest.mark.parametrize("halves", [False, True], ids=["one-pass", "x-halves"])
@pytest.mark.parametrize("dtype", ["f64", "f32"])
@pytest.mark.parametrize("name", sorted(SHAPES) + ["long:" + s for s in sorted(LONG_SHAPES)])
def test_hybrid_search_every_call(name, dtype, halves):
    # Calls that search (the run tiles' rows inside their runs, each tile's run in the run table, the dense
    # rows' window bounds) give the y of the calls that read what the first call recorded, bit for bit, on
    # every edge shape: many equal runs (the run lookup's proportional window), one long run before many
    # short ones (its fallback search), empty runs, dense or long rows first and last.
    if name.startswith("long:"):
        rp, col, n = _long_case(name[5:], dtype, seed=41)
    else:
        rp, col, n = _case(name, seed=41)
    rng = np.random.default_rng(42)
    val = rng.uniform(-1, 1, len(col)).astype(NP[dtype])
    x = rng.uniform(-1, 1, n).astype(NP[dtype])
    d_rp, d_col, d_val, d_x = dev(rp), dev(col), dev(val), dev(x)
    m = len(rp) - 1
    y = torch.empty(m, dtype=TORCH[dtype], device="cuda")
    outs = {}
    with pf.Plan(d_rp, d_col, m, n, len(col), dtype, "flat") as p:
        assert p.info.hybrid == 1
        p.set_x_halves(halves)
        assert p.info.x_halves == int(halves)
        for label, remember in (("first", True), ("memo", True), ("search", False), ("search2", False),
                                ("memo2", True)):
            p.set_remember_rows(remember)
            y.fill_(float("nan"))
            p.execute(d_rp, d_col, d_val, d_x, y)
            p.check()
            outs[label] = y.cpu().numpy()
    for label in ("memo", "search", "search2", "memo2"):
        assert np.array_equal(outs[label], outs["first"]), label
    assert_parity(rp, col, val, x, outs["first"], dtype, what=f"{name}/search every call")
