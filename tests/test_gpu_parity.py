"""GPU parity of every variant against the CPU oracle (through the C ABI).

Known-answer inputs (the reference's initVec values, include/common.h:126-133)
must match the oracle bit for bit; U[-1,1] inputs must be within 1e-12 (f64)
or 1e-5 (f32) per row, normalised by sum_j |a_ij x_j|, with empty rows exactly
zero.  y is pre-filled with NaN, so every row must be written.
"""
import numpy as np
import pytest

import oracle
import prefree_amd as pf
from csr_cases import csr_from_lengths, edge_cases
from gpu_util import NP, assert_parity, gpu_spmv, kat_exact_possible

pytestmark = pytest.mark.gpu

CASES = edge_cases()
VARIANTS = ["adaptive", "flat", "prefree"]


@pytest.mark.parametrize("dtype", ["f64", "f32"])
@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("case", range(len(CASES)), ids=[c[0] for c in CASES])
def test_edge_case_kat(case, variant, dtype):
    name, rp, col, n = CASES[case]
    val = oracle.initvec(len(col), NP[dtype])
    x = oracle.initvec(n, NP[dtype])
    y, _ = gpu_spmv(rp, col, val, x, variant, dtype=dtype)
    assert_parity(rp, col, val, x, y, dtype, exact=kat_exact_possible(rp, dtype), what=f"{name}/{variant}")


@pytest.mark.parametrize("dtype", ["f64", "f32"])
@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("case", range(len(CASES)), ids=[c[0] for c in CASES])
def test_edge_case_random(case, variant, dtype):
    name, rp, col, n = CASES[case]
    rng = np.random.default_rng(case)
    val = rng.uniform(-1, 1, len(col)).astype(NP[dtype])
    x = rng.uniform(-1, 1, n).astype(NP[dtype])
    y, _ = gpu_spmv(rp, col, val, x, variant, dtype=dtype)
    assert_parity(rp, col, val, x, y, dtype, what=f"{name}/{variant}")


SCALED = [(1, 0), (2, 300), (3, 60000), (4, 400000), (5, 40000)]


@pytest.mark.parametrize("dtype", ["f64", "f32"])
@pytest.mark.parametrize("variant", ["auto"] + VARIANTS)
@pytest.mark.parametrize("cfg,scale", SCALED, ids=[f"C{c}" for c, _ in SCALED])
def test_scaled_configs(cfg, scale, variant, dtype):
    rp, col, v = pf.synth_csr(cfg, seed=11, scale_n=scale, dtypes=(dtype,))
    x = pf.synth_x(cfg, len(rp) - 1, seed=11, dtypes=(dtype,))[dtype]
    y, info = gpu_spmv(rp, col, v[dtype], x, variant, dtype=dtype)
    assert_parity(rp, col, v[dtype], x, y, dtype, what=f"C{cfg}/{variant}")
    kval = oracle.initvec(len(col), NP[dtype])
    kx = oracle.initvec(len(x), NP[dtype])
    ky, _ = gpu_spmv(rp, col, kval, kx, variant, dtype=dtype)
    assert_parity(rp, col, kval, kx, ky, dtype, exact=kat_exact_possible(rp, dtype), what=f"C{cfg}/{variant}/kat")


@pytest.mark.parametrize("variant", ["adaptive", "flat"])
def test_tile_sizes(variant):
    for dtype in ("f64", "f32"):
        for tile in pf.supported_tiles(variant, dtype):
            for name, rp, col, n in CASES[::3]:
                rng = np.random.default_rng(tile)
                val = rng.uniform(-1, 1, len(col)).astype(NP[dtype])
                x = rng.uniform(-1, 1, n).astype(NP[dtype])
                y, info = gpu_spmv(rp, col, val, x, variant, tile=tile, dtype=dtype)
                assert info["tile"] == tile
                assert_parity(rp, col, val, x, y, dtype, what=f"{name}/{variant}/{tile}")


@pytest.mark.parametrize("run", [1, 2, 5, 16, 64])
def test_adaptive_run_lengths(run):
    """Any number of consecutive tiles per wave gives the same (bit-identical) y."""
    import torch
    from gpu_util import DEV, dev
    for cfg, scale in ((3, 60000), (5, 40000), (4, 400000)):
        rp, col, v = pf.synth_csr(cfg, seed=8, scale_n=scale)
        m = len(rp) - 1
        x = pf.synth_x(cfg, m, seed=8)["f64"]
        d = [dev(rp), dev(col), dev(v["f64"]), dev(x)]
        ys = []
        for r in (8, run):
            y = torch.full((m,), float("nan"), dtype=torch.float64, device=DEV)
            with pf.Plan(d[0], d[1], m, m, len(col), "f64", "adaptive") as p:
                p.set_run_tiles(r)
                p.execute(*d, y)
                torch.cuda.synchronize()
                p.check()
            ys.append(y.cpu().numpy())
        assert np.array_equal(ys[0], ys[1])
        assert_parity(rp, col, v["f64"], x, ys[1], "f64", what=f"C{cfg} run {run}")


@pytest.mark.parametrize("run", [1, 2, 3, 8, 64])
def test_flow_run_lengths(run):
    """FLAT 256 (rows carried across tile edges): any run length, KAT exact, U[-1,1] within tolerance."""
    import torch
    from gpu_util import DEV, dev
    for cfg, scale in ((2, 300), (3, 60000), (5, 40000), (4, 400000), (1, 0)):
        rp, col, v = pf.synth_csr(cfg, seed=13, scale_n=scale)
        m = len(rp) - 1
        x = pf.synth_x(cfg, m, seed=13)["f64"]
        d = [dev(rp), dev(col), dev(v["f64"]), dev(x)]
        kv, kx = oracle.initvec(len(col), np.float64), oracle.initvec(m, np.float64)
        with pf.Plan(d[0], d[1], m, m, len(col), "f64", "flat", 256) as p:
            p.set_run_tiles(run)
            for vals, xs, exact in ((v["f64"], x, False), (kv, kx, kat_exact_possible(rp, "f64"))):
                y = torch.full((m,), float("nan"), dtype=torch.float64, device=DEV)
                p.execute(d[0], d[1], dev(vals), dev(xs), y)
                torch.cuda.synchronize()
                assert_parity(rp, col, vals, xs, y.cpu().numpy(), "f64", exact=exact, what=f"C{cfg} flow run {run}")
            p.check()


def test_flow_short_rows_bit_exact_within_runs():
    """Rows of <= 16 nnz that do not cross a run edge are summed in nnz order, even across tile edges."""
    import torch
    from gpu_util import DEV, dev
    rp, col, v = pf.synth_csr(2, seed=14, scale_n=300)
    m = len(rp) - 1
    x = pf.synth_x(2, m, seed=14)["f64"]
    d = [dev(rp), dev(col), dev(v["f64"]), dev(x)]
    with pf.Plan(d[0], d[1], m, m, len(col), "f64", "flat", 256) as p:
        p.set_run_tiles(1 << 8)   # runs of 256 tiles: 65536 nnz, so the matrix spans few runs
        y = torch.full((m,), float("nan"), dtype=torch.float64, device=DEV)
        p.execute(*d, y)
        torch.cuda.synchronize()
    ref = oracle.spmv_serial(rp, col, v["f64"], x)
    got = y.cpu().numpy()
    run_nnz = 256 * 256
    crossing = (rp[:-1] // run_nnz) != ((np.maximum(rp[1:], rp[:-1] + 1) - 1) // run_nnz)
    assert np.array_equal(got[~crossing], ref[~crossing])
    assert_parity(rp, col, v["f64"], x, got, "f64", what="flow C2")


def test_adaptive_cache_policy_bit_identical():
    """Ordinary and non-temporal col/val loads give the same y bit for bit."""
    import torch
    from gpu_util import DEV, dev
    for cfg, scale in ((2, 300), (5, 40000)):
        rp, col, v = pf.synth_csr(cfg, seed=12, scale_n=scale)
        m = len(rp) - 1
        x = pf.synth_x(cfg, m, seed=12)["f64"]
        d = [dev(rp), dev(col), dev(v["f64"]), dev(x)]
        ys = []
        with pf.Plan(d[0], d[1], m, m, len(col), "f64", "adaptive") as p:
            for keep in (0, 1):
                p.set_keep_cached(keep)
                y = torch.full((m,), float("nan"), dtype=torch.float64, device=DEV)
                p.execute(*d, y)
                torch.cuda.synchronize()
                ys.append(y.cpu().numpy())
            p.check()
        assert np.array_equal(ys[0], ys[1])
        assert_parity(rp, col, v["f64"], x, ys[0], "f64", what=f"C{cfg} cache policy")


def test_adaptive_short_rows_bit_exact():
    """Rows of <= 16 products are summed in nnz order by one lane: the oracle's order exactly."""
    for cfg, scale in ((2, 300), (4, 400000), (1, 0)):
        rp, col, v = pf.synth_csr(cfg, seed=3, scale_n=scale)
        x = pf.synth_x(cfg, len(rp) - 1, seed=3)["f64"]
        y, info = gpu_spmv(rp, col, v["f64"], x, "adaptive")
        assert info["needs_fixup"] == 0
        assert_parity(rp, col, v["f64"], x, y, "f64", exact=True, what=f"C{cfg}")


ALIGN_MAX = 256   # PFK_ALIGN_ROW_MAX


def short_row_cases():
    out = [(name, rp, col, n) for name, rp, col, n in CASES if len(rp) > 1 and np.diff(rp).max() <= ALIGN_MAX]
    for cfg, scale in ((1, 0), (2, 300), (4, 400000)):
        rp, col, _ = pf.synth_csr(cfg, seed=21, scale_n=scale, dtypes=())
        out.append((f"C{cfg}", rp, col, len(rp) - 1))
    return out


@pytest.mark.parametrize("dtype", ["f64", "f32"])
@pytest.mark.parametrize("tile", [1024, 2048])
def test_flat_row_aligned_and_split_tiles(tile, dtype):
    """Short-row matrices: FLAT plans pick row-aligned tiles (one launch, no split row); forcing
    split-row tiles gives the same y.  KAT inputs are bit-exact both ways; with U[-1,1] inputs the
    row-aligned y of rows <= 16 nnz is bit-exact too, each row being summed whole by one lane."""
    for name, rp, col, n in short_row_cases():
        ys = {}
        for ra in (None, 0):
            kv = oracle.initvec(len(col), NP[dtype])
            kx = oracle.initvec(n, NP[dtype])
            y, info = gpu_spmv(rp, col, kv, kx, "flat", tile=tile, dtype=dtype, row_aligned=ra)
            assert info["tile"] == tile
            if ra is None:
                assert info["row_aligned"] == 1 and info["needs_fixup"] == 0, name
            else:
                assert info["row_aligned"] == 0 and info["needs_fixup"] == int(info["ntiles"] > 1), name
            if kat_exact_possible(rp, dtype):
                assert_parity(rp, col, kv, kx, y, dtype, exact=True, what=f"{name}/kat/ra={ra}")
            rng = np.random.default_rng(tile + len(col))
            val = rng.uniform(-1, 1, len(col)).astype(NP[dtype])
            x = rng.uniform(-1, 1, n).astype(NP[dtype])
            y, _ = gpu_spmv(rp, col, val, x, "flat", tile=tile, dtype=dtype, row_aligned=ra)
            assert_parity(rp, col, val, x, y, dtype, what=f"{name}/random/ra={ra}")
            ys[ra] = y
        ref = oracle.spmv_serial(rp, col, val, x)
        short = np.diff(rp) <= 16
        assert np.array_equal(ys[None][short], ref[short]), name


CHUNKS = [0, 1, 3000, 1 << 15, 1 << 40]   # one chunk per XCD, one tile per chunk, ..., one round


@pytest.mark.parametrize("dtype", ["f64", "f32", "f16"])
@pytest.mark.parametrize("tile", [1024, 2048])
def test_flat_xcd_chunks_same_y(tile, dtype):
    """FLAT tiles dealt to the XCDs in chunks of any size give the same y bit for bit, row-aligned
    and split-row, on tile counts that fill no round of chunks evenly; y starts as NaN, so a tile
    left out or computed twice shows."""
    cases = [(name, rp, col, n) for name, rp, col, n in short_row_cases() if len(col) > 0]
    rng = np.random.default_rng(41)
    lens = rng.integers(0, 40, size=9001)                       # ragged rows, 180k nnz
    rp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    col = rng.integers(0, 9001, size=int(rp[-1])).astype(np.int32)
    cases.append(("ragged", rp, col, 9001))
    for name, rp, col, n in cases:
        rng = np.random.default_rng(len(col))
        val = rng.uniform(-1, 1, len(col)).astype(NP[dtype])
        x = rng.uniform(-1, 1, n).astype(NP[dtype])
        for ra in (None, 0):
            ys = []
            for chunk in CHUNKS:
                y, info = gpu_spmv(rp, col, val, x, "flat", tile=tile, dtype=dtype, row_aligned=ra, chunk_nnz=chunk)
                assert info["chunk_nnz"] == chunk and info["grid"] % 8 == 0 and info["grid"] >= info["ntiles"]
                ys.append(y)
            for chunk, y in zip(CHUNKS[1:], ys[1:]):
                assert np.array_equal(y, ys[0], equal_nan=True), (name, ra, chunk)
            assert_parity(rp, col, val, x, ys[0], dtype, what=f"{name}/ra={ra}")


def test_chunk_setter_rejects():
    from gpu_util import dev
    rp, col, _ = pf.synth_csr(2, seed=3, scale_n=64, dtypes=())
    d_rp, d_col = dev(rp), dev(col)
    with pf.Plan(d_rp, d_col, len(rp) - 1, len(rp) - 1, len(col), "f64", "flat", 1024) as p:
        assert p.info.chunk_nnz == 1 << 15                    # 5 nnz per row: chunks of 2^15 nnz
        with pytest.raises(pf.PrefreeError):
            p.set_chunk_nnz(-1)
    with pf.Plan(d_rp, d_col, len(rp) - 1, len(rp) - 1, len(col), "f64", "adaptive", 0) as p:
        with pytest.raises(pf.PrefreeError):
            p.set_chunk_nnz(1 << 15)


def test_row_aligned_refused_for_long_rows():
    import torch
    from gpu_util import dev
    for name, rp, col, n in CASES:
        if len(rp) < 2 or np.diff(rp).max() <= ALIGN_MAX or len(col) < 2048:
            continue
        d_rp, d_col = dev(rp), dev(col)
        with pf.Plan(d_rp, d_col, len(rp) - 1, n, len(col), "f64", "flat", 1024) as p:
            assert p.info.row_aligned == 0, name
            with pytest.raises(pf.PrefreeError):
                p.set_row_aligned(1)
            p.set_row_aligned(0)
        torch.cuda.synchronize()


def x_window_cases():
    out = [(name, rp, col, n) for name, rp, col, n in CASES if len(col) > 4096]
    for cfg, scale in ((5, 40000), (3, 60000)):
        rp, col, _ = pf.synth_csr(cfg, seed=23, scale_n=scale, dtypes=())
        out.append((f"C{cfg}", rp, col, len(rp) - 1))
    # long rows whose columns all lie in the first eighth of x: every tile picks list 0, so all but
    # cap of them go through the overflow list to the other XCDs' spare slots
    rng = np.random.default_rng(31)
    lens = rng.integers(3000, 9000, size=40)
    rp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    n = 80000
    col = np.concatenate([np.sort(rng.choice(n // 8, size=k, replace=False)) for k in lens]).astype(np.int32)
    out.append(("skewed_first_eighth", rp, col, n))
    return out


@pytest.mark.parametrize("dtype", ["f64", "f32", "f16"])
@pytest.mark.parametrize("tile", [1024, 2048])
def test_flat_x_window_schedule_same_y(tile, dtype):
    """Split-row FLAT with tiles dealt to XCDs by x window (recorded by the first call, used from the
    second) gives exactly the y of the positional mapping, on KAT and U[-1,1] inputs."""
    for name, rp, col, n in x_window_cases():
        for kat in (True, False):
            if kat:
                val, x = oracle.initvec(len(col), NP[dtype]), oracle.initvec(n, NP[dtype])
            else:
                rng = np.random.default_rng(len(col))
                val = rng.uniform(-1, 1, len(col)).astype(NP[dtype])
                x = rng.uniform(-1, 1, n).astype(NP[dtype])
            ys = []
            for xw in (1, 0):
                y, info = gpu_spmv(rp, col, val, x, "flat", tile=tile, dtype=dtype, row_aligned=0, x_windows=xw,
                                   repeat=3)
                assert info["x_windows"] == xw and info["row_aligned"] == 0
                ys.append(y)
            assert np.array_equal(ys[0], ys[1], equal_nan=True), name
            assert_parity(rp, col, val, x, ys[0], dtype, exact=kat and kat_exact_possible(rp, dtype), what=name)


def test_x_window_schedule_planning_rule():
    """On for split-row FLAT when rows span 4+ tiles over an x beyond 4 MB; refused for row-aligned plans."""
    from gpu_util import dev
    rp, col, _ = pf.synth_csr(5, seed=2, scale_n=600000, dtypes=())   # x 4.8 MB, rows up to 500k
    m = len(rp) - 1
    with pf.Plan(dev(rp), dev(col), m, m, len(col), "f64", "flat", 1024) as p:
        assert p.info.row_aligned == 0 and p.info.x_windows == 1
    rp, col, _ = pf.synth_csr(2, seed=2, scale_n=300, dtypes=())
    m = len(rp) - 1
    with pf.Plan(dev(rp), dev(col), m, m, len(col), "f64", "flat", 1024) as p:
        assert p.info.row_aligned == 1 and p.info.x_windows == 0
        with pytest.raises(pf.PrefreeError):
            p.set_x_windows(1)


@pytest.mark.parametrize("variant", ["adaptive", "flat"])
def test_deterministic(variant):
    rp, col, v = pf.synth_csr(5, seed=4, scale_n=40000)
    x = pf.synth_x(5, len(rp) - 1, seed=4)["f64"]
    y1, _ = gpu_spmv(rp, col, v["f64"], x, variant)
    y2, _ = gpu_spmv(rp, col, v["f64"], x, variant, repeat=3)
    assert np.array_equal(y1, y2)


def test_plan_reuse_and_one_shot():
    import torch
    from gpu_util import DEV, dev
    rp, col, v = pf.synth_csr(3, seed=5, scale_n=50000)
    m = len(rp) - 1
    d_rp, d_col, d_val = dev(rp), dev(col), dev(v["f64"])
    stream = torch.cuda.current_stream()
    with pf.Plan(d_rp, d_col, m, m, len(col), "f64", "auto", stream=stream) as p:
        for seed in (1, 2):
            x = pf.synth_x(3, m, seed=seed)["f64"]
            y = torch.full((m,), float("nan"), dtype=torch.float64, device=DEV)
            p.execute(d_rp, d_col, d_val, dev(x), y, stream=stream)
            torch.cuda.synchronize()
            assert_parity(rp, col, v["f64"], x, y.cpu().numpy(), "f64", what=f"reuse {seed}")
        p.check(stream=stream)
    x = pf.synth_x(3, m, seed=9)["f64"]
    y = torch.full((m,), float("nan"), dtype=torch.float64, device=DEV)
    pf.spmv(d_rp, d_col, d_val, dev(x), y, m, m, len(col), "f64", "auto", stream=stream)
    assert_parity(rp, col, v["f64"], x, y.cpu().numpy(), "f64", what="one-shot")


def test_malformed_csr_rejected_at_planning():
    from gpu_util import dev
    rp = np.array([0, 2, 1, 4], dtype=np.int32)        # decreasing
    col = np.array([0, 1, 2, 0], dtype=np.int32)
    with pytest.raises(pf.PrefreeError) as e:
        pf.Plan(dev(rp), dev(col), 3, 3, 4, "f64")
    assert e.value.status == 6
    rp = np.array([0, 2, 4], dtype=np.int32)
    col = np.array([0, 5, 1, 2], dtype=np.int32)       # column out of range
    with pytest.raises(pf.PrefreeError) as e:
        pf.Plan(dev(rp), dev(col), 2, 3, 4, "f64")
    assert e.value.status == 6
    with pytest.raises(pf.PrefreeError) as e:          # row_ptr[m] != nnz
        pf.Plan(dev(rp), dev(col), 2, 3, 3, "f64")
    assert e.value.status == 6


@pytest.mark.parametrize("long_row", [400, 200])
@pytest.mark.parametrize("tile", [1024, 2048])
def test_kernel_error_flag_on_changed_row_ptr(tile, long_row):
    # A row-aligned FLAT plan accepts rows of at most 256 nnz, and loads a
    # tile's overflow past its nominal range for rows no longer than the
    # planned matrix's longest (5 here).  A different but valid row_ptr (same
    # m and nnz, monotone, row 0 at 0, row m at nnz, every column in range)
    # with one row of 400 nnz (past 256) or 200 nnz (past the planned 5) makes
    # a tile's last row overflow it by 300 or 100: the search sets the plan's
    # error flag (every access stays clamped to the tile), pf_plan_check
    # reports PF_ERR_KERNEL once and clears the flag, and the next call on the
    # planned row_ptr is clean and exact.
    import torch

    m, n = 4000, 4000
    rng = np.random.default_rng(tile)
    rp, col = csr_from_lengths([5] * m, n, rng)
    lengths = np.full(m, 5)
    r = tile - 20                   # starts at 5r = 5 tile - 100: runs long_row - 100 nnz into the next tile
    lengths[r] = long_row
    lengths[r + 1:r + 1 + long_row - 5] = 4  # nnz unchanged
    assert lengths.sum() == 5 * m
    rp_bad = np.zeros(m + 1, dtype=np.int32)
    np.cumsum(lengths, out=rp_bad[1:])
    val, x = oracle.initvec(len(col)), oracle.initvec(n)
    d_rp, d_bad, d_col = (torch.from_numpy(a).cuda() for a in (rp, rp_bad, col))
    d_val, d_x = torch.from_numpy(val).cuda(), torch.from_numpy(x).cuda()
    y = torch.full((m,), float("nan"), dtype=torch.float64, device="cuda")
    with pf.Plan(d_rp, d_col, m, n, len(col), "f64", "flat", tile) as p:
        assert p.info.row_aligned
        p.execute(d_rp, d_col, d_val, d_x, y)       # records the row map
        p.check()
        p.set_remember_rows(False)                  # every call searches row_ptr
        p.execute(d_bad, d_col, d_val, d_x, y)
        with pytest.raises(pf.PrefreeError) as e:
            p.check()
        assert e.value.status == 7  # PF_ERR_KERNEL
        p.check()                                   # the flag was cleared
        y.fill_(float("nan"))
        p.execute(d_rp, d_col, d_val, d_x, y)
        p.check()
        assert np.array_equal(y.cpu().numpy(), oracle.spmv_serial(rp, col, val, x))
        p.set_remember_rows(True)                   # records the map again on this call
        y.fill_(float("nan"))
        p.execute(d_rp, d_col, d_val, d_x, y)
        p.check()
        assert np.array_equal(y.cpu().numpy(), oracle.spmv_serial(rp, col, val, x))
