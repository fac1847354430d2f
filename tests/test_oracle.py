"""Pins of the CPU oracle (oracle/oracle.c) — CPU only.

The reference holds no golden vectors, known-answer fixtures or automated
tests for this path (its only check, eQcheck, never fails).  The oracle is
therefore pinned by: dense brute force, scipy.sparse on integer data (exact),
closed forms, cases where a wrong summation order or a fused multiply-add gives
a different exact answer, and brute-force restatements of the integer maps.
"""
import numpy as np
import pytest
import scipy.sparse as sp

import oracle
from csr_cases import csr_from_lengths, edge_cases


def random_csr(rng, m, n, max_len, empty_frac=0.2):
    lengths = rng.integers(0, max_len + 1, size=m)
    lengths[rng.random(m) < empty_frac] = 0
    return csr_from_lengths(lengths, n, rng)


def test_spmv_serial_matches_dense_brute_force():
    rng = np.random.default_rng(1)
    rp, col = random_csr(rng, 60, 45, 12)
    val = rng.uniform(-1, 1, len(col))
    x = rng.uniform(-1, 1, 45)
    dense = np.zeros((60, 45))
    for i in range(60):
        for j in range(rp[i], rp[i + 1]):
            dense[i, col[j]] += val[j]
    # brute force with the same left-to-right row order
    ref = np.array([sum((val[j] * x[col[j]] for j in range(rp[i], rp[i + 1])), 0.0) for i in range(60)])
    y = oracle.spmv_serial(rp, col, val, x)
    assert np.array_equal(y, ref)
    np.testing.assert_allclose(y, dense @ x, rtol=1e-13, atol=1e-13)


@pytest.mark.parametrize("dt", [np.float64, np.float32])
def test_spmv_serial_exact_on_integers_vs_scipy(dt):
    rng = np.random.default_rng(2)
    rp, col = random_csr(rng, 500, 300, 40)
    val = rng.integers(-14, 15, len(col)).astype(dt)
    x = rng.integers(-14, 15, 300).astype(dt)
    A = sp.csr_matrix((val.astype(np.float64), col, rp), shape=(500, 300))
    y = oracle.spmv_serial(rp, col, val, x)
    assert np.array_equal(y.astype(np.float64), A @ x.astype(np.float64))


def test_closed_forms():
    n = 100
    rng = np.random.default_rng(3)
    x = rng.uniform(-1, 1, n)
    eye_rp = np.arange(n + 1, dtype=np.int32)
    eye_col = np.arange(n, dtype=np.int32)
    assert np.array_equal(oracle.spmv_serial(eye_rp, eye_col, np.ones(n), x), x)
    d = rng.uniform(-1, 1, n)
    assert np.array_equal(oracle.spmv_serial(eye_rp, eye_col, d, x), d * x)
    # 5-point Laplacian on a 12x12 grid with x = c: (4 - degree) * c, interior rows 0.
    s = 12
    rows, cols, vals = [], [], []
    for r in range(s):
        for c in range(s):
            i = r * s + c
            for (rr, cc, v) in ((r - 1, c, -1.0), (r, c - 1, -1.0), (r, c, 4.0), (r, c + 1, -1.0), (r + 1, c, -1.0)):
                if 0 <= rr < s and 0 <= cc < s:
                    rows.append(i); cols.append(rr * s + cc); vals.append(v)
    A = sp.csr_matrix((vals, (rows, cols)), shape=(s * s, s * s))
    A.sort_indices()
    cst = 0.75
    y = oracle.spmv_serial(A.indptr.astype(np.int32), A.indices.astype(np.int32), A.data, np.full(s * s, cst))
    deg = np.diff(A.indptr) - 1
    assert np.array_equal(y, (4 - deg) * cst)
    assert np.count_nonzero(y) == 4 * (s - 2) + 4


def test_sequential_order_pinned():
    # left to right: ((0 + 1) + 1e16) - 1e16 = 0; any other order of this row gives 1.
    rp = np.array([0, 3], dtype=np.int32)
    col = np.array([0, 1, 2], dtype=np.int32)
    y = oracle.spmv_serial(rp, col, np.array([1.0, 1e16, -1e16]), np.ones(3))
    assert y[0] == 0.0


def test_no_fused_multiply_add():
    # a*x rounded before the add: -(1+2^-29) + round((1+2^-30)^2) == 0; an FMA gives 2^-60.
    e = 2.0 ** -30
    rp = np.array([0, 2], dtype=np.int32)
    col = np.array([0, 1], dtype=np.int32)
    y = oracle.spmv_serial(rp, col, np.array([-(1 + 2 * e), 1 + e]), np.array([1.0, 1 + e]))
    assert y[0] == 0.0


def test_accumulates_into_y():
    rp = np.array([0, 1, 1], dtype=np.int32)
    y = oracle.spmv_serial(rp, np.array([0], dtype=np.int32), np.array([2.0]), np.array([3.0]), y=[1.0, 5.0])
    assert list(y) == [7.0, 5.0]  # Y_val[i] = Y_val[i] + t, test_cdspmv.cpp:18


@pytest.mark.parametrize("threads", [1, 2, 3, 8])
@pytest.mark.parametrize("dt", [np.float64, np.float32])
def test_omp_bit_identical_to_serial(threads, dt):
    rng = np.random.default_rng(4)
    lengths = np.minimum(5000, np.floor((1.0 - rng.random(3000)) ** (-1 / 1.1))).astype(int)
    rp, col = csr_from_lengths(lengths, 8000, rng)
    val = rng.uniform(-1, 1, len(col)).astype(dt)
    x = rng.uniform(-1, 1, 8000).astype(dt)
    assert np.array_equal(oracle.spmv_omp(rp, col, val, x, nthreads=threads), oracle.spmv_serial(rp, col, val, x))


def test_pre_start_row_closed_form():
    rng = np.random.default_rng(5)
    for trial in range(30):
        lengths = rng.integers(0, 2000 if trial % 3 == 0 else 20, size=rng.integers(1, 400))
        lengths[rng.random(len(lengths)) < 0.3] = 0
        if lengths.sum() == 0:
            lengths[-1] = 1
        rp, _ = csr_from_lengths(lengths, 10, rng, distinct=False)
        for tile in (1, 7, 512, 1024):
            sr = oracle.pre_start_row(rp, tile)
            ntiles = len(sr) - 1
            t = np.arange(ntiles, dtype=np.int64) * tile
            closed = np.searchsorted(rp, t, side="right") - 1
            assert np.array_equal(sr[:ntiles], closed), (trial, tile)
            assert sr[ntiles] == 0  # the memset sentinel, preFreeSpMV.cu:594


def test_tile_row_range_sentinel_quirk():
    """Reference quirk: start_row[b+1]==0 is read as "m" even when row 0 legitimately spans the tile edge."""
    rp, col = csr_from_lengths([1500, 3, 3], 2000, np.random.default_rng(0))
    sr = oracle.pre_start_row(rp, 512)
    assert list(sr) == [0, 0, 0, 0]  # 1506 nnz: 3 tiles, all starting inside row 0
    assert oracle.tile_row_range(rp, 512, sr, 0, faithful_sentinel=True) == (0, 3)   # wrong: spans all rows
    assert oracle.tile_row_range(rp, 512, sr, 0, faithful_sentinel=False) == (0, 1)
    assert oracle.tile_row_range(rp, 512, sr, 2, faithful_sentinel=False) == (0, 3)


def test_tile_row_range_covers_tile_rows():
    rng = np.random.default_rng(6)
    for _ in range(20):
        lengths = rng.integers(0, 700, size=rng.integers(2, 200))
        lengths[rng.random(len(lengths)) < 0.3] = 0
        lengths[0] = max(lengths[0], 1)
        rp, _ = csr_from_lengths(lengths, 10, rng, distinct=False)
        sr = oracle.pre_start_row(rp, 512)
        for b in range(len(sr) - 1):
            s, e = oracle.tile_row_range(rp, 512, sr, b)
            lo, hi = b * 512, min((b + 1) * 512, rp[-1])
            touching = [r for r in range(len(rp) - 1) if rp[r] < hi and rp[r + 1] > lo]
            assert all(s <= r < e for r in touching)


@pytest.mark.parametrize("name,rp,col,n", edge_cases(), ids=[c[0] for c in edge_cases()])
def test_prefree_sim_exact_on_kat(name, rp, col, n):
    val = oracle.initvec(len(col))
    x = oracle.initvec(n)
    ref = oracle.spmv_serial(rp, col, val, x)
    assert np.array_equal(oracle.prefree_sim(rp, col, val, x), ref)
    assert np.array_equal(oracle.prefree_sim(rp, col, val, x, reverse_tiles=True), ref)


def test_prefree_sim_reproduces_sentinel_bug():
    rp, col = csr_from_lengths([1500, 3, 3], 2000, np.random.default_rng(0))
    val = oracle.initvec(len(col))
    x = oracle.initvec(2000)
    ref = oracle.spmv_serial(rp, col, val, x)
    assert np.array_equal(oracle.prefree_sim(rp, col, val, x), ref)
    # Tile 0 reads start_row[1] == 0 as "m" and stores 0 into rows 1..2; when it
    # runs after the tile that computed them (a legal GPU schedule) they are lost.
    assert np.array_equal(oracle.prefree_sim(rp, col, val, x, faithful_sentinel=True), ref)
    bad = oracle.prefree_sim(rp, col, val, x, faithful_sentinel=True, reverse_tiles=True)
    assert bad[1] == 0.0 and ref[1] != 0.0


def test_prefree_sim_random_within_tolerance():
    rng = np.random.default_rng(8)
    for name, rp, col, n in edge_cases(9):
        val = rng.uniform(-1, 1, len(col))
        x = rng.uniform(-1, 1, n)
        err, zb, _ = oracle.rownorm_maxerr(rp, col, val, x, oracle.spmv_serial(rp, col, val, x),
                                           oracle.prefree_sim(rp, col, val, x))
        assert err <= 1e-14 and zb == 0, name


def test_eqcheck_restatement():
    a = np.array([1.0, 2.0, 3.0, 0.0])
    assert oracle.eqcheck(a, a) == 0
    assert oracle.eqcheck(a, np.array([1.0, 2.1, 3.0, 0.0])) == 1
    assert oracle.eqcheck(a, np.array([1.0, 2.0, 3.0 * (1 + 1e-9), 0.0])) == 0  # 0/0 passes, as in :31


def test_rownorm_detects_planted_error():
    rng = np.random.default_rng(10)
    rp, col = random_csr(rng, 200, 200, 30)
    val = rng.uniform(-1, 1, len(col))
    x = rng.uniform(-1, 1, 200)
    y = oracle.spmv_serial(rp, col, val, x)
    assert oracle.rownorm_maxerr(rp, col, val, x, y, y)[0] == 0.0
    bad = y.copy()
    r = int(np.argmax(np.diff(rp)))
    bad[r] += 1e-9 * np.abs(val[rp[r]:rp[r + 1]] * x[col[rp[r]:rp[r + 1]]]).sum()
    err, _, worst = oracle.rownorm_maxerr(rp, col, val, x, y, bad)
    assert worst == r and 0.9e-9 < err < 1.1e-9
    empty = int(np.flatnonzero(np.diff(rp) == 0)[0])
    bad2 = y.copy()
    bad2[empty] = 1e-300
    assert oracle.rownorm_maxerr(rp, col, val, x, y, bad2)[1] == 1
    bad3 = y.copy()
    bad3[3] = np.nan
    assert oracle.rownorm_maxerr(rp, col, val, x, y, bad3)[0] == np.inf


def test_byte_models():
    # C2: nnz = 5*2048^2 - 4*2048, rows = cols = 2048^2
    assert oracle.bytes_effective(4194304, 4194304, 20963328, 8) == 335446020
    assert oracle.bytes_gather(4194304, 4194304, 20963328, 8) == (2 * 20963328 + 4194304) * 8 + 20963328 * 4 + 4194305 * 4
    assert oracle.bytes_effective(4096, 4096, 65536, 8) == 868356


def test_initvec():
    v = oracle.initvec(40)
    assert list(v[:16]) == [float(i % 15) for i in range(16)]
    assert np.array_equal(oracle.initvec(40, np.float32), v.astype(np.float32))


# ---- every reduction ladder of the reference kernel (preFreeSpMV.cu:440-559) ----

LADDERS = [(code, p) for code in (1, 2, 3, 4, 5) for p in (4, 8)]


@pytest.mark.parametrize("code,p_nnz", LADDERS, ids=[f"code{c}-p{p}" for c, p in LADDERS])
def test_prefree_sim_ladders_exact_on_kat(code, p_nnz):
    # initVec values: every product and row sum is an exact integer, so any
    # summation tree and any order of the boundary-row atomics give the serial sum.
    for name, rp, col, n in edge_cases():
        val, x = oracle.initvec(len(col)), oracle.initvec(n)
        ref = oracle.spmv_serial(rp, col, val, x)
        for rev in (False, True):
            got = oracle.prefree_sim(rp, col, val, x, code=code, p_nnz=p_nnz, reverse_tiles=rev)
            assert np.array_equal(got, ref), (name, code, p_nnz, rev)


@pytest.mark.parametrize("code,p_nnz", LADDERS, ids=[f"code{c}-p{p}" for c, p in LADDERS])
def test_prefree_sim_ladders_random_within_tolerance(code, p_nnz):
    rng = np.random.default_rng(code * 10 + p_nnz)
    for name, rp, col, n in edge_cases(11):
        val = rng.uniform(-1, 1, len(col))
        x = rng.uniform(-1, 1, n)
        y, plain, atomics = oracle.prefree_sim(rp, col, val, x, code=code, p_nnz=p_nnz, counts=True)
        err, zb, _ = oracle.rownorm_maxerr(rp, col, val, x, oracle.spmv_serial(rp, col, val, x), y)
        assert err <= 1e-14 and zb == 0, (name, code, p_nnz)
        # every non-empty row is written: by exactly one plain store, or by atomic adds alone
        lens = np.diff(rp)
        ok = ((plain == 1) & (atomics == 0)) | ((plain == 0) & (atomics >= 1))
        if code == 4:  # the long/short split skips rows whose sum is exactly zero
            ok |= (plain == 0) & (atomics == 0) & (y == 0)
        assert np.all(ok[lens > 0]), (name, code, p_nnz)


def test_prefree_sim_thread_ladder_is_sequential():
    # Code 1 sums every row with one thread in nnz order (red_row_thread): a row
    # inside one tile, stored plainly, is bit-identical to spmv_serial even where
    # cancellation makes other summation orders round differently.
    rng = np.random.default_rng(3)
    lengths = rng.integers(1, 12, size=4000)
    rp, col = csr_from_lengths(lengths, 3000, rng)
    val = rng.uniform(-1, 1, len(col)) * 10.0 ** rng.integers(-8, 9, size=len(col))
    x = rng.uniform(-1, 1, 3000)
    ref = oracle.spmv_serial(rp, col, val, x)
    for p_nnz in (4, 8):
        y, plain, _ = oracle.prefree_sim(rp, col, val, x, code=1, p_nnz=p_nnz, counts=True)
        assert plain.sum() > 3000
        assert np.array_equal(y[plain == 1], ref[plain == 1])


def test_prefree_vector_size_table():
    # calculate_vector_size<128> (preFreeSpMV.cu:394-405): 2^floor(log2(128 // n)) clamped to [2, 32],
    # 2 from 128 rows on; values worked by hand.
    want = {1: 32, 2: 32, 3: 32, 4: 32, 5: 16, 8: 16, 9: 8, 16: 8, 17: 4, 32: 4, 33: 2, 42: 2, 43: 2, 64: 2,
            65: 2, 127: 2, 128: 2, 500: 2}
    for n, vs in want.items():
        assert oracle.prefree_vector_size(n) == vs, n


def test_prefree_sim_long_short_split():
    # One 512-nnz tile holding rows of 2, 3, 500 and 7 nnz: the 500-nnz row holds
    # 97.7% of the tile, so ladder 4 takes red_row_long_short_specialized
    # (:485-511).  Row 1 (interior) sums to exactly zero: ladder 4 never writes
    # it (:326), ladder 3 stores the zero.  Row 0 opens the tile (atomic add of
    # its two-term sum, left to right).
    rng = np.random.default_rng(5)
    lengths = [2, 3, 500, 7, 4, 600]
    rp, col = csr_from_lengths(lengths, 2000, rng)
    val = rng.uniform(-1, 1, len(col))
    x = rng.uniform(-1, 1, 2000)
    val[rp[1]:rp[2]] = [1.0, 1.0, -2.0]
    x[col[rp[1]:rp[2]]] = 1.0
    ref = oracle.spmv_serial(rp, col, val, x)
    sentinel = np.full(len(lengths), 7.0)
    y4 = oracle.prefree_sim(rp, col, val, x, code=4, y=sentinel)
    y3 = oracle.prefree_sim(rp, col, val, x, code=3, y=sentinel)
    assert y4[1] == 7.0 and y3[1] == 0.0
    assert y4[0] == 7.0 + (val[0] * x[col[0]] + val[1] * x[col[1]])
    # the long row (interior, stored plainly) is within rounding of the serial sum
    r2 = slice(rp[2], rp[3])
    assert y4[2] != 7.0 and abs(y4[2] - ref[2]) <= 1e-14 * np.abs(val[r2] * x[col[r2]]).sum()
    kat_v, kat_x = oracle.initvec(len(col)), oracle.initvec(2000)
    assert np.array_equal(oracle.prefree_sim(rp, col, kat_v, kat_x, code=4),
                          oracle.spmv_serial(rp, col, kat_v, kat_x))


def test_prefree_sim_rejects_unknown_ladder():
    rp, col = csr_from_lengths([3, 3], 4, np.random.default_rng(0))
    v = oracle.initvec(6)
    with pytest.raises(ValueError):
        oracle.prefree_sim(rp, col, v, oracle.initvec(4), code=6)
    with pytest.raises(ValueError):
        oracle.prefree_sim(rp, col, v, oracle.initvec(4), code=3, p_nnz=16)
