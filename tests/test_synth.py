"""Synthetic configuration generators (pf_synth_*) — CPU only.

Checks the shapes and distributions the benchmark configurations state, that
columns are sorted, distinct and in range, and that generation is
deterministic in the seed and independent of the OpenMP thread count.
"""
import hashlib
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import prefree_amd as pf

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def check_rows(rp, col, n):
    assert rp[0] == 0 and np.all(np.diff(rp) >= 0)
    assert col.min(initial=0) >= 0 and col.max(initial=0) < n
    d = np.diff(col.astype(np.int64))
    starts = rp[1:-1]
    # within a row strictly increasing (sorted, distinct); across row starts anything goes
    ok = d > 0
    ok[starts[(starts > 0) & (starts < len(col))] - 1] = True
    assert np.all(ok)


def test_c1_full_shape():
    rp, col, v = pf.synth_csr(1, seed=1)
    assert len(rp) == 4097 and rp[-1] == 65536
    assert np.all(np.diff(rp) == 16)
    check_rows(rp, col, 4096)
    val = v["f64"]
    assert val.min() >= -1 and val.max() < 1 and abs(val.mean()) < 0.02


def test_c2_stencil():
    side = 64
    rp, col, v = pf.synth_csr(2, seed=1, scale_n=side)
    n = side * side
    assert rp[-1] == 5 * side * side - 4 * side
    check_rows(rp, col, n)
    val = v["f64"]
    for i in (0, 1, side, n // 2 + 3, n - 1):
        cols = col[rp[i]:rp[i + 1]]
        vals = val[rp[i]:rp[i + 1]]
        r, c = divmod(i, side)
        expect = sorted(rr * side + cc for rr, cc in ((r - 1, c), (r, c - 1), (r, c), (r, c + 1), (r + 1, c))
                        if 0 <= rr < side and 0 <= cc < side)
        assert list(cols) == expect
        assert list(vals) == [4.0 if cc == i else -1.0 for cc in cols]
    m, n2, nnz = pf.synth_dims(2, 1)
    assert (m, n2, nnz) == (4194304, 4194304, 20963328)


def test_c3_power_law():
    n = 200000
    rp, col, _ = pf.synth_csr(3, seed=1, scale_n=n)
    L = np.diff(rp)
    assert L.min() >= 1 and L.max() <= 200000
    assert 5.5 < L.mean() < 11
    # P(L >= k) = k^-1.1 for the Pareto tail
    for k in (2, 10, 100):
        assert abs((L >= k).mean() / k ** -1.1 - 1) < 0.1
    check_rows(rp, col, n)


def test_c4_very_sparse():
    n = 300000
    rp, col, _ = pf.synth_csr(4, seed=1, scale_n=n)
    L = np.diff(rp)
    assert abs(L.mean() - 2.5) < 0.02
    assert abs((L == 0).mean() - np.exp(-2.5)) < 0.003
    check_rows(rp, col, n)
    rows = np.repeat(np.arange(n), L)
    near = np.abs(col.astype(np.int64) - rows) <= 4096
    assert 0.89 < near.mean() < 0.92


def test_c5_mixed():
    n = 50000
    rp, col, _ = pf.synth_csr(5, seed=1, scale_n=n)
    L = np.diff(rp)
    dense = L > 64
    assert dense.sum() == n // 1000
    assert np.all((L[dense] >= n // 20) & (L[dense] <= n // 2))
    assert np.all((L[~dense] >= 8) & (L[~dense] <= 64))
    check_rows(rp, col, n)


def test_full_dims_c5_and_c3():
    m, n, nnz = pf.synth_dims(5, 1)
    assert m == n == 1000000
    assert 2.9e8 < nnz < 3.3e8  # ~311M by the stated distribution (text says ~200M)
    m, n, nnz = pf.synth_dims(3, 1)
    assert m == 2000000 and 1.2e7 < nnz < 2.0e7


def test_seed_determinism_and_values():
    a = pf.synth_csr(3, seed=5, scale_n=20000, dtypes=("f64", "f32"))
    b = pf.synth_csr(3, seed=5, scale_n=20000, dtypes=("f64", "f32"))
    c = pf.synth_csr(3, seed=6, scale_n=20000)
    assert digest(a[0], a[1], a[2]["f64"]) == digest(b[0], b[1], b[2]["f64"])
    assert digest(a[0], a[1]) != digest(c[0], c[1])
    assert np.array_equal(a[2]["f32"], a[2]["f64"].astype(np.float32))
    kat = pf.synth_csr(3, seed=5, scale_n=20000, vals=1)[2]["f64"]
    assert np.array_equal(kat, (np.arange(len(kat)) % 15).astype(np.float64))
    x = pf.synth_x(3, 1000, seed=5, vals=1)["f64"]
    assert np.array_equal(x, (np.arange(1000) % 15).astype(np.float64))


def test_thread_count_independent():
    code = ("import sys; sys.path.insert(0, %r); import conftest, prefree_amd as pf, hashlib, numpy as np;"
            "rp, col, v = pf.synth_csr(5, seed=3, scale_n=30000); x = pf.synth_x(5, 30000, seed=3)['f64'];"
            "print(hashlib.sha256(rp.tobytes() + col.tobytes() + v['f64'].tobytes() + x.tobytes()).hexdigest())"
            % os.path.dirname(os.path.abspath(__file__)))
    outs = set()
    for t in ("1", "3", "8"):
        env = dict(os.environ, OMP_NUM_THREADS=t)
        outs.add(subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                                check=True).stdout.strip())
    assert len(outs) == 1


def test_golden_c1_digest():
    with open(os.path.join(GOLDEN, "c1_seed1.json")) as f:
        g = json.load(f)
    rp, col, v = pf.synth_csr(1, seed=1)
    x = pf.synth_x(1, 4096, seed=1)["f64"]
    assert digest(rp, col, v["f64"], x) == g["csr_x_sha256"]


def test_golden_c1_oracle_output():
    import oracle
    with open(os.path.join(GOLDEN, "c1_seed1.json")) as f:
        g = json.load(f)
    rp, col, v = pf.synth_csr(1, seed=1)
    x = pf.synth_x(1, 4096, seed=1)["f64"]
    y = oracle.spmv_serial(rp, col, v["f64"], x)
    assert digest(y) == g["y_sha256"]
    assert [float(t).hex() for t in y[:16]] == g["y_head_hex"]
    ky = oracle.spmv_serial(rp, col, oracle.initvec(len(col)), oracle.initvec(4096))
    assert digest(ky) == g["kat_y_sha256"]
