"""The planning scan (pfk_plan_scan) on the GPU: statistics, column check and long-row sortedness in one pass.

pf_plan_create reads row_ptr once and col once: the row statistics, the column range check, the list of
long rows (over 256 nnz) and the column descents inside them.  Checked here:

* the statistics a plan holds equal pf_row_stats_compute's (the separate statistics pass) field by field;
* a single descent inside a dense row refuses the hybrid path wherever it falls, also across the
  boundary between two workgroups' ranges of col; a descent between two rows, or inside a short row, does
  not;
* more long rows than the scan lists (8192) fall back to a scan of their own and decide the same way;
* a single column out of range is refused wherever it falls;
* plan timing: the wall time covers the GPU time, both positive.
"""
import numpy as np
import pytest
import torch

import oracle
import prefree_amd as pf
from csr_cases import csr_from_lengths, edge_cases
from gpu_util import assert_parity, dev, gpu_spmv

pytestmark = pytest.mark.gpu

FIELDS = [f for f, _ in pf.RowStats._fields_]


def _chunk(nnz):
    """nnz per workgroup range of k_col_check (its launch in prefree_kernels.hip)."""
    grid = max(1, min(4096, -(-((nnz + 15) // 16) // 1024)))
    return (-(-nnz // grid) + 1023) & ~1023


def _cases():
    out = [(name, rp, col, n) for name, rp, col, n in edge_cases()]
    for cfg, scale in ((1, 0), (2, 300), (3, 60000), (4, 400000), (5, 40000)):
        rp, col, _ = pf.synth_csr(cfg, seed=4, scale_n=scale, dtypes=())
        out.append((f"C{cfg}", rp, col, len(rp) - 1))
    return out


CASES = _cases()


@pytest.mark.parametrize("case", range(len(CASES)), ids=[c[0] for c in CASES])
def test_plan_stats_equal_separate_pass(case):
    name, rp, col, n = CASES[case]
    m, nnz = len(rp) - 1, len(col)
    if m == 0:
        return
    d_rp, d_col = dev(rp), dev(col)
    want = pf.row_stats(d_rp, d_col, m, n, nnz)
    with pf.Plan(d_rp, d_col, m, n, nnz, "f64", "auto") as p:
        got = p.stats
        plan_ms, gpu_ms = p.timing
    for f in FIELDS:
        g, w = getattr(got, f), getattr(want, f)
        if hasattr(g, "__len__"):
            g, w = list(g), list(w)
        assert g == w, (name, f, g, w)
    assert plan_ms > 0 and 0 < gpu_ms <= plan_ms, (plan_ms, gpu_ms)
    torch.cuda.synchronize()


def _dense_matrix(seed=2, n=60000, pattern="300 D 400 D 500 D 200"):
    rng = np.random.default_rng(seed)
    lengths = []
    for p in pattern.split():
        lengths += [int(rng.integers(9000, 30000))] if p == "D" else [int(v) for v in rng.integers(0, 61, size=int(p))]
    rp, col = csr_from_lengths(lengths, n, rng)
    return rp, col, n


def _plan_info(rp, col, n):
    """A FLAT plan (the hybrid path is a FLAT plan's; AUTO picks ADAPTIVE for small matrices)."""
    with pf.Plan(dev(rp), dev(col), len(rp) - 1, n, len(col), "f64", "flat") as p:
        return p.info.as_dict()


def test_sorted_dense_rows_go_hybrid():
    rp, col, n = _dense_matrix()
    assert _plan_info(rp, col, n)["hybrid"] == 1


@pytest.mark.parametrize("where", ["middle", "first_pair", "last_pair", "chunk_edge", "chunk_edge_next",
                                   "wave_edge", "lane_block_edge"])
def test_one_descent_in_a_dense_row_refuses_hybrid(where):
    rp, col, n = _dense_matrix()
    lens = np.diff(rp)
    dense = np.flatnonzero(lens > 256)
    ch = _chunk(len(col))
    r = int(dense[1])
    a, b = int(rp[r]), int(rp[r + 1])
    if where == "middle":
        j = (a + b) // 2
    elif where == "first_pair":
        j = a
    elif where == "last_pair":
        j = b - 2
    elif where in ("wave_edge", "lane_block_edge"):
        # k_col_check: lane i of a wave holds 4 consecutive nnz of its range, so the pair (j, j + 1) with
        # j + 1 a multiple of 256 past the range's start crosses from a wave's last lane to the next wave
        # (taken by a load, not from the neighbouring lane); 1024 crosses into the next block of vectors
        step = 256 if where == "wave_edge" else 1024
        k0 = (a // ch) * ch  # start of the range holding the row's first nnz
        j = k0 + step - 1
        while j < a + 1:
            j += step
        assert j + 1 < b
    else:  # the pair (j, j + 1) straddles two workgroups' ranges, or starts the next range
        k = -(-a // ch) * ch
        while k < a + 2:
            k += ch
        assert k < b - 1, "the dense row must cross a range boundary"
        j = k - 1 if where == "chunk_edge" else k
    c = col.copy()
    c[j], c[j + 1] = c[j + 1], c[j]  # col[j] > col[j + 1] (the row's columns are distinct): one descent
    assert c[j] > c[j + 1]
    info = _plan_info(rp, c, n)
    assert info["hybrid"] == 0, where
    val, x = oracle.initvec(len(c)), oracle.initvec(n)
    y, _ = gpu_spmv(rp, c, val, x, "flat")
    assert_parity(rp, c, val, x, y, "f64", exact=True, what=where)


def test_descents_between_rows_or_in_short_rows_keep_hybrid():
    rp, col, n = _dense_matrix()
    lens = np.diff(rp)
    c = col.copy()
    short = [r for r in np.flatnonzero((lens >= 3) & (lens <= 256))[:50]]
    for r in short:  # reverse a few short rows: descents outside the dense rows
        c[rp[r]:rp[r + 1]] = c[rp[r]:rp[r + 1]][::-1]
    assert _plan_info(rp, c, n)["hybrid"] == 1


def test_more_long_rows_than_the_scan_lists():
    """8300 dense rows (over the scan's list of 8192): the plan scans again and decides as before."""
    rng = np.random.default_rng(6)
    n, nd, dl = 20000, 8300, 4100
    short = rng.integers(0, 8, size=(nd, 2))
    lengths = np.stack([np.full(nd, dl), short[:, 0], short[:, 1]], axis=1).ravel()
    rp = np.zeros(len(lengths) + 1, dtype=np.int64)
    np.cumsum(lengths, out=rp[1:])
    key = np.repeat(np.arange(len(lengths), dtype=np.int64) * n, lengths) + rng.integers(0, n, size=int(rp[-1]))
    col = (np.sort(key) % n).astype(np.int32)  # sorted within each row (repeats allowed)
    rp = rp.astype(np.int32)
    info = _plan_info(rp, col, n)
    assert info["hybrid"] == 1 and info["dense_rows"] == nd, info
    r = int(np.flatnonzero(np.diff(rp) > 256)[-1])
    j = int(rp[r]) + 100
    c = col.copy()
    while c[j] == c[j + 1]:
        j += 1
    c[j], c[j + 1] = c[j + 1], c[j]
    assert c[j] > c[j + 1]
    assert _plan_info(rp, c, n)["hybrid"] == 0
    val, x = oracle.initvec(len(col)), oracle.initvec(n)
    y, _ = gpu_spmv(rp, col, val, x, "flat")
    assert_parity(rp, col, val, x, y, "f64", exact=True, what="8300 dense rows")


@pytest.mark.parametrize("where", ["first", "last", "chunk_edge", "middle"])
def test_one_bad_column_refused(where):
    rp, col, n = _dense_matrix(seed=5)
    ch = _chunk(len(col))
    j = {"first": 0, "last": len(col) - 1, "chunk_edge": ch, "middle": len(col) // 2}[where]
    for bad in (n, -1):
        c = col.copy()
        c[j] = bad
        with pytest.raises(pf.PrefreeError) as e:
            pf.Plan(dev(rp), dev(c), len(rp) - 1, n, len(c), "f64", "auto")
        assert e.value.status == 6, where  # PF_ERR_CSR
    torch.cuda.synchronize()
