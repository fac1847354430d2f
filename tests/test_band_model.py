"""CPU model of the band kernel's steps, windows and LDS ring (k_band in prefree_kernels.hip), no GPU.

The band kernel keeps, per workgroup, x[f - w, l + w) of its current step in an LDS ring (x[c] at slot
c mod PFK_BAND_RING) and loads between steps only the entries the next step adds.  Its correctness rests on
index arithmetic alone: windows that only move forward and never span more than the ring, the entries a
step adds, the prefetch of at most kBandExt of them, row bounds staged for at most kBandRp - 1 rows.  This
model replays that arithmetic step by step over whole workgroups, for the edge cases, scaled C2 and C4,
banded matrices with outliers and steps of very many (empty) rows, and checks:

* every read the kernel makes stays inside its array (row map, col/val ranges, row_ptr, x, the ring);
* every column the kernel reads from the ring was written there for that column and not overwritten since
  (the ring invariant), and every other column is gathered from memory;
* each step's nnz range is whole rows of at most kBandSlots products;
* the y the model forms from its ring and gathers equals spmv_serial bit for bit (one lane per row in nnz
  order), so a wrong window or a stale ring slot would change the sums.
"""
import numpy as np
import pytest

import oracle
import prefree_amd as pf
from csr_cases import csr_from_lengths, edge_cases

BAND_STEP = 4096   # PFK_BAND_STEP
RING = 12288       # PFK_BAND_RING
BS = 1024          # kBandBS
PER = 5            # kBandPer
SLOTS = PER * BS
RP = 2 * BS        # kBandRp
EXT = 2 * BS       # kBandExt


def row_map(rp, tile):
    """The row map the plan's first call records: tile t -> (first row with row_ptr >= t*tile, row_ptr there);
    the last entry (m, nnz)."""
    m, nnz = len(rp) - 1, int(rp[-1])
    nt = max(1, -(-nnz // tile))
    out = np.zeros((nt + 1, 2), dtype=np.int64)
    for t in range(nt):
        f = int(np.searchsorted(rp, t * tile, side="left")) if t > 0 else 0
        out[t] = (f, rp[f])
    out[nt] = (m, nnz)
    return out, nt


class Model:
    def __init__(self, rp, col, x, w, tile, wgs, ext_shift=0):
        self.rp, self.col, self.x, self.w = rp, col, x, w
        self.ext_shift = ext_shift  # a planted mistake in the entries a step adds (tests of the model only)
        self.m, self.n, self.nnz = len(rp) - 1, len(x), int(rp[-1])
        self.map, self.ntiles = row_map(rp, tile)
        self.group = BAND_STEP // tile
        self.nsteps = -(-self.ntiles // self.group)
        wgs = max(1, min(self.nsteps, wgs))
        self.per = -(-self.nsteps // wgs)
        self.y = np.full(self.m, np.nan)

    def step(self, s, begin, end):
        """band_step: (f, l, A, B) or the empty step."""
        if s < begin or s >= end:
            return [0, 0, 0, 0, 0, 0]
        t0 = s * self.group
        t1 = min(t0 + self.group, self.ntiles)
        assert 0 <= t0 < self.ntiles and 0 <= t1 <= self.ntiles, "row map read out of range"
        (f, A), (l, B) = self.map[t0], self.map[t1]
        ok = 0 <= f <= l <= self.m and 0 <= A <= B <= self.nnz and B - A <= SLOTS
        assert ok, (s, f, l, A, B)
        return [int(f), int(l), int(A), int(B), 0, 0]

    def window(self, d, p):
        """band_window: d's window after p's."""
        if d[1] == d[0]:
            d[4], d[5] = p[4], p[5]
            return
        hi = max(min(d[1] + self.w, self.n), p[5])
        lo = max(d[0] - self.w, p[4])
        lo = min(max(lo, 0), hi)
        lo = max(lo, hi - RING)
        d[4], d[5] = lo, hi

    def run_workgroup(self, g):
        s0 = g * self.per
        s1 = min(self.nsteps, s0 + self.per)
        if s0 >= s1:
            return 0
        ring = np.full(RING, -1, dtype=np.int64)    # the column each slot holds (-1: nothing yet)
        empty = [0, 0, 0, 0, 0, 0]
        prev = list(empty)                            # the step before s0: empty, with an empty window
        nxt = self.step(s0, s0, s1)
        self.window(nxt, prev)
        gathered = 0
        for s in range(s0, s1):
            cur = nxt
            nxt = self.step(s + 1, s0, s1)
            self.window(nxt, cur)
            # entries step s adds: [max(prev.hi, cur.lo), cur.hi)
            e = max(prev[5], cur[4]) + self.ext_shift
            ne = cur[5] - e
            assert ne >= 0 and e >= 0 and e + ne <= self.n
            assert cur[5] - cur[4] <= RING and cur[4] >= prev[4] and cur[5] >= prev[5]
            for c in range(e, e + ne):  # the prefetched first EXT of them, then the rest
                ring[c % RING] = c
            f, l, A, B, lo, hi = cur
            nq = B - A
            assert 0 <= nq <= SLOTS
            cols = self.col[A:B]
            inwin = (cols >= lo) & (cols < hi)
            if inwin.any():
                slots = cols[inwin] % RING
                assert np.array_equal(ring[slots], cols[inwin]), f"stale ring slot in step {s}"
            gathered += int((~inwin).sum())
            xv = self.x[cols]  # the ring holds x[c] for every in-window c (checked above)
            prod = self.val[A:B] * xv
            nr = l - f
            for i in range(nr):
                ra, rb = int(self.rp[f + i]) - A, int(self.rp[f + i + 1]) - A
                assert 0 <= ra <= rb <= nq, (s, i, ra, rb, nq)
                acc = 0.0
                if rb - ra <= 16:
                    for j in range(ra, rb):
                        acc += prod[j]
                    self.y[f + i] = acc
                else:
                    self.y[f + i] = np.nan  # wave-summed rows: order not modelled here
            prev = cur
        return gathered

    def run(self, val):
        self.val = val
        g = 0
        wg = 0
        while wg * self.per < self.nsteps:
            g += self.run_workgroup(wg)
            wg += 1
        return g


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
    for name, rp, col, n in edge_cases():
        if len(rp) > 1 and np.diff(rp).max() <= 256 and n > 0:
            out.append((name, rp, col, n, 64))
    rp, col, _ = pf.synth_csr(4, seed=2, scale_n=300000, dtypes=())
    out.append(("C4", rp, col, len(rp) - 1, 4096))
    rp, col, _ = pf.synth_csr(2, seed=2, scale_n=300, dtypes=())
    out.append(("C2", rp, col, len(rp) - 1, 512))
    for i, (lam, w, o) in enumerate(((2.5, 4096, 0.1), (1.0, 1024, 0.3), (6.0, 64, 0.0), (0.2, 8192, 0.1))):
        rp, col, n = _banded(60000, lam, w, o, seed=i)
        out.append((f"banded{i}", rp, col, n, w))
    # steps of very many rows (long runs of empty rows), windows that jump, a wide rectangular x
    rng = np.random.default_rng(9)
    lengths = np.where(rng.random(200000) < 0.02, rng.integers(1, 40, 200000), 0)
    rp, col = csr_from_lengths(lengths, 200000, rng)
    out.append(("sparse_jumps", rp, col, 200000, 2048))
    rp, col, n = _banded(30000, 3.0, 2048, 0.05, seed=11, n=90000)
    out.append(("wide", rp, col, n, 2048))
    return out


CASES = _cases()


@pytest.mark.parametrize("tile", [1024, 2048])
@pytest.mark.parametrize("wgs", [1, 7, 256])
@pytest.mark.parametrize("case", range(len(CASES)), ids=[c[0] for c in CASES])
def test_band_ring_model(case, wgs, tile):
    name, rp, col, n, w = CASES[case]
    if int(np.diff(rp).max()) > 256:
        pytest.skip("row-aligned plans only")
    val = oracle.initvec(len(col))
    x = oracle.initvec(n)
    mdl = Model(rp, col, x, w, tile, wgs)
    mdl.run(val)
    ref = oracle.spmv_serial(rp, col, val, x)
    lane = ~np.isnan(mdl.y)
    assert np.array_equal(mdl.y[lane], ref[lane]), name
    assert np.all(np.diff(rp)[~lane] > 16)


def test_model_catches_a_stale_ring():
    """The model is not vacuous: adding the next step's entries one column late leaves a slot stale."""
    name, rp, col, n, w = [c for c in CASES if c[0] == "C4"][0]
    mdl = Model(rp, col, oracle.initvec(n), w, 2048, 64, ext_shift=1)
    with pytest.raises(AssertionError, match="stale ring slot"):
        mdl.run(oracle.initvec(len(col)))
