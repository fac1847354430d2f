"""CPU emulation of the in-kernel searches, checking every index they read (no GPU).

The GPU kernels find their rows, runs and segment bounds with wave-cooperative searches whose index
arithmetic (probe positions, brackets, the closing round's 16-entry scalar load, readlane lanes) must
stay inside the arrays for ANY row_ptr, guess and spread, or a kernel reads out of bounds.  Each function
below restates one device function of prefree-public_amd/csrc lane by lane (64 lanes, C integer
semantics), routes every array read through a bounds-checked accessor, and returns what the device
function returns.  The tests assert that no read leaves the array, that every readlane lane is in
[0, 64), and that the result equals numpy's searchsorted (the answer the reference's pre-pass computes,
src/spmv_kernel/preFreeSpMV.cu:3-28), over the edge cases, scaled C1-C5, random matrices, guess spreads
0-1000 and fitted, absent and wrong guess lines.

Device functions restated (prefree_kernels.hip / device_common.hpp):
  row_probe_issue + row_probe_finish   (k_rows, whole-matrix search with its closing scalar round)
  row_window_run + row_window_finish   (k_rows over a hybrid plan's runs)
  run_of_tile                          (the run of a run tile)
  lane_lower_bound                     (k_dense, a dense row's window bounds)
  wave_search_lt / wave_search_lt_next (k_tiles, k_flat, k_prefree, k_wave)
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import prefree_amd as pf
from csr_cases import edge_cases

WAVE = 64
CLOSE = 16  # kClose: row bounds read by the closing round


class Checked:
    """An int32 array whose every read is bounds-checked and counted."""

    def __init__(self, a, name):
        self.a = np.asarray(a, dtype=np.int64)
        self.name = name
        self.reads = 0

    def __getitem__(self, i):
        i = int(i)
        assert 0 <= i < len(self.a), f"{self.name}[{i}] read outside [0, {len(self.a)})"
        self.reads += 1
        return int(self.a[i])


def cdiv(a, b):
    """C integer division (truncation toward zero)."""
    q = abs(a) // abs(b)
    return q if (a >= 0) == (b > 0) else -q


def u32(k):
    return k & 0xFFFFFFFF


def high_bit(mask):  # 63 - __clzll(mask)
    return mask.bit_length() - 1


def low_bit(mask):  # __ffsll(mask) - 1
    return (mask & -mask).bit_length() - 1


def readlane(vals, lane):
    assert 0 <= lane < WAVE, f"readlane of lane {lane}"
    return vals[lane]


# ---- k_rows: row_probe_at / row_probe_issue / row_probe_finish -----------------

def row_probe_at(rp, guess, spread, lo0, hi0):
    ks, valid = [0] * WAVE, [False] * WAVE
    for lane in range(WAVE):
        q = guess + (lane - 32) * spread
        valid[lane] = spread > 0 and lo0 < q < hi0
        if valid[lane]:
            ks[lane] = rp[q]
    return dict(guess=guess, spread=spread, lo0=lo0, hi0=hi0, k=ks, valid=valid)


def row_probe_issue(rp, m, v, nnz, spread, ga, gb):
    if ga > 0.0:
        g = ga * float(v) + gb
    else:
        g = float(v) * (float(m) / float(nnz)) if nnz > 0 else 0.0
    hi_clamp = float(m - 1 if m > 0 else 0)
    gc = 0.0 if math.isnan(g) else min(max(g, 0.0), hi_clamp)
    return row_probe_at(rp, int(gc), 1 if ga > 0.0 else spread, 0, m)


def row_probe_finish(rp, m, v, p):
    g, spread, lo, hi = p["guess"], p["spread"], p["lo0"], p["hi0"]
    hi_probed = False
    if spread > 0:
        okm = sum(1 << l for l in range(WAVE) if p["valid"][l] and u32(p["k"][l]) < v)
        badm = sum(1 << l for l in range(WAVE) if p["valid"][l] and u32(p["k"][l]) >= v)
        nlo = g + (high_bit(okm) - 32) * spread if okm else lo
        nhi = g + (low_bit(badm) - 32) * spread if badm else hi
        if nlo < nhi:
            lo, hi, hi_probed = nlo, nhi, badm != 0
    have, key = False, 0
    if hi_probed and hi - lo == 1:
        have, key = True, readlane(p["k"], cdiv(hi - g, spread) + 32)
    while hi - lo > 1:
        if hi - lo <= CLOSE and lo <= m - CLOSE:
            kk = [rp[lo + 1 + i] for i in range(CLOSE)]  # one 64-byte scalar load
            w = hi - lo - 1
            c = sum(1 for i in range(CLOSE - 1) if i < w and u32(kk[i]) < v)
            return lo + c, kk[c]
        step = (hi - lo + 63) >> 6
        ks = [0] * WAVE
        c = 0
        for lane in range(WAVE):
            pp = lo + lane * step
            if lane > 0 and pp < hi:
                ks[lane] = rp[pp]
                c += u32(ks[lane]) < v
        if step == 1 and c + 1 < WAVE and lo + c + 1 < hi:
            have, key = True, readlane(ks, c + 1)
        nlo = lo + c * step
        hi = min(nlo + step, hi)
        lo = nlo
    return lo, (key if have else rp[lo + 1])


# ---- k_rows over runs: row_window_run / row_window_finish ------------------------

def row_window_run(rp, m, r0, r1, n0, n1, v):
    f = (float(v) - n0) / (float(n1) - n0) if n1 > n0 else 0.0
    g = r0 + int(min(max(f * float(r1 - r0), 0.0), float(max(r1 - r0, 0))))
    base = max(0, g - 4 * WAVE // 2) & ~3
    n_ok = max(0, min(4 * WAVE, m + 1 - base))  # the resource's range check: entries past it read 0
    k = [rp[base + i] if i < n_ok else 0 for i in range(4 * WAVE)]
    return dict(base=base, lo0=max(r0 - 1, 0), hi0=r1, k=k)


def row_window_finish(rp, m, v, w):
    base, lo0, hi0 = w["base"], w["lo0"], w["hi0"]
    s = min(max(lo0 + 1 - base, 0), 4 * WAVE)
    e = min(max(hi0 - base, s), 4 * WAVE)
    c = sum(1 for i in range(4 * WAVE) if s <= i < e and u32(w["k"][i]) < v)
    nlo = base + s + c - 1 if c > 0 else lo0
    if s + c < e and (c > 0 or s + base == lo0 + 1):
        i = s + c
        lane = i >> 2
        assert 0 <= lane < WAVE
        return nlo, w["k"][i]
    nhi = base + s + c if s + c < e else hi0
    return row_probe_finish(rp, m, v, dict(guess=0, spread=0, lo0=nlo, hi0=nhi, k=[0] * WAVE, valid=[False] * WAVE))


# ---- run_of_tile ------------------------------------------------------------------

def run_of_tile(runs, nr, t, ntiles):
    if nr >= 16 and ntiles > 0:
        gl = (t * nr) // ntiles - 8
        g = min(max(gl, 0), nr - 16)
        kk = [runs[g + i] for i in range(16)]  # one scalar load of 16 entries
        c = sum(1 for i in range(16) if kk[i] <= t)
        if c > 0 and (c < 16 or g + 16 == nr):
            return g + c - 1
    lo, hi = 0, nr
    while hi - lo > 1:
        step = (hi - lo + 63) >> 6
        c = 0
        for lane in range(1, WAVE):
            p = lo + lane * step
            if p < hi and runs[p] <= t:
                c += 1
        lo += c * step
        hi = min(lo + step, hi)
    return lo


# ---- k_dense: lane_lower_bound -----------------------------------------------------

def lane_lower_bound(col, a, b, v, guess, sp):
    lo, hi = a - 1, b
    nlo, nhi = lo, hi
    for i in range(8):
        p = guess + (i - 4) * sp
        if a <= p < b:
            if col[p] < v:
                nlo = max(nlo, p)
            else:
                nhi = min(nhi, p)
    if nlo < nhi:
        lo, hi = nlo, nhi
    rounds = 0
    while hi - lo > 1:
        step = (hi - lo + 7) >> 3
        c = 0
        for i in range(1, 8):
            p = lo + i * step
            if p < hi and col[p] < v:
                c += 1
        nlo = lo + c * step
        hi = min(nlo + step, hi)
        lo = nlo
        rounds += 1
        assert rounds < 64, "lane_lower_bound does not converge"
    return hi


# ---- device_common.hpp: wave_search_lt / wave_search_lt_next -------------------------

def wave_search_lt(rp, m, v, guess, spread, merge):
    if v == 0:
        return -1

    def key(r):
        return u32(rp[r] + (r if merge else 0))

    lo, hi = 0, m
    if spread > 0:
        okm = badm = 0
        for lane in range(WAVE):
            p = guess + (lane - 32) * spread
            if lo < p < hi:
                if key(p) < v:
                    okm |= 1 << lane
                else:
                    badm |= 1 << lane
        nlo = guess + (high_bit(okm) - 32) * spread if okm else lo
        nhi = guess + (low_bit(badm) - 32) * spread if badm else hi
        if nlo < nhi:
            lo, hi = nlo, nhi
    while hi - lo > 1:
        step = (hi - lo + 63) >> 6
        c = sum(1 for lane in range(1, WAVE) if lo + lane * step < hi and key(lo + lane * step) < v)
        lo += c * step
        hi = min(lo + step, hi)
    return lo


def wave_search_lt_next(rp, m, v, guess, spread):
    lo, hi = 0, m
    if spread > 0:
        okm = badm = 0
        for lane in range(WAVE):
            p = guess + (lane - 32) * spread
            if lo < p < hi:
                if u32(rp[p]) < v:
                    okm |= 1 << lane
                else:
                    badm |= 1 << lane
        nlo = guess + (high_bit(okm) - 32) * spread if okm else lo
        nhi = guess + (low_bit(badm) - 32) * spread if badm else hi
        if nlo < nhi:
            lo, hi = nlo, nhi
    have, key = False, 0
    while hi - lo > 1:
        step = (hi - lo + 63) >> 6
        ks = [0] * WAVE
        c = 0
        for lane in range(1, WAVE):
            p = lo + lane * step
            if p < hi:
                ks[lane] = rp[p]
                c += u32(ks[lane]) < v
        if step == 1 and c + 1 < WAVE and lo + c + 1 < hi:
            have, key = True, readlane(ks, c + 1)
        lo += c * step
        hi = min(lo + step, hi)
    return lo, (key if have else rp[lo + 1])


# ---- inputs ---------------------------------------------------------------------------

def _cases():
    out = [(name, rp, col) for name, rp, col, _n in edge_cases()]
    for cfg, scale in ((1, 0), (2, 120), (3, 20000), (4, 60000), (5, 3000)):
        rp, col, _ = pf.synth_csr(cfg, seed=6, scale_n=scale, dtypes=())
        out.append((f"C{cfg}", rp, col))
    rng = np.random.default_rng(5)
    for i in range(10):
        m = int(rng.integers(1, 3000))
        lens = rng.integers(0, int(rng.integers(1, 300)), size=m)
        rp = np.zeros(m + 1, dtype=np.int64)
        np.cumsum(lens, out=rp[1:])
        out.append((f"rand{i}", rp.astype(np.int32), None))
    return out


CASES = _cases()
SPREADS = [0, 1, 2, 3, 16, 17, 64, 1000]


def _keys(rp, K, limit=160):
    """(kb, last, ke) of every row-aligned tile of K nnz (a deterministic sample of at most `limit`)."""
    nnz = int(rp[-1])
    nt = -(-nnz // K)
    ts = range(nt) if nt <= limit else sorted(set(np.linspace(0, nt - 1, limit).astype(int).tolist()))
    for t in ts:
        last = t == nt - 1
        kb = t * K
        yield t, kb, last, (nnz + 1 if last else kb + K)


def _lines(rp):
    """Guess lines: none, the plan's fitted quartile line, and four wrong ones."""
    m, nnz = len(rp) - 1, int(rp[-1])
    out = [(0.0, 0.0)]
    if m >= 4 and nnz > 0:
        a, b = int(rp[m // 4]), int(rp[3 * m // 4])
        if b > a:
            ga = (3 * m // 4 - m // 4) / (b - a)
            gb = m // 4 - ga * a
            out += [(ga, gb), (ga * 3.0, gb), (ga / 3.0, gb), (ga, gb + m / 2), (1e-9, -1e9)]
    return out


# ---- tests --------------------------------------------------------------------------------

@pytest.mark.parametrize("case", range(len(CASES)), ids=[c[0] for c in CASES])
def test_row_probe_search_stays_in_row_ptr(case):
    """k_rows search mode: waves 2 and 3 find f (key kb) and l (key ke) of every tile."""
    name, rp_np, _ = CASES[case]
    m, nnz = len(rp_np) - 1, int(rp_np[-1])
    if m == 0 or nnz == 0:
        return
    rp = Checked(rp_np, "row_ptr")
    for K in (1024, 2048):
        for spread in SPREADS:
            for ga, gb in (_lines(rp_np) if spread == SPREADS[0] else [(0.0, 0.0)]):
                for t, kb, last, ke in _keys(rp_np, K, 40):
                    for v, run in ((kb, kb != 0), (ke, not last)):
                        if not run:
                            continue
                        p = row_probe_issue(rp, m, v, nnz, spread, ga, gb)
                        r, nk = row_probe_finish(rp, m, v, p)
                        want = int(np.searchsorted(rp_np, v, side="left")) - 1
                        assert r == want, (name, K, spread, ga, t, v, r, want)
                        assert nk == int(rp_np[r + 1]), (name, K, spread, t, "next key")


def run_table(rp, apart_min=257, dtype_f64=True):
    """The run table of a hybrid plan (host/capi.cpp try_hybrid): rows of at least apart_min nnz are summed
    apart, the rows between them form runs cut into tiles from the run's first nnz rounded down to 64."""
    lens = np.diff(rp.astype(np.int64))
    apart = np.flatnonzero(lens >= apart_min)
    nd, m, nnz = len(apart), len(rp) - 1, int(rp[-1])
    nruns = nd + 1
    rb = [0] + [int(r) + 1 for r in apart]
    re = [int(r) for r in apart] + [m]
    nb = [0] + [int(rp[r + 1]) for r in apart]
    ne = [int(rp[r]) for r in apart] + [nnz]
    short_rows = sum(e - b for b, e in zip(rb, re))
    short_nnz = sum(e - b for b, e in zip(nb, ne))
    K = 1024 if dtype_f64 and short_nnz >= 4 * short_rows else 2048
    tb, tiles = [], 0
    for i in range(nruns):
        tb.append(tiles)
        rr = re[i] - rb[i]
        nz = ne[i] - (nb[i] & ~63)
        tiles += max(1, -(-nz // K)) if rr > 0 else 0
    tb.append(tiles)
    return tb + rb + [0] + re + [0] + nb + [0] + ne + [0], nruns, tiles, K


@pytest.mark.parametrize("case", range(len(CASES)), ids=[c[0] for c in CASES])
def test_run_window_search_stays_in_row_ptr(case):
    """k_rows over runs, search mode: run_of_tile, then the window search of f and l inside the run."""
    name, rp_np, _ = CASES[case]
    m, nnz = len(rp_np) - 1, int(rp_np[-1])
    if m == 0 or nnz == 0:
        return
    rp = Checked(rp_np, "row_ptr")
    # Rows summed apart hold over 256 nnz in a plan (65 keeps the run's first key above the row before
    # it: the window search's precondition); 17 breaks that precondition, where only the bounds of the
    # reads are checked, not the answer.
    for apart_min in (257, 65, 17):
        exact = apart_min > 64
        table, nruns, ntiles, K = run_table(rp_np, apart_min)
        if ntiles == 0:
            continue
        runs = Checked(table, "runs")
        R = nruns + 1
        tb = table[:R]
        ts = range(ntiles) if ntiles <= 300 else np.linspace(0, ntiles - 1, 300).astype(int)
        for t in ts:
            t = int(t)
            i = run_of_tile(runs, nruns, t, ntiles)
            want_i = int(np.searchsorted(np.asarray(tb[:nruns]), t, side="right")) - 1
            assert i == want_i, (name, apart_min, t, i, want_i)
            nb0, ne = table[3 * R + i] & ~63, table[4 * R + i]
            kb = nb0 + (t - tb[i]) * K
            last = ne - kb <= K
            B0 = ne if last else kb + K
            lend, r0 = table[2 * R + i], table[R + i]
            kb = min(max(kb, 0), nnz)
            B0 = min(max(B0, kb), min(nnz, kb + K))
            lend = min(max(lend, 0), m)
            r0 = min(max(r0, 0), lend)
            ke = ne + 1 if last else kb + K
            for v, run in ((kb, kb != 0), (ke, not last)):
                if not run:
                    continue
                w = row_window_run(rp, m, r0, lend, table[3 * R + i], ne, v)
                r, nk = row_window_finish(rp, m, v, w)
                assert -1 <= r < m, (name, apart_min, t, v, r)
                if not exact:
                    continue
                want = int(np.searchsorted(rp_np, v, side="left")) - 1
                assert r == want, (name, apart_min, t, v, r, want)
                assert nk == int(rp_np[r + 1]), (name, apart_min, t, "next key")


def test_run_of_tile_on_skewed_tables():
    """run_of_tile's scalar window and its fallback search on tables of very uneven runs."""
    rng = np.random.default_rng(3)
    for nr in (1, 2, 15, 16, 17, 40, 1001):
        sizes = rng.integers(0, 50, size=nr) * (rng.random(nr) < 0.7) + (rng.random(nr) < 0.05) * 5000
        tb = np.zeros(nr + 1, dtype=np.int64)
        np.cumsum(sizes, out=tb[1:])
        ntiles = int(tb[-1])
        runs = Checked(tb, "tile_begin")
        for t in range(0, ntiles, max(1, ntiles // 500)):
            i = run_of_tile(runs, nr, t, ntiles)
            assert i == int(np.searchsorted(tb[:nr], t, side="right")) - 1, (nr, t, i)


@pytest.mark.parametrize("case", range(len(CASES)), ids=[c[0] for c in CASES])
def test_lane_lower_bound_stays_in_row(case):
    """k_dense search mode: each row's first nnz at or past a window's first column, from the row's own
    interpolated guess; rows with unsorted columns must still read only inside the row."""
    name, rp_np, col_np = CASES[case]
    if col_np is None or len(col_np) == 0:
        return
    m = len(rp_np) - 1
    n = int(col_np.max()) + 1
    col = Checked(col_np, "col")
    lens = np.diff(rp_np.astype(np.int64))
    rows = np.argsort(-lens)[:12]
    for r in rows:
        a0, a1 = int(rp_np[r]), int(rp_np[r + 1])
        length = a1 - a0
        sp = int(max(1.0, math.ceil(math.sqrt(length) / 4.0)))
        seg = col_np[a0:a1].astype(np.int64)
        srt = bool(np.all(seg[1:] >= seg[:-1])) if length > 1 else True
        for W in (64, 1000, 8192):
            for c0 in list(range(0, n + W, W)) + [n, n + 5]:
                place = c0 * (length / n) if n > 0 else 0.0
                guess = a0 + int(min(max(place, 0.0), float(max(length - 1, 0))))
                got = lane_lower_bound(col, a0, a1, c0, guess, sp)
                assert a0 <= got <= a1, (name, r, c0, got)
                if srt:
                    assert got == a0 + int(np.searchsorted(seg, c0, side="left")), (name, r, c0)


@pytest.mark.parametrize("merge", [False, True])
@pytest.mark.parametrize("case", range(len(CASES)), ids=[c[0] for c in CASES])
def test_wave_search_stays_in_row_ptr(case, merge):
    """wave_search_lt (merged keys row_ptr[r] + r for ADAPTIVE, plain for FLAT/PREFREE) and
    wave_search_lt_next over every guess spread, with guesses at, before and past the answer."""
    name, rp_np, _ = CASES[case]
    m, nnz = len(rp_np) - 1, int(rp_np[-1])
    if m == 0:
        return
    rp = Checked(rp_np, "row_ptr")
    keys = rp_np.astype(np.int64) + (np.arange(m + 1) if merge else 0)
    top = int(keys[-1])
    vs = sorted(set([0, 1, top, top + 1] + np.linspace(0, top + 1, 60).astype(int).tolist()))
    for spread in SPREADS:
        for v in vs:
            want = int(np.searchsorted(keys[:m], v, side="left")) - 1
            for guess in (0, m - 1, max(want, 0), want + 7 * max(spread, 1), -5, m + 40):
                got = wave_search_lt(rp, m, v, guess, spread, merge)
                assert got == want, (name, merge, spread, v, guess, got, want)
                if not merge and v > 0 and want + 1 <= m:
                    r, nk = wave_search_lt_next(rp, m, v, guess, spread)
                    assert r == want and nk == int(rp_np[r + 1]), (name, spread, v, guess)
