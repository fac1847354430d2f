"""Shared test inputs and index-level models.

* `edge_cases()` — hand-built CSR matrices for the edge cases the reference's
  path has to survive (empty matrix, empty rows at either end, one row longer
  than a tile, one row spanning every tile, rows exactly on tile edges,
  rectangular shapes, duplicate and unsorted columns), plus random mixes.
* `tile_model()` — the tile descriptors the ADAPTIVE / FLAT kernels compute,
  restated with numpy searchsorted; `check_tiling()` verifies the invariants
  that make a tiling correct (every nnz in exactly one tile, every row written
  exactly once or split into a contiguous head/tail chain).  The GPU
  descriptors are compared bit-for-bit against the model, and the model is
  pinned by the invariants, not by retyping it.
"""
from __future__ import annotations

import numpy as np


def csr_from_lengths(lengths, n, rng, sorted_cols=True, distinct=True):
    lengths = np.asarray(lengths, dtype=np.int64)
    rp = np.zeros(len(lengths) + 1, dtype=np.int64)
    np.cumsum(lengths, out=rp[1:])
    col = np.empty(int(rp[-1]), dtype=np.int32)
    for i, L in enumerate(lengths):
        if L == 0:
            continue
        if distinct and L <= n:
            c = rng.choice(n, size=int(L), replace=False)
        else:
            c = rng.integers(0, n, size=int(L))
        if sorted_cols:
            c = np.sort(c)
        col[rp[i]:rp[i + 1]] = c
    return rp.astype(np.int32), col


def edge_cases(seed=7):
    """List of (name, row_ptr, col, n)."""
    rng = np.random.default_rng(seed)
    out = []

    def add(name, lengths, n, **kw):
        rp, col = csr_from_lengths(lengths, n, rng, **kw)
        out.append((name, rp, col, n))

    add("all_empty", [0] * 5, 5)
    add("single_nnz", [1], 1)
    add("one_row_7", [7], 16)
    add("one_row_3000", [3000], 4000)
    add("leading_trailing_empty", [0, 0, 0, 3, 1, 0, 5, 0, 0], 9)
    add("row0_longer_than_tile", [5000] + [2] * 40 + [0, 3], 6000)  # reference quirk A1
    add("row_spans_every_tile", [1, 20000, 1], 21000)
    add("rows_of_512", [512] * 9, 600)
    add("rows_511_512_513", [511, 512, 513] * 5 + [1], 700)
    add("rows_16_17", [16, 17] * 300, 100)
    add("rows_512_513_wave_edge", [512, 513, 3] * 8, 1000)
    add("rows_near_long_threshold", [1019, 1020, 1021, 2043, 2044, 2045, 4] * 3, 3000)
    add("rectangular_wide", list(rng.integers(0, 30, size=200)), 5000)
    add("rectangular_tall", list(rng.integers(0, 6, size=3000)), 7)
    add("duplicate_unsorted_cols", list(rng.integers(1, 40, size=300)), 50, sorted_cols=False, distinct=False)
    add("many_empty_runs", list(np.where(rng.random(5000) < 0.7, 0, rng.integers(1, 9, size=5000))), 5000)
    pl = np.minimum(20000, np.floor((1.0 - rng.random(4000)) ** (-1 / 1.1))).astype(int)
    add("power_law_mix", list(pl), 30000)
    add("mixed_dense", list(np.where(rng.random(2000) < 0.005, rng.integers(3000, 9000, size=2000),
                                     rng.integers(8, 65, size=2000))), 10000)
    # Rows of up to 256 nnz (row-aligned FLAT) whose last row runs 0..255 nnz past a tile's end: the
    # overflow reaches every wave of the workgroup, not only the first 64 lanes.
    add("rows_of_255", [255] * 160, 3000)
    add("rows_65_to_256", list(rng.integers(65, 257, size=300)), 4000)
    # Rows of at most 64 nnz (the longest row bounds the overflow a row-aligned tile loads with its nominal
    # range): overflows of up to 63 nnz, one wave of preloaded slots.
    add("rows_of_64", [64] * 200, 3000)
    add("rows_1_to_64", list(rng.integers(1, 65, size=700)), 5000)
    # The same overflows under 4 nnz per row on average (the row-aligned kernel's short-row mode).
    add("sparse_long_rows", list(np.where(rng.random(20000) < 0.02, rng.integers(65, 257, size=20000), 0)), 20000)
    return out


# ---- tiling model of k_tiles (ADAPTIVE: merged keys; FLAT: nnz keys) ----------

def tile_model(rp, K, merged, lmax, aligned=False):
    """Per-tile (lo_row, n_rows, A, B, head, tail): rows [lo, lo+n) and nnz [A, B).

    aligned (FLAT only): every tile owns the rows starting in its nnz range
    [kb, kb+K) (the last tile also the rows starting at nnz), whole, with the
    nnz [row_ptr[f], row_ptr[l]); no row is split.
    """
    rp = np.asarray(rp, dtype=np.int64)
    m = len(rp) - 1
    nnz = int(rp[-1])
    total = nnz + m if merged else nnz
    ntiles = max(1, -(-total // K))
    keys = rp[:m] + (np.arange(m, dtype=np.int64) if merged else 0)
    desc = np.zeros((ntiles, 6), dtype=np.int64)
    for t in range(ntiles):
        kb = t * K
        last = t == ntiles - 1
        ke = (total if merged else total + 1) if last else kb + K
        f = int(np.searchsorted(keys, kb, side="left"))
        l = m if last else int(np.searchsorted(keys, ke, side="left"))
        if aligned:
            desc[t] = (f, l - f, rp[f], rp[l], 0, 0)
            continue
        head = tail = 0
        A = B = 0
        h = f - 1
        if h >= 0:
            jk = kb - (h if merged else 0)
            if rp[h + 1] - rp[h] > lmax and jk < rp[h + 1]:
                head, A = 1, jk
        lo = h if head else f
        if f < l:
            if not head:
                A = rp[f]
            e = l - 1
            jend = ke - (e if merged else 0)
            if rp[e + 1] - rp[e] > lmax and rp[e + 1] > jend:
                B, tail = jend, 1
            else:
                B = rp[e + 1]
        elif head:
            B = min(rp[h + 1], ke - (h if merged else 0))
        desc[t] = (lo, l - lo, A, B, head, tail)
    return desc


def check_tiling(rp, desc, K, lmax, merged):
    """Invariants of a correct tiling; raises AssertionError with the first violation."""
    rp = np.asarray(rp, dtype=np.int64)
    m = len(rp) - 1
    nnz = int(rp[-1])
    covered = np.zeros(nnz, dtype=np.int32)
    written = np.zeros(m, dtype=np.int32)      # rows completed inside one tile
    pieces = {}                                # split row -> list of (tile, kind, a, b)
    for t, (lo, nr, A, B, head, tail) in enumerate(desc):
        assert 0 <= A <= B <= nnz, (t, A, B)
        assert nr >= 0 and lo >= 0 and lo + nr <= m, (t, lo, nr)
        assert B - (A & ~3) <= K + lmax + 2, ("span", t, A, B)
        covered[A:B] += 1
        for i in range(nr):
            r = lo + i
            a, b = max(rp[r], A), min(rp[r + 1], B)
            if head and i == 0:
                pieces.setdefault(r, []).append((t, "head", a, b))
            elif tail and i == nr - 1:
                pieces.setdefault(r, []).append((t, "tail", a, b))
            else:
                assert a == rp[r] and b == rp[r + 1], ("row not whole", t, r)
                written[r] += 1
    assert np.all(covered == 1), ("nnz coverage", np.flatnonzero(covered != 1)[:10])
    for r, ps in pieces.items():
        assert written[r] == 0, ("split row also written whole", r)
        assert rp[r + 1] - rp[r] > lmax, ("short row split", r)
        ps.sort()
        assert ps[0][1] == "tail" and all(p[1] == "head" for p in ps[1:]), ("chain", r, ps)
        tiles = [p[0] for p in ps]
        assert tiles == list(range(tiles[0], tiles[0] + len(tiles))), ("non-contiguous", r, tiles)
        assert ps[0][2] == rp[r] and ps[-1][3] == rp[r + 1], ("chain ends", r, ps)
        for p, q in zip(ps, ps[1:]):
            assert p[3] == q[2], ("chain gap", r, ps)
        written[r] += 1
    assert np.all(written == 1), ("rows written", np.flatnonzero(written != 1)[:10])
