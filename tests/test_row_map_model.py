"""CPU replay of the row-map search (k_row_map in prefree_kernels.hip), lane by lane.

Each map entry t of a row-aligned plan is (f, row_ptr[f]) with f = the first row whose row_ptr is at or above
t * tile: numpy's searchsorted(side="left").  The kernel searches each entry with a group of 16 lanes: a first
round of 16 probes around the interpolated guess, 4 x guess_spread apart, clamped to [0, m]; then rounds of 16
probes evenly inside the bracket (lo, hi], the last at most hi - 1.  The replay checks every probe index
against row_ptr's m + 1 entries, that the lanes below the key are the group's lowest, the answer, and the
number of rounds; a planted mistake (probes not clamped below hi) is caught.
"""
import numpy as np
import pytest

L = 16


def search(rp, v, spread, ga, gb, clamp_hi=True):
    """(f, row_ptr[f], rounds) for key v by the kernel's group search; asserts every index stays in bounds."""
    m, nnz = len(rp) - 1, int(rp[-1])
    lo, hi, khi = -1, m, int(rp[m])
    g = ga * v + gb if ga > 0 else v * (m / nnz)
    gc = int(min(max(g, 0.0), float(m)))
    step0 = 4 * max(spread, 1)
    p = [min(max(gc + (q - L // 2) * step0, 0), m) for q in range(L)]
    rounds = 0
    while True:
        rounds += 1
        assert all(0 <= i <= m for i in p), (p, lo, hi)
        k = [int(rp[i]) for i in p]
        below = [x < v for x in k]
        nb = sum(below)
        assert below == [True] * nb + [False] * (L - nb)  # probes non-decreasing in the lane
        if nb > 0:
            lo = max(lo, p[nb - 1])
        if nb < L and p[nb] < hi:
            hi, khi = p[nb], k[nb]
        if hi - lo <= 1:
            return hi, khi, rounds
        assert rounds < 64, "the bracket must shrink every round"
        step = (hi - lo + L) // (L + 1)
        p = [min(lo + (q + 1) * step, hi - 1) if clamp_hi else lo + (q + 1) * step for q in range(L)]


def _row_ptr(lens):
    rp = np.zeros(len(lens) + 1, dtype=np.int64)
    np.cumsum(lens, out=rp[1:])
    return rp


def _cases():
    rng = np.random.default_rng(5)
    lens = rng.poisson(2.5, 60000)
    lens[rng.random(60000) < 0.3] = 0
    yield "poisson_empty", lens
    yield "exact_256", np.full(2048, 256)
    lens = rng.integers(0, 9, 40000)
    lens[10000:30000] = 0
    yield "empty_stretch", lens
    lens = rng.integers(0, 3, 80000)
    lens[-300:] = 200
    yield "dense_tail", lens


@pytest.mark.parametrize("name,lens", list(_cases()), ids=[c[0] for c in _cases()])
@pytest.mark.parametrize("tile", [1024, 2048])
def test_group_search_finds_the_lower_bound(name, lens, tile):
    rp = _row_ptr(lens)
    m, nnz = len(lens), int(rp[-1])
    for spread, ga, gb in ((0, 0.0, 0.0), (16, 0.0, 0.0), (64, 0.0, 0.0), (1, m / nnz, 3.0), (4, 1e-3, -5.0)):
        worst = 0
        for t in range(1, -(-nnz // tile)):
            f, r, rounds = search(rp, t * tile, spread, ga, gb)
            want = int(np.searchsorted(rp, t * tile, side="left"))
            assert (f, r) == (want, rp[want]), (name, tile, spread, t)
            worst = max(worst, rounds)
        # the bracket is cut about 17-fold per round after the guess: log17(m) + 2 rounds at most
        assert worst <= int(np.log(max(m, 2)) / np.log(17)) + 2, (name, spread, worst)


def test_a_planted_mistake_is_caught():
    """Probes allowed up to hi (not hi - 1) read row_ptr[m + 1] on a bracket that ends at m."""
    rp = _row_ptr(np.full(100, 3))
    with pytest.raises((AssertionError, IndexError)):
        for t in range(1, 300 // 8):
            search(rp, t * 8, 1, 0.0, 0.0, clamp_hi=False)
