"""The fp16 oracle functions (oracle.spmv_serial_f16, oracle.spmv_f16_rounded) — CPU only.

Pinned against an exact restatement built from the binary16 format itself
(Fraction arithmetic and round-to-nearest-even to 11 significant bits, an
exponent range of [-14, 15], subnormals in steps of 2^-24, overflow to
infinity), independent of numpy's float16:

* spmv_serial_f16 restates test/test_cdspmv.cpp:4-20 in the reference's fp16
  build (valT = half, include/common.h:43-46): every product and every
  addition rounded to binary16;
* spmv_f16_rounded is this library's fp16 result model: exact products summed
  exactly (fp64 here), one rounding per row.

A row [2048, 1, 1] times ones separates the two (2048 vs 2050).
"""
from fractions import Fraction

import numpy as np
import pytest

import oracle

MAX_HALF = Fraction(65504)


def round_half(q):
    """Nearest binary16 value to the rational q (ties to even); +-inf beyond the largest finite."""
    if q == 0:
        return Fraction(0)
    sign = -1 if q < 0 else 1
    a = abs(q)
    e = 0
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -14)                       # subnormals share the exponent of the smallest normal
    ulp = Fraction(2) ** (e - 10)
    n = a / ulp
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    r = fl * ulp
    if r > MAX_HALF:
        return float("inf") * sign
    return sign * r


def as_f16(q):
    return np.float16(float(q))


def csr(rows):
    rp = np.zeros(len(rows) + 1, dtype=np.int32)
    cols, vals = [], []
    for i, r in enumerate(rows):
        rp[i + 1] = rp[i] + len(r)
        for c, v in r:
            cols.append(c)
            vals.append(v)
    return rp, np.array(cols, dtype=np.int32), np.array(vals, dtype=np.float16)


@pytest.mark.parametrize("q,want", [
    (Fraction(2049), 2048.0), (Fraction(2051), 2052.0), (Fraction(2050), 2050.0),
    (Fraction(65519), 65504.0), (Fraction(65520), float("inf")), (Fraction(-65520), float("-inf")),
    (Fraction(1, 2 ** 25), 0.0), (Fraction(3, 2 ** 25), 2.0 ** -23), (Fraction(1, 3), 0.333251953125),
    (Fraction(1, 2 ** 24), 2.0 ** -24), (Fraction(2 ** 15 + 16), 32768.0), (Fraction(2 ** 15 + 48), 32832.0),
])
def test_round_half_restatement_matches_numpy_rounding(q, want):
    """The exact rounding above and numpy's float16 conversion agree on ties, overflow and subnormals."""
    assert float(round_half(q)) == want
    assert float(np.float64(float(q)).astype(np.float16)) == want


def test_two_semantics_differ_on_a_planted_row():
    rp, col, val = csr([[(0, 2048), (1, 1), (2, 1)], [], [(2, 3)]])
    x = np.ones(3, dtype=np.float16)
    ref = oracle.spmv_serial_f16(rp, col, val, x)
    ours = oracle.spmv_f16_rounded(rp, col, val, x)
    assert ref.tolist() == [2048.0, 0.0, 3.0]           # 2048 + 1 -> 2048 (tie to even), + 1 -> 2048
    assert ours.tolist() == [2050.0, 0.0, 3.0]          # exact 2050, representable
    assert ref.dtype == np.float16 and ours.dtype == np.float16


@pytest.mark.parametrize("seed", range(6))
def test_f16_oracles_match_exact_restatement(seed):
    """Random small CSR: both oracle functions equal the Fraction restatement bit for bit.  Values
    are binary16 with magnitudes in [0.5, 2) (and zeros), so the fp64 sums of the rounded model are
    exact and the only rounding is the binary16 one."""
    rng = np.random.default_rng(seed)
    m, n = 40, 30
    rows = []
    for _ in range(m):
        k = int(rng.integers(0, 12))
        cs = rng.choice(n, size=k, replace=True)
        vs = (rng.uniform(0.5, 2.0, k) * rng.choice([-1, 1], k)).astype(np.float16)
        rows.append(list(zip(cs.tolist(), vs.tolist())))
    rp, col, val = csr(rows)
    x = (rng.uniform(0.5, 2.0, n) * rng.choice([-1, 1], n)).astype(np.float16)
    x[rng.integers(0, n, 3)] = 0
    ref = oracle.spmv_serial_f16(rp, col, val, x)
    ours = oracle.spmv_f16_rounded(rp, col, val, x)
    for i in range(m):
        t = Fraction(0)
        exact = Fraction(0)
        for j in range(rp[i], rp[i + 1]):
            p = Fraction(float(val[j])) * Fraction(float(x[col[j]]))
            exact += p
            t = round_half(t + round_half(p))
        assert float(ref[i]) == float(t), (i, ref[i], t)
        assert float(ours[i]) == float(round_half(exact)), (i, ours[i], exact)


def test_f16_kat_values():
    """initVec in the fp16 build: (half)(float)(i % 15); products <= 196 and their sums up to 2048 are
    exact integers in binary16, so both semantics give the exact row sum there."""
    v = oracle.initvec(40, np.float16)
    assert v.dtype == np.float16 and v.tolist() == [float(i % 15) for i in range(40)]
    rp = np.array([0, 10, 20], dtype=np.int32)
    col = np.arange(20, dtype=np.int32) % 15
    val = oracle.initvec(20, np.float16)
    x = oracle.initvec(15, np.float16)
    exact = [sum((j % 15) * ((j % 15) % 15) for j in range(0, 10)), sum((j % 15) * (j % 15) for j in range(10, 20))]
    assert oracle.spmv_serial_f16(rp, col, val, x).tolist() == exact
    assert oracle.spmv_f16_rounded(rp, col, val, x).tolist() == exact


def test_f16_overflow_is_infinite_in_both():
    rp, col, val = csr([[(0, 60000), (1, 60000)]])
    x = np.ones(2, dtype=np.float16)
    assert np.isinf(oracle.spmv_serial_f16(rp, col, val, x)[0])
    assert np.isinf(oracle.spmv_f16_rounded(rp, col, val, x)[0])
