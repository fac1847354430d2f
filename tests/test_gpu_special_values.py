"""NaN and infinities in val and x, every variant, against the oracle.

With integer (initVec-style) values the finite row sums are exact (fp16: in the
fp32 sums, then rounded once, against the oracle's once-rounded sum), and special
values propagate through a row sum the same way in any order (a NaN or
+inf + -inf gives NaN, a single-signed infinity survives, 0 * inf is NaN), so y
must equal the oracle's (test/test_cdspmv.cpp:4-20) bit for bit, NaNs in the
same rows, in every variant and for row-aligned and split-row FLAT tiles.
"""
import numpy as np
import pytest

import oracle
from csr_cases import edge_cases
from gpu_util import NP, gpu_spmv

pytestmark = pytest.mark.gpu

CASES = [c for c in edge_cases() if len(c[2]) > 0]


def plant(a, rng, frac):
    """Integer values 0..14 with a fraction frac each of NaN, +inf and -inf."""
    a = a.copy()
    k = max(1, int(frac * len(a)))
    for v in (np.nan, np.inf, -np.inf):
        a[rng.choice(len(a), size=min(k, len(a)), replace=False)] = v
    return a


@pytest.mark.parametrize("dtype", ["f64", "f32", "f16"])
@pytest.mark.parametrize("variant,row_aligned", [("auto", None), ("flat", 0), ("adaptive", None), ("prefree", None)])
def test_special_values_match_oracle(variant, row_aligned, dtype):
    checked = 0
    for name, rp, col, n in CASES:
        rng = np.random.default_rng(len(col) + 7)
        val = plant(oracle.initvec(len(col), NP[dtype]), rng, 0.001)
        x = plant(oracle.initvec(n, NP[dtype]), rng, 0.002)
        if variant == "flat" and np.diff(rp).max() > 256:
            continue                                   # split tiles are the default there anyway
        y, info = gpu_spmv(rp, col, val, x, variant, dtype=dtype,
                           row_aligned=row_aligned if variant == "flat" else None)
        with np.errstate(invalid="ignore", over="ignore"):
            # fp16: exact products and sums, rounded once to binary16 (this library's fp16 semantics)
            ref = oracle.spmv_f16_rounded(rp, col, val, x) if dtype == "f16" else oracle.spmv_serial(rp, col, val, x)
        if dtype != "f64" and np.diff(rp).max() * 196 >= 2 ** 24:
            # finite sums beyond 2^24 may round differently in fp32: compare the specials only
            assert np.array_equal(np.isnan(y), np.isnan(ref)), name
            assert np.array_equal(np.isposinf(y), np.isposinf(ref)), name
            assert np.array_equal(np.isneginf(y), np.isneginf(ref)), name
        else:
            assert np.array_equal(y, ref, equal_nan=True), (name, info["variant_name"])
        checked += int(np.isnan(ref).any() or np.isinf(ref).any())
    assert checked >= 5        # the planted values reach y in most cases
