"""Randomly drawn CSR shapes on the GPU, every variant and value type, against the oracle.

Forty matrices from fixed seeds, each drawn from one of several row-length models (Poisson, power law,
dense rows among short ones, banded with outliers, mostly empty rows), with uniform or banded columns,
sorted or not within rows, square or rectangular.  Each runs under PF_AUTO (whatever plan it makes:
row-aligned or split-row FLAT, hybrid, band, ADAPTIVE), FLAT at both tiles, ADAPTIVE and PREFREE (a drawn
ladder), in a drawn value type: initVec values bit for bit against the oracle, U[-1,1] values within the
tolerance.  The case's parameters are in every assertion message.
"""
import numpy as np
import pytest

import oracle
import prefree_amd as pf
from gpu_util import NP, assert_parity, gpu_spmv, kat_exact_possible

pytestmark = pytest.mark.gpu

MODELS = ("poisson", "power", "dense_mix", "banded", "sparse")


def _lengths(model, m, rng):
    if model == "poisson":
        return rng.poisson(rng.uniform(0.5, 40.0), size=m)
    if model == "power":
        return np.minimum(rng.zipf(rng.uniform(1.6, 3.0), size=m), 20000)
    if model == "dense_mix":
        lens = rng.integers(0, 40, size=m)
        k = int(rng.integers(1, 12))
        lens[rng.choice(m, size=min(k, m), replace=False)] = rng.integers(5000, 30000, size=min(k, m))
        return lens
    if model == "banded":
        return rng.poisson(rng.uniform(1.0, 6.0), size=m)
    return np.where(rng.random(m) < 0.03, rng.integers(1, 60, size=m), 0)  # mostly empty rows


def _case(seed):
    rng = np.random.default_rng(1000 + seed)
    model = MODELS[seed % len(MODELS)]
    big = seed % 10 in (3, 7)  # x over 4 MB: band (banded) and hybrid (dense rows) candidates
    m = int(rng.integers(600000, 800000)) if big else int(rng.integers(1, 60000))
    n = m if rng.random() < 0.6 else int(rng.integers(1, 2 * m + 2))
    lens = _lengths(model, m, rng).astype(np.int64)
    lens = np.minimum(lens, 4_000_000 // max(m, 1) + 30000)  # keep every case under a few M nnz
    rp = np.zeros(m + 1, dtype=np.int64)
    np.cumsum(lens, out=rp[1:])
    row = np.repeat(np.arange(m, dtype=np.int64), lens)
    if model == "banded":
        w = int(rng.choice([64, 512, 4096]))
        col = np.clip(row * n // max(m, 1) + rng.integers(-w, w + 1, size=len(row)), 0, n - 1)
        out = rng.random(len(row)) < 0.1
        col[out] = rng.integers(0, n, size=int(out.sum()))
    else:
        col = rng.integers(0, n, size=len(row))
    sort = rng.random() < 0.8
    if sort:
        col = np.sort(row * n + col) % n
    dtype = str(rng.choice(["f64", "f32", "f16"], p=[0.5, 0.3, 0.2]))
    ladder = int(rng.integers(1, 6))
    what = f"seed={seed} model={model} m={m} n={n} nnz={len(col)} sorted={sort} dtype={dtype}"
    return rp.astype(np.int32), col.astype(np.int32), n, dtype, ladder, what


CASES = list(range(40))


@pytest.mark.parametrize("seed", CASES)
def test_random_shape_every_variant(seed):
    rp, col, n, dtype, ladder, what = _case(seed)
    rng = np.random.default_rng(seed)
    kv, kx = oracle.initvec(len(col), NP[dtype]), oracle.initvec(n, NP[dtype])
    uv = rng.uniform(-1, 1, len(col)).astype(NP[dtype])
    ux = rng.uniform(-1, 1, n).astype(NP[dtype])
    runs = [("auto", 0, None), ("flat", 1024, None), ("flat", 2048, None)]
    runs.append(("adaptive", pf.supported_tiles("adaptive", dtype)[0], None))
    runs.append(("prefree", 512 if seed % 2 else 1024, ladder))
    for variant, tile, lad in runs:
        tag = f"{what} {variant}/{tile}" + (f"/ladder {lad}" if lad else "")
        y, info = gpu_spmv(rp, col, kv, kx, variant, tile=tile, dtype=dtype, ladder=lad)
        assert_parity(rp, col, kv, kx, y, dtype, exact=kat_exact_possible(rp, dtype),
                      what=f"{tag} kat plan={info['variant_name']} hybrid={info['hybrid']} band={info['band_w']}")
        y, info = gpu_spmv(rp, col, uv, ux, variant, tile=tile, dtype=dtype, ladder=lad)
        assert_parity(rp, col, uv, ux, y, dtype,
                      what=f"{tag} random plan={info['variant_name']} hybrid={info['hybrid']} band={info['band_w']}")
