"""fp16 mode on the GPU (the reference's non-fp64 build, valT = half, include/common.h:43-46), through
the C ABI.  val, x and y are binary16; this library forms products and row sums in fp32 and rounds
each row sum once (oracle.spmv_f16_rounded), where the reference rounds every operation
(oracle.spmv_serial_f16).

* initVec inputs: bit-exact against the rounded model; against the reference's own fp16 semantics
  too wherever every row sum stays <= 2048 (all integers up to 2048 are binary16 values, so both
  are exact there);
* U[-1,1] inputs (fp64 draws rounded to binary16): per-row error against fp64 on the same fp16
  data at most 1e-3 * sum_j |a_ij x_j| + 2^-24 (one binary16 rounding: 2^-11 relative, or 2^-25
  absolute for a subnormal result; plus fp32 accumulation); empty rows exactly 0;
* both FLAT tilings (row-aligned and split rows), both tile sizes; ADAPTIVE at each of its tiles and
  PREFREE (the reference algorithm, every reduction ladder) under the same bars.  PREFREE keeps its
  tile-boundary rows' partials in fp32 and adds them in tile order (k_prefree_join) instead of the
  reference's half atomics: rows spanning hundreds of tiles are checked exactly.
"""
import numpy as np
import pytest
import torch

import oracle
import prefree_amd as pf
from csr_cases import csr_from_lengths, edge_cases
from gpu_util import DEV, assert_parity, dev, gpu_spmv, kat_exact_possible

pytestmark = pytest.mark.gpu

CASES = edge_cases()


def scaled():
    out = []
    for cfg, scale in ((1, 0), (2, 300), (3, 60000), (4, 400000), (5, 40000)):
        rp, col, _ = pf.synth_csr(cfg, seed=5, scale_n=scale, dtypes=())
        out.append((f"C{cfg}", rp, col, len(rp) - 1))
    return out


ALL = CASES + scaled()


@pytest.mark.parametrize("tile", [1024, 2048])
@pytest.mark.parametrize("case", range(len(ALL)), ids=[c[0] for c in ALL])
def test_f16_kat_bit_exact(case, tile):
    name, rp, col, n = ALL[case]
    val = oracle.initvec(len(col), np.float16)
    x = oracle.initvec(n, np.float16)
    aligned = [None] if len(rp) < 2 or np.diff(rp).max() > 256 else [None, 0]
    for ra in aligned:
        y, info = gpu_spmv(rp, col, val, x, "flat", tile=tile, dtype="f16", row_aligned=ra)
        assert info["tile"] == tile
        assert_parity(rp, col, val, x, y, "f16", exact=kat_exact_possible(rp, "f16"), what=f"{name}/ra={ra}")
        sums = oracle.spmv_f16_rounded(rp, col, val, x).astype(np.float64)
        if len(sums) and np.abs(sums).max() <= 2048:
            ref = oracle.spmv_serial_f16(rp, col, val, x)
            assert np.array_equal(ref.view(np.uint16), y.view(np.uint16)), f"{name}: reference fp16 semantics"


@pytest.mark.parametrize("tile", [1024, 2048])
@pytest.mark.parametrize("case", range(len(ALL)), ids=[c[0] for c in ALL])
def test_f16_random_within_tolerance(case, tile):
    name, rp, col, n = ALL[case]
    rng = np.random.default_rng(case + tile)
    val = rng.uniform(-1, 1, len(col)).astype(np.float16)
    x = rng.uniform(-1, 1, n).astype(np.float16)
    y, info = gpu_spmv(rp, col, val, x, "auto", tile=tile, dtype="f16")
    assert info["variant_name"] == "flat"
    assert_parity(rp, col, val, x, y, "f16", what=name)


def test_f16_rounds_once_not_per_operation():
    """Row [2048, 1, 1] times ones: one rounding of the fp32 sum gives 2050; the reference's per-operation
    binary16 rounding would give 2048 (2048 + 1 ties to even).  This library keeps the exact value."""
    rp = np.array([0, 3], dtype=np.int32)
    col = np.array([0, 1, 2], dtype=np.int32)
    val = np.array([2048, 1, 1], dtype=np.float16)
    x = np.ones(3, dtype=np.float16)
    y, _ = gpu_spmv(rp, col, val, x, "flat", tile=1024, dtype="f16")
    assert float(y[0]) == 2050.0
    assert float(oracle.spmv_serial_f16(rp, col, val, x)[0]) == 2048.0


OTHER = [("adaptive", 440), ("adaptive", 494), ("adaptive", 1024), ("prefree", 512), ("prefree", 1024)]


@pytest.mark.parametrize("variant,tile", OTHER, ids=[f"{v}-{t}" for v, t in OTHER])
@pytest.mark.parametrize("case", range(len(ALL)), ids=[c[0] for c in ALL])
def test_f16_adaptive_prefree(case, variant, tile):
    """initVec values bit-exact against the once-rounded sums (and the reference's per-operation fp16
    wherever its sums stay <= 2048); U[-1,1] values within the fp16 tolerance."""
    name, rp, col, n = ALL[case]
    val = oracle.initvec(len(col), np.float16)
    x = oracle.initvec(n, np.float16)
    y, info = gpu_spmv(rp, col, val, x, variant, tile=tile, dtype="f16")
    assert info["variant_name"] == variant and info["tile"] == tile
    assert_parity(rp, col, val, x, y, "f16", exact=kat_exact_possible(rp, "f16"), what=f"{name}/{variant}")
    sums = oracle.spmv_f16_rounded(rp, col, val, x).astype(np.float64)
    if len(sums) and np.abs(sums).max() <= 2048:
        ref = oracle.spmv_serial_f16(rp, col, val, x)
        assert np.array_equal(ref.view(np.uint16), y.view(np.uint16)), f"{name}: reference fp16 semantics"
    rng = np.random.default_rng(case + tile)
    val = rng.uniform(-1, 1, len(col)).astype(np.float16)
    x = rng.uniform(-1, 1, n).astype(np.float16)
    y, _ = gpu_spmv(rp, col, val, x, variant, tile=tile, dtype="f16")
    assert_parity(rp, col, val, x, y, "f16", what=f"{name}/{variant}")


def _spanning_rows(seed=3):
    """Short rows around rows of 40k-200k nnz (up to 390 tiles of 512 nnz each, beyond one wave's 64 tiles
    per round of k_prefree_join), single-row tiles between them; values whose sums stay exact in fp16."""
    rng = np.random.default_rng(seed)
    lengths = []
    for big in (200000, 40000, 65 * 512, 64 * 512 + 1, 513):
        lengths += [int(v) for v in rng.integers(0, 30, size=300)] + [big]
    lengths += [int(v) for v in rng.integers(0, 30, size=300)]
    n = 300000
    rp, col = csr_from_lengths(lengths, n, rng)
    val = np.ones(len(col), dtype=np.float16)
    x = rng.integers(-3, 4, size=n).astype(np.float16)
    return rp, col, val, x, n


@pytest.mark.parametrize("ladder", [1, 2, 3, 4, 5])
@pytest.mark.parametrize("tile", [512, 1024])
def test_f16_prefree_ladders_and_spanning_rows(ladder, tile):
    """Every ladder; rows whose partials span up to 390 tiles are joined in tile order exactly."""
    rp, col, val, x, n = _spanning_rows()
    y, info = gpu_spmv(rp, col, val, x, "prefree", tile=tile, dtype="f16", ladder=ladder)
    assert info["ladder"] == ladder
    want = oracle.spmv_f16_rounded(rp, col, val, x)
    assert np.abs(want.astype(np.float64)).max() <= 2048  # integer sums, exact in fp16 and fp32
    assert np.array_equal(want.view(np.uint16), y.view(np.uint16))
    for name, rp2, col2, n2 in CASES:  # the edge shapes under this ladder
        v2, x2 = oracle.initvec(len(col2), np.float16), oracle.initvec(n2, np.float16)
        y2, _ = gpu_spmv(rp2, col2, v2, x2, "prefree", tile=tile, dtype="f16", ladder=ladder)
        assert_parity(rp2, col2, v2, x2, y2, "f16", exact=kat_exact_possible(rp2, "f16"), what=f"{name}/{ladder}")


def test_f16_overflow_gives_infinity():
    rp = np.array([0, 2, 3], dtype=np.int32)
    col = np.array([0, 1, 0], dtype=np.int32)
    val = np.array([60000, 60000, 1], dtype=np.float16)
    x = np.ones(2, dtype=np.float16)
    y, _ = gpu_spmv(rp, col, val, x, "flat", tile=1024, dtype="f16")
    assert np.isinf(y[0]) and y[1] == 1.0
