"""Tiling of the ADAPTIVE and FLAT kernels — CPU only.

The model (csr_cases.tile_model) states what each workgroup of k_tiles
computes from row_ptr; check_tiling verifies the invariants that make any
tiling correct.  The GPU descriptors are compared against the model in
tests/test_gpu_index.py.  Planted mistakes confirm the checker catches a wrong
descriptor.
"""
import numpy as np
import pytest

import prefree_amd as pf
from csr_cases import check_tiling, edge_cases, tile_model

LMAX = {188: 64, 238: 16, 440: 64, 494: 16, 512: 252, 1024: 508, 2048: 1020, 4096: 2044}


def all_cases():
    cases = [(name, rp) for name, rp, _col, _n in edge_cases()]
    for cfg, scale in ((1, 4096), (2, 40), (3, 30000), (4, 20000), (5, 20000)):
        rp, _, _ = pf.synth_csr(cfg, seed=2, scale_n=scale, dtypes=())
        cases.append((f"C{cfg}", rp))
    return cases


@pytest.mark.parametrize("tile", [188, 238, 440, 494, 512, 1024, 2048, 4096])
@pytest.mark.parametrize("merged", [True, False], ids=["adaptive", "flat"])
def test_model_satisfies_invariants(tile, merged):
    lmax = LMAX[tile] if merged else 0
    for name, rp in all_cases():
        desc = tile_model(rp, tile, merged, lmax)
        check_tiling(rp, desc, tile, lmax, merged)


ALIGN_MAX = 256   # PFK_ALIGN_ROW_MAX: longest row of a row-aligned FLAT plan


@pytest.mark.parametrize("tile", [1024, 2048])
def test_row_aligned_model_satisfies_invariants(tile):
    """Row-aligned FLAT tiles: every nnz and row exactly once, no split, and
    the span the kernel's product buffer holds (K + 255 nnz past kb)."""
    n = 0
    for name, rp in all_cases():
        if len(rp) < 2 or np.diff(rp).max() > ALIGN_MAX:
            continue
        n += 1
        desc = tile_model(rp, tile, False, 0, aligned=True)
        check_tiling(rp, desc, tile, ALIGN_MAX, False)
        kb = np.arange(len(desc)) * tile
        assert np.all(desc[:, 2] >= kb), name
        assert np.all(desc[:, 3] - kb < tile + ALIGN_MAX), name
        # same row map (first row of each tile) as the split tiling
        split = tile_model(rp, tile, False, 0)
        rows_split = np.where(split[:, 4] == 1, split[:, 0] + 1, split[:, 0])
        assert np.array_equal(desc[:, 0], rows_split), name
    assert n >= 10


def test_adaptive_tiles_are_balanced():
    for name, rp in all_cases():
        desc = tile_model(rp, 188, True, 64)
        work = desc[:, 1] + (desc[:, 3] - desc[:, 2])   # rows + nnz of each tile
        assert work.max() <= 188 + 64 + 1, name


def test_lmax_matches_kernel_library():
    for dt in ("f64", "f32"):
        for tile in pf.supported_tiles("adaptive", dt):
            assert pf.adaptive_long_row_min(dt, tile) == LMAX[tile]


@pytest.mark.parametrize("mutation", ["shift_A", "drop_row", "flip_head", "flip_tail", "short_B"])
def test_checker_catches_planted_mistakes(mutation):
    rp = [c[1] for c in all_cases() if c[0] == "power_law_mix"][0]
    desc = tile_model(rp, 1024, True, 508)
    t = int(np.flatnonzero((desc[:, 4] == 1) | (desc[:, 5] == 1))[0]) if mutation.startswith("flip") else len(desc) // 2
    bad = desc.copy()
    if mutation == "shift_A":
        bad[t, 2] += 1
    elif mutation == "drop_row":
        bad[t, 1] -= 1
    elif mutation == "flip_head":
        bad[t, 4] ^= 1
    elif mutation == "flip_tail":
        bad[t, 5] ^= 1
    else:
        bad[t, 3] -= 1
    with pytest.raises(AssertionError):
        check_tiling(rp, bad, 1024, 508, True)
