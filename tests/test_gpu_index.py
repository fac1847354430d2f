"""Index-level parity on the GPU (bit-exact integer work).

* The row search each workgroup of k_tiles runs (with and without the
  interpolated first probe round) must give exactly the tile descriptors of
  the model in csr_cases.tile_model, which tests/test_tiling_model.py pins by
  invariants.
* k_prefree's in-kernel first row per tile must equal the reference pre-pass
  map, oracle.pre_start_row (restating src/spmv_kernel/preFreeSpMV.cu:3-28).
"""
import numpy as np
import pytest
import torch

import oracle
import prefree_amd as pf
from csr_cases import edge_cases, tile_model
from gpu_util import DEV, dev

pytestmark = pytest.mark.gpu

LMAX = {188: 64, 238: 16, 440: 64, 494: 16, 512: 252, 1024: 508, 2048: 1020, 4096: 2044}


def cases():
    out = [(name, rp) for name, rp, _c, _n in edge_cases()]
    for cfg, scale in ((1, 0), (2, 300), (3, 60000), (4, 400000), (5, 40000)):
        rp, _, _ = pf.synth_csr(cfg, seed=6, scale_n=scale, dtypes=())
        out.append((f"C{cfg}", rp))
    return out


CASES = cases()


# FLAT 256 (k_flow) finds rows by scanning forward and FLAT 2..32 (row groups) index rows directly, not by
# tile descriptors; parity tests cover both.
TILES = [(True, t) for t in pf.supported_tiles("adaptive", "f64")] + \
        [(False, t) for t in pf.supported_tiles("flat", "f64") if t > 256]


@pytest.mark.parametrize("spread,run", [(0, 0), (1, 1), (64, 3), (1000, 8), (64, 64)])
@pytest.mark.parametrize("merged,tile", TILES, ids=[("adaptive" if mg else "flat") + str(t) for mg, t in TILES])
def test_tile_descriptors_match_model(merged, tile, spread, run):
    for name, rp in CASES:
        m, nnz = len(rp) - 1, int(rp[-1])
        if m == 0:
            continue
        model = tile_model(rp, tile, merged, LMAX[tile] if merged else 0)
        ntiles = len(model)
        out = torch.full((8 * ntiles,), -7, dtype=torch.int32, device=DEV)
        err = torch.zeros(64, dtype=torch.int32, device=DEV)
        got_tiles = pf.tile_descriptors(dev(rp), m, nnz, tile, merged, out, err, guess_spread=spread, run_tiles=run)
        torch.cuda.synchronize()
        assert got_tiles == ntiles
        got = out.cpu().numpy().reshape(ntiles, 8)[:, :6].astype(np.int64)
        assert int(err.cpu()[0]) == 0, name
        bad = np.flatnonzero(np.any(got != model, axis=1))
        assert bad.size == 0, f"{name}: tile {bad[0]} got {got[bad[0]]} model {model[bad[0]]}"


LINES = [None, "fit", "steep", "shallow", "offset", "huge"]


def _line(rp, kind):
    """A first-guess line row = a * key + b for the row-aligned tiles' searches: the plan's fit through the
    quartile rows, or deliberately wrong ones (any line must give the same rows)."""
    m, nnz = len(rp) - 1, int(rp[-1])
    if kind is None or nnz == 0:
        return 0.0, 0.0
    a = m / nnz
    return {"fit": (a, 0.0), "steep": (3.0 * a, 0.0), "shallow": (a / 7.0, 5.0), "offset": (a, -0.3 * m),
            "huge": (1e12, 1e15)}[kind]


@pytest.mark.parametrize("line", LINES, ids=[str(k) for k in LINES])
@pytest.mark.parametrize("spread,chunk", [(0, 0), (1, 1 << 15), (2, 3000), (16, 1 << 15), (64, 1 << 15),
                                          (1000, 3000)])
@pytest.mark.parametrize("tile", [1024, 2048])
def test_row_aligned_descriptors_match_model(tile, spread, chunk, line):
    """Row-aligned FLAT tiles (rows starting in the tile, whole): exact descriptors wherever no
    tile's last row reaches 256 or more nnz past the tile's nominal end (always so when rows hold at
    most 256 nnz, the planning rule); otherwise the kernel refuses (error flag), since its product
    buffer holds K + 255 nnz.  Every tile reports once whatever the XCD chunk (slots start at -7)."""
    for name, rp in CASES:
        m, nnz = len(rp) - 1, int(rp[-1])
        if m == 0:
            continue
        model = tile_model(rp, tile, False, 0, aligned=True)
        ntiles = len(model)
        out = torch.full((8 * ntiles,), -7, dtype=torch.int32, device=DEV)
        err = torch.zeros(64, dtype=torch.int32, device=DEV)
        ga, gb = _line(rp, line)
        got_tiles = pf.tile_descriptors(dev(rp), m, nnz, tile, False, out, err, guess_spread=spread,
                                        row_aligned=True, chunk_nnz=chunk, guess_a=ga, guess_b=gb)
        torch.cuda.synchronize()
        assert got_tiles == ntiles
        kb = np.arange(ntiles - 1, dtype=np.int64) * tile
        if np.any(model[:-1, 3] - (kb + tile) >= 256):
            assert int(err.cpu()[0]) != 0, name
            continue
        assert int(err.cpu()[0]) == 0, name
        got = out.cpu().numpy().reshape(ntiles, 8)[:, :6].astype(np.int64)
        bad = np.flatnonzero(np.any(got != model, axis=1))
        assert bad.size == 0, f"{name}: tile {bad[0]} got {got[bad[0]]} model {model[bad[0]]}"


OWNER_TILES = [(dt, t) for dt in ("f64", "f32") for t in pf.supported_tiles("adaptive", dt)]


@pytest.mark.parametrize("dtype,tile", OWNER_TILES, ids=[f"{d}-{t}" for d, t in OWNER_TILES])
def test_adaptive_owner_table_matches_model(dtype, tile):
    """The per-pattern owner table (row whose split starts in a tile, else -1) the plan builds."""
    for name, rp in CASES:
        m, nnz = len(rp) - 1, int(rp[-1])
        if m == 0:
            continue
        model = tile_model(rp, tile, True, LMAX[tile])
        want = np.where(model[:, 5] == 1, model[:, 0] + model[:, 1] - 1, -1)
        out = torch.full((len(model),), -7, dtype=torch.int32, device=DEV)
        err = torch.zeros(64, dtype=torch.int32, device=DEV)
        nt = pf.adaptive_owners(dev(rp), m, nnz, tile, out, err, dtype=dtype, guess_spread=64, run_tiles=3)
        torch.cuda.synchronize()
        assert nt == len(model)
        assert int(err.cpu()[0]) == 0, name
        got = out.cpu().numpy().astype(np.int64)
        bad = np.flatnonzero(got != want)
        assert bad.size == 0, f"{name}: tile {bad[0]} owner {got[bad[0]]} model {want[bad[0]]}"


@pytest.mark.parametrize("tile", [512, 1024])
def test_prefree_rows_match_prepass(tile):
    for name, rp in CASES:
        m, nnz = len(rp) - 1, int(rp[-1])
        if nnz == 0:
            continue
        ref = oracle.pre_start_row(rp, tile)
        ntiles = len(ref) - 1
        out = torch.full((ntiles + 1,), -7, dtype=torch.int32, device=DEV)
        pf.prefree_rows(dev(rp), m, nnz, tile, out)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert np.array_equal(got[:ntiles], ref[:ntiles]), name
        assert got[ntiles] == m
