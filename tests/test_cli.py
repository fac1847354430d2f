"""The cdspmv harness (prefree-public_amd/bin/cdspmv), the counterpart of the
reference's test/test_cdspmv.cpp driver: Matrix Market in, initVec values,
preFreeSpMV, a sequential CPU check, our_perf / our_pre lines out.
"""
import os
import re
import subprocess

import numpy as np
import pytest

import prefree_amd as pf

CLI = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "prefree-public_amd", "bin", "cdspmv")


def run(args, env_extra=None, timeout=120):
    env = dict(os.environ)
    env.update({"PREFREE_WARMUP": "5", "PREFREE_ITERS": "20"})
    env.update(env_extra or {})
    return subprocess.run([CLI] + args, capture_output=True, text=True, timeout=timeout, env=env)


def write_mtx(path, rp, col, symmetric=False, val=None):
    m = len(rp) - 1
    n = int(col.max()) + 1 if len(col) else m
    rows = np.repeat(np.arange(m), np.diff(rp))
    keep = rows >= col if symmetric else np.ones(len(col), bool)
    lines = [f"%%MatrixMarket matrix coordinate real {'symmetric' if symmetric else 'general'}",
             f"{m} {max(n, m) if symmetric else n} {int(keep.sum())}"]
    vals = val if val is not None else np.ones(len(col))
    lines += [f"{r + 1} {c + 1} {float(v)!r}" for r, c, v, k in zip(rows, col, vals, keep) if k]
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")


def test_usage_without_arguments():
    r = run([])
    assert r.returncode == 0 and "cdspmv matrix.mtx" in r.stdout


def test_unreadable_file_is_an_error():
    r = run(["/nonexistent/x.mtx"])
    assert r.returncode == 2 and "cannot read" in r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("prec", ["f64", "f32"])
@pytest.mark.parametrize("variant", ["auto", "prefree", "adaptive", "flat"])
def test_cli_laplacian_passes_check(tmp_path, prec, variant):
    rp, col, _ = pf.synth_csr(2, seed=1, scale_n=64, dtypes=())
    f = str(tmp_path / "lap.mtx")
    write_mtx(f, rp, col)
    args = [f, "--variant", variant] + (["--f32"] if prec == "f32" else [])
    r = run(args)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "Success!" in r.stdout
    m = re.search(r"our_perf:\s*([0-9.]+) ms, our_pre:\s*([0-9.]+) ms", r.stdout)
    assert m and float(m.group(1)) > 0
    assert f"nnz = {len(col)}" in r.stdout
    # the vendor line the reference's tuner parses (scripts/profile_and_generate.py:299-300), from rocSPARSE
    v = re.search(r"cusparse_perf:\s*([0-9.]+) ms, cusparse_pre:\s*([0-9.]+) ms", r.stdout)
    assert v and float(v.group(1)) > 0 and float(v.group(2)) >= 0, r.stdout
    assert "vendor: rocSPARSE" in r.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("cfg,scale", [(2, 64), (3, 5000)])
@pytest.mark.parametrize("variant", ["auto", "flat"])
def test_cli_f16_passes_check(tmp_path, cfg, scale, variant):
    """The reference's fp16 build: binary16 values, the sequential check rounds every operation."""
    rp, col, _ = pf.synth_csr(cfg, seed=3, scale_n=scale, dtypes=())
    f = str(tmp_path / "a.mtx")
    write_mtx(f, rp, col)
    r = run([f, "--f16", "--variant", variant])
    assert r.returncode == 0, r.stdout + r.stderr
    assert "Success!" in r.stdout and "our_perf:" in r.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("variant", ["prefree", "adaptive"])
def test_cli_f16_reference_algorithm(tmp_path, variant):
    """--f16 with the reference algorithm (PREFREE) and ADAPTIVE passes the harness's fp16 check."""
    rp, col, _ = pf.synth_csr(2, seed=1, scale_n=32, dtypes=())
    f = str(tmp_path / "lap.mtx")
    write_mtx(f, rp, col)
    r = run([f, "--f16", "--variant", variant])
    assert r.returncode == 0, r.stdout + r.stderr
    assert "Success!" in r.stdout and "our_perf:" in r.stdout


@pytest.mark.gpu
def test_cli_symmetric_power_law(tmp_path):
    rp, col, _ = pf.synth_csr(3, seed=2, scale_n=5000, dtypes=())
    f = str(tmp_path / "pl.mtx")
    write_mtx(f, rp, col, symmetric=True)
    r = run([f])
    assert r.returncode == 0, r.stdout + r.stderr
    assert "Success!" in r.stdout and "our_total:" in r.stdout


PFSTAT = os.path.join(os.path.dirname(CLI), "pfstat")


def test_pfstat_usage_and_bad_file():
    r = subprocess.run([PFSTAT], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "usage: pfstat" in r.stdout
    r = subprocess.run([PFSTAT, "/nonexistent/x.mtx"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2


@pytest.mark.gpu
@pytest.mark.parametrize("variant", ["prefree", "adaptive", "flat"])
def test_pfstat_tile_statistics(tmp_path, variant):
    """Per-tile spans and row-piece lengths: pieces partition the nnz, spans cover the rows in order."""
    import csv
    import oracle
    rp, col, _ = pf.synth_csr(3, seed=4, scale_n=20000, dtypes=())
    f = str(tmp_path / "pl.mtx")
    write_mtx(f, rp, col)
    out = tmp_path / "stat"
    r = subprocess.run([PFSTAT, f, "--variant", variant, "--out", str(out)], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    name = "pl.csv" if variant == "prefree" else f"pl_{variant}.csv"
    rows = list(csv.DictReader(open(out / name)))
    nnz = int(rp[-1])
    tile = int(re.search(r"tiling: \w+, (\d+)", r.stdout).group(1))
    m = len(rp) - 1
    pieces, tol = 0.0, 0.0
    for t in rows:
        s, e = int(t["start_row"]), int(t["end_row"])
        assert 0 <= s <= e <= m
        assert int(t["max_row_length"]) <= (tile if variant != "adaptive" else tile + 252)
        pieces += float(t["avg_row_length"]) * (e - s)
        tol += 0.005 * (e - s)                                   # averages are printed to 2 decimals
    assert abs(pieces - nnz) <= tol + 1e-9 * nnz
    if variant == "prefree":
        ref = oracle.pre_start_row(rp, tile)
        assert [int(t["start_row"]) for t in rows] == [int(v) for v in ref[:len(rows)]]
        assert len(rows) == -(-nnz // tile)
    assert "PF_AUTO:" in r.stdout
