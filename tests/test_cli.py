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


@pytest.mark.gpu
def test_cli_symmetric_power_law(tmp_path):
    rp, col, _ = pf.synth_csr(3, seed=2, scale_n=5000, dtypes=())
    f = str(tmp_path / "pl.mtx")
    write_mtx(f, rp, col, symmetric=True)
    r = run([f])
    assert r.returncode == 0, r.stdout + r.stderr
    assert "Success!" in r.stdout and "our_total:" in r.stdout
