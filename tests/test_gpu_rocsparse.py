"""The vendor comparator (prefree-public_amd/bin/rocsparse_spmv): rocSPARSE's v2
SpMV on the synthetic benchmark matrices beside this library's y, the
counterpart of the cuSPARSE comparison in the reference harness
(test/test_cdspmv.cpp:155-267).  rocSPARSE's y is not pinned against the oracle
here (the reference never checks cuSPARSE's either); the comparator's own
row-normalised difference from this library's y must stay within the fp64
tolerance, and every algorithm must run and report a time, with this
library's time from the same C++ launch loop beside it."""
import json
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "prefree-public_amd", "bin",
                   "rocsparse_spmv")
CASES = [(1, "adaptive", 0), (1, "rowsplit", 0), (2, "adaptive", 300), (2, "nnzsplit", 300), (3, "lrb", 60000),
         (5, "adaptive", 20000)]


@pytest.mark.parametrize("cfg,alg,scale", CASES, ids=[f"C{c}-{a}" for c, a, _ in CASES])
def test_rocsparse_matches_this_library(cfg, alg, scale):
    print(f"rocsparse_spmv C{cfg} {alg} scale {scale}", flush=True)
    args = [BIN, str(cfg), alg, "--iters", "20"] + (["--scale", str(scale)] if scale else [])
    r = subprocess.run(args, capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, r.stderr[-2000:]
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["cfg"] == f"C{cfg}" and line["rocsparse_alg"] == alg
    assert line["us"] > 0 and line["preprocess_ms"] >= 0 and line["prefree_us"] > 0
    assert line["max_rownorm_diff_vs_prefree"] <= 1e-12, line
