"""Tuning: the size-class table PF_AUTO consults (pf_set_tuning_table) and the
online tuner (pf_plan_autotune)."""
import numpy as np
import pytest

import prefree_amd as pf
from test_abi import make_stats


@pytest.fixture
def table(tmp_path):
    path = tmp_path / "table.txt"
    yield path
    pf.set_tuning_table(None)


def test_table_rows_drive_auto(table):
    table.write_text("# class nnz_upper dtype variant tile run keep\n"
                     "small  1000000  f64 flat     2048 0 0\n"
                     "medium 30000000 f64 adaptive 238  5 1   # comment\n"
                     "large  -1       f64 adaptive 512  0 0\n"
                     "all    -1       f32 flat     4096 0 0\n")
    pf.set_tuning_table(str(table))
    small = pf.select(make_stats(10000, 160000, 16), "f64", "auto")
    assert small.variant == pf.FLAT and small.tile == 2048
    mid = pf.select(make_stats(4194304, 20963328, 5), "f64", "auto")
    assert mid.variant == pf.ADAPTIVE and mid.tile == 238 and mid.run_tiles == 5 and mid.keep_cached == 1
    big = pf.select(make_stats(1000000, 315000000, 499000), "f64", "auto")
    assert big.variant == pf.ADAPTIVE and big.tile == 512 and big.keep_cached == 0
    f32 = pf.select(make_stats(4194304, 20963328, 5), "f32", "auto")
    assert f32.variant == pf.FLAT and f32.tile == 4096
    # an explicit variant ignores the table
    assert pf.select(make_stats(4194304, 20963328, 5), "f64", "adaptive").tile == 512


def test_table_rows_with_unsupported_tiles_are_skipped(table):
    table.write_text("x -1 f64 adaptive 777 0 0\n")
    pf.set_tuning_table(str(table))
    assert pf.select(make_stats(4194304, 20963328, 5), "f64", "auto").tile == 1024   # built-in rule


def test_clearing_the_table_restores_the_rules(table):
    table.write_text("x -1 f64 flat 1024 0 0\n")
    pf.set_tuning_table(str(table))
    assert pf.select(make_stats(4194304, 20963328, 5), "f64", "auto").tile == 1024
    table.write_text("x -1 f64 adaptive 494 3 0\n")
    pf.set_tuning_table(str(table))
    assert pf.select(make_stats(4194304, 20963328, 5), "f64", "auto").variant == pf.ADAPTIVE
    pf.set_tuning_table(None)
    assert pf.select(make_stats(4194304, 20963328, 5), "f64", "auto").variant == pf.FLAT


@pytest.mark.parametrize("text", ["x 10 f64 adaptive\n", "x 10 f8 flat 1024 0 0\n", "x 10 f64 dense 4096 0 0\n",
                                  "x 10 f64 flat 4096 0 3\n", "x 10 f64 flat -5 0 0\n"])
def test_malformed_tables_are_rejected(table, text):
    table.write_text(text)
    with pytest.raises(pf.PrefreeError) as e:
        pf.set_tuning_table(str(table))
    assert e.value.status == 8


def test_missing_table_file():
    with pytest.raises(pf.PrefreeError) as e:
        pf.set_tuning_table("/nonexistent/table.txt")
    assert e.value.status == 8


@pytest.mark.gpu
@pytest.mark.parametrize("cfg,scale", [(2, 300), (5, 40000), (4, 200000)])
def test_autotune_picks_a_correct_faster_configuration(cfg, scale):
    import torch
    from gpu_util import DEV, assert_parity, dev
    rp, col, v = pf.synth_csr(cfg, seed=21, scale_n=scale)
    m = len(rp) - 1
    x = pf.synth_x(cfg, m, seed=21)["f64"]
    d = [dev(rp), dev(col), dev(v["f64"]), dev(x)]
    y = torch.full((m,), float("nan"), dtype=torch.float64, device=DEV)
    with pf.Plan(d[0], d[1], m, m, len(col), "f64", "auto") as p:
        r = p.autotune(*d, y, reps=5, flags=pf.TUNE_PREFREE)
        torch.cuda.synchronize()
        assert r["candidates"] > 10
        assert r["us"] <= r["default_us"]
        info = p.info
        assert (info.variant, info.tile) == (r["variant"], r["tile"])
        if info.variant == pf.ADAPTIVE:
            assert info.run_tiles == r["run_tiles"]
        if info.variant == pf.FLAT and info.tile in (1024, 2048):   # XCD chunk: the plan's rule or a tried size
            assert info.chunk_nnz == r["chunk_nnz"]
            assert r["chunk_nnz"] in (0, 1 << 13, 1 << 15, 1 << 17)
        assert_parity(rp, col, v["f64"], x, y.cpu().numpy(), "f64", what=f"C{cfg} autotune y")
        y2 = torch.full((m,), float("nan"), dtype=torch.float64, device=DEV)
        p.execute(*d, y2)
        torch.cuda.synchronize()
        p.check()
        assert_parity(rp, col, v["f64"], x, y2.cpu().numpy(), "f64", what=f"C{cfg} tuned plan")


def _autotune_module():
    import importlib.util
    import os
    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "prefree-public_amd", "tune",
                        "autotune.py")
    spec = importlib.util.spec_from_file_location("pf_autotune", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_offline_tuner_choice_and_table(table):
    at = _autotune_module()
    th = {"small_upper": 5000000, "medium_upper": 20000000}
    assert [at.classify(n, th) for n in (10, 4999999, 5000000, 19999999, 20000000)] == \
        ["small", "small", "medium", "medium", "large"]

    def mat(name, rows):
        return {"matrix": name, "candidates": [{"variant": v, "tile": t, "run": r, "keep": 0, "gbps": g}
                                               for v, t, r, g in rows]}
    per_class = {
        "small": [mat("a", [("adaptive", 188, 1, 100), ("flat", 4096, 0, 90)]),
                  mat("b", [("adaptive", 188, 1, 50), ("flat", 4096, 0, 80)])],    # flat wins on the mean: 85 > 75
        "medium": [],
        "large": [mat("c", [("adaptive", 494, 3, 4000), ("adaptive", 512, 16, 3900)])],
    }
    best = at.choose(per_class)
    assert best["small"]["variant"] == "flat" and best["small"]["mean_gbps"] == 85
    assert "medium" not in best
    assert (best["large"]["tile"], best["large"]["run"]) == (494, 3)
    at.write_table({"f64": best}, th, str(table))
    pf.set_tuning_table(str(table))
    assert pf.select(make_stats(10000, 160000, 16), "f64", "auto").variant == pf.FLAT
    large = pf.select(make_stats(4194304, 20963328, 5), "f64", "auto")
    assert (large.variant, large.tile, large.run_tiles) == (pf.ADAPTIVE, 494, 3)
    # a medium matrix falls through to the large row (no medium row, large has no bound)
    assert pf.select(make_stats(1000000, 6000000, 8), "f64", "auto").tile == 494


@pytest.mark.gpu
def test_offline_tuner_runs_end_to_end(tmp_path):
    import subprocess
    import sys
    import os
    at_path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "prefree-public_amd", "tune",
                           "autotune.py")
    cfg = tmp_path / "cfg.yaml"
    cfg.write_text("""size_thresholds: {small_upper: 100000, medium_upper: 1000000}
test_matrices:
  small: ["synthetic:C1"]
  medium: ["synthetic:C2:300"]
  large: ["synthetic:C4:400000"]
dtypes: [f64]
values: initvec
performance_test: {warmup_iterations: 2, test_iterations: 5}
candidates: {adaptive_runs: [1, 4], include_prefree: false}
""")
    r = subprocess.run([sys.executable, at_path, str(cfg), "--out", str(tmp_path)], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    pf.set_tuning_table(str(tmp_path / "tuning_table.txt"))
    try:
        text = (tmp_path / "tuning_table.txt").read_text()
        assert "small 100000 f64" in text and "large -1 f64" in text
    finally:
        pf.set_tuning_table(None)
