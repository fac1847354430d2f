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
                                  "x 10 f64 flat 4096 0 3\n", "x 10 f64 flat -5 0 0\n",
                                  "x 10 wide f64 flat 1024 0 0 0 1\n", "x 10 short f64 flat 1024 0 0 3 1\n",
                                  "x 10 short f64 prefree 512 0 0 6 1\n", "x 10 short f64 flat 1024 0 0 0 2\n",
                                  "x 1e5 short f64 flat 1024 0 0 0 1\n", "x 10 short f64 flat 1024 0 0 0\n",
                                  "x 10 short f64 auto 512 0 0 0 1\n", "x 10 short f64 flat 0 0 0 0 1\n"])
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


@pytest.mark.gpu
def test_autotune_times_launch_bound_plans_as_graphs():
    """C1 (65k nnz) launched call by call is bound by the host's launch rate: pf_plan_autotune then times every
    candidate as a captured graph, so its figures fall below the eager per-call time, and it keeps a correct
    plan whose graph time is no worse than the default's."""
    import torch
    from gpu_util import DEV, assert_parity, dev
    rp, col, v = pf.synth_csr(1, seed=4)
    m = len(rp) - 1
    x = pf.synth_x(1, m, seed=4)["f64"]
    d = [dev(rp), dev(col), dev(v["f64"]), dev(x)]
    y = torch.full((m,), float("nan"), dtype=torch.float64, device=DEV)
    with pf.Plan(d[0], d[1], m, m, len(col), "f64", "auto") as p:
        s = torch.cuda.current_stream()
        for _ in range(5):
            p.execute(*d, y, stream=s)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(200):
            p.execute(*d, y, stream=s)
        e1.record(s)
        torch.cuda.synchronize()
        eager_us = e0.elapsed_time(e1) * 1e3 / 200
        print(f"C1 eager {eager_us:.2f} us per call", flush=True)
        r = p.autotune(*d, y, reps=50)
        torch.cuda.synchronize()
        print(f"C1 autotune {r}", flush=True)
        assert r["us"] <= r["default_us"]
        assert r["default_us"] < eager_us, (r, eager_us)  # graph-timed: below the launch-bound eager time
        assert_parity(rp, col, v["f64"], x, y.cpu().numpy(), "f64", what="C1 autotune y")
        y.fill_(float("nan"))
        p.execute(*d, y)
        torch.cuda.synchronize()
        p.check()
        assert_parity(rp, col, v["f64"], x, y.cpu().numpy(), "f64", what="C1 tuned plan")


def _autotune_module():
    import importlib.util
    import os
    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "prefree-public_amd", "tune",
                        "autotune.py")
    spec = importlib.util.spec_from_file_location("pf_autotune", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_offline_tuner_classes_match_the_library():
    at = _autotune_module()
    th = {"small_upper": 5000000, "medium_upper": 20000000}
    assert [at.classify(n, th) for n in (10, 4999999, 5000000, 19999999, 20000000)] == \
        ["small", "small", "medium", "medium", "large"]
    # the row classes of host/capi.cpp row_class: C1 regular, C2 regular, C3 skewed, C4 short, C5 dense
    assert at.row_class(4096, 65536, 16) == "regular"
    assert at.row_class(4194304, 20963328, 5) == "regular"
    assert at.row_class(2000000, 15266620, 200000) == "skewed"
    assert at.row_class(20000000, 49994499, 16) == "short"
    assert at.row_class(1000000, 315647995, 498998) == "dense"
    assert at.row_class(10, 40, 256) == "regular" and at.row_class(10, 39, 256) == "short"
    assert at.row_class(10, 160, 257) == "dense" and at.row_class(10, 159, 257) == "skewed"


def _cand(v, t, us, gbps, run=0, ladder=0, hybrid=0, ok=True):
    return {"variant": v, "tile": t, "run": run, "keep": 0, "ladder": ladder, "hybrid": hybrid, "us": us,
            "gbps": gbps, "y_ok": ok}


def _mat(name, auto, cands):
    """A matrix as time_candidates returns it: AUTO's built-in rules first, timed as AUTO's own plan."""
    same = [c for c in cands if all(c[k] == auto[k] for k in ("variant", "tile", "run", "ladder", "hybrid"))]
    rules = dict(_cand("auto", 0, auto["us"], same[0]["gbps"], hybrid=1))
    return {"matrix": name, "auto": auto, "candidates": [rules] + cands}


def test_offline_tuner_score_time_then_counters_then_guard(table):
    at = _autotune_module()
    auto_flat = {"variant": "flat", "tile": 1024, "run": 0, "keep": 0, "ladder": 0, "hybrid": 0, "us": 10.0}
    per_class = {
        # time decides: prefree ladder 4 is fastest on the mean and no slower than AUTO anywhere
        ("small", "regular"): [
            _mat("a", auto_flat, [_cand("flat", 1024, 10.0, 100), _cand("prefree", 512, 8.0, 125, ladder=4)]),
            _mat("b", auto_flat, [_cand("flat", 1024, 10.0, 100), _cand("prefree", 512, 9.0, 111, ladder=4)])],
        # a tie on time (within 1%): the counters decide, the fewest bytes win
        ("large", "dense"): [
            _mat("c", dict(auto_flat, tile=2048, hybrid=1),
                 [_cand("flat", 2048, 10.0, 500, hybrid=1), _cand("flat", 2048, 10.04, 498.0),
                  _cand("adaptive", 512, 30.0, 166, run=4)])],
        # faster on the mean but slower than AUTO on one matrix: the built-in rules stay
        ("medium", "skewed"): [
            _mat("d", auto_flat, [_cand("flat", 1024, 10.0, 100), _cand("flat", 2048, 5.0, 200)]),
            _mat("e", auto_flat, [_cand("flat", 1024, 10.0, 100), _cand("flat", 2048, 10.5, 95)])],
        # a candidate with a wrong y never wins
        ("large", "short"): [
            _mat("f", auto_flat, [_cand("flat", 1024, 10.0, 100), _cand("flat", 4096, 5.0, 200, ok=False)])],
    }
    traffic = {("flat", 2048, 0, 0, 0, 1): 900, ("flat", 2048, 0, 0, 0, 0): 800}
    seen = []

    def counters(matrix, c):
        seen.append((matrix, c["variant"], c["tile"], c["hybrid"]))
        return {"traffic_bytes": traffic.get(at.cand_key(c), 1000)}
    best = at.choose(per_class, band=0.01, guard=0.005, counter_fn=counters)
    assert (best[("small", "regular")]["variant"], best[("small", "regular")]["ladder"]) == ("prefree", 4)
    dense = best[("large", "dense")]
    assert (dense["variant"], dense["tile"], dense["hybrid"]) == ("flat", 2048, 0)
    assert dense["fastest"]["hybrid"] == 1 and "fewest HBM bytes" in dense["why"]
    assert sorted(x for x in seen if x[0] == "c") == [("c", "auto", 0, 1), ("c", "flat", 2048, 0),
                                                       ("c", "flat", 2048, 1)]
    assert best[("medium", "skewed")]["variant"] == "auto" and "built-in rules" in best[("medium", "skewed")]["why"]
    assert best[("large", "short")]["variant"] == "auto"  # AUTO's flat 1024 and the rules tie; the rules come first
    # without counters the fastest of the tie wins; on equal time the rules (listed first) stay
    best2 = at.choose(per_class, band=0.01, guard=0.005)
    assert best2[("large", "dense")]["variant"] == "auto"
    per_class[("large", "dense")][0]["candidates"][1]["gbps"] = 503.0  # the hybrid plan 0.6% faster
    assert at.choose(per_class, band=0.01, guard=0.005)[("large", "dense")]["hybrid"] == 1

    th = {"small_upper": 5000000, "medium_upper": 20000000}
    at.write_table({"f64": best}, th, str(table), "test device")
    text = table.read_text()
    assert "small 5000000 regular f64 prefree 512 0 0 4 0" in text
    assert "large -1 dense f64 flat 2048 0 0 0 0" in text
    assert "medium 20000000 skewed f64 auto 0 0 0 0 1" in text
    pf.set_tuning_table(str(table))
    assert pf.tuning_table() == str(table)
    sel = pf.select(make_stats(10000, 160000, 16), "f64", "auto")          # small, regular
    assert (sel.variant, sel.tile, sel.ladder) == (pf.PREFREE, 512, 4)
    assert "small 5000000 short f64 auto 0 0 0 0 1" in text
    sel = pf.select(make_stats(10000, 20000, 3), "f64", "auto")            # small, short: not measured, the rules
    assert (sel.variant, sel.tile) == (pf.FLAT, 4)                         # row groups: the longest row, 3 nnz
    sel = pf.select(make_stats(2000000, 15266620, 200000), "f64", "auto")  # medium, skewed
    assert (sel.variant, sel.tile) == (pf.FLAT, 1024)


def test_step_bytes_sums_the_kernels_of_a_step():
    at = _autotune_module()
    rows = []
    for i in range(20):      # k_a 20 dispatches (one per call), k_b 19 (recorded rows), k_b search 1, planning 1
        rows.append({"Counter_Name": "FETCH_SIZE", "Kernel_Name": "k_a<double>", "Counter_Value": "100"})
        if i:
            rows.append({"Counter_Name": "FETCH_SIZE", "Kernel_Name": "k_b<double, 1>", "Counter_Value": "50"})
    rows.append({"Counter_Name": "FETCH_SIZE", "Kernel_Name": "k_b<double, 0>", "Counter_Value": "999"})
    rows.append({"Counter_Name": "FETCH_SIZE", "Kernel_Name": "k_row_stats", "Counter_Value": "999"})
    for _ in range(3):
        rows.append({"Counter_Name": "FETCH_SIZE", "Kernel_Name": "neg_kernel", "Counter_Value": str(131072)})
    b, scale = at.step_bytes(rows, "FETCH_SIZE")
    assert scale == (256 << 20) / 131072
    assert b == int(150 * scale)


def test_step_count_sums_the_kernels_of_a_step_unscaled():
    at = _autotune_module()
    rows = []
    for i in range(20):
        rows.append({"Counter_Name": "TCC_HIT_sum", "Kernel_Name": "k_a<double>", "Counter_Value": "30"})
        rows.append({"Counter_Name": "TCC_HIT_sum", "Kernel_Name": "k_b<double, 1>", "Counter_Value": "12"})
        rows.append({"Counter_Name": "TCC_MISS_sum", "Kernel_Name": "k_a<double>", "Counter_Value": "10"})
    rows.append({"Counter_Name": "TCC_HIT_sum", "Kernel_Name": "k_row_stats", "Counter_Value": "999"})
    rows.append({"Counter_Name": "TCC_HIT_sum", "Kernel_Name": "neg_kernel", "Counter_Value": "5000"})
    assert at.step_count(rows, "TCC_HIT_sum") == 42
    assert at.step_count(rows, "TCC_MISS_sum") == 10
    assert at.step_count(rows, "TCC_EA0_RDREQ_sum") is None


def test_offline_tuner_merges_runs_per_dtype(tmp_path):
    import json
    at = _autotune_module()
    dirs = []
    for dt, row in (("f64", "large -1 dense f64 flat 2048 0 0 0 1"), ("f32", "large -1 dense f32 flat 2048 0 0 0 1")):
        d = tmp_path / dt
        d.mkdir()
        (d / "tuning_table.txt").write_text(f"# head {dt}\n# columns\n{row}  # note\n")
        (d / "tuning_results.json").write_text(json.dumps({"device": "x", "dtypes": {dt: {"classes": {}, "matrices": [
            {"matrix": "m", "nnz": 1, "m": 1, "size_class": "small", "row_class": "short", "auto": {},
             "candidates": [{"us": 1.0}]}]}}}))
        dirs.append(str(d))
    out = tmp_path / "out"
    assert at.merge(dirs, str(out), {}) == 0
    lines = (out / "tuning_table.txt").read_text().splitlines()
    assert lines[0] == "# head f64" and len([x for x in lines if not x.startswith("#")]) == 2
    assert set(json.load(open(out / "tuning_results.json"))["dtypes"]) == {"f64", "f32"}
    summary = json.load(open(out / "tuning_summary.json"))
    assert set(summary["dtypes"]) == {"f64", "f32"}
    assert "candidates" not in summary["dtypes"]["f64"]["matrices"][0]
    pf.set_tuning_table(str(out / "tuning_table.txt"))
    pf.set_tuning_table(None)


def test_v2_rows_key_by_row_class(table):
    table.write_text("# class nnz_upper rows dtype variant tile run keep ladder hybrid\n"
                     "a -1 short   f64 flat     2048 0 0 0 1\n"
                     "b -1 regular f64 adaptive 238  3 0 0 1\n"
                     "c -1 skewed  f64 prefree  1024 0 0 5 1\n"
                     "d -1 dense   f64 flat     2048 0 0 0 0\n"
                     "e -1 any     f32 flat     4096 0 0 0 1\n")
    pf.set_tuning_table(str(table))
    assert pf.select(make_stats(20000000, 49994499, 16), "f64", "auto").tile == 2048
    r = pf.select(make_stats(4194304, 20963328, 5), "f64", "auto")
    assert (r.variant, r.tile, r.run_tiles) == (pf.ADAPTIVE, 238, 3)
    r = pf.select(make_stats(2000000, 15266620, 200000), "f64", "auto")
    assert (r.variant, r.tile, r.ladder) == (pf.PREFREE, 1024, 5)
    r = pf.select(make_stats(1000000, 315647995, 498998), "f64", "auto")
    assert (r.variant, r.tile) == (pf.FLAT, 2048)
    assert pf.select(make_stats(2000000, 15266620, 200000), "f32", "auto").tile == 4096


def test_default_table_is_loaded_unless_switched_off():
    import os
    import subprocess
    import sys
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = ("import importlib.util, sys; d = sys.argv[1]; "
            "s = importlib.util.spec_from_file_location('prefree_amd', d + '/__init__.py', "
            "submodule_search_locations=[d]); m = importlib.util.module_from_spec(s); "
            "sys.modules['prefree_amd'] = m; s.loader.exec_module(m); print(repr(m.tuning_table()))")
    pkg = os.path.join(repo, "prefree-public_amd")
    env = {k: v for k, v in os.environ.items() if k != "PREFREE_TUNING_TABLE"}
    out = subprocess.run([sys.executable, "-c", code, pkg], env=env, capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    path = eval(out.stdout.strip())
    assert path.endswith("tune/mi355x_tuning_table.txt")
    assert os.path.samefile(path, os.path.join(pkg, "tune", "mi355x_tuning_table.txt"))
    out = subprocess.run([sys.executable, "-c", code, pkg], env=dict(env, PREFREE_TUNING_TABLE=""),
                         capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and eval(out.stdout.strip()) == ""


def test_committed_table_parses_and_names_the_row_classes(table):
    import os
    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "prefree-public_amd", "tune",
                        "mi355x_tuning_table.txt")
    pf.set_tuning_table(path)
    for line in open(path):
        line = line.split("#")[0].split()
        if line:
            assert len(line) == 10 and line[2] in ("short", "regular", "skewed", "dense", "any"), line


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
candidates: {adaptive_runs: [1, 4], include_prefree: true, prefree_ladders: [2, 4]}
counters: false
""")
    r = subprocess.run([sys.executable, at_path, str(cfg), "--out", str(tmp_path)], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    pf.set_tuning_table(str(tmp_path / "tuning_table.txt"))
    try:
        text = (tmp_path / "tuning_table.txt").read_text()
        assert "small 100000 regular f64" in text and "medium 1000000 regular f64" in text
        assert "large -1 short f64" in text
        import json
        res = json.load(open(tmp_path / "tuning_results.json"))
        mats = res["dtypes"]["f64"]["matrices"]
        assert {m["row_class"] for m in mats} == {"regular", "short"}
        for m in mats:
            kinds = {(c["variant"], c["ladder"]) for c in m["candidates"]}
            assert ("prefree", 2) in kinds and ("prefree", 4) in kinds
            assert all(c["y_ok"] for c in m["candidates"]), m["matrix"]
            assert m["auto"]["us"] > 0
    finally:
        pf.set_tuning_table(None)


@pytest.mark.gpu
def test_table_hybrid_flag_and_ladder_reach_the_plan(table):
    import torch
    from gpu_util import DEV, assert_parity, dev
    rp, col, v = pf.synth_csr(5, seed=4, scale_n=100000)   # every long row dense: a hybrid plan applies
    m = len(rp) - 1
    x = pf.synth_x(5, m, seed=4)["f64"]
    d = [dev(rp), dev(col), dev(v["f64"]), dev(x)]
    for hybrid in (0, 1):
        table.write_text(f"t -1 dense f64 flat 2048 0 0 0 {hybrid}\n")
        pf.set_tuning_table(str(table))
        y = torch.full((m,), float("nan"), dtype=torch.float64, device=DEV)
        with pf.Plan(d[0], d[1], m, m, len(col), "f64", "auto") as p:
            assert (p.info.variant, p.info.tile, p.info.hybrid) == (pf.FLAT, 2048, hybrid)
            p.execute(*d, y)
            torch.cuda.synchronize()
            p.check()
        assert_parity(rp, col, v["f64"], x, y.cpu().numpy(), "f64", what=f"table hybrid {hybrid}")
    table.write_text("t -1 dense f64 prefree 1024 0 0 4 1\n")
    pf.set_tuning_table(str(table))
    y = torch.full((m,), float("nan"), dtype=torch.float64, device=DEV)
    with pf.Plan(d[0], d[1], m, m, len(col), "f64", "auto") as p:
        assert (p.info.variant, p.info.tile, p.info.ladder) == (pf.PREFREE, 1024, 4)
        p.execute(*d, y)
        torch.cuda.synchronize()
    assert_parity(rp, col, v["f64"], x, y.cpu().numpy(), "f64", what="table ladder 4")


@pytest.mark.gpu
@pytest.mark.parametrize("cfg,scale", [(1, 0), (2, 512), (3, 400000), (4, 1600000), (5, 20000)])
@pytest.mark.parametrize("dtype", ["f64", "f32"])
def test_committed_table_plans_are_correct(table, cfg, scale, dtype):
    """PF_AUTO under the table that ships with the library: parity on scaled C1-C5."""
    import os
    import torch
    from gpu_util import DEV, NP, assert_parity, dev
    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "prefree-public_amd", "tune",
                        "mi355x_tuning_table.txt")
    pf.set_tuning_table(path)
    rp, col, v = pf.synth_csr(cfg, seed=8, scale_n=scale, dtypes=(dtype,))
    m = len(rp) - 1
    x = pf.synth_x(cfg, m, seed=8, dtypes=(dtype,))[dtype]
    d = [dev(rp), dev(col), dev(v[dtype]), dev(x)]
    y = torch.full((m,), float("nan"), dtype=d[2].dtype, device=DEV)
    with pf.Plan(d[0], d[1], m, m, len(col), dtype, "auto") as p:
        for _ in range(2):
            p.execute(*d, y)
        torch.cuda.synchronize()
        p.check()
    assert_parity(rp, col, v[dtype], x, y.cpu().numpy(), dtype, what=f"C{cfg} {dtype} under the committed table")
