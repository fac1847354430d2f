#!/usr/bin/env python3
"""Offline tuner for gfx950: the reference's run_autotuning.sh +
scripts/profile_and_generate.py flow (:319-418 profile and analyse, :420-453
generate), re-targeted.

Each matrix of config.yaml falls in a class: its size class by nnz (the
reference's small / medium / large) and its row-length class from the same
statistics PF_AUTO reads (short, regular, skewed, dense; host/capi.cpp
row_class).  On one MI355X the tuner times, per matrix, every compiled
configuration of this library — FLAT tiles, the hybrid FLAT plan where the
matrix has dense rows, ADAPTIVE tiles x run lengths, PREFREE tiles (the
reference's P_NNZ 4 / 8) x its five reduction ladders (the reference tuner's
code axis, :99-235) — and PF_AUTO's own rule-based plan, each as the best of
two batches of back-to-back SpMVs, and checks each candidate's y against
AUTO's.  A matrix whose AUTO step takes under 20 us when launched one by one
is bound by the host's launch rate, which hides the kernels' differences: its
batches run as captured HIP graphs instead.  AUTO's built-in rules are a
candidate of their own (table variant "auto"), timed as the plan they made on
each matrix.  A class's score:

  1. time: the mean effective bandwidth (test/test_cdspmv.cpp:305 byte model)
     over the class's matrices;
  2. counters: among the candidates within `tie_band` of the best time that
     are no slower than AUTO's plan on any matrix of the class (beyond the
     timing noise `auto_guard`), rocprofv3 FETCH_SIZE + WRITE_SIZE per SpMV
     (every kernel of a step, scaled by a 256 MiB copy kernel measured in the
     same profiled process) decides: the fewest HBM bytes wins.  A third pass
     (TCC_HIT_sum, TCC_MISS_sum) records each counted candidate's L2 hit rate
     in the results beside its bytes.  (MALL hits are not separable on gfx950:
     TCC_EA0_RDREQ_DRAM_sum reads the same as TCC_EA0_RDREQ_sum.)  Equal time,
     fewer bytes leaves more of HBM to whatever runs beside the SpMV and
     loses less when the 256 MB MALL does not hold the matrix.
  3. guard: a winner must not be slower than AUTO's plan on any matrix of the
     class; otherwise the class's row is "auto", the built-in rules.  On equal
     time and bytes the rules win over a fixed configuration.

It writes
  * a tuning table (text) that PF_AUTO reads: by default from
    tune/mi355x_tuning_table.txt, else pf_set_tuning_table or
    $PREFREE_TUNING_TABLE — no source is generated or patched, no rebuild;
  * a results file (JSON) with every timing and counter reading.

The reference scored candidates by speedup over cuSPARSE; this tuner scores
them by time and measured traffic, which needs no vendor library.

usage: autotune.py [config.yaml] [--out DIR] [--counters | --no-counters]
       autotune.py --measure MATRIX DTYPE VARIANT TILE RUN KEEP LADDER HYBRID   (one profiled run)
"""
from __future__ import annotations

import argparse
import collections
import csv
import importlib.util
import json
import os
import subprocess
import sys
import tempfile
import time

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.dirname(HERE)
CLASSES = ("small", "medium", "large")
ROW_CLASSES = ("short", "regular", "skewed", "dense")
ALIGN_ROW_MAX = 256  # PFK_ALIGN_ROW_MAX, include/prefree_kernels.h
ROW_GROUP_MAX = 32   # FLAT "tiles" 2..32 are row groups (PFK_ROW_GROUP_TILE)
GRAPH_US = 20.0      # AUTO's step below this (eager): the matrix is timed as captured graphs
RULES = {"variant": "auto", "tile": 0, "run": 0, "keep": 0, "ladder": 0, "hybrid": 1}  # PF_AUTO's built-in rules
COPY_BYTES = 256 << 20


def load_pkg():
    if "prefree_amd" in sys.modules:
        return sys.modules["prefree_amd"]
    spec = importlib.util.spec_from_file_location("prefree_amd", os.path.join(PKG_DIR, "__init__.py"),
                                                  submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["prefree_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def classify(nnz, thresholds):
    if nnz < thresholds["small_upper"]:
        return "small"
    if nnz < thresholds["medium_upper"]:
        return "medium"
    return "large"


def row_class(m, nnz, max_row_len):
    """The row-length class of host/capi.cpp row_class (the cuts of PF_AUTO's rules)."""
    if max_row_len <= ALIGN_ROW_MAX:
        return "short" if nnz < 4 * m else "regular"
    return "skewed" if nnz < 16 * m else "dense"


def load_matrix(spec, dtype, values, seed=1):
    """(row_ptr, col, val, x, m, n) on the host for a .mtx path or 'synthetic:C<cfg>[:scale]'."""
    import numpy as np
    pf = load_pkg()
    np_t = {"f64": np.float64, "f32": np.float32, "f16": np.float16}[dtype]
    if spec.startswith("synthetic:"):
        parts = spec.split(":")
        cfg = int(parts[1].lstrip("Cc"))
        scale = int(parts[2]) if len(parts) > 2 else 0
        rp, col, vals = pf.synth_csr(cfg, seed=seed, scale_n=scale, vals=1 if values == "initvec" else 0,
                                     dtypes=(dtype,))
        m = n = len(rp) - 1
        val = vals[dtype]
        x = pf.synth_x(cfg, n, seed=seed, vals=1 if values == "initvec" else 0, dtypes=(dtype,))[dtype]
    else:
        rp, col, val64, m, n, _sym = pf.mtx_read(spec)
        if values == "initvec":    # test_cdspmv.cpp:291-292 with include/common.h:126-133
            val = (np.arange(len(col)) % 15).astype(np_t)
            x = (np.arange(n) % 15).astype(np_t)
        else:
            rng = np.random.default_rng(seed)
            val = rng.uniform(-1, 1, len(col)).astype(np_t)
            x = rng.uniform(-1, 1, n).astype(np_t)
    return rp, col, val, x, m, n


def cand_key(c):
    return (c["variant"], c["tile"], c["run"], c["keep"], c["ladder"], c["hybrid"])


def candidates(pf, dtype, cand_cfg):
    """Every configuration to time (the hybrid one is added per matrix when it applies)."""
    out = []

    def add(variant, tile, run=0, keep=0, ladder=0, hybrid=0):
        out.append({"variant": variant, "tile": tile, "run": run, "keep": keep, "ladder": ladder, "hybrid": hybrid})
    for t in pf.supported_tiles("flat", dtype):
        add("flat", t)
    for t in pf.supported_tiles("adaptive", dtype):
        for r in cand_cfg.get("adaptive_runs", [1, 2, 4, 8, 16]):
            for keep in ([0, 1] if cand_cfg.get("include_keep_cached") else [0]):
                add("adaptive", t, r, keep)
    if cand_cfg.get("include_prefree", True):
        for t in pf.supported_tiles("prefree", dtype):
            for ladder in cand_cfg.get("prefree_ladders", [1, 2, 3, 4, 5]):
                add("prefree", t, ladder=ladder)
    return out


def make_plan(pf, d, m, n, nnz, dtype, c, stream):
    """A plan for candidate c (variant 'auto': PF_AUTO's own choice); None if c does not apply."""
    if c["variant"] == "auto":
        return pf.Plan(d[0], d[1], m, n, nnz, dtype, "auto", 0, stream=stream)
    if c["hybrid"]:
        p = pf.Plan(d[0], d[1], m, n, nnz, dtype, "flat", 0, stream=stream)   # default tile: hybrid if it applies
        if not p.info.hybrid:
            p.close()
            return None
        return p
    p = pf.Plan(d[0], d[1], m, n, nnz, dtype, c["variant"], c["tile"], stream=stream)
    if c["variant"] == "flat" and c["tile"] <= ROW_GROUP_MAX and p.stats.max_row_len > ALIGN_ROW_MAX:
        p.close()  # row groups (lanes per row) are for short rows: a dense row would take one group
        return None
    if c["variant"] == "adaptive":
        p.set_run_tiles(c["run"])
        p.set_keep_cached(c["keep"])
    if c["variant"] == "prefree" and c["ladder"]:
        p.set_ladder(c["ladder"])
    return p


def describe_auto(info):
    """AUTO's plan as a candidate of the table."""
    v = load_pkg().VARIANT_NAMES.get(int(info.variant), "?")
    return {"variant": v, "tile": int(info.tile), "run": int(info.run_tiles) if v == "adaptive" else 0,
            "keep": int(info.keep_cached) if v == "adaptive" else 0,
            "ladder": int(info.ladder) if v == "prefree" else 0, "hybrid": int(info.hybrid)}


def time_candidates(spec, dtype, cfg, thresholds):
    """Mean microseconds per SpMV of every candidate on one matrix, and AUTO's plan."""
    import torch
    pf = load_pkg()
    values = cfg.get("values", "initvec")
    rp, col, val, x, m, n = load_matrix(spec, dtype, values)
    lens = rp[1:] - rp[:-1]
    nnz = len(col)
    rows = row_class(m, nnz, int(lens.max()) if m else 0)
    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream()
    d = [torch.from_numpy(a).to(dev) for a in (rp, col, val, x)]
    y = torch.empty(m, dtype=d[2].dtype, device=dev)
    y_auto = torch.empty_like(y)
    perf = cfg.get("performance_test", {})
    warm, iters = int(perf.get("warmup_iterations", 10)), int(perf.get("test_iterations", 100))
    vb = {"f64": 8, "f32": 4, "f16": 2}[dtype]
    bytes_eff = (nnz + m + n) * vb + nnz * 4 + (m + 1) * 4

    def run(c, out, graph=False):
        p = make_plan(pf, d, m, n, nnz, dtype, c, st)
        if p is None:
            return None, None
        with p:
            for _ in range(warm):
                p.execute(*d, out, stream=st)
            torch.cuda.synchronize()
            g = None
            if graph:  # the batch as one captured HIP graph: kernels back to back, no host launch in between
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    cs = torch.cuda.current_stream()
                    for _ in range(iters):
                        p.execute(*d, out, stream=cs)
                torch.cuda.synchronize()
                g.replay()
                torch.cuda.synchronize()
            best = float("inf")
            for _ in range(2):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(st)
                if g is not None:
                    g.replay()
                else:
                    for _ in range(iters):
                        p.execute(*d, out, stream=st)
                e1.record(st)
                torch.cuda.synchronize()
                best = min(best, e0.elapsed_time(e1) * 1e3 / iters)
            del g
            p.check(stream=st)
            return best, p.info

    us, info = run({"variant": "auto"}, y_auto)
    # A step under GRAPH_US is bound by the host's launch rate, which hides the kernels' own differences:
    # such matrices are timed as captured graphs, AUTO's plan again among them.
    graph = us < GRAPH_US
    if graph:
        us, info = run({"variant": "auto"}, y_auto, graph=True)
    auto = describe_auto(info)
    auto.update({"us": round(us, 3), "gbps": round(bytes_eff / (us * 1e3), 1), "graph": graph})
    print(json.dumps({"matrix": spec, "auto": auto}), flush=True)
    cands = candidates(pf, dtype, cfg.get("candidates", {}))
    cands.append({"variant": "flat", "tile": 0, "run": 0, "keep": 0, "ladder": 0, "hybrid": 1})
    exact = values == "initvec"
    # AUTO's built-in rules as a candidate of their own (a table row "auto"): per matrix, the plan they made
    out_rows = [dict(RULES, us=auto["us"], gbps=auto["gbps"], y_ok=True)]
    for c in cands:
        us, info = run(c, y, graph)
        if us is None:
            continue
        c = dict(c)
        if c["hybrid"]:
            # A hybrid step (dense rows, runs, partial sums) does not depend on the plan's base FLAT tile;
            # name it by AUTO's tile when AUTO's plan is the same hybrid plan, so the two share a key.
            c["tile"] = auto["tile"] if auto["variant"] == "flat" and auto["hybrid"] else int(info.tile)
        same = bool(torch.equal(y, y_auto)) if exact else \
            bool(torch.allclose(y.double(), y_auto.double(), rtol=1e-9, atol=1e-12))
        c.update({"us": round(us, 3), "gbps": round(bytes_eff / (us * 1e3), 1), "y_ok": same})
        out_rows.append(c)
        print(json.dumps({"matrix": spec, **c}), flush=True)
    del d, y, y_auto
    torch.cuda.empty_cache()
    return {"matrix": spec, "nnz": nnz, "m": m, "n": n, "bytes": bytes_eff, "size_class": classify(nnz, thresholds),
            "row_class": rows, "auto": auto, "candidates": out_rows}


def tie_set(mats, band, guard):
    """Candidates measured (and correct) on every matrix of a class: (best by time, the tie set)."""
    score = collections.defaultdict(list)
    for mat in mats:
        for c in mat["candidates"]:
            if c["y_ok"]:
                score[cand_key(c)].append((c["gbps"], c["us"], mat["auto"]["us"]))
    full = {k: v for k, v in score.items() if len(v) == len(mats)}
    if not full:
        return None, []
    mean = {k: sum(g for g, _, _ in v) / len(v) for k, v in full.items()}
    best = max(mean, key=mean.get)
    ties = [k for k in full if mean[k] >= mean[best] * (1 - band)
            and all(us <= a * (1 + guard) for _, us, a in full[k])]
    ties.sort(key=lambda k: -mean[k])
    return (best, mean), ties


def choose(per_class, band=0.01, guard=0.005, counter_fn=None, max_counted=3):
    """Winner per class key (size class, row class); see the module docstring for the score."""
    best = {}
    for key, mats in per_class.items():
        if not mats:
            continue
        top, ties = tie_set(mats, band, guard)
        if top is None:
            continue
        fastest, mean = top
        counted = {}
        if counter_fn and ties:
            for k in ties[:max_counted]:
                counted[k] = counter_fn(mats[0]["matrix"], dict(zip(("variant", "tile", "run", "keep", "ladder",
                                                                     "hybrid"), k)))
        ok = {k: v for k, v in counted.items() if "traffic_bytes" in v}
        if len(ok) > 1:
            pick = min(ok, key=lambda k: (ok[k]["traffic_bytes"], -mean[k]))
            why = f"fewest HBM bytes among {len(ok)} candidates tied on time"
        elif ok:
            pick = next(iter(ok))
            why = "time (the only candidate within the band; HBM bytes measured)"
        elif ties:
            pick = ties[0]
            why = "time"
        else:
            pick = cand_key(RULES)
            why = "no candidate beat AUTO's plan on every matrix: the built-in rules"
            if pick not in mean:  # AUTO's own timings
                mean[pick] = sum(m["bytes"] / (m["auto"]["us"] * 1e3) for m in mats) / len(mats)
        row = dict(zip(("variant", "tile", "run", "keep", "ladder", "hybrid"), pick))
        row.update({"mean_gbps": round(mean.get(pick, 0.0), 1), "fastest": dict(zip(
            ("variant", "tile", "run", "keep", "ladder", "hybrid"), fastest)), "why": why,
            "matrices": [m["matrix"] for m in mats],
            "auto": [{k: m["auto"][k] for k in ("variant", "tile", "run", "ladder", "hybrid", "us")} for m in mats],
            "us": [next((c["us"] for c in m["candidates"] if cand_key(c) == pick), m["auto"]["us"]) for m in mats]})
        if counted:
            row["counters"] = {"|".join(map(str, k)): v for k, v in counted.items()}
        best[key] = row
    return best


def write_table(best_by_dtype, thresholds, path, device=""):
    """The pf_set_tuning_table format: class nnz_upper rows dtype variant tile run keep ladder hybrid."""
    bounds = {"small": thresholds["small_upper"], "medium": thresholds["medium_upper"], "large": -1}
    lines = ["# preFree-MI355X tuning table, written by prefree-public_amd/tune/autotune.py"
             + (f" on {device}" if device else ""),
             "# class nnz_upper rows dtype variant tile run keep ladder hybrid"]
    for dtype, best in best_by_dtype.items():
        for rows in ROW_CLASSES:
            if not any((cls, rows) in best for cls in CLASSES):
                continue
            for cls in CLASSES:   # first match by nnz: a size class without a row keeps the built-in rules
                b = best.get((cls, rows))
                if not b:
                    lines.append(f"{cls} {bounds[cls]} {rows} {dtype} auto 0 0 0 0 1  # not measured")
                    continue
                note = f"{b['mean_gbps']} GB/s mean; {b['why']}"
                lines.append(f"{cls} {bounds[cls]} {rows} {dtype} {b['variant']} {b['tile']} {b['run']} "
                             f"{b['keep']} {b['ladder']} {b['hybrid']}  # {note}")
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")


def measure(args):
    """One profiled process: 20 SpMVs of one candidate, then 3 copies of 256 MiB for the counter scale."""
    import torch
    torch.cuda.init()  # before this library's first HIP call (see main)
    pf = load_pkg()
    pf.set_tuning_table(None)
    matrix, dtype, variant, tile, run, keep, ladder, hybrid = args
    c = {"variant": variant, "tile": int(tile), "run": int(run), "keep": int(keep), "ladder": int(ladder),
         "hybrid": int(hybrid)}
    rp, col, val, x, m, n = load_matrix(matrix, dtype, "initvec")
    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream()
    d = [torch.from_numpy(a).to(dev) for a in (rp, col, val, x)]
    y = torch.empty(m, dtype=d[2].dtype, device=dev)
    p = make_plan(pf, d, m, n, len(col), dtype, c, st)
    if p is None:
        raise SystemExit("candidate does not apply to this matrix")
    with p:
        for _ in range(20):
            p.execute(*d, y, stream=st)
        torch.cuda.synchronize()
    src = torch.ones(COPY_BYTES // 8, dtype=torch.float64, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()


def step_count(rows, counter, calls=20):
    """A counter's reading per SpMV step (every kernel dispatched once per call, `calls` times or more, summed
    per step; the copy kernel and the once-only planning and searching dispatches left out), unscaled."""
    by_kernel = collections.defaultdict(list)
    for r in rows:
        if r["Counter_Name"] == counter and "neg" not in r["Kernel_Name"]:
            by_kernel[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    step = [v for v in by_kernel.values() if len(v) >= calls - 1]
    return sum(sum(v) / len(v) for v in step) if step else None


def step_bytes(rows, counter, calls=20):
    """Bytes per SpMV step from one counter pass: every kernel dispatched once per call (`calls` times or
    more; planning kernels and the plan's first, searching call run once) summed per step, scaled by the
    copy kernel's reading for its known 256 MiB."""
    by_kernel = collections.defaultdict(list)
    copy = []
    for r in rows:
        if r["Counter_Name"] != counter:
            continue
        v = float(r["Counter_Value"])
        if "neg" in r["Kernel_Name"]:
            copy.append(v)
        else:
            by_kernel[r["Kernel_Name"]].append(v)
    step = [v for v in by_kernel.values() if len(v) >= calls - 1]
    if not step or not copy:
        return None, None
    scale = COPY_BYTES / (sum(copy) / len(copy))
    return int(sum(sum(v) / len(v) for v in step) * scale), scale


def counters_for(matrix, dtype, c):
    """rocprofv3 FETCH_SIZE and WRITE_SIZE of candidate c (two passes), in bytes per SpMV."""
    out = {}
    tmp = tempfile.mkdtemp(prefix="pf_tune_")
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        d = os.path.join(tmp, counter)
        cmd = ["timeout", "-s", "KILL", "120", "rocprofv3", "--pmc", counter, "--output-format", "csv", "-d", d,
               "-o", "run", "--", sys.executable, os.path.abspath(__file__), "--measure", matrix, dtype,
               c["variant"], str(c["tile"]), str(c["run"]), str(c["keep"]), str(c["ladder"]), str(c["hybrid"])]
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=150, cwd="/tmp",
                           env=dict(os.environ, TMPDIR="/tmp"))
        if r.returncode != 0:
            return {"error": f"rocprofv3 {counter} exit {r.returncode}"}
        rows = list(csv.DictReader(open(os.path.join(d, "run_counter_collection.csv"))))
        b, scale = step_bytes(rows, counter)
        if b is None:
            return {"error": f"no {counter} rows"}
        out[counter.lower() + "_bytes"] = b
        out[counter.lower() + "_scale"] = round(scale / 1024, 4)
    out["traffic_bytes"] = out["fetch_size_bytes"] + out["write_size_bytes"]
    # L2 hit rate of the step (reported beside the bytes, not scored): one more pass with two TCC counters
    d = os.path.join(tmp, "TCC")
    cmd = ["timeout", "-s", "KILL", "120", "rocprofv3", "--pmc", "TCC_HIT_sum", "TCC_MISS_sum", "--output-format", "csv",
           "-d", d, "-o", "run", "--", sys.executable, os.path.abspath(__file__), "--measure", matrix, dtype,
           c["variant"], str(c["tile"]), str(c["run"]), str(c["keep"]), str(c["ladder"]), str(c["hybrid"])]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=150, cwd="/tmp", env=dict(os.environ, TMPDIR="/tmp"))
    if r.returncode == 0:
        rows = list(csv.DictReader(open(os.path.join(d, "run_counter_collection.csv"))))
        hit, miss = step_count(rows, "TCC_HIT_sum"), step_count(rows, "TCC_MISS_sum")
        if hit is not None and miss is not None and hit + miss > 0:
            out["l2_hit_rate"] = round(hit / (hit + miss), 4)
    print(json.dumps({"matrix": matrix, "counters": c, **out}), flush=True)
    return out


def summary_of(results):
    """The results without the per-candidate timings: per class the winner, why, AUTO's plan and times."""
    out = {k: v for k, v in results.items() if k != "dtypes"}
    out["dtypes"] = {}
    for dt, r in results["dtypes"].items():
        mats = [{k: m[k] for k in ("matrix", "nnz", "m", "size_class", "row_class", "auto")} for m in r["matrices"]]
        out["dtypes"][dt] = {"classes": r["classes"], "matrices": mats}
    return out


def merge(dirs, out_dir, cfg):
    """One table and one results file from runs that each tuned other value types."""
    names = cfg.get("output", {})
    table_name = names.get("table_file", "tuning_table.txt")
    res_name = names.get("results_file", "tuning_results.json")
    head, rows, results = [], [], None
    for d in dirs:
        for line in open(os.path.join(d, table_name)):
            (head if line.startswith("#") else rows).append(line.rstrip("\n"))
        r = json.load(open(os.path.join(d, res_name)))
        if results is None:
            results = r
        else:
            results["dtypes"].update(r["dtypes"])
    os.makedirs(out_dir, exist_ok=True)
    with open(os.path.join(out_dir, table_name), "w") as f:
        f.write("\n".join(head[:2] + rows) + "\n")
    with open(os.path.join(out_dir, res_name), "w") as f:
        json.dump(results, f, indent=1)
    with open(os.path.join(out_dir, names.get("summary_file", "tuning_summary.json")), "w") as f:
        json.dump(summary_of(results), f, indent=1)
    print(json.dumps({"merged": dirs, "rows": len(rows)}), flush=True)
    return 0


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("config", nargs="?", default=os.path.join(HERE, "config.yaml"))
    ap.add_argument("--out", default=None, help="output directory (default: the config's directory)")
    ap.add_argument("--counters", dest="counters", action="store_true", default=None,
                    help="rank the time-tied candidates by rocprofv3 FETCH_SIZE + WRITE_SIZE (config 'counters')")
    ap.add_argument("--no-counters", dest="counters", action="store_false")
    ap.add_argument("--dtypes", default=None, help="comma list overriding the config's dtypes (e.g. f64)")
    ap.add_argument("--merge", nargs="+", metavar="DIR", default=None,
                    help="combine the tables and results of earlier runs (one per dtype) into --out")
    ap.add_argument("--measure", nargs=8,
                    metavar=("MATRIX", "DTYPE", "VARIANT", "TILE", "RUN", "KEEP", "LADDER", "HYBRID"),
                    help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.measure:
        measure(args.measure)
        return 0
    import yaml
    with open(args.config) as f:
        cfg = yaml.safe_load(f)
    if args.merge:
        return merge(args.merge, args.out or os.path.dirname(os.path.abspath(args.config)), cfg)
    # torch's bundled HIP runtime must initialise before this library's first
    # HIP call in the process (two runtimes share the device; the later one to
    # start otherwise finds no GPU).
    import torch
    torch.cuda.init()
    pf = load_pkg()
    pf.set_tuning_table(None)   # AUTO's built-in rules are the baseline, not a previous table
    out_dir = args.out or os.path.dirname(os.path.abspath(args.config))
    os.makedirs(out_dir, exist_ok=True)
    thresholds = cfg["size_thresholds"]
    use_counters = cfg.get("counters", True) if args.counters is None else args.counters
    score_cfg = cfg.get("score", {})
    band, guard = float(score_cfg.get("tie_band", 0.01)), float(score_cfg.get("auto_guard", 0.005))
    device = pf.device_name()
    results = {"timestamp": time.strftime("%Y-%m-%d %H:%M:%S"), "device": device, "tie_band": band,
               "auto_guard": guard, "counters": bool(use_counters), "dtypes": {}}
    best_by_dtype = {}
    for dtype in (args.dtypes.split(",") if args.dtypes else cfg.get("dtypes", ["f64"])):
        per_class = collections.defaultdict(list)
        for cls in CLASSES:
            for spec in cfg.get("test_matrices", {}).get(cls, []) or []:
                if not spec.startswith("synthetic:") and not os.path.exists(spec):
                    print(json.dumps({"warning": f"matrix not found: {spec}"}), flush=True)
                    continue
                r = time_candidates(spec, dtype, cfg, thresholds)
                if r["size_class"] != cls:
                    print(json.dumps({"note": f"{spec} has nnz {r['nnz']}: class {r['size_class']}, "
                                              f"listed under {cls}"}), flush=True)
                per_class[(r["size_class"], r["row_class"])].append(r)
        fn = (lambda mat, c, _dt=dtype: counters_for(mat, _dt, c)) if use_counters else None
        best = choose(per_class, band, guard, fn)
        best_by_dtype[dtype] = best
        results["dtypes"][dtype] = {"classes": {f"{k[0]}/{k[1]}": v for k, v in best.items()},
                                    "matrices": [m for mats in per_class.values() for m in mats]}
    table = os.path.join(out_dir, cfg.get("output", {}).get("table_file", "tuning_table.txt"))
    res = os.path.join(out_dir, cfg.get("output", {}).get("results_file", "tuning_results.json"))
    write_table(best_by_dtype, thresholds, table, device)
    with open(res, "w") as f:
        json.dump(results, f, indent=1)
    with open(os.path.join(out_dir, cfg.get("output", {}).get("summary_file", "tuning_summary.json")), "w") as f:
        json.dump(summary_of(results), f, indent=1)
    print(json.dumps({"table": table, "results": res,
                      "best": {dt: {f"{k[0]}/{k[1]}": {x: b[x] for x in ("variant", "tile", "run", "ladder",
                                                                          "hybrid", "mean_gbps", "why")}
                                    for k, b in best.items()} for dt, best in best_by_dtype.items()}}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
