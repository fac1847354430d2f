#!/usr/bin/env python3
"""Offline tuner for gfx950: the reference's run_autotuning.sh +
scripts/profile_and_generate.py flow (:319-418 profile and analyse, :420-453
generate), re-targeted.

For every matrix of every size class (config.yaml) it times every compiled
configuration of this library — (variant, tile) and, for ADAPTIVE, the run
length — as back-to-back SpMVs on one MI355X, averages the effective bandwidth
(test/test_cdspmv.cpp:305 byte model) per class and writes

  * a tuning table (text) that PF_AUTO reads through pf_set_tuning_table or
    $PREFREE_TUNING_TABLE — no source is generated or patched, no rebuild;
  * a results file (JSON) with every timing and, with `counters: true`, the
    rocprofv3 FETCH_SIZE / WRITE_SIZE bytes of each class's winner, scaled by
    a 256 MiB copy kernel measured in the same profiled process.

The reference scored candidates by speedup over cuSPARSE; this tuner scores
them by achieved bandwidth, which needs no vendor library.

usage: autotune.py [config.yaml] [--out DIR] [--counters]
       autotune.py --measure <matrix> <dtype> <variant> <tile> <run>   (one profiled run)
"""
from __future__ import annotations

import argparse
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
# The tile kernels of prefree-public_amd/csrc/prefree_kernels.hip (the dominant kernel of a step).
TILE_KERNELS = ("k_wave", "k_rows", "k_flat", "k_flow", "k_tiles", "k_prefree")


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


def candidates(pf, dtype, cand_cfg):
    out = []
    for t in pf.supported_tiles("adaptive", dtype):
        for r in cand_cfg.get("adaptive_runs", [1, 2, 4, 8, 16]):
            for keep in ([0, 1] if cand_cfg.get("include_keep_cached") else [0]):
                out.append(("adaptive", t, r, keep))
    for t in pf.supported_tiles("flat", dtype):
        out.append(("flat", t, 0, 0))
    if cand_cfg.get("include_prefree"):
        for t in pf.supported_tiles("prefree", dtype):
            out.append(("prefree", t, 0, 0))
    return out


def time_candidates(spec, dtype, cfg):
    """Mean microseconds per SpMV of every candidate on one matrix."""
    import torch
    pf = load_pkg()
    rp, col, val, x, m, n = load_matrix(spec, dtype, cfg.get("values", "initvec"))
    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream()
    d = [torch.from_numpy(a).to(dev) for a in (rp, col, val, x)]
    y = torch.empty(m, dtype=d[2].dtype, device=dev)
    perf = cfg.get("performance_test", {})
    warm, iters = int(perf.get("warmup_iterations", 10)), int(perf.get("test_iterations", 100))
    vb = 8 if dtype == "f64" else 4
    nnz = len(col)
    bytes_eff = (nnz + m + n) * vb + nnz * 4 + (m + 1) * 4
    rows = []
    for variant, tile, run, keep in candidates(pf, dtype, cfg.get("candidates", {})):
        with pf.Plan(d[0], d[1], m, n, nnz, dtype, variant, tile, stream=st) as p:
            if variant == "adaptive":
                p.set_run_tiles(run)
                p.set_keep_cached(keep)
            for _ in range(warm):
                p.execute(*d, y, stream=st)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(st)
            for _ in range(iters):
                p.execute(*d, y, stream=st)
            e1.record(st)
            torch.cuda.synchronize()
            p.check(stream=st)
            us = e0.elapsed_time(e1) * 1e3 / iters
        rows.append({"variant": variant, "tile": tile, "run": run, "keep": keep, "us": round(us, 3),
                     "gbps": round(bytes_eff / (us * 1e3), 1)})
        print(json.dumps({"matrix": spec, **rows[-1]}), flush=True)
    del d, y
    torch.cuda.empty_cache()
    return {"matrix": spec, "nnz": nnz, "m": m, "n": n, "bytes": bytes_eff, "candidates": rows}


def choose(per_class):
    """Best candidate per class: the highest mean effective bandwidth over the class's matrices."""
    best = {}
    for cls, mats in per_class.items():
        if not mats:
            continue
        score = {}
        for mat in mats:
            for c in mat["candidates"]:
                key = (c["variant"], c["tile"], c["run"], c["keep"])
                score.setdefault(key, []).append(c["gbps"])
        full = {k: sum(v) / len(v) for k, v in score.items() if len(v) == len(mats)}
        if not full:
            continue
        key = max(full, key=full.get)
        best[cls] = {"variant": key[0], "tile": key[1], "run": key[2], "keep": key[3],
                     "mean_gbps": round(full[key], 1), "matrices": [m["matrix"] for m in mats]}
    return best


def write_table(best_by_dtype, thresholds, path):
    """The pf_set_tuning_table format: class nnz_upper dtype variant tile run keep."""
    bounds = {"small": thresholds["small_upper"], "medium": thresholds["medium_upper"], "large": -1}
    lines = ["# preFree-MI355X tuning table, written by prefree-public_amd/tune/autotune.py",
             "# class nnz_upper dtype variant tile run keep"]
    for dtype, best in best_by_dtype.items():
        for cls in CLASSES:
            if cls in best:
                b = best[cls]
                lines.append(f"{cls} {bounds[cls]} {dtype} {b['variant']} {b['tile']} {b['run']} {b['keep']}"
                             f"  # {b['mean_gbps']} GB/s mean")
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")


def measure(args):
    """One profiled process: 20 SpMVs of one candidate, then 3 copies of 256 MiB for the counter scale."""
    import torch
    torch.cuda.init()  # before this library's first HIP call (see main)
    pf = load_pkg()
    matrix, dtype, variant, tile, run = args
    rp, col, val, x, m, n = load_matrix(matrix, dtype, "initvec")
    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream()
    d = [torch.from_numpy(a).to(dev) for a in (rp, col, val, x)]
    y = torch.empty(m, dtype=d[2].dtype, device=dev)
    with pf.Plan(d[0], d[1], m, n, len(col), dtype, variant, int(tile), stream=st) as p:
        if variant == "adaptive" and int(run):
            p.set_run_tiles(int(run))
        for _ in range(20):
            p.execute(*d, y, stream=st)
        torch.cuda.synchronize()
    src = torch.ones(1 << 25, dtype=torch.float64, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()


def counters_for(matrix, dtype, b):
    """rocprofv3 FETCH_SIZE and WRITE_SIZE of the winner (two passes), in bytes per SpMV."""
    out = {}
    tmp = tempfile.mkdtemp(prefix="pf_tune_")
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        d = os.path.join(tmp, counter)
        cmd = ["rocprofv3", "--pmc", counter, "--output-format", "csv", "-d", d, "-o", "run", "--",
               sys.executable, os.path.abspath(__file__), "--measure", matrix, dtype, b["variant"], str(b["tile"]),
               str(b["run"])]
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=120, cwd="/tmp",
                           env=dict(os.environ, TMPDIR="/tmp"))
        if r.returncode != 0:
            return {"error": f"rocprofv3 {counter} exit {r.returncode}"}
        rows = list(csv.DictReader(open(os.path.join(d, "run_counter_collection.csv"))))
        main = [float(x["Counter_Value"]) for x in rows if x["Counter_Name"] == counter and
                any(k in x["Kernel_Name"] for k in TILE_KERNELS)]
        copy = [float(x["Counter_Value"]) for x in rows if x["Counter_Name"] == counter and "neg" in x["Kernel_Name"]]
        if not main or not copy:
            return {"error": f"no {counter} rows"}
        scale = (256 << 20) / (sum(copy) / len(copy))
        out[counter.lower() + "_bytes"] = int(sum(main) / len(main) * scale)
        out[counter.lower() + "_scale"] = round(scale / 1024, 4)
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("config", nargs="?", default=os.path.join(HERE, "config.yaml"))
    ap.add_argument("--out", default=None, help="output directory (default: the config's directory)")
    ap.add_argument("--counters", action="store_true", help="collect rocprofv3 counters of each class's winner")
    ap.add_argument("--measure", nargs=5, metavar=("MATRIX", "DTYPE", "VARIANT", "TILE", "RUN"),
                    help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.measure:
        measure(args.measure)
        return 0
    import yaml
    with open(args.config) as f:
        cfg = yaml.safe_load(f)
    # torch's bundled HIP runtime must initialise before this library's first
    # HIP call in the process (two runtimes share the device; the later one to
    # start otherwise finds no GPU).
    import torch
    torch.cuda.init()
    out_dir = args.out or os.path.dirname(os.path.abspath(args.config))
    os.makedirs(out_dir, exist_ok=True)
    thresholds = cfg["size_thresholds"]
    results = {"timestamp": time.strftime("%Y-%m-%d %H:%M:%S"), "device": load_pkg().device_name(), "dtypes": {}}
    best_by_dtype = {}
    for dtype in cfg.get("dtypes", ["f64"]):
        per_class = {c: [] for c in CLASSES}
        for cls in CLASSES:
            for spec in cfg.get("test_matrices", {}).get(cls, []) or []:
                if not spec.startswith("synthetic:") and not os.path.exists(spec):
                    print(json.dumps({"warning": f"matrix not found: {spec}"}), flush=True)
                    continue
                r = time_candidates(spec, dtype, cfg)
                actual = classify(r["nnz"], thresholds)
                if actual != cls:
                    print(json.dumps({"note": f"{spec} has nnz {r['nnz']}: class {actual}, listed under {cls}"}))
                per_class[actual].append(r)
        best = choose(per_class)
        if cfg.get("counters") or args.counters:
            for cls, b in best.items():
                b["counters"] = counters_for(b["matrices"][0], dtype, b)
        best_by_dtype[dtype] = best
        results["dtypes"][dtype] = {"classes": best, "matrices": per_class}
    table = os.path.join(out_dir, cfg.get("output", {}).get("table_file", "tuning_table.txt"))
    res = os.path.join(out_dir, cfg.get("output", {}).get("results_file", "tuning_results.json"))
    write_table(best_by_dtype, thresholds, table)
    with open(res, "w") as f:
        json.dump(results, f, indent=1)
    print(json.dumps({"table": table, "results": res,
                      "best": {dt: {c: {k: b[k] for k in ("variant", "tile", "run", "mean_gbps")}
                                    for c, b in best.items()} for dt, best in best_by_dtype.items()}}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
