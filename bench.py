#!/usr/bin/env python3
"""bench.py — CSR SpMV throughput on one MI355X, every benchmark configuration.

One step = one y = A·x (pf_plan_execute) over the whole matrix, inputs already
resident in HBM.  The headline (`value`, `roofline`, `cpu_baseline`) is C5, the
largest single-GPU configuration of BASELINE.json (mixed dense rows, n = 10^6,
about 316M nnz, fp64); `configs` holds the same record for C1, C2, C3, C4,
C4 in fp32 and C5.  --config N measures configuration N alone (and makes it
the headline).

Per configuration:
  * hot      `steps` back-to-back steps.  `ms` is the host clock around them,
             bracketed by device synchronisation; `kernel_ms` the HIP events on
             the launch stream (the roofline's time base); a median of 40
             event-timed batches when steps are launched one by one.
  * rotated  the same steps alternating between enough device copies of the
             whole working set (row_ptr, col, val, x, y) to exceed 768 MB, so a
             step cannot find the previous step's lines in the 256 MB MALL.
  * cold     a 1 GiB write before each step (evicts L2 and MALL; the flush's
             own write-back overlaps the step's start).
  * search   a plan that finds every tile's rows by searching row_ptr in the
             kernel on every call, instead of reading the rows its first call
             recorded (pf_plan_set_remember_rows(plan, 0)).
  * cpu_baseline  the OpenMP restatement of the reference's spmv_serial
             (oracle/, all host cores) on the same matrix, and `parity`, the
             north-star row error of the GPU y against it.
`roofline.achieved` is the reference harness's effective-byte model
(test/test_cdspmv.cpp:305: nnz*(val+4) + (rows+cols)*val + (rows+1)*4) over
`kernel_ms`; `roofline.traffic` the HBM bytes per step measured by rocprofv3
(profiles/traffic.json) when committed for that plan.

Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(REPO, "prefree-public_amd")
METRIC = "fp64 SpMV GFLOP/s and achieved HBM GB/s (% of peak) on 1 MI355X"
PEAK_HBM_GBS = 8000.0
WORKLOADS = {
    1: "C1 uniform random 4096x4096, 16 nnz/row",
    2: "C2 5-point Laplacian 2048x2048",
    3: "C3 power-law n=2,000,000 (Pareto 2.1, cap 200,000)",
    4: "C4 very sparse n=20,000,000 (Poisson 2.5, banded +-4096, 10% outliers)",
    5: "C5 mixed n=1,000,000 (0.1% dense rows of 50k-500k nnz)",
}
VALUES = {
    1: "val, x ~ U[-1,1]",
    2: "val 4 on the diagonal, -1 off it; x ~ U[-1,1]",
    3: "val, x ~ U[-1,1]",
    4: "val, x ~ U[-1,1]",
    5: "val, x ~ U[-1,1]",
}
ALL_CONFIGS = [(1, "f64"), (2, "f64"), (3, "f64"), (4, "f64"), (4, "f32"), (5, "f64")]
HEADLINE = (5, "f64")
TOL = {"f64": 1e-12, "f32": 1e-5, "f16": 1e-3}
ROTATE_BYTES = 768 << 20     # rotated copies together exceed 3x the 256 MB MALL
ROTATE_MAX_COPIES = 1024


def cfg_name(cfg, dt):
    return f"C{cfg}" + ("" if dt == "f64" else f"_{dt}")


def kernel_name(info):
    """The dominant kernel of a plan's step (prefree-public_amd/csrc/prefree_kernels.hip)."""
    v = info["variant_name"]
    if info.get("hybrid"):
        return "k_long + k_rows (runs)" if info.get("long_tiles") else "k_dense + k_rows (runs)"
    if v == "adaptive":
        return "k_wave"
    if v == "prefree":
        return "k_prefree"
    if info["row_aligned"] and info.get("band_w"):
        return "k_band"
    if info["tile"] <= 32:  # FLAT 2..32: row groups of that many lanes
        return "k_vector"
    return {256: "k_flow", 4096: "k_tiles"}.get(info["tile"], "k_rows" if info["row_aligned"] else "k_flat")


def load_pkg():
    spec = importlib.util.spec_from_file_location("prefree_amd", os.path.join(PKG_DIR, "__init__.py"),
                                                  submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["prefree_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def traffic_from_profiles(key):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE), if committed."""
    path = os.path.join(REPO, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f).get(key)
        return None if t is None else int(t["hbm_bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(rp, col, val, x, seconds, nnz):
    """The OpenMP oracle timed on the host cores: 3 warm-up runs, then runs until
    `seconds` have passed and at least 10 were made.  Returns (record, y)."""
    sys.path.insert(0, REPO)
    import numpy as np
    import oracle

    threads = oracle.omp_max_threads()
    f16 = val.dtype == np.float16
    if f16:  # the fp16 values widened to fp64: the sums this library's fp16 result is rounded from
        val, x = val.astype(np.float64), x.astype(np.float64)
    y = np.zeros(len(rp) - 1, dtype=val.dtype)
    for _ in range(3):                      # warm-up (page-in, clocks)
        oracle.spmv_omp(rp, col, val, x, y=y)
    reps, t0 = 0, time.perf_counter()
    while True:
        y[:] = 0
        oracle.spmv_omp(rp, col, val, x, y=y)
        reps += 1
        el = time.perf_counter() - t0
        if (el >= seconds and reps >= 10) or reps >= 100000:
            break
    ms = el * 1e3 / reps
    m, n, vb = len(rp) - 1, len(x), val.dtype.itemsize
    bytes_eff = (nnz + m + n) * vb + nnz * 4 + (m + 1) * 4          # test/test_cdspmv.cpp:305, on the data timed
    return {"value": round(2.0 * nnz / (ms * 1e6), 3), "unit": "GFLOP/s", "cores": threads, "kind": "port",
            "ms_per_spmv": round(ms, 4), "gbps_effective": round(bytes_eff / (ms * 1e6), 1),
            "cpu_model": cpu_model(), "nproc": os.cpu_count(),
            "sample": f"full matrix, {reps} SpMVs in {el:.1f} s after 3 warm-up SpMVs (OpenMP restatement of "
                      f"spmv_serial, test/test_cdspmv.cpp:4-20, nnz-balanced row chunks, {threads} threads"
                      + (", on the fp16 values widened to fp64" if f16 else "") + ")"}, y


class Stepper:
    """Times `steps` calls of step(i) on `stream`: host clock and HIP events, eagerly
    (with 40 event-timed batches for a median) or as one captured HIP graph."""

    def __init__(self, torch, stream, use_graph):
        self.torch, self.stream, self.use_graph = torch, stream, use_graph

    def run(self, step, steps):
        torch, stream = self.torch, self.stream
        graph = None
        if self.use_graph:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for i in range(steps):
                    step(i, torch.cuda.current_stream())
            torch.cuda.synchronize()
            graph.replay()                   # untimed replay: the graph's first run
            torch.cuda.synchronize()
        n_batch = 0 if graph is not None else min(40, steps)
        bounds = [round(j * steps / n_batch) for j in range(n_batch + 1)] if n_batch else []
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        marks = ([e0] + [torch.cuda.Event(enable_timing=True) for _ in range(n_batch - 1)] + [e1]) if n_batch else []
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(stream)
        if graph is not None:
            graph.replay()
        else:
            k = 1
            for i in range(steps):
                if k < n_batch and i == bounds[k]:
                    marks[k].record(stream)
                    k += 1
                step(i, stream)
        e1.record(stream)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        host_ms = (t1 - t0) * 1e3 / steps
        ev_ms = e0.elapsed_time(e1) / steps
        median = None
        if n_batch:
            import numpy as np
            per = [marks[j].elapsed_time(marks[j + 1]) / (bounds[j + 1] - bounds[j]) for j in range(n_batch)]
            median = float(np.median(per))
        desc = (f"median of {n_batch} event-timed batches of the steps, launched one by one" if n_batch
                else "no median: the steps ran as one captured HIP graph replay")
        del graph
        return host_ms, ev_ms, median, desc


def prewarm(pf, torch):
    """One plan and call on a small matrix before anything is timed: the process's first use of the kernel
    library loads its code and sets up the device, a cost no later plan pays (it would otherwise land in the
    first configuration's plan_ms)."""
    import numpy as np

    rp, col, vals = pf.synth_csr(2, seed=1, scale_n=64, dtypes=("f64",))
    dev = torch.device("cuda:0")
    m = len(rp) - 1
    d = [torch.from_numpy(a).to(dev) for a in (rp, col, vals["f64"], np.ones(m))]
    y = torch.empty(m, dtype=torch.float64, device=dev)
    with pf.Plan(d[0], d[1], m, m, len(col), "f64", "auto") as p:
        p.execute(d[0], d[1], d[2], d[3], y)
    torch.cuda.synchronize()


def measure(pf, torch, cfg, dt, args, steps, warmup, want_cpu):
    """One configuration: every leg of the module docstring.  Returns its record."""
    import numpy as np

    dev = torch.device("cuda:0")
    vb = {"f64": 8, "f32": 4, "f16": 2}[dt]
    tdt = {"f64": torch.float64, "f32": torch.float32, "f16": torch.float16}[dt]
    legs = set(args.legs.split(","))

    rp, col, vals = pf.synth_csr(cfg, seed=args.seed, dtypes=(dt,))
    val = vals[dt]
    m = len(rp) - 1
    n = m
    nnz = len(col)
    x = pf.synth_x(cfg, n, seed=args.seed, dtypes=(dt,))[dt]
    bytes_eff = (nnz + m + n) * vb + nnz * 4 + (m + 1) * 4          # test/test_cdspmv.cpp:305
    bytes_gather = (2 * nnz + m) * vb + nnz * 4 + (m + 1) * 4       # test/test_cdspmv.cpp:306
    flops = 2.0 * nnz

    stream = torch.cuda.current_stream()
    d_rp = torch.from_numpy(rp).to(dev)
    d_col = torch.from_numpy(col).to(dev)
    d_val = torch.from_numpy(val).to(dev)
    d_x = torch.from_numpy(x).to(dev)
    d_y = torch.full((m,), float("nan"), dtype=tdt, device=dev)
    torch.cuda.synchronize()

    def make_plan(tile=None):
        p = pf.Plan(d_rp, d_col, m, n, nnz, dt, args.variant, args.tile if tile is None else tile, stream=stream)
        if args.x_windows >= 0:
            p.set_x_windows(args.x_windows)
        if args.chunk_nnz >= 0:
            p.set_chunk_nnz(args.chunk_nnz)
        if args.ladder and p.info.variant == pf.PREFREE:
            p.set_ladder(args.ladder)
        if args.hybrid == 0 and p.info.hybrid:
            p.set_hybrid(False)
        if args.x_halves >= 0 and p.info.hybrid:
            p.set_x_halves(args.x_halves)
        if args.band == 0 and p.info.band_w:
            p.set_band(False)
        elif args.band == 1 and not p.info.band_w:
            p.set_band(True)
        return p

    t_plan = time.perf_counter()
    plan = make_plan()
    t_plan = (time.perf_counter() - t_plan) * 1e3
    plan_wall, plan_gpu = plan.timing
    info = plan.info.as_dict()
    deterministic = info["variant_name"] != "prefree"   # PREFREE adds tile-boundary rows with atomics

    # Warm-up (eager), then the launch mode: a captured graph when a step is
    # launch-bound (under 20 us), otherwise launches one by one.
    w0 = torch.cuda.Event(enable_timing=True)
    w1 = torch.cuda.Event(enable_timing=True)
    w0.record(stream)
    for _ in range(max(1, warmup)):
        plan.execute(d_rp, d_col, d_val, d_x, d_y, stream=stream)
    w1.record(stream)
    torch.cuda.synchronize()
    warm_us = w0.elapsed_time(w1) * 1e3 / max(1, warmup)
    plan.check(stream=stream)
    y_ref = d_y.clone()
    use_graph = args.launch == "graph" or (args.launch == "auto" and warm_us < 20.0)
    st = Stepper(torch, stream, use_graph)

    def hot_step(i, s):
        plan.execute(d_rp, d_col, d_val, d_x, d_y, stream=s)

    d_y.fill_(float("nan"))
    host_ms, ev_ms, median, median_desc = st.run(hot_step, steps)
    plan.check(stream=stream)
    same_hot = bool(torch.equal(d_y, y_ref)) if deterministic else None
    gbs = bytes_eff / (ev_ms * 1e6)
    key = f"C{cfg}-{dt}-{info['variant_name']}-{info['tile']}" + (
        f"-r{info['run_tiles']}" if info["variant_name"] == "adaptive" else "") + (
        "-rows" if info["row_aligned"] else "") + ("-band" if info.get("band_w") else "") + (
        ("-long" if info["long_tiles"] else "-hybrid") if info["hybrid"] else "")
    traffic = traffic_from_profiles(key)
    rec = {
        "workload": WORKLOADS[cfg] + {"f64": "", "f32": " (fp32)", "f16": " (fp16)"}[dt],
        "cfg": f"C{cfg}", "dtype": dt, "rows": m, "cols": n, "nnz": nnz, "seed": args.seed,
        "values": VALUES[cfg],
        "variant": info["variant_name"], "tile": info["tile"], "tiles": info["ntiles"],
        "run_tiles": info["run_tiles"] if info["variant_name"] == "adaptive" else None,
        "row_aligned": bool(info["row_aligned"]), "x_windows": bool(info["x_windows"]),
        "xcd_chunk_nnz": info["chunk_nnz"] if info["variant_name"] == "flat" else None,
        "split_row_combine": bool(info["needs_fixup"]) and not info["hybrid"], "plan_ms": round(t_plan, 3),
        "plan_split": {"create_ms": round(plan_wall, 3), "gpu_ms": round(plan_gpu, 3),
                       "host_ms": round(plan_wall - plan_gpu, 3),
                       "what": "pf_plan_create's wall time (statistics, column check, selection, workspace, hybrid "
                               "tables), the event-timed GPU time of its kernels, and the rest (host work: "
                               "allocation, copies, synchronisation); paid once per sparsity pattern, not in "
                               "cdPre or the timed steps"},
        "ladder": info["ladder"] if info["variant_name"] == "prefree" else None,
        "hybrid": bool(info["hybrid"]), "dense_rows": info["dense_rows"] if info["hybrid"] else None,
        "long_tiles": info["long_tiles"] if info["hybrid"] and info["long_tiles"] else None,
        "x_halves": bool(info["x_halves"]) if info["hybrid"] else None,
        "band_w": info["band_w"] or None,
        "tuning_table": os.path.relpath(os.path.realpath(pf.tuning_table()), REPO) if pf.tuning_table() else None,
        "steps": steps, "warmup": warmup,
        "launch": ("one captured HIP graph of the timed steps" if use_graph else "eager launches from Python")
                  + f"; eager warm-up step {warm_us:.1f} us",
        "ms": round(host_ms, 6), "kernel_ms": round(ev_ms, 6),
        "kernel_ms_median": round(median, 6) if median is not None else None, "median_of": median_desc,
        "gflops": round(flops / (host_ms * 1e6), 3),
        "gbps_effective": round(gbs, 1), "pct_peak_hbm": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "bytes_model": {"effective": bytes_eff, "gather": bytes_gather, "source": "test/test_cdspmv.cpp:305-306"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic, "kernel": kernel_name(info),
                     "launch_ms": round(ev_ms, 6), "algorithmic_bytes": bytes_eff,
                     "traffic_gbps": round(traffic / (ev_ms * 1e6), 1) if traffic else None,
                     "traffic_key": key,
                     "note": ("step = k_rows over the runs of short rows + k_long over the long rows' tiles "
                              "+ k_long_sum (k_combine, which also adds the x halves, with x halves); "
                              "launch_ms covers them all"
                              if info["hybrid"] and info["long_tiles"] else
                              "step = k_rows over the runs of short rows + k_dense over the dense rows' x windows "
                              "+ k_dense_sum (k_combine, which also adds the x halves, with x halves); "
                              "launch_ms covers them all"
                              if info["hybrid"] else
                              "step = tile kernel + split-row combine kernel; launch_ms covers both"
                              if info["needs_fixup"] else "step = one tile-kernel launch")},
    }

    # Rotated copies of the whole working set: no step finds its matrix in the MALL.
    if "rotated" in legs:
        copies = max(2, min(ROTATE_MAX_COPIES, math.ceil(ROTATE_BYTES / bytes_eff)))
        bufs = [(d_rp, d_col, d_val, d_x, d_y)]
        for _ in range(copies - 1):
            bufs.append((d_rp.clone(), d_col.clone(), d_val.clone(), d_x.clone(),
                         torch.full((m,), float("nan"), dtype=tdt, device=dev)))
        torch.cuda.synchronize()

        def rot_step(i, s):
            b = bufs[i % copies]
            plan.execute(b[0], b[1], b[2], b[3], b[4], stream=s)

        for i in range(copies):                 # every copy once, untimed
            rot_step(i, stream)
        r_host, r_ev, r_med, _ = st.run(rot_step, max(steps, copies))
        plan.check(stream=stream)
        same_rot = all(bool(torch.equal(b[4], y_ref)) for b in bufs[1:]) if deterministic else None
        rec["rotated"] = {"ms": round(r_host, 6), "kernel_ms": round(r_ev, 6),
                          "kernel_ms_median": round(r_med, 6) if r_med is not None else None,
                          "steps": max(steps, copies), "copies": copies,
                          "working_set_bytes": copies * bytes_eff,
                          "gbps_effective": round(bytes_eff / (r_ev * 1e6), 1),
                          "frac": round(bytes_eff / (r_ev * 1e6) / PEAK_HBM_GBS, 4),
                          "y_equal_to_hot": same_rot}
        del bufs
        torch.cuda.synchronize()

    # Cold: a 1 GiB write between steps evicts L2 and MALL.
    if "cold" in legs and args.cold_steps > 0:
        flush = torch.empty(1 << 28, dtype=torch.float32, device=dev)
        cold_ms = 0.0
        c0 = torch.cuda.Event(enable_timing=True)
        c1 = torch.cuda.Event(enable_timing=True)
        for _ in range(args.cold_steps):
            flush.zero_()
            c0.record(stream)
            plan.execute(d_rp, d_col, d_val, d_x, d_y, stream=stream)
            c1.record(stream)
            c1.synchronize()
            cold_ms += c0.elapsed_time(c1)
        cold_ms /= args.cold_steps
        del flush
        rec["cold"] = {"ms": round(cold_ms, 6), "gbps_effective": round(bytes_eff / (cold_ms * 1e6), 1),
                       "frac": round(bytes_eff / (cold_ms * 1e6) / PEAK_HBM_GBS, 4),
                       "steps": args.cold_steps, "flush": "1 GiB write before each step"}

    # Rows searched inside the kernel on every call (no recorded row map): the
    # plan's own tile and, for a large row-aligned plan of 1024-nnz tiles, also
    # 2048-nnz tiles (the search's dependent round is paid once per tile, so a
    # caller who searches every call gains by planning half as many tiles); the
    # faster is reported, both are in the record.
    if "search" in legs:
        def search_time(tile):
            sp = make_plan(tile)
            sp.set_remember_rows(False)
            d_ys = torch.full((m,), float("nan"), dtype=tdt, device=dev)
            for _ in range(max(1, min(warmup, 50))):
                sp.execute(d_rp, d_col, d_val, d_x, d_ys, stream=stream)

            def search_step(i, s):
                sp.execute(d_rp, d_col, d_val, d_x, d_ys, stream=s)

            s_host, s_ev, s_med, _ = st.run(search_step, steps)
            sp.check(stream=stream)
            out = {"ms": round(s_host, 6), "kernel_ms": round(s_ev, 6),
                   "kernel_ms_median": round(s_med, 6) if s_med is not None else None,
                   "vs_recorded_rows": round(s_ev / ev_ms, 4),
                   "gbps_effective": round(bytes_eff / (s_ev * 1e6), 1),
                   "tile": sp.info.tile,
                   "y_equal_to_hot": bool(torch.equal(d_ys, y_ref)) if deterministic else None}
            sp.close()
            del d_ys
            return out

        own = search_time(None)
        if (info["variant_name"] == "flat" and info["row_aligned"] and info["tile"] == 1024 and not info.get("hybrid")
                and info["ntiles"] >= 2048):
            own = dict(own, tile_2048=search_time(2048))
        rec["search"] = dict(own, what="every call searches row_ptr for each tile's rows inside the tile kernel (a band plan: in a row-map kernel before the band kernel), with "
                                       "the plan's own tile (tile_2048: the same with 2048-nnz tiles); "
                                       "vs_recorded_rows against the hot plan's recorded-rows time")

    # The drop-in boundary (preFreeSpMV) takes host buffers: one SpMV including
    # the host->device copies of the CSR and x, planning and the copy of y back.
    if "host" in legs:
        torch.cuda.synchronize()
        h0 = time.perf_counter()
        h_rp = torch.from_numpy(rp).to(dev)
        h_col = torch.from_numpy(col).to(dev)
        h_val = torch.from_numpy(val).to(dev)
        h_x = torch.from_numpy(x).to(dev)
        h_y = torch.empty(m, dtype=tdt, device=dev)
        pf.spmv(h_rp, h_col, h_val, h_x, h_y, m, n, nnz, dt, args.variant, stream=stream)
        y_host = h_y.cpu()
        pcie_ms = (time.perf_counter() - h0) * 1e3
        del h_rp, h_col, h_val, h_x, h_y, y_host
        rec["host_buffers"] = {"ms": round(pcie_ms, 3), "gflops": round(flops / (pcie_ms * 1e6), 3),
                               "what": "one SpMV from pageable host arrays: copies in, plan, execute, copy of y out"}

    rec["y_equal_to_warmup"] = same_hot
    y_gpu = d_y.cpu().numpy()
    plan.close()
    del d_rp, d_col, d_val, d_x, d_y, y_ref
    torch.cuda.synchronize()
    torch.cuda.empty_cache()

    if want_cpu:
        import oracle
        cpu, y_cpu = cpu_baseline(rp, col, val, x, args.cpu_seconds, nnz)
        if dt == "f16":  # against the fp64 sums of the same fp16 data: one binary16 rounding per row,
            # 2^-11 relative or, for a subnormal result, 2^-25 absolute (allowed for as 2^-24)
            den = oracle.spmv_serial(rp, col, np.abs(val.astype(np.float64)), np.abs(x.astype(np.float64)))
            dev_ = np.abs(y_gpu.astype(np.float64) - y_cpu)
            zero_bad = int(np.count_nonzero((den == 0) & (y_gpu != 0)))
            nz = den > 0
            err = float((np.maximum(dev_[nz] - 2.0 ** -24, 0) / den[nz]).max()) if nz.any() else 0.0
        else:
            err, zero_bad, _ = oracle.rownorm_maxerr(rp, col, val, x, y_cpu, y_gpu)
        rec["cpu_baseline"] = cpu
        rec["parity"] = {"max_rownorm_err_vs_cpu": err, "zero_rows_bad": zero_bad, "tol": TOL[dt],
                         "ok": bool(err <= TOL[dt] and zero_bad == 0),
                         "bit_identical_rows": int(np.count_nonzero(y_gpu == y_cpu)), "rows": m}
        rec["speedup_vs_cpu"] = round(cpu["ms_per_spmv"] / host_ms, 1)
    else:
        rec["cpu_baseline"] = None
    return rec


def run_probe(pf, torch, args):
    """--probe gather: the x gathers alone (pfk_probe_gather), hot, as a ceiling for the SpMV kernels.

    Random 8-byte reads over a 16 MB and an 8 MB array (16M indices each), and each configuration's own
    column indices over its own x, with every compiled cache policy of the x loads for the random and
    C3 / C5 cases.  Events around `reps` back-to-back launches after 5 untimed ones."""
    import numpy as np

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    rng = np.random.default_rng(args.seed)
    policies = [0, 1, 2, 3, 16, 17, 18, 19]
    cases = []
    for mb in (16, 8):
        n = (mb << 20) // 8
        cases.append((f"random-{mb}MB", rng.integers(0, n, 16 << 20, dtype=np.int32), n, policies))
    for cfg in (1, 2, 3, 4, 5):
        m, n, nnz = pf.synth_dims(cfg, seed=args.seed)
        _, col, _ = pf.synth_csr(cfg, seed=args.seed, dtypes=("f64",))
        cases.append((f"C{cfg}-columns", col, n, policies if cfg in (3, 5) else [0]))
    out = {}
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    for name, idx, n, pols in cases:
        d_idx = torch.from_numpy(np.ascontiguousarray(idx)).to(dev)
        d_x = torch.rand(n, dtype=torch.float64, device=dev)
        d_out = torch.empty(4 * (-(-len(idx) // 1024)), dtype=torch.float64, device=dev)
        rec = {"gathers": int(len(idx)), "x_bytes": int(n * 8), "policy_us": {}}
        for pol in pols:
            for _ in range(5):
                pf.probe_gather("f64", d_idx, d_x, d_out, pol, stream=stream)
            reps = max(5, min(args.probe_reps, int(2e9 // max(1, len(idx)))))
            e0.record(stream)
            for _ in range(reps):
                pf.probe_gather("f64", d_idx, d_x, d_out, pol, stream=stream)
            e1.record(stream)
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / reps
            rec["policy_us"][str(pol)] = round(us, 2)
        us0 = rec["policy_us"]["0"]
        rec["us"] = us0
        rec["ggathers_per_s"] = round(len(idx) / us0 / 1e3, 2)
        out[name] = rec
        print(f"probe {name}: {rec['policy_us']}", file=sys.stderr, flush=True)
        del d_idx, d_x, d_out
    print(json.dumps({"probe": "gather", "device": pf.device_name(), "seed": args.seed,
                      "what": "x gathers alone: 16-byte non-temporal index loads + one x read per index, "
                              "cache policy bits of the x loads (1 sc0, 2 nt, 16 sc1) as keys, microseconds per launch",
                      "cases": out}), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4000,
                    help="timed steps of the headline configuration (exactly); the other configurations run "
                         "max(steps, --min-steps)")
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--min-steps", type=int, default=200)
    ap.add_argument("--config", type=int, default=0, choices=[0] + sorted(WORKLOADS),
                    help="0 = every configuration (C1-C5 fp64, C4 fp32) with C5 fp64 as the headline; "
                         "N = configuration N alone, in --dtype")
    ap.add_argument("--dtype", default="f64", choices=["f64", "f32", "f16"])
    ap.add_argument("--variant", default="auto", choices=["auto", "adaptive", "flat", "prefree"])
    ap.add_argument("--tile", type=int, default=0)
    ap.add_argument("--x-windows", type=int, default=-1, choices=[-1, 0, 1],
                    help="split-row FLAT: force the x-window tile schedule off (0) or on (1); -1 = the plan's choice")
    ap.add_argument("--chunk-nnz", type=int, default=-1,
                    help="FLAT 1024/2048: nnz per XCD chunk of tiles (0 = one chunk per XCD); -1 = the plan's choice")
    ap.add_argument("--hybrid", type=int, default=-1, choices=[-1, 0, 1],
                    help="plans with dense rows: 0 = split-row tiles instead of the hybrid path; -1 = the plan's choice")
    ap.add_argument("--band", type=int, default=-1, choices=[-1, 0, 1],
                    help="row-aligned plans with a band: force the band kernel off (0) or on (1); -1 = AUTO's rule")
    ap.add_argument("--x-halves", type=int, default=-1, choices=[-1, 0, 1],
                    help="hybrid plans: run tiles once per half of x (1) or once (0); -1 = the plan's choice")
    ap.add_argument("--ladder", type=int, default=0, choices=[0, 1, 2, 3, 4, 5],
                    help="PREFREE: the reference's reduction ladder 1..5 (0 = its active ladder, 3)")
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--legs", default="rotated,cold,search,host",
                    help="legs measured besides the hot steps (comma list of rotated, cold, search, host)")
    ap.add_argument("--cold-steps", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=3.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--launch", default="auto", choices=["auto", "graph", "eager"],
                    help="timed steps as one captured HIP graph or launched one by one from Python; auto: graph "
                         "when an eager warm-up step takes under 20 us (launch-bound), eager otherwise (a graph "
                         "adds about 0.5 us per kernel on MI355X)")
    ap.add_argument("--probe", default="", choices=["", "gather"],
                    help="gather: time the x gathers alone (random indices and each configuration's columns) "
                         "instead of the SpMV")
    ap.add_argument("--probe-reps", type=int, default=50)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="after the measurement, run a plain copy kernel over 256 MiB 3 times (known bytes, "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}); "
              "across GPUs the matrix would be split into row blocks of equal nnz, each GPU holding the x entries "
              "its columns touch; no multi-GPU figure is produced.", file=sys.stderr)
        sys.exit(2)
    for leg in args.legs.split(","):
        if leg and leg not in ("rotated", "cold", "search", "host"):
            ap.error(f"unknown leg {leg}")

    import torch

    pf = load_pkg()
    torch.cuda.set_device(torch.device("cuda:0"))
    if args.probe == "gather":
        run_probe(pf, torch, args)
        return
    if args.config:
        todo = [(args.config, args.dtype)]
        head = todo[0]
    else:
        todo, head = ALL_CONFIGS, HEADLINE
    prewarm(pf, torch)
    records = {}
    for cfg, dt in todo:
        is_head = (cfg, dt) == head
        steps = args.steps if is_head else max(args.steps, args.min_steps)
        print(f"bench: {cfg_name(cfg, dt)} ({'headline, ' if is_head else ''}{steps} steps)", file=sys.stderr,
              flush=True)
        records[cfg_name(cfg, dt)] = measure(pf, torch, cfg, dt, args, steps, args.warmup, not args.no_cpu)

    if args.copy_calibration:
        src = torch.ones(1 << 25, dtype=torch.float64, device="cuda:0")  # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)  # an elementwise kernel: reads 256 MiB, writes 256 MiB
        torch.cuda.synchronize()
        del src, dst

    h = records[cfg_name(*head)]
    result = {
        "metric": METRIC,
        "value": h["gflops"],
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": h["steps"],
        "warmup": h["warmup"],
        "ms_per_step": h["ms"],
        "ms_per_step_median": h["kernel_ms_median"],
        "median_of": h["median_of"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": h["dtype"],
        "data": (f"synthetic, seed {args.seed} (seeded generator prefree-public_amd/host/synth.cpp); "
                 f"{h['cfg']}: {h['values']}"),
        "config": {k: h[k] for k in ("workload", "cfg", "rows", "cols", "nnz", "seed", "variant", "tile", "tiles",
                                     "run_tiles", "row_aligned", "x_windows", "xcd_chunk_nnz", "split_row_combine",
                                     "hybrid", "dense_rows", "long_tiles", "x_halves", "band_w", "plan_ms",
                                     "plan_split",
                                     "tuning_table")},
        "gbps_effective": h["gbps_effective"],
        "pct_peak_hbm": h["pct_peak_hbm"],
        "bytes_model": h["bytes_model"],
        "roofline": h["roofline"],
        "rotated": h.get("rotated"),
        "cold": h.get("cold"),
        "search": h.get("search"),
        "launch": h["launch"],
        "host_buffers": h.get("host_buffers"),
        "device": pf.device_name(),
        "cpu_baseline": h["cpu_baseline"],
        "parity": h.get("parity"),
        "speedup_vs_cpu": h.get("speedup_vs_cpu"),
        "configs": records,
    }
    print(json.dumps(result), flush=True)
    print_summary(records)


def print_summary(records):
    """One short line per configuration on stderr, after the JSON line: a reader of the end of the output
    sees every configuration even when the start of the long JSON line is cut off."""
    def f(v, fmt):
        return format(v, fmt) if isinstance(v, (int, float)) else "-"

    for name, r in records.items():
        rot, cold, srch = r.get("rotated") or {}, r.get("cold") or {}, r.get("search") or {}
        roof, par, cpu = r["roofline"], r.get("parity") or {}, r.get("cpu_baseline") or {}
        ratio = roof["traffic"] / roof["algorithmic_bytes"] if roof.get("traffic") else None
        plan = r["variant"] + f"-{r['tile']}" + ("-rows" if r["row_aligned"] else "") + (
            f"-band{r['band_w']}" if r.get("band_w") else "") + (
            ("-long" if r["long_tiles"] else "-dense") + ("-halves" if r["x_halves"] else "") if r["hybrid"] else "")
        print(f"summary {name}: plan={plan} kernel_us={f(r['kernel_ms'] * 1e3, '.2f')} "
              f"frac={f(roof['frac'], '.4f')} rotated_frac={f(rot.get('frac'), '.4f')} "
              f"cold_frac={f(cold.get('frac'), '.4f')} search_x={f(srch.get('vs_recorded_rows'), '.3f')} "
              f"traffic_ratio={f(ratio, '.2f')} plan_ms={f(r['plan_ms'], '.3f')} "
              f"plan_gpu_ms={f(r['plan_split']['gpu_ms'], '.3f')} "
              f"parity={'ok' if par.get('ok') else ('FAIL' if par else '-')} "
              f"max_err={f(par.get('max_rownorm_err_vs_cpu'), '.1e')} gpu_gflops={f(r['gflops'], '.1f')} "
              f"cpu_gflops={f(cpu.get('value'), '.1f')}", file=sys.stderr, flush=True)


if __name__ == "__main__":
    main()
