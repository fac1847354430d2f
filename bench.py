#!/usr/bin/env python3
"""bench.py — CSR SpMV throughput on one MI355X.

One step = one y = A·x (pf_plan_execute) over the whole matrix, inputs already
resident in HBM.  Default workload: C2, the 5-point Laplacian on a 2048x2048
grid (n = 4,194,304, nnz = 20,963,328, fp64) — configs[1] of BASELINE.json,
the single-GPU configuration the metric is quoted on.  --config 1..5 selects
the other configurations (C4 also in fp32 with --dtype f32).

Prints ONE JSON line.  `value` is GFLOP/s (2*nnz per step) from the host clock
around exactly --steps back-to-back steps, bracketed by device
synchronisation.  `roofline.achieved` is the effective-byte model of the
reference harness (test/test_cdspmv.cpp:305: nnz*(val+4) + (rows+cols)*val +
(rows+1)*4) divided by the kernel time per step measured with HIP events on
the launch stream.  `cold` repeats the measurement with a 1 GiB write between
steps so that no part of the matrix is served from the 256 MB MALL.
`cpu_baseline` times the OpenMP restatement of the reference's spmv_serial
(oracle/, all host cores) on the same matrix.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
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


def kernel_name(info):
    """The dominant kernel of a plan's step (prefree-public_amd/csrc/prefree_kernels.hip)."""
    v = info["variant_name"]
    if v == "adaptive":
        return "k_wave"
    if v == "prefree":
        return "k_prefree"
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
            "sample": f"full matrix, {reps} SpMVs in {el:.1f} s (OpenMP restatement of spmv_serial, "
                      f"test/test_cdspmv.cpp:4-20, nnz-balanced row chunks, {threads} threads"
                      + (", on the fp16 values widened to fp64" if f16 else "") + ")"}, y


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--config", type=int, default=2, choices=sorted(WORKLOADS))
    ap.add_argument("--dtype", default="f64", choices=["f64", "f32", "f16"])
    ap.add_argument("--variant", default="auto", choices=["auto", "adaptive", "flat", "prefree"])
    ap.add_argument("--tile", type=int, default=0)
    ap.add_argument("--x-windows", type=int, default=-1, choices=[-1, 0, 1],
                    help="split-row FLAT: force the x-window tile schedule off (0) or on (1); -1 = the plan's choice")
    ap.add_argument("--chunk-nnz", type=int, default=-1,
                    help="FLAT 1024/2048: nnz per XCD chunk of tiles (0 = one chunk per XCD); -1 = the plan's choice")
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--cold-steps", type=int, default=100)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--launch", default="auto", choices=["auto", "graph", "eager"],
                    help="timed steps as one captured HIP graph or launched one by one from Python; auto: graph "
                         "when an eager warm-up step takes under 20 us (launch-bound), eager otherwise (a graph "
                         "adds about 0.5 us per kernel on MI355X)")
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

    import numpy as np
    import torch

    pf = load_pkg()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    dt = args.dtype
    vb = {"f64": 8, "f32": 4, "f16": 2}[dt]
    tdt = {"f64": torch.float64, "f32": torch.float32, "f16": torch.float16}[dt]

    rp, col, vals = pf.synth_csr(args.config, seed=args.seed, dtypes=(dt,))
    val = vals[dt]
    m = len(rp) - 1
    n = m
    nnz = len(col)
    x = pf.synth_x(args.config, n, seed=args.seed, dtypes=(dt,))[dt]

    stream = torch.cuda.current_stream()
    d_rp = torch.from_numpy(rp).to(dev)
    d_col = torch.from_numpy(col).to(dev)
    d_val = torch.from_numpy(val).to(dev)
    d_x = torch.from_numpy(x).to(dev)
    d_y = torch.full((m,), float("nan"), dtype=tdt, device=dev)
    torch.cuda.synchronize()

    t_plan = time.perf_counter()
    plan = pf.Plan(d_rp, d_col, m, n, nnz, dt, args.variant, args.tile, stream=stream)
    t_plan = (time.perf_counter() - t_plan) * 1e3
    if args.x_windows >= 0:
        plan.set_x_windows(args.x_windows)
    if args.chunk_nnz >= 0:
        plan.set_chunk_nnz(args.chunk_nnz)
    info = plan.info.as_dict()

    def step():
        plan.execute(d_rp, d_col, d_val, d_x, d_y, stream=stream)

    w0 = torch.cuda.Event(enable_timing=True)
    w1 = torch.cuda.Event(enable_timing=True)
    w0.record(stream)
    for _ in range(args.warmup):
        step()
    w1.record(stream)
    torch.cuda.synchronize()
    warm_us = w0.elapsed_time(w1) * 1e3 / max(1, args.warmup)
    plan.check(stream=stream)
    y_eager = d_y.clone()
    use_graph = args.launch == "graph" or (args.launch == "auto" and warm_us < 20.0)

    # The timed steps as one HIP graph of exactly --steps SpMV launches (the
    # plan's kernels only: no memset, no host synchronisation), so that the
    # launch-bound small configurations measure the GPU rather than the rate
    # at which Python can launch (--launch chooses; see its help).
    graph = None
    if use_graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            cs = torch.cuda.current_stream()
            for _ in range(args.steps):
                plan.execute(d_rp, d_col, d_val, d_x, d_y, stream=cs)
        torch.cuda.synchronize()
        d_y.fill_(float("nan"))
        graph.replay()                       # untimed replay, checked against the eager y below
        torch.cuda.synchronize()
        graph_same = bool(torch.equal(d_y, y_eager)) if info["variant_name"] != "prefree" else None

    # Timed region: exactly --steps steps, device-synchronised on both sides.
    # Launched one by one, the steps are also cut into batches by events on the
    # launch stream, for a median of the per-step time next to the mean.
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    n_batch = 40 if graph is None and args.steps >= 40 else 0
    bounds = [round(j * args.steps / n_batch) for j in range(n_batch + 1)] if n_batch else []
    marks = [e0] + [torch.cuda.Event(enable_timing=True) for _ in range(n_batch - 1)] + [e1] if n_batch else []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    if graph is not None:
        graph.replay()
    else:
        k = 1
        for i in range(args.steps):
            if n_batch and k < n_batch and i == bounds[k]:
                marks[k].record(stream)
                k += 1
            step()
    e1.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / args.steps
    ms_kernel = e0.elapsed_time(e1) / args.steps
    ms_median = None
    if n_batch:
        per = [marks[j].elapsed_time(marks[j + 1]) / (bounds[j + 1] - bounds[j]) for j in range(n_batch)]
        ms_median = float(np.median(per))
    plan.check(stream=stream)

    # Cold: a 1 GiB write between steps evicts the matrix from L2 and MALL.
    flush = torch.empty(1 << 28, dtype=torch.float32, device=dev)
    cold_ms = 0.0
    c0 = torch.cuda.Event(enable_timing=True)
    c1 = torch.cuda.Event(enable_timing=True)
    for _ in range(args.cold_steps):
        flush.zero_()
        c0.record(stream)
        step()
        c1.record(stream)
        c1.synchronize()
        cold_ms += c0.elapsed_time(c1)
    cold_ms /= max(1, args.cold_steps)
    del flush

    # The drop-in boundary (preFreeSpMV) takes host buffers: one SpMV including
    # the host->device copies of the CSR and x, planning and the copy of y back.
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

    if args.copy_calibration:
        src = torch.ones(1 << 25, dtype=torch.float64, device=dev)  # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)  # an elementwise kernel: reads 256 MiB, writes 256 MiB
        torch.cuda.synchronize()
        del src, dst

    y_gpu = d_y.cpu().numpy()
    bytes_eff = (nnz + m + n) * vb + nnz * 4 + (m + 1) * 4          # test/test_cdspmv.cpp:305
    bytes_gather = (2 * nnz + m) * vb + nnz * 4 + (m + 1) * 4       # test/test_cdspmv.cpp:306
    gbs = bytes_eff / (ms_kernel * 1e-3) / 1e9
    key = f"C{args.config}-{dt}-{info['variant_name']}-{info['tile']}" + (
        f"-r{info['run_tiles']}" if info["variant_name"] == "adaptive" else "") + (
        "-rows" if info["row_aligned"] else "")

    result = {
        "metric": METRIC,
        "value": round(2.0 * nnz / (ms_step * 1e6), 3),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 6),
        "ms_per_step_median": (round(ms_median, 6) if ms_median is not None else None),
        "median_of": (f"{n_batch} batches of the timed steps, HIP events on the launch stream" if n_batch
                      else "not measured: the timed steps are one graph replay"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dt,
        "data": "synthetic (seeded generator prefree-public_amd/host/synth.cpp, U[-1,1] values)",
        "config": {"workload": WORKLOADS[args.config] + {"f64": "", "f32": " (fp32)", "f16": " (fp16)"}[dt],
                   "cfg": f"C{args.config}", "rows": m, "cols": n, "nnz": nnz, "seed": args.seed,
                   "variant": info["variant_name"], "tile": info["tile"], "tiles": info["ntiles"],
                   "run_tiles": info["run_tiles"] if info["variant_name"] == "adaptive" else None,
                   "row_aligned": bool(info["row_aligned"]), "x_windows": bool(info["x_windows"]),
                   "xcd_chunk_nnz": info["chunk_nnz"] if info["variant_name"] == "flat" else None,
                   "split_row_combine": bool(info["needs_fixup"]), "plan_ms": round(t_plan, 3)},
        "gbps_effective": round(gbs, 1),
        "pct_peak_hbm": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "bytes_model": {"effective": bytes_eff, "gather": bytes_gather,
                        "source": "test/test_cdspmv.cpp:305-306"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic_from_profiles(key),
                     "kernel": kernel_name(info),
                     "launch_ms": round(ms_kernel, 6), "algorithmic_bytes": bytes_eff,
                     # the measured HBM bytes of the step kernel (profiles/traffic.json) over its time
                     "traffic_gbps": (round(traffic_from_profiles(key) / (ms_kernel * 1e6), 1)
                                      if traffic_from_profiles(key) else None),
                     "note": ("step = tile kernel + split-row combine kernel; launch_ms covers both"
                              if info["needs_fixup"] else "step = one tile-kernel launch")},
        "cold": ({"ms": round(cold_ms, 6), "gbps_effective": round(bytes_eff / (cold_ms * 1e-3) / 1e9, 1),
                  "flush": "1 GiB write before each step"} if args.cold_steps > 0 else None),
        "launch": ("one captured HIP graph of the timed steps (y checked bit for bit against an eager step: "
                   f"{'equal' if graph_same else ('n/a' if graph_same is None else 'DIFFERENT')})"
                   if graph is not None else "eager launches from Python")
                  + f"; eager warm-up step {warm_us:.1f} us",
        "host_buffers": {"ms": round(pcie_ms, 3), "gflops": round(2.0 * nnz / (pcie_ms * 1e6), 3),
                         "what": "one SpMV from pageable host arrays: copies in, plan, execute, copy of y out"},
        "device": pf.device_name(),
    }
    if not args.no_cpu:
        cpu, y_cpu = cpu_baseline(rp, col, val, x, args.cpu_seconds, nnz)
        import oracle
        if dt == "f16":  # against the fp64 sums of the same fp16 data: one binary16 rounding per row,
            # 2^-11 relative or, for a subnormal result, 2^-25 absolute (allowed for as 2^-24)
            den = oracle.spmv_serial(rp, col, np.abs(val.astype(np.float64)), np.abs(x.astype(np.float64)))
            dev_ = np.abs(y_gpu.astype(np.float64) - y_cpu)
            zero_bad = int(np.count_nonzero((den == 0) & (y_gpu != 0)))
            nz = den > 0
            err = float((np.maximum(dev_[nz] - 2.0 ** -24, 0) / den[nz]).max()) if nz.any() else 0.0
        else:
            err, zero_bad, _ = oracle.rownorm_maxerr(rp, col, val, x, y_cpu, y_gpu)
        result["cpu_baseline"] = cpu
        result["parity"] = {"max_rownorm_err_vs_cpu": err, "zero_rows_bad": zero_bad,
                            "tol": {"f64": 1e-12, "f32": 1e-5, "f16": 1e-3}[dt]}
        result["speedup_vs_cpu"] = round(cpu["ms_per_spmv"] / ms_step, 1)
    else:
        result["cpu_baseline"] = None
    plan.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
