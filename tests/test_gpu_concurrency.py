"""Plans are independent: each keeps its own workspace (row map, split-row
slots, error flag), errors are per host thread, and the tuning table is read
under a lock.  Two plans whose calls interleave on two streams, and two host
threads each driving its own plan (ctypes releases the GIL during the calls,
so the host calls overlap), must each give the oracle's y.  Streams keep the
default priority.
"""
import threading

import numpy as np
import pytest
import torch

import oracle
import prefree_amd as pf
from gpu_util import DEV, assert_parity, dev

pytestmark = pytest.mark.gpu


def matrices():
    out = []
    for cfg, scale, seed in ((2, 200, 1), (3, 20000, 2), (4, 200000, 3), (5, 20000, 4)):
        rp, col, v = pf.synth_csr(cfg, seed=seed, scale_n=scale)
        x = pf.synth_x(cfg, len(rp) - 1, seed=seed)["f64"]
        out.append((f"C{cfg}", rp, col, v["f64"], x))
    return out


def test_two_plans_interleaved_on_two_streams():
    mats = matrices()[:2]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    state = []
    for (name, rp, col, val, x), s in zip(mats, streams):
        m = len(rp) - 1
        d = (dev(rp), dev(col), dev(val), dev(x))
        y = torch.full((m,), float("nan"), dtype=torch.float64, device=DEV)
        torch.cuda.synchronize()                       # inputs and y ready before the plan's stream reads them
        plan = pf.Plan(d[0], d[1], m, m, len(col), "f64", "auto", stream=s)
        state.append((name, rp, col, val, x, d, y, plan, s))
    torch.cuda.synchronize()
    for _ in range(20):
        for name, rp, col, val, x, d, y, plan, s in state:
            plan.execute(d[0], d[1], d[2], d[3], y, stream=s)
    torch.cuda.synchronize()
    for name, rp, col, val, x, d, y, plan, s in state:
        plan.check(stream=s)
        assert_parity(rp, col, val, x, y.cpu().numpy(), "f64", what=f"interleaved {name}")
        plan.close()


def test_host_threads_each_with_a_plan():
    mats = matrices()
    results, errors = {}, []

    def worker(name, rp, col, val, x):
        try:
            s = torch.cuda.Stream()
            m = len(rp) - 1
            with torch.cuda.stream(s):
                d = (dev(rp), dev(col), dev(val), dev(x))
                y = torch.full((m,), float("nan"), dtype=torch.float64, device=DEV)
            s.synchronize()
            with pf.Plan(d[0], d[1], m, m, len(col), "f64", "auto", stream=s) as plan:
                for _ in range(30):
                    plan.execute(d[0], d[1], d[2], d[3], y, stream=s)
                s.synchronize()
                plan.check(stream=s)
            results[name] = y.cpu().numpy()
        except Exception as e:       # reported below, in the test's own thread
            errors.append(f"{name}: {e!r}")

    threads = [threading.Thread(target=worker, args=mat) for mat in mats]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not errors, errors
    assert all(not t.is_alive() for t in threads)
    for name, rp, col, val, x in mats:
        assert_parity(rp, col, val, x, results[name], "f64", what=f"thread {name}")
