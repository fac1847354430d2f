"""Plans executed inside a captured HIP graph (torch.cuda.CUDAGraph on the
plan's stream): every replay must give the eager y bit for bit, with eager
work and synchronisation between replays.  Each variant's step is kernels
only (no memset, no host synchronisation), which is what makes it capturable.
"""
import numpy as np
import pytest
import torch

import prefree_amd as pf
from gpu_util import DEV, dev

pytestmark = pytest.mark.gpu

PLANS = [("flat", 1024, 2), ("flat", 1024, 3), ("flat", 2048, 4), ("flat", 256, 2), ("flat", 4096, 3),
         ("adaptive", 512, 5), ("adaptive", 188, 2), ("flat", 2, 2), ("flat", 16, 1), ("flat", 32, 3),
         ("prefree", 1024, 3), ("prefree", 512, 2)]


@pytest.mark.parametrize("variant,tile,cfg", PLANS, ids=[f"{v}{t}-C{c}" for v, t, c in PLANS])
def test_graph_replays_match_eager(variant, tile, cfg):
    scale = {1: 20000, 2: 300, 3: 60000, 4: 400000, 5: 40000}[cfg]
    # PREFREE adds a spanning row's tile partials with atomics, in whatever order they land: initVec values
    # (small integers) make every such sum exact, so the comparison stays bit for bit.
    vals = 1 if variant == "prefree" else 0
    rp, col, v = pf.synth_csr(cfg, seed=9, scale_n=scale, vals=vals)
    m = len(rp) - 1
    x = pf.synth_x(cfg, m, seed=9, vals=vals)["f64"]
    d_rp, d_col, d_val, d_x = dev(rp), dev(col), dev(v["f64"]), dev(x)
    y = torch.full((m,), float("nan"), dtype=torch.float64, device=DEV)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        plan = pf.Plan(d_rp, d_col, m, m, len(col), "f64", variant, tile, stream=s)
        plan.execute(d_rp, d_col, d_val, d_x, y, stream=s)     # first call (FLAT records its row map)
        s.synchronize()
        eager = y.clone()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for _ in range(3):
                plan.execute(d_rp, d_col, d_val, d_x, y, stream=s)
        for rep in range(4):
            y.fill_(float("nan"))
            g.replay()
            s.synchronize()
            assert torch.equal(y, eager), f"replay {rep} differs from the eager result"
            y.fill_(0.0)                                        # eager work between replays
            plan.execute(d_rp, d_col, d_val, d_x, y, stream=s)
            s.synchronize()
            assert torch.equal(y, eager)
        plan.check(stream=s)
        plan.close()
    assert not np.isnan(eager.cpu().numpy()).any()
