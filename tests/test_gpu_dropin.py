"""The C++ drop-in preFreeSpMV (include/PreFree.h) against the oracle, called through its mangled symbols.

The reference harness checks preFreeSpMV's y against spmv_serial (test/test_cdspmv.cpp:311-317); here the
same call (src/spmv_kernel/preFreeSpMV.cu:563-662 restated by host/dropin.cpp: host buffers in, device
copies, plan, timed calls, one checked call, y back) is made through ctypes with host numpy arrays and its
y compared with the pinned oracle:

* initVec values (include/common.h:126-133): bit for bit (fp64, fp32 while row sums stay exact; fp16
  against the once-rounded model);
* U[-1,1] values: per-row error within 1e-12 (fp64) / 1e-5 (fp32) / 1e-3 + 2^-24 (fp16) of
  sum_j |a_ij x_j|, empty rows exactly 0;
* *cdTime > 0 and *cdPre >= 0 (both finite), y overwritten even where it held NaN.

Cases: the edge cases, C1 at its own size and C2-C5 scaled.  The drop-in exits its process on a fatal
error, as the reference's CUDA_CHECK_ERROR does, so it runs in a worker process (tests/dropin_worker.py)
and a failure reports the error it printed.
"""
import math
import os
import subprocess
import sys
import tempfile

import numpy as np
import pytest

import oracle
import prefree_amd as pf
from csr_cases import edge_cases
from gpu_util import NP, assert_parity, kat_exact_possible

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(os.path.dirname(HERE), "prefree-public_amd", "lib", "libprefree.so")


def _scaled():
    out = []
    for cfg, scale in ((1, 0), (2, 300), (3, 60000), (4, 400000), (5, 40000)):
        rp, col, _ = pf.synth_csr(cfg, seed=9, scale_n=scale, dtypes=())
        out.append((f"C{cfg}", rp, col, len(rp) - 1))
    return out


ALL = edge_cases() + _scaled()


class Worker:
    """tests/dropin_worker.py in a child process: the drop-in exits its process on a fatal error, so a
    failure here reports what it printed instead of ending the test run."""

    def __init__(self, tmp):
        self.tmp, self.proc, self.n = tmp, None, 0
        self.err_path = os.path.join(tmp, "worker.err")

    def _start(self):
        env = dict(os.environ, PREFREE_WARMUP="3", PREFREE_ITERS="10", PREFREE_PRE_ITERS="5")
        env.pop("PREFREE_TILE", None)
        self.err = open(self.err_path, "ab")
        self.proc = subprocess.Popen([sys.executable, os.path.join(HERE, "dropin_worker.py"), LIB],
                                     stdin=subprocess.PIPE, stdout=subprocess.PIPE, stderr=self.err, env=env)

    def call(self, rp, col, val, x, dtype, variant=""):
        if self.proc is None or self.proc.poll() is not None:
            self._start()
        self.n += 1
        path = os.path.join(self.tmp, f"case{self.n}.npz")
        np.savez(path, row_ptr=rp, col=col, val=val, x=x, dtype=np.array(dtype), variant=np.array(variant))
        self.proc.stdin.write((path + "\n").encode())
        self.proc.stdin.flush()
        reply = self.proc.stdout.readline().decode().strip()
        if reply != "ok":
            self.proc.wait(timeout=60)
            self.err.flush()
            with open(self.err_path, "rb") as f:
                tail = f.read()[-2000:].decode(errors="replace")
            raise AssertionError(f"drop-in process ended (status {self.proc.returncode}): {tail}")
        out = np.load(path + ".out.npz")
        return out["y"], float(out["cd_time"]), float(out["cd_pre"])

    def close(self):
        if self.proc is not None and self.proc.poll() is None:
            self.proc.stdin.close()
            self.proc.wait(timeout=60)


@pytest.fixture(scope="module")
def worker():
    with tempfile.TemporaryDirectory() as tmp:
        w = Worker(tmp)
        yield w
        w.close()


def _check_times(t, pre, m):
    assert math.isfinite(t) and math.isfinite(pre)
    assert pre >= 0.0
    if m > 0:
        assert t > 0.0


@pytest.mark.parametrize("dtype", ["f64", "f32", "f16"])
@pytest.mark.parametrize("case", range(len(ALL)), ids=[c[0] for c in ALL])
def test_dropin_kat_bit_exact(case, dtype, worker):
    name, rp, col, n = ALL[case]
    val = oracle.initvec(len(col), NP[dtype])
    x = oracle.initvec(n, NP[dtype])
    y, t, pre = worker.call(rp, col, val, x, dtype)
    _check_times(t, pre, len(rp) - 1)
    assert_parity(rp, col, val, x, y, dtype, exact=kat_exact_possible(rp, dtype), what=f"{name}/{dtype}")


@pytest.mark.parametrize("dtype", ["f64", "f32", "f16"])
@pytest.mark.parametrize("case", range(len(ALL)), ids=[c[0] for c in ALL])
def test_dropin_random_within_tolerance(case, dtype, worker):
    name, rp, col, n = ALL[case]
    rng = np.random.default_rng(100 + case)
    val = rng.uniform(-1, 1, len(col)).astype(NP[dtype])
    x = rng.uniform(-1, 1, n).astype(NP[dtype])
    y, t, pre = worker.call(rp, col, val, x, dtype)
    _check_times(t, pre, len(rp) - 1)
    assert_parity(rp, col, val, x, y, dtype, what=f"{name}/{dtype}")


@pytest.mark.parametrize("variant", ["prefree", "flat", "adaptive"])
def test_dropin_variants(variant, worker):
    """PREFREE_VARIANT selects the tiling, as the environment knob of the drop-in documents."""
    rp, col, _ = pf.synth_csr(3, seed=11, scale_n=40000, dtypes=())
    n = len(rp) - 1
    rng = np.random.default_rng(11)
    val, x = rng.uniform(-1, 1, len(col)), rng.uniform(-1, 1, n)
    y, t, pre = worker.call(rp, col, val, x, "f64", variant)
    _check_times(t, pre, n)
    assert_parity(rp, col, val, x, y, "f64", what=variant)
    kv, kx = oracle.initvec(len(col)), oracle.initvec(n)
    y, _, _ = worker.call(rp, col, kv, kx, "f64", variant)
    assert np.array_equal(y, oracle.spmv_serial(rp, col, kv, kx))
