"""pf_spmv_noalloc (the entry point that allocates nothing) against pf_spmv, through the C ABI.

pf_spmv_noalloc takes its statistics block and plan workspace from the
library's fixed device scratch array.  Two calls in a row, the second on a
smaller matrix, must each give exactly pf_spmv's y (same plan choice, same
kernels: bit for bit; PREFREE on known-answer values, whose sums are exact in
any order).  The scratch keeps the previous call's contents, so the second
call also checks that everything that must start cleared is cleared.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
import prefree_amd as pf
from gpu_util import DEV, NP, TORCH, dev

pytestmark = pytest.mark.gpu


def _noalloc():
    L = pf.lib()
    f = L.pf_spmv_noalloc
    f.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 5 + [ctypes.c_void_p]
    f.restype = ctypes.c_int
    return f


def _run(entry, rp, col, val, x, dtype, variant):
    m, n, nnz = len(rp) - 1, len(x), len(col)
    d_rp, d_col, d_val, d_x = dev(rp), dev(col), dev(val), dev(x)
    y = torch.full((max(m, 1),), float("nan"), dtype=TORCH[dtype], device=DEV)
    stream = torch.cuda.current_stream()
    st = entry(d_rp.data_ptr(), d_col.data_ptr(), d_val.data_ptr(), d_x.data_ptr(), y.data_ptr(), m, n, nnz,
               pf.dtype_code(dtype), pf.variant_code(variant), stream.cuda_stream)
    assert st == 0, f"status {st}: {pf.lib().pf_last_error().decode()}"
    torch.cuda.synchronize()
    return y[:m].cpu().numpy()


def _reference(rp, col, val, x, dtype, variant):
    return _run(lambda *a: pf.lib().pf_spmv(*a), rp, col, val, x, dtype, variant)


# (cfg, scale) pairs: the first matrix of each pair is the larger one.
PAIRS = [((3, 200000), (1, 0)), ((5, 20000), (2, 200)), ((4, 400000), (3, 30000))]


@pytest.mark.parametrize("dtype", ["f64", "f32"])
@pytest.mark.parametrize("variant", ["auto", "flat", "adaptive", "prefree"])
@pytest.mark.parametrize("pair", range(len(PAIRS)), ids=[f"C{a[0]}-then-C{b[0]}" for a, b in PAIRS])
def test_noalloc_matches_pf_spmv(pair, variant, dtype):
    f = _noalloc()
    kat = variant == "prefree"  # atomics on tile-boundary rows: exact sums only with integer values
    for cfg, scale in PAIRS[pair]:
        rp, col, v = pf.synth_csr(cfg, seed=5, scale_n=scale, dtypes=(dtype,))
        x = pf.synth_x(cfg, len(rp) - 1, seed=5, dtypes=(dtype,))[dtype]
        val = v[dtype]
        if kat:
            val, x = oracle.initvec(len(col), NP[dtype]), oracle.initvec(len(x), NP[dtype])
        want = _reference(rp, col, val, x, dtype, variant)
        got = _run(f, rp, col, val, x, dtype, variant)
        assert np.array_equal(got, want), f"C{cfg}/{variant}/{dtype}: {np.count_nonzero(got != want)} rows differ"
        if kat:
            assert np.array_equal(got, oracle.spmv_serial(rp, col, val, x))



def test_noalloc_two_host_threads():
    """Two host threads call pf_spmv_noalloc at once on their own streams and matrices, several times each:
    the per-device lock orders their use of the one scratch array, so every result equals pf_spmv's."""
    import threading

    f = _noalloc()
    jobs = []
    for cfg, scale in ((3, 200000), (5, 20000)):
        rp, col, v = pf.synth_csr(cfg, seed=7, scale_n=scale, dtypes=("f64",))
        x = pf.synth_x(cfg, len(rp) - 1, seed=7, dtypes=("f64",))["f64"]
        want = _reference(rp, col, v["f64"], x, "f64", "auto")
        m, n, nnz = len(rp) - 1, len(x), len(col)
        bufs = (dev(rp), dev(col), dev(v["f64"]), dev(x))
        y = torch.full((m,), float("nan"), dtype=torch.float64, device=DEV)
        jobs.append((bufs, y, m, n, nnz, want, torch.cuda.Stream()))
    torch.cuda.synchronize()
    rounds = 6
    start = threading.Barrier(len(jobs))
    failures = []

    def worker(k):
        (d_rp, d_col, d_val, d_x), y, m, n, nnz, want, s = jobs[k]
        try:
            for it in range(rounds):
                y.fill_(float("nan"))
                torch.cuda.synchronize()
                start.wait()
                st = f(d_rp.data_ptr(), d_col.data_ptr(), d_val.data_ptr(), d_x.data_ptr(), y.data_ptr(), m, n, nnz,
                       pf.dtype_code("f64"), pf.variant_code("auto"), s.cuda_stream)
                if st != 0:
                    failures.append(f"thread {k} call {it}: status {st}")
                    continue
                got = y.cpu().numpy()  # the call synchronised its stream before returning
                if not np.array_equal(got, want):
                    failures.append(f"thread {k} call {it}: {np.count_nonzero(got != want)} rows differ")
        except Exception as e:  # reported below; a thread's exception would otherwise be lost
            failures.append(f"thread {k}: {e!r}")
            start.abort()

    threads = [threading.Thread(target=worker, args=(k,)) for k in range(len(jobs))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not failures, failures
