"""Worker process of tests/test_gpu_dropin.py: runs the C++ drop-in preFreeSpMV on request.

The drop-in ends the process on a fatal error, as the reference's CUDA_CHECK_ERROR does
(include/common.h:49-58), so the tests call it in this separate process and read the error it printed
when it dies.  Protocol, one request per line on stdin: the path of an .npz file holding dtype, row_ptr,
col, val, x and variant ("" for the default); the worker writes y, cdTime and cdPre to <path>.out.npz
and prints "ok".  Usage: python dropin_worker.py <path of libprefree.so>.
"""
import ctypes
import os
import sys

import numpy as np

SYMBOLS = {  # g++ (Itanium ABI) names of the three overloads in include/PreFree.h
    "f64": "_Z11preFreeSpMVPdPiS0_S_S_iiiS_S_",
    "f32": "_Z11preFreeSpMVPfPiS0_S_S_iiiPdS1_",
    "f16": "_Z11preFreeSpMVP7pf_halfPiS1_S0_S0_iiiPdS2_",
}
NP = {"f64": np.float64, "f32": np.float32, "f16": np.float16}


def main():
    lib = ctypes.CDLL(sys.argv[1])
    fns = {}
    for dt, sym in SYMBOLS.items():
        f = getattr(lib, sym)
        f.restype = None
        f.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 3 + [ctypes.POINTER(ctypes.c_double)] * 2
        fns[dt] = f
    for line in sys.stdin:
        path = line.strip()
        if not path:
            continue
        d = np.load(path)
        dt = str(d["dtype"])
        variant = str(d["variant"])
        if variant:
            os.environ["PREFREE_VARIANT"] = variant
        else:
            os.environ.pop("PREFREE_VARIANT", None)
        rp = np.ascontiguousarray(d["row_ptr"], dtype=np.int32)
        col = np.ascontiguousarray(d["col"], dtype=np.int32)
        val = np.ascontiguousarray(d["val"], dtype=NP[dt])
        x = np.ascontiguousarray(d["x"], dtype=NP[dt])
        m = len(rp) - 1
        y = np.full(max(m, 1), np.nan, dtype=NP[dt])
        t, pre = ctypes.c_double(-1.0), ctypes.c_double(-1.0)
        fns[dt](val.ctypes.data, rp.ctypes.data, col.ctypes.data, x.ctypes.data, y.ctypes.data, m, len(x), len(col),
                ctypes.byref(t), ctypes.byref(pre))
        np.savez(path + ".out.npz", y=y[:m], cd_time=t.value, cd_pre=pre.value)
        print("ok", flush=True)


if __name__ == "__main__":
    main()
