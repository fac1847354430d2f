"""Writes tests/golden/c1_seed1.json: digests of the C1 (seed 1) CSR + x as the
synthetic generator makes them, and the oracle's y for U[-1,1] and for the
initVec known-answer values.  Run from the repo root after a deliberate
change to the generator or the oracle:  python tests/golden/make_golden.py
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import conftest  # noqa: E402,F401  (registers prefree_amd)
import oracle  # noqa: E402
import prefree_amd as pf  # noqa: E402


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def main():
    rp, col, v = pf.synth_csr(1, seed=1)
    x = pf.synth_x(1, 4096, seed=1)["f64"]
    y = oracle.spmv_serial(rp, col, v["f64"], x)
    kval = oracle.initvec(len(col))
    kx = oracle.initvec(4096)
    ky = oracle.spmv_serial(rp, col, kval, kx)
    out = {
        "config": "C1 uniform 4096^2, 16 distinct sorted columns per row, seed 1",
        "csr_x_sha256": sha(rp, col, v["f64"], x),
        "y_sha256": sha(y),
        "y_head_hex": [float(t).hex() for t in y[:16]],
        "kat_y_sha256": sha(ky),
        "kat_y_head": [float(t) for t in ky[:16]],
    }
    with open(os.path.join(HERE, "c1_seed1.json"), "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out, indent=1))


if __name__ == "__main__":
    main()
