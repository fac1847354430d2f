"""CPU oracle for the CSR SpMV hot path — TEST INFRASTRUCTURE ONLY.

ctypes wrappers over ``oracle/liboracle.so`` (built from ``oracle/oracle.c`` by
``oracle/Makefile``).  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker or the CPU baseline; the product never does.

Each wrapper names the reference file:line its C function restates
(wang-luhan/preFree-public).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_dp = ctypes.POINTER(ctypes.c_double)
_fp = ctypes.POINTER(ctypes.c_float)
_ip = ctypes.POINTER(ctypes.c_int)
_llp = ctypes.POINTER(ctypes.c_longlong)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"{_LIB_PATH} is missing: run `make -C oracle` (or __graft_entry__.build())")
        L = ctypes.CDLL(_LIB_PATH)
        for name, vp in (("f64", _dp), ("f32", _fp)):
            getattr(L, f"oracle_spmv_serial_{name}").argtypes = [vp, _ip, _ip, vp, vp, ctypes.c_int]
            getattr(L, f"oracle_spmv_omp_{name}").argtypes = [vp, _ip, _ip, vp, vp, ctypes.c_int, ctypes.c_int]
            f = getattr(L, f"oracle_rownorm_maxerr_{name}")
            f.argtypes = [vp, _ip, _ip, vp, vp, vp, ctypes.c_int, _llp, _ip]
            f.restype = ctypes.c_double
        L.oracle_omp_max_threads.restype = ctypes.c_int
        L.oracle_pre_start_row.argtypes = [_ip, ctypes.c_int, ctypes.c_int, _ip, ctypes.c_int]
        L.oracle_tile_row_range.argtypes = [_ip, ctypes.c_int, ctypes.c_int, _ip, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_int, _ip, _ip]
        L.oracle_prefree_sim_f64.argtypes = [_dp, _ip, _ip, _dp, _dp, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                             ctypes.c_int]
        L.oracle_prefree_sim_code_f64.argtypes = [_dp, _ip, _ip, _dp, _dp] + [ctypes.c_int] * 6 + [_ip, _ip]
        L.oracle_prefree_sim_code_f64.restype = ctypes.c_int
        L.oracle_prefree_vector_size.argtypes = [ctypes.c_int]
        L.oracle_prefree_vector_size.restype = ctypes.c_int
        L.oracle_eqcheck_f64.argtypes = [_dp, _dp, ctypes.c_int, ctypes.c_double]
        L.oracle_eqcheck_f64.restype = ctypes.c_longlong
        for f in (L.oracle_bytes_effective, L.oracle_bytes_gather):
            f.argtypes = [ctypes.c_longlong, ctypes.c_longlong, ctypes.c_longlong, ctypes.c_int]
            f.restype = ctypes.c_longlong
        L.oracle_initvec_f64.argtypes = [_dp, ctypes.c_longlong]
        L.oracle_initvec_f32.argtypes = [_fp, ctypes.c_longlong]
        _lib = L
    return _lib


def _ptr(a: np.ndarray, ctype):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def _vtype(a: np.ndarray):
    if a.dtype == np.float64:
        return "f64", ctypes.c_double
    if a.dtype == np.float32:
        return "f32", ctypes.c_float
    raise TypeError(f"unsupported value dtype {a.dtype}")


def _check_csr(row_ptr, col):
    assert row_ptr.dtype == np.int32 and col.dtype == np.int32


def spmv_serial(row_ptr, col, val, x, y=None):
    """spmv_serial, test/test_cdspmv.cpp:4-20.  Returns y + A·x (y defaults to 0)."""
    _check_csr(row_ptr, col)
    name, ct = _vtype(val)
    m = len(row_ptr) - 1
    y = np.zeros(m, dtype=val.dtype) if y is None else np.array(y, dtype=val.dtype, copy=True)
    getattr(lib(), f"oracle_spmv_serial_{name}")(_ptr(val, ct), _ptr(row_ptr, ctypes.c_int),
                                                 _ptr(col, ctypes.c_int), _ptr(x, ct), _ptr(y, ct), m)
    return y


def spmv_omp(row_ptr, col, val, x, nthreads=0, y=None):
    """Row-parallel spmv_serial with nnz-balanced chunks (bit-identical to the serial one)."""
    _check_csr(row_ptr, col)
    name, ct = _vtype(val)
    m = len(row_ptr) - 1
    y = np.zeros(m, dtype=val.dtype) if y is None else y
    getattr(lib(), f"oracle_spmv_omp_{name}")(_ptr(val, ct), _ptr(row_ptr, ctypes.c_int),
                                              _ptr(col, ctypes.c_int), _ptr(x, ct), _ptr(y, ct), m, int(nthreads))
    return y


def omp_max_threads() -> int:
    return int(lib().oracle_omp_max_threads())


def pre_start_row(row_ptr, tile):
    """pre_start_rowPerTile brute force, src/spmv_kernel/preFreeSpMV.cu:3-28 (zeroed as :591-595)."""
    m = len(row_ptr) - 1
    nnz = int(row_ptr[-1])
    ntiles = (nnz + tile - 1) // tile
    out = np.empty(ntiles + 1, dtype=np.int32)
    lib().oracle_pre_start_row(_ptr(row_ptr, ctypes.c_int), m, int(tile), _ptr(out, ctypes.c_int), ntiles)
    return out


def tile_row_range(row_ptr, tile, start_row, b, faithful_sentinel=False):
    """Row range of tile b, preFreeSpMV.cu:429-438."""
    m = len(row_ptr) - 1
    s, e = ctypes.c_int(), ctypes.c_int()
    lib().oracle_tile_row_range(_ptr(row_ptr, ctypes.c_int), m, int(tile), _ptr(start_row, ctypes.c_int),
                                len(start_row) - 1, int(b), int(bool(faithful_sentinel)),
                                ctypes.byref(s), ctypes.byref(e))
    return s.value, e.value


def prefree_sim(row_ptr, col, val, x, faithful_sentinel=False, reverse_tiles=False, code=3, p_nnz=4, y=None,
                counts=False):
    """One execution of preFreeSpMV_kernel<p_nnz,128> with reduction ladder `code`
    (preFreeSpMV.cu:407-561; code 3 is the active ladder :466-483, 1/2/4/5 the
    tuner's alternatives :440-461 and :485-559) on the CPU.  y defaults to zeros
    (the reference memsets it, :644).  counts=True also returns, per row, the
    number of plain stores and of atomic adds it received."""
    _check_csr(row_ptr, col)
    assert val.dtype == np.float64
    m = len(row_ptr) - 1
    y = np.zeros(m, dtype=np.float64) if y is None else np.array(y, dtype=np.float64, copy=True)
    plain = np.zeros(max(m, 1), dtype=np.int32)
    atomics = np.zeros(max(m, 1), dtype=np.int32)
    st = lib().oracle_prefree_sim_code_f64(_ptr(val, ctypes.c_double), _ptr(row_ptr, ctypes.c_int),
                                           _ptr(col, ctypes.c_int), _ptr(x, ctypes.c_double),
                                           _ptr(y, ctypes.c_double), m, int(row_ptr[-1]), int(code), int(p_nnz),
                                           int(bool(faithful_sentinel)), int(bool(reverse_tiles)),
                                           _ptr(plain, ctypes.c_int), _ptr(atomics, ctypes.c_int))
    if st != 0:
        raise ValueError(f"unknown ladder code {code} or P_NNZ {p_nnz}")
    return (y, plain[:m], atomics[:m]) if counts else y


def prefree_vector_size(n):
    """calculate_vector_size<128>, preFreeSpMV.cu:394-405 (0 for n <= 0)."""
    return int(lib().oracle_prefree_vector_size(int(n)))


def eqcheck(ref, ours, tol=1e-8):
    """eQcheck, test/test_cdspmv.cpp:22-54: count of elements failing the legacy relative test."""
    ref = np.ascontiguousarray(ref, dtype=np.float64)
    ours = np.ascontiguousarray(ours, dtype=np.float64)
    return int(lib().oracle_eqcheck_f64(_ptr(ref, ctypes.c_double), _ptr(ours, ctypes.c_double), len(ref), tol))


def rownorm_maxerr(row_ptr, col, val, x, yref, y):
    """max_i |y_i - yref_i| / sum_j |a_ij x_j|; returns (max_err, zero_row_violations, worst_row)."""
    _check_csr(row_ptr, col)
    name, ct = _vtype(val)
    yref = np.ascontiguousarray(yref, dtype=val.dtype)
    y = np.ascontiguousarray(y, dtype=val.dtype)
    zb = ctypes.c_longlong()
    wr = ctypes.c_int()
    e = getattr(lib(), f"oracle_rownorm_maxerr_{name}")(
        _ptr(val, ct), _ptr(row_ptr, ctypes.c_int), _ptr(col, ctypes.c_int), _ptr(x, ct),
        _ptr(yref, ct), _ptr(y, ct), len(row_ptr) - 1, ctypes.byref(zb), ctypes.byref(wr))
    return float(e), int(zb.value), int(wr.value)


def bytes_effective(rows, cols, nnz, val_bytes):
    """Byte model test/test_cdspmv.cpp:305."""
    return int(lib().oracle_bytes_effective(rows, cols, nnz, val_bytes))


def bytes_gather(rows, cols, nnz, val_bytes):
    """Byte model test/test_cdspmv.cpp:306."""
    return int(lib().oracle_bytes_gather(rows, cols, nnz, val_bytes))


def initvec(n, dtype=np.float64):
    """initVec, include/common.h:126-133 (fp16: the reference's valT = half cast of (float)(i % 15))."""
    if np.dtype(dtype) == np.float16:
        return initvec(n, np.float32).astype(np.float16)
    v = np.empty(n, dtype=dtype)
    if dtype == np.float64:
        lib().oracle_initvec_f64(_ptr(v, ctypes.c_double), n)
    else:
        lib().oracle_initvec_f32(_ptr(v, ctypes.c_float), n)
    return v


# ---- fp16 (the reference's non-fp64 build: valT = half, include/common.h:43-46) ----------
#
# numpy's binary16 arithmetic converts both operands to float, operates, and
# rounds the result to the nearest binary16 (ties to even): for a product or a
# sum of two binary16 values this is the correctly rounded binary16 result.


def spmv_serial_f16(row_ptr, col, val, x):
    """spmv_serial, test/test_cdspmv.cpp:4-20, in the reference's fp16 build: the accumulator t and
    every product are binary16, each product and each addition rounded to binary16, in nnz order.
    Vectorised over rows (position k of every row at step k); returns float16[m]."""
    _check_csr(row_ptr, col)
    val = np.asarray(val, dtype=np.float16)
    x = np.asarray(x, dtype=np.float16)
    m = len(row_ptr) - 1
    lens = np.diff(row_ptr).astype(np.int64)
    t = np.zeros(m, dtype=np.float16)
    for k in range(int(lens.max()) if m else 0):
        with np.errstate(over="ignore"):
            rows = np.flatnonzero(lens > k)
            j = row_ptr[rows].astype(np.int64) + k
            prod = val[j] * x[col[j]]          # binary16 product
            t[rows] = t[rows] + prod           # binary16 sum
    return t


def spmv_f16_rounded(row_ptr, col, val, x):
    """This library's fp16 result model: exact products of the binary16 inputs, summed in fp64 in nnz
    order (spmv_serial, test/test_cdspmv.cpp:4-20, on the values widened to double), each row
    sum rounded once to binary16.  Returns float16[m]."""
    v64 = np.asarray(val, dtype=np.float16).astype(np.float64)
    x64 = np.asarray(x, dtype=np.float16).astype(np.float64)
    with np.errstate(over="ignore"):       # sums beyond 65504 round to +-inf, as intended
        return spmv_serial(row_ptr, col, v64, x64).astype(np.float16)
