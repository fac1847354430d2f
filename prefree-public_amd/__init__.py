"""prefree_amd — Python binding of the MI355X CSR SpMV library.

ctypes over the C ABI of ``lib/libprefree.so`` (include/prefree_c.h) and, for
index-level tests, ``lib/libprefree_kernels.so`` (include/prefree_kernels.h).
Device buffers are passed as raw pointers; anything with ``data_ptr()`` (a
torch tensor on the GPU) is accepted.  Streams are HIP stream handles (torch's
``stream.cuda_stream``); ``None`` is the null stream.

The binding never falls back to a CPU path: if the native libraries are not
built, importing the functions raises ``RuntimeError``.

Reference counterpart: the single entry point ``preFreeSpMV`` of
include/PreFree.h:3-5 (wang-luhan/preFree-public), kept in C++ as the drop-in
(include/PreFree.h of this repo); ``Plan`` exposes its two halves, analysis
and SpMV, on device memory.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(_HERE, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libprefree.so")
KLIB_PATH = os.path.join(LIB_DIR, "libprefree_kernels.so")

F64, F32, F16 = 0, 1, 2
AUTO, PREFREE, ADAPTIVE, FLAT = 0, 1, 2, 3
VARIANTS = {"auto": AUTO, "prefree": PREFREE, "adaptive": ADAPTIVE, "flat": FLAT}
VARIANT_NAMES = {v: k for k, v in VARIANTS.items()}
DTYPES = {"f64": F64, "f32": F32, "f16": F16}
STATUS = {0: "PF_OK", 1: "PF_ERR_INVALID", 2: "PF_ERR_ALIGN", 3: "PF_ERR_HIP", 4: "PF_ERR_NOMEM",
          5: "PF_ERR_UNSUPPORTED", 6: "PF_ERR_CSR", 7: "PF_ERR_KERNEL", 8: "PF_ERR_IO"}


class PrefreeError(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = status
        super().__init__(f"{what}: {STATUS.get(status, status)} ({_last_error()})")


class RowStats(ctypes.Structure):
    _fields_ = [("m", ctypes.c_longlong), ("nnz", ctypes.c_longlong), ("max_row_len", ctypes.c_longlong),
                ("min_row_len", ctypes.c_longlong), ("n_empty_rows", ctypes.c_longlong),
                ("n_decreasing", ctypes.c_longlong), ("row_ptr_first", ctypes.c_longlong),
                ("row_ptr_last", ctypes.c_longlong), ("n_bad_cols", ctypes.c_longlong),
                ("hist_log2", ctypes.c_longlong * 33), ("n_long_rows", ctypes.c_longlong),
                ("max_short_row_len", ctypes.c_longlong), ("guess_dev", ctypes.c_longlong),
                ("line_q1_row_ptr", ctypes.c_longlong), ("line_q3_row_ptr", ctypes.c_longlong),
                ("line_far_rows", ctypes.c_longlong)]

    def as_dict(self):
        d = {k: getattr(self, k) for k, _ in self._fields_ if k != "hist_log2"}
        d["hist_log2"] = list(self.hist_log2)
        return d


class PlanInfo(ctypes.Structure):
    _fields_ = [("variant", ctypes.c_int), ("dtype", ctypes.c_int), ("tile", ctypes.c_int),
                ("long_row_min", ctypes.c_int), ("guess_spread", ctypes.c_int), ("needs_fixup", ctypes.c_int),
                ("run_tiles", ctypes.c_int), ("keep_cached", ctypes.c_int), ("ntiles", ctypes.c_longlong),
                ("grid", ctypes.c_longlong),
                ("workspace_bytes", ctypes.c_size_t), ("row_aligned", ctypes.c_int), ("x_windows", ctypes.c_int),
                ("chunk_nnz", ctypes.c_longlong), ("ladder", ctypes.c_int), ("hybrid", ctypes.c_int),
                ("dense_rows", ctypes.c_longlong), ("x_halves", ctypes.c_int), ("long_tiles", ctypes.c_int),
                ("guess_a", ctypes.c_double), ("guess_b", ctypes.c_double), ("band_w", ctypes.c_int)]

    def as_dict(self):
        d = {k: getattr(self, k) for k, _ in self._fields_}
        d["variant_name"] = VARIANT_NAMES.get(self.variant, "?")
        return d


class TuneResult(ctypes.Structure):
    """pf_tune_result, include/prefree_c.h."""
    _fields_ = [("variant", ctypes.c_int), ("tile", ctypes.c_int), ("run_tiles", ctypes.c_int),
                ("keep_cached", ctypes.c_int), ("candidates", ctypes.c_int), ("us", ctypes.c_double),
                ("default_us", ctypes.c_double), ("chunk_nnz", ctypes.c_longlong), ("ladder", ctypes.c_int),
                ("hybrid", ctypes.c_int)]

    def as_dict(self):
        d = {k: getattr(self, k) for k, _ in self._fields_}
        d["variant_name"] = VARIANT_NAMES.get(self.variant, "?")
        return d


TUNE_PREFREE = 1
TUNE_KEEP_CACHED = 2


class SpmvArgs(ctypes.Structure):
    """pfk_spmv_args, include/prefree_kernels.h."""
    _fields_ = [("row_ptr", ctypes.c_void_p), ("col", ctypes.c_void_p), ("val", ctypes.c_void_p),
                ("x", ctypes.c_void_p), ("y", ctypes.c_void_p), ("m", ctypes.c_int), ("n", ctypes.c_int),
                ("nnz", ctypes.c_int), ("tile", ctypes.c_int), ("guess_spread", ctypes.c_int),
                ("run_tiles", ctypes.c_int), ("keep_cached", ctypes.c_int), ("ntiles", ctypes.c_longlong), ("head_slot", ctypes.c_void_p), ("tail_slot", ctypes.c_void_p),
                ("owner_row", ctypes.c_void_p), ("err_flag", ctypes.c_void_p), ("row_map", ctypes.c_void_p),
                ("map_ready", ctypes.c_int), ("row_aligned", ctypes.c_int), ("sched", ctypes.c_void_p),
                ("sched_cap", ctypes.c_longlong), ("chunk_nnz", ctypes.c_longlong), ("ladder", ctypes.c_int),
                ("head_bytes", ctypes.c_size_t), ("tail_bytes", ctypes.c_size_t), ("owner_bytes", ctypes.c_size_t),
                ("row_map_bytes", ctypes.c_size_t), ("sched_bytes", ctypes.c_size_t),
                ("dense_rows", ctypes.c_void_p), ("n_dense", ctypes.c_int), ("n_win", ctypes.c_int),
                ("n_runs", ctypes.c_int), ("runs", ctypes.c_void_p), ("run_map", ctypes.c_void_p),
                ("dense_seg", ctypes.c_void_p), ("dense_part", ctypes.c_void_p), ("runs_bytes", ctypes.c_size_t),
                ("run_map_bytes", ctypes.c_size_t), ("dense_seg_bytes", ctypes.c_size_t),
                ("dense_part_bytes", ctypes.c_size_t), ("x_halves", ctypes.c_int), ("half_part", ctypes.c_void_p),
                ("half_part_bytes", ctypes.c_size_t), ("long_mode", ctypes.c_int), ("n_long_tiles", ctypes.c_int),
                ("long_tiles", ctypes.c_void_p), ("long_deal", ctypes.c_void_p), ("long_row_tiles", ctypes.c_void_p),
                ("long_part", ctypes.c_void_p), ("long_tiles_bytes", ctypes.c_size_t),
                ("long_deal_bytes", ctypes.c_size_t), ("long_row_tiles_bytes", ctypes.c_size_t),
                ("long_part_bytes", ctypes.c_size_t), ("ovf_cap", ctypes.c_int),
                ("aux_stream", ctypes.c_void_p), ("ev_fork", ctypes.c_void_p), ("ev_join", ctypes.c_void_p),
                ("guess_a", ctypes.c_double), ("guess_b", ctypes.c_double),
                ("row_apart", ctypes.c_void_p), ("row_apart_bytes", ctypes.c_size_t), ("band_w", ctypes.c_int)]


_lib = None
_klib = None
_vp = ctypes.c_void_p
_i = ctypes.c_int
_ll = ctypes.c_longlong


def _sig(f, args, res=ctypes.c_int):
    f.argtypes = args
    f.restype = res


def lib() -> ctypes.CDLL:
    """The C ABI library; raises if it is not built (no fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"native library {LIB_PATH} is missing: run __graft_entry__.build() "
                               "(make -C prefree-public_amd)")
        # One HIP runtime per process: the library needs libamdhip64.so.7, which torch's own HIP libraries
        # also provide under that name.  Loaded after torch, the library binds to torch's runtime; loaded
        # first, it brings in the system one, torch then loads its own copy beside it (its libraries ask for
        # the unversioned name), and whichever of the two starts second finds no device.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = ctypes.CDLL(LIB_PATH)
        _sig(L.pf_version, [])
        _sig(L.pf_status_string, [_i], ctypes.c_char_p)
        _sig(L.pf_last_error, [], ctypes.c_char_p)
        _sig(L.pf_row_stats_compute, [_vp, _vp, _i, _i, _ll, ctypes.POINTER(RowStats), _vp])
        _sig(L.pf_select, [ctypes.POINTER(RowStats), _i, _i, ctypes.POINTER(PlanInfo)])
        _sig(L.pf_plan_create, [ctypes.POINTER(_vp), _vp, _vp, _i, _i, _i, _i, _i, _vp])
        _sig(L.pf_plan_create_tuned, [ctypes.POINTER(_vp), _vp, _vp, _i, _i, _i, _i, _i, _i, _vp])
        _sig(L.pf_plan_get_info, [_vp, ctypes.POINTER(PlanInfo)])
        _sig(L.pf_plan_get_timing, [_vp, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)])
        _sig(L.pf_plan_set_band, [_vp, _i])
        _sig(L.pf_plan_set_run_tiles, [_vp, _i])
        _sig(L.pf_plan_set_keep_cached, [_vp, _i])
        _sig(L.pf_plan_set_row_aligned, [_vp, _i])
        _sig(L.pf_plan_set_x_windows, [_vp, _i])
        _sig(L.pf_plan_set_chunk_nnz, [_vp, _ll])
        _sig(L.pf_plan_set_remember_rows, [_vp, _i])
        _sig(L.pf_plan_set_ladder, [_vp, _i])
        _sig(L.pf_plan_set_hybrid, [_vp, _i])
        _sig(L.pf_plan_set_x_halves, [_vp, _i])
        _sig(L.pf_plan_autotune, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, ctypes.POINTER(TuneResult)])
        _sig(L.pf_set_tuning_table, [ctypes.c_char_p])
        _sig(L.pf_tuning_table, [], ctypes.c_char_p)
        _sig(L.pf_plan_get_stats, [_vp, ctypes.POINTER(RowStats)])
        _sig(L.pf_plan_execute, [_vp, _vp, _vp, _vp, _vp, _vp, _vp])
        _sig(L.pf_plan_check, [_vp, _vp])
        _sig(L.pf_plan_destroy, [_vp])
        _sig(L.pf_spmv, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp])
        _sig(L.pf_synth_dims, [_i, ctypes.c_uint64, _i, ctypes.POINTER(_i), ctypes.POINTER(_i),
                               ctypes.POINTER(_ll)])
        _sig(L.pf_synth_csr, [_i, ctypes.c_uint64, _i, _i, _vp, _vp, _vp, _vp])
        _pi = ctypes.POINTER(ctypes.c_int)
        _sig(L.pf_mtx_read, [ctypes.c_char_p, _pi, _pi, _pi, _pi, ctypes.POINTER(_pi), ctypes.POINTER(_pi),
                             ctypes.POINTER(ctypes.POINTER(ctypes.c_double))])
        L.pf_mtx_last_error.restype = ctypes.c_char_p
        L.pf_mtx_last_error.argtypes = []
        L.pf_host_free.restype = None
        L.pf_host_free.argtypes = [_vp]
        _sig(L.pf_synth_x, [_i, ctypes.c_uint64, _i, _i, _vp, _vp])
        _sig(L.pf_device_malloc, [ctypes.POINTER(_vp), ctypes.c_size_t])
        _sig(L.pf_device_free, [_vp])
        _sig(L.pf_memcpy_h2d, [_vp, _vp, ctypes.c_size_t, _vp])
        _sig(L.pf_memcpy_d2h, [_vp, _vp, ctypes.c_size_t, _vp])
        _sig(L.pf_stream_synchronize, [_vp])
        _lib = L
    return _lib


def klib() -> ctypes.CDLL:
    """The thin HIP layer (for the index-level debug entry points)."""
    global _klib
    if _klib is None:
        lib()
        K = ctypes.CDLL(KLIB_PATH)
        _sig(K.pfk_debug_tile_desc, [_i, _i, ctypes.POINTER(SpmvArgs), _vp, _vp])
        _sig(K.pfk_adaptive_owners, [_i, ctypes.POINTER(SpmvArgs), _vp])
        _sig(K.pfk_spmv_flat, [_i, ctypes.POINTER(SpmvArgs), _vp])
        _sig(K.pfk_spmv_adaptive, [_i, ctypes.POINTER(SpmvArgs), _vp])
        _sig(K.pfk_spmv_fixup, [_i, _i, ctypes.POINTER(SpmvArgs), _vp])
        _sig(K.pfk_spmv_prefree, [_i, ctypes.POINTER(SpmvArgs), _vp])
        _sig(K.pfk_debug_prefree_rows, [_vp, _i, _i, _i, _vp, _vp])
        _sig(K.pfk_adaptive_long_row_min, [_i, _i])
        _sig(K.pfk_supported_tiles, [_i, _i, ctypes.POINTER(_i), _i])
        _sig(K.pfk_flat_grid, [ctypes.c_longlong, _i, ctypes.c_longlong], ctypes.c_longlong)
        _sig(K.pfk_device_name, [ctypes.c_char_p, _i])
        _sig(K.pfk_probe_gather, [_i, _vp, _ll, _vp, _ll, _vp, _ll, _i, _vp])
        _sig(K.pfk_band_stats, [_vp, _vp, _i, _vp, _vp])
        _sig(K.pfk_row_map, [ctypes.POINTER(SpmvArgs), _vp])
        _sig(K.pfk_last_error, [], ctypes.c_char_p)
        _klib = K
    return _klib


def _last_error() -> str:
    try:
        return (lib().pf_last_error() or b"").decode()
    except Exception:  # pragma: no cover - the library itself failed to load
        return ""


def _check(status: int, what: str):
    if status != 0:
        detail = lib().pf_last_error().decode(errors="replace")
        raise PrefreeError(status, f"{what}: {detail}" if detail else what)


def _p(obj):
    """Raw device pointer of a torch tensor / int / None."""
    if obj is None:
        return None
    if isinstance(obj, int):
        return obj
    return obj.data_ptr()


def _s(stream):
    if stream is None:
        return None
    return stream if isinstance(stream, int) else stream.cuda_stream


def dtype_code(d) -> int:
    if isinstance(d, int):
        return d
    if d in DTYPES:
        return DTYPES[d]
    name = getattr(d, "name", None) or str(d)
    if "float64" in name or name == "double":
        return F64
    if "float32" in name or name == "float":
        return F32
    if "float16" in name or name == "half":
        return F16
    raise ValueError(f"unsupported dtype {d}")


def variant_code(v) -> int:
    return v if isinstance(v, int) else VARIANTS[v]


# ---- analysis and execution -------------------------------------------------

def row_stats(row_ptr, col, m, n, nnz, stream=None) -> RowStats:
    s = RowStats()
    _check(lib().pf_row_stats_compute(_p(row_ptr), _p(col), m, n, nnz, ctypes.byref(s), _s(stream)),
           "pf_row_stats_compute")
    return s


def select(stats: RowStats, dtype="f64", variant="auto") -> PlanInfo:
    info = PlanInfo()
    _check(lib().pf_select(ctypes.byref(stats), dtype_code(dtype), variant_code(variant), ctypes.byref(info)),
           "pf_select")
    return info


class Plan:
    """Analysis of one CSR structure (pf_plan_create); execute() computes y = A·x."""

    def __init__(self, row_ptr, col, m, n, nnz, dtype="f64", variant="auto", tile=0, stream=None):
        h = ctypes.c_void_p()
        _check(lib().pf_plan_create_tuned(ctypes.byref(h), _p(row_ptr), _p(col), int(m), int(n), int(nnz),
                                          dtype_code(dtype), variant_code(variant), int(tile), _s(stream)),
               "pf_plan_create")
        self._h = h
        self.m, self.n, self.nnz = int(m), int(n), int(nnz)

    @property
    def info(self) -> PlanInfo:
        i = PlanInfo()
        _check(lib().pf_plan_get_info(self._h, ctypes.byref(i)), "pf_plan_get_info")
        return i

    @property
    def timing(self):
        """(plan_ms, plan_gpu_ms): wall time of the plan's creation and the GPU time of its kernels."""
        a, b = ctypes.c_double(), ctypes.c_double()
        _check(lib().pf_plan_get_timing(self._h, ctypes.byref(a), ctypes.byref(b)), "pf_plan_get_timing")
        return a.value, b.value

    @property
    def stats(self) -> RowStats:
        s = RowStats()
        _check(lib().pf_plan_get_stats(self._h, ctypes.byref(s)), "pf_plan_get_stats")
        return s

    def set_run_tiles(self, run_tiles):
        _check(lib().pf_plan_set_run_tiles(self._h, int(run_tiles)), "pf_plan_set_run_tiles")

    def autotune(self, row_ptr, col, val, x, y, reps=20, flags=0, stream=None):
        """pf_plan_autotune: time the compiled configurations on this matrix, keep the fastest."""
        r = TuneResult()
        _check(lib().pf_plan_autotune(self._h, _p(row_ptr), _p(col), _p(val), _p(x), _p(y), int(reps), int(flags),
                                      _s(stream), ctypes.byref(r)), "pf_plan_autotune")
        return r.as_dict()

    def set_keep_cached(self, keep_cached):
        _check(lib().pf_plan_set_keep_cached(self._h, int(bool(keep_cached))), "pf_plan_set_keep_cached")

    def set_row_aligned(self, row_aligned):
        _check(lib().pf_plan_set_row_aligned(self._h, int(bool(row_aligned))), "pf_plan_set_row_aligned")

    def set_x_windows(self, x_windows):
        _check(lib().pf_plan_set_x_windows(self._h, int(bool(x_windows))), "pf_plan_set_x_windows")

    def set_chunk_nnz(self, chunk_nnz):
        _check(lib().pf_plan_set_chunk_nnz(self._h, int(chunk_nnz)), "pf_plan_set_chunk_nnz")

    def set_ladder(self, ladder):
        """pf_plan_set_ladder: PREFREE reduction ladder 1..5 (the reference tuner's code)."""
        _check(lib().pf_plan_set_ladder(self._h, int(ladder)), "pf_plan_set_ladder")

    def set_band(self, band):
        """pf_plan_set_band: the band kernel on (True) or off (False) for calls after the first."""
        _check(lib().pf_plan_set_band(self._h, int(bool(band))), "pf_plan_set_band")

    def set_hybrid(self, hybrid):
        """pf_plan_set_hybrid: switch a hybrid plan to split-row tiles (False) and back (True)."""
        _check(lib().pf_plan_set_hybrid(self._h, int(bool(hybrid))), "pf_plan_set_hybrid")

    def set_x_halves(self, x_halves):
        """pf_plan_set_x_halves: hybrid plans' run tiles once per half of x (True) or once (False)."""
        _check(lib().pf_plan_set_x_halves(self._h, int(bool(x_halves))), "pf_plan_set_x_halves")

    def set_remember_rows(self, remember):
        """pf_plan_set_remember_rows: False = every call searches row_ptr (no recorded row map)."""
        _check(lib().pf_plan_set_remember_rows(self._h, int(bool(remember))), "pf_plan_set_remember_rows")

    def execute(self, row_ptr, col, val, x, y, stream=None):
        _check(lib().pf_plan_execute(self._h, _p(row_ptr), _p(col), _p(val), _p(x), _p(y), _s(stream)),
               "pf_plan_execute")

    def check(self, stream=None):
        _check(lib().pf_plan_check(self._h, _s(stream)), "pf_plan_check")

    def close(self):
        if getattr(self, "_h", None):
            lib().pf_plan_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def spmv(row_ptr, col, val, x, y, m, n, nnz, dtype="f64", variant="auto", stream=None):
    """One-shot y = A·x (plan, execute, synchronise, destroy)."""
    _check(lib().pf_spmv(_p(row_ptr), _p(col), _p(val), _p(x), _p(y), int(m), int(n), int(nnz),
                         dtype_code(dtype), variant_code(variant), _s(stream)), "pf_spmv")


def tile_descriptors(row_ptr, m, nnz, tile, merged, out, err_flag, guess_spread=0, run_tiles=0, stream=None,
                     row_aligned=False, chunk_nnz=0, guess_a=0.0, guess_b=0.0):
    """pfk_debug_tile_desc: per-tile descriptors of ADAPTIVE (merged) / FLAT (split or row-aligned
    tiles, dealt to the XCDs in chunks of chunk_nnz) into `out` (int32[8*ntiles])."""
    total = nnz + m if merged else nnz
    ntiles = max(1, -(-total // tile))
    a = SpmvArgs(row_ptr=_p(row_ptr), m=m, n=m, nnz=nnz, tile=tile, guess_spread=guess_spread,
                 run_tiles=run_tiles, ntiles=ntiles, err_flag=_p(err_flag), row_aligned=int(bool(row_aligned)),
                 chunk_nnz=int(chunk_nnz), guess_a=float(guess_a), guess_b=float(guess_b))
    _check(klib().pfk_debug_tile_desc(F64, int(bool(merged)), ctypes.byref(a), _p(out), _s(stream)),
           "pfk_debug_tile_desc")
    return ntiles


def adaptive_owners(row_ptr, m, nnz, tile, out, err_flag, dtype="f64", guess_spread=0, run_tiles=0, stream=None):
    """pfk_adaptive_owners: split-row owner of every ADAPTIVE tile into `out` (int32[ntiles])."""
    ntiles = max(1, -(-(nnz + m) // tile))
    a = SpmvArgs(row_ptr=_p(row_ptr), m=m, n=m, nnz=nnz, tile=tile, guess_spread=guess_spread,
                 run_tiles=run_tiles, ntiles=ntiles, owner_row=_p(out), err_flag=_p(err_flag),
                 owner_bytes=int(out.numel()) * 4)
    _check(klib().pfk_adaptive_owners(dtype_code(dtype), ctypes.byref(a), _s(stream)), "pfk_adaptive_owners")
    return ntiles


def prefree_rows(row_ptr, m, nnz, tile, out, stream=None):
    """pfk_debug_prefree_rows: in-kernel first row of every tile (ntiles+1 entries, last = m)."""
    _check(klib().pfk_debug_prefree_rows(_p(row_ptr), m, nnz, tile, _p(out), _s(stream)),
           "pfk_debug_prefree_rows")


def band_stats(row_ptr, col, m, out, stream=None):
    """pfk_band_stats: over every BAND_SAMPLE-th block of 256 rows, out[i] = the nnz with |col - row| <= 64 << i
    (i < BAND_WIDTHS), out[BAND_WIDTHS] = the sampled nnz; `out` int64[BAND_WIDTHS + 1]."""
    _check(klib().pfk_band_stats(_p(row_ptr), _p(col), int(m), _p(out), _s(stream)), "pfk_band_stats")


BAND_WIDTHS = 9   # PFK_BAND_WIDTHS
BAND_SAMPLE = 16  # PFK_BAND_SAMPLE


def adaptive_long_row_min(dtype, tile) -> int:
    return int(klib().pfk_adaptive_long_row_min(dtype_code(dtype), int(tile)))


def supported_tiles(variant, dtype):
    buf = (ctypes.c_int * 16)()
    n = min(16, klib().pfk_supported_tiles(variant_code(variant), dtype_code(dtype), buf, 16))
    return [buf[i] for i in range(n)]


def probe_gather(dtype, idx, x, out, policy=0, stream=None):
    """pfk_probe_gather: the x gathers of an SpMV alone (measurement only); `out` holds
    4 * ceil(len(idx) / 1024) values of dtype."""
    _check(klib().pfk_probe_gather(dtype_code(dtype), _p(idx), int(idx.numel()), _p(x), int(x.numel()), _p(out),
                                   int(out.numel()), int(policy), _s(stream)), "pfk_probe_gather")


def device_name() -> str:
    buf = ctypes.create_string_buffer(256)
    _check(klib().pfk_device_name(buf, 256), "pfk_device_name")
    return buf.value.decode()


# ---- synthetic matrices ------------------------------------------------------

CONFIGS = {1: "C1 uniform 4096^2 16/row", 2: "C2 5-point Laplacian 2048^2", 3: "C3 power-law n=2M",
           4: "C4 very sparse n=20M", 5: "C5 mixed dense rows n=1M"}


def synth_dims(cfg, seed=1, scale_n=0):
    m, n, nnz = ctypes.c_int(), ctypes.c_int(), ctypes.c_longlong()
    _check(lib().pf_synth_dims(int(cfg), int(seed), int(scale_n), ctypes.byref(m), ctypes.byref(n),
                               ctypes.byref(nnz)), "pf_synth_dims")
    return m.value, n.value, nnz.value


def set_tuning_table(path):
    """pf_set_tuning_table: the table PF_AUTO consults (None clears it)."""
    _check(lib().pf_set_tuning_table(None if path is None else os.fsencode(path)), "pf_set_tuning_table")


def tuning_table():
    """pf_tuning_table: path of the table PF_AUTO consults ('' when none)."""
    return os.fsdecode(lib().pf_tuning_table() or b"")


def mtx_read(path):
    """pf_mtx_read: a Matrix Market file as (row_ptr, col, val, m, n, is_symmetric), numpy arrays."""
    import numpy as np
    L = lib()
    m, n, nnz, sym = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    rp = ctypes.POINTER(ctypes.c_int)()
    col = ctypes.POINTER(ctypes.c_int)()
    val = ctypes.POINTER(ctypes.c_double)()
    st = L.pf_mtx_read(os.fsencode(path), ctypes.byref(m), ctypes.byref(n), ctypes.byref(nnz), ctypes.byref(sym),
                       ctypes.byref(rp), ctypes.byref(col), ctypes.byref(val))
    if st != 0:
        raise PrefreeError(st, f"pf_mtx_read: {L.pf_mtx_last_error().decode()}")
    try:
        r = np.ctypeslib.as_array(rp, shape=(m.value + 1,)).copy()
        c = np.ctypeslib.as_array(col, shape=(max(nnz.value, 1),))[:nnz.value].copy()
        v = np.ctypeslib.as_array(val, shape=(max(nnz.value, 1),))[:nnz.value].copy()
    finally:
        for ptr in (rp, col, val):
            L.pf_host_free(ctypes.cast(ptr, ctypes.c_void_p))
    return r, c, v, m.value, n.value, bool(sym.value)


def synth_csr(cfg, seed=1, scale_n=0, vals=0, dtypes=("f64",), out=None):
    """(row_ptr, col, {dtype: val}) of configuration `cfg` as numpy arrays.

    `out` may supply preallocated arrays (dict with keys row_ptr, col, f64, f32),
    e.g. pinned host memory.  "f16" values are the f64 draws rounded to the
    nearest IEEE binary16 (ties to even)."""
    m, n, nnz = synth_dims(cfg, seed, scale_n)
    out = dict(out or {})
    rp = out.get("row_ptr")
    rp = np.empty(m + 1, dtype=np.int32) if rp is None else rp
    col = out.get("col")
    col = np.empty(nnz, dtype=np.int32) if col is None else col
    vals_out = {}
    gen = [d for d in dtypes if d != "f16"] + (["f64"] if "f16" in dtypes and "f64" not in dtypes else [])
    for d in gen:
        a = out.get(d)
        vals_out[d] = np.empty(nnz, dtype=np.float64 if d == "f64" else np.float32) if a is None else a
    _check(lib().pf_synth_csr(int(cfg), int(seed), int(scale_n), int(vals), rp.ctypes.data, col.ctypes.data,
                              vals_out["f64"].ctypes.data if "f64" in vals_out else None,
                              vals_out["f32"].ctypes.data if "f32" in vals_out else None), "pf_synth_csr")
    if "f16" in dtypes:
        vals_out["f16"] = vals_out["f64"].astype(np.float16)
        if "f64" not in dtypes:
            del vals_out["f64"]
    return rp, col, vals_out


def synth_x(cfg, n, seed=1, vals=0, dtypes=("f64",)):
    gen = [d for d in dtypes if d != "f16"] + (["f64"] if "f16" in dtypes and "f64" not in dtypes else [])
    xs = {d: np.empty(n, dtype=np.float64 if d == "f64" else np.float32) for d in gen}
    _check(lib().pf_synth_x(int(cfg), int(seed), int(n), int(vals),
                            xs["f64"].ctypes.data if "f64" in xs else None,
                            xs["f32"].ctypes.data if "f32" in xs else None), "pf_synth_x")
    if "f16" in dtypes:
        xs["f16"] = xs["f64"].astype(np.float16)
        if "f64" not in dtypes:
            del xs["f64"]
    return xs


def version() -> int:
    return int(lib().pf_version())
