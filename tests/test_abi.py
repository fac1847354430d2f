"""C ABI surface and host logic — CPU only (no GPU call is made).

* both libraries load and export every function their headers declare;
* the C++ drop-in preFreeSpMV keeps the reference's signature
  (include/PreFree.h:3-5 of wang-luhan/preFree-public) with C++ linkage;
* pf_select (host only) resolves variants, tiles and tile counts;
* argument validation fails before any GPU call.
"""
import ctypes
import os
import re
import subprocess

import pytest

import prefree_amd as pf

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = {
    "prefree_c.h": pf.LIB_PATH,
    "prefree_kernels.h": pf.KLIB_PATH,
}


def declared_functions(header):
    """Functions the header declares for the library to export (its static inline helpers are header-only)."""
    text = open(os.path.join(REPO, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"static inline[^{;]*\{.*?\n\}", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pfk?_[a-z0-9_]+)\s*\(", text)))


def exported(lib_path):
    out = subprocess.run(["nm", "-D", "--defined-only", lib_path], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


@pytest.mark.parametrize("header", sorted(HEADERS))
def test_every_declared_symbol_is_exported(header):
    names = declared_functions(header)
    assert len(names) > 10
    syms = exported(HEADERS[header])
    missing = [n for n in names if n not in syms]
    assert not missing, missing
    lib = ctypes.CDLL(HEADERS[header])
    for n in names:
        getattr(lib, n)


def test_dropin_cxx_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", "-C", pf.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    assert "preFreeSpMV(double*, int*, int*, double*, double*, int, int, int, double*, double*)" in out
    assert "preFreeSpMV(float*, int*, int*, float*, float*, int, int, int, double*, double*)" in out
    assert "preFreeSpMV(pf_half*, int*, int*, pf_half*, pf_half*, int, int, int, double*, double*)" in out


def test_kernel_library_targets_gfx950():
    # the offload bundle embedded in our own build names its only target
    blob = open(pf.KLIB_PATH, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob
    assert b"gfx942" not in blob and b"gfx90a" not in blob


def test_status_strings_and_version():
    L = pf.lib()
    for code in range(8):
        assert L.pf_status_string(code)
    assert L.pf_status_string(99) == b"unknown status"
    assert pf.version() == 100


def make_stats(m, nnz, max_len, empty=0):
    s = pf.RowStats()
    s.m, s.nnz, s.max_row_len, s.min_row_len, s.n_empty_rows = m, nnz, max_len, 0, empty
    s.row_ptr_last = nnz
    return s


@pytest.mark.parametrize("dev,spread", [(0, 1), (28, 1), (29, 2), (59, 2), (60, 4), (411, 16), (1981, 64),
                                        (1982, 64), (10 ** 9, 64)])
def test_guess_spread_covers_the_deviation(dev, spread):
    """The first probe round spans guess - 32 s .. guess + 31 s, and a row search's answer lies within
    guess_dev + 2 rows of the guess: s is the smallest power of two with 31 s >= guess_dev + 3, at most
    64; rows longer than 64 nnz take no interpolated round."""
    s = make_stats(1 << 20, 5 << 20, 5)
    s.guess_dev = dev
    assert pf.select(s, "f64", "flat").guess_spread == spread
    s.max_row_len = 65
    assert pf.select(s, "f64", "flat").guess_spread == 0


def test_line_guess_when_nearly_every_row_is_near_the_quartile_line():
    """Row-aligned searches centre their first round on the line through (row_ptr[m/4], m/4) and
    (row_ptr[3m/4], 3m/4) when at most m/256 rows lie over 28 rows from it (guess_a, guess_b); otherwise, or
    when the line is undefined or the rows are longer than 64 nnz, on the mean-density guess (guess_a 0)."""
    m, nnz = 1 << 20, 5 << 20
    s = make_stats(m, nnz, 5)
    s.guess_dev = 410
    s.line_q1_row_ptr, s.line_q3_row_ptr = 5 * (m // 4) - 2048, 5 * (3 * m // 4) - 2048
    s.line_far_rows = m // 256
    i = pf.select(s, "f64", "flat")
    a = (3 * m // 4 - m // 4) / (s.line_q3_row_ptr - s.line_q1_row_ptr)
    assert i.guess_a == a and i.guess_b == m // 4 - a * s.line_q1_row_ptr and i.guess_spread == 16
    s.line_far_rows = m // 256 + 1  # one row too many
    assert pf.select(s, "f64", "flat").guess_a == 0.0
    s.line_far_rows = 0
    s.line_q3_row_ptr = s.line_q1_row_ptr  # no line through two equal row_ptr values
    assert pf.select(s, "f64", "flat").guess_a == 0.0
    s.line_q3_row_ptr = 5 * (3 * m // 4) - 2048
    s.max_row_len = 65
    assert pf.select(s, "f64", "flat").guess_a == 0.0


def run_for(ntiles, resident, cap=16):
    return max(1, min(cap, -(-ntiles // resident)))


def test_select_auto_banded_is_flat():
    """C2 shape: short regular rows -> FLAT, 1024 nnz per tile (fp64) / 2048 (fp32)."""
    s = make_stats(4194304, 20963328, 5)
    s.guess_dev = 410  # C2's rows lie up to 410 rows from where the mean density puts them
    i = pf.select(s, "f64", "auto")
    assert i.variant == pf.FLAT and i.tile == 1024
    assert i.ntiles == -(-20963328 // 1024)
    assert i.row_aligned == 1 and i.needs_fixup == 0     # rows <= 256 nnz: tiles own whole rows
    # tiles go to the XCDs in chunks of 2^15 nnz (32 tiles); the grid pads each XCD to whole chunks,
    # fewer than 8 workgroups per round of chunks
    assert i.chunk_nnz == 1 << 15
    rounds = -(-(-(-i.ntiles // 8)) // 32)
    assert i.grid % 8 == 0 and i.grid >= i.ntiles and i.grid - i.ntiles < 8 * rounds
    assert i.guess_spread == 16      # 64 probes 16 rows apart cover 410 + 2 rows either side
    i32 = pf.select(s, "f32", "auto")
    assert i32.variant == pf.FLAT and i32.tile == 2048
    wide = pf.select(make_stats(4194304, 4194304 * 40, 60), "f64", "auto")   # rows up to 60 nnz: still FLAT
    assert wide.variant == pf.FLAT and wide.tile == 1024


def test_chunk_rule_boundary():
    """Chunks of 2^15 nnz from 4 nnz per row on average; below that, one chunk per XCD (the same bound
    that selects the row-aligned kernel's short-row mode)."""
    m = 1000000
    assert pf.select(make_stats(m, 4 * m - 1, 20), "f64", "flat").chunk_nnz == 0
    assert pf.select(make_stats(m, 4 * m, 20), "f64", "flat").chunk_nnz == 1 << 15
    for dt in ("f32", "f16"):
        assert pf.select(make_stats(m, 4 * m, 20), dt, "flat").chunk_nnz == 1 << 15


def test_chunk_rule_and_grid():
    """Very short rows (under 4 nnz on average, C4's shape) keep one XCD chunk of an eighth of the tiles;
    the grid then pads the tiles to a multiple of 8 only."""
    c4 = pf.select(make_stats(20000000, 50000000, 30), "f64", "auto")
    assert c4.variant == pf.FLAT and c4.row_aligned == 1 and c4.chunk_nnz == 0
    assert c4.grid % 8 == 0 and c4.grid >= c4.ntiles and c4.grid - 8 < c4.ntiles
    split = pf.select(make_stats(2000000, 16000000, 200000), "f64", "flat")
    assert split.row_aligned == 0 and split.chunk_nnz == 1 << 15
    assert pf.select(make_stats(2000000, 16000000, 200000), "f64", "prefree").chunk_nnz == 0
    K = pf.klib()
    for ntiles in (1, 7, 8, 9, 255, 20464, 24414):
        for tile in (1024, 2048):
            for chunk in (0, 1, tile, 1 << 15, 1 << 40):
                grid = K.pfk_flat_grid(ntiles, tile, chunk)
                g = -(-ntiles // 8)
                per = g if chunk == 0 else max(1, chunk // tile)
                rounds = -(-g // per)
                assert grid % 8 == 0 and ntiles <= grid < ntiles + 8 * rounds, (ntiles, tile, chunk, grid)


def _lanes(m, nnz, max_len):
    """The row-group lanes rule restated: at most one pass for the longest row; at least the power of two
    nearest half the mean row, or the most lanes (up to 4x the mean row or a quarter of the longest) that
    fit the chip's 2^19 resident lanes; 2..32."""
    lat = min(32, max(2, 1 << (max_len - 1).bit_length()))
    thr = 2
    while thr < 32 and nnz / m / 2 >= thr * 2 ** 0.5:
        thr *= 2
    fill = 2
    while fill < 32 and 2 * fill * m <= 1 << 19 and 2 * fill <= max(4 * nnz / m, max_len / 4):
        fill *= 2
    return min(lat, max(thr, fill))


def test_row_group_lanes_properties():
    """Over random shapes inside AUTO's row-group bounds: the lanes are a power of two in 2..32, never more than
    one pass of the longest row needs (beyond 2), at least the power of two nearest half the mean row (up to
    that bound), and the plan reports one workgroup per 256 lanes."""
    import math
    import random
    rnd = random.Random(5)
    for _ in range(400):
        m = rnd.randint(1, 1 << 18)
        mean = rnd.uniform(0.05, 200.0)
        mx = rnd.randint(max(1, int(mean)), 256)
        nnz = min(int(mean * m), mx * m)
        i = pf.select(make_stats(m, nnz, mx), "f32", "auto")
        if nnz * 8 > 256 << 20:
            assert i.tile >= 1024, (m, nnz, mx)
            continue
        L = i.tile
        assert i.variant == pf.FLAT and L in (2, 4, 8, 16, 32), (m, nnz, mx, L)
        lat = min(32, max(2, 1 << (mx - 1).bit_length()))
        assert L <= lat, (m, nnz, mx, L)
        h = nnz / m / 2
        thr = 2 if h <= 0 else min(32, max(2, 2 ** math.floor(math.log2(h) + 0.5)))
        assert L >= min(lat, thr), (m, nnz, mx, L)
        assert i.grid == i.ntiles == max(1, -(-m * L // 256))


def test_select_auto_small_matrix():
    """C1 shape (rows of 16): FLAT row groups of 16 lanes per row (the longest row, in one pass); up to 2^18
    rows of at most 256 nnz whose values and columns fit 256 MB: row groups; beyond: row-aligned tiles.
    With a row beyond 256 nnz, too few 512-key tiles for the device -> ADAPTIVE, 188-key tiles, one per run."""
    i = pf.select(make_stats(4096, 65536, 16), "f64", "auto")
    assert i.variant == pf.FLAT and i.tile == 16 and i.row_aligned == 1 and i.needs_fixup == 0
    assert i.ntiles == 4096 * 16 // 256 and i.grid == i.ntiles  # workgroups of 256 lanes, launched as many
    cases = ((100000, 500000, 200, 4),      # lanes that fill the chip
             (1000, 1000, 200, 32),         # latency: the longest row, capped at 32
             (10000, 70000, 8, 8),          # latency: the longest row
             (32768, 65536, 10, 8),         # the longest row would overfill the chip: the filling lanes
             (262144, 262144 * 32, 60, 16),  # throughput: half the mean row
             (262144, 262144 * 8, 40, 4),
             (262144, 262144 * 5, 5, 2),    # C2 at 512^2
             (200000, 200000 * 128, 200, 32))
    for m, nnz, mx, lanes in cases:
        assert _lanes(m, nnz, mx) == lanes, (m, nnz, mx)
        i = pf.select(make_stats(m, nnz, mx), "f32", "auto")
        assert (i.variant, i.tile) == (pf.FLAT, lanes), (m, nnz, mx)
    i = pf.select(make_stats(1000000, 5000000, 20), "f64", "auto")  # over 2^18 rows: tiles
    assert i.variant == pf.FLAT and i.tile == 1024 and i.row_aligned == 1
    i = pf.select(make_stats(262145, 262145 * 5, 20), "f64", "auto")
    assert i.variant == pf.FLAT and i.tile == 1024
    i = pf.select(make_stats(200000, 200000 * 128, 200), "f64", "auto")  # 307 MB of values and columns: tiles
    assert i.variant == pf.FLAT and i.tile == 1024
    i = pf.select(make_stats(4096, 65536, 300), "f64", "auto")
    assert i.variant == pf.ADAPTIVE and i.tile == 188 and i.run_tiles == 1
    assert i.long_row_min == 64


def test_select_auto_very_short_rows_is_flat():
    """C4 shape: 2.5 nnz per row -> FLAT."""
    s = make_stats(20000000, 50000000, 14, empty=1640000)
    for dt, tile in (("f64", 2048), ("f32", 2048)):   # under 4 nnz per row: 2048-nnz tiles
        i = pf.select(s, dt, "auto")
        assert i.variant == pf.FLAT and i.tile == tile and i.row_aligned == 1 and i.needs_fixup == 0


def test_select_auto_long_rows_are_split_row_flat():
    """C3 shape (short rows plus a few long ones) -> split-row FLAT 1024; C5 shape (dense rows hold most nnz)
    -> split-row FLAT 2048; both with the x-window schedule when x exceeds one XCD's 4 MB L2."""
    c3 = pf.select(make_stats(2000000, 15200000, 200000), "f64", "auto")
    assert c3.variant == pf.FLAT and c3.tile == 1024 and c3.row_aligned == 0 and c3.needs_fixup == 1
    assert c3.x_windows == 1                                     # x = 16 MB
    c5 = pf.select(make_stats(1000000, 315647995, 499000), "f64", "auto")
    assert c5.variant == pf.FLAT and c5.tile == 2048 and c5.row_aligned == 0 and c5.needs_fixup == 1
    assert c5.x_windows == 1                                     # x = 8 MB
    c5f = pf.select(make_stats(1000000, 315647995, 499000), "f32", "auto")
    assert c5f.variant == pf.FLAT and c5f.tile == 2048 and c5f.x_windows == 0   # x = 4 MB fits one L2
    small = pf.select(make_stats(30000, 200000, 3000), "f64", "auto")
    assert small.variant == pf.ADAPTIVE and small.tile == 188    # too small for 512-key tiles


def test_select_long_rows_need_the_combine_kernel():
    s = make_stats(2000000, 15000000, 200000)
    i = pf.select(s, "f64", "adaptive")
    assert i.needs_fixup == 1 and i.guess_spread == 0 and i.tile == 512
    f = pf.select(s, "f64", "flat")
    assert f.variant == pf.FLAT and f.ntiles == -(-15000000 // 1024) and f.needs_fixup == 1
    p = pf.select(s, "f64", "prefree")
    assert p.variant == pf.PREFREE and p.tile == 512 and p.ntiles == -(-15000000 // 512)


def test_select_row_aligned_threshold():
    """FLAT 1024/2048 tiles own whole rows when no row exceeds PFK_ALIGN_ROW_MAX (256) nnz."""
    for max_len, aligned in ((256, 1), (257, 0)):
        for dt, tile in (("f64", 1024), ("f32", 2048)):
            i = pf.select(make_stats(1000000, 20000000, max_len), dt, "flat")
            assert i.tile == tile and i.row_aligned == aligned and i.needs_fixup == 1 - aligned
    for variant in ("adaptive", "prefree"):
        assert pf.select(make_stats(1000000, 20000000, 5), "f64", variant).row_aligned == 0


def test_select_f16_auto_is_flat():
    """fp16 values: AUTO picks FLAT (2048 nnz per tile) for every matrix, row-aligned when rows fit;
    ADAPTIVE (fp32's tiles) and PREFREE are there when asked for."""
    short = pf.select(make_stats(4194304, 20963328, 5), "f16", "auto")
    assert short.variant == pf.FLAT and short.tile == 2048 and short.row_aligned == 1 and short.needs_fixup == 0
    dense = pf.select(make_stats(1000000, 315647995, 499000), "f16", "auto")
    assert dense.variant == pf.FLAT and dense.tile == 2048 and dense.row_aligned == 0 and dense.needs_fixup == 1
    assert pf.supported_tiles("flat", "f16") == [1024, 2048, 2, 4, 8, 16, 32]
    assert pf.supported_tiles("adaptive", "f16") == pf.supported_tiles("adaptive", "f32") == [440, 494, 1024]
    assert pf.supported_tiles("prefree", "f16") == [512, 1024]
    a = pf.select(make_stats(1000, 5000, 5), "f16", "adaptive")
    assert a.variant == pf.ADAPTIVE and a.tile == 440
    p = pf.select(make_stats(1000, 5000, 5), "f16", "prefree")
    assert p.variant == pf.PREFREE and p.tile == 512 and p.ladder == 3


def test_select_rejects_bad_arguments():
    s = make_stats(10, 10, 1)
    with pytest.raises(pf.PrefreeError):
        pf.select(s, 7, "auto")


def test_supported_tiles():
    assert pf.supported_tiles("adaptive", "f64") == [188, 238, 494, 512]
    assert pf.supported_tiles("adaptive", "f32") == [440, 494, 1024]
    groups = [2, 4, 8, 16, 32]  # FLAT row groups: lanes per row
    assert pf.supported_tiles("flat", "f64") == [256, 1024, 2048, 4096] + groups
    assert pf.supported_tiles("flat", "f32") == [256, 1024, 2048, 4096] + groups
    assert pf.supported_tiles("flat", "f16") == [1024, 2048] + groups
    assert pf.supported_tiles("prefree", "f64") == [512, 1024]


def test_validation_before_gpu():
    L = pf.lib()
    h = ctypes.c_void_p()
    assert L.pf_plan_create(ctypes.byref(h), None, None, -1, 4, 0, 0, 0, None) == 1
    assert L.pf_plan_create(ctypes.byref(h), None, None, 4, 4, 0, 9, 0, None) == 1
    assert L.pf_plan_create(ctypes.byref(h), None, None, 4, 4, 0, 0, 11, None) == 1
    assert L.pf_plan_create(ctypes.byref(h), 256, 8, 4, 4, 4, 0, 0, None) == 2   # misaligned col
    assert L.pf_plan_execute(None, None, None, None, None, None, None) == 1
    m, n, z = ctypes.c_int(), ctypes.c_int(), ctypes.c_longlong()
    assert L.pf_synth_dims(9, 1, 0, ctypes.byref(m), ctypes.byref(n), ctypes.byref(z)) == 1
    assert L.pf_plan_destroy(None) == 0


def test_noalloc_rejects_oversized_workspace_before_launch():
    # pf_spmv_noalloc: FLAT with 1024-nnz tiles on 300M nnz needs about 10 MB of workspace, more than the
    # 8 MiB scratch; refused from the sizes alone, before any GPU call (the pointers are never read).
    L = pf.lib()
    f = L.pf_spmv_noalloc
    f.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 5 + [ctypes.c_void_p]
    f.restype = ctypes.c_int
    st = f(0x1000, 0x1000, 0x1000, 0x1000, 0x1000, 1, 1, 300_000_000, pf.F64, pf.FLAT, None)
    assert st == 5  # PF_ERR_UNSUPPORTED
    assert b"scratch" in L.pf_last_error()


# ---- the thin HIP layer checks the workspace sizes it is given (no launch happens) ----

def _args(ntiles=100, **kw):
    fake = 0x10000  # never dereferenced: every case below is refused on the host
    a = dict(row_ptr=fake, col=fake, val=fake, x=fake, y=fake, m=1000, n=1000, nnz=100 * 1024, tile=1024,
             ntiles=ntiles, head_slot=fake, tail_slot=fake, owner_row=fake, err_flag=fake,
             head_bytes=ntiles * 8, tail_bytes=ntiles * 8, owner_bytes=ntiles * 4)
    a.update(kw)
    return pf.SpmvArgs(**a)


@pytest.mark.parametrize("field,value", [("head_bytes", 99 * 8), ("tail_bytes", 100 * 8 - 1), ("owner_bytes", 396),
                                         ("head_slot", None)])
def test_flat_split_rejects_small_slots(field, value):
    K = pf.klib()
    a = _args(**{field: value})
    assert K.pfk_spmv_flat(pf.F64, ctypes.byref(a), None) == 1  # PF_ERR_INVALID
    assert K.pfk_spmv_fixup(pf.F64, 0, ctypes.byref(a), None) == 1
    assert K.pfk_spmv_adaptive(pf.F64, ctypes.byref(_args(tile=512, **{field: value})), None) == 1


def test_fp16_slots_are_fp32():
    # fp16 partial sums are fp32: 2-byte slots per tile are too small.
    K = pf.klib()
    a = _args(head_bytes=100 * 2, tail_bytes=100 * 2)
    assert K.pfk_spmv_flat(pf.F16, ctypes.byref(a), None) == 1
    assert b"head slots" in K.pfk_last_error()


def test_row_map_and_schedule_sizes_checked():
    K = pf.klib()
    fake = 0x20000
    assert K.pfk_spmv_flat(pf.F64, ctypes.byref(_args(row_map=fake, row_map_bytes=100 * 8)), None) == 1
    assert b"row map" in K.pfk_last_error()
    cap = 13  # ceil(100 / 8)
    ints = 16 + 8 * cap + 100
    a = _args(row_map=fake, row_map_bytes=101 * 8, sched=fake, sched_cap=cap, sched_bytes=ints * 4 - 4)
    assert K.pfk_spmv_flat(pf.F64, ctypes.byref(a), None) == 1
    assert b"schedule" in K.pfk_last_error()
    a = _args(row_map=fake, row_map_bytes=101 * 8, sched=fake, sched_cap=12, sched_bytes=1 << 20)
    assert K.pfk_spmv_flat(pf.F64, ctypes.byref(a), None) == 1  # lists shorter than an even share


def test_adaptive_owner_table_size_checked():
    K = pf.klib()
    a = _args(tile=512, owner_bytes=10)
    assert K.pfk_adaptive_owners(pf.F64, ctypes.byref(a), None) == 1


def test_prefree_ladder_range_checked():
    K = pf.klib()
    K.pfk_spmv_prefree.argtypes = [ctypes.c_int, ctypes.POINTER(pf.SpmvArgs), ctypes.c_void_p]
    for bad in (-1, 6):
        a = _args(tile=512, ladder=bad)
        assert K.pfk_spmv_prefree(pf.F64, ctypes.byref(a), None) == 1
        assert b"ladder" in K.pfk_last_error()


def test_plan_info_layout_has_ladder():
    s = pf.RowStats(m=1000, nnz=5000, max_row_len=7, min_row_len=3)
    assert pf.select(s, "f64", "prefree").ladder == 3
    assert pf.select(s, "f64", "flat").ladder == 0


def _hyb_args(**kw):
    fake = 0x30000
    nd, nl, R = 3, 20, 5
    a = dict(row_ptr=fake, col=fake, val=fake, x=fake, y=fake, m=1000, n=1000, nnz=100 * 1024, tile=1024,
             ntiles=10, err_flag=fake, dense_rows=fake, n_dense=nd, n_runs=R - 1, runs=fake, runs_bytes=5 * R * 4,
             long_mode=1, n_long_tiles=nl, long_tiles=fake, long_deal=fake, long_row_tiles=fake, long_part=fake,
             long_tiles_bytes=nl * 16, long_deal_bytes=nl * 4, long_row_tiles_bytes=(nd + 1) * 4,
             long_part_bytes=nl * 8)
    a.update(kw)
    return pf.SpmvArgs(**a)


@pytest.mark.parametrize("field,value,what", [("long_tiles_bytes", 20 * 16 - 1, b"long-row tiles"),
                                              ("long_deal_bytes", 76, b"long-row tile deal"),
                                              ("long_row_tiles_bytes", 12, b"long-row tile index"),
                                              ("long_part_bytes", 20 * 4, b"long-row partial sums"),
                                              ("long_deal", None, b"missing tables"),
                                              ("n_long_tiles", 0, b"missing tables"),
                                              ("row_apart_bytes", 999, b"rows summed apart")])
def test_hybrid_long_mode_tables_checked(field, value, what):
    # pfk_spmv_hybrid in long mode refuses a short or missing long-row table before any launch
    K = pf.klib()
    K.pfk_spmv_hybrid.argtypes = [ctypes.c_int, ctypes.POINTER(pf.SpmvArgs), ctypes.c_void_p]
    a = _hyb_args(**{field: value})
    if field == "row_apart_bytes":  # with x halves, one byte per row (m = 1000) is required
        a.row_apart, a.x_halves, a.half_part, a.half_part_bytes = 0x30000, 1, 0x30000, 8000
    assert K.pfk_spmv_hybrid(pf.F64, ctypes.byref(a), None) == 1
    assert what in K.pfk_last_error()


def test_gather_cols_rejects_bad_arguments():
    K = pf.klib()
    K.pfk_gather_cols.argtypes = [ctypes.c_void_p, ctypes.c_longlong, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                  ctypes.c_void_p]
    assert K.pfk_gather_cols(None, 10, 0x1000, 4, 0x1000, None) == 1
    assert K.pfk_gather_cols(0x1000, 10, 0x1000, -1, 0x1000, None) == 1
    assert K.pfk_gather_cols(0x1000, 10, 0x1000, 0, 0x1000, None) == 0  # nothing to gather: no launch


STRUCTS = [("pf_row_stats", "RowStats", "prefree_c.h"), ("pf_plan_info", "PlanInfo", "prefree_c.h"),
           ("pf_tune_result", "TuneResult", "prefree_c.h"), ("pfk_spmv_args", "SpmvArgs", "prefree_kernels.h")]


def test_ctypes_mirrors_match_the_c_structs(tmp_path):
    """Every ctypes mirror in prefree-public_amd/__init__.py has the size, field order and field offsets of its
    struct in include/*.h, as the C compiler lays it out (a small C program prints sizeof / offsetof)."""
    inc = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "include")
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "prefree_c.h"', '#include "prefree_kernels.h"',
             "int main(void) {"]
    for cname, pyname, _ in STRUCTS:
        lines.append(f'printf("{pyname} sizeof %zu\\n", sizeof({cname}));')
        for fname, _t in getattr(pf, pyname)._fields_:
            lines.append(f'printf("{pyname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines += ["return 0; }"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", inc, "-o", str(exe), str(src)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    got = {}
    for line in filter(None, out):
        py, field, value = line.split()
        got[(py, field)] = int(value)
    for _cname, pyname, _ in STRUCTS:
        cls = getattr(pf, pyname)
        assert got[(pyname, "sizeof")] == ctypes.sizeof(cls), pyname
        for fname, _t in cls._fields_:
            assert got[(pyname, fname)] == getattr(cls, fname).offset, (pyname, fname)


def test_dense_windows_cover_x_evenly(tmp_path):
    """pfk_dense_nwin / pfk_dense_width (include/prefree_kernels.h): a multiple of 8 windows (one share per XCD),
    each a multiple of 64 columns and at most PFK_DENSE_WINDOW(dtype), together covering [0, n), with no more
    windows than the fewest of that width rounded up to a multiple of 8."""
    inc = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "include")
    src = tmp_path / "win.c"
    src.write_text("\n".join([
        "#include <stdio.h>", '#include "prefree_kernels.h"', "int main(void) {",
        "  const long long ns[] = {1, 63, 64, 65, 8191, 8192, 8193, 60000, 65536, 65537, 600000, 1000000, 1100000,",
        "                          2000000, 4194304, 20000000, 2147483647LL};",
        "  for (int t = 0; t < 2; ++t) for (unsigned i = 0; i < sizeof ns / sizeof ns[0]; ++i) {",
        "    const int nw = pfk_dense_nwin(ns[i], t), w = pfk_dense_width(ns[i], nw);",
        '    printf("%d %lld %d %d\\n", t, ns[i], nw, w);',
        "  }", "  return 0; }"]) + "\n")
    exe = tmp_path / "win"
    subprocess.run(["gcc", "-std=c11", "-I", inc, "-o", str(exe), str(src)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    rows = [tuple(int(v) for v in line.split()) for line in out if line]
    assert len(rows) == 34
    for dtype, n, nw, w in rows:
        cap = 8192 if dtype == 0 else 16384
        fewest = -(-n // cap)
        assert nw % 8 == 0 and fewest <= nw < fewest + 8, (dtype, n, nw)
        assert w % 64 == 0 and 0 < w <= cap, (dtype, n, w)
        assert nw * w >= n, (dtype, n, nw, w)
    c5 = {(d, n): (nw, w) for d, n, nw, w in rows}
    assert c5[(0, 1000000)] == (128, 7872) and c5[(1, 1000000)] == (64, 15680)
