"""The cdspmv harness's fp16 arithmetic (prefree-public_amd/host/cdspmv.cpp), on the CPU.

The --f16 mode of the harness checks the library against a sequential SpMV that
rounds every product and sum to binary16, as the reference's fp16 build does
(test/test_cdspmv.cpp:4-20 with valT = half, include/common.h:43-46).  Its
binary16 conversions and that SpMV are checked here:
  * widening: every one of the 65,536 bit patterns against numpy's float16;
  * narrowing: round to nearest even, against numpy, on every binary16 value,
    the midpoints between neighbours and the floats next to them, random floats
    over the whole range, zeros, infinities, overflow and subnormals;
  * the sequential SpMV: bit for bit against oracle.spmv_serial_f16 on random
    CSR, including rows that overflow to infinity.
A small driver compiled here includes cdspmv.cpp with its main renamed (and the
vendor SpMV, which the fp16 paths never call, stubbed).
"""
import os
import subprocess

import numpy as np
import pytest

import oracle
import prefree_amd as pf

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(REPO, "prefree-public_amd", "host", "cdspmv.cpp")
LIB = os.path.join(REPO, "prefree-public_amd", "lib")

DRIVER = r'''
#define main cdspmv_main
#include CDSPMV_SRC
#undef main
#include <cstdio>
#include <vector>
// the fp16 paths run no vendor SpMV; these stand in for host/vendor_rocsparse.cpp, not linked here
int vendor_spmv(const double *, const int *, const int *, const double *, double *, int, int, int, int, int,
                double *, double *, char *why, int why_len) { std::snprintf(why, why_len, "not linked"); return 1; }
int vendor_spmv(const float *, const int *, const int *, const float *, float *, int, int, int, int, int,
                double *, double *, char *why, int why_len) { std::snprintf(why, why_len, "not linked"); return 1; }
// usage: drv widen OUT | drv narrow IN OUT | drv spmv IN OUT
int main(int argc, char **argv)
{
    const std::string mode = argv[1];
    if (mode == "widen") {
        FILE *o = std::fopen(argv[2], "wb");
        for (int b = 0; b < 65536; ++b) {
            const float f = widen(pf_half{(unsigned short)b});
            std::fwrite(&f, 4, 1, o);
        }
        std::fclose(o);
        return 0;
    }
    FILE *in = std::fopen(argv[2], "rb");
    FILE *o = std::fopen(argv[3], "wb");
    if (mode == "narrow") {
        float v;
        while (std::fread(&v, 4, 1, in) == 1) {
            const unsigned short b = narrow(v).bits;
            std::fwrite(&b, 2, 1, o);
        }
    } else {
        int m = 0, n = 0, nnz = 0;
        if (std::fread(&m, 4, 1, in) != 1 || std::fread(&n, 4, 1, in) != 1 || std::fread(&nnz, 4, 1, in) != 1)
            return 2;
        std::vector<int> rp(m + 1), col(nnz);
        std::vector<pf_half> val(nnz), x(n), y(m);
        if (std::fread(rp.data(), 4, m + 1, in) != (size_t)(m + 1) || std::fread(col.data(), 4, nnz, in) != (size_t)nnz ||
            std::fread(val.data(), 2, nnz, in) != (size_t)nnz || std::fread(x.data(), 2, n, in) != (size_t)n)
            return 2;
        serial_spmv(val.data(), rp.data(), col.data(), x.data(), y.data(), m);
        std::fwrite(y.data(), 2, m, o);
    }
    std::fclose(in);
    std::fclose(o);
    return 0;
}
'''


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    d = tmp_path_factory.mktemp("cdspmv_f16")
    src = d / "drv.cpp"
    src.write_text(DRIVER)
    exe = d / "drv"
    r = subprocess.run(["g++", "-O2", "-std=c++17", f'-DCDSPMV_SRC="{SRC}"', "-I", os.path.join(REPO, "include"),
                        str(src), "-o", str(exe), f"-L{LIB}", "-lprefree", f"-Wl,-rpath,{LIB}"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return d, str(exe)


def test_widen_every_pattern(driver):
    d, exe = driver
    subprocess.run([exe, "widen", str(d / "w.bin")], check=True, timeout=60)
    got = np.fromfile(d / "w.bin", np.float32)
    ref = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    assert np.array_equal(got, ref, equal_nan=True)


def test_narrow_round_to_nearest_even(driver):
    d, exe = driver
    rng = np.random.default_rng(5)
    h = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    f = np.sort(h[np.isfinite(h)])
    mids = ((f[:-1].astype(np.float64) + f[1:]) / 2).astype(np.float32)     # exact ties
    up = np.nextafter(mids, np.float32(np.inf)).astype(np.float32)
    down = np.nextafter(mids, np.float32(-np.inf)).astype(np.float32)
    rand = (rng.standard_normal(200000) * 10.0 ** rng.integers(-9, 6, 200000)).astype(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, 65504, 65519.99, 65520, 65536, 1e30, -1e30,
                        2.0 ** -24, 2.0 ** -25, 2.0 ** -25 + 2.0 ** -40, 2.0 ** -26, 3 * 2.0 ** -25, 2.0 ** -14],
                       dtype=np.float32)
    vals = np.concatenate([f, mids, up, down, rand, special]).astype(np.float32)
    vals.tofile(d / "n_in.bin")
    subprocess.run([exe, "narrow", str(d / "n_in.bin"), str(d / "n_out.bin")], check=True, timeout=60)
    got = np.fromfile(d / "n_out.bin", np.uint16)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    bad = np.flatnonzero(got != ref)
    assert bad.size == 0, f"{bad.size} values, first {vals[bad[:5]]}: got {got[bad[:5]]} want {ref[bad[:5]]}"


@pytest.mark.parametrize("cfg,scale,spread", [(2, 64, 4.0), (3, 5000, 4.0), (3, 5000, 40.0), (5, 3000, 40.0)])
def test_serial_half_spmv_matches_oracle(driver, cfg, scale, spread):
    d, exe = driver
    rp, col, _ = pf.synth_csr(cfg, seed=1, scale_n=scale, dtypes=())
    rp, col = rp.astype(np.int32), col.astype(np.int32)
    m, n, nnz = len(rp) - 1, int(col.max()) + 1, len(col)
    rng = np.random.default_rng(cfg + int(spread))
    val = (rng.standard_normal(nnz) * spread).astype(np.float16)
    x = (rng.standard_normal(n) * spread).astype(np.float16)
    with open(d / "s_in.bin", "wb") as fh:
        np.array([m, n, nnz], np.int32).tofile(fh)
        rp.tofile(fh); col.tofile(fh); val.tofile(fh); x.tofile(fh)
    subprocess.run([exe, "spmv", str(d / "s_in.bin"), str(d / "s_out.bin")], check=True, timeout=60)
    got = np.fromfile(d / "s_out.bin", np.float16)
    ref = np.asarray(oracle.spmv_serial_f16(rp, col, val, x), np.float16)
    if spread >= 40 and cfg != 2:
        assert np.isinf(ref).any()          # the case reaches binary16 overflow
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
