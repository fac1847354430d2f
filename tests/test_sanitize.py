"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer — CPU only.

The Matrix Market reader (host/mtx.cpp) parses untrusted files and the
generators (host/synth.cpp) do the index arithmetic of the benchmark matrices.
Both are compiled with g++ -fsanitize=address,undefined (host code only, no
HIP) together with tests/sanitize/host_driver.cpp, and run over valid,
malformed and randomly corrupted .mtx files and over every configuration at
scaled sizes.  Any sanitizer report aborts the driver; every readable file must
give a valid CSR and every unreadable one a PF_ERR_IO status.
"""
import os
import shutil
import subprocess

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = [os.path.join(REPO, "prefree-public_amd", "host", f) for f in ("mtx.cpp", "synth.cpp")]
DRIVER = os.path.join(REPO, "tests", "sanitize", "host_driver.cpp")
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1",
           UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1", OMP_NUM_THREADS="4")

VALID = {
    "general.mtx": "%%MatrixMarket matrix coordinate real general\n% c\n\n3 4 6\n2 3 1.5\n1 1 -2\n2 1 3e-1\n"
                   "3 4 7\n2 3 0.25\n1 4 9\n",
    "symmetric.mtx": "%%MatrixMarket matrix coordinate real symmetric\n3 3 4\n2 1 5\n1 1 1\n3 2 6\n3 1 7\n",
    "pattern.mtx": "%%MatrixMarket MATRIX Coordinate PATTERN General\n2 2 2\n1 2\n2 1\n",
    "integer.mtx": "%%MatrixMarket matrix coordinate integer general\r\n2 2 1\r\n2 2 -4\r\n",
    "complex.mtx": "%%MatrixMarket matrix coordinate complex hermitian\n2 2 2\n1 1 1 0\n2 1 2 -3\n",
    "skew.mtx": "%%MatrixMarket matrix coordinate real skew-symmetric\n3 3 2\n2 1 4\n3 2 -1\n",
    "empty_rows.mtx": "%%MatrixMarket matrix coordinate real general\n5 5 1\n5 5 2\n",
    "no_entries.mtx": "%%MatrixMarket matrix coordinate real general\n4 3 0\n",
}
MALFORMED = {
    "empty.mtx": "",
    "no_banner.mtx": "3 3 1\n1 1 1\n",
    "short_banner.mtx": "%%MatrixMarket matrix coordinate real\n1 1 1\n1 1 1\n",
    "array_format.mtx": "%%MatrixMarket matrix array real general\n2 2\n1\n2\n3\n4\n",
    "bad_field.mtx": "%%MatrixMarket matrix coordinate quaternion general\n1 1 1\n1 1 1\n",
    "bad_size.mtx": "%%MatrixMarket matrix coordinate real general\n3 x 1\n1 1 1\n",
    "negative_size.mtx": "%%MatrixMarket matrix coordinate real general\n-3 3 1\n1 1 1\n",
    "huge_count.mtx": "%%MatrixMarket matrix coordinate real general\n3 3 2147483647\n1 1 1\n2 2 2\n",
    "index_zero.mtx": "%%MatrixMarket matrix coordinate real general\n3 3 1\n0 1 1\n",
    "index_past_end.mtx": "%%MatrixMarket matrix coordinate real general\n3 3 1\n4 1 1\n",
    "col_past_end.mtx": "%%MatrixMarket matrix coordinate real general\n3 3 1\n1 4 1\n",
    "not_a_number.mtx": "%%MatrixMarket matrix coordinate real general\n3 3 1\n1 1 abc\n",
    "truncated.mtx": "%%MatrixMarket matrix coordinate real general\n3 3 3\n1 1 1\n2 2",
    "symmetric_not_square.mtx": "%%MatrixMarket matrix coordinate real symmetric\n2 3 1\n1 3 1\n",
    "no_size_line.mtx": "%%MatrixMarket matrix coordinate real general\n% only comments\n",
}


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    out = str(tmp_path_factory.mktemp("san") / "host_driver")
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
           "-fno-omit-frame-pointer", "-fopenmp", "-I", os.path.join(REPO, "include"), *SRC, DRIVER, "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0 and "asan" in (r.stderr or "").lower():
        pytest.skip("this toolchain has no AddressSanitizer runtime")
    assert r.returncode == 0, r.stderr[-2000:]
    return out


def _run(driver, args):
    r = subprocess.run([driver, *args], capture_output=True, text=True, env=ENV, timeout=600)
    assert r.returncode == 0, (r.stdout[-3000:], r.stderr[-3000:])
    assert r.stdout.rstrip().endswith("ok")
    return r.stdout


def test_mtx_valid_and_malformed_files(driver, tmp_path):
    paths = []
    for name, text in {**VALID, **MALFORMED}.items():
        p = tmp_path / name
        p.write_bytes(text.encode())
        paths.append(str(p))
    out = _run(driver, ["mtx", *paths, str(tmp_path / "missing.mtx")])
    for name in VALID:
        assert f"{name}:" in out and "valid" in out.split(f"{name}:")[1].splitlines()[0]
    for name in MALFORMED:
        assert "status 8" in out.split(f"{name}:")[1].splitlines()[0], name


def test_mtx_corrupted_files(driver, tmp_path):
    # byte flips, deletions and truncations of the entry lines of valid files
    rng = np.random.default_rng(20)
    paths = []
    alphabet = b"0123456789 -+.eE\n%x"
    for k in range(300):
        base = list(VALID.values())[k % len(VALID)].encode()
        head = base.index(b"\n", base.index(b"\n") + 1) + 1 if k % 3 else 0  # keep the size line two times in three
        body = bytearray(base[head:])
        for _ in range(int(rng.integers(1, 6))):
            if not body:
                break
            i = int(rng.integers(0, len(body)))
            op = int(rng.integers(0, 3))
            if op == 0:
                body[i] = alphabet[int(rng.integers(0, len(alphabet)))]
            elif op == 1:
                del body[i]
            else:
                body = body[:i]
        p = tmp_path / f"c{k}.mtx"
        p.write_bytes(base[:head] + bytes(body))
        paths.append(str(p))
    _run(driver, ["mtx", *paths])


def test_mtx_random_matrices(driver, tmp_path):
    import scipy.io
    import scipy.sparse as sp

    rng = np.random.default_rng(21)
    paths = []
    for k, sym in enumerate(["general", "symmetric", "general", "skew-symmetric"]):
        n = int(rng.integers(50, 400))
        a = sp.random(n, n, density=0.03, random_state=int(rng.integers(1 << 30)), format="coo")
        if sym == "symmetric":
            a = sp.tril(a + a.T).tocoo()
        elif sym == "skew-symmetric":
            a = sp.tril(a - a.T, -1).tocoo()
        p = str(tmp_path / f"r{k}.mtx")
        scipy.io.mmwrite(p, a, symmetry=sym)
        paths.append(p)
    out = _run(driver, ["mtx", *paths])
    assert out.count("valid") == len(paths)


def test_synth_generators(driver):
    out = _run(driver, ["synth"])
    assert out.count("valid") == 10
