"""Matrix Market reader (pf_mtx_read) against the reference harness's conventions
(utilities/mmio.cpp:1543-1713): 1-based -> 0-based, file order within a row,
duplicates kept, symmetric/hermitian entries mirrored right after the entry,
skew-symmetric files not mirrored, pattern -> 1.0, complex -> real part.

Pinned two ways: hand-derived CSR for small files (order and layout), and
scipy.io.mmread (an independent reader) for the matrix values of random files.
"""
import numpy as np
import pytest
import scipy.io
import scipy.sparse as sp

import prefree_amd as pf


def write(tmp_path, name, text):
    p = tmp_path / name
    p.write_text(text)
    return str(p)


def test_general_real_file_order_and_duplicates(tmp_path):
    f = write(tmp_path, "g.mtx", """%%MatrixMarket matrix coordinate real general
% a comment
3 4 6
2 3 1.5
1 1 -2
2 1 3e-1
3 4 7
2 3 0.25
1 4 9
""")
    rp, col, val, m, n, sym = pf.mtx_read(f)
    assert (m, n, sym) == (3, 4, False)
    assert rp.tolist() == [0, 2, 5, 6]
    assert col.tolist() == [0, 3, 2, 0, 2, 3]            # row 1: file order 2,1,2 (0-based) with the duplicate
    assert val.tolist() == [-2.0, 9.0, 1.5, 0.3, 0.25, 7.0]


def test_symmetric_mirror_follows_each_entry(tmp_path):
    f = write(tmp_path, "s.mtx", """%%MatrixMarket matrix coordinate real symmetric
3 3 4
2 1 5
1 1 1
3 2 6
3 1 7
""")
    rp, col, val, m, n, sym = pf.mtx_read(f)
    assert sym and (m, n) == (3, 3)
    # one pass in file order: (1,0) then mirror (0,1); (0,0); (2,1) then (1,2); (2,0) then (0,2)
    assert rp.tolist() == [0, 3, 5, 7]
    assert col.tolist() == [1, 0, 2, 0, 2, 1, 0]
    assert val.tolist() == [5, 1, 7, 5, 6, 6, 7]


def test_field_types_and_banner_case(tmp_path):
    pat = pf.mtx_read(write(tmp_path, "p.mtx", "%%MatrixMarket MATRIX Coordinate PATTERN General\n2 2 2\n1 2\n2 1\n"))
    assert pat[2].tolist() == [1.0, 1.0] and pat[1].tolist() == [1, 0]
    itg = pf.mtx_read(write(tmp_path, "i.mtx", "%%MatrixMarket matrix coordinate integer general\n2 2 1\n2 2 -4\n"))
    assert itg[2].tolist() == [-4.0] and itg[0].tolist() == [0, 0, 1]
    cpx = pf.mtx_read(write(tmp_path, "c.mtx", "%%MatrixMarket matrix coordinate complex hermitian\n2 2 2\n1 1 2 0\n2 1 3 -1\n"))
    assert cpx[5] and cpx[1].tolist() == [0, 1, 0] and cpx[2].tolist() == [2.0, 3.0, 3.0]


def test_skew_symmetric_is_not_mirrored(tmp_path):
    f = write(tmp_path, "k.mtx", "%%MatrixMarket matrix coordinate real skew-symmetric\n3 3 2\n2 1 4\n3 2 -1\n")
    rp, col, val, m, n, sym = pf.mtx_read(f)
    assert not sym and rp.tolist() == [0, 0, 1, 2] and col.tolist() == [0, 1] and val.tolist() == [4, -1]


def test_comments_blank_lines_crlf_and_empty_rows(tmp_path):
    f = write(tmp_path, "e.mtx", "%%MatrixMarket matrix coordinate real general\r\n%c1\r\n%c2\r\n\r\n5 2 2\r\n"
                               "4 2 1.0\r\n% inline comment\r\n1 1 2.0\r\n")
    rp, col, val, m, n, sym = pf.mtx_read(f)
    assert (m, n) == (5, 2) and rp.tolist() == [0, 1, 1, 1, 2, 2] and col.tolist() == [0, 1]


def test_empty_matrix(tmp_path):
    rp, col, val, m, n, sym = pf.mtx_read(write(tmp_path, "z.mtx", "%%MatrixMarket matrix coordinate real general\n4 4 0\n"))
    assert rp.tolist() == [0, 0, 0, 0, 0] and len(col) == 0 and len(val) == 0


@pytest.mark.parametrize("text,why", [
    ("%%MatrixMarket matrix array real general\n2 2\n1\n2\n3\n4\n", "array"),
    ("%MatrixMarket matrix coordinate real general\n1 1 1\n1 1 1\n", "banner"),
    ("%%MatrixMarket matrix coordinate real general\n2 2 2\n1 1 1\n", "truncated"),
    ("%%MatrixMarket matrix coordinate real general\n2 2 1\n3 1 1\n", "row out of range"),
    ("%%MatrixMarket matrix coordinate real general\n2 2 1\n1 0 1\n", "column out of range"),
    ("%%MatrixMarket matrix coordinate real weird\n2 2 1\n1 1 1\n", "symmetry"),
    ("%%MatrixMarket vector coordinate real general\n2 2 1\n1 1 1\n", "object"),
])
def test_malformed_files_are_rejected(tmp_path, text, why):
    with pytest.raises(pf.PrefreeError) as e:
        pf.mtx_read(write(tmp_path, "bad.mtx", text))
    assert e.value.status == 8, why


def test_missing_file():
    with pytest.raises(pf.PrefreeError) as e:
        pf.mtx_read("/nonexistent/none.mtx")
    assert e.value.status == 8


@pytest.mark.parametrize("symmetry", ["general", "symmetric"])
def test_random_files_match_scipy(tmp_path, symmetry):
    rng = np.random.default_rng(7)
    n = 300
    nz = 2000
    i = rng.integers(1, n + 1, nz)
    j = rng.integers(1, n + 1, nz)
    if symmetry == "symmetric":
        i, j = np.maximum(i, j), np.minimum(i, j)       # lower triangle, as the format requires
    v = rng.uniform(-1, 1, nz)
    lines = [f"%%MatrixMarket matrix coordinate real {symmetry}", f"{n} {n} {nz}"]
    lines += [f"{a} {b} {float(c)!r}" for a, b, c in zip(i, j, v)]
    f = write(tmp_path, "r.mtx", "\n".join(lines) + "\n")
    rp, col, val, m, nn, sym = pf.mtx_read(f)
    ours = sp.csr_matrix((val, col, rp), shape=(m, nn)).toarray()   # duplicates summed
    ref = scipy.io.mmread(f)
    ref = ref.toarray() if sp.issparse(ref) else np.asarray(ref)
    assert np.allclose(ours, ref, rtol=0, atol=1e-12)
    assert np.all(np.diff(rp) >= 0) and rp[-1] == len(col)
