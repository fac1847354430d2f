"""Row statistics on the GPU (pf_row_stats_compute: k_row_stats, k_col_check) against numpy, exactly."""
import numpy as np
import pytest

import prefree_amd as pf
from csr_cases import edge_cases
from gpu_util import dev

pytestmark = pytest.mark.gpu

ALIGN_MAX = 256  # PFK_ALIGN_ROW_MAX


def cases():
    out = [(name, rp, col, n) for name, rp, col, n in edge_cases()]
    for cfg, scale in ((1, 0), (2, 300), (3, 60000), (4, 400000), (5, 40000)):
        rp, col, _ = pf.synth_csr(cfg, seed=4, scale_n=scale, dtypes=())
        out.append((f"C{cfg}", rp, col, len(rp) - 1))
    # more rows than the statistics' workgroups take at 8 rows per lane (a workgroup per CU, several passes)
    rp, col, _ = pf.synth_csr(3, seed=5, scale_n=2600001, dtypes=())
    out.append(("C3_2.6M", rp, col, len(rp) - 1))
    return out


def expected(rp, col, n):
    m, nnz = len(rp) - 1, int(rp[-1])
    lens = np.diff(rp.astype(np.int64))
    bits = np.where(lens > 0, np.frexp(lens.astype(np.float64))[1], 0)  # bit_length of each length
    hist = np.bincount(bits, minlength=33).astype(np.int64)
    short = lens[lens <= ALIGN_MAX]
    dev = 0
    if m > 0 and nnz > 0:
        # the kernel's own arithmetic in binary64, no contraction: r - row_ptr[r] * (m / nnz)
        d = np.abs(np.arange(m, dtype=np.float64) - rp[:m].astype(np.float64) * (m / nnz))
        dev = int(np.ceil(d.max()))
    # the line through (row_ptr[m / 4], m / 4) and (row_ptr[3m / 4], 3m / 4): rows over 28 rows from it
    q1, q3 = m // 4, 3 * m // 4
    p1, p3 = (int(rp[q1]), int(rp[q3])) if m >= 4 else (0, 0)
    far = m
    if m >= 4 and p3 > p1:
        la = (q3 - q1) / (p3 - p1)
        lb = q1 - la * p1
        far = int((np.abs(np.arange(m, dtype=np.float64) - (la * rp[:m].astype(np.float64) + lb)) > 28.0).sum())
    return dict(m=m, nnz=nnz, max_row_len=int(lens.max(initial=0)), min_row_len=int(lens.min()) if m else 0,
                n_empty_rows=int((lens == 0).sum()), n_decreasing=0, row_ptr_first=int(rp[0]),
                row_ptr_last=nnz, n_bad_cols=int(((col < 0) | (col >= n)).sum()), n_long_rows=int((lens > ALIGN_MAX).sum()),
                max_short_row_len=int(short.max(initial=0)), guess_dev=dev, line_q1_row_ptr=p1, line_q3_row_ptr=p3,
                line_far_rows=far, hist=hist)


CASES = cases()


@pytest.mark.parametrize("name,rp,col,n", CASES, ids=[c[0] for c in CASES])
def test_row_stats_match_numpy(name, rp, col, n):
    m, nnz = len(rp) - 1, int(rp[-1])
    s = pf.row_stats(dev(rp), dev(col) if nnz else None, m, n, nnz)
    want = expected(rp, col, n)
    for k, v in want.items():
        if k == "hist":
            assert list(s.hist_log2) == list(v), name
        elif k == "min_row_len" and m == 0:
            continue
        else:
            assert getattr(s, k) == v, (name, k, getattr(s, k), v)


def test_c2_plan_takes_the_deviation_spread():
    """C2 at full size: rows up to 410 from the mean-density guess -> 64 probes 16 rows apart; but only the
    rows of the first and last grid rows lie over 28 rows from the line through the quartile rows, so the row-aligned tiles
    search around that line instead, 1 row apart."""
    rp, col, _ = pf.synth_csr(2, seed=1, dtypes=())
    m, nnz = len(rp) - 1, int(rp[-1])
    s = pf.row_stats(dev(rp), dev(col), m, m, nnz)
    want = expected(rp, col, m)
    assert s.guess_dev == want["guess_dev"] == 410
    assert s.line_far_rows == want["line_far_rows"] and 0 < s.line_far_rows * 256 <= m  # 3817 of 4,194,304
    with pf.Plan(dev(rp), dev(col), m, m, nnz, "f64") as p:
        assert p.info.guess_spread == 16
        la = (3 * m // 4 - m // 4) / (s.line_q3_row_ptr - s.line_q1_row_ptr)
        assert p.info.guess_a == la and p.info.guess_b == m // 4 - la * s.line_q1_row_ptr


def test_irregular_plan_keeps_the_mean_density_guess():
    """C4 (Poisson rows, a random walk off any line): most rows lie far from the quartile line, so the plan
    keeps the mean-density guess (guess_a 0)."""
    rp, col, _ = pf.synth_csr(4, seed=1, scale_n=400000, dtypes=())
    m, nnz = len(rp) - 1, int(rp[-1])
    s = pf.row_stats(dev(rp), dev(col), m, m, nnz)
    assert s.line_far_rows == expected(rp, col, m)["line_far_rows"] and s.line_far_rows * 256 > m
    with pf.Plan(dev(rp), dev(col), m, m, nnz, "f64") as p:
        assert p.info.guess_a == 0.0
