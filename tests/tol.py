"""Tolerances of the parity tests (stated once, used everywhere).

Forward fp32 outputs (LayerNorm y, GELU y):      |gpu - ref| <= 1e-6 + 1e-5 |ref|
Element-wise backward outputs (dx, grad_in):     |gpu - ref| <= 1e-5 s + 1e-4 |ref|,
                                                 s = max(1, rms(ref))
    (the near-zero floor 1e-5 s covers gradients that are cancelling sums of
    O(1) terms, e.g. the residual-stream gradient gtop + dx2 + dx1, whose
    fp32 rounding is ~1e-6 absolute while the value itself may be ~1e-3)
Column sums (dgamma, dbeta, dbias):              |gpu - ref| <= 1e-4 (|ref| + ||t_c||_2)
    where t_c are the per-row terms summed into column c; the float error of
    any summation order scales with ||t_c||_2, so a column whose sum cancels
    to near zero is still held to 1e-4 of its natural size.  Where the terms
    are approximations of a function (GELU dbias against float64), the
    element-wise backward floor 1e-5 s is added, times sqrt(rows).
    On every column that does not cancel (|ref| >= ||t_c||_2, and for
    approximated terms 1e-4 |ref| at least their floor 1e-5 s sqrt(rows))
    the north star's literal bound also holds: |gpu - ref| <= 1e-4 |ref|.  The largest
    |gpu - ref| / |ref| over those columns is recorded per call (COLSUM_LOG)
    and printed at the end of a pytest session.
Gather / copies / single adds / selects:         bit-exact.

Where a float oracle is itself inexact in a region (the textbook float GELU
formula where 1 + tanhf(z) cancels), the comparison with it adds that
oracle's own error |oracle_f32 - oracle_f64| to the bound, and the GPU is
also held to the plain tolerance against the float64 oracle.
"""
import numpy as np

FWD_RTOL, FWD_ATOL = 1e-5, 1e-6
BWD_RTOL, BWD_ATOL = 1e-4, 1e-5
COL_RTOL = 1e-4

# (pytest node id, name, max relative error over non-cancelling columns,
#  number of such columns, number of columns), one entry per column-sum check.
COLSUM_LOG = []


def _node():
    import os
    return os.environ.get("PYTEST_CURRENT_TEST", "").rsplit(" (", 1)[0]


def colsum_relative(name, gpu, ref, l2, floor=0.0):
    """Asserts |gpu - ref| <= COL_RTOL |ref| on the columns whose sum does not
    cancel (|ref| >= l2, the 2-norm of the column's terms) and whose
    relative bound is not below `floor`, the absolute error its terms may
    carry (nonzero for terms that approximate a function, e.g. a GELU
    gradient near its zero at u = -0.75, held element-wise to BWD_ATOL s);
    records the largest relative error there in COLSUM_LOG and returns it."""
    g = np.asarray(gpu, np.float64)
    r = np.asarray(ref, np.float64)
    # a column of zero terms sums to exactly 0 and is checked bit for bit by
    # the absolute bound; it has no relative error
    keep = (np.abs(r) >= np.asarray(l2, np.float64)) & (r != 0) & (COL_RTOL * np.abs(r) >= floor)
    rel = np.abs(g - r)[keep] / np.abs(r)[keep]
    worst = float(rel.max()) if rel.size else 0.0
    COLSUM_LOG.append((_node(), name, worst, int(keep.sum()), int(r.size)))
    assert worst <= COL_RTOL, (
        f"{name}: relative error {worst:.3e} on a non-cancelling column exceeds {COL_RTOL:g}")
    return worst


def _report(name, gpu, ref, bound):
    err = np.abs(gpu.astype(np.float64) - ref.astype(np.float64))
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(
            f"{name}: {int(bad.sum())} of {err.size} elements out of tolerance; worst at {i}: "
            f"gpu={gpu[i]!r} ref={ref[i]!r} err={err[i]:.3e} bound={bound[i] if np.ndim(bound) else bound:.3e}")
    return float(err.max()) if err.size else 0.0


def assert_fwd(name, gpu, ref):
    ref = np.asarray(ref)
    bound = FWD_ATOL + FWD_RTOL * np.abs(ref.astype(np.float64))
    return _report(name, np.asarray(gpu), ref, bound)


def assert_bwd(name, gpu, ref):
    ref = np.asarray(ref)
    r64 = ref.astype(np.float64)
    s = max(1.0, float(np.sqrt(np.mean(r64 * r64)))) if r64.size else 1.0
    bound = BWD_ATOL * s + BWD_RTOL * np.abs(r64)
    return _report(name, np.asarray(gpu), ref, bound)


def assert_colsum(name, gpu, ref, terms, approx_terms=False):
    """terms: [rows, cols] array of the per-row summands (float64 ok).

    approx_terms: the summands are themselves fp32 approximations of a
    function (the GELU gradient against its float64 value), each held to the
    element-wise backward tolerance; their absolute floor BWD_ATOL * s, with
    s = max(1, rms(terms)), then also bounds the column sum, accumulated as
    independent errors (times sqrt(rows)).  Without it a column of one row
    would be held to 1e-4 of a gradient value whose own element bound is
    BWD_ATOL * s."""
    ref = np.asarray(ref)
    t = np.asarray(terms, dtype=np.float64)
    l2 = np.sqrt((t * t).sum(axis=0))
    bound = COL_RTOL * (np.abs(ref.astype(np.float64)) + l2)
    floor = 0.0
    if approx_terms and t.size:
        s = max(1.0, float(np.sqrt(np.mean(t * t))))
        floor = BWD_ATOL * s * np.sqrt(t.shape[0])
        bound = bound + floor
    worst = _report(name, np.asarray(gpu), ref, bound)
    colsum_relative(name, gpu, ref, l2, floor)
    return worst


def assert_exact(name, gpu, ref):
    gpu, ref = np.asarray(gpu), np.asarray(ref)
    assert gpu.shape == ref.shape, f"{name}: shape {gpu.shape} vs {ref.shape}"
    same = (gpu.view(np.uint32) == ref.view(np.uint32)) if gpu.dtype == np.float32 else (gpu == ref)
    if not same.all():
        i = np.unravel_index(np.argmin(same), same.shape)
        raise AssertionError(f"{name}: {int((~same).sum())} elements differ bitwise; first at "
                             f"{i}: gpu={gpu[i]!r} ref={ref[i]!r}")


def assert_fwd_within_oracle_error(name, gpu, ref32, ref64):
    ref32 = np.asarray(ref32)
    own = np.abs(ref32.astype(np.float64) - np.asarray(ref64, np.float64))
    bound = FWD_ATOL + FWD_RTOL * np.abs(ref32.astype(np.float64)) + own
    return _report(name, np.asarray(gpu), ref32, bound)


def assert_bwd_within_oracle_error(name, gpu, ref32, ref64):
    ref32 = np.asarray(ref32)
    r64 = ref32.astype(np.float64)
    s = max(1.0, float(np.sqrt(np.mean(r64 * r64)))) if r64.size else 1.0
    own = np.abs(r64 - np.asarray(ref64, np.float64))
    bound = BWD_ATOL * s + BWD_RTOL * np.abs(r64) + own
    return _report(name, np.asarray(gpu), ref32, bound)
