"""Comparison helpers shared by the parity tests."""
import numpy as np


def bits(a):
    a = np.asarray(a)
    return a.view({8: np.uint64, 4: np.uint32, 2: np.uint16, 1: np.uint8}[a.dtype.itemsize])


def assert_bit_equal(got, want, what=""):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    bad = np.nonzero(bits(got).ravel() != bits(want).ravel())[0]
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[:5]}: " \
                          f"{got.ravel()[bad[:5]]} vs {want.ravel()[bad[:5]]}"


def rel_err(got, want):
    """max|got - want| / max|want| over the whole tensor (NaN-safe: both NaN = equal)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    both_nan = np.isnan(got) & np.isnan(want)
    d = np.where(both_nan, 0.0, np.abs(got - want))
    scale = np.max(np.abs(np.where(np.isnan(want), 0, want))) if want.size else 0.0
    if not np.all(np.isfinite(d)):
        return np.inf
    return float(d.max() / scale) if scale > 0 else float(d.max())


def tol_for_k(k):
    """The stated forward/backward tolerance: 1e-5 relative, 1e-4 when K >= 8192."""
    return 1e-4 if k >= 8192 else 1e-5


def assert_close(got, want, k, what=""):
    e = rel_err(got, want)
    assert e <= tol_for_k(k), f"{what}: rel err {e:.3e} > {tol_for_k(k):.0e} (K={k})"
    return e
