"""Shared comparison helpers for the parity tests."""
import numpy as np

CANON_NAN = 0x7FC00000


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def assert_bit_exact(got, want, what):
    g, w = bits(got).ravel(), bits(want).ravel()
    bad = np.nonzero(g != w)[0]
    assert bad.size == 0, (f"{what}: {bad.size} of {g.size} differ; first at {bad[0]}: "
                           f"got {g[bad[0]]:#010x} want {w[bad[0]]:#010x}")


def rel_l2(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    den = np.linalg.norm(want)
    return float(np.linalg.norm(got - want) / (den if den > 0 else 1.0))


# Tolerance stated by the benchmark contract for matmul outputs: 1e-3 relative L2 against
# the fp32 reference path on the same inputs.
REL_L2_TOL = 1e-3


def assert_rel_l2(got, want, what, tol=REL_L2_TOL):
    assert np.array_equal(np.isnan(got), np.isnan(want)), f"{what}: NaN pattern differs"
    fin = ~np.isnan(want)
    e = rel_l2(np.asarray(got)[fin], np.asarray(want)[fin])
    assert e < tol, f"{what}: relative L2 {e:.3e} >= {tol}"
    return e
