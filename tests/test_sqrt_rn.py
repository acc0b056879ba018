"""The correction the RMS factors apply to the hardware square root
(heph_device.h sqrt_rn): from any estimate within one ulp of sqrt(a), the
sign tests a <= d*y and a > u*y pick the correctly rounded root. Checked on
the host against numpy's correctly rounded float32 sqrt, for estimates one
ulp low, exact and one ulp high, over random, boundary and near-midpoint
inputs (float64 holds d*y exactly, so a - d*y has the sign one FMA gives)."""
import numpy as np


def corrected(a, y):
    a64, y32 = np.float64(a), np.float32(y)
    b = y32.view(np.uint32)
    d = np.uint32(b - 1).view(np.float32)
    u = np.uint32(b + 1).view(np.float32)
    if a64 - np.float64(d) * np.float64(y32) <= 0.0:
        return d
    if a64 - np.float64(u) * np.float64(y32) > 0.0:
        return u
    return y32


def inputs():
    rng = np.random.default_rng(0)
    a = rng.random(20000, dtype=np.float32) * np.float32(4.0) + np.float32(1e-3)
    wide = (2.0 ** rng.uniform(-100, 100, 5000)).astype(np.float32)
    # squares of floats and squares of float midpoints sit at the edges
    y = (rng.random(5000, dtype=np.float32) + np.float32(1.0)).astype(np.float32)
    sq = (y.astype(np.float64) ** 2).astype(np.float32)
    mid = ((y.astype(np.float64) + np.spacing(y).astype(np.float64) / 2) ** 2).astype(np.float32)
    near = np.concatenate([np.nextafter(mid, np.float32(0)), mid, np.nextafter(mid, np.float32(9))])
    return np.concatenate([a, wide, sq, near, np.float32([1.0, 2.0, 1e-6, 1.1285120])])


def test_sqrt_rn_picks_the_nearest_root_from_any_one_ulp_estimate():
    bad = []
    for a in inputs():
        want = np.sqrt(a)
        for k in (-1, 0, 1):
            y = np.uint32(want.view(np.uint32) + np.int64(k)).view(np.float32)
            if corrected(a, y) != want:
                bad.append((float(a), k))
    assert not bad, bad[:5]


def test_a_plain_one_ulp_estimate_is_not_enough():
    # without the correction an estimate one ulp off stays off: the test
    # above would catch an implementation that skipped it
    a = np.float32(1.1285120)
    want = np.sqrt(a)
    y = np.uint32(want.view(np.uint32) - 1).view(np.float32)
    assert y != want and corrected(a, y) == want
