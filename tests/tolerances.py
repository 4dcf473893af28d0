"""Parity tolerance for fp32-accumulated outputs.

Accumulated outputs may differ from the reference's sequential f32 sums only by
summation order. The bar: per output
    |got - want| <= max(1e-2 * |want|, 2 bf16 ulps of |want|, 1e-5 * sum_k |w_k x_k|)
The last term covers outputs that cancel to near zero, where a relative bound
is meaningless; it is the magnitude-scaled bound the reference's own hybrid
tests use (crates/stark-engine/src/engine/hybrid/weight_metal.rs:2390-2395 allows
2e-5 * max(sum|w x|, 1)), tightened by 2x.
"""
import numpy as np

REL = 1e-2
ULPS = 2
ABS_SCALE = 1e-5


def bf16_ulp(v):
    v = np.abs(np.asarray(v, np.float64))
    e = np.floor(np.log2(np.maximum(v, 2.0 ** -126)))
    return 2.0 ** (e - 7)


def check(got, want, mag=None, label=""):
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    assert got.shape == want.shape, f"{label}: shape {got.shape} vs {want.shape}"
    nan_g, nan_w = np.isnan(got), np.isnan(want)
    assert np.array_equal(nan_g, nan_w), f"{label}: NaN pattern differs"
    g, w = got[~nan_w], want[~nan_w]
    tol = np.maximum(REL * np.abs(w), ULPS * bf16_ulp(w))
    if mag is not None:
        tol = np.maximum(tol, ABS_SCALE * np.asarray(mag, np.float64).ravel()[~nan_w])
    err = np.abs(g - w)
    bad = err > tol
    if bad.any():
        i = int(np.argmax(err - tol))
        raise AssertionError(f"{label}: {int(bad.sum())}/{bad.size} outside tolerance; worst idx {i} "
                             f"got {g[i]!r} want {w[i]!r} tol {tol[i]!r}")
    return float((err / np.maximum(np.abs(w), 1e-30)).max()) if err.size else 0.0
