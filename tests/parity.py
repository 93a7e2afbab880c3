"""Parity metric for fp32 outputs against the fp64 oracle.

BASELINE's contract: final fp32 outputs within max relative error 1e-3
(reduction-order differences).  Gated:
  normwise    max_i |y_i - r_i| / max_j |r_j|
  elementwise max_i |y_i - r_i| / |r_i| over outputs with |r_i| >= 1e-3 * max_j |r_j|
Reported only: the raw elementwise maximum (outputs near zero make it meaningless:
at K = 4096, sigma_w = 0.02, y ~ N(0, 1.28^2) and ~0.3 % of outputs are < 5e-3).
"""
import numpy as np

TOL = 1e-3


def parity(y, ref) -> dict:
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    assert y.shape == r.shape, (y.shape, r.shape)
    scale = float(np.max(np.abs(r))) if r.size else 0.0
    err = np.abs(y - r)
    if scale == 0.0:
        return {"normwise": float(np.max(err)) if err.size else 0.0, "elementwise": 0.0, "raw": 0.0}
    mask = np.abs(r) >= 1e-3 * scale
    rel = err[mask] / np.abs(r[mask])
    return {
        "normwise": float(np.max(err) / scale),
        "elementwise": float(np.max(rel)) if rel.size else 0.0,
        "raw": float(np.max(err / np.maximum(np.abs(r), 1e-30))),
    }


def assert_parity(y, ref, tol: float = TOL, label: str = "") -> dict:
    p = parity(y, ref)
    assert np.all(np.isfinite(y)), f"{label}: non-finite output"
    assert p["normwise"] <= tol and p["elementwise"] <= tol, f"{label}: {p}"
    return p
