"""Parity metrics shared by the tests.

The reference's own metric (tests/gpu_parity.rs:45-55) is a pointwise
max relative error with denominator max(|x|, |y|, 1e-6).  Pointwise relative
error is ill-conditioned for outputs near zero (any two fp32 summation orders
differ there), so the gates at the BASELINE sizes are normalised:

* GEMM: max_ij |C − C64|_ij / (|A|·|B|)_ij   (componentwise error bound)
        and ‖C − C64‖_F / ‖C64‖_F,           both against a float64 product;
* attention / model tensors: ‖x − r‖_F / ‖r‖_F and max|x − r| / max|r|.
"""
import numpy as np


def max_rel_err(a, b) -> float:
    """tests/gpu_parity.rs:45-55 — pointwise, denominator max(|a|,|b|,1e-6)."""
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    den = np.maximum(np.maximum(np.abs(a), np.abs(b)), 1e-6)
    return float(np.max(np.abs(a - b) / den)) if a.size else 0.0


def fro_rel(x, ref) -> float:
    x = np.asarray(x, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(x - ref) / den) if den > 0 else float(np.linalg.norm(x))


def max_norm_rel(x, ref) -> float:
    x = np.asarray(x, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    den = np.max(np.abs(ref)) if ref.size else 0.0
    err = np.max(np.abs(x - ref)) if ref.size else 0.0
    return float(err / den) if den > 0 else float(err)


def componentwise(c, c64, bound) -> float:
    """max |c − c64| / bound, bound = |A|·|B| (float64), guarded at 0."""
    c = np.asarray(c, np.float64)
    bound = np.maximum(np.asarray(bound, np.float64), 1e-30)
    return float(np.max(np.abs(c - c64) / bound))
