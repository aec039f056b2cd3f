"""Tolerance checks shared by the config-size GPU parity tests.

The bar of the path is a maximum relative error of 2e-3 against the fp32/fp64-accumulated
reference result on the same inputs.  Two statements of it are checked together:
- norm-wise: max|y - ref| / max|ref| < tol (the whole output vector as the scale);
- element-wise: |y - ref| <= tol * (|ref| + rms(ref)) for every element, so that an element of
  typical magnitude is within tol of its own value, and only elements far below the typical
  magnitude (where a relative error is undefined) are held to an absolute bound of tol * rms.
"""
import numpy as np


def errors(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    d = np.abs(y - ref)
    scale = np.abs(ref).max()
    rms = float(np.sqrt(np.mean(ref * ref)))
    norm = float(d.max() / max(scale, 1e-30))
    elem = float((d / (np.abs(ref) + rms + 1e-30)).max())
    return norm, elem


def assert_close(y, ref, tol=2e-3, what=""):
    y = np.asarray(y, np.float64)
    assert np.all(np.isfinite(y)), f"{what}: non-finite output"
    norm, elem = errors(y, ref)
    assert norm < tol and elem < tol, f"{what}: norm-wise {norm:.3e}, element-wise {elem:.3e} (tol {tol})"
