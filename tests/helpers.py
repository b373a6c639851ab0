"""Shared helpers for the test suite (decoding fixtures, tolerances)."""
import numpy as np

NP = {"int32": np.int32, "uint8": np.uint8, "float64": np.float64, "float32": np.float32, "int64": np.int64}


def dec(v, dtype):
    out = []
    for x in v:
        if isinstance(x, str):
            out.append({"nan": np.nan, "inf": np.inf, "-inf": -np.inf}[x])
        else:
            out.append(x)
    return np.array(out, dtype=dtype)


def same_float(a, b):
    """Elementwise equal with NaN == NaN and zero signs compared."""
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    both_nan = np.isnan(a) & np.isnan(b)
    eq = (a == b) & (np.signbit(a) == np.signbit(b))
    return bool(np.all(both_nan | eq))


def assert_close(got, ref, rtol, atol=0.0, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    lim = atol + rtol * np.abs(ref)
    bad = np.nonzero(~(err <= lim))[0]
    if bad.size:
        i = bad[0]
        raise AssertionError(f"{what}: {bad.size} elements out of tolerance (rtol={rtol}, atol={atol}); "
                             f"first at {i}: got {got[i]!r}, expected {ref[i]!r}")


def assert_mixed(got, ref, tol, what=""):
    """|got - ref| <= tol * max(|ref|, 1): the affine-scan criterion (products
    underflow toward 0 and b crosses zero)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    lim = tol * np.maximum(np.abs(ref), 1.0)
    bad = np.nonzero(~(err <= lim))[0]
    if bad.size:
        i = bad[0]
        raise AssertionError(f"{what}: {bad.size} out of tolerance {tol}; first at {i}: "
                             f"got {got[i]!r}, expected {ref[i]!r}")
