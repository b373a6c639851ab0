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


def pow2_factors(rng, n, dt, contiguous=True):
    """Factors +-2^k whose products are exact in Float32 and Float64, so a
    product scan or reduction can be compared bit for bit. contiguous=True
    (scans, which only multiply contiguous runs): every factor is 2 or 1/2
    and the running exponent is a triangle wave in [-20, 20], so any dropped,
    repeated or reordered factor changes an exponent. contiguous=False
    (reductions, whose partial products cover strided subsets): about 8
    factors are +-2 or +-1/2, the rest +-1. Signs are random."""
    i = np.arange(n + 1)
    if contiguous:
        e = 20 - np.abs(((i + 20) % 80) - 40)   # e[0] = 0
        k = np.diff(e)
    else:
        k = rng.choice([-1, 1], n) * (rng.random(n) < 8.0 / n)
    return (rng.choice([-1.0, 1.0], n) * np.exp2(k)).astype(dt)


def product_rtol(dt, n):
    """Forward error bound of any product of n floating-point factors
    (n - 1 roundings): |computed - exact| <= gamma_{n-1} |exact| with
    gamma_m = m u / (1 - m u), u = 2^-24 (Float32) or 2^-53 (Float64)."""
    u = 2.0 ** -24 if np.dtype(dt) == np.float32 else 2.0 ** -53
    m = max(n - 1, 1)
    return m * u / (1 - m * u)


# The quaternion group Q8 = {+-1, +-i, +-j, +-k} as (s, v1, v2, v3): its
# products stay in the group and are exact in any float type, and it is
# non-commutative (i j = k, j i = -k), so a scan of Q8 elements checks the
# order of every product bit for bit.
Q8 = np.array([[1, 0, 0, 0], [-1, 0, 0, 0], [0, 1, 0, 0], [0, -1, 0, 0],
               [0, 0, 1, 0], [0, 0, -1, 0], [0, 0, 0, 1], [0, 0, 0, -1]], np.float64)


def q8_sequence(rng, n, dt):
    return Q8[rng.integers(0, 8, n)].astype(dt)


def quat_as_complex2(q):
    """2x2 complex matrices of quaternions (s, v1, v2, v3): s + v1 i + v2 j
    + v3 k -> [[s + v1 i, v2 + v3 i], [-v2 + v3 i, s - v1 i]], an algebra
    homomorphism, so matrix products are quaternion products."""
    q = np.asarray(q, np.float64)
    m = np.empty(q.shape[:-1] + (2, 2), np.complex128)
    m[..., 0, 0] = q[..., 0] + 1j * q[..., 1]
    m[..., 0, 1] = q[..., 2] + 1j * q[..., 3]
    m[..., 1, 0] = -q[..., 2] + 1j * q[..., 3]
    m[..., 1, 1] = q[..., 0] - 1j * q[..., 1]
    return m


def complex2_as_quat(m):
    return np.stack([m[..., 0, 0].real, m[..., 0, 0].imag, m[..., 0, 1].real, m[..., 0, 1].imag], -1)
