"""Pins the CPU oracle (oracle/kf_oracle.c) before any GPU result is checked
against it: golden vectors computed independently with numpy / plain Python,
closed forms, and the special cases Julia's operators define."""
import numpy as np
import pytest

from helpers import NP, dec, same_float


def test_scan_golden(oracle, golden):
    for c in golden["scan"]:
        dt = NP[c["dtype"]]
        x = dec(c["x"], dt)
        for mode in ("inclusive", "exclusive"):
            got = oracle.scan(x, c["op"], exclusive=mode == "exclusive")
            exp = dec(c[mode], np.float64 if dt == np.float64 else dt)
            if dt == np.float64:
                if c.get("signed_zero"):
                    assert same_float(got, exp), (c["op"], mode, got, exp)
                else:
                    # numpy's cumsum adds in the same left-to-right order: equal bits
                    assert same_float(got, exp), (c["dtype"], c["op"], c["n"], mode)
            else:
                assert np.array_equal(got, exp), (c["dtype"], c["op"], c["n"], mode)


def test_affine_golden(oracle, golden):
    for c in golden["affine"]:
        ab = np.stack([dec(c["a"], np.float32), dec(c["b"], np.float32)], axis=1)
        for mode in ("inclusive", "exclusive"):
            got = oracle.scan(ab, "affine", exclusive=mode == "exclusive")
            assert np.array_equal(got, np.array(c[mode], np.float64)), (c["n"], mode)


def test_reduce_golden(oracle, golden):
    for c in golden["reduce"]:
        dt = NP[c["dtype"]]
        x = np.arange(1, c["n"] + 1).astype(dt) if c["x"] == "arange1" else dec(c["x"], dt)
        got = oracle.reduce(x, c["op"], c["f"])
        assert got == c["expected"], (c, got)


def test_reduce_dim_golden(oracle, golden):
    for c in golden["reduce_dim"]:
        buf = dec(c["buf"], np.float64)
        r, k, cs = c["rows"], c["cols"], c["col_stride"]
        np.testing.assert_allclose(oracle.reduce_dim(buf, r, k, cs, 1), dec(c["dim1"], np.float64), rtol=1e-14)
        np.testing.assert_allclose(oracle.reduce_dim(buf, r, k, cs, 2), dec(c["dim2"], np.float64), rtol=1e-14)
        assert np.array_equal(oracle.reduce_dim(buf, r, k, cs, 1, "max"), dec(c["dim1_max"], np.float64))
        assert np.array_equal(oracle.reduce_dim(buf, r, k, cs, 2, "min"), dec(c["dim2_min"], np.float64))


# ---- closed forms and invariants -------------------------------------------
@pytest.mark.parametrize("n", [1, 2, 17, 4096, 100_003])
def test_scan_closed_forms(oracle, n):
    ones = np.ones(n, np.int32)
    assert np.array_equal(oracle.scan(ones), np.arange(1, n + 1, dtype=np.int32))
    assert np.array_equal(oracle.scan(ones, exclusive=True), np.arange(0, n, dtype=np.int32))
    r = np.arange(1, n + 1, dtype=np.int64)
    tri = r * (r + 1) // 2
    assert np.array_equal(oracle.scan(r), tri)
    # abs2 map: running sum of squares
    assert np.array_equal(oracle.scan(r, "+", "abs2"), r * (r + 1) * (2 * r + 1) // 6)
    # max of an increasing sequence is itself; min of it is the first element
    assert np.array_equal(oracle.scan(r, "max"), r)
    assert np.array_equal(oracle.scan(r, "min"), np.ones(n, np.int64))


def test_scan_int_wraps(oracle):
    x = np.array([2**31 - 1, 1, 1], np.int32)
    assert oracle.scan(x).tolist() == [2**31 - 1, -2**31, -2**31 + 1]
    u = np.array([250, 10, 255], np.uint8)
    assert oracle.scan(u).tolist() == [250, 4, 3]
    assert oracle.scan(u, "+", "abs2").tolist() == [(250 * 250) % 256, (250 * 250 + 100) % 256,
                                                    (250 * 250 + 100 + 255 * 255) % 256]


def _wrap_signed(v, bits):
    v %= 1 << bits
    return v - (1 << bits) if v >= 1 << (bits - 1) else v


@pytest.mark.parametrize("n", [1, 2, 12, 13, 21, 40, 1000])
def test_product_scan_closed_forms(oracle, n):
    # scan!(*) of 1:n is n!, exact in Python integers and then wrapped to the
    # element width (Julia Int32/Int64/UInt8 `*` wrap around)
    facts, f = [], 1
    for k in range(1, n + 1):
        f *= k
        facts.append(f)
    for dt, bits, signed in ((np.int32, 32, True), (np.int64, 64, True), (np.uint8, 8, False)):
        x = np.arange(1, n + 1).astype(dt)
        want = [(_wrap_signed(v, bits) if signed else v % (1 << bits)) for v in facts]
        assert oracle.scan(x, "*").tolist() == want, (dt, n)
        exc = oracle.scan(x, "*", exclusive=True)
        assert exc[0] == 1 and exc[1:].tolist() == want[:-1]
        assert int(oracle.reduce(x, "*")) == want[-1]
    # powers of two are exact in binary floating point
    for dt in (np.float32, np.float64):
        k = min(n, 1000)
        got = oracle.scan(np.full(k, 2.0, dt), "*")
        assert np.array_equal(got, 2.0 ** np.arange(1, k + 1, dtype=np.float64))
        got = oracle.scan(np.full(k, 0.5, dt), "*", exclusive=True)
        assert np.array_equal(got, 0.5 ** np.arange(0, k, dtype=np.float64))


def test_product_scan_matches_numpy(oracle):
    # the reference's product-scan test draws U[0, 1) (scan_test.jl:1-19); numpy's
    # cumprod in Float64 is an independent left-to-right product
    rng = np.random.default_rng(5)
    x = rng.uniform(0.9, 1.1, 4097)
    assert np.allclose(oracle.scan(x, "*"), np.cumprod(x), rtol=1e-12, atol=0)
    assert np.isclose(oracle.reduce(x, "*"), np.prod(x), rtol=1e-12)
    xf = x.astype(np.float32)
    assert np.allclose(oracle.scan(xf, "*"), np.cumprod(xf.astype(np.float64)), rtol=1e-12, atol=0)


def test_pow2_product_fixtures_are_exact(oracle):
    # the GPU product tests compare bit for bit on these factors: every
    # prefix (scan) or subset (reduction) product must be a representable
    # power of two, here checked against the exponent and sign sums
    import sys, os
    sys.path.insert(0, os.path.dirname(__file__))
    from helpers import pow2_factors, product_rtol
    rng = np.random.default_rng(3)
    for dt in (np.float32, np.float64):
        for n in (1, 7, 4097, 1_000_000):
            x = pow2_factors(rng, n, dt)
            e = np.cumsum(np.log2(np.abs(x.astype(np.float64))))
            sgn = np.cumprod(np.sign(x.astype(np.float64)))
            assert np.abs(e).max() <= 20
            assert np.array_equal(oracle.scan(x, "*"), sgn * np.exp2(e))
            y = pow2_factors(rng, n, dt, contiguous=False)
            assert np.abs(np.log2(np.abs(y.astype(np.float64)))).sum() <= 60
            assert oracle.reduce(y, "*") == np.prod(np.sign(y)) * np.exp2(np.log2(np.abs(y.astype(np.float64))).sum())
    # the error bound covers a float32 pairwise tree of near-1 factors (whose
    # rounding drifts one way: about -8e-5 at 10^5)
    x = rng.uniform(0.999, 1.001, 100_000).astype(np.float32)
    y = x.copy()
    while y.size > 1:
        y = np.append(y, np.float32(1)) if y.size % 2 else y
        y = (y[0::2] * y[1::2]).astype(np.float32)
    exact = oracle.reduce(x, "*")
    assert abs(float(y[0]) - exact) <= product_rtol(np.float32, x.size) * abs(exact)


def test_quaternion_scan_pins(oracle):
    import sys, os
    sys.path.insert(0, os.path.dirname(__file__))
    from helpers import Q8, q8_sequence, quat_as_complex2, complex2_as_quat
    one, i, j, k = Q8[0], Q8[2], Q8[4], Q8[6]
    # Hamilton's rules: i j = k, j k = i, k i = j, j i = -k, i^2 = -1
    for a, b, want in ((i, j, k), (j, k, i), (k, i, j), (j, i, -k), (i, i, -one), (k, j, -i)):
        assert np.array_equal(oracle.scan(np.stack([a, b]), "*")[1], want)
    # Q8 sequences: exact, and equal to running products of the 2x2 complex
    # representation (an independent formula for the same algebra)
    rng = np.random.default_rng(9)
    for dt in (np.float32, np.float64):
        q = q8_sequence(rng, 2000, dt)
        got = oracle.scan(q, "*")
        m = quat_as_complex2(q)
        run = np.eye(2, dtype=np.complex128)
        want = np.empty((len(q), 4))
        for t in range(len(q)):
            run = run @ m[t]
            want[t] = complex2_as_quat(run)
        assert np.array_equal(got, want)
        exc = oracle.scan(q, "*", exclusive=True)
        assert np.array_equal(exc[0], one) and np.array_equal(exc[1:], got[:-1])
    # random quaternions: matrix representation within rounding, norms
    # multiply, and the order matters
    q = rng.standard_normal((500, 4))
    q *= rng.uniform(0.9, 1.1, (500, 1)) / np.linalg.norm(q, axis=1, keepdims=True)
    got = oracle.scan(q, "*")
    m = quat_as_complex2(q)
    run = np.eye(2, dtype=np.complex128)
    norms = np.cumprod(np.linalg.norm(q, axis=1))
    for t in range(len(q)):
        run = run @ m[t]
        assert np.linalg.norm(got[t] - complex2_as_quat(run)) <= 1e-12 * norms[t]
    assert np.allclose(np.linalg.norm(got, axis=1), norms, rtol=1e-12)
    assert not np.allclose(oracle.scan(q[::-1], "*")[-1], got[-1])


@pytest.mark.parametrize("n", [1, 2, 100, 1000, 40_000])
def test_reduce3_closed_forms(oracle, n):
    # sum_{i<=n} i*i*i = (n(n+1)/2)^2 (Nicomachus), exact in Int64 and, wrapped,
    # in Int32; max of an increasing product is the last one
    r = np.arange(1, n + 1, dtype=np.int64)
    want = (n * (n + 1) // 2) ** 2
    assert int(oracle.reduce3(r, r, r)) == want
    r32 = r.astype(np.int32)
    w32 = want % (1 << 32)
    assert int(oracle.reduce3(r32, r32, r32)) == (w32 - (1 << 32) if w32 >= 1 << 31 else w32)
    assert int(oracle.reduce3(r, r, r, "max")) == n ** 3
    rng = np.random.default_rng(n)
    a, b, c = rng.random((3, n))
    assert np.isclose(oracle.reduce3(a, b, c), np.sum(a * b * c), rtol=1e-12)


def test_reduce2_weighted_squares_and_expdiff(oracle):
    # sum_i i * i^2 = (n(n+1)/2)^2 (exact integers); exp(x - y) against numpy;
    # exp(x - x) = 1, so the sum is n exactly
    n = 3000
    r = np.arange(1, n + 1, dtype=np.int64)
    assert int(oracle.reduce2(r, r, "+", "wsq")) == (n * (n + 1) // 2) ** 2
    rng = np.random.default_rng(12)
    w, x = rng.random((2, n))
    assert np.isclose(oracle.reduce2(w, x, "+", "wsq"), np.sum(w * x * x), rtol=1e-12)
    a, b = rng.random((2, n)) * 2
    assert np.isclose(oracle.reduce2(a, b, "+", "expdiff"), np.sum(np.exp(a - b)), rtol=1e-12)
    assert oracle.reduce2(a, a, "+", "expdiff") == n


def test_exclusive_is_shifted_inclusive(oracle):
    rng = np.random.default_rng(1)
    for dt, op, ident in ((np.int32, "max", np.iinfo(np.int32).min), (np.int32, "min", np.iinfo(np.int32).max),
                          (np.int64, "+", 0), (np.uint8, "min", 255)):
        x = rng.integers(0, 100, 999).astype(dt)
        inc, exc = oracle.scan(x, op), oracle.scan(x, op, exclusive=True)
        assert exc[0] == ident and np.array_equal(exc[1:], inc[:-1])


def test_julia_max_min_special_values(oracle):
    # Julia: max(-0.0, 0.0) == 0.0, min(0.0, -0.0) == -0.0, NaN propagates
    x = np.array([-0.0, 0.0], np.float64)
    assert not np.signbit(oracle.scan(x, "max")[1])
    y = np.array([0.0, -0.0], np.float64)
    assert np.signbit(oracle.scan(y, "min")[1])
    z = np.array([1.0, np.nan, 5.0], np.float64)
    assert np.isnan(oracle.scan(z, "max")[2]) and np.isnan(oracle.reduce(z, "min"))


def test_affine_closed_forms(oracle):
    n = 1000
    rng = np.random.default_rng(2)
    b = rng.standard_normal(n).astype(np.float32)
    # a = 1: x_t is the prefix sum of b
    ab = np.stack([np.ones(n, np.float32), b], 1)
    out = oracle.scan(ab, "affine")
    np.testing.assert_allclose(out[:, 1], np.cumsum(b.astype(np.float64)), rtol=1e-12, atol=1e-12)
    assert np.all(out[:, 0] == 1.0)
    # b = 0: the a-component is the running product
    a = rng.uniform(0.9, 1.0, n).astype(np.float32)
    out = oracle.scan(np.stack([a, np.zeros(n, np.float32)], 1), "affine")
    np.testing.assert_allclose(out[:, 0], np.cumprod(a.astype(np.float64)), rtol=1e-12)
    assert np.all(out[:, 1] == 0.0)
    # constant a, b = 1: geometric series x_t = (1 - a^t) / (1 - a)
    a0 = np.float32(0.5)
    out = oracle.scan(np.stack([np.full(60, a0), np.ones(60, np.float32)], 1), "affine")
    t = np.arange(1, 61)
    np.testing.assert_allclose(out[:, 1], (1 - 0.5**t) / 0.5, rtol=1e-14)
    # non-commutativity: swapping two elements changes the result
    p = np.array([[2, 1], [3, 5]], np.float32)
    assert oracle.scan(p, "affine")[1].tolist() == [6.0, 3 * 1 + 5]
    assert oracle.scan(p[::-1], "affine")[1].tolist() == [6.0, 2 * 5 + 1]


@pytest.mark.parametrize("n", [1, 33, 100, 10001, 100000])
def test_reduce_closed_forms(oracle, n):
    for dt in (np.float32, np.float64, np.int32, np.int64):
        x = np.arange(1, n + 1).astype(dt)
        tri = n * (n + 1) // 2
        if dt == np.int32:
            tri = int(np.uint32(tri % 2**32).astype(np.int32))
        assert oracle.reduce(x) == tri
        assert oracle.reduce(x, "max") == n and oracle.reduce(x, "min") == 1
    u = np.full(n, 3, np.uint8)
    assert oracle.reduce(u) == (3 * n) % 256


def test_reduce_matches_numpy(oracle):
    rng = np.random.default_rng(3)
    x = rng.standard_normal(100_000).astype(np.float32)
    np.testing.assert_allclose(oracle.reduce(x, "+", "abs2"), np.sum(x.astype(np.float64) ** 2), rtol=1e-12)
    i = rng.integers(-2**31, 2**31 - 1, 100_000).astype(np.int32)
    assert oracle.reduce(i, "max") == i.max() and oracle.reduce(i, "min") == i.min()


def test_reduce_dim_matches_numpy_fortran(oracle):
    rng = np.random.default_rng(4)
    rows, cols = 37, 23
    A = np.asfortranarray(rng.standard_normal((rows, 2 * cols)))
    buf = A.reshape(-1, order="F")
    V = A[:, ::2]  # view(A, :, 1:2:end): col_stride = 2*rows
    np.testing.assert_allclose(oracle.reduce_dim(buf, rows, cols, 2 * rows, 1), V.sum(0), rtol=1e-13)
    np.testing.assert_allclose(oracle.reduce_dim(buf, rows, cols, 2 * rows, 2), V.sum(1), rtol=1e-13)
    np.testing.assert_allclose(oracle.reduce_dim(buf, rows, cols, 2 * rows, 2, "+", "abs2"), (V**2).sum(1),
                               rtol=1e-13)
    I = rng.integers(-1000, 1000, (rows, cols)).astype(np.int32)
    ib = I.reshape(-1, order="F")
    assert np.array_equal(oracle.reduce_dim(ib, rows, cols, rows, 1), I.sum(0).astype(np.int32))
    assert np.array_equal(oracle.reduce_dim(ib, rows, cols, rows, 2, "max"), I.max(1))


def test_cpu_baseline_agrees(oracle):
    rng = np.random.default_rng(5)
    x = rng.random(200_000, dtype=np.float32)
    ref = oracle.scan(x)
    y1 = np.empty_like(x)
    y4 = np.empty_like(x)
    oracle.baseline_scan_add_f32(x, y1, 1)
    oracle.baseline_scan_add_f32(x, y4, 4)
    np.testing.assert_allclose(y1, ref, rtol=1e-4)
    np.testing.assert_allclose(y4, ref, rtol=1e-4)
    s = oracle.reduce(x)
    assert abs(oracle.baseline_sum_f32(x, 1) - s) <= 1e-4 * s
    assert abs(oracle.baseline_sum_f32(x, 4) - s) <= 1e-4 * s


@pytest.mark.parametrize("threads", [1, 3, 16])
@pytest.mark.parametrize("n", [5, 100_003])
def test_cpu_baselines_of_every_config(oracle, threads, n):
    # the timed CPU paths of C2-C5 against numpy (ragged chunks, and fewer
    # elements than threads at n = 5)
    rng = np.random.default_rng(n + threads)
    xi = rng.integers(-2**31, 2**31 - 1, n).astype(np.int32)
    for excl in (False, True):
        y = np.empty_like(xi)
        oracle.baseline_scan_add_i32(xi, y, excl, threads)
        incl = np.cumsum(xi, dtype=np.int32)  # numpy's int32 cumsum wraps like Julia's Int32 +
        ref = np.concatenate([[0], incl[:-1]]).astype(np.int32) if excl else incl
        assert np.array_equal(y, ref), (excl, threads)
    assert oracle.baseline_max_i32(xi, threads) == int(xi.max())
    xf = rng.standard_normal(n).astype(np.float32)
    assert abs(oracle.baseline_sum_abs2(xf, threads) - float((xf.astype(np.float64) ** 2).sum())) <= 1e-5 * n
    xd = rng.standard_normal(n)
    assert abs(oracle.baseline_sum_abs2(xd, threads) - float((xd ** 2).sum())) <= 1e-12 * n
    # affine: a constant a = 1/2 and b = 1 give x_t = 2 - 2^(1-t) (closed
    # form), and random pairs agree with the Float64 checker
    ab = np.tile(np.array([[0.5, 1.0]], np.float32), (n, 1))
    out = np.empty_like(ab)
    oracle.baseline_scan_affine_f32(ab, out, threads)
    t = np.arange(1, n + 1)
    np.testing.assert_allclose(out[:, 1], 2.0 - 2.0 ** (1.0 - t), rtol=1e-6)
    np.testing.assert_allclose(out[:, 0], 0.5 ** np.minimum(t, 200), rtol=1e-6, atol=1e-37)
    ab = np.stack([rng.uniform(0.9, 1.0, n), rng.standard_normal(n)], 1).astype(np.float32)
    oracle.baseline_scan_affine_f32(ab, out, threads)
    ref = oracle.scan(ab, "affine")
    assert np.all(np.abs(out - ref) <= 1e-4 * np.maximum(np.abs(ref), 1))


@pytest.mark.parametrize("threads", [1, 4])
def test_cpu_baseline_dims_matches_numpy(oracle, threads):
    rng = np.random.default_rng(threads)
    rows, cols = 37, 53
    M = rng.uniform(-1, 1, (rows, 2 * cols)).astype(np.float32)
    buf = M.reshape(-1, order="F")
    for cs, view in ((rows, M[:, :cols]), (2 * rows, M[:, ::2])):
        # the plain matrix (col stride = rows) and every second column
        b = buf if cs == 2 * rows else M[:, :cols].reshape(-1, order="F")
        for dim, ref in ((1, view.astype(np.float64).sum(0)), (2, view.astype(np.float64).sum(1))):
            out = np.empty(cols if dim == 1 else rows, np.float32)
            oracle.baseline_sum_dims_f32(b, rows, cols, cs, dim, out, threads)
            np.testing.assert_allclose(out, ref, rtol=1e-4, atol=1e-5)


def test_reduce2_matches_numpy_and_closed_forms(oracle):
    rng = np.random.default_rng(6)
    x = rng.standard_normal(10_000)
    y = rng.standard_normal(10_000)
    np.testing.assert_allclose(oracle.reduce2(x, y), np.dot(x, y), rtol=1e-12)
    np.testing.assert_allclose(oracle.reduce2(x, y, "+", "sqdiff"), np.sum((x - y) ** 2), rtol=1e-12)
    assert oracle.reduce2(x, y, "max") == np.max(x * y)
    n = 1000
    r = np.arange(1, n + 1, dtype=np.int64)
    assert oracle.reduce2(r, r) == n * (n + 1) * (2 * n + 1) // 6          # sum of squares
    assert oracle.reduce2(r, r - 1, "+", "sqdiff") == n                     # unit differences
    i = np.array([2**16, 3], np.int32)
    assert oracle.reduce2(i, i) == np.int32(9)                              # 2^32 wraps to 0


def test_matvec_vecmat_oracle_matches_numpy(oracle):
    rng = np.random.default_rng(8)
    rows, cols = 29, 17
    A = np.asfortranarray(rng.standard_normal((rows, 2 * cols)))
    buf = A.reshape(-1, order="F")
    V = A[:, ::2]
    x2, x1 = rng.standard_normal(cols), rng.standard_normal(rows)
    np.testing.assert_allclose(oracle.reduce_dim_x(buf, rows, cols, 2 * rows, x2, 2), V @ x2, rtol=1e-12)
    np.testing.assert_allclose(oracle.reduce_dim_x(buf, rows, cols, 2 * rows, x1, 1), x1 @ V, rtol=1e-12)
    np.testing.assert_allclose(oracle.reduce_dim_x(buf, rows, cols, 2 * rows, x2, 2, "+", "sqdiff"),
                               ((V - x2[None, :]) ** 2).sum(1), rtol=1e-12)
    I = rng.integers(-9, 9, (rows, cols)).astype(np.int32)
    xi = rng.integers(-9, 9, cols).astype(np.int32)
    assert np.array_equal(oracle.reduce_dim_x(I.reshape(-1, order="F"), rows, cols, rows, xi, 2), I @ xi)
    assert np.array_equal(oracle.reduce_dim_x(I.reshape(-1, order="F"), rows, cols, rows, xi, 2, "max"),
                          (I * xi[None, :]).max(1))
