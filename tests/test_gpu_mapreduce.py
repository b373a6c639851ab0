"""mapreduce parity on the GPU (full reduction and dims), through the C ABI,
against the pinned CPU oracle. Integers and max/min are exact; float sums
are checked against a Float64 host sum with |err| <= rtol * sum(|f(x)|)
(the error bound of any summation order), rtol stated per test."""
import sys

import numpy as np
import pytest
import torch

from helpers import NP, assert_close, dec, pow2_factors, product_rtol

pytestmark = pytest.mark.gpu

SIZES = list(range(1, 11)) + [33, 100, 1023, 1025, 10001, 100_000, 1 << 20, (1 << 22) + 7]
F = {"identity": None, "abs2": None}


def fmap(kf, f):
    return {"identity": kf.identity, "abs2": kf.abs2}[f]


def gen(rng, dt, n):
    if dt == np.int32:
        return rng.integers(-2**31, 2**31 - 1, n, dtype=np.int64).astype(np.int32)
    if dt == np.int64:
        return rng.integers(-1000, 1000, n).astype(np.int64)
    if dt == np.uint8:
        return rng.integers(0, 256, n).astype(np.uint8)
    return rng.standard_normal(n).astype(dt)


def sum_abs(x, f):
    x = x.astype(np.float64)
    return float(np.sum(x * x if f == "abs2" else np.abs(x)))


@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int32, np.int64, np.uint8])
@pytest.mark.parametrize("op", ["+", "max", "min"])
@pytest.mark.parametrize("f", ["identity", "abs2"])
def test_full_reduce(kf, oracle, dev, dt, op, f):
    rng = np.random.default_rng(31)
    rtol = 1e-6 if dt == np.float32 else 1e-12
    for n in SIZES:
        x = gen(rng, dt, n)
        got = kf.mapreduce(fmap(kf, f), op, torch.from_numpy(x).to(dev))
        ref = oracle.reduce(x, op, f)
        if dt in (np.float32, np.float64) and op == "+":
            assert abs(got - ref) <= rtol * sum_abs(x, f) + 1e-300, (n, got, ref)
        elif dt in (np.float32, np.float64):
            # max/min select an element: exact once the oracle's Float64
            # f(x) is rounded to the element type (exact for abs2 too, as
            # the double product of two floats rounds to the float product)
            assert dt(got) == dt(ref), (n, got, ref)
        else:
            assert got == int(ref), (n, got, ref)


@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int32, np.int64, np.uint8])
def test_product_reduce(kf, oracle, dev, dt):
    # mapreduce(identity, *, x): odd integer factors (wrapping, exact);
    # float factors +-2^k (exact products, compared bit for bit) and factors
    # in [0.999, 1.001] within the forward error bound gamma_{n-1} of a
    # product in any association order
    rng = np.random.default_rng(37)
    for n in SIZES:
        if np.dtype(dt).kind == "f":
            x = pow2_factors(rng, n, dt, contiguous=False)
            got = kf.mapreduce(kf.identity, "*", torch.from_numpy(x).to(dev))
            assert got == oracle.reduce(x, "*"), n
            x = rng.uniform(0.999, 1.001, n).astype(dt)
            got = kf.mapreduce(kf.identity, "*", torch.from_numpy(x).to(dev))
            ref = oracle.reduce(x, "*")
            assert abs(got - ref) <= product_rtol(dt, n) * abs(ref), (n, got, ref)
        else:
            x = 2 * rng.integers(-3, 3, n) + 1
            x = (x % 256).astype(dt) if dt == np.uint8 else x.astype(dt)
            got = kf.mapreduce(kf.identity, "*", torch.from_numpy(x).to(dev))
            assert got == int(oracle.reduce(x, "*")), n
    # along dims, on a column view
    rows, cols = 300, 70
    buf = rng.uniform(0.99, 1.01, (2 * cols, rows)).reshape(-1)
    A = torch.from_numpy(buf).to(dev).as_strided((rows, cols), (1, 2 * rows))
    for dim in (1, 2):
        got = kf.mapreduce(kf.identity, "*", A, dims=dim).reshape(-1).cpu().numpy()
        ref = oracle.reduce_dim(buf, rows, cols, 2 * rows, dim, "*")
        assert_close(got, ref, product_rtol(np.float64, rows if dim == 1 else cols), what=f"dims={dim}")


@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int32])
def test_reference_arange_sums(kf, dev, golden, dt):
    # reference test/tests/mapreduce/mapreduce1d_test.jl:10-55 (sums of 1:n, reused tmp)
    cases = [c for c in golden["reduce"] if c["dtype"] == np.dtype(dt).name and c["x"] == "arange1"]
    assert cases
    src0 = torch.arange(1, 100_001, device=dev).to(getattr(torch, np.dtype(dt).name))
    tmp = kf.get_allocation(kf.MapReduce1D, kf.identity, "+", src0)
    for c in cases:
        x = torch.arange(1, c["n"] + 1, device=dev).to(src0.dtype)
        f = fmap(kf, c["f"])
        for t in (None, tmp):
            got = kf.mapreduce(f, c["op"], x, tmp=t)
            if dt == np.int32:
                assert got == c["expected"]
            else:
                assert abs(got - c["expected"]) <= 1e-6 * c["expected"]
        dst = torch.zeros(1, dtype=x.dtype, device=dev)
        kf.mapreduce_(f, c["op"], dst, x, tmp=tmp)
        if dt == np.int32:
            assert dst.item() == c["expected"]


def test_views_and_strides(kf, oracle, dev):
    # reference test/tests/views/views_test.jl:44-65
    rng = np.random.default_rng(37)
    x = rng.standard_normal(100_003)
    src = torch.from_numpy(x).to(dev)
    for sl in (slice(2, None), slice(1, None), slice(3, -5), slice(None, None, 3), slice(5, None, 7)):
        v = x[sl]
        got = kf.mapreduce(kf.identity, "+", src[sl])
        assert abs(got - oracle.reduce(np.ascontiguousarray(v))) <= 1e-12 * np.abs(v).sum()
        assert kf.mapreduce(kf.identity, min, src[sl]) == v.min()
        assert kf.mapreduce(kf.abs2, "+", src[sl], g=np.sqrt) == pytest.approx(np.sqrt((v * v).sum()), rel=1e-12)


@pytest.mark.parametrize("dt", [np.int32, np.uint8, np.int64, np.float32])
def test_short_stride_views_vector_path(kf, oracle, dev, dt):
    # strided 1-D views whose stride spans at most 32 bytes stream the whole
    # span with 16-byte loads and combine the elements at multiples of the
    # stride: every stride up to that, start offsets that put the 128-byte
    # head at every phase, lengths from a single element to several
    # persistent rounds, + (integers exact) and max
    rng = np.random.default_rng(97)
    es = np.dtype(dt).itemsize
    for stride in range(2, 32 // es + 1):
        for n in (1, 2, 3, 40, 1000, 65_537, 3_000_001 // stride):
            for off in (0, 1, 5):
                flat = (rng.integers(0, 256, n * stride + off + 1).astype(dt) if dt != np.float32 else
                        (rng.random(n * stride + off + 1) < 0.25).astype(dt))
                t = torch.from_numpy(flat).to(dev)
                v = flat[off:off + (n - 1) * stride + 1:stride]
                assert v.shape[0] == n
                got = kf.mapreduce(kf.identity, "+", t[off:off + (n - 1) * stride + 1:stride])
                ref = v.astype(np.int64).sum()
                if dt == np.float32:
                    assert got == float(ref), (stride, n, off)  # sparse 0/1: exact in any order
                else:
                    assert int(got) == int(np.array(ref).astype(dt)), (stride, n, off)
                assert kf.mapreduce(kf.identity, max, t[off:off + (n - 1) * stride + 1:stride]) == v.max(), \
                    (stride, n, off)


def test_full_reduce_of_2d_and_3d(kf, dev):
    # reference test/tests/mapreduce/mapreduce_test.jl:9-28
    rng = np.random.default_rng(41)
    a = rng.random((6, 5, 4)).astype(np.float32)       # torch (6,5,4) C-order == Julia 4x5x6
    x = torch.from_numpy(a).to(dev).permute(2, 1, 0)   # Julia-shaped 4x5x6, column-major
    s = float(a.astype(np.float64).sum())
    assert kf.mapreduce(kf.identity, "+", x) == pytest.approx(s, rel=1e-6)
    assert kf.mapreduce(kf.identity, "+", x, dims=":") == pytest.approx(s, rel=1e-6)
    r = kf.mapreduce(kf.identity, "+", x, dims=(1, 2, 3))
    assert tuple(r.shape) == (1, 1, 1) and r.item() == pytest.approx(s, rel=1e-6)
    # a strided 2-D view that is not one strided vector: two passes
    A = torch.from_numpy(rng.random((64, 33))).to(dev).T   # 33 x 64 column-major
    V = A[:, ::2]
    assert kf.mapreduce(kf.identity, "+", V) == pytest.approx(float(V.sum()), rel=1e-12)


def colmajor(rng, rows, cols, dt, view=False, low=-1.0, high=1.0):
    pc = 2 * cols if view else cols
    if np.dtype(dt).kind == "f":
        parent = rng.uniform(low, high, (pc, rows)).astype(dt)
    else:
        parent = rng.integers(-1000, 1000, (pc, rows)).astype(dt)
    buf = parent.reshape(-1)
    return buf, (2 * rows if view else rows)


@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int32, np.uint8])
@pytest.mark.parametrize("shape", [(128, 64), (1, 64), (128, 1), (1024, 256), (3, 7), (5, 7), (33, 17),
                                   (1, 1), (4096, 3), (7, 5000), (70000, 2), (100_000, 9)])
@pytest.mark.parametrize("view", [False, True])
def test_dims_2d(kf, oracle, dev, dt, shape, view):
    # reference test/tests/mapreduce/mapreduce2d_test.jl:1-47 and
    # test/tests/views/views_test.jl:66-160 (column views)
    rows, cols = shape
    rng = np.random.default_rng(rows * 131 + cols)
    buf, cs = colmajor(rng, rows, cols, dt, view)
    t = torch.from_numpy(buf).to(dev)
    A = t.as_strided((rows, cols), (1, cs))
    for dim in (1, 2):
        for op, f in (("+", "identity"), ("max", "identity"), ("min", "abs2"), ("+", "abs2")):
            if dt == np.uint8 and f == "abs2":
                continue
            got = kf.mapreduce(fmap(kf, f), op, A, dims=dim)
            assert tuple(got.shape) == ((1, cols) if dim == 1 else (rows, 1))
            g = got.reshape(-1).cpu().numpy()
            ref = oracle.reduce_dim(buf, rows, cols, cs, dim, op, f)
            if np.dtype(dt).kind == "f" and op == "+":
                M = buf.astype(np.float64)[np.arange(cols)[None, :] * cs + np.arange(rows)[:, None]]
                M = M * M if f == "abs2" else np.abs(M)
                bound = M.sum(axis=dim - 1) * (1e-6 if dt == np.float32 else 1e-12)
                assert np.all(np.abs(g - ref) <= bound + 1e-300), (dim, op, f)
            elif np.dtype(dt).kind == "f":
                assert np.array_equal(g, ref.astype(dt)), (dim, op, f)
            else:
                assert np.array_equal(g, ref), (dim, op, f)


@pytest.mark.parametrize("dt", [np.int32, np.int64, np.uint8])
@pytest.mark.parametrize("shape", [
    (2_100_000, 5),        # 4-byte: 8-vector strips, 257 of them; column tail
    (1_048_580, 9),        # 4-byte: 4-vector strips, the last one ragged
    (1_000_003, 6),        # 4-byte: 2-vector strips, fewer columns than one pass
    (300_000, 37),         # 1-vector strips, no split
    (70_000, 300),         # 1-vector strips split over column ranges
    (8197, 11, 130),       # batched: 8-vector strips reached through the batch count
])
def test_dims2_strip_widths(kf, dev, dt, shape):
    # The dims=2 launch picks its strip width (16-byte vectors per thread per
    # column) from rows x batch; these shapes reach every width for each
    # element size, with ragged last strips and column tails. Exact: integer
    # sums wrap in the element type, max is order-free.
    rng = np.random.default_rng(sum(shape))
    hi = 256 if dt == np.uint8 else 1 << 20
    a = rng.integers(0, hi, shape[::-1]).astype(dt)            # C order == Julia column-major shape
    x = torch.from_numpy(a).to(dev).permute(*reversed(range(len(shape))))
    xn = x.cpu().numpy()
    for op in ("+", "max"):
        got = kf.mapreduce(kf.identity, op, x, dims=2).cpu().numpy()
        ref = xn.sum(axis=1, keepdims=True, dtype=dt) if op == "+" else xn.max(axis=1, keepdims=True)
        assert got.shape == ref.shape and np.array_equal(got, ref), (shape, op)


def _exact_dims_case(kf, dev, rng, dt, rows, cols, dim, pad=0, ops=("+", "max")):
    # column-major rows x cols with column stride rows + pad; integer sums
    # wrap in the element type, max is order-free: both exact
    hi = 256 if dt == np.uint8 else 1 << 20
    cs = rows + pad
    buf = rng.integers(0, hi, cs * cols).astype(dt)
    A = torch.from_numpy(buf).to(dev).as_strided((rows, cols), (1, cs))
    M = buf.reshape(cols, cs)[:, :rows].T
    for op in ops:
        got = kf.mapreduce(kf.identity, op, A, dims=dim).cpu().numpy().reshape(-1)
        ref = M.sum(axis=dim - 1, dtype=dt) if op == "+" else M.max(axis=dim - 1)
        assert np.array_equal(got, ref), (rows, cols, pad, dim, op)


@pytest.mark.parametrize("dt", [np.int32, np.int64, np.uint8])
def test_dims1_short_columns(kf, dev, dt):
    # Columns of up to 128 vector (256 element) units take L = 1..16 lanes per column
    # (16-byte units when rows is a multiple of the vector width and the
    # columns are aligned, elements otherwise); longer ones one wave each.
    rng = np.random.default_rng(11)
    for rows in (1, 2, 3, 4, 5, 8, 12, 16, 31, 32, 64, 100, 128, 255, 256, 512, 513, 1000, 2048, 2064):
        for pad in (0, 1, 16):
            _exact_dims_case(kf, dev, rng, dt, rows, 3001, 1, pad)


@pytest.mark.parametrize("dt", [np.int32, np.uint8])
@pytest.mark.parametrize("shape", [(1_000_003, 3), (1 << 20, 2), (777_777, 5), (300_001, 17), (65536, 100)])
def test_dims1_few_long_columns(kf, dev, dt, shape):
    # few long columns split into up to 4096 row segments per column; the
    # cols x S partials are combined by the narrow dims=2 kernel
    _exact_dims_case(kf, dev, np.random.default_rng(sum(shape)), dt, *shape, 1)


@pytest.mark.parametrize("dt", [np.int32, np.int64, np.uint8])
def test_dims2_narrow(kf, dev, dt):
    # At most 256 row units: thread (unit, phase) over column phases, split
    # over column ranges whose partials the same kernel combines.
    rng = np.random.default_rng(12)
    for rows in (1, 2, 3, 4, 7, 16, 64, 100, 256, 257, 1000, 1024):
        for cols in (1, 5, 1000, 100_003):
            for pad in (0, 3):
                if rows * cols > 30_000_000:
                    continue
                _exact_dims_case(kf, dev, rng, dt, rows, cols, 2, pad)


@pytest.mark.parametrize("shape", [(16, 1000, 7), (3, 5000, 4), (64, 33, 300), (2, 100_000, 3)])
def test_dims2_narrow_batched(kf, dev, shape):
    # middle-dims reductions with narrow rows: batch in grid.z, split partials per batch
    rng = np.random.default_rng(sum(shape))
    a = rng.integers(-1000, 1000, shape[::-1]).astype(np.int32)
    x = torch.from_numpy(a).to(dev).permute(2, 1, 0)
    xn = x.cpu().numpy()
    for op in ("+", "max"):
        got = kf.mapreduce(kf.identity, op, x, dims=2).cpu().numpy()
        ref = xn.sum(axis=1, keepdims=True, dtype=np.int32) if op == "+" else xn.max(axis=1, keepdims=True)
        assert np.array_equal(got, ref), (shape, op)


def test_dims1_column_count_beyond_one_grid(kf, dev):
    # more columns than one capped grid covers: both dims=1 kernels
    # grid-stride over column blocks (1-lane columns past 8192 x 256 columns;
    # wave-per-column past 65536 x 4)
    rng = np.random.default_rng(13)
    _exact_dims_case(kf, dev, rng, np.uint8, 1, (1 << 26) + 5, 1, ops=("+",))
    _exact_dims_case(kf, dev, rng, np.uint8, 2064, 270_000, 1, ops=("max",))


@pytest.mark.parametrize("dt", [np.int32, np.int64, np.uint8])
def test_dims2_misaligned_base_peeled(kf, dev, dt):
    # A misaligned by k elements with a 16-byte-multiple column stride: the
    # first 16/es - k rows take an element-path launch, the rest the vector
    # paths from an aligned base; plain, batched (grid.z) and matvec forms
    rng = np.random.default_rng(14)
    ev = 16 // np.dtype(dt).itemsize
    hi = 256 if dt == np.uint8 else 1 << 20
    for rows, cols in ((5, 9), (100, 1000), (1000, 77), (5000, 3000), (70_000, 40), (1 << 20, 3)):
        cs = -(-(rows + ev) // ev) * ev
        buf = torch.from_numpy(rng.integers(0, hi, cs * cols + ev).astype(dt)).to(dev)
        for k in sorted({0, 1, ev // 2, ev - 1}):
            A = buf.as_strided((rows, cols), (1, cs), k)
            M = A.cpu().numpy()
            for op in ("+", "max"):
                got = kf.mapreduce(kf.identity, op, A, dims=2).cpu().numpy().reshape(-1)
                ref = M.sum(axis=1, dtype=dt) if op == "+" else M.max(axis=1)
                assert np.array_equal(got, ref), (rows, cols, k, op)
    # batched: Julia rows x cols x nb with a 16-byte-multiple batch stride
    rows, cols, nb = 37, 50, 6
    cs = -(-(rows + ev) // ev) * ev
    buf = torch.from_numpy(rng.integers(0, hi, cs * cols * nb + ev).astype(dt)).to(dev)
    X = buf.as_strided((rows, cols, nb), (1, cs, cs * cols), 1)
    got = kf.mapreduce(kf.identity, "+", X, dims=2).cpu().numpy()
    assert np.array_equal(got, X.cpu().numpy().sum(axis=1, keepdims=True, dtype=dt))
    if dt != np.uint8:
        x = torch.from_numpy(rng.integers(-5, 5, cols).astype(dt)).to(dev)
        A = buf[: cs * cols + ev].as_strided((rows, cols), (1, cs), 2)
        got = kf.matvec(A, x).cpu().numpy()
        ref = (A.cpu().numpy() * x.cpu().numpy()[None, :]).sum(axis=1, dtype=dt)
        assert np.array_equal(got, ref)


def test_vecmat_scratch_contract_with_misaligned_operand(kf, dev):
    # The C ABI decides scratch from the alignment the launch uses (here the
    # misaligned x sends vecmat to the element path). A shape whose launch
    # splits its rows is refused without scratch, on the host, before any
    # launch; one that does not split runs without scratch; both are exact
    # with the queried scratch.
    import ctypes
    L = sys.modules["kernelforge_amd._lib"]
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    for rows, cols, splits in ((100_000, 40, True), (512, 40, False)):
        A = torch.randint(-9, 9, (cols, rows), dtype=torch.int32, device=dev).T
        x = torch.randint(-9, 9, (rows + 1,), dtype=torch.int32, device=dev)[1:]
        dst = torch.zeros(cols, dtype=torch.int32, device=dev)
        args = (L.OP_ADD, L.MAP2_MUL, L.I32, P(A), rows, cols, rows, 1, P(x), 1, P(dst), 1)
        ref = (A.cpu().numpy().astype(np.int64) * x.cpu().numpy()[:, None]).sum(axis=0).astype(np.int32)
        rc = L.lib().kf_reduce_dim_x(*args, None, 0, stream)
        if splits:
            assert rc == L.KF_ENOSCRATCH
        else:
            assert rc == L.KF_OK and np.array_equal(dst.cpu().numpy(), ref)
        need = L.lib().kf_reduce_dim_scratch_bytes(L.I32, rows, cols, 1)
        tmp = torch.zeros(need, dtype=torch.uint8, device=dev)
        dst.zero_()
        assert L.lib().kf_reduce_dim_x(*args, P(tmp), need, stream) == L.KF_OK
        assert np.array_equal(dst.cpu().numpy(), ref), (rows, cols)


def test_dims_golden(kf, dev, golden):
    for c in golden["reduce_dim"]:
        buf = dec(c["buf"], np.float64)
        t = torch.from_numpy(buf).to(dev)
        A = t.as_strided((c["rows"], c["cols"]), (1, c["col_stride"]))
        assert_close(kf.mapreduce(kf.identity, "+", A, dims=1).reshape(-1).cpu().numpy(),
                     dec(c["dim1"], np.float64), 1e-12, 1e-12, what="golden dim1")
        assert_close(kf.mapreduce(kf.identity, "+", A, dims=2).reshape(-1).cpu().numpy(),
                     dec(c["dim2"], np.float64), 1e-12, 1e-12, what="golden dim2")
        assert np.array_equal(kf.mapreduce(kf.identity, max, A, dims=1).reshape(-1).cpu().numpy(),
                              dec(c["dim1_max"], np.float64))
        assert np.array_equal(kf.mapreduce(kf.identity, min, A, dims=2).reshape(-1).cpu().numpy(),
                              dec(c["dim2_min"], np.float64))


@pytest.mark.parametrize("dims", [1, (1, 2), 3, (2, 3), (1, 3), (1, 2, 3)])
def test_dims_nd_routing(kf, dev, dims):
    # reference test/tests/mapreduce/mapreduce_test.jl:30-131
    rng = np.random.default_rng(43)
    a = rng.random((6, 5, 8))                            # C-order (6,5,8) == Julia 8x5x6
    x = torch.from_numpy(a).to(dev).permute(2, 1, 0)     # Julia 8x5x6
    got = kf.mapreduce(kf.identity, "+", x, dims=dims)
    d = (dims,) if isinstance(dims, int) else dims
    ref = x.cpu().numpy().sum(axis=tuple(k - 1 for k in d), keepdims=True)
    assert tuple(got.shape) == ref.shape
    np.testing.assert_allclose(got.cpu().numpy(), ref, rtol=1e-12)


@pytest.mark.parametrize("dims,same", [(-1, 3), ((-1, 1), (1, 3)), (-3, 1), ((-2, -1), (2, 3))])
def test_negative_dims_count_from_the_end(kf, dev, dims, same):
    # reference src/helpers.jl:194-198: d <= 0 means dim nd + d + 1
    rng = np.random.default_rng(47)
    x = torch.from_numpy(rng.integers(-9, 9, (6, 5, 8)).astype(np.int64)).to(dev).permute(2, 1, 0)
    got = kf.mapreduce(kf.identity, "+", x, dims=dims)
    ref = kf.mapreduce(kf.identity, "+", x, dims=same)
    assert torch.equal(got, ref)


def test_dims_errors(kf, dev):
    x = torch.zeros(4, 5, device=dev).T
    with pytest.raises(kf.ArgumentError):
        kf.mapreduce(kf.identity, "+", x, dims=3)
    with pytest.raises(kf.ArgumentError):
        kf.mapreduce(kf.identity, "+", x, dims=(1, 1))
    with pytest.raises(kf.ArgumentError):
        kf.mapreduce(kf.identity, kf.affine, x)
    with pytest.raises(kf.ArgumentError):
        kf.mapreduce(kf.identity, "+", (x, x), dims=1)   # multi-array: full reduction only


# ---- BASELINE.json configurations at full size -------------------------------
def test_config3a_abs2_sum_f32_2pow30(kf, oracle, dev):
    g = torch.Generator(device=dev).manual_seed(20261201 + 3)
    x = torch.randn(2**30, device=dev, generator=g, dtype=torch.float32)
    got = kf.mapreduce(kf.abs2, "+", x)
    ref = oracle.reduce(x.cpu().numpy(), "+", "abs2")
    assert abs(got - ref) <= 1e-5 * ref, (got, ref)  # rel tol 1e-5 vs the Float64 host sum


def test_config3b_abs2_sum_f64_2pow28(kf, oracle, dev):
    g = torch.Generator(device=dev).manual_seed(20261201 + 31)
    x = torch.randn(2**28, device=dev, generator=g, dtype=torch.float64)
    got = kf.mapreduce(kf.abs2, "+", x)
    ref = oracle.reduce(x.cpu().numpy(), "+", "abs2")
    assert abs(got - ref) <= 1e-10 * ref, (got, ref)  # the host Float64 sum itself errs ~sqrt(n)*eps


def test_config3c_int32_max_2pow28(kf, oracle, dev):
    rng = np.random.default_rng(20261201 + 32)
    x = rng.integers(-2**31, 2**31 - 1, 2**28, dtype=np.int64).astype(np.int32)
    t = torch.from_numpy(x).to(dev)
    assert kf.mapreduce(kf.identity, max, t) == oracle.reduce(x, "max")
    assert kf.mapreduce(kf.identity, min, t) == oracle.reduce(x, "min")


@pytest.mark.parametrize("which", ["dims1", "dims2", "dims1_view", "dims2_view"])
def test_config5_dims(kf, oracle, dev, which):
    g = torch.Generator(device=dev).manual_seed(20261201 + 5)
    if which.startswith("dims1"):
        rows, cols, dim = 4096, 65536, 1
    else:
        rows, cols, dim = 65536, 4096, 2
    t = torch.rand(rows * cols, device=dev, generator=g) * 2 - 1
    A = t.as_strided((rows, cols), (1, rows))
    if which.endswith("view"):
        A = A[:, ::2]
    kcols = A.shape[1]
    got = kf.mapreduce(kf.identity, "+", A, dims=dim).reshape(-1).cpu().numpy()
    buf = t.cpu().numpy()
    cs = A.stride(1)
    ref = oracle.reduce_dim(buf, rows, kcols, cs, dim)
    absA = np.abs(buf.astype(np.float64))
    absA = absA.reshape(cols, rows)[:: (2 if which.endswith("view") else 1)]  # (kcols, rows)
    bound = absA.sum(axis=1 if dim == 1 else 0) * 1e-6
    assert np.all(np.abs(got - ref) <= bound), which


@pytest.mark.parametrize("dt", [np.int32, np.int64, np.uint8])
def test_multilevel_full_reduce_exact(kf, oracle, dev, dt):
    # every launch regime of the vector path, at its edges, with aligned and
    # unaligned starts (exact integer results): one launch of one-shot
    # workgroups at 2 and 4 vectors per lane (2048 * 256 * 2 vectors), the
    # same just past 128 MiB (one-shot level 0 + folding level 1), and from
    # 256 MiB the persistent chunked single launch: whole rounds only, and
    # (2^24 + 5000 vectors) chunks rounded up to whole rounds, so one
    # workgroup ends in a partial round and the last 682 get no vectors
    rng = np.random.default_rng(47)
    epv = 16 // np.dtype(dt).itemsize
    for n in (2048 * 512 * epv - 1, 2048 * 512 * epv + 5, 2048 * 256 * 16 * epv + 5, 2**24 * epv + 3,
              (2**24 + 5000) * epv + 7):
        print(f"multilevel {np.dtype(dt).name} n={n}", flush=True)
        x = gen(rng, dt, n + 3)
        t = torch.from_numpy(x).to(dev)
        for off in (0, 1, 3):
            v = x[off:off + n]
            for op in ("+", "max"):
                assert kf.mapreduce(kf.identity, op, t[off:off + n]) == int(oracle.reduce(v, op)), (n, off, op)


@pytest.mark.parametrize("shape,dims", [
    ((8, 5, 6), 2),                  # middle dim (the reference's mapreducedims fallback)
    ((4, 5, 6, 7), (2, 3)),          # middle block
    ((4, 5, 6, 7, 3), (2, 4)),       # two separate blocks, neither at an end
    ((3, 4, 5, 6, 7), (1, 3, 5)),    # three blocks
    ((64, 33, 40), 2),               # larger middle reduction (vector path, splits)
    ((1000, 7, 3), 2),
    ((5, 1, 4), 2),                  # size-1 reduced dim
])
@pytest.mark.parametrize("dt", [np.float64, np.int32])
def test_general_dims(kf, dev, shape, dims, dt):
    # reference test/tests/mapreduce/mapreducedims_test.jl: any dims set
    rng = np.random.default_rng(53)
    a = (rng.integers(-50, 50, shape[::-1]) if dt == np.int32 else rng.standard_normal(shape[::-1])).astype(dt)
    x = torch.from_numpy(a).to(dev).permute(*reversed(range(len(shape))))   # Julia-shaped, column-major
    d = (dims,) if isinstance(dims, int) else dims
    axes = tuple(k - 1 for k in d)
    xn = x.cpu().numpy()
    for f, op, ref in (("identity", "+", xn.sum(axis=axes, keepdims=True)),
                       ("abs2", "+", (xn * xn).sum(axis=axes, keepdims=True)),
                       ("identity", "max", xn.max(axis=axes, keepdims=True))):
        got = kf.mapreduce(fmap(kf, f), op, x, dims=dims)
        assert tuple(got.shape) == ref.shape
        if dt == np.int32:
            assert np.array_equal(got.cpu().numpy(), ref.astype(np.int32)), (f, op)
        else:
            np.testing.assert_allclose(got.cpu().numpy(), ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int32, np.int64, np.uint8])
def test_two_array_mapreduce(kf, oracle, dev, dt):
    # reference test/tests/mapreduce/mapreduce1d_test.jl:231-319 (dot products,
    # distances, g = sqrt); exact for integers, rtol * sum|f| for floats
    import operator
    rng = np.random.default_rng(59)
    for n in (1, 7, 33, 4097, 100_003, (1 << 22) + 5):
        x, y = gen(rng, dt, n), gen(rng, dt, n)
        tx, ty = torch.from_numpy(x).to(dev), torch.from_numpy(y).to(dev)
        for f, name in ((operator.mul, "mul"), (kf.sqdiff, "sqdiff")):
            for op in ("+", "max"):
                got = kf.mapreduce(f, op, (tx, ty))
                ref = oracle.reduce2(x, y, op, name)
                if np.dtype(dt).kind == "f" and op == "+":
                    xf, yf = x.astype(np.float64), y.astype(np.float64)
                    bound = np.sum(np.abs(xf * yf) if name == "mul" else (xf - yf) ** 2)
                    tol = 1e-6 if dt == np.float32 else 1e-12
                    assert abs(got - ref) <= tol * bound + 1e-300, (n, name, got, ref)
                elif np.dtype(dt).kind == "f" and name == "mul":
                    assert dt(got) == dt(ref), (n, name, op)   # one rounding: exact
                elif np.dtype(dt).kind == "f":
                    # (x-y)^2 rounds twice in the element type, once in the oracle
                    assert got == pytest.approx(ref, rel=1e-6 if dt == np.float32 else 1e-15), (n, name, op)
                else:
                    assert got == int(ref), (n, name, op)
        # strided / unaligned operands take the scalar path
        if n > 8:
            got = kf.mapreduce(operator.mul, "+", (tx[1::2], ty[:-1:2]))
            ref = oracle.reduce2(x[1::2], y[:-1:2], "+", "mul")
            if np.dtype(dt).kind != "f":
                assert got == int(ref)
    # g = sqrt: Euclidean distance
    x = rng.random(15_000)
    y = rng.random(15_000)
    d = kf.mapreduce(kf.sqdiff, "+", (torch.from_numpy(x).to(dev), torch.from_numpy(y).to(dev)), g=np.sqrt)
    assert d == pytest.approx(np.sqrt(np.sum((x - y) ** 2)), rel=1e-12)


@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int32, np.int64, np.uint8])
def test_three_array_mapreduce(kf, oracle, dev, dt):
    # reference test/tests/mapreduce/mapreduce1d_test.jl:180-194: sum(a .* b .* c)
    # and cbrt(sum(a .* b .* c)); exact for integers, floats within
    # 2 roundings of each product plus the sum's rtol * sum|a b c|
    rng = np.random.default_rng(61)
    for n in (1, 5, 33, 4097, 12_000, 100_003, (1 << 22) + 3):
        x, y, z = gen(rng, dt, n), gen(rng, dt, n), gen(rng, dt, n)
        t = [torch.from_numpy(a).to(dev) for a in (x, y, z)]
        for op in ("+", "max"):
            got = kf.mapreduce(kf.prod3, op, tuple(t))
            ref = oracle.reduce3(x, y, z, op)
            if np.dtype(dt).kind == "f":
                bound = np.sum(np.abs(x.astype(np.float64) * y * z)) if op == "+" else abs(ref)
                tol = 1e-6 if dt == np.float32 else 1e-12
                assert abs(got - ref) <= tol * bound + 1e-300, (n, op, got, ref)
            else:
                assert got == int(ref), (n, op)
        if n > 8:   # strided operands take the scalar path
            got = kf.mapreduce(kf.prod3, "+", (t[0][1::2], t[1][:-1:2], t[2][::2][: len(x[1::2])]))
            ref = oracle.reduce3(x[1::2], y[:-1:2], z[::2][: len(x[1::2])])
            if np.dtype(dt).kind != "f":
                assert got == int(ref), n
    # the reference's cases: U[0,1) of length 12000, g = cbrt; the
    # lower-level names with a reused buffer
    import operator
    a, b, c = (rng.random(12_000) for _ in range(3))
    ta, tb, tc = (torch.from_numpy(v).to(dev) for v in (a, b, c))
    assert kf.mapreduce1d(operator.mul, "+", (ta, tb, tc)) == pytest.approx(np.sum(a * b * c), rel=1e-12)
    tmp = kf.get_allocation(kf.MapReduce1D, kf.prod3, "+", (ta, tb, tc))
    r = kf.mapreduce1d(kf.prod3, "+", (ta, tb, tc), g=np.cbrt, tmp=tmp)
    assert r == pytest.approx(np.cbrt(np.sum(a * b * c)), rel=1e-12)
    d = torch.empty(1, dtype=torch.float64, device=dev)
    kf.mapreduce1d_(kf.prod3, "+", d, (ta, tb, tc), tmp=tmp)
    assert d.item() == pytest.approx(np.sum(a * b * c), rel=1e-12)


@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int32, np.int64])
def test_two_array_weighted_squares_and_expdiff(kf, oracle, dev, dt):
    # reference test/tests/mapreduce/mapreduce1d_test.jl:117-131:
    # sum(w .* x .^ 2) (n = 50000) and sum(exp.(a .- b)) (n = 10000, a, b in
    # [0, 2)); exact for integers, floats within rtol * the sum of |terms|
    # (each term rounds at most 3 times in the element type, exp within a few ulps)
    rng = np.random.default_rng(67)
    tol = 1e-6 if dt == np.float32 else 1e-12
    for n in (1, 9, 4097, 50_000, (1 << 21) + 1):
        w, x = gen(rng, dt, n), gen(rng, dt, n)
        tw, tx = torch.from_numpy(w).to(dev), torch.from_numpy(x).to(dev)
        got = kf.mapreduce1d(kf.wsq, "+", (tw, tx))
        ref = oracle.reduce2(w, x, "+", "wsq")
        if np.dtype(dt).kind == "f":
            bound = np.sum(np.abs(w.astype(np.float64) * x * x))
            assert abs(got - ref) <= tol * bound + 1e-300, (n, got, ref)
        else:
            assert got == int(ref), n
    if np.dtype(dt).kind != "f":
        with pytest.raises(kf.ArgumentError):
            kf.mapreduce1d(kf.expdiff, "+", (tw, tx))
        return
    for n in (1, 10_000, 1 << 20):
        a, b = (rng.random(n) * 2).astype(dt), (rng.random(n) * 2).astype(dt)
        got = kf.mapreduce1d(kf.expdiff, "+", (torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)))
        ref = oracle.reduce2(a, b, "+", "expdiff")
        assert abs(got - ref) <= 4 * tol * ref, (n, got, ref)
    # the matvec / vecmat entry point takes the symmetric maps only
    A = torch.ones(8, 4, dtype=torch.from_numpy(a).dtype, device=dev)
    with pytest.raises(kf.ArgumentError):
        kf.matvec(kf.wsq, "+", A.T, torch.ones(8, dtype=A.dtype, device=dev))


def test_post_map_g(kf, dev):
    # reference test/tests/mapreduce/mapreduce2d_test.jl:30-35: abs2 + g = sqrt row norms
    import math
    rng = np.random.default_rng(61)
    a = rng.standard_normal((64, 128))                     # C-order (64,128) == Julia 128x64
    A = torch.from_numpy(a).to(dev).T
    An = A.cpu().numpy()
    got = kf.mapreduce(kf.abs2, "+", A, dims=2, g=math.sqrt).reshape(-1).cpu().numpy()
    np.testing.assert_allclose(got, np.sqrt((An ** 2).sum(axis=1)), rtol=1e-13)
    got = kf.mapreduce(kf.identity, "+", A, dims=1, g=kf.abs2).reshape(-1).cpu().numpy()
    np.testing.assert_allclose(got, An.sum(axis=0) ** 2, rtol=1e-12)
    dst = torch.zeros(1, dtype=torch.float64, device=dev)
    kf.mapreduce_(kf.abs2, "+", dst, A, g="sqrt")
    assert dst.item() == pytest.approx(np.sqrt((An ** 2).sum()), rel=1e-13)
    # scan!(f, op, dst, src; g): g applied to every prefix
    x = torch.from_numpy(rng.random(10_001)).to(dev)
    y = kf.scan("+", x, g=torch.sqrt).cpu().numpy()
    np.testing.assert_allclose(y, np.sqrt(np.cumsum(x.cpu().numpy())), rtol=1e-12)
    with pytest.raises(kf.ArgumentError):
        kf.mapreduce(kf.identity, "+", A, dims=1, g=lambda v: v / 2)   # arbitrary g only on host scalars
    assert kf.mapreduce(kf.identity, "+", x, g=lambda v: v / 2) == pytest.approx(x.sum().item() / 2, rel=1e-12)


def test_one_reduction_buffer_across_kinds_and_levels(kf, oracle, dev):
    # One MapReduce buffer serves full reductions of one, two and three
    # levels, two-array reductions, strided reductions and split dims
    # reductions, in interleaved order, three times: any state a call left
    # in the buffer that a later call relied on would corrupt a result.
    import operator
    rng = np.random.default_rng(101)
    buf = kf.KernelBuffer(kf.MapReduce1D, 64 << 20, dev)
    sizes = (1000, 300_000, 524_288, 524_289, (1 << 22) + 3, (1 << 24) + 5)
    xs = {n: gen(rng, np.int32, n) for n in sizes}
    ts = {n: torch.from_numpy(x).to(dev) for n, x in xs.items()}
    rows, cols = 65536, 64
    a = gen(rng, np.int32, rows * cols)
    A = torch.from_numpy(a).to(dev).view(cols, rows).T          # column-major rows x cols
    for rep in range(3):
        for n in sizes:
            for op in ("+", "max"):
                got = kf.mapreduce(kf.identity, op, ts[n], tmp=buf)
                assert got == int(oracle.reduce(xs[n], op)), (rep, n, op)
            y = ts[n].flip(0).contiguous()
            got = kf.mapreduce(operator.mul, "+", (ts[n], y), tmp=buf)
            assert got == int(oracle.reduce2(xs[n], xs[n][::-1].copy(), "+", "mul")), (rep, n)
            got = kf.mapreduce(kf.identity, "+", ts[n][::3], tmp=buf)
            assert got == int(oracle.reduce(xs[n][::3], "+")), (rep, n, "strided")
            for dim in (1, 2):
                got = kf.mapreduce(kf.identity, "+", A, dims=dim, tmp=buf).cpu().numpy().ravel()
                ref = oracle.reduce_dim(a, rows, cols, rows, dim, "+")
                assert np.array_equal(got, ref), (rep, n, dim)


def test_scan_buffer_is_refused_for_reductions(kf, dev):
    x = torch.arange(100, dtype=torch.int32, device=dev)
    sbuf = kf.get_allocation(kf.Scan1D, kf.identity, "+", x)
    with pytest.raises(kf.ArgumentError):
        kf.mapreduce(kf.identity, "+", x, tmp=sbuf)
    rbuf = kf.KernelBuffer(kf.MapReduce1D, 1 << 20, dev)
    with pytest.raises(kf.ArgumentError):
        kf.scan_("+", torch.empty_like(x), x, tmp=rbuf)


@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int32, np.uint8])
def test_maximum_minimum(kf, oracle, dev, dt):
    # reference src/mapreduce/reductions.jl (maximum(src), minimum(src),
    # maximum!(rel, dst, src)), on views as test/tests/views/views_test.jl:62-63
    # does with min; exact: max/min select an input
    import operator
    rng = np.random.default_rng(151)
    for n in (1, 33, 10001, 1_000_003):
        x = gen(rng, dt, n + 2)
        t = torch.from_numpy(x).to(dev)
        assert kf.maximum(t) == x.max()
        assert kf.minimum(t) == x.min()
        assert kf.minimum(t[2:]) == x[2:].min()
        assert kf.maximum(operator.gt, t[1:-1]) == x[1:-1].min()
        out = torch.empty(1, dtype=t.dtype, device=dev)
        kf.maximum_(operator.lt, out, t)
        assert out.item() == x.max()
    with pytest.raises(kf.ArgumentError):
        kf.maximum(operator.le, torch.ones(3, device=dev))


def test_lower_level_entry_points(kf, oracle, dev):
    # the names the reference's tests call besides mapreduce/mapreduce!:
    # mapreduce1d(!), mapreduce2d(!), mapreducedims(!) (mapreduce1d_test.jl,
    # mapreduce2d_test.jl, mapreducedims_test.jl); exact on Int32
    import operator
    rng = np.random.default_rng(163)
    x = gen(rng, np.int32, 100_003)
    y = gen(rng, np.int32, 100_003)
    tx, ty = torch.from_numpy(x).to(dev), torch.from_numpy(y).to(dev)
    assert kf.mapreduce1d(kf.identity, "+", tx) == int(oracle.reduce(x, "+"))
    d = kf.mapreduce1d(kf.abs2, "max", tx, to_cpu=False)
    assert d.device.type == "cuda" and d.shape == (1,) and d.item() == int(oracle.reduce(x, "max", "abs2"))
    out = torch.zeros(3, dtype=torch.int32, device=dev)
    kf.mapreduce1d_(operator.mul, "+", out, (tx, ty))
    assert out[0].item() == int(oracle.reduce2(x, y, "+", "mul")) and out[1:].eq(0).all()
    assert kf.mapreduce1d(operator.mul, "+", (tx, ty)) == int(oracle.reduce2(x, y, "+", "mul"))
    rows, cols = 300, 170
    a = gen(rng, np.int32, rows * cols)
    A = torch.from_numpy(a).to(dev).view(cols, rows).T
    for dim in (1, 2):
        ref = oracle.reduce_dim(a, rows, cols, rows, dim, "+")
        assert np.array_equal(kf.mapreduce2d(kf.identity, "+", A, dim).cpu().numpy(), ref), dim
        dst = torch.empty(ref.shape[0], dtype=torch.int32, device=dev)
        kf.mapreduce2d_(kf.identity, "+", dst, A, dim)
        assert np.array_equal(dst.cpu().numpy(), ref), dim
    with pytest.raises(kf.ArgumentError):
        kf.mapreduce2d(kf.identity, "+", A, 3)
    B = torch.from_numpy(gen(rng, np.int32, 6 * 7 * 8)).to(dev).view(8, 7, 6).permute(2, 1, 0)  # column-major 6x7x8
    ref = B.cpu().numpy().astype(np.int64).sum(axis=(0, 2), keepdims=True).astype(np.int32)
    got = kf.mapreducedims(kf.identity, "+", B, (1, 3))
    assert tuple(got.shape) == (1, 7, 1) and np.array_equal(got.cpu().numpy(), ref)
    dst = torch.empty(1, 7, 1, dtype=torch.int32, device=dev)
    kf.mapreducedims_(kf.identity, "+", dst, B, (1, 3))
    assert np.array_equal(dst.cpu().numpy(), ref)


@pytest.mark.parametrize("dt", [np.float32, np.int32])
def test_multi_array_chunked_large(kf, oracle, dev, dt):
    # from 1 GiB of operands the multi-array reductions run the persistent
    # chunk kernel (2048 workgroups over contiguous chunks of every array,
    # folded in the same launch); ragged lengths leave a scalar tail for
    # workgroup 0. Exact for integers (wrapping), rtol * sum|f| for floats.
    import operator
    rng = np.random.default_rng(67)
    for k, n in ((2, (1 << 27) + 5), (3, 100_000_003)):
        arrs = [gen(rng, dt, n) for _ in range(k)]
        t = tuple(torch.from_numpy(a).to(dev) for a in arrs)
        for op in ("+", "max"):
            got = kf.mapreduce(operator.mul if k == 2 else kf.prod3, op, t)
            ref = oracle.reduce2(arrs[0], arrs[1], op, "mul") if k == 2 else oracle.reduce3(*arrs, op)
            if dt == np.float32 and op == "+":
                p = arrs[0].astype(np.float64) * arrs[1]
                if k == 3:
                    p = p * arrs[2]
                assert abs(got - ref) <= 1e-6 * np.sum(np.abs(p)), (k, n, op, got, ref)
            elif dt == np.float32:
                assert got == pytest.approx(ref, rel=1e-6), (k, n, op)
            else:
                assert got == int(ref), (k, n, op)
        del t
