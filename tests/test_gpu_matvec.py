"""matvec / vecmat with a vector operand on the GPU against the oracle
(reference test/tests/mapreduce/matvec_test.jl, vecmat_test.jl shape sweeps:
square, tall, wide, small and large n; views). Integers exact; floats within
rtol * sum|f| (the bound of any summation order)."""
import operator

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1), (3, 3), (101, 101), (512, 512), (1000, 1000), (1024, 10), (4096, 32), (65536, 16),
          (3, 10_000), (32, 50_000), (4, 1000), (63, 1000), (2048, 1000), (32768, 50),
          (8, 300_000), (12, 100_000), (300_000, 3), (100, 20_000),
          # one row (matvec) / one column (vecmat): the 1-D dot-product route
          (1, 3), (1, 100_003), (1, 2**20 + 5), (5, 1), (200_001, 1)]


def mk(rng, dt, shape):
    if np.dtype(dt).kind == "f":
        return rng.random(shape).astype(dt)
    return rng.integers(-20, 20, shape).astype(dt)


@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int32])
@pytest.mark.parametrize("view", [False, True])
def test_matvec_vecmat(kf, oracle, dev, dt, view):
    rng = np.random.default_rng(71)
    for rows, cols in SHAPES:
        pc = 2 * cols if view else cols
        parent = mk(rng, dt, (pc, rows))           # row k of parent = column k of the matrix
        buf = parent.reshape(-1)
        cs = 2 * rows if view else rows
        A = torch.from_numpy(buf).to(dev).as_strided((rows, cols), (1, cs))
        x2, x1 = mk(rng, dt, cols), mk(rng, dt, rows)
        tx2, tx1 = torch.from_numpy(x2).to(dev), torch.from_numpy(x1).to(dev)
        M = buf.astype(np.float64)[np.arange(cols)[None, :] * cs + np.arange(rows)[:, None]]
        for name, f in (("mul", operator.mul), ("sqdiff", kf.sqdiff)):
            for dim, fn, x, tx in ((2, kf.matvec, x2, tx2), (1, kf.vecmat, x1, tx1)):
                args = (tx, A) if dim == 1 else (A, tx)
                got = fn(f, "+", *args).cpu().numpy()
                ref = oracle.reduce_dim_x(buf, rows, cols, cs, x, dim, "+", name)
                if np.dtype(dt).kind == "f":
                    xv = x.astype(np.float64)
                    T = M * (xv[None, :] if dim == 2 else xv[:, None]) if name == "mul" else \
                        (M - (xv[None, :] if dim == 2 else xv[:, None])) ** 2
                    bound = np.abs(T).sum(axis=1 if dim == 2 else 0) * (1e-6 if dt == np.float32 else 1e-12)
                    assert np.all(np.abs(got - ref) <= bound + 1e-300), (rows, cols, name, dim)
                else:
                    assert np.array_equal(got, ref), (rows, cols, name, dim)


def test_api_forms_and_errors(kf, dev):
    rng = np.random.default_rng(73)
    a = rng.random((40, 30))                                   # Julia 30 x 40
    A = torch.from_numpy(a).to(dev).T
    x = torch.from_numpy(rng.random(40)).to(dev)
    y = torch.from_numpy(rng.random(30)).to(dev)
    An = A.cpu().numpy()
    np.testing.assert_allclose(kf.matvec(A, x).cpu().numpy(), An @ x.cpu().numpy(), rtol=1e-12)
    np.testing.assert_allclose(kf.vecmat(y, A).cpu().numpy(), y.cpu().numpy() @ An, rtol=1e-12)
    dst = torch.zeros(30, dtype=torch.float64, device=dev)
    kf.matvec_(operator.mul, "+", dst, A, x)
    np.testing.assert_allclose(dst.cpu().numpy(), An @ x.cpu().numpy(), rtol=1e-12)
    dst2 = torch.zeros(40, dtype=torch.float64, device=dev)
    kf.vecmat_(dst2, y, A)
    np.testing.assert_allclose(dst2.cpu().numpy(), y.cpu().numpy() @ An, rtol=1e-12)
    # x = nothing: plain row / column reductions; g = sqrt: row norms
    np.testing.assert_allclose(kf.matvec(A, None).cpu().numpy(), An.sum(1), rtol=1e-12)
    np.testing.assert_allclose(kf.matvec(kf.abs2, "+", A, None, g="sqrt").cpu().numpy(),
                               np.sqrt((An ** 2).sum(1)), rtol=1e-12)
    np.testing.assert_allclose(kf.vecmat(None, A).cpu().numpy(), An.sum(0), rtol=1e-12)
    with pytest.raises(kf.ArgumentError):
        kf.matvec(A, y)                                        # wrong length
    with pytest.raises(kf.ArgumentError):
        kf.matvec(A, x.float())                                # mixed types


def test_get_allocation_kinds_reference_order(kf, oracle, dev):
    # reference get_allocation(MatVec, f, op, A, x), get_allocation(VecMat, f, op, x, A)
    # (matvec.jl:182, vecmat.jl:265) and get_allocation(MapReduce1D, f, op, (x, y), blocks)
    # (mapreduce1d_test.jl:161); each buffer is reused for several calls
    rng = np.random.default_rng(173)
    rows, cols = 3000, 40
    a = rng.integers(-20, 20, (cols, rows)).astype(np.int32)
    A = torch.from_numpy(a).to(dev).T                  # column-major rows x cols
    xr = torch.from_numpy(rng.integers(-20, 20, rows).astype(np.int32)).to(dev)
    xc = torch.from_numpy(rng.integers(-20, 20, cols).astype(np.int32)).to(dev)
    tmv = kf.get_allocation(kf.MatVec, operator.mul, "+", A, xc)
    tvm = kf.get_allocation(kf.VecMat, operator.mul, "+", xr, A)
    M = a.T.astype(np.int64)
    for _ in range(3):
        got = kf.matvec(operator.mul, "+", A, xc, tmp=tmv).cpu().numpy()
        assert np.array_equal(got, (M @ xc.cpu().numpy().astype(np.int64)).astype(np.int32))
        got = kf.vecmat(operator.mul, "+", xr, A, tmp=tvm).cpu().numpy()
        assert np.array_equal(got, (xr.cpu().numpy().astype(np.int64) @ M).astype(np.int32))
    x = torch.from_numpy(rng.integers(-9, 9, 100_001).astype(np.int32)).to(dev)
    y = torch.from_numpy(rng.integers(-9, 9, 100_001).astype(np.int32)).to(dev)
    t2 = kf.get_allocation(kf.MapReduce1D, operator.mul, "+", (x, y), 1000)
    ref = int((x.cpu().numpy().astype(np.int64) * y.cpu().numpy()).sum())
    for _ in range(3):
        assert kf.mapreduce(operator.mul, "+", (x, y), tmp=t2) == ref


@pytest.mark.parametrize("dt", [np.int32, np.uint8, np.float64])
def test_single_row_or_column_dims_route(kf, oracle, dev, dt):
    # mapreduce(f, op, A; dims) over one row (dims=2) or one column (dims=1)
    # is handed to the 1-D reduction: contiguous, strided (column stride of a
    # view) and element-offset operands, against numpy (integers exact)
    rng = np.random.default_rng(79)
    for n in (1, 7, 4099, 1_000_003):
        for off in (0, 1):
            flat = mk(rng, dt, 2 * n + 2)
            t = torch.from_numpy(flat).to(dev)
            for dims, shape, strides, take in ((2, (1, n), (1, 1), flat[off:off + n]),
                                               (2, (1, n), (1, 2), flat[off:off + 2 * n:2]),
                                               (1, (n, 1), (1, n), flat[off:off + n])):
                A = t[off:].as_strided(shape, strides)
                for op, npf in (("+", np.sum), (max, np.max)):
                    got = kf.mapreduce(kf.identity, op, A, dims=dims).cpu().numpy().reshape(-1)
                    if np.dtype(dt).kind == "f":
                        ref = npf(take.astype(np.float64))
                        assert abs(got[0] - ref) <= 1e-12 * max(1.0, np.abs(take).sum()), (n, off, dims, op)
                    else:
                        ref = npf(take.astype(np.int64)) if op == "+" else npf(take)
                        assert int(got[0]) == int(np.array(ref).astype(dt)), (n, off, dims, op)


@pytest.mark.parametrize("dt", [np.uint8, np.int32, np.int64])
def test_short_contiguous_columns_flat_path(kf, oracle, dev, dt):
    # dims=1 over contiguous matrices with columns of at most 2 KiB: blocks of
    # whole columns staged through LDS (column counts that leave a ragged
    # last block, rows that are and are not a multiple of the vector width,
    # every lanes-per-column choice), vecmat and plain mapreduce, exact
    rng = np.random.default_rng(83)
    es = np.dtype(dt).itemsize
    for rows in (1, 2, 3, 5, 10, 16, 17, 63, 100, 127, 2048 // es - 1, 2048 // es, 2048 // es + 1):
        for cols in (1, 7, 4099, 100_003 // max(1, rows // 8)):
            buf = mk(rng, dt, rows * cols)
            A = torch.from_numpy(buf).to(dev).as_strided((rows, cols), (1, rows))
            x = mk(rng, dt, rows)
            got = kf.vecmat(operator.mul, "+", torch.from_numpy(x).to(dev), A).cpu().numpy()
            ref = oracle.reduce_dim_x(buf, rows, cols, rows, x, 1, "+", "mul")
            assert np.array_equal(got, ref), (rows, cols, "vecmat")
            M = buf.reshape(cols, rows)
            for op, npf in (("+", np.sum), (max, np.max)):
                got = kf.mapreduce(kf.identity, op, A, dims=1).cpu().numpy().reshape(-1)
                ref = (M.astype(np.int64).sum(axis=1).astype(dt) if op == "+" else M.max(axis=1))
                assert np.array_equal(got, ref), (rows, cols, op)
            # sum of squares (UInt8: dot4 of each column's bytes with themselves)
            got = kf.mapreduce(kf.abs2, "+", A, dims=1).cpu().numpy().reshape(-1)
            M64 = M.astype(np.int64)
            assert np.array_equal(got, (M64 * M64).sum(axis=1).astype(dt)), (rows, cols, "abs2")


@pytest.mark.parametrize("dt", [np.int32, np.int64, np.uint8])
def test_short_contiguous_columns_flat_rows_path(kf, oracle, dev, dt):
    # dims=2 over contiguous matrices with columns of at most 2 KiB (8-byte
    # types, and 4-byte types whose rows are not a multiple of 4): blocks of
    # whole columns through LDS, row phases, partial rows-vectors per
    # workgroup and the split combine; matvec and plain mapreduce, exact
    rng = np.random.default_rng(89)
    es = np.dtype(dt).itemsize
    rows_set = (2, 3, 5, 10, 63, 255, 257, 2048 // es - 1, 2048 // es)
    if es >= 4:  # 4- and 8-byte types up to 4 KiB columns
        rows_set += (300, 511, 512, 700, 1000, 1023, 1024) if es == 8 else (513, 600, 1000, 1023, 1024, 1500, 2048)
    if dt == np.uint8:  # + over 32-bit words (packed 16-bit sums) when rows % 4 == 0, else over
        # the words of the rows' period (lcm(rows, 4) bytes; up to 255 odd / 510 even rows)
        rows_set = (4, 8, 12, 100, 252, 1000, 1020, 1028, 2044, 2048, 10, 2, 3, 5, 7, 14, 255, 257, 510)
    for rows in rows_set:
        for cols in (1000, 40_003, 1_000_003 // rows):
            buf = mk(rng, dt, rows * cols)
            A = torch.from_numpy(buf).to(dev).as_strided((rows, cols), (1, rows))
            x = mk(rng, dt, cols)
            got = kf.matvec(operator.mul, "+", A, torch.from_numpy(x).to(dev)).cpu().numpy()
            ref = oracle.reduce_dim_x(buf, rows, cols, rows, x, 2, "+", "mul")
            assert np.array_equal(got, ref), (rows, cols, "matvec")
            M = buf.reshape(cols, rows)
            for op in ("+", max):
                got = kf.mapreduce(kf.identity, op, A, dims=2).cpu().numpy().reshape(-1)
                ref = (M.astype(np.int64).sum(axis=0).astype(dt) if op == "+" else M.max(axis=0))
                assert np.array_equal(got, ref), (rows, cols, op)
            got = kf.mapreduce(kf.abs2, "+", A, dims=2).cpu().numpy().reshape(-1)
            ref = (M.astype(np.int64) ** 2).sum(axis=0).astype(dt)
            assert np.array_equal(got, ref), (rows, cols, "abs2")


@pytest.mark.parametrize("dt", [np.int32, np.uint8, np.int64])
def test_flat_paths_with_strided_x_and_dst(kf, oracle, dev, dt):
    # the LDS-staged dims kernels with an every-other-element x and an
    # every-third-element destination (vecmat!: dims=1; matvec!: dims=2)
    rng = np.random.default_rng(101)
    for rows, cols in ((4, 50_003), (10, 30_001), (100, 4_001), (256, 2_003)):
        buf = mk(rng, dt, rows * cols)
        A = torch.from_numpy(buf).to(dev).as_strided((rows, cols), (1, rows))
        for dim, m, k in ((1, cols, rows), (2, rows, cols)):
            xb = mk(rng, dt, 2 * k)
            x = torch.from_numpy(xb).to(dev)[::2]
            dbuf = torch.zeros(3 * m, dtype=A.dtype, device=dev)
            d = dbuf[::3]
            if dim == 1:
                kf.vecmat_(operator.mul, "+", d, x, A)
            else:
                kf.matvec_(operator.mul, "+", d, A, x)
            ref = oracle.reduce_dim_x(buf, rows, cols, rows, np.ascontiguousarray(xb[::2]), dim, "+", "mul")
            assert np.array_equal(d.cpu().numpy(), ref), (rows, cols, dim)
            assert not dbuf.cpu().numpy()[1::3].any() and not dbuf.cpu().numpy()[2::3].any()


@pytest.mark.parametrize("dt", [np.int32, np.float64])
def test_batched_middle_dims_many_splits(kf, dev, dt):
    # mapreducedims over the middle dim of a Julia pre x mid x post array with
    # few rows and long reduced dims: the batched narrow kernel splits the
    # reduced columns and the many-wave combine folds every batch entry
    rng = np.random.default_rng(103)
    for pre, mid, post in ((40, 20_000, 3), (70, 9_001, 5), (20, 30_000, 2)):
        a = mk(rng, dt, (post, mid, pre))  # numpy C order == Julia pre x mid x post
        x = torch.from_numpy(a).to(dev).permute(2, 1, 0)
        got = kf.mapreduce(kf.identity, "+", x, dims=2).cpu().numpy()
        ref = a.astype(np.float64 if dt == np.float64 else np.int64).sum(axis=1)  # post x pre
        ref = np.ascontiguousarray(ref.T)[:, None, :]
        if dt == np.float64:
            assert np.allclose(got.reshape(pre, 1, post), ref, rtol=1e-12, atol=1e-9), (pre, mid, post)
        else:
            assert np.array_equal(got.reshape(pre, 1, post).astype(np.int64), ref.astype(dt).astype(np.int64)), \
                (pre, mid, post)


@pytest.mark.parametrize("dt", [np.uint8, np.int32, np.float32, np.float64])
def test_few_long_columns(kf, dev, dt):
    # 2..16 long columns along dims=1: every workgroup reads all columns of
    # its row range and the operand x once (one or many row ranges; rows off
    # the 16-byte vector length leave a tail; a strided destination)
    rng = np.random.default_rng(107)
    # (matrices from 80 MiB take the one-workgroup-for-all-columns kernel)
    extra = [(10_000_003, 10)] if dt == np.uint8 else []
    for rows, cols in [(600, 16), (777_777, 2), (100_003, 7), (2**20 + 3, 16), (50_001, 9), (4_000_000, 10)] + extra:
        if np.dtype(dt).kind == "f":
            a = rng.random((cols, rows)).astype(dt)
            xv = rng.random(rows).astype(dt)
        else:
            a = rng.integers(0, 256 if dt == np.uint8 else 100, (cols, rows)).astype(dt)
            xv = rng.integers(0, 256 if dt == np.uint8 else 100, rows).astype(dt)
        A = torch.from_numpy(a).to(dev).T                      # rows x cols, column-major
        x = torch.from_numpy(xv).to(dev)
        a64 = a.astype(np.float64 if np.dtype(dt).kind == "f" else np.int64)
        x64 = xv.astype(a64.dtype)
        dbuf = torch.zeros(3 * cols, dtype=A.dtype, device=dev)
        d = dbuf.as_strided((1, cols), (3 * cols, 3))
        kf.mapreduce_(kf.identity, "+", d, A, dims=1)
        got_sum = dbuf[::3].cpu().numpy()
        got_max = kf.mapreduce(kf.identity, max, A, dims=1).cpu().numpy().reshape(-1)
        got_vm = kf.vecmat(operator.mul, "+", x, A).cpu().numpy()
        ref_sum, ref_vm = a64.sum(axis=1), (a64 * x64[None, :]).sum(axis=1)
        assert np.array_equal(got_max, a.max(axis=1)), (rows, cols)
        if np.dtype(dt).kind == "f":
            tol = 1e-5 if dt == np.float32 else 1e-12
            assert np.allclose(got_sum, ref_sum, rtol=tol), (rows, cols)
            assert np.allclose(got_vm, ref_vm, rtol=tol), (rows, cols)
        else:
            m = 256 if dt == np.uint8 else 2**32
            wrap = lambda v: (v % m).astype(np.uint64 if dt == np.uint8 else np.int64)
            assert np.array_equal(wrap(got_sum.astype(np.int64)), wrap(ref_sum)), (rows, cols)
            assert np.array_equal(wrap(got_vm.astype(np.int64)), wrap(ref_vm)), (rows, cols)
        assert not dbuf.cpu().numpy()[1::3].any()


@pytest.mark.parametrize("dt", [np.uint8, np.int32, np.float32, np.float64])
def test_few_columns_dims2(kf, dev, dt):
    # 2..16 columns along dims=2 (matvec and mapreducedims): one batch of
    # loads over every column per output vector; rows off the vector width
    # (peeled head/tail rows), a strided destination, UInt8 packed sums
    rng = np.random.default_rng(109)
    for rows, cols in ((4096, 16), (1_000_000, 10), (300_003, 3), (2**20, 2), (77_777, 7)):
        if np.dtype(dt).kind == "f":
            a = rng.random((cols, rows)).astype(dt)
            xv = rng.random(cols).astype(dt)
        else:
            a = rng.integers(0, 256 if dt == np.uint8 else 100, (cols, rows)).astype(dt)
            xv = rng.integers(0, 256 if dt == np.uint8 else 100, cols).astype(dt)
        A = torch.from_numpy(a).to(dev).T                      # rows x cols, column-major
        x = torch.from_numpy(xv).to(dev)
        a64 = a.astype(np.float64 if np.dtype(dt).kind == "f" else np.int64)
        x64 = xv.astype(a64.dtype)
        dbuf = torch.zeros(2 * rows, dtype=A.dtype, device=dev)
        d = dbuf.as_strided((rows, 1), (2, 2 * rows))
        kf.mapreduce_(kf.identity, "+", d, A, dims=2)
        got_sum = dbuf[::2].cpu().numpy()
        got_sq = kf.mapreduce(kf.abs2, "+", A, dims=2).cpu().numpy().reshape(-1)
        got_max = kf.mapreduce(kf.identity, max, A, dims=2).cpu().numpy().reshape(-1)
        got_mv = kf.matvec(operator.mul, "+", A, x).cpu().numpy()
        ref_sum, ref_sq, ref_mv = a64.sum(axis=0), (a64 * a64).sum(axis=0), (a64 * x64[:, None]).sum(axis=0)
        assert np.array_equal(got_max, a.max(axis=0)), (rows, cols)
        if np.dtype(dt).kind == "f":
            tol = 1e-5 if dt == np.float32 else 1e-12
            for g_, r_ in ((got_sum, ref_sum), (got_sq, ref_sq), (got_mv, ref_mv)):
                assert np.allclose(g_, r_, rtol=tol), (rows, cols)
        else:
            m = 256 if dt == np.uint8 else 2**32
            for g_, r_ in ((got_sum, ref_sum), (got_sq, ref_sq), (got_mv, ref_mv)):
                assert np.array_equal(g_.astype(np.int64) % m, r_ % m), (rows, cols)
        assert not dbuf.cpu().numpy()[1::2].any()


# 126 and 127 rows: the longest periods (63 and 127 words per period; at 127
# each workgroup sees only two column phases)
@pytest.mark.parametrize("rows", [7, 10, 126, 127])
def test_u8_rows_off_the_word_large(kf, dev, rows):
    # UInt8 dims=2 over short columns off the word boundary, large enough for
    # the flat path's period kernel (sums from 96 MiB, matvec from 256 MiB):
    # each word phase keeps packed 16-bit sums for fixed rows, exact mod 256
    rng = np.random.default_rng(113 + rows)
    for cols, with_x in ((105_000_000 // rows, False), (281_000_000 // rows, True)):
        a = rng.integers(0, 256, (cols, rows), dtype=np.uint8)   # Julia rows x cols, column-major
        A = torch.from_numpy(a).to(dev).T
        if with_x:
            xv = rng.integers(0, 256, cols, dtype=np.uint8)
            got = kf.matvec(operator.mul, "+", A, torch.from_numpy(xv).to(dev)).cpu().numpy()
            ref = np.zeros(rows, np.int64)
            for c0 in range(0, cols, 1 << 24):  # products mod 2^16 in chunks
                blk = a[c0:c0 + (1 << 24)].astype(np.uint16) * xv[c0:c0 + (1 << 24), None].astype(np.uint16)
                ref += blk.sum(axis=0, dtype=np.int64)
            assert np.array_equal(got.astype(np.int64), ref % 256), (rows, cols, "matvec")
        else:
            got = kf.mapreduce(kf.identity, "+", A, dims=2).cpu().numpy().reshape(-1)
            assert np.array_equal(got.astype(np.int64), a.sum(axis=0, dtype=np.int64) % 256), (rows, cols, "+")
            got = kf.mapreduce(kf.abs2, "+", A, dims=2).cpu().numpy().reshape(-1)
            sq = np.zeros(rows, np.int64)
            for c0 in range(0, cols, 1 << 24):
                b = a[c0:c0 + (1 << 24)].astype(np.uint16)
                sq += (b * b).sum(axis=0, dtype=np.int64)
            assert np.array_equal(got.astype(np.int64), sq % 256), (rows, cols, "abs2")


@pytest.mark.parametrize("dt", [np.uint8, np.int32, np.float32, np.float64])
def test_length_one_dimension_is_a_map(kf, dev, dt):
    # dims=1 over a single row / dims=2 over a single column: every output is
    # f of one element (no combine), with and without a vector operand, for
    # aligned, element-offset (off the 16-byte vector) and strided views;
    # one IEEE operation per output, so floats are exact too
    rng = np.random.default_rng(83)
    for n in (2, 17, 4099, 1_000_003):
        for off in (0, 1):
            flat = mk(rng, dt, 2 * n + 2)
            t = torch.from_numpy(flat).to(dev)
            for dims, shape, strides, take in ((1, (1, n), (1, 1), flat[off:off + n]),
                                               (1, (1, n), (1, 2), flat[off:off + 2 * n:2]),
                                               (2, (n, 1), (1, n), flat[off:off + n])):
                A = t[off:].as_strided(shape, strides)
                got = kf.mapreduce(kf.abs2, "+", A, dims=dims).cpu().numpy().reshape(-1)
                assert np.array_equal(got, (take * take).astype(dt)), (n, off, dims, strides)
                x = mk(rng, dt, 1)
                tx = torch.from_numpy(x).to(dev)
                got = (kf.vecmat(operator.mul, "+", tx, A) if dims == 1 else
                       kf.matvec(operator.mul, "+", A, tx)).cpu().numpy().reshape(-1)
                assert np.array_equal(got, (take * x[0]).astype(dt)), (n, off, dims, strides)


@pytest.mark.parametrize("dt", [np.int32, np.int64, np.float64])
def test_flat_path_columns_up_to_4k(kf, oracle, dev, dt):
    # dims=1 over contiguous columns of 2-4 KiB of 4- and 8-byte types: the
    # flat path when a block's columns take one pass of the workgroup's lanes
    # (Int32 1000 / 1023 rows, Int64 300 / 500 / 511 rows), the wave per
    # column otherwise (Int32 600 / 700 rows); ragged last blocks; integers
    # exact, Float64 within 1e-12 of the column's sum of |f|
    rng = np.random.default_rng(89)
    es = np.dtype(dt).itemsize
    for rows in ((600, 700, 1000, 1023, 1024) if es == 4 else (300, 500, 511, 512)):
        for cols in (1, 5, 4099):
            buf = mk(rng, dt, rows * cols)
            A = torch.from_numpy(buf).to(dev).as_strided((rows, cols), (1, rows))
            x = mk(rng, dt, rows)
            got = kf.vecmat(operator.mul, "+", torch.from_numpy(x).to(dev), A).cpu().numpy()
            ref = oracle.reduce_dim_x(buf, rows, cols, rows, x, 1, "+", "mul")
            M = buf.reshape(cols, rows).astype(np.float64)
            if np.dtype(dt).kind == "f":
                bound = np.abs(M * x.astype(np.float64)[None, :]).sum(axis=1) * 1e-12
                assert np.all(np.abs(got - ref) <= bound), (rows, cols, "vecmat")
                got = kf.mapreduce(kf.identity, "+", A, dims=1).cpu().numpy().reshape(-1)
                assert np.all(np.abs(got - M.sum(axis=1)) <= np.abs(M).sum(axis=1) * 1e-12), (rows, cols)
            else:
                assert np.array_equal(got, ref), (rows, cols, "vecmat")
                Mi = buf.reshape(cols, rows)
                for op, npf in (("+", np.sum), (max, np.max)):
                    got = kf.mapreduce(kf.identity, op, A, dims=1).cpu().numpy().reshape(-1)
                    ref = Mi.astype(np.int64).sum(axis=1).astype(dt) if op == "+" else Mi.max(axis=1)
                    assert np.array_equal(got, ref), (rows, cols, op)


@pytest.mark.parametrize("dt", [np.uint8, np.int32, np.int64])
def test_dims2_partial_last_strip(kf, dev, dt):
    # dims=2 over tall aligned columns whose row count is not a whole number
    # of the vector kernel's strips (256 threads x 1-8 vectors): the last
    # strip is partial, its vectors past the end load and store nothing. The
    # matrix is a tensor of exactly rows * cols elements, so a load past the
    # last column's end would leave the allocation. Integers: exact.
    rng = np.random.default_rng(211)
    ev = 16 // np.dtype(dt).itemsize
    for rows, cols in ((10_000, 700), (100_000, 90), (1_000_000, 12), (4096 + ev, 300), (65536 - ev, 64)):
        a = rng.integers(0, 100, (cols, rows)).astype(dt)       # Julia rows x cols, column-major
        A = torch.from_numpy(a).to(dev).T
        x = rng.integers(0, 7, cols).astype(dt)
        print(f"partial strip {np.dtype(dt).name} {rows}x{cols}", flush=True)
        got = kf.mapreduce(kf.identity, "+", A, dims=2).cpu().numpy().reshape(-1)
        a64 = a.astype(np.int64)
        m = 256 if dt == np.uint8 else 2**32 if dt == np.int32 else None
        ref = a64.sum(axis=0)
        if m:
            assert np.array_equal(got.astype(np.int64) % m, ref % m), (rows, cols)
        else:
            assert np.array_equal(got.astype(np.int64), ref), (rows, cols)
        got = kf.matvec(operator.mul, "+", A, torch.from_numpy(x).to(dev)).cpu().numpy()
        ref = (a64 * x.astype(np.int64)[:, None]).sum(axis=0)
        if m:
            assert np.array_equal(got.astype(np.int64) % m, ref % m), (rows, cols, "matvec")
        else:
            assert np.array_equal(got.astype(np.int64), ref), (rows, cols, "matvec")
