"""kf_reduce_noalloc (the allocation-free variant of kf_reduce, scratch in a
static device array) against kf_reduce with a caller buffer, through the C
ABI: same kernels and combine order, so every result must match bit for
bit, on two calls in a row (the second smaller) and across dtypes, maps,
operators, strides and the one-launch / two-level size classes."""
import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

_TORCH = {"F32": torch.float32, "F64": torch.float64, "I32": torch.int32, "I64": torch.int64, "U8": torch.uint8}


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _pair(kf, dev, op, f, dtn, x, stride=1):
    """(kf_reduce result, kf_reduce_noalloc result) as host numpy scalars."""
    L, K = kf._lib.lib(), kf._lib
    dt = getattr(K, dtn)
    n = (x.numel() + stride - 1) // stride
    ref = torch.empty(1, dtype=x.dtype, device=dev)
    got = torch.empty(1, dtype=x.dtype, device=dev)
    need = L.kf_reduce_scratch_bytes(dt, n)
    buf = kf.KernelBuffer(kf.MapReduce1D, need, dev)
    rc = L.kf_reduce(op, f, dt, ctypes.c_void_p(x.data_ptr()), n, stride, ctypes.c_void_p(ref.data_ptr()),
                     ctypes.c_void_p(buf.ptr), buf.nbytes, _stream())
    assert rc == K.KF_OK, L.kf_last_error()
    rc = L.kf_reduce_noalloc(op, f, dt, ctypes.c_void_p(x.data_ptr()), n, stride, ctypes.c_void_p(got.data_ptr()),
                             _stream())
    assert rc == K.KF_OK, L.kf_last_error()
    torch.cuda.synchronize()
    return ref.cpu().numpy()[0], got.cpu().numpy()[0]


def _data(dtn, n, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    dt = _TORCH[dtn]
    if dt.is_floating_point:
        return torch.randn(n, device=dev, generator=g, dtype=dt)
    lo, hi = (0, 255) if dt == torch.uint8 else (-1000, 1000)
    return torch.randint(lo, hi, (n,), device=dev, generator=g, dtype=dt)


def _bits_equal(a, b):
    return np.asarray(a).tobytes() == np.asarray(b).tobytes()


@pytest.mark.parametrize("dtn", ["F32", "F64", "I32", "I64", "U8"])
def test_two_calls_in_a_row_second_smaller(kf, dev, dtn):
    K = kf._lib
    # first call: two-level (level 0 writes partials, level 1 folds) for
    # F32/I32, one launch otherwise; second call: far smaller (one launch)
    for n in (2**25 + 12345, 100_003):
        x = _data(dtn, n, dev, seed=n)
        print(f"noalloc {dtn} n={n}", flush=True)
        for op, f in ((K.OP_ADD, K.MAP_IDENTITY), (K.OP_ADD, K.MAP_ABS2), (K.OP_MAX, K.MAP_IDENTITY)):
            ref, got = _pair(kf, dev, op, f, dtn, x)
            assert _bits_equal(ref, got), (dtn, n, op, f, ref, got)


def test_views_and_strides(kf, dev):
    K = kf._lib
    x = _data("F32", 3 * 10**6 + 7, dev, seed=5)
    for view, stride in ((x[1:], 1), (x[3:], 1), (x, 2), (x[1:], 3)):
        ref, got = _pair(kf, dev, K.OP_ADD, K.MAP_IDENTITY, "F32", view, stride)
        assert _bits_equal(ref, got), (stride, ref, got)
    # and the oracle-independent closed form: the sum of 1..n (exact in Int64)
    n = 10**6
    xi = torch.arange(1, n + 1, dtype=torch.int64, device=dev)
    ref, got = _pair(kf, dev, K.OP_ADD, K.MAP_IDENTITY, "I64", xi)
    assert int(got) == n * (n + 1) // 2 == int(ref)


def test_sizes_beyond_the_static_scratch_are_refused(kf, dev):
    L, K = kf._lib.lib(), kf._lib
    n = 1
    while L.kf_reduce_scratch_bytes(K.F64, n) <= 4 << 20:
        n *= 2
    p = ctypes.c_void_p(4096)
    assert L.kf_reduce_noalloc(K.OP_ADD, 0, K.F64, p, n, 1, p, None) == K.KF_EINVAL
    assert "static" in L.kf_last_error().decode()
    # zero-length is a no-op, bad arguments are refused before any launch
    assert L.kf_reduce_noalloc(K.OP_ADD, 0, K.F64, p, 0, 1, p, None) == K.KF_OK
    assert L.kf_reduce_noalloc(K.OP_AFFINE, 0, K.F32X2, p, 10, 1, p, None) == K.KF_EINVAL
