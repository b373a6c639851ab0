"""Give-up paths, forced from the host: a scan tile or a reduction
workgroup withholds its publication (kf_debug_scan_giveup /
kf_debug_reduce_giveup, exported by the instrumented library only) and the
waiting workgroup runs out of a small poll budget. Every kernel still exits
normally. What is checked: nothing is stored as a result, the give-up is
reported (KF_EGIVEUP from the next entry point, kf_async_status, the
scratch status queries), and the calls after the report are exact again."""
import ctypes
import contextlib

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _async(D):
    flag = ctypes.c_int(-1)
    assert D.kf_async_status(ctypes.byref(flag)) == 0
    return flag.value


def _status(fn, buf):
    flag = ctypes.c_int(-1)
    assert fn(ctypes.c_void_p(buf.ptr), _stream(), ctypes.byref(flag)) == 0
    return flag.value


@contextlib.contextmanager
def _hook(fn, who, limit=4096):
    assert fn(who, limit) == 0
    try:
        yield
    finally:
        assert fn(-1, 0) == 0


@pytest.fixture
def D(kf, dev):
    D = kf._lib.debug_lib()
    torch.cuda.synchronize()
    _async(D)  # start from a clear report
    return D


# one wave reads all predecessors / every wave of the workgroup reads a share /
# more tiles than the GPU holds at once (64-tile windows)
@pytest.mark.parametrize("n", [300_000, 3_000_000, 30_000_000])
def test_scan_giveup_is_reported_and_recovered(kf, oracle, dev, D, n):
    K = kf._lib
    x = np.random.default_rng(41).integers(0, 16, n).astype(np.int32)
    src = torch.from_numpy(x).to(dev)
    dst = torch.empty_like(src)
    tmp = kf.KernelBuffer(kf.Scan1D, D.kf_scan_scratch_bytes(K.I32, K.OP_ADD, n), dev)

    def scan(out):
        return D.kf_scan(K.OP_ADD, K.MAP_IDENTITY, K.POST_IDENTITY, K.I32, 0, _p(src), 1, _p(out), 1, n,
                         ctypes.c_void_p(tmp.ptr), tmp.nbytes, _stream())

    print(f"scan give-up n={n}", flush=True)
    with _hook(D.kf_debug_scan_giveup, 3):
        assert scan(dst) == K.KF_OK  # queued; tile 4 gives up, every waiting tile stops
        torch.cuda.synchronize()
    sentinel = torch.full_like(src, -7)
    # the next entry point reports it and queues nothing
    assert scan(sentinel) == K.KF_EGIVEUP
    assert "gave up" in D.kf_last_error().decode()
    # the report is consumed; the buffer stays inert (stores nothing) until
    # its status is queried, and that skipped call is reported in turn
    assert scan(sentinel) == K.KF_OK
    torch.cuda.synchronize()
    assert bool((sentinel == -7).all())
    assert _async(D) == 1 and _async(D) == 0
    assert _status(D.kf_scan_scratch_status, tmp) == 1
    assert _status(D.kf_scan_scratch_status, tmp) == 0
    for _ in range(2):
        assert scan(dst) == K.KF_OK
        assert np.array_equal(dst.cpu().numpy(), oracle.scan(x, "+"))
    assert _async(D) == 0


# the one-shot folding launch (10^7), the persistent chunk kernel (2^26 + 5),
# the two-level path whose level 1 folds (3 * 2^24) and the short-stride
# span kernel (stride 2)
@pytest.mark.parametrize("n,stride", [(10**7, 1), (2**26 + 5, 1), (3 * 2**24, 1), (4 * 10**6 + 1, 2)])
def test_fold_giveup_is_reported_and_recovered(kf, oracle, dev, D, n, stride):
    K = kf._lib
    x = np.random.default_rng(n).integers(-1000, 1000, n).astype(np.int32)
    src = torch.from_numpy(x).to(dev)
    m = (n + stride - 1) // stride
    out = torch.full((1,), 12345, dtype=torch.int32, device=dev)
    need = D.kf_reduce_scratch_bytes(K.I32, m)
    tmp = kf.KernelBuffer(kf.MapReduce1D, need, dev)

    def red():
        return D.kf_reduce(K.OP_ADD, K.MAP_IDENTITY, K.I32, _p(src), m, stride, _p(out), ctypes.c_void_p(tmp.ptr),
                           tmp.nbytes, _stream())

    print(f"fold give-up n={n} stride={stride}", flush=True)
    ref = oracle.reduce(x[::stride], "+")
    assert red() == K.KF_OK
    assert int(out.item()) == int(ref)
    out.fill_(12345)
    with _hook(D.kf_debug_reduce_giveup, 5):
        assert red() == K.KF_OK
        torch.cuda.synchronize()
    assert int(out.item()) == 12345  # no result was stored
    assert _status(D.kf_reduce_scratch_status, tmp) == 1
    assert _status(D.kf_reduce_scratch_status, tmp) == 0
    assert red() == K.KF_EGIVEUP  # the report, once; nothing queued
    assert int(out.item()) == 12345
    # the fold moved its epoch past the failed call's slots: exact at once
    for _ in range(2):
        assert red() == K.KF_OK
        assert int(out.item()) == int(ref)
    assert _async(D) == 0


@contextlib.contextmanager
def _package_on(kf, D):
    """Route the Python package through the instrumented library."""
    saved = kf._lib._lib
    kf._lib._lib = D
    try:
        yield
    finally:
        kf._lib._lib = saved


def test_python_mapreduce_and_scan_raise_and_recover(kf, oracle, dev, D):
    x = np.random.default_rng(3).integers(-50, 50, 10**7).astype(np.int32)
    src = torch.from_numpy(x).to(dev)
    with _package_on(kf, D):
        # mapreduce reads its result back, so it raises at once
        with _hook(D.kf_debug_reduce_giveup, 7):
            with pytest.raises(kf._lib.KernelForgeError, match="gave up"):
                kf.mapreduce(kf.identity, "+", src)
        assert kf.mapreduce(kf.identity, "+", src) == int(oracle.reduce(x, "+"))
        # scan! is asynchronous: the library's next call raises, after every
        # live scan buffer has been re-validated
        tmp = kf.get_allocation(kf.Scan1D, kf.identity, "+", src)
        dst = torch.empty_like(src)
        with _hook(D.kf_debug_scan_giveup, 3):
            kf.scan_("+", dst, src, tmp=tmp)
            torch.cuda.synchronize()
        with pytest.raises(kf._lib.KernelForgeError, match="valid again"):
            kf.scan_("+", dst, src, tmp=tmp)
        kf.scan_("+", dst, src, tmp=tmp)
        assert np.array_equal(dst.cpu().numpy(), oracle.scan(x, "+"))
        # check=True raises at the call itself
        with _hook(D.kf_debug_scan_giveup, 3):
            with pytest.raises(kf._lib.KernelForgeError):
                kf.scan_("+", dst, src, tmp=tmp, check=True)
        kf.scan_("+", dst, src, tmp=tmp, check=True)
        assert np.array_equal(dst.cpu().numpy(), oracle.scan(x, "+"))
        kf.check_async()


def test_noalloc_fold_giveup_is_reported(kf, oracle, dev, D):
    # kf_reduce_noalloc never allocates: with the report word set up by
    # kf_init, its fold give-up is reported like any other, dst is left
    # untouched, and the static scratch serves the next call exactly
    K = kf._lib
    assert D.kf_init() == 0
    n = 10**7
    x = np.random.default_rng(7).integers(-1000, 1000, n).astype(np.int32)
    src = torch.from_numpy(x).to(dev)
    out = torch.full((1,), 12345, dtype=torch.int32, device=dev)

    def red():
        return D.kf_reduce_noalloc(K.OP_ADD, K.MAP_IDENTITY, K.I32, _p(src), n, 1, _p(out), _stream())

    print("noalloc fold give-up", flush=True)
    with _hook(D.kf_debug_reduce_giveup, 5):
        assert red() == K.KF_OK
        torch.cuda.synchronize()
    assert int(out.item()) == 12345
    assert _async(D) == 1
    for _ in range(2):
        assert red() == K.KF_OK
        assert int(out.item()) == int(oracle.reduce(x, "+"))
    assert _async(D) == 0
