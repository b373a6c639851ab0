"""vcopy! and setvalue! on the GPU (reference test/tests/copy/copy_test.jl):
exact byte equality for every size, element type and alignment."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,n", [
    (torch.float32, 100_000_007), (torch.uint8, 100_000_001), (torch.float32, 33), (torch.float64, 100_000),
    (torch.uint8, 33), (torch.int32, 100_001), (torch.int32, 1), (torch.float32, 1_000_000),
])
def test_vcopy(kf, dev, dtype, n):
    # reference copy_test.jl:1-63 (sizes and types)
    g = torch.Generator(device=dev).manual_seed(n)
    if dtype.is_floating_point:
        src = torch.rand(n, device=dev, dtype=dtype, generator=g)
    else:
        src = torch.randint(0, 100, (n,), device=dev, dtype=dtype, generator=g)
    dst = torch.zeros_like(src)
    kf.vcopy_(dst, src)
    assert torch.equal(dst, src)


def test_vcopy_three_byte_struct(kf, dev):
    # reference copy_test.jl:25-39: a 3-byte isbits struct; here (n, 3) uint8 rows
    n = 100_005
    src = torch.ones(n, 3, dtype=torch.uint8, device=dev)
    src[::7] = torch.tensor([1, 2, 3], dtype=torch.uint8, device=dev)
    dst = torch.zeros_like(src)
    kf.vcopy_(dst, src)
    assert torch.equal(dst, src)


def test_vcopy_misaligned_offsets(kf, dev):
    # equal and unequal misalignment of dst and src, ragged lengths: only the
    # copied range changes, byte for byte
    base = torch.arange(4096 + 64, dtype=torch.int64, device=dev).to(torch.uint8)
    for so in (0, 1, 3, 8, 15):
        for do in (0, 1, 3, 8, 15):
            for n in (0, 1, 15, 16, 17, 100, 4000):
                dst = torch.full((4096 + 64,), 0xAB, dtype=torch.uint8, device=dev)
                kf.vcopy_(dst[do:do + n], base[so:so + n])
                ref = torch.full_like(dst, 0xAB)
                ref[do:do + n] = base[so:so + n]
                assert torch.equal(dst, ref), (so, do, n)


@pytest.mark.parametrize("dtype,val,n", [
    (torch.uint8, 0, 100_003), (torch.float32, 0.0, 100_007), (torch.int32, 0, 99_999),
    (torch.uint8, 0x5A, 100_000_001), (torch.float64, -1.5, 1_000_003), (torch.int64, -7, 33),
    (torch.float32, float("nan"), 1025),
])
def test_setvalue(kf, dev, dtype, val, n):
    # reference copy_test.jl:41-50, 65-75: fill a typemax-filled buffer
    info = torch.finfo(dtype) if dtype.is_floating_point else torch.iinfo(dtype)
    dst = torch.full((n,), info.max, dtype=dtype, device=dev)
    kf.setvalue_(dst, val)
    ref = torch.full((n,), val, dtype=dtype, device=dev)
    assert torch.equal(dst.view(torch.uint8), ref.view(torch.uint8))


def test_setvalue_offsets_and_pairs(kf, dev):
    # unaligned starts and ragged ends leave the bytes outside untouched;
    # 8-byte (a, b) rows and 12-byte rows (a size that does not divide 16)
    for off in (0, 1, 2, 3, 5):
        for n in (1, 3, 4, 5, 100, 4097):
            buf = torch.full((n + 16,), -1, dtype=torch.int32, device=dev)
            kf.setvalue_(buf[off:off + n], 42)
            ref = torch.full_like(buf, -1)
            ref[off:off + n] = 42
            assert torch.equal(buf, ref), (off, n)
    pairs = torch.zeros(10_001, 2, dtype=torch.float32, device=dev)
    kf.setvalue_(pairs, (0.5, -2.0))
    assert torch.equal(pairs, torch.tensor([[0.5, -2.0]], device=dev).expand(10_001, 2))
    rows = torch.zeros(5_003, 3, dtype=torch.float32, device=dev)
    kf.setvalue_(rows[1:], (1.0, 2.0, 3.0))
    assert torch.equal(rows[0], torch.zeros(3, device=dev))
    assert torch.equal(rows[1:], torch.tensor([[1.0, 2.0, 3.0]], device=dev).expand(5_002, 3))


def test_setvalue_rejects(kf, dev):
    x = torch.zeros(10, 4, device=dev)
    with pytest.raises(kf.ArgumentError):
        kf.setvalue_(x[:, 0], 1.0)          # not contiguous
    with pytest.raises(kf.ArgumentError):
        kf.setvalue_(x, (1.0, 2.0))         # tuple length does not match the rows


# ---- the bandwidth probes behind bench.py's ceilings --------------------------
@pytest.mark.parametrize("nbytes", [16, 4096, 4096 * 3 + 16, 1 << 20, (96 << 10) * 5 + 48, 64 << 20])
def test_bw_probe_copies_are_exact(kf, dev, nbytes):
    # every copy kind moves the bytes exactly (the ordered copy twice in a row:
    # its flags from the first call must not let the second skip its order)
    import ctypes
    L, K = kf._lib.lib(), kf._lib
    g = torch.Generator(device=dev).manual_seed(nbytes)
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=dev, generator=g)
    scratch = torch.empty(L.kf_bw_probe_scratch_bytes(nbytes), dtype=torch.uint8, device=dev)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for kind in (K.BW_COPY, K.BW_COPY_TILED, K.BW_COPY_ORDERED, K.BW_COPY_ORDERED):
        dst = torch.zeros_like(src)
        rc = L.kf_bw_probe(kind, ctypes.c_void_p(dst.data_ptr()), ctypes.c_void_p(src.data_ptr()), nbytes,
                           ctypes.c_void_p(scratch.data_ptr()), scratch.numel(), s)
        assert rc == K.KF_OK, L.kf_last_error()
        torch.cuda.synchronize()
        assert torch.equal(dst, src), (kind, nbytes)


def test_bw_probe_reads_write_nothing_but_their_sink(kf, dev):
    import ctypes
    L, K = kf._lib.lib(), kf._lib
    nbytes = 1 << 24
    src = torch.arange(nbytes // 4, dtype=torch.int32, device=dev)
    sink = torch.full((4,), 7, dtype=torch.int32, device=dev)
    before = src.clone()
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for kind in (K.BW_READ, K.BW_READ_TILED):
        rc = L.kf_bw_probe(kind, ctypes.c_void_p(sink.data_ptr()), ctypes.c_void_p(src.data_ptr()), nbytes, None, 0, s)
        assert rc == K.KF_OK, L.kf_last_error()
    torch.cuda.synchronize()
    assert torch.equal(src, before)
    assert sink[1:].tolist() == [7, 7, 7]   # the sink's first word is the only one a probe may touch
    # argument checks: misaligned sizes and a missing scratch for the ordered copy
    assert L.kf_bw_probe(K.BW_COPY, ctypes.c_void_p(sink.data_ptr()), ctypes.c_void_p(src.data_ptr()), 15, None, 0,
                         s) == K.KF_EINVAL
    assert L.kf_bw_probe(K.BW_COPY_ORDERED, ctypes.c_void_p(sink.data_ptr()), ctypes.c_void_p(src.data_ptr()), 16,
                         None, 0, s) == K.KF_ENOSCRATCH
    assert L.kf_bw_probe(99, ctypes.c_void_p(sink.data_ptr()), ctypes.c_void_p(src.data_ptr()), 16, None, 0,
                         s) == K.KF_EINVAL


@pytest.mark.parametrize("nbytes", [16, 4096 + 16, 1 << 24])
def test_bw_probe_write_stores_every_vector_and_nothing_past_it(kf, dev, nbytes):
    # the write probe stores vector i as (i, i >> 32, 0, 0) over dst[0:bytes]
    # and reads nothing; the word after the buffer stays untouched
    import ctypes
    L, K = kf._lib.lib(), kf._lib
    n4 = nbytes // 4
    dst = torch.full((n4 + 4,), -1, dtype=torch.int32, device=dev)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = L.kf_bw_probe(K.BW_WRITE, ctypes.c_void_p(dst.data_ptr()), None, nbytes, None, 0, s)
    assert rc == K.KF_OK, L.kf_last_error()
    torch.cuda.synchronize()
    v = dst[:n4].view(-1, 4).cpu()
    nvec = nbytes // 16
    assert torch.equal(v[:, 0], torch.arange(nvec, dtype=torch.int32))
    assert bool((v[:, 1:] == 0).all())
    assert dst[n4:].tolist() == [-1, -1, -1, -1]
