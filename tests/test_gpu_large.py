"""Operands past 2^31 elements (64-bit index arithmetic in every kernel),
checked on the device against closed forms (the host oracle would take
minutes at these sizes)."""
import pytest
import torch

pytestmark = pytest.mark.gpu

CHUNK = 1 << 28


def u8_ramp_prefix(i):
    """Inclusive prefix sum mod 256 of x[k] = k mod 256 at positions i
    (int64): with q, r = divmod(i + 1, 256) the sum is
    q * (0 + ... + 255) + (0 + ... + r-1) = q * 32640 + r (r - 1) / 2,
    and 32640 = 128 (mod 256)."""
    q, r = torch.div(i + 1, 256, rounding_mode="floor"), (i + 1) % 256
    return ((q * 128 + r * (r - 1) // 2) % 256).to(torch.uint8)


def test_uint8_scan_beyond_2pow31(kf, dev):
    n = (1 << 31) + 77
    x = torch.empty(n, dtype=torch.uint8, device=dev)
    for s in range(0, n, CHUNK):
        e = min(n, s + CHUNK)
        x[s:e] = (torch.arange(s, e, device=dev) % 256).to(torch.uint8)
    for exclusive in (False, True):
        y = kf.scan("+", x, exclusive=exclusive)
        for s in range(0, n, CHUNK):
            e = min(n, s + CHUNK)
            i = torch.arange(s, e, device=dev)
            want = u8_ramp_prefix(i - 1 if exclusive else i)
            if exclusive and s == 0:
                want[0] = 0
            assert torch.equal(y[s:e], want), (exclusive, s)
        del y
    torch.cuda.synchronize()


def test_uint8_scan_wide_shape_switchover(kf, dev):
    # UInt8 arrays switch to 512 x 12-vector tiles at 384 MiB and to
    # 512 x 16 at 2^30: both sides of each switch, inclusive and exclusive,
    # against the closed-form prefix of x[k] = k mod 256
    for edge in (384 << 20, 1 << 30):
        for n in (edge - 1, edge, edge + 1):
            x = torch.empty(n, dtype=torch.uint8, device=dev)
            for s in range(0, n, CHUNK):
                e = min(n, s + CHUNK)
                x[s:e] = (torch.arange(s, e, device=dev) % 256).to(torch.uint8)
            for exclusive in (False, True):
                y = kf.scan("+", x, exclusive=exclusive)
                for s in range(0, n, CHUNK):
                    e = min(n, s + CHUNK)
                    i = torch.arange(s, e, device=dev)
                    want = u8_ramp_prefix(i - 1 if exclusive else i)
                    if exclusive and s == 0:
                        want[0] = 0
                    assert torch.equal(y[s:e], want), (n, exclusive, s)
                del y
            del x
    torch.cuda.synchronize()


def test_int32_reductions_beyond_2pow31(kf, dev):
    n = (1 << 31) + 5
    x = torch.ones(n, dtype=torch.int32, device=dev)
    want = n - (1 << 32)                 # Int32 + wraps: 2^31 + 5 -> -2^31 + 5
    assert kf.mapreduce(kf.identity, "+", x) == want
    x[n - 1] = 7                          # a maximum only the tail handling sees
    assert kf.mapreduce(kf.identity, "max", x) == 7
    x[n - 1] = 1
    x[(1 << 31) + 1] = -3
    assert kf.mapreduce(kf.identity, "min", x) == -3
    assert kf.mapreduce(kf.identity, "+", x[1::2]) == (n - 1) // 2 - 4   # stride 2: one -3 among ones
    del x
    torch.cuda.synchronize()


def test_uint8_reductions_beyond_2pow32(kf, dev):
    n = (1 << 32) + 3
    x = torch.ones(n, dtype=torch.uint8, device=dev)
    assert kf.mapreduce(kf.identity, "+", x) == 3          # (2^32 + 3) mod 256
    x[n - 2] = 200
    assert kf.mapreduce(kf.identity, "max", x) == 200
    del x
    torch.cuda.synchronize()


def test_dims_reductions_beyond_2pow31(kf, dev):
    # a 65536 x (32768 + 3) column-major Int32 matrix (2^31 + 196608
    # elements): column and row sums of ones, with one marked column and row
    rows, cols = 1 << 16, (1 << 15) + 3
    buf = torch.ones(cols, rows, dtype=torch.int32, device=dev)     # column j is buf[j]
    buf[cols - 1, rows - 1] = 5
    A = buf.T                                                        # rows x cols, column-major
    c = kf.mapreduce(kf.identity, "+", A, dims=1).reshape(-1)
    assert c.shape[0] == cols and int(c[0]) == rows and int(c[cols - 1]) == rows + 4
    assert torch.equal(c[:-1], torch.full((cols - 1,), rows, dtype=torch.int32, device=dev))
    r = kf.mapreduce(kf.identity, "+", A, dims=2).reshape(-1)
    assert r.shape[0] == rows and int(r[rows - 1]) == cols + 4
    assert torch.equal(r[:-1], torch.full((rows - 1,), cols, dtype=torch.int32, device=dev))
    assert kf.mapreduce(kf.identity, "max", A) == 5
    del buf, A
    torch.cuda.synchronize()
