"""The kernels record into HIP graphs (no memset nodes; scratch is kept valid
by the kernels themselves) and every replay matches eager execution, with
eager work and synchronisations between replays."""
import operator

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(kf, oracle, dev):
    rng = np.random.default_rng(29)
    n = 1_000_003
    x = torch.from_numpy(rng.integers(-8, 9, n).astype(np.int32)).to(dev)
    A = torch.from_numpy(rng.integers(-8, 9, (300, 5000)).astype(np.int32)).to(dev).T  # 5000 x 300 col-major
    y = torch.empty_like(x)
    tot = torch.empty(1, dtype=torch.int32, device=dev)
    dot = torch.empty(1, dtype=torch.int32, device=dev)
    rows = torch.empty(5000, dtype=torch.int32, device=dev)
    t_scan = kf.get_allocation(kf.Scan1D, kf.identity, "+", x)
    t_red = kf.get_allocation(kf.MapReduce1D, kf.identity, "+", x)
    t_dim = kf.get_allocation(kf.MapReduce2D, kf.identity, "+", A, dims=2)

    def work():
        kf.scan_("+", y, x, tmp=t_scan, exclusive=True)
        kf.mapreduce_(kf.identity, max, tot, x, tmp=t_red)         # single-level fold (489 workgroups)
        kf.mapreduce1d_(operator.mul, "+", dot, (x, x), tmp=t_red)  # the same, two arrays
        kf.mapreduce_(kf.identity, "+", rows, A, dims=2, tmp=t_dim)

    work()  # eager warm-up
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        work()
    for rep in range(4):
        x.add_(rep)        # eager work between replays
        A.mul_(-1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        xs, As = x.cpu().numpy(), A.cpu().numpy()
        assert np.array_equal(y.cpu().numpy(), oracle.scan(xs, "+", exclusive=True)), rep
        assert tot.item() == xs.max(), rep
        assert dot.item() == int(np.sum(xs.astype(np.int64) ** 2) % 2**32 - (2**32 if np.sum(xs.astype(np.int64) ** 2) % 2**32 >= 2**31 else 0)), rep
        assert np.array_equal(rows.cpu().numpy(), As.sum(axis=1).astype(np.int32)), rep
        # the same calls eagerly agree with the replay
        y2 = torch.empty_like(y)
        kf.scan_("+", y2, x, tmp=t_scan, exclusive=True)
        assert torch.equal(y2, y), rep


def test_two_streams_concurrently(kf, oracle, dev):
    # calls on different streams use different default scratch buffers and
    # may overlap; each stream's results must match its own data
    rng = np.random.default_rng(31)
    xs = [rng.integers(-8, 9, 3_000_017).astype(np.int32) for _ in range(2)]
    streams = [torch.cuda.Stream(device=dev) for _ in range(2)]
    outs = [None, None]
    srcs = [torch.from_numpy(x).to(dev) for x in xs]
    torch.cuda.synchronize()
    for rep in range(3):
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                outs[i] = kf.scan("+", srcs[i])
                kf.scan_("max", outs[i], outs[i])   # in place on the same stream
        torch.cuda.synchronize()
        for i in range(2):
            ref = np.maximum.accumulate(oracle.scan(xs[i], "+"))
            assert np.array_equal(outs[i].cpu().numpy(), ref), (rep, i)


_FRESH = r"""
import sys, ctypes
sys.path.insert(0, sys.argv[1])
import torch
import __graft_entry__
kf = __graft_entry__.load_package()
dev = torch.device("cuda:0")
x = torch.arange(1, 100_001, dtype=torch.int64, device=dev)
y = torch.empty_like(x)
tmp = kf.get_allocation(kf.Scan1D, kf.identity, "+", x)
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):          # the library's very first call happens under capture
    kf.scan_("+", y, x, tmp=tmp)
for _ in range(3):
    y.zero_()
    g.replay()
    torch.cuda.synchronize()
    assert int(y[-1]) == 100_000 * 100_001 // 2, int(y[-1])
kf.scan_("+", y, x, tmp=tmp)       # and eagerly afterwards (the report word is allocated now)
assert int(y[-1]) == 100_000 * 100_001 // 2
flag = ctypes.c_int(-1)
assert kf._lib.lib().kf_async_status(ctypes.byref(flag)) == 0 and flag.value == 0
print("FRESH_OK")
"""


def test_first_library_call_under_capture(tmp_path):
    # the give-up report word is allocated on first use, never while the
    # caller's stream is being captured: a process whose first call is
    # captured into a graph must capture and replay cleanly
    import os
    import subprocess
    import sys
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    script = tmp_path / "fresh.py"
    script.write_text(_FRESH)
    r = subprocess.run([sys.executable, str(script), repo], capture_output=True, text=True, timeout=110)
    assert r.returncode == 0 and "FRESH_OK" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]
