"""The C ABI from a plain host program (kernelforge.jl_amd/csrc/kf_driver.cpp,
built by build()): hipMalloc'd buffers, scratch from the *_scratch_bytes
queries, exact checks against host loops; no Python or torch in between."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

DRIVER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "kernelforge.jl_amd", "kf_driver")


def test_c_driver_end_to_end():
    if not os.path.exists(DRIVER):
        pytest.fail("kernelforge.jl_amd/kf_driver is not built; run __graft_entry__.build()")
    r = subprocess.run([DRIVER, str(1 << 22)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "kf_driver: ok" in r.stdout
    for check in ("Int32 inclusive scan exact", "Int32 exclusive scan exact", "mapreduce(abs2, +) exact",
                  "mapreduce(abs2, max) exact", "dims=1) on a column view exact", "dims=2) on a column view exact"):
        assert check in r.stdout, check
