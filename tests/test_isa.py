"""Machine-code checks of the built libkfhip.so (CPU tier, no GPU needed):
every device code object targets gfx950, and none contains a store or
atomic through the scalar data cache or a packed-FP32 VALU instruction
(both are kept out of all kernels on this hardware pool). The code objects
are this repository's own build, disassembled with ROCm's llvm-objdump."""
import glob
import os
import re
import shutil
import subprocess

import pytest

OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"
LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "kernelforge.jl_amd", "libkfhip.so")
SCALAR_WRITE = re.compile(r"^\s*s_(store|atomic|buffer_store|buffer_atomic|scratch_store|dcache_wb)\w*\b", re.M)
PACKED_F32 = re.compile(r"^\s*v_pk_(add|mul|fma)_f32\b", re.M)


@pytest.fixture(scope="module")
def disassembly(tmp_path_factory):
    if not os.path.exists(OBJDUMP):
        pytest.skip("llvm-objdump not installed")
    if not os.path.exists(LIB):
        pytest.fail("libkfhip.so is not built")
    d = tmp_path_factory.mktemp("isa")
    lib = d / "libkfhip.so"
    shutil.copy(LIB, lib)
    subprocess.run([OBJDUMP, "--offloading", str(lib)], check=True, capture_output=True, cwd=d)
    bundles = sorted(glob.glob(str(d / "libkfhip.so.*")))
    dev = [b for b in bundles if "amdgcn" in b]
    assert dev, bundles
    return {b: subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", b], check=True, capture_output=True,
                              text=True).stdout for b in dev}


def test_every_code_object_is_gfx950(disassembly):
    for b in disassembly:
        assert b.endswith("--gfx950"), b


def test_no_scalar_cache_writes(disassembly):
    for b, text in disassembly.items():
        assert "s_endpgm" in text                      # it is a disassembly of kernels
        hits = SCALAR_WRITE.findall(text)
        assert not hits, (os.path.basename(b), hits[:5])


def test_no_packed_fp32_valu(disassembly):
    for b, text in disassembly.items():
        hits = PACKED_F32.findall(text)
        assert not hits, (os.path.basename(b), hits[:5])


def test_patterns_match_what_they_exclude():
    # negative control: the patterns do recognise the instructions
    assert SCALAR_WRITE.search("\ts_store_dword s4, s[0:1], 0x0")
    assert SCALAR_WRITE.search("\ts_atomic_add s2, s[4:5], 0x10")
    assert not SCALAR_WRITE.search("\ts_load_dwordx2 s[0:1], s[4:5], 0x0")
    assert PACKED_F32.search("\tv_pk_fma_f32 v[0:1], v[2:3], v[4:5], v[6:7]")
    assert not PACKED_F32.search("\tv_pk_add_u16 v0, v1, v2")
