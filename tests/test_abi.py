"""The C-ABI library loads, exports every symbol include/kf.h declares, and
rejects bad arguments before touching a GPU (no compute calls here)."""
import ctypes
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols(header="kf.h"):
    text = open(os.path.join(REPO, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kf_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_expected_surface():
    assert declared_symbols() == sorted([
        "kf_version", "kf_last_error", "kf_scratch_reset", "kf_scan_scratch_bytes", "kf_scan",
        "kf_reduce_scratch_bytes", "kf_reduce", "kf_reduce_dim_scratch_bytes", "kf_reduce_dim", "kf_copy",
        "kf_reduce2_scratch_bytes", "kf_reduce2", "kf_reduce_dim_batched_scratch_bytes", "kf_reduce_dim_batched", "kf_post_map", "kf_reduce_dim_x",
        "kf_fill", "kf_scan_scratch_status", "kf_reduce3_scratch_bytes", "kf_reduce3",
        "kf_reduce_noalloc", "kf_init", "kf_async_status", "kf_reduce_scratch_status",
        "kf_bw_probe_scratch_bytes", "kf_bw_probe",
        "kf_scan_shaped_scratch_bytes", "kf_scan_shape", "kf_scan_shaped"])


def test_library_exports_every_declared_symbol(kf):
    L = kf._lib.lib()
    for name in declared_symbols():
        assert hasattr(L, name), name
        assert name in kf._lib.SIGNATURES, name


def test_test_hooks_live_only_in_the_instrumented_library(kf):
    # the production library exports no kf_debug_* symbol; the instrumented
    # one exports every symbol include/kf_debug.h declares
    L = kf._lib.lib()
    debug = declared_symbols("kf_debug.h")
    assert debug == sorted(kf._lib.DEBUG_SIGNATURES)
    for name in debug:
        assert not hasattr(L, name), name
    D = kf._lib.debug_lib()
    for name in debug + list(kf._lib.DEBUG_LIB_EXPORTS):
        assert hasattr(D, name), name


def test_async_status_is_clear_without_a_gpu(kf):
    # no kernel has run, so nothing can have given up (the report word is
    # not even allocated yet); the query neither blocks nor needs a device
    flag = ctypes.c_int(7)
    assert kf._lib.lib().kf_async_status(ctypes.byref(flag)) == kf._lib.KF_OK
    assert flag.value == 0
    assert kf._lib.lib().kf_async_status(None) == kf._lib.KF_EINVAL
    kf.check_async()


def test_version(kf):
    assert kf._lib.lib().kf_version() == 100


def test_scratch_queries(kf):
    L = kf._lib.lib()
    # one 128-byte descriptor line per tile + a 256-byte header; large arrays
    # use 8 x 16-byte vectors per thread, 768 threads from 17 MiB on for
    # 4- and 8-byte types (96 KiB tiles); the tile count covers
    # operands that start up to 15 bytes past a 16-byte boundary
    tiles = -(-(2**28 + 3) // (768 * 8 * 4))
    assert L.kf_scan_scratch_bytes(kf._lib.F32, kf._lib.OP_ADD, 2**28) == 256 + tiles * 128
    assert L.kf_scan_scratch_bytes(kf._lib.F32X2, kf._lib.OP_AFFINE, 2**26) == 256 + -(-(2**26 + 1) // (768 * 8 * 2)) * 128
    assert L.kf_scan_scratch_bytes(kf._lib.F32X2, kf._lib.OP_AFFINE, 2**25) == 256 + -(-(2**25 + 1) // (768 * 8 * 2)) * 128
    # just below 17 MiB: 1024 threads x 4 vectors (64 KiB tiles)
    n = (17 << 20) // 4 - 1
    assert L.kf_scan_scratch_bytes(kf._lib.F32, kf._lib.OP_ADD, n) == 256 + -(-(n + 3) // (1024 * 4 * 4)) * 128
    assert L.kf_scan_scratch_bytes(kf._lib.U8, kf._lib.OP_ADD, 1) == 256 + 128
    assert L.kf_reduce_scratch_bytes(kf._lib.F64, 10) >= 256 + 4096 * 8
    assert L.kf_reduce_dim_scratch_bytes(kf._lib.F32, 4096, 65536, 1) >= 256
    # few columns -> split rows: partials for every (split, column)
    assert L.kf_reduce_dim_scratch_bytes(kf._lib.F32, 2**24, 2, 1) > 256


def test_dims_scratch_queries_over_shapes(kf):
    # host-only plan walk (no GPU): every dtype, both dims, plain and
    # batched, over row counts around the vector width, the narrow limit and
    # whole-strip boundaries; each query returns a positive size (the
    # largest need over every alignment case) without faulting on the host
    L = kf._lib.lib()
    rows_set = sorted({1, 2, 3, 5, 15, 16, 17, 255, 256, 257, 511, 512, 513, 1000, 1023, 1024, 1025, 2047,
                       4093, 4096, 4099, 8191, 8192, 8195, 65535, 65536, 1048572, 1048575, 2_100_003})
    for dt in (kf._lib.F32, kf._lib.F64, kf._lib.I32, kf._lib.I64, kf._lib.U8):
        for rows in rows_set:
            for cols in (1, 3, 40, 4096, 100_003):
                for dim in (1, 2):
                    assert L.kf_reduce_dim_scratch_bytes(dt, rows, cols, dim) >= 256
                assert L.kf_reduce_dim_batched_scratch_bytes(dt, rows, cols, 7) >= 256


def _shape(kf, dt, n, wg, ni):
    t, i = ctypes.c_int(0), ctypes.c_int(0)
    assert kf._lib.lib().kf_scan_shape(dt, n, wg, ni, ctypes.byref(t), ctypes.byref(i)) == kf._lib.KF_OK
    return t.value, i.value


def test_scan_shape_keywords_pick_the_nearest_compiled_shape(kf):
    # host-only: the shape table, no GPU. Default shapes follow the size.
    K, L = kf._lib, kf._lib.lib()
    assert _shape(kf, K.F32, 2**28, 0, 0) == (768, 32)
    assert _shape(kf, K.F32, 10**6, 0, 0) == (1024, 8)
    assert _shape(kf, K.U8, 2**30, 0, 0) == (512, 256)
    assert _shape(kf, K.F64, 2**27, 0, 0) == (768, 16)
    # exact requests: elements per thread = vectors x elements per vector
    for ni, want in ((4, 4), (8, 8), (16, 16), (32, 32)):
        assert _shape(kf, K.F32, 2**28, 1024, ni) == (1024, want)
    assert _shape(kf, K.F32, 10**6, 768, 32) == (768, 32)
    assert _shape(kf, K.U8, 10**6, 512, 192) == (512, 192)
    assert _shape(kf, K.F64, 10**6, 1024, 2) == (1024, 2)
    # nearest: the reference's 256-thread workgroups take the nearest block
    # (512 for UInt8, whose only block size it is; 768 is nearer than 1024)
    assert _shape(kf, K.U8, 10**7, 256, 16) == (512, 16)
    assert _shape(kf, K.F32, 10**7, 256, 16)[1] == 16
    # a keyword not given stands for the default's value: workgroup 1024
    # alone at 2^28 Float32 (default 768 x 32) -> 1024 x 32, Nitem 32 alone
    # -> the default itself
    assert _shape(kf, K.F32, 2**28, 1024, 0) == (1024, 32)
    assert _shape(kf, K.F32, 2**28, 0, 32) == (768, 32)
    assert _shape(kf, K.F32, 2**28, 0, 8) == (1024, 8)  # 768 threads come with 32 only
    # Nitem beyond the compiled range clamps to the widest shape
    assert _shape(kf, K.F32, 2**20, 0, 10**6)[1] == 32
    # quaternions: 1024 x 1, 2 or 4 units (QuaternionF64 1 or 2) and the wide
    # shapes 768 x 8 (QuaternionF32) and 1024 x 8 (QuaternionF64) from 17 MiB
    assert _shape(kf, K.Q64, 100, 1024, 64) == (1024, 8)  # the widest QuaternionF64 shape
    assert _shape(kf, K.Q64, 100, 1024, 2) == (1024, 2)
    assert _shape(kf, K.Q64, 100, 1024, 4) == (1024, 2)  # no 1024 x 4 for QuaternionF64
    assert _shape(kf, K.Q32, 100, 1024, 64) == (768, 8)
    assert _shape(kf, K.Q32, 2**26, 0, 0) == (768, 8)
    assert _shape(kf, K.Q32, 2**22, 0, 0) == (768, 8)
    assert _shape(kf, K.Q32, 10**6, 0, 0) == (1024, 4)
    assert _shape(kf, K.Q64, 10**6, 0, 0) == (1024, 8)
    assert _shape(kf, K.Q64, 5 * 10**5, 0, 0) == (1024, 2)
    # scratch follows the shape: one 128-byte line per tile + the header
    n = 10**6
    assert L.kf_scan_shaped_scratch_bytes(K.F32, K.OP_ADD, n, 0, 0) == L.kf_scan_scratch_bytes(K.F32, K.OP_ADD, n)
    assert L.kf_scan_shaped_scratch_bytes(K.F32, K.OP_ADD, n, 1024, 4) == 256 + -(-(n + 3) // 4096) * 128
    assert L.kf_scan_shaped_scratch_bytes(K.F32, K.OP_ADD, n, 1024, 32) == 256 + -(-(n + 3) // 32768) * 128
    t = ctypes.c_int(0)
    assert L.kf_scan_shape(99, 10, 0, 0, ctypes.byref(t), ctypes.byref(t)) == K.KF_EINVAL
    assert L.kf_scan_shape(K.F32, 10, 0, 0, None, ctypes.byref(t)) == K.KF_EINVAL
    # a hinted call with a default-sized scratch that is too small is refused
    p, q = ctypes.c_void_p(4096), ctypes.c_void_p(1 << 24)
    small = L.kf_scan_scratch_bytes(K.F32, K.OP_ADD, n)
    assert L.kf_scan_shaped(K.OP_ADD, 0, 0, K.F32, 0, p, 1, q, 1, n, 1024, 4, ctypes.c_void_p(1 << 30), small,
                            None) == K.KF_ENOSCRATCH


def _err(kf):
    return kf._lib.lib().kf_last_error().decode()


def test_invalid_arguments_rejected_without_gpu(kf):
    L, K = kf._lib.lib(), kf._lib
    p = ctypes.c_void_p(4096)
    assert L.kf_scan(99, 0, 0, K.F32, 0, p, 1, p, 1, 10, p, 1 << 20, None) == K.KF_EINVAL
    assert "op" in _err(kf)
    # affine needs the pair type and vice versa
    assert L.kf_scan(K.OP_AFFINE, 0, 0, K.F32, 0, p, 1, p, 1, 10, p, 1 << 20, None) == K.KF_EINVAL
    assert L.kf_scan(K.OP_ADD, 0, 0, K.F32X2, 0, p, 1, p, 1, 10, p, 1 << 20, None) == K.KF_EINVAL
    # the multiply operator takes the scalar types and the quaternions
    assert L.kf_scan(K.OP_MUL, 0, 0, K.F32X2, 0, p, 1, p, 1, 10, p, 1 << 20, None) == K.KF_EINVAL
    # quaternions: the product only, no map or post-map, scan only
    for q in (K.Q32, K.Q64):
        assert L.kf_scan(K.OP_ADD, 0, 0, q, 0, p, 1, p, 1, 10, p, 1 << 20, None) == K.KF_EINVAL
        assert L.kf_scan(K.OP_MUL, K.MAP_ABS2, 0, q, 0, p, 1, p, 1, 10, p, 1 << 20, None) == K.KF_EINVAL
        assert L.kf_scan(K.OP_MUL, 0, K.POST_ABS2, q, 0, p, 1, p, 1, 10, p, 1 << 20, None) == K.KF_EINVAL
        assert L.kf_reduce(K.OP_MUL, 0, q, p, 10, 1, p, p, 1 << 20, None) == K.KF_EINVAL
        assert "scan only" in _err(kf) or "kf_scan only" in _err(kf)
    # affine is scan-only
    assert L.kf_reduce(K.OP_AFFINE, 0, K.F32X2, p, 10, 1, p, p, 1 << 20, None) == K.KF_EINVAL
    # post-map g: unknown code, sqrt on integers, any g on the affine scan
    assert L.kf_scan(K.OP_ADD, 0, 7, K.F32, 0, p, 1, p, 1, 10, p, 1 << 20, None) == K.KF_EINVAL
    assert L.kf_scan(K.OP_ADD, 0, K.POST_SQRT, K.I32, 0, p, 1, p, 1, 10, p, 1 << 20, None) == K.KF_EINVAL
    assert L.kf_scan(K.OP_AFFINE, 0, K.POST_ABS2, K.F32X2, 0, p, 1, p, 1, 10, p, 1 << 20, None) == K.KF_EINVAL
    # n == 0 is a successful no-op, n < 0 an error
    assert L.kf_scan(K.OP_ADD, 0, 0, K.F32, 0, p, 1, p, 1, 0, None, 0, None) == K.KF_OK
    assert L.kf_scan(K.OP_ADD, 0, 0, K.F32, 0, p, 1, p, 1, -1, None, 0, None) == K.KF_EINVAL
    # scratch too small
    q = ctypes.c_void_p(1 << 20)
    assert L.kf_scan(K.OP_ADD, 0, 0, K.F32, 0, p, 1, q, 1, 10, p, 8, None) == K.KF_ENOSCRATCH
    # partial overlap of src and dst
    assert L.kf_scan(K.OP_ADD, 0, 0, K.F32, 0, ctypes.c_void_p(4096), 1, ctypes.c_void_p(4100), 1, 10, q, 1 << 20,
                     None) == K.KF_EINVAL
    assert "overlap" in _err(kf)
    # misaligned element pointer
    assert L.kf_scan(K.OP_ADD, 0, 0, K.F32, 0, ctypes.c_void_p(4097), 1, q, 1, 10, q, 1 << 20, None) == K.KF_EINVAL
    # reduce_dim: bad dim, col_stride < rows
    assert L.kf_reduce_dim(K.OP_ADD, 0, K.F32, p, 4, 4, 4, 3, q, 1, q, 1 << 20, None) == K.KF_EINVAL
    assert L.kf_reduce_dim(K.OP_ADD, 0, K.F32, p, 4, 4, 2, 1, q, 1, q, 1 << 20, None) == K.KF_EINVAL
    assert L.kf_copy(p, p, 0, None) == K.KF_OK
    flag = ctypes.c_int(0)
    assert L.kf_scan_scratch_status(None, None, ctypes.byref(flag)) == K.KF_EINVAL
    assert L.kf_reduce_scratch_status(None, None, ctypes.byref(flag)) == K.KF_EINVAL
    # fill: count 0 is a no-op; bad count, missing value, value size 0 or > 64
    v = ctypes.create_string_buffer(b"\x01" * 65, 65)
    assert L.kf_fill(p, 0, v, 4, None) == K.KF_OK
    assert L.kf_fill(p, -1, v, 4, None) == K.KF_EINVAL
    assert L.kf_fill(p, 10, None, 4, None) == K.KF_EINVAL
    assert L.kf_fill(p, 10, v, 0, None) == K.KF_EINVAL
    assert L.kf_fill(p, 10, v, 65, None) == K.KF_EINVAL
    assert "64" in _err(kf)
