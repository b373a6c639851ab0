"""ctypes binding of libkfhip.so (the C ABI declared in include/kf.h).

The library must have been built (kernelforge.jl_amd/build.py); there is no
fallback: a missing library raises at first use.
"""
import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkfhip.so")

# enums mirrored from include/kf.h
KF_OK, KF_EINVAL, KF_ENOSCRATCH, KF_EHIP, KF_EGIVEUP = 0, 1, 2, 3, 4
OP_ADD, OP_MAX, OP_MIN, OP_AFFINE, OP_MUL = 0, 1, 2, 3, 4
MAP_IDENTITY, MAP_ABS2 = 0, 1
MAP2_MUL, MAP2_SQDIFF, MAP2_WSQ, MAP2_EXPDIFF = 0, 1, 2, 3
MAP3_MUL = 0
POST_IDENTITY, POST_SQRT, POST_ABS2 = 0, 1, 2
F32, F64, I32, I64, U8, F32X2, Q32, Q64 = 0, 1, 2, 3, 4, 5, 6, 7
BW_COPY, BW_COPY_TILED, BW_COPY_ORDERED, BW_READ, BW_READ_TILED, BW_WRITE = 0, 1, 2, 3, 4, 5

# Every symbol include/kf.h declares, with its ctypes signature.
_P, _I, _I64, _SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t
SIGNATURES = {
    "kf_version": ([], _I),
    "kf_last_error": ([], ctypes.c_char_p),
    "kf_scratch_reset": ([_P, _SZ, _P], _I),
    "kf_scan_scratch_bytes": ([_I, _I, _I64], _SZ),
    "kf_scan": ([_I, _I, _I, _I, _I, _P, _I64, _P, _I64, _I64, _P, _SZ, _P], _I),
    "kf_scan_shaped_scratch_bytes": ([_I, _I, _I64, _I, _I], _SZ),
    "kf_scan_shape": ([_I, _I64, _I, _I, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)], _I),
    "kf_scan_shaped": ([_I, _I, _I, _I, _I, _P, _I64, _P, _I64, _I64, _I, _I, _P, _SZ, _P], _I),
    "kf_reduce_scratch_bytes": ([_I, _I64], _SZ),
    "kf_reduce": ([_I, _I, _I, _P, _I64, _I64, _P, _P, _SZ, _P], _I),
    "kf_reduce_dim_scratch_bytes": ([_I, _I64, _I64, _I], _SZ),
    "kf_reduce_dim": ([_I, _I, _I, _P, _I64, _I64, _I64, _I, _P, _I64, _P, _SZ, _P], _I),
    "kf_reduce2_scratch_bytes": ([_I, _I64], _SZ),
    "kf_reduce2": ([_I, _I, _I, _P, _I64, _P, _I64, _I64, _P, _P, _SZ, _P], _I),
    "kf_reduce3_scratch_bytes": ([_I, _I64], _SZ),
    "kf_reduce3": ([_I, _I, _I, _P, _I64, _P, _I64, _P, _I64, _I64, _P, _P, _SZ, _P], _I),
    "kf_reduce_dim_batched_scratch_bytes": ([_I, _I64, _I64, _I64], _SZ),
    "kf_reduce_dim_batched": ([_I, _I, _I, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P, _SZ, _P], _I),
    "kf_reduce_dim_x": ([_I, _I, _I, _P, _I64, _I64, _I64, _I, _P, _I64, _P, _I64, _P, _SZ, _P], _I),
    "kf_post_map": ([_I, _I, _P, _I64, _I64, _P], _I),
    "kf_copy": ([_P, _P, _SZ, _P], _I),
    "kf_scan_scratch_status": ([_P, _P, ctypes.POINTER(ctypes.c_int)], _I),
    "kf_fill": ([_P, _I64, _P, _SZ, _P], _I),
    "kf_reduce_noalloc": ([_I, _I, _I, _P, _I64, _I64, _P, _P], _I),
    "kf_init": ([], _I),
    "kf_async_status": ([ctypes.POINTER(ctypes.c_int)], _I),
    "kf_reduce_scratch_status": ([_P, _P, ctypes.POINTER(ctypes.c_int)], _I),
    "kf_bw_probe_scratch_bytes": ([_SZ], _SZ),
    "kf_bw_probe": ([_I, _P, _P, _SZ, _P, _SZ, _P], _I),
}

# The instrumented library (include/kf_debug.h): the same C ABI plus the test
# and timeline hooks, built with -DKF_TIMELINE from the scan and full-reduction
# sources only.
DEBUG_LIB_PATH = os.path.join(HERE, "libkfhip_timeline.so")
DEBUG_SIGNATURES = {
    "kf_debug_scan_giveup": ([_I64, ctypes.c_uint32], _I),
    "kf_debug_reduce_giveup": ([_I, ctypes.c_uint32], _I),
    "kf_debug_scan_timeline": ([_P], _I),
    "kf_debug_reduce_timeline": ([_P], _I),
}
DEBUG_LIB_EXPORTS = ("kf_version", "kf_last_error", "kf_init", "kf_async_status", "kf_scratch_reset",
                     "kf_scan", "kf_scan_shaped", "kf_scan_scratch_bytes", "kf_scan_shaped_scratch_bytes",
                     "kf_scan_shape", "kf_scan_scratch_status", "kf_reduce", "kf_reduce_scratch_bytes",
                     "kf_reduce_scratch_status", "kf_reduce2", "kf_reduce2_scratch_bytes", "kf_reduce3",
                     "kf_reduce3_scratch_bytes", "kf_reduce_noalloc", "kf_post_map")

_lib = None
_debug_lib = None
_lock = threading.Lock()


class KernelForgeError(RuntimeError):
    """A HIP-level failure reported by libkfhip (KF_EHIP)."""


def lib():
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise RuntimeError(
                        f"{LIB_PATH} is not built; run kernelforge.jl_amd/build.py "
                        "(or __graft_entry__.build()) first")
                L = ctypes.CDLL(LIB_PATH)
                for name, (args, res) in SIGNATURES.items():
                    fn = getattr(L, name)
                    fn.argtypes = args
                    fn.restype = res
                _lib = L
    return _lib


def debug_lib():
    """The instrumented library (test hooks and timelines); a separate
    handle with its own kernels and its own give-up report word."""
    global _debug_lib
    if _debug_lib is None:
        with _lock:
            if _debug_lib is None:
                if not os.path.exists(DEBUG_LIB_PATH):
                    raise RuntimeError(f"{DEBUG_LIB_PATH} is not built; run kernelforge.jl_amd/build.py")
                L = ctypes.CDLL(DEBUG_LIB_PATH)
                for name in DEBUG_LIB_EXPORTS:
                    fn = getattr(L, name)
                    fn.argtypes, fn.restype = SIGNATURES[name]
                for name, (args, res) in DEBUG_SIGNATURES.items():
                    fn = getattr(L, name)
                    fn.argtypes, fn.restype = args, res
                _debug_lib = L
    return _debug_lib


def check(rc, what):
    """Translate a kf_status into the exception the reference raises."""
    if rc == KF_OK:
        return
    msg = lib().kf_last_error().decode(errors="replace")
    if rc in (KF_EINVAL, KF_ENOSCRATCH):
        from . import ArgumentError
        raise ArgumentError(f"{what}: {msg}")
    if rc == KF_EGIVEUP:
        from . import _revalidate_scan_buffers
        raise KernelForgeError(f"{what}: {msg} {_revalidate_scan_buffers()}")
    raise KernelForgeError(f"{what}: {msg}")
