"""ctypes wrapper of liboracle.so — the CPU checker and CPU baseline.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg. The product (kernelforge.jl_amd) never imports
it. Semantics and reference citations are in kf_oracle.c.

Every function takes numpy arrays. Float results come back as float64
(the Float64 host accumulation tolerances are stated against); integer
results come back exactly, in the input's dtype.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")

DT = {np.dtype(np.float32): 0, np.dtype(np.float64): 1, np.dtype(np.int32): 2,
      np.dtype(np.int64): 3, np.dtype(np.uint8): 4}
OPS = {"+": 0, "max": 1, "min": 2, "affine": 3, "*": 4}
MAPS = {"identity": 0, "abs2": 1}

_lib = None


def build():
    r = subprocess.run(["make", "-s", "-B", "-C", HERE, "liboracle.so"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + r.stderr)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        P, I64, I, D = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_double
        L.kfo_scan_f.argtypes = [P, I, I64, I64, I, I, I, P]
        L.kfo_scan_i.argtypes = [P, I, I64, I64, I, I, I, P]
        L.kfo_scan_affine.argtypes = [P, I64, I, P]
        L.kfo_scan_quat.argtypes = [P, I, I64, I, P]
        L.kfo_reduce_f.argtypes = [P, I, I64, I64, I, I]
        L.kfo_reduce_f.restype = D
        L.kfo_reduce_i.argtypes = [P, I, I64, I64, I, I, P]
        L.kfo_reduce2_f.argtypes = [P, P, I, I64, I, I]
        L.kfo_reduce2_f.restype = D
        L.kfo_reduce2_i.argtypes = [P, P, I, I64, I, I, P]
        L.kfo_reduce3_f.argtypes = [P, P, P, I, I64, I]
        L.kfo_reduce3_f.restype = D
        L.kfo_reduce3_i.argtypes = [P, P, P, I, I64, I, P]
        L.kfo_reduce_dim_x_f.argtypes = [P, P, I, I64, I64, I64, I, I, I, P]
        L.kfo_reduce_dim_x_i.argtypes = [P, P, I, I64, I64, I64, I, I, I, P]
        L.kfo_reduce_dim_f.argtypes = [P, I, I64, I64, I64, I, I, I, P]
        L.kfo_reduce_dim_i.argtypes = [P, I, I64, I64, I64, I, I, I, P]
        L.kfb_scan_add_f32_seq.argtypes = [P, P, I64]
        L.kfb_scan_add_f32_par.argtypes = [P, P, I64, I]
        L.kfb_sum_f32_seq.argtypes = [P, I64]
        L.kfb_sum_f32_seq.restype = ctypes.c_float
        L.kfb_sum_f32_par.argtypes = [P, I64, I]
        L.kfb_sum_f32_par.restype = ctypes.c_float
        L.kfo_omp_max_threads.restype = I
        L.kfb_scan_add_i32.argtypes = [P, P, I64, I, I]
        L.kfb_scan_affine_f32.argtypes = [P, P, I64, I]
        L.kfb_sum_abs2_f32.argtypes = [P, I64, I]
        L.kfb_sum_abs2_f32.restype = ctypes.c_float
        L.kfb_sum_abs2_f64.argtypes = [P, I64, I]
        L.kfb_sum_abs2_f64.restype = D
        L.kfb_max_i32.argtypes = [P, I64, I]
        L.kfb_max_i32.restype = ctypes.c_int32
        L.kfb_sum_dims_f32.argtypes = [P, I64, I64, I64, I, P, I]
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _is_float(a):
    return a.dtype in (np.float32, np.float64)


def scan(x, op="+", f="identity", exclusive=False):
    """Base.accumulate(op, f.(x)) (exclusive: shifted right, identity first).
    x: 1-D numpy array (any stride); (n, 2) float32 pairs for op='affine';
    (n, 4) float32/float64 quaternions (s, v1, v2, v3) for op='*' (Hamilton
    product)."""
    L = lib()
    if op == "*" and x.ndim == 2:
        q = np.ascontiguousarray(x)
        assert q.shape[1] == 4 and q.dtype in (np.float32, np.float64)
        out = np.empty((q.shape[0], 4), np.float64)
        L.kfo_scan_quat(_p(q), int(q.dtype == np.float64), q.shape[0], int(exclusive), _p(out))
        return out
    if op == "affine":
        ab = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, 2)
        out = np.empty((ab.shape[0], 2), np.float64)
        L.kfo_scan_affine(_p(ab), ab.shape[0], int(exclusive), _p(out))
        return out
    x = np.ascontiguousarray(x)
    n = x.shape[0]
    if _is_float(x):
        out = np.empty(n, np.float64)
        L.kfo_scan_f(_p(x), DT[x.dtype], n, 1, OPS[op], MAPS[f], int(exclusive), _p(out))
    else:
        out = np.empty(n, x.dtype)
        L.kfo_scan_i(_p(x), DT[x.dtype], n, 1, OPS[op], MAPS[f], int(exclusive), _p(out))
    return out


def reduce(x, op="+", f="identity"):
    """Base.mapreduce(f, op, x) over a non-empty 1-D array."""
    L = lib()
    x = np.ascontiguousarray(x)
    if _is_float(x):
        return L.kfo_reduce_f(_p(x), DT[x.dtype], x.shape[0], 1, OPS[op], MAPS[f])
    out = np.empty(1, x.dtype)
    L.kfo_reduce_i(_p(x), DT[x.dtype], x.shape[0], 1, OPS[op], MAPS[f], _p(out))
    return out[0]


def reduce2(x, y, op="+", f2="mul"):
    """Base.mapreduce(f2, op, x, y) for f2 in {"mul": x*y, "sqdiff": (x-y)^2, "wsq": x*y*y, "expdiff": exp(x-y)}."""
    L = lib()
    x, y = np.ascontiguousarray(x), np.ascontiguousarray(y)
    assert x.dtype == y.dtype and x.shape == y.shape and x.ndim == 1
    code = {"mul": 0, "sqdiff": 1, "wsq": 2, "expdiff": 3}[f2]
    if _is_float(x):
        return L.kfo_reduce2_f(_p(x), _p(y), DT[x.dtype], x.shape[0], OPS[op], code)
    out = np.empty(1, x.dtype)
    L.kfo_reduce2_i(_p(x), _p(y), DT[x.dtype], x.shape[0], OPS[op], code, _p(out))
    return out[0]



def reduce3(x, y, z, op="+"):
    """Base.mapreduce((a, b, c) -> a*b*c, op, x, y, z); float products in Float64."""
    L = lib()
    x, y, z = (np.ascontiguousarray(a) for a in (x, y, z))
    assert x.dtype == y.dtype == z.dtype and x.shape == y.shape == z.shape and x.ndim == 1
    if _is_float(x):
        return L.kfo_reduce3_f(_p(x), _p(y), _p(z), DT[x.dtype], x.shape[0], OPS[op])
    out = np.empty(1, x.dtype)
    L.kfo_reduce3_i(_p(x), _p(y), _p(z), DT[x.dtype], x.shape[0], OPS[op], _p(out))
    return out[0]

def reduce_dim(buf, rows, cols, col_stride, dim, op="+", f="identity"):
    """Base.mapreduce(f, op, A; dims=dim) of the column-major matrix
    A[i, j] = buf[i + j*col_stride] (buf 1-D). Returns the 1-D result."""
    L = lib()
    buf = np.ascontiguousarray(buf)
    assert buf.ndim == 1 and (cols - 1) * col_stride + rows <= buf.shape[0]
    m = cols if dim == 1 else rows
    if _is_float(buf):
        out = np.empty(m, np.float64)
        L.kfo_reduce_dim_f(_p(buf), DT[buf.dtype], rows, cols, col_stride, dim, OPS[op], MAPS[f], _p(out))
    else:
        out = np.empty(m, buf.dtype)
        L.kfo_reduce_dim_i(_p(buf), DT[buf.dtype], rows, cols, col_stride, dim, OPS[op], MAPS[f], _p(out))
    return out


def reduce_dim_x(buf, rows, cols, col_stride, x, dim, op="+", f2="mul"):
    """matvec (dim 2) / vecmat (dim 1) of the column-major matrix in buf with x."""
    L = lib()
    buf, x = np.ascontiguousarray(buf), np.ascontiguousarray(x)
    assert buf.dtype == x.dtype and x.shape[0] == (cols if dim == 2 else rows)
    m = rows if dim == 2 else cols
    code = {"mul": 0, "sqdiff": 1}[f2]
    if _is_float(buf):
        out = np.empty(m, np.float64)
        L.kfo_reduce_dim_x_f(_p(buf), _p(x), DT[buf.dtype], rows, cols, col_stride, dim, OPS[op], code, _p(out))
    else:
        out = np.empty(m, buf.dtype)
        L.kfo_reduce_dim_x_i(_p(buf), _p(x), DT[buf.dtype], rows, cols, col_stride, dim, OPS[op], code, _p(out))
    return out


# --- CPU baseline (element-type arithmetic, as Base computes on the host) ---
def baseline_scan_add_f32(x, y, threads=1):
    L = lib()
    if threads <= 1:
        L.kfb_scan_add_f32_seq(_p(x), _p(y), x.shape[0])
    else:
        L.kfb_scan_add_f32_par(_p(x), _p(y), x.shape[0], threads)


def baseline_sum_f32(x, threads=1):
    L = lib()
    if threads <= 1:
        return L.kfb_sum_f32_seq(_p(x), x.shape[0])
    return L.kfb_sum_f32_par(_p(x), x.shape[0], threads)


def baseline_scan_add_i32(x, y, exclusive=False, threads=1):
    lib().kfb_scan_add_i32(_p(x), _p(y), x.shape[0], int(bool(exclusive)), threads)


def baseline_scan_affine_f32(ab, out, threads=1):
    """ab, out: (n, 2) float32 C-contiguous."""
    lib().kfb_scan_affine_f32(_p(ab), _p(out), ab.shape[0], threads)


def baseline_sum_abs2(x, threads=1):
    L = lib()
    if x.dtype == np.float32:
        return L.kfb_sum_abs2_f32(_p(x), x.shape[0], threads)
    return L.kfb_sum_abs2_f64(_p(x), x.shape[0], threads)


def baseline_max_i32(x, threads=1):
    return lib().kfb_max_i32(_p(x), x.shape[0], threads)


def baseline_sum_dims_f32(buf, rows, cols, col_stride, dim, out, threads=1):
    """buf: the flat Float32 storage of a column-major rows x cols matrix with
    column stride col_stride; out: cols (dim=1) or rows (dim=2) values."""
    lib().kfb_sum_dims_f32(_p(buf), rows, cols, col_stride, dim, _p(out), threads)


def omp_max_threads():
    return lib().kfo_omp_max_threads()
