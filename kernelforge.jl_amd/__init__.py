"""kernelforge_amd — host side of the MI355X scan / mapreduce path.

A Python mirror of KernelForge.jl's operator interface for this path, over
the C ABI of libkfhip.so (include/kf.h). Names follow the reference with
Julia's `!` spelled as a trailing underscore:

    scan_(op, dst, src)            KernelForge.scan!(op, dst, src)
    scan_(f, op, dst, src)         KernelForge.scan!(f, op, dst, src)
    scan(op, src) / scan(f, op, src)
    mapreduce(f, op, src, dims=None)   -> scalar (dims=None) or tensor
    mapreduce_(f, op, dst, src, dims=None)
    get_allocation(kind, f, op, src)   -> KernelBuffer (the reference's `tmp`)
    vcopy_(dst, src)

(reference src/scan/scan.jl:218-284, src/mapreduce/mapreduce.jl:51-212,
src/allocations.jl:16-41, src/copy/copy.jl:24-28).

Arrays are torch tensors on a ROCm device, read with Julia's conventions:
tensor dim k is Julia dim k+1, `dims` are 1-based, and a Julia column-major
matrix is a tensor whose first dim has stride 1 (e.g. `torch.empty(n, m).T`
is an m x n column-major matrix; `A[:, ::2]` is `view(A, :, 1:2:end)`).
Affine pairs are float32 tensors of shape (n, 2) holding (a, b); a vector
of quaternions (Julia's QuaternionF32 / QuaternionF64) is a float32 /
float64 tensor of shape (n, 4) holding (s, v1, v2, v3).

Operators: `+` (operator.add or "+"), `*` (operator.mul or "*"; on
quaternions the Hamilton product, scan only), `max`, `min`, `affine` (scan
only);
maps: `identity`, `abs2`. Anything else raises ArgumentError, as does a
shape/dtype mismatch. The reference's launch-shape keywords of scan!
(Nitem, workgroup) pick the nearest of the compiled gfx950 tile shapes
(`scan_shape`); its other tuning keywords (blocks, family, arch, and the
reductions' Nitem / workgroup) are accepted and ignored: the reduction
shapes are fixed for gfx950. Calls are asynchronous on torch's current stream except the full
`mapreduce`, which returns a host scalar (like the reference's
`Array(dst)[1]`, src/mapreduce/1D/mapreduce1d.jl:203).
"""
import contextlib
import ctypes
import operator
import weakref

import torch

from . import _lib as _L

__all__ = [
    "ArgumentError", "KernelBuffer", "AffineOp", "affine", "identity", "abs2", "sqdiff", "wsq", "expdiff", "prod3",
    "scan_shape",
    "scan", "scan_", "mapreduce", "mapreduce_", "get_allocation", "vcopy_", "setvalue_", "scan_status",
    "check_async", "maximum", "maximum_", "minimum", "mapreduce1d", "mapreduce1d_", "mapreduce2d", "mapreduce2d_",
    "mapreducedims", "mapreducedims_",
    "Scan1D", "MapReduce1D", "MapReduce2D", "MatVec", "VecMat", "matvec", "matvec_", "vecmat", "vecmat_",
]


class ArgumentError(ValueError):
    """Invalid argument (Julia's ArgumentError)."""


def identity(x):
    return x


def abs2(x):
    return x * x


class AffineOp:
    """(a1, b1) o (a2, b2) = (a2*a1, a2*b1 + b2): composition of the maps
    x -> a*x + b, older map first. Scanning it solves x_t = a_t x_{t-1} + b_t."""

    def __call__(self, p, q):
        return (q[0] * p[0], q[0] * p[1] + q[1])

    def __repr__(self):
        return "affine"


affine = AffineOp()


def prod3(a, b, c):
    """a * b * c: the three-array map of mapreduce(prod3, +, (a, b, c))."""
    return a * b * c


def sqdiff(a, b):
    """(a - b)^2: the two-array map of a squared Euclidean distance."""
    return (a - b) * (a - b)


def wsq(w, x):
    """w * x^2: the two-array map of a weighted sum of squares."""
    return w * x * x


def expdiff(a, b):
    """exp(a - b) (floating-point types)."""
    import math
    return math.exp(a - b)


_MAP2 = {"mul": _L.MAP2_MUL, "*": _L.MAP2_MUL, "sqdiff": _L.MAP2_SQDIFF, "wsq": _L.MAP2_WSQ,
         "expdiff": _L.MAP2_EXPDIFF}


def _map2_code(f):
    if f is operator.mul:
        return _L.MAP2_MUL
    if f is sqdiff:
        return _L.MAP2_SQDIFF
    if f is wsq:
        return _L.MAP2_WSQ
    if f is expdiff:
        return _L.MAP2_EXPDIFF
    if isinstance(f, str) and f in _MAP2:
        return _MAP2[f]
    raise ArgumentError(f"unsupported two-array map {f!r}: expected operator.mul, sqdiff, wsq or expdiff")

# Allocation kinds (reference src/algorithms.jl:16-31 tags).
Scan1D, MapReduce1D, MapReduce2D = "Scan1D", "MapReduce1D", "MapReduce2D"
MatVec, VecMat = "MatVec", "VecMat"

_OPS = {"+": _L.OP_ADD, "max": _L.OP_MAX, "min": _L.OP_MIN, "affine": _L.OP_AFFINE, "*": _L.OP_MUL}
_MAPS = {"identity": _L.MAP_IDENTITY, "abs2": _L.MAP_ABS2}
_DTYPES = {torch.float32: _L.F32, torch.float64: _L.F64, torch.int32: _L.I32,
           torch.int64: _L.I64, torch.uint8: _L.U8}


def _op_code(op):
    if op is operator.add or op is operator.iadd or op is sum:
        return _L.OP_ADD
    if op is operator.mul or op is operator.imul:
        return _L.OP_MUL
    if op is max:
        return _L.OP_MAX
    if op is min:
        return _L.OP_MIN
    if isinstance(op, AffineOp):
        return _L.OP_AFFINE
    if isinstance(op, str) and op in _OPS:
        return _OPS[op]
    raise ArgumentError(f"unsupported operator {op!r}: expected +, *, max, min or affine")


def _map_code(f):
    if f is None or f is identity:
        return _L.MAP_IDENTITY
    if f is abs2:
        return _L.MAP_ABS2
    if isinstance(f, str) and f in _MAPS:
        return _MAPS[f]
    raise ArgumentError(f"unsupported map {f!r}: expected identity or abs2")


def _post_code(g):
    """Post-map g on device results: identity, sqrt or abs2 (else None)."""
    import math
    if g is None or g is identity:
        return _L.POST_IDENTITY
    if g is abs2 or g == "abs2":
        return _L.POST_ABS2
    if g in (math.sqrt, torch.sqrt) or g == "sqrt" or getattr(g, "__name__", "") == "sqrt":
        return _L.POST_SQRT
    return None


def _apply_post(g, t, n, stride):
    """t[i*stride] = g(t[i*stride]) on the device for the supported post-maps."""
    code = _post_code(g)
    if code is None:
        raise ArgumentError(f"unsupported post-map g={g!r} on device results: expected identity, sqrt or abs2")
    if code == _L.POST_IDENTITY or n == 0:
        return
    dt = _DTYPES.get(t.dtype)
    if dt is None:
        raise ArgumentError(f"post-map on unsupported element type {t.dtype}")
    with _on(t.device):
        rc = _L.lib().kf_post_map(code, dt, ctypes_void(t.data_ptr()), n, stride, _stream_ptr(t))
    _L.check(rc, "post-map g")


_raw_stream_of = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _raw_stream(device):
    """hipStream_t (as an int) of the current stream on `device`."""
    if _raw_stream_of is not None:
        return _raw_stream_of(device.index)
    return torch.cuda.current_stream(device).cuda_stream


def _stream_ptr(t):
    return _raw_stream(t.device)


def ctypes_void(x):
    """A device address for a c_void_p argument (ctypes converts ints)."""
    return x


_NO_SWITCH = contextlib.nullcontext()


def _on(device):
    """Make `device` current for the launches in the block (no switch, and
    no cost, when it already is)."""
    return _NO_SWITCH if device.index == torch.cuda.current_device() else torch.cuda.device(device)


def _require_device(*ts):
    for t in ts:
        if not isinstance(t, torch.Tensor):
            raise ArgumentError(f"expected a torch.Tensor, got {type(t).__name__}")
        if t.device.type != "cuda":
            raise ArgumentError("kernelforge_amd operates on GPU tensors (device 'cuda'); "
                                f"got a tensor on {t.device}")
    dev = ts[0].device
    for t in ts[1:]:
        if t.device != dev:
            raise ArgumentError(f"tensors on different devices: {dev} and {t.device}")


# ---------------------------------------------------------------------------
# Scratch buffers (the reference's `tmp` KernelBuffer)
# ---------------------------------------------------------------------------
class KernelBuffer:
    """Caller-owned scratch for one kind of call. Zero-filled at creation;
    the kernels keep it valid across calls, so it can be reused with
    different data (reference test/tests/scan/scan_test.jl:103-125)."""

    def __init__(self, kind, nbytes, device):
        self.kind = kind
        self.nbytes = int(max(nbytes, 256))
        raw = torch.zeros(self.nbytes + 256, dtype=torch.uint8, device=device)
        off = (-raw.data_ptr()) % 256
        self._raw = raw
        self.arr = raw[off:off + self.nbytes]
        if kind == Scan1D:
            _scan_buffers.add(self)

    @property
    def ptr(self):
        return self.arr.data_ptr()

    def __repr__(self):
        return f"KernelBuffer({self.kind}, {self.nbytes} bytes, {self.arr.device})"


_default_tmp = {}
# every live Scan1D buffer, re-validated when the library reports a give-up
_scan_buffers = weakref.WeakSet()


def _revalidate_scan_buffers():
    """Clear the sticky give-up flag of every live Scan1D buffer (each query
    synchronises its device's current stream); returns a sentence for the
    error message saying which scans are affected."""
    hit = 0
    for buf in list(_scan_buffers):
        flag = ctypes.c_int(0)
        with _on(buf.arr.device):
            rc = _L.lib().kf_scan_scratch_status(buf.ptr, _raw_stream(buf.arr.device), ctypes.byref(flag))
        if rc == _L.KF_OK and flag.value:
            hit += 1
    if hit:
        return (f"{hit} scan scratch buffer(s) had given up: the scans on them since then stored nothing; "
                "they are valid again")
    return "(a reduction fold gave up: its destination was left untouched; its buffer is valid again)"


def check_async():
    """Raise KernelForgeError if a kernel queued earlier gave up waiting on
    its scratch buffer (kf_async_status), after re-validating every scan
    buffer. Non-blocking: it covers the kernels that have finished, so call
    it after a synchronisation to cover all of them. No counterpart in the
    reference, whose waits are unbounded."""
    flag = ctypes.c_int(0)
    _L.check(_L.lib().kf_async_status(ctypes.byref(flag)), "check_async")
    if flag.value:
        raise _L.KernelForgeError(
            "a scan lookback or reduction fold gave up waiting on its scratch buffer; its results are invalid. "
            + _revalidate_scan_buffers())


def _scratch(kind, need, device, tmp, stream=None):
    if tmp is not None:
        if not isinstance(tmp, KernelBuffer):
            raise ArgumentError(f"tmp must be a KernelBuffer, got {type(tmp).__name__}")
        if (tmp.kind == Scan1D) != (kind == Scan1D):
            # scan descriptors and reduction partials must not share memory:
            # a stale partial could read as a current-epoch descriptor
            raise ArgumentError(f"tmp was allocated for {tmp.kind}; this call needs a "
                                f"{'Scan1D' if kind == Scan1D else 'MapReduce'} buffer")
        if tmp.nbytes < need:
            raise ArgumentError(f"tmp holds {tmp.nbytes} bytes, this call needs {need}")
        return tmp
    key = (kind, device, _raw_stream(device) if stream is None else stream)
    buf = _default_tmp.get(key)
    if buf is None or buf.nbytes < need:
        buf = KernelBuffer(kind, max(need, 2 * (buf.nbytes if buf else 0)), device)
        _default_tmp[key] = buf
    return buf


# ---------------------------------------------------------------------------
# scan! (reference src/scan/scan.jl:218-284)
# ---------------------------------------------------------------------------
def _scan_operand(t, op):
    """(dtype code, n, element stride) of a scan operand."""
    if op == _L.OP_AFFINE:
        if t.dtype != torch.float32 or t.dim() != 2 or t.shape[1] != 2:
            raise ArgumentError("the affine scan takes float32 (a, b) pairs of shape (n, 2)")
        if t.shape[0] > 0 and (t.stride(1) != 1 or t.stride(0) % 2 != 0):
            raise ArgumentError("affine pairs must be stored as adjacent (a, b) float32 values")
        return _L.F32X2, t.shape[0], max(t.stride(0) // 2, 1)
    if op == _L.OP_MUL and t.dim() == 2 and t.shape[1] == 4 and t.dtype in (torch.float32, torch.float64):
        # a vector of quaternions (s, v1, v2, v3), the layout of Julia's
        # QuaternionF32 / QuaternionF64; `*` is the Hamilton product
        if t.shape[0] > 0 and (t.stride(1) != 1 or t.stride(0) % 4 != 0):
            raise ArgumentError("quaternions must be stored as 4 adjacent (s, v1, v2, v3) values")
        return (_L.Q32 if t.dtype == torch.float32 else _L.Q64), t.shape[0], max(t.stride(0) // 4, 1)
    if t.dim() != 1:
        raise ArgumentError(f"scan! takes vectors; got a {t.dim()}-d tensor")
    if t.dtype not in _DTYPES:
        raise ArgumentError(f"unsupported element type {t.dtype}")
    return _DTYPES[t.dtype], t.shape[0], t.stride(0) if t.shape[0] > 1 else 1


def _split_f_op(args, n_arrays, name):
    if len(args) == n_arrays + 1:
        return identity, args[0], args[1:]
    if len(args) == n_arrays + 2:
        return args[0], args[1], args[2:]
    raise ArgumentError(f"{name} takes ([f,] op, {', '.join(['array'] * n_arrays)})")


_SCAN_TUNING = ("Nitem", "workgroup", "family", "arch")


def _shape_keywords(tuning, name):
    """(workgroup, Nitem) of the reference's scan! keywords (0: not given);
    family and arch are accepted and ignored (the descriptor layout is fixed
    per element type here)."""
    for k in tuning:
        if k not in _SCAN_TUNING:
            raise ArgumentError(f"{name}: unknown keyword {k}")
    out = []
    for k in ("workgroup", "Nitem"):
        v = tuning.get(k)
        if v is None:
            out.append(0)
        elif isinstance(v, bool) or not isinstance(v, int) or v <= 0:
            raise ArgumentError(f"{name}: {k} must be a positive integer, got {v!r}")
        else:
            out.append(int(v))
    return tuple(out)


def scan_shape(src, op="+", Nitem=None, workgroup=None):
    """(threads per workgroup, elements per thread) of the tile shape a
    scan! of `src` takes for these keywords: the compiled shape nearest to
    the request (kf_scan_shape), the size-based default when neither is
    given. No counterpart in the reference, which compiles any shape."""
    wg, ni = _shape_keywords({"Nitem": Nitem, "workgroup": workgroup}, "scan_shape")
    dt, n, _ = _scan_operand(src, _op_code(op))
    threads, items = ctypes.c_int(0), ctypes.c_int(0)
    _L.check(_L.lib().kf_scan_shape(dt, n, wg, ni, ctypes.byref(threads), ctypes.byref(items)), "scan_shape")
    return threads.value, items.value


def scan_(*args, exclusive=False, tmp=None, g=None, check=False, **tuning):
    """scan!([f,] op, dst, src; exclusive=False, tmp=None, check=False,
    Nitem=None, workgroup=None) -> dst.

    dst[i] = f(src[1]) op ... op f(src[i]) (inclusive, the reference's only
    mode), or the exclusive variant dst[1] = identity(op),
    dst[i] = inclusive[i-1]. In place (dst is src) is allowed.
    A lookback that gives up (see scan_status) is never silent: the next
    call into the library after that kernel has finished raises
    KernelForgeError, and so do check_async() and the full mapreduce's
    read-back; check=True synchronises after the launch and raises at once. Nitem / workgroup select the nearest compiled tile shape
    (scan_shape); a tmp for such a call comes from
    get_allocation(Scan1D, f, op, src, workgroup, blocks) or is sized for
    the shape (ArgumentError if it is too small)."""
    f, op, (dst, src) = _split_f_op(args, 2, "scan!")
    wg, ni = _shape_keywords(tuning, "scan!")
    opc, fc = _op_code(op), _map_code(f)
    if _post_code(g) is None or (g not in (None, identity) and (opc == _L.OP_AFFINE or src.dim() == 2)):
        raise ArgumentError(f"scan!: unsupported post-map g={g!r}: expected identity, sqrt or abs2")
    _require_device(dst, src)
    dt, n, ss = _scan_operand(src, opc)
    ddt, dn, ds = _scan_operand(dst, opc)
    if ddt != dt:
        raise ArgumentError(f"dst eltype {dst.dtype} differs from src eltype {src.dtype}")
    if dn != n:
        raise ArgumentError(f"dst has length {dn}, src has length {n}")
    if n == 0:
        return dst
    L = _L.lib()
    need = L.kf_scan_shaped_scratch_bytes(dt, opc, n, wg, ni)
    buf = _scratch(Scan1D, need, src.device, tmp)
    with _on(src.device):
        rc = L.kf_scan_shaped(opc, fc, _post_code(g), dt, int(bool(exclusive)), ctypes_void(src.data_ptr()), ss,
                              ctypes_void(dst.data_ptr()), ds, n, wg, ni, ctypes_void(buf.ptr), buf.nbytes,
                              _stream_ptr(src))
    _L.check(rc, "scan!")  # g is applied by the kernel as each value is stored
    if check and scan_status(buf):
        # this give-up is raised here, so its pending report is consumed
        _L.check(_L.lib().kf_async_status(ctypes.byref(ctypes.c_int(0))), "scan!")
        raise _L.KernelForgeError(
            "scan!: a tile's lookback gave up waiting for its predecessor; the results are invalid "
            "(the scratch buffer has been re-validated) " + _revalidate_scan_buffers())
    return dst


def scan_status(tmp):
    """True if a scan! on the Scan1D buffer `tmp` gave up waiting for a
    predecessor tile since the last query (its results are then invalid:
    only out-of-order workgroup dispatch, a corrupted buffer or overlapping
    calls can cause it; until the query, later scans on `tmp` store
    nothing, and each of them is reported by the next library call).
    Clears the flag and re-validates the buffer; synchronises the current
    stream. No counterpart in the reference."""
    if not isinstance(tmp, KernelBuffer) or tmp.kind != Scan1D:
        raise ArgumentError("scan_status takes the Scan1D KernelBuffer of a scan! call")
    flag = ctypes.c_int(0)
    with _on(tmp.arr.device):
        rc = _L.lib().kf_scan_scratch_status(tmp.ptr, _raw_stream(tmp.arr.device), ctypes.byref(flag))
    _L.check(rc, "scan_status")
    return bool(flag.value)


def scan(*args, exclusive=False, tmp=None, g=None, check=False, **tuning):
    """scan([f,] op, src) -> new dst (reference src/scan/scan.jl:218-244)."""
    f, op, (src,) = _split_f_op(args, 1, "scan")
    _require_device(src)
    dst = torch.empty_like(src, memory_format=torch.contiguous_format)
    return scan_(f, op, dst, src, exclusive=exclusive, tmp=tmp, g=g, check=check, **tuning)


# ---------------------------------------------------------------------------
# mapreduce (reference src/mapreduce/mapreduce.jl:51-298)
# ---------------------------------------------------------------------------
def _normalize_dims(dims, nd):
    """Sorted dims tuple; a non-positive d counts from the end (d -> nd + d + 1),
    then range and duplicate checks with the reference's messages
    (src/helpers.jl:194-198, src/mapreduce/mapreduce.jl:250-257)."""
    if isinstance(dims, int):
        dims = (dims,)
    try:
        dims = tuple(int(d) for d in dims)
    except TypeError:
        raise ArgumentError(f"dims must be an int or a tuple of ints, got {dims!r}")
    dims = tuple(sorted(d if d > 0 else nd + d + 1 for d in dims))
    for d in dims:
        if not 1 <= d <= nd:
            raise ArgumentError(f"dimension {d} out of range for {nd}-dimensional array")
    if len(set(dims)) != len(dims):
        raise ArgumentError(f"duplicate dimensions in dims={dims}")
    return dims


def _classify_dims(dims, nd):
    """(lead_end, tail_start) with the reference's meaning
    (src/mapreduce/mapreduce.jl:272-298): dims[:lead_end] are 1..lead_end,
    dims[tail_start-1:] are the last dims; (0, N+1) = general layout."""
    N = len(dims)
    lead_end = 0
    for k in range(1, N + 1):
        if dims[k - 1] == k:
            lead_end = k
        else:
            break
    tail_start = N + 1
    for k in range(N, 0, -1):
        if dims[k - 1] == nd - (N - k):
            tail_start = k
        else:
            break
    if lead_end > 0 and tail_start <= N:
        if all(dims[i + 1] == dims[i] + 1 for i in range(N - 1)):
            return lead_end, N + 1
    n_tail = N - tail_start + 1 if tail_start <= N else 0
    if lead_end + n_tail != N:
        return 0, N + 1
    return lead_end, tail_start


def _merge(sizes, strides):
    """Single (count, stride) for a run of dims in column-major order, or None."""
    count, stride, expect = 1, None, None
    for s, st in zip(sizes, strides):
        if s == 1:
            continue
        if stride is None:
            stride, expect = st, st * s
        elif st != expect:
            return None
        else:
            expect = st * s
        count *= s
    return count, (stride if stride is not None else 1)


def _as_matrix(t, k):
    """View dims [0, k) as rows and [k, nd) as columns of a column-major
    matrix: (rows, cols, col_stride). Rows must be unit-stride."""
    sizes, strides = list(t.shape), list(t.stride())
    r = _merge(sizes[:k], strides[:k])
    c = _merge(sizes[k:], strides[k:])
    if r is None or c is None or (r[0] > 1 and r[1] != 1):
        raise NotImplementedError(
            f"layout with shape {tuple(sizes)} and strides {tuple(strides)} cannot be viewed as a "
            f"column-major matrix split at dim {k}")
    rows, cols = r[0], c[0]
    col_stride = c[1] if cols > 1 else max(rows, 1)
    if cols > 1 and col_stride < rows:
        raise NotImplementedError("overlapping or row-major layout is not supported")
    return rows, cols, col_stride


def _colmajor_empty(shape, dtype, device):
    nd = len(shape)
    if nd == 0:
        return torch.empty((), dtype=dtype, device=device)
    return torch.empty(tuple(reversed(shape)), dtype=dtype, device=device).permute(*reversed(range(nd)))


def _check_reducible(src, opc, fc):
    if opc == _L.OP_AFFINE:
        raise ArgumentError("mapreduce needs a commutative operator; the affine operator is scan-only")
    if src.dtype not in _DTYPES:
        raise ArgumentError(f"unsupported element type {src.dtype}")


def _reduce_full_into(fc, opc, dst, src, tmp):
    """dst[0] = mapreduce(f, op, src) for any layout expressible as a
    column-major matrix (1-D strided views included)."""
    L = _L.lib()
    dt = _DTYPES[src.dtype]
    n = src.numel()
    if n == 0:
        raise ArgumentError("reducing over an empty collection is not allowed")
    merged = _merge(list(src.shape), list(src.stride()))
    stream = _stream_ptr(src)
    with _on(src.device):
        if merged is not None:
            need = L.kf_reduce_scratch_bytes(dt, n)
            buf = _scratch(MapReduce1D, need, src.device, tmp)
            rc = L.kf_reduce(opc, fc, dt, ctypes_void(src.data_ptr()), n, merged[1], ctypes_void(dst.data_ptr()),
                             ctypes_void(buf.ptr), buf.nbytes, stream)
            _L.check(rc, "mapreduce")
            return
        # two passes: columns of the first-dim-contiguous matrix, then the column results
        rows, cols, cs = _as_matrix(src, 1)
        part = torch.empty(cols, dtype=src.dtype, device=src.device)
        _reduce_dim_into(fc, opc, part, 1, src, rows, cols, cs, 1, None)
        need = L.kf_reduce_scratch_bytes(dt, cols)
        buf = _scratch(MapReduce1D, need, src.device, tmp)
        rc = L.kf_reduce(opc, _L.MAP_IDENTITY, dt, ctypes_void(part.data_ptr()), cols, 1,
                         ctypes_void(dst.data_ptr()), ctypes_void(buf.ptr), buf.nbytes, stream)
        _L.check(rc, "mapreduce")


def _reduce_dim_into(fc, opc, dst, dst_stride, src, rows, cols, cs, dim, tmp, base_ptr=None):
    L = _L.lib()
    dt = _DTYPES[src.dtype]
    need = L.kf_reduce_dim_scratch_bytes(dt, rows, cols, dim)
    buf = _scratch(MapReduce2D, need, src.device, tmp)
    ptr = src.data_ptr() if base_ptr is None else base_ptr
    with _on(src.device):
        rc = L.kf_reduce_dim(opc, fc, dt, ctypes_void(ptr), rows, cols, cs, dim, ctypes_void(dst.data_ptr()),
                             dst_stride, ctypes_void(buf.ptr), buf.nbytes, _stream_ptr(src))
    _L.check(rc, f"mapreduce(dims={dim})")


def _to_scalar(t):
    v = t.item()  # synchronises: every kernel queued so far has finished
    check_async()
    return v


def mapreduce(f, op, src, dims=None, g=None, tmp=None, **tuning):
    """mapreduce(f, op, src; dims=None) (reference src/mapreduce/mapreduce.jl:51-120).

    dims=None or ":" -> host scalar; otherwise a tensor with size 1 along the
    reduced dims, laid out column-major. `g` (post-map) is supported for the
    full reduction, where it is applied to the returned scalar."""
    if isinstance(src, (tuple, list)):
        return _mapreduce_multi(f, op, src, dims, g, tmp)
    fc, opc = _map_code(f), _op_code(op)
    _require_device(src)
    _check_reducible(src, opc, fc)
    if dims is None or dims == ":" or dims is Ellipsis:
        out = torch.empty(1, dtype=src.dtype, device=src.device)
        _reduce_full_into(fc, opc, out, src, tmp)
        val = _to_scalar(out)
        return g(val) if g is not None else val
    nd = src.dim()
    dims_t = _normalize_dims(dims, nd)
    shape = list(src.shape)
    out_shape = [1 if (i + 1) in dims_t else s for i, s in enumerate(shape)]
    dst = _colmajor_empty(out_shape, src.dtype, src.device)
    mapreduce_(f, op, dst, src, dims=dims_t, g=g, tmp=tmp)
    return dst


def _mapreduce_multi(f, op, srcs, dims, g, tmp):
    """mapreduce(f, op, (x, y[, z])) (reference src/mapreduce/mapreduce.jl:228-239):
    full reduction only, f(x, y) = x*y or (x-y)^2, f(x, y, z) = x*y*z,
    equal-length vectors."""
    if dims is not None and dims != ":" and dims is not Ellipsis:
        raise ArgumentError("Multi-array mapreduce only supports full reduction (dims=nothing)")
    _require_device(*srcs)
    out = torch.empty(1, dtype=srcs[0].dtype, device=srcs[0].device)
    _reduce2_into(f, op, out, srcs, tmp)
    val = _to_scalar(out)
    return g(val) if g is not None else val


def _map3_code(f):
    if f is operator.mul or f is prod3 or (isinstance(f, str) and f in ("mul", "*")):
        return _L.MAP3_MUL
    raise ArgumentError(f"unsupported three-array map {f!r}: expected prod3 (x*y*z) or operator.mul")


def _reduce2_into(f, op, out, srcs, tmp):
    """out[0] = op_i f(x[i], y[i]) through kf_reduce2, or op_i f(x[i], y[i],
    z[i]) through kf_reduce3 for three arrays."""
    if len(srcs) not in (2, 3):
        raise ArgumentError(f"multi-array mapreduce takes two or three arrays, got {len(srcs)}")
    fc = _map2_code(f) if len(srcs) == 2 else _map3_code(f)
    opc = _op_code(op)
    _require_device(out, *srcs)
    x = srcs[0]
    if any(a.dtype != x.dtype for a in srcs) or x.dtype not in _DTYPES or out.dtype != x.dtype:
        raise ArgumentError(f"element types {[a.dtype for a in srcs]} -> {out.dtype}: expected one supported type")
    if any(a.dim() != 1 or a.shape[0] != x.shape[0] for a in srcs):
        raise ArgumentError("multi-array mapreduce takes vectors of equal length")
    if opc == _L.OP_AFFINE:
        raise ArgumentError("mapreduce needs a commutative operator; the affine operator is scan-only")
    n = x.shape[0]
    if n == 0:
        raise ArgumentError("reducing over an empty collection is not allowed")
    L = _L.lib()
    dt = _DTYPES[x.dtype]
    args = []
    for a in srcs:
        args += [ctypes_void(a.data_ptr()), a.stride(0) if n > 1 else 1]
    if len(srcs) == 2:
        buf = _scratch(MapReduce1D, L.kf_reduce2_scratch_bytes(dt, n), x.device, tmp)
        entry = L.kf_reduce2
    else:
        buf = _scratch(MapReduce1D, L.kf_reduce3_scratch_bytes(dt, n), x.device, tmp)
        entry = L.kf_reduce3
    with _on(x.device):
        rc = entry(opc, fc, dt, *args, n, ctypes_void(out.data_ptr()), ctypes_void(buf.ptr), buf.nbytes,
                   _stream_ptr(x))
    _L.check(rc, "mapreduce")


def mapreduce1d(f, op, src, g=None, tmp=None, to_cpu=True, **tuning):
    """mapreduce1d(f, op, src_or_srcs; g, tmp, to_cpu=true) (reference
    src/mapreduce/1D/mapreduce1d.jl:177-209): a host scalar, or with
    to_cpu=False the 1-element device array holding it."""
    if to_cpu:
        return mapreduce(f, op, src, g=g, tmp=tmp)
    first = src[0] if isinstance(src, (tuple, list)) else src
    _require_device(first)
    dst = torch.empty(1, dtype=first.dtype, device=first.device)
    return mapreduce1d_(f, op, dst, src, g=g, tmp=tmp)


def mapreduce1d_(f, op, dst, src, g=None, tmp=None, **tuning):
    """mapreduce1d!(f, op, dst, src_or_srcs; g, tmp) (reference
    src/mapreduce/1D/mapreduce1d.jl:211-345): dst[1] = g(op_i f(src[i]))."""
    if not isinstance(src, (tuple, list)):
        return mapreduce_(f, op, dst, src, g=g, tmp=tmp)
    if _post_code(g) is None:
        raise ArgumentError(f"mapreduce1d!: unsupported post-map g={g!r}: expected identity, sqrt or abs2")
    if dst.numel() < 1:
        raise ArgumentError("dst must hold at least one element")
    _reduce2_into(f, op, dst.as_strided((1,), (1,)), src, tmp)
    _apply_post(g, dst, 1, 1)
    return dst


def mapreduce2d(f, op, src, dim, g=None, tmp=None, **tuning):
    """mapreduce2d(f, op, A, dim; g, tmp) (reference src/mapreduce/2D/mapreduce2d.jl:49-64):
    the vector of column (dim=1) or row (dim=2) reductions of a matrix."""
    if dim not in (1, 2):
        raise ArgumentError(f"dim must be 1 or 2, got {dim}")
    return vecmat(f, op, None, src, g=g, tmp=tmp) if dim == 1 else matvec(f, op, src, None, g=g, tmp=tmp)


def mapreduce2d_(f, op, dst, src, dim, g=None, tmp=None, **tuning):
    """mapreduce2d!(f, op, dst, A, dim; g, tmp) (reference src/mapreduce/2D/mapreduce2d.jl:111-126)."""
    if dim not in (1, 2):
        raise ArgumentError(f"dim must be 1 or 2, got {dim}")
    if dim == 1:
        return vecmat_(f, op, dst, None, src, g=g, tmp=tmp)
    return matvec_(f, op, dst, src, None, g=g, tmp=tmp)


def mapreducedims(f, op, src, dims, g=None, tmp=None, **tuning):
    """mapreducedims(f, op, src, dims; g) (reference src/mapreduce/ND/mapreducedims.jl:117-140):
    size 1 along `dims`, the source size elsewhere."""
    return mapreduce(f, op, src, dims=dims, g=g, tmp=tmp)


def mapreducedims_(f, op, dst, src, dims, g=None, tmp=None, **tuning):
    """mapreducedims!(f, op, dst, src, dims; g) (reference src/mapreduce/ND/mapreducedims.jl:146-163)."""
    return mapreduce_(f, op, dst, src, dims=dims, g=g, tmp=tmp)


def mapreduce_(f, op, dst, src, dims=None, g=None, tmp=None, **tuning):
    """mapreduce!(f, op, dst, src; dims=None) (reference src/mapreduce/mapreduce.jl:151-212)."""
    fc, opc = _map_code(f), _op_code(op)
    _require_device(dst, src)
    _check_reducible(src, opc, fc)
    if _post_code(g) is None:
        raise ArgumentError(f"mapreduce!: unsupported post-map g={g!r} on device results: "
                            "expected identity, sqrt or abs2")
    if dst.dtype != src.dtype:
        raise ArgumentError(f"dst eltype {dst.dtype} differs from src eltype {src.dtype}")
    if dims is None or dims == ":" or dims is Ellipsis:
        if dst.numel() < 1:
            raise ArgumentError("dst must hold at least one element")
        _reduce_full_into(fc, opc, dst.as_strided((1,), (1,)), src, tmp)
        _apply_post(g, dst, 1, 1)
        return dst
    nd = src.dim()
    dims_t = _normalize_dims(dims, nd)
    shape = list(src.shape)
    keep = [s for i, s in enumerate(shape) if (i + 1) not in dims_t]
    nkeep = 1
    for s in keep:
        nkeep *= s
    if dst.numel() != nkeep:
        raise ArgumentError(f"dst has {dst.numel()} elements, the reduction produces {nkeep}")
    dflat = _merge(list(dst.shape), list(dst.stride()))
    if dflat is None:
        raise ArgumentError("dst must be expressible as a strided vector")
    dst_stride = dflat[1]
    if src.numel() == 0:
        if nkeep:
            raise ArgumentError("reducing over an empty dimension is not allowed")
        return dst
    _mapreduce_dims_into(fc, opc, dst, dst_stride, src, dims_t, tmp)
    _apply_post(g, dst, nkeep, dst_stride)
    return dst


def _mapreduce_dims_into(fc, opc, dst, dst_stride, src, dims_t, tmp):
    """Route a dims reduction (reference src/mapreduce/mapreduce.jl:151-212)."""
    nd = src.dim()
    shape = list(src.shape)
    if len(dims_t) == nd:  # every dim: a full reduction into a (1,...,1) array
        _reduce_full_into(fc, opc, dst, src, tmp)
        return dst
    lead_end, tail_start = _classify_dims(dims_t, nd)
    leading, trailing = lead_end > 0, tail_start <= len(dims_t)
    if leading and not trailing:
        rows, cols, cs = _as_matrix(src, lead_end)
        _reduce_dim_into(fc, opc, dst, dst_stride, src, rows, cols, cs, 1, tmp)
        return dst
    if trailing and not leading:
        k = dims_t[tail_start - 1] - 1
        rows, cols, cs = _as_matrix(src, k)
        _reduce_dim_into(fc, opc, dst, dst_stride, src, rows, cols, cs, 2, tmp)
        return dst
    if leading and trailing:
        # trailing block first (no map afterwards), then the leading block
        k = dims_t[tail_start - 1] - 1
        rows, cols, cs = _as_matrix(src, k)
        mid = torch.empty(rows, dtype=src.dtype, device=src.device)
        _reduce_dim_into(fc, opc, mid, 1, src, rows, cols, cs, 2, tmp)
        lead = 1
        for s in shape[:lead_end]:
            lead *= s
        _reduce_dim_into(_L.MAP_IDENTITY, opc, dst, dst_stride, mid, lead, rows // lead, lead, 1, tmp)
        return dst
    _reduce_dims_general(fc, opc, dst, dst_stride, src, dims_t, tmp)
    return dst


def _blocks_of(dims0):
    """Contiguous runs [(d0, d1), ...] (0-based, half-open) of sorted dims."""
    out = []
    for d in dims0:
        if out and out[-1][1] == d:
            out[-1] = (out[-1][0], d + 1)
        else:
            out.append((d, d + 1))
    return out


def _reduce_dims_general(fc, opc, dst, dst_stride, src, dims_t, tmp):
    """Any set of dims: reduce one contiguous block of dims at a time, each
    block as the middle of a (pre, mid, post) view, with the batched dim-2
    kernel (or the dim-1 kernel when pre == 1). The reference does this
    with one thread per output in mapreducedims_kernel!
    (reference src/mapreduce/ND/mapreducedims_kernel.jl:1-23); the
    block-by-block form keeps every pass a coalesced streaming reduction.
    Valid for the commutative operators accepted here."""
    L = _L.lib()
    dt = _DTYPES[src.dtype]
    blocks = _blocks_of([d - 1 for d in dims_t])
    cur, cur_fc = src, fc
    for bi, (d0, d1) in enumerate(blocks):
        shape, strides = list(cur.shape), list(cur.stride())
        pre_m = _merge(shape[:d0], strides[:d0])
        mid_m = _merge(shape[d0:d1], strides[d0:d1])
        post_m = _merge(shape[d1:], strides[d1:])
        if pre_m is None or mid_m is None or post_m is None or (pre_m[0] > 1 and pre_m[1] != 1):
            raise NotImplementedError(
                f"layout with shape {tuple(shape)} and strides {tuple(strides)} cannot be reduced over "
                f"dims {d0 + 1}..{d1} without a copy")
        pre, mid, post = pre_m[0], mid_m[0], post_m[0]
        mid_stride = mid_m[1] if mid > 1 else max(pre, 1)
        post_stride = post_m[1] if post > 1 else 0
        last = bi == len(blocks) - 1
        out_shape = [1 if d0 <= i < d1 else v for i, v in enumerate(shape)]
        if last:
            out, out_stride = dst, dst_stride
        else:
            out, out_stride = _colmajor_empty(out_shape, src.dtype, src.device), 1
        with _on(src.device):
            if pre == 1 and mid_stride == 1:
                # leading block of a (mid, post) matrix: dim-1 kernel
                need = L.kf_reduce_dim_scratch_bytes(dt, mid, post, 1)
                buf = _scratch(MapReduce2D, need, src.device, tmp)
                rc = L.kf_reduce_dim(opc, cur_fc, dt, ctypes_void(cur.data_ptr()), mid, post,
                                     post_stride if post > 1 else mid, 1, ctypes_void(out.data_ptr()), out_stride,
                                     ctypes_void(buf.ptr), buf.nbytes, _stream_ptr(src))
            else:
                need = L.kf_reduce_dim_batched_scratch_bytes(dt, pre, mid, post)
                buf = _scratch(MapReduce2D, need, src.device, tmp)
                rc = L.kf_reduce_dim_batched(opc, cur_fc, dt, ctypes_void(cur.data_ptr()), pre, mid, mid_stride,
                                             post, post_stride, ctypes_void(out.data_ptr()), out_stride,
                                             ctypes_void(buf.ptr), buf.nbytes, _stream_ptr(src))
        _L.check(rc, f"mapreduce(dims={dims_t})")
        cur, cur_fc = out if not last else None, _L.MAP_IDENTITY


# ---------------------------------------------------------------------------
# matvec / vecmat (reference src/mapreduce/2D/matvec.jl:393-474,
# src/mapreduce/2D/vecmat.jl:328-405)
# ---------------------------------------------------------------------------
def _split_fop_kw(args, n_arrays, f, op, name):
    if len(args) == n_arrays + 2:
        return args[0], args[1], args[2:]
    if len(args) == n_arrays:
        return f, op, args
    raise ArgumentError(f"{name} takes ([f, op,] {n_arrays} arrays)")


def _dim_x_into(f, op, dst, A, x, dim, g, tmp, name):
    opc = _op_code(op)
    _require_device(dst, A, *(() if x is None else (x,)))
    if A.dim() != 2:
        raise ArgumentError(f"{name}: expected a matrix, got a {A.dim()}-d tensor")
    if A.dtype not in _DTYPES or dst.dtype != A.dtype or (x is not None and x.dtype != A.dtype):
        raise ArgumentError(f"{name}: operands must share one supported element type")
    if opc == _L.OP_AFFINE:
        raise ArgumentError(f"{name} needs a commutative operator")
    if _post_code(g) is None:
        raise ArgumentError(f"{name}: unsupported post-map g={g!r}: expected identity, sqrt or abs2")
    rows, cols, cs = _as_matrix(A, 1)
    m = rows if dim == 2 else cols
    k = cols if dim == 2 else rows
    dflat = _merge(list(dst.shape), list(dst.stride()))
    if dflat is None or dst.numel() != m:
        raise ArgumentError(f"{name}: dst must be a vector of length {m}")
    if x is None:  # the reference's x = nothing: a plain reduction with f applied to A
        fc = _L.MAP_ABS2 if (f is abs2 or f == "abs2") else _L.MAP_IDENTITY
        _reduce_dim_into(fc, opc, dst, dflat[1], A, rows, cols, cs, dim, tmp)
    else:
        if x.dim() != 1 or x.shape[0] != k:
            raise ArgumentError(f"{name}: x must be a vector of length {k}")
        fc = _map2_code(f)
        L = _L.lib()
        dt = _DTYPES[A.dtype]
        buf = _scratch(MapReduce2D, L.kf_reduce_dim_scratch_bytes(dt, rows, cols, dim), A.device, tmp)
        with _on(A.device):
            rc = L.kf_reduce_dim_x(opc, fc, dt, ctypes_void(A.data_ptr()), rows, cols, cs, dim,
                                   ctypes_void(x.data_ptr()), x.stride(0) if k > 1 else 1,
                                   ctypes_void(dst.data_ptr()), dflat[1], ctypes_void(buf.ptr), buf.nbytes,
                                   _stream_ptr(A))
        _L.check(rc, name)
    _apply_post(g, dst, m, dflat[1])
    return dst


def matvec(*args, f=operator.mul, op="+", g=None, tmp=None, **tuning):
    """matvec(A, x; f=*, op=+) or matvec(f, op, A, x): dst[i] = op_j f(A[i,j], x[j]).
    f: operator.mul or sqdiff; x=None reduces the rows of A (f unary)."""
    f, op, (A, x) = _split_fop_kw(args, 2, f, op, "matvec")
    _require_device(A)
    dst = torch.empty(A.shape[0], dtype=A.dtype, device=A.device)
    return _dim_x_into(f, op, dst, A, x, 2, g, tmp, "matvec")


def matvec_(*args, f=operator.mul, op="+", g=None, tmp=None, **tuning):
    """matvec!(dst, A, x; f=*, op=+) or matvec!(f, op, dst, A, x)."""
    f, op, (dst, A, x) = _split_fop_kw(args, 3, f, op, "matvec!")
    return _dim_x_into(f, op, dst, A, x, 2, g, tmp, "matvec!")


def vecmat(*args, f=operator.mul, op="+", g=None, tmp=None, **tuning):
    """vecmat(x, A; f=*, op=+) or vecmat(f, op, x, A): dst[j] = op_i f(x[i], A[i,j])."""
    f, op, (x, A) = _split_fop_kw(args, 2, f, op, "vecmat")
    _require_device(A)
    dst = torch.empty(A.shape[1], dtype=A.dtype, device=A.device)
    return _dim_x_into(f, op, dst, A, x, 1, g, tmp, "vecmat")


def vecmat_(*args, f=operator.mul, op="+", g=None, tmp=None, **tuning):
    """vecmat!(dst, x, A; f=*, op=+) or vecmat!(f, op, dst, x, A)."""
    f, op, (dst, x, A) = _split_fop_kw(args, 3, f, op, "vecmat!")
    return _dim_x_into(f, op, dst, A, x, 1, g, tmp, "vecmat!")


def get_allocation(kind, f, op, src, *args, **kwargs):
    """Scratch for a later call with the same operands (reference
    src/scan/scan.jl:121-211, src/mapreduce/1D/mapreduce1d.jl:113-170,
    src/mapreduce/2D/matvec.jl:182, src/mapreduce/2D/vecmat.jl:265).

    kind: Scan1D (src), MapReduce1D (src, or a tuple (x, y) of two arrays),
    MatVec (A, x) and VecMat (x, A) as the reference orders them, or
    MapReduce2D (A, dims=1 or 2). For Scan1D the reference's positional
    (workgroup, blocks) are honoured: the buffer fits the tile shape
    `workgroup` selects and at least `blocks` tiles (get_allocation(Scan1D,
    f, op, src, blocks) takes blocks alone, as an int). Other tuning
    arguments (arch, and those of the reductions) are accepted and
    ignored."""
    L = _L.lib()
    opc = _op_code(op)
    if kind == Scan1D:
        _map_code(f)
        _require_device(src)
        dt, n, _ = _scan_operand(src, opc)
        if len(args) == 1 and isinstance(args[0], int) and not isinstance(args[0], bool):
            workgroup, blocks = None, args[0]  # get_allocation(Scan1D, f, op, src, blocks; arch)
        else:
            workgroup = args[0] if len(args) > 0 else kwargs.get("workgroup")
            blocks = args[1] if len(args) > 1 else kwargs.get("blocks")
        wg, _ = _shape_keywords({"workgroup": workgroup}, "get_allocation")
        if blocks is not None and (isinstance(blocks, bool) or not isinstance(blocks, int) or blocks < 0):
            raise ArgumentError(f"get_allocation: blocks must be a non-negative integer, got {blocks!r}")
        need = L.kf_scan_shaped_scratch_bytes(dt, opc, n, wg, 0)
        if blocks is not None:
            need = max(need, 256 + 128 * blocks)  # header + one 128-byte descriptor line per tile
        device = src.device
    elif kind == MapReduce1D:
        if isinstance(src, (tuple, list)):
            _map2_code(f) if len(src) == 2 else _map3_code(f)
            _require_device(*src)
            need = L.kf_reduce2_scratch_bytes(_DTYPES[src[0].dtype], src[0].numel())
            device = src[0].device
        else:
            _map_code(f)
            _require_device(src)
            need = L.kf_reduce_scratch_bytes(_DTYPES[src.dtype], src.numel())
            device = src.device
    elif kind in (MatVec, VecMat, MapReduce2D):
        if kind == MatVec:
            A, dim = src, 2
        elif kind == VecMat:
            A, dim = (args[0] if args else kwargs["A"]), 1
        else:
            A, dim = src, int(kwargs.get("dims", args[0] if args else 1))
        _require_device(A)
        rows, cols, _ = _as_matrix(A, 1) if A.dim() == 2 else (A.numel(), 1, A.numel())
        need = L.kf_reduce_dim_scratch_bytes(_DTYPES[A.dtype], rows, cols, dim)
        device = A.device
    else:
        raise ArgumentError(f"unknown allocation kind {kind!r}")
    return KernelBuffer(kind, need, device)


def _rel_op(rel):
    """The reduction operator of maximum!(rel, ...): `<` keeps the larger, `>` the smaller."""
    if rel is operator.lt or rel == "<":
        return "max"
    if rel is operator.gt or rel == ">":
        return "min"
    raise ArgumentError(f"maximum!: the relation must be < or > (got {rel!r})")


def maximum_(rel, dst, src, tmp=None):
    """maximum!(rel, dst, src) (reference src/mapreduce/reductions.jl:3-6): the
    full reduction with op(x, y) = rel(x, y) ? y : x, i.e. max for `<`, min
    for `>`. Equal to the reference's on every input without NaN or a signed
    zero tie; there it follows Base max/min (NaN-propagating, -0.0 < +0.0)
    where the reference's select depends on its combine order."""
    return mapreduce_(identity, _rel_op(rel), dst, src, tmp=tmp)


def maximum(*args, tmp=None):
    """maximum([rel,] src) -> host scalar (reference src/mapreduce/reductions.jl:8-15)."""
    rel, (src,) = (operator.lt, args) if len(args) == 1 else (args[0], args[1:])
    return mapreduce(identity, _rel_op(rel), src, tmp=tmp)


def minimum(src, tmp=None):
    """minimum(src) = maximum(>, src) (reference src/mapreduce/reductions.jl:16)."""
    return maximum(operator.gt, src, tmp=tmp)


def vcopy_(dst, src):
    """vcopy!(dst, src) (reference src/copy/copy.jl:24-28): dst .= src for
    contiguous tensors of equal size in bytes."""
    _require_device(dst, src)
    if not (dst.is_contiguous() and src.is_contiguous()):
        raise ArgumentError("vcopy! needs contiguous tensors")
    nb = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() != nb:
        raise ArgumentError("vcopy!: size mismatch")
    with _on(src.device):
        rc = _L.lib().kf_copy(ctypes_void(dst.data_ptr()), ctypes_void(src.data_ptr()), nb, _stream_ptr(src))
    _L.check(rc, "vcopy!")
    return dst


def setvalue_(dst, val):
    """setvalue!(dst, val) (reference src/copy/copy.jl:52-56): every element
    of the contiguous tensor dst becomes val. A tuple val fills the rows of a
    2-D dst (one element = one row, e.g. affine (a, b) pairs)."""
    _require_device(dst)
    if not dst.is_contiguous():
        raise ArgumentError("setvalue! needs a contiguous tensor")
    if isinstance(val, (tuple, list)):
        if dst.dim() != 2 or dst.shape[1] != len(val):
            raise ArgumentError(f"a {len(val)}-tuple fills the rows of an (n, {len(val)}) tensor")
        elem = torch.tensor(list(val), dtype=dst.dtype)
        count = dst.shape[0]
    else:
        elem = torch.tensor([val], dtype=dst.dtype)
        count = dst.numel()
    raw = bytes(elem.view(torch.uint8).tolist())
    buf = ctypes.create_string_buffer(raw, len(raw))
    with _on(dst.device):
        rc = _L.lib().kf_fill(ctypes_void(dst.data_ptr()), count, ctypes.cast(buf, ctypes.c_void_p), len(raw),
                              _stream_ptr(dst))
    _L.check(rc, "setvalue!")
    return dst
