# KernelForgeHIP.jl: the Julia side of the MI355X drop-in for KernelForge.jl's
# scan! / mapreduce hot path. The public functions keep the reference's names,
# positional arguments and keywords (cited per function); underneath, every call
# goes through the C ABI of libkfhip.so (include/kf.h) with `ccall`, on the
# task-local AMDGPU stream. scan!'s launch-shape keywords (Nitem, workgroup)
# select the nearest compiled gfx950 tile shape (kf_scan_shaped); the other
# tuning keywords of the reference (blocks, family, arch, chunksz, and the
# reductions' shapes) are accepted and ignored: the library picks its own
# gfx950 launch shapes there.
#
# Supported operands: ROCArrays and strided views of them with eltype Float32,
# Float64, Int32, Int64, UInt8; NTuple{2,Float32} affine pairs (scan only);
# quaternion structs with fields (s, v1, v2, v3) of Float32 / Float64 (scan
# with *, Quaternions.jl's layout). Operators: +, max, min, *, and `affine`.
# Maps f: identity, abs2 (one array); *, sqdiff, wsq, expdiff (two arrays);
# prod3 / * (three arrays). Post-maps g on device results: identity, sqrt,
# abs2; a full reduction returned to the host takes any g.
#
# Errors follow the reference: ArgumentError for bad arguments (library codes
# KF_EINVAL / KF_ENOSCRATCH), ErrorException for HIP failures (KF_EHIP) and
# for a give-up of an earlier kernel (KF_EGIVEUP, see `check_async`).
module KernelForgeHIP

using AMDGPU

const libkf = normpath(joinpath(@__DIR__, "..", "libkfhip.so"))

# ---------------------------------------------------------------------------
# Algorithm tags and buffers (reference src/algorithms.jl:5-43,
# src/allocations.jl:16-41)
# ---------------------------------------------------------------------------
abstract type ForgeAlgorithm end
struct Scan1D <: ForgeAlgorithm end
struct MapReduce1D <: ForgeAlgorithm end
struct MapReduce2D <: ForgeAlgorithm end
struct MapReduceDims <: ForgeAlgorithm end
struct MatVec <: ForgeAlgorithm end
struct VecMat <: ForgeAlgorithm end

# `@allocate f(args...)` looks the algorithm up by the lowercase name of its
# tag type, with or without `!`, as the reference's table does.
const KERNEL_TAGS = Dict{Symbol,DataType}()
for T in (Scan1D, MapReduce1D, MapReduce2D, MapReduceDims, MatVec, VecMat)
    s = Symbol(lowercase(string(nameof(T))))
    KERNEL_TAGS[s] = T
    KERNEL_TAGS[Symbol(s, :!)] = T
end

"""
    KernelBuffer{Arrays<:NamedTuple}

Caller-owned scratch, as the reference's `KernelBuffer`: `arrays` holds one
zero-filled `ROCVector{UInt8}` under the key of its family, `scan` (tile
descriptors) or `reduce` (partials), so one buffer never serves both. It may
be reused across calls of its family; the kernels keep it valid (epoch tags).
"""
struct KernelBuffer{Arrays<:NamedTuple}
    arrays::Arrays
end

function _buffer(family::Symbol, nbytes::Integer)
    v = AMDGPU.zeros(UInt8, max(Int(nbytes), 256))
    family === :scan && (SCAN_BUFFERS[v] = nothing)
    return KernelBuffer(NamedTuple{(family,)}((v,)))
end

function _scratch(tmp::KernelBuffer, family::Symbol, need::Integer)
    haskey(tmp.arrays, family) ||
        throw(ArgumentError("tmp holds a $(keys(tmp.arrays)[1]) buffer; this call needs a $family buffer"))
    buf = tmp.arrays[family]
    length(buf) >= need || throw(ArgumentError("tmp holds $(length(buf)) bytes, this call needs $need"))
    return buf
end
_scratch(::Nothing, family::Symbol, need::Integer) = _buffer(family, need).arrays[family]

"""
    @allocate f(args...; kwargs...)

`get_allocation(Tag, args...; kwargs...)` for the algorithm named by `f`
(reference src/allocations.jl:20-41): `@allocate scan1d(identity, +, src)`.
"""
macro allocate(expr)
    (expr isa Expr && expr.head == :call) || error("@allocate expects a function call")
    tag = get(KERNEL_TAGS, expr.args[1], nothing)
    tag === nothing && error("Unknown ForgeAlgorithm: $(expr.args[1])")
    args = expr.args[2:end]
    call = Expr(:call, GlobalRef(@__MODULE__, :get_allocation))
    if !isempty(args) && args[1] isa Expr && args[1].head == :parameters
        push!(call.args, args[1], tag)   # keyword block stays right after the callee
        append!(call.args, args[2:end])
    else
        push!(call.args, tag)
        append!(call.args, args)
    end
    return esc(call)
end

# ---------------------------------------------------------------------------
# Codes of include/kf.h
# ---------------------------------------------------------------------------
"""
    affine

The non-commutative composition of affine maps, older map on the left:
`(a1, b1) ∘ (a2, b2) = (a2*a1, a2*b1 + b2)`; `scan!(affine, dst, ab)` runs the
recurrence `x_t = a_t x_{t-1} + b_t` over `NTuple{2,Float32}` pairs.
"""
struct AffineCompose <: Function end
(::AffineCompose)(p, q) = (q[1] * p[1], muladd(q[1], p[2], q[2]))
const affine = AffineCompose()

sqdiff(x, y) = abs2(x - y)
wsq(x, y) = x * y * y
expdiff(x, y) = exp(x - y)
prod3(x, y, z) = x * y * z

opcode(::typeof(+)) = Cint(0)
opcode(::typeof(max)) = Cint(1)
opcode(::typeof(min)) = Cint(2)
opcode(::AffineCompose) = Cint(3)
opcode(::typeof(*)) = Cint(4)
opcode(op) = throw(ArgumentError("unsupported operator $op: expected +, max, min, * or affine"))

mapcode(::typeof(identity)) = Cint(0)
mapcode(::typeof(abs2)) = Cint(1)
mapcode(f) = throw(ArgumentError("unsupported map $f: expected identity or abs2"))

map2code(::typeof(*)) = Cint(0)
map2code(::typeof(sqdiff)) = Cint(1)
map2code(::typeof(wsq)) = Cint(2)
map2code(::typeof(expdiff)) = Cint(3)
map2code(f) = throw(ArgumentError("unsupported two-array map $f: expected *, sqdiff, wsq or expdiff"))

map3code(::Union{typeof(prod3),typeof(*)}) = Cint(0)
map3code(f) = throw(ArgumentError("unsupported three-array map $f: expected prod3"))

postcode(::typeof(identity)) = Cint(0)
postcode(::typeof(sqrt)) = Cint(1)
postcode(::typeof(abs2)) = Cint(2)
postcode(g) = nothing

_isquat(T) = isbitstype(T) && fieldnames(T) == (:s, :v1, :v2, :v3)
function dtcode(::Type{T}) where {T}
    T === Float32 && return Cint(0)
    T === Float64 && return Cint(1)
    T === Int32 && return Cint(2)
    T === Int64 && return Cint(3)
    T === UInt8 && return Cint(4)
    T === NTuple{2,Float32} && return Cint(5)
    if _isquat(T)
        fieldtype(T, 1) === Float32 && return Cint(6)
        fieldtype(T, 1) === Float64 && return Cint(7)
    end
    throw(ArgumentError("unsupported element type $T"))
end

# Every live scan scratch vector, so that a give-up report can re-validate
# them all (their sticky flags would otherwise keep later scans inert).
const SCAN_BUFFERS = WeakKeyDict{ROCVector{UInt8},Nothing}()

function _check(rc::Cint, what)
    rc == 0 && return nothing
    msg = unsafe_string(ccall((:kf_last_error, libkf), Cstring, ()))
    rc in (Cint(1), Cint(2)) && throw(ArgumentError("$what: $msg"))
    rc == Cint(4) && error("$what: $msg $(_revalidate_scan_buffers())")
    error("$what: $msg")
end

function _revalidate_scan_buffers()
    hit = count(_scan_status, collect(keys(SCAN_BUFFERS)))
    hit > 0 && return "$hit scan scratch buffer(s) had given up: the scans on them since then stored " *
                      "nothing; they are valid again"
    return "(a reduction fold gave up: its destination was left untouched; its buffer is valid again)"
end

"""
    check_async()

Throw if a kernel queued earlier gave up waiting on its scratch buffer
(`kf_async_status`), after re-validating every scan buffer. Non-blocking: it
covers the kernels that have finished, so call it after a synchronisation
to cover them all. No counterpart in the reference, whose waits are unbounded.
"""
function check_async()
    flag = Ref{Cint}(0)
    _check(ccall((:kf_async_status, libkf), Cint, (Ptr{Cint},), flag), "check_async")
    flag[] != 0 && error("a scan lookback or reduction fold gave up waiting on its scratch buffer; " *
                         "its results are invalid. $(_revalidate_scan_buffers())")
    return nothing
end

_stream() = AMDGPU.stream().stream                        # hipStream_t of the task-local stream
devptr(A::AbstractArray) = Base.unsafe_convert(Ptr{eltype(A)}, A)

# (count, stride) of an array read in column-major order when one stride
# covers it (dense arrays, strided vectors, column views), else nothing.
function _merge(sz, st)
    count, stride, expect = 1, 0, 0
    for (s, t) in zip(sz, st)
        s == 1 && continue
        if stride == 0
            stride, expect = t, t * s
        elseif t != expect
            return nothing
        else
            expect = t * s
        end
        count *= s
    end
    return (count, stride == 0 ? 1 : stride)
end

function _linear(A::AbstractArray, what)
    m = _merge(size(A), strides(A))
    m === nothing && throw(ArgumentError("$what: the operand is not a strided vector"))
    return m[2]
end

# Dims [1, k] as rows and [k+1, nd] as columns of a column-major matrix:
# (rows, cols, col_stride); rows must be unit-stride.
function _as_matrix(A::AbstractArray, k::Int)
    sz, st = size(A), strides(A)
    r = _merge(sz[1:k], st[1:k])
    c = _merge(sz[k+1:end], st[k+1:end])
    (r === nothing || c === nothing || (r[1] > 1 && r[2] != 1)) &&
        throw(ArgumentError("layout $(sz) with strides $(st) is not a column-major matrix split at dim $k"))
    cs = c[1] > 1 ? c[2] : max(r[1], 1)
    c[1] > 1 && cs < r[1] && throw(ArgumentError("overlapping or row-major layout"))
    return r[1], c[1], cs
end

function _post!(g, dst::AbstractArray, n::Integer, stride::Integer)
    gc = postcode(g)
    gc === nothing && throw(ArgumentError("unsupported post-map g=$g on device results: expected identity, sqrt or abs2"))
    gc == 0 && return dst
    rc = ccall((:kf_post_map, libkf), Cint, (Cint, Cint, Ptr{Cvoid}, Int64, Int64, Ptr{Cvoid}),
               gc, dtcode(eltype(dst)), devptr(dst), n, stride, _stream())
    _check(rc, "post-map g")
    return dst
end

# ---------------------------------------------------------------------------
# scan! / scan (reference src/scan/scan.jl:121-284)
# ---------------------------------------------------------------------------
_shape_kw(v, name) = v === nothing ? Cint(0) :
    (v isa Integer && v > 0 ? Cint(v) : throw(ArgumentError("$name must be a positive integer, got $v")))

_scan_bytes(op, src, workgroup=nothing, Nitem=nothing) =
    ccall((:kf_scan_shaped_scratch_bytes, libkf), Csize_t, (Cint, Cint, Int64, Cint, Cint),
          dtcode(eltype(src)), opcode(op), length(src), _shape_kw(workgroup, "workgroup"), _shape_kw(Nitem, "Nitem"))

"""
    get_allocation(::Type{Scan1D}, f, op, src, workgroup=nothing, blocks=nothing, arch=nothing)
    get_allocation(::Type{Scan1D}, f, op, src, blocks::Int; arch=nothing)

A `KernelBuffer` for `scan!` on arrays like `src` (reference
src/scan/scan.jl:156-211): the size of the tile shape `workgroup` selects
(kf_scan_shaped_scratch_bytes), and at least a 256-byte header plus one
128-byte descriptor per tile of `blocks`. `arch` is accepted for
compatibility.
"""
function get_allocation(::Type{Scan1D}, f::F, op::O, src::AbstractArray, blocks::Int;
                        arch=nothing) where {F<:Function,O<:Function}
    blocks >= 0 || throw(ArgumentError("blocks must be non-negative, got $blocks"))
    return _buffer(:scan, max(_scan_bytes(op, src), 256 + 128 * blocks))
end

function get_allocation(::Type{Scan1D}, f::F, op::O, src::AbstractArray, workgroup=nothing,
                        blocks=nothing, arch=nothing) where {F<:Function,O<:Function}
    bytes = _scan_bytes(op, src, workgroup)
    blocks === nothing || (bytes = max(bytes, 256 + 128 * blocks))
    return _buffer(:scan, bytes)
end

"""
    scan_shape(src, op=+; Nitem=nothing, workgroup=nothing) -> (threads, items)

Threads per workgroup and elements per thread of the compiled tile shape a
`scan!` of `src` takes for these keywords (kf_scan_shape). No reference
counterpart: the reference compiles whatever shape it is given.
"""
function scan_shape(src::AbstractArray, op::O=+; Nitem=nothing, workgroup=nothing) where {O<:Function}
    threads, items = Ref{Cint}(0), Ref{Cint}(0)
    rc = ccall((:kf_scan_shape, libkf), Cint, (Cint, Int64, Cint, Cint, Ptr{Cint}, Ptr{Cint}),
               dtcode(eltype(src)), length(src), _shape_kw(workgroup, "workgroup"), _shape_kw(Nitem, "Nitem"),
               threads, items)
    _check(rc, "scan_shape")
    return (Int(threads[]), Int(items[]))
end

"""
    scan!([f,] op, dst, src; g=identity, tmp=nothing, Nitem, workgroup, family, arch,
          exclusive=false, check=false) -> dst

`dst[i] = g(f(src[1]) op ... op f(src[i]))` (reference src/scan/scan.jl:251-284).
`exclusive=true` gives `dst[1] = g(identity of op)`, `dst[i] = g(inclusive[i-1])`
(no reference counterpart). A lookback that gives up (see `scan_status`) is
reported by the library's next call after that kernel has finished (an
error), by `check_async` and by the full `mapreduce`'s read-back;
`check=true` synchronises and throws at once. `Nitem` (elements per thread) and
`workgroup` (threads per workgroup) select the nearest compiled tile shape
(`scan_shape`); `family` and `arch` are accepted for compatibility.
"""
function scan!(op::O, dst::AbstractArray, src::AbstractArray; kwargs...) where {O<:Function}
    return scan!(identity, op, dst, src; kwargs...)
end

function scan!(f::F, op::O, dst::AbstractArray, src::AbstractArray; g::G=identity, tmp=nothing,
               Nitem=nothing, workgroup=nothing, family=nothing, arch=nothing,
               exclusive::Bool=false, check::Bool=false) where {F<:Function,O<:Function,G<:Function}
    n = length(src)
    n == 0 && return dst
    length(dst) == n || throw(ArgumentError("dst has length $(length(dst)), src has length $n"))
    eltype(dst) === eltype(src) ||
        throw(ArgumentError("dst eltype $(eltype(dst)) differs from src eltype $(eltype(src))"))
    gc = postcode(g)
    gc === nothing && throw(ArgumentError("unsupported post-map g=$g: expected identity, sqrt or abs2"))
    wg, ni = _shape_kw(workgroup, "workgroup"), _shape_kw(Nitem, "Nitem")
    buf = _scratch(tmp, :scan, _scan_bytes(op, src, workgroup, Nitem))
    rc = ccall((:kf_scan_shaped, libkf), Cint,
               (Cint, Cint, Cint, Cint, Cint, Ptr{Cvoid}, Int64, Ptr{Cvoid}, Int64, Int64, Cint, Cint,
                Ptr{Cvoid}, Csize_t, Ptr{Cvoid}),
               opcode(op), mapcode(f), gc, dtcode(eltype(src)), Cint(exclusive),
               devptr(src), _linear(src, "scan!"), devptr(dst), _linear(dst, "scan!"), n, wg, ni,
               devptr(buf), length(buf), _stream())
    _check(rc, "scan!")
    if check && _scan_status(buf)
        # raised here, so the pending report is consumed
        _check(ccall((:kf_async_status, libkf), Cint, (Ptr{Cint},), Ref{Cint}(0)), "scan!")
        error("scan!: a tile's lookback gave up waiting for its predecessor; the results are invalid " *
              "(the scratch buffer has been re-validated) $(_revalidate_scan_buffers())")
    end
    return dst
end

"""
    scan([f,] op, src; kwargs...) -> dst

Allocating form of `scan!` (reference src/scan/scan.jl:218-244).
"""
function scan(op::O, src::AbstractArray; kwargs...) where {O<:Function}
    return scan(identity, op, src; kwargs...)
end

function scan(f::F, op::O, src::AbstractArray; g::G=identity, kwargs...) where {F<:Function,O<:Function,G<:Function}
    # a vector of length(src) with eltype promote_op(g, promote_op(f, T)), as
    # the reference allocates it (src/scan/scan.jl:226-244), for any shape of src
    H = Base.promote_op(g, Base.promote_op(f, eltype(src)))
    dst = similar(src, H, length(src))
    return scan!(f, op, dst, src; g, kwargs...)
end

function _scan_status(buf::ROCVector{UInt8})
    flag = Ref{Cint}(0)
    rc = ccall((:kf_scan_scratch_status, libkf), Cint, (Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cint}),
               devptr(buf), _stream(), flag)
    _check(rc, "scan_status")
    return flag[] != 0
end

"""
    scan_status(tmp::KernelBuffer) -> Bool

True if a `scan!` on `tmp` gave up waiting for a predecessor tile since the
last query; its results are invalid, and until this query later scans on
`tmp` store nothing. Clears the flag and re-validates the buffer;
synchronises the stream. No counterpart in the reference.
"""
scan_status(tmp::KernelBuffer) = _scan_status(_scratch(tmp, :scan, 0))

# ---------------------------------------------------------------------------
# Full reductions: mapreduce1d(!) (reference src/mapreduce/1D/mapreduce1d.jl:111-345)
# ---------------------------------------------------------------------------
_reduce_bytes(T, n) = ccall((:kf_reduce_scratch_bytes, libkf), Csize_t, (Cint, Int64), dtcode(T), n)
_reduce_bytes(T, n, k::Int) = k == 2 ?
    ccall((:kf_reduce2_scratch_bytes, libkf), Csize_t, (Cint, Int64), dtcode(T), n) :
    ccall((:kf_reduce3_scratch_bytes, libkf), Csize_t, (Cint, Int64), dtcode(T), n)

"""
    get_allocation(::Type{MapReduce1D}, f, op, src_or_srcs, workgroup=nothing, blocks=nothing, arch=nothing)

A `KernelBuffer` for `mapreduce1d!` / `mapreduce` over `src` or a tuple of
two or three arrays (reference src/mapreduce/1D/mapreduce1d.jl:140-170).
"""
function get_allocation(::Type{MapReduce1D}, f::F, op::O, src::AbstractArray, workgroup=nothing,
                        blocks=nothing, arch=nothing) where {F<:Function,O<:Function}
    return _buffer(:reduce, _reduce_bytes(eltype(src), length(src)))
end

function get_allocation(::Type{MapReduce1D}, f::F, op::O, srcs::NTuple{U,AbstractArray}, workgroup=nothing,
                        blocks=nothing, arch=nothing) where {U,F<:Function,O<:Function}
    U == 1 && return get_allocation(MapReduce1D, f, op, srcs[1])
    return _buffer(:reduce, _reduce_bytes(eltype(srcs[1]), length(srcs[1]), U))
end

# dst[1] = op_i f(src[i]) for a strided vector or any array viewable as a
# column-major matrix (reduced by columns, then the column results).
function _reduce_full!(f, op, dst::AbstractArray, src::AbstractArray, tmp)
    T = eltype(src)
    n = length(src)
    n == 0 && throw(ArgumentError("reducing over an empty collection is not allowed"))
    m = _merge(size(src), strides(src))
    if m !== nothing
        buf = _scratch(tmp, :reduce, _reduce_bytes(T, n))
        rc = ccall((:kf_reduce, libkf), Cint,
                   (Cint, Cint, Cint, Ptr{Cvoid}, Int64, Int64, Ptr{Cvoid}, Ptr{Cvoid}, Csize_t, Ptr{Cvoid}),
                   opcode(op), mapcode(f), dtcode(T), devptr(src), n, m[2], devptr(dst), devptr(buf),
                   length(buf), _stream())
        return _check(rc, "mapreduce")
    end
    rows, cols, cs = _as_matrix(src, 1)
    part = ROCVector{T}(undef, cols)
    _reduce_dim!(f, op, part, 1, devptr(src), T, rows, cols, cs, 1, nothing)
    _reduce_full!(identity, op, dst, part, tmp)
end

function _reduce_multi!(f, op, dst::AbstractArray, srcs::NTuple{U,AbstractArray}, tmp) where {U}
    T = eltype(srcs[1])
    n = length(srcs[1])
    all(s -> eltype(s) === T && length(s) == n, srcs) ||
        throw(ArgumentError("multi-array mapreduce takes arrays of one element type and length"))
    n == 0 && throw(ArgumentError("reducing over an empty collection is not allowed"))
    buf = _scratch(tmp, :reduce, _reduce_bytes(T, n, U))
    x, y = srcs[1], srcs[2]
    if U == 2
        rc = ccall((:kf_reduce2, libkf), Cint,
                   (Cint, Cint, Cint, Ptr{Cvoid}, Int64, Ptr{Cvoid}, Int64, Int64, Ptr{Cvoid}, Ptr{Cvoid}, Csize_t,
                    Ptr{Cvoid}),
                   opcode(op), map2code(f), dtcode(T), devptr(x), _linear(x, "mapreduce"), devptr(y),
                   _linear(y, "mapreduce"), n, devptr(dst), devptr(buf), length(buf), _stream())
    elseif U == 3
        z = srcs[3]
        rc = ccall((:kf_reduce3, libkf), Cint,
                   (Cint, Cint, Cint, Ptr{Cvoid}, Int64, Ptr{Cvoid}, Int64, Ptr{Cvoid}, Int64, Int64, Ptr{Cvoid},
                    Ptr{Cvoid}, Csize_t, Ptr{Cvoid}),
                   opcode(op), map3code(f), dtcode(T), devptr(x), _linear(x, "mapreduce"), devptr(y),
                   _linear(y, "mapreduce"), devptr(z), _linear(z, "mapreduce"), n, devptr(dst), devptr(buf),
                   length(buf), _stream())
    else
        throw(ArgumentError("multi-array mapreduce takes two or three arrays, got $U"))
    end
    _check(rc, "mapreduce")
end

"""
    mapreduce1d(f, op, src_or_srcs; g=identity, tmp=nothing, to_cpu=true, kwargs...)

Full reduction (reference src/mapreduce/1D/mapreduce1d.jl:177-209): a host
scalar `g(op_i f(src[i]))`, or with `to_cpu=false` the one-element device array.
"""
function mapreduce1d(f::F, op::O, src::AbstractArray; kwargs...) where {F<:Function,O<:Function}
    return mapreduce1d(f, op, (src,); kwargs...)
end

function mapreduce1d(f::F, op::O, srcs::NTuple{U,AbstractArray}; g::G=identity, tmp=nothing,
                     to_cpu::Bool=true, kwargs...) where {U,F<:Function,O<:Function,G<:Function}
    dst = ROCVector{eltype(srcs[1])}(undef, 1)
    if to_cpu
        mapreduce1d!(f, op, dst, srcs; tmp)
        v = Array(dst)[1]                 # the read-back synchronises; any g on the host
        check_async()
        return g(v)
    end
    return mapreduce1d!(f, op, dst, srcs; g, tmp)
end

"""
    mapreduce1d!(f, op, dst, src_or_srcs; g=identity, tmp=nothing, kwargs...)

`dst[1] = g(op_i f(src[i]))` on the device (reference
src/mapreduce/1D/mapreduce1d.jl:211-295).
"""
function mapreduce1d!(f::F, op::O, dst::AbstractArray, src::AbstractArray; kwargs...) where {F<:Function,O<:Function}
    return mapreduce1d!(f, op, dst, (src,); kwargs...)
end

function mapreduce1d!(f::F, op::O, dst::AbstractArray, srcs::NTuple{U,AbstractArray}; g::G=identity,
                      tmp=nothing, kwargs...) where {U,F<:Function,O<:Function,G<:Function}
    length(dst) >= 1 || throw(ArgumentError("dst must hold at least one element"))
    eltype(dst) === eltype(srcs[1]) ||
        throw(ArgumentError("dst eltype $(eltype(dst)) differs from src eltype $(eltype(srcs[1]))"))
    U == 1 ? _reduce_full!(f, op, dst, srcs[1], tmp) : _reduce_multi!(f, op, dst, srcs, tmp)
    return _post!(g, dst, 1, 1)
end

# ---------------------------------------------------------------------------
# Reductions along a dimension: matvec / vecmat / mapreduce2d
# (reference src/mapreduce/2D/matvec.jl:150-611, vecmat.jl:1-531,
# mapreduce2d.jl:49-126)
# ---------------------------------------------------------------------------
_dim_bytes(T, rows, cols, dim) = ccall((:kf_reduce_dim_scratch_bytes, libkf), Csize_t,
                                       (Cint, Int64, Int64, Cint), dtcode(T), rows, cols, dim)

# dst[k*dst_stride] for the rows x cols column-major matrix at p
function _reduce_dim!(f, op, dst, dst_stride, p, T, rows, cols, cs, dim, tmp)
    buf = _scratch(tmp, :reduce, _dim_bytes(T, rows, cols, dim))
    rc = ccall((:kf_reduce_dim, libkf), Cint,
               (Cint, Cint, Cint, Ptr{Cvoid}, Int64, Int64, Int64, Cint, Ptr{Cvoid}, Int64, Ptr{Cvoid}, Csize_t,
                Ptr{Cvoid}),
               opcode(op), mapcode(f), dtcode(T), p, rows, cols, cs, dim, devptr(dst), dst_stride, devptr(buf),
               length(buf), _stream())
    _check(rc, "mapreduce(dims=$dim)")
end

function _reduce_dim_x!(f, op, dst, A, x, dim, tmp)
    T = eltype(A)
    rows, cols = size(A)
    buf = _scratch(tmp, :reduce, _dim_bytes(T, rows, cols, dim))
    rc = ccall((:kf_reduce_dim_x, libkf), Cint,
               (Cint, Cint, Cint, Ptr{Cvoid}, Int64, Int64, Int64, Cint, Ptr{Cvoid}, Int64, Ptr{Cvoid}, Int64,
                Ptr{Cvoid}, Csize_t, Ptr{Cvoid}),
               opcode(op), map2code(f), dtcode(T), devptr(A), rows, cols, stride(A, 2), dim, devptr(x),
               _linear(x, "matvec"), devptr(dst), _linear(dst, "matvec"), devptr(buf), length(buf), _stream())
    _check(rc, dim == 2 ? "matvec" : "vecmat")
end

function _matrix_reduce!(f, op, dst, A::AbstractMatrix, x, dim, g, tmp)
    stride(A, 1) == 1 || throw(ArgumentError("the matrix must have unit row stride (column-major)"))
    n_out = dim == 1 ? size(A, 2) : size(A, 1)
    length(dst) == n_out || throw(ArgumentError("dst has length $(length(dst)), the reduction produces $n_out"))
    if x === nothing
        _reduce_dim!(f, op, dst, _linear(dst, "mapreduce2d!"), devptr(A), eltype(A), size(A, 1), size(A, 2),
                     stride(A, 2), dim, tmp)
    else
        length(x) == size(A, 3 - dim) || throw(ArgumentError("x has length $(length(x)), expected $(size(A, 3 - dim))"))
        _reduce_dim_x!(f, op, dst, A, x, dim, tmp)
    end
    return _post!(g, dst, n_out, _linear(dst, "mapreduce2d!"))
end

"""
    get_allocation(::Type{MatVec}, f, op, src, x, chunksz=nothing, Nblocks=nothing, workgroup=nothing,
                   blocks_row=nothing, Nitem=nothing, arch=nothing)

A `KernelBuffer` for `matvec!` (reference src/mapreduce/2D/matvec.jl:210-250).
"""
function get_allocation(::Type{MatVec}, f::F, op::O, src::AbstractMatrix, x::Union{AbstractArray,Nothing},
                        chunksz=nothing, Nblocks=nothing, workgroup=nothing, blocks_row=nothing, Nitem=nothing,
                        arch=nothing) where {F<:Function,O<:Function}
    return _buffer(:reduce, _dim_bytes(eltype(src), size(src, 1), size(src, 2), 2))
end

"""
    get_allocation(::Type{VecMat}, f, op, x, src, Nitem=nothing, Nthreads=nothing, workgroup=nothing,
                   blocks=nothing, arch=nothing; flag_alloc=Val(true))

A `KernelBuffer` for `vecmat!` (reference src/mapreduce/2D/vecmat.jl:292-330).
"""
function get_allocation(::Type{VecMat}, f::F, op::O, x::Union{AbstractArray,Nothing}, src::AbstractMatrix,
                        Nitem=nothing, Nthreads=nothing, workgroup=nothing, blocks=nothing, arch=nothing;
                        flag_alloc=Val(true)) where {F<:Function,O<:Function}
    return _buffer(:reduce, _dim_bytes(eltype(src), size(src, 1), size(src, 2), 1))
end

"""
    get_allocation(::Type{MapReduce2D}, f, op, src, dim)

A `KernelBuffer` for `mapreduce2d!` along `dim` (the reference sizes it
inside matvec / vecmat).
"""
function get_allocation(::Type{MapReduce2D}, f::F, op::O, src::AbstractMatrix, dim::Int) where {F<:Function,O<:Function}
    return _buffer(:reduce, _dim_bytes(eltype(src), size(src, 1), size(src, 2), dim))
end

"""
    matvec([f, op,] src, x; g=identity, tmp=nothing, kwargs...)

`dst[i] = g(op_j f(src[i,j], x[j]))`, or `op_j f(src[i,j])` with `x = nothing`
(reference src/mapreduce/2D/matvec.jl:393-438).
"""
function matvec(src::AbstractMatrix, x::Union{AbstractArray,Nothing}; f::F=*, op::O=+, kwargs...) where {F<:Function,O<:Function}
    return matvec(f, op, src, x; kwargs...)
end

function matvec(f::F, op::O, src::AbstractMatrix, x::Union{AbstractArray,Nothing}; g::G=identity, tmp=nothing,
                kwargs...) where {F<:Function,O<:Function,G<:Function}
    dst = ROCVector{eltype(src)}(undef, size(src, 1))
    return _matrix_reduce!(f, op, dst, src, x, 2, g, tmp)
end

function matvec!(dst::AbstractArray, src::AbstractMatrix, x::Union{AbstractArray,Nothing}; f::F=*, op::O=+,
                 kwargs...) where {F<:Function,O<:Function}
    return matvec!(f, op, dst, src, x; kwargs...)
end

function matvec!(f::F, op::O, dst::AbstractArray, src::AbstractMatrix, x::Union{AbstractArray,Nothing};
                 g::G=identity, tmp=nothing, kwargs...) where {F<:Function,O<:Function,G<:Function}
    return _matrix_reduce!(f, op, dst, src, x, 2, g, tmp)
end

"""
    vecmat([f, op,] x, src; g=identity, tmp=nothing, kwargs...)

`dst[j] = g(op_i f(x[i], src[i,j]))`, or `op_i f(src[i,j])` with `x = nothing`
(reference src/mapreduce/2D/vecmat.jl:328-405).
"""
function vecmat(x::Union{AbstractArray,Nothing}, src::AbstractMatrix; f::F=*, op::O=+, kwargs...) where {F<:Function,O<:Function}
    return vecmat(f, op, x, src; kwargs...)
end

function vecmat(f::F, op::O, x::Union{AbstractArray,Nothing}, src::AbstractMatrix; g::G=identity, tmp=nothing,
                kwargs...) where {F<:Function,O<:Function,G<:Function}
    dst = ROCVector{eltype(src)}(undef, size(src, 2))
    return _matrix_reduce!(f, op, dst, src, x, 1, g, tmp)
end

function vecmat!(dst::AbstractArray, x::Union{AbstractArray,Nothing}, src::AbstractMatrix; f::F=*, op::O=+,
                 kwargs...) where {F<:Function,O<:Function}
    return vecmat!(f, op, dst, x, src; kwargs...)
end

function vecmat!(f::F, op::O, dst::AbstractArray, x::Union{AbstractArray,Nothing}, src::AbstractMatrix;
                 g::G=identity, tmp=nothing, kwargs...) where {F<:Function,O<:Function,G<:Function}
    return _matrix_reduce!(f, op, dst, src, x, 1, g, tmp)
end

"""
    mapreduce2d(f, op, src, dim; g=identity, tmp=nothing, kwargs...)
    mapreduce2d!(f, op, dst, src, dim; g=identity, tmp=nothing, kwargs...)

Column (`dim=1`) or row (`dim=2`) reductions of a matrix (reference
src/mapreduce/2D/mapreduce2d.jl:49-126).
"""
function mapreduce2d(f::F, op::O, src::AbstractMatrix, dim::Int; g::G=identity, tmp=nothing,
                     kwargs...) where {F<:Function,O<:Function,G<:Function}
    dim == 1 && return vecmat(f, op, nothing, src; g, tmp)
    dim == 2 && return matvec(f, op, src, nothing; g, tmp)
    throw(ArgumentError("dim must be 1 or 2, got $dim"))
end

function mapreduce2d!(f::F, op::O, dst::AbstractArray, src::AbstractMatrix, dim::Int; g::G=identity,
                      tmp=nothing, kwargs...) where {F<:Function,O<:Function,G<:Function}
    dim == 1 && return vecmat!(f, op, dst, nothing, src; g, tmp)
    dim == 2 && return matvec!(f, op, dst, src, nothing; g, tmp)
    throw(ArgumentError("dim must be 1 or 2, got $dim"))
end

# ---------------------------------------------------------------------------
# mapreduce(f, op, src; dims) and its routing (reference
# src/mapreduce/mapreduce.jl:51-298, src/helpers.jl:194-198)
# ---------------------------------------------------------------------------
_normalize_dims(dims::Int, nd::Int) = (dims > 0 ? dims : nd + dims + 1,)
_normalize_dims(dims::NTuple{N,Int}, nd::Int) where {N} = Tuple(sort!([d > 0 ? d : nd + d + 1 for d in dims]))
_normalize_dims(dims::AbstractVector{<:Integer}, nd::Int) = _normalize_dims(Tuple(Int.(dims)), nd)

function _validate_dims(dims::NTuple{N,Int}, nd::Int) where {N}
    for d in dims
        1 <= d <= nd || throw(ArgumentError("dimension $d out of range for $nd-dimensional array"))
    end
    allunique(dims) || throw(ArgumentError("duplicate dimensions in dims=$dims"))
    return nothing
end

# (lead_end, tail_start) over the sorted dims: dims[1:lead_end] == 1:lead_end
# and dims[tail_start:end] are the last dims; (0, N+1) when the dims are not
# one leading block, one trailing block, or one of each.
function _classify_dims(dims::NTuple{N,Int}, nd::Int) where {N}
    lead_end = 0
    while lead_end < N && dims[lead_end+1] == lead_end + 1
        lead_end += 1
    end
    tail_start = N + 1
    while tail_start > 1 && dims[tail_start-1] == nd - (N - tail_start + 1)
        tail_start -= 1
    end
    if lead_end > 0 && tail_start <= N && all(i -> dims[i+1] == dims[i] + 1, 1:N-1)
        return (lead_end, N + 1)          # one block touching both ends: leading
    end
    lead_end + (N + 1 - tail_start) == N || return (0, N + 1)
    return (lead_end, tail_start)
end

"""
    mapreduce(f, op, src; dims=nothing, g=identity, tmp=nothing, kwargs...)

`dims = nothing` or `:`: the host scalar `g(op_i f(src[i]))`. Otherwise a
device array with size 1 along the reduced dims (reference
src/mapreduce/mapreduce.jl:51-120).
"""
function mapreduce(f::F, op::O, src::AbstractArray{T}; dims=nothing, g::G=identity,
                   kwargs...) where {T,F<:Function,O<:Function,G<:Function}
    dims === Colon() && (dims = nothing)
    dims === nothing && return mapreduce1d(f, op, src; g, to_cpu=true, kwargs...)
    nd = ndims(src)
    d = _normalize_dims(dims, nd)
    _validate_dims(d, nd)
    dst = ROCArray{T}(undef, ntuple(i -> i in d ? 1 : size(src, i), nd))
    return mapreduce!(f, op, dst, src; dims=d, g, kwargs...)
end

"""
    mapreduce(f, op, srcs::NTuple; dims=nothing, g=identity, kwargs...)

Two- or three-array full reduction (reference src/mapreduce/mapreduce.jl:228-239).
"""
function mapreduce(f::F, op::O, srcs::NTuple{U,AbstractArray}; dims=nothing, g::G=identity,
                   kwargs...) where {U,F<:Function,O<:Function,G<:Function}
    (dims === nothing || dims === Colon()) ||
        throw(ArgumentError("Multi-array mapreduce only supports full reduction (dims=nothing)"))
    return mapreduce1d(f, op, srcs; g, to_cpu=true, kwargs...)
end

"""
    mapreduce!(f, op, dst, src; dims=nothing, g=identity, tmp=nothing, kwargs...)

In-place form (reference src/mapreduce/mapreduce.jl:151-212): `dims = nothing`
writes `dst[1]`; otherwise `dst` holds the kept dims' elements.
"""
function mapreduce!(f::F, op::O, dst::AbstractArray, src::AbstractArray; dims=nothing, g::G=identity,
                    tmp=nothing, kwargs...) where {F<:Function,O<:Function,G<:Function}
    dims === Colon() && (dims = nothing)
    dims === nothing && return mapreduce1d!(f, op, dst, src; g, tmp)
    nd = ndims(src)
    d = _normalize_dims(dims, nd)
    _validate_dims(d, nd)
    length(d) == nd && return mapreducedims!(f, op, dst, src, d; g, tmp)
    nkeep = prod(i -> i in d ? 1 : size(src, i), 1:nd)
    length(dst) == nkeep || throw(ArgumentError("dst has $(length(dst)) elements, the reduction produces $nkeep"))
    T = eltype(src)
    ds = _linear(dst, "mapreduce!")
    lead_end, tail_start = _classify_dims(d, nd)
    leading, trailing = lead_end > 0, tail_start <= length(d)
    if leading && !trailing
        rows, cols, cs = _as_matrix(src, lead_end)
        _reduce_dim!(f, op, dst, ds, devptr(src), T, rows, cols, cs, 1, tmp)
    elseif trailing && !leading
        rows, cols, cs = _as_matrix(src, d[tail_start] - 1)
        _reduce_dim!(f, op, dst, ds, devptr(src), T, rows, cols, cs, 2, tmp)
    elseif leading && trailing
        # the trailing block first, then the leading block of its result
        rows, cols, cs = _as_matrix(src, d[tail_start] - 1)
        mid = ROCVector{T}(undef, rows)
        _reduce_dim!(f, op, mid, 1, devptr(src), T, rows, cols, cs, 2, tmp)
        lead = prod(size(src)[1:lead_end])
        _reduce_dim!(identity, op, dst, ds, devptr(mid), T, lead, rows ÷ lead, lead, 1, tmp)
    else
        _reduce_blocks!(f, op, dst, ds, src, d, tmp)
    end
    return _post!(g, dst, nkeep, ds)
end

# Any set of dims, one contiguous block of dims at a time: the block is the
# middle of a (pre, mid, post) view of the current array, reduced by
# kf_reduce_dim_batched (or kf_reduce_dim when pre == 1). Valid for the
# commutative operators the reductions accept. The reference's fallback is
# one thread per output (src/mapreduce/ND/mapreducedims_kernel.jl:1-23).
function _reduce_blocks!(f, op, dst, ds, src, d, tmp)
    T = eltype(src)
    blocks = Tuple{Int,Int}[]
    for k in d
        if !isempty(blocks) && blocks[end][2] == k - 1
            blocks[end] = (blocks[end][1], k)
        else
            push!(blocks, (k, k))
        end
    end
    cur, fcur = src, f
    for (bi, (d0, d1)) in enumerate(blocks)
        sz, st = size(cur), strides(cur)
        pre_m = _merge(sz[1:d0-1], st[1:d0-1])
        mid_m = _merge(sz[d0:d1], st[d0:d1])
        post_m = _merge(sz[d1+1:end], st[d1+1:end])
        (pre_m === nothing || mid_m === nothing || post_m === nothing || (pre_m[1] > 1 && pre_m[2] != 1)) &&
            throw(ArgumentError("layout $(sz) with strides $(st) cannot be reduced over dims $d0:$d1 without a copy"))
        pre, mid, post = pre_m[1], mid_m[1], post_m[1]
        mid_stride = mid > 1 ? mid_m[2] : max(pre, 1)
        post_stride = post > 1 ? post_m[2] : 0
        last = bi == length(blocks)
        out = last ? dst : ROCArray{T}(undef, ntuple(i -> d0 <= i <= d1 ? 1 : sz[i], length(sz)))
        os = last ? ds : 1
        if pre == 1 && mid_stride == 1
            _reduce_dim!(fcur, op, out, os, devptr(cur), T, mid, post, post > 1 ? post_stride : mid, 1, tmp)
        else
            need = ccall((:kf_reduce_dim_batched_scratch_bytes, libkf), Csize_t, (Cint, Int64, Int64, Int64),
                         dtcode(T), pre, mid, post)
            buf = _scratch(tmp, :reduce, need)
            rc = ccall((:kf_reduce_dim_batched, libkf), Cint,
                       (Cint, Cint, Cint, Ptr{Cvoid}, Int64, Int64, Int64, Int64, Int64, Ptr{Cvoid}, Int64, Ptr{Cvoid},
                        Csize_t, Ptr{Cvoid}),
                       opcode(op), mapcode(fcur), dtcode(T), devptr(cur), pre, mid, mid_stride, post, post_stride,
                       devptr(out), os, devptr(buf), length(buf), _stream())
            _check(rc, "mapreduce(dims=$d)")
        end
        cur, fcur = out, identity
    end
    return dst
end

"""
    mapreducedims(f, op, src, dims; g=identity, kwargs...)
    mapreducedims!(f, op, dst, src, dims; g=identity, kwargs...)

Reduction over any set of dims (reference src/mapreduce/ND/mapreducedims.jl:117-163).
"""
function mapreducedims(f::F, op::O, src::AbstractArray{T}, dims; g::G=identity, tmp=nothing,
                       kwargs...) where {T,F<:Function,O<:Function,G<:Function}
    nd = ndims(src)
    d = _normalize_dims(dims, nd)
    _validate_dims(d, nd)
    dst = ROCArray{T}(undef, ntuple(i -> i in d ? 1 : size(src, i), nd))
    return mapreducedims!(f, op, dst, src, d; g, tmp)
end

function mapreducedims!(f::F, op::O, dst::AbstractArray, src::AbstractArray, dims; g::G=identity, tmp=nothing,
                        kwargs...) where {F<:Function,O<:Function,G<:Function}
    nd = ndims(src)
    d = _normalize_dims(dims, nd)
    _validate_dims(d, nd)
    if length(d) == nd
        _reduce_full!(f, op, dst, src, tmp)
        return _post!(g, dst, 1, 1)
    end
    return mapreduce!(f, op, dst, src; dims=d, g, tmp)
end

"""
    maximum([rel,] src), minimum(src)

Largest / smallest element (reference src/mapreduce/reductions.jl:1-16);
`rel` = `<` or `>` select max / min.
"""
maximum(src::AbstractArray) = mapreduce1d(identity, max, src)
minimum(src::AbstractArray) = mapreduce1d(identity, min, src)
function maximum(rel::F, src::AbstractArray) where {F<:Function}
    rel === (<) && return mapreduce1d(identity, max, src)
    rel === (>) && return mapreduce1d(identity, min, src)
    throw(ArgumentError("maximum(rel, src) supports rel = < or >"))
end

# ---------------------------------------------------------------------------
# vcopy! / setvalue! (reference src/copy/copy.jl:24-56)
# ---------------------------------------------------------------------------
function vcopy!(dst::AbstractArray, src::AbstractArray)
    length(dst) == length(src) && eltype(dst) === eltype(src) ||
        throw(ArgumentError("vcopy! needs arrays of one element type and length"))
    (_linear(dst, "vcopy!") == 1 && _linear(src, "vcopy!") == 1) ||
        throw(ArgumentError("vcopy! needs contiguous arrays"))
    rc = ccall((:kf_copy, libkf), Cint, (Ptr{Cvoid}, Ptr{Cvoid}, Csize_t, Ptr{Cvoid}),
               devptr(dst), devptr(src), sizeof(eltype(src)) * length(src), _stream())
    _check(rc, "vcopy!")
    return dst
end

function setvalue!(dst::AbstractArray{T}, val) where {T}
    _linear(dst, "setvalue!") == 1 || throw(ArgumentError("setvalue! needs a contiguous array"))
    v = Ref{T}(convert(T, val))
    rc = GC.@preserve v ccall((:kf_fill, libkf), Cint, (Ptr{Cvoid}, Int64, Ptr{Cvoid}, Csize_t, Ptr{Cvoid}),
                              devptr(dst), length(dst), Base.unsafe_convert(Ptr{T}, v), sizeof(T), _stream())
    _check(rc, "setvalue!")
    return dst
end

end # module
