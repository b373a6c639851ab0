"""The Julia binding (kernelforge.jl_amd/julia/KernelForgeHIP.jl) against
include/kf.h and against the reference's public signatures. There is no
julia in this environment, so the binding is checked as text: every
`ccall((:kf_..., libkf), R, (A...), ...)` must name a declared C function
with the matching return and argument types, and the reference's entry
points (reference src/scan/scan.jl:156-284, src/allocations.jl:16-41,
src/mapreduce/mapreduce.jl:51-212, src/mapreduce/1D/mapreduce1d.jl:140-295,
src/mapreduce/2D/mapreduce2d.jl:49-126, src/mapreduce/ND/mapreducedims.jl:117-163)
must be defined with their positional arguments."""
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
JL = os.path.join(REPO, "kernelforge.jl_amd", "julia", "KernelForgeHIP.jl")
HEADER = os.path.join(REPO, "include", "kf.h")

ENUMS = {"kf_op", "kf_map", "kf_post", "kf_dtype", "kf_map2", "kf_map3"}
C_TO_JULIA = {"int": "Cint", "int64_t": "Int64", "size_t": "Csize_t", "uint32_t": "UInt32",
              "void*": "Ptr{Cvoid}", "int*": "Ptr{Cint}", "char*": "Cstring"}


def _ctype(decl):
    """Julia ccall type of one C parameter or return declaration."""
    decl = decl.replace("const ", "").strip()
    decl = re.sub(r"\s*\*\s*", "* ", decl).strip()
    parts = decl.split()
    # drop the parameter name (the last word, unless the whole decl is a type)
    if len(parts) > 1 and not parts[-1].endswith("*"):
        base = " ".join(parts[:-1])
    else:
        base = " ".join(parts)
    base = base.replace(" ", "").replace("*", "*")
    if base in ENUMS:
        return "Cint"
    if base not in C_TO_JULIA:
        raise AssertionError(f"no Julia mapping for C type {decl!r}")
    return C_TO_JULIA[base]


def header_prototypes():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"typedef enum\s*\{.*?\}\s*\w+\s*;", "", text, flags=re.S)
    protos = {}
    for m in re.finditer(r"([\w\s\*]+?)\b(kf_\w+)\s*\(([^)]*)\)\s*;", text):
        ret, name, args = m.group(1).strip(), m.group(2), m.group(3).strip()
        ret = ret.split("\n")[-1].strip()
        params = [] if args in ("", "void") else [_ctype(a) for a in args.split(",")]
        protos[name] = (_ctype(ret + " r"), params)
    return protos


CCALL = re.compile(r"ccall\(\(:(kf_\w+),\s*libkf\),\s*([\w{}]+),\s*\(([^()]*)\)", re.S)


def julia_ccalls(text):
    out = []
    for m in CCALL.finditer(text):
        args = [a.strip() for a in m.group(3).replace("\n", " ").split(",") if a.strip()]
        out.append((m.group(1), m.group(2), args))
    return out


def test_header_parses_every_declared_function():
    protos = header_prototypes()
    assert protos["kf_scan"] == ("Cint", ["Cint", "Cint", "Cint", "Cint", "Cint", "Ptr{Cvoid}", "Int64",
                                          "Ptr{Cvoid}", "Int64", "Int64", "Ptr{Cvoid}", "Csize_t", "Ptr{Cvoid}"])
    assert protos["kf_last_error"] == ("Cstring", [])
    assert protos["kf_scan_scratch_status"][1] == ["Ptr{Cvoid}", "Ptr{Cvoid}", "Ptr{Cint}"]


def test_every_ccall_matches_kf_h():
    protos = header_prototypes()
    calls = julia_ccalls(open(JL).read())
    assert len(calls) >= 15
    for name, ret, args in calls:
        assert name in protos, f"{name} is not declared in include/kf.h"
        cret, cargs = protos[name]
        assert ret == cret, f"{name}: returns {cret} in kf.h, {ret} in the binding"
        assert args == cargs, f"{name}: kf.h {cargs} vs binding {args}"
    # the hot path's entry points are all bound
    bound = {c[0] for c in calls}
    for name in ("kf_scan_shaped", "kf_scan_shaped_scratch_bytes", "kf_scan_shape", "kf_scan_scratch_status",
                 "kf_reduce", "kf_reduce_scratch_bytes",
                 "kf_reduce2", "kf_reduce3", "kf_reduce_dim", "kf_reduce_dim_x", "kf_reduce_dim_scratch_bytes",
                 "kf_reduce_dim_batched", "kf_reduce_dim_batched_scratch_bytes", "kf_post_map", "kf_copy", "kf_fill",
                 "kf_last_error"):
        assert name in bound, name


def test_integration_md_names_the_binding_and_its_ccalls_match():
    text = open(os.path.join(REPO, "INTEGRATION.md")).read()
    assert "kernelforge.jl_amd/julia/KernelForgeHIP.jl" in text
    protos = header_prototypes()
    for block in re.findall(r"```julia\n(.*?)```", text, flags=re.S):
        for name, ret, args in julia_ccalls(block):
            assert protos[name] == (ret, args), name


# (function name, regex of its positional signature) per reference entry point
SIGNATURES = [
    ("get_allocation(::Type{Scan1D}, f, op, src, workgroup, blocks, arch)",
     r"function get_allocation\(::Type\{Scan1D\}, f::F, op::O, src::AbstractArray, workgroup=nothing,\s*blocks=nothing, arch=nothing\)"),
    ("get_allocation(::Type{Scan1D}, f, op, src, blocks::Int; arch)",
     r"function get_allocation\(::Type\{Scan1D\}, f::F, op::O, src::AbstractArray, blocks::Int;\s*arch=nothing\)"),
    ("get_allocation(::Type{MapReduce1D}, f, op, src, workgroup, blocks, arch)",
     r"function get_allocation\(::Type\{MapReduce1D\}, f::F, op::O, src::AbstractArray, workgroup=nothing,\s*blocks=nothing, arch=nothing\)"),
    ("get_allocation(::Type{MapReduce1D}, f, op, srcs::NTuple, ...)",
     r"function get_allocation\(::Type\{MapReduce1D\}, f::F, op::O, srcs::NTuple\{U,AbstractArray\}"),
    ("get_allocation(::Type{MatVec}, f, op, src, x, ...)",
     r"function get_allocation\(::Type\{MatVec\}, f::F, op::O, src::AbstractMatrix, x::Union\{AbstractArray,Nothing\}"),
    ("get_allocation(::Type{VecMat}, f, op, x, src, ...; flag_alloc)",
     r"function get_allocation\(::Type\{VecMat\}, f::F, op::O, x::Union\{AbstractArray,Nothing\}, src::AbstractMatrix,[^;]*;\s*flag_alloc=Val\(true\)\)"),
    ("scan!(op, dst, src; kw...)", r"function scan!\(op::O, dst::AbstractArray, src::AbstractArray; kwargs\.\.\.\)"),
    ("scan!(f, op, dst, src; g, tmp, Nitem, workgroup, family, arch)",
     r"function scan!\(f::F, op::O, dst::AbstractArray, src::AbstractArray; g::G=identity, tmp=nothing,\s*Nitem=nothing, workgroup=nothing, family=nothing, arch=nothing"),
    ("scan(op, src; kw...)", r"function scan\(op::O, src::AbstractArray; kwargs\.\.\.\)"),
    ("scan(f, op, src; kw...)", r"function scan\(f::F, op::O, src::AbstractArray; g::G=identity, kwargs\.\.\.\)"),
    ("mapreduce(f, op, src; dims, g, kwargs...)",
     r"function mapreduce\(f::F, op::O, src::AbstractArray\{T\}; dims=nothing, g::G=identity,\s*kwargs\.\.\.\)"),
    ("mapreduce(f, op, srcs::NTuple; dims, g)", r"function mapreduce\(f::F, op::O, srcs::NTuple\{U,AbstractArray\}; dims=nothing"),
    ("mapreduce!(f, op, dst, src; dims, g, kwargs...)",
     r"function mapreduce!\(f::F, op::O, dst::AbstractArray, src::AbstractArray; dims=nothing, g::G=identity"),
    ("mapreduce1d(f, op, src; kw...)", r"function mapreduce1d\(f::F, op::O, src::AbstractArray; kwargs\.\.\.\)"),
    ("mapreduce1d(f, op, srcs; g, tmp, to_cpu)",
     r"function mapreduce1d\(f::F, op::O, srcs::NTuple\{U,AbstractArray\}; g::G=identity, tmp=nothing,\s*to_cpu::Bool=true"),
    ("mapreduce1d!(f, op, dst, src; kw...)", r"function mapreduce1d!\(f::F, op::O, dst::AbstractArray, src::AbstractArray; kwargs\.\.\.\)"),
    ("mapreduce1d!(f, op, dst, srcs; g, tmp)", r"function mapreduce1d!\(f::F, op::O, dst::AbstractArray, srcs::NTuple\{U,AbstractArray\}; g::G=identity,\s*tmp=nothing"),
    ("mapreduce2d(f, op, src, dim; g, tmp)", r"function mapreduce2d\(f::F, op::O, src::AbstractMatrix, dim::Int; g::G=identity, tmp=nothing"),
    ("mapreduce2d!(f, op, dst, src, dim; g, tmp)", r"function mapreduce2d!\(f::F, op::O, dst::AbstractArray, src::AbstractMatrix, dim::Int; g::G=identity,\s*tmp=nothing"),
    ("mapreducedims(f, op, src, dims; g)", r"function mapreducedims\(f::F, op::O, src::AbstractArray\{T\}, dims; g::G=identity"),
    ("mapreducedims!(f, op, dst, src, dims; g)", r"function mapreducedims!\(f::F, op::O, dst::AbstractArray, src::AbstractArray, dims; g::G=identity"),
    ("matvec(f, op, src, x; g, tmp)", r"function matvec\(f::F, op::O, src::AbstractMatrix, x::Union\{AbstractArray,Nothing\}; g::G=identity, tmp=nothing"),
    ("matvec!(f, op, dst, src, x; g, tmp)", r"function matvec!\(f::F, op::O, dst::AbstractArray, src::AbstractMatrix, x::Union\{AbstractArray,Nothing\};\s*g::G=identity, tmp=nothing"),
    ("vecmat(f, op, x, src; g, tmp)", r"function vecmat\(f::F, op::O, x::Union\{AbstractArray,Nothing\}, src::AbstractMatrix; g::G=identity, tmp=nothing"),
    ("vecmat!(f, op, dst, x, src; g, tmp)", r"function vecmat!\(f::F, op::O, dst::AbstractArray, x::Union\{AbstractArray,Nothing\}, src::AbstractMatrix;\s*g::G=identity, tmp=nothing"),
    ("@allocate", r"macro allocate\(expr\)"),
    ("KernelBuffer{Arrays<:NamedTuple}", r"struct KernelBuffer\{Arrays<:NamedTuple\}\n\s+arrays::Arrays\nend"),
]


@pytest.mark.parametrize("what,pattern", SIGNATURES, ids=[s[0] for s in SIGNATURES])
def test_reference_signature_is_defined(what, pattern):
    assert re.search(pattern, open(JL).read()), what


def test_dims_routing_restates_the_reference_rules():
    # the routing branches of reference src/mapreduce/mapreduce.jl:151-212:
    # all dims -> mapreducedims!, leading -> dim 1, trailing -> dim 2, both ->
    # two passes (trailing first), else the general fallback; negative dims
    # count from the end (src/helpers.jl:194-198)
    text = open(JL).read()
    body = text[text.index("function mapreduce!("):text.index("# Any set of dims, one contiguous block")]
    order = [body.index(s) for s in ("length(d) == nd && return mapreducedims!", "if leading && !trailing",
                                     "elseif trailing && !leading", "elseif leading && trailing", "_reduce_blocks!")]
    assert order == sorted(order)
    assert "_normalize_dims(dims::Int, nd::Int) = (dims > 0 ? dims : nd + dims + 1,)" in text


def _strip_strings_and_comments(src):
    src = re.sub(r'"""(.*?)"""', '""', src, flags=re.S)
    src = re.sub(r'"(\\.|[^"\\])*"', '""', src)
    src = re.sub(r"#.*", "", src)
    return src


def test_blocks_are_balanced():
    # a coarse syntax check (no julia here): every block opener has its `end`;
    # `end` inside brackets (indexing, comprehensions) is not a block end
    src = _strip_strings_and_comments(open(JL).read())
    prev = None
    while prev != src:
        prev, src = src, re.sub(r"\[[^\[\]]*\]", "[]", src)
    openers = ends = 0
    for line in src.splitlines():
        s = line.strip()
        openers += len(re.findall(r"\b(module|function|macro|struct|for|while|let|begin|quote|do|try)\b", s))
        openers += s.startswith("abstract type") + s.startswith("if ")
        ends += len(re.findall(r"\bend\b", s))
    assert openers == ends > 50


def test_allocating_scan_returns_a_vector_of_the_promoted_eltype():
    # reference src/scan/scan.jl:226-244: dst = similar(src, H, length(src))
    # with H = promote_op(g, promote_op(f, T)), whatever the shape of src
    text = open(JL).read()
    m = re.search(r"function scan\(f::F, op::O, src::AbstractArray;(.*?)\nend", text, re.S)
    assert m, "allocating scan(f, op, src) not found"
    body = m.group(1)
    assert "Base.promote_op(g, Base.promote_op(f, eltype(src)))" in body
    assert "similar(src, H, length(src))" in body
    assert "scan!(f, op, dst, src; g, kwargs...)" in body


def test_give_up_reports_reach_the_julia_caller():
    # KF_EGIVEUP (4) raises, and the full mapreduce checks the report after
    # its synchronising read-back
    text = open(JL).read()
    assert "rc == Cint(4) && error(" in text
    m = re.search(r"v = Array\(dst\)\[1\].*?\n\s*check_async\(\)", text, re.S)
    assert m, "mapreduce1d does not call check_async after the read-back"
