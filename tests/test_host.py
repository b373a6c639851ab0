"""Host-side logic of the Python mirror of the reference API (no GPU):
operator/map resolution, dims normalisation and routing, layout merging."""
import operator

import pytest
import torch


def test_operator_and_map_resolution(kf):
    L = kf._lib
    assert kf._op_code(operator.add) == L.OP_ADD == kf._op_code("+")
    assert kf._op_code(max) == L.OP_MAX and kf._op_code(min) == L.OP_MIN
    assert kf._op_code(kf.affine) == L.OP_AFFINE
    assert kf._map_code(kf.identity) == L.MAP_IDENTITY and kf._map_code(kf.abs2) == L.MAP_ABS2
    assert kf._op_code(operator.mul) == L.OP_MUL == kf._op_code("*")
    with pytest.raises(kf.ArgumentError):
        kf._op_code(operator.truediv)
    with pytest.raises(kf.ArgumentError):
        kf._map_code(lambda x: x)


def test_affine_op_is_the_recurrence(kf):
    # (a1,b1) o (a2,b2) applied to x equals applying map 1 then map 2
    p, q, x = (2.0, 1.0), (3.0, 5.0), 7.0
    a, b = kf.affine(p, q)
    assert a * x + b == q[0] * (p[0] * x + p[1]) + q[1]


def test_normalize_and_validate_dims(kf):
    assert kf._normalize_dims(2, 3) == (2,)
    assert kf._normalize_dims((3, 1), 3) == (1, 3)
    with pytest.raises(kf.ArgumentError):
        kf._normalize_dims(4, 3)
    with pytest.raises(kf.ArgumentError):
        kf._normalize_dims(0, 3)
    with pytest.raises(kf.ArgumentError):
        kf._normalize_dims((1, 1), 3)
    # non-positive dims count from the end (reference src/helpers.jl:194-198):
    # d -> nd + d + 1, so -1 is the last dim and 0 is one past it
    assert kf._normalize_dims(-1, 3) == (3,)
    assert kf._normalize_dims((-1, 1), 3) == (1, 3)
    assert kf._normalize_dims(-3, 3) == (1,)
    with pytest.raises(kf.ArgumentError):
        kf._normalize_dims(-4, 3)
    with pytest.raises(kf.ArgumentError):
        kf._normalize_dims((3, -1), 3)


@pytest.mark.parametrize("dims,nd,expected", [
    ((1,), 3, (1, 2)),          # leading only
    ((1, 2), 3, (2, 3)),        # leading block
    ((3,), 3, (0, 1)),          # trailing only
    ((2, 3), 3, (0, 1)),        # trailing block
    ((1, 3), 3, (1, 2)),        # leading + trailing
    ((1, 2, 3), 3, (3, 4)),     # one block touching both ends -> leading
    ((2,), 3, (0, 2)),          # middle -> general
    ((2, 4, 5), 5, (0, 4)),     # not two blocks covering dims -> general
    ((1, 4, 5), 5, (1, 2)),     # lead {1}, tail {4,5}
])
def test_classify_dims_matches_reference_rules(kf, dims, nd, expected):
    # rules of reference src/mapreduce/mapreduce.jl:272-298
    assert kf._classify_dims(dims, nd) == expected


def test_merge_and_matrix_views(kf):
    A = torch.empty(65536, 4096).T          # 4096 x 65536 column-major
    assert kf._as_matrix(A, 1) == (4096, 65536, 4096)
    V = A[:, ::2]                            # view(A, :, 1:2:end)
    assert kf._as_matrix(V, 1) == (4096, 32768, 8192)
    B = torch.empty(4, 5, 6).permute(2, 1, 0)  # 6x5x4 column-major
    assert kf._as_matrix(B, 2) == (30, 4, 30)
    assert kf._as_matrix(B, 1) == (6, 20, 6)
    with pytest.raises(NotImplementedError):
        kf._as_matrix(torch.empty(3, 4), 1)   # row-major: rows are not unit-stride


def test_cpu_tensors_are_rejected(kf):
    x = torch.zeros(10)
    with pytest.raises(kf.ArgumentError, match="GPU"):
        kf.scan("+", x)
    with pytest.raises(kf.ArgumentError, match="GPU"):
        kf.mapreduce(kf.identity, "+", x)


def test_scratch_family_check(kf):
    # a scan buffer must not serve reductions and vice versa (reduction
    # partials written over scan descriptors could read as current ones)
    cpu = torch.device("cpu")
    sbuf = kf.KernelBuffer(kf.Scan1D, 1024, cpu)
    rbuf = kf.KernelBuffer(kf.MapReduce1D, 1024, cpu)
    with pytest.raises(kf.ArgumentError):
        kf._scratch(kf.MapReduce1D, 256, cpu, sbuf)
    with pytest.raises(kf.ArgumentError):
        kf._scratch(kf.MapReduce2D, 256, cpu, sbuf)
    with pytest.raises(kf.ArgumentError):
        kf._scratch(kf.Scan1D, 256, cpu, rbuf)
    assert kf._scratch(kf.MapReduce2D, 256, cpu, rbuf) is rbuf      # one family: shared
    with pytest.raises(kf.ArgumentError):
        kf._scratch(kf.MapReduce1D, 4096, cpu, rbuf)                  # too small
