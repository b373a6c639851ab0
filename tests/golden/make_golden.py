"""Writes tests/golden/fixtures.json: small seeded input/output vectors for
scan! and mapreduce, computed with numpy and plain Python only (independent
of oracle/kf_oracle.c, which the CPU tests check against these vectors).

The reference ships no golden files (its tests compare against Julia Base on
random inputs, reference test/tests/scan/scan_test.jl:35-125,
test/tests/mapreduce/mapreduce1d_test.jl:10-55); these fixtures restate the
same known-answer cases with fixed seeds:
  * scans of Int32 / UInt8 / Float64 with +, max, min at the reference's
    sizes (1..10, 100, 1000, 10001), inclusive and exclusive;
  * the affine recurrence x_t = a_t x_{t-1} + b_t;
  * mapreduce(identity, +) over 1:n (closed form n(n+1)/2), abs2 sums,
    max/min;
  * dims=1 / dims=2 on small column-major matrices and a stride-2 column view.

Run: python tests/golden/make_golden.py
"""
import json
import os

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fixtures.json")
SEED = 20261201


def jl_max(x, y):
    if np.isnan(x) or np.isnan(y):
        return float("nan")
    if x == y:
        return y if np.signbit(x) else x
    return x if x > y else y


def jl_min(x, y):
    if np.isnan(x) or np.isnan(y):
        return float("nan")
    if x == y:
        return x if np.signbit(x) else y
    return x if x < y else y


def np_scan(x, op):
    if op == "+":
        return np.cumsum(x, dtype=x.dtype if x.dtype.kind in "iu" else np.float64)
    if op == "max":
        return np.maximum.accumulate(x)
    return np.minimum.accumulate(x)


IDENT = {("+", "i"): 0, ("+", "u"): 0, ("+", "f"): 0.0,
         ("max", "i"): None, ("min", "i"): None}


def identity(op, dtype):
    if op == "+":
        return 0
    info = np.iinfo(dtype) if np.dtype(dtype).kind in "iu" else None
    if info is None:
        return float("-inf") if op == "max" else float("inf")
    return int(info.min) if op == "max" else int(info.max)


def enc(v):
    """JSON-safe floats (inf / nan as strings)."""
    out = []
    for x in np.asarray(v).tolist():
        if isinstance(x, float) and not np.isfinite(x):
            out.append("nan" if np.isnan(x) else ("inf" if x > 0 else "-inf"))
        else:
            out.append(x)
    return out


def main():
    rng = np.random.default_rng(SEED)
    cases = {"scan": [], "affine": [], "reduce": [], "reduce_dim": []}
    sizes = list(range(1, 11)) + [100, 1000, 10001]  # 10001: UInt8 only (reference scan_test.jl:67-86)
    for dt in ("int32", "uint8", "float64"):
        for op in ("+", "max", "min"):
            for n in (sizes if dt == "uint8" else sizes[:-1]):
                if dt == "int32":
                    x = rng.integers(1, 11, n).astype(np.int32)  # rand(1:10) as in the reference
                elif dt == "uint8":
                    x = rng.integers(0, 256, n).astype(np.uint8)
                else:
                    x = rng.random(n)
                incl = np_scan(x, op).astype(x.dtype if dt != "float64" else np.float64)
                excl = np.concatenate([[identity(op, x.dtype)], incl[:-1]]).astype(incl.dtype)
                cases["scan"].append({"dtype": dt, "op": op, "n": n, "x": enc(x),
                                      "inclusive": enc(incl), "exclusive": enc(excl)})
    # signed zeros and NaN for Julia's max/min (hand-built sequence)
    sz = np.array([0.0, -0.0, 1.0, float("nan"), 2.0], np.float64)
    for op, fn in (("max", jl_max), ("min", jl_min)):
        acc, incl = None, []
        for v in sz:
            acc = v if acc is None else fn(acc, v)
            incl.append(acc)
        cases["scan"].append({"dtype": "float64", "op": op, "n": 5, "x": enc(sz), "inclusive": enc(incl),
                              "exclusive": enc([identity(op, np.float64)] + incl[:-1]), "signed_zero": True})
    # int32 wrap-around
    w = np.array([2**31 - 1, 1, 5], np.int32)
    cases["scan"].append({"dtype": "int32", "op": "+", "n": 3, "x": enc(w),
                          "inclusive": enc(np.cumsum(w, dtype=np.int32)),
                          "exclusive": enc(np.concatenate([[0], np.cumsum(w, dtype=np.int32)[:-1]]))})
    # affine recurrence, plain Python float64 loop
    for n in (1, 2, 7, 100, 1500):
        a = rng.uniform(0.9, 1.0, n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        A, B, incl = 1.0, 0.0, []
        for ai, bi in zip(a.tolist(), b.tolist()):
            A, B = ai * A, ai * B + bi
            incl.append([A, B])
        excl = [[1.0, 0.0]] + incl[:-1]
        cases["affine"].append({"n": n, "a": enc(a), "b": enc(b), "inclusive": incl, "exclusive": excl})
    # reductions
    for dt in ("float32", "float64", "int32"):
        for n in (33, 100, 10001, 100000):
            x = np.arange(1, n + 1).astype(dt)  # the reference's 1:n sums
            tri = n * (n + 1) // 2
            if dt == "int32":  # Julia's Int32 `+` wraps (mapreduce does not widen, unlike sum)
                tri = int(np.array(tri % 2**32, np.uint32).astype(np.int32))
            cases["reduce"].append({"dtype": dt, "op": "+", "f": "identity", "n": n, "x": "arange1",
                                    "expected": tri})
            if dt != "int32":
                cases["reduce"].append({"dtype": dt, "op": "+", "f": "abs2", "n": n, "x": "arange1",
                                        "expected": n * (n + 1) * (2 * n + 1) // 6})
    for dt in ("int32", "float64"):
        for op in ("max", "min"):
            x = rng.integers(-2**31, 2**31 - 1, 777).astype(dt)
            cases["reduce"].append({"dtype": dt, "op": op, "f": "identity", "n": 777, "x": enc(x),
                                    "expected": (x.max() if op == "max" else x.min()).item()})
    # dims on column-major matrices; buffer holds the full parent, view uses col_stride
    for rows, cols in ((5, 7), (64, 32), (3, 7), (1, 64), (128, 1), (33, 17)):
        for view in (False, True):
            pc = cols * 2 if view else cols
            parent = rng.uniform(-1, 1, (pc, rows)).astype(np.float64)  # row k of `parent` = column k
            cs = 2 * rows if view else rows
            M = parent[::2] if view else parent  # (cols, rows): columns of the matrix
            cases["reduce_dim"].append({
                "dtype": "float64", "rows": rows, "cols": cols, "col_stride": cs,
                "buf": enc(parent.reshape(-1)),
                "dim1": enc(M.sum(axis=1)), "dim2": enc(M.sum(axis=0)),
                "dim1_max": enc(M.max(axis=1)), "dim2_min": enc(M.min(axis=0))})
    with open(OUT, "w") as fh:
        json.dump({"seed": SEED, "generator": "numpy.random.default_rng", "cases": cases}, fh)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
