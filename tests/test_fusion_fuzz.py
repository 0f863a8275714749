"""Malformed node arrays through the library's host code on the CPU: the fusion
matcher (lbr_fusion_windows) and the host half of plan creation
(lbr_check_nodes: every node decoder, the fused steps and the step joins, with
and without fusion).  The real node streams of six workloads get a few fields
of a few nodes replaced by out-of-range or inconsistent values (negative and
huge dims and extras, n_dims and n_inputs past their arrays, wrong op codes,
swapped, shared and null pointers).  Each call must return runs, steps or an
error, never read past a record or overflow; tests/test_host_sanitizer.py runs
this file against the ASan + UBSan build, where either would stop the process.

`execute()` and `lbr_plan_create[_fused]` take node arrays from any caller, so
a malformed record is an input like any other (the reference's executor,
csrc/executor.c:409-452, trusts the host layer instead).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from runtime.executor.common import COpNode
from runtime.executor.hip_lib import open_library

from test_fusion import _workload_nodes

OPS = [100, 101, 102, 103, 104, 105, 106, 107, 108, 109, 200, 201, 202, 203, 300, 301, 302, 400, 500, 501,
       502, 503, 504, 505, 600, 601, 1000, 1001, 1002, 1003]
INTS = [-(1 << 31), -7, -1, 0, 1, 2, 3, 4, 5, 8, 16, 17, 31, 64, 100, 128, 1000, 4096, 65535, 1 << 20,
        (1 << 31) - 1]


def _lib():
    try:
        return open_library()
    except RuntimeError as e:
        pytest.skip(str(e))


def _copy(arr):
    out = (COpNode * len(arr))()
    ctypes.memmove(out, arr, ctypes.sizeof(arr))
    return out


def _mutate(r: np.random.Generator, arr, n: int) -> str:
    i = int(r.integers(n))
    nd = arr[i]
    k = int(r.integers(10))
    pick = lambda xs: xs[int(r.integers(len(xs)))]   # noqa: E731
    if k == 0:
        j = int(r.integers(8))
        nd.extra[j] = pick(INTS)
        return f"node {i} extra[{j}]={nd.extra[j]}"
    if k == 1 and nd.n_dims > 0:
        j = int(r.integers(max(1, min(nd.n_dims, 24))))
        nd.out_shape[j] = pick(INTS)
        return f"node {i} out_shape[{j}]={nd.out_shape[j]}"
    if k == 2:
        nd.n_dims = pick([-1, 0, 1, 2, 3, 4, 5, 24, 25, 1000, -(1 << 31)])
        return f"node {i} n_dims={nd.n_dims}"
    if k == 3:
        nd.n_inputs = pick([-1, 0, 1, 2, 3, 4, 12, 13, 1 << 20])
        return f"node {i} n_inputs={nd.n_inputs}"
    if k == 4:
        j, o = int(r.integers(12)), arr[int(r.integers(n))]
        nd.inputs[j] = pick([None, o.output, o.inputs[0], nd.output])
        return f"node {i} inputs[{j}]"
    if k == 5:
        nd.op = pick(OPS + [0, -1, 399, 9999])
        return f"node {i} op={nd.op}"
    if k == 6:
        o = arr[int(r.integers(n))]
        nd.output = pick([None, o.output, o.inputs[0]])
        return f"node {i} output"
    if k == 7:
        nd.elem_size = pick([0, 1, 2, 4, 8, -4])
        return f"node {i} elem_size={nd.elem_size}"
    # every dim of a node huge (element counts past 2^63 if multiplied unchecked), or one
    # of them 0 (no elements, but products over the other dims still huge)
    nd.n_dims = pick([4, 8, 24])
    for j in range(nd.n_dims):
        nd.out_shape[j] = pick([65535, (1 << 31) - 1])
    if k == 9:
        nd.out_shape[int(r.integers(nd.n_dims))] = 0
    return f"node {i} huge dims x{nd.n_dims}{' with a 0' if k == 9 else ''}"


@pytest.mark.parametrize("key,seq", [("toy", 32), ("gpt2w", 64), ("gpt2", 64), ("qwen3_4b", 64),
                                     ("7b4k", 64), ("gpt2_lm", 48)])
def test_fusion_matcher_takes_malformed_nodes(key, seq):
    lib = _lib()
    base, _, live = _workload_nodes(key, seq)
    n = len(base)
    for nd in base:
        if nd.op == 504:   # EMBEDDING: the table's row count, as the compiled executor writes it
            nd.extra[1] = 1 << 16
    assert lib.fusion_windows(base, n, live)   # the unmodified stream fuses
    assert 0 < lib.check_nodes(base, n, live) < lib.check_nodes(base, n, live, fuse=False) == n
    r = np.random.default_rng(seq * 7919 + len(key))
    errors = [0, 0, 0]
    for trial in range(150):
        arr = _copy(base)
        what = [_mutate(r, arr, n) for _ in range(int(r.integers(1, 4)))]
        for fuse in (False, True):
            try:
                steps = lib.check_nodes(arr, n, live, fuse=fuse)
                assert 1 <= steps <= n, (trial, what, fuse, steps)
            except RuntimeError:
                errors[fuse] += 1
        try:
            runs = lib.fusion_windows(arr, n, live)
        except RuntimeError:
            errors[2] += 1
            continue
        for first, count, kind in runs:
            assert 0 <= first and count >= 1 and first + count <= n and kind != "?", (trial, what, runs)
        firsts = [f for f, _, _ in runs]
        assert firsts == sorted(firsts), (trial, what)
    print(f"{key}: 150 malformed arrays; refused unfused {errors[0]}, fused {errors[1]}, matcher {errors[2]}")


def test_fusion_matcher_rejects_out_of_range_records():
    # n_dims / n_inputs outside their arrays and element counts past what any device holds
    # are errors of the call, before any matcher reads the record
    lib = _lib()
    base, _, live = _workload_nodes("gpt2w", 64)
    n = len(base)
    calls = [lambda a: lib.fusion_windows(a, n, live), lambda a: lib.check_nodes(a, n, live),
             lambda a: lib.check_nodes(a, n, live, fuse=False)]
    for call in calls:
        for field, value in [("n_dims", 25), ("n_dims", -1), ("n_inputs", 13), ("n_inputs", -1)]:
            arr = _copy(base)
            setattr(arr[3], field, value)
            with pytest.raises(RuntimeError, match="node 3"):
                call(arr)
        arr = _copy(base)
        arr[3].n_dims = 8
        for j in range(8):
            arr[3].out_shape[j] = 65535
        with pytest.raises(RuntimeError, match="node 3 has more than 2\\^40 elements"):
            call(arr)
        arr[3].out_shape[0] = 0   # no elements, but the other dims' product is bounded too
        with pytest.raises(RuntimeError, match="node 3 has more than 2\\^40 elements"):
            call(arr)
        arr = _copy(base)
        arr[5].out_shape[0] = -2
        with pytest.raises(RuntimeError, match="node 5"):
            call(arr)
    # extras that disagree with the output's shape (the kernels would index past it)
    ops = [nd.op for nd in base]
    for op, field, j, value, msg in [(1002, "extra", 0, 32, "seq_len"), (1002, "extra", 1, 32, "head_dim"),
                                     (503, "extra", 3, 1, "slice"), (501, "extra", 4, 1, "transpose")]:
        k = ops.index(op)
        arr = _copy(base)
        getattr(arr[k], field)[j] = value
        for call in calls[1:]:
            with pytest.raises(RuntimeError, match=msg):
                call(arr)
