"""The single-workgroup plan (csrc/tiny.hip, opt-in with LBR_TINY=1) on the GPU.

Graphs whose intermediates fit one CU's LDS run as one workgroup that walks
the node array itself.  Each case here is a small graph `op → NEG` (NEG is
exact, and makes the op's output an intermediate held in LDS) or a longer
chain, run three ways on the same input: the single-workgroup plan, the
multi-kernel plan of the same graph (LBR_TINY=0) and the CPU oracle.

Tolerances: copies are bit-exact against the oracle; element-wise ops and
norms ≤ 1e-5 normwise; GEMM and attention ≤ 1e-4 (the interpreter sums in
its own order, so it matches the other plans within fp32 rounding, not bit
for bit).
"""

from __future__ import annotations

import numpy as np
import pytest

from runtime.ir import Graph, OpType
from runtime.planner import plan
from conftest import normwise_rel

pytestmark = [pytest.mark.gpu, pytest.mark.tiny]


def _graph(inputs, consts, nodes, outputs):
    """nodes: (op, input names, output name, output shape, attrs[, dtype])."""
    g = Graph()
    for name, arr in inputs.items():
        g.add_tensor(name, tuple(arr.shape), str(arr.dtype))
        g.inputs.append(name)
    for name, arr in consts.items():
        g.add_tensor(name, tuple(arr.shape), str(arr.dtype)).buffer = arr
        g.constants.append(name)
    for spec in nodes:
        op, ins, out, shape, attrs = spec[:5]
        dtype = spec[5] if len(spec) > 5 else "float32"
        g.add_tensor(out, tuple(shape), dtype)
        g.add_node(op, list(ins), out, attrs)
    g.outputs.extend(outputs)
    return g


def _run(g, feeds, monkeypatch, tiny: bool):
    from runtime.executor.compiled import CompiledExecutor
    monkeypatch.setenv("LBR_TINY", "1" if tiny else "0")
    ex = CompiledExecutor()
    ex.compile(plan(g))
    try:
        kinds = [p["kind"] for p in ex.step_params()]
        out = ex.run(feeds)
        return {k: np.array(v) for k, v in out.items()}, kinds
    finally:
        ex.close()


def _check(g, feeds, monkeypatch, tol, exact=False, ref=None):
    from oracle.host_exec import OracleRun
    y, kinds = _run(g, feeds, monkeypatch, tiny=True)
    assert kinds == ["tiny"], f"expected the single-workgroup plan, got steps {kinds}"
    z, kinds_z = _run(g, feeds, monkeypatch, tiny=False)
    assert "tiny" not in kinds_z
    o = OracleRun(plan(g)).run(feeds)
    for name in g.outputs:
        if exact:
            np.testing.assert_array_equal(y[name], o[name])
            np.testing.assert_array_equal(y[name], z[name])
            continue
        e_o, e_z = normwise_rel(y[name], o[name]), normwise_rel(y[name], z[name])
        print(f"{name}: tiny-vs-oracle {e_o:.2e} tiny-vs-kernels {e_z:.2e}")
        assert np.isfinite(y[name]).all()
        assert e_o <= tol and e_z <= tol
        if ref is not None and name in ref:
            assert normwise_rel(y[name], ref[name]) <= tol


def _r(seed=0):
    return np.random.default_rng(seed)


def _f(r, *shape, scale=1.0):
    return (r.standard_normal(shape) * scale).astype(np.float32)


# ---------------------------------------------------------------- element-wise

UNARY = [OpType.RELU, OpType.EXP, OpType.TANH, OpType.POW, OpType.GELU, OpType.RSQRT, OpType.SILU,
         OpType.NEG, OpType.COS, OpType.SIN]


@pytest.mark.parametrize("op", UNARY, ids=lambda o: o.name)
def test_unary(monkeypatch, op):
    r = _r(1)
    x = _f(r, 7, 45)
    if op == OpType.RSQRT:
        x = np.abs(x) + 0.1
    attrs = {"scalar": 3.0} if op == OpType.POW else {}
    g = _graph({"x": x}, {}, [(op, ["x"], "t", x.shape, attrs), (OpType.NEG, ["t"], "y", x.shape, {})], ["y"])
    _check(g, {"x": x}, monkeypatch, 1e-5)


BINARY_CASES = [
    # (op, a shape, b shape or None for scalar)
    (OpType.ADD, (6, 40), (40,)),          # bias row
    (OpType.ADD, (6, 40), (6, 40)),        # same shape
    (OpType.ADD, (6, 40), None),           # scalar
    (OpType.ADD, (2, 6, 40), (2, 1, 40)),  # broadcast
    (OpType.SUB, (6, 40), (6, 40)),
    (OpType.SUB, (6, 40), None),
    (OpType.MUL, (3, 5, 8), (5, 1)),
    (OpType.MUL, (6, 40), None),
    (OpType.DIV, (6, 40), (6, 40)),
    (OpType.DIV, (4, 6, 10), (4, 1, 10)),
]


@pytest.mark.parametrize("op,ashape,bshape", BINARY_CASES, ids=lambda v: str(v))
def test_binary(monkeypatch, op, ashape, bshape):
    r = _r(2)
    a = _f(r, *ashape)
    feeds = {"a": a}
    if bshape is None:
        nodes = [(op, ["a"], "t", ashape, {"scalar": 1.75})]
        out_shape = ashape
    else:
        b = _f(r, *bshape)
        if op == OpType.DIV:
            b = np.abs(b) + 0.5
        feeds["b"] = b
        out_shape = tuple(np.broadcast_shapes(ashape, bshape))
        nodes = [(op, ["a", "b"], "t", out_shape, {})]
    nodes.append((OpType.NEG, ["t"], "y", out_shape, {}))
    g = _graph(feeds, {}, nodes, ["y"])
    _check(g, feeds, monkeypatch, 1e-5)


def test_bias_relu_and_gated(monkeypatch):
    r = _r(3)
    x, u = _f(r, 9, 48), _f(r, 9, 48)
    bias = _f(r, 48)
    nodes = [
        (OpType.FUSED_BIAS_RELU, ["x", "bias"], "t0", x.shape, {}),
        (OpType.GATED_ACT, ["x", "u"], "t1", x.shape, {"act": "silu"}),
        (OpType.GATED_ACT, ["t0", "bias", "u"], "t2", x.shape, {"act": "gelu", "has_bias": True}),
        (OpType.ADD, ["t1", "t2"], "y", x.shape, {}),
    ]
    g = _graph({"x": x, "u": u}, {"bias": bias}, nodes, ["y"])
    _check(g, {"x": x, "u": u}, monkeypatch, 1e-5)


# ---------------------------------------------------------------- row ops

@pytest.mark.parametrize("cols", [16, 64, 100, 200])
def test_norms_and_softmax(monkeypatch, cols):
    r = _r(4)
    x = _f(r, 11, cols, scale=2.0)
    gam, bet = _f(r, cols), _f(r, cols)
    nodes = [
        (OpType.LAYERNORM, ["x", "g", "b"], "ln", x.shape, {"eps": 1e-5}),
        (OpType.RMSNORM, ["ln", "g"], "rms", x.shape, {"eps": 1e-6}),
        (OpType.SOFTMAX, ["rms"], "sm", x.shape, {}),
        (OpType.NEG, ["sm"], "y", x.shape, {}),
    ]
    g = _graph({"x": x}, {"g": gam, "b": bet}, nodes, ["y"])
    _check(g, {"x": x}, monkeypatch, 1e-5)


# ---------------------------------------------------------------- GEMM

MATMUL_CASES = [
    # (a shape, b shape, transpose_b, alpha, bias)
    ((20, 17), (30, 17), True, 1.0, False),        # ragged M, N, K
    ((20, 17), (17, 30), False, 1.0, False),       # B stored [K, N]
    ((2, 3, 33, 24), (2, 3, 24, 40), False, 0.5, False),   # batched, alpha
    ((2, 40, 64), (48, 64), True, 1.0, True),      # 3-D A by a 2-D B, bias (MATMUL_ADD)
    ((1, 64), (64, 96), False, 1.0, True),         # M = 1, K split in 2 over the wavefronts
    ((8, 256), (16, 256), True, 1.0, False),       # one output block, K split 16 ways
    ((32, 2048), (64, 2048), True, 1.0, True),     # B and A staged in K chunks
    ((16, 1024), (1024, 48), False, 2.0, False),   # B [K, N] staged in K chunks
]


@pytest.mark.parametrize("ashape,bshape,tb,alpha,bias", MATMUL_CASES, ids=lambda v: str(v))
def test_matmul(monkeypatch, ashape, bshape, tb, alpha, bias):
    r = _r(5)
    a = _f(r, *ashape)
    b = _f(r, *bshape, scale=0.2)
    n = bshape[-2] if tb else bshape[-1]
    out_shape = (*ashape[:-1], n)
    attrs = {"transpose_b": tb}
    if alpha != 1.0:
        attrs["alpha"] = alpha
    consts = {"w": b}
    if bias:
        consts["bias"] = _f(r, n)
        nodes = [(OpType.MATMUL_ADD, ["a", "w", "bias"], "t", out_shape, attrs)]
    else:
        nodes = [(OpType.MATMUL, ["a", "w"], "t", out_shape, attrs)]
    nodes.append((OpType.NEG, ["t"], "y", out_shape, {}))
    g = _graph({"a": a}, consts, nodes, ["y"])
    bb = b.astype(np.float64)
    ref = a.astype(np.float64) @ (np.swapaxes(bb, -1, -2) if tb else bb) * alpha
    if bias:
        ref = ref + consts["bias"]
    _check(g, {"a": a}, monkeypatch, 1e-4, ref={"y": -ref})


# ---------------------------------------------------------------- attention

ATTN_CASES = [
    # (B·H, S, hd, causal, mask, group)
    (4, 40, 16, True, False, 1),
    (2, 64, 64, False, False, 1),
    (2, 100, 32, True, False, 2),     # GQA: 2 query heads per kv head
    (2, 30, 128, False, True, 1),     # additive mask
    (1, 128, 8, True, False, 1),      # one head's 128 x 132 scores fill most of the staging area
]


@pytest.mark.parametrize("bh,S,hd,causal,mask,group", ATTN_CASES, ids=lambda v: str(v))
def test_attention(monkeypatch, bh, S, hd, causal, mask, group):
    from helpers import cf_attention
    r = _r(6)
    q = _f(r, bh, S, hd)
    k = _f(r, bh // group, S, hd)
    v = _f(r, bh // group, S, hd)
    feeds = {"q": q, "k": k, "v": v}
    ins = ["q", "k", "v"]
    m = None
    if mask:
        m = np.where(r.random((bh, S, S)) < 0.2, -1e9, 0.0).astype(np.float32)
        for i in range(S):
            m[:, i, i] = 0.0
        feeds["m"] = m
        ins.append("m")
    attrs = {"causal": causal, "group_size": group}
    nodes = [(OpType.ATTENTION, ins, "t", (bh, S, hd), attrs), (OpType.NEG, ["t"], "y", (bh, S, hd), {})]
    g = _graph(feeds, {}, nodes, ["y"])
    ref = -cf_attention(q, k, v, causal=causal, group=group, mask=m)
    _check(g, feeds, monkeypatch, 1e-4, ref={"y": ref})


# ---------------------------------------------------------------- copies

@pytest.mark.parametrize("dtype", ["float32", "int64"])
def test_copies(monkeypatch, dtype):
    r = _r(7)
    if dtype == "float32":
        x = _f(r, 3, 10, 12)
    else:
        x = r.integers(-2**40, 2**40, size=(3, 10, 12)).astype(np.int64)
    nodes = [
        (OpType.TRANSPOSE, ["x"], "t0", (3, 12, 10), {"dim0": 1, "dim1": 2}, dtype),
        (OpType.SLICE, ["t0"], "t1", (3, 7, 10), {"dim": 1, "start": 2, "end": 9}, dtype),
        (OpType.RESHAPE, ["t1"], "t2", (21, 10), {"shape": [21, 10]}, dtype),
        (OpType.TRANSPOSE, ["t2"], "t3", (10, 21), {}, dtype),
        (OpType.CAT, ["t3", "t3"], "y", (10, 42), {"dim": 1}, dtype),
    ]
    g = _graph({"x": x}, {}, nodes, ["y"])
    _check(g, {"x": x}, monkeypatch, 0, exact=True)
    xt = np.swapaxes(x, 1, 2)[:, 2:9, :].reshape(21, 10).T
    np.testing.assert_array_equal(_run(g, {"x": x}, monkeypatch, tiny=True)[0]["y"], np.concatenate([xt, xt], 1))


# ---------------------------------------------------------------- whole workloads

def test_toy_block_plan_is_one_step(monkeypatch):
    """The toy block at its benchmark shape (S = 32, D = 64, 4 heads) is one
    workgroup; its output against the multi-kernel plan and the oracle, and
    the captured graph replayed with fresh inputs."""
    from workloads import export_workload, WORKLOADS
    from runtime.passes import run_pipeline
    _, x, graph = export_workload("toy")
    run_pipeline(graph, None)
    _check(graph, {graph.inputs[0]: x}, monkeypatch, 1e-4)
    from runtime.executor.compiled import CompiledExecutor
    from oracle.host_exec import OracleRun
    ex = CompiledExecutor()
    mp = plan(graph)
    ex.compile(mp)
    orc = OracleRun(mp)
    try:
        for seed in range(3):
            xi = WORKLOADS["toy"].input(seed=seed + 20)
            y = ex.run({graph.inputs[0]: xi})[graph.outputs[0]]
            o = orc.run({graph.inputs[0]: xi})[graph.outputs[0]]
            assert normwise_rel(y, o) <= 1e-4
    finally:
        ex.close()
