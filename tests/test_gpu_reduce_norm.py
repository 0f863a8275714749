"""Split-K GEMM + residual ADD → RMSNORM / LAYERNORM with the norm inside the
split-K reduce kernel (one row per wavefront up to 1024 columns, one row per
workgroup above): the reduce writes the residual sum C and the normalised rows.
It uses the norm kernels' own per-lane layout and sums, so both outputs equal
the plan with the norm kernel apart bit for bit; against the CPU oracle and a
float64 closed form, 1e-4 normwise.
"""

import numpy as np
import pytest

from conftest import normwise_rel
from helpers import cf_layernorm, cf_rmsnorm, randn, rng, run_oracle
from runtime.ir import Graph, OpType

pytestmark = pytest.mark.gpu


def _graph(r, M, N, K, norm, bias):
    g = Graph()
    a, x = randn(r, 1, M, K), randn(r, 1, M, N)
    for name, arr in (("a", a), ("x", x)):
        g.add_tensor(name, arr.shape)
        g.inputs.append(name)

    def const(name, arr):
        g.add_tensor(name, arr.shape).buffer = arr
        g.constants.append(name)

    w = randn(r, N, K, scale=0.05)
    const("w", w)
    c = a.astype(np.float64) @ w.T.astype(np.float64)
    g.add_tensor("c", (1, M, N))
    if bias:
        b = randn(r, N)
        const("b", b)
        g.add_node(OpType.MATMUL_ADD, ["a", "w", "b"], "c", {"transpose_b": True})
        c = c + b
    else:
        g.add_node(OpType.MATMUL, ["a", "w"], "c", {"transpose_b": True})
    g.add_tensor("h", (1, M, N))
    g.add_node(OpType.ADD, ["x", "c"], "h", {})
    h = c + x
    gam = (1.0 + 0.5 * randn(r, N)).astype(np.float32)
    const("gam", gam)
    g.add_tensor("n", (1, M, N))
    if norm == "rms":
        g.add_node(OpType.RMSNORM, ["h", "gam"], "n", {"eps": 1e-6})
        n = cf_rmsnorm(h, gam, 1e-6)
    else:
        bet = randn(r, N)
        const("bet", bet)
        g.add_node(OpType.LAYERNORM, ["h", "gam", "bet"], "n", {"eps": 1e-5})
        n = cf_layernorm(h, gam, bet, 1e-5)
    g.outputs += ["h", "n"]
    return g, {"a": a, "x": x}, h, n


def _run(graph, inputs):
    from runtime.executor.compiled import CompiledExecutor
    from runtime.planner import plan
    ex = CompiledExecutor(fuse=True)
    ex.compile(plan(graph))
    try:
        out = ex.run(inputs)
        return out["h"], out["n"], [p["name"] for p in ex.step_params()]
    finally:
        ex.close()


@pytest.mark.parametrize("norm", ["rms", "layer"])
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("M,N,K", [(64, 768, 1536), (40, 1000, 1024), (96, 2560, 2048), (33, 4096, 1024),
                                   (16, 2000, 768)])
def test_reduce_norm(monkeypatch, norm, bias, M, N, K):
    monkeypatch.setenv("LBR_GEMM_KSPLIT", "3")
    g, ins, h64, n64 = _graph(rng(M + N + K), M, N, K, norm, bias)
    h, n, names = _run(g, ins)
    monkeypatch.setenv("LBR_REDUCE_NORM", "0")
    h2, n2, names2 = _run(g, ins)
    print(names, names2)
    assert any(nm.endswith("+rmsnorm" if norm == "rms" else "+layernorm") for nm in names), names
    assert not any(nm in ("rmsnorm", "layernorm") for nm in names), names
    assert any(nm in ("rmsnorm", "layernorm") for nm in names2), names2
    np.testing.assert_array_equal(h, h2)
    np.testing.assert_array_equal(n, n2)
    from oracle.host_exec import OracleRun
    from runtime.planner import plan
    o = OracleRun(plan(g)).run(ins)
    for got, ref, name in ((h, h64, "h"), (n, n64, "n")):
        assert normwise_rel(got, ref) <= 1e-4, name
        assert normwise_rel(o[name], ref) <= 1e-4, name
        assert normwise_rel(got, o[name]) <= 1e-4, name


def _tin_graph(r, H, S, hd, N, norm):
    """O [1, H, S, hd] → TRANSPOSE(1, 2) → RESHAPE [1, S, H·hd] → MATMUL_ADD → ADD(x, C) → norm: the
    GEMM reads O in its head layout (GPT-2-width's attention projection and second LayerNorm)."""
    K = H * hd
    o, x = randn(r, 1, H, S, hd), randn(r, 1, S, N)
    w, b = randn(r, N, K, scale=0.05), randn(r, N)
    gam = (1.0 + 0.5 * randn(r, N)).astype(np.float32)
    bet = randn(r, N)
    g = Graph()
    for name, arr in (("o", o), ("x", x)):
        g.add_tensor(name, arr.shape)
        g.inputs.append(name)
    for name, arr in (("w", w), ("b", b), ("gam", gam), ("bet", bet)):
        g.add_tensor(name, arr.shape).buffer = arr
        g.constants.append(name)
    g.add_tensor("t", (1, S, H, hd))
    g.add_node(OpType.TRANSPOSE, ["o"], "t", {"dim0": 1, "dim1": 2})
    g.add_tensor("a", (1, S, K))
    g.add_node(OpType.RESHAPE, ["t"], "a", {"shape": (1, S, K)})
    g.add_tensor("c", (1, S, N))
    g.add_node(OpType.MATMUL_ADD, ["a", "w", "b"], "c", {"transpose_b": True})
    g.add_tensor("h", (1, S, N))
    g.add_node(OpType.ADD, ["x", "c"], "h", {})
    h = np.swapaxes(o, 1, 2).reshape(1, S, K).astype(np.float64) @ w.T.astype(np.float64) + b + x
    g.add_tensor("n", (1, S, N))
    if norm == "rms":
        g.add_node(OpType.RMSNORM, ["h", "gam"], "n", {"eps": 1e-6})
        n = cf_rmsnorm(h, gam, 1e-6)
    else:
        g.add_node(OpType.LAYERNORM, ["h", "gam", "bet"], "n", {"eps": 1e-5})
        n = cf_layernorm(h, gam, bet, 1e-5)
    g.outputs += ["h", "n"]
    return g, {"o": o, "x": x}, h, n


@pytest.mark.parametrize("norm", ["rms", "layer"])
@pytest.mark.parametrize("H,S,hd,N", [(12, 512, 64, 768), (4, 100, 32, 520), (8, 64, 128, 1024)])
def test_reduce_norm_after_head_layout_gemm(monkeypatch, norm, H, S, hd, N):
    """The attention projection reading its A in head layout, + residual, + norm: one GEMM
    (two K ranges when its own choice is unsplit) whose reduce writes C and the normalised
    rows, bit-equal to the plan with the norm kernel apart (both in two K ranges)."""
    monkeypatch.setenv("LBR_GEMM_KSPLIT", "2")
    g, ins, h64, n64 = _tin_graph(rng(H + S + hd + N), H, S, hd, N, norm)
    h, n, names = _run(g, ins)
    monkeypatch.setenv("LBR_REDUCE_NORM", "0")
    h2, n2, names2 = _run(g, ins)
    print(names, names2)
    suffix = "+tin+resid+rmsnorm" if norm == "rms" else "+tin+resid+layernorm"
    assert any(nm.endswith(suffix) for nm in names), names
    assert any(nm.endswith("+tin+resid") for nm in names2), names2
    np.testing.assert_array_equal(h, h2)
    np.testing.assert_array_equal(n, n2)
    from oracle.host_exec import OracleRun
    from runtime.planner import plan
    o = OracleRun(plan(g)).run(ins)
    assert normwise_rel(n, n64) <= 1e-4 and normwise_rel(h, h64) <= 1e-4
    assert normwise_rel(n, o["n"]) <= 1e-4 and normwise_rel(o["n"], n64) <= 1e-4


@pytest.mark.parametrize("N", [6000, 256])
def test_reduce_norm_other_widths_stay_apart(monkeypatch, N):
    """Rows above 4096 or of at most 256 columns keep the norm kernel."""
    monkeypatch.setenv("LBR_GEMM_KSPLIT", "3")
    g, ins, h64, n64 = _graph(rng(9), 16, N, 768, "rms", False)
    h, n, names = _run(g, ins)
    assert "rmsnorm" in names, names
    assert normwise_rel(h, h64) <= 1e-4 and normwise_rel(n, n64) <= 1e-4



def _params(graph, inputs):
    from runtime.executor.compiled import CompiledExecutor
    from runtime.planner import plan
    ex = CompiledExecutor(fuse=True)
    ex.compile(plan(graph))
    try:
        out = ex.run(inputs)
        return out["h"], out["n"], ex.step_params()
    finally:
        ex.close()


@pytest.mark.parametrize("norm", ["rms", "layer"])
def test_unsplit_gemm_takes_two_ranges_for_the_norm(monkeypatch, norm):
    """A small unsplit residual GEMM (GPT-2's attention projection shape) takes two K
    ranges so its reduce carries the norm: the K sum then rounds otherwise than the
    unsplit GEMM (within 1e-5 of the plan that keeps them apart)."""
    g, ins, h64, n64 = _graph(rng(21), 1024, 768, 768, norm, True)
    h, n, steps = _params(g, ins)
    monkeypatch.setenv("LBR_REDUCE_NORM_SPLIT", "0")
    h2, n2, steps2 = _params(g, ins)
    joined = [p for p in steps if p.get("split_for_norm")]
    assert len(joined) == 1 and joined[0]["ksplit"] == 2 and joined[0]["reduce_norm"], steps
    assert not any(p.get("split_for_norm") or p.get("reduce_norm") for p in steps2), steps2
    assert normwise_rel(h, h2) <= 1e-5 and normwise_rel(n, n2) <= 1e-5
    assert normwise_rel(h, h64) <= 1e-4 and normwise_rel(n, n64) <= 1e-4


def _add_norm_graph(r, B, S, N, norm, same_shape):
    """x [B, S, N] + p ([B, S, N], or a [S, N] table broadcast over the batch) →
    norm; outputs the sum and the norm."""
    g = Graph()
    x = randn(r, B, S, N)
    g.add_tensor("x", x.shape)
    g.inputs.append("x")
    if same_shape:
        p = randn(r, B, S, N)
        g.add_tensor("p", p.shape)
        g.inputs.append("p")
    else:
        p = randn(r, S, N)
        g.add_tensor("p", p.shape).buffer = p
        g.constants.append("p")
    g.add_tensor("h", (B, S, N))
    g.add_node(OpType.ADD, ["x", "p"], "h", {})
    h = x.astype(np.float64) + p
    gam = (1.0 + 0.5 * randn(r, N)).astype(np.float32)
    g.add_tensor("gam", (N,)).buffer = gam
    g.constants.append("gam")
    g.add_tensor("n", (B, S, N))
    if norm == "rms":
        g.add_node(OpType.RMSNORM, ["h", "gam"], "n", {"eps": 1e-6})
        n = cf_rmsnorm(h, gam, 1e-6)
    else:
        bet = randn(r, N)
        g.add_tensor("bet", (N,)).buffer = bet
        g.constants.append("bet")
        g.add_node(OpType.LAYERNORM, ["h", "gam", "bet"], "n", {"eps": 1e-5})
        n = cf_layernorm(h, gam, bet, 1e-5)
    g.outputs += ["h", "n"]
    ins = {"x": x, "p": p} if same_shape else {"x": x}
    return g, ins, h, n


@pytest.mark.parametrize("norm", ["rms", "layer"])
@pytest.mark.parametrize("same_shape", [False, True])
@pytest.mark.parametrize("B,S,N", [(1, 1024, 768), (2, 100, 2560), (3, 7, 64)])
def test_add_norm(monkeypatch, norm, same_shape, B, S, N):
    """ADD → norm as one norm kernel that adds (the position table of GPT-2's input):
    bit-equal to the two kernels apart; 1e-4 of float64 and the oracle."""
    g, ins, h64, n64 = _add_norm_graph(rng(B + S + N), B, S, N, norm, same_shape)
    h, n, names = _run(g, ins)
    monkeypatch.setenv("LBR_ADD_NORM", "0")
    h2, n2, names2 = _run(g, ins)
    print(names, names2)
    assert names == [("rmsnorm" if norm == "rms" else "layernorm") + "+add"], names
    assert len(names2) == 2, names2
    np.testing.assert_array_equal(h, h2)
    np.testing.assert_array_equal(n, n2)
    o = run_oracle_all(g, ins)
    for got, ref, name in ((h, h64, "h"), (n, n64, "n")):
        assert normwise_rel(got, ref) <= 1e-4 and normwise_rel(o[name], ref) <= 1e-4, name


def run_oracle_all(graph, inputs):
    from oracle.host_exec import OracleRun
    from runtime.planner import plan
    return OracleRun(plan(graph)).run(inputs)
