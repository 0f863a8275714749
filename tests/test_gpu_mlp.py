"""Fused MLP on the GPU: [LAYERNORM | RMSNORM →] MATMUL_ADD → RELU | GELU |
SILU → MATMUL_ADD [→ ADD(residual)] as one mlp_rows kernel (16 rows per
workgroup, the hidden rows in LDS, each wavefront's weight fragments in
registers: tiny MLPs, where the unfused chain is launch-bound).

Each case runs fused, node by node (fusion off), on the CPU oracle, and
against a float64 closed form.  The kernel repeats the unfused kernels'
arithmetic (norm_wave_rows' lane sums; the DMA GEMM's per-output K order),
so where the node-by-node plan runs those kernels — widths that are
multiples of the DMA GEMM's 32-wide K step, one K range — the two outputs
are equal bit for bit; otherwise within 1e-5.  Everything against float64
and the oracle: 1e-4 normwise.
"""

import numpy as np
import pytest

from conftest import normwise_rel
from helpers import cf_gelu_tanh, cf_layernorm, cf_rmsnorm, cf_silu, randn, rng, run_oracle
from runtime.ir import Graph, OpType

pytestmark = pytest.mark.gpu

ACTS = {"gelu": (OpType.GELU, cf_gelu_tanh), "relu": (OpType.RELU, lambda v: np.maximum(v, 0.0)),
        "silu": (OpType.SILU, cf_silu)}


def _run(graph, inputs, fuse):
    from runtime.executor.compiled import CompiledExecutor
    from runtime.planner import plan
    ex = CompiledExecutor(fuse=fuse)
    ex.compile(plan(graph))
    try:
        y = ex.run(inputs)[graph.outputs[0]]
        return y, [k for _, _, k in ex.fused_runs()], [p["kernel"] for p in ex.step_params()]
    finally:
        ex.close()


def _graph(r, M, D, H, norm, act, resid, bias2=True):
    g = Graph()
    x = randn(r, 1, M, D)
    g.add_tensor("x", (1, M, D))
    g.inputs.append("x")
    a, a64 = "x", x.astype(np.float64)
    if norm:
        gam = (1.0 + 0.5 * randn(r, D)).astype(np.float32)
        g.add_tensor("gam", (D,)).buffer = gam
        g.constants.append("gam")
        g.add_tensor("n", (1, M, D))
        if norm == "layer":
            bet = randn(r, D)
            g.add_tensor("bet", (D,)).buffer = bet
            g.constants.append("bet")
            g.add_node(OpType.LAYERNORM, ["x", "gam", "bet"], "n", {"eps": 1e-5})
            a64 = cf_layernorm(x, gam, bet, 1e-5)
        else:
            g.add_node(OpType.RMSNORM, ["x", "gam"], "n", {"eps": 1e-6})
            a64 = cf_rmsnorm(x, gam, 1e-6)
        a = "n"
    w1, b1 = randn(r, H, D, scale=0.05), randn(r, H)
    w2, b2 = randn(r, D, H, scale=0.05), randn(r, D)
    for name, arr in (("w1", w1), ("b1", b1), ("w2", w2), ("b2", b2)):
        g.add_tensor(name, arr.shape).buffer = arr
        g.constants.append(name)
    opk, f = ACTS[act]
    g.add_tensor("c1", (1, M, H))
    g.add_node(OpType.MATMUL_ADD, [a, "w1", "b1"], "c1", {"transpose_b": True})
    g.add_tensor("h", (1, M, H))
    g.add_node(opk, ["c1"], "h", {})
    g.add_tensor("c2", (1, M, D))
    if bias2:
        g.add_node(OpType.MATMUL_ADD, ["h", "w2", "b2"], "c2", {"transpose_b": True})
    else:
        g.add_node(OpType.MATMUL, ["h", "w2"], "c2", {"transpose_b": True})
    h64 = f(a64 @ w1.T.astype(np.float64) + b1)
    y64 = h64 @ w2.T.astype(np.float64) + (b2 if bias2 else 0.0)
    out = "c2"
    if resid:
        g.add_tensor("y", (1, M, D))
        g.add_node(OpType.ADD, ["x", "c2"], "y", {})
        y64 = y64 + x
        out = "y"
    g.outputs.append(out)
    return g, x, y64


@pytest.mark.parametrize("norm", ["layer", "rms", None])
@pytest.mark.parametrize("act", ["gelu", "relu", "silu"])
@pytest.mark.parametrize("resid", [True, False])
@pytest.mark.parametrize("M,D,H", [(32, 64, 256), (50, 64, 192), (16, 128, 128), (7, 32, 256), (33, 96, 128)])
def test_mlp(monkeypatch, norm, act, resid, M, D, H):
    monkeypatch.setenv("LBR_GEMM_KSPLIT", "1")
    g, x, ref = _graph(rng(M + D + H), M, D, H, norm, act, resid)
    _check(g, x, ref, exact=D % 32 == 0 and H % 32 == 0)


def test_mlp_no_bias_on_second_gemm(monkeypatch):
    monkeypatch.setenv("LBR_GEMM_KSPLIT", "1")
    g, x, ref = _graph(rng(3), 40, 64, 128, "layer", "gelu", True, bias2=False)
    _check(g, x, ref, exact=True)


def _check(g, x, ref, exact):
    y, runs, kernels = _run(g, {"x": x}, True)
    z, plain, _ = _run(g, {"x": x}, False)
    o = run_oracle(g, {"x": x})
    e_f, e_r, e_o = normwise_rel(y, z), normwise_rel(y, ref), normwise_rel(o, ref)
    print(f"{kernels}: fused-vs-nodes {e_f:.2e} (max |d| {np.abs(y - z).max():.1e}) gpu-vs-ref {e_r:.2e} "
          f"oracle-vs-ref {e_o:.2e}")
    assert runs == ["mlp"] and plain == []
    assert any(k.startswith("mlp_rows") for k in kernels)
    if exact:
        np.testing.assert_array_equal(y, z)
    else:
        assert e_f <= 1e-5
    assert e_r <= 1e-4 and e_o <= 1e-4 and normwise_rel(y, o) <= 1e-4


def _tail_graph(r, M, D, Ha, hd, H, norm, act, tail_resid, proj_bias=True):
    """Attention block tail: O [1, Ha, M, hd] → TRANSPOSE → RESHAPE → o-projection
    (+ bo) → x1 = x + · → [norm] → MLP → y = x1 + · (tail_resid "x1"), x + · ("x")
    or no residual (None).  The projection (a TRANSPOSE_GEMM run) joins the MLP's
    kernel."""
    g = Graph()
    x, o = randn(r, 1, M, D), randn(r, 1, Ha, M, hd)
    for name, arr in (("x", x), ("o", o)):
        g.add_tensor(name, arr.shape)
        g.inputs.append(name)
    K0 = Ha * hd

    def const(name, arr):
        g.add_tensor(name, arr.shape).buffer = arr
        g.constants.append(name)

    wo, bo = randn(r, D, K0, scale=0.05), randn(r, D)
    const("wo", wo)
    const("bo", bo)
    g.add_tensor("ot", (1, M, Ha, hd))
    g.add_node(OpType.TRANSPOSE, ["o"], "ot", {"dim0": 1, "dim1": 2})
    g.add_tensor("or", (1, M, K0))
    g.add_node(OpType.RESHAPE, ["ot"], "or", {"shape": [1, M, K0]})
    g.add_tensor("c0", (1, M, D))
    o2 = np.swapaxes(o, 1, 2).reshape(1, M, K0).astype(np.float64)
    c0 = o2 @ wo.T.astype(np.float64)
    if proj_bias:
        g.add_node(OpType.MATMUL_ADD, ["or", "wo", "bo"], "c0", {"transpose_b": True})
        c0 = c0 + bo
    else:
        g.add_node(OpType.MATMUL, ["or", "wo"], "c0", {"transpose_b": True})
    g.add_tensor("x1", (1, M, D))
    g.add_node(OpType.ADD, ["x", "c0"], "x1", {})
    x1 = x + c0
    a, a64 = "x1", x1
    if norm:
        gam = (1.0 + 0.5 * randn(r, D)).astype(np.float32)
        const("gam", gam)
        g.add_tensor("n", (1, M, D))
        if norm == "layer":
            bet = randn(r, D)
            const("bet", bet)
            g.add_node(OpType.LAYERNORM, ["x1", "gam", "bet"], "n", {"eps": 1e-5})
            a64 = cf_layernorm(x1, gam, bet, 1e-5)
        else:
            g.add_node(OpType.RMSNORM, ["x1", "gam"], "n", {"eps": 1e-6})
            a64 = cf_rmsnorm(x1, gam, 1e-6)
        a = "n"
    w1, b1 = randn(r, H, D, scale=0.05), randn(r, H)
    w2, b2 = randn(r, D, H, scale=0.05), randn(r, D)
    for name, arr in (("w1", w1), ("b1", b1), ("w2", w2), ("b2", b2)):
        const(name, arr)
    opk, f = ACTS[act]
    g.add_tensor("c1", (1, M, H))
    g.add_node(OpType.MATMUL_ADD, [a, "w1", "b1"], "c1", {"transpose_b": True})
    g.add_tensor("h", (1, M, H))
    g.add_node(opk, ["c1"], "h", {})
    g.add_tensor("c2", (1, M, D))
    g.add_node(OpType.MATMUL_ADD, ["h", "w2", "b2"], "c2", {"transpose_b": True})
    y64 = f(a64 @ w1.T.astype(np.float64) + b1) @ w2.T.astype(np.float64) + b2
    out = "c2"
    if tail_resid:
        g.add_tensor("y", (1, M, D))
        g.add_node(OpType.ADD, [tail_resid, "c2"], "y", {})
        y64 = y64 + (x1 if tail_resid == "x1" else x)
        out = "y"
    g.outputs.append(out)
    return g, {"x": x, "o": o}, y64


def _run_named(graph, inputs, fuse):
    from runtime.executor.compiled import CompiledExecutor
    from runtime.planner import plan
    ex = CompiledExecutor(fuse=fuse)
    ex.compile(plan(graph))
    try:
        return ex.run(inputs)[graph.outputs[0]], ex.step_params()
    finally:
        ex.close()


@pytest.mark.parametrize("tail_resid", ["x1", "x", None])
@pytest.mark.parametrize("norm,act", [("layer", "gelu"), ("rms", "silu"), (None, "relu")])
@pytest.mark.parametrize("M,D,Ha,hd,H", [(32, 64, 4, 16, 256), (50, 64, 2, 32, 192), (16, 128, 8, 16, 128),
                                         (33, 96, 3, 32, 128), (7, 64, 2, 32, 128)])
def test_mlp_with_projection(monkeypatch, tail_resid, norm, act, M, D, Ha, hd, H):
    """The attention output projection inside the MLP kernel: bit-equal to the same
    plan with the two kernels apart, within 1e-5 of the node-by-node plan, and
    1e-4 of float64 and the oracle."""
    monkeypatch.setenv("LBR_GEMM_KSPLIT", "1")
    g, ins, ref = _tail_graph(rng(M + D + H + hd), M, D, Ha, hd, H, norm, act, tail_resid)
    y, steps = _run_named(g, ins, True)
    monkeypatch.setenv("LBR_PROJ_MLP", "0")
    z, apart = _run_named(g, ins, True)
    monkeypatch.delenv("LBR_PROJ_MLP")
    monkeypatch.setenv("LBR_FUSE", "0")
    w, _ = _run_named(g, ins, True)
    o = run_oracle(g, ins)
    names = [s["name"] for s in steps]
    print(f"{names}: joined-vs-apart max |d| {np.abs(y - z).max():.1e}, vs nodes {normwise_rel(y, w):.2e}, "
          f"vs ref {normwise_rel(y, ref):.2e}")
    assert len(steps) == 1 and "+proj" in names[0], names
    assert sorted(s["kind"] for s in apart) == ["mlp", "transpose_gemm"], apart
    np.testing.assert_array_equal(y, z)
    assert normwise_rel(y, w) <= 1e-5
    assert normwise_rel(y, ref) <= 1e-4 and normwise_rel(o, ref) <= 1e-4 and normwise_rel(y, o) <= 1e-4


def test_mlp_with_projection_no_bias(monkeypatch):
    monkeypatch.setenv("LBR_GEMM_KSPLIT", "1")
    g, ins, ref = _tail_graph(rng(5), 40, 64, 4, 16, 128, "layer", "gelu", "x1", proj_bias=False)
    y, steps = _run_named(g, ins, True)
    monkeypatch.setenv("LBR_PROJ_MLP", "0")
    z, _ = _run_named(g, ins, True)
    assert any("+proj" in s["name"] for s in steps)
    np.testing.assert_array_equal(y, z)
    assert normwise_rel(y, ref) <= 1e-4
