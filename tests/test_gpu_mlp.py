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
