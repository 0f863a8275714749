"""Norm prologue on the GPU: RMSNORM / LAYERNORM → MATMUL[_ADD] [→ activation]
run as one DMA GEMM that reads the norm's input and applies the norm to the A
fragments on the fly (statistics accumulated from the same fragments, the
row factors applied in the epilogue).

Each case runs fused, node by node (fusion off), on the CPU oracle, and
against a float64 closed form.  The fused GEMM sums the normalised row in
another order than the norm kernel then the GEMM do, so fused-vs-unfused is
held to 1e-5 normwise, not bit for bit; everything against float64 and the
oracle to 1e-4.  One LayerNorm case has rows whose mean is 500× their spread,
the case a one-pass variance without the row shift would lose: there the
fused GEMM stays within 1e-6 of float64 while the reference's fp32 two-pass
norm (node by node, and the oracle) is ~1e-4 off, so the fused result is
held to float64 at 1e-5 and to the node-by-node path at 1e-4.
"""

import numpy as np
import pytest

from conftest import normwise_rel
from helpers import cf_gelu_tanh, cf_layernorm, cf_rmsnorm, randn, rng, run_oracle
from runtime.ir import Graph, OpType

pytestmark = pytest.mark.gpu

TOL = 1e-4
FUSED_TOL = 1e-5


def _run(graph, inputs, fuse):
    from runtime.executor.compiled import CompiledExecutor
    from runtime.planner import plan
    ex = CompiledExecutor(fuse=fuse)
    ex.compile(plan(graph))
    try:
        y = ex.run(inputs)[graph.outputs[0]]
        return y, [k for _, _, k in ex.fused_runs()], [p["name"] for p in ex.step_params()]
    finally:
        ex.close()


def _graph(r, norm, M, N, K, bias, act, offset):
    """x [1, M, K] → norm → n; c = n·wᵀ (+ b) [→ GELU]; returns (graph, x, float64 result)."""
    g = Graph()
    x = randn(r, 1, M, K)
    if offset:
        x = (500.0 + x).astype(np.float32)
    g.add_tensor("x", (1, M, K))
    g.inputs.append("x")
    gam = (1.0 + 0.5 * randn(r, K)).astype(np.float32)
    g.add_tensor("gam", (K,)).buffer = gam
    g.constants.append("gam")
    if norm == "layer":
        bet = randn(r, K)
        g.add_tensor("bet", (K,)).buffer = bet
        g.constants.append("bet")
        g.add_tensor("n", (1, M, K))
        g.add_node(OpType.LAYERNORM, ["x", "gam", "bet"], "n", {"eps": 1e-5})
        n64 = cf_layernorm(x, gam, bet, 1e-5)
    else:
        g.add_tensor("n", (1, M, K))
        g.add_node(OpType.RMSNORM, ["x", "gam"], "n", {"eps": 1e-6})
        n64 = cf_rmsnorm(x, gam, 1e-6)
    w = randn(r, N, K, scale=0.05)
    g.add_tensor("w", (N, K)).buffer = w
    g.constants.append("w")
    ins = ["n", "w"]
    c = n64 @ w.T.astype(np.float64)
    if bias:
        b = randn(r, N)
        g.add_tensor("b", (N,)).buffer = b
        g.constants.append("b")
        ins.append("b")
        c = c + b
    g.add_tensor("c", (1, M, N))
    g.add_node(OpType.MATMUL_ADD if bias else OpType.MATMUL, ins, "c", {"transpose_b": True})
    out = "c"
    if act:
        g.add_tensor("y", (1, M, N))
        g.add_node(OpType.GELU, ["c"], "y", {})
        c = cf_gelu_tanh(c)
        out = "y"
    g.outputs.append(out)
    return g, x, c


@pytest.mark.parametrize("norm", ["layer", "rms"])
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("tile", [None, "128x128", "128x64", "64x128", "64x64", "32x48", "32x48s4", "64x96",
                                  "32x160", "64x32", "32x64", "32x96", "32x96k64", "64x64k64"])
@pytest.mark.parametrize("M,N,K", [(300, 520, 96), (32, 192, 64), (1000, 300, 768)])
def test_norm_gemm(monkeypatch, norm, bias, tile, M, N, K):
    monkeypatch.setenv("LBR_NORM_PROLOGUE", "always")   # the default takes small GEMMs only
    if tile:
        monkeypatch.setenv("LBR_GEMM_TILE", tile)
    monkeypatch.setenv("LBR_GEMM_KSPLIT", "1")
    g, x, ref = _graph(rng(M + K), norm, M, N, K, bias, False, False)
    _check(g, x, ref, "norm_gemm")


@pytest.mark.parametrize("norm,offset", [("layer", False), ("rms", False), ("layer", True)])
def test_norm_gemm_act(monkeypatch, norm, offset):
    """The prologue under an activation epilogue; the shifted rows (mean 500) too."""
    monkeypatch.setenv("LBR_GEMM_KSPLIT", "1")
    monkeypatch.setenv("LBR_NORM_PROLOGUE", "always")
    g, x, ref = _graph(rng(7), norm, 200, 256, 128, True, True, offset)
    _check(g, x, ref, "gemm_act", shifted=offset)


def _check(g, x, ref, kind, shifted=False):
    y, runs, kernels = _run(g, {"x": x}, True)
    z, plain, _ = _run(g, {"x": x}, False)
    o = run_oracle(g, {"x": x})
    e_f, e_r, e_o, e_or = normwise_rel(y, z), normwise_rel(y, ref), normwise_rel(y, o), normwise_rel(o, ref)
    print(f"{kind}: {kernels}; fused-vs-nodes {e_f:.2e} gpu-vs-ref {e_r:.2e} gpu-vs-oracle {e_o:.2e} "
          f"oracle-vs-ref {e_or:.2e}")
    assert runs == [kind] and plain == []
    assert any("+norm" in k for k in kernels)
    if shifted:   # the fused result is the accurate one
        assert e_r <= FUSED_TOL and e_f <= TOL
    else:
        assert e_f <= FUSED_TOL
    assert e_or <= TOL and e_r <= TOL and e_o <= TOL
