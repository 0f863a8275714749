"""Pins the CPU oracle (oracle/oracle_executor.c, the restated reference
executor) against what the mathematics fixes, on the CPU.

Each op is checked against an independent float64 closed form on inputs
chosen so that plausible mistakes show: non-square and non-symmetric
operands (a transposed operand fails), distinct KV heads under GQA (a wrong
head index fails), causal rows checked against brute-force softmax (an
off-by-one on the diagonal fails), shifted/scaled LayerNorm inputs (a
dropped mean or eps fails), both attention paths (S ≤ 256 standard,
S > 256 flash with ragged tiles).  The reference holds no golden vectors
for this path (its tests draw unseeded random inputs against closed forms);
its known-answer tests are in test_host_layer.py.
"""

import numpy as np
import pytest

from runtime.ir import OpType
from helpers import (cf_attention, cf_gelu_tanh, cf_layernorm, cf_rmsnorm, cf_silu, one_node_graph, randn, rng,
                     run_oracle)
from conftest import normwise_rel


def _ok(graph, inputs, ref, tol):
    y = run_oracle(graph, inputs)
    assert y.shape == ref.shape
    err = normwise_rel(y, ref)
    assert err <= tol, err
    return y


@pytest.mark.parametrize("M,N,K,trans_b,batches,b2d", [
    (65, 70, 300, True, 1, True), (33, 17, 9, False, 1, True), (12, 20, 16, True, 3, False),
    (1, 40, 64, True, 1, True), (1, 40, 64, False, 2, False), (130, 66, 257, False, 1, True)])
@pytest.mark.parametrize("bias", [False, True])
def test_oracle_gemm(M, N, K, trans_b, batches, b2d, bias):
    r = rng(M + N + K)
    a = randn(r, 1, M, K) if b2d else randn(r, batches, M, K)
    bshape = (N, K) if trans_b else (K, N)
    b = randn(r, *bshape) if b2d else randn(r, batches, *bshape)
    ref = a.astype(np.float64) @ (np.swapaxes(b, -2, -1) if trans_b else b).astype(np.float64)
    consts = {"b": b}
    attrs = {"transpose_b": trans_b}
    op = OpType.MATMUL
    if bias:
        consts["bias"] = randn(r, N)
        ref = ref + consts["bias"]
        op = OpType.MATMUL_ADD
    else:
        attrs["alpha"] = -0.75
        ref = ref * -0.75
    out_shape = (1, M, N) if b2d else (batches, M, N)
    _ok(one_node_graph(op, {"a": a}, out_shape, attrs, consts), {"a": a}, ref, 1e-5)


@pytest.mark.parametrize("B,H,S,hd,causal,group", [
    (1, 4, 32, 16, True, 1), (2, 2, 19, 8, False, 1), (1, 4, 300, 32, True, 1), (1, 8, 270, 16, False, 4),
    (1, 4, 257, 8, True, 2), (1, 2, 1, 8, True, 1)])
def test_oracle_attention(B, H, S, hd, causal, group):
    r = rng(S + hd)
    q, k, v = randn(r, B, H, S, hd), randn(r, B, H // group, S, hd), randn(r, B, H // group, S, hd)
    attrs = {"causal": True} if causal else {}
    if group > 1:
        attrs["group_size"] = group
    g = one_node_graph(OpType.ATTENTION, {"q": q, "k": k, "v": v}, (B, H, S, hd), attrs)
    _ok(g, {"q": q, "k": k, "v": v}, cf_attention(q, k, v, causal=causal, group=group), 1e-5)


def test_oracle_attention_brute_force_causal_rows():
    """Row i of causal attention = softmax over keys 0..i only (tiny, explicit loop)."""
    r = rng(99)
    S, hd = 6, 8
    q, k, v = randn(r, 1, 1, S, hd), randn(r, 1, 1, S, hd), randn(r, 1, 1, S, hd)
    g = one_node_graph(OpType.ATTENTION, {"q": q, "k": k, "v": v}, q.shape, {"causal": True})
    y = run_oracle(g, {"q": q, "k": k, "v": v})[0, 0]
    for i in range(S):
        s = np.array([float(q[0, 0, i].astype(np.float64) @ k[0, 0, j].astype(np.float64)) / np.sqrt(hd)
                      for j in range(i + 1)])
        p = np.exp(s - s.max())
        p /= p.sum()
        want = sum(p[j] * v[0, 0, j].astype(np.float64) for j in range(i + 1))
        np.testing.assert_allclose(y[i], want, rtol=1e-5, atol=1e-6)
    # row 0 sees only key 0
    np.testing.assert_allclose(y[0], v[0, 0, 0], rtol=1e-6)


def test_oracle_attention_mask_long_sequence():
    r = rng(7)
    S = 280
    q, k, v = randn(r, 1, 2, S, 16), randn(r, 1, 2, S, 16), randn(r, 1, 2, S, 16)
    mask = np.where(r.random((1, 2, S, S)) < 0.3, -1e9, 0.0).astype(np.float32)
    g = one_node_graph(OpType.ATTENTION, {"q": q, "k": k, "v": v, "mask": mask}, q.shape, {})
    _ok(g, {"q": q, "k": k, "v": v, "mask": mask}, cf_attention(q, k, v, mask=mask), 1e-5)


@pytest.mark.parametrize("S", [12, 280])
def test_oracle_attention_mask_replaces_causal(S):
    """A node with both a mask and the causal flag: the reference applies the additive mask
    alone (attn.c:40-48, "either custom additive mask or causal (never both)"), and with a
    mask never takes the flash path (executor.c:389).  The closed form of the mask alone
    holds; the mask plus the causal pattern, which differs in every row but the last, does not."""
    r = rng(S + 3)
    q, k, v = randn(r, 1, 2, S, 16), randn(r, 1, 2, S, 16), randn(r, 1, 2, S, 16)
    mask = np.where(r.random((1, 2, S, S)) < 0.3, -1e9, 0.0).astype(np.float32)
    for i in range(S):
        mask[..., i, i] = 0.0
    g = one_node_graph(OpType.ATTENTION, {"q": q, "k": k, "v": v, "mask": mask}, q.shape, {"causal": True})
    _ok(g, {"q": q, "k": k, "v": v, "mask": mask}, cf_attention(q, k, v, mask=mask), 1e-5)
    both = cf_attention(q, k, v, mask=mask, causal=True)
    assert normwise_rel(both, cf_attention(q, k, v, mask=mask)) > 1e-2


def test_oracle_norms_softmax():
    r = rng(1)
    x = randn(r, 1, 9, 300) * 4 + 2.5
    gm, bt = randn(r, 300), randn(r, 300)
    _ok(one_node_graph(OpType.LAYERNORM, {"x": x}, x.shape, {"eps": 1e-5}, {"g": gm, "b": bt}), {"x": x},
        cf_layernorm(x, gm, bt, 1e-5), 1e-5)
    _ok(one_node_graph(OpType.RMSNORM, {"x": x}, x.shape, {"eps": 1e-6}, {"w": gm}), {"x": x},
        cf_rmsnorm(x, gm, 1e-6), 1e-5)
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(-1, keepdims=True))
    _ok(one_node_graph(OpType.SOFTMAX, {"x": x}, x.shape, {"axis": 2}), {"x": x}, e / e.sum(-1, keepdims=True), 1e-5)


def test_oracle_layernorm_known_answer():
    """[1, 2, 3, 4] with γ=1, β=0: mean 2.5, var 1.25 → (x-2.5)/sqrt(1.25+eps)."""
    x = np.array([[1, 2, 3, 4]], dtype=np.float32)
    g = one_node_graph(OpType.LAYERNORM, {"x": x}, x.shape, {"eps": 0.0},
                       {"g": np.ones(4, np.float32), "b": np.zeros(4, np.float32)})
    y = run_oracle(g, {"x": x})
    np.testing.assert_allclose(y, (x - 2.5) / np.sqrt(1.25), rtol=1e-6)


def test_oracle_elementwise():
    r = rng(2)
    x = randn(r, 4, 50) * 2
    up, bias = randn(r, 4, 50), randn(r, 50)
    cases = [
        (OpType.GELU, {}, cf_gelu_tanh(x)), (OpType.SILU, {}, cf_silu(x)), (OpType.TANH, {}, np.tanh(x)),
        (OpType.NEG, {}, -x.astype(np.float64)), (OpType.RELU, {}, np.maximum(x, 0)),
        (OpType.EXP, {}, np.exp(x.astype(np.float64))), (OpType.SIN, {}, np.sin(x)), (OpType.COS, {}, np.cos(x)),
    ]
    for op, attrs, ref in cases:
        _ok(one_node_graph(op, {"x": x}, x.shape, attrs), {"x": x}, ref, 1e-6)
    _ok(one_node_graph(OpType.GATED_ACT, {"x": x, "up": up}, x.shape, {"act": "silu"}), {"x": x, "up": up},
        cf_silu(x) * up, 1e-6)
    _ok(one_node_graph(OpType.GATED_ACT, {"x": x, "up": up}, x.shape, {"act": "gelu", "has_bias": True},
                       {"bias": bias}, order=["x", "bias", "up"]), {"x": x, "up": up},
        cf_gelu_tanh(x.astype(np.float64) + bias) * up, 1e-6)
    _ok(one_node_graph(OpType.FUSED_BIAS_RELU, {"x": x}, x.shape, {}, {"bias": bias}), {"x": x},
        np.maximum(x.astype(np.float64) + bias, 0), 1e-7)


def test_oracle_broadcast_and_modes():
    r = rng(3)
    a = randn(r, 2, 3, 4, 5)
    for b in (randn(r, 1, 3, 1, 5), randn(r, 5), randn(r, 2, 3, 4, 5), randn(r, 4, 1)):
        for op, f in ((OpType.ADD, np.add), (OpType.SUB, np.subtract), (OpType.MUL, np.multiply)):
            _ok(one_node_graph(op, {"a": a}, a.shape, {}, {"b": b}), {"a": a}, f(a.astype(np.float64), b), 1e-7)
    _ok(one_node_graph(OpType.DIV, {"a": a}, a.shape, {"scalar": 4.0}), {"a": a}, a / 4.0, 1e-7)


def test_oracle_data_movement_exact():
    x = np.arange(2 * 3 * 4 * 5, dtype=np.float32).reshape(2, 3, 4, 5)
    g = one_node_graph(OpType.TRANSPOSE, {"x": x}, (2, 4, 3, 5), {"dim0": 1, "dim1": 2})
    np.testing.assert_array_equal(run_oracle(g, {"x": x}), np.swapaxes(x, 1, 2))
    g = one_node_graph(OpType.SLICE, {"x": x}, (2, 3, 2, 5), {"dim": 2, "start": 1, "end": 3})
    np.testing.assert_array_equal(run_oracle(g, {"x": x}), x[:, :, 1:3])
    y = np.arange(2 * 3 * 2 * 5, dtype=np.float32).reshape(2, 3, 2, 5) + 1000
    g = one_node_graph(OpType.CAT, {"x": x, "y": y}, (2, 3, 6, 5), {"dim": 2})
    np.testing.assert_array_equal(run_oracle(g, {"x": x, "y": y}), np.concatenate([x, y], axis=2))
    m = np.arange(12, dtype=np.float32).reshape(3, 4)
    g = one_node_graph(OpType.TRANSPOSE, {"m": m}, (4, 3), {"dim0": 0, "dim1": 1})
    np.testing.assert_array_equal(run_oracle(g, {"m": m}), m.T)


def test_oracle_reductions():
    r = rng(4)
    x = randn(r, 3, 7, 11)
    for op, f in ((OpType.SUM, np.sum), (OpType.MAX, np.max)):
        for axis in (0, 1, 2):
            ref = f(x.astype(np.float64), axis=axis, keepdims=True)
            _ok(one_node_graph(op, {"x": x}, ref.shape, {"axis": axis, "keepdim": True}), {"x": x}, ref, 1e-6)


@pytest.mark.parametrize("key", ["toy", "gpt2w"])
def test_oracle_end_to_end_vs_torch(key):
    """Whole plans on the oracle vs PyTorch eager in float64."""
    from workloads import export_workload, reference_forward
    from runtime.passes import run_pipeline
    from runtime.planner import plan
    from oracle.host_exec import OracleRun
    model, x, graph = export_workload(key)
    run_pipeline(graph)
    y = OracleRun(plan(graph)).run({graph.inputs[0]: x})[graph.outputs[0]]
    assert normwise_rel(y, reference_forward(model, x)) < 1e-5
