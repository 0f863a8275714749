"""Helpers for op-level tests: one-node graphs run on the GPU executor, the
CPU oracle, and checked against a float64 numpy closed form."""

from __future__ import annotations

import numpy as np

from runtime.ir import Graph, OpType
from runtime.planner import plan


def one_node_graph(op: OpType, inputs: dict[str, np.ndarray], out_shape, attrs=None,
                   consts: dict[str, np.ndarray] | None = None, order: list[str] | None = None,
                   out_dtype: str = "float32") -> Graph:
    """Graph with runtime inputs ``inputs``, constant tensors ``consts`` and one node.

    ``order`` lists the node's input names (default: inputs then consts).
    """
    g = Graph()
    consts = consts or {}
    for name, arr in inputs.items():
        g.add_tensor(name, tuple(arr.shape), str(arr.dtype))
        g.inputs.append(name)
    for name, arr in consts.items():
        g.add_tensor(name, tuple(arr.shape), str(arr.dtype)).buffer = arr
        g.constants.append(name)
    g.add_tensor("out", tuple(out_shape), out_dtype)
    g.add_node(op, order or (list(inputs) + list(consts)), "out", attrs or {})
    g.outputs.append("out")
    return g


def run_gpu(graph: Graph, inputs: dict[str, np.ndarray], use_graph: bool = True,
            kernels: list | None = None) -> np.ndarray:
    """The graph's first output through the compiled executor; `kernels` (a list) receives
    the plan's step names."""
    from runtime.executor.compiled import CompiledExecutor
    ex = CompiledExecutor(use_graph=use_graph)
    ex.compile(plan(graph))
    try:
        if kernels is not None:
            kernels.extend(ex.kernel_names())
        return ex.run(inputs)[graph.outputs[0]]
    finally:
        ex.close()


def run_oracle(graph: Graph, inputs: dict[str, np.ndarray]) -> np.ndarray:
    from oracle.host_exec import OracleRun
    return OracleRun(plan(graph)).run(inputs)[graph.outputs[0]]


def rng(seed: int = 0) -> np.random.Generator:
    return np.random.default_rng(seed)


def randn(r: np.random.Generator, *shape, scale: float = 1.0) -> np.ndarray:
    return (r.standard_normal(shape) * scale).astype(np.float32)


# ---------------------------------------------------------------- float64 closed forms

def cf_attention(q, k, v, causal=False, group=1, mask=None):
    """softmax(q·kᵀ/√hd [+ mask] [+ causal]) · v per (batch·head), kv head = bh // group."""
    q = q.astype(np.float64)
    k = k.astype(np.float64)
    v = v.astype(np.float64)
    bh, s, hd = q.shape[0], q.shape[-2], q.shape[-1]
    qf = q.reshape(-1, s, hd)
    kf = k.reshape(-1, s, hd)
    vf = v.reshape(-1, s, v.shape[-1])
    out = np.empty((qf.shape[0], s, vf.shape[-1]))
    for b in range(qf.shape[0]):
        kvh = b // group
        sc = qf[b] @ kf[kvh].T / np.sqrt(hd)
        if mask is not None:
            sc = sc + mask.reshape(-1, s, s)[b]
        if causal:
            sc = sc + np.triu(np.full((s, s), -np.inf), k=1)
        sc = sc - sc.max(axis=-1, keepdims=True)
        e = np.exp(sc)
        out[b] = (e / e.sum(axis=-1, keepdims=True)) @ vf[kvh]
    return out.reshape(q.shape[:-1] + (v.shape[-1],))


def cf_layernorm(x, g, b, eps):
    x = x.astype(np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * g + b


def cf_rmsnorm(x, w, eps):
    x = x.astype(np.float64)
    return x / np.sqrt((x ** 2).mean(-1, keepdims=True) + eps) * w


def cf_gelu_tanh(x):
    x = x.astype(np.float64)
    return 0.5 * x * (1 + np.tanh(np.sqrt(2 / np.pi) * (x + 0.044715 * x ** 3)))


def cf_silu(x):
    x = x.astype(np.float64)
    return x / (1 + np.exp(-x))
