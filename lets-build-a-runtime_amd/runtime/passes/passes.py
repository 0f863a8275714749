"""Graph optimisation passes and the pass pipelines.

A pass is ``(Graph) -> bool`` (True if it changed the graph) and mutates in
place.  The passes and the pipeline order restate runtime/passes/passes.py
of the reference (94-534): they decide which ops — and which node ids —
reach the executor, so they are kept rule for rule:

* ``absorb_into_matmul``: TRANSPOSE-on-B → transpose_b, constant 2-D B
  pre-transposed, scalar MUL/DIV on inputs/output folded into alpha
  (passes.py:94-225);
* ``constant_fold`` with the registry's numpy evaluators (305-350);
* ``absorb_mask_into_attention``: constant causal masks → causal=True
  (232-287);
* ``eliminate_dead_code`` (357-389);
* ``merge_parallel_matmuls``: MATMULs sharing an input and constant
  weights → one MATMUL + SLICEs (397-502).
"""

from __future__ import annotations

from collections import defaultdict
from dataclasses import dataclass
from typing import Callable

import numpy as np

from ..ir import Graph, Node, OpType
from ..ops import OP_REGISTRY

Pass = Callable[[Graph], bool]

DEFAULT_PIPELINE: list[Pass] = []


@dataclass
class PassResult:
    name: str
    changed: bool
    nodes_before: int
    nodes_after: int

    def __str__(self) -> str:
        if not self.changed:
            return f"[pass] {self.name}: no changes"
        delta = self.nodes_after - self.nodes_before
        return f"[pass] {self.name}: {self.nodes_before} -> {self.nodes_after} nodes ({'+' if delta >= 0 else ''}{delta})"


def _run_one(graph: Graph, p: Pass, log: list[PassResult] | None) -> bool:
    before = len(graph.nodes)
    changed = p(graph)
    if log is not None:
        log.append(PassResult(getattr(p, "__name__", str(p)), changed, before, len(graph.nodes)))
    return changed


def run_pipeline(graph: Graph, pipeline: list[Pass] | None = None, log: list[PassResult] | None = None) -> None:
    """Run each pass once, in order."""
    for p in (pipeline or DEFAULT_PIPELINE):
        _run_one(graph, p, log)


def run_until_stable(graph: Graph, pipeline: list[Pass] | None = None, max_iterations: int = 10,
                     log: list[PassResult] | None = None) -> int:
    """Repeat the pipeline until no pass changes the graph; returns iterations run."""
    passes = pipeline or DEFAULT_PIPELINE
    for it in range(max_iterations):
        changed = False
        for p in passes:
            changed |= _run_one(graph, p, log)
        if not changed:
            return it + 1
    return max_iterations


# ---------------------------------------------------------------- matmul absorption

def _absorb_transpose_b(node: Node, graph: Graph) -> bool:
    if node.attrs.get("transpose_b"):
        return False
    b = node.inputs[1]
    prod = graph.producer(b)
    if prod is None or prod.op != OpType.TRANSPOSE or len(graph.consumers(b)) != 1:
        return False
    nd = len(graph.tensors[prod.inputs[0]].shape)
    if {prod.attrs.get("dim0", 0), prod.attrs.get("dim1", 1)} != {nd - 2, nd - 1}:
        return False
    graph.rewire_input(node.id, b, prod.inputs[0])
    node.attrs["transpose_b"] = True
    graph.remove_node(prod.id)
    graph.remove_tensor(b)
    return True


def _pretranspose_constant_b(node: Node, graph: Graph) -> bool:
    if node.attrs.get("transpose_b"):
        return False
    b = node.inputs[1]
    if b not in graph.constants:
        return False
    info = graph.tensors[b]
    if info.buffer is None or len(info.shape) != 2:
        return False
    info.buffer = np.ascontiguousarray(info.buffer.T)
    info.shape = info.buffer.shape
    node.attrs["transpose_b"] = True
    return True


def _fold_scalar_into_alpha(node: Node, scalar: float, op: OpType) -> None:
    alpha = node.attrs.get("alpha", 1.0)
    node.attrs["alpha"] = alpha * scalar if op == OpType.MUL else alpha / scalar


def _absorb_input_scalars(node: Node, graph: Graph) -> bool:
    changed = False
    for name in list(node.inputs):
        prod = graph.producer(name)
        if (prod is not None and prod.op in (OpType.MUL, OpType.DIV) and "scalar" in prod.attrs
                and len(graph.consumers(name)) == 1):
            _fold_scalar_into_alpha(node, prod.attrs["scalar"], prod.op)
            graph.rewire_input(node.id, name, prod.inputs[0])
            graph.remove_node(prod.id)
            graph.remove_tensor(name)
            changed = True
    return changed


def _absorb_output_scalar(node: Node, graph: Graph) -> bool:
    users = graph.consumers(node.output)
    if len(users) != 1 or users[0].op not in (OpType.MUL, OpType.DIV) or "scalar" not in users[0].attrs:
        return False
    scal = users[0]
    _fold_scalar_into_alpha(node, scal.attrs["scalar"], scal.op)
    for down in graph.consumers(scal.output):
        graph.rewire_input(down.id, scal.output, node.output)
    if scal.output in graph.outputs:
        graph.outputs[graph.outputs.index(scal.output)] = node.output
    graph.remove_node(scal.id)
    graph.remove_tensor(scal.output)
    return True


def absorb_into_matmul(graph: Graph) -> bool:
    """Fold adjacent transposes and scalars into MATMUL flags/alpha (run before folding)."""
    changed = False
    for node in list(graph):
        if node.op != OpType.MATMUL:
            continue
        changed |= _absorb_transpose_b(node, graph)
        changed |= _pretranspose_constant_b(node, graph)
        changed |= _absorb_input_scalars(node, graph)
        changed |= _absorb_output_scalar(node, graph)
    return changed


# ---------------------------------------------------------------- causal masks

def _is_causal_mask(buf: np.ndarray) -> bool:
    """Lower-triangular-True bool mask, or float mask with ~0 on/below and < -1e4 above the diagonal."""
    if buf.ndim < 2 or buf.shape[-1] != buf.shape[-2]:
        return False
    s = buf.shape[-1]
    if s < 2:
        return True
    m = buf.reshape(-1, s, s)[0]
    if buf.dtype == np.bool_:
        return np.array_equal(m, np.tril(np.ones((s, s), dtype=np.bool_)))
    if np.issubdtype(buf.dtype, np.floating):
        return bool(np.allclose(np.tril(m), 0, atol=1e-6) and np.all(m[np.triu_indices(s, k=1)] < -1e4))
    return False


def absorb_mask_into_attention(graph: Graph) -> bool:
    """ATTENTION(Q, K, V, constant causal mask) → ATTENTION(Q, K, V, causal=True)."""
    changed = False
    consts = set(graph.constants)
    for node in list(graph):
        if node.op != OpType.ATTENTION or len(node.inputs) != 4 or node.attrs.get("causal"):
            continue
        mask = node.inputs[3]
        if mask not in consts:
            continue
        buf = graph.tensors[mask].buffer
        if buf is None or not _is_causal_mask(buf):
            continue
        node.attrs["causal"] = True
        graph._consumers[mask].remove(node.id)
        node.inputs = node.inputs[:3]
        graph._order = None
        changed = True
    return changed


# ---------------------------------------------------------------- constant folding

def _has_unresolved_symbols(attrs: dict, symbols: set[str]) -> bool:
    for v in attrs.values():
        if isinstance(v, str) and v in symbols:
            return True
        if isinstance(v, (tuple, list)) and any(isinstance(x, str) and x in symbols for x in v):
            return True
    return False


def constant_fold(graph: Graph) -> bool:
    """Evaluate nodes whose inputs are all constants; results become constants."""
    changed = False
    consts = set(graph.constants)
    symbols = set(graph.dynamic_dims.keys())
    for node in list(graph):
        if not all(t in consts for t in node.inputs):
            continue
        op_def = OP_REGISTRY.get(node.op)
        if op_def is None or op_def.evaluator is None:
            continue
        if symbols and _has_unresolved_symbols(node.attrs, symbols):
            continue
        result = op_def.evaluator([graph.tensors[t].buffer for t in node.inputs], node.attrs)
        want = np.dtype(graph.tensors[node.output].dtype)
        if result.dtype != want:
            result = result.astype(want)
        out = graph.tensors[node.output]
        out.buffer = np.ascontiguousarray(result)
        out.shape = result.shape
        graph.constants.append(node.output)
        consts.add(node.output)
        graph.remove_node(node.id)
        changed = True
    return changed


# ---------------------------------------------------------------- dead code

def eliminate_dead_code(graph: Graph) -> bool:
    """Drop nodes nobody reads (repeatedly) and constants nobody reads."""
    changed = False
    outs = set(graph.outputs)
    while True:
        dead = [n for n in graph.nodes.values() if not graph.consumers(n.output) and n.output not in outs]
        if not dead:
            break
        for n in dead:
            graph.remove_node(n.id)
            graph.remove_tensor(n.output)
        changed = True
    for name in [c for c in graph.constants if not graph.consumers(c) and c not in outs]:
        graph.constants.remove(name)
        graph.remove_tensor(name)
        changed = True
    return changed


# ---------------------------------------------------------------- parallel matmul merge

def merge_parallel_matmuls(graph: Graph) -> bool:
    """Merge MATMULs that read the same activation with compatible constant weights.

    N matmuls become one matmul over the concatenated weight plus N SLICEs
    of its output along the last dim (keeping the original output names).
    """
    changed = False
    consts = set(graph.constants)
    groups: dict[str, list[Node]] = defaultdict(list)
    for node in graph:
        if node.op == OpType.MATMUL and node.inputs[1] in consts:
            groups[node.inputs[0]].append(node)

    for shared, group in groups.items():
        if len(group) < 2:
            continue
        first = group[0]
        trans_b = first.attrs.get("transpose_b", False)
        alpha = first.attrs.get("alpha", 1.0)
        w0 = graph.tensors[first.inputs[1]].shape
        if len(w0) != 2:
            continue
        K = w0[1] if trans_b else w0[0]
        ok = True
        for node in group[1:]:
            ws = graph.tensors[node.inputs[1]].shape
            if (node.attrs.get("transpose_b", False) != trans_b or node.attrs.get("alpha", 1.0) != alpha
                    or len(ws) != 2 or (ws[1] if trans_b else ws[0]) != K):
                ok = False
                break
        if not ok:
            continue

        merged_w = np.concatenate([graph.tensors[n.inputs[1]].buffer for n in group], axis=0 if trans_b else 1)
        w_name = f"_merged_weight_{first.output}"
        graph.add_tensor(w_name, merged_w.shape, "float32").buffer = merged_w
        graph.constants.append(w_name)
        consts.add(w_name)

        in_shape = graph.tensors[shared].shape
        n_total = merged_w.shape[0] if trans_b else merged_w.shape[1]
        out_shape = (*in_shape[:-1], n_total)
        out_name = f"_merged_matmul_{first.output}"
        graph.add_tensor(out_name, out_shape, "float32")
        attrs = {"transpose_b": trans_b}
        if alpha != 1.0:
            attrs["alpha"] = alpha
        graph.add_node(OpType.MATMUL, [shared, w_name], out_name, attrs)

        last = len(out_shape) - 1
        start = 0
        for node in group:
            ws = graph.tensors[node.inputs[1]].shape
            width = ws[0] if trans_b else ws[1]
            old_out, old_w = node.output, node.inputs[1]
            graph.remove_node(node.id)
            graph.add_node(OpType.SLICE, [out_name], old_out, {"dim": last, "start": start, "end": start + width})
            start += width
            if not graph.consumers(old_w):
                if old_w in graph.constants:
                    graph.constants.remove(old_w)
                graph.remove_tensor(old_w)
        changed = True
    return changed


# ---------------------------------------------------------------- pipelines

from .fusion import fuse, fuse_dags  # noqa: E402

PRE_RESOLUTION_PIPELINE: list[Pass] = [
    absorb_into_matmul,
    constant_fold,
    absorb_mask_into_attention,
    fuse_dags,
    merge_parallel_matmuls,
    fuse,
    eliminate_dead_code,
]

POST_RESOLUTION_PIPELINE: list[Pass] = [
    constant_fold,
    absorb_mask_into_attention,
    eliminate_dead_code,
]

DEFAULT_PIPELINE.extend(PRE_RESOLUTION_PIPELINE)
