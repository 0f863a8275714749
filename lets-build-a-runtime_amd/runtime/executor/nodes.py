"""Building the OpNode array from a memory plan, and the device-safety check.

``dispatch_order`` / ``fill_node`` restate the reference's compile step
(runtime/executor/compiled.py:34-157): skip alias nodes whose input is not
external, reject fold-only ops, resolve input/output addresses, append the
node's scratch slot as an extra input, record out_shape / n_dims /
elem_size, and pack extras with the op registry.  Addresses come from a
caller-supplied resolver, so the same builder serves device pointers (the
GPU executor) and host pointers (the CPU oracle used by the tests).

``required_elements`` states, per op, how many elements the kernel reads
from each input given the node's extras — the reference's C code trusts
these blindly; on a GPU an over-read faults the device, so the executor
compares them with the tensors' real sizes before anything is launched.
"""

from __future__ import annotations

import ctypes
from typing import Callable

import numpy as np

from ..ir import FOLD_ONLY_BASE, Graph, Node, OpType
from ..ops import OP_REGISTRY
from ..planner import MemoryPlan
from .common import MAX_DIMS, MAX_INPUTS, COpNode


def is_dispatch_alias(node: Node) -> bool:
    op_def = OP_REGISTRY.get(node.op)
    return op_def is not None and op_def.is_alias(node)


def dispatch_order(plan: MemoryPlan) -> list[Node]:
    """Nodes that reach the executor, in plan order (compiled.py:50-60)."""
    graph = plan.graph
    external = set(graph.inputs) | set(graph.constants)
    out = []
    for node in plan.order:
        if is_dispatch_alias(node) and node.inputs[0] not in external:
            continue
        if node.op.value >= FOLD_ONLY_BASE:
            raise RuntimeError(f"Fold-only op {node.op.name} reached compiled executor — "
                               f"should have been eliminated by constant folding")
        out.append(node)
    return out


def fill_node(c: COpNode, node: Node, graph: Graph, addr: Callable[[str], int], scratch: int | None) -> None:
    """Populate one COpNode (compiled.py:108-157)."""
    c.op = node.op.value
    n_in = len(node.inputs) + (1 if scratch is not None else 0)
    if n_in > MAX_INPUTS:
        raise ValueError(f"node {node.id} ({node.op.name}) has {n_in} inputs; the ABI holds {MAX_INPUTS}")
    c.n_inputs = len(node.inputs)
    for j, name in enumerate(node.inputs):
        c.inputs[j] = addr(name)
    if scratch is not None:
        c.inputs[c.n_inputs] = scratch
        c.n_inputs += 1
    c.output = addr(node.output)
    out = graph.tensors[node.output]
    if len(out.shape) > MAX_DIMS:
        raise ValueError(f"node {node.id}: {len(out.shape)} dims exceed the ABI's {MAX_DIMS}")
    c.n_dims = len(out.shape)
    for d, v in enumerate(out.shape):
        c.out_shape[d] = v
    c.elem_size = np.dtype(out.dtype).itemsize
    op_def = OP_REGISTRY.get(node.op)
    if op_def is not None and op_def.extras is not None:
        vals = op_def.extras(node, graph)
        if len(vals) > MAX_DIMS:
            raise ValueError(f"node {node.id} ({node.op.name}): {len(vals)} extras exceed the ABI's {MAX_DIMS}")
        for i, v in enumerate(vals):
            c.extra[i] = v


def build_nodes(plan: MemoryPlan, addr: Callable[[str], int],
                scratch_addr: Callable[[int, int], int]) -> tuple[ctypes.Array, list[Node]]:
    """COpNode array for the plan.  ``scratch_addr(offset, size)`` maps a scratch slot."""
    order = dispatch_order(plan)
    arr = (COpNode * max(len(order), 1))()
    for i, node in enumerate(order):
        sc = None
        if node.id in plan.scratch:
            off, size = plan.scratch[node.id]
            sc = scratch_addr(off, size)
        fill_node(arr[i], node, plan.graph, addr, sc)
    return arr, order


# ---------------------------------------------------------------- extents

def _numel(shape) -> int:
    n = 1
    for d in shape:
        n *= int(d)
    return n


def _bcast_need(extras: list[int], base: int) -> tuple[int, int]:
    nd = extras[base]
    a_st = extras[base + 1: base + 1 + nd]
    b_st = extras[base + 1 + nd: base + 1 + 2 * nd]
    shape = extras[base + 1 + 2 * nd: base + 1 + 3 * nd]
    if any(s == 0 for s in shape):
        return 0, 0
    a = sum((s - 1) * st for s, st in zip(shape, a_st)) + 1
    b = sum((s - 1) * st for s, st in zip(shape, b_st)) + 1
    return a, b


def required_elements(node: Node, graph: Graph) -> list[tuple[str, int]]:
    """(input name, elements the kernel reads) for each data input of the node."""
    op = node.op
    ex = OP_REGISTRY[op].extras(node, graph) if OP_REGISTRY[op].extras else []
    out_shape = graph.tensors[node.output].shape
    total = _numel(out_shape)
    last = out_shape[-1] if out_shape else 1
    lead = total // last if last else 0
    ins = node.inputs
    if op in (OpType.RELU, OpType.EXP, OpType.TANH, OpType.POW, OpType.GELU, OpType.RSQRT, OpType.SILU,
              OpType.NEG, OpType.COS, OpType.SIN, OpType.SOFTMAX):
        return [(ins[0], total)]
    if op == OpType.ADD:
        mode = ex[0]
        if mode == 2:
            return [(ins[0], total)]
        if mode == 1:
            return [(ins[0], total), (ins[1], total)]
        if mode == 3:
            a, b = _bcast_need(ex, 1)
            return [(ins[0], a), (ins[1], b)]
        return [(ins[0], total), (ins[1], last)]
    if op in (OpType.SUB, OpType.MUL, OpType.DIV):
        mode = ex[0]
        if mode == 1:
            return [(ins[0], total)]
        if mode == 2:
            a, b = _bcast_need(ex, 1)
            return [(ins[0], a), (ins[1], b)]
        return [(ins[0], total), (ins[1], total)]
    if op in (OpType.MAX, OpType.SUM):
        axis, axis_size = ex[0], ex[1]
        outer = _numel(out_shape[:axis]) if axis >= 0 else 1
        inner = _numel(out_shape[axis:]) if axis >= 0 else total
        return [(ins[0], outer * axis_size * inner)]
    if op in (OpType.MATMUL, OpType.MATMUL_ADD):
        K, trans_b, b_is_2d = ex[0], ex[1], ex[2]
        N = out_shape[-1]
        if b_is_2d:
            M, batches = lead, 1
        else:
            M = out_shape[-2]
            batches = _numel(out_shape[:-2])
        need = [(ins[0], batches * M * K), (ins[1], batches * N * K)]
        if op == OpType.MATMUL_ADD:
            need.append((ins[2], N))
        return need
    if op == OpType.RESHAPE:
        return [(ins[0], total)]
    if op == OpType.TRANSPOSE:
        if len(out_shape) == 2:
            return [(ins[0], ex[0] * ex[1])]
        return [(ins[0], ex[0] * ex[1] * ex[2] * ex[3] * ex[4])]
    if op == OpType.SLICE:
        outer, orig, start, length, inner = ex[:5]
        if start < 0 or length < 0 or start + length > orig:
            raise ValueError(f"SLICE node {node.id}: range [{start}, {start + length}) outside dim {orig}")
        return [(ins[0], outer * orig * inner)]
    if op == OpType.CAT:
        dim = ex[0]
        outer = _numel(out_shape[:dim])
        inner = _numel(out_shape[dim + 1:])
        return [(t, outer * ex[1 + k] * inner) for k, t in enumerate(ins)]
    if op == OpType.EMBEDDING:
        return [(ins[0], lead), (ins[1], 0)]  # ids are range-checked on the device
    if op == OpType.LAYERNORM:
        return [(ins[0], total), (ins[1], last), (ins[2], last)]
    if op == OpType.RMSNORM:
        return [(ins[0], total), (ins[1], last)]
    if op == OpType.FUSED_BIAS_RELU:
        return [(ins[0], total), (ins[1], last)]
    if op == OpType.GATED_ACT:
        if ex[0]:
            return [(ins[0], total), (ins[1], last), (ins[2], total)]
        return [(ins[0], total), (ins[1], total)]
    if op == OpType.ATTENTION:
        S, hd, _, has_mask, group = ex[0], ex[1], ex[2], ex[3], max(ex[4], 1)
        bh = _numel(out_shape[:-2])
        kv_heads = (bh - 1) // group + 1 if bh else 0
        need = [(ins[0], bh * S * hd), (ins[1], kv_heads * S * hd), (ins[2], kv_heads * S * hd)]
        if has_mask:
            need.append((ins[3], bh * S * S))
        return need
    return []


def check_extents(order: list[Node], graph: Graph) -> None:
    """Raise ValueError if any node would read past the end of one of its inputs."""
    for node in order:
        out_dtype = graph.tensors[node.output].dtype
        for name, need in required_elements(node, graph):
            have = _numel(graph.tensors[name].shape)
            if need > have:
                raise ValueError(f"node {node.id} ({node.op.name}) would read {need} elements of '{name}', "
                                 f"which holds {have}")
        if node.op not in (OpType.RESHAPE, OpType.TRANSPOSE, OpType.SLICE, OpType.CAT) and out_dtype != "float32":
            raise ValueError(f"node {node.id} ({node.op.name}) produces {out_dtype}; device kernels compute fp32")
