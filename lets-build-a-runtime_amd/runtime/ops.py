"""Per-op definitions: numpy evaluators, alias/in-place flags, extras packers,
scratch sizes and shape rules — the single registry every layer reads.

Mirrors runtime/ops.py:52-690 of the reference.  What must be identical,
and is therefore restated rule for rule:

* extras packers (ops.py:137-329) — they define the integers in
  ``OpNode.extra`` that the device dispatch decodes, including float
  bit-casts (ops.py:34-39);
* scratch calculators (ops.py:427-459) — they size the planner's scratch
  lifetimes and so shift every later arena offset;
* alias / in-place flags (ops.py:498-583) — they decide memory sharing;
* shape rules (ops.py:339-420) and numpy evaluators, which produce the
  constant-folded weights (RoPE tables, masks) the device consumes.
"""

from __future__ import annotations

import struct
from dataclasses import dataclass
from typing import Any, Callable

import numpy as np

from .ir import Graph, Node, OpType

NumpyEvaluator = Callable[[list[np.ndarray], dict[str, Any]], np.ndarray]
ScratchCalculator = Callable[[list[tuple[int, ...]], tuple[int, ...], dict], int]
ExtrasPacker = Callable[[Node, Graph], list[int]]
ShapeInfer = Callable[[list[tuple[int, ...]], dict[str, Any]], tuple[int, ...]]
AliasPredicate = bool | Callable[[Node], bool]
AliasOffset = Callable[[Node], int]


def _float_bits(f: float) -> int:
    """float32 bit pattern as a signed int32 (read back in C through a union)."""
    return struct.unpack("<i", struct.pack("<f", f))[0]


@dataclass
class OpDef:
    """Everything the host layer knows about one op.

    evaluator     numpy implementation (constant folding)
    scratch       bytes of single-step workspace the op needs (planner)
    alias         output is a view of input 0 (bool or predicate on the node)
    alias_offset  byte offset of that view inside input 0
    inplace       output may take over a dying input 0's arena slot
    extras        packer for OpNode.extra
    shape         output-shape rule; None = shape of input 0
    """
    evaluator: NumpyEvaluator | None = None
    scratch: ScratchCalculator | None = None
    alias: AliasPredicate = False
    alias_offset: AliasOffset | None = None
    inplace: bool = False
    extras: ExtrasPacker | None = None
    shape: ShapeInfer | None = None

    def is_alias(self, node: Node) -> bool:
        return self.alias(node) if callable(self.alias) else bool(self.alias)


# ---------------------------------------------------------------- evaluators

def _eval_softmax(ins, attrs):
    x = ins[0]
    ax = attrs["axis"]
    e = np.exp(x - np.max(x, axis=ax, keepdims=True))
    return e / np.sum(e, axis=ax, keepdims=True)


def _eval_layernorm(ins, attrs):
    x, gamma, beta = ins[0], ins[1], ins[2]
    eps = attrs.get("eps", 1e-5)
    mu = np.mean(x, axis=-1, keepdims=True)
    var = np.var(x, axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * gamma + beta


def _eval_attention(ins, attrs):
    q, k, v = ins[0], ins[1], ins[2]
    scores = np.matmul(q, np.swapaxes(k, -2, -1)) * (1.0 / np.sqrt(q.shape[-1]))
    if len(ins) > 3:
        scores = scores + ins[3]
    if attrs.get("causal"):
        s = q.shape[-2]
        scores = scores + np.triu(np.full((s, s), -np.inf, dtype=np.float32), k=1)
    scores -= np.max(scores, axis=-1, keepdims=True)
    e = np.exp(scores)
    return np.matmul(e / np.sum(e, axis=-1, keepdims=True), v)


def _eval_gated_act(ins, attrs):
    if attrs.get("has_bias", False):
        v = ins[0] + ins[1]
        up = ins[2]
    else:
        v = ins[0]
        up = ins[1]
    if attrs.get("act", "silu") == "silu":
        act = v / (1.0 + np.exp(-v))
    else:
        act = 0.5 * v * (1 + np.tanh(0.7978845608 * (v + 0.044715 * v ** 3)))
    return act * up


def _eval_slice_tensor(ins, attrs):
    x, dim = ins[0], attrs["dim"]
    start = attrs.get("start", 0)
    end = attrs.get("end", x.shape[dim])
    idx = tuple(slice(start, end) if d == dim else slice(None) for d in range(x.ndim))
    return x[idx]


def _eval_diff(ins, attrs):
    prepend = ins[1] if len(ins) > 1 else None
    return np.diff(ins[0], n=attrs.get("n", 1), axis=attrs.get("dim", -1), prepend=prepend)


def _eval_index(ins, attrs):
    n_idx = attrs.get("n_indices", len(ins) - 1)
    nones = set(attrs.get("none_positions", []))
    picks: list[Any] = []
    k = 1
    for i in range(n_idx):
        if i in nones:
            picks.append(slice(None))
        else:
            picks.append(ins[k])
            k += 1
    return ins[0][tuple(picks)]


def _binary_eval(fn):
    return lambda ins, a: fn(ins[0], a["scalar"] if "scalar" in a else ins[1])


def _matmul_eval(ins, a):
    b = np.swapaxes(ins[1], -2, -1) if a.get("transpose_b") else ins[1]
    return ins[0] @ b * a.get("alpha", 1.0)


def _matmul_add_eval(ins, a):
    return _matmul_eval(ins, a) + ins[2]


def _rmsnorm_eval(ins, a):
    x = ins[0]
    return x / np.sqrt(np.mean(x ** 2, axis=-1, keepdims=True) + a.get("eps", 1e-5)) * ins[1]


def _gelu_eval(ins, a):
    x = ins[0]
    return 0.5 * x * (1 + np.tanh(0.7978845608 * (x + 0.044715 * x ** 3)))


# ---------------------------------------------------------------- extras packers

def _matmul_extras(node: Node, graph: Graph) -> list[int]:
    """[K, trans_b, b_is_2d, alpha_bits]; alpha_bits = 0 means alpha 1.0."""
    a_shape = graph.tensors[node.inputs[0]].shape
    b_shape = graph.tensors[node.inputs[1]].shape
    alpha = node.attrs.get("alpha", 1.0)
    return [
        a_shape[-1],
        1 if node.attrs.get("transpose_b") else 0,
        1 if (len(b_shape) == 2 and len(a_shape) > 2) else 0,
        _float_bits(alpha) if alpha != 1.0 else 0,
    ]


def _transpose_extras(node: Node, graph: Graph) -> list[int]:
    """2-D: [rows, cols]; N-D swapaxes: [outer, A, middle, B, inner]."""
    shape = graph.tensors[node.inputs[0]].shape
    if len(shape) == 2:
        return [shape[0], shape[1]]
    d0, d1 = sorted((node.attrs.get("dim0", 0), node.attrs.get("dim1", 1)))
    prod = lambda dims: int(np.prod(dims, dtype=np.int64)) if len(dims) else 1
    return [prod(shape[:d0]), shape[d0], prod(shape[d0 + 1:d1]), shape[d1], prod(shape[d1 + 1:])]


def _broadcast_strides(shape: tuple, out_shape: tuple) -> list[int]:
    """Element strides of ``shape`` broadcast against ``out_shape`` (0 on broadcast dims)."""
    nd = len(out_shape)
    lead = nd - len(shape)
    strides = []
    for d in range(nd):
        if d < lead or shape[d - lead] == 1:
            strides.append(0)
        else:
            s = 1
            for k in range(d - lead + 1, len(shape)):
                s *= shape[k]
            strides.append(s)
    return strides


def _pack_broadcast(a_shape: tuple, b_shape: tuple, out_shape: tuple) -> list[int]:
    """[ndim, a_strides..., b_strides..., out_shape...]"""
    return ([len(out_shape)] + _broadcast_strides(a_shape, out_shape)
            + _broadcast_strides(b_shape, out_shape) + list(out_shape))


def _add_extras(node: Node, graph: Graph) -> list[int]:
    """Mode in extra[0]: 0 bias row, 1 same shape, 2 scalar (+bits), 3 broadcast (+packing)."""
    if "scalar" in node.attrs:
        return [2, _float_bits(node.attrs["scalar"])]
    a_shape = graph.tensors[node.inputs[0]].shape
    b_shape = graph.tensors[node.inputs[1]].shape
    if a_shape == b_shape:
        return [1]
    if len(b_shape) == 1 and b_shape[-1] == a_shape[-1]:
        return [0]
    out_shape = node.attrs.get("_out_shape") or graph.tensors[node.output].shape
    return [3] + _pack_broadcast(a_shape, b_shape, out_shape)


def _scalar_binop_extras(node: Node, graph: Graph) -> list[int]:
    """SUB/MUL/DIV mode in extra[0]: 0 same shape, 1 scalar (+bits), 2 broadcast (+packing)."""
    if "scalar" in node.attrs:
        return [1, _float_bits(node.attrs["scalar"])]
    a_shape = graph.tensors[node.inputs[0]].shape
    b_shape = graph.tensors[node.inputs[1]].shape
    if a_shape == b_shape:
        return [0]
    return [2] + _pack_broadcast(a_shape, b_shape, graph.tensors[node.output].shape)


def _reduction_extras(node: Node, graph: Graph) -> list[int]:
    axis = node.attrs.get("axis", -1)
    return [axis, graph.tensors[node.inputs[0]].shape[axis]]


def _eps_extras(node: Node, graph: Graph) -> list[int]:
    return [_float_bits(node.attrs.get("eps", 1e-5))]


def _attention_extras(node: Node, graph: Graph) -> list[int]:
    """[seq_len, head_dim, causal, has_mask, group_size]"""
    q = graph.tensors[node.inputs[0]].shape
    return [q[-2], q[-1], 1 if node.attrs.get("causal") else 0, 1 if len(node.inputs) > 3 else 0,
            node.attrs.get("group_size", 1)]


def _pow_extras(node: Node, graph: Graph) -> list[int]:
    return [_float_bits(node.attrs.get("scalar", 2.0))]


def _embedding_extras(node: Node, graph: Graph) -> list[int]:
    return [graph.tensors[node.inputs[1]].shape[-1]]


def _cat_extras(node: Node, graph: Graph) -> list[int]:
    dim = node.attrs["dim"]
    return [dim] + [graph.tensors[t].shape[dim] for t in node.inputs]


def _gated_act_extras(node: Node, graph: Graph) -> list[int]:
    return [1 if node.attrs.get("has_bias") else 0, 0 if node.attrs.get("act", "silu") == "silu" else 1]


def _slice_alias(node: Node) -> bool:
    """dim-0 slices are views; any other dim needs a strided copy."""
    return node.attrs.get("dim", 0) == 0


def _slice_extras(node: Node, graph: Graph) -> list[int]:
    """[outer, orig_dim_size, start, len, inner] for the strided copy."""
    shape = graph.tensors[node.inputs[0]].shape
    dim = node.attrs["dim"]
    start = node.attrs["start"]
    end = min(node.attrs["end"], shape[dim])
    outer = 1
    for d in range(dim):
        outer *= shape[d]
    inner = 1
    for d in range(dim + 1, len(shape)):
        inner *= shape[d]
    return [outer, shape[dim], start, end - start, inner]


# ---------------------------------------------------------------- shape rules

def _shape_broadcast_binary(in_shapes, attrs):
    if "scalar" in attrs:
        return in_shapes[0]
    return tuple(np.broadcast_shapes(in_shapes[0], in_shapes[1]))


def _shape_matmul(in_shapes, attrs):
    a, b = in_shapes[0], in_shapes[1]
    return (*a[:-1], b[-2] if attrs.get("transpose_b") else b[-1])


def _shape_reshape(in_shapes, attrs):
    target = list(attrs["shape"])
    if any(isinstance(d, str) for d in target):
        return tuple(target)
    total = 1
    for d in in_shapes[0]:
        total *= d
    free = None
    known = 1
    for i, d in enumerate(target):
        if d == -1:
            free = i
        else:
            known *= d
    if free is not None:
        target[free] = total // known
    return tuple(target)


def _shape_transpose(in_shapes, attrs):
    s = list(in_shapes[0])
    d0, d1 = attrs["dim0"], attrs["dim1"]
    s[d0], s[d1] = s[d1], s[d0]
    return tuple(s)


def _shape_permute(in_shapes, attrs):
    return tuple(in_shapes[0][i] for i in attrs["axes"])


def _shape_slice(in_shapes, attrs):
    s = list(in_shapes[0])
    dim = attrs["dim"]
    s[dim] = min(attrs["end"], s[dim]) - attrs.get("start", 0)
    return tuple(s)


def _shape_reduce(in_shapes, attrs):
    s = list(in_shapes[0])
    if attrs.get("keepdim", False):
        s[attrs["axis"]] = 1
    else:
        s.pop(attrs["axis"])
    return tuple(s)


def _shape_attention(in_shapes, attrs):
    return (*in_shapes[0][:-1], in_shapes[2][-1])


def _shape_embedding(in_shapes, attrs):
    return (*in_shapes[0], in_shapes[1][-1])


def _shape_cat(in_shapes, attrs):
    dim = attrs["dim"]
    s = list(in_shapes[0])
    s[dim] = sum(x[dim] for x in in_shapes)
    return tuple(s)


# ---------------------------------------------------------------- scratch

# Attention kernel switch and tile sizes of the reference's CPU kernels
# (csrc/ops/attn.c:106-111, csrc/executor.c:23).  They only size the
# planner's scratch slot here, which keeps arena offsets identical.
FLASH_SEQ_THRESHOLD = 256
FLASH_BR = 128
FLASH_BC = 256


def _use_flash_attention(seq_len: int, attrs: dict) -> bool:
    return seq_len > FLASH_SEQ_THRESHOLD


def _attention_scratch(input_shapes, output_shape, attrs) -> int:
    """bh·BR·BC floats on the flash path, bh·S·S on the standard path."""
    q = input_shapes[0]
    bh = 1
    for d in q[:-2]:
        bh *= d
    s = q[-2]
    per = FLASH_BR * FLASH_BC if _use_flash_attention(s, attrs) else s * s
    return bh * per * 4


# ---------------------------------------------------------------- registry

OP_REGISTRY: dict[OpType, OpDef] = {
    OpType.ADD: OpDef(inplace=True, extras=_add_extras, shape=_shape_broadcast_binary,
                      evaluator=_binary_eval(lambda a, b: a + b)),
    OpType.SUB: OpDef(inplace=True, extras=_scalar_binop_extras, shape=_shape_broadcast_binary,
                      evaluator=_binary_eval(lambda a, b: a - b)),
    OpType.MUL: OpDef(inplace=True, extras=_scalar_binop_extras, shape=_shape_broadcast_binary,
                      evaluator=_binary_eval(lambda a, b: a * b)),
    OpType.DIV: OpDef(inplace=True, extras=_scalar_binop_extras, shape=_shape_broadcast_binary,
                      evaluator=_binary_eval(lambda a, b: a / b)),
    OpType.RELU: OpDef(inplace=True, evaluator=lambda ins, a: np.maximum(ins[0], 0)),
    OpType.EXP: OpDef(inplace=True, evaluator=lambda ins, a: np.exp(ins[0])),
    OpType.POW: OpDef(inplace=True, extras=_pow_extras, evaluator=lambda ins, a: np.power(ins[0], a["scalar"])),
    OpType.TANH: OpDef(inplace=True, evaluator=lambda ins, a: np.tanh(ins[0])),
    # not in-place in the reference (its macOS kernel reads x after writing out)
    OpType.GELU: OpDef(inplace=False, evaluator=_gelu_eval),
    OpType.RSQRT: OpDef(inplace=True, evaluator=lambda ins, a: 1.0 / np.sqrt(ins[0])),
    OpType.SILU: OpDef(inplace=True, evaluator=lambda ins, a: ins[0] / (1.0 + np.exp(-ins[0]))),
    OpType.NEG: OpDef(inplace=True, evaluator=lambda ins, a: -ins[0]),
    OpType.COS: OpDef(inplace=True, evaluator=lambda ins, a: np.cos(ins[0])),
    OpType.SIN: OpDef(inplace=True, evaluator=lambda ins, a: np.sin(ins[0])),

    OpType.MAX: OpDef(extras=_reduction_extras, shape=_shape_reduce,
                      evaluator=lambda ins, a: np.max(ins[0], axis=a["axis"], keepdims=a.get("keepdim", False))),
    OpType.SUM: OpDef(extras=_reduction_extras, shape=_shape_reduce,
                      evaluator=lambda ins, a: np.sum(ins[0], axis=a["axis"], keepdims=a.get("keepdim", False))),
    OpType.SOFTMAX: OpDef(evaluator=_eval_softmax),

    OpType.RESHAPE: OpDef(alias=True, shape=_shape_reshape, evaluator=lambda ins, a: ins[0].reshape(a["shape"])),
    OpType.TRANSPOSE: OpDef(extras=_transpose_extras, shape=_shape_transpose,
                            evaluator=lambda ins, a: np.swapaxes(ins[0], a["dim0"], a["dim1"])),
    OpType.PERMUTE: OpDef(shape=_shape_permute, evaluator=lambda ins, a: np.transpose(ins[0], a["axes"])),
    OpType.SLICE: OpDef(alias=_slice_alias, alias_offset=lambda n: n.attrs.get("byte_offset", 0),
                        extras=_slice_extras, shape=_shape_slice, evaluator=_eval_slice_tensor),

    OpType.LAYERNORM: OpDef(extras=_eps_extras, evaluator=_eval_layernorm),
    OpType.RMSNORM: OpDef(extras=_eps_extras, evaluator=_rmsnorm_eval),
    OpType.MATMUL: OpDef(extras=_matmul_extras, shape=_shape_matmul, evaluator=_matmul_eval),
    OpType.EMBEDDING: OpDef(extras=_embedding_extras, shape=_shape_embedding,
                            evaluator=lambda ins, a: ins[1][ins[0].astype(int)]),
    OpType.CAT: OpDef(extras=_cat_extras, shape=_shape_cat,
                      evaluator=lambda ins, a: np.concatenate(ins, axis=a["dim"])),

    OpType.MATMUL_ADD: OpDef(extras=_matmul_extras, shape=_shape_matmul, evaluator=_matmul_add_eval),
    OpType.FUSED_BIAS_RELU: OpDef(inplace=True, evaluator=lambda ins, a: np.maximum(ins[0] + ins[1], 0)),
    OpType.ATTENTION: OpDef(extras=_attention_extras, scratch=_attention_scratch, shape=_shape_attention,
                            evaluator=_eval_attention),
    OpType.GATED_ACT: OpDef(extras=_gated_act_extras, evaluator=_eval_gated_act),

    # fold-only
    OpType.ARANGE: OpDef(evaluator=lambda ins, a: np.arange(a["start"], a["end"], dtype=np.dtype(a["dtype"])),
                         shape=lambda in_shapes, a: (a["end"] - a["start"],)),
    OpType.CAST: OpDef(evaluator=lambda ins, a: ins[0].astype(a["target_dtype"])),
    OpType.EXPAND: OpDef(evaluator=lambda ins, a: np.broadcast_to(ins[0], a["shape"])),
    OpType.DIFF: OpDef(evaluator=_eval_diff),
    OpType.CMP_NE: OpDef(evaluator=_binary_eval(lambda a, b: a != b)),
    OpType.CMP_LE: OpDef(evaluator=lambda ins, a: ins[0] <= ins[1]),
    OpType.CMP_EQ: OpDef(evaluator=lambda ins, a: ins[0] == ins[1]),
    OpType.CUMSUM: OpDef(evaluator=lambda ins, a: np.cumsum(ins[0], axis=a["dim"])),
    OpType.BITWISE_AND: OpDef(evaluator=lambda ins, a: ins[0] & ins[1]),
    OpType.INDEX: OpDef(evaluator=_eval_index),
}


# ---------------------------------------------------------------- dynamic shapes

def resolve_graph(graph: Graph, bindings: dict[str, int]) -> Graph:
    """Concrete copy of a (possibly symbolic) optimised graph.

    Tensor metadata, node attrs and connectivity are copied with every
    symbol replaced by its binding; weight buffers are shared.  Shapes are
    re-inferred from the bound inputs, RESHAPE targets are made concrete,
    and the post-resolution passes fold what the bindings made constant
    (runtime/ops.py:590-662).
    """
    out = Graph()
    for name, t in graph.tensors.items():
        out.add_tensor(name, t.shape, t.dtype).buffer = t.buffer

    def sub(v):
        if isinstance(v, str) and v in bindings:
            return bindings[v]
        if isinstance(v, tuple):
            return tuple(sub(x) for x in v)
        if isinstance(v, list):
            return [sub(x) for x in v]
        return v

    for node in graph:
        out.add_node(node.op, list(node.inputs), node.output, {k: sub(v) for k, v in node.attrs.items()})
    out.inputs = list(graph.inputs)
    out.outputs = list(graph.outputs)
    out.constants = list(graph.constants)
    out.dynamic_dims = graph.dynamic_dims

    new_shapes = {}
    for name in out.inputs:
        shape = list(out.tensors[name].shape)
        for sym, specs in graph.dynamic_dims.items():
            if sym not in bindings:
                continue
            for tname, dim in specs:
                if tname == name:
                    shape[dim] = bindings[sym]
        new_shapes[name] = tuple(shape)
    infer_shapes(out, new_shapes)

    for node in out:
        if node.op == OpType.RESHAPE:
            node.attrs["shape"] = out.tensors[node.output].shape

    from .passes import POST_RESOLUTION_PIPELINE, run_pipeline
    run_pipeline(out, POST_RESOLUTION_PIPELINE)
    return out


def infer_shapes(graph: Graph, input_shapes: dict[str, tuple[int, ...]]) -> None:
    """Set input shapes and propagate output shapes in topological order."""
    for name, shape in input_shapes.items():
        graph.tensors[name].shape = shape
    for node in graph:
        op_def = OP_REGISTRY.get(node.op)
        shapes = [graph.tensors[t].shape for t in node.inputs]
        if op_def is not None and op_def.shape is not None:
            graph.tensors[node.output].shape = op_def.shape(shapes, node.attrs)
        else:
            graph.tensors[node.output].shape = shapes[0]
