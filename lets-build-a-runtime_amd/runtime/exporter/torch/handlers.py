"""ATen → IR handlers used by the exporter.

Restates runtime/exporter/torch/handlers.py of the reference (600-688):
same ATen coverage, same decomposition (linear → TRANSPOSE + MATMUL [+ ADD],
addmm → MATMUL + ADD, mean → SUM + DIV, permute → TRANSPOSE when it swaps
exactly two axes, split + getitem → SLICE with a byte offset, SDPA →
ATTENTION with causal / GQA group_size), same tensor naming (fx node names
plus ``_weight_t`` / ``_mm`` / ``_sum`` suffixes).  Note: ``aten.gelu`` maps
to the tanh-approximation GELU whatever its ``approximate`` argument, as in
the reference (handlers.py:605).
"""

from __future__ import annotations

import operator
import sys
from typing import Callable

import numpy as np
import torch

from ...ir import Graph, OpType

OpHandler = Callable[[object, Graph, dict, dict], None]


# ---------------------------------------------------------------- helpers

def _sym_or_val(d, symbol_map: dict[str, str]):
    """int stays int; a SymInt becomes its user symbol (or is concretised without a map)."""
    if isinstance(d, int):
        return d
    if symbol_map:
        s = str(d)
        return symbol_map.get(s, s)
    return int(d.node.hint)


def _output_meta(fx) -> tuple[tuple[int, ...], str]:
    val = fx.meta["val"]
    return tuple(d if isinstance(d, int) else int(d.node.hint) for d in val.shape), \
        str(val.dtype).replace("torch.", "")


def _emit(fx, graph: Graph, node_map: dict, op: OpType, inputs: list[str], attrs: dict | None = None) -> None:
    shape, dtype = _output_meta(fx)
    graph.add_tensor(fx.name, shape, dtype)
    graph.add_node(op, inputs, fx.name, attrs)
    node_map[fx.name] = fx.name


def _get_axis(fx, arg_index: int = 1, default: int = -1):
    ndim = len(fx.args[0].meta["val"].shape)
    axis = fx.args[arg_index] if len(fx.args) > arg_index else fx.kwargs.get("dim", default)
    if isinstance(axis, (list, tuple)) and len(axis) == 1:
        axis = axis[0]
    if isinstance(axis, int):
        axis = axis % ndim
    return axis


def _is_transpose(axes: list[int]) -> bool:
    return sum(1 for i, a in enumerate(axes) if a != i) == 2


def _keepdim(fx) -> bool:
    return fx.args[2] if len(fx.args) > 2 else fx.kwargs.get("keepdim", False)


# ---------------------------------------------------------------- factories

def _binary(op: OpType) -> OpHandler:
    def handler(fx, graph, node_map, symbol_map):
        inputs = [node_map[fx.args[0].name]]
        attrs = {}
        rhs = fx.args[1]
        if hasattr(rhs, "name"):
            inputs.append(node_map[rhs.name])
        else:
            attrs["scalar"] = float(rhs)
        _emit(fx, graph, node_map, op, inputs, attrs or None)
    return handler


def _simple(op: OpType) -> OpHandler:
    def handler(fx, graph, node_map, symbol_map):
        _emit(fx, graph, node_map, op, [node_map[a.name] for a in fx.args if hasattr(a, "name")])
    return handler


def _reduction(op: OpType) -> OpHandler:
    def handler(fx, graph, node_map, symbol_map):
        _emit(fx, graph, node_map, op, [node_map[fx.args[0].name]], {"axis": _get_axis(fx), "keepdim": _keepdim(fx)})
    return handler


# ---------------------------------------------------------------- handlers

def _handle_max_dim(fx, graph, node_map, symbol_map):
    """aten.max.dim → MAX on the values; getitem 0 aliases it."""
    val = fx.meta["val"][0]
    graph.add_tensor(fx.name, tuple(val.shape), str(val.dtype).replace("torch.", ""))
    graph.add_node(OpType.MAX, [node_map[fx.args[0].name]], fx.name, {"axis": _get_axis(fx), "keepdim": _keepdim(fx)})
    node_map[fx.name] = fx.name


def _handle_softmax(fx, graph, node_map, symbol_map):
    _emit(fx, graph, node_map, OpType.SOFTMAX, [node_map[fx.args[0].name]], {"axis": _get_axis(fx)})


def _handle_mean(fx, graph, node_map, symbol_map):
    """mean.dim → SUM (name ``<fx>_sum``) + DIV by the axis size (symbolic if dynamic)."""
    shape, dtype = _output_meta(fx)
    axis = _get_axis(fx)
    sum_name = f"{fx.name}_sum"
    graph.add_tensor(sum_name, shape, dtype)
    graph.add_node(OpType.SUM, [node_map[fx.args[0].name]], sum_name, {"axis": axis, "keepdim": _keepdim(fx)})
    count = _sym_or_val(fx.args[0].meta["val"].shape[axis], symbol_map)
    if isinstance(count, int):
        count = float(count)
    graph.add_tensor(fx.name, shape, dtype)
    graph.add_node(OpType.DIV, [sum_name], fx.name, {"scalar": count})
    node_map[fx.name] = fx.name


def _handle_transpose_2d(fx, graph, node_map, symbol_map):
    _emit(fx, graph, node_map, OpType.TRANSPOSE, [node_map[fx.args[0].name]], {"dim0": 0, "dim1": 1})


def _handle_transpose_int(fx, graph, node_map, symbol_map):
    nd = len(fx.args[0].meta["val"].shape)
    _emit(fx, graph, node_map, OpType.TRANSPOSE, [node_map[fx.args[0].name]],
          {"dim0": fx.args[1] % nd, "dim1": fx.args[2] % nd})


def _handle_permute(fx, graph, node_map, symbol_map):
    axes = list(fx.args[1])
    src = [node_map[fx.args[0].name]]
    if _is_transpose(axes):
        d0, d1 = [i for i, a in enumerate(axes) if a != i]
        _emit(fx, graph, node_map, OpType.TRANSPOSE, src, {"dim0": d0, "dim1": d1})
    else:
        _emit(fx, graph, node_map, OpType.PERMUTE, src, {"axes": axes})


def _handle_reshape(fx, graph, node_map, symbol_map):
    """view / reshape / unflatten / unsqueeze / squeeze → RESHAPE to the traced output shape."""
    target = tuple(_sym_or_val(d, symbol_map) for d in fx.meta["val"].shape)
    _emit(fx, graph, node_map, OpType.RESHAPE, [node_map[fx.args[0].name]], {"shape": target})


def _handle_linear(fx, graph, node_map, symbol_map):
    """linear(x, W[N,K], b?) → TRANSPOSE(W) + MATMUL (+ ADD bias)."""
    x = node_map[fx.args[0].name]
    w = node_map[fx.args[1].name]
    bias = fx.args[2] if len(fx.args) > 2 else None
    shape, dtype = _output_meta(fx)
    wt = f"{fx.name}_weight_t"
    ws = graph.tensors[w].shape
    graph.add_tensor(wt, (ws[1], ws[0]), dtype)
    graph.add_node(OpType.TRANSPOSE, [w], wt, {"dim0": 0, "dim1": 1})
    if bias is None:
        _emit(fx, graph, node_map, OpType.MATMUL, [x, wt])
        return
    mm = f"{fx.name}_mm"
    graph.add_tensor(mm, shape, dtype)
    graph.add_node(OpType.MATMUL, [x, wt], mm)
    graph.add_tensor(fx.name, shape, dtype)
    graph.add_node(OpType.ADD, [mm, node_map[bias.name]], fx.name)
    node_map[fx.name] = fx.name


def _handle_addmm(fx, graph, node_map, symbol_map):
    """addmm(b, x, W[K,N]) (HF Conv1D) → MATMUL + ADD."""
    bias, x, w = (node_map[fx.args[i].name] for i in range(3))
    shape, dtype = _output_meta(fx)
    mm = f"{fx.name}_mm"
    graph.add_tensor(mm, shape, dtype)
    graph.add_node(OpType.MATMUL, [x, w], mm)
    graph.add_tensor(fx.name, shape, dtype)
    graph.add_node(OpType.ADD, [mm, bias], fx.name)
    node_map[fx.name] = fx.name


def _handle_layer_norm(fx, graph, node_map, symbol_map):
    inputs = [node_map[fx.args[0].name], node_map[fx.args[2].name], node_map[fx.args[3].name]]
    _emit(fx, graph, node_map, OpType.LAYERNORM, inputs, {"eps": fx.args[4] if len(fx.args) > 4 else 1e-5})


def _handle_pow(fx, graph, node_map, symbol_map):
    _emit(fx, graph, node_map, OpType.POW, [node_map[fx.args[0].name]], {"scalar": float(fx.args[1])})


def _handle_ne_scalar(fx, graph, node_map, symbol_map):
    _emit(fx, graph, node_map, OpType.CMP_NE, [node_map[fx.args[0].name]], {"scalar": fx.args[1]})


def _handle_embedding(fx, graph, node_map, symbol_map):
    """embedding(table, ids) → EMBEDDING(ids, table)."""
    _emit(fx, graph, node_map, OpType.EMBEDDING, [node_map[fx.args[1].name], node_map[fx.args[0].name]])


def _handle_sdpa(fx, graph, node_map, symbol_map):
    """scaled_dot_product_attention → ATTENTION (mask input, causal flag, GQA group size)."""
    inputs = [node_map[fx.args[i].name] for i in range(3)]
    if len(fx.args) > 3 and fx.args[3] is not None and hasattr(fx.args[3], "name"):
        inputs.append(node_map[fx.args[3].name])
    causal = bool(fx.args[5]) if len(fx.args) > 5 else bool(fx.kwargs.get("is_causal", False))
    attrs = {"causal": True} if causal else {}
    qs = fx.args[0].meta["val"].shape
    ks = fx.args[1].meta["val"].shape
    if len(qs) >= 3 and len(qs) == len(ks):
        nq, nkv = qs[-3], ks[-3]
        if isinstance(nq, int) and isinstance(nkv, int) and nq > nkv and nq % nkv == 0:
            attrs["group_size"] = nq // nkv
    _emit(fx, graph, node_map, OpType.ATTENTION, inputs, attrs)


def _handle_getitem(fx, graph, node_map, symbol_map):
    """getitem of split → SLICE (with byte offset); getitem 0 of max.dim → alias."""
    src = fx.args[0]
    index = fx.args[1]
    if src.target == torch.ops.aten.split.Tensor:
        x = node_map[src.args[0].name]
        chunk = src.args[1]
        dim = src.args[2] if len(src.args) > 2 else 0
        xs = graph.tensors[x].shape
        if dim < 0:
            dim += len(xs)
        _, dtype = _output_meta(fx)
        trailing = 1
        for d in xs[dim + 1:]:
            trailing *= d
        _emit(fx, graph, node_map, OpType.SLICE, [x],
              {"byte_offset": index * chunk * trailing * np.dtype(dtype).itemsize, "dim": dim,
               "start": index * chunk, "end": index * chunk + chunk})
        return
    if index == 0 and src.name in node_map:
        node_map[fx.name] = node_map[src.name]


def _handle_noop(fx, graph, node_map, symbol_map):
    node_map[fx.name] = node_map[fx.args[0].name]


def _handle_assert_metadata(fx, graph, node_map, symbol_map):
    pass


def _materialize_constant(fx, graph, node_map, data: np.ndarray) -> None:
    shape, dtype = _output_meta(fx)
    graph.add_tensor(fx.name, shape, dtype).buffer = data
    graph.constants.append(fx.name)
    node_map[fx.name] = fx.name


def _resolve_scalar_arg(arg, symbol_map):
    if isinstance(arg, (int, float)):
        return arg
    val = arg.meta.get("val")
    if val is not None:
        return _sym_or_val(val, symbol_map)
    return int(arg)


def _handle_arange(fx, graph, node_map, symbol_map):
    end = _resolve_scalar_arg(fx.args[0], symbol_map)
    _, dtype = _output_meta(fx)
    _emit(fx, graph, node_map, OpType.ARANGE, [], {"start": 0, "end": end, "dtype": dtype})


def _handle_arange_start(fx, graph, node_map, symbol_map):
    start = _resolve_scalar_arg(fx.args[0], symbol_map)
    end = _resolve_scalar_arg(fx.args[1], symbol_map)
    _, dtype = _output_meta(fx)
    _emit(fx, graph, node_map, OpType.ARANGE, [], {"start": start, "end": end, "dtype": dtype})


def _handle_new_ones(fx, graph, node_map, symbol_map):
    shape, dtype = _output_meta(fx)
    _materialize_constant(fx, graph, node_map, np.ones(shape, dtype=np.dtype(dtype)))


def _handle_to_dtype(fx, graph, node_map, symbol_map):
    _, out_dtype = _output_meta(fx)
    in_dtype = str(fx.args[0].meta["val"].dtype).replace("torch.", "")
    if in_dtype == out_dtype:
        node_map[fx.name] = node_map[fx.args[0].name]
    else:
        _emit(fx, graph, node_map, OpType.CAST, [node_map[fx.args[0].name]], {"target_dtype": out_dtype})


def _handle_expand(fx, graph, node_map, symbol_map):
    target = tuple(_sym_or_val(d, symbol_map) for d in fx.meta["val"].shape)
    _emit(fx, graph, node_map, OpType.EXPAND, [node_map[fx.args[0].name]], {"shape": target})


def _handle_slice_tensor(fx, graph, node_map, symbol_map):
    """slice.Tensor → SLICE; a full [0:maxsize] slice aliases its input."""
    dim = fx.args[1] if len(fx.args) > 1 else 0
    start = fx.args[2] if len(fx.args) > 2 else 0
    if len(fx.args) > 3:
        raw = fx.args[3]
        if isinstance(raw, int):
            end = raw
        else:
            hint = int(raw.node.hint)
            end = hint if hint >= sys.maxsize else _sym_or_val(raw, symbol_map)
    else:
        end = _sym_or_val(fx.args[0].meta["val"].shape[dim], symbol_map)
    if isinstance(start, int) and start == 0 and isinstance(end, int) and end >= sys.maxsize:
        node_map[fx.name] = node_map[fx.args[0].name]
        return
    _emit(fx, graph, node_map, OpType.SLICE, [node_map[fx.args[0].name]], {"dim": dim, "start": start, "end": end})


def _handle_diff(fx, graph, node_map, symbol_map):
    inputs = [node_map[fx.args[0].name]]
    attrs = {"n": fx.args[1] if len(fx.args) > 1 else 1, "dim": fx.args[2] if len(fx.args) > 2 else -1}
    if len(fx.args) > 3 and fx.args[3] is not None and hasattr(fx.args[3], "name"):
        inputs.append(node_map[fx.args[3].name])
        attrs["has_prepend"] = True
    _emit(fx, graph, node_map, OpType.DIFF, inputs, attrs)


def _handle_cumsum(fx, graph, node_map, symbol_map):
    _emit(fx, graph, node_map, OpType.CUMSUM, [node_map[fx.args[0].name]], {"dim": fx.args[1]})


def _handle_index(fx, graph, node_map, symbol_map):
    idx_list = fx.args[1]
    inputs = [node_map[fx.args[0].name]]
    attrs = {"n_indices": len(idx_list)}
    nones = []
    for i, idx in enumerate(idx_list):
        if idx is None:
            nones.append(i)
        else:
            inputs.append(node_map[idx.name])
    if nones:
        attrs["none_positions"] = nones
    _emit(fx, graph, node_map, OpType.INDEX, inputs, attrs)


def _handle_cat(fx, graph, node_map, symbol_map):
    tensors = fx.args[0]
    dim = fx.args[1] if len(fx.args) > 1 else 0
    if isinstance(dim, int) and dim < 0:
        dim += len(tensors[0].meta["val"].shape)
    _emit(fx, graph, node_map, OpType.CAT, [node_map[t.name] for t in tensors], {"dim": dim})


aten = torch.ops.aten

ATEN_HANDLERS: dict[object, OpHandler] = {
    aten.relu.default: _simple(OpType.RELU),
    aten.exp.default: _simple(OpType.EXP),
    aten.tanh.default: _simple(OpType.TANH),
    aten.gelu.default: _simple(OpType.GELU),
    aten.rsqrt.default: _simple(OpType.RSQRT),
    aten.silu.default: _simple(OpType.SILU),
    aten.neg.default: _simple(OpType.NEG),
    aten.cos.default: _simple(OpType.COS),
    aten.sin.default: _simple(OpType.SIN),
    aten.mm.default: _simple(OpType.MATMUL),
    aten.matmul.default: _simple(OpType.MATMUL),
    aten.bmm.default: _simple(OpType.MATMUL),
    aten.le.Tensor: _simple(OpType.CMP_LE),
    aten.eq.Tensor: _simple(OpType.CMP_EQ),
    aten.__and__.Tensor: _simple(OpType.BITWISE_AND),
    aten.add.Tensor: _binary(OpType.ADD),
    aten.sub.Tensor: _binary(OpType.SUB),
    aten.mul.Tensor: _binary(OpType.MUL),
    aten.div.Tensor: _binary(OpType.DIV),
    aten.amax.default: _reduction(OpType.MAX),
    aten.sum.dim_IntList: _reduction(OpType.SUM),
    aten.max.dim: _handle_max_dim,
    aten.mean.dim: _handle_mean,
    aten._softmax.default: _handle_softmax,
    aten.softmax.int: _handle_softmax,
    aten.t.default: _handle_transpose_2d,
    aten.numpy_T.default: _handle_transpose_2d,
    aten.transpose.int: _handle_transpose_int,
    aten.permute.default: _handle_permute,
    aten.view.default: _handle_reshape,
    aten.reshape.default: _handle_reshape,
    aten.unflatten.int: _handle_reshape,
    aten.unsqueeze.default: _handle_reshape,
    aten.squeeze.dim: _handle_reshape,
    aten.linear.default: _handle_linear,
    aten.addmm.default: _handle_addmm,
    aten.layer_norm.default: _handle_layer_norm,
    aten.pow.Tensor_Scalar: _handle_pow,
    aten.ne.Scalar: _handle_ne_scalar,
    aten.embedding.default: _handle_embedding,
    aten.scaled_dot_product_attention.default: _handle_sdpa,
    aten.split.Tensor: _handle_noop,
    operator.getitem: _handle_getitem,
    aten.arange.default: _handle_arange,
    aten.arange.start: _handle_arange_start,
    aten.new_ones.default: _handle_new_ones,
    aten.to.dtype_layout: _handle_to_dtype,
    aten.to.dtype: _handle_to_dtype,
    aten.expand.default: _handle_expand,
    aten.slice.Tensor: _handle_slice_tensor,
    aten.diff.default: _handle_diff,
    aten.cumsum.default: _handle_cumsum,
    aten.index.Tensor: _handle_index,
    aten.cat.default: _handle_cat,
    aten.contiguous.default: _handle_noop,
    aten.dropout.default: _handle_noop,
    aten.alias.default: _handle_noop,
    aten._assert_tensor_metadata.default: _handle_assert_metadata,
}
