"""PyTorch → graph IR via torch.export.

Restates runtime/exporter/torch/exporter.py of the reference (28-208):
``torch.export`` traces the model in eval/no-grad mode (with deferred
runtime asserts when dims are dynamic), placeholders become graph inputs or
weight constants according to the export signature, every ``call_function``
node is mapped by the ATen handler registry, and the output node names the
graph outputs.  Tensor names are the fx node names, so node and tensor
naming — and with it node ids and planner order — match the reference for
the same model and torch version.
"""

from __future__ import annotations

import torch
import torch.nn as nn
from torch.export.graph_signature import InputKind

from ...ir import Graph
from .handlers import ATEN_HANDLERS


def export_pytorch(model: nn.Module, example_inputs: tuple,
                   dynamic_dims: dict[str, list[tuple[str, int]]] | None = None,
                   example_kwargs: dict | None = None) -> Graph:
    """Export ``model`` to a Graph.

    dynamic_dims maps a symbol to the (input name, dim) pairs it stands for,
    e.g. ``{"L": [("x", 1)]}``; those dims stay symbolic in RESHAPE/EXPAND
    attrs until ``resolve_graph`` binds them.
    """
    model.eval()
    with torch.no_grad():
        return _export_core(model, example_inputs, dynamic_dims, example_kwargs)


def _export_core(model, example_inputs, dynamic_dims=None, example_kwargs=None) -> Graph:
    torch_dynamic = None
    extra = {}
    if dynamic_dims:
        torch_dynamic = {}
        for sym, specs in dynamic_dims.items():
            dim = torch.export.Dim(sym, min=1)
            for input_name, idx in specs:
                torch_dynamic.setdefault(input_name, {})[idx] = dim
        extra = {"strict": False, "prefer_deferred_runtime_asserts_over_guards": True}

    exported = torch.export.export(model, example_inputs, kwargs=example_kwargs or {},
                                   dynamic_shapes=torch_dynamic, **extra)

    symbol_map: dict[str, str] = {}
    if dynamic_dims:
        for fx in exported.graph_module.graph.nodes:
            if fx.op != "placeholder":
                continue
            val = fx.meta["val"]
            for sym, specs in dynamic_dims.items():
                for input_name, idx in specs:
                    if fx.name == input_name and not isinstance(val.shape[idx], int):
                        symbol_map[str(val.shape[idx])] = sym

    graph = Graph()
    node_map: dict[str, str] = {}
    _process_placeholders(exported, graph, node_map)
    _process_compute_nodes(exported, graph, node_map, symbol_map)
    _process_outputs(exported, graph, node_map)
    if dynamic_dims:
        graph.dynamic_dims = dynamic_dims
    return graph


def _concrete_shape(val) -> tuple[int, ...]:
    return tuple(d if isinstance(d, int) else int(d.node.hint) for d in val.shape)


def _process_placeholders(exported, graph: Graph, node_map: dict[str, str]) -> None:
    kinds, targets = {}, {}
    for spec in exported.graph_signature.input_specs:
        kinds[spec.arg.name] = spec.kind
        if spec.target is not None:
            targets[spec.arg.name] = spec.target
    for fx in exported.graph_module.graph.nodes:
        if fx.op != "placeholder":
            continue
        val = fx.meta["val"]
        info = graph.add_tensor(fx.name, _concrete_shape(val), str(val.dtype).replace("torch.", ""))
        node_map[fx.name] = fx.name
        kind = kinds[fx.name]
        if kind == InputKind.USER_INPUT:
            graph.inputs.append(fx.name)
        elif kind in (InputKind.PARAMETER, InputKind.BUFFER):
            graph.constants.append(fx.name)
            key = targets[fx.name]
            if key in exported.state_dict:
                info.buffer = exported.state_dict[key].numpy(force=True)
            elif hasattr(exported, "constants") and key in exported.constants:
                info.buffer = exported.constants[key].numpy(force=True)
            else:
                raise ValueError(f"Weight/buffer '{key}' not found in state_dict or constants")


def _process_compute_nodes(exported, graph: Graph, node_map: dict[str, str], symbol_map: dict[str, str]) -> None:
    for fx in exported.graph_module.graph.nodes:
        if fx.op != "call_function":
            continue
        val = fx.meta.get("val")
        if val is None:
            continue  # deferred runtime assertions
        if not isinstance(val, torch.Tensor) and not (isinstance(val, tuple) and val
                                                      and isinstance(val[0], torch.Tensor)):
            continue  # SymInt arithmetic, sym_size
        handler = ATEN_HANDLERS.get(fx.target)
        if handler is None:
            raise ValueError(f"Unsupported ATen op: {fx.target}")
        handler(fx, graph, node_map, symbol_map)


def _process_outputs(exported, graph: Graph, node_map: dict[str, str]) -> None:
    for fx in exported.graph_module.graph.nodes:
        if fx.op == "output":
            for arg in fx.args[0]:
                if hasattr(arg, "name"):
                    graph.outputs.append(node_map[arg.name])
