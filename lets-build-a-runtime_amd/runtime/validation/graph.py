"""Graph-phase validators (POST_EXPORT, POST_OPTIMIZE, POST_RESOLVE,
POST_RESOLVE_OPTIMIZE) — the checks of runtime/validation/graph.py:16-210."""

from __future__ import annotations

from ..ir import FOLD_ONLY_BASE, Graph, OpType
from ..ops import OP_REGISTRY
from .core import Phase, Severity, ValidationResult, register_validator


def _check_structure(graph: Graph, who: str) -> list[ValidationResult]:
    out: list[ValidationResult] = []

    def add(sev, msg):
        out.append(ValidationResult(who, sev, msg))

    for node in graph.nodes.values():
        for t in node.inputs:
            if t not in graph.tensors:
                add(Severity.ERROR, f"Node {node.id} ({node.op.name}) references unknown input tensor '{t}'")
        if node.output not in graph.tensors:
            add(Severity.ERROR, f"Node {node.id} ({node.op.name}) output tensor '{node.output}' not in registry")
    for role, names in (("input", graph.inputs), ("constant", graph.constants), ("output", graph.outputs)):
        for n in names:
            if n not in graph.tensors:
                add(Severity.ERROR, f"Graph {role} '{n}' not in tensor registry")
    for n in graph.inputs:
        if graph.producer(n) is not None:
            add(Severity.ERROR, f"Graph input '{n}' has a producer node (should be external)")
    for n in graph.constants:
        if graph.producer(n) is not None:
            add(Severity.ERROR, f"Graph constant '{n}' has a producer node (should be external)")
    for n in graph.outputs:
        if graph.producer(n) is None:
            add(Severity.ERROR, f"Graph output '{n}' has no producer node")
    external = set(graph.inputs) | set(graph.constants)
    for node in graph.nodes.values():
        for t in node.inputs:
            if t not in external and graph.producer(t) is None:
                add(Severity.ERROR, f"Node {node.id} ({node.op.name}) consumes '{t}' which has no producer "
                                    f"and is not an input/constant")
    order = graph._toposort()
    if len(order) != len(graph.nodes):
        done = {n.id for n in order}
        add(Severity.ERROR, f"Graph has cycles involving nodes: {[i for i in graph.nodes if i not in done]}")
    read = set()
    for node in graph.nodes.values():
        read.update(node.inputs)
    outs = set(graph.outputs)
    for node in graph.nodes.values():
        if node.output not in read and node.output not in outs:
            add(Severity.WARNING, f"Dead node {node.id} ({node.op.name}): output '{node.output}' is never consumed")
    return out


@register_validator("structural_integrity", Phase.POST_EXPORT)
def validate_post_export(graph: Graph) -> list[ValidationResult]:
    return _check_structure(graph, "structural_integrity")


@register_validator("structural_integrity", Phase.POST_OPTIMIZE)
def validate_post_optimize(graph: Graph) -> list[ValidationResult]:
    return _check_structure(graph, "structural_integrity")


def _has_symbol(v, symbols: set[str]) -> bool:
    if isinstance(v, str) and v in symbols:
        return True
    if isinstance(v, (tuple, list)):
        return any(_has_symbol(x, symbols) for x in v)
    return False


@register_validator("resolution_completeness", Phase.POST_RESOLVE)
def validate_post_resolve(graph: Graph) -> list[ValidationResult]:
    who = "resolution_completeness"
    out = []
    for name, t in graph.tensors.items():
        for i, d in enumerate(t.shape):
            if not isinstance(d, int):
                out.append(ValidationResult(who, Severity.ERROR,
                                            f"Tensor '{name}' has non-integer dimension at index {i}: {d!r}"))
    symbols = set(graph.dynamic_dims.keys()) if graph.dynamic_dims else set()
    if symbols:
        for node in graph.nodes.values():
            for k, v in node.attrs.items():
                if _has_symbol(v, symbols):
                    out.append(ValidationResult(who, Severity.ERROR, f"Node {node.id} ({node.op.name}) attr '{k}' "
                                                                     f"contains unresolved symbol: {v!r}"))
    return out


@register_validator("execution_readiness", Phase.POST_RESOLVE_OPTIMIZE)
def validate_execution_readiness(graph: Graph) -> list[ValidationResult]:
    who = "execution_readiness"
    out = []
    for node in graph.nodes.values():
        if node.op.value >= FOLD_ONLY_BASE:
            out.append(ValidationResult(who, Severity.ERROR, f"Fold-only op {node.op.name} (node {node.id}) "
                                                             f"was not eliminated by constant folding"))
    for node in graph.nodes.values():
        if node.op not in OP_REGISTRY:
            out.append(ValidationResult(who, Severity.ERROR,
                                        f"Op {node.op.name} (node {node.id}) has no OP_REGISTRY entry"))
    for node in graph.nodes.values():
        op_def = OP_REGISTRY.get(node.op)
        if op_def is None or not op_def.is_alias(node):
            continue
        if len(node.inputs) != 1:
            out.append(ValidationResult(who, Severity.ERROR, f"Alias op {node.op.name} (node {node.id}) has "
                                                             f"{len(node.inputs)} inputs, expected 1"))
            continue
        seen = {node.output}
        cur = node.inputs[0]
        while cur is not None:
            if cur in seen:
                out.append(ValidationResult(who, Severity.ERROR,
                                            f"Circular alias chain at node {node.id} ({node.op.name})"))
                break
            seen.add(cur)
            prod = graph.producer(cur)
            if prod is None:
                break
            pd = OP_REGISTRY.get(prod.op)
            if pd is None or not pd.is_alias(prod):
                break
            cur = prod.inputs[0] if prod.inputs else None
        if node.op == OpType.SLICE:
            off = node.attrs.get("byte_offset", 0)
            if isinstance(off, int) and off < 0:
                out.append(ValidationResult(who, Severity.ERROR,
                                            f"SLICE node {node.id} has negative byte_offset: {off}"))
    return out
