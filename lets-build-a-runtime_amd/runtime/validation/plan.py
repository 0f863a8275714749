"""POST_PLAN validator: arena integrity (runtime/validation/plan.py:20-138).

Every intermediate has an offset, the arena covers every allocation, scratch
entries name scheduled nodes, and no two co-live allocations partially
overlap (containment is allowed: aliases live inside their root).  On the
GPU the same invariant is what keeps concurrently-live device buffers from
corrupting each other.
"""

from __future__ import annotations

import numpy as np

from ..ir import Graph
from ..planner import MemoryPlan
from .core import Phase, Severity, ValidationResult, register_validator


def _tensor_bytes(graph: Graph, name: str) -> int:
    t = graph.tensors[name]
    return int(np.prod(t.shape)) * np.dtype(t.dtype).itemsize


@register_validator("memory_plan_integrity", Phase.POST_PLAN)
def validate_memory_plan(plan: MemoryPlan) -> list[ValidationResult]:
    who = "memory_plan_integrity"
    out: list[ValidationResult] = []
    graph = plan.graph
    external = set(graph.inputs) | set(graph.constants)

    for node in plan.order:
        if node.output not in external and node.output not in plan.offsets:
            out.append(ValidationResult(who, Severity.ERROR, f"Intermediate tensor '{node.output}' (node {node.id}, "
                                                             f"{node.op.name}) has no arena offset"))

    extent = 0
    for name, off in plan.offsets.items():
        if name in external or name not in graph.tensors:
            continue
        extent = max(extent, off + _tensor_bytes(graph, name))
    for _, (off, size) in plan.scratch.items():
        extent = max(extent, off + size)
    if plan.arena_size < extent:
        out.append(ValidationResult(who, Severity.ERROR,
                                    f"Arena undersized: {plan.arena_size} bytes < required {extent} bytes"))
    elif plan.arena_size > extent:
        out.append(ValidationResult(who, Severity.WARNING,
                                    f"Arena oversized: {plan.arena_size} bytes > minimum {extent} bytes "
                                    f"({plan.arena_size - extent} bytes wasted)"))

    ids = {n.id for n in plan.order}
    for nid in plan.scratch:
        if nid not in ids:
            out.append(ValidationResult(who, Severity.ERROR, f"Scratch allocation for node {nid} references a "
                                                             f"node not in the execution order"))

    step_of = {node.output: s for s, node in enumerate(plan.order)}
    last_use: dict[str, int] = {}
    for s, node in enumerate(plan.order):
        for t in node.inputs:
            if t not in external:
                last_use[t] = s
    allocs = []
    for name, off in plan.offsets.items():
        if name in external or name not in graph.tensors:
            continue
        size = _tensor_bytes(graph, name)
        born = step_of.get(name)
        if born is None or size == 0:
            continue
        allocs.append((name, off, size, born, last_use.get(name, born)))
    step_by_id = {node.id: i for i, node in enumerate(plan.order)}
    for nid, (off, size) in plan.scratch.items():
        if size and nid in step_by_id:
            s = step_by_id[nid]
            allocs.append((f"__scratch_{nid}", off, size, s, s))

    for i in range(len(allocs)):
        ni, oi, si, bi, di = allocs[i]
        ei = oi + si
        for j in range(i + 1, len(allocs)):
            nj, oj, sj, bj, dj = allocs[j]
            if bi > dj or bj > di:
                continue
            ej = oj + sj
            if ei <= oj or ej <= oi:
                continue
            if (oi <= oj and ei >= ej) or (oj <= oi and ej >= ei):
                continue
            out.append(ValidationResult(who, Severity.ERROR,
                                        f"Partial overlap between co-live tensors: '{ni}' [{oi}:{ei}) "
                                        f"(steps {bi}-{di}) and '{nj}' [{oj}:{ej}) (steps {bj}-{dj})"))
    return out
