"""POST_PLAN validator: the device arena a memory plan describes.

On the GPU a plan becomes one hipMalloc of ``arena_size`` bytes; every
intermediate tensor and every scratch slot is a byte range of it.  The
phase, validator name and severities follow the reference's validation
contract (runtime/validation/plan.py); the model and the checks are this
backend's.

The check reasons about *values* rather than tensor names.  A value is what
one node computes into memory; a view (RESHAPE, dim-0 SLICE) of an arena
tensor names the same value at an offset inside it, so reading a view keeps
the viewed value alive.  A value is live from the step that writes it to
the last step that reads it, and a graph output stays live past the end
of the order, because the host copies it back only after the last kernel.
What the executor relies on:

* every intermediate the order writes has an offset, every byte range lies
  inside the arena (an arena longer than the highest range end only wastes
  memory: a warning), a view lies inside the buffer it views, and every
  scratch slot belongs to a scheduled node;
* two values live at the same step never share a byte — with one
  exception, the in-place hand-off: an element-wise node whose output takes
  exactly the bytes of its first input's buffer, when that input's value is
  read for the last time by this very node (each lane reads its element
  before writing it back);
* information only: ranges that do not start on a 16-byte boundary — every
  kernel picks its 16-byte vector path per node from the addresses, so such
  a node runs a scalar variant.
"""

from __future__ import annotations

import numpy as np

from ..ir import Graph, Node
from ..ops import OP_REGISTRY
from ..planner import MemoryPlan
from .core import Phase, Severity, ValidationResult, register_validator

_VECTOR_ALIGN = 16


def _nbytes(graph: Graph, name: str) -> int:
    t = graph.tensors[name]
    return int(np.prod(t.shape)) * np.dtype(t.dtype).itemsize


class _Value:
    """One computed value: its bytes [lo, hi), the steps it is live, the tensors naming it."""

    def __init__(self, label: str, lo: int, hi: int, born: int) -> None:
        self.label, self.lo, self.hi, self.born, self.dies = label, lo, hi, born, born
        self.names = [label]

    def shares_bytes(self, other: "_Value") -> bool:
        return self.lo < other.hi and other.lo < self.hi

    def live_with(self, other: "_Value") -> bool:
        return self.born <= other.dies and other.born <= self.dies


@register_validator("memory_plan_integrity", Phase.POST_PLAN)
def validate_memory_plan(plan: MemoryPlan) -> list[ValidationResult]:
    who = "memory_plan_integrity"
    results: list[ValidationResult] = []

    def report(sev: Severity, msg: str) -> None:
        results.append(ValidationResult(who, sev, msg))

    graph = plan.graph
    external = set(graph.inputs) | set(graph.constants)
    read_back = len(plan.order)   # the host copies outputs back after the last step
    step_of_node = {node.id: s for s, node in enumerate(plan.order)}

    # ---- values, in execution order
    value_of: dict[str, _Value] = {}          # tensor name -> the value it names
    values: list[_Value] = []
    handoff: dict[int, tuple[_Value, int]] = {}   # id(new value) -> (value it overwrites in place, step)
    misaligned = 0
    for s, node in enumerate(plan.order):
        out = node.output
        if out in external or out not in graph.tensors:
            continue
        if out not in plan.offsets:
            report(Severity.ERROR, f"node {node.id} ({node.op.name}) writes '{out}', which has no arena offset")
            continue
        lo = plan.offsets[out]
        hi = lo + _nbytes(graph, out)
        if lo % _VECTOR_ALIGN:
            misaligned += 1
        op_def = OP_REGISTRY.get(node.op)
        src = value_of.get(node.inputs[0]) if node.inputs else None
        if op_def is not None and src is not None and op_def.is_alias(node):
            if not (src.lo <= lo and hi <= src.hi):
                report(Severity.ERROR, f"view '{out}' [{lo}:{hi}) of node {node.id} ({node.op.name}) is not inside "
                                       f"the buffer of '{src.label}' [{src.lo}:{src.hi}) it views")
            src.names.append(out)
            value_of[out] = src
            continue
        v = _Value(out, lo, hi, s)
        if op_def is not None and op_def.inplace and src is not None and (lo, hi) == (src.lo, src.hi):
            handoff[id(v)] = (src, s)   # same bytes as the input's buffer: an element-wise overwrite
        value_of[out] = v
        values.append(v)

    # ---- lifetimes: the last read of any name of a value; outputs to the end
    for s, node in enumerate(plan.order):
        for t in node.inputs:
            v = value_of.get(t)
            if v is not None:
                v.dies = max(v.dies, s)
    for t in graph.outputs:
        v = value_of.get(t)
        if v is not None:
            v.dies = read_back

    # ---- scratch slots: live at their node's step only
    for nid, (off, size) in plan.scratch.items():
        if nid not in step_of_node:
            report(Severity.ERROR, f"scratch slot [{off}:{off + size}) is assigned to node {nid}, which is not in "
                                   f"the execution order")
            continue
        if size:
            values.append(_Value(f"scratch of node {nid}", off, off + size, step_of_node[nid]))

    # ---- the arena holds every range
    top = max((v.hi for v in values), default=0)
    for v in values:
        if v.hi > plan.arena_size:
            report(Severity.ERROR, f"'{v.label}' [{v.lo}:{v.hi}) runs past the end of the {plan.arena_size}-byte "
                                   f"arena")
    if plan.arena_size > top:
        report(Severity.WARNING, f"arena of {plan.arena_size} bytes is longer than its highest range end {top}: "
                                 f"{plan.arena_size - top} bytes are never used")

    # ---- no two live values share a byte, except the in-place hand-off
    def clash_allowed(a: _Value, b: _Value) -> bool:
        for new, old in ((a, b), (b, a)):
            h = handoff.get(id(new))
            if h is not None and h[0] is old and old.dies == h[1] == new.born:
                return True
        return False

    by_birth = sorted((v for v in values if v.hi > v.lo), key=lambda v: (v.born, v.lo))
    live: list[_Value] = []
    for v in by_birth:
        live = [u for u in live if u.dies >= v.born]
        for u in live:
            if u.shares_bytes(v) and u.live_with(v) and not clash_allowed(u, v):
                report(Severity.ERROR,
                       f"'{v.label}' [{v.lo}:{v.hi}) (live at steps {v.born}-{v.dies}) shares bytes with "
                       f"'{u.label}' [{u.lo}:{u.hi}) (live at steps {u.born}-{u.dies}), which still holds a "
                       f"needed value")
        live.append(v)

    if misaligned:
        report(Severity.INFO, f"{misaligned} intermediate(s) start off a {_VECTOR_ALIGN}-byte boundary; the device "
                              f"kernels for them take scalar paths")
    return results
