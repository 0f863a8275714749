"""PRE_EXECUTE validators (runtime/validation/execution.py:16-136).

``compiled_dispatch`` checks that every op the compiled executor will
dispatch has a device kernel.  The set below is the device library's
dispatch table (include/lbr_executor.h, lbr_op_supported); it equals the
reference's ``_C_DISPATCH_OPS`` (execution.py:16-34) — PERMUTE is the one
registered op without a kernel on either side.

``device_extents`` is specific to this backend: it refuses a plan in which
a kernel would read past the end of an input (the reference's CPU code has
no such guard; on the GPU an over-read is a memory fault).
"""

from __future__ import annotations

from ..ir import FOLD_ONLY_BASE, OpType
from ..ops import OP_REGISTRY
from ..planner import ExecutionPlan
from .core import Phase, Severity, ValidationResult, register_validator

_HIP_DISPATCH_OPS: frozenset[OpType] = frozenset({
    OpType.RELU, OpType.EXP, OpType.TANH, OpType.POW, OpType.GELU,
    OpType.RSQRT, OpType.SILU, OpType.NEG, OpType.COS, OpType.SIN,
    OpType.ADD, OpType.SUB, OpType.MUL, OpType.DIV,
    OpType.MAX, OpType.SUM, OpType.SOFTMAX,
    OpType.MATMUL,
    OpType.RESHAPE, OpType.TRANSPOSE, OpType.SLICE, OpType.EMBEDDING, OpType.CAT,
    OpType.LAYERNORM, OpType.RMSNORM,
    OpType.MATMUL_ADD, OpType.FUSED_BIAS_RELU, OpType.ATTENTION, OpType.GATED_ACT,
})

# name kept for callers written against the reference
_C_DISPATCH_OPS = _HIP_DISPATCH_OPS


def _ops_needing_dispatch(plan: ExecutionPlan) -> list[tuple[int, OpType]]:
    graph = plan.graph
    external = set(graph.inputs) | set(graph.constants)
    out = []
    for node in plan.memory.order:
        op_def = OP_REGISTRY.get(node.op)
        if op_def is not None and op_def.is_alias(node) and node.inputs[0] not in external:
            continue
        out.append((node.id, node.op))
    return out


@register_validator("compiled_dispatch", Phase.PRE_EXECUTE)
def validate_compiled_dispatch(plan: ExecutionPlan) -> list[ValidationResult]:
    if plan.executor_type != "compiled":
        return []
    who = "compiled_dispatch"
    out = []
    for nid, op in _ops_needing_dispatch(plan):
        if op.value >= FOLD_ONLY_BASE:
            out.append(ValidationResult(who, Severity.ERROR, f"Fold-only op {op.name} (node {nid}) cannot be compiled"))
        elif op not in _HIP_DISPATCH_OPS:
            out.append(ValidationResult(who, Severity.ERROR, f"Op {op.name} (node {nid}) has no device kernel"))
    return out


@register_validator("device_extents", Phase.PRE_EXECUTE)
def validate_device_extents(plan: ExecutionPlan) -> list[ValidationResult]:
    if plan.executor_type != "compiled":
        return []
    from ..executor.nodes import dispatch_order, required_elements
    who = "device_extents"
    graph = plan.graph
    out = []
    try:
        order = dispatch_order(plan.memory)
    except RuntimeError:
        return []  # fold-only ops are reported by compiled_dispatch
    for node in order:
        if node.op not in _HIP_DISPATCH_OPS:
            continue
        try:
            needs = required_elements(node, graph)
        except ValueError as e:
            out.append(ValidationResult(who, Severity.ERROR, str(e)))
            continue
        for name, need in needs:
            have = 1
            for d in graph.tensors[name].shape:
                have *= d
            if need > have:
                out.append(ValidationResult(who, Severity.ERROR, f"node {node.id} ({node.op.name}) would read "
                                                                 f"{need} elements of '{name}', which holds {have}"))
    return out
