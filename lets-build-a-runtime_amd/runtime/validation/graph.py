"""Graph-phase validators: POST_EXPORT, POST_OPTIMIZE, POST_RESOLVE and
POST_RESOLVE_OPTIMIZE.

Phases, validator names and severities follow the reference's validation
contract (runtime/validation/graph.py); the checks are derived from what
this backend's compiled executor needs from a graph before it can turn it
into an OpNode stream:

* structure (after export and after optimisation) — the graph is indexed
  once into writers and readers per tensor, and the checks are facts about
  tensors: every name used is in the tensor table, every tensor has exactly
  one source (it is an input or a constant, or exactly one node writes it),
  everything read or returned has one, the writer→reader relation has no
  cycle (the executor runs one topological order), and a value nobody reads
  and the graph does not return is reported as dead (a warning);
* resolution — after binding dynamic dimensions every shape entry is a
  concrete integer and no attribute still names a dimension symbol;
* execution readiness — no fold-only op is left, every op has a definition,
  views (RESHAPE, dim-0 SLICE) take one input, sit on a chain of views that
  ends at a real buffer, and start inside it, and every node that reaches
  the device fits the OpNode record the library decodes (at most 24 output
  dims, each below 2^31, at most 12 inputs counting the scratch slot, at
  most 24 extras).
"""

from __future__ import annotations

from collections import defaultdict
from numbers import Integral

from ..ir import FOLD_ONLY_BASE, Graph, Node, OpType
from ..ops import OP_REGISTRY
from .core import Phase, Severity, ValidationResult, register_validator

_ABI_DIMS = 24       # OpNode.out_shape / extra entries
_ABI_INPUTS = 12     # OpNode.inputs, the scratch slot included
_INT32_MAX = 2**31 - 1


def _who(node: Node) -> str:
    return f"node {node.id} ({node.op.name})"


class _Report:
    def __init__(self, validator: str) -> None:
        self.validator = validator
        self.results: list[ValidationResult] = []

    def error(self, msg: str) -> None:
        self.results.append(ValidationResult(self.validator, Severity.ERROR, msg))

    def warning(self, msg: str) -> None:
        self.results.append(ValidationResult(self.validator, Severity.WARNING, msg))


def _writers_and_readers(graph: Graph) -> tuple[dict[str, list[Node]], dict[str, list[Node]]]:
    writers: dict[str, list[Node]] = defaultdict(list)
    readers: dict[str, list[Node]] = defaultdict(list)
    for node in graph.nodes.values():
        writers[node.output].append(node)
        for t in node.inputs:
            readers[t].append(node)
    return writers, readers


def _cycle(graph: Graph, writers: dict[str, list[Node]]) -> list[int] | None:
    """Node ids along one dependence cycle, or None (iterative depth-first colouring)."""
    def deps(nid: int) -> list[int]:
        return [w.id for t in graph.nodes[nid].inputs for w in writers.get(t, ())]

    state: dict[int, int] = {}            # absent: unseen, 1: on the current path, 2: finished
    for start in graph.nodes:
        if start in state:
            continue
        path, stack = [start], [iter(deps(start))]
        state[start] = 1
        while stack:
            nxt = next(stack[-1], None)
            if nxt is None:
                state[path.pop()] = 2
                stack.pop()
            elif state.get(nxt) == 1:
                return path[path.index(nxt):]
            elif nxt not in state:
                state[nxt] = 1
                path.append(nxt)
                stack.append(iter(deps(nxt)))
    return None


def _structure(graph: Graph, validator: str) -> list[ValidationResult]:
    rep = _Report(validator)
    table = graph.tensors
    writers, readers = _writers_and_readers(graph)
    external = {t: "input" for t in graph.inputs}
    external.update({t: "constant" for t in graph.constants})

    for role, names in (("input", graph.inputs), ("constant", graph.constants), ("output", graph.outputs)):
        for t in names:
            if t not in table:
                rep.error(f"graph {role} '{t}' is not in the tensor table")
    for t, nodes in readers.items():
        if t not in table:
            for n in nodes:
                rep.error(f"{_who(n)} reads '{t}', which is not in the tensor table")
    for t, nodes in writers.items():
        if t not in table:
            for n in nodes:
                rep.error(f"{_who(n)} writes '{t}', which is not in the tensor table")

    # one source per tensor
    for t, nodes in writers.items():
        if t in external:
            for n in nodes:
                rep.error(f"'{t}' is a graph {external[t]} (external) but {_who(n)} also writes it")
        elif len(nodes) > 1:
            rep.error(f"'{t}' has {len(nodes)} writers ({', '.join(_who(n) for n in nodes)}); a tensor has one")
    for t in graph.outputs:
        if t in table and t not in external and not writers.get(t):
            rep.error(f"graph output '{t}' is never written: no node produces it")
    for t, nodes in readers.items():
        if t in table and t not in external and not writers.get(t):
            rep.error(f"{_who(nodes[0])} reads '{t}', which has no source: no node produces it and it is "
                      f"neither an input nor a constant")

    cyc = _cycle(graph, writers)
    if cyc:
        rep.error("dependence cycle through nodes " + " -> ".join(str(i) for i in cyc + cyc[:1]))

    returned = set(graph.outputs)
    for node in graph.nodes.values():
        if not readers.get(node.output) and node.output not in returned:
            rep.warning(f"{_who(node)} is dead: nothing reads its output '{node.output}' and the graph does "
                        f"not return it")
    return rep.results


@register_validator("structural_integrity", Phase.POST_EXPORT)
def validate_post_export(graph: Graph) -> list[ValidationResult]:
    return _structure(graph, "structural_integrity")


@register_validator("structural_integrity", Phase.POST_OPTIMIZE)
def validate_post_optimize(graph: Graph) -> list[ValidationResult]:
    return _structure(graph, "structural_integrity")


def _symbols_named(value, symbols: set[str]) -> set[str]:
    """Dimension symbols a (possibly nested) attribute value still names."""
    if isinstance(value, str):
        return {value} & symbols
    if isinstance(value, dict):
        value = list(value.keys()) + list(value.values())
    if isinstance(value, (tuple, list)):
        found: set[str] = set()
        for v in value:
            found |= _symbols_named(v, symbols)
        return found
    return set()


def _concrete(d) -> bool:
    return isinstance(d, Integral) and not isinstance(d, bool)


@register_validator("resolution_completeness", Phase.POST_RESOLVE)
def validate_post_resolve(graph: Graph) -> list[ValidationResult]:
    rep = _Report("resolution_completeness")
    for name, t in graph.tensors.items():
        bad = [f"dim {i} = {d!r}" for i, d in enumerate(t.shape) if not _concrete(d)]
        if bad:
            rep.error(f"tensor '{name}' has a non-integer dimension after resolution ({', '.join(bad)})")
    symbols = set(graph.dynamic_dims or {})
    if symbols:
        for node in graph.nodes.values():
            for key, value in node.attrs.items():
                left = _symbols_named(value, symbols)
                if left:
                    rep.error(f"{_who(node)} attribute '{key}' = {value!r} still holds unresolved symbol(s) "
                              f"{sorted(left)}")
    return rep.results


def _view_chain_ok(graph: Graph, node: Node, rep: _Report) -> None:
    """A view's chain of views must end at a buffer, not loop back on itself."""
    visited = {node.output}
    cur = node.inputs[0]
    while True:
        if cur in visited:
            rep.error(f"{_who(node)} is a view on a chain of views that loops back to '{cur}'")
            return
        visited.add(cur)
        prod = graph.producer(cur)
        op_def = OP_REGISTRY.get(prod.op) if prod is not None else None
        if prod is None or op_def is None or not op_def.is_alias(prod) or not prod.inputs:
            return
        cur = prod.inputs[0]


def _abi_fit(graph: Graph, node: Node, rep: _Report) -> None:
    """The node fits the OpNode record (include/lbr_executor.h) the device library decodes."""
    op_def = OP_REGISTRY[node.op]
    shape = graph.tensors[node.output].shape if node.output in graph.tensors else ()
    if len(shape) > _ABI_DIMS:
        rep.error(f"{_who(node)} output has {len(shape)} dims; the node record holds {_ABI_DIMS}")
    if any(_concrete(d) and not 0 <= d <= _INT32_MAX for d in shape):
        rep.error(f"{_who(node)} output shape {tuple(shape)} has a dimension outside the record's int32 range")
    slots = len(node.inputs) + (1 if op_def.scratch is not None else 0)
    if slots > _ABI_INPUTS:
        rep.error(f"{_who(node)} needs {slots} input slots (scratch included); the node record holds "
                  f"{_ABI_INPUTS}")
    if op_def.extras is not None and all(_concrete(d) for d in shape):
        try:
            n_extras = len(op_def.extras(node, graph))
        except Exception as e:   # a packer that cannot read this node's attributes
            rep.error(f"{_who(node)}: its extras cannot be packed ({type(e).__name__}: {e})")
            return
        if n_extras > _ABI_DIMS:
            rep.error(f"{_who(node)} packs {n_extras} extras; the node record holds {_ABI_DIMS}")


@register_validator("execution_readiness", Phase.POST_RESOLVE_OPTIMIZE)
def validate_execution_readiness(graph: Graph) -> list[ValidationResult]:
    rep = _Report("execution_readiness")
    external = set(graph.inputs) | set(graph.constants)
    for node in graph.nodes.values():
        if node.op.value >= FOLD_ONLY_BASE:
            rep.error(f"{_who(node)} is a fold-only op left in the graph; constant folding must remove it "
                      f"before execution")
            continue
        op_def = OP_REGISTRY.get(node.op)
        if op_def is None:
            rep.error(f"{_who(node)} has no op definition in the registry")
            continue
        dispatched = True
        if op_def.is_alias(node):
            if len(node.inputs) != 1:
                rep.error(f"{_who(node)} is a view with {len(node.inputs)} inputs, expected 1")
                continue
            _view_chain_ok(graph, node, rep)
            if node.op == OpType.SLICE:
                off = node.attrs.get("byte_offset", 0)
                if _concrete(off) and off < 0:
                    rep.error(f"{_who(node)} views its input at negative byte_offset {off}, before the buffer")
            dispatched = node.inputs[0] in external   # a view of an external tensor is a device copy
        if dispatched:
            _abi_fit(graph, node, rep)
    return rep.results
