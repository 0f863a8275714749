"""Pattern fusion: linear-chain patterns and small DAG patterns.

Restates runtime/passes/fusion.py of the reference (58-683): the registry,
the matching rules (sole-consumer chains; DAGs anchored at a root with
commutative backtracking and exact internal consumer counts), the
priorities, and the registered patterns — these decide the fused ops and
node ids the executor sees, so they are kept rule for rule.

Chain patterns:   ADD+RELU → FUSED_BIAS_RELU; ADD+SILU/GELU+MUL and
                  SILU/GELU+MUL → GATED_ACT; MATMUL+ADD(1-D bias) →
                  MATMUL_ADD; MATMUL+SOFTMAX+MATMUL (± causal mask ADD) →
                  ATTENTION; RESHAPE+EXPAND+RESHAPE+ATTENTION → GQA
                  group_size.
DAG patterns:     tanh-GELU (8 nodes) → GELU; x/(1+exp(-x)) → SILU;
                  pow/sum/div/add/rsqrt/mul/mul → RMSNORM.
"""

from __future__ import annotations

from dataclasses import dataclass
from itertools import groupby
from typing import Callable

from ..ir import Graph, Node, OpType


# ================================================================ chain fusion

@dataclass
class FusionPattern:
    """A linear chain of ops fused into one op.

    Lower ``priority`` values are applied first (each level sweeps the whole
    graph before the next); within a level longer patterns are tried first.
    ``validator`` adds structural checks, ``build_attrs`` / ``build_inputs``
    shape the fused node.
    """
    name: str
    pattern: list[OpType]
    fused_op: OpType
    priority: int = 0
    validator: Callable[[list[Node], Graph], bool] | None = None
    build_attrs: Callable[[list[Node], Graph], dict] | None = None
    build_inputs: Callable[[list[Node], Graph, list[str]], list[str]] | None = None


FUSION_PATTERNS: list[FusionPattern] = []


def register_fusion(pattern: FusionPattern) -> None:
    FUSION_PATTERNS.append(pattern)


def fuse(graph: Graph, patterns: list[FusionPattern] | None = None) -> bool:
    """Apply chain patterns, one full topological sweep per priority level."""
    pats = patterns if patterns is not None else FUSION_PATTERNS
    if not pats:
        return False
    changed = False
    for _, level in groupby(sorted(pats, key=lambda p: p.priority), key=lambda p: p.priority):
        level = sorted(level, key=lambda p: len(p.pattern), reverse=True)
        claimed: set[int] = set()
        for node in list(graph):
            if node.id in claimed:
                continue
            for pat in level:
                chain = _try_match(node, pat, graph, claimed)
                if chain is not None:
                    _apply_fusion(chain, pat, graph)
                    claimed.update(n.id for n in chain)
                    changed = True
                    break
    return changed


def _try_match(start: Node, pat: FusionPattern, graph: Graph, claimed: set[int]) -> list[Node] | None:
    if start.op != pat.pattern[0]:
        return None
    chain = [start]
    cur = start
    for op in pat.pattern[1:]:
        users = graph.consumers(cur.output)
        if len(users) != 1:
            return None
        nxt = users[0]
        if nxt.id in claimed or nxt.op != op:
            return None
        chain.append(nxt)
        cur = nxt
    if pat.validator and not pat.validator(chain, graph):
        return None
    return chain


def _apply_fusion(chain: list[Node], pat: FusionPattern, graph: Graph) -> None:
    last = chain[-1]
    internal = {n.output for n in chain}
    ext: list[str] = []
    for n in chain:
        for t in n.inputs:
            if t not in internal and t not in ext:
                ext.append(t)
    attrs = pat.build_attrs(chain, graph) if pat.build_attrs else {}
    if pat.build_inputs:
        ext = pat.build_inputs(chain, graph, ext)
    # remove first: removing the last node pops the producer entry of its output
    for n in chain:
        graph.remove_node(n.id)
        if n.output != last.output:
            graph.remove_tensor(n.output)
    graph.add_node(pat.fused_op, ext, last.output, attrs)


# ---- registered chain patterns ----------------------------------------------

from .passes import _is_causal_mask  # noqa: E402


def _add_is_bias(add: Node, graph: Graph) -> bool:
    a = graph.tensors[add.inputs[0]].shape
    b = graph.tensors[add.inputs[1]].shape
    return len(b) == 1 and b[0] == a[-1]


register_fusion(FusionPattern(
    name="bias_relu", pattern=[OpType.ADD, OpType.RELU], fused_op=OpType.FUSED_BIAS_RELU, priority=0,
    validator=lambda chain, g: _add_is_bias(chain[0], g),
))


def _biased_gated_inputs(chain: list[Node], graph: Graph, ext: list[str]) -> list[str]:
    add, act, mul = chain
    up = [t for t in mul.inputs if t not in {act.output}][0]
    return [add.inputs[0], add.inputs[1], up]


for _act, _op in (("silu", OpType.SILU), ("gelu", OpType.GELU)):
    register_fusion(FusionPattern(
        name=f"bias_{_act}_mul", pattern=[OpType.ADD, _op, OpType.MUL], fused_op=OpType.GATED_ACT, priority=0,
        validator=lambda chain, g: _add_is_bias(chain[0], g),
        build_attrs=(lambda a: (lambda chain, g: {"act": a, "has_bias": True}))(_act),
        build_inputs=_biased_gated_inputs,
    ))


def _gated_inputs(chain: list[Node], graph: Graph, ext: list[str]) -> list[str]:
    act, mul = chain
    up = [t for t in mul.inputs if t not in {act.output}][0]
    return [act.inputs[0], up]


for _act, _op in (("silu", OpType.SILU), ("gelu", OpType.GELU)):
    register_fusion(FusionPattern(
        name=f"{_act}_mul", pattern=[_op, OpType.MUL], fused_op=OpType.GATED_ACT, priority=1,
        build_attrs=(lambda a: (lambda chain, g: {"act": a, "has_bias": False}))(_act),
        build_inputs=_gated_inputs,
    ))


def _validate_matmul_add(chain: list[Node], graph: Graph) -> bool:
    mm, add = chain
    for t in add.inputs:
        if t != mm.output:
            return len(graph.tensors[t].shape) == 1
    return False


register_fusion(FusionPattern(
    name="matmul_add", pattern=[OpType.MATMUL, OpType.ADD], fused_op=OpType.MATMUL_ADD, priority=1,
    validator=_validate_matmul_add, build_attrs=lambda chain, g: dict(chain[0].attrs),
))


def _softmax_on_last_axis(sm: Node, graph: Graph) -> bool:
    return sm.attrs.get("axis") == len(graph.tensors[sm.output].shape) - 1


register_fusion(FusionPattern(
    name="attention", pattern=[OpType.MATMUL, OpType.SOFTMAX, OpType.MATMUL], fused_op=OpType.ATTENTION,
    priority=0,
    validator=lambda chain, g: bool(chain[0].attrs.get("transpose_b")) and _softmax_on_last_axis(chain[1], g),
))


def _mask_operand(chain: list[Node]) -> str | None:
    qk, add = chain[0], chain[1]
    for t in add.inputs:
        if t != qk.output:
            return t
    return None


def _validate_causal_attention(chain: list[Node], graph: Graph) -> bool:
    if not chain[0].attrs.get("transpose_b") or not _softmax_on_last_axis(chain[2], graph):
        return False
    mask = _mask_operand(chain)
    if mask is None:
        return False
    info = graph.tensors[mask]
    return mask in graph.constants and info.buffer is not None and _is_causal_mask(info.buffer)


register_fusion(FusionPattern(
    name="causal_attention", pattern=[OpType.MATMUL, OpType.ADD, OpType.SOFTMAX, OpType.MATMUL],
    fused_op=OpType.ATTENTION, priority=0, validator=_validate_causal_attention,
    build_attrs=lambda chain, g: {"causal": True},
    build_inputs=lambda chain, g, ext: [t for t in ext if t != _mask_operand(chain)],
))


def _validate_gqa(chain: list[Node], graph: Graph) -> bool:
    r1, expand, r2, attn = chain
    shape = expand.attrs.get("shape")
    orig = graph.tensors[r1.inputs[0]].shape
    if shape is None or len(shape) != len(orig) + 1:
        return False
    group = shape[2]
    if not isinstance(group, int) or group <= 1:
        return False
    return r2.output in (attn.inputs[1], attn.inputs[2])


def _gqa_attrs(chain: list[Node], graph: Graph) -> dict:
    attrs = dict(chain[-1].attrs)
    attrs["group_size"] = chain[1].attrs["shape"][2]
    return attrs


def _gqa_inputs(chain: list[Node], graph: Graph, ext: list[str]) -> list[str]:
    inner = {n.output for n in chain[:-1]}
    src = chain[0].inputs[0]
    return [src if t in inner else t for t in chain[-1].inputs]


register_fusion(FusionPattern(
    name="gqa_attention", pattern=[OpType.RESHAPE, OpType.EXPAND, OpType.RESHAPE, OpType.ATTENTION],
    fused_op=OpType.ATTENTION, priority=0, validator=_validate_gqa, build_attrs=_gqa_attrs,
    build_inputs=_gqa_inputs,
))


# ================================================================ DAG fusion

@dataclass
class DAGNode:
    """Pattern node; inputs name other pattern nodes or external slots "x0", "x1", ..."""
    op: OpType
    inputs: list[str]
    scalar: float | None = None
    commutative: bool = False


@dataclass
class DAGFusionPattern:
    name: str
    nodes: dict[str, DAGNode]
    root: str
    fused_op: OpType
    external_inputs: list[str]
    priority: int = 0
    build_attrs: Callable[[dict[str, Node], Graph], dict] | None = None


DAG_FUSION_PATTERNS: list[DAGFusionPattern] = []


def register_dag_fusion(pattern: DAGFusionPattern) -> None:
    DAG_FUSION_PATTERNS.append(pattern)


_APPROX_TOL = 1e-4


def _match_dag_node(name: str, gnode: Node, pat: DAGFusionPattern, graph: Graph, bind: dict[str, Node],
                    ext: dict[str, str], claimed: set[int]) -> bool:
    if name in bind:
        return bind[name].id == gnode.id
    pn = pat.nodes[name]
    if gnode.op != pn.op or gnode.id in claimed:
        return False
    if pn.scalar is not None:
        s = gnode.attrs.get("scalar")
        if s is None or abs(s - pn.scalar) >= _APPROX_TOL:
            return False
    if len(pn.inputs) != len(gnode.inputs):
        return False
    orders = [pn.inputs]
    if pn.commutative and len(pn.inputs) == 2:
        orders.append([pn.inputs[1], pn.inputs[0]])
    for refs in orders:
        saved_b, saved_e = dict(bind), dict(ext)
        bind[name] = gnode
        ok = True
        for ref, tensor in zip(refs, gnode.inputs):
            if ref.startswith("x"):
                if ref in ext and ext[ref] != tensor:
                    ok = False
                    break
                ext[ref] = tensor
            else:
                prod = graph.producer(tensor)
                if prod is None or not _match_dag_node(ref, prod, pat, graph, bind, ext, claimed):
                    ok = False
                    break
        if ok:
            return True
        bind.clear()
        bind.update(saved_b)
        ext.clear()
        ext.update(saved_e)
    return False


def _try_match_dag(root: Node, pat: DAGFusionPattern, graph: Graph,
                   claimed: set[int]) -> tuple[dict[str, Node], dict[str, str]] | None:
    bind: dict[str, Node] = {}
    ext: dict[str, str] = {}
    if not _match_dag_node(pat.root, root, pat, graph, bind, ext, claimed):
        return None
    refs: dict[str, int] = {}
    for pn in pat.nodes.values():
        for r in pn.inputs:
            if not r.startswith("x"):
                refs[r] = refs.get(r, 0) + 1
    for r, expected in refs.items():
        if len(graph.consumers(bind[r].output)) != expected:
            return None
    return bind, ext


def _apply_dag_fusion(bind: dict[str, Node], ext: dict[str, str], pat: DAGFusionPattern, graph: Graph) -> None:
    out = bind[pat.root].output
    inputs = [ext[x] for x in pat.external_inputs]
    attrs = pat.build_attrs(bind, graph) if pat.build_attrs else {}
    for gn in bind.values():
        graph.remove_node(gn.id)
        if gn.output != out:
            graph.remove_tensor(gn.output)
    graph.add_node(pat.fused_op, inputs, out, attrs)


def fuse_dags(graph: Graph, patterns: list[DAGFusionPattern] | None = None) -> bool:
    """Apply DAG patterns anchored at their root op, one sweep per priority level."""
    pats = patterns if patterns is not None else DAG_FUSION_PATTERNS
    if not pats:
        return False
    changed = False
    for _, level in groupby(sorted(pats, key=lambda p: p.priority), key=lambda p: p.priority):
        level = sorted(level, key=lambda p: len(p.nodes), reverse=True)
        claimed: set[int] = set()
        for node in list(graph):
            if node.id in claimed:
                continue
            for pat in level:
                if node.op != pat.nodes[pat.root].op:
                    continue
                res = _try_match_dag(node, pat, graph, claimed)
                if res is not None:
                    bind, ext = res
                    _apply_dag_fusion(bind, ext, pat, graph)
                    claimed.update(n.id for n in bind.values())
                    changed = True
                    break
    return changed


# ---- registered DAG patterns -------------------------------------------------

# tanh-GELU as exported from GPT-2's gelu_new:
#   0.5·x · (1 + tanh(√(2/π)·(x + 0.044715·x³)))
register_dag_fusion(DAGFusionPattern(
    name="gelu_tanh",
    nodes={
        "pow": DAGNode(OpType.POW, ["x0"], scalar=3.0),
        "mul_c": DAGNode(OpType.MUL, ["pow"], scalar=0.044715),
        "add_x": DAGNode(OpType.ADD, ["x0", "mul_c"], commutative=True),
        "mul_s": DAGNode(OpType.MUL, ["add_x"], scalar=0.7978845608),
        "tanh": DAGNode(OpType.TANH, ["mul_s"]),
        "add_1": DAGNode(OpType.ADD, ["tanh"], scalar=1.0),
        "half_x": DAGNode(OpType.MUL, ["x0"], scalar=0.5),
        "out": DAGNode(OpType.MUL, ["add_1", "half_x"], commutative=True),
    },
    root="out", fused_op=OpType.GELU, external_inputs=["x0"],
))

# SiLU as x / (1 + exp(-x))
register_dag_fusion(DAGFusionPattern(
    name="silu",
    nodes={
        "neg": DAGNode(OpType.NEG, ["x0"]),
        "exp": DAGNode(OpType.EXP, ["neg"]),
        "denom": DAGNode(OpType.ADD, ["exp"], scalar=1.0),
        "out": DAGNode(OpType.DIV, ["x0", "denom"]),
    },
    root="out", fused_op=OpType.SILU, external_inputs=["x0"],
))

# RMSNorm after mean → SUM + DIV:  x · rsqrt(Σx²/N + eps) · w
register_dag_fusion(DAGFusionPattern(
    name="rmsnorm",
    nodes={
        "pow": DAGNode(OpType.POW, ["x0"], scalar=2.0),
        "sum": DAGNode(OpType.SUM, ["pow"]),
        "div": DAGNode(OpType.DIV, ["sum"]),
        "add_eps": DAGNode(OpType.ADD, ["div"]),
        "rsqrt": DAGNode(OpType.RSQRT, ["add_eps"]),
        "norm": DAGNode(OpType.MUL, ["x0", "rsqrt"], commutative=True),
        "out": DAGNode(OpType.MUL, ["norm", "x1"], commutative=True),
    },
    root="out", fused_op=OpType.RMSNORM, external_inputs=["x0", "x1"],
    build_attrs=lambda bind, g: {"eps": bind["add_eps"].attrs["scalar"]},
))
