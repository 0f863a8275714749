"""Validators on deliberately broken artifacts (the reference's strategy,
tests/test_validation.py): each case breaks one invariant of a small valid
graph or plan and checks that the matching phase reports it at the right
severity, and that the intact artifact passes.

Beyond the reference's checks, the arena model here also catches a graph
output overwritten before the host reads it back, an unrelated value placed
inside a live one, and a view outside its buffer; and it reports unaligned
ranges as information.
"""

import numpy as np
import pytest

from runtime.ir import Graph, OpType
from runtime.planner import ExecutionPlan, MemoryPlan, plan
from runtime.validation import Phase, Severity, ValidationError, run_validators


def _errors(results):
    return [r.message for r in results if r.severity == Severity.ERROR]


def _warnings(results):
    return [r.message for r in results if r.severity == Severity.WARNING]


def _chain(n=2, shape=(4, 64)):
    """x → RELU → t1 → RELU → ... → t_n (output)."""
    g = Graph()
    g.add_tensor("x", shape)
    g.inputs.append("x")
    prev = "x"
    for i in range(1, n + 1):
        g.add_tensor(f"t{i}", shape)
        g.add_node(OpType.RELU, [prev], f"t{i}")
        prev = f"t{i}"
    g.outputs.append(prev)
    return g


def _structure(g):
    return run_validators(Phase.POST_EXPORT, g, fail_on=None)


# ---------------------------------------------------------------- structure

def test_valid_graph_has_no_findings():
    g = _chain(3)
    assert _structure(g) == []
    assert run_validators(Phase.POST_OPTIMIZE, g, fail_on=None) == []


def test_unknown_tensors():
    g = _chain()
    g.add_tensor("o", (4, 64))
    g.add_tensor("ghost", (4, 64))
    g.add_node(OpType.ADD, ["t2", "ghost"], "o")
    del g.tensors["ghost"]          # Graph.add_node refuses unknown names; break the table afterwards
    g.outputs = ["o", "missing"]
    errs = _errors(_structure(g))
    assert any("reads 'ghost'" in m for m in errs)
    assert any("output 'missing'" in m for m in errs)


def test_external_tensor_written_by_a_node():
    g = _chain()
    g.add_node(OpType.NEG, ["t1"], "x")
    errs = _errors(_structure(g))
    assert any("'x' is a graph input" in m and "also writes it" in m for m in errs)


def test_two_writers():
    g = _chain()
    g.add_node(OpType.NEG, ["x"], "t1")
    assert any("has 2 writers" in m for m in _errors(_structure(g)))


def test_value_without_source():
    g = _chain()
    g.add_tensor("orphan", (4, 64))
    g.add_tensor("o", (4, 64))
    g.add_node(OpType.ADD, ["t2", "orphan"], "o")
    g.outputs = ["o"]
    assert any("'orphan', which has no source" in m for m in _errors(_structure(g)))
    g2 = _chain()
    g2.add_tensor("never", (4, 64))
    g2.outputs.append("never")
    assert any("output 'never' is never written" in m for m in _errors(_structure(g2)))


def test_cycle_is_reported_with_its_path():
    g = Graph()
    g.add_tensor("x", (4,))
    g.inputs.append("x")
    for t in ("a", "b", "c"):
        g.add_tensor(t, (4,))
    n1 = g.add_node(OpType.ADD, ["x", "c"], "a")
    n2 = g.add_node(OpType.RELU, ["a"], "b")
    n3 = g.add_node(OpType.RELU, ["b"], "c")
    g.outputs.append("c")
    errs = _errors(_structure(g))
    cyc = [m for m in errs if "dependence cycle" in m]
    assert cyc and all(str(n.id) in cyc[0] for n in (n1, n2, n3))


def test_dead_value_is_a_warning_only():
    g = _chain()
    g.add_tensor("unused", (4, 64))
    g.add_node(OpType.NEG, ["t1"], "unused")
    res = _structure(g)
    assert not _errors(res)
    assert any("is dead" in m and "'unused'" in m for m in _warnings(res))
    with pytest.raises(ValidationError):
        run_validators(Phase.POST_EXPORT, g, fail_on=Severity.WARNING)


# ---------------------------------------------------------------- resolution

def test_unresolved_dimensions_and_symbols():
    g = _chain()
    g.dynamic_dims = {"L": [("x", 0)]}
    g.tensors["t1"].shape = ("L", 64)
    g.add_tensor("r", (4, 64))
    g.add_node(OpType.RESHAPE, ["t2"], "r", {"shape": [("L", 2), {"k": "L"}]})
    g.outputs = ["r"]
    errs = _errors(run_validators(Phase.POST_RESOLVE, g, fail_on=None))
    assert any("'t1' has a non-integer dimension" in m for m in errs)
    assert any("attribute 'shape'" in m and "['L']" in m for m in errs)
    g.tensors["t1"].shape = (np.int64(4), 64)     # a numpy integer is concrete
    g.nodes[max(g.nodes)].attrs["shape"] = (4, 64)
    assert _errors(run_validators(Phase.POST_RESOLVE, g, fail_on=None)) == []


# ---------------------------------------------------------------- execution readiness

def _ready(g):
    return _errors(run_validators(Phase.POST_RESOLVE_OPTIMIZE, g, fail_on=None))


def test_fold_only_and_view_rules():
    from runtime.ir import FOLD_ONLY_BASE
    fold_only = [op for op in OpType if op.value >= FOLD_ONLY_BASE]
    g = _chain()
    g.add_tensor("c", (4, 64))
    g.add_node(fold_only[0], ["t2"], "c")
    g.add_tensor("v", (256,))
    g.add_node(OpType.RESHAPE, ["t1", "t2"], "v", {"shape": (256,)})
    g.add_tensor("s", (2, 64))
    g.add_node(OpType.SLICE, ["t1"], "s", {"dim": 0, "start": 0, "end": 2, "byte_offset": -4})
    errs = _ready(g)
    assert any(f"{fold_only[0].name}" in m and "fold-only" in m for m in errs)
    assert any("view with 2 inputs" in m for m in errs)
    assert any("negative byte_offset -4" in m for m in errs)
    assert _ready(_chain()) == []


def test_node_must_fit_the_opnode_record():
    g = Graph()
    ins = [f"i{k}" for k in range(12)]
    for name in ins:
        g.add_tensor(name, (4,))
        g.inputs.append(name)
    g.add_tensor("y", (4,))
    g.add_node(OpType.CAT, ins, "y", {"dim": 0})
    g.outputs.append("y")
    assert _ready(g) == []           # 12 inputs, no scratch slot
    g.add_tensor("q", (1, 2, 8, 4))
    g.add_tensor("att", (1, 2, 8, 4))
    g.add_node(OpType.ATTENTION, ["q"] * 12, "att", {})
    g.outputs.append("att")
    assert any("13 input slots" in m for m in _ready(g))   # 12 + the attention scratch slot
    deep = Graph()
    deep.add_tensor("x", (1,) * 25)
    deep.inputs.append("x")
    deep.add_tensor("y", (1,) * 25)
    deep.add_node(OpType.RELU, ["x"], "y")
    deep.outputs.append("y")
    assert any("25 dims" in m for m in _ready(deep))


# ---------------------------------------------------------------- memory plan

NB = 4 * 64 * 4   # bytes of one (4, 64) fp32 tensor


def _mplan(g, offsets, arena, scratch=None):
    return MemoryPlan(graph=g, order=list(g.nodes.values()), arena_size=arena, offsets=offsets,
                      scratch=scratch or {})


def _plan_findings(p):
    return run_validators(Phase.POST_PLAN, p, fail_on=None)


def test_planner_output_is_clean():
    g = _chain(4)
    assert _errors(_plan_findings(plan(g))) == []
    assert _warnings(_plan_findings(plan(g))) == []


def test_missing_offset_and_arena_bounds():
    g = _chain()
    assert any("'t2', which has no arena offset" in m for m in _errors(_plan_findings(_mplan(g, {"t1": 0}, NB))))
    errs = _errors(_plan_findings(_mplan(g, {"t1": 0, "t2": NB}, NB)))
    assert any("'t2'" in m and "runs past the end" in m for m in errs)
    res = _plan_findings(_mplan(g, {"t1": 0, "t2": NB}, 5 * NB))
    assert not _errors(res)
    assert any(f"{3 * NB} bytes are never used" in m for m in _warnings(res))


def test_co_live_values_may_not_share_bytes():
    g = _chain()
    # t1 is read at step 1 while t2 is written there: they must not overlap at all
    assert any("shares bytes" in m for m in _errors(_plan_findings(_mplan(g, {"t1": 0, "t2": 128}, 2 * NB))))
    # ... not even by containment: a later value inside a live one is just as wrong
    g3 = _chain(3)                    # t1, t2, t3 at steps 0-2; small = NEG(t2) at step 3
    g3.add_tensor("small", (8,))
    g3.add_node(OpType.NEG, ["t2"], "small")
    g3.outputs.append("small")
    errs = _errors(_plan_findings(_mplan(g3, {"t1": 0, "t2": NB, "t3": 0, "small": 2 * NB + 64}, 3 * NB)))
    assert errs == []
    errs = _errors(_plan_findings(_mplan(g3, {"t1": 0, "t2": NB, "t3": 0, "small": NB + 64}, 3 * NB)))
    assert any("'small'" in m and "'t2'" in m for m in errs)


def test_graph_output_must_survive_to_the_end():
    # t1 is an output read back after the last step: t3 may not reuse its bytes, although
    # no node reads t1 after step 1
    g = _chain(3)
    g.outputs = ["t1", "t3"]
    errs = _errors(_plan_findings(_mplan(g, {"t1": 0, "t2": NB, "t3": 0}, 2 * NB)))
    assert any("'t3'" in m and "'t1'" in m for m in errs)
    g.outputs = ["t3"]
    assert _errors(_plan_findings(_mplan(g, {"t1": 0, "t2": NB, "t3": 0}, 2 * NB))) == []


def test_views_and_in_place_hand_off():
    # a RESHAPE view names the same value as its buffer: same bytes, no conflict
    g = Graph()
    for name, shape in (("x", (4, 64)), ("y", (4, 64)), ("v", (256,)), ("z", (4, 64))):
        g.add_tensor(name, shape)
    g.inputs.append("x")
    g.add_node(OpType.RELU, ["x"], "y")
    g.add_node(OpType.RESHAPE, ["y"], "v", {"shape": (256,)})
    g.add_node(OpType.RELU, ["v"], "z")
    g.outputs.append("z")
    assert _errors(_plan_findings(_mplan(g, {"y": 0, "v": 0, "z": NB}, 2 * NB))) == []
    # a view outside its buffer is refused
    assert any("is not inside" in m for m in _errors(_plan_findings(_mplan(g, {"y": 0, "v": 64, "z": NB}, 2 * NB))))
    # z written in place over y (RELU reads each element before writing it) on y's last read
    assert _errors(_plan_findings(_mplan(g, {"y": 0, "v": 0, "z": 0}, NB))) == []
    # ... but not when y is still needed afterwards (returned too)
    g.outputs.append("y")
    assert any("shares bytes" in m for m in _errors(_plan_findings(_mplan(g, {"y": 0, "v": 0, "z": 0}, NB))))


def test_scratch_slots():
    g = Graph()
    for name in ("q", "k", "v"):
        g.add_tensor(name, (1, 2, 8, 4))
        g.inputs.append(name)
    g.add_tensor("o", (1, 2, 8, 4))
    att = g.add_node(OpType.ATTENTION, ["q", "k", "v"], "o", {})
    g.outputs.append("o")
    nb = 2 * 8 * 4 * 4
    ok = _mplan(g, {"o": 0}, nb + 512, scratch={att.id: (nb, 512)})
    assert _errors(_plan_findings(ok)) == []
    bad = _mplan(g, {"o": 0}, nb + 512, scratch={att.id: (nb - 64, 512)})
    assert any("scratch of node" in m and "shares bytes" in m for m in _errors(_plan_findings(bad)))
    stray = _mplan(g, {"o": 0}, nb + 512, scratch={999: (nb, 512)})
    assert any("node 999, which is not in the execution order" in m for m in _errors(_plan_findings(stray)))


def test_unaligned_ranges_are_information():
    g = _chain()
    res = _plan_findings(_mplan(g, {"t1": 4, "t2": NB + 16}, 2 * NB + 16))
    assert not _errors(res)
    info = [r.message for r in res if r.severity == Severity.INFO]
    assert info and "1 intermediate(s) start off a 16-byte boundary" in info[0]


# ---------------------------------------------------------------- whole pipeline

@pytest.mark.parametrize("key,seq", [("toy", None), ("gpt2", 64), ("qwen3_4b", 32)])
def test_real_pipeline_passes_every_phase(key, seq):
    from runtime.passes import run_pipeline
    from workloads import export_workload
    _, _, g = export_workload(key, seq_len=seq)
    run_pipeline(g, None)
    for phase in (Phase.POST_OPTIMIZE, Phase.POST_RESOLVE, Phase.POST_RESOLVE_OPTIMIZE):
        assert _errors(run_validators(phase, g, fail_on=None)) == []
    p = plan(g)
    assert _errors(run_validators(Phase.POST_PLAN, p, fail_on=None)) == []
    assert _errors(run_validators(Phase.PRE_EXECUTE, ExecutionPlan(g, p, "compiled", "hip"), fail_on=None)) == []
