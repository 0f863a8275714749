"""The host contract against the reference's own output.

tests/golden/plan_<workload>.json were written by the reference's exporter,
pipeline and planner (tests/golden/make_plan_fixtures.py) for the same
seeded models.  This repository's host layer must reproduce them exactly:
the plan order with node ids, ops, tensor names and attrs; which nodes are
dispatched; the extras each dispatched node carries; the scratch slots; and
every arena offset.  Identical offsets mean the device arena has the
reference's layout byte for byte.
"""

import json
from pathlib import Path

import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"
KEYS = ["toy", "gpt2w", "gpt2", "7b4k", "qwen3_4b", "gpt2_lm", "qwen3_4b_lm"]


def _jsonable(v):
    if isinstance(v, (list, tuple)):
        return [_jsonable(x) for x in v]
    if isinstance(v, dict):
        return {k: _jsonable(x) for k, x in v.items()}
    if hasattr(v, "item"):
        return v.item()
    return v


@pytest.mark.parametrize("key", KEYS)
def test_plan_matches_reference(key):
    import torch
    import transformers
    from runtime.exporter import export_model
    from runtime.ir import FOLD_ONLY_BASE
    from runtime.ops import OP_REGISTRY
    from runtime.passes import run_pipeline
    from runtime.planner import plan
    from workloads import WORKLOADS

    fx = json.loads((GOLDEN / f"plan_{key}.json").read_text())
    gen = fx["generated_with"]
    if gen["torch"] != torch.__version__ or gen["transformers"] != transformers.__version__:
        pytest.skip(f"fixture made with torch {gen['torch']} / transformers {gen['transformers']}")

    w = WORKLOADS[key]
    g = export_model(w.model(0), (torch.from_numpy(w.input(0)),))
    run_pipeline(g)
    p = plan(g)
    external = set(g.inputs) | set(g.constants)

    assert g.inputs == fx["inputs"] and g.outputs == fx["outputs"]
    assert {c: list(g.tensors[c].shape) for c in g.constants} == fx["constants"]
    assert len(p.order) == len(fx["order"])
    for node, want in zip(p.order, fx["order"]):
        op_def = OP_REGISTRY.get(node.op)
        alias = op_def is not None and op_def.is_alias(node)
        dispatched = not (alias and node.inputs[0] not in external) and node.op.value < FOLD_ONLY_BASE
        got = {"id": node.id, "op": node.op.name, "inputs": list(node.inputs), "output": node.output,
               "attrs": _jsonable(node.attrs), "dispatched": dispatched,
               "out_shape": list(g.tensors[node.output].shape)}
        if dispatched and op_def is not None and op_def.extras is not None:
            got["extras"] = [int(v) for v in op_def.extras(node, g)]
        if node.id in p.scratch:
            got["scratch"] = list(p.scratch[node.id])
        assert got == want, f"node {node.id}: {got} != {want}"
    assert {k: int(v) for k, v in p.offsets.items()} == fx["offsets"]
    assert p.arena_size == fx["arena_size"]
