"""Write the plan fixtures: what the reference's host layer produces for each
BASELINE workload, as small JSON files (structure only, no tensor data).

    python tests/golden/make_plan_fixtures.py [workload ...]

Runs in the build container only (it imports the reference from
/root/reference, which does not exist on the GPU box).  For each workload it
exports the model defined in lets-build-a-runtime_amd/workloads.py with the
reference's exporter, runs its default pipeline and planner, and records:

* the optimised graph's nodes in plan order (id, op, inputs, output, attrs),
* which of them the reference's compiled executor dispatches, with the
  extras its registry packs and the scratch slot the planner assigns,
* every arena offset and the arena size.

tests/test_plan_fixtures.py checks this repository's host layer against
these files.  The torch / transformers versions used are recorded in each
file; the fixtures are only comparable under the same versions.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
REFERENCE = Path("/root/reference")


def _jsonable(v):
    if isinstance(v, (list, tuple)):
        return [_jsonable(x) for x in v]
    if isinstance(v, dict):
        return {k: _jsonable(x) for k, x in v.items()}
    if hasattr(v, "item"):
        return v.item()
    return v


def main(keys: list[str]) -> None:
    sys.path.insert(0, str(REPO / "lets-build-a-runtime_amd"))
    sys.path.insert(0, str(REFERENCE))           # `runtime` = the reference's package
    import torch
    import transformers
    import runtime
    assert str(REFERENCE) in runtime.__file__, runtime.__file__
    from runtime.exporter import export_model
    from runtime.ir import FOLD_ONLY_BASE
    from runtime.ops import OP_REGISTRY
    from runtime.passes import run_pipeline
    from runtime.planner import plan
    from workloads import WORKLOADS, CONFIG_ORDER

    for key in keys or CONFIG_ORDER:
        w = WORKLOADS[key]
        model = w.model(0)
        x = torch.from_numpy(w.input(0))
        g = export_model(model, (x,))
        run_pipeline(g)
        p = plan(g)
        external = set(g.inputs) | set(g.constants)
        nodes = []
        for node in p.order:
            op_def = OP_REGISTRY.get(node.op)
            alias = op_def is not None and op_def.is_alias(node)
            dispatched = not (alias and node.inputs[0] not in external) and node.op.value < FOLD_ONLY_BASE
            entry = {"id": node.id, "op": node.op.name, "inputs": list(node.inputs), "output": node.output,
                     "attrs": _jsonable(node.attrs), "dispatched": dispatched,
                     "out_shape": list(g.tensors[node.output].shape)}
            if dispatched and op_def is not None and op_def.extras is not None:
                entry["extras"] = [int(v) for v in op_def.extras(node, g)]
            if node.id in p.scratch:
                entry["scratch"] = list(p.scratch[node.id])
            nodes.append(entry)
        fixture = {
            "workload": key, "title": w.title,
            "generated_with": {"torch": torch.__version__, "transformers": transformers.__version__,
                               "reference": "kaselby/lets-build-a-runtime (read-only mount)"},
            "inputs": list(g.inputs), "outputs": list(g.outputs),
            "constants": {c: list(g.tensors[c].shape) for c in g.constants},
            "order": nodes,
            "offsets": {k: int(v) for k, v in p.offsets.items()},
            "arena_size": int(p.arena_size),
        }
        out = HERE / f"plan_{key}.json"
        out.write_text(json.dumps(fixture, indent=1) + "\n")
        print(f"{key}: {len(nodes)} nodes, arena {p.arena_size} → {out.name}")


if __name__ == "__main__":
    main(sys.argv[1:])
