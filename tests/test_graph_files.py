"""On-disk graph format ({stem}.json + {stem}.weights, runtime/ir.py:363-447).

tests/golden/graph_tiny.* was written by the reference's own Graph.save
(tests/golden/make_graph_fixture.py).  This repository's Graph.load must read
it back to the same graph its own exporter builds, and its Graph.save must
write the same files, so graphs move between the two in both directions.
"""

from __future__ import annotations

import importlib.util
import json
from pathlib import Path

import numpy as np
import torch

from runtime.exporter import export_model
from runtime.ir import Graph

GOLDEN = Path(__file__).resolve().parent / "golden"


def _fixture_module():
    spec = importlib.util.spec_from_file_location("make_graph_fixture", GOLDEN / "make_graph_fixture.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _our_export():
    fx = _fixture_module()
    return export_model(fx.tiny_model(), (torch.from_numpy(fx.tiny_input()),))


def _normalised(d):
    return json.loads(json.dumps(d))


def _strip_ids(d):
    d = _normalised(d)
    for n in d["nodes"]:
        n.pop("id", None)
    return d


def test_reference_file_loads_to_our_export(tmp_path):
    ref = Graph.load(GOLDEN / "graph_tiny")
    ours = _our_export()
    # load renumbers node ids in file order (ir.py from_dict → add_node), so the
    # direct export matches up to ids and a save/load round trip matches exactly
    assert _strip_ids(ref.to_dict()) == _strip_ids(ours.to_dict())
    ours.save(tmp_path / "g")
    assert _normalised(ref.to_dict()) == _normalised(Graph.load(tmp_path / "g").to_dict())
    for name in ours.constants:
        a, b = ref.tensors[name].buffer, ours.tensors[name].buffer
        assert a is not None and a.dtype == b.dtype and a.shape == b.shape
        assert a.tobytes() == np.ascontiguousarray(b).tobytes(), name


def test_our_save_writes_the_reference_files(tmp_path):
    _our_export().save(tmp_path / "g")
    ours = json.loads((tmp_path / "g.json").read_text())
    ref = json.loads((GOLDEN / "graph_tiny.json").read_text())
    assert ours == ref
    assert (tmp_path / "g.weights").read_bytes() == (GOLDEN / "graph_tiny.weights").read_bytes()


def test_loaded_graph_plans_like_the_export():
    from runtime.executor.nodes import dispatch_order
    from runtime.ops import OP_REGISTRY
    from runtime.passes import run_pipeline
    from runtime.planner import plan
    streams = []
    for g in (Graph.load(GOLDEN / "graph_tiny"), _our_export()):
        run_pipeline(g)
        p = plan(g)
        streams.append(([(n.op.name, tuple(n.inputs), n.output,
                          tuple(OP_REGISTRY[n.op].extras(n, g)) if OP_REGISTRY[n.op].extras else ())
                         for n in dispatch_order(p)], dict(p.offsets), p.arena_size))
    assert streams[0] == streams[1]


def test_missing_weights_file_leaves_constants_empty(tmp_path):
    (tmp_path / "g.json").write_text((GOLDEN / "graph_tiny.json").read_text())
    g = Graph.load(tmp_path / "g")
    assert g.constants and all(g.tensors[c].buffer is None for c in g.constants)
