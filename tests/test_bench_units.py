"""bench.py's algorithmic work per kernel step, on the CPU: the byte counts of
fused runs against closed forms of the workload's shapes (no device).

A fused run reads what comes from outside it and writes what leaves it.  A
view (RESHAPE, dim-0 SLICE) of a tensor made inside the run is not an
outside read: Qwen3's q head prologue reads its per-head RMSNorm input
through a RESHAPE of the run's own SLICE output.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from runtime.executor.hip_lib import open_library  # noqa: E402

ARENA, EXT = 1 << 40, 1 << 44


def _units(key: str, seq: int):
    import bench
    from runtime.executor.nodes import build_nodes
    from runtime.passes import run_pipeline
    from runtime.planner import plan
    from workloads import export_workload
    try:
        lib = open_library()
    except RuntimeError as e:
        pytest.skip(str(e))
    _, _, g = export_workload(key, seq_len=seq)
    run_pipeline(g, None)
    mem = plan(g)
    ext: dict[str, int] = {}

    def addr(name):
        if name in mem.offsets and name not in g.inputs and name not in g.constants:
            return ARENA + mem.offsets[name]
        if name not in ext:
            ext[name] = EXT + len(ext) * (1 << 32)
        return ext[name]

    arr, order = build_nodes(mem, addr, lambda off, size: ARENA + off)
    live = [(addr(n), int(np.prod(g.tensors[n].shape)) * 4) for n in g.outputs]
    runs = lib.fusion_windows(arr, len(order), live)
    names = [n.op.name for n in order]
    units = bench.step_units(names, order, mem.graph, [0.0] * len(order), runs)
    return units, runs, order, mem.graph


def test_qwen3_head_prologue_bytes_closed_form():
    S, Hq, Hkv, hd = 1024, 32, 8, 128
    units, runs, _, graph = _units("qwen3_4b", S)
    heads = [u for u in units if len(u["nodes"]) == 10 and u["nodes"][0].op.name == "SLICE"]
    assert len(heads) == 4, [(u["name"], len(u["nodes"])) for u in units]
    seen = []
    for u in heads:
        h = graph.tensors[u["nodes"][0].output].shape[-1] // hd   # q: 32 heads, k: 8
        seen.append(h)
        rows = S * h * hd * 4                 # the q (or k) columns read, the head layout written
        tables = 2 * S * hd * 4               # cos and sin, [S, hd] each
        weight = hd * 4                       # the per-head RMSNorm weight
        assert u["bytes"] == rows + tables + weight + rows, (u["name"], h, u["bytes"])
    # one q and one k run per layer
    assert sorted(seen) == [Hkv, Hkv, Hq, Hq]


def test_unfused_node_bytes_are_inputs_plus_output():
    units, runs, order, _ = _units("gpt2w", 512)
    covered = {i for f, c, _ in runs for i in range(f, f + c)}
    singles = [u for i, u in enumerate(units) if len(u["nodes"]) == 1]
    assert singles
    for u in singles:
        n = u["nodes"][0]
        if n.op.name in ("MATMUL", "MATMUL_ADD", "ATTENTION"):
            continue
        assert u["flops"] == 0.0
    # every node is in exactly one unit
    assert sum(len(u["nodes"]) for u in units) == len(order)
    assert len(covered) == sum(c for _, c, _ in runs)
