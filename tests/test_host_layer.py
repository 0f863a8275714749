"""Host contract on the CPU: ABI layout, library exports, the reference's
known-answer tests, node streams per workload, planner invariants,
validation errors, serialisation and dynamic shapes."""

import ctypes
import os
import re
import struct
from pathlib import Path

import numpy as np
import pytest
import torch

from runtime.executor.common import COpNode
from runtime.ir import Graph, OpType
from runtime.ops import OP_REGISTRY, _float_bits
from runtime.planner import OrderStrategy, PlannerConfig, plan

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "lbr_executor.h"
LIB = ROOT / "lets-build-a-runtime_amd" / "csrc" / "liblbr_executor.so"


# ---------------------------------------------------------------- ABI

def test_opnode_layout_matches_reference_abi():
    """312-byte OpNode with the field offsets of csrc/runtime.h:60-69."""
    assert ctypes.sizeof(COpNode) == 312
    assert COpNode.inputs.offset == 8
    assert COpNode.output.offset == 104
    assert COpNode.out_shape.offset == 112
    assert COpNode.n_dims.offset == 208
    assert COpNode.elem_size.offset == 212
    assert COpNode.extra.offset == 216


def test_header_op_codes_match_ir():
    text = HEADER.read_text()
    codes = dict(re.findall(r"OP_([A-Z_]+)\s*=\s*(\d+)", text))
    assert len(codes) == 30          # csrc/runtime.h:11-55: 29 dispatchable ops + PERMUTE
    for name, val in codes.items():
        assert OpType[name].value == int(val)


def _declared_symbols():
    return re.findall(r"^\s*(?:const char\*|int)\s+(lbr_[a-z_0-9]+|execute)\s*\(", HEADER.read_text(), re.M)


def test_library_exports_every_declared_symbol():
    if not LIB.exists():
        pytest.skip("device library not built")
    lib = ctypes.CDLL(str(LIB))
    syms = _declared_symbols()
    assert len(syms) >= 20
    assert "execute" in syms   # the reference's own symbol, csrc/executor.c:458
    for s in syms:
        assert hasattr(lib, s), s
    # the reference's binding (runtime/executor/common.py:157-159) resolves unchanged
    lib.execute.argtypes = [ctypes.POINTER(COpNode), ctypes.c_int]
    lib.execute.restype = None
    lib.lbr_opnode_size.restype = ctypes.c_int
    assert lib.lbr_opnode_size() == 312
    lib.lbr_version.restype = ctypes.c_char_p
    assert b"gfx950" in lib.lbr_version()


def test_library_dispatch_table_matches_validator_set():
    if not LIB.exists():
        pytest.skip("device library not built")
    from runtime.validation.execution import _HIP_DISPATCH_OPS
    lib = ctypes.CDLL(str(LIB))
    for op in OpType:
        assert bool(lib.lbr_op_supported(op.value)) == (op in _HIP_DISPATCH_OPS), op


def test_library_reports_missing_device_instead_of_crashing():
    if not LIB.exists():
        pytest.skip("device library not built")
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present")
    lib = ctypes.CDLL(str(LIB))
    lib.lbr_last_error.restype = ctypes.c_char_p
    assert lib.lbr_init(0) != 0
    assert lib.lbr_last_error()


# ---------------------------------------------------------------- reference KATs (tests/test_ops.py, test_planner.py, test_backends.py)

def test_float_bits_roundtrip():
    for v in [0.0, 1.0, -1.0, 3.14159, 1e-6, float("inf")]:
        assert struct.unpack("f", struct.pack("i", _float_bits(v)))[0] == pytest.approx(v)


def test_evaluator_known_answers():
    a = np.array([1, 2, 3], dtype=np.float32)
    np.testing.assert_allclose(OP_REGISTRY[OpType.ADD].evaluator([a, np.array([4, 5, 6], np.float32)], {}), [5, 7, 9])
    np.testing.assert_allclose(OP_REGISTRY[OpType.ADD].evaluator([a], {"scalar": 10.0}), [11, 12, 13])
    np.testing.assert_allclose(OP_REGISTRY[OpType.RELU].evaluator([np.array([-1, 0, 1, -5, 3], np.float32)], {}),
                               [0, 0, 1, 0, 3])
    r = OP_REGISTRY[OpType.RESHAPE].evaluator([np.arange(12, dtype=np.float32)], {"shape": (3, 4)})
    assert r.shape == (3, 4)


def test_attention_scratch_size_known_answer():
    """[2,4,16,32] → 8 slices · 16² · 4 B (reference test_ops.py:161-170)."""
    s = OP_REGISTRY[OpType.ATTENTION].scratch([(2, 4, 16, 32)] * 3, (2, 4, 16, 32), {})
    assert s == 8 * 16 * 16 * 4
    # flash path: S > 256 → BR·BC per slice
    assert OP_REGISTRY[OpType.ATTENTION].scratch([(1, 2, 512, 64)] * 3, (1, 2, 512, 64), {}) == 2 * 128 * 256 * 4


def test_dim0_slice_alias_arena_known_answer():
    """dim-0 SLICE aliases its input at byte_offset; arena = 384 + 128 B (reference test_backends.py:300-319)."""
    chunk, idx = 4, 1
    g = Graph()
    g.add_tensor("x", (12, 8))
    g.inputs.append("x")
    g.add_tensor("relu_out", (12, 8))
    g.add_node(OpType.RELU, ["x"], "relu_out")
    g.add_tensor("sliced", (chunk, 8))
    off = idx * chunk * 8 * 4
    g.add_node(OpType.SLICE, ["relu_out"], "sliced", {"byte_offset": off, "dim": 0, "start": 4, "end": 8})
    g.add_tensor("out", (chunk, 8))
    g.add_node(OpType.ADD, ["sliced"], "out", {"scalar": 0.0})
    g.outputs.append("out")
    p = plan(g)
    assert p.offsets["sliced"] == p.offsets["relu_out"] + off
    assert p.arena_size == 12 * 8 * 4 + chunk * 8 * 4
    from oracle.host_exec import OracleRun
    x = np.random.default_rng(0).standard_normal((12, 8)).astype(np.float32)
    np.testing.assert_array_equal(OracleRun(p).run({"x": x})["out"], np.maximum(x, 0)[4:8])


# ---------------------------------------------------------------- node streams
# The dispatched node sequence of a custom block after the reference's default
# passes (runtime/passes/passes.py pipeline; merged QKV, three head chains).

BLOCK_STREAM = ["LAYERNORM", "MATMUL", "SLICE", "SLICE", "SLICE", "ADD", "ADD", "ADD", "TRANSPOSE", "TRANSPOSE",
                "TRANSPOSE", "ATTENTION", "TRANSPOSE", "MATMUL_ADD", "ADD", "LAYERNORM", "MATMUL_ADD", "GELU",
                "MATMUL_ADD", "ADD"]


def _stream(key, seq=None):
    from workloads import export_workload
    from runtime.executor.nodes import dispatch_order
    from runtime.passes import run_pipeline
    _, _, g = export_workload(key, seq_len=seq)
    run_pipeline(g)
    p = plan(g)
    return g, p, dispatch_order(p)


def test_custom_block_stream():
    g, p, order = _stream("toy")
    assert sorted(n.op.name for n in order) == sorted(BLOCK_STREAM)
    assert len(order) == 20
    attn = [n for n in order if n.op == OpType.ATTENTION][0]
    assert attn.attrs.get("causal") is True
    mm = [n for n in order if n.op == OpType.MATMUL][0]
    assert g.tensors[mm.output].shape == (1, 32, 192)          # merged QKV
    assert OP_REGISTRY[OpType.MATMUL].extras(mm, g) == [64, 1, 1, 0]
    slices = [n for n in order if n.op == OpType.SLICE]
    assert [OP_REGISTRY[OpType.SLICE].extras(n, g) for n in slices] == [[32, 192, 0, 64, 1], [32, 192, 64, 64, 1],
                                                                         [32, 192, 128, 64, 1]]
    assert OP_REGISTRY[OpType.ATTENTION].extras(attn, g) == [32, 16, 1, 0, 1]


def test_qwen3_stream_counts():
    g, p, order = _stream("qwen3_4b", seq=16)
    from collections import Counter
    c = Counter(n.op.name for n in order)
    assert c == Counter({"SLICE": 18, "RMSNORM": 9, "MATMUL": 8, "TRANSPOSE": 8, "MUL": 8, "ADD": 8, "NEG": 4,
                         "CAT": 4, "ATTENTION": 2, "GATED_ACT": 2})
    attn = [n for n in order if n.op == OpType.ATTENTION]
    assert all(OP_REGISTRY[OpType.ATTENTION].extras(n, g)[4] == 4 for n in attn)   # GQA 32/8
    muls = [n for n in order if n.op == OpType.MUL]
    assert all(OP_REGISTRY[OpType.MUL].extras(n, g)[0] == 2 for n in muls)         # RoPE broadcast mode


def test_gpt2_stream_counts():
    g, p, order = _stream("gpt2", seq=16)
    from collections import Counter
    assert Counter(n.op.name for n in order) == Counter({"MATMUL_ADD": 8, "TRANSPOSE": 8, "SLICE": 6, "ADD": 5,
                                                         "LAYERNORM": 5, "ATTENTION": 2, "GELU": 2})


# ---------------------------------------------------------------- planner invariants

@pytest.mark.parametrize("key,seq", [("toy", None), ("gpt2", 64), ("qwen3_4b", 32)])
@pytest.mark.parametrize("order", [OrderStrategy.MEMORY_AWARE_V1, OrderStrategy.NAIVE])
def test_plan_integrity(key, seq, order):
    from runtime.validation.plan import validate_memory_plan
    from runtime.validation.core import Severity
    from workloads import export_workload
    from runtime.passes import run_pipeline
    _, _, g = export_workload(key, seq_len=seq)
    run_pipeline(g)
    p = plan(g, PlannerConfig(order=order))
    errs = [r for r in validate_memory_plan(p) if r.severity == Severity.ERROR]
    assert not errs, errs
    assert p.arena_size <= p.stats.naive_bytes + sum(s for _, s in p.scratch.values())


def test_unsupported_order_strategy_raises():
    g = Graph()
    g.add_tensor("x", (2,))
    g.inputs.append("x")
    g.add_tensor("y", (2,))
    g.add_node(OpType.RELU, ["x"], "y")
    with pytest.raises(NotImplementedError):
        plan(g, PlannerConfig(order=OrderStrategy.MEMORY_AWARE_V3))


# ---------------------------------------------------------------- validation / errors

def test_compiled_dispatch_rejects_permute_and_fold_only():
    from runtime.planner import ExecutionPlan
    from runtime.validation import Phase, ValidationError, run_validators
    g = Graph()
    g.add_tensor("x", (2, 3, 4))
    g.inputs.append("x")
    g.add_tensor("y", (4, 2, 3))
    g.add_node(OpType.PERMUTE, ["x"], "y", {"axes": [2, 0, 1]})
    g.outputs.append("y")
    p = plan(g)
    with pytest.raises(ValidationError, match="no device kernel"):
        run_validators(Phase.PRE_EXECUTE, ExecutionPlan(g, p, "compiled", "hip"))


def test_device_extents_refuses_overread():
    from runtime.planner import ExecutionPlan
    from runtime.validation import Phase, ValidationError, run_validators
    g = Graph()
    g.add_tensor("q", (1, 4, 8, 16))
    g.add_tensor("k", (1, 1, 8, 16))   # too few KV heads for group_size 2
    g.add_tensor("v", (1, 1, 8, 16))
    g.inputs += ["q", "k", "v"]
    g.add_tensor("o", (1, 4, 8, 16))
    g.add_node(OpType.ATTENTION, ["q", "k", "v"], "o", {"group_size": 2})
    g.outputs.append("o")
    with pytest.raises(ValidationError, match="would read"):
        run_validators(Phase.PRE_EXECUTE, ExecutionPlan(g, plan(g), "compiled", "hip"))


def test_session_modes():
    from runtime.session import Session
    g = Graph()
    s = Session(g)
    with pytest.raises(RuntimeError, match="create"):
        s.run({})
    with pytest.raises(NotImplementedError):
        s.create(execution_mode="interpreted")
    with pytest.raises(ValueError):
        Session(Graph()).create(execution_mode="bogus")


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from runtime.executor import hip_lib
    monkeypatch.setattr(hip_lib, "_LIB", None)
    monkeypatch.setenv("LBR_EXECUTOR_LIB", str(tmp_path / "nope.so"))
    with pytest.raises(RuntimeError, match="not found"):
        hip_lib.load_library(0)


# ---------------------------------------------------------------- serialisation, dynamic shapes

def test_graph_save_load_roundtrip(tmp_path):
    from workloads import export_workload
    from runtime.passes import run_pipeline
    _, x, g = export_workload("toy")
    run_pipeline(g)
    g.save(tmp_path / "toy")
    g2 = Graph.load(tmp_path / "toy")
    import json
    norm = lambda d: json.loads(json.dumps(d, default=list))          # tuples come back as lists
    d1, d2 = norm(g.to_dict()), norm(g2.to_dict())
    strip = lambda d: [{k: v for k, v in n.items() if k != "id"} for n in d["nodes"]]   # ids are renumbered on load
    assert strip(d1) == strip(d2)
    assert {k: d1[k] for k in ("tensors", "inputs", "constants", "outputs")} == \
           {k: d2[k] for k in ("tensors", "inputs", "constants", "outputs")}
    for c in g.constants:
        np.testing.assert_array_equal(g2.tensors[c].buffer, g.tensors[c].buffer)
    from oracle.host_exec import OracleRun
    y1 = OracleRun(plan(g)).run({g.inputs[0]: x})[g.outputs[0]]
    y2 = OracleRun(plan(g2)).run({g2.inputs[0]: x})[g2.outputs[0]]
    np.testing.assert_array_equal(y1, y2)


def test_dynamic_seq_resolve():
    from runtime.exporter import export_model
    from runtime.ops import resolve_graph
    from runtime.passes import run_pipeline
    from workloads import CausalGeluBlock, init_weights
    m = init_weights(CausalGeluBlock(64, 4))
    g = export_model(m, (torch.randn(1, 16, 64),), dynamic_dims={"L": [("x", 1)]})
    run_pipeline(g)
    for L in (3, 40, 300):
        r = resolve_graph(g, {"L": L})
        assert r.tensors[r.outputs[0]].shape == (1, L, 64)
        p = plan(r)
        from oracle.host_exec import OracleRun
        x = np.random.default_rng(L).standard_normal((1, L, 64)).astype(np.float32)
        with torch.no_grad():
            ref = m(torch.from_numpy(x)).numpy()
        y = OracleRun(p).run({r.inputs[0]: x})[r.outputs[0]]
        np.testing.assert_allclose(y, ref, atol=1e-4)


@pytest.mark.parametrize("bh,seq,causal", [(12, 1024, 1), (12, 512, 1), (4, 32, 1), (32, 1024, 1), (5, 1000, 1),
                                           (3, 7, 1), (1, 1, 1), (2, 130, 0), (8, 300, 1), (6, 48, 0), (16, 17, 1),
                                           (24, 1024, 1), (96, 1024, 1)])
def test_attn_kq_grid_covers_every_block_once(bh, seq, causal):
    """The key-quartered attention grid (host mirror of the launch's assignment and the kernel's
    index arithmetic): every (head, 16-row block) exactly once.  When the grid fits on the 256
    CUs at once (4 workgroups a CU), workgroups w, w + 256, ... share CU w mod 256 (XCD w mod 8):
    the busiest CU carries at most the heaviest block more than the average load, and each XCD
    holds whole heads or alternate blocks of them.  Otherwise block levels run heaviest first."""
    import ctypes
    from runtime.executor.hip_lib import open_library
    lib = open_library()
    nq, C = (seq + 15) // 16, 256
    n = bh * nq
    heads, blocks = (ctypes.c_int * n)(), (ctypes.c_int * n)()
    assert lib.lbr_attn_kq_grid(bh, seq, causal, C, heads, blocks, n) == n
    pairs = sorted(zip(heads[:n], blocks[:n]))
    assert pairs == [(h, b) for h in range(bh) for b in range(nq)]
    nt = (seq + 31) // 32

    def tiles(b):
        return min(nt, min(seq - 1, 16 * b + 15) // 32 + 1) if causal else nt

    P = next((p for p in (1, 2, 4, 8) if p <= nq and nq % p == 0 and bh * p % 8 == 0), None)
    if n > 4 * C or P is None and n > 4 * C:
        # the kernel's own order: block levels from the last (heaviest under causal masking) down
        assert [blocks[w] for w in range(n)] == sorted(blocks[:n], reverse=True)
        return
    load = [0] * C
    for w in range(n):
        load[w % C] += tiles(blocks[w])
    heaviest = max(tiles(b) for b in range(nq))
    assert max(load) <= sum(load) / min(n, C) + heaviest, (max(load), sum(load) / min(n, C))
    if P is not None:
        for x in range(8):
            mine = {(heads[w], blocks[w] % P) for w in range(x, n, 8)}
            assert len(mine) == bh * P // 8
