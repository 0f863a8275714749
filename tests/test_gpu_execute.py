"""The reference's entry point by name: `execute(OpNode*, int)` bound exactly as
runtime/executor/common.py:157-159 binds it (argtypes [POINTER(COpNode),
c_int], restype None), called on node arrays the host layer built with
device addresses.

Each case runs the plan's one-kernel-per-node array through `execute` and
compares it with the same array replayed as a plan (same decoded kernels,
so bit-identical) and with the CPU oracle.  The GPT-2 body uses both
workspace users (split-K FFN2, key-range-split attention); the one-shot
workspace must then be reused, not re-allocated, by a smaller call.
"""

import ctypes

import numpy as np
import pytest

from conftest import normwise_rel

pytestmark = pytest.mark.gpu


def _reference_binding():
    from runtime.executor.common import COpNode
    from runtime.executor.hip_lib import library_path
    lib = ctypes.CDLL(str(library_path()))
    lib.execute.argtypes = [ctypes.POINTER(COpNode), ctypes.c_int]
    lib.execute.restype = None
    status = ctypes.CDLL(str(library_path())).execute   # same symbol, read as int
    status.argtypes = [ctypes.POINTER(COpNode), ctypes.c_int]
    status.restype = ctypes.c_int
    return lib.execute, status


def _workspace_bytes(lib) -> int:
    out = ctypes.c_size_t(0)
    lib.check(lib.lbr_execute_workspace_bytes(ctypes.byref(out)), "lbr_execute_workspace_bytes")
    return int(out.value)


def _via_execute(key, seq, execute_fn):
    from oracle.host_exec import OracleRun
    from runtime.executor.compiled import CompiledExecutor
    from runtime.planner import plan
    from workloads import export_workload
    from runtime.passes import run_pipeline
    _, x, graph = export_workload(key, seq_len=seq)
    run_pipeline(graph, None)   # the Session's optimisation passes (pre-transposed weights, merges)
    mp = plan(graph)
    ex = CompiledExecutor(fuse=False)
    ex.compile(mp)
    try:
        name_in, name_out = graph.inputs[0], graph.outputs[0]
        y_plan = ex.run({name_in: x})[name_out]
        ex._lib.lbr_memset(ctypes.c_void_p(ex.device_address(name_out)), 0, y_plan.nbytes)
        ex.upload_inputs({name_in: x})
        rc = execute_fn(ex._nodes, len(ex.dispatch_order))
        y = ex.download_outputs()[name_out]
    finally:
        ex.close()
    o = OracleRun(mp).run({name_in: x})[name_out]
    return rc, y, y_plan, o


def test_execute_by_reference_name(hip_lib):
    execute, execute_status = _reference_binding()
    rc, y, y_plan, o = _via_execute("gpt2", None, execute)
    assert rc is None
    np.testing.assert_array_equal(y, y_plan)
    e = normwise_rel(y, o)
    print(f"gpt2 body via execute: vs oracle rel {e:.2e}")
    assert e <= 1e-3
    held = _workspace_bytes(hip_lib)
    assert held > 0, "split-K / split attention must have used the one-shot workspace"
    # a smaller call reuses the block (grow-only, nothing re-allocated)
    rc, y, y_plan, o = _via_execute("toy", None, execute_status)
    assert rc == 0
    np.testing.assert_array_equal(y, y_plan)
    assert normwise_rel(y, o) <= 1e-3
    assert _workspace_bytes(hip_lib) == held


def test_execute_reports_unknown_op(hip_lib):
    from runtime.executor.common import COpNode
    from runtime.ir import OpType
    _, execute_status = _reference_binding()
    bad = (COpNode * 1)()
    bad[0].op = OpType.PERMUTE.value
    assert execute_status(bad, 1) == 2   # LBR_ERR_UNSUPPORTED where the reference aborts
    assert "unknown op" in hip_lib.last_error()
