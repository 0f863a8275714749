"""lbr_execute_noalloc — the entry point that allocates nothing — against
lbr_execute on the same node arrays (same decoded kernels, so the outputs
must be bit-identical), on two calls in a row, the second smaller.

The GPT-2 body's one-kernel-per-node array uses the workspace twice over,
both forced here: every GEMM runs in 2 K ranges whose partial sums go to
the workspace, and the attention takes the key-range split with shares of
4 key tiles, so most query blocks are cut into segments whose partials go
to the workspace.  The second call runs the same body at
S=512.  Every benchmark workload's one-kernel-per-node array fits the scratch
array and runs through it.  A node array whose workspace need exceeds the
scratch array is rejected before any launch.
"""

import ctypes

import numpy as np
import pytest

from conftest import normwise_rel

pytestmark = pytest.mark.gpu


def _run_both(lib, key, seq):
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
        kinds = ex.step_params()
        att = [s for s in kinds if s["kernel"].startswith("attn_fwd_mfma16")]
        gem = [s for s in kinds if s["kernel"].startswith("gemm_")]
        assert att and all(s["split_wg"] > 0 for s in att), att
        assert gem and all(s["ksplit"] == 2 and s["dma_tile"] >= 0 for s in gem), gem
        name_in, name_out = graph.inputs[0], graph.outputs[0]
        n = len(ex.dispatch_order)
        out_ptr = ctypes.c_void_p(ex.device_address(name_out))
        ex.upload_inputs({name_in: x})
        lib.check(lib.lbr_execute(ex._nodes, n), "lbr_execute")
        y_exec = ex.download_outputs()[name_out]
        lib.check(lib.lbr_memset(out_ptr, 0, y_exec.nbytes), "lbr_memset")
        ex.upload_inputs({name_in: x})
        lib.check(lib.lbr_execute_noalloc(ex._nodes, n), "lbr_execute_noalloc")
        y = ex.download_outputs()[name_out]
    finally:
        ex.close()
    o = OracleRun(mp).run({name_in: x})[name_out]
    return y, y_exec, o


def test_noalloc_matches_execute_twice(hip_lib, monkeypatch):
    monkeypatch.setenv("LBR_ATTN_SPLIT", "4")
    monkeypatch.setenv("LBR_GEMM_KSPLIT", "2")
    for seq in (1024, 512):
        y, y_exec, o = _run_both(hip_lib, "gpt2", seq)
        e = normwise_rel(y, o)
        print(f"gpt2 body S={seq}: noalloc == execute bitwise: {np.array_equal(y, y_exec)}; vs oracle rel {e:.2e}")
        np.testing.assert_array_equal(y, y_exec)
        assert np.isfinite(y).all() and e <= 1e-3


@pytest.mark.parametrize("key", ["toy", "gpt2w", "gpt2", "gpt2_lm", "7b4k", "qwen3_4b", "qwen3_4b_lm"])
def test_noalloc_takes_every_workload(hip_lib, key):
    """The scratch array holds the workspace of every benchmark workload's one-kernel-per-node
    array at its benchmark size: lbr_execute_noalloc runs it and matches lbr_execute bit for
    bit.  (lbr_execute's grow-only workspace, printed, is the largest need so far.)"""
    from runtime.executor.compiled import CompiledExecutor
    from runtime.planner import plan
    from workloads import export_workload
    from runtime.passes import run_pipeline
    lib = hip_lib
    _, x, graph = export_workload(key)
    run_pipeline(graph, None)
    ex = CompiledExecutor(fuse=False)
    ex.compile(plan(graph))
    try:
        n = len(ex.dispatch_order)
        name_in, name_out = graph.inputs[0], graph.outputs[0]
        ex.upload_inputs({name_in: x})
        lib.check(lib.lbr_execute(ex._nodes, n), "lbr_execute")
        ws = ctypes.c_size_t(0)
        lib.check(lib.lbr_execute_workspace_bytes(ctypes.byref(ws)), "lbr_execute_workspace_bytes")
        print(f"{key}: lbr_execute workspace so far {ws.value / 2**20:.1f} MiB")
        y_exec = ex.download_outputs()[name_out]
        out_ptr = ctypes.c_void_p(ex.device_address(name_out))
        lib.check(lib.lbr_memset(out_ptr, 0, y_exec.nbytes), "lbr_memset")
        ex.upload_inputs({name_in: x})
        lib.check(lib.lbr_execute_noalloc(ex._nodes, n), "lbr_execute_noalloc")
        y = ex.download_outputs()[name_out]
    finally:
        ex.close()
    print(f"{key}: noalloc == execute bitwise: {np.array_equal(y, y_exec)}")
    np.testing.assert_array_equal(y, y_exec)


def test_noalloc_rejects_oversized_workspace(hip_lib, monkeypatch):
    """16 K ranges of a 2048 x 2048 product need 256 MiB of partial sums, more than the
    scratch array holds: refused before any launch, the output left untouched."""
    from runtime.executor.common import COpNode
    from runtime.ir import OpType
    monkeypatch.setenv("LBR_GEMM_KSPLIT", "16")
    M = N = 2048
    K = 512
    lib = hip_lib
    a, b, c = lib.alloc(M * K * 4), lib.alloc(N * K * 4), lib.alloc(M * N * 4)
    try:
        lib.check(lib.lbr_memset(ctypes.c_void_p(c), 0x7f, M * N * 4), "lbr_memset")
        node = (COpNode * 1)()
        node[0].op = OpType.MATMUL.value
        node[0].n_inputs = 2
        node[0].inputs[0] = a
        node[0].inputs[1] = b
        node[0].output = c
        node[0].n_dims = 2
        node[0].out_shape[0] = M
        node[0].out_shape[1] = N
        node[0].elem_size = 4
        node[0].extra[0] = K
        node[0].extra[1] = 1   # trans_b
        node[0].extra[2] = 1   # b_is_2d
        assert lib.lbr_execute_noalloc(node, 1) == 1   # LBR_ERR_INVALID
        assert "workspace" in lib.last_error()
        host = np.empty(16, dtype=np.uint8)
        lib.d2h(host.ctypes.data, c, 16)
        assert (host == 0x7f).all()
    finally:
        for p in (a, b, c):
            lib.free(p)
