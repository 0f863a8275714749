"""GEMM tile choice at plan creation.  By default a committed table of measured
tiles (kTunedTiles) sets the tile of the workloads' listed GEMM steps and the
model's pick holds elsewhere, so a plan is the same run to run.
LBR_GEMM_AUTOTUNE=1 also times the other small one-batch, unsplit DMA GEMMs
over every tile their launcher family has, and the fastest replaces the
model's choice; LBR_GEMM_AUTOTUNE=0 keeps the model's pick everywhere.

Every DMA tile sums each output's K terms in the same order (K steps in
order, the same 4-wide MFMA reduction inside a step), so a tuned plan and
the model's plan give bit-identical outputs; plan creation restores the
ranges the timed launches wrote, so memory is as the caller left it.
"""

import ctypes

import numpy as np
import pytest

from conftest import normwise_rel

pytestmark = pytest.mark.gpu


def _gemm_node(M, N, K, a, b, bias, c):
    from runtime.executor.common import COpNode
    from runtime.ir import OpType
    node = (COpNode * 1)()
    node[0].op = OpType.MATMUL_ADD.value
    node[0].n_inputs = 3
    node[0].inputs[0] = a
    node[0].inputs[1] = b
    node[0].inputs[2] = bias
    node[0].output = c
    node[0].n_dims = 3
    node[0].out_shape[0] = 1
    node[0].out_shape[1] = M
    node[0].out_shape[2] = N
    node[0].elem_size = 4
    node[0].extra[0] = K
    node[0].extra[1] = 1   # trans_b
    node[0].extra[2] = 1   # b_is_2d
    return node


@pytest.mark.parametrize("M,N,K", [(512, 2304, 768), (1024, 2304, 768), (512, 3072, 768), (1024, 768, 768)])
def test_autotune_restores_memory_and_matches_model(hip_lib, monkeypatch, M, N, K):
    lib = hip_lib
    r = np.random.default_rng(M + N + K)
    a_h = r.standard_normal((M, K)).astype(np.float32)
    b_h = (0.05 * r.standard_normal((N, K))).astype(np.float32)
    bias_h = r.standard_normal(N).astype(np.float32)
    a, b, bias, c = (lib.alloc(x) for x in (a_h.nbytes, b_h.nbytes, bias_h.nbytes, M * N * 4))
    try:
        for dev, host in ((a, a_h), (b, b_h), (bias, bias_h)):
            lib.h2d(dev, host.ctypes.data, host.nbytes)
        node = _gemm_node(M, N, K, a, b, bias, c)
        outs = {}
        for tune in ("1", "0"):
            monkeypatch.setenv("LBR_GEMM_AUTOTUNE", tune)
            lib.check(lib.lbr_memset(ctypes.c_void_p(c), 0x7f, M * N * 4), "lbr_memset")
            plan = ctypes.c_void_p()
            lib.check(lib.lbr_plan_create(node, 1, 1, ctypes.byref(plan)), "lbr_plan_create")
            try:
                host = np.empty(M * N, dtype=np.uint8)
                lib.d2h(host.ctypes.data, c, host.nbytes)
                assert (host == 0x7f).all(), "plan creation left the output changed"
                lib.check(lib.lbr_plan_launch(plan), "lbr_plan_launch")
                lib.check(lib.lbr_synchronize(), "lbr_synchronize")
                y = np.empty((M, N), dtype=np.float32)
                lib.d2h(y.ctypes.data, c, y.nbytes)
                outs[tune] = y
            finally:
                lib.check(lib.lbr_plan_destroy(plan), "lbr_plan_destroy")
    finally:
        for p in (a, b, bias, c):
            lib.free(p)
    ref = a_h.astype(np.float64) @ b_h.T.astype(np.float64) + bias_h
    print(f"{M}x{N}x{K}: tuned == model bitwise {np.array_equal(outs['1'], outs['0'])}, "
          f"vs float64 {normwise_rel(outs['1'], ref):.2e}")
    np.testing.assert_array_equal(outs["1"], outs["0"])
    assert normwise_rel(outs["1"], ref) <= 1e-5


@pytest.mark.parametrize("key,seq", [("gpt2w", 512), ("gpt2", 256), ("toy", 32)])
def test_autotune_workload_bitwise(monkeypatch, key, seq):
    """Whole fused bodies (head scatter, activation, residual, norm prologue
    epilogues): the timed plan (LBR_GEMM_AUTOTUNE=1: the table, then timing of the
    other steps' tiles) equals the default table plan bit for bit, and the model's
    plan (=0) too where the table keeps each step's K ranges; where the table sets
    other K ranges (GPT-2-width's O projection and FFN2) the model's plan sums other
    partial sums and agrees to float32 rounding."""
    from runtime.executor.compiled import CompiledExecutor
    from runtime.passes import run_pipeline
    from runtime.planner import plan
    from workloads import export_workload
    _, x, graph = export_workload(key, seq_len=seq)
    run_pipeline(graph, None)
    mp = plan(graph)
    name_in, name_out = graph.inputs[0], graph.outputs[0]
    outs, tiles = {}, {}
    for tune in ("1", None, "0"):
        if tune is None:
            monkeypatch.delenv("LBR_GEMM_AUTOTUNE", raising=False)
        else:
            monkeypatch.setenv("LBR_GEMM_AUTOTUNE", tune)
        ex = CompiledExecutor()
        ex.compile(mp)
        try:
            tiles[tune] = [(p["tile"], p["ksplit"]) for p in ex.step_params() if p["kernel"].startswith("gemm_dma")]
            outs[tune] = ex.run({name_in: x})[name_out]
        finally:
            ex.close()
    print(f"{key} S={seq}: DMA tiles timed {tiles['1']} table {tiles[None]} model {tiles['0']}")
    np.testing.assert_array_equal(outs["1"], outs[None])
    if [ks for _, ks in tiles[None]] == [ks for _, ks in tiles["0"]]:
        np.testing.assert_array_equal(outs[None], outs["0"])
    else:
        assert normwise_rel(outs[None], outs["0"]) <= 1e-6


def test_default_plan_takes_the_table_tiles_every_time():
    """GPT-2-width at S=512: every GEMM step takes the table's tile and K ranges (QKV
    32x160, O projection with LayerNorm 2 in its reduce 32x96 in 2 ranges, FFN1 32x64,
    FFN2 32x96 in 2 ranges), identically in every plan creation."""
    from runtime.executor.compiled import CompiledExecutor
    from runtime.passes import run_pipeline
    from runtime.planner import plan
    from workloads import export_workload
    _, x, graph = export_workload("gpt2w", seq_len=512)
    run_pipeline(graph, None)
    mp = plan(graph)
    picks = []
    for _ in range(3):
        ex = CompiledExecutor()
        ex.compile(mp)
        try:
            picks.append([(p["name"], p["m"], p["n"], p["k"], p["tile"], p["ksplit"]) for p in ex.step_params()
                          if p["kernel"].startswith("gemm_dma")])
        finally:
            ex.close()
    assert picks[0] == picks[1] == picks[2], picks
    by_name = {name: (tile, ks) for name, m, n, k, tile, ks in picks[0]}
    assert by_name == {"gemm_dma_f32_nt+heads": ("32x160", 1), "gemm_dma_f32_nt+tin+resid+layernorm": ("32x96", 2),
                       "gemm_dma_f32_nt+act": ("32x64", 1), "gemm_dma_f32_nt+resid": ("32x96", 2)}, picks[0]
