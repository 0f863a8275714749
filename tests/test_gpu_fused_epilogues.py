"""Fused GEMM epilogues on the GPU, through the compiled executor:

* MATMUL[_ADD] → RELU / GELU / SILU, the activation applied in the GEMM
  epilogue (or in the split-K reduction), and
* the gated pair MATMUL[_ADD] with 2F columns → SLICE [0,F) and [F,2F) →
  GATED_ACT(gate, [bias], up), computed by one GEMM whose tiles pair gate
  and up columns,
* TRANSPOSE → MATMUL[_ADD] → [ADD], the GEMM reading A in head layout, and
  SLICE → TRANSPOSE → ATTENTION → TRANSPOSE, the attention reading V from
  the sliced tensor's columns,
* ATTENTION → TRANSPOSE with the output over V (split attention, the merge
  kernel writing every row),

each against the float64 closed form, the CPU oracle, and the same graph run
node by node (fusion off): the bits must be identical, since the epilogue
rounds every step in the order the separate nodes do.
"""

import numpy as np
import pytest

from conftest import normwise_rel
from helpers import cf_gelu_tanh, cf_silu, randn, rng, run_oracle
from runtime.ir import Graph, OpType

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _run(graph, inputs, fuse):
    from runtime.executor.compiled import CompiledExecutor
    from runtime.planner import plan
    ex = CompiledExecutor(fuse=fuse)
    ex.compile(plan(graph))
    try:
        y = ex.run(inputs)[graph.outputs[0]]
        return y, [kind for _, _, kind in ex.fused_runs()]
    finally:
        ex.close()


def _check(graph, inputs, ref, kind):
    y, runs = _run(graph, inputs, True)
    z, plain = _run(graph, inputs, False)
    o = run_oracle(graph, inputs)
    print(f"{kind}: fused runs {runs}; gpu-vs-ref {normwise_rel(y, ref):.2e} oracle-vs-ref {normwise_rel(o, ref):.2e}")
    assert runs == [kind] and plain == []
    np.testing.assert_array_equal(y, z)
    assert normwise_rel(o, ref) <= TOL
    assert normwise_rel(y, ref) <= TOL
    assert normwise_rel(y, o) <= TOL


def _gemm_graph(g, r, M, N, K, bias):
    """a [1, M, K] input, w [N, K] (and b [N]) constants, c = a·wᵀ (+ b); returns a, c64."""
    a = randn(r, 1, M, K)
    w = randn(r, N, K)
    g.add_tensor("a", (1, M, K))
    g.inputs.append("a")
    g.add_tensor("w", (N, K)).buffer = w
    g.constants.append("w")
    ins = ["a", "w"]
    c = a.astype(np.float64) @ w.T.astype(np.float64)
    if bias:
        b = randn(r, N)
        g.add_tensor("b", (N,)).buffer = b
        g.constants.append("b")
        ins.append("b")
        c = c + b
    g.add_tensor("c", (1, M, N))
    g.add_node(OpType.MATMUL_ADD if bias else OpType.MATMUL, ins, "c", {"transpose_b": True})
    return a, c


ACTS = {OpType.RELU: lambda v: np.maximum(v, 0.0), OpType.GELU: cf_gelu_tanh, OpType.SILU: cf_silu}


# Kernel-selection overrides (read when the plan is built): LBR_GEMM_TILE forces
# a DMA tile, LBR_GEMM_KSPLIT the number of K ranges (the activation then runs
# in the split-K reduction).
@pytest.mark.parametrize("op", list(ACTS), ids=lambda o: o.name)
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("tile,ks,M,N,K", [(None, None, 300, 520, 96), ("256x256", "1", 300, 520, 96),
                                           ("64x128", "1", 70, 130, 64), ("128x128", "3", 200, 300, 3072),
                                           ("32x64", "1", 70, 130, 64), ("32x96", "2", 200, 300, 768),
                                           ("32x96k64", "1", 70, 130, 128), ("64x64k64", "2", 200, 300, 768)])
def test_gemm_activation_epilogue(monkeypatch, op, bias, tile, ks, M, N, K):
    if tile:
        monkeypatch.setenv("LBR_GEMM_TILE", tile)
        monkeypatch.setenv("LBR_GEMM_KSPLIT", ks)
    r = rng(M + N + K)
    g = Graph()
    a, c = _gemm_graph(g, r, M, N, K, bias)
    g.add_tensor("y", (1, M, N))
    g.add_node(op, ["c"], "y", {})
    g.outputs.append("y")
    _check(g, {"a": a}, ACTS[op](c), "gemm_act")


@pytest.mark.parametrize("tile", [None, "256x256", "128x128", "128x64", "64x128", "64x64", "64x96", "32x64",
                                  "64x64k64"])
@pytest.mark.parametrize("act,gbias,order,mm_bias", [("silu", False, 0, False), ("gelu", True, 1, True),
                                                      ("silu", True, 0, True), ("gelu", False, 1, False)])
def test_gemm_gated_epilogue(monkeypatch, tile, act, gbias, order, mm_bias):
    """gate = the half picked by `order` (0: columns [0, F)), F ragged against the 16-column
    blocks and the tiles."""
    if tile:
        monkeypatch.setenv("LBR_GEMM_TILE", tile)
        monkeypatch.setenv("LBR_GEMM_KSPLIT", "1")
    M, F, K = 300, 200, 128   # K: two steps of the 64-wide-step tiles, four of the others
    r = rng(M + F + K + order)
    g = Graph()
    a, c = _gemm_graph(g, r, M, 2 * F, K, mm_bias)
    for k, (lo, hi) in enumerate([(0, F), (F, 2 * F)]):
        g.add_tensor(f"s{k}", (1, M, F))
        g.add_node(OpType.SLICE, ["c"], f"s{k}", {"dim": 2, "start": lo, "end": hi})
    halves = [c[..., :F], c[..., F:]]
    x, up = (halves[0], halves[1]) if order == 0 else (halves[1], halves[0])
    ins = ["s0", "s1"] if order == 0 else ["s1", "s0"]
    if gbias:
        gb = randn(r, F)
        g.add_tensor("gb", (F,)).buffer = gb
        g.constants.append("gb")
        ins.insert(1, "gb")
        x = x + gb
    g.add_tensor("y", (1, M, F))
    g.add_node(OpType.GATED_ACT, ins, "y", {"has_bias": gbias, "act": act})
    g.outputs.append("y")
    ref = (cf_silu(x) if act == "silu" else cf_gelu_tanh(x)) * up
    _check(g, {"a": a}, ref, "gemm_gated")


@pytest.mark.parametrize("tile,ks", [(None, None), ("256x256", "1"), ("128x64", "1"), ("64x64", "1"),
                                     ("32x48", "1"), ("32x48s4", "1"), ("64x96", "1"), ("32x64", "1"), ("64x32", "2"),
                                     ("32x96", "1"), ("32x160", "1"),
                                     ("128x128", "3")])
@pytest.mark.parametrize("H,S,hd,N,bias,resid", [(4, 300, 64, 200, True, True), (2, 130, 128, 96, False, True),
                                                  (8, 64, 32, 520, True, False), (4, 40, 16, 64, True, True),
                                                  (12, 70, 8, 100, False, True)])
def test_transpose_gemm(monkeypatch, tile, ks, H, S, hd, N, bias, resid):
    """O [1, H, S, hd] → TRANSPOSE(1, 2) → [1, S, H·hd] → MATMUL[_ADD] → [ADD(C, R)]: the GEMM reads
    O in its head layout (the transposed copy is never made).  ks=3 splits K into ranges that
    start inside a head (e.g. k0 = 96 with hd = 64); hd = 16 and 8 put 2 and 4 whole heads in
    one 32-wide K step."""
    if tile:
        monkeypatch.setenv("LBR_GEMM_TILE", tile)
        monkeypatch.setenv("LBR_GEMM_KSPLIT", ks)
    r = rng(H * S + hd + N)
    K = H * hd
    o = randn(r, 1, H, S, hd)
    w = randn(r, N, K)
    g = Graph()
    g.add_tensor("o", (1, H, S, hd))
    g.inputs.append("o")
    g.add_tensor("t", (1, S, H, hd))
    g.add_node(OpType.TRANSPOSE, ["o"], "t", {"dim0": 1, "dim1": 2})
    g.add_tensor("a", (1, S, K))
    g.add_node(OpType.RESHAPE, ["t"], "a", {"shape": (1, S, K)})
    g.add_tensor("w", (N, K)).buffer = w
    g.constants.append("w")
    ins = ["a", "w"]
    c = np.swapaxes(o, 1, 2).reshape(1, S, K).astype(np.float64) @ w.T.astype(np.float64)
    if bias:
        b = randn(r, N)
        g.add_tensor("b", (N,)).buffer = b
        g.constants.append("b")
        ins.append("b")
        c = c + b
    g.add_tensor("c", (1, S, N))
    g.add_node(OpType.MATMUL_ADD if bias else OpType.MATMUL, ins, "c", {"transpose_b": True})
    inputs = {"o": o}
    out = "c"
    if resid:
        res = randn(r, 1, S, N)
        g.add_tensor("r", (1, S, N))
        g.inputs.append("r")
        inputs["r"] = res
        g.add_tensor("y", (1, S, N))
        g.add_node(OpType.ADD, ["c", "r"], "y", {})
        c = c + res
        out = "y"
    g.outputs.append(out)
    _check(g, inputs, c, "transpose_gemm")


@pytest.mark.parametrize("split", [None, "3"])
@pytest.mark.parametrize("H,Hkv,S,hd,causal", [(8, 2, 300, 128, True), (4, 4, 200, 64, False),
                                               (12, 4, 1024, 64, True)])
def test_attention_sliced_v(monkeypatch, split, H, Hkv, S, hd, causal):
    """kv [1, S, 2·Hkv·hd] → SLICE (V columns) → RESHAPE → TRANSPOSE(1, 2) → V of a GQA ATTENTION →
    TRANSPOSE(1, 2): one attention kernel reading the V rows from kv's columns with kv's row
    stride (the sliced and transposed copies are never made), under the plain and the split
    (LBR_ATTN_SPLIT=3: shares of 3 key tiles) schedules."""
    from helpers import cf_attention
    if split:
        monkeypatch.setenv("LBR_ATTN_SPLIT", split)
        monkeypatch.setenv("LBR_ATTN_FOLD", "0")
    r = rng(H * S + hd)
    W = Hkv * hd
    q = randn(r, 1, H, S, hd)
    k = randn(r, 1, Hkv, S, hd)
    kv = randn(r, 1, S, 2 * W)
    g = Graph()
    for name, arr in (("q", q), ("k", k), ("kv", kv)):
        g.add_tensor(name, arr.shape)
        g.inputs.append(name)
    g.add_tensor("v2", (1, S, W))
    g.add_node(OpType.SLICE, ["kv"], "v2", {"dim": 2, "start": W, "end": 2 * W})
    g.add_tensor("v4", (1, S, Hkv, hd))
    g.add_node(OpType.RESHAPE, ["v2"], "v4", {"shape": (1, S, Hkv, hd)})
    g.add_tensor("vt", (1, Hkv, S, hd))
    g.add_node(OpType.TRANSPOSE, ["v4"], "vt", {"dim0": 1, "dim1": 2})
    attrs = {"group_size": H // Hkv}
    if causal:
        attrs["causal"] = True
    g.add_tensor("att", (1, H, S, hd))
    g.add_node(OpType.ATTENTION, ["q", "k", "vt"], "att", attrs)
    g.add_tensor("out", (1, S, H, hd))
    g.add_node(OpType.TRANSPOSE, ["att"], "out", {"dim0": 1, "dim1": 2})
    g.outputs.append("out")
    v = np.ascontiguousarray(kv[..., W:].reshape(1, S, Hkv, hd).transpose(0, 2, 1, 3))
    ref = np.swapaxes(cf_attention(q, k, v, causal=causal, group=H // Hkv), 1, 2)
    _check(g, {"q": q, "k": k, "kv": kv}, ref, "attn_sliced_v")


@pytest.mark.parametrize("fold64", [False, True], ids=["default", "fold64"])
@pytest.mark.parametrize("H,S,hd", [(12, 1024, 64), (8, 640, 128)])
def test_attention_sliced_v_over_its_source(monkeypatch, H, S, hd, fold64):
    """kv = RELU(kv_in) in the arena → SLICE (V columns) → RESHAPE → TRANSPOSE → V of a causal
    ATTENTION small enough for the key-range split → TRANSPOSE: the planner puts the output over
    kv's rows, which the fused kernel reads V from.  The run is still one kernel: every row
    goes through the split's workspace and the merge kernel writes the output after kv has
    been read (bit-identical to the plan without fusion).  fold64: the 16x16 kernel on folded
    64-row blocks (LBR_ATTN_FOLD64=1) stages its rows and attn_kq_flush stores them."""
    from helpers import cf_attention
    from runtime.executor.compiled import CompiledExecutor
    from runtime.planner import plan
    if fold64:
        monkeypatch.setenv("LBR_ATTN_FOLD64", "1")
        monkeypatch.setenv("LBR_ATTN_KQ", "0")
    r = rng(H * S + hd + 1)
    W = H * hd
    q, k, kv_in = randn(r, 1, H, S, hd), randn(r, 1, H, S, hd), randn(r, 1, S, 2 * W)
    g = Graph()
    for name, arr in (("q", q), ("k", k), ("kv_in", kv_in)):
        g.add_tensor(name, arr.shape)
        g.inputs.append(name)
    g.add_tensor("kv", (1, S, 2 * W))
    g.add_node(OpType.RELU, ["kv_in"], "kv", {})
    g.add_tensor("v2", (1, S, W))
    g.add_node(OpType.SLICE, ["kv"], "v2", {"dim": 2, "start": W, "end": 2 * W})
    g.add_tensor("v4", (1, S, H, hd))
    g.add_node(OpType.RESHAPE, ["v2"], "v4", {"shape": (1, S, H, hd)})
    g.add_tensor("vt", (1, H, S, hd))
    g.add_node(OpType.TRANSPOSE, ["v4"], "vt", {"dim0": 1, "dim1": 2})
    g.add_tensor("att", (1, H, S, hd))
    g.add_node(OpType.ATTENTION, ["q", "k", "vt"], "att", {"causal": True})
    g.add_tensor("out", (1, S, H, hd))
    g.add_node(OpType.TRANSPOSE, ["att"], "out", {"dim0": 1, "dim1": 2})
    g.outputs.append("out")
    mem = plan(g)
    kv0, out0 = mem.offsets["kv"], mem.offsets["out"]
    assert out0 < kv0 + S * 2 * W * 4 and kv0 < out0 + S * W * 4   # the output lies over kv
    ex = CompiledExecutor(fuse=True)
    ex.compile(mem)
    try:
        assert any(n.endswith("+v+transpose+defer") for n in ex.kernel_names())
        if fold64:
            att = [p for p in ex.step_params() if p["kernel"].startswith("attn_fwd_mfma16")]
            assert att and all(p["block_rows"] == 64 and p["defer"] for p in att), att
    finally:
        ex.close()
    kv = np.maximum(kv_in, 0.0)
    v = np.ascontiguousarray(kv[..., W:].reshape(1, S, H, hd).transpose(0, 2, 1, 3))
    ref = np.swapaxes(cf_attention(q, k, v, causal=True), 1, 2)
    _check(g, {"q": q, "k": k, "kv_in": kv_in}, ref, "attn_sliced_v")


@pytest.mark.parametrize("H,S,hd,causal,fold64", [(12, 1024, 64, True, False), (8, 640, 128, True, False),
                                                  (4, 700, 64, False, False), (8, 640, 128, True, True),
                                                  (3, 333, 64, True, True)])
def test_attention_transpose_over_v(monkeypatch, H, S, hd, causal, fold64):
    """V = RELU(x) lives in the arena and is dead after an ATTENTION small enough for the
    key-range split; the planner puts the output TRANSPOSE(1, 2) over V's memory.  The fused
    kernel sends every row through the split's workspace and the merge kernel, which runs
    after V has been read, writes the [B, S, H, hd] output (bit-identical to the direct store).
    fold64: the folded 64-row schedule, rows staged for attn_kq_flush."""
    from helpers import cf_attention
    from runtime.executor.compiled import CompiledExecutor
    from runtime.planner import plan
    if fold64:
        monkeypatch.setenv("LBR_ATTN_FOLD64", "1")
        monkeypatch.setenv("LBR_ATTN_KQ", "0")
    r = rng(H * S + hd)
    q, k, x = randn(r, 1, H, S, hd), randn(r, 1, H, S, hd), randn(r, 1, H, S, hd)
    g = Graph()
    for name in ("q", "k", "x"):
        g.add_tensor(name, (1, H, S, hd))
        g.inputs.append(name)
    g.add_tensor("v", (1, H, S, hd))
    g.add_node(OpType.RELU, ["x"], "v", {})
    g.add_tensor("att", (1, H, S, hd))
    g.add_node(OpType.ATTENTION, ["q", "k", "v"], "att", {"causal": True} if causal else {})
    g.add_tensor("out", (1, S, H, hd))
    g.add_node(OpType.TRANSPOSE, ["att"], "out", {"dim0": 1, "dim1": 2})
    g.outputs.append("out")
    mem = plan(g)
    assert mem.offsets["out"] == mem.offsets["v"]
    ex = CompiledExecutor(fuse=True)
    ex.compile(mem)
    try:
        assert any(n.endswith("+transpose+defer") for n in ex.kernel_names())
        if fold64:
            att = [p for p in ex.step_params() if p["kernel"].startswith("attn_fwd_mfma16")]
            assert att and all(p["block_rows"] == 64 and p["defer"] for p in att), att
    finally:
        ex.close()
    ref = np.swapaxes(cf_attention(q, k, np.maximum(x, 0.0), causal=causal), 1, 2)
    _check(g, {"q": q, "k": k, "x": x}, ref, "attn_transpose")


@pytest.mark.parametrize("H,S,hd,causal,fold64", [(12, 1024, 64, True, False), (8, 640, 128, True, False),
                                                  (4, 700, 64, False, False), (8, 640, 128, True, True)])
def test_attention_output_relay(monkeypatch, H, S, hd, causal, fold64):
    """The output TRANSPOSE over V, as above, read only by the projection GEMM after it: the plan
    gives the attention a buffer of its own and points the GEMM's A there, so the store is not
    deferred (only cut blocks go through the merge kernel).  Bit-equal to the deferred plan
    (LBR_ATTN_RELAY=0), and to the closed form within the fused tolerance."""
    from helpers import cf_attention
    from runtime.executor.compiled import CompiledExecutor
    from runtime.planner import plan
    if fold64:
        monkeypatch.setenv("LBR_ATTN_FOLD64", "1")
        monkeypatch.setenv("LBR_ATTN_KQ", "0")
    r = rng(H * S + hd + 2)
    W, N = H * hd, 96
    q, k, x = randn(r, 1, H, S, hd), randn(r, 1, H, S, hd), randn(r, 1, H, S, hd)
    w = randn(r, N, W, scale=0.05)
    g = Graph()
    for name in ("q", "k", "x"):
        g.add_tensor(name, (1, H, S, hd))
        g.inputs.append(name)
    g.add_tensor("w", (N, W)).buffer = w
    g.constants.append("w")
    g.add_tensor("v", (1, H, S, hd))
    g.add_node(OpType.RELU, ["x"], "v", {})
    g.add_tensor("att", (1, H, S, hd))
    g.add_node(OpType.ATTENTION, ["q", "k", "v"], "att", {"causal": True} if causal else {})
    g.add_tensor("out", (1, S, H, hd))
    g.add_node(OpType.TRANSPOSE, ["att"], "out", {"dim0": 1, "dim1": 2})
    g.add_tensor("o2", (1, S, W))
    g.add_node(OpType.RESHAPE, ["out"], "o2", {"shape": (1, S, W)})
    g.add_tensor("c", (1, S, N))
    g.add_node(OpType.MATMUL, ["o2", "w"], "c", {"transpose_b": True})
    g.outputs.append("c")
    ins = {"q": q, "k": k, "x": x}
    ys = {}
    for relay in ("1", "0"):
        monkeypatch.setenv("LBR_ATTN_RELAY", relay)
        ex = CompiledExecutor(fuse=True)
        ex.compile(plan(g))
        try:
            names = ex.kernel_names()
            print(relay, names)
            assert any(n.endswith("+transpose+relay" if relay == "1" else "+transpose+defer") for n in names)
            ys[relay] = [ex.run(ins)["c"] for _ in range(3)]
        finally:
            ex.close()
    for y in ys["1"] + ys["0"][1:]:
        assert np.array_equal(y, ys["0"][0])
    att = np.swapaxes(cf_attention(q, k, np.maximum(x, 0.0), causal=causal), 1, 2).reshape(1, S, W)
    ref = att.astype(np.float64) @ w.T.astype(np.float64)
    assert normwise_rel(ys["1"][0], ref) <= 1e-4


@pytest.mark.parametrize("H,Hkv,S,hd,causal,k_live,D", [(12, 12, 256, 64, True, False, 96),
                                                        (8, 2, 512, 64, True, False, 96),
                                                        (4, 4, 128, 32, False, False, 96),
                                                        (12, 12, 256, 64, True, True, 96),
                                                        (4, 4, 192, 64, True, False, 100)])
def test_attention_fragment_major_keys(monkeypatch, H, Hkv, S, hd, causal, k_live, D):
    """x → MATMUL_ADD → q/k/v (SLICE → RESHAPE → TRANSPOSE(1, 2)) → key-quartered ATTENTION: the
    QKV GEMM's head scatter stores K fragment-major (16-row × 16-column chunks of 1 KiB) and the
    attention loads it so, whole cache lines per load.  Bit-equal to the row-major plan
    (LBR_KQ_FRAG=0), within 1e-4 of the float64 closed form.  With K also a graph output the
    plan keeps K row-major (the caller reads it), and the returned K matches the closed form.
    D = 100 is not a multiple of the DMA GEMM's K step: the other MFMA kernel's head scatter."""
    from helpers import cf_attention
    from runtime.executor.compiled import CompiledExecutor
    from runtime.planner import plan
    r = rng(H * S + hd + 7)
    widths = [H * hd, Hkv * hd, Hkv * hd]
    N = sum(widths)
    x = randn(r, 1, S, D)
    w = randn(r, N, D, scale=0.1)
    b = randn(r, N, scale=0.1)
    g = Graph()
    g.add_tensor("x", (1, S, D))
    g.inputs.append("x")
    g.add_tensor("w", (N, D)).buffer = w
    g.add_tensor("b", (N,)).buffer = b
    g.constants += ["w", "b"]
    g.add_tensor("c", (1, S, N))
    g.add_node(OpType.MATMUL_ADD, ["x", "w", "b"], "c", {"transpose_b": True})
    col = 0
    for name, heads, wd in (("q", H, widths[0]), ("k", Hkv, widths[1]), ("v", Hkv, widths[2])):
        g.add_tensor(name + "2", (1, S, wd))
        g.add_node(OpType.SLICE, ["c"], name + "2", {"dim": 2, "start": col, "end": col + wd})
        g.add_tensor(name + "4", (1, S, heads, hd))
        g.add_node(OpType.RESHAPE, [name + "2"], name + "4", {"shape": (1, S, heads, hd)})
        g.add_tensor(name + "t", (1, heads, S, hd))
        g.add_node(OpType.TRANSPOSE, [name + "4"], name + "t", {"dim0": 1, "dim1": 2})
        col += wd
    attrs = {"group_size": H // Hkv} if Hkv != H else {}
    if causal:
        attrs["causal"] = True
    g.add_tensor("att", (1, H, S, hd))
    g.add_node(OpType.ATTENTION, ["qt", "kt", "vt"], "att", attrs)
    g.outputs.append("att")
    if k_live:
        g.outputs.append("kt")
    c64 = x.astype(np.float64) @ w.T.astype(np.float64) + b
    heads = []
    col = 0
    for hh, wd in zip((H, Hkv, Hkv), widths):
        heads.append(np.ascontiguousarray(c64[..., col:col + wd].reshape(1, S, hh, hd).transpose(0, 2, 1, 3)))
        col += wd
    ref = cf_attention(*heads, causal=causal, group=H // Hkv)
    ys = {}
    for frag in ("1", "0"):
        monkeypatch.setenv("LBR_KQ_FRAG", frag)
        ex = CompiledExecutor(fuse=True)
        ex.compile(plan(g))
        try:
            params = ex.step_params()
            att = [p for p in params if p["kernel"].startswith("attn_fwd_kq")]
            gem = [p for p in params if p["kernel"].startswith("gemm_")]
            print(frag, [p["name"] for p in params], [p.get("k_frag") for p in att], [p.get("frag_splits") for p in gem])
            assert len(att) == 1 and len(gem) == 1
            assert gem[0]["kernel"].startswith("gemm_dma" if D % 32 == 0 else "gemm_mfma")
            on = frag == "1" and not k_live
            assert att[0]["k_frag"] == on and gem[0]["frag_splits"] == (2 if on else 0)
            ys[frag] = ex.run({"x": x})
        finally:
            ex.close()
    np.testing.assert_array_equal(ys["1"]["att"], ys["0"]["att"])
    assert normwise_rel(ys["1"]["att"], ref) <= 1e-4
    if k_live:
        assert normwise_rel(ys["1"]["kt"], heads[1]) <= 1e-5
