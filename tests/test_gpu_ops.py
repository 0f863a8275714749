"""Per-op parity on the GPU: each device kernel (through the C ABI, via the
compiled executor) against the CPU oracle and a float64 closed form.

Tolerances: normwise max relative error ≤ 1e-5 for element-wise/norm ops,
≤ 1e-4 for GEMM and attention (fp32 accumulation over K); copies are exact.
"""

import numpy as np
import pytest

from runtime.ir import OpType
from helpers import (cf_attention, cf_gelu_tanh, cf_layernorm, cf_rmsnorm, cf_silu, one_node_graph, randn, rng,
                     run_gpu, run_oracle)
from conftest import normwise_rel

pytestmark = pytest.mark.gpu


def _check(graph, inputs, ref, tol, kernels=None):
    y = run_gpu(graph, inputs, kernels=kernels)
    o = run_oracle(graph, inputs)
    assert y.shape == ref.shape
    e_gpu, e_orc, e_go = normwise_rel(y, ref), normwise_rel(o, ref), normwise_rel(y, o)
    print(f"gpu-vs-ref {e_gpu:.2e} oracle-vs-ref {e_orc:.2e} gpu-vs-oracle {e_go:.2e}")
    assert e_orc <= tol, f"oracle off the closed form: {e_orc}"
    assert e_gpu <= tol, f"gpu off the closed form: {e_gpu}"
    assert e_go <= tol
    return y, o


# ---------------------------------------------------------------- GEMM

GEMM_CASES = [
    # (M, N, K, trans_b, batches, b_is_2d)
    (128, 128, 32, True, 1, True),
    (256, 384, 512, True, 1, True),
    (100, 70, 33, True, 1, True),     # ragged tiles, K % 4 != 0 (scalar path)
    (1000, 2304, 768, True, 1, True),
    (64, 96, 40, False, 1, True),     # B stored [K, N]
    (37, 130, 64, False, 3, False),   # batched, ragged
    (1, 512, 256, True, 1, True),     # M == 1 → GEMV
    (1, 300, 128, False, 2, False),   # batched GEMV, B [K, N]
    (5, 7, 1, True, 1, True),         # K = 1
    (256, 384, 4096, True, 1, True),  # few tiles, long K → split-K + reduction
    (200, 300, 2050, True, 1, True),  # split-K, ragged K on the scalar path
    (64, 128, 3000, False, 2, False), # split-K, batched, B [K, N]
]


# Kernel-selection overrides read when the plan is built: LBR_GEMM_TILE=legacy
# keeps the register-staged 32x32 kernel, a tile name (256x256, 128x128,
# 128x64, 64x128) forces that DMA tile, LBR_GEMM_KSPLIT=n forces n K ranges.
@pytest.mark.parametrize("kernel", ["auto", "legacy"])
@pytest.mark.parametrize("M,N,K,trans_b,batches,b2d", GEMM_CASES)
@pytest.mark.parametrize("with_bias", [False, True])
def test_gemm(monkeypatch, kernel, M, N, K, trans_b, batches, b2d, with_bias):
    if kernel == "legacy":
        monkeypatch.setenv("LBR_GEMM_TILE", "legacy")
    name = _gemm_case(M, N, K, trans_b, batches, b2d, with_bias)
    if kernel == "legacy":
        assert "dma" not in name


DMA_CASES = [
    # (M, N, K, batches, b_is_2d)
    (300, 520, 96, 1, True),      # ragged M and N edges, 3 K steps (a 64-wide-step tile falls back)
    (200, 330, 192, 1, True),     # 3 steps of 64
    (513, 257, 64, 1, True),
    (64, 64, 32, 1, True),        # a single K step
    (96, 200, 160, 3, False),     # batched, B [batches, N, K]
]


@pytest.mark.parametrize("tile", ["256x256", "128x128", "128x64", "64x128", "64x64",
                                  "32x48", "32x48s4", "64x96", "32x160", "64x32", "32x64", "32x96",
                                  "32x96k64", "64x64k64"])
@pytest.mark.parametrize("M,N,K,batches,b2d", DMA_CASES)
@pytest.mark.parametrize("with_bias", [False, True])
def test_gemm_dma_tiles(monkeypatch, tile, M, N, K, batches, b2d, with_bias):
    monkeypatch.setenv("LBR_GEMM_TILE", tile)
    monkeypatch.setenv("LBR_GEMM_KSPLIT", "1")
    assert _gemm_case(M, N, K, True, batches, b2d, with_bias) == "gemm_dma_f32_nt"


@pytest.mark.parametrize("tile,ks,M,N,K,batches", [("128x128", 3, 200, 300, 3072, 1), ("256x256", 5, 70, 90, 800, 2),
                                                   ("64x128", 2, 130, 260, 64, 1), ("64x64", 3, 100, 70, 960, 1),
                                                   ("32x48s4", 3, 100, 130, 960, 1), ("64x96", 2, 70, 200, 512, 2),
                                                   ("32x96", 2, 100, 130, 960, 1), ("64x32", 3, 70, 200, 512, 2),
                                                   ("32x160", 2, 130, 260, 640, 1), ("32x64", 4, 100, 70, 1024, 1),
                                                   ("32x96k64", 3, 100, 130, 960, 1), ("64x64k64", 2, 70, 200, 512, 2)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_gemm_dma_ksplit(monkeypatch, tile, ks, M, N, K, batches, with_bias):
    monkeypatch.setenv("LBR_GEMM_TILE", tile)
    monkeypatch.setenv("LBR_GEMM_KSPLIT", str(ks))
    assert _gemm_case(M, N, K, True, batches, batches == 1, with_bias) == "gemm_dma_f32_nt"


def _gemm_case(M, N, K, trans_b, batches, b2d, with_bias):
    r = rng(M * 7 + N + K)
    if b2d:
        a = randn(r, 1, M, K)
        b = randn(r, *( (N, K) if trans_b else (K, N) ))
        out_shape = (1, M, N)
    else:
        a = randn(r, batches, M, K)
        b = randn(r, batches, *((N, K) if trans_b else (K, N)))
        out_shape = (batches, M, N)
    bt = np.swapaxes(b, -2, -1) if trans_b else b
    ref = a.astype(np.float64) @ bt.astype(np.float64)
    consts = {"b": b}
    op = OpType.MATMUL
    alpha = 1.0 if with_bias else 0.5
    attrs = {"transpose_b": trans_b}
    if with_bias:
        bias = randn(r, N)
        consts["bias"] = bias
        op = OpType.MATMUL_ADD
        ref = ref + bias
    else:
        attrs["alpha"] = alpha
        ref = ref * alpha
    g = one_node_graph(op, {"a": a}, out_shape, attrs, consts)
    _check(g, {"a": a}, ref, 1e-4)
    return _kernel_of(g)


def _kernel_of(graph) -> str:
    """Kernel the plan of a one-node graph launches (kernel selection happens at plan build)."""
    from runtime.executor.compiled import CompiledExecutor
    from runtime.planner import plan
    ex = CompiledExecutor()
    ex.compile(plan(graph))
    try:
        return ex.kernel_names()[0]
    finally:
        ex.close()


def test_matmul_add_ignores_alpha():
    """MATMUL_ADD applies bias with alpha fixed to 1, like the reference's C dispatch (executor.c:341)."""
    r = rng(3)
    a, b, bias = randn(r, 1, 64, 32), randn(r, 48, 32), randn(r, 48)
    g = one_node_graph(OpType.MATMUL_ADD, {"a": a}, (1, 64, 48), {"transpose_b": True, "alpha": 2.0},
                       {"b": b, "bias": bias})
    ref = a.astype(np.float64) @ b.T.astype(np.float64) + bias
    _check(g, {"a": a}, ref, 1e-4)


# ---------------------------------------------------------------- attention

ATTN_CASES = [
    # (B, H, S, hd, causal, group)
    (1, 4, 32, 16, True, 1),
    (1, 4, 32, 16, False, 1),
    (2, 3, 7, 64, True, 1),
    (1, 2, 100, 64, False, 1),
    (1, 12, 512, 64, True, 1),
    (1, 4, 257, 128, True, 1),
    (1, 8, 300, 128, False, 4),
    (1, 32, 256, 128, True, 4),
    (1, 2, 1, 64, True, 1),
    (1, 2, 40, 24, True, 1),        # hd % 8 == 0, padded to 32
    (1, 2, 33, 12, False, 1),       # hd % 8 != 0 → row fallback kernel
    (1, 2, 200, 256, True, 1),      # hd > 128 → 32x32 MFMA kernel
    (1, 3, 70, 160, False, 1),      # hd > 128, padded to 256
    (1, 32, 1024, 128, True, 4),    # Qwen3-4B attention: small grid → key-range split
    (1, 12, 1024, 64, True, 1),     # GPT-2 attention: split with 4-tile shares
]


def _attention_case(B, H, S, hd, causal, group, kernel=None):
    r = rng(S * 3 + hd + H)
    q = randn(r, B, H, S, hd)
    k = randn(r, B, H // group, S, hd)
    v = randn(r, B, H // group, S, hd)
    attrs = {"causal": True} if causal else {}
    if group > 1:
        attrs["group_size"] = group
    g = one_node_graph(OpType.ATTENTION, {"q": q, "k": k, "v": v}, (B, H, S, hd), attrs)
    ref = cf_attention(q, k, v, causal=causal, group=group)
    names = []
    _check(g, {"q": q, "k": k, "v": v}, ref, 1e-4, kernels=names)
    if kernel is not None:
        assert names == [kernel], names


@pytest.mark.parametrize("B,H,S,hd,causal,group", ATTN_CASES)
def test_attention(B, H, S, hd, causal, group):
    _attention_case(B, H, S, hd, causal, group)


# Kernel-selection overrides read when the plan is built: LBR_ATTN_FOLD=1
# forces the paired causal schedule (workgroup j runs query blocks n-1-j and
# j; odd n leaves the middle block alone), LBR_ATTN_TILE=32 the 32x32 kernel,
# LBR_ATTN_SPLIT=c the key-range split: every workgroup an equal share of c
# key tiles (32 keys) of the whole (head, query block, tile) sequence, plus
# the merge kernel (c=1: every tile its own segment; c=3, 7: shares that cut
# blocks at varying offsets and span several blocks and heads);
# LBR_ATTN_SPLIT_WG=7 seven workgroups, shares of a non-integer tile count.
@pytest.mark.parametrize("env", [{"LBR_ATTN_FOLD": "1"}, {"LBR_ATTN_TILE": "32"},
                                 {"LBR_ATTN_SPLIT": "1", "LBR_ATTN_FOLD": "0"},
                                 {"LBR_ATTN_SPLIT": "3", "LBR_ATTN_FOLD": "0"},
                                 {"LBR_ATTN_SPLIT": "7", "LBR_ATTN_FOLD": "0"},
                                 {"LBR_ATTN_SPLIT": "8", "LBR_ATTN_FOLD": "0"},
                                 {"LBR_ATTN_SPLIT_WG": "7", "LBR_ATTN_FOLD": "0"}],
                         ids=["fold", "tile32", "split1", "split3", "split7", "split8", "wg7"])
@pytest.mark.parametrize("B,H,S,hd,causal,group", [
    (1, 4, 257, 128, True, 1),      # 3 query blocks: pair (2, 0) and the middle block 1 alone
    (1, 8, 512, 64, True, 2),       # 4 query blocks: pairs (3, 0), (2, 1)
    (2, 2, 1000, 32, True, 1),
    (1, 2, 130, 128, False, 1),     # non-causal ignores the fold flag
    (1, 3, 300, 40, True, 1),       # hd/4 = 10 threads a row: merge rows straddle workgroups
    (1, 2, 520, 96, True, 2),       # hd/4 = 24
])
def test_attention_schedules(monkeypatch, env, B, H, S, hd, causal, group):
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    _attention_case(B, H, S, hd, causal, group)


# The key-quartered kernel: 16 query rows per workgroup, the key tiles dealt over its four
# wavefronts, partial rows combined in LDS.  It takes small grids of head dim 32 or 64 by
# default (GPT-2 and GPT-2-width); LBR_ATTN_KQ=1 forces it for head dims 32, 64 and 128.
# Cases: blocks with fewer tiles than wavefronts (S ≤ 96), S not a multiple of 16 or 32
# (clamped rows past S), GQA, batches, the XCD layout with alternate blocks (12 heads) and
# without (5 and 3 heads), head dim 128.
KQ_CASES = [
    (1, 4, 32, 32, True, 1),
    (1, 4, 32, 32, False, 1),
    (2, 3, 7, 64, True, 1),
    (1, 2, 1, 64, True, 1),
    (1, 2, 100, 64, False, 1),
    (1, 12, 512, 64, True, 1),
    (1, 12, 1024, 64, True, 1),
    (1, 5, 1000, 32, True, 1),
    (2, 8, 200, 64, True, 4),
    (1, 4, 257, 128, True, 1),
    (1, 8, 300, 128, False, 4),
    (1, 32, 256, 128, True, 4),
    (1, 16, 333, 64, False, 2),
]


@pytest.mark.parametrize("B,H,S,hd,causal,group", KQ_CASES)
def test_attention_kq(monkeypatch, B, H, S, hd, causal, group):
    monkeypatch.setenv("LBR_ATTN_KQ", "1")
    _attention_case(B, H, S, hd, causal, group, kernel="attn_fwd_kq_f32")


# The 16x16 kernel on folded 64-row query blocks (4 wavefronts, one workgroup a CU at Qwen3's
# 32 heads × S1024, the default there): forced on ragged, padded, GQA, odd-block-count and
# one-row shapes, and on Qwen3's own.
@pytest.mark.parametrize("B,H,S,hd,group", [(1, 4, 257, 128, 1), (1, 8, 300, 128, 4), (2, 3, 70, 64, 1),
                                            (1, 2, 1, 128, 1), (1, 4, 100, 48, 1), (1, 2, 64, 16, 1),
                                            (1, 4, 130, 96, 2), (1, 6, 200, 32, 3), (1, 32, 1024, 128, 4)])
def test_attention_fold64(monkeypatch, B, H, S, hd, group):
    if (H, S) != (32, 1024):
        monkeypatch.setenv("LBR_ATTN_FOLD64", "1")
    monkeypatch.setenv("LBR_ATTN_KQ", "0")
    _attention_case(B, H, S, hd, True, group, kernel="attn_fwd_mfma16_f32")


@pytest.mark.parametrize("B,H,S,hd", [(1, 12, 512, 64), (1, 12, 1024, 64), (1, 4, 32, 16)])
def test_attention_small_grid_default(B, H, S, hd):
    # the schedule small grids take by default: the key-quartered kernel for head dim 32 / 64,
    # the 16x16 kernel (here with the padded head dim 16) otherwise
    kernel = "attn_fwd_kq_f32" if hd in (32, 64) else "attn_fwd_mfma16_f32"
    _attention_case(B, H, S, hd, True, 1, kernel=kernel)


@pytest.mark.parametrize("S", [16, 300])
@pytest.mark.parametrize("split", ["0", "2", "kq", "causal_flag"])
def test_attention_mask(monkeypatch, S, split):
    # causal_flag: the node also sets causal; the reference then applies the mask alone
    # (attn.c:40-48, "either custom additive mask or causal (never both)")
    if split == "kq":
        monkeypatch.setenv("LBR_ATTN_KQ", "1")
    elif split != "causal_flag":
        monkeypatch.setenv("LBR_ATTN_SPLIT", split)
    r = rng(S)
    B, H, hd = 1, 2, 64
    q, k, v = randn(r, B, H, S, hd), randn(r, B, H, S, hd), randn(r, B, H, S, hd)
    mask = np.where(r.random((B, H, S, S)) < 0.2, -1e9, 0.0).astype(np.float32)
    for i in range(S):
        mask[..., i, i] = 0.0
    g = one_node_graph(OpType.ATTENTION, {"q": q, "k": k, "v": v, "mask": mask}, (B, H, S, hd),
                       {"causal": True} if split == "causal_flag" else {})
    ref = cf_attention(q, k, v, mask=mask)
    _check(g, {"q": q, "k": k, "v": v, "mask": mask}, ref, 1e-4)


# ---------------------------------------------------------------- norms

@pytest.mark.parametrize("rows,cols", [(32, 64), (17, 768), (9, 2560), (5, 4096), (3, 130), (2, 20000)])
def test_layernorm(rows, cols):
    r = rng(rows + cols)
    x = randn(r, 1, rows, cols) * 3 + 1
    g_, b_ = randn(r, cols), randn(r, cols)
    g = one_node_graph(OpType.LAYERNORM, {"x": x}, x.shape, {"eps": 1e-5}, {"g": g_, "b": b_})
    _check(g, {"x": x}, cf_layernorm(x, g_, b_, 1e-5), 1e-5)


@pytest.mark.parametrize("rows,cols", [(1024, 128), (16, 2560), (3, 100), (2, 9000)])
def test_rmsnorm(rows, cols):
    r = rng(rows * cols)
    x = randn(r, rows, cols)
    w = randn(r, cols)
    g = one_node_graph(OpType.RMSNORM, {"x": x}, x.shape, {"eps": 1e-6}, {"w": w})
    _check(g, {"x": x}, cf_rmsnorm(x, w, 1e-6), 1e-5)


def test_softmax():
    r = rng(5)
    x = randn(r, 3, 37, 300, scale=4.0)
    g = one_node_graph(OpType.SOFTMAX, {"x": x}, x.shape, {"axis": 2})
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(-1, keepdims=True))
    _check(g, {"x": x}, e / e.sum(-1, keepdims=True), 1e-5)


@pytest.mark.parametrize("op,axis,keep", [(OpType.SUM, 1, True), (OpType.MAX, 2, False), (OpType.SUM, 0, False)])
def test_reduce(op, axis, keep):
    r = rng(axis)
    x = randn(r, 4, 33, 70)
    ref = (np.sum if op == OpType.SUM else np.max)(x.astype(np.float64), axis=axis, keepdims=keep)
    g = one_node_graph(op, {"x": x}, ref.shape, {"axis": axis, "keepdim": keep})
    _check(g, {"x": x}, ref, 1e-5)


# ---------------------------------------------------------------- element-wise

UNARY = [
    (OpType.RELU, lambda x: np.maximum(x, 0), {}),
    (OpType.EXP, np.exp, {}),
    (OpType.TANH, np.tanh, {}),
    (OpType.GELU, cf_gelu_tanh, {}),
    (OpType.SILU, cf_silu, {}),
    (OpType.NEG, lambda x: -x, {}),
    (OpType.COS, np.cos, {}),
    (OpType.SIN, np.sin, {}),
    (OpType.POW, lambda x: np.abs(x) ** 3.0, {"scalar": 3.0}),
    (OpType.RSQRT, lambda x: 1 / np.sqrt(np.abs(x) + 0.5), {}),
]


@pytest.mark.parametrize("op,fn,attrs", UNARY, ids=[u[0].name for u in UNARY])
@pytest.mark.parametrize("n", [1000, 4096 * 3 + 1])
def test_unary(op, fn, attrs, n):
    r = rng(n)
    x = randn(r, n)
    if op == OpType.POW:
        x = np.abs(x)
    if op == OpType.RSQRT:
        x = np.abs(x) + 0.5
        fn = lambda v: 1 / np.sqrt(v)
    g = one_node_graph(op, {"x": x}, x.shape, attrs)
    _check(g, {"x": x}, fn(x.astype(np.float64)), 1e-5)


@pytest.mark.parametrize("op,npf", [(OpType.ADD, np.add), (OpType.SUB, np.subtract), (OpType.MUL, np.multiply),
                                    (OpType.DIV, np.divide)])
def test_binary_modes(op, npf):
    r = rng(op.value)
    a = randn(r, 2, 16, 96)
    b_same = randn(r, 2, 16, 96) + (3.0 if op == OpType.DIV else 0.0)
    b_bcast = randn(r, 1, 16, 96) + (3.0 if op == OpType.DIV else 0.0)
    b_col = randn(r, 2, 16, 1) + (3.0 if op == OpType.DIV else 0.0)
    for b in (b_same, b_bcast, b_col):
        g = one_node_graph(op, {"a": a}, a.shape, {}, {"b": b})
        _check(g, {"a": a}, npf(a.astype(np.float64), b.astype(np.float64)), 1e-5)
    g = one_node_graph(op, {"a": a}, a.shape, {"scalar": 1.7})
    _check(g, {"a": a}, npf(a.astype(np.float64), np.float32(1.7)), 1e-5)


def test_add_bias_row():
    r = rng(11)
    a, bias = randn(r, 3, 50, 96), randn(r, 96)
    g = one_node_graph(OpType.ADD, {"a": a}, a.shape, {}, {"bias": bias})
    _check(g, {"a": a}, a.astype(np.float64) + bias, 1e-6)


def test_rope_broadcast_mul():
    r = rng(12)
    q, cos = randn(r, 1, 8, 64, 128), randn(r, 1, 1, 64, 128)
    g = one_node_graph(OpType.MUL, {"q": q}, q.shape, {}, {"cos": cos})
    _check(g, {"q": q}, q.astype(np.float64) * cos, 1e-6)


def test_bias_relu_and_gated():
    r = rng(13)
    x, bias, up = randn(r, 4, 64), randn(r, 64), randn(r, 4, 64)
    g = one_node_graph(OpType.FUSED_BIAS_RELU, {"x": x}, x.shape, {}, {"bias": bias})
    _check(g, {"x": x}, np.maximum(x.astype(np.float64) + bias, 0), 1e-6)
    for act, fn in (("silu", cf_silu), ("gelu", cf_gelu_tanh)):
        g = one_node_graph(OpType.GATED_ACT, {"x": x, "up": up}, x.shape, {"act": act, "has_bias": False})
        _check(g, {"x": x, "up": up}, fn(x) * up, 1e-5)
        g = one_node_graph(OpType.GATED_ACT, {"x": x, "up": up}, x.shape, {"act": act, "has_bias": True},
                           {"bias": bias}, order=["x", "bias", "up"])
        _check(g, {"x": x, "up": up}, fn(x.astype(np.float64) + bias) * up, 1e-5)


# ---------------------------------------------------------------- data movement (exact)

def _exact(graph, inputs, ref):
    y = run_gpu(graph, inputs)
    o = run_oracle(graph, inputs)
    np.testing.assert_array_equal(y, ref)
    np.testing.assert_array_equal(o, ref)


@pytest.mark.parametrize("shape,d0,d1", [((1, 64, 4, 16), 1, 2), ((2, 5, 3, 7), 1, 3), ((33, 65), 0, 1),
                                         ((1, 12, 40, 64), 1, 2)])
def test_transpose(shape, d0, d1):
    x = randn(rng(1), *shape)
    ref = np.swapaxes(x, d0, d1)
    g = one_node_graph(OpType.TRANSPOSE, {"x": x}, ref.shape, {"dim0": d0, "dim1": d1})
    _exact(g, {"x": x}, ref)


@pytest.mark.parametrize("shape,dim,start,end", [((1, 32, 192), 2, 64, 128), ((4, 10, 6), 1, 3, 9),
                                                 ((1, 8, 16, 128), 3, 0, 64), ((7, 5), 0, 2, 5), ((3, 9), 1, 1, 2)])
def test_slice(shape, dim, start, end):
    x = randn(rng(2), *shape)
    idx = [slice(None)] * len(shape)
    idx[dim] = slice(start, end)
    ref = x[tuple(idx)]
    attrs = {"dim": dim, "start": start, "end": end}
    if dim == 0:
        attrs["byte_offset"] = start * int(np.prod(shape[1:])) * 4
    g = one_node_graph(OpType.SLICE, {"x": x}, ref.shape, attrs)
    _exact(g, {"x": x}, ref)


def test_slice_int64():
    x = np.arange(60, dtype=np.int64).reshape(3, 20)
    g = one_node_graph(OpType.SLICE, {"x": x}, (3, 5), {"dim": 1, "start": 7, "end": 12}, out_dtype="int64")
    _exact(g, {"x": x}, x[:, 7:12])


@pytest.mark.parametrize("dim", [0, 1, 3])
def test_cat(dim):
    r = rng(dim)
    shapes = [[1, 8, 16, 64], [1, 8, 16, 64], [1, 8, 16, 64]]
    for s, w in zip(shapes, (5, 3, 1)):
        s[dim] = w if dim else s[dim]
    xs = {f"x{i}": randn(r, *s) for i, s in enumerate(shapes)}
    ref = np.concatenate(list(xs.values()), axis=dim)
    g = one_node_graph(OpType.CAT, xs, ref.shape, {"dim": dim})
    _exact(g, xs, ref)


def test_reshape_of_input_copies():
    x = randn(rng(3), 2, 3, 8)
    g = one_node_graph(OpType.RESHAPE, {"x": x}, (6, 8), {"shape": (6, 8)})
    _exact(g, {"x": x}, x.reshape(6, 8))


def test_embedding():
    r = rng(4)
    table = randn(r, 50, 32)
    ids = np.array([[3, 0, 49, 7, 7]], dtype=np.int64)
    g = one_node_graph(OpType.EMBEDDING, {"ids": ids}, (1, 5, 32), {}, {"table": table})
    _exact(g, {"ids": ids}, table[ids])


def test_execute_entry_point(hip_lib):
    """lbr_execute — the drop-in for execute(OpNode*, int) — on a hand-built node array."""
    import ctypes
    from runtime.executor.common import COpNode
    lib = hip_lib
    x = randn(rng(9), 256)
    nbytes = x.nbytes
    dx, dy = lib.alloc(nbytes), lib.alloc(nbytes)
    try:
        lib.h2d(dx, x.ctypes.data, nbytes)
        nodes = (COpNode * 2)()
        nodes[0].op = OpType.NEG.value
        nodes[0].n_inputs = 1
        nodes[0].inputs[0] = dx
        nodes[0].output = dy
        nodes[0].n_dims = 1
        nodes[0].out_shape[0] = 256
        nodes[0].elem_size = 4
        nodes[1] = nodes[0]
        nodes[1].op = OpType.RELU.value
        nodes[1].inputs[0] = dy
        lib.check(lib.lbr_execute(nodes, 2), "lbr_execute")
        y = np.empty_like(x)
        lib.d2h(y.ctypes.data, dy, nbytes)
        np.testing.assert_array_equal(y, np.maximum(-x, 0))
        bad = (COpNode * 1)()
        bad[0].op = OpType.PERMUTE.value
        assert lib.lbr_execute(bad, 1) == 2  # LBR_ERR_UNSUPPORTED, where the reference aborts
        assert "unknown op" in lib.last_error()
    finally:
        lib.free(dx)
        lib.free(dy)
