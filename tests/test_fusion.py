"""Peephole fusion matcher (lbr_fusion_windows) on the CPU: no device is
touched, node pointers are fake addresses that are only compared.

* the runs found on each BASELINE workload's real node stream (planner
  offsets at S=64), and
* every refusal rule on hand-built node arrays: a final output over memory
  the fused kernel reads, an intermediate read later, an intermediate inside
  a live-out range — each built so that the same array without the hazard
  does fuse.
"""

from __future__ import annotations

import ctypes
from collections import Counter

import numpy as np
import pytest

from runtime.executor.common import COpNode
from runtime.executor.hip_lib import open_library
from runtime.ir import OpType

ARENA, EXT = 1 << 40, 1 << 44


def _lib():
    try:
        return open_library()
    except RuntimeError as e:
        pytest.skip(str(e))


def _workload_nodes(key: str, seq: int):
    from runtime.executor.nodes import build_nodes
    from runtime.passes import run_pipeline
    from runtime.planner import plan
    from workloads import export_workload
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
    return arr, order, live


EXPECTED = {
    # merged QKV → three (slice, bias add, transpose) chains in the GEMM epilogue; the O-proj residual
    # add writes over the GEMM's own A input (refused), the FFN2 one fuses
    # FFN1 → GELU runs in the GEMM epilogue; the attention output transpose → O-proj → residual
    # ADD is one GEMM reading the [B,H,S,hd] layout (hd = 16 in the toy block: a 32-wide K step
    # of the O projection covers two whole heads); both LayerNorms run inside the (small) GEMM
    # that reads their output (the heads run and the FFN1 run start at the norm)
    "toy": Counter({("gemm_heads", 11): 1, ("mlp", 5): 1, ("transpose_gemm", 3): 1}),
    "gpt2w": Counter({("gemm_heads", 10): 1, ("gemm_resid", 2): 1, ("gemm_act", 2): 1, ("transpose_gemm", 3): 1}),
    "7b4k": Counter({("gemm_heads", 10): 1, ("gemm_resid", 2): 1, ("gemm_act", 2): 1, ("transpose_gemm", 3): 1}),
    # c_attn is MATMUL_ADD (bias already in the GEMM): three (slice, transpose) chains per layer;
    # c_proj's output lands over the attention output it would read (transpose kept); the
    # attention's output transpose, which the planner puts over the dead V, joins it: this
    # small grid runs the key-quartered kernel, whose flush kernel stores every row after V
    # has been read (deferred store)
    "gpt2": Counter({("gemm_heads", 7): 2, ("gemm_resid", 2): 4, ("gemm_act", 2): 2,
                     ("attn_transpose", 2): 2}),
    # q/k: slice → per-head RMSNorm → transpose → 7-node RoPE as one kernel; v's slice copy
    # stays (its transpose would land over the QKV rows it reads, and the attention output lands
    # over QKV too), while v's transpose, the attention and its output transpose are one kernel
    # reading V from the slice (in the other workloads the planner places the output transpose
    # over the dead V: refused); at S=64 the gated FFN output lands over the gate/up GEMM's
    # input (refused)
    "qwen3_4b": Counter({("head_prologue", 10): 4, ("gemm_resid", 2): 4, ("attn_sliced_v", 3): 2}),
    # at the benchmark length the merged gate/up GEMM → two half slices → SiLU gate is one GEMM,
    # and the attention takes the key-range split, whose merge kernel writes every output row
    # after all of Q, K and V have been read: v's slice joins the attention run although the
    # output lands over the QKV rows
    "qwen3_4b@1024": Counter({("head_prologue", 10): 4, ("gemm_resid", 2): 4, ("attn_sliced_v", 4): 2,
                              ("gemm_gated", 4): 2}),
    # likewise the output transpose over the dead V at the benchmark length
    "gpt2@1024": Counter({("gemm_heads", 7): 2, ("gemm_resid", 2): 4, ("gemm_act", 2): 2,
                          ("attn_transpose", 2): 2}),
    # ... but where the transpose can go into the O projection instead, that is taken
    "gpt2w@512": Counter({("gemm_heads", 10): 1, ("gemm_resid", 2): 1, ("gemm_act", 2): 1,
                          ("transpose_gemm", 3): 1}),
}


@pytest.mark.parametrize("key", list(EXPECTED))
def test_workload_fusion_windows(key):
    lib = _lib()
    name, _, seq = key.partition("@")
    arr, order, live = _workload_nodes(name, int(seq) if seq else 64)
    wins = lib.fusion_windows(arr, len(order), live)
    assert Counter((kind, count) for _, count, kind in wins) == EXPECTED[key]
    # runs are disjoint, in order, inside the array
    end = 0
    for first, count, _ in wins:
        assert first >= end and first + count <= len(order)
        end = first + count
    # no live-out declared → intermediates that are graph outputs are unknown; with an
    # explicit empty list fusion still runs (the caller asserts nothing is read back)
    assert len(lib.fusion_windows(arr, len(order), [])) >= len(wins)


# ------------------------------------------------------------ hand-built arrays

def _node(op, inputs, output, shape, extra=()):
    n = COpNode()
    n.op = op.value
    n.n_inputs = len(inputs)
    for i, p in enumerate(inputs):
        n.inputs[i] = p
    n.output = output
    n.n_dims = len(shape)
    for i, d in enumerate(shape):
        n.out_shape[i] = d
    n.elem_size = 4
    for i, e in enumerate(extra):
        n.extra[i] = e
    return n


def _array(nodes):
    arr = (COpNode * len(nodes))()
    for i, n in enumerate(nodes):
        arr[i] = n
    return arr


M, K, N = 256, 128, 384          # GEMM rows, depth, columns
A_, W_, R_ = EXT, EXT + (1 << 32), EXT + (2 << 32)
MB = 1 << 20


def _gemm_resid(c_off, y_off, a_ptr=A_, later=()):
    """MATMUL A·Wᵀ → C, ADD(C, R) → Y, then `later` nodes."""
    mm = _node(OpType.MATMUL, [a_ptr, W_], ARENA + c_off, (1, M, N), (K, 1, 1, 0))
    ad = _node(OpType.ADD, [ARENA + c_off, R_], ARENA + y_off, (1, M, N), (1,))
    return [mm, ad, *later]


def _windows(nodes, live=()):
    lib = _lib()
    arr = _array(nodes)
    return lib.fusion_windows(arr, len(nodes), list(live))


def test_gemm_resid_fuses():
    assert _windows(_gemm_resid(0, 4 * MB)) == [(0, 2, "gemm_resid")]
    # Y over the dead C is fine: C is never written
    assert _windows(_gemm_resid(0, 0)) == [(0, 2, "gemm_resid")]


def test_gemm_resid_refuses_output_over_gemm_input():
    # the GEMM reads A while other workgroups would already write Y over it
    assert _windows(_gemm_resid(0, 4 * MB, a_ptr=ARENA + 4 * MB)) == []


def test_gemm_resid_refuses_live_intermediate():
    c_off = 0
    reader = _node(OpType.RELU, [ARENA + c_off + 64], ARENA + 16 * MB, (16,))
    assert _windows(_gemm_resid(c_off, 4 * MB, later=[reader])) == []
    # ... unless the memory was overwritten before that read
    writer = _node(OpType.RELU, [R_], ARENA + c_off, (1, M, N))
    assert _windows(_gemm_resid(c_off, 4 * MB, later=[writer, reader])) == [(0, 2, "gemm_resid")]


def test_gemm_resid_refuses_intermediate_read_from_below():
    # a later input that starts below C and extends over it still reads C's values: the
    # liveness walk compares each input's read extent, not just its first byte
    c_off = 64 * MB
    reader = _node(OpType.RELU, [ARENA + c_off - 4096], ARENA + 16 * MB, (MB // 4,))
    assert _windows(_gemm_resid(c_off, 4 * MB, later=[reader])) == []
    # ... the same read ending where C begins does not
    short = _node(OpType.RELU, [ARENA + c_off - 4096], ARENA + 16 * MB, (1024,))
    assert _windows(_gemm_resid(c_off, 4 * MB, later=[short])) == [(0, 2, "gemm_resid")]
    # a broadcast operand's extent follows its strides: a [M, N] read of a row-broadcast
    # tensor spans N elements only, so one starting 4 KiB below C ends before it ...
    bc = [2, 2, N, 1, 0, 1, M, N]   # mode 2 (broadcast), ndim 2, a strides, b strides, shape
    brd = _node(OpType.MUL, [R_, ARENA + c_off - 4096], ARENA + 16 * MB, (M, N), bc)
    assert _windows(_gemm_resid(c_off, 4 * MB, later=[brd])) == [(0, 2, "gemm_resid")]
    # ... while a full-stride one reaches into it
    full = _node(OpType.MUL, [R_, ARENA + c_off - 4096], ARENA + 16 * MB, (M, N), [2, 2, N, 1, N, 1, M, N])
    assert _windows(_gemm_resid(c_off, 4 * MB, later=[full])) == []


def test_gemm_resid_refuses_intermediate_in_live_out():
    nodes = _gemm_resid(0, 4 * MB)
    assert _windows(nodes, live=[(ARENA + 8, 4)]) == []
    assert _windows(nodes, live=[(ARENA + 4 * MB, M * N * 4)]) == [(0, 2, "gemm_resid")]


def _qkv(c_off, outs, heads=(4, 4, 4), hd=32, S=M, bias=True):
    """MATMUL → C [1,S,Σ heads·hd]; per split: SLICE → [ADD bias] → TRANSPOSE(S,H)."""
    width = [h * hd for h in heads]
    ncol = sum(width)
    nodes = [_node(OpType.MATMUL, [A_, W_], ARENA + c_off, (1, S, ncol), (K, 1, 1, 0))]
    col = 0
    for k, (h, w) in enumerate(zip(heads, width)):
        tmp = ARENA + 32 * MB + k * MB
        nodes.append(_node(OpType.SLICE, [ARENA + c_off], tmp, (1, S, w), (S, ncol, col, w, 1)))
        src = tmp
        if bias:
            nodes.append(_node(OpType.ADD, [tmp, EXT + (3 + k << 32)], tmp, (1, S, w), (0,)))
        nodes.append(_node(OpType.TRANSPOSE, [src], ARENA + outs[k], (1, h, S, hd), (1, S, 1, h, hd)))
        col += w
    return nodes


def test_gemm_heads_fuses_with_gqa_splits():
    nodes = _qkv(0, [8 * MB, 9 * MB, 10 * MB], heads=(8, 2, 2))
    assert _windows(nodes) == [(0, 10, "gemm_heads")]
    # an output inside the dead C is fine for the epilogue form (C is never written)
    nodes = _qkv(0, [8 * MB, 9 * MB, 0], heads=(8, 2, 2), bias=False)
    assert _windows(nodes) == [(0, 7, "gemm_heads")]


def test_gemm_heads_refuses_when_C_is_read_later():
    nodes = _qkv(0, [8 * MB, 9 * MB, 10 * MB])
    nodes.append(_node(OpType.RELU, [ARENA + 4], ARENA + 40 * MB, (8,)))
    wins = _windows(nodes)
    assert all(kind != "gemm_heads" for _, _, kind in wins)


def _rope_chain(src_off, out_off, S=64, H=4, hd=128, norm=True, rope=True):
    """SLICE(C) → [RMSNORM] → TRANSPOSE → [RoPE 7 nodes] over C [1, S, H·hd + 64]."""
    ld = H * hd + 64
    C = ARENA + src_off
    t = [ARENA + 40 * MB + k * MB for k in range(12)]
    nodes = [_node(OpType.SLICE, [C], t[0], (1, S, H * hd), (S, ld, 0, H * hd, 1))]
    cur = t[0]
    if norm:
        nodes.append(_node(OpType.RMSNORM, [cur, EXT + (5 << 32)], t[1], (1, S, H, hd), (0x358637BD,)))
        cur = t[1]
    nodes.append(_node(OpType.TRANSPOSE, [cur], t[2] if rope else ARENA + out_off, (1, H, S, hd),
                       (1, S, 1, H, hd)))
    if not rope:
        return nodes
    x = t[2]
    cos, sin = EXT + (6 << 32), EXT + (7 << 32)
    half = hd // 2
    bc = (2, 4, 0, S * hd, hd, 1, 0, 0, hd, 1, 1, H, S, hd)
    rows = H * S
    nodes += [
        _node(OpType.MUL, [x, cos], t[3], (1, H, S, hd), bc),
        _node(OpType.SLICE, [x], t[4], (1, H, S, half), (rows, hd, 0, half, 1)),
        _node(OpType.SLICE, [x], t[5], (1, H, S, half), (rows, hd, half, half, 1)),
        _node(OpType.NEG, [t[5]], t[5], (1, H, S, half)),
        _node(OpType.CAT, [t[5], t[4]], t[6], (1, H, S, hd), (3, half, half)),
        _node(OpType.MUL, [t[6], sin], t[6], (1, H, S, hd), bc),
        _node(OpType.ADD, [t[3], t[6]], ARENA + out_off, (1, H, S, hd), (1,)),
    ]
    return nodes


def test_head_prologue_fuses_norm_and_rope():
    assert _windows(_rope_chain(0, 8 * MB)) == [(0, 10, "head_prologue")]
    assert _windows(_rope_chain(0, 8 * MB, norm=False)) == [(0, 9, "head_prologue")]
    assert _windows(_rope_chain(0, 8 * MB, rope=False)) == [(0, 3, "head_prologue")]


def test_head_prologue_refuses_output_over_its_source():
    # out overlaps the rows of C the kernel reads (different index map)
    assert _windows(_rope_chain(0, 4096)) == []


def test_head_prologue_refuses_when_an_intermediate_is_read():
    nodes = _rope_chain(0, 8 * MB)
    # a later reader of the transposed (pre-RoPE) tensor keeps it live
    nodes.append(_node(OpType.RELU, [ARENA + 42 * MB], ARENA + 60 * MB, (8,)))
    assert _windows(nodes) == []


def test_rope_tables_take_any_broadcast_strides():
    # a sin table that also varies along heads is still RoPE: the kernel indexes it by strides
    nodes = _rope_chain(0, 8 * MB)
    nodes[8].extra[7] = 64 * 128
    assert _windows(nodes) == [(0, 10, "head_prologue")]


def test_not_rotate_half_is_not_rope():
    # cat(x1, −x2) is not rotate_half: the chain stops at the transpose
    nodes = _rope_chain(0, 8 * MB)
    nodes[7].inputs[0], nodes[7].inputs[1] = nodes[7].inputs[1], nodes[7].inputs[0]
    assert _windows(nodes) == [(0, 3, "head_prologue")]


def _attn_transpose(out_off, v_off=20 * MB, B=1, H=4, S=128, hd=64, q_off=16 * MB, k_off=18 * MB,
                    att_off=24 * MB):
    q, k, v = ARENA + q_off, ARENA + k_off, ARENA + v_off
    att = _node(OpType.ATTENTION, [q, k, v, ARENA + 30 * MB], ARENA + att_off, (B, H, S, hd), (S, hd, 1, 0, 1))
    att.n_inputs = 4          # Q, K, V + the planner's scratch slot
    tr = _node(OpType.TRANSPOSE, [ARENA + att_off], ARENA + out_off, (B, S, H, hd), (B, H, 1, S, hd))
    return [att, tr]


def test_attention_transpose_fuses():
    assert _windows(_attn_transpose(26 * MB)) == [(0, 2, "attn_transpose")]
    # the dead attention output's own memory is fine
    assert _windows(_attn_transpose(24 * MB)) == [(0, 2, "attn_transpose")]


def test_attention_transpose_refuses_misaligned_output():
    # the fused kernel stores the transposed rows as float4s: a planner offset that is not
    # 16-byte aligned keeps the two nodes apart
    assert _windows(_attn_transpose(26 * MB + 4)) == []
    assert _windows(_attn_transpose(26 * MB + 16)) == [(0, 2, "attn_transpose")]
    # with V read from the source rows, the attention still joins but its output transpose does not
    assert _windows(_sliced_v(0, 24 * MB, 26 * MB + 8)) == [(0, 2, "attn_sliced_v")]


def _no_deferred_store(monkeypatch):
    """Attention schedules without a deferred store: no key-range split."""
    monkeypatch.setenv("LBR_ATTN_SPLIT", "0")


def test_attention_transpose_output_over_v(monkeypatch):
    # 4 heads × S 128 take the key-range split, whose merge kernel stores every output row after
    # the attention kernel has read V: the output may lie over V (deferred store)
    assert _windows(_attn_transpose(20 * MB)) == [(0, 2, "attn_transpose")]
    # the same grid without the split: the planner may reuse V's memory once attention is done,
    # but one fused kernel still reads V
    _no_deferred_store(monkeypatch)
    assert _windows(_attn_transpose(20 * MB)) == []
    assert _windows(_attn_transpose(26 * MB)) == [(0, 2, "attn_transpose")]


def test_tiny_attention_grid_takes_no_split():
    # head dim 48 (no key-quartered form): 4 heads × S 128 hold 4 key tiles a block, too few
    # for the key-range split to pay for its merge launch, so there is no deferred store and
    # an output over V is refused; at S 256 (8 tiles a block) the split, and the fusion, return
    assert _windows(_attn_transpose(20 * MB, hd=48)) == []
    assert _windows(_attn_transpose(26 * MB, hd=48)) == [(0, 2, "attn_transpose")]
    assert _windows(_attn_transpose(20 * MB, S=256, hd=48)) == [(0, 2, "attn_transpose")]


def test_attention_transpose_refuses_output_over_v_on_a_full_grid():
    # 32 heads × S 4096 × hd 128 fill the CUs with folded query blocks: no split, no deferred
    # store, so an output over V is refused while one elsewhere fuses
    big = dict(H=32, S=4096, hd=128, q_off=0, k_off=64 * MB, v_off=128 * MB, att_off=192 * MB)
    assert _windows(_attn_transpose(256 * MB, **big)) == [(0, 2, "attn_transpose")]
    assert _windows(_attn_transpose(128 * MB, **big)) == []
    assert _windows(_attn_transpose(160 * MB, **big)) == []


def _split_attn_transpose(out_off, H=12, S=1024, hd=64, later=()):
    """A causal attention small enough to take the key-range split (12 heads × 8 query blocks
    of 128 rows on 256 CUs) → output TRANSPOSE(H,S) at out_off; Q, K, V at 16, 24, 32 MB."""
    q, k, v = ARENA + 16 * MB, ARENA + 24 * MB, ARENA + 32 * MB
    att = _node(OpType.ATTENTION, [q, k, v, ARENA + 60 * MB], ARENA + 40 * MB, (1, H, S, hd), (S, hd, 1, 0, 1))
    att.n_inputs = 4
    tr = _node(OpType.TRANSPOSE, [ARENA + 40 * MB], ARENA + out_off, (1, S, H, hd), (1, H, 1, S, hd))
    return [att, tr, *later]


def test_split_attention_transpose_may_write_over_its_inputs():
    # the split's merge kernel writes every row once the split kernel has read Q, K and V
    for off in (16, 24, 32):
        assert _windows(_split_attn_transpose(off * MB)) == [(0, 2, "attn_transpose")]
    # ... unless a GEMM right after takes the transpose (reading the head layout): that
    # costs no extra pass over the rows
    w = _node(OpType.MATMUL, [ARENA + 32 * MB, W_], ARENA + 48 * MB, (1, 1024, 256), (768, 1, 1, 0))
    assert _windows(_split_attn_transpose(32 * MB, later=[w])) == [(1, 2, "transpose_gemm")]


def test_attention_transpose_needs_the_16x16_kernel():
    # head dim 256 runs the 32x32 kernel, which writes [bh, S, hd] only
    assert _windows(_attn_transpose(40 * MB, hd=256)) == []


def _sliced_v(v_src_off, att_off, out_off, sliced=False, hd=64, later=()):
    """[SLICE of the V columns of [S, 3·Hkv·hd] rows at v_src_off →] TRANSPOSE(S,H) → V of a GQA
    ATTENTION (8 query heads, 2 K/V heads) → output TRANSPOSE(H,S) at out_off, then `later`."""
    B, H, Hkv, S = 1, 8, 2, 128
    nodes = []
    t_in = ARENA + v_src_off
    if sliced:
        ld = 3 * Hkv * hd
        nodes.append(_node(OpType.SLICE, [t_in], ARENA + 40 * MB, (B, S, Hkv * hd),
                           (B * S, ld, 2 * Hkv * hd, Hkv * hd, 1)))
        t_in = ARENA + 40 * MB
    tv = _node(OpType.TRANSPOSE, [t_in], ARENA + 44 * MB, (B, Hkv, S, hd), (B, S, 1, Hkv, hd))
    att = _node(OpType.ATTENTION, [ARENA + 16 * MB, ARENA + 18 * MB, ARENA + 44 * MB, ARENA + 30 * MB],
                ARENA + att_off, (B, H, S, hd), (S, hd, 1, 0, H // Hkv))
    tr = _node(OpType.TRANSPOSE, [ARENA + att_off], ARENA + out_off, (B, S, H, hd), (B, H, 1, S, hd))
    return nodes + [tv, att, tr, *later]


def test_attention_sliced_v_fuses():
    # V's transpose, the attention and its output transpose: the kernel reads V from the
    # transpose's [B, S, Hkv·hd] input
    assert _windows(_sliced_v(0, 24 * MB, 26 * MB)) == [(0, 3, "attn_sliced_v")]
    # from the slice's source rows (its columns 2·Hkv·hd ..), without the slice copy
    assert _windows(_sliced_v(0, 24 * MB, 26 * MB, sliced=True)) == [(0, 4, "attn_sliced_v")]


def test_attention_sliced_v_refusals(monkeypatch):
    # the attention output over the rows V is read from is fine while the output transpose
    # joins the run (the fused kernel never writes it)
    assert _windows(_sliced_v(24 * MB, 24 * MB, 26 * MB)) == [(0, 3, "attn_sliced_v")]
    # 8 heads × S 128 take the key-range split (deferred store): the final output may land over
    # V's source rows, and so may the output transpose
    assert _windows(_sliced_v(24 * MB, 24 * MB, 24 * MB)) == [(0, 3, "attn_sliced_v")]
    assert _windows(_sliced_v(26 * MB, 24 * MB, 26 * MB)) == [(0, 3, "attn_sliced_v")]
    # without the split: the final output over V's source leaves the plain output transpose
    # fusion only, and the output transpose over V's source stays out of the run
    _no_deferred_store(monkeypatch)
    assert _windows(_sliced_v(24 * MB, 24 * MB, 26 * MB)) == [(0, 3, "attn_sliced_v")]
    assert _windows(_sliced_v(24 * MB, 24 * MB, 24 * MB)) == [(1, 2, "attn_transpose")]
    assert _windows(_sliced_v(26 * MB, 24 * MB, 26 * MB)) == [(0, 2, "attn_sliced_v")]
    monkeypatch.delenv("LBR_ATTN_SPLIT")
    # the transposed V read again later: it must be written
    reader = _node(OpType.RELU, [ARENA + 44 * MB], ARENA + 50 * MB, (1, 2, 128, 64))
    assert _windows(_sliced_v(0, 24 * MB, 26 * MB, later=[reader])) == [(1, 2, "attn_transpose")]
    # head dim 256 runs the 32x32 kernel, which reads V as [bh, S, hd] only
    assert _windows(_sliced_v(0, 24 * MB, 26 * MB, hd=256)) == []


# ------------------------------------------------------------ activation epilogues

def _gemm_act(c_off, y_off, a_ptr=A_, op=OpType.GELU, k=K, later=()):
    """MATMUL A·Wᵀ → C, activation(C) → Y, then `later` nodes."""
    mm = _node(OpType.MATMUL, [a_ptr, W_], ARENA + c_off, (1, M, N), (k, 1, 1, 0))
    ac = _node(op, [ARENA + c_off], ARENA + y_off, (1, M, N))
    return [mm, ac, *later]


def test_gemm_act_fuses():
    for op in (OpType.RELU, OpType.GELU, OpType.SILU):
        assert _windows(_gemm_act(0, 4 * MB, op=op)) == [(0, 2, "gemm_act")]
    # in place over the dead C
    assert _windows(_gemm_act(0, 0)) == [(0, 2, "gemm_act")]
    # only RELU, GELU and SILU have an epilogue form
    assert _windows(_gemm_act(0, 4 * MB, op=OpType.TANH)) == []


def test_gemm_act_refusals():
    # Y over the GEMM's A input
    assert _windows(_gemm_act(0, 4 * MB, a_ptr=ARENA + 4 * MB)) == []
    # C read by a later node, or C a graph output
    reader = _node(OpType.RELU, [ARENA + 64], ARENA + 16 * MB, (16,))
    assert _windows(_gemm_act(0, 4 * MB, later=[reader])) == []
    assert _windows(_gemm_act(0, 4 * MB), live=[(ARENA, 4)]) == []
    # K % 32 != 0 keeps the register-staged kernel, which has no activation epilogue
    assert _windows(_gemm_act(0, 4 * MB, k=K + 4)) == []


F = 192   # gated pair: output columns


def _gated(y_off, order=(0, 1), a_ptr=A_, bias=False, act=0, later=(), halves=(0, F)):
    """MATMUL → C [1, M, 2F]; SLICE(C) at columns halves[0] and halves[1]; GATED_ACT(x, [b], up)
    with x, up the slices picked by `order`."""
    C = ARENA
    mm = _node(OpType.MATMUL, [a_ptr, W_], C, (1, M, 2 * F), (K, 1, 1, 0))
    s = [_node(OpType.SLICE, [C], ARENA + (8 + k) * MB, (1, M, F), (M, 2 * F, halves[k], F, 1)) for k in (0, 1)]
    x, up = s[order[0]].output, s[order[1]].output
    ins = [x, EXT + (6 << 32), up] if bias else [x, up]
    ga = _node(OpType.GATED_ACT, ins, ARENA + y_off, (1, M, F), (int(bias), act))
    return [mm, s[0], s[1], ga, *later]


def test_gemm_gated_fuses():
    assert _windows(_gated(16 * MB)) == [(0, 4, "gemm_gated")]
    # the gate is the upper half
    assert _windows(_gated(16 * MB, order=(1, 0))) == [(0, 4, "gemm_gated")]
    assert _windows(_gated(16 * MB, bias=True, act=1)) == [(0, 4, "gemm_gated")]
    # output over the dead C and slices
    assert _windows(_gated(0)) == [(0, 4, "gemm_gated")]


def test_gemm_gated_refusals():
    # output over the GEMM's A input (the Qwen3 LM plan places it there)
    assert _windows(_gated(16 * MB, a_ptr=ARENA + 16 * MB)) == []
    # a slice read by a later node, or a graph output
    reader = _node(OpType.RELU, [ARENA + 8 * MB], ARENA + 40 * MB, (16,))
    assert _windows(_gated(16 * MB, later=[reader])) == []
    assert _windows(_gated(16 * MB), live=[(ARENA + 9 * MB, 4)]) == []
    # slices that are not the two halves of C
    assert _windows(_gated(16 * MB, halves=(0, 64))) == []
    # output over the gated bias
    nodes = _gated(16 * MB, bias=True)
    nodes[3].inputs[1] = ARENA + 16 * MB + 64
    assert _windows(nodes) == []


# ------------------------------------------------------------ transpose → GEMM

TB, TH, TS, THD = 1, 4, 64, 32      # attention output [B, H, S, hd] → [B, S, H·hd] for the GEMM
TK = TH * THD


def _tgemm(o_off, t_off, c_off, y_off=None, hd=THD, later=()):
    """O [B,H,S,hd] → TRANSPOSE(H,S) → T; MATMUL T·Wᵀ → C [B·S, N]; [ADD(C, R) → Y]."""
    heads = TK // hd
    tr = _node(OpType.TRANSPOSE, [ARENA + o_off], ARENA + t_off, (TB, TS, heads, hd), (TB, heads, 1, TS, hd))
    mm = _node(OpType.MATMUL, [ARENA + t_off, W_], ARENA + c_off, (TB, TS, N), (TK, 1, 1, 0))
    nodes = [tr, mm]
    if y_off is not None:
        nodes.append(_node(OpType.ADD, [ARENA + c_off, R_], ARENA + y_off, (TB, TS, N), (1,)))
    return [*nodes, *later]


def test_transpose_gemm_fuses():
    assert _windows(_tgemm(0, 1 * MB, 2 * MB, 3 * MB)) == [(0, 3, "transpose_gemm")]
    assert _windows(_tgemm(0, 1 * MB, 2 * MB)) == [(0, 2, "transpose_gemm")]
    # C or Y over the dead transposed copy T is fine: T is never written
    assert _windows(_tgemm(0, 1 * MB, 1 * MB, 1 * MB)) == [(0, 3, "transpose_gemm")]


def test_transpose_gemm_refusals():
    # the GEMM's output over the attention output it now reads (GPT-2's c_proj): with no
    # residual ADD, C is that output; with one, Y is (C itself is never written)
    assert _windows(_tgemm(0, 1 * MB, 0)) == []
    assert _windows(_tgemm(0, 1 * MB, 0, 3 * MB)) == [(0, 3, "transpose_gemm")]
    # Y over O: the residual ADD stays a node of its own, the transpose is still absorbed
    assert _windows(_tgemm(0, 1 * MB, 2 * MB, 0)) == [(0, 2, "transpose_gemm")]
    # head dim 2: a lane's 4-float chunk of the K step would straddle two heads; 16
    # divides the 32-wide step (two whole heads per step)
    assert _windows(_tgemm(0, 1 * MB, 2 * MB, hd=2)) == []
    assert _windows(_tgemm(0, 1 * MB, 2 * MB, hd=16)) == [(0, 2, "transpose_gemm")]
    # T read by a later node
    reader = _node(OpType.RELU, [ARENA + 1 * MB], ARENA + 8 * MB, (16,))
    assert all(k != "transpose_gemm" for _, _, k in _windows(_tgemm(0, 1 * MB, 2 * MB, 3 * MB, later=[reader])))


def test_transpose_gemm_needs_a_head_layout_tile(monkeypatch):
    """The 64-wide-K-step tiles have no head-layout form: a GEMM forced onto one keeps
    its TRANSPOSE as a node of its own (instead of a fused step with no kernel)."""
    monkeypatch.setenv("LBR_GEMM_TILE", "32x96k64")
    assert _windows(_tgemm(0, 1 * MB, 2 * MB, 3 * MB)) == [(1, 2, "gemm_resid")]   # GEMM + ADD only
    monkeypatch.setenv("LBR_GEMM_TILE", "32x96")
    assert _windows(_tgemm(0, 1 * MB, 2 * MB, 3 * MB)) == [(0, 3, "transpose_gemm")]


# ------------------------------------------------------------ index arithmetic

def test_fast_divisor_matches_integer_division():
    """The attention key-range split and the head prologue divide by a multiply and a shift (x < 2^31):
    the host computation of the same (m, s) against plain division on every
    divisor up to 4096 with the dividends at each multiple's edges, on divisors
    around powers of two, and on random pairs."""
    f = _lib().lbr_fast_div
    r = np.random.default_rng(11)
    top = (1 << 31) - 1
    divisors = list(range(1, 4097)) + [(1 << k) + e for k in range(12, 31) for e in (-1, 0, 1)] + [top]
    for d in divisors:
        q_hi = top // d
        xs = {0, 1, d - 1, d, d + 1, top, top - 1, q_hi * d, q_hi * d - 1}
        xs |= {int(v) for v in r.integers(0, top, 4)}
        for x in xs:
            if 0 <= x <= top:
                assert f(x, d) == x // d, (x, d)
    for x, d in zip(r.integers(0, top, 20000), r.integers(1, top, 20000)):
        assert f(int(x), int(d)) == int(x) // int(d)


# ------------------------------------------------------------ norm prologue

def _norm_gemm(rms=False, K=128, M=256, N=384, x=EXT + (5 << 32), ln_off=0, c_off=MB, later=()):
    """RMSNORM | LAYERNORM(x) → n, MATMUL(n, W) → C, then `later` nodes."""
    eps = int(np.float32(1e-5).view(np.int32))
    ins = [x, EXT + (6 << 32)] if rms else [x, EXT + (6 << 32), EXT + (7 << 32)]
    nm = _node(OpType.RMSNORM if rms else OpType.LAYERNORM, ins, ARENA + ln_off, (M, K), (eps,))
    mm = _node(OpType.MATMUL, [ARENA + ln_off, W_], ARENA + c_off, (1, M, N), (K, 1, 1, 0))
    return [nm, mm, *later]


def test_norm_prologue_fuses_layer_and_rms_norms():
    assert _windows(_norm_gemm()) == [(0, 2, "norm_gemm")]
    assert _windows(_norm_gemm(rms=True)) == [(0, 2, "norm_gemm")]
    # a GEMM epilogue run takes the norm at its head
    act = _node(OpType.GELU, [ARENA + MB], ARENA + 2 * MB, (1, 256, 384))
    assert _windows(_norm_gemm(later=[act])) == [(0, 3, "gemm_act")]


def test_norm_prologue_refusals():
    # the norm's output is read again later
    reader = _node(OpType.RELU, [ARENA + 64], ARENA + 4 * MB, (16,))
    assert _windows(_norm_gemm(later=[reader])) == []
    # the GEMM's output lands on the norm's input, which the GEMM reads to the end
    assert _windows(_norm_gemm(x=ARENA + 2 * MB, c_off=2 * MB)) == []
    # misaligned input rows for the DMA loads
    assert _windows(_norm_gemm(x=EXT + (5 << 32) + 4)) == []
    # the norm's output is a declared live-out
    assert _windows(_norm_gemm(), live=[(ARENA, 256 * 128 * 4)]) == []


# ---------------------------------------------------------------- MLP

def _mlp(M=32, D=64, H=256, norm="layer", resid=True, act=OpType.GELU, y_off=None, x=EXT + (8 << 32), later=()):
    """[norm(x) → n,] n·W1ᵀ + b1 → c1, act → h, h·W2ᵀ + b2 → c2, [ADD(x, c2) → y], then `later`."""
    W1, B1, W2, B2 = (EXT + (k << 32) for k in (9, 10, 11, 12))
    eps = int(np.float32(1e-5).view(np.int32))
    nodes = []
    a = x
    if norm:
        ins = [x, EXT + (6 << 32)] if norm == "rms" else [x, EXT + (6 << 32), EXT + (7 << 32)]
        nodes.append(_node(OpType.RMSNORM if norm == "rms" else OpType.LAYERNORM, ins, ARENA, (1, M, D), (eps,)))
        a = ARENA
    nodes.append(_node(OpType.MATMUL_ADD, [a, W1, B1], ARENA + MB, (1, M, H), (D, 1, 1, 0)))
    nodes.append(_node(act, [ARENA + MB], ARENA + 2 * MB, (1, M, H)))
    nodes.append(_node(OpType.MATMUL_ADD, [ARENA + 2 * MB, W2, B2], ARENA + 3 * MB, (1, M, D), (H, 1, 1, 0)))
    if resid:
        nodes.append(_node(OpType.ADD, [x, ARENA + 3 * MB], ARENA + (y_off if y_off is not None else 4 * MB),
                           (1, M, D), (1,)))
    return nodes + list(later)


def test_mlp_fuses(monkeypatch):
    assert _windows(_mlp()) == [(0, 5, "mlp")]
    assert _windows(_mlp(norm="rms", act=OpType.SILU)) == [(0, 5, "mlp")]
    assert _windows(_mlp(norm=None)) == [(0, 4, "mlp")]
    assert _windows(_mlp(resid=False)) == [(0, 4, "mlp")]
    # the output written row for row over the norm's input (the residual)
    assert _windows(_mlp(x=ARENA + 8 * MB, y_off=8 * MB)) == [(0, 5, "mlp")]
    monkeypatch.setenv("LBR_MLP_FUSE", "0")
    assert "mlp" not in {k for _, _, k in _windows(_mlp())}


def test_mlp_refusals():
    # hidden rows too wide for LDS ((D + H + 8) · 64 B > 64 KiB)
    assert "mlp" not in {k for _, _, k in _windows(_mlp(D=256, H=1024))}
    # too much work for one launch-bound kernel (2·M·(H·D + D·H) > 2^25)
    assert "mlp" not in {k for _, _, k in _windows(_mlp(M=2048))}
    # widths not multiples of 16
    assert "mlp" not in {k for _, _, k in _windows(_mlp(D=72, H=256))}
    # the hidden activation is read again later
    reader = _node(OpType.RELU, [ARENA + 2 * MB], ARENA + 9 * MB, (1, 32, 256))
    assert "mlp" not in {k for _, _, k in _windows(_mlp(later=[reader]))}
    # the output partly over the norm's input (other rows than its own)
    assert "mlp" not in {k for _, _, k in _windows(_mlp(x=ARENA + 8 * MB, y_off=8 * MB + 256))}
    # the norm's output is a declared live-out: the MLP runs without it
    assert _windows(_mlp(), live=[(ARENA, 32 * 64 * 4)]) == [(1, 4, "mlp")]
