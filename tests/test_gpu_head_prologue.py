"""The fused head prologue (SLICE → [bias] → RMSNorm → TRANSPOSE → RoPE as one
kernel) on Qwen3-style attention layers of head dim 64, 128 and 256, with and
without q/k/v biases, in both kernel forms: the float4 one (hd/4 lanes per
row, R rows a lane; the Q and K prologues joined into one launch, and apart)
and the one-wavefront-per-row one kept for unaligned rows.

Each case runs the fused plan against the one-kernel-per-node plan of the
same graph (equal up to the RMSNorm sum order: normwise 1e-5) and against
float64 PyTorch (1e-3).
"""

import copy

import numpy as np
import pytest
import torch

from conftest import normwise_rel

pytestmark = pytest.mark.gpu


class _Layer(torch.nn.Module):
    def __init__(self, hd, bias):
        super().__init__()
        from transformers import Qwen3Config
        from transformers.models.qwen3 import modeling_qwen3 as mq
        cfg = Qwen3Config(hidden_size=4 * hd, intermediate_size=256, num_hidden_layers=1, num_attention_heads=4,
                          num_key_value_heads=2, head_dim=hd, rms_norm_eps=1e-6, vocab_size=16,
                          max_position_embeddings=256, attention_bias=bias,
                          rope_parameters={"rope_type": "default", "rope_theta": 1e6})
        cfg._attn_implementation = "sdpa"
        self.layer = mq.Qwen3DecoderLayer(cfg, 0)
        self.rot = mq.Qwen3RotaryEmbedding(cfg)

    def forward(self, x):
        pos = torch.arange(x.shape[1]).unsqueeze(0)
        out = self.layer(x, attention_mask=None, position_ids=pos, position_embeddings=self.rot(x, pos))
        return out[0] if isinstance(out, tuple) else out


@pytest.mark.parametrize("kernel", ["vec", "vec-unmerged", "scalar"])
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("hd", [64, 128, 256])
def test_head_prologue_forms(monkeypatch, hd, bias, kernel):
    from runtime.exporter import export_model
    from runtime.session import Session
    from workloads import init_weights, reference_forward
    monkeypatch.setenv("LBR_QKV_EPILOGUE", "0")   # the prologue kernels themselves (hd 128 joins the GEMM)
    m = init_weights(_Layer(hd, bias), seed=hd + bias)
    if bias:   # non-zero biases, so the bias add is exercised
        with torch.no_grad():
            for name, p in m.named_parameters():
                if name.endswith("bias"):
                    p.normal_(0.0, 0.5)
    x = np.random.default_rng(hd).standard_normal((1, 48, 4 * hd)).astype(np.float32)
    g = export_model(m, (torch.from_numpy(x),))
    g2 = copy.deepcopy(g)
    if kernel == "scalar":
        monkeypatch.setenv("LBR_HEAD_PROLOGUE", "scalar")
    if kernel == "vec-unmerged":
        monkeypatch.setenv("LBR_HEAD_MERGE", "0")
    fused = Session(g)
    fused.create()
    heads = [s for s in fused.executor.step_params() if s["kind"] == "head_prologue"]
    if kernel == "vec":   # q and k in one launch
        assert len(heads) == 1 and heads[0]["vec"] and heads[0]["parts"] == 2, heads
    else:                 # q and k launched apart
        assert len(heads) == 2 and all(s["vec"] == (kernel != "scalar") and s["parts"] == 1 for s in heads), heads
    y = fused.run({g.inputs[0]: x})[g.outputs[0]]
    fused.close()
    monkeypatch.setenv("LBR_FUSE", "0")
    plain = Session(g2)
    plain.create()
    z = plain.run({g2.inputs[0]: x})[g2.outputs[0]]
    plain.close()
    ref = reference_forward(m, x)
    e_fz, e_ref = normwise_rel(y, z), normwise_rel(y, ref)
    print(f"hd={hd} bias={bias} {kernel}: fused-vs-unfused {e_fz:.2e}, vs torch64 {e_ref:.2e}")
    assert np.isfinite(y).all()
    assert e_fz <= 1e-5
    assert e_ref <= 1e-3


def _rotate_half(x):   # written as transformers' Qwen3 does, so the export gives the same node chain
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


class _PerHeadTables(torch.nn.Module):
    """Q and K prologues whose RoPE tables vary over heads ([1, H, S, hd], broadcast
    over the batch): the float4 kernel's per-head table loads."""

    def __init__(self, H, hd, S):
        super().__init__()
        from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm
        self.H, self.hd = H, hd
        self.qp = torch.nn.Linear(2 * H * hd, H * hd, bias=False)
        self.kp = torch.nn.Linear(2 * H * hd, H * hd, bias=False)
        self.vp = torch.nn.Linear(2 * H * hd, H * hd, bias=False)   # keeps the projection live past K
        self.qn, self.kn = Qwen3RMSNorm(hd, eps=1e-6), Qwen3RMSNorm(hd, eps=1e-5)
        g = torch.Generator().manual_seed(H * hd)
        self.register_buffer("cos", torch.randn(1, H, S, hd, generator=g))
        self.register_buffer("sin", torch.randn(1, H, S, hd, generator=g))

    def forward(self, x):
        B, S, _ = x.shape
        H, hd = self.H, self.hd
        q = self.qn(self.qp(x).view(B, S, H, hd)).transpose(1, 2)
        k = self.kn(self.kp(x).view(B, S, H, hd)).transpose(1, 2)
        v = self.vp(x).view(B, S, H, hd).transpose(1, 2)
        q = q * self.cos + _rotate_half(q) * self.sin
        k = k * self.cos + _rotate_half(k) * self.sin
        return torch.cat([q, k, v], dim=1)


@pytest.mark.parametrize("merge", [True, False])
@pytest.mark.parametrize("hd,H", [(64, 6), (128, 4), (256, 3)])
def test_head_prologue_per_head_tables(monkeypatch, hd, H, merge):
    from runtime.exporter import export_model
    from runtime.session import Session
    from workloads import init_weights, reference_forward
    monkeypatch.setenv("LBR_QKV_EPILOGUE", "0")
    S = 40
    m = init_weights(_PerHeadTables(H, hd, S), seed=hd)
    with torch.no_grad():   # non-trivial norm weights
        m.qn.weight.normal_(1.0, 0.3)
        m.kn.weight.normal_(1.0, 0.3)
    x = np.random.default_rng(H).standard_normal((2, S, 2 * H * hd)).astype(np.float32)
    g = export_model(m, (torch.from_numpy(x),))
    g2 = copy.deepcopy(g)
    if not merge:
        monkeypatch.setenv("LBR_HEAD_MERGE", "0")
    fused = Session(g)
    fused.create()
    heads = [s for s in fused.executor.step_params() if s["kind"] == "head_prologue"]
    assert [s["parts"] for s in heads] == ([2] if merge else [1, 1]) and all(s["vec"] for s in heads), heads
    y = fused.run({g.inputs[0]: x})[g.outputs[0]]
    fused.close()
    monkeypatch.setenv("LBR_FUSE", "0")
    plain = Session(g2)
    plain.create()
    z = plain.run({g2.inputs[0]: x})[g2.outputs[0]]
    plain.close()
    ref = reference_forward(m, x)
    e_fz, e_ref = normwise_rel(y, z), normwise_rel(y, ref)
    print(f"per-head tables hd={hd} H={H} merge={merge}: fused-vs-unfused {e_fz:.2e}, vs torch64 {e_ref:.2e}")
    assert e_fz <= 1e-5
    assert e_ref <= 1e-3


class _SharedTables(torch.nn.Module):
    """Q/K prologues with RoPE rows shared by the heads ([1, 1, S, hd], as Qwen3's rotary
    embedding gives them), head dim 128."""

    def __init__(self, H, S, bias):
        super().__init__()
        from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm
        hd = 128
        self.H, self.hd = H, hd
        self.qp = torch.nn.Linear(2 * H * hd, H * hd, bias=bias)
        self.kp = torch.nn.Linear(2 * H * hd, H * hd, bias=bias)
        self.vp = torch.nn.Linear(2 * H * hd, H * hd, bias=bias)
        self.qn, self.kn = Qwen3RMSNorm(hd, eps=1e-6), Qwen3RMSNorm(hd, eps=1e-5)
        g = torch.Generator().manual_seed(H + S)
        self.register_buffer("cos", torch.randn(1, 1, S, hd, generator=g))
        self.register_buffer("sin", torch.randn(1, 1, S, hd, generator=g))

    def forward(self, x):
        B, S, _ = x.shape
        H, hd = self.H, self.hd
        q = self.qn(self.qp(x).view(B, S, H, hd)).transpose(1, 2)
        k = self.kn(self.kp(x).view(B, S, H, hd)).transpose(1, 2)
        v = self.vp(x).view(B, S, H, hd).transpose(1, 2)
        q = q * self.cos + _rotate_half(q) * self.sin
        k = k * self.cos + _rotate_half(k) * self.sin
        return torch.cat([q, k, v], dim=1)


@pytest.mark.parametrize("bias,merge,S", [(False, True, 64), (True, True, 40), (False, False, 64), (True, True, 100)])
def test_head_prologue_in_qkv_epilogue(monkeypatch, bias, merge, S):
    """At head dim 128 the Q and K prologues run in the QKV GEMM's epilogue: 64×128 tiles, one
    head each, normalised and rotated from LDS with the float4 prologue kernel's lanes and sums,
    so the output equals the GEMM + prologue-kernel plan (LBR_QKV_EPILOGUE=0) bit for bit.
    Apart (LBR_HEAD_MERGE=0) only the Q prologue, right after the GEMM, joins it.  S = 40 and 100 leave partial 64-row tiles and a batch boundary inside a tile (B = 2).  The
    join needs a GEMM without K ranges."""
    from runtime.exporter import export_model
    from runtime.executor.compiled import CompiledExecutor
    from runtime.ir import OpType
    from runtime.passes import run_pipeline
    from runtime.planner import plan
    from workloads import init_weights, reference_forward
    H = 4
    m = init_weights(_SharedTables(H, S, bias), seed=S + bias)
    with torch.no_grad():
        m.qn.weight.normal_(1.0, 0.3)
        m.kn.weight.normal_(1.0, 0.3)
        if bias:
            for p in (m.qp.bias, m.kp.bias, m.vp.bias):
                p.normal_(0.0, 0.5)
    x = np.random.default_rng(S).standard_normal((2, S, 2 * H * 128)).astype(np.float32)
    g = export_model(m, (torch.from_numpy(x),))
    run_pipeline(g, None)
    mm = [n for n in g.nodes.values() if n.op in (OpType.MATMUL, OpType.MATMUL_ADD)]
    assert len(mm) == 1   # q, k and v projections merged into one GEMM
    out = g.outputs[0]
    if not merge:
        monkeypatch.setenv("LBR_HEAD_MERGE", "0")
    # at M = 2·S the model would cut K of this GEMM into ranges, and the epilogue needs one
    # (Qwen3's M = 1024 takes one anyway); the same single range in every plan compared
    monkeypatch.setenv("LBR_GEMM_KSPLIT", "1")
    ys = []
    for env in ("1", "0", "nofuse"):
        monkeypatch.setenv("LBR_QKV_EPILOGUE", "0" if env == "0" else "1")
        ex = CompiledExecutor(fuse=env != "nofuse")
        ex.compile(plan(g))
        try:
            params = ex.step_params()
            joined = [p for p in params if p["kind"] == "gemm_head_prologue"]
            heads = [p for p in params if p["kind"] == "head_prologue"]
            print(env, [(p["name"], p.get("head_parts")) for p in params])
            if env == "1":
                assert len(joined) == 1 and joined[0]["tile"] == "64x128", params
                assert joined[0]["head_parts"] == (2 if merge else 1) and len(heads) == (0 if merge else 1)
            elif env != "nofuse":
                assert not joined and len(heads) == (1 if merge else 2)
            ys.append(ex.run({g.inputs[0]: x})[out])
        finally:
            ex.close()
    np.testing.assert_array_equal(ys[0], ys[1])
    ref = reference_forward(m, x)
    e_fz, e_ref = normwise_rel(ys[0], ys[2]), normwise_rel(ys[0], ref)
    print(f"qkv epilogue bias={bias} merge={merge} S={S}: fused-vs-unfused {e_fz:.2e}, "
          f"vs torch64 {e_ref:.2e}")
    assert e_fz <= 1e-5
    assert e_ref <= 1e-3


@pytest.mark.parametrize("S", [512, 1024])
def test_qkv_epilogue_in_qwen3_layer(monkeypatch, S):
    """A Qwen3-4B-shaped layer (32/8 heads of 128, hidden 2560): the planner puts the Q/K
    prologue outputs over the QKV GEMM's input, which the epilogue cannot write while other
    workgroups still read it, so the plan moves them to a buffer of its own and points the
    attention's Q and K there.  Bit-equal to the GEMM + prologue-kernel plan."""
    from runtime.exporter import export_model
    from runtime.session import Session
    from workloads import Qwen3Body, init_weights
    m = init_weights(Qwen3Body(n_layer=1), seed=0)
    x = np.random.default_rng(S).standard_normal((1, S, 2560)).astype(np.float32)
    g = export_model(m, (torch.from_numpy(x),))
    ys = []
    for env in ("1", "0"):
        monkeypatch.setenv("LBR_QKV_EPILOGUE", env)
        sess = Session(copy.deepcopy(g))
        sess.create()
        kinds = [p["kind"] for p in sess.executor.step_params()]
        print(env, [p["name"] for p in sess.executor.step_params()])
        assert ("gemm_head_prologue" in kinds) == (env == "1") and ("head_prologue" in kinds) == (env == "0")
        ys.append(sess.run({g.inputs[0]: x})[g.outputs[0]])
        sess.close()
    np.testing.assert_array_equal(ys[0], ys[1])
