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
