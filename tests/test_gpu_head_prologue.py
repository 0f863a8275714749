"""The fused head prologue (SLICE → [bias] → RMSNorm → TRANSPOSE → RoPE as one
kernel) on Qwen3-style attention layers of head dim 64, 128 and 256, with and
without q/k/v biases, in both kernel forms: the float4 one (hd/4 lanes per
row) and the one-wavefront-per-row one kept for unaligned rows.

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


@pytest.mark.parametrize("kernel", ["vec", "scalar"])
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
    fused = Session(g)
    fused.create()
    heads = [s for s in fused.executor.step_params() if s["kind"] == "head_prologue"]
    assert len(heads) == 2 and all(s["vec"] == (kernel == "vec") for s in heads), heads   # q and k
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
