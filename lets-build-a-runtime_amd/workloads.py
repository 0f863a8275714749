"""The five benchmark workloads as seeded PyTorch models.

Each workload builds a random-init fp32 model of the stated architecture and
a seeded input, following one convention everywhere (GPU run, CPU oracle,
PyTorch reference):

* weights: ``torch.manual_seed(seed)``; every Linear weight and every
  embedding ~ N(0, 0.02); biases 0; LayerNorm γ = 1, β = 0; RMSNorm w = 1;
* input: ``np.random.default_rng(seed).standard_normal((1, S, D))`` as fp32.

Architectures:
  toy      custom pre-norm block  S=32   D=64   H=4   causal SDPA, tanh-GELU FFN 4×
  gpt2w    custom pre-norm block  S=512  D=768  H=12
  gpt2     GPT-2 body, 2 layers   S=1024 D=768  H=12  (HF GPT2Block + ln_f, learned
           position embeddings added to the input)
  7b4k     custom pre-norm block  S=4096 D=4096 H=32
  qwen3_4b Qwen3 body, 2 layers   S=1024 D=2560 Hq=32 Hkv=8 hd=128, q/k RMSNorm,
           RoPE θ=1e6, SiLU-gated FFN 9728, RMSNorm eps 1e-6 (HF Qwen3DecoderLayer)
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F


class CausalGeluBlock(nn.Module):
    """Pre-norm transformer block: LN → QKV (bias) → causal SDPA → O (bias) → residual,
    LN → FFN (bias) with tanh-GELU → residual."""

    def __init__(self, d_model: int, n_heads: int, ffn_mult: int = 4) -> None:
        super().__init__()
        self.n_heads = n_heads
        self.d_k = d_model // n_heads
        self.ln1 = nn.LayerNorm(d_model)
        self.wq = nn.Linear(d_model, d_model)
        self.wk = nn.Linear(d_model, d_model)
        self.wv = nn.Linear(d_model, d_model)
        self.wo = nn.Linear(d_model, d_model)
        self.ln2 = nn.LayerNorm(d_model)
        self.ffn1 = nn.Linear(d_model, d_model * ffn_mult)
        self.ffn2 = nn.Linear(d_model * ffn_mult, d_model)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        B, S, D = x.shape
        h = self.ln1(x)
        q = self.wq(h).reshape(B, S, self.n_heads, self.d_k).permute(0, 2, 1, 3)
        k = self.wk(h).reshape(B, S, self.n_heads, self.d_k).permute(0, 2, 1, 3)
        v = self.wv(h).reshape(B, S, self.n_heads, self.d_k).permute(0, 2, 1, 3)
        a = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        a = a.permute(0, 2, 1, 3).reshape(B, S, D)
        x = x + self.wo(a)
        return x + self.ffn2(F.gelu(self.ffn1(self.ln2(x)), approximate="tanh"))


class GPT2Body(nn.Module):
    """GPT-2 transformer body: learned position embeddings + blocks + ln_f."""

    def __init__(self, n_layer: int = 2, n_head: int = 12, n_embd: int = 768, n_positions: int = 1024) -> None:
        super().__init__()
        from transformers import GPT2Config
        from transformers.models.gpt2.modeling_gpt2 import GPT2Block
        cfg = GPT2Config(n_layer=n_layer, n_head=n_head, n_embd=n_embd, n_positions=n_positions, vocab_size=1,
                         bos_token_id=0, eos_token_id=0, attn_pdrop=0.0, resid_pdrop=0.0, embd_pdrop=0.0)
        cfg._attn_implementation = "sdpa"
        self.wpe = nn.Parameter(torch.zeros(n_positions, n_embd))
        self.h = nn.ModuleList([GPT2Block(cfg, layer_idx=i) for i in range(n_layer)])
        self.ln_f = nn.LayerNorm(n_embd, eps=cfg.layer_norm_epsilon)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        h = x + self.wpe[: x.shape[1]]
        for block in self.h:
            out = block(h)
            h = out[0] if isinstance(out, tuple) else out
        return self.ln_f(h)


class Qwen3Body(nn.Module):
    """Qwen3 decoder body: rotary tables + decoder layers + final RMSNorm."""

    def __init__(self, hidden: int = 2560, n_layer: int = 2, n_heads: int = 32, n_kv: int = 8, head_dim: int = 128,
                 ffn: int = 9728, eps: float = 1e-6, theta: float = 1e6, max_pos: int = 4096) -> None:
        super().__init__()
        from transformers import Qwen3Config
        from transformers.models.qwen3 import modeling_qwen3 as mq
        cfg = Qwen3Config(hidden_size=hidden, intermediate_size=ffn, num_hidden_layers=n_layer,
                          num_attention_heads=n_heads, num_key_value_heads=n_kv, head_dim=head_dim,
                          rms_norm_eps=eps, vocab_size=16, max_position_embeddings=max_pos,
                          rope_parameters={"rope_type": "default", "rope_theta": theta}, attention_bias=False)
        cfg._attn_implementation = "sdpa"
        self.layers = nn.ModuleList([mq.Qwen3DecoderLayer(cfg, i) for i in range(n_layer)])
        self.norm = mq.Qwen3RMSNorm(hidden, eps=eps)
        self.rotary_emb = mq.Qwen3RotaryEmbedding(cfg)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        pos = torch.arange(x.shape[1], device=x.device).unsqueeze(0)
        pe = self.rotary_emb(x, pos)
        for layer in self.layers:
            out = layer(x, attention_mask=None, position_ids=pos, position_embeddings=pe)
            x = out[0] if isinstance(out, tuple) else out
        return self.norm(x)


def init_weights(model: nn.Module, seed: int = 0) -> nn.Module:
    """N(0, 0.02) linear/embedding weights, zero biases, unit norm scales (deterministic per seed)."""
    torch.manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            leaf = name.rsplit(".", 1)[-1]
            if leaf == "bias":
                p.zero_()
            elif p.dim() >= 2 or name == "wpe":
                p.normal_(0.0, 0.02)
            else:  # LayerNorm / RMSNorm scales
                p.fill_(1.0)
    return model.eval()


class CausalLM(nn.Module):
    """A HuggingFace causal LM returning logits for token ids — the reference's
    full-model benchmark wrapper (ablation/bench_transformer_ablation.py:186-208)."""

    def __init__(self, lm: nn.Module) -> None:
        super().__init__()
        self.lm = lm

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        return self.lm(ids, use_cache=False).logits


def gpt2_lm(n_layer: int = 2, n_head: int = 12, n_embd: int = 768, vocab: int = 50257) -> nn.Module:
    """GPT2LMHeadModel as the reference builds it (bench_transformer_ablation.py:170-183): tied LM head."""
    from transformers import GPT2Config, GPT2LMHeadModel
    cfg = GPT2Config(n_layer=n_layer, n_head=n_head, n_embd=n_embd, vocab_size=vocab, attn_pdrop=0.0,
                     resid_pdrop=0.0, embd_pdrop=0.0)
    cfg._attn_implementation = "sdpa"
    m = GPT2LMHeadModel(cfg)
    m.config.use_cache = False
    return CausalLM(m)


def qwen3_lm(hidden: int = 2560, n_layer: int = 2, n_heads: int = 32, n_kv: int = 8, head_dim: int = 128,
             ffn: int = 9728, vocab: int = 151936, eps: float = 1e-6, theta: float = 1e6) -> nn.Module:
    """Qwen3ForCausalLM with Qwen3-4B's shape, two layers and tied embeddings (the reference
    loads the same config from the hub, bench_transformer_ablation.py:196-208; no network here)."""
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(hidden_size=hidden, intermediate_size=ffn, num_hidden_layers=n_layer,
                      num_attention_heads=n_heads, num_key_value_heads=n_kv, head_dim=head_dim,
                      rms_norm_eps=eps, vocab_size=vocab, max_position_embeddings=40960,
                      rope_parameters={"rope_type": "default", "rope_theta": theta}, attention_bias=False,
                      tie_word_embeddings=True)
    cfg._attn_implementation = "sdpa"
    m = Qwen3ForCausalLM(cfg)
    m.config.use_cache = False
    return CausalLM(m)


@dataclass(frozen=True)
class Workload:
    key: str
    title: str
    seq_len: int
    d_model: int
    build: Callable[[], nn.Module]
    causal: bool = True
    vocab: int = 0               # > 0: the model takes int64 token ids [1, S] in [0, vocab)

    def model(self, seed: int = 0) -> nn.Module:
        return init_weights(self.build(), seed)

    def input(self, seed: int = 0, seq_len: int | None = None, batch: int = 1) -> np.ndarray:
        s = self.seq_len if seq_len is None else seq_len
        rng = np.random.default_rng(seed)
        if self.vocab:
            return rng.integers(0, self.vocab, (batch, s), dtype=np.int64)
        return rng.standard_normal((batch, s, self.d_model)).astype(np.float32)


WORKLOADS: dict[str, Workload] = {
    "toy": Workload("toy", "Toy custom block S32 D64 H4", 32, 64, lambda: CausalGeluBlock(64, 4)),
    "gpt2w": Workload("gpt2w", "Custom block at GPT-2 width S512 D768 H12", 512, 768,
                      lambda: CausalGeluBlock(768, 12)),
    "gpt2": Workload("gpt2", "GPT-2 body 2 layers S1024 D768 H12", 1024, 768, lambda: GPT2Body(2, 12, 768, 1024)),
    "7b4k": Workload("7b4k", "7B-shaped block S4096 D4096 H32", 4096, 4096, lambda: CausalGeluBlock(4096, 32)),
    "qwen3_4b": Workload("qwen3_4b", "Qwen3-4B-shaped body 2 layers S1024 D2560 GQA 32/8", 1024, 2560,
                         lambda: Qwen3Body()),
    # the reference's published full-model rows (README.md:41-57): embeddings + 2 layers + LM head
    "gpt2_lm": Workload("gpt2_lm", "GPT-2 LM 2 layers S1024 D768 vocab 50257 (token ids in, logits out)", 1024,
                        768, lambda: gpt2_lm(), vocab=50257),
    "qwen3_4b_lm": Workload("qwen3_4b_lm", "Qwen3-4B-shaped LM 2 layers S1024 D2560 vocab 151936 (ids in, logits out)",
                            1024, 2560, lambda: qwen3_lm(), vocab=151936),
}

# BASELINE.json configs[i] → workload key
CONFIG_ORDER = ["toy", "gpt2w", "gpt2", "7b4k", "qwen3_4b"]
# the full language models (embeddings + LM head) the reference quotes latencies for
# (README.md:41-57), measured after the BASELINE shapes
LM_ORDER = ["gpt2_lm", "qwen3_4b_lm"]


def export_workload(key: str, seed: int = 0, seq_len: int | None = None, batch: int = 1):
    """(model, input numpy, exported Graph) for a workload (the BASELINE configs are batch 1)."""
    from runtime.exporter import export_model
    w = WORKLOADS[key]
    model = w.model(seed)
    x = w.input(seed, seq_len, batch)
    graph = export_model(model, (torch.from_numpy(x),))
    return model, x, graph


def reference_forward(model: nn.Module, x: np.ndarray, dtype=torch.float64) -> np.ndarray:
    """PyTorch eager forward on the CPU in ``dtype`` (float64 by default)."""
    with torch.no_grad():
        m = model.to(dtype)
        xt = torch.from_numpy(x)
        try:
            y = m(xt if not xt.is_floating_point() else xt.to(dtype))   # token ids stay int64
        finally:
            model.to(torch.float32)
    return y.to(torch.float64).numpy()
