"""Seeded weights of the small Qwen2 used for the Hugging Face fixture
tests/golden/hf_qwen2.npz: the same tensors in the fixture generator (which
loads them into transformers' Qwen2ForCausalLM) and in the GPU tests (which
load them into PagedQwen3 with the Qwen2 options). The attention has
configuration 1's head shape -- Qwen2-1.5B's: 12 query heads and 2 kv heads of
128 (hidden 1536) -- with q/k/v biases, no q/k norms and a tied LM head, as
that model has; two layers and a small vocabulary keep it small. Drawn on the
CPU with a seeded torch.Generator in a fixed order; the fixture stores their
SHA-256 so that a different draw is caught before any comparison."""
from __future__ import annotations

import hashlib

import torch

SMALL_HF = dict(vocab_size=1000, hidden_size=1536, intermediate_size=1024, num_hidden_layers=2,
                num_attention_heads=12, num_key_value_heads=2, rope_theta=1.0e6,
                rms_norm_eps=1.0e-6, max_position_embeddings=4096, tie_word_embeddings=True)
HEAD_DIM = SMALL_HF["hidden_size"] // SMALL_HF["num_attention_heads"]   # 128
SEED = 20251202
STD = 0.03
BIAS_STD = 0.5   # large enough that a dropped bias moves q and k visibly


def shapes(cfg: dict = SMALL_HF) -> dict:
    E, I, V = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"]
    H, KV = cfg["num_attention_heads"], cfg["num_key_value_heads"]
    D = E // H
    out = {"model.embed_tokens.weight": (V, E), "model.norm.weight": (E,)}
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}."
        out.update({p + "input_layernorm.weight": (E,), p + "post_attention_layernorm.weight": (E,),
                    p + "self_attn.q_proj.weight": (H * D, E), p + "self_attn.q_proj.bias": (H * D,),
                    p + "self_attn.k_proj.weight": (KV * D, E), p + "self_attn.k_proj.bias": (KV * D,),
                    p + "self_attn.v_proj.weight": (KV * D, E), p + "self_attn.v_proj.bias": (KV * D,),
                    p + "self_attn.o_proj.weight": (E, H * D),
                    p + "mlp.gate_proj.weight": (I, E), p + "mlp.up_proj.weight": (I, E),
                    p + "mlp.down_proj.weight": (E, I)})
    return out


def weights(cfg: dict = SMALL_HF) -> dict:
    """bf16 CPU tensors by HF parameter name (in sorted-name order of the
    draw): matrices N(0, STD), biases N(0, BIAS_STD), norm weights
    1 + N(0, 0.1)."""
    g = torch.Generator().manual_seed(SEED)
    out = {}
    for n, sh in sorted(shapes(cfg).items()):
        x = torch.randn(sh, generator=g, dtype=torch.float32)
        if n.endswith(".bias"):
            x = x * BIAS_STD
        elif len(sh) == 1:
            x = 1.0 + 0.1 * x
        else:
            x = x * STD
        out[n] = x.to(torch.bfloat16)
    return out


def sha(ws: dict) -> str:
    h = hashlib.sha256()
    for n in sorted(ws):
        h.update(n.encode())
        h.update(ws[n].view(torch.int16).numpy().tobytes())
    return h.hexdigest()
