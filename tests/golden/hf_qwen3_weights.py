"""Seeded weights of the small Qwen3 used for the Hugging Face fixtures
(tests/golden/hf_qwen3.npz): the same tensors in the fixture generator (which
loads them into transformers' Qwen3ForCausalLM) and in the GPU tests (which
load them into PagedQwen3). Drawn on the CPU with a seeded torch.Generator in
a fixed order; the fixture stores their SHA-256 so that a different draw is
caught before any comparison."""
from __future__ import annotations

import hashlib

import torch

SMALL_HF = dict(vocab_size=1000, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                num_attention_heads=4, num_key_value_heads=2, head_dim=128, rope_theta=1.0e6,
                rms_norm_eps=1.0e-6, max_position_embeddings=4096, tie_word_embeddings=False,
                attention_bias=False)
SEED = 20241202
STD = 0.05


def names(num_layers: int) -> list:
    out = ["model.embed_tokens.weight", "model.norm.weight", "lm_head.weight"]
    for i in range(num_layers):
        p = f"model.layers.{i}."
        out += [p + n for n in ("input_layernorm.weight", "post_attention_layernorm.weight",
                                "self_attn.q_proj.weight", "self_attn.k_proj.weight",
                                "self_attn.v_proj.weight", "self_attn.o_proj.weight",
                                "self_attn.q_norm.weight", "self_attn.k_norm.weight",
                                "mlp.gate_proj.weight", "mlp.up_proj.weight",
                                "mlp.down_proj.weight")]
    return out


def shapes(cfg: dict) -> dict:
    E, I, V = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"]
    H, KV, D = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"]
    out = {"model.embed_tokens.weight": (V, E), "model.norm.weight": (E,),
           "lm_head.weight": (V, E)}
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}."
        out.update({p + "input_layernorm.weight": (E,), p + "post_attention_layernorm.weight": (E,),
                    p + "self_attn.q_proj.weight": (H * D, E), p + "self_attn.k_proj.weight": (KV * D, E),
                    p + "self_attn.v_proj.weight": (KV * D, E), p + "self_attn.o_proj.weight": (E, H * D),
                    p + "self_attn.q_norm.weight": (D,), p + "self_attn.k_norm.weight": (D,),
                    p + "mlp.gate_proj.weight": (I, E), p + "mlp.up_proj.weight": (I, E),
                    p + "mlp.down_proj.weight": (E, I)})
    return out


def weights(cfg: dict = SMALL_HF) -> dict:
    """bf16 CPU tensors by HF parameter name: projections N(0, STD), norm
    weights 1 + N(0, 0.1) (so that the norms' weights matter)."""
    g = torch.Generator().manual_seed(SEED)
    sh = shapes(cfg)
    out = {}
    for n in names(cfg["num_hidden_layers"]):
        x = torch.randn(sh[n], generator=g, dtype=torch.float32)
        out[n] = ((1.0 + 0.1 * x) if len(sh[n]) == 1 else x * STD).to(torch.bfloat16)
    return out


def sha(ws: dict) -> str:
    h = hashlib.sha256()
    for n in sorted(ws):
        h.update(n.encode())
        h.update(ws[n].view(torch.int16).numpy().tobytes())
    return h.hexdigest()
