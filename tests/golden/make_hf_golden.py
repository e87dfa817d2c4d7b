"""Writes tests/golden/hf_qwen3.npz: vectors from Hugging Face transformers'
own Qwen3 (the model the reference wraps, nanoPD/engine/model_runner.py:8-13,
:53-58, :97-115), run on the CPU with eager attention, for the parity tests of
the fused prologue and of PagedQwen3. Run in a container with transformers
installed: python -m tests.golden.make_hf_golden

The model is loaded the way the reference loads it (model_runner.py:9-13):
the seeded weights are saved with save_pretrained and read back with
AutoModelForCausalLM.from_pretrained(dtype=...), once in float16 (the
reference's dtype) and once in bfloat16. That path keeps the rotary
embedding's inv_freq in float32 (casting a built model with .to(dtype) would
round it to the model dtype and shift every angle by up to 2^-9 relative).

Contents (`<dt>` is "fp16" or "bf16"):
- weights_sha: SHA-256 of the seeded weights (tests/golden/hf_qwen3_weights.py);
- <dt>_prologue_*: layer 0 of sequence 0: the q/k/v projection output (input
  of the prologue), and HF's q and k after q_norm / k_norm and
  apply_rotary_pos_emb with Qwen3RotaryEmbedding's cos / sin, as 16-bit
  patterns of the model dtype;
- <dt>_seq<i>_*: three prompts (37, 130, 300 tokens) and three greedy decode
  steps each; HF's logits (model dtype, as 16-bit patterns) at every 8th
  prompt position, the prompt's last position and each decode position, and
  the greedy tokens.
"""
from __future__ import annotations

import os
import sys
import tempfile

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from tests.golden import hf_qwen3_weights as W  # noqa: E402

PROMPTS = (37, 130, 300)
DECODE_STEPS = 3
OUT = os.path.join(HERE, "hf_qwen3.npz")


DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16}


def bits(t: torch.Tensor) -> np.ndarray:
    assert t.dtype in (torch.float16, torch.bfloat16)
    return t.detach().contiguous().view(torch.int16).numpy().view(np.uint16)


def main() -> None:
    from transformers import AutoModelForCausalLM, Qwen3Config, Qwen3ForCausalLM

    torch.manual_seed(0)
    cfg = Qwen3Config(**W.SMALL_HF, attn_implementation="eager")
    ws = W.weights()
    src = Qwen3ForCausalLM(cfg)
    missing, unexpected = src.load_state_dict({n: t.float() for n, t in ws.items()}, strict=False)
    assert not unexpected and all("rotary" in m for m in missing), (missing, unexpected)
    out = {"weights_sha": np.array(W.sha(ws))}

    g = torch.Generator().manual_seed(7)
    prompts = [torch.randint(0, W.SMALL_HF["vocab_size"], (n,), generator=g) for n in PROMPTS]
    with tempfile.TemporaryDirectory() as d:
        src.save_pretrained(d)
        for tag, dt in DTYPES.items():
            model = AutoModelForCausalLM.from_pretrained(d, dtype=dt,
                                                         attn_implementation="eager").eval()
            assert model.model.rotary_emb.inv_freq.dtype == torch.float32
            record(model, prompts, tag, out)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


def record(model, prompts: list, tag: str, out: dict) -> None:
    from transformers.models.qwen3 import modeling_qwen3 as hfq

    # prologue of layer 0 on prompt 0, HF's own modules
    layer = model.model.layers[0]
    attn = layer.self_attn
    ids = prompts[0][None]
    pos = torch.arange(ids.size(1))[None]
    with torch.no_grad():
        h = layer.input_layernorm(model.model.embed_tokens(ids))
        qp, kp, vp = attn.q_proj(h), attn.k_proj(h), attn.v_proj(h)
        D = W.SMALL_HF["head_dim"]
        q = attn.q_norm(qp.view(1, -1, W.SMALL_HF["num_attention_heads"], D)).transpose(1, 2)
        k = attn.k_norm(kp.view(1, -1, W.SMALL_HF["num_key_value_heads"], D)).transpose(1, 2)
        cos, sin = model.model.rotary_emb(h, pos)
        qr, kr = hfq.apply_rotary_pos_emb(q, k, cos, sin)
    out[f"{tag}_prologue_qkv"] = bits(torch.cat([qp, kp, vp], dim=-1)[0])    # [T, (H+2KV)*D]
    out[f"{tag}_prologue_q"] = bits(qr[0].transpose(0, 1))                    # [T, H, D]
    out[f"{tag}_prologue_k"] = bits(kr[0].transpose(0, 1))                    # [T, KV, D]
    out[f"{tag}_prologue_v"] = bits(vp[0].view(-1, W.SMALL_HF["num_key_value_heads"], D))

    # whole model: prompts, then greedy decode steps (full re-forward each time)
    for i, p in enumerate(prompts):
        seq = p.clone()
        with torch.no_grad():
            lg = model(seq[None]).logits[0]                  # model dtype
        rows = sorted(set(range(0, len(p), 8)) | {len(p) - 1})
        out[f"{tag}_seq{i}_prompt"] = p.numpy().astype(np.int32)
        out[f"{tag}_seq{i}_rows"] = np.array(rows, dtype=np.int32)
        out[f"{tag}_seq{i}_prompt_logits"] = bits(lg[rows])
        out[f"{tag}_seq{i}_prompt_argmax"] = lg.float().argmax(-1).numpy().astype(np.int32)
        toks, dec = [], []
        nxt = int(lg[-1].argmax())
        for _ in range(DECODE_STEPS):
            toks.append(nxt)
            seq = torch.cat([seq, torch.tensor([nxt])])
            with torch.no_grad():
                l1 = model(seq[None]).logits[0, -1]
            dec.append(bits(l1))
            nxt = int(l1.float().argmax())
        out[f"{tag}_seq{i}_decode_tokens"] = np.array(toks, dtype=np.int32)
        out[f"{tag}_seq{i}_decode_logits"] = np.stack(dec)


if __name__ == "__main__":
    main()
