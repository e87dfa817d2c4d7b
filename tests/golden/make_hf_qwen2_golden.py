"""Writes tests/golden/hf_qwen2.npz: vectors from Hugging Face transformers'
own Qwen2 (the reference's runner serves qwen2 models as well as qwen3,
nanoPD/engine/model_runner.py:53-58; its q_norm / k_norm step applies only
when the attention module has them, :101-104, which Qwen2's does not), run on
the CPU with eager attention, for the parity tests of the norm-free fused
prologue and of PagedQwen3 with the Qwen2 options. Run in a container with
transformers installed: python -m tests.golden.make_hf_qwen2_golden

The attention has configuration 1's head shape (Qwen2-1.5B: 12 query and 2 kv
heads of 128, q/k/v biases, tied embeddings; tests/golden/hf_qwen2_weights.py).
The model is loaded the way the reference loads it (model_runner.py:9-13):
the seeded weights are saved with save_pretrained and read back with
AutoModelForCausalLM.from_pretrained(dtype=...), once in float16 (the
reference's dtype) and once in bfloat16, which keeps the rotary embedding's
inv_freq in float32.

Contents (`<dt>` is "fp16" or "bf16"):
- weights_sha: SHA-256 of the seeded weights;
- <dt>_prologue_*: layer 0 of sequence 0: the q/k/v projection output with
  its biases (the input of the prologue), and HF's q and k after
  apply_rotary_pos_emb with Qwen2RotaryEmbedding's cos / sin, as 16-bit
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

from tests.golden import hf_qwen2_weights as W  # noqa: E402
from tests.golden.make_hf_golden import DTYPES, bits  # noqa: E402

PROMPTS = (37, 130, 300)
DECODE_STEPS = 3
OUT = os.path.join(HERE, "hf_qwen2.npz")


def main() -> None:
    from transformers import AutoModelForCausalLM, Qwen2Config, Qwen2ForCausalLM

    torch.manual_seed(0)
    cfg = Qwen2Config(**W.SMALL_HF, attn_implementation="eager")
    ws = W.weights()
    src = Qwen2ForCausalLM(cfg)
    missing, unexpected = src.load_state_dict({n: t.float() for n, t in ws.items()}, strict=False)
    assert not unexpected, unexpected
    assert all("rotary" in m or m == "lm_head.weight" for m in missing), missing
    src.tie_weights()
    assert src.lm_head.weight.data_ptr() == src.model.embed_tokens.weight.data_ptr()
    out = {"weights_sha": np.array(W.sha(ws))}

    g = torch.Generator().manual_seed(11)
    prompts = [torch.randint(0, W.SMALL_HF["vocab_size"], (n,), generator=g) for n in PROMPTS]
    with tempfile.TemporaryDirectory() as d:
        src.save_pretrained(d)
        for tag, dt in DTYPES.items():
            model = AutoModelForCausalLM.from_pretrained(d, dtype=dt,
                                                         attn_implementation="eager").eval()
            assert model.model.rotary_emb.inv_freq.dtype == torch.float32
            assert not hasattr(model.model.layers[0].self_attn, "q_norm")
            record(model, prompts, tag, out)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


def record(model, prompts: list, tag: str, out: dict) -> None:
    from transformers.models.qwen2 import modeling_qwen2 as hfq

    H, KV, D = W.SMALL_HF["num_attention_heads"], W.SMALL_HF["num_key_value_heads"], W.HEAD_DIM
    layer = model.model.layers[0]
    attn = layer.self_attn
    ids = prompts[0][None]
    pos = torch.arange(ids.size(1))[None]
    with torch.no_grad():
        h = layer.input_layernorm(model.model.embed_tokens(ids))
        qp, kp, vp = attn.q_proj(h), attn.k_proj(h), attn.v_proj(h)
        q = qp.view(1, -1, H, D).transpose(1, 2)
        k = kp.view(1, -1, KV, D).transpose(1, 2)
        cos, sin = model.model.rotary_emb(h, pos)
        qr, kr = hfq.apply_rotary_pos_emb(q, k, cos, sin)
    out[f"{tag}_prologue_qkv"] = bits(torch.cat([qp, kp, vp], dim=-1)[0])    # [T, (H+2KV)*D]
    out[f"{tag}_prologue_q"] = bits(qr[0].transpose(0, 1))                    # [T, H, D]
    out[f"{tag}_prologue_k"] = bits(kr[0].transpose(0, 1))                    # [T, KV, D]
    out[f"{tag}_prologue_v"] = bits(vp[0].view(-1, KV, D))

    for i, p in enumerate(prompts):
        seq = p.clone()
        with torch.no_grad():
            lg = model(seq[None]).logits[0]
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
