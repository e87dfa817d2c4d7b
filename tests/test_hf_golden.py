"""CPU checks of the Hugging Face fixture (tests/golden/hf_qwen3.npz, written
by tests/golden/make_hf_golden.py from transformers' own Qwen3, loaded with
from_pretrained in float16 and in bfloat16): the seeded weights the GPU tests
load reproduce the weights the fixture was made with, the fixture is
self-consistent (HF's greedy tokens are the argmax of its logits), and its
prologue vectors are exactly what transformers' published formulas give
(Qwen3RMSNorm, Qwen3RotaryEmbedding with a float32 inv_freq, and
apply_rotary_pos_emb with every product and sum rounded to the model dtype),
restated here in torch on the CPU. The restatement with inv_freq rounded to
the model dtype (what casting a built model with .to(dtype) does) must not
match: it moves every angle by up to 2^-9 relative."""
import numpy as np
import pytest
import torch

from tests.golden import hf_qwen3_weights as W

GOLD = np.load("tests/golden/hf_qwen3.npz")
DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16}
H, KV, D = (W.SMALL_HF[k] for k in ("num_attention_heads", "num_key_value_heads", "head_dim"))


def _t16(a: np.ndarray, dt) -> torch.Tensor:
    return torch.from_numpy(a.view(np.int16).copy()).view(dt)


def _hf_prologue(x: torch.Tensor, w: torch.Tensor, inv_freq: torch.Tensor) -> torch.Tensor:
    """q_norm / k_norm then apply_rotary_pos_emb on x [T, heads, D] in the
    model dtype, in transformers' order of roundings."""
    dt = x.dtype
    xf = x.float()
    n = w.to(dt) * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True)
                                     + W.SMALL_HF["rms_norm_eps"])).to(dt)
    ang = torch.arange(x.size(0)).float()[:, None] * inv_freq[None, :]
    emb = torch.cat([ang, ang], -1)
    cos, sin = emb.cos().to(dt)[:, None, :], emb.sin().to(dt)[:, None, :]
    half = D // 2
    return n * cos + torch.cat([-n[..., half:], n[..., :half]], -1) * sin


def test_seeded_weights_reproduce_the_fixture_weights():
    assert W.sha(W.weights()) == str(GOLD["weights_sha"])


@pytest.mark.parametrize("tag", list(DTYPES))
def test_fixture_is_self_consistent(tag):
    for i in range(3):
        assert np.array_equal(GOLD[f"{tag}_seq{i}_prompt"], GOLD[f"bf16_seq{i}_prompt"])
        lg = _t16(GOLD[f"{tag}_seq{i}_prompt_logits"], DTYPES[tag]).float().numpy()
        rows = GOLD[f"{tag}_seq{i}_rows"]
        assert np.array_equal(lg.argmax(-1), GOLD[f"{tag}_seq{i}_prompt_argmax"][rows])
        dec = _t16(GOLD[f"{tag}_seq{i}_decode_logits"], DTYPES[tag]).float().numpy()
        toks = GOLD[f"{tag}_seq{i}_decode_tokens"]
        assert toks[0] == GOLD[f"{tag}_seq{i}_prompt_argmax"][-1]
        assert np.array_equal(dec[:-1].argmax(-1), toks[1:])
    T = len(GOLD[f"{tag}_seq0_prompt"])
    assert GOLD[f"{tag}_prologue_q"].shape == (T, H, D)
    assert GOLD[f"{tag}_prologue_k"].shape == (T, KV, D)


@pytest.mark.parametrize("tag", list(DTYPES))
def test_fixture_prologue_is_hf_formula(tag):
    dt = DTYPES[tag]
    ws = W.weights()
    qkv = _t16(GOLD[f"{tag}_prologue_qkv"], dt)
    T = qkv.size(0)
    inv = 1.0 / (W.SMALL_HF["rope_theta"] ** (torch.arange(0, D, 2, dtype=torch.float) / D))
    assert torch.equal(qkv[:, (H + KV) * D:].reshape(T, KV, D), _t16(GOLD[f"{tag}_prologue_v"], dt))
    for name, off, nh in (("q", 0, H), ("k", H * D, KV)):
        x = qkv[:, off:off + nh * D].reshape(T, nh, D)
        w = ws[f"model.layers.0.self_attn.{name}_norm.weight"]
        want = _t16(GOLD[f"{tag}_prologue_{name}"], dt)
        assert torch.equal(_hf_prologue(x, w, inv).view(torch.int16), want.view(torch.int16))
        # planted mistake: the angles of a dtype-rounded inv_freq
        bad = _hf_prologue(x, w, inv.to(dt).float())
        assert (bad.view(torch.int16) == want.view(torch.int16)).float().mean() < 0.95
