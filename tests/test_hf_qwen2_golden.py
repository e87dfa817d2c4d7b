"""CPU checks of the Hugging Face Qwen2 fixture (tests/golden/hf_qwen2.npz,
written by tests/golden/make_hf_qwen2_golden.py from transformers' own Qwen2 at
configuration 1's head shape, loaded with from_pretrained in float16 and in
bfloat16): the seeded weights the GPU tests load reproduce the fixture's, the
fixture is self-consistent (HF's greedy tokens are the argmax of its logits),
its projection output holds the q/k/v biases, and its q / k are exactly what
transformers' published formulas give without a q/k norm (Qwen2RotaryEmbedding
with a float32 inv_freq, apply_rotary_pos_emb with every product and sum
rounded to the model dtype), restated here in torch. Planted mistakes -- the
angles of a dtype-rounded inv_freq, a projection without its bias, a Qwen3
q_norm applied where Qwen2 has none -- must not match."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from tests.golden import hf_qwen2_weights as W

GOLD = np.load("tests/golden/hf_qwen2.npz")
DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16}
H, KV = W.SMALL_HF["num_attention_heads"], W.SMALL_HF["num_key_value_heads"]
D = W.HEAD_DIM
EPS = W.SMALL_HF["rms_norm_eps"]


def _t16(a: np.ndarray, dt) -> torch.Tensor:
    return torch.from_numpy(a.view(np.int16).copy()).view(dt)


def _rope_hf(x: torch.Tensor, inv_freq: torch.Tensor) -> torch.Tensor:
    """apply_rotary_pos_emb on x [T, heads, D] in the model dtype at positions
    0..T-1, in transformers' order of roundings."""
    dt = x.dtype
    ang = torch.arange(x.size(0)).float()[:, None] * inv_freq[None, :]
    emb = torch.cat([ang, ang], -1)
    cos, sin = emb.cos().to(dt)[:, None, :], emb.sin().to(dt)[:, None, :]
    half = D // 2
    return x * cos + torch.cat([-x[..., half:], x[..., :half]], -1) * sin


def _inv_freq():
    return 1.0 / (W.SMALL_HF["rope_theta"] ** (torch.arange(0, D, 2, dtype=torch.float) / D))


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
def test_fixture_projection_holds_the_biases(tag):
    """Layer 0's input (Qwen2RMSNorm of the embedding rows) through F.linear
    with and without the biases: the fixture's q/k/v is the biased one."""
    dt = DTYPES[tag]
    ws = {n: t.to(dt) for n, t in W.weights().items()}
    ids = torch.from_numpy(GOLD[f"{tag}_seq0_prompt"]).long()
    x = ws["model.embed_tokens.weight"][ids]
    xf = x.float()
    h = ws["model.layers.0.input_layernorm.weight"] * \
        (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + EPS)).to(dt)
    p = "model.layers.0.self_attn."
    got = torch.cat([F.linear(h, ws[p + f"{n}_proj.weight"], ws[p + f"{n}_proj.bias"])
                     for n in "qkv"], -1)
    nob = torch.cat([F.linear(h, ws[p + f"{n}_proj.weight"]) for n in "qkv"], -1)
    want = _t16(GOLD[f"{tag}_prologue_qkv"], dt)
    u = 2.0 ** -8 if dt == torch.bfloat16 else 2.0 ** -11
    # the CPU GEMM's summation order may differ from the one HF ran: within a
    # few roundings of the output's magnitude
    assert ((got.float() - want.float()).abs() <= 4 * u * want.float().abs() + 1e-3).all()
    assert ((nob.float() - want.float()).abs().max() > 0.1)


@pytest.mark.parametrize("tag", list(DTYPES))
def test_fixture_prologue_is_hf_formula(tag):
    dt = DTYPES[tag]
    qkv = _t16(GOLD[f"{tag}_prologue_qkv"], dt)
    T = qkv.size(0)
    inv = _inv_freq()
    assert torch.equal(qkv[:, (H + KV) * D:].reshape(T, KV, D), _t16(GOLD[f"{tag}_prologue_v"], dt))
    for name, off, nh in (("q", 0, H), ("k", H * D, KV)):
        x = qkv[:, off:off + nh * D].reshape(T, nh, D)
        want = _t16(GOLD[f"{tag}_prologue_{name}"], dt)
        assert torch.equal(_rope_hf(x, inv).view(torch.int16), want.view(torch.int16))
        # planted mistakes: a dtype-rounded inv_freq; a Qwen3-style q/k norm
        bad = _rope_hf(x, inv.to(dt).float())
        assert (bad.view(torch.int16) == want.view(torch.int16)).float().mean() < 0.95
        xf = x.float()
        normed = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + EPS)).to(dt)
        bad = _rope_hf(normed, inv)
        assert (bad.view(torch.int16) == want.view(torch.int16)).float().mean() < 0.5
