"""The Qwen2 caller side against Hugging Face transformers' own Qwen2, through
the fixture tests/golden/hf_qwen2.npz (tests/golden/make_hf_qwen2_golden.py:
transformers on the CPU, eager attention, from_pretrained in float16 and
bfloat16; configuration 1's head shape -- 12 query and 2 kv heads of 128, q/k/v
biases, no q/k norms, tied LM head). The reference's runner serves qwen2
models (nanoPD/engine/model_runner.py:53-58) and applies q_norm / k_norm only
where the attention module has them (:101-104).

- The norm-free fused prologue (npd_qk_norm_rope_store with null norm
  weights) on HF's biased q/k/v projection output against HF's q and k after
  apply_rotary_pos_emb: V bit-exact; q and k at least 75% bit-identical and
  within 2.5 ulps (of the model dtype) of each rotated pair's norm (the bound
  of tests/test_gpu_hf_parity.py: the kernel rotates in fp32 and rounds once,
  HF rounds cos, sin, both products and the sum).
- The same prologue against the unfused PyTorch composite PagedQwen3 runs
  with fused_prologue=False (fp32 RoPE, then paged_kv_store_slots): q and the
  stored k at least 98% bit-identical, V bit-exact.
- PagedQwen3 with the Qwen2 options and HF's weights over the paged kernels:
  chunked prefills on paged prefixes, mixed prefill + decode steps and pure
  decodes, teacher-forced with HF's greedy tokens, against HF's logits: max
  |diff| relative to max |logit| <= 1e-2 (fp16) / 3e-2 (bf16), argmax flips at
  most 1 in 20 rows."""
import numpy as np
import pytest
import torch

from nanopd_amd import paged_kernels as pk
from nanopd_amd.qwen3 import PagedQwen3, Qwen3Config, StepBatch
from tests.golden import hf_qwen2_weights as W

pytestmark = pytest.mark.gpu

GOLD = np.load("tests/golden/hf_qwen2.npz")
C = W.SMALL_HF
CFG = Qwen3Config(num_layers=C["num_hidden_layers"], hidden=C["hidden_size"],
                  num_heads=C["num_attention_heads"], num_kv_heads=C["num_key_value_heads"],
                  head_dim=W.HEAD_DIM, intermediate=C["intermediate_size"],
                  vocab=C["vocab_size"], rope_theta=C["rope_theta"], rms_eps=C["rms_norm_eps"],
                  qk_norm=False, qkv_bias=True, tie_word_embeddings=True)
BS = 16
DTYPES = {"fp16": (torch.float16, 2.0 ** -10), "bf16": (torch.bfloat16, 2.0 ** -7)}


def _t16(a: np.ndarray, dt, device) -> torch.Tensor:
    return torch.from_numpy(a.view(np.int16).copy()).view(dt).to(device)


def _logits(a: np.ndarray, dt) -> np.ndarray:
    return torch.from_numpy(a.view(np.int16).copy()).view(dt).float().numpy()


@pytest.fixture(scope="module", params=list(DTYPES))
def hf(request, device):
    """(tag, dtype, ulp at 1, PagedQwen3 with the Qwen2 options and the
    fixture's weights in dtype)."""
    tag = request.param
    dt, ulp = DTYPES[tag]
    m = PagedQwen3(CFG, num_blocks=96, block_size=BS, device=device, dtype=dt, seed=0)
    m.load_hf_state_dict(W.weights())
    assert m.lm_head is m.embed
    yield tag, dt, ulp, m
    del m
    torch.cuda.empty_cache()


def _prologue(model, qkv, dt, device, fused):
    T = qkv.size(0)
    H, KV, D = CFG.num_heads, CFG.num_kv_heads, CFG.head_dim
    kc = torch.zeros(8, KV, BS, D, dtype=dt, device=device)
    vc = torch.zeros_like(kc)
    q_out = torch.empty(T, H, D, dtype=dt, device=device)
    slots = torch.arange(T, dtype=torch.int32, device=device)          # blocks 0, 1, 2
    if fused:
        pk.qk_norm_rope_store(q_out, kc, vc, qkv, slots, slots.clone(), model.inv_freq, None, None,
                              CFG.rms_eps)
    else:   # the model's PyTorch prologue: fp32 RoPE, then the slot store
        freqs = slots.float()[:, None] * model.inv_freq[None, :]
        cos, sin = freqs.cos()[:, None, :], freqs.sin()[:, None, :]
        q_out.copy_(model._rope(qkv[:, :H * D].view(T, H, D), cos, sin))
        k = model._rope(qkv[:, H * D:(H + KV) * D].view(T, KV, D), cos, sin)
        pk.paged_kv_store_slots(kc, vc, k, qkv[:, (H + KV) * D:].view(T, KV, D), slots)
    torch.cuda.synchronize()
    k_got = kc.permute(0, 2, 1, 3).reshape(-1, KV, D)[:T]
    v_got = vc.permute(0, 2, 1, 3).reshape(-1, KV, D)[:T]
    return q_out, k_got, v_got


def test_norm_free_prologue_matches_hf(device, hf):
    tag, dt, ulp, model = hf
    qkv = _t16(GOLD[f"{tag}_prologue_qkv"], dt, device)
    q_out, k_got, v_got = _prologue(model, qkv, dt, device, fused=True)
    assert torch.equal(v_got, _t16(GOLD[f"{tag}_prologue_v"], dt, device))
    half = CFG.head_dim // 2
    for name, got in (("q", q_out), ("k", k_got)):
        want = _t16(GOLD[f"{tag}_prologue_{name}"], dt, device)
        same = (got.view(torch.int16) == want.view(torch.int16)).float().mean().item()
        wf = want.float()
        pair = torch.sqrt(wf[..., :half] ** 2 + wf[..., half:] ** 2).repeat(1, 1, 2)
        rel = ((got.float() - wf).abs() / pair.clamp_min(1e-30)).max().item()
        print(f"{tag} Qwen2 prologue {name}: {same:.2%} bit-identical to HF; max |diff| = "
              f"{rel / ulp:.2f} ulps of the rotated pair's norm")
        assert same >= 0.75 and rel <= 2.5 * ulp


def test_norm_free_prologue_matches_unfused_composite(device, hf):
    tag, dt, _, model = hf
    qkv = _t16(GOLD[f"{tag}_prologue_qkv"], dt, device)
    fq, fk, fv = _prologue(model, qkv, dt, device, fused=True)
    uq, uk, uv = _prologue(model, qkv, dt, device, fused=False)
    assert torch.equal(fv, uv)
    for nm, a, b in (("q", fq, uq), ("k", fk, uk)):
        same = (a.view(torch.int16) == b.view(torch.int16)).float().mean().item()
        assert same >= 0.98, f"{nm}: {same:.2%} bit-identical to the unfused composite"
        u = 2.0 ** -8 if dt == torch.bfloat16 else 2.0 ** -11
        assert ((a.float() - b.float()).abs() <= 2 * u * b.float().abs() + 1e-6).all()


def _steps():
    """The fixture's three sequences as mixed engine steps: (prefill chunk of a
    sequence or None, decodes [(seq, k)]); chunks of 128 tokens."""
    L = [len(GOLD[f"bf16_seq{i}_prompt"]) for i in range(3)]
    return [((0, 0, L[0]), []), ((1, 0, 128), []), ((1, 128, L[1]), [(0, 0)]),
            ((2, 0, 128), [(0, 1), (1, 0)]), ((2, 128, 256), [(0, 2), (1, 1)]),
            ((2, 256, L[2]), [(1, 2)]), (None, [(2, 0)]), (None, [(2, 1)]), (None, [(2, 2)])]


def test_paged_qwen2_matches_hf(device, hf):
    tag, dt, _, model = hf
    model.k_cache.zero_()
    model.v_cache.zero_()
    L = [len(GOLD[f"{tag}_seq{i}_prompt"]) for i in range(3)]
    tables = []
    nxt = 0
    for n in L:   # room for the prompt and 3 decode tokens
        nb = (n + 3 + BS - 1) // BS
        tables.append(list(range(nxt, nxt + nb)))
        nxt += nb
    worst, flips, total = 0.0, 0, 0
    for pre, decs in _steps():
        seqs, ids = [], []
        if pre is not None:
            i, a, e = pre
            seqs.append((e - a, a, tables[i]))
            ids += GOLD[f"{tag}_seq{i}_prompt"][a:e].tolist()
        for i, k in decs:
            seqs.append((1, L[i] + k, tables[i]))
            ids.append(int(GOLD[f"{tag}_seq{i}_decode_tokens"][k]))
        tp = seqs[0][0] if pre is not None else 0
        meta = pk.pack_metadata(seqs, BS, device, max_blocks_per_seq=max(len(t) for t in tables))
        b = StepBatch(input_ids=torch.tensor(ids, dtype=torch.int64, device=device), meta=meta,
                      num_prefill_seqs=1 if pre is not None else 0, num_prefill_tokens=tp,
                      sample_rows=None, max_prefill_q=tp)
        lg = model.forward(b).float().cpu().numpy()
        got, want = [], []
        if pre is not None:
            i, a, e = pre
            rows = GOLD[f"{tag}_seq{i}_rows"]
            sel = [j for j, r in enumerate(rows) if a <= r < e]
            got.append(lg[[rows[j] - a for j in sel]])
            want.append(_logits(GOLD[f"{tag}_seq{i}_prompt_logits"], dt)[sel])
        for j, (i, k) in enumerate(decs):
            got.append(lg[tp + j][None])
            want.append(_logits(GOLD[f"{tag}_seq{i}_decode_logits"], dt)[k][None])
        got, want = np.concatenate(got), np.concatenate(want)
        worst = max(worst, float(np.abs(got - want).max() / max(1.0, np.abs(want).max())))
        flips += int((got.argmax(-1) != want.argmax(-1)).sum())
        total += len(got)
    print(f"{tag} PagedQwen3 (Qwen2 options) vs HF Qwen2: worst relative logits diff {worst:.2e}, "
          f"argmax flips {flips}/{total}")
    assert worst <= (1e-2 if dt == torch.float16 else 3e-2)
    assert flips <= max(1, total // 20)
