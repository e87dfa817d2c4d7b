"""Fused Qwen3 attention prologue (q/k RMSNorm + RoPE + paged K/V store)
against PyTorch composites of the same steps.

The reference runs HF Qwen3RMSNorm for q_norm / k_norm, HF
apply_rotary_pos_emb and paged_kv_store (nanoPD/engine/model_runner.py:97-115,
:142-146, :189-192). Two composites are checked:
- fp32 rotation (the kernel's order): bit-identical on at least 98% of the
  elements, the rest within the rounding that a one-ulp change of the fp32
  statistics or of cos / sin can cause;
- HF's rotation, which rounds cos / sin and each product to the storage dtype:
  within a few ulps.
V rows are copied, so the V cache must match bit for bit; slots that are
negative leave the pool untouched. Without norm weights (the Qwen2 / Llama
prologue: the reference applies q_norm / k_norm only where the attention has
them, nanoPD/engine/model_runner.py:101-104) the same composites without the
norm step."""
import pytest
import torch

from nanopd_amd import paged_kernels as pk

pytestmark = pytest.mark.gpu

D = 128


def hf_rms_norm(x, w, eps):
    """HF Qwen3RMSNorm: fp32 statistics, round, then times the weight."""
    xf = x.float()
    r = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return w * (xf * r).to(x.dtype)


def rope_fp32(x, cos, sin):
    h = x.size(-1) // 2
    xf = x.float()
    x1, x2 = xf[..., :h], xf[..., h:]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1).to(x.dtype)


def rope_hf(x, cos, sin):
    """HF apply_rotary_pos_emb: cos / sin in the model dtype, dtype arithmetic."""
    c = torch.cat([cos, cos], -1).to(x.dtype)
    s = torch.cat([sin, sin], -1).to(x.dtype)
    h = x.size(-1) // 2
    rot = torch.cat([-x[..., h:], x[..., :h]], dim=-1)
    return x * c + rot * s


def _case(device, dtype, T, H, KV, num_blocks, bs, pad=0, seed=0, max_pos=40000, D=D):
    g = torch.Generator(device=device).manual_seed(seed)
    width = (H + 2 * KV) * D
    base = torch.randn(T, width + pad, generator=g, device=device, dtype=torch.float32) * 1.5
    qkv = base.to(dtype)[:, :width]                         # token stride width + pad
    qw = (1.0 + 0.2 * torch.randn(D, generator=g, device=device)).to(dtype)
    kw = (1.0 + 0.2 * torch.randn(D, generator=g, device=device)).to(dtype)
    slots = torch.randperm(num_blocks * bs, generator=g, device=device)[:T].to(torch.int32)
    if T > 3:
        slots[::7] = -1                                       # not stored
    pos = torch.randint(0, max_pos, (T,), generator=g, device=device, dtype=torch.int32)
    inv_freq = 1.0 / (1.0e6 ** (torch.arange(0, D, 2, dtype=torch.float32, device=device) / D))
    return qkv, qw, kw, slots, pos, inv_freq


def _run(device, dtype, T, H, KV, num_blocks=64, bs=16, pad=0, seed=0, D=D, norms=True):
    qkv, qw, kw, slots, pos, inv_freq = _case(device, dtype, T, H, KV, num_blocks, bs, pad, seed,
                                              D=D)
    if not norms:
        qw = kw = None
    sentinel = torch.tensor(7.0, dtype=dtype)
    kc = torch.full((num_blocks, KV, bs, D), float(sentinel), dtype=dtype, device=device)
    vc = kc.clone()
    q = torch.empty(T, H, D, dtype=dtype, device=device)
    pk.qk_norm_rope_store(q, kc, vc, qkv, slots, pos, inv_freq, qw, kw, 1e-6)
    torch.cuda.synchronize()

    freqs = pos.float()[:, None] * inv_freq[None, :]
    cos, sin = freqs.cos()[:, None, :], freqs.sin()[:, None, :]
    qs = qkv[:, : H * D].reshape(T, H, D)
    ks = qkv[:, H * D:(H + KV) * D].reshape(T, KV, D)
    vs = qkv[:, (H + KV) * D:].reshape(T, KV, D)
    if norms:
        qn, kn = hf_rms_norm(qs, qw, 1e-6), hf_rms_norm(ks, kw, 1e-6)
    else:
        qn, kn = qs, ks
    ref = {"fp32": (rope_fp32(qn, cos, sin), rope_fp32(kn, cos, sin)),
           "hf": (rope_hf(qn, cos, sin), rope_hf(kn, cos, sin))}
    keep = slots >= 0
    sl = slots[keep].long()
    blk, off = sl // bs, sl % bs
    vref = torch.full_like(vc, float(sentinel))
    vref[blk, :, off] = vs[keep]
    k_got = kc[blk, :, off]                                   # [kept, KV, D]
    return {"q": (q, ref["fp32"][0], ref["hf"][0], qn),
            "k": (k_got, ref["fp32"][1][keep], ref["hf"][1][keep], kn[keep])}, kc, vc, vref


def _ulp(ref, dtype):
    mant = 7 if dtype == torch.bfloat16 else 10
    tiny = 2.0 ** -24 if dtype == torch.float16 else 1e-30
    e = torch.floor(torch.log2(ref.float().abs().clamp_min(tiny)))
    return torch.pow(2.0, e - mant)


def _check(res, kc, vc, vref, dtype, D):
    assert torch.equal(vc, vref), "v cache differs"
    # unit roundoff of the storage dtype
    u = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    h = D // 2
    for nm, (got, w32, whf, n) in res.items():
        nf = n.float()
        mag = nf.abs() + torch.cat([nf[..., h:], nf[..., :h]], -1).abs()
        # same steps; the fp32 mean (summation order) may move a normalised
        # input by one ulp, which the rotation carries into its output
        d = (got.float() - w32.float()).abs()
        tol = _ulp(w32, dtype) + 3 * u * mag
        assert (d <= tol).all(), f"{nm}: {(d - tol).max().item():.3e} beyond the fp32 composite"
        assert (d == 0).float().mean().item() >= 0.98, f"{nm}: too few exact elements"
        # HF rounds cos / sin, both products and the sum: |err| <= ~2u (|a| + |b|) + u |out|
        d = (got.float() - whf.float()).abs()
        tol = 2.5 * u * mag + 1.5 * u * whf.float().abs() + 1e-6
        assert (d <= tol).all(), f"{nm}: {(d - tol).max().item():.3e} beyond the HF composite bound"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T,H,KV,pad", [(1, 32, 8, 0), (37, 32, 8, 0), (512, 32, 8, 256),
                                        (300, 16, 4, 64), (64, 8, 8, 0)])
def test_matches_composites(device, dtype, T, H, KV, pad):
    print(f"qk_norm_rope_store dtype={dtype} T={T} H={H} KV={KV} pad={pad}", flush=True)
    res, kc, vc, vref = _run(device, dtype, T, H, KV, pad=pad, seed=T + H)
    _check(res, kc, vc, vref, dtype, D)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hd", [64, 256])
@pytest.mark.parametrize("T,H,KV,pad", [(1, 5, 1, 0), (37, 5, 1, 0), (130, 16, 4, 32),
                                        (257, 8, 2, 0)])
def test_head_dims_64_and_256(device, dtype, hd, T, H, KV, pad):
    """D 64: two rows per wave (an odd row count leaves the last wave half
    idle); D 256: two rotate-half pairs per lane."""
    print(f"qk_norm_rope_store D={hd} dtype={dtype} T={T} H={H} KV={KV} pad={pad}", flush=True)
    res, kc, vc, vref = _run(device, dtype, T, H, KV, pad=pad, seed=T + H + hd, D=hd)
    _check(res, kc, vc, vref, dtype, hd)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hd", [64, 128, 256])
@pytest.mark.parametrize("T,H,KV,pad", [(1, 12, 2, 0), (45, 12, 2, 0), (300, 12, 2, 64),
                                        (129, 32, 8, 0)])
def test_norm_free_matches_composites(device, dtype, hd, T, H, KV, pad):
    """No q/k norm weights: RoPE of the projection output (12 / 2 heads is
    configuration 1's Qwen2-1.5B shape)."""
    print(f"rope_store (no norms) D={hd} dtype={dtype} T={T} H={H} KV={KV} pad={pad}", flush=True)
    res, kc, vc, vref = _run(device, dtype, T, H, KV, pad=pad, seed=T + H + hd + 1, D=hd,
                             norms=False)
    _check(res, kc, vc, vref, dtype, hd)


def test_one_norm_weight_is_refused(device):
    dtype = torch.bfloat16
    kc = torch.zeros(4, 2, 16, D, dtype=dtype, device=device)
    q = torch.empty(3, 12, D, dtype=dtype, device=device)
    qkv = torch.zeros(3, 16 * D, dtype=dtype, device=device)
    i32 = torch.zeros(3, dtype=torch.int32, device=device)
    w = torch.ones(D, dtype=dtype, device=device)
    f = torch.ones(D // 2, device=device)
    with pytest.raises(RuntimeError, match="both norm weights"):
        pk.qk_norm_rope_store(q, kc, kc.clone(), qkv, i32, i32, f, w, None, 1e-6)


def test_untouched_slots_and_empty(device):
    dtype = torch.bfloat16
    res, kc, vc, vref = _run(device, dtype, 40, 32, 8, num_blocks=8, bs=16)
    # 40 tokens, every 7th skipped: 34 of the 128 slots written, the rest keep the sentinel
    assert (kc != 7.0).any(-1).sum().item() == 34 * 8
    assert torch.equal(vc, vref)
    kc0 = kc.clone()
    q = res["q"][0]
    pk.qk_norm_rope_store(q[:0], kc, vc, torch.empty(0, 48 * D, dtype=dtype, device=device),
                          torch.empty(0, dtype=torch.int32, device=device),
                          torch.empty(0, dtype=torch.int32, device=device),
                          torch.ones(D // 2, device=device), torch.ones(D, dtype=dtype, device=device),
                          torch.ones(D, dtype=dtype, device=device), 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(kc, kc0)


def test_python_checks(device):
    dtype = torch.bfloat16
    kc = torch.zeros(4, 8, 16, D, dtype=dtype, device=device)
    q = torch.empty(3, 32, D, dtype=dtype, device=device)
    qkv = torch.zeros(3, 48 * D, dtype=dtype, device=device)
    i32 = torch.zeros(3, dtype=torch.int32, device=device)
    w = torch.ones(D, dtype=dtype, device=device)
    f = torch.ones(D // 2, device=device)
    with pytest.raises(RuntimeError, match="qkv must be"):
        pk.qk_norm_rope_store(q, kc, kc.clone(), qkv[:, :-D], i32, i32, f, w, w, 1e-6)
    with pytest.raises(RuntimeError, match="int32"):
        pk.qk_norm_rope_store(q, kc, kc.clone(), qkv, i32.long(), i32, f, w, w, 1e-6)
    with pytest.raises(RuntimeError, match="inv_freq"):
        pk.qk_norm_rope_store(q, kc, kc.clone(), qkv, i32, i32, f.half(), w, w, 1e-6)
