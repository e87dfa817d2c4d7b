"""FP8 (OCP e4m3) KV pool on the GPU, through the C-ABI: the store is
bit-exact against the oracle's e4m3 rounding (itself pinned to
torch.float8_e4m3fn), and decode attention over the pool is within the
2-byte path's tolerance of the float64 oracle over the dequantised pool
(e4m3 values are exact in fp16 and bf16; the per-head scales are applied in
fp32, to the scores and to the output)."""
import math

import numpy as np
import pytest
import torch

from nanopd_amd import paged_kernels as pk
from oracle import paged_oracle as O
from tests.helpers import ATOL, f32, max_abs

pytestmark = pytest.mark.gpu


def _u8(t):
    return t.contiguous().view(torch.uint8).cpu().numpy()


def _scales(kvh, seed):
    g = torch.Generator().manual_seed(seed)
    return (0.01 + 0.05 * torch.rand(kvh, generator=g)).float()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("kvh,D,bs", [(2, 128, 16), (8, 128, 32), (4, 64, 16), (1, 256, 8)])
def test_store_bit_exact(device, dtype, kvh, D, bs):
    g = torch.Generator().manual_seed(kvh * D + bs)
    N, T = 20, 37
    kc = torch.full((N, kvh, bs, D), 0x5A, dtype=torch.uint8)
    vc = kc.clone()
    k = (torch.randn(T, kvh, D, generator=g) * 2).to(dtype)
    v = (torch.randn(T, kvh, D, generator=g) * 2).to(dtype)
    k[0, 0, :4] = torch.tensor([1e4, -1e4, 0.0, -0.0]).to(dtype)     # saturation, signed zeros
    slots = torch.randperm(N * bs, generator=g)[:T].to(torch.int32)
    slots[3] = -1
    slots[5] = N * bs + 7                                          # outside the pool: skipped
    ks, vs = _scales(kvh, 1), _scales(kvh, 2)
    want_k, want_v = kc.numpy().copy(), vc.numpy().copy()
    O.kv_store_slots_fp8(want_k, want_v, f32(k), f32(v), slots.numpy(), ks.numpy(), vs.numpy())
    dk, dv = kc.to(device).view(torch.float8_e4m3fn), vc.to(device).view(torch.float8_e4m3fn)
    pk.paged_kv_store_slots_fp8(dk, dv, k.to(device), v.to(device), slots.to(device),
                                ks.to(device), vs.to(device))
    torch.cuda.synchronize()
    assert np.array_equal(_u8(dk), want_k) and np.array_equal(_u8(dv), want_v)


def _fp8_case(device, seq_lens, H, kvh, bs, dtype, seed):
    """Random e4m3 pool (no NaN codes), shuffled tables, per-head scales."""
    g = torch.Generator().manual_seed(seed)
    nbs = [(s + bs - 1) // bs for s in seq_lens]
    mb, total = max(nbs + [1]), max(sum(nbs), 1)
    codes = torch.randint(0, 0x7E, (2, total, kvh, bs, 128), generator=g, dtype=torch.int32)
    codes = codes | (torch.randint(0, 2, codes.shape, generator=g, dtype=torch.int32) << 7)
    kc, vc = codes[0].to(torch.uint8), codes[1].to(torch.uint8)
    q = torch.randn(len(seq_lens), H, 128, generator=g).to(dtype)
    order = torch.randperm(total, generator=g)
    bt = torch.zeros(len(seq_lens), mb, dtype=torch.int32)
    o = 0
    for i, n in enumerate(nbs):
        bt[i, :n] = order[o:o + n]
        o += n
    sl = torch.tensor(seq_lens, dtype=torch.int32)
    # element magnitudes up to about 1.5 (like the 2-byte tests' values): the
    # absolute tolerance is then above the output's own rounding
    ks = (0.5 + torch.rand(kvh, generator=g)) / 448
    vs = (0.5 + torch.rand(kvh, generator=g)) / 448
    return q, kc, vc, bt, sl, ks.float(), vs.float(), mb


def _run_and_check(device, q, kc, vc, bt, sl, ks, vs, mb, bs, dtype):
    scale = 1 / math.sqrt(128)
    out = torch.full_like(q, float("nan")).to(device)
    pk.paged_attention_forward_fp8(out, q.to(device), kc.to(device).view(torch.float8_e4m3fn),
                                   vc.to(device).view(torch.float8_e4m3fn), bt.to(device),
                                   sl.to(device), scale, bs, mb, ks.to(device), vs.to(device))
    torch.cuda.synchronize()
    want = O.decode_attention(f32(q), O.fp8_pool_values(kc.numpy(), ks.numpy()),
                              O.fp8_pool_values(vc.numpy(), vs.numpy()), bt.numpy(), sl.numpy(),
                              scale)
    assert np.isfinite(f32(out)).all()
    err = max_abs(out, want)
    assert err <= ATOL[dtype], f"max-abs {err}"
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("G", [1, 2, 4, 6, 8, 12, 16])
def test_decode_group_sizes(device, dtype, G):
    kvh = 2
    args = _fp8_case(device, [1, 17, 300, 777, 0], G * kvh, kvh, 16, dtype, seed=G)
    _run_and_check(device, *args, 16, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("G", [3, 5, 7])
def test_decode_nan_rows_past_the_context(device, dtype, G):
    """Rows of a sequence's last block past its context hold e4m3 NaN codes
    (0x7F / 0xFF): the scores of those tokens are selected out and their V
    rows zeroed before the products, so the output stays finite and equal to
    the oracle's over the context alone (odd group sizes: padded head slots)."""
    kvh, bs = 2, 16
    q, kc, vc, bt, sl, ks, vs, mb = _fp8_case(device, [1, 17, 300, 777, 5, 40], G * kvh, kvh, bs,
                                              dtype, seed=100 + G)
    for i, n in enumerate(sl.tolist()):
        if n % bs:
            b = int(bt[i, (n - 1) // bs])
            kc[b, :, n % bs:, :] = 0x7F
            vc[b, :, n % bs:, :] = 0xFF
    _run_and_check(device, q, kc, vc, bt, sl, ks, vs, mb, bs, dtype)


@pytest.mark.parametrize("bs", [16, 32])
def test_decode_block_sizes_and_long_context(device, bs):
    args = _fp8_case(device, [4097, 64, 2500], 32, 8, bs, torch.bfloat16, seed=bs)
    _run_and_check(device, *args, bs, torch.bfloat16)


@pytest.mark.parametrize("H,kvh,bs", [(64, 4, 16), (32, 1, 32), (96, 3, 16)])
def test_decode_group_of_16_long_context(device, H, kvh, bs):
    """16 and 32 query heads per kv head over an FP8 pool (16-head units),
    up to 32k tokens."""
    args = _fp8_case(device, [32768, 1, 4097, 0], H, kvh, bs, torch.bfloat16, seed=H + bs)
    _run_and_check(device, *args, bs, torch.bfloat16)


@pytest.mark.parametrize("G", [4, 16])
def test_decode_rescale_mid_partition(device, G):
    """Scores that jump far above the earlier ones twice inside a partition
    (the first by about 2^16, the second by about 2^33 in log2 units of the
    softmax), over an FP8 pool: the probability reference formed from the
    first steps moves, and the probabilities already stored are rescaled."""
    from tests.test_gpu_decode import jumping_scores_case
    dtype = torch.bfloat16
    kvh = 2
    q, kc, vc, bt, sl, scale, mb = jumping_scores_case(device, G, kvh, [200, 700, 3000, 40], dtype,
                                                       seed=78 + G)
    ks = (kc.float().abs().amax(dim=(0, 2, 3)) / 448).clamp_min(1e-8).cpu()
    vs = (vc.float().abs().amax(dim=(0, 2, 3)) / 448).clamp_min(1e-8).cpu()
    k8 = (kc.float().cpu() / ks[None, :, None, None]).to(torch.float8_e4m3fn).view(torch.uint8)
    v8 = (vc.float().cpu() / vs[None, :, None, None]).to(torch.float8_e4m3fn).view(torch.uint8)
    _run_and_check(device, q.cpu(), k8, v8, bt.cpu(), sl.cpu(), ks, vs, mb, 16, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("G,bs", [(1, 16), (4, 16), (4, 32), (8, 16), (12, 16)])
def test_decode_many_units(device, dtype, G, bs):
    """40 sequences x 8 kv heads = 320 work units: groups of up to 8 heads
    take the four-wave form (two steps in flight), 12 heads the three-wave
    one; contexts from 0 to 9000 tokens, some past several partitions, rows
    past the context holding NaN codes."""
    g = np.random.default_rng(G * bs)
    lens = [int(x) for x in g.integers(0, 9000, 40)]
    lens[:4] = [0, 1, 17, 9000]
    q, kc, vc, bt, sl, ks, vs, mb = _fp8_case(device, lens, G * 8, 8, bs, dtype, seed=300 + G + bs)
    for i, n in enumerate(sl.tolist()):
        if n % bs:
            b = int(bt[i, (n - 1) // bs])
            kc[b, :, n % bs:, :] = 0x7F
            vc[b, :, n % bs:, :] = 0xFF
    _run_and_check(device, q, kc, vc, bt, sl, ks, vs, mb, bs, dtype)


def test_decode_long_context_merge_groups(device):
    """80 units with a 32769-token context and 9 other lengths: many
    partitions merged in groups of 16 (the last a group of one)."""
    lens = [32769, 5000, 17, 1, 2048, 2049, 4097, 100, 0, 9000]
    args = _fp8_case(device, lens, 16, 8, 16, torch.bfloat16, seed=2048)
    _run_and_check(device, *args, 16, torch.bfloat16)


def test_store_then_decode_matches_bf16_pool(device):
    """Config-2 shape, 16 sequences: the same bf16 K/V stored into a bf16 pool
    and into an fp8 pool; attention over the fp8 pool is the fp64 attention
    over its dequantised values, and stays close to the bf16 pool's."""
    g = torch.Generator().manual_seed(5)
    H, kvh, bs, S = 32, 8, 16, 16
    lens = torch.randint(128, 1500, (S,), generator=g).tolist()
    nbs = [(n + bs - 1) // bs for n in lens]
    N, mb = sum(nbs), max(nbs)
    order = torch.randperm(N, generator=g)
    bt = torch.zeros(S, mb, dtype=torch.int32)
    slots = []
    o = 0
    for i, (n, nb) in enumerate(zip(lens, nbs)):
        bt[i, :nb] = order[o:o + nb]
        o += nb
        slots += [int(bt[i, p // bs]) * bs + p % bs for p in range(n)]
    T = len(slots)
    k = (torch.randn(T, kvh, 128, generator=g) * 0.5).to(torch.bfloat16).to(device)
    v = (torch.randn(T, kvh, 128, generator=g) * 0.5).to(torch.bfloat16).to(device)
    sm = torch.tensor(slots, dtype=torch.int32, device=device)
    ks = torch.full((kvh,), 2.0 / 448, device=device)
    vs = torch.full((kvh,), 2.0 / 448, device=device)
    k8 = torch.zeros((N, kvh, bs, 128), dtype=torch.float8_e4m3fn, device=device)
    v8 = torch.zeros_like(k8)
    k16 = torch.zeros((N, kvh, bs, 128), dtype=torch.bfloat16, device=device)
    v16 = torch.zeros_like(k16)
    pk.paged_kv_store_slots_fp8(k8, v8, k, v, sm, ks, vs)
    pk.paged_kv_store_slots(k16, v16, k, v, sm)
    q = (torch.randn(S, H, 128, generator=g) * 0.5).to(torch.bfloat16).to(device)
    sl = torch.tensor(lens, dtype=torch.int32, device=device)
    btd = bt.to(device)
    o8, o16 = torch.empty_like(q), torch.empty_like(q)
    pk.paged_attention_forward_fp8(o8, q, k8, v8, btd, sl, 128 ** -0.5, bs, mb, ks, vs)
    pk.paged_attention_forward(o16, q, k16, v16, btd, sl, 128 ** -0.5, bs, mb)
    torch.cuda.synchronize()
    want = O.decode_attention(f32(q), O.fp8_pool_values(_u8(k8), ks.cpu().numpy()),
                              O.fp8_pool_values(_u8(v8), vs.cpu().numpy()), bt.numpy(),
                              sl.cpu().numpy(), 128 ** -0.5)
    assert max_abs(o8, want) <= ATOL[torch.bfloat16]
    # e4m3 keeps 3 mantissa bits: the outputs move by about 2^-5 of the V values
    assert (o8.float() - o16.float()).abs().max().item() <= 0.05


def test_argument_checks(device):
    q = torch.zeros(1, 8, 64, dtype=torch.bfloat16, device=device)
    kc = torch.zeros(4, 2, 16, 64, dtype=torch.float8_e4m3fn, device=device)
    sc = torch.ones(2, device=device)
    bt = torch.zeros(1, 1, dtype=torch.int32, device=device)
    sl = torch.ones(1, dtype=torch.int32, device=device)
    with pytest.raises(RuntimeError, match="head_dim"):
        pk.paged_attention_forward_fp8(torch.empty_like(q), q, kc, kc, bt, sl, 0.1, 16, 1, sc, sc)
    kc = torch.zeros(4, 2, 8, 128, dtype=torch.float8_e4m3fn, device=device)
    q = torch.zeros(1, 8, 128, dtype=torch.bfloat16, device=device)
    with pytest.raises(RuntimeError, match="block_size"):
        pk.paged_attention_forward_fp8(torch.empty_like(q), q, kc, kc, bt, sl, 0.1, 8, 1, sc, sc)
    with pytest.raises(RuntimeError, match="k_scale"):
        pk.paged_attention_forward_fp8(torch.empty_like(q), q, kc, kc, bt, sl, 0.1, 8, 1,
                                       torch.ones(3, device=device), sc)


def _fp8_prefill_case(device, prefixes, chunks, H, kvh, dtype, seed, bs=16, D=128):
    """Random e4m3 pool (no NaN codes) with per-head scales, shuffled tables
    of prefix + chunk blocks, and the chunks' queries packed varlen."""
    g = torch.Generator().manual_seed(seed)
    ctx = [p + c for p, c in zip(prefixes, chunks)]
    nbs = [(n + bs - 1) // bs for n in ctx]
    total = sum(nbs) + 3
    codes = torch.randint(0, 0x7E, (2, total, kvh, bs, D), generator=g, dtype=torch.int32)
    codes = codes | (torch.randint(0, 2, codes.shape, generator=g, dtype=torch.int32) << 7)
    kc, vc = codes[0].to(torch.uint8), codes[1].to(torch.uint8)
    order = torch.randperm(total, generator=g)
    bt = torch.zeros(len(ctx), max(nbs), dtype=torch.int32)
    o = 0
    for s, n in enumerate(nbs):
        bt[s, :n] = order[o:o + n]
        o += n
    q = (torch.randn(sum(chunks), H, D, generator=g) * 0.5).to(dtype)
    cu = torch.tensor([0] + list(np.cumsum(chunks)), dtype=torch.int32)
    ks = (0.5 + torch.rand(kvh, generator=g)) / 448
    vs = (0.5 + torch.rand(kvh, generator=g)) / 448
    return q, kc, vc, bt, cu, torch.tensor(ctx, dtype=torch.int32), ks.float(), vs.float(), max(chunks)


def _prefill_run_and_check(device, q, kc, vc, bt, cu, ctx, ks, vs, max_q, dtype):
    scale = 1 / math.sqrt(q.size(-1))
    out = torch.full_like(q, float("nan")).to(device)
    pk.paged_prefill_attention_fp8(out, q.to(device), kc.to(device).view(torch.float8_e4m3fn),
                                   vc.to(device).view(torch.float8_e4m3fn), bt.to(device),
                                   cu.to(device), ctx.to(device), scale, kc.size(2), bt.size(1),
                                   max_q, ks.to(device), vs.to(device))
    torch.cuda.synchronize()
    want = O.prefill_attention(f32(q), O.fp8_pool_values(kc.numpy(), ks.numpy()),
                               O.fp8_pool_values(vc.numpy(), vs.numpy()), bt.numpy(), cu.numpy(),
                               ctx.numpy(), scale)
    assert np.isfinite(f32(out)).all()
    err = max_abs(out, want)
    assert err <= ATOL[dtype], f"max-abs {err}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("G", [1, 2, 4, 6])
def test_prefill_group_sizes(device, dtype, G):
    """Every heads-per-workgroup tiling (1, 2, 4) over an FP8 pool, with an
    empty prefix, a ragged chunk and a key range long enough to be split."""
    kvh = 2
    case = _fp8_prefill_case(device, [0, 100, 1500], [64, 37, 200], G * kvh, kvh, dtype, seed=G)
    _prefill_run_and_check(device, *case, dtype)


@pytest.mark.parametrize("hd", [64, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_head_dims_64_and_256(device, hd, dtype):
    """Head dims 64 (prefill_kernel, the 1700-key range in key splits) and
    256 (prefill_generic_kernel) over an FP8 pool: empty and paged prefixes,
    ragged chunks, a decode row."""
    case = _fp8_prefill_case(device, [0, 100, 1500, 77], [64, 37, 200, 1], 8, 2, dtype,
                             seed=hd, D=hd)
    _prefill_run_and_check(device, *case, dtype)


def test_prefill_config3_shape(device):
    """Configuration 3's chunks and prefixes (4 x 512 on {0, 512, 1536, 3072}),
    Qwen3-8B heads, over an FP8 pool."""
    case = _fp8_prefill_case(device, [0, 512, 1536, 3072], [512] * 4, 32, 8, torch.bfloat16,
                             seed=3)
    _prefill_run_and_check(device, *case, torch.bfloat16)


def test_prefill_fp8_argument_checks(device):
    case = _fp8_prefill_case(device, [0], [16], 8, 2, torch.bfloat16, seed=5)
    q, kc, vc, bt, cu, ctx, ks, vs, max_q = case
    dk, dv = kc.to(device).view(torch.float8_e4m3fn), vc.to(device).view(torch.float8_e4m3fn)
    out = torch.empty_like(q).to(device)
    args = (out, q.to(device), dk, dv, bt.to(device), cu.to(device), ctx.to(device), 0.1, 16,
            bt.size(1), max_q)
    with pytest.raises(RuntimeError):   # one scale per kv head
        pk.paged_prefill_attention_fp8(*args, ks[:1].to(device), vs.to(device))
    with pytest.raises(RuntimeError):   # 2-byte caches are not FP8 pools
        pk.paged_prefill_attention_fp8(out, q.to(device), dk.to(torch.bfloat16),
                                       dv.to(torch.bfloat16), *args[4:], ks.to(device),
                                       vs.to(device))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hd", [64, 128, 256])
def test_fused_prologue_fp8_bytes(device, dtype, hd):
    """The fused q/k-norm + RoPE prologue into an FP8 pool writes the same
    bytes as the 2-byte prologue followed by the FP8 store of its K/V rows,
    and the same q; negative slots leave the pool untouched (head dims 64,
    128, 256)."""
    g = torch.Generator(device=device).manual_seed(11 + hd)
    T, H, KV, N, bs = 45, 16, 4, 32, 16
    width = (H + 2 * KV) * hd
    qkv = (torch.randn(T, width + 8, generator=g, device=device) * 1.5).to(dtype)[:, :width]
    qw = (1.0 + 0.2 * torch.randn(hd, generator=g, device=device)).to(dtype)
    kw = (1.0 + 0.2 * torch.randn(hd, generator=g, device=device)).to(dtype)
    slots = torch.randperm(N * bs, generator=g, device=device)[:T].to(torch.int32)
    slots[::7] = -1
    pos = torch.randint(0, 40000, (T,), generator=g, device=device, dtype=torch.int32)
    inv_freq = 1.0 / (1.0e6 ** (torch.arange(0, hd, 2, dtype=torch.float32, device=device) / hd))
    ks = (0.01 + 0.05 * torch.rand(KV, generator=g, device=device)).float()
    vs = (0.01 + 0.05 * torch.rand(KV, generator=g, device=device)).float()
    # 2-byte prologue into a 2-byte pool, then the FP8 store of the stored rows
    kc = torch.zeros(N, KV, bs, hd, dtype=dtype, device=device)
    vc = torch.zeros_like(kc)
    q2 = torch.empty(T, H, hd, dtype=dtype, device=device)
    pk.qk_norm_rope_store(q2, kc, vc, qkv, slots, pos, inv_freq, qw, kw, 1e-6)
    keep = slots >= 0
    sl = slots[keep].long()
    k_rows = kc.permute(0, 2, 1, 3).reshape(N * bs, KV, hd)[sl]
    v_rows = vc.permute(0, 2, 1, 3).reshape(N * bs, KV, hd)[sl]
    want_k = torch.full((N, KV, bs, hd), 0x5A, dtype=torch.uint8, device=device)
    want_v = want_k.clone()
    pk.paged_kv_store_slots_fp8(want_k.view(torch.float8_e4m3fn), want_v.view(torch.float8_e4m3fn),
                                k_rows, v_rows, slots[keep].contiguous(), ks, vs)
    # fused FP8 prologue
    got_k = torch.full_like(want_k, 0x5A)
    got_v = torch.full_like(want_v, 0x5A)
    q8 = torch.empty_like(q2)
    pk.qk_norm_rope_store(q8, got_k.view(torch.float8_e4m3fn), got_v.view(torch.float8_e4m3fn), qkv,
                          slots, pos, inv_freq, qw, kw, 1e-6, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    assert torch.equal(q8, q2)
    assert torch.equal(got_k, want_k) and torch.equal(got_v, want_v)
