"""Config 5's caller side on the GPU, A/B: the same random-weight Qwen3 (small
shapes, head_dim 128, GQA 4) through the engine with the HIP attention ops
and with a PyTorch fp32 restatement of the attention (gather the context
through the block table, causal softmax over prefix + chunk, as
ref_paged_attention does, PA/tests/test_paged_attention.py:33-71). The
reference pins config 5 only by generated tokens (test_mixed_batch.py:7-29);
here the logits of a mixed prefill + decode step are compared directly, and
the greedy tokens of a served batch must agree."""
import math

import pytest
import torch

from nanopd_amd import paged_kernels as pk
from nanopd_amd.engine import Engine, Request, make_requests, serve
from nanopd_amd.qwen3 import PagedQwen3, Qwen3Config, StepBatch

pytestmark = pytest.mark.gpu

SMALL = Qwen3Config(num_layers=3, hidden=1024, num_heads=16, num_kv_heads=4, head_dim=128,
                    intermediate=2048, vocab=4096, init_std=0.05)


def torch_attention(layer, q, kc, vc, b: StepBatch, out):
    """fp32 attention over each sequence's paged context (after the step's
    store): row i of a q_len-row sequence sits at position ctx - q_len + i."""
    m = b.meta
    cu = m.cu_seqlens_q.tolist()
    sl = m.seq_lens.tolist()
    bt = m.block_tables
    bs = kc.size(2)
    g = q.size(1) // kc.size(1)
    scale = 1.0 / math.sqrt(q.size(2))
    for s in range(len(sl)):
        a, e, ctx = cu[s], cu[s + 1], sl[s]
        nb = (ctx + bs - 1) // bs
        idx = bt[s, :nb].long()
        K = kc[idx].transpose(0, 1).reshape(kc.size(1), nb * bs, -1)[:, :ctx].float()
        V = vc[idx].transpose(0, 1).reshape(vc.size(1), nb * bs, -1)[:, :ctx].float()
        K = K.repeat_interleave(g, dim=0)
        V = V.repeat_interleave(g, dim=0)
        qs = q[a:e].float().transpose(0, 1)                          # [H, ql, D]
        sc = torch.matmul(qs, K.transpose(1, 2).contiguous()) * scale
        pos = ctx - (e - a) + torch.arange(e - a, device=q.device)
        mask = torch.arange(ctx, device=q.device)[None, :] > pos[:, None]
        sc = sc.masked_fill(mask[None], float("-inf"))
        out[a:e] = torch.matmul(torch.softmax(sc, dim=-1), V).transpose(0, 1).to(out.dtype)


def _model(device, attention=None, fused_prologue=True):
    return PagedQwen3(SMALL, num_blocks=512, block_size=16, device=device, seed=3,
                      attention=attention, fused_prologue=fused_prologue)


def _mixed_batch(model, device):
    """One prefill chunk of 200 tokens on a 300-token prefix (the prefix
    stored by an earlier chunk) and 5 decodes, packed prefill first."""
    torch.manual_seed(0)
    seqs, ids, rows = [], [], []
    table0 = list(range(40, 72))
    seqs.append((200, 300, table0))
    ids += torch.randint(0, SMALL.vocab, (200,)).tolist()
    rows.append(199)
    for i, ctx in enumerate([17, 64, 255, 400, 33]):
        t = list(range(100 + 40 * i, 100 + 40 * i + (ctx + 16) // 16))
        seqs.append((1, ctx, t))
        ids.append(int(torch.randint(0, SMALL.vocab, (1,))))
        rows.append(200 + i)
    meta = pk.pack_metadata(seqs, 16, device, max_blocks_per_seq=max(len(t) for _, _, t in seqs))
    return StepBatch(input_ids=torch.tensor(ids, device=device), meta=meta, num_prefill_seqs=1,
                     num_prefill_tokens=200, sample_rows=torch.tensor(rows, device=device),
                     max_prefill_q=200)


def test_mixed_step_logits_match_torch_attention(device):
    hip = _model(device)
    ref = _model(device, attention=torch_attention)
    # identical random prefix/context in both caches
    g = torch.Generator(device=device).manual_seed(9)
    kc = torch.randn(hip.k_cache.shape, generator=g, device=device, dtype=torch.float32) * 0.5
    vc = torch.randn(hip.v_cache.shape, generator=g, device=device, dtype=torch.float32) * 0.5
    for m in (hip, ref):
        m.k_cache.copy_(kc)
        m.v_cache.copy_(vc)
    del kc, vc
    b = _mixed_batch(hip, device)
    lh = hip.forward(b)
    lr = ref.forward(b)
    torch.cuda.synchronize()
    err = (lh - lr).abs().max().item()
    spread = lr.abs().max().item()
    print(f"logits max-abs {err:.3e} (|logits| max {spread:.2f})")
    assert err <= 2e-2 * max(1.0, spread)
    assert (lh.argmax(-1) == lr.argmax(-1)).float().mean().item() >= 5 / 6
    # layer 0's K/V come from identical inputs: the stores wrote identical caches
    assert torch.equal(hip.k_cache[0], ref.k_cache[0]) and torch.equal(hip.v_cache[0], ref.v_cache[0])


def test_fused_prologue_matches_pytorch_prologue(device):
    """qk_norm_rope_store against the PyTorch prologue (HF q/k norm, fp32
    RoPE, paged_kv_store_slots) inside the model: same step, same caches."""
    fused = _model(device)
    comp = _model(device, fused_prologue=False)
    b = _mixed_batch(fused, device)
    lf, lc = fused.forward(b), comp.forward(b)
    torch.cuda.synchronize()
    # layer 0 sees identical inputs: its K/V rows agree up to a rare
    # last-place rounding difference, V exactly
    assert torch.equal(fused.v_cache[0], comp.v_cache[0])
    d = (fused.k_cache[0].float() - comp.k_cache[0].float()).abs()
    assert (d == 0).float().mean().item() > 0.999 and d.max().item() <= 0.05
    err = (lf - lc).abs().max().item()
    spread = lc.abs().max().item()
    print(f"fused vs PyTorch prologue: logits max-abs {err:.3e} (|logits| max {spread:.2f})")
    assert err <= 1e-2 * max(1.0, spread)
    assert (lf.argmax(-1) == lc.argmax(-1)).float().mean().item() >= 5 / 6


def test_teacher_forced_steps_agree_with_torch_attention(device):
    """Two engines, HIP and PyTorch attention, run the same requests in
    lockstep; both consume the HIP engine's greedy tokens (teacher forcing),
    so every step has identical inputs and the logits must stay close over a
    whole served batch: chunked prefills, decodes, block allocation."""
    reqs = make_requests(6, seed=11, prompt_median=150, prompt_clip=(20, 700), out_median=12,
                         out_clip=(4, 24), vocab=SMALL.vocab)
    engs = [Engine(_model(device, attention=a), max_batch_size=4, budget=256, chunk=128)
            for a in (None, torch_attention)]
    seqs = [[e.add(Request(r.rid, list(r.prompt), r.max_new_tokens)) for r in reqs] for e in engs]
    worst, steps, flips = 0.0, 0, 0
    while engs[0].sched.has_work():
        preps = [e.prepare() for e in engs]
        assert (preps[0] is None) == (preps[1] is None)
        if preps[0] is None:
            continue
        (p0, b0), (p1, b1) = preps
        assert torch.equal(b0.input_ids, b1.input_ids) and b0.num_prefill_tokens == b1.num_prefill_tokens
        l0, l1 = engs[0].model.forward(b0), engs[1].model.forward(b1)
        toks = l0.argmax(-1).tolist() if b0.sample_rows.numel() else []
        if toks:
            worst = max(worst, ((l0 - l1).abs().max() / l1.abs().max().clamp_min(1.0)).item())
            flips += sum(int(a != b) for a, b in zip(toks, l1.argmax(-1).tolist()))
        for e, p in zip(engs, (p0, p1)):
            e.commit(p, toks)
        steps += 1
    total = sum(r.max_new_tokens for r in reqs)
    print(f"{steps} steps, worst relative logits diff {worst:.2e}, argmax flips {flips}/{total}")
    for e, ss in zip(engs, seqs):
        assert all(len(s.output) == s.req.max_new_tokens for s in ss)
        assert e.blocks.num_free_blocks == 512          # every block returned
    # bf16 attention outputs (P rounded to bf16 for the PV MFMA) against fp32,
    # through 3 random layers: ~1.5e-2 relative observed
    assert worst <= 3e-2
    assert flips <= 0.1 * total


def test_serve_reports_throughput(device):
    eng = Engine(_model(device), max_batch_size=4, budget=256, chunk=128)
    reqs = make_requests(5, seed=2, rate=50.0, prompt_median=100, prompt_clip=(20, 300),
                         out_median=8, out_clip=(4, 16), vocab=SMALL.vocab)
    res = serve(eng, reqs)
    assert res["requests"] == 5
    assert res["output_tokens"] == sum(r.max_new_tokens for r in reqs)
    assert res["tok_per_s"] > 0 and res["wall_s"] > 0


def test_fp8_pool_step_matches_torch_attention(device):
    """The model with an FP8 (e4m3) KV pool: the fused prologue stores e4m3
    bytes, the FP8 prefill and decode ops read them. Against the same model
    with the fp32 PyTorch attention over the dequantised pool (e4m3 * scale),
    after identical random prefix/context bytes in both pools: the logits agree
    as closely as the 2-byte pools' A/B, and the step's own K/V bytes are the
    same in both pools (layer 0 sees identical inputs)."""
    def torch_attention_fp8(model):
        def attend(layer, q, kc, vc, b, out):
            ks = model.k_scale[layer][None, :, None, None]
            vs = model.v_scale[layer][None, :, None, None]
            torch_attention(layer, q, kc.float() * ks, vc.float() * vs, b, out)
        return attend

    hip = PagedQwen3(SMALL, num_blocks=512, block_size=16, device=device, seed=3,
                     kv_cache_dtype="fp8")
    ref = PagedQwen3(SMALL, num_blocks=512, block_size=16, device=device, seed=3,
                     kv_cache_dtype="fp8")
    ref.attention = torch_attention_fp8(ref)
    g = torch.Generator(device=device).manual_seed(9)
    codes = torch.randint(0, 0x7E, hip.k_cache.shape, generator=g, device=device,
                          dtype=torch.int32) | (torch.randint(0, 2, hip.k_cache.shape, generator=g,
                                                              device=device, dtype=torch.int32) << 7)
    for m in (hip, ref):
        m.k_cache.view(torch.uint8).copy_(codes.to(torch.uint8))
        m.v_cache.view(torch.uint8).copy_(codes.flip(0).to(torch.uint8))
    del codes
    b = _mixed_batch(hip, device)
    lh = hip.forward(b)
    lr = ref.forward(b)
    torch.cuda.synchronize()
    assert torch.isfinite(lh).all()
    err = (lh - lr).abs().max().item()
    spread = lr.abs().max().item()
    print(f"fp8 pool: logits max-abs {err:.3e} (|logits| max {spread:.2f})")
    assert err <= 2e-2 * max(1.0, spread)
    assert (lh.argmax(-1) == lr.argmax(-1)).float().mean().item() >= 5 / 6
    assert torch.equal(hip.k_cache[0].view(torch.uint8), ref.k_cache[0].view(torch.uint8))
    assert torch.equal(hip.v_cache[0].view(torch.uint8), ref.v_cache[0].view(torch.uint8))


def test_fp8_pool_served_batch(device):
    """An engine over the FP8-pool model serves a small batch to completion
    (prefill chunks, decodes, graph-replayed decode steps) with finite logits
    and the requested output lengths."""
    from nanopd_amd.graphs import DecodeGraphs
    model = PagedQwen3(SMALL, num_blocks=512, block_size=16, device=device, seed=3,
                       kv_cache_dtype="fp8")
    reqs = make_requests(5, seed=5, prompt_median=120, prompt_clip=(20, 400), out_median=10,
                         out_clip=(4, 16), vocab=SMALL.vocab)
    eng = Engine(model, max_batch_size=4, budget=256, chunk=128,
                 graphs=DecodeGraphs(model, max_width=32))
    seqs = [eng.add(Request(r.rid, list(r.prompt), r.max_new_tokens)) for r in reqs]
    while eng.sched.has_work():
        eng.step()
    for r, s in zip(reqs, seqs):
        assert len(s.output) == r.max_new_tokens
