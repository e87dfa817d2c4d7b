"""Config 5's shape on the GPU: the full Qwen3-8B architecture (36 layers,
hidden 4096, 32 / 8 heads of 128, MLP 12288, vocab 151936, random init, bf16
pool) through the paged kernels, as ModelRunner.paged_forward runs it
(nanoPD/engine/model_runner.py:75-213).

- A mixed step (one 512-token prefill chunk on a 1024-token prefix and 15
  decodes of up to 3000 tokens) against the same model with fp32 PyTorch
  attention over the paged context (ref_paged_attention's computation,
  PA/tests/test_paged_attention.py:33-71, made causal over prefix + chunk).
- A short served batch (8 requests, chunked prefill, 16-way batch cap) with
  graph-replayed decode steps: every replay is checked against the same padded
  step launched kernel by kernel (identical tokens), every token id is inside
  the vocabulary and every request reaches its output length."""
import pytest
import torch

from nanopd_amd import paged_kernels as pk
from nanopd_amd.engine import Engine, Request, make_requests
from nanopd_amd.graphs import DecodeGraphs
from nanopd_amd.qwen3 import QWEN3_8B, PagedQwen3, StepBatch
from tests.test_gpu_e2e import torch_attention

pytestmark = pytest.mark.gpu

NUM_BLOCKS = 2048


@pytest.fixture(scope="module")
def model(device):
    m = PagedQwen3(QWEN3_8B, num_blocks=NUM_BLOCKS, block_size=16, device=device, seed=0)
    yield m
    del m
    torch.cuda.empty_cache()


def _mixed_batch(device):
    g = torch.Generator().manual_seed(5)
    seqs, ids, rows = [], [], []
    seqs.append((512, 1024, list(range(0, 96))))        # chunk on a 1024-token prefix
    ids += torch.randint(0, QWEN3_8B.vocab, (512,), generator=g).tolist()
    rows.append(511)
    nxt = 96
    for i in range(15):
        ctx = int(torch.randint(16, 3000, (1,), generator=g))
        nb = ctx // 16 + 1
        seqs.append((1, ctx, list(range(nxt, nxt + nb))))
        nxt += nb
        ids.append(int(torch.randint(0, QWEN3_8B.vocab, (1,), generator=g)))
        rows.append(512 + i)
    assert nxt <= NUM_BLOCKS
    meta = pk.pack_metadata(seqs, 16, device, max_blocks_per_seq=max(len(t) for _, _, t in seqs))
    return StepBatch(input_ids=torch.tensor(ids, device=device), meta=meta, num_prefill_seqs=1,
                     num_prefill_tokens=512, sample_rows=torch.tensor(rows, device=device),
                     max_prefill_q=512)


def _torch_attention_storage_precision(layer, q, kc, vc, b, out):
    """torch_attention with the rounding the reference's own attention has
    (SDPA in the model dtype, model_runner.py:168): scores and probabilities
    rounded to the storage type, fp32 accumulation."""
    def rnd(x):
        return x.to(out.dtype).float()
    m = b.meta
    cu, sl = m.cu_seqlens_q.tolist(), m.seq_lens.tolist()
    bs, g = kc.size(2), q.size(1) // kc.size(1)
    scale = q.size(2) ** -0.5
    for s in range(len(sl)):
        a, e, ctx = cu[s], cu[s + 1], sl[s]
        nb = (ctx + bs - 1) // bs
        idx = m.block_tables[s, :nb].long()
        K = kc[idx].transpose(0, 1).reshape(kc.size(1), nb * bs, -1)[:, :ctx].float()
        V = vc[idx].transpose(0, 1).reshape(vc.size(1), nb * bs, -1)[:, :ctx].float()
        K, V = K.repeat_interleave(g, dim=0), V.repeat_interleave(g, dim=0)
        qs = q[a:e].float().transpose(0, 1)
        sc = rnd(torch.matmul(qs, K.transpose(1, 2).contiguous()) * scale)
        pos = ctx - (e - a) + torch.arange(e - a, device=q.device)
        sc = sc.masked_fill(torch.arange(ctx, device=q.device)[None, :] > pos[:, None], float("-inf"))
        p = rnd(torch.softmax(sc, dim=-1))
        out[a:e] = torch.matmul(p, V).transpose(0, 1).to(out.dtype)


def test_qwen3_8b_mixed_step_matches_torch_attention(device, model):
    """Per layer, the HIP attention of the step (prefill chunk over its paged
    prefix, and 15 decodes) against fp32 attention over the same q and pool,
    within the bf16 tolerance (max-abs 1e-2, relative to values above 1).
    End to end, the logits after 36 layers stay as close to the fp32-attention
    model as the reference's own storage-precision attention does."""
    g = torch.Generator(device=device).manual_seed(9)
    for c in (model.k_cache, model.v_cache):
        c.copy_((torch.randn(c.shape, generator=g, device=device, dtype=torch.float32) * 0.5)
                .to(c.dtype))
    saved = (model.k_cache.clone(), model.v_cache.clone())
    b = _mixed_batch(device)

    errs = []

    def checking(layer, q, kc, vc, batch, out):
        model._paged_attention(layer, q, kc, vc, batch, out)
        ref = torch.empty(out.shape, dtype=torch.float32, device=out.device)
        torch_attention(layer, q, kc, vc, batch, ref)
        errs.append(((out.float() - ref).abs().max() / ref.abs().max().clamp_min(1.0)).item())

    def run(attention):
        model.k_cache.copy_(saved[0])
        model.v_cache.copy_(saved[1])
        model.attention = attention
        try:
            return model.forward(b)
        finally:
            model.attention = model._paged_attention

    lh = run(checking)
    lr = run(torch_attention)
    lf = run(_torch_attention_storage_precision)
    torch.cuda.synchronize()
    print(f"Qwen3-8B per-layer attention max-abs (rel. to values > 1): worst {max(errs):.2e} "
          f"over {len(errs)} layers")
    assert len(errs) == QWEN3_8B.num_layers and max(errs) <= 1e-2
    assert torch.isfinite(lh).all()
    spread = lr.abs().max().item()
    err = (lh - lr).abs().max().item()
    floor = (lf - lr).abs().max().item()
    agree = (lh.argmax(-1) == lr.argmax(-1)).float().mean().item()
    print(f"logits vs fp32 attention: HIP {err:.3e}, storage-precision reference {floor:.3e} "
          f"(|logits| max {spread:.2f}); HIP argmax agreement {agree:.2f}")
    assert err <= max(2.0 * floor, 2e-2 * spread)


def _eager_padded_tokens(model, positions, tables, last, batch, width):
    """The graph's padded step, launched op by op (same kernels, same shapes)."""
    n = len(positions)
    seqs = [(1, p, t) for p, t in zip(positions, tables)] + [(1, -1, [])] * (batch - n)
    meta = pk.pack_metadata(seqs, model.block_size, model.device, max_blocks_per_seq=width)
    ids = torch.tensor(list(last) + [0] * (batch - n), dtype=torch.int64, device=model.device)
    cfg = model.cfg
    ws = torch.zeros(pk.attention_workspace_bytes(batch, cfg.num_heads, cfg.num_kv_heads,
                                                  cfg.head_dim, model.block_size, width),
                     dtype=torch.uint8, device=model.device)
    b = StepBatch(input_ids=ids, meta=meta, num_prefill_seqs=0, num_prefill_tokens=0,
                  sample_rows=None, decode_workspace=ws)
    return model.forward(b).argmax(-1)[:n].tolist()


def test_qwen3_8b_served_batch_with_graphs(device, model):
    model.k_cache.zero_()
    model.v_cache.zero_()
    reqs = make_requests(8, seed=21, rate=1e9, prompt_median=300, prompt_clip=(32, 1500),
                         out_median=16, out_clip=(8, 32))
    graphs = DecodeGraphs(model, max_width=128)
    eng = Engine(model, max_batch_size=16, budget=1024, chunk=512, graphs=graphs)
    seqs = [eng.add(Request(r.rid, list(r.prompt), r.max_new_tokens)) for r in reqs]
    replays = 0
    while eng.sched.has_work():
        plan = eng.sched.schedule(0.0)
        if plan.prefill is None and not plan.decodes:
            continue
        rows = eng._rows(plan)
        _, sq, ids, _, _ = rows
        toks = None
        if plan.prefill is None:
            pos = [c for _, c, _ in sq]
            tabs = [t for _, _, t in sq]
            toks = graphs.decode(pos, tabs, ids)
            if toks is not None:
                g = graphs.capture(len(pos), max(len(t) for t in tabs))
                want = _eager_padded_tokens(model, pos, tabs, ids, g.batch, g.width)
                assert toks == want, f"replay {replays}: {toks} != {want}"
                replays += 1
        if toks is None:
            batch = eng._pack(*rows)
            toks = model.forward(batch).argmax(-1).tolist() if batch.sample_rows.numel() else []
        eng.commit(plan, toks)      # raises on an id outside [0, vocab)
    assert replays >= 8
    for r, s in zip(reqs, seqs):
        assert len(s.output) == r.max_new_tokens
        assert all(0 <= t < QWEN3_8B.vocab for t in s.output)
    assert eng.blocks.num_free_blocks == NUM_BLOCKS
