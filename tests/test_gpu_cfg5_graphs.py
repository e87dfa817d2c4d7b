"""Graph-replayed decode steps at configuration 5's widths, over a bf16 and
an FP8 (e4m3) pool of the full Qwen3-8B architecture (random init).

Configuration 5 serves prompts of up to 8192 tokens, so decode steps carry
block tables of up to 576 blocks (8192 + 1024 tokens in blocks of 16). For
each pool:

- DecodeGraphs.capture_all() with max_width 576 captures every (batch bucket,
  width bucket) graph: batches 1..16 by powers of two, widths 16 .. 512 and
  576;
- the buckets are replayed in an alternating order (widest, narrowest, second
  widest, ...), each over a step whose real rows fill all or all but one of
  its batch rows, with a widest table inside the bucket, random context
  lengths and eager work (the same padded step launched op by op) between
  replays; each replay's tokens must equal that eager step's, and every id
  must lie in the vocabulary;
- one request with an 8192-token prompt is served through chunked prefill
  (16 chunks of 512) and then decodes through the graphs (tables of 513+
  blocks: the 576 bucket), each replay checked the same way.

This runs the decode-graph code as it stands (argmax writing the graph's
token buffer, a blocking staging upload, kernel nodes only); the engine's own
check raises on any id outside [0, vocab). Reference: the engine step
nanoPD/engine/engine.py:42-113 and the fp16 KV cache of
nanoPD/engine/model_runner.py:24-31 (the FP8 pool has no reference
counterpart)."""
import numpy as np
import pytest
import torch

from nanopd_amd import paged_kernels as pk
from nanopd_amd.engine import Engine, Request
from nanopd_amd.graphs import BATCH_BUCKETS, DecodeGraphs
from nanopd_amd.qwen3 import QWEN3_8B, PagedQwen3, StepBatch

pytestmark = pytest.mark.gpu

BS = 16
MAX_WIDTH = 576
NUM_BLOCKS = 2048


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


@pytest.fixture(scope="module", params=["bf16", "fp8"])
def model(request, device):
    """Qwen3-8B shape; the pool filled with random K/V (e4m3 codes without
    NaN for the FP8 pool)."""
    fp8 = request.param == "fp8"
    m = PagedQwen3(QWEN3_8B, num_blocks=NUM_BLOCKS, block_size=BS, device=device, seed=0,
                   kv_cache_dtype="fp8" if fp8 else "auto")
    g = torch.Generator(device=device).manual_seed(17)
    for c in (m.k_cache, m.v_cache):
        if fp8:
            codes = torch.randint(0, 0x7E, c.shape, generator=g, device=device, dtype=torch.int32)
            sign = torch.randint(0, 2, c.shape, generator=g, device=device, dtype=torch.int32)
            c.view(torch.uint8).copy_((codes | (sign << 7)).to(torch.uint8))
            del codes, sign
        else:
            c.normal_(0.0, 0.5, generator=g)
    torch.cuda.synchronize()
    yield request.param, m
    del m
    torch.cuda.empty_cache()


def _alternating(widths):
    """Widest, narrowest, second widest, second narrowest, ..."""
    out, lo, hi = [], 0, len(widths) - 1
    while lo <= hi:
        out.append(widths[hi])
        if lo != hi:
            out.append(widths[lo])
        hi, lo = hi - 1, lo + 1
    return out


def test_every_bucket_up_to_576_blocks(device, model):
    tag, m = model
    graphs = DecodeGraphs(m, max_width=MAX_WIDTH)
    n = graphs.capture_all()
    widths = sorted({w for (_, w) in graphs._graphs})
    print(f"{tag}: captured {n} graphs, widths {widths}", flush=True)
    assert n == len(BATCH_BUCKETS) * len(widths) and widths[-1] == MAX_WIDTH
    rng = np.random.default_rng(5)
    replays = 0
    order = [(b, w) for k, w in enumerate(_alternating(widths))
             for b in (BATCH_BUCKETS if k % 2 else BATCH_BUCKETS[::-1])]
    for i, (bb, wb) in enumerate(order):
        # every other step leaves a padding row (where bb - 1 rows still map to bb)
        nreal = bb - 1 if i % 2 and bb >= 4 else bb
        # each row writes its new token into a block of its own; the context
        # blocks (read only) come from the others and may repeat
        last_blocks = rng.choice(NUM_BLOCKS, size=nreal, replace=False)
        readable = np.setdiff1d(np.arange(NUM_BLOCKS), last_blocks)
        positions, tables = [], []
        for r in range(nreal):
            width = wb if r == 0 else int(rng.integers(1, wb + 1))   # row 0: the bucket's width
            ctx = (width - 1) * BS + int(rng.integers(0, BS))        # position of the new token
            tab = list(rng.choice(readable, size=width - 1)) + [last_blocks[r]]
            positions.append(ctx)
            tables.append([int(x) for x in tab])
        last = [int(x) for x in rng.integers(0, QWEN3_8B.vocab, size=nreal)]
        print(f"{tag}: replay {i}: bucket ({bb}, {wb}), {nreal} rows, widest "
              f"{max(len(t) for t in tables)} blocks", flush=True)
        assert graphs.bucket(nreal, max(len(t) for t in tables)) == (bb, wb)
        got = graphs.decode(positions, tables, last)
        torch.cuda.synchronize()
        want = _eager_padded_tokens(m, positions, tables, last, bb, wb)
        torch.cuda.synchronize()
        assert got == want, f"{tag} replay {i} ({bb}, {wb}): {got} != {want}"
        assert all(0 <= t < QWEN3_8B.vocab for t in got)
        replays += 1
    assert replays == len(order)


def test_8192_token_prompt_then_graph_decodes(device, model):
    tag, m = model
    graphs = DecodeGraphs(m, max_width=MAX_WIDTH)
    eng = Engine(m, max_batch_size=16, budget=1024, chunk=512, graphs=graphs)
    g = torch.Generator().manual_seed(23)
    prompt = torch.randint(0, QWEN3_8B.vocab, (8192,), generator=g).tolist()
    seq = eng.add(Request(0, prompt, 6))
    prefill_steps, replays = 0, 0
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
            assert toks is not None, f"no graph for {len(pos)} rows / {max(map(len, tabs))} blocks"
            gr = graphs.capture(len(pos), max(len(t) for t in tabs))
            assert gr.width == MAX_WIDTH
            want = _eager_padded_tokens(m, pos, tabs, ids, gr.batch, gr.width)
            assert toks == want, f"{tag} replay {replays}: {toks} != {want}"
            replays += 1
        else:
            prefill_steps += 1
            batch = eng._pack(*rows)
            toks = m.forward(batch).argmax(-1).tolist() if batch.sample_rows.numel() else []
        eng.commit(plan, toks)      # raises on an id outside [0, vocab)
    print(f"{tag}: 8192-token prompt in {prefill_steps} chunks, {replays} graph decodes",
          flush=True)
    assert prefill_steps == 16 and replays == 5
    assert len(seq.output) == 6 and all(0 <= t < QWEN3_8B.vocab for t in seq.output)
    assert eng.blocks.num_free_blocks == NUM_BLOCKS
