"""CPU bounds checks of every device store of the serving path, through the
address model in tests/address_model.py (no GPU needed).

Shapes covered:
- every HIP-graph bucket of config 5 (batch 1/2/4/8/16 x table widths
  16 ... 576), real rows plus padding rows (position -1, context 0), with the
  2-byte and the FP8 pool's partition rules;
- every step of a simulated config-5 run (256 seeded requests through the
  engine's own Scheduler and BlockSpaceManager on a virtual clock), eager
  mixed steps and graph-replayed decode steps alike, both pool types;
- configurations 1-4 and batches beyond the inline work list (> 64
  sequences).
The sizes are the ones the host allocates (graphs.py, qwen3.py, engine.py),
and the workspace sizes come from the built library's own size functions.
A planted mistake (a buffer one row or one byte short) must be reported."""
from __future__ import annotations

import numpy as np
import pytest

from nanopd_amd import _lib
from nanopd_amd.block_manager import BlockSpaceManager
from nanopd_amd.engine import Scheduler, Sequence, make_requests
from tests import address_model as A

H, KV, D, BS = 32, 8, 128, 16
GRAPH_BATCHES = (1, 2, 4, 8, 16)
MAX_WIDTH = (8192 + 1024 + 15) // 16          # bench.py's graph width cap
GRAPH_WIDTHS = (16, 32, 64, 128, 256, 512, MAX_WIDTH)
NUM_BLOCKS = 12288                            # bench.py's config-5 pool


def _decode_ws(S, max_bps, bs=BS, h=H, kv=KV, d=D):
    return int(_lib.load().npd_paged_attention_workspace_size(S, h, kv, d, bs, max_bps))


def _prefill_ws(S, tq, mq, mctx, h=H):
    return int(_lib.load().npd_paged_prefill_workspace_size(S, tq, h, D, mq, mctx))


def check_decode(W, S, max_bps, seq_lens, fp8, out_rows=None, ws_bytes=None, h=H, kv=KV, bs=BS,
                 d=D):
    L = A.decode_host(S, h, kv, bs, max_bps, fp8, D=d)
    out = A.Buf("decode out", (out_rows if out_rows is not None else S) * h * d * 2)
    ws = A.Buf("decode workspace",
               ws_bytes if ws_bytes is not None else _decode_ws(S, max_bps, bs, h, kv, d))
    A.decode(W, L, out, ws, np.asarray(seq_lens), h * d, d, D=d)
    return L


def check_graph_step(W, bb, wb, real_lens, fp8):
    """A graph replay of bucket (bb, wb): real rows, then padding rows."""
    n = len(real_lens)
    lens = list(real_lens) + [0] * (bb - n)
    # the graph's metadata kernel: bb sequences of one token, tables of wb
    bufs = {k: A.Buf(f"graph {k}", 4 * m) for k, m in
            (("cu", bb + 1), ("seq_lens", bb), ("tables", bb * wb), ("positions", bb),
             ("slots", bb), ("token_seq", bb))}
    desc = np.zeros(3 * bb, np.int64)
    desc[0::3] = 1
    desc[1::3] = [x - 1 for x in lens]
    desc[2::3] = wb
    A.pack_metadata(W, bufs, desc, bb, bb, wb)
    elt = 1 if fp8 else 2
    cache = A.Buf("layer cache", NUM_BLOCKS * KV * BS * D * elt)
    slots = np.array([x - 1 if x > 0 else -1 for x in lens])   # any slot inside the pool
    A.prologue(W, A.Buf("graph q_out", bb * H * D * 2), cache, cache, slots, bb, H, KV,
               NUM_BLOCKS, BS, H * D, fp8)
    check_decode(W, bb, wb, lens, fp8,
                 ws_bytes=_decode_ws(bb, wb))   # graphs.py allocates exactly this


@pytest.mark.parametrize("fp8", [False, True])
def test_graph_buckets(fp8):
    rng = np.random.default_rng(7)
    W = A.Writes()
    for bb in GRAPH_BATCHES:
        for wb in GRAPH_WIDTHS:
            cap = wb * BS
            for n in sorted({0, 1, bb // 2, bb}):
                check_graph_step(W, bb, wb, [cap] * n, fp8)                      # longest
                check_graph_step(W, bb, wb, list(rng.integers(1, cap + 1, n)), fp8)
                check_graph_step(W, bb, wb, [1] * n, fp8)
                check_graph_step(W, bb, wb, [min(cap, 16 * k + 1) for k in range(n)], fp8)
    W.check()
    assert W.count > 0


def simulate_serve(n_requests=256, seed=5, step_s=0.0062, per_token_s=2e-5):
    """Steps of config 5 through the engine's Scheduler / BlockSpaceManager on
    a virtual clock: [(prefill (q_len, ctx, table) or None, [(pos, table)])]."""
    reqs = sorted(make_requests(n_requests, seed=seed), key=lambda r: r.arrival)
    blocks = BlockSpaceManager(BS, NUM_BLOCKS)
    sched = Scheduler(blocks, 16, 1024, 512)
    now, i, steps = 0.0, 0, []
    while i < len(reqs) or sched.has_work():
        while i < len(reqs) and reqs[i].arrival <= now:
            sched.waiting.append(Sequence(reqs[i]))
            i += 1
        if not sched.has_work():
            now = reqs[i].arrival
            continue
        plan = sched.schedule(now)
        if plan.prefill is None and not plan.decodes:
            continue
        pre = None
        if plan.prefill is not None:
            a, e = plan.chunk
            pre = (e - a, a, list(blocks.block_table(plan.prefill.req.rid)))
        decs = []
        for s in plan.decodes:
            assert blocks.append_slot(s.req.rid, s.num_computed) is None   # no forks here
            decs.append((s.num_computed, list(blocks.block_table(s.req.rid))))
        # commit, as Engine.commit does
        if plan.prefill is not None:
            s = plan.prefill
            s.num_computed = plan.chunk[1]
            if plan.is_last:
                s.output.append(0)
                sched.running.append(s)
        for s in plan.decodes:
            s.output.append(0)
            s.num_computed += 1
        steps.append((pre, decs))
        now += step_s + per_token_s * (pre[0] if pre else 0)
    return steps


def bucket(batch, width):
    """DecodeGraphs.bucket of graphs.py."""
    bb = next((x for x in GRAPH_BATCHES if x >= batch), None)
    if bb is None or width > MAX_WIDTH:
        return None
    wb = 16
    while wb < width:
        wb *= 2
    return bb, min(wb, MAX_WIDTH)


def check_eager_step(W, pre, decs, fp8):
    """One eager engine step (qwen3.py forward + engine.py _pack)."""
    seqs = ([pre] if pre else []) + [(1, p, t) for p, t in decs]
    tp = pre[0] if pre else 0
    T = tp + len(decs)
    ns = len(seqs)
    mb = max(len(t) for _, _, t in seqs)
    total_q = sum(q for q, _, _ in seqs)
    bufs = {k: A.Buf(f"meta {k}", 4 * m) for k, m in
            (("cu", ns + 1), ("seq_lens", ns), ("tables", ns * mb), ("positions", total_q),
             ("slots", total_q), ("token_seq", total_q))}
    desc = np.array([[q, c, len(t)] for q, c, t in seqs]).ravel()
    A.pack_metadata(W, bufs, desc, ns, total_q, mb)
    elt = 1 if fp8 else 2
    cache = A.Buf("layer cache", NUM_BLOCKS * KV * BS * D * elt)
    slots = []
    for q, c, t in seqs:
        for k in range(q):
            pos = c + k
            slots.append(t[pos // BS] * BS + pos % BS if pos // BS < len(t) else -1)
    A.prologue(W, A.Buf("q", T * H * D * 2), cache, cache, np.array(slots), T, H, KV, NUM_BLOCKS,
               BS, H * D, fp8)
    max_sl = max(q + c for q, c, _ in seqs)
    if pre:
        L = A.prefill_host(1, H, KV, BS, mb, tp, max_sl)
        ws = A.Buf("prefill workspace", _prefill_ws(1, tp, tp, max_sl))
        assert ws.nbytes == L.total
        A.prefill(W, L, A.Buf("attn[:tp]", tp * H * D * 2), ws, np.array([0, tp]),
                  np.array([pre[0] + pre[1]]), H * D, D)
    if decs:
        check_decode(W, len(decs), mb, [p + 1 for p, _ in decs], fp8)


@pytest.mark.parametrize("fp8", [False, True])
def test_config5_served_steps(fp8):
    steps = simulate_serve()
    W = A.Writes()
    n_graph = n_eager = 0
    for pre, decs in steps:
        if pre is None and decs:
            key = bucket(len(decs), max(len(t) for _, t in decs))
            if key is not None:
                check_graph_step(W, key[0], key[1], [p + 1 for p, _ in decs], fp8)
                n_graph += 1
                continue
        check_eager_step(W, pre, decs, fp8)
        n_eager += 1
    W.check()
    assert n_graph > 1000 and n_eager > 200, (n_graph, n_eager)


def test_configs_1_to_4_and_large_batches():
    W = A.Writes()
    rng = np.random.default_rng(3)
    # config 1 (12/2 heads, fp16), 2, 3's decode part, 4
    check_decode(W, 4, 32, [17, 64, 200, 511], False, h=12, kv=2)
    check_decode(W, 64, 256, rng.integers(128, 4097, 64), False)
    check_decode(W, 64, 256, rng.integers(128, 4097, 64), True)
    check_decode(W, 48, 128, rng.integers(256, 2049, 48), False)
    check_decode(W, 8, 2049, [k * 1024 + 1 for k in (8, 12, 16, 20, 24, 28, 32, 32)], False)
    check_decode(W, 8, 2049, [k * 1024 + 1 for k in (8, 12, 16, 20, 24, 28, 32, 32)], True)
    # beyond the inline work list: the schedule kernel's list
    check_decode(W, 96, 256, rng.integers(1, 4097, 96), False)
    check_decode(W, 300, 64, np.concatenate([[0], rng.integers(1, 1025, 299)]), True)
    # config 3's prefill: 4 chunks of 512 on prefixes {0, 512, 1536, 3072}
    pre = [0, 512, 1536, 3072]
    cu = np.array([0, 512, 1024, 1536, 2048])
    ctx = np.array([p + 512 for p in pre])
    L = A.prefill_host(4, H, KV, BS, 224, 512, 3584)
    A.prefill(W, L, A.Buf("out", 2048 * H * D * 2), A.Buf("ws", _prefill_ws(4, 2048, 512, 3584)),
              cu, ctx, H * D, D)
    # a wide batch of prefills (fixed-grid path): 70 chunks of 1..300 rows
    q = rng.integers(1, 301, 70)
    cu = np.concatenate([[0], np.cumsum(q)])
    c = q + rng.integers(0, 3000, 70)
    mb = int((c.max() + BS - 1) // BS)
    L = A.prefill_host(70, H, KV, BS, mb, int(q.max()), int(c.max()))
    assert 70 * L.tiles > 64
    A.prefill(W, L, A.Buf("out", int(cu[-1]) * H * D * 2),
              A.Buf("ws", _prefill_ws(70, int(cu[-1]), int(q.max()), int(c.max()))), cu, c, H * D, D)
    # other head groupings of prefill (G = 6 -> 2 heads per workgroup, G = 1)
    for h, kv in ((12, 2), (8, 8)):
        L = A.prefill_host(2, h, kv, BS, 64, 300, 1000)
        A.prefill(W, L, A.Buf("out", 600 * h * D * 2),
                  A.Buf("ws", _prefill_ws(2, 600, 300, 1000, h=h)), np.array([0, 300, 600]),
                  np.array([1000, 300]), h * D, D)
    # copy-on-write fork of config 4 (two 64 KiB blocks), ids outside the pool skipped
    cache = A.Buf("cache", 100 * KV * BS * D * 2)
    A.copy_blocks(W, cache, cache, [[3, 99], [7, 42], [-1, 5], [5, 100]], 100, KV * BS * D * 2)
    W.check()


def test_group_sizes_above_8():
    """One-pass units at head dim 128: 64 q / 4 kv heads (G = 16: one unit
    per pool kv head), 128 / 4 (G = 32: two units of 16), 96 / 4 (two of 12),
    9 / 1 and 48 / 4 (one unit of 9 or 12, padded to 16 columns), 14 / 1 and
    26 / 1 (units of 14 and 13, whose K goes through the LDS tile), and groups
    of 5 and 8: the decode stores and LDS accesses stay inside their buffers,
    in both work-list forms and both pool types (every FP8 group runs as a
    16-column unit)."""
    W = A.Writes()
    rng = np.random.default_rng(16)
    assert A.kv_split_of(64, 4) == 1 and A.kv_split_of(128, 4) == 2 and A.kv_split_of(48, 4) == 1
    assert A.kv_split_of(96, 4) == 2 and A.kv_split_of(9, 1) == 1 and A.kv_split_of(17, 1) == 17
    assert A.kv_split_of(64, 4, D=64) == 2 and A.kv_split_of(64, 4, bs=8) == 2
    assert A.kv_split_of(48, 4, D=64) == 2 and A.kv_split_of(9, 1, bs=64) == 3
    assert A.kv_split_of(26, 1) == 2 and A.wide_k_lds(False, 13) and not A.wide_k_lds(False, 12)
    assert not A.wide_k_lds(True, 16)
    for h, kv in ((64, 4), (128, 4), (96, 4), (9, 1), (48, 4), (40, 8), (64, 8), (14, 1), (26, 1)):
        for fp8 in (False, True):
            check_decode(W, 6, 2048, [1, 17, 300, 4097, 32768, 0], fp8, h=h, kv=kv)
            check_decode(W, 70, 400, rng.integers(0, 6400, 70), fp8, h=h, kv=kv)
            check_decode(W, 16, 576, [9216] * 16, fp8, h=h, kv=kv)
    W.check()


def test_planted_mistakes_are_reported():
    # decode output one row short
    W = A.Writes()
    check_decode(W, 16, 576, [9216] + [0] * 15, True, out_rows=15)
    check_decode(W, 16, 576, [1] * 16, True, out_rows=15)
    with pytest.raises(A.OutOfBounds, match="decode"):
        W.check()
    # a workspace one byte short of what a long context writes (two-level merge)
    W = A.Writes()
    check_decode(W, 8, 2049, [32769] * 8, False)
    W.check()
    top = W.ranges["decode workspace"][2]   # the highest byte this call stores to
    assert top <= _decode_ws(8, 2049)
    W = A.Writes()
    check_decode(W, 8, 2049, [32769] * 8, False, ws_bytes=top - 1)
    with pytest.raises(A.OutOfBounds, match="workspace"):
        W.check()
    # a prefill output one token short
    W = A.Writes()
    L = A.prefill_host(1, H, KV, BS, 64, 512, 1024)
    A.prefill(W, L, A.Buf("out", 511 * H * D * 2), A.Buf("ws", _prefill_ws(1, 512, 512, 1024)),
              np.array([0, 512]), np.array([1024]), H * D, D)
    with pytest.raises(A.OutOfBounds, match="prefill output"):
        W.check()
    # a slot past the pool is skipped, a slot one row short of the cache is not
    W = A.Writes()
    cache = A.Buf("cache", 10 * KV * BS * D - 1)
    A.prologue(W, A.Buf("q", H * D * 2), cache, cache, np.array([159]), 1, H, KV, 10, BS, H * D,
               True)
    with pytest.raises(A.OutOfBounds, match="prologue cache"):
        W.check()


def test_head_dims_64_and_256():
    """The fused prologue (two rows per wave at D 64, two rotate-half pairs
    per lane at D 256) and prefill at those head dims (prefill_kernel at 64,
    with its partials in the workspace the library sizes; the generic kernel
    at 256): every K/V row read and every store inside its buffer, over
    ragged chunks on paged prefixes, an empty chunk, a chunk longer than its
    context (rows before position 0) and block tables at their full width; a
    planted wrong row stride is caught."""
    rng = np.random.default_rng(64)
    for d in (64, 256):
        W = A.Writes()
        h, kv, bs, nblk = 6, 2, 16, 400
        # prologue: 37 tokens, every 7th slot skipped, q rows with a padded stride
        T = 37
        slots = rng.permutation(nblk * bs)[:T]
        slots[::7] = -1
        A.prologue(W, A.Buf("q_out", T * (h * d + 64) * 2), A.Buf("k", nblk * kv * bs * d * 2),
                   A.Buf("v", nblk * kv * bs * d * 2), slots, T, h, kv, nblk, bs, h * d + 64,
                   False, D=d)
        q = np.array([300, 1, 0, 129, 64])
        cu = np.concatenate([[0], np.cumsum(q)])
        mb = 100
        ctx = np.array([1300, 1, 0, mb * bs, 20])   # full-width table; 64 rows on 20 keys
        tables = np.stack([rng.permutation(nblk)[:mb] for _ in q]).astype(np.int64)
        out = A.Buf("out", int(cu[-1]) * h * d * 2)
        if d == 64:
            mctx = int(ctx.max())
            L = A.prefill_host(len(q), h, kv, bs, mb, int(q.max()), mctx, D=d)
            ws_bytes = int(_lib.load().npd_paged_prefill_workspace_size(
                len(q), int(cu[-1]), h, d, int(q.max()), mctx))
            assert ws_bytes == L.total > 0
            A.prefill(W, L, out, A.Buf("ws", ws_bytes), cu, ctx, h * d, d, D=d)
            W.check()
            bad = A.Writes()   # planted: output rows addressed with twice the row stride
            A.prefill(bad, L, out, A.Buf("ws", ws_bytes), cu, ctx, 2 * h * d, d, D=d)
        else:
            A.prefill_generic(W, len(q), h, kv, bs, mb, nblk, int(q.max()), out, cu, ctx, h * d,
                              d, tables, d)
            W.check()
            bad = A.Writes()   # planted: output rows addressed with twice the row stride
            A.prefill_generic(bad, len(q), h, kv, bs, mb, nblk, int(q.max()), out, cu, ctx,
                              2 * h * d, d, tables, d)
        with pytest.raises(A.OutOfBounds):
            bad.check()


@pytest.mark.parametrize("S,H,KV,mq", [(4, 32, 8, 512), (3, 12, 2, 130), (5, 6, 1, 64),
                                        (1, 16, 16, 700), (64, 8, 2, 65), (70, 4, 4, 64)])
def test_prefill_generic_grid_covers_every_tile_once(S, H, KV, mq):
    """Head dim 256: the XCD-grouped grid of prefill_generic_kernel runs every
    (sequence, 64-row tile, query head) exactly once (tied and clamped
    contexts included), the workgroups of one (sequence, kv head) all go to
    one XCD, and up to 64 sequences start longest context first."""
    rng = np.random.default_rng(S * 100 + H)
    cap = 4096
    ctx = rng.integers(-5, 5000, size=S)
    ctx[: S // 3] = ctx[0]                       # ties
    units = A.prefill_generic_units(S, H, KV, mq, ctx, cap)
    tiles = -(-mq // 64)
    assert sorted(u[1:] for u in units) == \
        [(s, t, h) for s in range(S) for t in range(tiles) for h in range(H)]
    assert len({u[0] for u in units}) == len(units)
    xcds = {}
    for bid, s, t, h in units:   # blockIdx % 8 is the XCD
        xcds.setdefault((s, h // (H // KV)), set()).add(bid % 8)
    assert all(len(x) == 1 for x in xcds.values())
    if S <= 64:   # first workgroup of each sequence in grid order: by clamped context, descending
        first = {}
        for bid, s, t, h in units:
            first.setdefault(s, bid)
        key = np.clip(ctx, 0, cap)
        by_start = sorted(first, key=lambda s: first[s])
        assert [int(key[s]) for s in by_start] == sorted((int(k) for k in key), reverse=True)


def test_decode_fast_path_head_dims_64_and_256():
    """The fast path at head dims 64 and 256 (block sizes 16 and 32): output,
    partial, group-slot and counter stores inside the workspace the library
    sizes, over short and 32k contexts, both work-list forms and G up to 16."""
    rng = np.random.default_rng(256)
    W = A.Writes()
    for d in (64, 256):
        for bs in (16, 32):
            for h, kv in ((32, 8), (16, 2), (14, 2), (64, 4)):
                mb = 32768 // bs + 1
                check_decode(W, 8, mb, [1, 17, 300, 4097, 32768, 0, 9000, 12], False, h=h, kv=kv,
                             bs=bs, d=d)
                check_decode(W, 70, 4096 // bs, rng.integers(0, 4097, 70), False, h=h, kv=kv,
                             bs=bs, d=d)
    W.check()


@pytest.mark.parametrize("case", ["cfg3", "ragged", "long_prefix", "groups_2"])
def test_prefill_work_list_covers_every_part_once(case):
    """The in-kernel work list (<= 64 tiles): every (sequence, tile, key part,
    kv head, head group) is run by exactly one workgroup, and each tile's parts
    cut its key range [0, steps) into consecutive, non-empty pieces of near
    equal length (prefill_attention.hip prefill_item and the part bounds of
    prefill_kernel)."""
    rng = np.random.default_rng(7)
    if case == "cfg3":
        S, h, kv, q, p = 4, H, KV, [512] * 4, [0, 512, 1536, 3072]
    elif case == "ragged":
        S, h, kv = 5, H, KV
        q = [int(x) for x in rng.integers(1, 700, S)]
        p = [int(x) for x in rng.integers(0, 5000, S)]
    elif case == "long_prefix":
        S, h, kv, q, p = 2, H, KV, [300, 64], [30000, 9000]
    else:
        S, h, kv, q, p = 3, 16, 8, [200, 130, 400], [100, 2000, 700]
    cu = np.concatenate([[0], np.cumsum(q)])
    ctx = np.array(q) + np.array(p)
    max_bps = int(np.ceil(ctx.max() / BS))
    L = A.prefill_host(S, h, kv, BS, max_bps, max(q), int(ctx.max()))
    assert L.S * L.tiles <= 64
    items = [it for it in A.prefill_items(L, cu, ctx) if it is not None]
    TR = 64 * L.rt
    seen = set()
    parts = {}
    for s, t, j, kh, hg, q0, qlen, cx, ks, eq in items:
        assert eq
        key = (s, t, j, kh, hg)
        assert key not in seen, key
        seen.add(key)
        rows = min(qlen - t * TR, TR)
        nsteps = -(-max(cx - qlen + t * TR + rows, 0) // 64)
        nsp = min(max(-(-nsteps // ks), 1), L.splits)
        assert j < nsp
        base, rm = divmod(nsteps, nsp)
        st0 = j * base + min(j, rm)
        st1 = st0 + base + (1 if j < rm else 0)
        parts.setdefault((s, t, kh, hg), []).append((st0, st1, nsteps, nsp))
    expected = 0
    for s in range(S):
        for t in range(-(-q[s] // TR)):
            for kh in range(kv):
                for hg in range(L.hgroups):
                    got = sorted(parts.get((s, t, kh, hg), []))
                    assert got, (s, t, kh, hg)
                    nsteps, nsp = got[0][2], got[0][3]
                    assert len(got) == nsp
                    expected += nsp
                    assert got[0][0] == 0 and got[-1][1] == nsteps
                    for (a0, a1, _, _), (b0, _, _, _) in zip(got, got[1:]):
                        assert a1 == b0
                    lens = [b - a for a, b, _, _ in got]
                    assert max(lens) - min(lens) <= 1
                    assert nsteps == 0 or min(lens) >= 1
    assert len(items) == expected


def test_bench_names_the_kernel_the_library_runs():
    """bench.py's fast_path (which kernel its decode line names and whether a
    stored counter reading applies) follows the library's use_fast_path for
    every head dim and block size bench can be given."""
    from types import SimpleNamespace

    import bench
    for S in (64, 4096, 4097):
        for D in (32, 64, 96, 128, 160, 192, 256):
            for bs in (8, 16, 24, 32, 48, 64, 128, 256):
                w = SimpleNamespace(num_seqs=S, head_dim=D, block_size=bs)
                assert bench.fast_path(w) == A.use_fast_path(D, bs, S), (S, D, bs)
