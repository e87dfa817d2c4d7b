"""Pins the CPU oracle (oracle/paged_oracle.py) before it is trusted.

The reference holds no golden vectors for this path (its tests regenerate
inputs on a CUDA device); its pins are case lists and tolerances. Each oracle
function is therefore checked against something that does not share its code:

* bits_to_f32 / f32_to_bits  -- torch's own fp16/bf16 casts (library routine).
* e4m3_to_f32 / f32_to_e4m3  -- torch.float8_e4m3fn casts (library routine) on
  every code and on random, tie, subnormal and boundary values in range;
  saturation beyond 448 by hand.
* kv_store_slots_fp8         -- dequantised bytes are within half an e4m3 step
  of x (relative 2^-4) at the right slots; untouched slots keep their poison.
* kv_store                   -- the reference's Python scatter loop restated in
  torch (oracle/torch_ref.py), plus: untouched slots keep their poison, the
  reference test cases (start_pos 8 mid-block; seq_len {1,8,16,32,64}; 8 heads),
  idempotence, and out-of-range tokens are skipped.
* kv_store_slots             -- equals kv_store on the same tokens.
* decode_attention           -- explicit scalar loops with math.exp on tiny
  inputs; torch SDPA on an unpaged contiguous copy (library routine); the
  reference oracle restated with torch ops (repeat_interleave + bmm); special
  cases: seq_len 1 -> V[0], constant keys -> mean of V, GQA == MHA with
  replicated KV, block-table permutation invariance, seq_len 0 -> zeros.
* prefill_attention          -- prefix 0 equals torch SDPA(is_causal=True) and
  the reference's chunk-only computation (chunk_only_prefill); the last row
  equals decode_attention at the same context; splitting a chunk in two gives
  the same rows.
* chunk_only_prefill         -- torch SDPA with the reference's block-diagonal
  mask (oracle/torch_ref.py ref_prefill_sdpa).
* partition_partials + lse_merge -- merged partials equal the unsplit softmax
  for several partition sizes (a dropped rescale term fails it).
* copy_blocks                -- bytes of dst equal src; others untouched.
* extract_kv / load_kv       -- the reference's per-block copy loops
  (kv_transfer.py:45-69) restated in torch (oracle/torch_ref.py); a round trip
  into a second pool at another block list reproduces the blocks and leaves
  every other block's poison.
* pack_metadata              -- hand-written expected tensors for a small batch.
* BlockAllocator / append_slot -- the reference block-manager test facts
  (LIFO order, CoW pair on a shared last block).
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import paged_oracle as O
from oracle import torch_ref as R


def _rand_bits(rng, shape, dtype):
    x = (rng.standard_normal(shape) * 0.5).astype(np.float32)
    return O.f32_to_bits(x, dtype)


# ---------------------------------------------------------------------------
# storage formats
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype,tdt", [("f16", torch.float16), ("bf16", torch.bfloat16)])
def test_format_round_trip_matches_torch(dtype, tdt):
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(4096).astype(np.float32) * 3,
                        np.array([0.0, -0.0, 1e-30, 65504.0, 1e38, np.inf, -np.inf], np.float32)])
    mine = O.f32_to_bits(x, dtype)
    theirs = torch.from_numpy(x).to(tdt).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(mine, theirs)
    back = O.bits_to_f32(mine, dtype)
    assert np.array_equal(back, torch.from_numpy(x).to(tdt).float().numpy())


# ---------------------------------------------------------------------------
# store
# ---------------------------------------------------------------------------

def _store_case(kvh, T, D, bs, start, total_blocks=None, seed=0, perm=False):
    rng = np.random.default_rng(seed)
    nb = (start + T + bs - 1) // bs
    total = total_blocks or nb + 3
    k_src = _rand_bits(rng, (kvh, T, D), "f16")
    v_src = _rand_bits(rng, (kvh, T, D), "f16")
    table = rng.permutation(total)[:nb] if perm else np.arange(nb)
    tables = np.tile(table.astype(np.int32), (T, 1))
    pos = np.arange(start, start + T, dtype=np.int32)
    return k_src, v_src, tables, pos, total


@pytest.mark.parametrize("kvh,T,start,bs", [(4, 16, 0, 16), (2, 8, 8, 16), (2, 1, 0, 16),
                                            (2, 8, 0, 16), (2, 32, 0, 16), (2, 64, 0, 16),
                                            (8, 16, 0, 16), (3, 40, 5, 32), (2, 33, 7, 4)])
def test_store_matches_reference_loop(kvh, T, start, bs):
    D = 128
    k_src, v_src, tables, pos, total = _store_case(kvh, T, D, bs, start, perm=True, seed=T)
    poison = np.uint16(0x7E01)   # a NaN pattern no source produces
    kc = np.full((total, kvh, bs, D), poison, np.uint16)
    vc = kc.copy()
    O.kv_store(kc, vc, k_src, v_src, tables, pos)
    tk = torch.from_numpy(np.full((total, kvh, bs, D), poison, np.uint16).view(np.int16))
    tv = tk.clone()
    R.ref_kv_store_loop(tk, tv, torch.from_numpy(k_src.view(np.int16)),
                        torch.from_numpy(v_src.view(np.int16)), torch.from_numpy(tables),
                        torch.from_numpy(pos))
    assert np.array_equal(kc, tk.numpy().view(np.uint16))
    assert np.array_equal(vc, tv.numpy().view(np.uint16))
    # untouched slots keep the poison: exactly T*kvh rows were written
    written = np.any(kc != poison, axis=-1).sum()
    assert written == T * kvh
    # idempotent
    kc2, vc2 = kc.copy(), vc.copy()
    O.kv_store(kc2, vc2, k_src, v_src, tables, pos)
    assert np.array_equal(kc, kc2) and np.array_equal(vc, vc2)


def test_store_skips_out_of_range_tokens():
    kvh, T, D, bs = 2, 4, 128, 16
    k_src, v_src, tables, pos, total = _store_case(kvh, T, D, bs, 0)
    tables[1, 0] = total + 5        # block outside the pool
    pos = pos.copy()
    pos[2] = -1                     # negative position
    pos[3] = bs * tables.shape[1]   # past the end of the table
    kc = np.zeros((total, kvh, bs, D), np.uint16)
    vc = kc.copy()
    O.kv_store(kc, vc, k_src, v_src, tables, pos)
    assert np.array_equal(kc[tables[0, 0], :, 0], k_src[:, 0])
    assert np.any(kc != 0, axis=-1).sum() == kvh  # only token 0 landed


def test_store_slots_equals_table_store():
    kvh, T, D, bs = 4, 37, 64, 8
    k_src, v_src, tables, pos, total = _store_case(kvh, T, D, bs, 3, perm=True, seed=5)
    a_k = np.zeros((total, kvh, bs, D), np.uint16); a_v = a_k.copy()
    O.kv_store(a_k, a_v, k_src, v_src, tables, pos)
    slots = np.array([tables[t, p // bs] * bs + p % bs for t, p in enumerate(pos)], np.int32)
    slots[5] = -1
    b_k = np.zeros_like(a_k); b_v = b_k.copy()
    O.kv_store_slots(b_k, b_v, k_src.transpose(1, 0, 2), v_src.transpose(1, 0, 2), slots)
    blk, off = tables[5, pos[5] // bs], pos[5] % bs
    a_k[blk, :, off] = 0
    a_v[blk, :, off] = 0
    assert np.array_equal(a_k, b_k) and np.array_equal(a_v, b_v)


def test_copy_blocks():
    rng = np.random.default_rng(1)
    kc = _rand_bits(rng, (10, 2, 4, 64), "bf16")
    vc = _rand_bits(rng, (10, 2, 4, 64), "bf16")
    k0, v0 = kc.copy(), vc.copy()
    O.copy_blocks(kc, vc, [(3, 7), (1, 2), (4, 99)])
    assert np.array_equal(kc[7], k0[3]) and np.array_equal(vc[2], v0[1])
    keep = [i for i in range(10) if i not in (7, 2)]
    assert np.array_equal(kc[keep], k0[keep]) and np.array_equal(vc[keep], v0[keep])


def test_e4m3_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = O.e4m3_to_f32(codes)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin], want[fin])
    rng = np.random.default_rng(7)
    pos = O._E4M3_POS
    mids = (pos[:-1] + pos[1:]) / 2                       # exact ties between neighbours
    x = np.concatenate([rng.standard_normal(20000) * 40, rng.standard_normal(2000) * 1e-2,
                        mids, -mids, pos, -pos, [0.0, -0.0, 448.0, -448.0, 2.0 ** -10]])
    x = x.astype(np.float32)
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = O.f32_to_e4m3(x)
    assert np.array_equal(got, want)
    assert np.array_equal(O.f32_to_e4m3(np.array([1e4, -500.0, np.nan], np.float32)),
                          np.array([0x7E, 0xFE, 0x7F], np.uint8))


def test_kv_store_slots_fp8():
    rng = np.random.default_rng(8)
    kc = np.full((6, 2, 4, 16), 0x33, np.uint8)
    vc = kc.copy()
    ks, vs = np.array([0.05, 0.2], np.float32), np.array([0.1, 0.01], np.float32)
    k = rng.standard_normal((3, 2, 16)).astype(np.float32)
    v = rng.standard_normal((3, 2, 16)).astype(np.float32)
    O.kv_store_slots_fp8(kc, vc, k, v, np.array([5, -1, 22]), ks, vs)
    kf, vf = O.fp8_pool_values(kc, ks), O.fp8_pool_values(vc, vs)
    for t, slot in ((0, 5), (2, 22)):
        b, o = divmod(slot, 4)
        assert np.all(np.abs(kf[b, :, o] - k[t]) <= np.abs(k[t]) * 2.0 ** -4 + ks[:, None] * 2.0 ** -10)
        assert np.all(np.abs(vf[b, :, o] - v[t]) <= np.abs(v[t]) * 2.0 ** -4 + vs[:, None] * 2.0 ** -10)
    written = {(1, 1), (5, 2)}
    for b in range(6):
        for o in range(4):
            if (b, o) not in written:
                assert (kc[b, :, o] == 0x33).all() and (vc[b, :, o] == 0x33).all()


def test_extract_and_load_kv():
    rng = np.random.default_rng(2)
    kp = _rand_bits(rng, (3, 12, 2, 4, 16), "bf16")
    vp = _rand_bits(rng, (3, 12, 2, 4, 16), "bf16")
    ids = [7, 0, 11, 3]
    wk, wv = O.extract_kv(kp, vp, ids)
    rk, rv = R.ref_extract_kv(torch.from_numpy(kp.view(np.int16)),
                              torch.from_numpy(vp.view(np.int16)), ids)
    assert np.array_equal(wk, rk.numpy().view(np.uint16))
    assert np.array_equal(wv, rv.numpy().view(np.uint16))
    zk, _ = O.extract_kv(kp, vp, [5, 99])             # out of the pool -> zero block
    assert np.array_equal(zk[:, 0], kp[:, 5]) and not zk[:, 1].any()
    dk = np.full((3, 20, 2, 4, 16), 0x7fc1, np.uint16)
    dv = dk.copy()
    dst = [19, 2, 8, 13]
    O.load_kv(dk, dv, dst, wk, wv)
    tk = torch.from_numpy(np.full((3, 20, 2, 4, 16), 0x7fc1, np.uint16).view(np.int16))
    tv = tk.clone()
    R.ref_load_kv(tk, tv, dst, torch.from_numpy(wk.view(np.int16)), torch.from_numpy(wv.view(np.int16)))
    assert np.array_equal(dk, tk.numpy().view(np.uint16)) and np.array_equal(dv, tv.numpy().view(np.uint16))
    for s_, d_ in zip(ids, dst):
        assert np.array_equal(dk[:, d_], kp[:, s_]) and np.array_equal(dv[:, d_], vp[:, s_])
    rest = [b for b in range(20) if b not in dst]
    assert (dk[:, rest] == 0x7fc1).all() and (dv[:, rest] == 0x7fc1).all()


# ---------------------------------------------------------------------------
# decode attention
# ---------------------------------------------------------------------------

def _decode_case(S, H, kvh, D, bs, seq_lens, seed=0, dtype="f16", perm=True):
    rng = np.random.default_rng(seed)
    nbs = [(n + bs - 1) // bs for n in seq_lens]
    total = sum(nbs) + 2
    order = rng.permutation(total) if perm else np.arange(total)
    mb = max(nbs + [1])
    bt = np.zeros((S, mb), np.int32)
    o = 0
    for s, k in enumerate(nbs):
        bt[s, :k] = order[o:o + k]
        o += k
    q = O.bits_to_f32(_rand_bits(rng, (S, H, D), dtype), dtype)
    kc = O.bits_to_f32(_rand_bits(rng, (total, kvh, bs, D), dtype), dtype)
    vc = O.bits_to_f32(_rand_bits(rng, (total, kvh, bs, D), dtype), dtype)
    return q, kc, vc, bt, np.array(seq_lens, np.int32)


def _loops_decode(q, kc, vc, bt, sl, scale):
    S, H, D = q.shape
    kvh, bs = kc.shape[1], kc.shape[2]
    out = np.zeros((S, H, D))
    for s in range(S):
        for h in range(H):
            g = h // (H // kvh)
            sc = []
            for t in range(int(sl[s])):
                b, off = bt[s, t // bs], t % bs
                sc.append(sum(float(q[s, h, d]) * float(kc[b, g, off, d]) for d in range(D)) * scale)
            if not sc:
                continue
            m = max(sc)
            w = [math.exp(x - m) for x in sc]
            z = sum(w)
            for t in range(int(sl[s])):
                b, off = bt[s, t // bs], t % bs
                for d in range(D):
                    out[s, h, d] += w[t] / z * float(vc[b, g, off, d])
    return out


def test_decode_matches_scalar_loops():
    q, kc, vc, bt, sl = _decode_case(3, 4, 2, 8, 4, [1, 6, 9], seed=3)
    got = O.decode_attention(q, kc, vc, bt, sl, 0.3)
    want = _loops_decode(q, kc, vc, bt, sl, 0.3)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("H,kvh,bs,lens", [(4, 4, 8, [4, 8, 12]), (8, 2, 8, [16, 8]),
                                           (12, 2, 16, [17, 64, 200]), (32, 8, 16, [1, 15, 16, 17]),
                                           (6, 1, 32, [40])])
def test_decode_matches_sdpa_on_unpaged_copy(H, kvh, bs, lens):
    D = 64
    q, kc, vc, bt, sl = _decode_case(len(lens), H, kvh, D, bs, lens, seed=H + bs)
    scale = 1 / math.sqrt(D)
    got = O.decode_attention(q, kc, vc, bt, sl, scale)
    for s, n in enumerate(lens):
        # build the contiguous context by explicit per-token indexing
        K = np.stack([kc[bt[s, t // bs], :, t % bs] for t in range(n)], axis=1)  # [kvh, n, D]
        V = np.stack([vc[bt[s, t // bs], :, t % bs] for t in range(n)], axis=1)
        qt = torch.from_numpy(q[s]).double().unsqueeze(1)                       # [H, 1, D]
        Kt = torch.from_numpy(K).double().repeat_interleave(H // kvh, 0)
        Vt = torch.from_numpy(V).double().repeat_interleave(H // kvh, 0)
        ref = F.scaled_dot_product_attention(qt, Kt, Vt, scale=scale)[:, 0]
        assert np.allclose(got[s], ref.numpy(), rtol=1e-10, atol=1e-10)


def test_decode_matches_reference_torch_restatement():
    q, kc, vc, bt, sl = _decode_case(4, 12, 2, 128, 16, [17, 64, 200, 511], seed=9)
    got = O.decode_attention(q, kc, vc, bt, sl, 1 / math.sqrt(128))
    ref = R.ref_paged_attention(torch.from_numpy(q).double(), torch.from_numpy(kc).double(),
                                torch.from_numpy(vc).double(), torch.from_numpy(bt),
                                torch.from_numpy(sl), 1 / math.sqrt(128))
    assert np.allclose(got, ref.numpy(), rtol=1e-6, atol=1e-6)


def test_decode_special_cases():
    q, kc, vc, bt, sl = _decode_case(2, 8, 2, 64, 16, [1, 37], seed=4)
    out = O.decode_attention(q, kc, vc, bt, sl, 0.125)
    # seq_len 1: the output is the single value row
    for h in range(8):
        assert np.allclose(out[0, h], vc[bt[0, 0], h // 4, 0])
    # constant keys: uniform weights, output = mean of V over the context
    kc2 = kc.copy()
    kc2[:] = 0.25
    out2 = O.decode_attention(q, kc2, vc, bt, sl, 0.125)
    V = np.stack([vc[bt[1, t // 16], :, t % 16] for t in range(37)], axis=1)
    for h in range(8):
        assert np.allclose(out2[1, h], V[h // 4].mean(axis=0))
    # seq_len 0 -> zeros
    out3 = O.decode_attention(q, kc, vc, bt, np.array([0, 37], np.int32), 0.125)
    assert np.all(out3[0] == 0) and np.allclose(out3[1], out[1])


def test_decode_gqa_equals_replicated_mha():
    q, kc, vc, bt, sl = _decode_case(2, 8, 2, 64, 8, [19, 33], seed=6)
    gqa = O.decode_attention(q, kc, vc, bt, sl, 0.1)
    mha = O.decode_attention(q, np.repeat(kc, 4, axis=1), np.repeat(vc, 4, axis=1), bt, sl, 0.1)
    assert np.allclose(gqa, mha, rtol=1e-12, atol=1e-12)


def test_decode_block_table_permutation_invariance():
    q, kc, vc, bt, sl = _decode_case(3, 4, 2, 64, 4, [5, 17, 30], seed=7)
    a = O.decode_attention(q, kc, vc, bt, sl, 0.2)
    rng = np.random.default_rng(0)
    perm = rng.permutation(kc.shape[0])          # move block b to perm[b]
    kc2 = np.empty_like(kc); vc2 = np.empty_like(vc)
    kc2[perm] = kc; vc2[perm] = vc
    b = O.decode_attention(q, kc2, vc2, perm[bt].astype(np.int32), sl, 0.2)
    assert np.allclose(a, b, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# split-context merge
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("part", [1, 7, 16, 100, 1000])
def test_lse_merge_equals_unsplit_softmax(part):
    rng = np.random.default_rng(part)
    n, D = 300, 16
    q = rng.standard_normal(D) * 2
    K = rng.standard_normal((n, D)) * 2
    V = rng.standard_normal((n, D))
    merged = O.lse_merge(O.partition_partials(q, K, V, 0.7, part))
    sc = K @ q * 0.7
    w = np.exp(sc - sc.max())
    assert np.allclose(merged, w @ V / w.sum(), rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# prefill
# ---------------------------------------------------------------------------

def _prefill_case(prefixes, chunks, H=8, kvh=2, D=32, bs=8, seed=0):
    rng = np.random.default_rng(seed)
    ctx = [p + c for p, c in zip(prefixes, chunks)]
    q_all, kc, vc, bt, _ = _decode_case(len(ctx), H, kvh, D, bs, ctx, seed=seed, dtype="bf16")
    T = sum(chunks)
    q = O.bits_to_f32(_rand_bits(rng, (T, H, D), "bf16"), "bf16")
    cu = np.concatenate([[0], np.cumsum(chunks)]).astype(np.int32)
    return q, kc, vc, bt, cu, np.array(ctx, np.int32)


def test_prefill_prefix0_equals_causal_sdpa_and_chunk_only():
    chunks = [7, 20, 1]
    q, kc, vc, bt, cu, ctx = _prefill_case([0, 0, 0], chunks, seed=2)
    got = O.prefill_attention(q, kc, vc, bt, cu, ctx, 0.2)
    kvh, bs = kc.shape[1], kc.shape[2]
    k_tok = np.concatenate([np.stack([kc[bt[s, t // bs], :, t % bs] for t in range(n)])
                            for s, n in enumerate(chunks)])   # [T, kvh, D]
    v_tok = np.concatenate([np.stack([vc[bt[s, t // bs], :, t % bs] for t in range(n)])
                            for s, n in enumerate(chunks)])
    chunk_only = O.chunk_only_prefill(q, k_tok, v_tok, cu, 0.2)
    assert np.allclose(got, chunk_only, rtol=1e-12, atol=1e-12)
    for s, n in enumerate(chunks):
        a, b = cu[s], cu[s + 1]
        qt = torch.from_numpy(q[a:b]).double().transpose(0, 1)
        kt = torch.from_numpy(k_tok[a:b]).double().transpose(0, 1).repeat_interleave(4, 0)
        vt = torch.from_numpy(v_tok[a:b]).double().transpose(0, 1).repeat_interleave(4, 0)
        ref = F.scaled_dot_product_attention(qt, kt, vt, is_causal=True, scale=0.2)
        assert np.allclose(got[a:b], ref.transpose(0, 1).numpy(), rtol=1e-10, atol=1e-10)


def test_chunk_only_matches_reference_sdpa_restatement():
    chunks = [5, 9]
    rng = np.random.default_rng(4)
    T = sum(chunks)
    q = rng.standard_normal((T, 8, 16))
    k = rng.standard_normal((T, 2, 16))
    v = rng.standard_normal((T, 2, 16))
    cu = np.array([0, 5, 14], np.int32)
    mine = O.chunk_only_prefill(q, k, v, cu, 0.25)
    ref = R.ref_prefill_sdpa(torch.from_numpy(q).double(), torch.from_numpy(k).double(),
                             torch.from_numpy(v).double(), chunks, 0.25)
    assert np.allclose(mine, ref.numpy(), rtol=1e-6, atol=1e-6)


def test_prefill_last_row_equals_decode_and_split_invariance():
    prefixes, chunks = [0, 13, 40], [9, 16, 5]
    q, kc, vc, bt, cu, ctx = _prefill_case(prefixes, chunks, seed=8)
    full = O.prefill_attention(q, kc, vc, bt, cu, ctx, 0.3)
    # last row of each sequence == decode at the full context
    last = np.stack([q[cu[s + 1] - 1] for s in range(3)])
    dec = O.decode_attention(last, kc, vc, bt, ctx, 0.3)
    for s in range(3):
        assert np.allclose(full[cu[s + 1] - 1], dec[s], rtol=1e-12, atol=1e-12)
    # split every chunk in two calls: prefix grows by the first part
    for s in range(3):
        c = chunks[s]
        h1 = c // 2
        a = cu[s]
        part1 = O.prefill_attention(q[a:a + h1], kc, vc, bt[s:s + 1], np.array([0, h1], np.int32),
                                    np.array([prefixes[s] + h1], np.int32), 0.3)
        part2 = O.prefill_attention(q[a + h1:a + c], kc, vc, bt[s:s + 1],
                                    np.array([0, c - h1], np.int32), np.array([ctx[s]], np.int32), 0.3)
        assert np.allclose(np.concatenate([part1, part2]), full[a:a + c], rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# metadata and block policy
# ---------------------------------------------------------------------------

def test_pack_metadata_small_batch():
    seqs = [(3, 5, [7, 2]), (1, 9, [4]), (1, 16, [1, 0])]   # prefill chunk, 2 decodes
    m = O.pack_metadata(seqs, block_size=8, max_blocks_per_seq=3)
    assert m["cu_seqlens_q"].tolist() == [0, 3, 4, 5]
    assert m["seq_lens"].tolist() == [8, 10, 17]
    assert m["block_tables"].tolist() == [[7, 2, 0], [4, 0, 0], [1, 0, 0]]
    assert m["positions"].tolist() == [5, 6, 7, 9, 16]
    # pos 5,6,7 -> block 7 offsets 5..7; pos 9 -> table[1] missing -> -1;
    # pos 16 -> table[2] missing -> -1
    assert m["slot_mapping"].tolist() == [61, 62, 63, -1, -1]
    assert m["token_seq"].tolist() == [0, 0, 0, 1, 2]


def test_block_allocator_lifo_and_cow():
    a = O.BlockAllocator(4)
    assert [a.allocate(), a.allocate()] == [3, 2]     # highest index first
    t = [3]
    assert O.append_slot(a, t, 4, 4) is None and t == [3, 1]   # token 4 opens block 1
    child = list(t)
    for b in child:
        a.fork(b)
    pair = O.append_slot(a, child, 5, 4)              # shared last block -> CoW
    assert pair == (1, 0) and child == [3, 0]
    with pytest.raises(MemoryError):
        a.allocate()
