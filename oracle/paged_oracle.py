"""Numpy restatement of nanoPD's paged KV store / paged attention path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker. The product (nanopd_amd) never
imports it.

Storage tensors are handled as raw uint16 bit patterns plus a dtype tag
("f16" / "bf16") so that the store and copy ops can be checked bit for bit;
arithmetic is float64 (attention) unless stated.

Pinning of every function (what fixes it independently of this file) is listed
in the module docstring of tests/test_oracle.py; a function without such a
check would be marked "parity unpinned" here. Every function below is pinned.
Citations are relative to the reference tree; PA/ = nanoPD/paged_attention/.
"""
from __future__ import annotations

import math
from typing import Sequence

import numpy as np

# ---------------------------------------------------------------------------
# 2-byte storage formats
# ---------------------------------------------------------------------------


def bits_to_f32(bits: np.ndarray, dtype: str) -> np.ndarray:
    """uint16 bit patterns -> float32 (exact for both formats)."""
    bits = np.asarray(bits, dtype=np.uint16)
    if dtype == "bf16":
        return (bits.astype(np.uint32) << 16).view(np.float32)
    if dtype == "f16":
        return bits.view(np.float16).astype(np.float32)
    raise ValueError(dtype)


def f32_to_bits(x: np.ndarray, dtype: str) -> np.ndarray:
    """float -> uint16 bit patterns, round to nearest even (NaN -> quiet NaN)."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "f16":
        with np.errstate(over="ignore"):
            return x.astype(np.float16).view(np.uint16)
    if dtype == "bf16":
        u = x.view(np.uint32).astype(np.uint64)
        nan = (u & 0x7FFFFFFF) > 0x7F800000
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        return np.where(nan, np.uint16(0x7FC0), r).astype(np.uint16)
    raise ValueError(dtype)


# ---------------------------------------------------------------------------
# FP8 (OCP e4m3, "e4m3fn") storage: 1 sign, 4 exponent (bias 7), 3 mantissa
# bits; no infinities; S.1111.111 is NaN; largest finite 448.
# ---------------------------------------------------------------------------


def e4m3_to_f32(codes: np.ndarray) -> np.ndarray:
    """e4m3 bytes -> float32 (exact)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int32)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e, m = (c >> 3) & 0xF, c & 0x7
    mag = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * 2.0 ** (e - 7))
    out = (sign * mag).astype(np.float32)
    out[(c & 0x7F) == 0x7F] = np.nan
    return out


_E4M3_POS = e4m3_to_f32(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)   # codes 0..126, ascending


def f32_to_e4m3(x: np.ndarray) -> np.ndarray:
    """float -> e4m3 bytes, round to nearest, ties to the even code; values
    beyond 448 saturate; NaN -> 0x7F. Negative values keep the sign bit (a
    negative value that rounds to zero gives 0x80)."""
    x = np.asarray(x, dtype=np.float32).astype(np.float64)
    a = np.minimum(np.abs(x), 448.0)
    hi = np.searchsorted(_E4M3_POS, a, side="left").clip(0, 0x7E)
    lo = np.maximum(hi - 1, 0)
    dl, dh = a - _E4M3_POS[lo], _E4M3_POS[hi] - a
    pick = np.where(dl < dh, lo, np.where(dh < dl, hi, np.where(lo % 2 == 0, lo, hi)))
    pick = np.where(a == _E4M3_POS[hi], hi, pick)
    out = (pick | np.where(np.signbit(x), 0x80, 0)).astype(np.uint8)
    out[np.isnan(x)] = 0x7F
    return out


def kv_store_slots_fp8(k_cache: np.ndarray, v_cache: np.ndarray, k_src: np.ndarray,
                       v_src: np.ndarray, slots: np.ndarray, k_scale: np.ndarray,
                       v_scale: np.ndarray) -> None:
    """FP8 pool store: caches uint8 [N, kvh, bs, D], sources float [T, kvh, D]
    (the exact values of the 2-byte inputs); byte = e4m3(clamp(x / scale[h])),
    the division in fp32. Slots outside the pool are skipped."""
    n, kvh, bs, _ = k_cache.shape
    ks = np.asarray(k_scale, np.float32)[:, None]
    vs = np.asarray(v_scale, np.float32)[:, None]
    for t, slot in enumerate(np.asarray(slots)):
        if 0 <= slot < n * bs:
            b, o = divmod(int(slot), bs)
            k_cache[b, :, o] = f32_to_e4m3(np.asarray(k_src[t], np.float32) / ks)
            v_cache[b, :, o] = f32_to_e4m3(np.asarray(v_src[t], np.float32) / vs)


def fp8_pool_values(cache: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """Element values of an fp8 pool: e4m3(byte) * scale[kv head] (float64)."""
    return e4m3_to_f32(cache).astype(np.float64) * np.asarray(scale, np.float64)[None, :, None, None]


# ---------------------------------------------------------------------------
# KV store (bit-exact scatter)
# ---------------------------------------------------------------------------


def kv_store(k_cache: np.ndarray, v_cache: np.ndarray, k_src: np.ndarray, v_src: np.ndarray,
             block_tables: np.ndarray, positions: np.ndarray) -> None:
    """In-place scatter; index math of PA/csrc/kvstore/paged_kv_store_kernel.cu:40-57.

    caches [num_blocks, kvh, bs, D]; k_src/v_src [kvh, T, D]; block_tables
    [T, max_bps] (one row per token); positions [T]. Tokens whose slot falls
    outside the table or the pool are skipped (the reference has no check and
    would write out of bounds, PA/csrc/kvstore/paged_kv_store_kernel.cu:45-57).
    """
    num_blocks, kvh, bs, _ = k_cache.shape
    T = k_src.shape[1]
    max_bps = block_tables.shape[1]
    for t in range(T):
        pos = int(positions[t])
        if pos < 0 or pos // bs >= max_bps:
            continue
        blk = int(block_tables[t, pos // bs])
        if blk < 0 or blk >= num_blocks:
            continue
        k_cache[blk, :, pos % bs, :] = k_src[:, t, :]
        v_cache[blk, :, pos % bs, :] = v_src[:, t, :]


def kv_store_slots(k_cache: np.ndarray, v_cache: np.ndarray, k_src: np.ndarray, v_src: np.ndarray,
                   slot_mapping: np.ndarray) -> None:
    """In-place scatter by flat slot; k_src/v_src [T, kvh, D]; negative or
    out-of-pool slots are skipped."""
    num_blocks, _, bs, _ = k_cache.shape
    slots = np.asarray(slot_mapping, dtype=np.int64)
    ok = (slots >= 0) & (slots < num_blocks * bs)
    idx = np.nonzero(ok)[0]
    blk, off = slots[idx] // bs, slots[idx] % bs
    k_cache[blk, :, off, :] = k_src[idx]
    v_cache[blk, :, off, :] = v_src[idx]


def copy_blocks(k_cache: np.ndarray, v_cache: np.ndarray, pairs: Sequence[tuple[int, int]]) -> None:
    """CoW block copy: cache[dst] = cache[src] for each pair, in order.
    Pairs the kernel would skip (index outside the pool) are skipped."""
    n = k_cache.shape[0]
    for src, dst in pairs:
        if 0 <= src < n and 0 <= dst < n:
            k_cache[dst] = k_cache[src]
            v_cache[dst] = v_cache[src]


def extract_kv(k_pool: np.ndarray, v_pool: np.ndarray, ids: Sequence[int]):
    """Transfer layout of a block list (nanoPD/workers/kv_transfer.py:45-53:
    buf[:, i] = cache[:, bid]): pools [L, N, ...] -> wire [L, len(ids), ...].
    An id outside the pool gives a zero block (the kernel's rule)."""
    n = k_pool.shape[1]
    out_k = np.zeros((k_pool.shape[0], len(ids)) + k_pool.shape[2:], dtype=k_pool.dtype)
    out_v = np.zeros_like(out_k)
    for i, b in enumerate(ids):
        if 0 <= b < n:
            out_k[:, i] = k_pool[:, b]
            out_v[:, i] = v_pool[:, b]
    return out_k, out_v


def load_kv(k_pool: np.ndarray, v_pool: np.ndarray, ids: Sequence[int], wire_k: np.ndarray,
            wire_v: np.ndarray) -> None:
    """Inverse of extract_kv (kv_transfer.py:56-69: cache[:, bid] = buf[:, i]);
    ids outside the pool are skipped."""
    n = k_pool.shape[1]
    for i, b in enumerate(ids):
        if 0 <= b < n:
            k_pool[:, b] = wire_k[:, i]
            v_pool[:, b] = wire_v[:, i]


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------


def gather_context(cache_f: np.ndarray, table: np.ndarray, n: int) -> np.ndarray:
    """[num_blocks, kvh, bs, D] -> [kvh, n, D] for the first n tokens of a table
    (the per-sequence gather of PA/tests/test_paged_attention.py:50-57)."""
    bs = cache_f.shape[2]
    nb = (n + bs - 1) // bs
    blocks = cache_f[np.asarray(table[:nb], dtype=np.int64)]          # [nb, kvh, bs, D]
    return blocks.transpose(1, 0, 2, 3).reshape(cache_f.shape[1], nb * bs, -1)[:, :n]


def decode_attention(q: np.ndarray, k_cache_f: np.ndarray, v_cache_f: np.ndarray,
                     block_tables: np.ndarray, seq_lens: np.ndarray, scale: float) -> np.ndarray:
    """Paged decode attention in float64, the oracle of
    PA/tests/test_paged_attention.py:33-71 (gather, GQA expand, softmax(q.K^T
    * scale) . V). q [S, H, D] float; caches float [blocks, kvh, bs, D]. The
    kv head of q-head h is h // (H / kvh) (PA/csrc/attention/
    paged_attention_kernel.cu:62). seq_len <= 0 gives zeros.
    Returns float64 [S, H, D]."""
    S, H, D = q.shape
    kvh = k_cache_f.shape[1]
    G = H // kvh
    out = np.zeros((S, H, D), dtype=np.float64)
    for s in range(S):
        n = int(seq_lens[s])
        if n <= 0:
            continue
        K = gather_context(k_cache_f, block_tables[s], n).astype(np.float64)   # [kvh, n, D]
        V = gather_context(v_cache_f, block_tables[s], n).astype(np.float64)
        Kx = np.repeat(K, G, axis=0)                                           # [H, n, D]
        Vx = np.repeat(V, G, axis=0)
        sc = np.einsum("hd,hnd->hn", q[s].astype(np.float64), Kx) * scale
        sc -= sc.max(axis=1, keepdims=True)
        p = np.exp(sc)
        p /= p.sum(axis=1, keepdims=True)
        out[s] = np.einsum("hn,hnd->hd", p, Vx)
    return out


def prefill_attention(q: np.ndarray, k_cache_f: np.ndarray, v_cache_f: np.ndarray,
                      block_tables: np.ndarray, cu_seqlens_q: np.ndarray,
                      context_lens: np.ndarray, scale: float) -> np.ndarray:
    """Causal attention over paged prefix + chunk, float64 (the mathematical
    contract of the chunked-prefill op; the reference computes it only for an
    empty prefix, nanoPD/engine/model_runner.py:152-168).
    q [total_q, H, D]; row i of sequence s is at position
    context_lens[s] - q_len + i and attends to keys 0..pos. Rows with pos < 0
    get zeros. Returns float64 [total_q, H, D]."""
    TQ, H, D = q.shape
    kvh = k_cache_f.shape[1]
    G = H // kvh
    out = np.zeros((TQ, H, D), dtype=np.float64)
    for s in range(len(cu_seqlens_q) - 1):
        a, b = int(cu_seqlens_q[s]), int(cu_seqlens_q[s + 1])
        ql, ctx = b - a, int(context_lens[s])
        if ql <= 0 or ctx <= 0:
            continue
        K = np.repeat(gather_context(k_cache_f, block_tables[s], ctx).astype(np.float64), G, axis=0)
        V = np.repeat(gather_context(v_cache_f, block_tables[s], ctx).astype(np.float64), G, axis=0)
        pos = ctx - ql + np.arange(ql)                                          # [ql]
        sc = np.einsum("qhd,hnd->hqn", q[a:b].astype(np.float64), K) * scale    # [H, ql, ctx]
        mask = np.arange(ctx)[None, :] > pos[:, None]                           # [ql, ctx]
        sc = np.where(mask[None], -np.inf, sc)
        valid = pos >= 0
        m = np.max(sc, axis=2, keepdims=True)
        m = np.where(np.isfinite(m), m, 0.0)
        p = np.exp(sc - m)
        den = p.sum(axis=2, keepdims=True)
        den = np.where(den > 0, den, 1.0)
        o = np.einsum("hqn,hnd->qhd", p / den, V)
        o[~valid] = 0.0
        out[a:b] = o
    return out


def chunk_only_prefill(q: np.ndarray, k: np.ndarray, v: np.ndarray, cu_seqlens_q: np.ndarray,
                       scale: float) -> np.ndarray:
    """The reference's actual prefill: SDPA over the chunk tokens only, with a
    block-diagonal causal mask across the packed prefills
    (nanoPD/engine/model_runner.py:152-168). q [T, H, D]; k/v [T, kvh, D].
    Equals prefill_attention when every prefix is empty."""
    T, H, D = q.shape
    G = H // k.shape[1]
    out = np.zeros((T, H, D), dtype=np.float64)
    for s in range(len(cu_seqlens_q) - 1):
        a, b = int(cu_seqlens_q[s]), int(cu_seqlens_q[s + 1])
        n = b - a
        if n <= 0:
            continue
        K = np.repeat(k[a:b].astype(np.float64).transpose(1, 0, 2), G, axis=0)  # [H, n, D]
        V = np.repeat(v[a:b].astype(np.float64).transpose(1, 0, 2), G, axis=0)
        sc = np.einsum("qhd,hnd->hqn", q[a:b].astype(np.float64), K) * scale
        sc = np.where(np.triu(np.ones((n, n), dtype=bool), 1)[None], -np.inf, sc)
        sc -= sc.max(axis=2, keepdims=True)
        p = np.exp(sc)
        p /= p.sum(axis=2, keepdims=True)
        out[a:b] = np.einsum("hqn,hnd->qhd", p, V)
    return out


def partition_partials(q: np.ndarray, K: np.ndarray, V: np.ndarray, scale: float,
                       partition: int) -> list[tuple[np.ndarray, np.ndarray, np.ndarray]]:
    """Split-context partials for one (sequence, head): per partition of
    `partition` tokens, (sum_t e^{s_t - m} v_t, m, sum_t e^{s_t - m})
    (the per-partition state of PA/csrc/paged_attention_optimized/
    paged_attention_optimized.cu:66-171). q [D]; K, V [n, D]."""
    sc = (K.astype(np.float64) @ q.astype(np.float64)) * scale
    out = []
    for t0 in range(0, len(sc), partition):
        s = sc[t0:t0 + partition]
        m = s.max()
        e = np.exp(s - m)
        out.append((e @ V[t0:t0 + partition].astype(np.float64), m, e.sum()))
    return out


def lse_merge(partials: Sequence[tuple[np.ndarray, float, float]]) -> np.ndarray:
    """Log-sum-exp merge of partition partials (PA/csrc/paged_attention_optimized/
    paged_attention_optimized.cu:185-217): g = max m_p; S = sum s_p e^{m_p - g};
    out = sum acc_p e^{m_p - g} / S."""
    g = max(m for _, m, _ in partials)
    S = sum(l * math.exp(m - g) for _, m, l in partials)
    acc = sum(a * math.exp(m - g) for a, m, _ in partials)
    return acc / S


# ---------------------------------------------------------------------------
# Ragged-batch metadata
# ---------------------------------------------------------------------------


def pack_metadata(seqs: Sequence[tuple[int, int, Sequence[int]]], block_size: int,
                  max_blocks_per_seq: int) -> dict:
    """Brute-force restatement of the per-step tensors paged_forward builds:
    positions start_position + i for a prefill chunk (nanoPD/engine/
    model_runner.py:133-137) and `position` for a decode (engine.py:55-60);
    seq_lens = position + 1 of the last new token (model_runner.py:183);
    block tables zero padded to max_blocks (model_runner.py:178-182); slot
    = table[pos // bs] * bs + pos % bs (PA/csrc/kvstore/paged_kv_store_kernel.cu:45-51),
    -1 past the end of the table. seqs: (q_len, ctx_before, table) in batch order."""
    cu = [0]
    seq_lens, tables, positions, slots, token_seq = [], [], [], [], []
    for s, (ql, ctx, table) in enumerate(seqs):
        ql = max(int(ql), 0)
        cu.append(cu[-1] + ql)
        seq_lens.append(int(ctx) + ql)
        row = [0] * max_blocks_per_seq
        for b in range(min(len(table), max_blocks_per_seq)):
            row[b] = int(table[b])
        tables.append(row)
        for i in range(ql):
            pos = int(ctx) + i
            lb = pos // block_size if pos >= 0 else -1
            slot = int(table[lb]) * block_size + pos % block_size if 0 <= lb < len(table) else -1
            positions.append(pos)
            slots.append(slot)
            token_seq.append(s)
    return {
        "cu_seqlens_q": np.array(cu, dtype=np.int32),
        "seq_lens": np.array(seq_lens, dtype=np.int32),
        "block_tables": np.array(tables, dtype=np.int32).reshape(len(seqs), max_blocks_per_seq),
        "positions": np.array(positions, dtype=np.int32),
        "slot_mapping": np.array(slots, dtype=np.int32),
        "token_seq": np.array(token_seq, dtype=np.int32),
    }


# ---------------------------------------------------------------------------
# Block allocation policy (for generating block tables like the reference)
# ---------------------------------------------------------------------------


class BlockAllocator:
    """LIFO free list starting as [0..N-1], so the first allocation returns the
    highest index (nanoPD/block_manager/block_manager.py:11-39); refcounted."""

    def __init__(self, num_blocks: int):
        self.free = list(range(num_blocks))
        self.ref = [0] * num_blocks

    def allocate(self) -> int:
        if not self.free:
            raise MemoryError("out of KV blocks")
        b = self.free.pop()
        self.ref[b] = 1
        return b

    def fork(self, b: int) -> int:
        self.ref[b] += 1
        return b

    def release(self, b: int) -> None:
        self.ref[b] -= 1
        if self.ref[b] == 0:
            self.free.append(b)


def append_slot(alloc: BlockAllocator, table: list[int], num_tokens: int, block_size: int):
    """Make room for token index `num_tokens` (0-based) in `table`; returns the
    CoW pair (old, new) when the last block is shared, else None
    (nanoPD/block_manager/block_manager.py:72-98)."""
    if num_tokens // block_size >= len(table):
        table.append(alloc.allocate())
        return None
    last = table[-1]
    if alloc.ref[last] > 1:
        new = alloc.allocate()
        alloc.release(last)
        table[-1] = new
        return (last, new)
    return None
