"""Seeded synthetic workloads for the paged-attention path (configs 1-4).

Shapes follow the configurations the path is measured on:
  1. Qwen2-1.5B shape decode: H 12, kvh 2, D 128, fp16, bs 16, pool 256 blocks,
     contexts {17, 64, 200, 511}; every context token goes through the store op.
  2. Qwen3-8B shape decode: H 32, kvh 8, D 128, bf16, bs 16, batch 64, contexts
     uniform in [128, 4096]; one new token per sequence goes through the store op.
  3. ragged mixed batch: 4 prefill chunks of 512 on prefixes {0, 512, 1536, 3072}
     plus 48 decodes with contexts uniform in [256, 2048], packed varlen.
  4. long-context decode: contexts {8k .. 32k} plus a copy-on-write fork of the
     last (partial) block of 2 sequences.
Values are N(0, 1) * 0.5; block tables are slices of a seeded permutation of
the pool (fragmented), zero padded like the reference's
(nanoPD/engine/model_runner.py:177-182). Random draws: numpy for lengths and
permutations, a seeded torch generator on the target device for values.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch


@dataclass
class DecodeWorkload:
    name: str
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    dtype: torch.dtype
    seq_lens_list: list          # tokens attended per sequence (after the store)
    num_blocks: int
    k_cache: torch.Tensor        # [num_blocks, kvh, bs, D]
    v_cache: torch.Tensor
    block_tables: torch.Tensor   # int32 [S, max_bps]
    seq_lens: torch.Tensor       # int32 [S]
    query: torch.Tensor          # [S, H, D]
    store_k: torch.Tensor        # [kvh, T, D] tokens written through the store op
    store_v: torch.Tensor
    store_tables: torch.Tensor   # int32 [T, max_bps]
    store_positions: torch.Tensor  # int32 [T]
    scale: float
    cow_pairs: list = field(default_factory=list)   # (src, dst) block copies

    @property
    def num_seqs(self) -> int:
        return len(self.seq_lens_list)

    @property
    def max_blocks_per_seq(self) -> int:
        return self.block_tables.size(1)

    def kv_bytes(self) -> int:
        """KV bytes the attention reads: each context row once per kv head."""
        elt = torch.finfo(self.dtype).bits // 8
        return sum(self.seq_lens_list) * self.num_kv_heads * self.head_dim * 2 * elt

    def unique_kv_bytes(self) -> int:
        """KV bytes of the distinct pool rows the call reads: a block shared by
        several tables (a copy-on-write fork's prefix) counts once, with the
        most tokens any sequence uses from it."""
        elt = torch.finfo(self.dtype).bits // 8
        used: dict = {}
        tables = self.block_tables.cpu().numpy()
        for s, n in enumerate(self.seq_lens_list):
            nb = (n + self.block_size - 1) // self.block_size
            for j in range(nb):
                b = int(tables[s, j])
                used[b] = max(used.get(b, 0), min(self.block_size, n - j * self.block_size))
        return sum(used.values()) * self.num_kv_heads * self.head_dim * 2 * elt

    def _qo_meta_bytes(self) -> int:
        elt = torch.finfo(self.dtype).bits // 8
        qo = 2 * self.num_seqs * self.num_heads * self.head_dim * elt
        meta = self.num_seqs * self.max_blocks_per_seq * 4 + self.num_seqs * 4
        return qo + meta

    def attention_bytes(self) -> int:
        """Algorithmic bytes of one decode-attention call, per sequence: its KV
        rows + Q + O + block-table row + seq_len (a shared block counts once
        per sequence that reads it)."""
        return self.kv_bytes() + self._qo_meta_bytes()

    def attention_unique_bytes(self) -> int:
        """Bytes one decode-attention call must move from HBM at least: the
        distinct KV rows (unique_kv_bytes) + Q + O + tables + seq_lens. The
        roofline counts these; they equal attention_bytes when no block is
        shared."""
        return self.unique_kv_bytes() + self._qo_meta_bytes()

    def store_bytes(self) -> int:
        """Algorithmic bytes of the store: K/V rows read + written, plus the
        position and the one table entry read per token."""
        elt = torch.finfo(self.dtype).bits // 8
        t = self.store_k.size(1)
        return 4 * t * self.num_kv_heads * self.head_dim * elt + 8 * t


def _values(gen: torch.Generator, shape, dtype, device) -> torch.Tensor:
    return (torch.randn(shape, generator=gen, dtype=torch.float32, device=device) * 0.5).to(dtype)


def _tables(rng: np.random.Generator, seq_lens: list, bs: int, pool: int):
    need = [(n + bs - 1) // bs for n in seq_lens]
    total = sum(need)
    assert total <= pool, "pool too small"
    perm = rng.permutation(pool)[:total]
    mb = max(need + [1])
    tables = np.zeros((len(seq_lens), mb), dtype=np.int32)
    o = 0
    for s, k in enumerate(need):
        tables[s, :k] = perm[o:o + k]
        o += k
    return tables


def make_decode_workload(name: str, *, num_heads: int, num_kv_heads: int, head_dim: int,
                         block_size: int, dtype: torch.dtype, seq_lens: list,
                         pool_blocks: int | None = None, pool_factor: float = 1.25,
                         store_all_context: bool = False, seed: int = 0,
                         device: str | torch.device = "cpu",
                         gen_device: str | torch.device | None = None) -> DecodeWorkload:
    """Build a decode workload. With store_all_context every context token is
    written through the store op into a zeroed pool (config 1); otherwise the
    pool is random and only the last token of each sequence is stored
    (configs 2 and 4). Values are drawn on gen_device (default: device) and
    moved; drawing on the CPU makes them identical on every machine."""
    rng = np.random.default_rng(seed)
    dev = torch.device(device)
    gdev = torch.device(gen_device) if gen_device is not None else dev
    gen = torch.Generator(device=gdev)
    gen.manual_seed(seed)
    bs = block_size
    total_blocks = sum((n + bs - 1) // bs for n in seq_lens)
    pool = pool_blocks if pool_blocks is not None else int(math.ceil(pool_factor * total_blocks))
    tables = _tables(rng, seq_lens, bs, pool)
    shape = (pool, num_kv_heads, bs, head_dim)
    if store_all_context:
        k_cache = torch.zeros(shape, dtype=dtype, device=gdev)
        v_cache = torch.zeros(shape, dtype=dtype, device=gdev)
        tok_seq = np.concatenate([np.full(n, s, dtype=np.int64) for s, n in enumerate(seq_lens)])
        positions = np.concatenate([np.arange(n, dtype=np.int32) for n in seq_lens])
    else:
        k_cache = _values(gen, shape, dtype, gdev)
        v_cache = _values(gen, shape, dtype, gdev)
        tok_seq = np.arange(len(seq_lens), dtype=np.int64)
        positions = np.array([n - 1 for n in seq_lens], dtype=np.int32)
    T = len(positions)
    store_k = _values(gen, (num_kv_heads, T, head_dim), dtype, gdev).to(dev)
    store_v = _values(gen, (num_kv_heads, T, head_dim), dtype, gdev).to(dev)
    query = _values(gen, (len(seq_lens), num_heads, head_dim), dtype, gdev).to(dev)
    k_cache, v_cache = k_cache.to(dev), v_cache.to(dev)
    return DecodeWorkload(
        name=name, num_heads=num_heads, num_kv_heads=num_kv_heads, head_dim=head_dim,
        block_size=bs, dtype=dtype, seq_lens_list=list(seq_lens), num_blocks=pool,
        k_cache=k_cache, v_cache=v_cache,
        block_tables=torch.from_numpy(tables).to(dev),
        seq_lens=torch.tensor(seq_lens, dtype=torch.int32, device=dev),
        query=query, store_k=store_k, store_v=store_v,
        store_tables=torch.from_numpy(np.ascontiguousarray(tables[tok_seq])).to(dev),
        store_positions=torch.from_numpy(positions).to(dev),
        scale=1.0 / math.sqrt(head_dim))


def config1(device="cpu", seed: int = 1) -> DecodeWorkload:
    """Drawn on the CPU, so the values (and the golden fixture) are the same
    on every machine."""
    return make_decode_workload(
        "cfg1_qwen2_1.5b_decode", num_heads=12, num_kv_heads=2, head_dim=128, block_size=16,
        dtype=torch.float16, seq_lens=[17, 64, 200, 511], pool_blocks=256,
        store_all_context=True, seed=seed, device=device, gen_device="cpu")


def config2_seq_lens(seed: int = 2, batch: int = 64) -> list:
    rng = np.random.default_rng(seed + 1000)
    return [int(x) for x in rng.integers(128, 4096, size=batch, endpoint=True)]


def config2(device="cpu", seed: int = 2, batch: int = 64, num_heads: int = 32,
            head_dim: int = 128, block_size: int = 16) -> DecodeWorkload:
    """Configuration 2 (32 q / 8 kv heads, head dim 128, blocks of 16). Other
    values give the same contexts and kv heads with another group size (e.g.
    num_heads 64: the 64 q / 8 kv heads of larger Qwen models), head dim or
    block size."""
    if (num_heads, head_dim, block_size) == (32, 128, 16):
        name = "cfg2_qwen3_8b_decode_b64"
    else:
        name = f"cfg2_contexts_h{num_heads}_kv8_b64"
        name += f"_d{head_dim}" if head_dim != 128 else ""
        name += f"_bs{block_size}" if block_size != 16 else ""
    return make_decode_workload(
        name, num_heads=num_heads, num_kv_heads=8, head_dim=head_dim, block_size=block_size,
        dtype=torch.bfloat16, seq_lens=config2_seq_lens(seed, batch), seed=seed, device=device)


def config4(device="cpu", seed: int = 4) -> DecodeWorkload:
    """Long-context decode with a CoW fork: 8 sequences of {8..32}k context get
    one new token each (which opens a new, partial block); sequences 6 and 7 are
    then forked, and each child's append_slot copies the shared partial block
    (nanoPD/block_manager/block_manager.py:72-98). Attention runs over the 8
    parents and the 2 children (10 sequences)."""
    ctx = [k * 1024 for k in (8, 12, 16, 20, 24, 28, 32, 32)]
    base = make_decode_workload(
        "cfg4_long_decode_cow", num_heads=32, num_kv_heads=8, head_dim=128, block_size=16,
        dtype=torch.bfloat16, seq_lens=[n + 1 for n in ctx], pool_factor=1.25, seed=seed,
        device=device)
    # Free blocks = the pool blocks no table uses; LIFO like BlockAllocator.
    used = set(base.block_tables.cpu().numpy().ravel().tolist())
    free = [b for b in range(base.num_blocks) if b not in used]
    tables = base.block_tables.cpu().numpy()
    parents = [6, 7]
    child_rows, pairs = [], []
    for p in parents:
        n_blk = (base.seq_lens_list[p] + base.block_size - 1) // base.block_size
        row = tables[p].copy()
        new = free.pop()
        pairs.append((int(row[n_blk - 1]), int(new)))
        row[n_blk - 1] = new
        child_rows.append(row)
    dev = base.k_cache.device
    base.block_tables = torch.from_numpy(np.concatenate([tables, np.stack(child_rows)])).to(dev)
    base.seq_lens_list = base.seq_lens_list + [base.seq_lens_list[p] for p in parents]
    base.seq_lens = torch.tensor(base.seq_lens_list, dtype=torch.int32, device=dev)
    base.query = torch.cat([base.query, base.query[parents]], dim=0)
    base.cow_pairs = pairs
    return base


@dataclass
class MixedWorkload:
    """Config 3: prefill chunks + decodes in one varlen batch (prefills first,
    as paged_forward orders tokens, nanoPD/engine/model_runner.py:120-125)."""
    name: str
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    dtype: torch.dtype
    chunk_lens: list       # q_len per sequence (chunk size or 1)
    ctx_before: list       # cached tokens before this step
    num_blocks: int
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    block_tables: torch.Tensor   # int32 [S, max_bps]
    cu_seqlens_q: torch.Tensor   # int32 [S + 1]
    context_lens: torch.Tensor   # int32 [S], ctx_before + q_len
    slot_mapping: torch.Tensor   # int32 [T]
    query: torch.Tensor          # [T, H, D]
    new_k: torch.Tensor          # [T, kvh, D] (token major, as k_proj produces)
    new_v: torch.Tensor
    num_prefill_seqs: int
    scale: float

    @property
    def num_prefill_tokens(self) -> int:
        return sum(self.chunk_lens[: self.num_prefill_seqs])

    def prefill_flops(self) -> int:
        """Useful (unmasked causal) FLOPs of the prefill part:
        4 * H * D * sum(C * P + C (C + 1) / 2)."""
        tot = 0
        for c, p in zip(self.chunk_lens[: self.num_prefill_seqs], self.ctx_before):
            tot += c * p + c * (c + 1) // 2
        return 4 * self.num_heads * self.head_dim * tot

    def store_bytes(self) -> int:
        """Algorithmic bytes of the step's slot store: every new token's K/V
        rows read + written, plus its int32 slot."""
        elt = torch.finfo(self.dtype).bits // 8
        t = self.new_k.size(0)
        return 4 * t * self.num_kv_heads * self.head_dim * elt + 4 * t


def config3(device="cpu", seed: int = 3, chunk: int = 512, prefixes=(0, 512, 1536, 3072),
            num_decodes: int = 48) -> MixedWorkload:
    rng = np.random.default_rng(seed)
    dev = torch.device(device)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    H, kvh, D, bs, dtype = 32, 8, 128, 16, torch.bfloat16
    dec_ctx = [int(x) for x in rng.integers(256, 2048, size=num_decodes, endpoint=True)]
    chunk_lens = [chunk] * len(prefixes) + [1] * num_decodes
    ctx_before = list(prefixes) + [n - 1 for n in dec_ctx]
    ctx_after = [c + q for c, q in zip(ctx_before, chunk_lens)]
    total_blocks = sum((n + bs - 1) // bs for n in ctx_after)
    pool = int(math.ceil(1.25 * total_blocks))
    tables = _tables(rng, ctx_after, bs, pool)
    shape = (pool, kvh, bs, D)
    k_cache = _values(gen, shape, dtype, dev)
    v_cache = _values(gen, shape, dtype, dev)
    cu = np.concatenate([[0], np.cumsum(chunk_lens)]).astype(np.int32)
    slots = []
    for s, (q, c) in enumerate(zip(chunk_lens, ctx_before)):
        for i in range(q):
            pos = c + i
            slots.append(int(tables[s, pos // bs]) * bs + pos % bs)
    T = int(cu[-1])
    return MixedWorkload(
        name="cfg3_mixed_chunked_prefill", num_heads=H, num_kv_heads=kvh, head_dim=D,
        block_size=bs, dtype=dtype, chunk_lens=chunk_lens, ctx_before=ctx_before,
        num_blocks=pool, k_cache=k_cache, v_cache=v_cache,
        block_tables=torch.from_numpy(tables).to(dev),
        cu_seqlens_q=torch.from_numpy(cu).to(dev),
        context_lens=torch.tensor(ctx_after, dtype=torch.int32, device=dev),
        slot_mapping=torch.tensor(slots, dtype=torch.int32, device=dev),
        query=_values(gen, (T, H, D), dtype, dev),
        new_k=_values(gen, (T, kvh, D), dtype, dev),
        new_v=_values(gen, (T, kvh, D), dtype, dev),
        num_prefill_seqs=len(prefixes), scale=1.0 / math.sqrt(D))
