"""The reference's own PyTorch paths, restated, run on host cores.

TEST INFRASTRUCTURE ONLY: used by tests/ as a second, structurally different
checker and by bench.py's cpu_baseline leg as the timed CPU baseline. The
reference's Python is never imported or shipped; these are restatements:

* ref_paged_attention -- PA/tests/test_paged_attention.py:33-71 (per-sequence
  gather over block_tables, repeat_interleave for GQA, fp32 bmm -> softmax ->
  bmm, cast to the storage dtype). PA/ = nanoPD/paged_attention/.
* ref_prefill_sdpa -- nanoPD/engine/model_runner.py:152-168 (block-diagonal
  causal mask over the packed chunks, repeat_interleave, SDPA; chunk only).
* ref_kv_store_loop -- the Python scatter loop of
  nanoPD/docs/en/03-cuda_kernels_en.md:69-78.
* ref_extract_kv / ref_load_kv -- the per-block copies of extract_kv_to_pinned
  and load_kv_from_pinned (nanoPD/workers/kv_transfer.py:45-69), into and out
  of an ordinary (not pinned) buffer.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def ref_paged_attention(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                        block_tables: torch.Tensor, seq_lens: torch.Tensor,
                        scale: float) -> torch.Tensor:
    num_seqs, num_heads, _ = query.shape
    num_kv_heads = key_cache.size(1)
    block_size = key_cache.size(2)
    group = num_heads // num_kv_heads
    outs = []
    for s in range(num_seqs):
        n = int(seq_lens[s])
        nb = (n + block_size - 1) // block_size
        idx = block_tables[s, :nb].long()
        keys = key_cache[idx].transpose(0, 1).reshape(num_kv_heads, nb * block_size, -1)[:, :n]
        vals = value_cache[idx].transpose(0, 1).reshape(num_kv_heads, nb * block_size, -1)[:, :n]
        keys = keys.repeat_interleave(group, dim=0).float()
        vals = vals.repeat_interleave(group, dim=0).float()
        q = query[s].unsqueeze(1).float()
        attn = torch.bmm(q, keys.transpose(1, 2).contiguous()) * scale
        attn = F.softmax(attn, dim=-1)
        outs.append(torch.bmm(attn, vals).squeeze(1))
    return torch.stack(outs).to(query.dtype)


def ref_prefill_sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, chunk_lens: list,
                     scale: float) -> torch.Tensor:
    """q [T, H, D], k/v [T, kvh, D] of the packed chunks; returns [T, H, D]."""
    T, H, D = q.shape
    group = H // k.size(1)
    mask = torch.full((T, T), float("-inf"), dtype=torch.float32)
    o = 0
    for n in chunk_lens:
        mask[o:o + n, o:o + n] = torch.triu(torch.full((n, n), float("-inf")), diagonal=1)
        o += n
    qh = q.transpose(0, 1).unsqueeze(0).float()                     # (1, H, T, D)
    kh = k.transpose(0, 1).repeat_interleave(group, dim=0).unsqueeze(0).float()
    vh = v.transpose(0, 1).repeat_interleave(group, dim=0).unsqueeze(0).float()
    out = F.scaled_dot_product_attention(qh, kh, vh, attn_mask=mask, scale=scale)
    return out[0].transpose(0, 1).to(q.dtype)


def ref_kv_store_loop(k_cache: torch.Tensor, v_cache: torch.Tensor, k_src: torch.Tensor,
                      v_src: torch.Tensor, block_tables: torch.Tensor,
                      positions: torch.Tensor) -> None:
    block_size = k_cache.size(2)
    for i in range(k_src.size(1)):
        position = int(positions[i])
        phys = int(block_tables[i, position // block_size])
        k_cache[phys, :, position % block_size, :] = k_src[:, i, :]
        v_cache[phys, :, position % block_size, :] = v_src[:, i, :]


def ref_extract_kv(k_cache: torch.Tensor, v_cache: torch.Tensor, block_table) -> tuple:
    """kv_transfer.py:45-53: buf.k[:, i].copy_(k_cache[:, bid]) per block."""
    shape = (k_cache.size(0), len(block_table)) + tuple(k_cache.shape[2:])
    bk = torch.empty(shape, dtype=k_cache.dtype)
    bv = torch.empty(shape, dtype=v_cache.dtype)
    for i, bid in enumerate(block_table):
        bk[:, i].copy_(k_cache[:, bid])
        bv[:, i].copy_(v_cache[:, bid])
    return bk, bv


def ref_load_kv(k_cache: torch.Tensor, v_cache: torch.Tensor, block_table, bk: torch.Tensor,
                bv: torch.Tensor) -> None:
    """kv_transfer.py:56-69: k_cache[:, bid].copy_(buf.k[:, i]) per block."""
    for i, bid in enumerate(block_table):
        k_cache[:, bid].copy_(bk[:, i])
        v_cache[:, bid].copy_(bv[:, i])
