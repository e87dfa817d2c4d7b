"""MI355X drop-in for nanoPD's ``paged_kernels`` extension.

Same Python-visible ops, argument meaning and error behaviour as the reference
module built by PA/setup.py:6-15 (PA/ = nanoPD/paged_attention/):

* :func:`paged_kv_store` -- PA/csrc/kvstore/paged_kv_store.h:23-27
* :func:`paged_attention_forward` -- PA/csrc/attention/paged_attention.h:24-34

plus the ops the MI355X path adds:

* :func:`paged_kv_store_slots` -- store by flat slot mapping, strided sources
* :func:`paged_prefill_attention` -- varlen chunked prefill over the paged prefix
* :func:`copy_blocks` -- copy-on-write block copy
* :func:`qk_norm_rope_store` -- Qwen3 q/k RMSNorm + RoPE + paged K/V store, fused
* :func:`pack_metadata` -- ragged-batch metadata built on the GPU

Every op validates its arguments here (``RuntimeError``, as ``TORCH_CHECK``
raises in the reference) and again in the C library, then enqueues HIP kernels
on the current stream of the tensors' device; nothing synchronises the host.
There is no CPU or PyTorch fallback: without the built library every op raises.
"""
from __future__ import annotations

import threading
from typing import NamedTuple, Sequence

import torch

from . import _lib

__all__ = [
    "paged_kv_store", "paged_kv_store_slots", "paged_attention_forward",
    "paged_prefill_attention", "copy_blocks", "pack_metadata", "BatchMetadata",
    "attention_workspace_bytes", "prefill_workspace_bytes", "qk_norm_rope_store",
]

_DTYPES = {torch.float16: _lib.NPD_DTYPE_F16, torch.bfloat16: _lib.NPD_DTYPE_BF16}


def _fail(msg: str) -> None:
    raise RuntimeError(msg)


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _dtype_code(t: torch.Tensor, what: str) -> int:
    code = _DTYPES.get(t.dtype)
    _check(code is not None, f"{what}: dtype {t.dtype} not supported (float16 / bfloat16)")
    return code


def _int32(t: torch.Tensor, what: str) -> None:
    _check(isinstance(t, torch.Tensor), f"{what} must be a tensor")
    _check(t.dtype == torch.int32, f"{what} must be int32 (got {t.dtype})")


def _same_device(dev: torch.device, *ts: torch.Tensor) -> None:
    for t in ts:
        _check(t.device == dev, f"tensor on {t.device}, expected {dev}")


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _cache_checks(k_cache: torch.Tensor, v_cache: torch.Tensor) -> None:
    _check(k_cache.dim() == 4 and v_cache.dim() == 4,
           "caches must be [num_blocks, num_kv_heads, block_size, head_dim]")
    _check(k_cache.shape == v_cache.shape, "k_cache and v_cache shapes differ")
    _check(k_cache.dtype == v_cache.dtype, "k_cache and v_cache dtypes differ")
    _check(k_cache.is_contiguous() and v_cache.is_contiguous(), "caches must be contiguous")


# ---------------------------------------------------------------------------
# KV store
# ---------------------------------------------------------------------------

def paged_kv_store(k_cache: torch.Tensor, v_cache: torch.Tensor, k_src: torch.Tensor,
                   v_src: torch.Tensor, block_tables: torch.Tensor, positions) -> None:
    """Scatter K/V rows into the paged pool (reference: paged_kv_store_ops.cu:7-50).

    k_src/v_src: [num_kv_heads, num_tokens, head_dim] (any strides with a
    contiguous last dim); block_tables: int32 [num_tokens, max_blocks_per_seq],
    one row per token; positions: int32 [num_tokens]. Token t goes to
    ``cache[block_tables[t, pos // bs], h, pos % bs]`` with ``pos = positions[t]``.

    The older form used by PA/tests/test_paged_kernels.py:250-261,
    ``(k_cache, v_cache, k_src[1, kvh, T, D], v_src, block_table[nb], start_pos: int)``,
    is accepted too and means positions ``start_pos + t`` on a shared table.
    """
    _check(isinstance(k_src, torch.Tensor) and k_src.is_cuda, "k src is must be on CUDA")
    _check(isinstance(v_src, torch.Tensor) and v_src.is_cuda, "v src is must be on CUDA")
    if isinstance(positions, int):
        _check(k_src.dim() == 4 and k_src.size(0) == 1 and v_src.dim() == 4,
               "start-position form needs k_src/v_src of shape [1, kvh, T, D]")
        _int32(block_tables, "block_table")
        _check(block_tables.dim() == 1, "start-position form needs a 1-D block table")
        k_src, v_src = k_src[0], v_src[0]
        n = k_src.size(1)
        positions = torch.arange(positions, positions + n, dtype=torch.int32, device=k_src.device)
        block_tables = block_tables.unsqueeze(0).expand(n, -1).contiguous()
    _check(k_src.dim() == 3, "k_src must be [num_kv_heads, num_tokens, head_dim]")
    _check(v_src.shape == k_src.shape, "k_src and v_src shapes differ")
    _cache_checks(k_cache, v_cache)
    _int32(block_tables, "block_tables")
    _int32(positions, "positions")
    dev = k_src.device
    _same_device(dev, v_src, k_cache, v_cache, block_tables, positions)
    kvh, n, d = k_src.shape
    num_blocks, ckvh, bs, cd = k_cache.shape
    _check(ckvh == kvh and cd == d, f"source [{kvh}, {n}, {d}] does not match cache {tuple(k_cache.shape)}")
    _check(k_src.dtype == k_cache.dtype and v_src.dtype == k_cache.dtype, "source/cache dtype mismatch")
    code = _dtype_code(k_cache, "paged_kv_store")
    _check(block_tables.dim() == 2 and block_tables.size(0) >= n,
           "block_tables must be [num_tokens, max_blocks_per_seq]")
    _check(block_tables.is_contiguous(), "block_tables must be contiguous")
    _check(positions.dim() == 1 and positions.numel() >= n and positions.is_contiguous(),
           "positions must be a contiguous [num_tokens] tensor")
    if n == 0:
        return
    if k_src.stride(2) != 1 or v_src.stride() != k_src.stride():
        k_src, v_src = k_src.contiguous(), v_src.contiguous()
    _lib.call("npd_paged_kv_store", k_cache.data_ptr(), v_cache.data_ptr(), k_src.data_ptr(),
              v_src.data_ptr(), block_tables.data_ptr(), positions.data_ptr(), n, kvh, d,
              num_blocks, bs, block_tables.size(1), k_src.stride(0), k_src.stride(1), code,
              _stream(dev))


def paged_kv_store_slots(k_cache: torch.Tensor, v_cache: torch.Tensor, k_src: torch.Tensor,
                         v_src: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """Scatter token-major K/V rows by flat slot (no reference counterpart).

    k_src/v_src: [num_tokens, num_kv_heads, head_dim] with any strides on the
    first two dims (a view of the k_proj output needs no copy); slot_mapping:
    int32 [num_tokens], ``slot = block * block_size + offset``; negative slots
    are skipped.
    """
    _check(isinstance(k_src, torch.Tensor) and k_src.is_cuda, "k src is must be on CUDA")
    _check(isinstance(v_src, torch.Tensor) and v_src.is_cuda, "v src is must be on CUDA")
    _check(k_src.dim() == 3, "k_src must be [num_tokens, num_kv_heads, head_dim]")
    _check(v_src.shape == k_src.shape, "k_src and v_src shapes differ")
    _cache_checks(k_cache, v_cache)
    _int32(slot_mapping, "slot_mapping")
    dev = k_src.device
    _same_device(dev, v_src, k_cache, v_cache, slot_mapping)
    n, kvh, d = k_src.shape
    num_blocks, ckvh, bs, cd = k_cache.shape
    _check(ckvh == kvh and cd == d, "source does not match cache shape")
    _check(k_src.dtype == k_cache.dtype and v_src.dtype == k_cache.dtype, "source/cache dtype mismatch")
    code = _dtype_code(k_cache, "paged_kv_store_slots")
    _check(slot_mapping.dim() == 1 and slot_mapping.numel() >= n and slot_mapping.is_contiguous(),
           "slot_mapping must be a contiguous [num_tokens] tensor")
    if n == 0:
        return
    if k_src.stride(2) != 1 or v_src.stride() != k_src.stride():
        k_src, v_src = k_src.contiguous(), v_src.contiguous()
    _lib.call("npd_paged_kv_store_slots", k_cache.data_ptr(), v_cache.data_ptr(), k_src.data_ptr(),
              v_src.data_ptr(), slot_mapping.data_ptr(), n, kvh, d, num_blocks, bs,
              k_src.stride(1), k_src.stride(0), code, _stream(dev))


FP8_DTYPES = (torch.uint8, torch.float8_e4m3fn)


def _fp8_cache_checks(k_cache: torch.Tensor, v_cache: torch.Tensor, k_scale: torch.Tensor,
                      v_scale: torch.Tensor) -> None:
    _check(k_cache.dim() == 4 and v_cache.dim() == 4 and k_cache.shape == v_cache.shape,
           "fp8 caches must be [num_blocks, num_kv_heads, block_size, head_dim]")
    _check(k_cache.dtype in FP8_DTYPES and v_cache.dtype == k_cache.dtype,
           "fp8 caches must be torch.float8_e4m3fn (or uint8 holding e4m3 bytes)")
    _check(k_cache.is_contiguous() and v_cache.is_contiguous(), "caches must be contiguous")
    kvh = k_cache.size(1)
    for sc, nm in ((k_scale, "k_scale"), (v_scale, "v_scale")):
        _check(isinstance(sc, torch.Tensor) and sc.dtype == torch.float32 and sc.dim() == 1
               and sc.numel() == kvh and sc.is_contiguous(),
               f"{nm} must be a contiguous float32 [num_kv_heads] tensor")


def paged_kv_store_slots_fp8(k_cache: torch.Tensor, v_cache: torch.Tensor, k_src: torch.Tensor,
                             v_src: torch.Tensor, slot_mapping: torch.Tensor,
                             k_scale: torch.Tensor, v_scale: torch.Tensor) -> None:
    """:func:`paged_kv_store_slots` into an FP8 (OCP e4m3) pool with
    per-kv-head scales (no reference counterpart; its caches are fp16):
    byte = e4m3(clamp(x / scale[h], -448, 448)), round to nearest even."""
    _check(isinstance(k_src, torch.Tensor) and k_src.is_cuda, "k src is must be on CUDA")
    _check(k_src.dim() == 3 and v_src.shape == k_src.shape,
           "k_src / v_src must be [num_tokens, num_kv_heads, head_dim]")
    _fp8_cache_checks(k_cache, v_cache, k_scale, v_scale)
    _int32(slot_mapping, "slot_mapping")
    dev = k_src.device
    _same_device(dev, v_src, k_cache, v_cache, slot_mapping, k_scale, v_scale)
    n, kvh, d = k_src.shape
    num_blocks, ckvh, bs, cd = k_cache.shape
    _check(ckvh == kvh and cd == d, "source does not match cache shape")
    _check(v_src.dtype == k_src.dtype, "k_src / v_src dtypes differ")
    code = _dtype_code(k_src, "paged_kv_store_slots_fp8")
    _check(slot_mapping.dim() == 1 and slot_mapping.numel() >= n and slot_mapping.is_contiguous(),
           "slot_mapping must be a contiguous [num_tokens] tensor")
    if n == 0:
        return
    if k_src.stride(2) != 1 or v_src.stride() != k_src.stride():
        k_src, v_src = k_src.contiguous(), v_src.contiguous()
    _lib.call("npd_paged_kv_store_slots_fp8", k_cache.data_ptr(), v_cache.data_ptr(),
              k_src.data_ptr(), v_src.data_ptr(), slot_mapping.data_ptr(), k_scale.data_ptr(),
              v_scale.data_ptr(), n, kvh, d, num_blocks, bs, k_src.stride(1), k_src.stride(0), code,
              _stream(dev))


# ---------------------------------------------------------------------------
# Decode attention
# ---------------------------------------------------------------------------

# Cached decode workspaces, one per (device, stream), so that calls on
# different streams never share one. They are zero-filled when made: the fast
# decode path keeps per-(sequence, kv-head) merge counters in the workspace and
# leaves them zero after every call, so zeroing once is enough.
_workspaces: dict = {}
_workspaces_lock = threading.Lock()


def _decode_workspace(dev: torch.device, stream: int, need: int, kind: str = "decode") -> torch.Tensor:
    """A zero-filled workspace cached per (device, stream, op): the kernels
    leave their merge counters at zero, so it is cleared only when allocated.
    The lookup and the insert hold a lock (callers on several host threads)."""
    key = (dev.index, stream, kind)
    with _workspaces_lock:
        ws = _workspaces.get(key)
        if ws is None or ws.numel() < need:
            ws = torch.zeros(need, dtype=torch.uint8, device=dev)
            _workspaces[key] = ws
        return ws


def attention_workspace_bytes(num_seqs: int, num_heads: int, num_kv_heads: int, head_dim: int,
                              block_size: int, max_num_blocks_per_seq: int) -> int:
    return int(_lib.load().npd_paged_attention_workspace_size(
        num_seqs, num_heads, num_kv_heads, head_dim, block_size, max_num_blocks_per_seq))


def paged_attention_forward(out: torch.Tensor, query: torch.Tensor, key_cache: torch.Tensor,
                            value_cache: torch.Tensor, block_tables: torch.Tensor,
                            seq_lens: torch.Tensor, scale: float, block_size: int,
                            max_num_blocks_per_seq: int, workspace: torch.Tensor | None = None) -> None:
    """Paged decode attention into ``out`` (reference: paged_attention_ops.cu:7-59).

    query/out: [num_seqs, num_heads, head_dim]; caches [num_blocks, kvh,
    block_size, head_dim]; block_tables: int32 [num_seqs, max_num_blocks_per_seq];
    seq_lens: int32 [num_seqs], the number of cached tokens to attend over
    (including the token just stored). ``out`` is fully overwritten. An optional
    uint8 ``workspace`` of at least :func:`attention_workspace_bytes` bytes,
    zero-filled before its first use, replaces the cached per-stream one; calls
    that share a workspace must run in stream order.
    """
    _check(isinstance(query, torch.Tensor) and query.is_cuda, "query is must be on CUDA")
    _check(query.dim() == 3, "query must be [num seqs, num_heads, head_size]")
    _check(key_cache.dim() == 4, "key_cache must be [num_blocks, num_kv_heads, block_size, head_size]")
    _int32(block_tables, "block_tables")
    _int32(seq_lens, "seq_lens")
    _cache_checks(key_cache, value_cache)
    dev = query.device
    _same_device(dev, out, key_cache, value_cache, block_tables, seq_lens)
    s, h, d = query.shape
    num_blocks, kvh, bs, cd = key_cache.shape
    _check(cd == d, f"head_dim {d} does not match cache head_dim {cd}")
    _check(int(block_size) == bs, f"block_size {block_size} does not match cache block size {bs}")
    _check(h % kvh == 0, f"num_heads {h} is not a multiple of num_kv_heads {kvh}")
    _check(out.shape == query.shape and out.dtype == query.dtype, "out must match query")
    _check(query.dtype == key_cache.dtype, "query/cache dtype mismatch")
    code = _dtype_code(query, "paged_attention_forward")
    mb = int(max_num_blocks_per_seq)
    _check(block_tables.dim() == 2 and block_tables.size(0) >= s and block_tables.size(1) == mb,
           "block_tables must be [num_seqs, max_num_blocks_per_seq]")
    _check(block_tables.is_contiguous(), "block_tables must be contiguous")
    _check(seq_lens.dim() == 1 and seq_lens.numel() >= s and seq_lens.is_contiguous(),
           "seq_lens must be a contiguous [num_seqs] tensor")
    _check(query.stride(2) == 1 and out.stride(2) == 1, "head_dim must be the contiguous dim")
    if s == 0:
        return
    need = attention_workspace_bytes(s, h, kvh, d, bs, mb)
    stream = _stream(dev)
    ws_ptr = 0
    if need > 0:
        if workspace is None:
            workspace = _decode_workspace(dev, stream, need)
        _check(workspace.numel() * workspace.element_size() >= need,
               f"workspace of {need} bytes needed")
        ws_ptr = workspace.data_ptr()
    _lib.call("npd_paged_attention", out.data_ptr(), query.data_ptr(), key_cache.data_ptr(),
              value_cache.data_ptr(), block_tables.data_ptr(), seq_lens.data_ptr(), s, h, kvh, d,
              num_blocks, bs, mb, float(scale), query.stride(0), query.stride(1), out.stride(0),
              out.stride(1), ws_ptr, need, code, stream)


def paged_attention_forward_fp8(out: torch.Tensor, query: torch.Tensor, key_cache: torch.Tensor,
                                value_cache: torch.Tensor, block_tables: torch.Tensor,
                                seq_lens: torch.Tensor, scale: float, block_size: int,
                                max_num_blocks_per_seq: int, k_scale: torch.Tensor,
                                v_scale: torch.Tensor,
                                workspace: torch.Tensor | None = None) -> None:
    """:func:`paged_attention_forward` over an FP8 pool written by
    :func:`paged_kv_store_slots_fp8`: K = e4m3(byte) * k_scale[kv head], V
    likewise. query/out fp16 or bf16; head_dim 128; block_size 16 or 32."""
    _check(isinstance(query, torch.Tensor) and query.is_cuda, "query is must be on CUDA")
    _check(query.dim() == 3, "query must be [num seqs, num_heads, head_size]")
    _fp8_cache_checks(key_cache, value_cache, k_scale, v_scale)
    _int32(block_tables, "block_tables")
    _int32(seq_lens, "seq_lens")
    dev = query.device
    _same_device(dev, out, key_cache, value_cache, block_tables, seq_lens, k_scale, v_scale)
    s, h, d = query.shape
    num_blocks, kvh, bs, cd = key_cache.shape
    _check(cd == d, f"head_dim {d} does not match cache head_dim {cd}")
    _check(int(block_size) == bs, f"block_size {block_size} does not match cache block size {bs}")
    _check(h % kvh == 0, f"num_heads {h} is not a multiple of num_kv_heads {kvh}")
    _check(out.shape == query.shape and out.dtype == query.dtype, "out must match query")
    code = _dtype_code(query, "paged_attention_forward_fp8")
    mb = int(max_num_blocks_per_seq)
    _check(block_tables.dim() == 2 and block_tables.size(0) >= s and block_tables.size(1) == mb,
           "block_tables must be [num_seqs, max_num_blocks_per_seq]")
    _check(block_tables.is_contiguous(), "block_tables must be contiguous")
    _check(seq_lens.dim() == 1 and seq_lens.numel() >= s and seq_lens.is_contiguous(),
           "seq_lens must be a contiguous [num_seqs] tensor")
    _check(query.stride(2) == 1 and out.stride(2) == 1, "head_dim must be the contiguous dim")
    if s == 0:
        return
    need = attention_workspace_bytes(s, h, kvh, d, bs, mb)
    stream = _stream(dev)
    ws_ptr = 0
    if need > 0:
        if workspace is None:
            workspace = _decode_workspace(dev, stream, need)
        _check(workspace.numel() * workspace.element_size() >= need,
               f"workspace of {need} bytes needed")
        ws_ptr = workspace.data_ptr()
    _lib.call("npd_paged_attention_fp8", out.data_ptr(), query.data_ptr(), key_cache.data_ptr(),
              value_cache.data_ptr(), block_tables.data_ptr(), seq_lens.data_ptr(),
              k_scale.data_ptr(), v_scale.data_ptr(), s, h, kvh, d, num_blocks, bs, mb,
              float(scale), query.stride(0), query.stride(1), out.stride(0), out.stride(1), ws_ptr,
              need, code, stream)


# ---------------------------------------------------------------------------
# Chunked prefill attention
# ---------------------------------------------------------------------------

def prefill_workspace_bytes(num_seqs: int, total_q: int, num_heads: int, head_dim: int,
                            max_q_len: int, max_context_len: int) -> int:
    return int(_lib.load().npd_paged_prefill_workspace_size(
        num_seqs, total_q, num_heads, head_dim, max_q_len, max_context_len))


def _prefill(out, query, key_cache, value_cache, block_tables, cu_seqlens_q, context_lens, scale,
             block_size, max_num_blocks_per_seq, max_q_len, max_context_len, workspace,
             fp8_scales):
    _check(isinstance(query, torch.Tensor) and query.is_cuda, "query is must be on CUDA")
    _check(query.dim() == 3, "query must be [total_q, num_heads, head_size]")
    _int32(block_tables, "block_tables")
    _int32(cu_seqlens_q, "cu_seqlens_q")
    _int32(context_lens, "context_lens")
    if fp8_scales is None:
        _cache_checks(key_cache, value_cache)
    else:
        _fp8_cache_checks(key_cache, value_cache, *fp8_scales)
    dev = query.device
    _same_device(dev, out, key_cache, value_cache, block_tables, cu_seqlens_q, context_lens,
                 *(fp8_scales or ()))
    tq, h, d = query.shape
    num_blocks, kvh, bs, cd = key_cache.shape
    _check(cd == d, f"head_dim {d} does not match cache head_dim {cd}")
    _check(int(block_size) == bs, f"block_size {block_size} does not match cache block size {bs}")
    _check(h % kvh == 0, f"num_heads {h} is not a multiple of num_kv_heads {kvh}")
    _check(out.shape == query.shape and out.dtype == query.dtype, "out must match query")
    if fp8_scales is None:
        _check(query.dtype == key_cache.dtype, "query/cache dtype mismatch")
    code = _dtype_code(query, "paged_prefill_attention")
    ns = cu_seqlens_q.numel() - 1
    mb = int(max_num_blocks_per_seq)
    _check(ns >= 0 and cu_seqlens_q.dim() == 1 and cu_seqlens_q.is_contiguous(),
           "cu_seqlens_q must be a contiguous [num_seqs + 1] tensor")
    _check(context_lens.dim() == 1 and context_lens.numel() >= ns and context_lens.is_contiguous(),
           "context_lens must be a contiguous [num_seqs] tensor")
    _check(block_tables.dim() == 2 and block_tables.size(0) >= ns and block_tables.size(1) == mb
           and block_tables.is_contiguous(), "block_tables must be [num_seqs, max_num_blocks_per_seq]")
    _check(query.stride(2) == 1 and out.stride(2) == 1, "head_dim must be the contiguous dim")
    if ns == 0 or tq == 0:
        return
    mctx = int(max_context_len) if max_context_len is not None else mb * bs
    need = prefill_workspace_bytes(ns, tq, h, d, int(max_q_len), mctx)
    stream = _stream(dev)
    ws_ptr = 0
    if need > 0:
        if workspace is None:
            workspace = _decode_workspace(dev, stream, need, "prefill")
        _check(workspace.numel() * workspace.element_size() >= need,
               f"workspace of {need} bytes needed")
        ws_ptr = workspace.data_ptr()
    ptrs = (out.data_ptr(), query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
            block_tables.data_ptr(), cu_seqlens_q.data_ptr(), context_lens.data_ptr())
    sizes = (ns, tq, h, kvh, d, num_blocks, bs, mb, int(max_q_len), mctx, float(scale),
             query.stride(0), query.stride(1), out.stride(0), out.stride(1), ws_ptr, need, code,
             stream)
    if fp8_scales is None:
        _lib.call("npd_paged_prefill_attention", *ptrs, *sizes)
    else:
        _lib.call("npd_paged_prefill_attention_fp8", *ptrs, fp8_scales[0].data_ptr(),
                  fp8_scales[1].data_ptr(), *sizes)


def paged_prefill_attention(out: torch.Tensor, query: torch.Tensor, key_cache: torch.Tensor,
                            value_cache: torch.Tensor, block_tables: torch.Tensor,
                            cu_seqlens_q: torch.Tensor, context_lens: torch.Tensor, scale: float,
                            block_size: int, max_num_blocks_per_seq: int, max_q_len: int,
                            max_context_len: int | None = None,
                            workspace: torch.Tensor | None = None) -> None:
    """Causal varlen attention over the paged prefix plus the new chunk.

    Replaces the SDPA prefill of paged_forward (nanoPD/engine/model_runner.py:
    152-168), which attends within the chunk only. query/out: [total_q,
    num_heads, head_dim]; sequence s owns rows cu_seqlens_q[s]:cu_seqlens_q[s+1];
    its chunk K/V must already be in the pool; context_lens[s] = prefix + chunk.
    Row i of s sits at position context_lens[s] - q_len + i and sees keys 0..pos.
    max_q_len / max_context_len are host-side upper bounds (grid sizing; the
    context bound, default max_num_blocks_per_seq * block_size, sets how long
    key ranges are split). An optional uint8 ``workspace`` of at least
    :func:`prefill_workspace_bytes` bytes, zero-filled before its first use,
    replaces the cached per-stream one; calls sharing one run in stream order.
    """
    _prefill(out, query, key_cache, value_cache, block_tables, cu_seqlens_q, context_lens, scale,
             block_size, max_num_blocks_per_seq, max_q_len, max_context_len, workspace, None)


def paged_prefill_attention_fp8(out: torch.Tensor, query: torch.Tensor, key_cache: torch.Tensor,
                                value_cache: torch.Tensor, block_tables: torch.Tensor,
                                cu_seqlens_q: torch.Tensor, context_lens: torch.Tensor,
                                scale: float, block_size: int, max_num_blocks_per_seq: int,
                                max_q_len: int, k_scale: torch.Tensor, v_scale: torch.Tensor,
                                max_context_len: int | None = None,
                                workspace: torch.Tensor | None = None) -> None:
    """:func:`paged_prefill_attention` over an FP8 pool written by
    :func:`paged_kv_store_slots_fp8` (no reference counterpart): K =
    e4m3(byte) * k_scale[kv head], V likewise, converted exactly to the
    query's type before the MFMAs. query/out fp16 or bf16; head_dim a
    multiple of 32 from 32 to 256."""
    _prefill(out, query, key_cache, value_cache, block_tables, cu_seqlens_q, context_lens, scale,
             block_size, max_num_blocks_per_seq, max_q_len, max_context_len, workspace,
             (k_scale, v_scale))


# ---------------------------------------------------------------------------
# Block copy and metadata
# ---------------------------------------------------------------------------

def copy_blocks(k_cache: torch.Tensor, v_cache: torch.Tensor, block_pairs) -> None:
    """Copy whole blocks src -> dst in both caches (copy-on-write fork).

    block_pairs: int32 [N, 2] device tensor of (src, dst), or a sequence of
    pairs (uploaded with one copy). Completes the CoW contract of
    BlockSpaceManager.append_slot (nanoPD/block_manager/block_manager.py:91-96).
    FP8 pools (torch.float8_e4m3fn / uint8) are copied as the same bytes.
    """
    if k_cache.dtype in FP8_DTYPES and v_cache.dtype == k_cache.dtype:
        # a block copy moves bytes: a 1-byte pool is passed as 2-byte
        # elements, half as many per row (head_dim is even)
        _check(k_cache.is_contiguous() and v_cache.is_contiguous() and k_cache.size(-1) % 2 == 0,
               "fp8 caches must be contiguous with an even head_dim")
        k_cache = k_cache.view(torch.uint8).view(torch.bfloat16)
        v_cache = v_cache.view(torch.uint8).view(torch.bfloat16)
    _cache_checks(k_cache, v_cache)
    dev = k_cache.device
    _check(k_cache.is_cuda, "caches must be on CUDA")
    if not isinstance(block_pairs, torch.Tensor):
        block_pairs = torch.tensor(list(block_pairs), dtype=torch.int32).reshape(-1, 2).to(dev)
    _int32(block_pairs, "block_pairs")
    _same_device(dev, block_pairs)
    _check(block_pairs.dim() == 2 and block_pairs.size(1) == 2 and block_pairs.is_contiguous(),
           "block_pairs must be a contiguous [N, 2] tensor")
    n = block_pairs.size(0)
    if n == 0:
        return
    code = _dtype_code(k_cache, "copy_blocks")
    per_block = k_cache[0].numel()
    _lib.call("npd_copy_blocks", k_cache.data_ptr(), v_cache.data_ptr(), block_pairs.data_ptr(), n,
              k_cache.size(0), per_block, code, _stream(dev))


def _block_list(block_table, dev: torch.device) -> torch.Tensor:
    if isinstance(block_table, torch.Tensor):
        _int32(block_table, "block_table")
        _check(block_table.dim() == 1 and block_table.is_contiguous(),
               "block_table must be a contiguous 1-D int32 tensor")
        _same_device(dev, block_table)
        return block_table
    return torch.tensor(list(block_table), dtype=torch.int32).to(dev)


def _pool_checks(k_cache: torch.Tensor, v_cache: torch.Tensor, what: str) -> None:
    _check(k_cache.is_cuda, f"{what}: caches must be on CUDA")
    _check(k_cache.dim() == 5 and v_cache.shape == k_cache.shape,
           f"{what}: caches must be [num_layers, num_blocks, num_kv_heads, block_size, head_dim]")
    _check(k_cache.dtype == v_cache.dtype, f"{what}: k_cache and v_cache dtypes differ")
    _check(k_cache.is_contiguous() and v_cache.is_contiguous(), f"{what}: caches must be contiguous")


def extract_kv(k_cache: torch.Tensor, v_cache: torch.Tensor, block_table,
               out_k: torch.Tensor | None = None, out_v: torch.Tensor | None = None):
    """Gathers the blocks of ``block_table`` from every layer of the pool into
    the transfer layout ``[num_layers, len(block_table), num_kv_heads,
    block_size, head_dim]``, one launch (reference: extract_kv_to_pinned,
    nanoPD/workers/kv_transfer.py:45-53, one copy per block). Caches are the
    multi-layer pool ``[num_layers, num_blocks, kvh, bs, D]``. Returns
    ``(wire_k, wire_v)``, allocated unless given; an id outside the pool gives
    a zero block."""
    _pool_checks(k_cache, v_cache, "extract_kv")
    dev = k_cache.device
    ids = _block_list(block_table, dev)
    L, nb = k_cache.shape[:2]
    shape = (L, ids.numel()) + tuple(k_cache.shape[2:])
    if out_k is None:
        out_k = torch.empty(shape, dtype=k_cache.dtype, device=dev)
    if out_v is None:
        out_v = torch.empty(shape, dtype=k_cache.dtype, device=dev)
    for o in (out_k, out_v):
        _check(tuple(o.shape) == shape and o.dtype == k_cache.dtype and o.is_contiguous(),
               f"extract_kv: wire buffers must be contiguous {list(shape)} of the cache dtype")
        _same_device(dev, o)
    block_bytes = k_cache[0, 0].numel() * k_cache.element_size()
    _lib.call("npd_kv_gather_blocks", k_cache.data_ptr(), v_cache.data_ptr(), L, nb, block_bytes,
              ids.data_ptr(), ids.numel(), out_k.data_ptr(), out_v.data_ptr(), _stream(dev))
    return out_k, out_v


def load_kv(k_cache: torch.Tensor, v_cache: torch.Tensor, block_table, wire_k: torch.Tensor,
            wire_v: torch.Tensor) -> None:
    """Scatters a transfer buffer (see :func:`extract_kv`) into the pool at
    ``block_table`` (reference: load_kv_from_pinned, kv_transfer.py:56-69).
    Ids outside the pool are skipped."""
    _pool_checks(k_cache, v_cache, "load_kv")
    dev = k_cache.device
    ids = _block_list(block_table, dev)
    L, nb = k_cache.shape[:2]
    shape = (L, ids.numel()) + tuple(k_cache.shape[2:])
    for w in (wire_k, wire_v):
        _check(tuple(w.shape) == shape and w.dtype == k_cache.dtype and w.is_contiguous(),
               f"load_kv: wire buffers must be contiguous {list(shape)} of the cache dtype")
        _same_device(dev, w)
    block_bytes = k_cache[0, 0].numel() * k_cache.element_size()
    _lib.call("npd_kv_scatter_blocks", k_cache.data_ptr(), v_cache.data_ptr(), L, nb, block_bytes,
              ids.data_ptr(), ids.numel(), wire_k.data_ptr(), wire_v.data_ptr(), _stream(dev))


def qk_norm_rope_store(q_out: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                       qkv: torch.Tensor, slot_mapping: torch.Tensor, positions: torch.Tensor,
                       inv_freq: torch.Tensor, q_norm_weight: torch.Tensor | None,
                       k_norm_weight: torch.Tensor | None, eps: float,
                       k_scale: torch.Tensor | None = None,
                       v_scale: torch.Tensor | None = None) -> None:
    """Qwen3 attention prologue in one launch (replaces q_norm / k_norm,
    rotary embedding, the K/V copies and paged_kv_store of
    nanoPD/engine/model_runner.py:97-115, :142-146, :189-192). With both norm
    weights None it is the Qwen2 / Llama prologue: RoPE of q and k as
    projected (the reference applies the norms only where the attention
    module has them, model_runner.py:101-104).

    qkv: [T, (H + 2 KV) * D] rows of the fused projection (q, k, v heads;
    token stride free, elements contiguous); q_out: [T, H, D], heads
    contiguous; slot_mapping / positions: int32 [T]; inv_freq: fp32 [D / 2];
    norm weights: [D] in the cache dtype. Writes normalised + rotated q to
    q_out, normalised + rotated k and raw v to the caches at slot_mapping
    (negative slots are not stored). D in {64, 128, 256}.
    With ``k_scale`` / ``v_scale`` (fp32 [num_kv_heads]) the caches are an FP8
    pool (torch.float8_e4m3fn or uint8): k and v are stored as the e4m3 bytes
    of value / scale, as :func:`paged_kv_store_slots_fp8` rounds them.
    """
    fp8 = k_scale is not None or v_scale is not None
    if fp8:
        _fp8_cache_checks(k_cache, v_cache, k_scale, v_scale)
    else:
        _cache_checks(k_cache, v_cache)
    dev = qkv.device
    _check(qkv.is_cuda, "qkv must be on CUDA")
    _check((q_norm_weight is None) == (k_norm_weight is None),
           "pass both norm weights (Qwen3) or neither (Qwen2 / Llama)")
    norms = [w for w in (q_norm_weight, k_norm_weight) if w is not None]
    _same_device(dev, q_out, k_cache, v_cache, slot_mapping, positions, inv_freq, *norms)
    _int32(slot_mapping, "slot_mapping")
    _int32(positions, "positions")
    num_blocks, kvh, bs, d = k_cache.shape
    _check(q_out.dim() == 3 and q_out.size(2) == d, "q_out must be [num_tokens, num_heads, head_dim]")
    t, h = q_out.size(0), q_out.size(1)
    _check(qkv.dim() == 2 and qkv.size(0) == t and qkv.size(1) == (h + 2 * kvh) * d,
           "qkv must be [num_tokens, (num_heads + 2 * num_kv_heads) * head_dim]")
    _check(qkv.stride(1) == 1, "qkv rows must be contiguous")
    _check(q_out.stride(2) == 1 and q_out.stride(1) == d, "q_out heads must be contiguous")
    for x in (q_out, qkv, *norms):
        _check(x.dtype == (qkv.dtype if fp8 else k_cache.dtype),
               "qkv / q_out / norm weights must have one dtype (the cache dtype of a 2-byte pool)")
    _check(all(w.numel() == d and w.is_contiguous() for w in norms),
           "norm weights must be contiguous [head_dim]")
    qw = q_norm_weight.data_ptr() if norms else None
    kw = k_norm_weight.data_ptr() if norms else None
    _check(inv_freq.dtype == torch.float32 and inv_freq.numel() == d // 2
           and inv_freq.is_contiguous(), "inv_freq must be contiguous float32 [head_dim / 2]")
    for x, nm in ((slot_mapping, "slot_mapping"), (positions, "positions")):
        _check(x.dim() == 1 and x.numel() >= t and x.is_contiguous(),
               f"{nm} must be a contiguous [num_tokens] tensor")
    code = _dtype_code(qkv if fp8 else k_cache, "qk_norm_rope_store")
    if t == 0:
        return
    if fp8:
        _same_device(dev, k_scale, v_scale)
        _lib.call("npd_qk_norm_rope_store_fp8", q_out.data_ptr(), k_cache.data_ptr(),
                  v_cache.data_ptr(), qkv.data_ptr(), slot_mapping.data_ptr(),
                  positions.data_ptr(), inv_freq.data_ptr(), qw, kw, k_scale.data_ptr(),
                  v_scale.data_ptr(), t, h, kvh, d,
                  num_blocks, bs, qkv.stride(0), q_out.stride(0), float(eps), code, _stream(dev))
        return
    _lib.call("npd_qk_norm_rope_store", q_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
              qkv.data_ptr(), slot_mapping.data_ptr(), positions.data_ptr(), inv_freq.data_ptr(),
              qw, kw, t, h, kvh, d, num_blocks, bs,
              qkv.stride(0), q_out.stride(0), float(eps), code, _stream(dev))


class BatchMetadata(NamedTuple):
    cu_seqlens_q: torch.Tensor   # int32 [S + 1]
    seq_lens: torch.Tensor       # int32 [S], context after the step
    block_tables: torch.Tensor   # int32 [S, max_blocks_per_seq], zero padded
    positions: torch.Tensor      # int32 [T]
    slot_mapping: torch.Tensor   # int32 [T]
    token_seq: torch.Tensor      # int32 [T]
    max_q_len: int
    max_seq_len: int
    max_blocks_per_seq: int


def pack_metadata(seqs: Sequence[tuple[int, int, Sequence[int]]], block_size: int,
                  device: torch.device | str, max_blocks_per_seq: int | None = None) -> BatchMetadata:
    """Pack a ragged batch on the GPU from one host upload.

    seqs: per sequence, in batch order, ``(q_len, ctx_before, block_table)``:
    a prefill chunk of q_len tokens on a prefix of ctx_before tokens, or a
    decode (q_len 1, ctx_before = its position). The outputs replace the
    per-layer tensors paged_forward builds (nanoPD/engine/model_runner.py:
    129-150, 177-187).
    """
    dev = torch.device(device)
    ns = len(seqs)
    tables = [list(t) for _, _, t in seqs]
    mb = max_blocks_per_seq if max_blocks_per_seq is not None else max([len(t) for t in tables] + [1])
    total_q = sum(int(q) for q, _, _ in seqs)
    flat = [b for t in tables for b in t]
    host = torch.empty(3 * ns + len(flat), dtype=torch.int32,
                       pin_memory=dev.type == "cuda")
    if ns:
        host[: 3 * ns] = torch.tensor([[int(q), int(c), len(t)] for (q, c, _), t in zip(seqs, tables)],
                                      dtype=torch.int32).reshape(-1)
    if flat:
        host[3 * ns:] = torch.tensor(flat, dtype=torch.int32)
    buf = host.to(dev, non_blocking=True)
    desc, flat_d = buf[: 3 * ns], buf[3 * ns:]
    out_i = torch.empty(ns + 1 + ns + ns * mb + 3 * total_q, dtype=torch.int32, device=dev)
    o = 0
    cu = out_i[o:o + ns + 1]; o += ns + 1
    sl = out_i[o:o + ns]; o += ns
    bt = out_i[o:o + ns * mb].view(ns, mb); o += ns * mb
    pos = out_i[o:o + total_q]; o += total_q
    slots = out_i[o:o + total_q]; o += total_q
    tseq = out_i[o:o + total_q]
    if dev.type != "cuda":
        _fail("pack_metadata needs a CUDA device")
    _lib.call("npd_pack_metadata", desc.data_ptr(), flat_d.data_ptr() if flat else 0, ns, total_q,
              len(flat), mb, int(block_size), cu.data_ptr(), sl.data_ptr(), bt.data_ptr(),
              pos.data_ptr(), slots.data_ptr(), tseq.data_ptr(), _stream(dev))
    max_q = max([int(q) for q, _, _ in seqs] + [0])
    max_sl = max([int(q) + int(c) for q, c, _ in seqs] + [0])
    return BatchMetadata(cu, sl, bt, pos, slots, tseq, max_q, max_sl, mb)
