"""Decode-only engine steps replayed from HIP graphs.

A decode step of the collocated engine (nanoPD/engine/engine.py:42-113 with
every running sequence decoding one token) launches about 400 kernels: for
each of 36 layers the norms, GEMMs, the fused attention prologue and paged
decode attention. Their host-side launch cost is paid once per shape here:
each (batch bucket, block-table width bucket) is captured into a graph whose
inputs are static device buffers:

  staging (int32): token ids [B] | descriptors [B, 3] | block tables [B, W]
  -> pack_metadata kernel (inside the graph) -> positions, slots, tables, ...
  -> embedding, 36 layers, final norm, LM head, argmax -> tokens [B]

A step fills a pinned host copy of `staging`, uploads it with one blocking
copy and replays the graph; argmax writes the graph's token buffer directly,
so the graph holds kernel nodes only, no memcpy node. Rows past the real
batch are padding: position -1 and an all-zero table give slot -1 (nothing
is stored) and a context of 0 (decode attention writes zeros), and their
tokens are dropped. Every kernel argument
(batch size, table width, workspace pointers) is fixed per graph, so the
table width is bucketed (powers of two) and the decode workspace is
allocated, zeroed, before capture; the graph records no memset.
"""
from __future__ import annotations

import torch

from . import _lib
from . import paged_kernels as pk
from .qwen3 import PagedQwen3, StepBatch

BATCH_BUCKETS = (1, 2, 4, 8, 16)


class _Graph:
    def __init__(self, model: PagedQwen3, batch: int, width: int, pool=None, debug: bool = False):
        """debug: keep the captured graph (its nodes can be listed through
        CUDAGraph.raw_cuda_graph)."""
        dev = model.device
        cfg = model.cfg
        self.batch, self.width = batch, width
        n = batch + 3 * batch + batch * width
        self.host = torch.zeros(n, dtype=torch.int32, pin_memory=True)
        self.host_np = self.host.numpy()
        self.staging = torch.zeros(n, dtype=torch.int32, device=dev)
        out = torch.zeros(batch + 1 + batch + batch * width + 3 * batch, dtype=torch.int32,
                          device=dev)
        o = 0
        self.cu = out[o:o + batch + 1]; o += batch + 1
        self.seq_lens = out[o:o + batch]; o += batch
        self.tables = out[o:o + batch * width].view(batch, width); o += batch * width
        self.positions = out[o:o + batch]; o += batch
        self.slots = out[o:o + batch]; o += batch
        self.token_seq = out[o:o + batch]
        need = pk.attention_workspace_bytes(batch, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim,
                                            model.block_size, width)
        self.workspace = torch.zeros(max(need, 1), dtype=torch.uint8, device=dev)
        self.tokens = torch.zeros(batch, dtype=torch.int64, device=dev)
        self.model = model
        # the warm-up runs see padding rows only (no slot is written)
        self._fill([], [], [])
        self.staging.copy_(self.host)
        self.graph = torch.cuda.CUDAGraph(keep_graph=debug)
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(2):   # warm-up: GEMM heuristics, workspaces
                self._body()
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        with torch.cuda.graph(self.graph, pool=pool):
            self._body()
        torch.cuda.synchronize(dev)

    def _body(self) -> None:
        b, w = self.batch, self.width
        st = self.staging
        desc, flat = st[b:4 * b], st[4 * b:]
        dev = self.model.device
        _lib.call("npd_pack_metadata", desc.data_ptr(), flat.data_ptr(), b, b, b * w, w,
                  self.model.block_size, self.cu.data_ptr(), self.seq_lens.data_ptr(),
                  self.tables.data_ptr(), self.positions.data_ptr(), self.slots.data_ptr(),
                  self.token_seq.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
        meta = pk.BatchMetadata(self.cu, self.seq_lens, self.tables, self.positions, self.slots,
                                self.token_seq, 1, 0, w)
        batch = StepBatch(input_ids=st[:b].long(), meta=meta, num_prefill_seqs=0,
                          num_prefill_tokens=0, sample_rows=None, max_prefill_q=0,
                          decode_workspace=self.workspace)
        # argmax writes the token buffer itself: no device-to-device copy node
        # follows it in the graph (the argmax result of a separate tensor would
        # sit in the shared graph pool, over other graphs' bf16 intermediates)
        torch.argmax(self.model.forward(batch), dim=-1, out=self.tokens)

    def _fill(self, positions: list, tables: list, last_tokens: list) -> None:
        """Writes a step's staging image into the pinned host buffer: real rows
        first, padding rows (position -1, empty table) after them."""
        b, w = self.batch, self.width
        n = len(positions)
        h = self.host_np
        h[:] = 0
        h[:n] = last_tokens
        desc = h[b:4 * b].reshape(b, 3)
        desc[:, 0] = 1
        desc[:, 1] = -1
        desc[:, 2] = w
        desc[:n, 1] = positions
        flat = h[4 * b:].reshape(b, w)
        for i, t in enumerate(tables):
            flat[i, :len(t)] = t

    def run(self, positions: list, tables: list, last_tokens: list) -> list:
        """One decode step of len(positions) <= batch sequences."""
        n = len(positions)
        self._fill(positions, tables, last_tokens)
        # a blocking upload: the replay starts from a complete staging image
        self.staging.copy_(self.host)
        self.graph.replay()
        return self.tokens[:n].tolist()   # synchronises: `host` is free again


class DecodeGraphs:
    """Graphs of decode-only steps for batches up to max(BATCH_BUCKETS) and
    block tables up to max_width blocks, captured on first use."""

    def __init__(self, model: PagedQwen3, max_width: int, min_width: int = 16):
        self.model = model
        self.max_width = max_width
        self.min_width = min_width
        self._graphs: dict = {}
        # one memory pool for every graph's intermediates: graphs replay one
        # at a time, in stream order
        self.pool = torch.cuda.graph_pool_handle()

    def bucket(self, batch: int, width: int):
        """(batch bucket, width bucket), or None if the step does not fit:
        widths are powers of two from min_width, capped at max_width."""
        bb = next((x for x in BATCH_BUCKETS if x >= batch), None)
        if bb is None or width > self.max_width:
            return None
        wb = self.min_width
        while wb < width:
            wb *= 2
        return bb, min(wb, self.max_width)

    def capture(self, batch: int, width: int) -> _Graph:
        key = self.bucket(batch, width)
        if key is None:
            raise ValueError(f"decode step of {batch} sequences / {width} blocks has no graph")
        g = self._graphs.get(key)
        if g is None:
            g = _Graph(self.model, *key, pool=self.pool)
            self._graphs[key] = g
        return g

    def capture_all(self) -> int:
        """Captures every bucket up front (serving loops then never pay a
        capture); returns the number of graphs."""
        w = self.min_width
        widths = []
        while w < self.max_width:
            widths.append(w)
            w *= 2
        widths.append(self.max_width)
        for b in BATCH_BUCKETS:
            for w in widths:
                self.capture(b, w)
        return len(self._graphs)

    def decode(self, positions: list, tables: list, last_tokens: list):
        """Greedy tokens of one decode-only step, or None if it has no graph."""
        width = max(len(t) for t in tables)
        if self.bucket(len(positions), width) is None:
            return None
        return self.capture(len(positions), width).run(positions, tables, last_tokens)
