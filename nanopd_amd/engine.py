"""Collocated continuous batching on one GPU: the step loop that drives the
paged kernels, as nanoPD's Engine and Scheduler do
(nanoPD/engine/engine.py:42-113, nanoPD/engine/scheduler.py:31-112).

Scheduling rules kept from the reference:
- sequences are admitted in arrival order while fewer than max_batch_size
  run and the pool holds the whole prompt (scheduler.py:82-101,
  block_manager.py:58-67);
- at most one sequence prefills per step. Its chunk is min(chunk, budget -
  #running) tokens (scheduler.py:47, :70-101); the reference's chunk is
  budget - #running with budget 1024, and here it is also capped at `chunk`;
- every running sequence decodes one token per step, after
  BlockSpaceManager.append_slot makes room (engine.py:56-60);
- greedy sampling (top-1), and a sequence stops after max_new_tokens (no
  EOS).

Differences, on purpose:
- the step's metadata (cu_seqlens, slot_mapping, block tables, positions) is
  packed once per step on the GPU (pack_metadata), not rebuilt per layer;
- copy-on-write pairs from append_slot are copied on the GPU;
- with `graphs`, decode-only steps replay a captured HIP graph of the whole
  model step (nanopd_amd/graphs.py) instead of launching it kernel by kernel.
"""
from __future__ import annotations

import math
import random
import sys
import time
from dataclasses import dataclass, field
from typing import Optional

import torch

from . import paged_kernels as pk
from .block_manager import BlockSpaceManager
from .graphs import DecodeGraphs
from .qwen3 import PagedQwen3, StepBatch


@dataclass
class Request:
    rid: int
    prompt: list            # token ids
    max_new_tokens: int
    arrival: float = 0.0    # seconds after the run starts


@dataclass
class Sequence:
    req: Request
    num_computed: int = 0
    output: list = field(default_factory=list)
    admitted: float = -1.0
    first_token: float = -1.0
    finished: float = -1.0

    @property
    def prompt_len(self) -> int:
        return len(self.req.prompt)

    @property
    def done(self) -> bool:
        return len(self.output) >= self.req.max_new_tokens


@dataclass
class StepPlan:
    prefill: Optional[Sequence]
    chunk: tuple            # (start, end) of the prefill chunk
    is_last: bool
    decodes: list


class Scheduler:
    """scheduler.py:20-112: waiting -> (prefilling) -> running -> finished."""

    def __init__(self, blocks: BlockSpaceManager, max_batch_size: int = 16, budget: int = 1024,
                 chunk: int = 512):
        self.blocks = blocks
        self.max_batch_size = max_batch_size
        self.budget = budget
        self.chunk = chunk
        self.waiting: list = []
        self.prefilling: list = []
        self.running: list = []
        self.finished: list = []

    def has_work(self) -> bool:
        return bool(self.waiting or self.prefilling or self.running)

    def schedule(self, now: float) -> StepPlan:
        still = []
        for s in self.running:
            if s.done:
                self.finished.append(s)
                self.blocks.free(s.req.rid)
            else:
                still.append(s)
        self.running = still
        decodes = list(self.running)
        room = min(self.budget - len(decodes), self.chunk)
        if room <= 0:
            return StepPlan(None, (0, 0), False, decodes)
        seq = None
        if self.prefilling:
            seq = self.prefilling[0]
        elif self.waiting:
            cand = self.waiting[0]
            if (len(self.running) < self.max_batch_size
                    and self.blocks.can_allocate(cand.prompt_len)):
                seq = self.waiting.pop(0)
                self.blocks.allocate(seq.req.rid, seq.prompt_len)
                seq.admitted = now
                self.prefilling.append(seq)
        if seq is None:
            return StepPlan(None, (0, 0), False, decodes)
        start = seq.num_computed
        end = min(start + room, seq.prompt_len)
        is_last = end >= seq.prompt_len
        if is_last:
            self.prefilling.pop(0)
        return StepPlan(seq, (start, end), is_last, decodes)


class Engine:
    def __init__(self, model: PagedQwen3, max_batch_size: int = 16, budget: int = 1024,
                 chunk: int = 512, clock=None, graphs: Optional[DecodeGraphs] = None):
        self.model = model
        self.graphs = graphs
        self.blocks = BlockSpaceManager(model.block_size, model.num_blocks)
        self.sched = Scheduler(self.blocks, max_batch_size, budget, chunk)
        self.device = model.device
        self.clock = clock or (lambda: 0.0)   # time stamps of first / last tokens
        self.steps = 0

    def add(self, req: Request) -> Sequence:
        seq = Sequence(req)
        self.sched.waiting.append(seq)
        return seq

    def prepare(self, now: float = 0.0):
        """Schedules a step and packs its batch: (plan, StepBatch), or None when
        there is nothing to run."""
        plan = self.sched.schedule(now)
        if plan.prefill is None and not plan.decodes:
            return None
        return plan, self._pack(*self._rows(plan))

    def _rows(self, plan: StepPlan):
        """The step's sequences (q_len, ctx_before, block table), token ids and
        sample rows; makes room for every decode token (append_slot) and runs
        the copy-on-write copies."""
        seqs, ids, sample_rows = [], [], []
        tp = 0
        if plan.prefill is not None:
            s = plan.prefill
            a, e = plan.chunk
            seqs.append((e - a, a, self.blocks.block_table(s.req.rid)))
            ids.extend(s.req.prompt[a:e])
            tp = e - a
            if plan.is_last:
                sample_rows.append(tp - 1)
        cow = []
        for i, s in enumerate(plan.decodes):
            pos = s.num_computed
            pair = self.blocks.append_slot(s.req.rid, pos)
            if pair is not None:
                cow.append(pair)
            seqs.append((1, pos, self.blocks.block_table(s.req.rid)))
            ids.append(s.output[-1])
            sample_rows.append(tp + i)
        self.model.copy_blocks(cow)
        return plan, seqs, ids, sample_rows, tp

    def _pack(self, plan: StepPlan, seqs: list, ids: list, sample_rows: list, tp: int) -> StepBatch:
        mb = max(len(t) for _, _, t in seqs)
        meta = pk.pack_metadata(seqs, self.model.block_size, self.device, max_blocks_per_seq=mb)
        batch = StepBatch(
            input_ids=torch.tensor(ids, dtype=torch.int64).to(self.device, non_blocking=True),
            meta=meta, num_prefill_seqs=1 if plan.prefill is not None else 0,
            num_prefill_tokens=tp,
            sample_rows=torch.tensor(sample_rows, dtype=torch.int64).to(self.device, non_blocking=True),
            max_prefill_q=tp)
        return batch

    def commit(self, plan: StepPlan, tokens: list, now: float = 0.0) -> None:
        """Applies a step's sampled tokens (one per sample row, in order).
        Raises if a token id is outside [0, vocab): argmax cannot produce one,
        so it means memory that held the step's tokens was overwritten."""
        vocab = self.model.cfg.vocab
        for x in tokens:
            if not 0 <= x < vocab:
                shapes = {"step": self.steps, "prefill": None if plan.prefill is None else
                          (plan.prefill.req.rid, plan.chunk, plan.is_last),
                          "decodes": [(s.req.rid, s.num_computed) for s in plan.decodes],
                          "tokens": tokens}
                raise RuntimeError(f"token id {x} (0x{x & 0xffffffffffffffff:016x}) outside "
                                   f"[0, {vocab}) in step {shapes}")
        k = 0
        t = self.clock() if tokens else now
        if plan.prefill is not None:
            s = plan.prefill
            s.num_computed = plan.chunk[1]
            if plan.is_last:
                s.output.append(tokens[k])
                s.first_token = t
                k += 1
                self.sched.running.append(s)
                if s.done:
                    s.finished = t
        for s in plan.decodes:
            s.output.append(tokens[k])
            s.num_computed += 1
            k += 1
            if s.done:
                s.finished = t
        self.steps += 1

    def step(self, now: float = 0.0) -> int:
        """One scheduled step, greedy sampling; returns the tokens sampled."""
        plan = self.sched.schedule(now)
        if plan.prefill is None and not plan.decodes:
            return 0
        rows = self._rows(plan)
        if self.graphs is not None and plan.prefill is None:
            _, seqs, ids, _, _ = rows
            tokens = self.graphs.decode([c for _, c, _ in seqs], [t for _, _, t in seqs], ids)
            if tokens is not None:
                self.commit(plan, tokens, now)
                return len(tokens)
        batch = self._pack(*rows)
        tokens = []
        if batch.sample_rows.numel():
            tokens = self.model.forward(batch).argmax(dim=-1).tolist()
        else:
            self.model.forward(batch)
        self.commit(plan, tokens, now)
        return len(tokens)

    def drain(self, now: float = 0.0) -> None:
        while self.sched.has_work():
            self.step(now)


def make_requests(n: int, seed: int = 5, rate: float = 8.0, prompt_median: int = 512,
                  prompt_clip=(32, 8192), out_median: int = 128, out_clip=(8, 1024),
                  sigma: float = 1.0, vocab: int = 151936) -> list:
    """Config-5 workload: lognormal prompt/output lengths (median, sigma,
    clipped), Poisson arrivals at `rate` per second from a seeded
    expovariate, random prompt token ids."""
    rng = random.Random(seed)
    reqs, t = [], 0.0
    for i in range(n):
        t += rng.expovariate(rate)
        p = int(min(max(round(rng.lognormvariate(math.log(prompt_median), sigma)), prompt_clip[0]),
                    prompt_clip[1]))
        o = int(min(max(round(rng.lognormvariate(math.log(out_median), sigma)), out_clip[0]),
                    out_clip[1]))
        reqs.append(Request(i, [rng.randrange(vocab) for _ in range(p)], o, t))
    return reqs


def serve(engine: Engine, requests: list, time_scale: float = 1.0,
          progress_every: int = 0) -> dict:
    """Runs requests arriving at their `arrival` times (wall clock, scaled by
    time_scale) through the engine until all finish. Reports output tokens per
    second over (last finish - first arrival), and the reference's formula
    (output tokens / arrival window, benchmark_poisson.py:93-99).
    progress_every > 0: a line on stderr each time that many more requests
    have finished."""
    pending = sorted(requests, key=lambda r: r.arrival)
    seqs = []
    t0 = time.perf_counter()
    engine.clock = lambda: time.perf_counter() - t0
    i = 0
    reported = 0
    while i < len(pending) or engine.sched.has_work():
        now = time.perf_counter() - t0
        while i < len(pending) and pending[i].arrival * time_scale <= now:
            seqs.append(engine.add(pending[i]))
            i += 1
        if not engine.sched.has_work():
            time.sleep(max(0.0, pending[i].arrival * time_scale - now))
            continue
        engine.step(now)
        if progress_every > 0:
            done = sum(1 for s in seqs if s.finished >= 0)
            if done >= reported + progress_every:
                reported = done - done % progress_every
                print(f"serve: {done}/{len(pending)} requests finished, {engine.steps} steps, "
                      f"{now:.1f} s", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t_end = time.perf_counter() - t0
    for s in seqs:
        if s.finished < 0:
            s.finished = t_end
    out_tokens = sum(len(s.output) for s in seqs)
    first = min(r.arrival for r in requests) * time_scale
    last_finish = max(s.finished for s in seqs)
    window = max(r.arrival for r in requests) * time_scale - first
    lat = sorted(s.finished - s.req.arrival * time_scale for s in seqs)
    return {
        "requests": len(seqs),
        "output_tokens": out_tokens,
        "prompt_tokens": sum(s.prompt_len for s in seqs),
        "tok_per_s": out_tokens / max(last_finish - first, 1e-9),
        "tok_per_s_arrival_window": out_tokens / max(window, 1e-9),
        "wall_s": t_end,
        "steps": engine.steps,
        "p50_e2e_s": lat[len(lat) // 2],
        "p99_e2e_s": lat[min(len(lat) - 1, int(len(lat) * 0.99))],
    }
