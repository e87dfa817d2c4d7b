"""Host logic of the caller side (CPU): block bookkeeping against the oracle's
restatement of nanoPD/block_manager/block_manager.py, the scheduler's
chunking / budget / admission rules (nanoPD/engine/scheduler.py:31-112), and
the config-5 workload generator."""
import math
import random

import pytest

from nanopd_amd.block_manager import BlockSpaceManager
from nanopd_amd.engine import Request, Scheduler, Sequence, make_requests
from oracle import paged_oracle as O


def test_block_manager_matches_oracle_on_random_ops():
    rng = random.Random(7)
    bs, nb = 16, 64
    mgr = BlockSpaceManager(bs, nb)
    alloc = O.BlockAllocator(nb)
    tables, lens, nxt = {}, {}, 0
    for _ in range(400):
        op = rng.random()
        if op < 0.25 or not tables:
            n = rng.randint(1, 70)
            if mgr.can_allocate(n) and len(alloc.free) >= (n + bs - 1) // bs:
                got = list(mgr.allocate(nxt, n))
                want = [alloc.allocate() for _ in range((n + bs - 1) // bs)]
                assert got == want
                tables[nxt], lens[nxt] = want, n
                nxt += 1
        elif op < 0.8:
            sid = rng.choice(list(tables))
            if not alloc.free:
                continue
            pos = lens[sid]
            got = mgr.append_slot(sid, pos)
            want = O.append_slot(alloc, tables[sid], pos, bs)
            assert got == want
            lens[sid] += 1
            assert mgr.block_table(sid) == tables[sid]
        elif op < 0.9:
            sid = rng.choice(list(tables))
            mgr.fork(sid, nxt)
            tables[nxt] = [alloc.fork(b) for b in tables[sid]]
            lens[nxt] = lens[sid]
            nxt += 1
        else:
            sid = rng.choice(list(tables))
            mgr.free(sid)
            for b in tables.pop(sid):
                alloc.release(b)
            lens.pop(sid)
        assert mgr.num_free_blocks == len(alloc.free)


def test_first_allocation_is_highest_block_and_cow_pair():
    mgr = BlockSpaceManager(4, 8)
    assert mgr.allocate(0, 5) == [7, 6]
    mgr.fork(0, 1)
    # position 5 lands in the shared last block -> private copy (old, new)
    assert mgr.append_slot(1, 5) == (6, 5)
    assert mgr.block_table(1) == [7, 5] and mgr.block_table(0) == [7, 6]
    # position 8 needs a third block, no copy
    assert mgr.append_slot(1, 8) is None and mgr.block_table(1) == [7, 5, 4]
    mgr.free(0)
    mgr.free(1)
    assert mgr.num_free_blocks == 8


def _seq(rid, n, out=4):
    return Sequence(Request(rid, list(range(n)), out))


def test_scheduler_chunks_a_long_prompt_one_sequence_at_a_time():
    sched = Scheduler(BlockSpaceManager(16, 1000), max_batch_size=16, budget=1024, chunk=512)
    a, b = _seq(0, 1300), _seq(1, 40)
    sched.waiting += [a, b]
    chunks = []
    for _ in range(3):
        p = sched.schedule(0.0)
        assert p.prefill is a and not p.decodes
        chunks.append((p.chunk, p.is_last))
        a.num_computed = p.chunk[1]
    assert chunks == [((0, 512), False), ((512, 1024), False), ((1024, 1300), True)]
    a.output.append(1)
    sched.running.append(a)
    p = sched.schedule(0.0)
    assert p.prefill is b and p.chunk == (0, 40) and p.is_last and p.decodes == [a]


def test_scheduler_budget_and_admission_caps():
    blocks = BlockSpaceManager(16, 1000)
    sched = Scheduler(blocks, max_batch_size=2, budget=600, chunk=512)
    run = [_seq(i, 10) for i in range(2)]
    for s in run:
        blocks.allocate(s.req.rid, 10)
        s.output.append(1)
    sched.running = list(run)
    sched.waiting.append(_seq(9, 100))
    p = sched.schedule(0.0)
    assert p.prefill is None and len(p.decodes) == 2        # batch full: no admission
    sched.max_batch_size = 3
    p = sched.schedule(0.0)
    assert p.prefill is not None and p.chunk == (0, 100)
    sched.budget = 100                                       # room = budget - #running
    sched.max_batch_size = 4
    s = _seq(10, 500)
    sched.waiting.append(s)
    sched.running.append(p.prefill)
    p.prefill.output.append(1)
    p2 = sched.schedule(0.0)
    assert p2.prefill is s and p2.chunk == (0, 97)
    small = Scheduler(BlockSpaceManager(16, 3), max_batch_size=4, budget=1024, chunk=512)
    small.waiting.append(_seq(0, 49))                        # needs 4 blocks of 3
    assert small.schedule(0.0).prefill is None


def test_finished_sequences_release_their_blocks():
    blocks = BlockSpaceManager(16, 20)
    sched = Scheduler(blocks, max_batch_size=4)
    s = _seq(0, 40, out=1)
    blocks.allocate(0, 40)
    s.output.append(5)
    sched.running.append(s)
    assert blocks.num_free_blocks == 17
    p = sched.schedule(1.0)
    assert p.decodes == [] and sched.finished == [s] and blocks.num_free_blocks == 20


def test_config5_workload_generator():
    reqs = make_requests(256, seed=5)
    assert reqs == make_requests(256, seed=5)
    assert all(32 <= len(r.prompt) <= 8192 and 8 <= r.max_new_tokens <= 1024 for r in reqs)
    gaps = [b.arrival - a.arrival for a, b in zip(reqs, reqs[1:])]
    assert all(g > 0 for g in gaps)
    assert abs(sum(gaps) / len(gaps) - 1 / 8.0) < 0.03       # Poisson at 8 req/s
    med = sorted(len(r.prompt) for r in reqs)[128]
    assert 350 < med < 750                                     # lognormal median 512
    assert abs(math.log(sorted(r.max_new_tokens for r in reqs)[128] / 128)) < 0.4
