"""Concurrent host-thread callers on one GPU.

nanoPD's central scheduler calls the paged ops from two host threads at once
(nanoPD/router/central_scheduler.py:132-135, one thread per worker). Here two
threads, each on its own HIP stream (default priority), interleave slot
stores, decode attention and chunked prefill through the Python layer (which
keeps one workspace per (device, stream) behind a lock) and invalid calls
through the C-ABI. A barrier before every op makes the threads' calls
overlap. Checked:

* every output of the threaded run equals the same sequence of calls made by
  one thread on one stream, bit for bit (the prefill shapes stay below the
  key-split length, where the merge order -- and so the rounding -- would
  depend on which split finishes last);
* npd_last_error() is per thread: each thread reads back the message of its
  own failed call, never the other thread's, and a later successful call does
  not overwrite it.
"""
import ctypes
import threading

import numpy as np
import pytest
import torch

from nanopd_amd import _lib
from nanopd_amd import paged_kernels as pk
from tests.helpers import bits

pytestmark = pytest.mark.gpu

ROUNDS = 4


def _workload(device, seed, dtype):
    """One caller's state: a pool, a decode batch and a prefill batch, and per
    round a slot store of new tokens (the decode rows' next token)."""
    g = torch.Generator().manual_seed(seed)
    H, kvh, D, bs = 32, 8, 128, 16
    # decode: 12 sequences of up to 2000 tokens (before the rounds' tokens)
    mb = (2000 + ROUNDS + bs - 1) // bs
    pmb = (1000 + bs - 1) // bs
    nblocks = 12 * mb + 3 * pmb + 8
    kc = (torch.randn(nblocks, kvh, bs, D, generator=g) * 0.5).to(dtype)
    vc = (torch.randn(nblocks, kvh, bs, D, generator=g) * 0.5).to(dtype)
    order = torch.randperm(nblocks, generator=g)
    dl = torch.randint(100, 2000, (12,), generator=g)
    bt = torch.zeros(12, mb, dtype=torch.int32)
    for i in range(12):
        bt[i] = order[i * mb:(i + 1) * mb]
    # prefill: 3 chunks on prefixes whose key ranges stay within 1024 keys
    pre, chunk = [0, 300, 700], [200, 256, 300]
    pbt = torch.stack([order[12 * mb + i * pmb:12 * mb + (i + 1) * pmb] for i in range(3)]).int()
    pq = (torch.randn(sum(chunk), H, D, generator=g) * 0.5).to(dtype)
    cu = torch.tensor([0, 200, 456, 756], dtype=torch.int32)
    ctx = torch.tensor([p + c for p, c in zip(pre, chunk)], dtype=torch.int32)
    rounds = []
    for r in range(ROUNDS):
        pos = dl + r   # the new token's position
        slots = (bt[torch.arange(12), pos // bs] * bs + pos % bs).int()
        rounds.append(dict(
            k=(torch.randn(12, kvh, D, generator=g) * 0.5).to(dtype),
            v=(torch.randn(12, kvh, D, generator=g) * 0.5).to(dtype),
            q=(torch.randn(12, H, D, generator=g) * 0.5).to(dtype),
            slots=slots, lens=(pos + 1).int()))
    to = lambda t: t.to(device)  # noqa: E731
    return dict(kc=to(kc), vc=to(vc), bt=to(bt), mb=mb, pbt=to(pbt), pmb=pmb, pq=to(pq),
                cu=to(cu), ctx=to(ctx), max_q=max(chunk),
                rounds=[{k: to(v) for k, v in rd.items()} for rd in rounds])


def _fresh(w):
    return dict(w, kc=w["kc"].clone(), vc=w["vc"].clone())


def _round(w, r, outs):
    rd = w["rounds"][r]
    scale = 128 ** -0.5
    pk.paged_kv_store_slots(w["kc"], w["vc"], rd["k"], rd["v"], rd["slots"])
    yield
    out = torch.full_like(rd["q"], float("nan"))
    pk.paged_attention_forward(out, rd["q"], w["kc"], w["vc"], w["bt"], rd["lens"], scale, 16,
                               w["mb"])
    outs.append(out)
    yield
    pout = torch.full_like(w["pq"], float("nan"))
    pk.paged_prefill_attention(pout, w["pq"], w["kc"], w["vc"], w["pbt"], w["cu"], w["ctx"],
                               scale, 16, w["pmb"], w["max_q"])
    outs.append(pout)
    yield


def _serial(w, device):
    outs = []
    stream = torch.cuda.Stream(device)
    with torch.cuda.stream(stream):
        for r in range(ROUNDS):
            for _ in _round(w, r, outs):
                pass
    stream.synchronize()
    return [bits(o) for o in outs] + [bits(w["kc"]), bits(w["vc"])]


def _bad_call(kind):
    """An invalid C-ABI call whose message names the thread's own mistake."""
    fake = 0x1000
    lib = _lib.load()
    if kind == "dtype":   # dtype code 7
        return lib.npd_paged_kv_store_slots(fake, fake, fake, fake, fake, 4, 8, 128, 64, 16, 1024,
                                            128, 7, None)
    # num_heads 12 over 5 kv heads
    return lib.npd_paged_attention(fake, fake, fake, fake, fake, fake, 2, 12, 5, 128, 64, 16, 4,
                                   ctypes.c_float(0.1), 1536, 128, 1536, 128, None, 0, 1, None)


def test_two_threads_match_serial_and_keep_their_own_errors(device):
    dtype = torch.bfloat16
    wa, wb = _workload(device, 1, dtype), _workload(device, 2, dtype)
    want = [_serial(_fresh(wa), device), _serial(_fresh(wb), device)]
    print("serial runs done", flush=True)

    barrier = threading.Barrier(2, timeout=60)
    results, errors = [None, None], [None, None]
    own = {0: ("dtype", b"unsupported dtype code 7"), 1: ("heads", b"not a multiple")}

    def worker(i, w):
        try:
            outs = []
            stream = torch.cuda.Stream(device)
            with torch.cuda.stream(stream):
                for r in range(ROUNDS):
                    for _ in _round(w, r, outs):
                        barrier.wait()   # both threads' next calls overlap
            stream.synchronize()
            got = [bits(o) for o in outs] + [bits(w["kc"]), bits(w["vc"])]
            # thread-local error messages
            kind, msg = own[i]
            barrier.wait()
            rc = _bad_call(kind)
            barrier.wait()   # both have failed before either reads back
            lib = _lib.load()
            mine = lib.npd_last_error()
            other = own[1 - i][1]
            # a successful call afterwards leaves the last failure in place
            pk.paged_kv_store_slots(w["kc"], w["vc"], w["rounds"][0]["k"], w["rounds"][0]["v"],
                                    w["rounds"][0]["slots"])
            stream.synchronize()
            after = lib.npd_last_error()
            results[i] = (got, rc, mine, other, msg, after)
        except BaseException as e:  # noqa: BLE001 -- reported by the main thread
            errors[i] = e
            barrier.abort()

    threads = [threading.Thread(target=worker, args=(i, w)) for i, w in
               enumerate((_fresh(wa), _fresh(wb)))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=300)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    for e in errors:
        if e is not None:
            raise e
    for i in range(2):
        got, rc, mine, other, msg, after = results[i]
        assert len(got) == len(want[i])
        for n, (x, y) in enumerate(zip(got, want[i])):
            assert np.array_equal(x, y), f"thread {i}: output {n} differs from the serial run"
        assert rc < 0
        assert msg in mine and other not in mine, (i, mine)
        assert after == mine, (i, after)
