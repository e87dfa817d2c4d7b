"""Decode over sequences whose tables share blocks: copy-on-write forks,
forks that grew past the fork point, and identical tables.

Each sequence's items read their own table, so a block two tables hold is read
by both (at config 4 the second reads mostly come from L2: over the FP8 pool,
whose loads are not nontemporal, the fetch counters read the distinct bytes).
A form in which the first sequence of such a set served the others' query
heads in its idle MFMA columns was built, passed these tests and was dropped:
it read each row once but left fewer waves streaming (config 4 over the FP8
pool: 81.1 against 73.4 us in the trace, the same bytes fetched).

Checks, for the one-pass units (head dim 128: 2-byte groups of 5-8 heads,
every FP8 group) and the two-pass kernel (2-byte, 4 heads):
- every row against the float64 oracle, at the decode tests' tolerance;
- bit-equality with the same batch over unshared tables (every block of the
  forks copied to a block of its own);
- bit-equality when the sequences come in reverse order.

Reference: the fork and the copy-on-write of the last block,
nanoPD/block_manager/block_manager.py:100-105 and :72-98."""
import math

import numpy as np
import pytest
import torch

from nanopd_amd import paged_kernels as pk
from oracle import paged_oracle as O
from tests.helpers import ATOL, f32, max_abs

pytestmark = pytest.mark.gpu

D = 128
# parents' contexts: one block, part of a block, a few partitions, and a long
# one whose 512-token partitions (the kernel halves the host's 2048 for this
# few items) merge in two levels
PARENTS = [1, 100, 2065, 3000, 5000, 12000]
# (parent, kind, extra tokens): "cow" shares every block but a copied last
# one; "grow" also appends tokens past the fork; "same" is an identical table
FORKS = [(3, "cow", 0), (3, "cow", 0), (4, "same", 0), (4, "same", 0), (4, "same", 0),
         (4, "same", 0), (2, "grow", 300), (5, "cow", 0), (5, "grow", 2500), (1, "same", 0)]


def compact(kc, vc, bt):
    """The pool blocks the tables use, renumbered (the oracle's input)."""
    ids = np.unique(bt.numpy())
    remap = np.zeros(int(ids.max()) + 1, dtype=np.int32)
    remap[ids] = np.arange(len(ids), dtype=np.int32)
    return kc[torch.from_numpy(ids).long()], vc[torch.from_numpy(ids).long()], remap[bt.numpy()]


def build(bs, fp8, seed):
    """Pool contents, the shared tables, and the same batch over unshared
    tables (every fork block copied to a fresh one)."""
    g = torch.Generator().manual_seed(seed)
    nblk = lambda n: (n + bs - 1) // bs
    ctx = list(PARENTS)
    need = sum(nblk(n) for n in PARENTS)
    for p, kind, extra in FORKS:
        ctx.append(PARENTS[p] + extra)
        need += 1 + nblk(PARENTS[p] + extra) - nblk(PARENTS[p])
    # the unshared copy needs every fork block again
    total = need + sum(nblk(c) for c in ctx[len(PARENTS):]) + 8
    order = torch.randperm(total, generator=g).tolist()
    take = lambda n: [order.pop() for _ in range(n)]
    rows = [take(nblk(n)) for n in PARENTS]
    copies = []   # (src, dst) block copies: the copied-on-write blocks
    for p, kind, extra in FORKS:
        row = list(rows[p])
        if kind in ("cow", "grow"):
            new = take(1)[0]
            copies.append((row[-1], new))
            row[-1] = new
        if kind == "grow":
            row += take(nblk(PARENTS[p] + extra) - nblk(PARENTS[p]))
        rows.append(row)
    # unshared: each fork's blocks copied to blocks of its own
    urows = [list(r) for r in rows[:len(PARENTS)]]
    for r in rows[len(PARENTS):]:
        nr = take(len(r))
        copies += list(zip(r, nr))
        urows.append(nr)
    S, mb = len(rows), max(len(r) for r in rows)
    bt, ubt = torch.zeros(S, mb, dtype=torch.int32), torch.zeros(S, mb, dtype=torch.int32)
    for i, (r, u) in enumerate(zip(rows, urows)):
        bt[i, :len(r)] = torch.tensor(r)
        ubt[i, :len(u)] = torch.tensor(u)
    shape = (total, 8, bs, D)
    if fp8:
        codes = torch.randint(0, 0x7E, (2,) + shape, generator=g, dtype=torch.int32)
        codes = codes | (torch.randint(0, 2, codes.shape, generator=g, dtype=torch.int32) << 7)
        kc, vc = codes[0].to(torch.uint8), codes[1].to(torch.uint8)
    else:
        kc, vc = torch.randn(shape, generator=g), torch.randn(shape, generator=g)
    for src, dst in copies:   # the copies hold the source block's contents
        kc[dst] = kc[src]
        vc[dst] = vc[src]
    return kc, vc, bt, ubt, torch.tensor(ctx, dtype=torch.int32), mb


def run(device, q, kc, vc, bt, sl, mb, bs, fp8, ks=None, vs=None):
    out = torch.full_like(q, float("nan"))
    scale = 1 / math.sqrt(D)
    if fp8:
        pk.paged_attention_forward_fp8(out, q, kc.to(device).view(torch.float8_e4m3fn),
                                       vc.to(device).view(torch.float8_e4m3fn), bt.to(device),
                                       sl.to(device), scale, bs, mb, ks.to(device), vs.to(device))
    else:
        pk.paged_attention_forward(out, q, kc, vc, bt.to(device), sl.to(device), scale, bs, mb)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("H,dtype,bs", [(48, torch.bfloat16, 16), (64, torch.bfloat16, 32),
                                        (40, torch.float16, 16), (32, torch.bfloat16, 16)])
def test_shared_blocks_2byte(device, H, dtype, bs):
    """G 6 / 8 / 5 (one-pass units) and G 4 (the two-pass kernel), 8 kv heads."""
    print(f"shared blocks: H={H} G={H // 8} {dtype} bs={bs}", flush=True)
    kc, vc, bt, ubt, sl, mb = build(bs, False, seed=H + bs)
    kc, vc = kc.to(dtype).to(device), vc.to(dtype).to(device)
    g = torch.Generator().manual_seed(H)
    q = torch.randn(len(sl), H, D, generator=g).to(dtype).to(device)
    out = run(device, q, kc, vc, bt, sl, mb, bs, False)
    ck, cv, cbt = compact(kc.cpu(), vc.cpu(), bt)
    want = O.decode_attention(f32(q), f32(ck), f32(cv), cbt, sl.numpy(), 1 / math.sqrt(D))
    assert np.isfinite(f32(out)).all()
    assert max_abs(out, want) <= ATOL[dtype]
    uout = run(device, q, kc, vc, ubt, sl, mb, bs, False)
    assert torch.equal(out.view(torch.int16), uout.view(torch.int16))


@pytest.mark.parametrize("G,bs", [(1, 16), (4, 16), (4, 32), (8, 16), (16, 16)])
def test_shared_blocks_fp8(device, G, bs):
    """FP8 pools, G 1 / 4 / 8 / 16."""
    print(f"shared blocks fp8: G={G} bs={bs}", flush=True)
    kc, vc, bt, ubt, sl, mb = build(bs, True, seed=100 + G + bs)
    g = torch.Generator().manual_seed(G)
    H = 8 * G
    q = torch.randn(len(sl), H, D, generator=g).to(torch.bfloat16).to(device)
    ks = (0.5 + torch.rand(8, generator=g)) / 448
    vs = (0.5 + torch.rand(8, generator=g)) / 448
    out = run(device, q, kc, vc, bt, sl, mb, bs, True, ks, vs)
    ck, cv, cbt = compact(kc, vc, bt)
    want = O.decode_attention(f32(q), O.fp8_pool_values(ck.numpy(), ks.numpy()),
                              O.fp8_pool_values(cv.numpy(), vs.numpy()), cbt, sl.numpy(),
                              1 / math.sqrt(D))
    assert np.isfinite(f32(out)).all()
    assert max_abs(out, want) <= ATOL[torch.bfloat16]
    uout = run(device, q, kc, vc, ubt, sl, mb, bs, True, ks, vs)
    assert torch.equal(out.view(torch.int16), uout.view(torch.int16))


def test_leader_order_does_not_matter(device):
    """The same batch with its sequences in reverse order: every row bit-equal
    (FP8, G 4, and bf16, G 8)."""
    for fp8, H in ((True, 32), (False, 64)):
        kc, vc, bt, _, sl, mb = build(16, fp8, seed=7)
        g = torch.Generator().manual_seed(3)
        q = torch.randn(len(sl), H, D, generator=g).to(torch.bfloat16).to(device)
        ks = (0.5 + torch.rand(8, generator=g)) / 448
        vs = (0.5 + torch.rand(8, generator=g)) / 448
        if not fp8:
            kc, vc = kc.to(torch.bfloat16).to(device), vc.to(torch.bfloat16).to(device)
        out = run(device, q, kc, vc, bt, sl, mb, 16, fp8, ks, vs)
        rev = torch.arange(len(sl) - 1, -1, -1)
        rout = run(device, q[rev.to(device)].contiguous(), kc, vc, bt[rev].contiguous(),
                   sl[rev].contiguous(), mb, 16, fp8, ks, vs)
        assert torch.equal(out.view(torch.int16), rout[rev.to(device)].view(torch.int16))
