"""Decode attention over seeded random shapes against the float64 oracle.

Each case draws its batch size, kv heads, group size (1-24 query heads per kv
head), head dim, block size, pool type and contexts from a fixed seed, so the
kernel forms meet shapes the hand-written cases do not pair up: the two-pass
VALU kernel, the one-pass matrix-core units (five to sixteen heads, units of
at most 16 for larger groups, the four-wave FP8 form past 256 units), the
generic kernel for other head dims and block sizes, the in-kernel work list
(up to 64 sequences) and the schedule kernel (more), single and split
partitions, two-level merges and empty contexts. Rows past a context hold NaN
(2-byte pools) or NaN codes (FP8 pools). Tolerance: the decode tests' max-abs
bar (2e-3 fp16, 1e-2 bf16). Reference oracle: PA/tests/test_paged_attention.py:33-71."""
import math

import numpy as np
import pytest
import torch

from nanopd_amd import paged_kernels as pk
from oracle import paged_oracle as O
from tests.helpers import ATOL, f32, max_abs

pytestmark = pytest.mark.gpu

NCASES = 48


def draw(seed):
    r = np.random.default_rng(seed)
    fp8 = bool(r.random() < 0.35)
    D = 128 if fp8 else int(r.choice([64, 128, 128, 128, 256, 96, 160]))
    if fp8 or D in (64, 256):
        bs = int(r.choice([16, 32]))
    else:
        bs = int(r.choice([8, 16, 16, 32, 64]))
    kvh = int(r.choice([1, 2, 4, 8]))
    G = int(r.choice([1, 2, 3, 4, 5, 6, 8, 9, 12, 16, 20, 24]))
    S = int(r.choice([1, 3, 7, 16, 40, 70]))
    if S * kvh * G > 2048:          # keep the float64 oracle within seconds
        S = max(1, 2048 // (kvh * G))
    lens = r.integers(0, 4500, S)
    lens[r.random(S) < 0.1] = 0
    if S > 1:
        lens[0] = int(r.integers(1, 40))
    dtype = torch.bfloat16 if r.random() < 0.6 else torch.float16
    return fp8, D, bs, kvh, G, [int(x) for x in lens], dtype


@pytest.mark.parametrize("case", range(NCASES))
def test_random_shape(device, case):
    fp8, D, bs, kvh, G, lens, dtype = draw(1000 + case)
    S, H = len(lens), G * kvh
    print(f"case {case}: fp8={fp8} D={D} bs={bs} kvh={kvh} G={G} S={S} {dtype} "
          f"max ctx {max(lens)}", flush=True)
    g = torch.Generator().manual_seed(case)
    nbs = [max(1, (n + bs - 1) // bs) for n in lens]
    mb, total = max(nbs), sum(nbs)
    order = torch.randperm(total, generator=g)
    bt = torch.zeros(S, mb, dtype=torch.int32)
    o = 0
    for i, n in enumerate(nbs):
        bt[i, :n] = order[o:o + n]
        o += n
    sl = torch.tensor(lens, dtype=torch.int32)
    q = torch.randn(S, H, D, generator=g).to(dtype)
    scale = 1 / math.sqrt(D)
    out = torch.full((S, H, D), float("nan"), dtype=dtype, device=device)
    if fp8:
        codes = torch.randint(0, 0x7E, (2, total, kvh, bs, D), generator=g, dtype=torch.int32)
        codes = codes | (torch.randint(0, 2, codes.shape, generator=g, dtype=torch.int32) << 7)
        kc, vc = codes[0].to(torch.uint8), codes[1].to(torch.uint8)
        for i, n in enumerate(lens):
            if n % bs:
                b = int(bt[i, (n - 1) // bs])
                kc[b, :, n % bs:, :] = 0x7F
                vc[b, :, n % bs:, :] = 0xFF
        ks = (0.5 + torch.rand(kvh, generator=g)) / 448
        vs = (0.5 + torch.rand(kvh, generator=g)) / 448
        pk.paged_attention_forward_fp8(out, q.to(device), kc.to(device).view(torch.float8_e4m3fn),
                                       vc.to(device).view(torch.float8_e4m3fn), bt.to(device),
                                       sl.to(device), scale, bs, mb, ks.to(device), vs.to(device))
        want = O.decode_attention(f32(q), O.fp8_pool_values(kc.numpy(), ks.numpy()),
                                  O.fp8_pool_values(vc.numpy(), vs.numpy()), bt.numpy(),
                                  sl.numpy(), scale)
    else:
        kc = torch.randn(total, kvh, bs, D, generator=g).to(dtype)
        vc = torch.randn(total, kvh, bs, D, generator=g).to(dtype)
        want = O.decode_attention(f32(q), f32(kc), f32(vc), bt.numpy(), sl.numpy(), scale)
        for i, n in enumerate(lens):
            if n % bs:
                b = int(bt[i, (n - 1) // bs])
                kc[b, :, n % bs:, :] = float("nan")
                vc[b, :, n % bs:, :] = float("nan")
        pk.paged_attention_forward(out, q.to(device), kc.to(device), vc.to(device), bt.to(device),
                                   sl.to(device), scale, bs, mb)
    torch.cuda.synchronize()
    assert np.isfinite(f32(out)).all()
    assert max_abs(out, want) <= ATOL[dtype]
