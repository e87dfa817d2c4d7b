"""Block-list pack / unpack of the multi-layer KV pool (the single-GPU half of
KV transfer, reference nanoPD/workers/kv_transfer.py:45-69) on the GPU,
through the C-ABI: bit-exact against the oracle and the reference's per-block
copy loop, a round trip into a second pool at another block list, and
attention over the moved blocks equal to attention over the originals."""
import numpy as np
import pytest
import torch

from nanopd_amd import paged_kernels as pk
from oracle import paged_oracle as O
from oracle import torch_ref as R

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _pool(device, L, N, kvh=8, bs=16, D=128, dtype=torch.bfloat16, seed=0):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    k = torch.randn((L, N, kvh, bs, D), generator=g, device=device).to(dtype)
    v = torch.randn((L, N, kvh, bs, D), generator=g, device=device).to(dtype)
    return k, v


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("L,N,n,kvh,bs", [(1, 8, 1, 2, 16), (3, 40, 17, 2, 8), (36, 300, 64, 8, 16)])
def test_extract_matches_oracle_and_reference_loop(device, dtype, L, N, n, kvh, bs):
    k, v = _pool(device, L, N, kvh=kvh, bs=bs, dtype=dtype, seed=n)
    ids = torch.randperm(N, generator=torch.Generator().manual_seed(n))[:n].tolist()
    wk, wv = pk.extract_kv(k, v, ids)
    torch.cuda.synchronize()
    ok, ov = O.extract_kv(_bits(k), _bits(v), ids)
    assert np.array_equal(_bits(wk), ok) and np.array_equal(_bits(wv), ov)
    rk, rv = R.ref_extract_kv(k.cpu(), v.cpu(), ids)
    assert torch.equal(wk.cpu(), rk) and torch.equal(wv.cpu(), rv)


def test_out_of_pool_ids(device):
    k, v = _pool(device, 2, 10)
    wk, wv = pk.extract_kv(k, v, [3, -1, 10, 9])
    torch.cuda.synchronize()
    assert torch.equal(wk[:, 0], k[:, 3]) and torch.equal(wv[:, 3], v[:, 9])
    assert not wk[:, 1:3].any() and not wv[:, 1:3].any()
    dk = torch.full_like(k, 7.0)
    dv = torch.full_like(v, 7.0)
    pk.load_kv(dk, dv, [0, 50, -3, 9], wk, wv)       # 50, -3: skipped
    torch.cuda.synchronize()
    assert torch.equal(dk[:, 0], k[:, 3]) and torch.equal(dv[:, 9], v[:, 9])
    assert (dk[:, 1:9] == 7).all() and (dv[:, 1:9] == 7).all()


def test_round_trip_and_attention_over_moved_blocks(device):
    """A sequence moves from pool A (table ta) to pool B (table tb): B's
    blocks equal A's bit for bit, every other block of B keeps its poison,
    and decode attention over B with tb equals attention over A with ta."""
    L, kvh, bs, D, H = 4, 8, 16, 128, 32
    ka, va = _pool(device, L, 200, seed=1)
    ctx = 1000
    nb = (ctx + bs - 1) // bs
    ta = torch.randperm(200, generator=torch.Generator().manual_seed(2))[:nb].tolist()
    tb = torch.randperm(150, generator=torch.Generator().manual_seed(3))[:nb].tolist()
    kb = torch.full((L, 150, kvh, bs, D), float("nan"), dtype=ka.dtype, device=device)
    vb = kb.clone()
    wk, wv = pk.extract_kv(ka, va, ta)
    pk.load_kv(kb, vb, tb, wk, wv)
    torch.cuda.synchronize()
    assert torch.equal(kb[:, tb], ka[:, ta]) and torch.equal(vb[:, tb], va[:, ta])
    rest = [b for b in range(150) if b not in set(tb)]
    assert torch.isnan(kb[:, rest].float()).all() and torch.isnan(vb[:, rest].float()).all()
    q = torch.randn((1, H, D), device=device).to(ka.dtype)
    sl = torch.tensor([ctx], dtype=torch.int32, device=device)
    for layer in range(L):
        oa, ob = torch.empty_like(q), torch.empty_like(q)
        pk.paged_attention_forward(oa, q, ka[layer], va[layer],
                                   torch.tensor([ta], dtype=torch.int32, device=device), sl,
                                   D ** -0.5, bs, nb)
        pk.paged_attention_forward(ob, q, kb[layer], vb[layer],
                                   torch.tensor([tb], dtype=torch.int32, device=device), sl,
                                   D ** -0.5, bs, nb)
        torch.cuda.synchronize()
        assert torch.equal(oa, ob)


def test_argument_checks(device):
    k, v = _pool(device, 2, 10)
    with pytest.raises(RuntimeError):
        pk.extract_kv(k[0], v[0], [1])                  # not a multi-layer pool
    with pytest.raises(RuntimeError):
        pk.load_kv(k, v, [1, 2], torch.empty_like(k[:, :1]), torch.empty_like(v[:, :1]))
    with pytest.raises(RuntimeError):
        pk.extract_kv(k, v, torch.tensor([1, 2], dtype=torch.int64, device=device))
