"""GPU parity of the KV store, slot store and block copy: bit-exact against the
oracle (PA/tests/test_paged_kernels.py:296-323 asserts atol=rtol=0).
Every call goes through the C-ABI library (nanopd_amd.paged_kernels)."""
import numpy as np
import pytest
import torch

from nanopd_amd import paged_kernels as pk
from nanopd_amd import workloads
from oracle import paged_oracle as O
from tests.helpers import bits, sha

pytestmark = pytest.mark.gpu

POISON = 0x7E01  # NaN bit pattern: rows the op must not touch keep it


def _poisoned(shape, dtype, device):
    return torch.full(shape, POISON, dtype=torch.int16, device=device).view(dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("kvh,T,start,bs,D", [(4, 16, 0, 16, 128), (2, 8, 8, 16, 128),
                                              (2, 1, 0, 16, 128), (2, 32, 0, 16, 128),
                                              (2, 64, 0, 16, 128), (8, 16, 0, 16, 128),
                                              (3, 40, 5, 32, 64), (2, 33, 7, 4, 256)])
def test_store_reference_cases(device, dtype, kvh, T, start, bs, D):
    """Cases of PA/tests/test_paged_kernels.py:263-355, per-token table form."""
    g = torch.Generator(device="cpu").manual_seed(T * 31 + start)
    nb = (start + T + bs - 1) // bs
    total = nb + 3
    k_src = torch.randn(kvh, T, D, generator=g).to(dtype).to(device)
    v_src = torch.randn(kvh, T, D, generator=g).to(dtype).to(device)
    table = torch.randperm(total, generator=g)[:nb].to(torch.int32)
    tables = table.unsqueeze(0).expand(T, -1).contiguous().to(device)
    pos = torch.arange(start, start + T, dtype=torch.int32, device=device)
    kc = _poisoned((total, kvh, bs, D), dtype, device)
    vc = _poisoned((total, kvh, bs, D), dtype, device)
    want_k, want_v = bits(kc), bits(vc)
    O.kv_store(want_k, want_v, bits(k_src), bits(v_src), tables.cpu().numpy(), pos.cpu().numpy())
    pk.paged_kv_store(kc, vc, k_src, v_src, tables, pos)
    torch.cuda.synchronize()
    assert np.array_equal(bits(kc), want_k)
    assert np.array_equal(bits(vc), want_v)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_store_start_position_form(device, dtype):
    """The older (k_src[1,kvh,T,D], 1-D table, start_pos) form of
    PA/tests/test_paged_kernels.py:302-323."""
    kvh, T, D, bs, start = 2, 8, 128, 16, 8
    k_src = torch.randn(1, kvh, T, D, device=device).to(dtype)
    v_src = torch.randn(1, kvh, T, D, device=device).to(dtype)
    table = torch.arange(1, dtype=torch.int32, device=device)
    kc = torch.zeros(1, kvh, bs, D, dtype=dtype, device=device)
    vc = torch.zeros_like(kc)
    pk.paged_kv_store(kc, vc, k_src, v_src, table, start)
    torch.cuda.synchronize()
    for tok in range(T):
        assert torch.equal(kc[0, :, start + tok], k_src[0, :, tok])
        assert torch.equal(vc[0, :, start + tok], v_src[0, :, tok])
    assert torch.count_nonzero(kc[0, :, :start]) == 0


def test_store_config1_all_context(device):
    w = workloads.config1(device)
    want_k, want_v = bits(w.k_cache), bits(w.v_cache)
    O.kv_store(want_k, want_v, bits(w.store_k), bits(w.store_v), w.store_tables.cpu().numpy(),
               w.store_positions.cpu().numpy())
    pk.paged_kv_store(w.k_cache, w.v_cache, w.store_k, w.store_v, w.store_tables, w.store_positions)
    torch.cuda.synchronize()
    got_k, got_v = bits(w.k_cache), bits(w.v_cache)
    assert np.array_equal(got_k, want_k) and np.array_equal(got_v, want_v)
    gold = np.load("tests/golden/cfg1.npz")
    assert sha(got_k, got_v) == str(gold["pool_sha"])


def test_store_config2_one_token_per_seq(device):
    w = workloads.config2(device)
    want_k, want_v = bits(w.k_cache), bits(w.v_cache)
    O.kv_store(want_k, want_v, bits(w.store_k), bits(w.store_v), w.store_tables.cpu().numpy(),
               w.store_positions.cpu().numpy())
    pk.paged_kv_store(w.k_cache, w.v_cache, w.store_k, w.store_v, w.store_tables, w.store_positions)
    torch.cuda.synchronize()
    assert np.array_equal(bits(w.k_cache), want_k) and np.array_equal(bits(w.v_cache), want_v)


def test_store_skips_out_of_range(device):
    kvh, T, D, bs, total = 2, 4, 128, 16, 3
    k_src = torch.randn(kvh, T, D, device=device).half()
    v_src = torch.randn(kvh, T, D, device=device).half()
    tables = torch.tensor([[0], [99], [1], [2]], dtype=torch.int32, device=device)
    pos = torch.tensor([0, 1, -5, 16], dtype=torch.int32, device=device)   # 16 -> table col 1: off table
    kc = _poisoned((total, kvh, bs, D), torch.float16, device)
    vc = _poisoned((total, kvh, bs, D), torch.float16, device)
    want_k, want_v = bits(kc), bits(vc)
    O.kv_store(want_k, want_v, bits(k_src), bits(v_src), tables.cpu().numpy(), pos.cpu().numpy())
    pk.paged_kv_store(kc, vc, k_src, v_src, tables, pos)
    torch.cuda.synchronize()
    assert np.array_equal(bits(kc), want_k) and np.array_equal(bits(vc), want_v)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [64, 128, 256])
def test_store_slots_token_major_view(device, dtype, D):
    """Slot store straight from a [T, kvh*D] projection output (a strided view)."""
    T, kvh, bs, total = 50, 4, 16, 12
    g = torch.Generator(device="cpu").manual_seed(D)
    proj = torch.randn(T, 3 * kvh * D, generator=g).to(dtype).to(device)   # fused kv-like buffer
    k_src = proj[:, : kvh * D].view(T, kvh, D)
    v_src = proj[:, kvh * D: 2 * kvh * D].view(T, kvh, D)
    slots = torch.randperm(total * bs, generator=g)[:T].to(torch.int32)
    slots[7] = -1
    slots = slots.to(device)
    kc = _poisoned((total, kvh, bs, D), dtype, device)
    vc = _poisoned((total, kvh, bs, D), dtype, device)
    want_k, want_v = bits(kc), bits(vc)
    O.kv_store_slots(want_k, want_v, bits(k_src), bits(v_src), slots.cpu().numpy())
    pk.paged_kv_store_slots(kc, vc, k_src, v_src, slots)
    torch.cuda.synchronize()
    assert np.array_equal(bits(kc), want_k) and np.array_equal(bits(vc), want_v)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_copy_blocks(device, dtype):
    total, kvh, bs, D = 20, 8, 16, 128
    kc = torch.randn(total, kvh, bs, D, device=device).to(dtype)
    vc = torch.randn(total, kvh, bs, D, device=device).to(dtype)
    pairs = [(3, 7), (1, 2), (11, 19), (5, 25)]   # the last is out of the pool: skipped
    want_k, want_v = bits(kc), bits(vc)
    O.copy_blocks(want_k, want_v, pairs)
    pk.copy_blocks(kc, vc, pairs)
    torch.cuda.synchronize()
    assert np.array_equal(bits(kc), want_k) and np.array_equal(bits(vc), want_v)
