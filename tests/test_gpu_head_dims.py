"""GPU parity at head dims other than 64, 128 and 256.

The reference accepts them: its store moves 8-byte pieces of any head_dim % 4
== 0 (PA/csrc/kvstore/paged_kv_store_ops.cu:25-26), its decode kernel any
multiple of 32 up to 1024 (PA/csrc/attention/paged_attention_kernel.cu:16-20,
:116-140), and its prefill is SDPA at any head size
(nanoPD/engine/model_runner.py:166-168). Here:

* the KV stores (per-token table and slot forms, FP8 pool) take any head dim
  that is a multiple of 4 (8 for the FP8 pool): bit-exact against the oracle;
* decode attention takes multiples of 8 from 32 to 256 (the generic kernel,
  lanes of a token row padded to a power of two): within max-abs 2e-3 (fp16)
  / 1e-2 (bf16) of the float64 oracle, split partitions and the merge
  included;
* chunked prefill takes multiples of 32 from 32 to 256 (the generic MFMA
  kernel at every head dim but 64 and 128): same tolerance, paged prefixes,
  ragged chunks, decode rows, rows before position 0, and the FP8 pool.
"""
import math

import numpy as np
import pytest
import torch

from nanopd_amd import paged_kernels as pk
from oracle import paged_oracle as O
from tests.helpers import ATOL, bits, f32, max_abs, oracle_decode
from tests.test_gpu_decode import make_inputs, run as run_decode
from tests.test_gpu_fp8 import _fp8_prefill_case, _prefill_run_and_check
from tests.test_gpu_prefill import check as check_prefill
from tests.test_gpu_prefill import make_case, run as run_prefill

pytestmark = pytest.mark.gpu


def _poisoned(shape, dtype, device):
    return torch.full(shape, -7.25, dtype=dtype, device=device)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [4, 12, 36, 96, 100, 160, 192, 320])
def test_store_any_head_dim(device, dtype, D):
    """Per-token tables (the reference's form) at head dims of 4 mod 8 (8-byte
    vectors) and other multiples of 8 (16-byte vectors, runtime lane count)."""
    kvh, T, start, bs = 3, 45, 5, 16
    g = torch.Generator().manual_seed(D)
    nb = (start + T + bs - 1) // bs
    total = nb + 3
    k_src = torch.randn(kvh, T, D, generator=g).to(dtype).to(device)
    v_src = torch.randn(kvh, T, D, generator=g).to(dtype).to(device)
    table = torch.randperm(total, generator=g)[:nb].to(torch.int32)
    tables = table.unsqueeze(0).expand(T, -1).contiguous().to(device)
    pos = torch.arange(start, start + T, dtype=torch.int32, device=device)
    pos[3] = -1   # skipped
    kc = _poisoned((total, kvh, bs, D), dtype, device)
    vc = _poisoned((total, kvh, bs, D), dtype, device)
    want_k, want_v = bits(kc), bits(vc)
    O.kv_store(want_k, want_v, bits(k_src), bits(v_src), tables.cpu().numpy(), pos.cpu().numpy())
    pk.paged_kv_store(kc, vc, k_src, v_src, tables, pos)
    torch.cuda.synchronize()
    assert np.array_equal(bits(kc), want_k) and np.array_equal(bits(vc), want_v)


@pytest.mark.parametrize("D", [20, 96, 160, 192])
def test_store_slots_any_head_dim(device, D):
    """Slot store from a strided token-major view of a fused projection."""
    dtype = torch.bfloat16
    T, kvh, bs, total = 50, 4, 16, 12
    g = torch.Generator().manual_seed(D + 1)
    proj = torch.randn(T, 3 * kvh * D, generator=g).to(dtype).to(device)
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


@pytest.mark.parametrize("D", [32, 96, 192])
def test_fp8_store_any_head_dim(device, D):
    dtype = torch.bfloat16
    kvh, bs, N, T = 2, 16, 20, 37
    g = torch.Generator().manual_seed(D + 2)
    kc = torch.full((N, kvh, bs, D), 0x5A, dtype=torch.uint8)
    vc = kc.clone()
    k = (torch.randn(T, kvh, D, generator=g) * 2).to(dtype)
    v = (torch.randn(T, kvh, D, generator=g) * 2).to(dtype)
    slots = torch.randperm(N * bs, generator=g)[:T].to(torch.int32)
    slots[3] = -1
    ks = (0.01 + 0.05 * torch.rand(kvh, generator=g)).float()
    vs = (0.01 + 0.05 * torch.rand(kvh, generator=g)).float()
    want_k, want_v = kc.numpy().copy(), vc.numpy().copy()
    O.kv_store_slots_fp8(want_k, want_v, f32(k), f32(v), slots.numpy(), ks.numpy(), vs.numpy())
    dk, dv = kc.to(device).view(torch.float8_e4m3fn), vc.to(device).view(torch.float8_e4m3fn)
    pk.paged_kv_store_slots_fp8(dk, dv, k.to(device), v.to(device), slots.to(device),
                                ks.to(device), vs.to(device))
    torch.cuda.synchronize()
    u8 = lambda t: t.view(torch.uint8).cpu().numpy()  # noqa: E731
    assert np.array_equal(u8(dk), want_k) and np.array_equal(u8(dv), want_v)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [32, 40, 96, 160, 192, 224])
@pytest.mark.parametrize("G,kvh,bs", [(1, 4, 16), (4, 2, 16), (6, 2, 8), (8, 1, 32)])
def test_decode_any_head_dim(device, dtype, D, G, kvh, bs):
    """Contexts from 1 token to several partitions (the merge kernel), a
    zero-length row, shuffled tables."""
    lens = [1, 37, 700, 3001, 0, 129]
    print(f"decode D={D} {dtype} G={G} kvh={kvh} bs={bs}", flush=True)
    q, kc, vc, bt, sl, scale, mb = make_inputs(len(lens), G * kvh, kvh, D, lens, bs, dtype,
                                               device, seed=D * 7 + G)
    out = run_decode(q, kc, vc, bt, sl, scale, mb, bs)
    assert torch.count_nonzero(out[4]) == 0   # seq_len 0 -> zeros
    want = oracle_decode(q, kc, vc, bt, sl, scale)
    assert np.isfinite(f32(out)).all()
    err = max_abs(out, want)
    assert err <= ATOL[dtype], f"max-abs {err}"


def test_decode_head_dim_96_group_of_16(device):
    """A group above 8 heads (served as two sub-groups) at head dim 96."""
    lens = [5, 1200, 4096]
    q, kc, vc, bt, sl, scale, mb = make_inputs(len(lens), 32, 2, 96, lens, 16, torch.bfloat16,
                                               device, seed=96)
    out = run_decode(q, kc, vc, bt, sl, scale, mb, 16)
    assert max_abs(out, oracle_decode(q, kc, vc, bt, sl, scale)) <= ATOL[torch.bfloat16]


@pytest.mark.parametrize("hd", [32, 96, 160, 192, 224])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("prefixes,chunks,G,kvh,bs", [
    ([0], [1], 4, 2, 16),
    ([0, 70, 300], [130, 45, 64], 4, 2, 16),
    ([1536, 0, 4000], [512, 200, 96], 1, 4, 8),
    ([0, 512, 2000, 99], [300, 128, 1, 1], 6, 1, 32),
])
def test_prefill_any_head_dim(device, hd, dtype, prefixes, chunks, G, kvh, bs):
    print(f"prefill D={hd} {dtype} prefixes={prefixes} chunks={chunks} G={G} kvh={kvh} bs={bs}",
          flush=True)
    args = make_case(device, prefixes, chunks, H=G * kvh, kvh=kvh, D=hd, bs=bs, dtype=dtype,
                     seed=hd + sum(chunks))
    q, kc, vc, bt, cu, ctx, mb, mq = args
    scale = 1 / math.sqrt(hd)
    check_prefill(run_prefill(*args, scale), q, kc, vc, bt, cu, ctx, scale)


@pytest.mark.parametrize("hd", [32, 96, 192])
def test_prefill_zero_rows_and_last_row_equals_decode(device, hd):
    """Rows before position 0 are zeros; the last row of a chunk equals a
    decode step over the same context."""
    args = make_case(device, [0], [40], D=hd, seed=hd + 3)
    q, kc, vc, bt, cu, ctx, mb, mq = args
    short = torch.tensor([25], dtype=torch.int32, device=device)
    out = run_prefill(q, kc, vc, bt, cu, short, mb, mq, 0.1)
    assert torch.count_nonzero(out[:15]) == 0
    check_prefill(out, q, kc, vc, bt, cu, short, 0.1)
    scale = 1 / math.sqrt(hd)
    args = make_case(device, [700], [300], D=hd, seed=hd + 11)
    q, kc, vc, bt, cu, ctx, mb, mq = args
    full = run_prefill(*args, scale)
    dec = torch.empty(1, 32, hd, dtype=q.dtype, device=device)
    pk.paged_attention_forward(dec, q[-1:].contiguous(), kc, vc, bt, ctx, scale, 16, mb)
    torch.cuda.synchronize()
    assert max_abs(full[-1:], f32(dec).astype(np.float64)) <= ATOL[torch.bfloat16]


@pytest.mark.parametrize("hd", [96, 192])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_fp8_pool_any_head_dim(device, hd, dtype):
    """Chunked prefill over an e4m3 pool at head dims 96 and 192, against the
    float64 oracle over the dequantised pool: empty and paged prefixes, ragged
    chunks, a decode row."""
    case = _fp8_prefill_case(device, [0, 100, 1500, 77], [64, 37, 200, 1], 8, 2, dtype,
                             seed=hd, D=hd)
    _prefill_run_and_check(device, *case, dtype)
