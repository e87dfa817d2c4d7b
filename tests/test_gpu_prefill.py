"""GPU parity of chunked-prefill attention (MFMA kernel) against the float64
oracle: causal attention over the paged prefix plus the chunk.

For an empty prefix this is the reference's own computation
(nanoPD/engine/model_runner.py:152-168, SDPA over the chunk with a causal
block-diagonal mask); for a non-empty prefix the reference ignores the prefix,
so the oracle is the mathematical definition (prefill_attention in
oracle/paged_oracle.py, pinned in tests/test_oracle.py). Tolerance: max-abs
2e-3 (fp16) / 1e-2 (bf16)."""
import math

import numpy as np
import pytest
import torch

from nanopd_amd import paged_kernels as pk
from nanopd_amd import workloads
from oracle import paged_oracle as O
from tests.helpers import ATOL, f32, max_abs

pytestmark = pytest.mark.gpu


def make_case(device, prefixes, chunks, H=32, kvh=8, D=128, bs=16, dtype=torch.bfloat16, seed=0,
              shuffle=True):
    """Pool with random values, tables of prefix + chunk blocks, queries of the
    chunks packed varlen; the chunk K/V already stored in the pool."""
    g = torch.Generator().manual_seed(seed)
    ctx = [p + c for p, c in zip(prefixes, chunks)]
    nbs = [(n + bs - 1) // bs for n in ctx]
    total = sum(nbs) + 3
    kc = (torch.randn(total, kvh, bs, D, generator=g) * 0.5).to(dtype)
    vc = (torch.randn(total, kvh, bs, D, generator=g) * 0.5).to(dtype)
    order = torch.randperm(total, generator=g) if shuffle else torch.arange(total)
    mb = max(nbs)
    bt = torch.zeros(len(ctx), mb, dtype=torch.int32)
    o = 0
    for s, n in enumerate(nbs):
        bt[s, :n] = order[o:o + n]
        o += n
    T = sum(chunks)
    q = (torch.randn(T, H, D, generator=g) * 0.5).to(dtype)
    cu = torch.tensor([0] + list(np.cumsum(chunks)), dtype=torch.int32)
    return (q.to(device), kc.to(device), vc.to(device), bt.to(device), cu.to(device),
            torch.tensor(ctx, dtype=torch.int32, device=device), mb, max(chunks))


def run(q, kc, vc, bt, cu, ctx, mb, max_q, scale):
    out = torch.full_like(q, float("nan"))
    pk.paged_prefill_attention(out, q, kc, vc, bt, cu, ctx, scale, kc.size(2), mb, max_q)
    torch.cuda.synchronize()
    return out


def oracle(q, kc, vc, bt, cu, ctx, scale):
    return O.prefill_attention(f32(q), f32(kc), f32(vc), bt.cpu().numpy(), cu.cpu().numpy(),
                               ctx.cpu().numpy(), scale)


def check(out, q, kc, vc, bt, cu, ctx, scale):
    want = oracle(q, kc, vc, bt, cu, ctx, scale)
    assert np.isfinite(f32(out)).all()
    err = max_abs(out, want)
    assert err <= ATOL[q.dtype], f"max-abs {err}"
    return err


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("chunk", [1, 7, 16, 63, 64, 65, 200, 512])
def test_empty_prefix_chunks(device, dtype, chunk):
    args = make_case(device, [0], [chunk], dtype=dtype, seed=chunk)
    q, kc, vc, bt, cu, ctx, mb, mq = args
    check(run(*args, 1 / math.sqrt(128)), q, kc, vc, bt, cu, ctx, 1 / math.sqrt(128))


@pytest.mark.parametrize("prefix,chunk", [(5, 1), (31, 33), (100, 64), (512, 512), (1000, 17),
                                          (1536, 512), (4000, 96)])
def test_prefix_plus_chunk(device, prefix, chunk):
    args = make_case(device, [prefix], [chunk], seed=prefix + chunk)
    q, kc, vc, bt, cu, ctx, mb, mq = args
    check(run(*args, 1 / math.sqrt(128)), q, kc, vc, bt, cu, ctx, 1 / math.sqrt(128))


@pytest.mark.parametrize("G,kvh", [(1, 4), (2, 4), (4, 2), (6, 2), (8, 1)])
def test_group_sizes(device, G, kvh):
    args = make_case(device, [0, 70, 300], [130, 45, 64], H=G * kvh, kvh=kvh, seed=G)
    q, kc, vc, bt, cu, ctx, mb, mq = args
    check(run(*args, 0.1), q, kc, vc, bt, cu, ctx, 0.1)


@pytest.mark.parametrize("bs", [8, 16, 32])
def test_block_sizes(device, bs):
    args = make_case(device, [37, 0], [90, 33], bs=bs, seed=bs)
    q, kc, vc, bt, cu, ctx, mb, mq = args
    check(run(*args, 1 / math.sqrt(128)), q, kc, vc, bt, cu, ctx, 1 / math.sqrt(128))


def test_varlen_with_decode_rows(device):
    """Prefill chunks and single-token decodes in one varlen call."""
    prefixes = [0, 512, 2000, 99, 1, 4095]
    chunks = [300, 128, 1, 1, 1, 1]
    args = make_case(device, prefixes, chunks, seed=7)
    q, kc, vc, bt, cu, ctx, mb, mq = args
    check(run(*args, 1 / math.sqrt(128)), q, kc, vc, bt, cu, ctx, 1 / math.sqrt(128))


def test_context_shorter_than_chunk_gives_zero_rows(device):
    args = make_case(device, [0], [40], seed=3)
    q, kc, vc, bt, cu, ctx, mb, mq = args
    ctx = torch.tensor([25], dtype=torch.int32, device=device)   # rows 0..14 sit before position 0
    out = run(q, kc, vc, bt, cu, ctx, mb, mq, 0.1)
    assert torch.count_nonzero(out[:15]) == 0
    check(out, q, kc, vc, bt, cu, ctx, 0.1)


def test_chunking_invariance_and_last_row_equals_decode(device):
    scale = 1 / math.sqrt(128)
    args = make_case(device, [700], [512], seed=11)
    q, kc, vc, bt, cu, ctx, mb, mq = args
    full = run(*args, scale)
    # the same rows in two calls of 256: the first sees a context 256 shorter
    a1 = run(q[:256], kc, vc, bt, torch.tensor([0, 256], dtype=torch.int32, device=device),
             torch.tensor([700 + 256], dtype=torch.int32, device=device), mb, 256, scale)
    a2 = run(q[256:], kc, vc, bt, torch.tensor([0, 256], dtype=torch.int32, device=device),
             ctx, mb, 256, scale)
    tol = ATOL[torch.bfloat16]
    assert max_abs(torch.cat([a1, a2]), f32(full).astype(np.float64)) <= tol
    # the last row attends to the whole context, like a decode step
    dec = torch.empty(1, 32, 128, dtype=q.dtype, device=device)
    pk.paged_attention_forward(dec, q[-1:].contiguous(), kc, vc, bt, ctx, scale, 16, mb)
    torch.cuda.synchronize()
    assert max_abs(full[-1:], f32(dec).astype(np.float64)) <= tol


def test_config3_store_then_prefill_and_decode(device):
    """Configuration 3: 4 chunks of 512 on prefixes {0, 512, 1536, 3072} plus 48
    decodes, packed varlen: store every new token by slot, then run the prefill
    op on the chunks and the decode op on the decodes."""
    w = workloads.config3(device)
    pk.paged_kv_store_slots(w.k_cache, w.v_cache, w.new_k, w.new_v, w.slot_mapping)
    npf = w.num_prefill_seqs
    tp = w.num_prefill_tokens
    mb = w.block_tables.size(1)
    out = torch.full_like(w.query, float("nan"))
    pk.paged_prefill_attention(out[:tp], w.query[:tp], w.k_cache, w.v_cache,
                               w.block_tables[:npf].contiguous(), w.cu_seqlens_q[:npf + 1].contiguous(),
                               w.context_lens[:npf].contiguous(), w.scale, 16, mb, 512)
    pk.paged_attention_forward(out[tp:], w.query[tp:], w.k_cache, w.v_cache,
                               w.block_tables[npf:].contiguous(), w.context_lens[npf:].contiguous(),
                               w.scale, 16, mb)
    torch.cuda.synchronize()
    want = O.prefill_attention(f32(w.query), f32(w.k_cache), f32(w.v_cache),
                               w.block_tables.cpu().numpy(), w.cu_seqlens_q.cpu().numpy(),
                               w.context_lens.cpu().numpy(), w.scale)
    err = max_abs(out, want)
    print(f"cfg3 max-abs {err:.2e}")
    assert err <= ATOL[torch.bfloat16]


@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_key_splits_match_whole_ranges(device, dtype, hd):
    """Long prefixes are cut into key splits merged by the last split to
    arrive; splitting off (max_context_len=0) runs every range whole. Both
    agree with the oracle and with each other (head dims 64 and 128)."""
    args = make_case(device, [3000, 1100, 0, 5000], [200, 64, 130, 33], D=hd, dtype=dtype,
                     seed=21)
    q, kc, vc, bt, cu, ctx, mb, mq = args
    scale = 1 / math.sqrt(hd)
    assert pk.prefill_workspace_bytes(4, int(q.size(0)), 32, hd, mq, mb * 16) > 0
    split = run(*args, scale)
    whole = torch.full_like(q, float("nan"))
    pk.paged_prefill_attention(whole, q, kc, vc, bt, cu, ctx, scale, 16, mb, mq, max_context_len=0)
    torch.cuda.synchronize()
    check(split, q, kc, vc, bt, cu, ctx, scale)
    check(whole, q, kc, vc, bt, cu, ctx, scale)
    assert max_abs(split, f32(whole).astype(np.float64)) <= ATOL[dtype]


def test_workspace_reuse_and_explicit_workspace(device):
    """The merge counters are left at zero: the same (explicit) workspace
    serves consecutive calls of different shapes; a short one is refused."""
    scale = 1 / math.sqrt(128)
    a1 = make_case(device, [2500, 700], [100, 300], seed=31)
    a2 = make_case(device, [4000], [64], seed=32)
    need = max(pk.prefill_workspace_bytes(2, 400, 32, 128, 300, a1[6] * 16),
               pk.prefill_workspace_bytes(1, 64, 32, 128, 64, a2[6] * 16))
    ws = torch.zeros(need, dtype=torch.uint8, device=device)
    for args in (a1, a2, a1):
        q, kc, vc, bt, cu, ctx, mb, mq = args
        out = torch.full_like(q, float("nan"))
        pk.paged_prefill_attention(out, q, kc, vc, bt, cu, ctx, scale, 16, mb, mq, workspace=ws)
        torch.cuda.synchronize()
        check(out, q, kc, vc, bt, cu, ctx, scale)
    q, kc, vc, bt, cu, ctx, mb, mq = a2
    with pytest.raises(RuntimeError, match="workspace"):
        pk.paged_prefill_attention(torch.empty_like(q), q, kc, vc, bt, cu, ctx, scale, 16, mb, mq,
                                   workspace=ws[:64])


@pytest.mark.parametrize("hd", [64, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("prefixes,chunks,G,kvh,bs", [
    ([0], [1], 4, 2, 16),
    ([0, 70, 300], [130, 45, 64], 4, 2, 16),
    ([5, 1000, 0], [1, 17, 65], 2, 4, 32),
    ([1536, 0, 4000], [512, 200, 96], 1, 4, 8),
    ([0, 512, 2000, 99], [300, 128, 1, 1], 6, 1, 16),
])
def test_head_dims_64_and_256(device, hd, dtype, prefixes, chunks, G, kvh, bs):
    """Head dims 64 (prefill_kernel) and 256 (prefill_generic_kernel): empty
    and paged prefixes, ragged chunks and decode rows in one call, group
    sizes 1-6, block sizes 8-32."""
    print(f"prefill D={hd} {dtype} prefixes={prefixes} chunks={chunks} G={G} kvh={kvh} bs={bs}",
          flush=True)
    args = make_case(device, prefixes, chunks, H=G * kvh, kvh=kvh, D=hd, bs=bs, dtype=dtype,
                     seed=hd + sum(chunks))
    q, kc, vc, bt, cu, ctx, mb, mq = args
    scale = 1 / math.sqrt(hd)
    check(run(*args, scale), q, kc, vc, bt, cu, ctx, scale)


@pytest.mark.parametrize("hd", [64, 128, 256])
def test_nan_rows_past_the_context(device, hd):
    """Rows of a sequence's last block past its context hold NaN: keys past
    the visible range are clamped to the last visible key, so those rows are
    never read and the output equals the oracle's (key splits included at
    head dims 64 and 128)."""
    prefixes, chunks, bs = [3000, 0, 700, 5], [200, 37, 130, 1], 16
    q, kc, vc, bt, cu, ctx, mb, mq = make_case(device, prefixes, chunks, D=hd, bs=bs, seed=hd + 5)
    for i, n in enumerate(ctx.tolist()):
        if n % bs:
            b = int(bt[i, (n - 1) // bs])
            kc[b, :, n % bs:, :] = float("nan")
            vc[b, :, n % bs:, :] = float("nan")
    scale = 1 / math.sqrt(hd)
    check(run(q, kc, vc, bt, cu, ctx, mb, mq, scale), q, kc, vc, bt, cu, ctx, scale)


@pytest.mark.parametrize("hd", [64, 256])
def test_head_dims_64_and_256_zero_rows_and_decode(device, hd):
    """Rows before position 0 are zeros; the last row of a chunk equals a
    decode step over the same context (decode's generic path for D 64/256)."""
    args = make_case(device, [0], [40], D=hd, seed=hd + 3)
    q, kc, vc, bt, cu, ctx, mb, mq = args
    short = torch.tensor([25], dtype=torch.int32, device=device)
    out = run(q, kc, vc, bt, cu, short, mb, mq, 0.1)
    assert torch.count_nonzero(out[:15]) == 0
    check(out, q, kc, vc, bt, cu, short, 0.1)
    scale = 1 / math.sqrt(hd)
    args = make_case(device, [700], [300], D=hd, seed=hd + 11)
    q, kc, vc, bt, cu, ctx, mb, mq = args
    full = run(*args, scale)
    dec = torch.empty(1, 32, hd, dtype=q.dtype, device=device)
    pk.paged_attention_forward(dec, q[-1:].contiguous(), kc, vc, bt, ctx, scale, 16, mb)
    torch.cuda.synchronize()
    assert max_abs(full[-1:], f32(dec).astype(np.float64)) <= ATOL[torch.bfloat16]
