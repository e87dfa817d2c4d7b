"""GPU test of npd_paged_attention_noalloc (the decode entry point that
allocates nothing: its workspace is a static device array) against
npd_paged_attention with a caller workspace, both called through the C-ABI.

Two calls in a row on the same GPU share the static array; the second has a
smaller input (fewer sequences, shorter contexts, another dtype), so it runs
over what the first left there. Outputs must be bit-identical to the existing
entry point's (same kernels, same partition and merge order), and within the
attention tolerance of the float64 oracle. Shapes beyond the scratch size are
refused before any launch."""
import ctypes

import numpy as np
import pytest
import torch

from nanopd_amd import _lib
from nanopd_amd import paged_kernels as pk
from tests.helpers import ATOL, bits, max_abs, oracle_decode

pytestmark = pytest.mark.gpu

_CODE = {torch.float16: _lib.NPD_DTYPE_F16, torch.bfloat16: _lib.NPD_DTYPE_BF16}


def _inputs(num_seqs, heads, kv_heads, ctx_max, dtype, device, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    bs, d = 16, 128
    lens = torch.randint(1, ctx_max + 1, (num_seqs,), generator=g)
    lens[0] = ctx_max
    nbs = [(int(s) + bs - 1) // bs for s in lens]
    mb, total = max(nbs), sum(nbs)
    q = (torch.randn(num_seqs, heads, d, generator=g) * 0.5).to(dtype)
    kc = (torch.randn(total, kv_heads, bs, d, generator=g) * 0.5).to(dtype)
    vc = (torch.randn(total, kv_heads, bs, d, generator=g) * 0.5).to(dtype)
    order = torch.randperm(total, generator=g)
    bt = torch.zeros(num_seqs, mb, dtype=torch.int32)
    o = 0
    for i, n in enumerate(nbs):
        bt[i, :n] = order[o:o + n]
        o += n
    sl = lens.to(torch.int32)
    return [t.to(device) for t in (q, kc, vc, bt, sl)] + [mb]


def _noalloc(out, q, kc, vc, bt, sl, mb):
    s, h, d = q.shape
    nb, kvh, bs, _ = kc.shape
    return _lib.load().npd_paged_attention_noalloc(
        out.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(), sl.data_ptr(),
        s, h, kvh, d, nb, bs, mb, d ** -0.5, q.stride(0), q.stride(1), out.stride(0),
        out.stride(1), _CODE[q.dtype], ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


def _with_workspace(q, kc, vc, bt, sl, mb):
    out = torch.full_like(q, float("nan"))
    pk.paged_attention_forward(out, q, kc, vc, bt, sl, q.size(2) ** -0.5, kc.size(2), mb)
    return out


def _graph_replays(device, eager_first, seed):
    """Captures one npd_paged_attention_noalloc call into a HIP graph (after
    an eager call when eager_first), then replays it three times over new
    query contents and new context lengths written into the captured input
    buffers, with eager work and synchronisations between the replays. Each
    replay must equal npd_paged_attention on a caller workspace bit for bit."""
    num_seqs, heads, kvh, ctx_max = 16, 32, 8, 4096
    q, kc, vc, bt, sl, mb = _inputs(num_seqs, heads, kvh, ctx_max, torch.bfloat16, device, seed)
    out = torch.full_like(q, float("nan"))
    if eager_first:
        assert _noalloc(out, q, kc, vc, bt, sl, mb) == 0, _lib.load().npd_last_error()
        torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    rcs = []
    with torch.cuda.graph(graph):
        rcs.append(_noalloc(out, q, kc, vc, bt, sl, mb))
    assert rcs == [0], _lib.load().npd_last_error()
    gen = torch.Generator(device="cpu").manual_seed(seed + 100)
    for rep in range(3):
        print(f"noalloc graph replay {rep} (eager first: {eager_first})", flush=True)
        q.copy_((torch.randn(q.shape, generator=gen) * 0.5).to(q.dtype))
        lens = torch.randint(1, ctx_max + 1, (num_seqs,), generator=gen)
        lens[rep] = ctx_max   # some sequence spans the whole table (the longest split)
        sl.copy_(lens.to(torch.int32))
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        want = _with_workspace(q, kc, vc, bt, sl, mb)
        torch.cuda.synchronize()
        assert np.array_equal(bits(out), bits(want)), f"replay {rep} differs"


def test_noalloc_under_graph_capture_first_call(device):
    # the first noalloc call of the process (the scratch look-up and the clear
    # of its counter region happen inside the capture)
    _graph_replays(device, eager_first=False, seed=11)


def test_noalloc_under_graph_capture_after_eager_call(device):
    _graph_replays(device, eager_first=True, seed=12)


@pytest.mark.parametrize("first,second", [
    # (num_seqs, heads, kv_heads, ctx_max, dtype, seed)
    ((96, 32, 8, 4096, torch.bfloat16, 1), (8, 32, 8, 2000, torch.float16, 2)),
    ((8, 32, 8, 32768, torch.bfloat16, 3), (4, 12, 2, 511, torch.float16, 4)),
    # one-pass units: 16 heads per kv head, then 32 (two units of 16 per kv head)
    ((12, 128, 8, 2500, torch.bfloat16, 5), (6, 64, 2, 9000, torch.float16, 6)),
])
def test_noalloc_matches_workspace_entry_point(device, first, second):
    for num_seqs, heads, kvh, ctx_max, dtype, seed in (first, second):
        print(f"noalloc case: seqs {num_seqs} heads {heads}/{kvh} ctx {ctx_max} {dtype}",
              flush=True)
        q, kc, vc, bt, sl, mb = _inputs(num_seqs, heads, kvh, ctx_max, dtype, device, seed)
        want = _with_workspace(q, kc, vc, bt, sl, mb)
        got = torch.full_like(q, float("nan"))
        rc = _noalloc(got, q, kc, vc, bt, sl, mb)
        assert rc == 0, _lib.load().npd_last_error()
        torch.cuda.synchronize()
        assert np.array_equal(bits(got), bits(want)), "differs from npd_paged_attention"
        err = max_abs(got, oracle_decode(q, kc, vc, bt, sl, q.size(2) ** -0.5))
        assert err <= ATOL[dtype], f"max-abs {err} vs the oracle"


def test_noalloc_refuses_shapes_beyond_scratch(device):
    # 64 sequences with 65536-token tables need far more than the scratch:
    # refused before any pointer is touched
    need = pk.attention_workspace_bytes(64, 32, 8, 128, 16, 4096)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    fake = 0x1000
    rc = _lib.load().npd_paged_attention_noalloc(fake, fake, fake, fake, fake, fake, 64, 32, 8,
                                                 128, 1 << 16, 16, 4096, 0.088, 4096, 128, 4096,
                                                 128, _lib.NPD_DTYPE_BF16, None)
    assert rc == -4 and b"static scratch" in _lib.load().npd_last_error()
