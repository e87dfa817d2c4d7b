"""GPU parity of ragged-batch metadata packing against the oracle's brute-force
restatement of paged_forward's per-layer tensors (bit-exact, int32)."""
import numpy as np
import pytest
import torch

from nanopd_amd import paged_kernels as pk
from oracle import paged_oracle as O

pytestmark = pytest.mark.gpu


def _check(device, seqs, bs, mb=None):
    mb = mb or max([len(t) for _, _, t in seqs] + [1])
    got = pk.pack_metadata(seqs, bs, device, max_blocks_per_seq=mb)
    torch.cuda.synchronize()
    want = O.pack_metadata(seqs, bs, mb)
    for name in ("cu_seqlens_q", "seq_lens", "block_tables", "positions", "slot_mapping", "token_seq"):
        assert np.array_equal(getattr(got, name).cpu().numpy(), want[name]), name


def test_small_mixed_batch(device):
    _check(device, [(3, 5, [7, 2]), (1, 9, [4]), (1, 16, [1, 0])], 8, 3)


def test_config3_shape_batch(device):
    rng = np.random.default_rng(0)
    bs = 16
    seqs = []
    next_blk = 0
    for p in (0, 512, 1536, 3072):
        n = (p + 512 + bs - 1) // bs
        seqs.append((512, p, list(range(next_blk, next_blk + n))))
        next_blk += n
    for _ in range(48):
        ctx = int(rng.integers(256, 2048))
        n = (ctx + 1 + bs - 1) // bs
        seqs.append((1, ctx, list(rng.permutation(20000)[:n])))
    _check(device, seqs, bs)


def test_many_sequences_and_empty_rows(device):
    rng = np.random.default_rng(1)
    seqs = []
    for i in range(3000):   # more than one scan chunk of 1024
        ql = int(rng.integers(0, 4))
        ctx = int(rng.integers(0, 100))
        n = int(rng.integers(0, (ctx + ql + 7) // 8 + 1))
        seqs.append((ql, ctx, list(rng.integers(0, 5000, size=n))))
    _check(device, seqs, 8)
