"""Writes the golden fixtures of tests/golden/ from the CPU oracle.

The reference stores no vectors for this path (its tests draw inputs on a CUDA
device), so the fixtures are produced here by the pinned oracle
(tests/test_oracle.py) on inputs drawn on the CPU, which are the same on every
machine:

* cfg1.npz   -- configuration 1 (Qwen2-1.5B shape, fp16): digests of the inputs
  and of the pool after all 792 context tokens are stored, plus the expected
  decode output bits (float64 oracle rounded once to fp16).
* tiny.npz   -- a fully explicit small case (inputs and outputs in the file):
  2 sequences {3, 9}, H 4, kvh 2, D 64, block 4, bf16.

Run from the repository root: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from nanopd_amd import workloads  # noqa: E402
from oracle import paged_oracle as O  # noqa: E402
from tests.helpers import bits, sha  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def cfg1():
    w = workloads.config1("cpu")
    kc, vc = bits(w.k_cache), bits(w.v_cache)
    O.kv_store(kc, vc, bits(w.store_k), bits(w.store_v), w.store_tables.numpy(),
               w.store_positions.numpy())
    out = O.decode_attention(O.bits_to_f32(bits(w.query), "f16"), O.bits_to_f32(kc, "f16"),
                             O.bits_to_f32(vc, "f16"), w.block_tables.numpy(), w.seq_lens.numpy(),
                             w.scale)
    np.savez(os.path.join(HERE, "cfg1.npz"),
             inputs_sha=np.array(sha(bits(w.query), bits(w.store_k), bits(w.store_v),
                                     w.block_tables.numpy(), w.store_positions.numpy())),
             pool_sha=np.array(sha(kc, vc)),
             out_bits=O.f32_to_bits(out.astype(np.float32), "f16"))


def tiny():
    rng = np.random.default_rng(1234)
    S, H, kvh, D, bs, lens = 2, 4, 2, 64, 4, [3, 9]
    nb = 5
    q = O.f32_to_bits((rng.standard_normal((S, H, D)) * 0.5).astype(np.float32), "bf16")
    kc = O.f32_to_bits((rng.standard_normal((nb, kvh, bs, D)) * 0.5).astype(np.float32), "bf16")
    vc = O.f32_to_bits((rng.standard_normal((nb, kvh, bs, D)) * 0.5).astype(np.float32), "bf16")
    bt = np.array([[4, 0, 0], [2, 0, 3]], np.int32)
    sl = np.array(lens, np.int32)
    out = O.decode_attention(O.bits_to_f32(q, "bf16"), O.bits_to_f32(kc, "bf16"),
                             O.bits_to_f32(vc, "bf16"), bt, sl, 0.125)
    np.savez(os.path.join(HERE, "tiny.npz"), q=q, k_cache=kc, v_cache=vc, block_tables=bt,
             seq_lens=sl, scale=np.float32(0.125), out=out)


if __name__ == "__main__":
    cfg1()
    tiny()
    print("wrote", os.listdir(HERE))
