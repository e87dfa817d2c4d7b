"""CPU tests of the drop-in boundary: the C-ABI library loads, exports every
symbol include/nanopd.h declares, and rejects bad arguments before touching
the GPU; the Python mirror raises RuntimeError where the reference's
TORCH_CHECKs do (PA/csrc/attention/paged_attention_ops.cu:18-22,
PA/csrc/kvstore/paged_kv_store_ops.cu:13-16; int64 tables ->
RuntimeError as in PA/tests/test_paged_attention.py:233-247)."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from nanopd_amd import _lib
from nanopd_amd import paged_kernels as pk

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols():
    text = (ROOT / "include" / "nanopd.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(npd_\w+)\s*\(", text, re.M)))


def test_header_and_binding_agree():
    assert _declared_symbols() == sorted(_lib.exported_symbols())


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared_symbols():
        assert hasattr(lib, name), name
    assert lib.npd_version() >= 100


def test_library_exports_are_plain_c():
    # no torch / C++ types across the boundary: the .so must not link libtorch
    import subprocess
    out = subprocess.run(["ldd", str(_lib.LIB_PATH)], capture_output=True, text=True).stdout
    assert "libtorch" not in out and "libc10" not in out


def _rc(name, *args):
    return getattr(_lib.load(), name)(*args)


@pytest.mark.skipif(torch.cuda.is_available(),
                    reason="fake pointers: validation-only test, never run where a launch could happen")
def test_c_validation_paths_need_no_gpu():
    lib = _lib.load()
    fake = 0x1000  # never dereferenced: validation fails first
    # unsupported dtype
    rc = _rc("npd_paged_kv_store", fake, fake, fake, fake, fake, fake, 4, 2, 128, 16, 16, 4, 512,
             128, 7, None)
    assert rc == -2 and b"dtype" in lib.npd_last_error()
    # bad head dims: not a multiple of 4 for the store, of 8 (or outside [32,
    # 256]) for decode; a head dim of 4 mod 8 needs 8-byte alignment only
    rc = _rc("npd_paged_kv_store", fake, fake, fake, fake, fake, fake, 4, 2, 98, 16, 16, 4, 392,
             98, 1, None)
    assert rc == -1 and b"head_dim" in lib.npd_last_error()
    # (an odd stride stops each call before any launch: the pointer check
    # passed when the message names the strides)
    rc = _rc("npd_paged_kv_store", fake + 8, fake, fake, fake, fake, fake, 4, 2, 100, 16, 16, 4,
             402, 100, 1, None)
    assert rc == -3 and b"strides" in lib.npd_last_error()
    rc = _rc("npd_paged_kv_store", fake + 4, fake, fake, fake, fake, fake, 4, 2, 100, 16, 16, 4,
             402, 100, 1, None)
    assert rc == -3 and b"8-byte aligned" in lib.npd_last_error()
    for d in (24, 100, 264):
        rc = _rc("npd_paged_attention", fake, fake, fake, fake, fake, fake, 2, 32, 8, d, 64, 16, 4,
                 ctypes.c_float(0.1), 32 * d, d, 32 * d, d, None, 0, 1, None)
        assert rc == -1 and b"head_dim" in lib.npd_last_error(), d
    # misaligned pointer
    rc = _rc("npd_paged_kv_store", fake + 2, fake, fake, fake, fake, fake, 4, 2, 128, 16, 16, 4,
             512, 128, 1, None)
    assert rc == -3
    # odd stride
    rc = _rc("npd_paged_kv_store_slots", fake, fake, fake, fake, fake, 4, 2, 128, 16, 16, 130,
             260, 1, None)
    assert rc == -3
    # heads not a multiple of kv heads
    rc = _rc("npd_paged_attention", fake, fake, fake, fake, fake, fake, 2, 12, 5, 128, 64, 16, 4,
             ctypes.c_float(0.1), 1536, 128, 1536, 128, None, 0, 1, None)
    assert rc == -1 and b"multiple" in lib.npd_last_error()
    # a group of 16 q-heads per kv head is accepted: at head dim 64 it is
    # served as two groups of 8 (a workspace sized for 4 units), at head dim
    # 128 with blocks of 16 as one 16-head unit per kv head (2 units, 256-token
    # partitions: 16 x 256 scores); validation gets as far as the missing
    # workspace
    need = lib.npd_paged_attention_workspace_size(2, 32, 2, 64, 16, 4)
    assert need == lib.npd_paged_attention_workspace_size(2, 32, 4, 64, 16, 4)
    wide = lib.npd_paged_attention_workspace_size(2, 32, 2, 128, 16, 4)
    # (4 units: too few items for longer partitions -> 64 tokens, 1 slot each)
    assert wide == (2**20 + 16 + 2 * 2 * 1 * 8 + 255) // 256 * 256 + 2 * 32 * 1 * 130 * 4
    rc = _rc("npd_paged_attention", fake, fake, fake, fake, fake, fake, 2, 32, 2, 128, 64, 16, 4,
             ctypes.c_float(0.1), 4096, 128, 4096, 128, None, 0, 1, None)
    assert rc == -4 and b"workspace" in lib.npd_last_error()
    # workspace required for a long context and missing
    rc = _rc("npd_paged_attention", fake, fake, fake, fake, fake, fake, 2, 32, 8, 128, 4096, 16,
             256, ctypes.c_float(0.1), 4096, 128, 4096, 128, None, 0, 1, None)
    assert rc == -4 and b"workspace" in lib.npd_last_error()
    # zero work is a no-op, not an error
    assert _rc("npd_paged_attention", 0, 0, 0, 0, 0, 0, 0, 32, 8, 128, 4096, 16, 256,
               ctypes.c_float(0.1), 4096, 128, 4096, 128, None, 0, 1, None) == 0
    assert _rc("npd_copy_blocks", fake, fake, fake, 0, 10, 1024, 1, None) == 0
    assert _rc("npd_copy_blocks", fake, fake, fake, 3, 10, 1004, 1, None) == -3
    # block-list gather / scatter: no-op, unaligned block size, null ids, too many layers
    for fn in ("npd_kv_gather_blocks", "npd_kv_scatter_blocks"):
        assert _rc(fn, fake, fake, 36, 100, 32768, fake, 0, fake, fake, None) == 0
        assert _rc(fn, fake, fake, 36, 100, 32760, fake, 4, fake, fake, None) == -3
        assert _rc(fn, fake, fake, 36, 100, 32768, None, 4, fake, fake, None) == -1
        assert _rc(fn, fake, fake, 70000, 100, 32768, fake, 4, fake, fake, None) == -1
    assert _rc("npd_pack_metadata", fake, fake, 5000, 1, 1, 4, 16, fake, fake, fake, fake, fake,
               fake, None) == -1
    # fused q/k norm + rope + store: head_dim, short token stride, dtype, no-op
    rope = lambda d, stride, code, t=4: _rc(  # noqa: E731
        "npd_qk_norm_rope_store", fake, fake, fake, fake, fake, fake, fake, fake, fake, t, 32, 8, d,
        64, 16, stride, 32 * d, ctypes.c_float(1e-6), code, None)
    assert rope(96, 48 * 96, 1) == -1 and b"head_dim" in lib.npd_last_error()
    assert rope(128, 40 * 128, 1) == -1 and b"stride" in lib.npd_last_error()
    assert rope(128, 48 * 128, 5) == -2
    assert rope(128, 48 * 128, 1, t=0) == 0


@pytest.mark.skipif(torch.cuda.is_available(),
                    reason="fake pointers: validation-only test, never run where a launch could happen")
def test_noalloc_validates_like_the_workspace_entry_point():
    # npd_paged_attention_noalloc checks its arguments before it looks at its
    # static scratch (or the device): every invalid call returns the code
    # npd_paged_attention returns, with the same message, and launches nothing
    lib = _lib.load()
    fake = 0x1000
    f = ctypes.c_float(0.1)
    cases = [
        # (seqs, heads, kv heads, head dim, blocks, block, max bps, strides, dtype, out ptr)
        (2, 32, 8, 128, 64, 16, 4, (4096, 128, 4096, 128), 7, fake),        # dtype
        (2, 12, 5, 128, 64, 16, 4, (1536, 128, 1536, 128), 1, fake),        # heads % kv heads
        (2, 32, 8, 100, 64, 16, 4, (3200, 100, 3200, 100), 1, fake),        # head dim
        (2, 32, 8, 128, 64, 16, 4, (4100, 128, 4096, 128), 1, fake),        # q stride
        (2, 32, 8, 128, 64, 16, 4, (4096, 128, 4096, 128), 1, fake + 8),    # out alignment
        (2, 32, 8, 128, 64, 16, 4, (4096, 128, 4096, 128), 1, 0),           # null out
        (-1, 32, 8, 128, 64, 16, 4, (4096, 128, 4096, 128), 1, fake),       # sizes
    ]
    for s, h, kvh, d, nb, bs, mb, (qs, qh, os_, oh), code, out in cases:
        rc_ws = _rc("npd_paged_attention", out, fake, fake, fake, fake, fake, s, h, kvh, d, nb, bs,
                    mb, f, qs, qh, os_, oh, None, 0, code, None)
        msg_ws = lib.npd_last_error().split(b":", 1)[1]
        rc_na = _rc("npd_paged_attention_noalloc", out, fake, fake, fake, fake, fake, s, h, kvh, d,
                    nb, bs, mb, f, qs, qh, os_, oh, code, None)
        msg_na = lib.npd_last_error().split(b":", 1)[1]
        assert rc_ws < 0 and rc_na == rc_ws and msg_na == msg_ws, (s, h, kvh, d, rc_ws, rc_na)
    # no work is a no-op for both
    assert _rc("npd_paged_attention_noalloc", 0, 0, 0, 0, 0, 0, 0, 32, 8, 128, 4096, 16, 256, f,
               4096, 128, 4096, 128, 1, None) == 0


def test_workspace_size():
    lib = _lib.load()
    # fast path (head_dim 128): the fixed 1 MiB counter region every workspace
    # starts with, a 16-byte item count, an 8-byte (unit, partition) work-list
    # entry per possible partition (padded to 256 bytes), then fp32 partials
    # (G*D + 2G floats per partition and, past 16 partitions, per group of 16
    # partitions: the first level of the two-level merge).
    def fast(S, H, kvh, P):
        units = S * kvh
        groups = (P + 15) // 16 if P > 16 else 0
        return (2**20 + 16 + units * P * 8 + 255) // 256 * 256 + S * H * (P + groups) * 130 * 4
    ws = lib.npd_paged_attention_workspace_size
    # 2-byte pools (block size 64 here, a size the FP8 entry point does not
    # take): the host partition is the longest of 2048 .. 64 tokens that gives
    # >= 1280 work items at the longest context, and for the two-pass kernel
    # (head dim 128 with up to 4 query heads per kv head, head dims 64 / 256)
    # at most 4096 / G tokens for G query heads per kv head, G rounded up to a
    # power of two; the one-pass units (head dim 128 from 5 heads on, every
    # FP8 group) keep no scores and have no such cap. The kernel may halve it
    # for shorter actual contexts, down to a quarter (and not below 64 tokens
    # or the block): the partials are sized for that one.
    # 1024 seqs x 8 kv heads x 256 tokens: one partition each
    assert ws(1024, 32, 8, 128, 64, 4) == fast(1024, 32, 8, 1)
    # 64 seqs x 8 kv heads x 256 tokens: 512 units -> the block (64), 4 each
    assert ws(64, 32, 8, 128, 64, 4) == fast(64, 32, 8, 4)
    # 8 seqs x 8 kv heads x 32k tokens: 2048 gives 1024 items, 1024 gives
    # 2048 -> 1024, slots for 256-token partitions (128)
    assert ws(8, 32, 8, 128, 64, 512) == fast(8, 32, 8, 128)
    # 10 seqs x 8 kv heads x 32832 tokens: G = 4 caps the partition at 1024
    # (slots for 256: 129); G = 8 (a one-pass unit) and G = 2 take 2048 (512: 65)
    assert ws(10, 32, 8, 128, 64, 513) == fast(10, 32, 8, 129)
    assert ws(10, 64, 8, 128, 64, 513) == fast(10, 64, 8, 65)
    assert ws(10, 16, 8, 128, 64, 513) == fast(10, 16, 8, 65)
    # 1 seq x 8 kv heads x 4k tokens: too few items at any length -> the block
    assert ws(1, 32, 8, 128, 64, 64) == fast(1, 32, 8, 64)
    # 4096 seqs x 8 kv heads x 128k tokens: slots for 512 partitions of 256,
    # but a counter per unit and per group (32768 x 33) would not fit the
    # 262144 counters -> one level, no group partials; 512 seqs (4096 x 33) fit
    assert ws(4096, 32, 8, 128, 64, 2048) == fast(4096, 32, 8, 512) - 4096 * 32 * 32 * 130 * 4
    assert ws(512, 32, 8, 128, 64, 2048) == fast(512, 32, 8, 512)
    # Blocks of 16 or 32 (which the FP8 entry point takes): the workspace also
    # covers an FP8 pool's partition (one-pass units: no score cap); here both
    # give 128 slots of 256 tokens
    assert ws(8, 32, 8, 128, 16, 2048) == fast(8, 32, 8, 128)
    assert ws(8, 32, 8, 128, 32, 1024) == fast(8, 32, 8, 128)
    # 1024 seqs x 256 tokens: both rules give one partition
    assert ws(1024, 32, 8, 128, 16, 16) == fast(1024, 32, 8, 1)
    # 1 seq x 8 kv heads x 4k tokens in blocks of 16: partitions of 64
    assert ws(1, 32, 8, 128, 16, 256) == fast(1, 32, 8, 64)
    # head dims 64 and 256 take the fast path for blocks of 16 and 32: the
    # same layout with G*D + 2G floats per partition (1 seq x 8 kv heads x 1k
    # tokens: partitions of 64, 16 slots)
    def fast_d(S, H, kvh, P, d):
        units = S * kvh
        return (2**20 + 16 + units * P * 8 + 255) // 256 * 256 + S * H * P * (d + 2) * 4
    assert ws(2, 8, 8, 64, 16, 64) == fast_d(2, 8, 8, 16, 64)
    assert ws(2, 8, 8, 256, 32, 32) == fast_d(2, 8, 8, 16, 256)
    # generic path (block size 8, any head dim): partitions of 256 below 4096 waves
    n = lib.npd_paged_attention_workspace_size(2, 8, 8, 64, 8, 128)
    assert n == 2**20 + 2 * 8 * 4 * (64 + 2) * 4


def test_prefill_workspace_size():
    lib = _lib.load()
    # key ranges up to 16 steps of 64 keys run whole: no workspace
    assert lib.npd_paged_prefill_workspace_size(4, 2048, 32, 128, 512, 1024) == 0
    assert lib.npd_paged_prefill_workspace_size(4, 2048, 32, 128, 512, 0) == 0
    # longer ranges are split (at most 8 ways): the 1 MiB counter region, then
    # per (sequence, row subtile of 32, head, split) an O record of 32 rows x
    # D fp32 and an (m, l) record of 32 rows x 2 x 4 lanes
    def split(S, H, max_q, splits, D=128):
        t32 = (max_q + 31) // 32 + 7
        units = S * t32 * H
        return 2**20 + units * splits * (32 * D * 4 + 1024)
    assert lib.npd_paged_prefill_workspace_size(4, 2048, 32, 128, 512, 3584) == split(4, 32, 512, 4)
    assert lib.npd_paged_prefill_workspace_size(1, 100, 32, 128, 100, 1025) == split(1, 32, 100, 2)
    assert lib.npd_paged_prefill_workspace_size(2, 1024, 32, 128, 512, 32768) == split(2, 32, 512, 8)
    # head dim 64 runs the same kernel with half-size O records
    assert lib.npd_paged_prefill_workspace_size(4, 2048, 32, 64, 512, 3584) == \
        split(4, 32, 512, 4, D=64)
    assert lib.npd_paged_prefill_workspace_size(4, 2048, 32, 64, 512, 1024) == 0
    # head dim 256 runs unsplit (prefill_generic_kernel): no workspace
    assert lib.npd_paged_prefill_workspace_size(2, 1024, 32, 256, 512, 32768) == 0


def test_python_mirror_raises_like_torch_check():
    q = torch.zeros(2, 4, 64, dtype=torch.float16)
    kc = torch.zeros(4, 4, 8, 64, dtype=torch.float16)
    bt = torch.zeros(2, 1, dtype=torch.int32)
    sl = torch.ones(2, dtype=torch.int32)
    out = torch.zeros_like(q)
    with pytest.raises(RuntimeError, match="CUDA"):
        pk.paged_attention_forward(out, q, kc, kc, bt, sl, 0.1, 8, 1)
    with pytest.raises(RuntimeError, match="CUDA"):
        pk.paged_kv_store(kc, kc, q, q, bt, sl)
    with pytest.raises(RuntimeError):
        pk.paged_prefill_attention(out, q, kc, kc, bt, torch.zeros(3, dtype=torch.int32), sl,
                                   0.1, 8, 1, 1)
