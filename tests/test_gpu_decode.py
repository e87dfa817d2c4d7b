"""GPU parity of paged decode attention against the float64 oracle.

Tolerance (max-abs, output vs oracle): 2e-3 for fp16, 1e-2 for bf16 -- the
bar of the task, tighter than the reference tests' atol=rtol=1e-2
(PA/tests/test_paged_attention.py:144). Cases restate the reference list
(PA/tests/test_paged_attention.py:127-247) and add the measured configurations
and properties (permutation invariance, seq_len 0/1, CoW fork, strided query,
every group size and head dim the kernel instantiates)."""
import math

import numpy as np
import pytest
import torch

from nanopd_amd import paged_kernels as pk
from nanopd_amd import workloads
from oracle import paged_oracle as O
from tests.helpers import ATOL, bits, f32, max_abs, oracle_decode, sha

pytestmark = pytest.mark.gpu


def make_inputs(num_seqs, num_heads, num_kv_heads, head_size, seq_lens, block_size, dtype,
                device, seed=42, shuffle=True):
    """Like make_inputs of PA/tests/test_paged_attention.py:78-110, with values
    drawn on the CPU and (optionally) a shuffled block order."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    nbs = [(s + block_size - 1) // block_size for s in seq_lens]
    mb, total = max(nbs), sum(nbs)
    q = torch.randn(num_seqs, num_heads, head_size, generator=g).to(dtype)
    kc = torch.randn(total, num_kv_heads, block_size, head_size, generator=g).to(dtype)
    vc = torch.randn(total, num_kv_heads, block_size, head_size, generator=g).to(dtype)
    order = torch.randperm(total, generator=g) if shuffle else torch.arange(total)
    bt = torch.zeros(num_seqs, mb, dtype=torch.int32)
    o = 0
    for i, n in enumerate(nbs):
        bt[i, :n] = order[o:o + n]
        o += n
    sl = torch.tensor(seq_lens, dtype=torch.int32)
    return (q.to(device), kc.to(device), vc.to(device), bt.to(device), sl.to(device),
            1.0 / math.sqrt(head_size), mb)


def run(q, kc, vc, bt, sl, scale, mb, bs):
    out = torch.full_like(q, float("nan"))   # the op must overwrite every element
    pk.paged_attention_forward(out, q, kc, vc, bt, sl, scale, bs, mb)
    torch.cuda.synchronize()
    return out


def check(out, q, kc, vc, bt, sl, scale):
    want = oracle_decode(q, kc, vc, bt, sl, scale)
    err = max_abs(out, want)
    assert np.isfinite(f32(out)).all()
    assert err <= ATOL[q.dtype], f"max-abs {err}"
    return err


@pytest.mark.parametrize("D,bs", [(64, 16), (128, 16), (128, 32), (256, 16), (128, 8)])
def test_nan_rows_past_the_context(device, D, bs):
    """Rows of a sequence's last block past its context hold NaN: the kernels
    mask those tokens' scores by selection and zero their V rows, so the
    output is finite and equals the oracle's over the context (fast path at
    head dims 64 / 128 / 256, block sizes 16 and 32; the generic path at block
    size 8)."""
    lens = [1, 17, 300, 777, 5, 40]
    q, kc, vc, bt, sl, scale, mb = make_inputs(len(lens), 12, 3, D, lens, bs, torch.bfloat16,
                                               device, seed=D + bs)
    for i, n in enumerate(lens):
        if n % bs:
            b = int(bt[i, (n - 1) // bs])
            kc[b, :, n % bs:, :] = float("nan")
            vc[b, :, n % bs:, :] = float("nan")
    check(run(q, kc, vc, bt, sl, scale, mb, bs), q, kc, vc, bt, sl, scale)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_single_seq_single_head(device, dtype):
    args = make_inputs(1, 1, 1, 64, [8], 16, dtype, device)
    q, kc, vc, bt, sl, scale, mb = args
    check(run(*args, 16), q, kc, vc, bt, sl, scale)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_multi_seq(device, dtype):
    args = make_inputs(3, 4, 4, 64, [4, 8, 12], 8, dtype, device)
    q, kc, vc, bt, sl, scale, mb = args
    check(run(*args, 8), q, kc, vc, bt, sl, scale)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_gqa(device, dtype):
    args = make_inputs(2, 8, 2, 64, [16, 8], 8, dtype, device)
    q, kc, vc, bt, sl, scale, mb = args
    check(run(*args, 8), q, kc, vc, bt, sl, scale)


@pytest.mark.parametrize("seq_len", [1, 7, 8, 9, 15, 16, 17, 32, 255, 256, 257, 511, 512, 513])
def test_various_seq_lens(device, seq_len):
    args = make_inputs(1, 4, 4, 64, [seq_len], 8, torch.float16, device)
    q, kc, vc, bt, sl, scale, mb = args
    check(run(*args, 8), q, kc, vc, bt, sl, scale)


@pytest.mark.parametrize("block_size", [4, 8, 16, 32])
def test_various_block_sizes(device, block_size):
    args = make_inputs(2, 4, 4, 64, [24, 16], block_size, torch.float16, device)
    q, kc, vc, bt, sl, scale, mb = args
    check(run(*args, block_size), q, kc, vc, bt, sl, scale)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("G", [1, 2, 3, 4, 5, 6, 7, 8])
def test_group_sizes_and_head_dims(device, dtype, D, G):
    kvh = 2
    args = make_inputs(3, G * kvh, kvh, D, [1, 300, 1100], 16, dtype, device, seed=G * D)
    q, kc, vc, bt, sl, scale, mb = args
    check(run(*args, 16), q, kc, vc, bt, sl, scale)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("G,kvh", [(12, 2), (16, 4), (16, 1), (9, 1), (11, 1), (13, 1), (14, 2),
                                   (15, 1), (26, 1)])
def test_group_sizes_above_8(device, dtype, G, kvh):
    """More than 8 query heads per kv head (e.g. 64 q / 4 kv heads): the kv
    head of q-head h is still h // G (PA/csrc/attention/
    paged_attention_kernel.cu:62); the op serves groups of up to 16 heads as
    one one-pass unit (direct K operand loads up to 12 heads, K staged through
    LDS for 13-16) and G = 26 as two units of 13. Contexts up to 32k tokens
    (two-level merges), an empty sequence and a one-token one."""
    lens = [1, 17, 300, 4097, 32768, 0]
    args = make_inputs(len(lens), G * kvh, kvh, 128, lens, 16, dtype, device, seed=G * 10 + kvh)
    q, kc, vc, bt, sl, scale, mb = args
    check(run(*args, 16), q, kc, vc, bt, sl, scale)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("G,kvh,bs", [(16, 2, 16), (16, 1, 32), (32, 2, 16), (48, 1, 32)])
def test_sixteen_head_units(device, dtype, G, kvh, bs):
    """Groups that are a multiple of 16 heads at head dim 128 with blocks of
    16 or 32 run as 16-head units (both passes on the matrix cores, each K/V
    row read once per unit): G = 16, 32 (two units per kv head) and 48.
    Contexts up to 32k (two-level merges), an empty and a one-token
    sequence, NaN rows past the last token of a partial block."""
    lens = [1, 17, 300, 4097, 32768, 0, 1000]
    print(f"16-head units G={G} kvh={kvh} bs={bs} {dtype}", flush=True)
    q, kc, vc, bt, sl, scale, mb = make_inputs(len(lens), G * kvh, kvh, 128, lens, bs, dtype,
                                               device, seed=G * 7 + kvh + bs)
    for i, n in enumerate(lens):
        if n % bs:
            b = int(bt[i, (n - 1) // bs])
            kc[b, :, n % bs:, :] = float("nan")
            vc[b, :, n % bs:, :] = float("nan")
    check(run(q, kc, vc, bt, sl, scale, mb, bs), q, kc, vc, bt, sl, scale)


def test_sixteen_head_units_short_contexts(device):
    """16-head units over few short sequences (the kernel halves the
    partition while the contexts give too few items) and config 2's contexts
    with 128 query heads over its 8 kv heads."""
    g = torch.Generator().manual_seed(128)
    for lens in ([33, 250, 9, 1000], torch.randint(128, 4097, (64,), generator=g).tolist()):
        args = make_inputs(len(lens), 16 * 8, 8, 128, lens, 16, torch.bfloat16, device,
                           seed=len(lens))
        q, kc, vc, bt, sl, scale, mb = args
        check(run(*args, 16), q, kc, vc, bt, sl, scale)


def jumping_scores_case(device, G, kvh, lens, dtype, seed):
    """Every query head of a group has the same vector u, and the K rows of a
    few tokens are multiples of u: their scores jump far above the earlier
    ones (log2 units: the first by about 16, the second by about 33) in the
    middle of a partition, so that a probability reference formed from the
    first steps must move twice. V rows random."""
    q, kc, vc, bt, sl, scale, mb = make_inputs(len(lens), G * kvh, kvh, 128, lens, 16, dtype,
                                               device, seed=seed)
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(kvh, 128, generator=g)
    q.copy_(u.repeat_interleave(G, 0)[None].expand(q.shape).to(dtype))
    for s_, n in enumerate(lens):
        for tok, alpha in ((n // 3, 1.0), ((2 * n) // 3, 2.0)):
            if n < 48:
                continue
            b, o = int(bt[s_, tok // 16]), tok % 16
            kc[b, :, o, :] = (alpha * u).to(dtype).to(device)
    return q, kc, vc, bt, sl, scale, mb


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_sixteen_head_units_rescale_mid_partition(device, dtype):
    """16-head units form probabilities against a per-head reference that
    moves only when a step's max exceeds it by more than 2^8; a move after
    the first step rescales the probabilities already stored. Scores that
    jump twice inside a partition exercise that path (contexts shorter and
    longer than a partition)."""
    lens = [200, 700, 3000, 40]
    q, kc, vc, bt, sl, scale, mb = jumping_scores_case(device, 16, 2, lens, dtype, seed=77)
    check(run(q, kc, vc, bt, sl, scale, mb, 16), q, kc, vc, bt, sl, scale)


@pytest.mark.parametrize("D,bs", [(64, 8), (256, 8), (128, 8)])
def test_group_of_16_generic_path(device, D, bs):
    """G = 16 on the generic kernel (block size 8)."""
    args = make_inputs(3, 32, 2, D, [1, 700, 3000], bs, torch.bfloat16, device, seed=D + bs)
    q, kc, vc, bt, sl, scale, mb = args
    check(run(*args, bs), q, kc, vc, bt, sl, scale)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("bs", [16, 32])
@pytest.mark.parametrize("G", [1, 3, 4, 8, 16])
def test_fast_path_head_dims_64_and_256(device, dtype, D, bs, G):
    """The fast path at head dims 64 (8 lanes per row) and 256 (32 lanes):
    contexts up to 32k (two-level merges), an empty and a one-token sequence,
    block sizes 16 and 32, G = 16 as two sub-groups of 8."""
    lens = [1, 17, 300, 4097, 32768, 0]
    kvh = 2 if G <= 8 else 1
    print(f"decode fast path D={D} bs={bs} G={G} {dtype}", flush=True)
    args = make_inputs(len(lens), G * kvh, kvh, D, lens, bs, dtype, device, seed=D * 100 + bs + G)
    q, kc, vc, bt, sl, scale, mb = args
    check(run(*args, bs), q, kc, vc, bt, sl, scale)


@pytest.mark.parametrize("D", [64, 256])
def test_fast_path_head_dims_scheduled(device, D):
    """More than 64 sequences at head dims 64 / 256: the schedule kernel's
    work list, config 2's head shape (32 q / 8 kv heads)."""
    g = torch.Generator().manual_seed(D)
    lens = torch.randint(0, 6000, (70,), generator=g).tolist()
    args = make_inputs(70, 32, 8, D, lens, 16, torch.bfloat16, device, seed=D + 1)
    q, kc, vc, bt, sl, scale, mb = args
    check(run(*args, 16), q, kc, vc, bt, sl, scale)


def test_group_of_16_scheduled_path(device):
    """G = 16 with more than 64 sequences (the schedule kernel's work list)."""
    g = torch.Generator().manual_seed(16)
    lens = torch.randint(0, 6000, (70,), generator=g).tolist()
    args = make_inputs(70, 32, 2, 128, lens, 16, torch.bfloat16, device, seed=160)
    q, kc, vc, bt, sl, scale, mb = args
    check(run(*args, 16), q, kc, vc, bt, sl, scale)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("G", [5, 8])
@pytest.mark.parametrize("bs", [64, 128, 256])
def test_one_pass_units_large_blocks(device, dtype, G, bs):
    """Head dim 128 with 5-8 heads per group runs as one-pass matrix-core
    units at every fast-path block size (a 16-token step inside a block of up
    to 256 tokens): contexts inside one block, across blocks and partitions,
    and rows past the context holding NaN."""
    lens = [1, 300, 1100, 5000, 17]
    q, kc, vc, bt, sl, scale, mb = make_inputs(len(lens), G * 2, 2, 128, lens, bs, dtype, device,
                                               seed=G * bs)
    for i, n in enumerate(lens):
        if n % bs:
            b = int(bt[i, (n - 1) // bs])
            kc[b, :, n % bs:, :] = float("nan")
            vc[b, :, n % bs:, :] = float("nan")
    check(run(q, kc, vc, bt, sl, scale, mb, bs), q, kc, vc, bt, sl, scale)


@pytest.mark.parametrize("lens", [[1025], [2049], [100, 1025, 3000, 5000, 17]])
def test_two_level_merge_one_pass_units(device, lens):
    """The two-level merge of the one-pass units (8 heads per group): 64- and
    128-token partitions, groups of 16 with a last group of one."""
    args = make_inputs(len(lens), 64, 8, 128, lens, 16, torch.bfloat16, device, seed=sum(lens) + 1)
    q, kc, vc, bt, sl, scale, mb = args
    check(run(*args, 16), q, kc, vc, bt, sl, scale)


@pytest.mark.parametrize("lens", [[1024], [1025], [2048], [2049], [100, 1025, 3000, 5000, 17]])
def test_two_level_merge_group_boundaries(device, lens):
    """A (sequence, kv-head) with more than 16 partitions merges in two
    levels: groups of 16, then the group results. One sequence (8 units) takes
    64-token partitions, so the lengths sit at the group boundaries: 16
    partitions (one level), 17 (the last group has one partition, published as
    its group's result), 32, 33; then a mix of one- and two-level units
    (128-token partitions)."""
    args = make_inputs(len(lens), 32, 8, 128, lens, 16, torch.bfloat16, device, seed=sum(lens))
    q, kc, vc, bt, sl, scale, mb = args
    check(run(*args, 16), q, kc, vc, bt, sl, scale)


@pytest.mark.parametrize("num_heads", [4, 16])
def test_two_level_merge_many_groups(device, num_heads):
    """1025 partitions of 64 tokens in one unit: 65 group results, so the
    second level reads them in two 64-lane chunks. With 8 heads per kv head a
    lane merges two (head, chunk) pairs, the second reading the chunk weights
    again."""
    args = make_inputs(1, num_heads, 2, 128, [65537], 16, torch.bfloat16, device, seed=7)
    q, kc, vc, bt, sl, scale, mb = args
    check(run(*args, 16), q, kc, vc, bt, sl, scale)


def test_two_level_merge_scheduled_path(device):
    """More than 64 sequences (the work list built by the schedule kernel):
    70 units with 256-token partitions, up to 32 of them per unit."""
    g = torch.Generator().manual_seed(70)
    lens = torch.randint(1, 8193, (70,), generator=g).tolist()
    lens[3] = 8192
    args = make_inputs(70, 4, 1, 128, lens, 16, torch.bfloat16, device, seed=70)
    q, kc, vc, bt, sl, scale, mb = args
    check(run(*args, 16), q, kc, vc, bt, sl, scale)


def test_2048_token_partitions_span_128_blocks(device):
    """A 32769-token context in a table 2049 blocks wide with 80 units and 2
    query heads per kv head: 17 partitions of 2048 tokens each, 128 blocks of
    16 (two block ids per lane). Short and empty sequences share the batch."""
    lens = [32769, 5000, 17, 1, 2048, 2049, 4097, 100, 0, 9000]
    args = make_inputs(len(lens), 16, 8, 128, lens, 16, torch.bfloat16, device, seed=2048)
    q, kc, vc, bt, sl, scale, mb = args
    assert mb == 2049
    check(run(*args, 16), q, kc, vc, bt, sl, scale)


def test_partition_halved_for_short_contexts(device):
    """A table 224 blocks wide (3584 tokens) makes the host take 1024-token
    partitions for 48 x 8 units; the actual contexts (256 .. 2048) give fewer
    than 1024 items at that length, so the kernel halves the partition (here
    to 256) from seq_lens alone."""
    g = torch.Generator().manual_seed(48)
    lens = torch.randint(256, 2049, (48,), generator=g).tolist()
    q, kc, vc, bt, sl, scale, mb = make_inputs(48, 32, 8, 128, lens, 16, torch.bfloat16, device,
                                               seed=48)
    btw = torch.zeros(48, 224, dtype=torch.int32, device=device)
    btw[:, :mb] = bt
    out = run(q, kc, vc, btw, sl, scale, 224, 16)
    check(out, q, kc, vc, btw, sl, scale)


def test_output_shape_and_int64_tables_raise(device):
    args = make_inputs(4, 8, 8, 128, [10] * 4, 16, torch.float16, device)
    q, kc, vc, bt, sl, scale, mb = args
    out = run(*args, 16)
    assert out.shape == (4, 8, 128)
    with pytest.raises(RuntimeError):
        pk.paged_attention_forward(torch.zeros_like(q), q, kc, vc, bt.to(torch.int64), sl, scale,
                                   16, mb)


def test_seq_len_zero_and_one(device):
    args = make_inputs(3, 8, 2, 128, [1, 40, 1], 16, torch.bfloat16, device)
    q, kc, vc, bt, sl, scale, mb = args
    sl = torch.tensor([1, 0, 1], dtype=torch.int32, device=device)
    out = run(q, kc, vc, bt, sl, scale, mb, 16)
    assert torch.count_nonzero(out[1]) == 0
    for s in (0, 2):   # one token: the output is that token's value row, exactly
        for h in range(8):
            assert torch.equal(out[s, h], vc[bt[s, 0], h // 4, 0])


def test_block_table_permutation_is_bit_invariant(device):
    args = make_inputs(4, 32, 8, 128, [100, 700, 1500, 3000], 16, torch.bfloat16, device, seed=3)
    q, kc, vc, bt, sl, scale, mb = args
    a = run(q, kc, vc, bt, sl, scale, mb, 16)
    perm = torch.randperm(kc.size(0), generator=torch.Generator().manual_seed(5)).to(device)
    kc2, vc2 = torch.empty_like(kc), torch.empty_like(vc)
    kc2[perm] = kc
    vc2[perm] = vc
    b = run(q, kc2, vc2, perm[bt.long()].to(torch.int32), sl, scale, mb, 16)
    assert torch.equal(a, b)


def test_strided_query_and_out(device):
    args = make_inputs(5, 16, 4, 128, [33, 64, 65, 400, 2000], 16, torch.bfloat16, device, seed=11)
    q, kc, vc, bt, sl, scale, mb = args
    # (H, S, D) storage viewed as (S, H, D): strides (D, S*D, 1)
    qt = q.transpose(0, 1).contiguous().transpose(0, 1)
    out = torch.full((16, 5, 128), float("nan"), dtype=q.dtype, device=device).transpose(0, 1)
    pk.paged_attention_forward(out, qt, kc, vc, bt, sl, scale, 16, mb)
    torch.cuda.synchronize()
    check(out, q, kc, vc, bt, sl, scale)


def test_tiny_golden_vector(device):
    gold = np.load("tests/golden/tiny.npz")
    t = lambda a: torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(device)  # noqa: E731
    q, kc, vc = t(gold["q"]), t(gold["k_cache"]), t(gold["v_cache"])
    bt = torch.from_numpy(gold["block_tables"]).to(device)
    sl = torch.from_numpy(gold["seq_lens"]).to(device)
    out = run(q, kc, vc, bt, sl, float(gold["scale"]), bt.size(1), kc.size(2))
    assert max_abs(out, gold["out"]) <= ATOL[torch.bfloat16]


def test_config1_store_then_decode_matches_golden(device):
    w = workloads.config1(device)
    gold = np.load("tests/golden/cfg1.npz")
    assert sha(bits(w.query), bits(w.store_k), bits(w.store_v), w.block_tables.cpu().numpy(),
               w.store_positions.cpu().numpy()) == str(gold["inputs_sha"])
    pk.paged_kv_store(w.k_cache, w.v_cache, w.store_k, w.store_v, w.store_tables, w.store_positions)
    out = run(w.query, w.k_cache, w.v_cache, w.block_tables, w.seq_lens, w.scale,
              w.max_blocks_per_seq, w.block_size)
    want = O.bits_to_f32(gold["out_bits"], "f16").astype(np.float64)
    # the golden output is itself rounded to fp16: allow one extra half-ulp
    assert max_abs(out, want) <= ATOL[torch.float16] + 2 ** -11
    check(out, w.query, w.k_cache, w.v_cache, w.block_tables, w.seq_lens, w.scale)


def test_config2_store_then_decode(device):
    w = workloads.config2(device)
    pk.paged_kv_store(w.k_cache, w.v_cache, w.store_k, w.store_v, w.store_tables, w.store_positions)
    out = run(w.query, w.k_cache, w.v_cache, w.block_tables, w.seq_lens, w.scale,
              w.max_blocks_per_seq, w.block_size)
    err = check(out, w.query, w.k_cache, w.v_cache, w.block_tables, w.seq_lens, w.scale)
    print(f"cfg2 max-abs {err:.2e}")


def test_config4_long_context_with_cow_fork(device):
    w = workloads.config4(device)
    pk.paged_kv_store(w.k_cache, w.v_cache, w.store_k, w.store_v, w.store_tables, w.store_positions)
    pk.copy_blocks(w.k_cache, w.v_cache, w.cow_pairs)
    out = run(w.query, w.k_cache, w.v_cache, w.block_tables, w.seq_lens, w.scale,
              w.max_blocks_per_seq, w.block_size)
    for (src, dst) in w.cow_pairs:
        assert torch.equal(w.k_cache[src], w.k_cache[dst]) and torch.equal(w.v_cache[src], w.v_cache[dst])
    # children (rows 8, 9) read a copied last block: identical to their parents
    assert torch.equal(out[8], out[6]) and torch.equal(out[9], out[7])
    # every row (8 parents of 8k-32k tokens, 2 children) against the oracle
    want = oracle_decode(w.query, w.k_cache, w.v_cache, w.block_tables, w.seq_lens, w.scale)
    err = max_abs(out, want)
    print(f"cfg4 max-abs {err:.2e} over all {out.size(0)} rows")
    assert err <= ATOL[torch.bfloat16]


@pytest.mark.parametrize("num_seqs", [6, 70])
def test_workspace_reuse_across_calls(device, num_seqs):
    """The fast path merges partitions in the last-arriving wave through
    counters in the workspace that every call leaves at zero: a workspace
    zeroed once and reused across calls with other lengths (other partition
    counts) stays right. 70 sequences take the scheduled (work-list) path,
    6 the in-kernel one."""
    g = torch.Generator().manual_seed(num_seqs)
    top = 4000 if num_seqs < 64 else 1500
    lens_a = torch.randint(1, top + 1, (num_seqs,), generator=g).tolist()
    lens_b = torch.randint(1, top + 1, (num_seqs,), generator=g).tolist()
    lens_a[0], lens_b[1] = top, top
    args = make_inputs(num_seqs, 32, 8, 128, [top] * num_seqs, 16, torch.bfloat16, device,
                       seed=21)
    q, kc, vc, bt, sl, scale, mb = args
    ws = torch.zeros(pk.attention_workspace_bytes(num_seqs, 32, 8, 128, 16, mb),
                     dtype=torch.uint8, device=device)
    for lens in (lens_a, lens_b, lens_a):
        sl = torch.tensor(lens, dtype=torch.int32, device=device)
        out = torch.full_like(q, float("nan"))
        pk.paged_attention_forward(out, q, kc, vc, bt, sl, scale, 16, mb, workspace=ws)
        torch.cuda.synchronize()
        check(out, q, kc, vc, bt, sl, scale)


def test_workspace_shared_across_shapes_and_ops(device):
    """One zero-filled workspace serves decode calls whose layouts differ
    (sequence count, table width -> partition count, work-list and partial
    offsets) and a chunked-prefill call in between: the merge counters sit in a
    fixed region that partial results never overwrite, and each call leaves
    its counters at zero. (A serving engine calls with a new shape every step.)"""
    from tests.test_gpu_prefill import make_case, oracle as prefill_oracle
    shapes = [(70, 1500, 94), (6, 4000, 250), (33, 700, 44), (70, 1500, 94), (64, 2500, 157)]
    need = max(pk.attention_workspace_bytes(n, 32, 8, 128, 16, mb) for n, _, mb in shapes)
    pq, pkc, pvc, pbt, pcu, pctx, pmb, pmq = make_case(device, [2500, 900], [200, 64], seed=41)
    need = max(need, pk.prefill_workspace_bytes(2, int(pq.size(0)), 32, 128, pmq, pmb * 16))
    ws = torch.zeros(need, dtype=torch.uint8, device=device)
    for i, (n, top, mb) in enumerate(shapes):
        g = torch.Generator().manual_seed(100 + i)
        lens = torch.randint(1, top + 1, (n,), generator=g).tolist()
        lens[0] = top
        q, kc, vc, bt, sl, scale, mbi = make_inputs(n, 32, 8, 128, lens, 16, torch.bfloat16,
                                                    device, seed=50 + i)
        assert mbi <= mb
        btw = torch.zeros(n, mb, dtype=torch.int32, device=device)
        btw[:, :mbi] = bt
        out = torch.full_like(q, float("nan"))
        pk.paged_attention_forward(out, q, kc, vc, btw, sl, scale, 16, mb, workspace=ws)
        torch.cuda.synchronize()
        check(out, q, kc, vc, btw, sl, scale)
        if i == 1:
            pout = torch.full_like(pq, float("nan"))
            pk.paged_prefill_attention(pout, pq, pkc, pvc, pbt, pcu, pctx, 1 / math.sqrt(128), 16,
                                       pmb, pmq, workspace=ws)
            torch.cuda.synchronize()
            want = prefill_oracle(pq, pkc, pvc, pbt, pcu, pctx, 1 / math.sqrt(128))
            assert max_abs(pout, want) <= ATOL[torch.bfloat16]
