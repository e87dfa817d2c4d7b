"""CPU check of the decode fast path's lane algebra (decode_attention.hip,
decode_fast_item) for head dims 64, 128 and 256 and group sizes 1-8.

A numpy model of one wave64 runs pass 1's reduce-scatter exactly as the
kernel orders it, with the cross-lane operations defined from the CDNA
instruction set:
- row_ror:8      lane i of a 16-lane row reads lane (i + 8) mod 16;
- row_half_mirror lane i of an 8-lane half row reads lane 7 - i;
- quad_perm       [2,3,0,1] reads i ^ 2, [1,0,3,2] reads i ^ 1;
- v_permlane16_swap(A, B): for each pair of 16-lane rows (2k, 2k + 1), A of
  row 2k + 1 and B of row 2k are exchanged;
- v_permlane32_swap: the same for 32-lane halves.
Each lane starts from partial dot products of its 8 head-dim elements
(integers, so every sum is exact) and must end holding the full dot product
of the (query head, token) pair the kernel stores it as: head hmask(lane),
token slot tokhi(lane) | e. The row combine of pass 3 (sum over the token
rows of the wave) is checked the same way. A planted mistake (the D 256
stage coordinates taken from the 16-lane basis alone) fails."""
import numpy as np
import pytest


def bfly_coord(j, s):
    j2 = (j >> 2) & 1
    return {1: (j >> 3) & 1, 2: j2, 3: ((j >> 1) & 1) ^ j2}.get(s, (j & 1) ^ j2)


def stage_coord(D, j, k, planted=False):
    if D == 64:
        return bfly_coord(j, k + 2)
    if D == 128:
        return bfly_coord(j, k + 1)
    if k < 4:
        return bfly_coord(j & 15, k + 1)
    return 0 if planted else (j >> 4) & 1


def ilog2(x):
    return x.bit_length() - 1


def pow2ceil(x):
    p = 1
    while p < x:
        p *= 2
    return p


def src_lane(ctrl, i):
    """Lane whose value lane i reads under a DPP control."""
    if ctrl == "ror8":
        return (i & ~15) | (((i & 15) + 8) & 15)
    if ctrl == "half_mirror":
        return (i & ~7) | (7 - (i & 7))
    if ctrl == "xor2":
        return i ^ 2
    return i ^ 1


def dpp(ctrl, x):
    return x[[src_lane(ctrl, i) for i in range(64)]]


def permlane_swap(width, a, b):
    a, b = a.copy(), b.copy()
    for i in range(64):
        if (i // width) % 2 == 1:   # odd row: its A swaps with B of the row below
            a[i], b[i - width] = b[i - width], a[i]
    return a, b


def stage_ctrl(D, k):
    seq = ["half_mirror", "xor2", "xor1"] if D == 64 else ["ror8", "half_mirror", "xor2", "xor1"]
    return seq[k] if k < len(seq) else "swap16"


def run_wave(D, G, rng, planted=False):
    LPT, TPL = D // 8, 64 // (D // 8)
    NL = 16 // TPL
    NLB, NS = ilog2(NL), ilog2(LPT)
    GP = pow2ceil(G)
    LGP = ilog2(GP)
    NV = NL * GP
    NB = ilog2(NV)
    NH = min(NB, NS)
    HELD = NV >> NH
    NTS = NH - LGP if NH > LGP else 0
    lanes = np.arange(64)
    r, j = lanes // LPT, lanes % LPT
    q = rng.integers(-9, 10, size=(G, D))             # query heads of the group
    k = rng.integers(-9, 10, size=(16, D))            # the 16 tokens of a step
    hmask = np.zeros(64, np.int64)
    tokhi = np.zeros(64, np.int64)
    for ln in range(64):
        for kk in range(min(LGP, NS)):
            hmask[ln] |= stage_coord(D, j[ln], kk, planted) << (LGP - 1 - kk)
        for t in range(NTS):
            tokhi[ln] |= stage_coord(D, j[ln], LGP + t, planted) << (NLB - 1 - t)
    # v[slot h * NL + i][lane]: q slot h holds head h ^ hmask, token slot i is row i * TPL + r
    v = np.zeros((NV, 64), np.int64)
    for ln in range(64):
        cols = slice(j[ln] * 8, j[ln] * 8 + 8)
        for h in range(GP):
            hh = h ^ hmask[ln]
            for i in range(NL):
                if hh < G:
                    v[h * NL + i, ln] = int(q[hh, cols] @ k[i * TPL + r[ln], cols])
    for kk in range(NS):
        cnt = NV >> kk if (NV >> kk) >= 2 else 1
        ctrl = stage_ctrl(D, kk)
        upper = np.array([stage_coord(D, j[ln], kk, planted) != 0 for ln in range(64)])
        free = kk < LGP
        if cnt >= 2:
            half = cnt // 2
            for p in range(half):
                if ctrl == "swap16":
                    a, b = permlane_swap(16, v[p], v[p + half])
                    v[p] = a + b
                elif free:
                    v[p] = v[p] + dpp(ctrl, v[p + half])
                else:
                    send = np.where(upper, v[p], v[p + half])
                    keep = np.where(upper, v[p + half], v[p])
                    v[p] = keep + dpp(ctrl, send)
        else:
            if ctrl == "swap16":
                a, b = permlane_swap(16, v[0], v[0])
                v[0] = a + b
            else:
                v[0] = v[0] + dpp(ctrl, v[0])
    checked = 0
    for ln in range(64):
        h = hmask[ln]
        for e in range(HELD):
            ti = tokhi[ln] | e
            tok = ti * TPL + r[ln]
            if h < G:
                if v[e, ln] != int(q[h] @ k[tok]):
                    return False, checked
                checked += 1
    # every (head, token) pair of the step is held by some lane
    held = {(hmask[ln], (tokhi[ln] | e) * TPL + r[ln]) for ln in range(64) for e in range(HELD)
            if hmask[ln] < G}
    return len(held) == G * 16, checked


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("G", list(range(1, 9)))
def test_reduce_scatter_holds_exact_dot_products(D, G):
    ok, n = run_wave(D, G, np.random.default_rng(D * 10 + G))
    assert ok and n > 0


@pytest.mark.parametrize("D", [64, 128, 256])
def test_row_combine_sums_the_token_rows(D):
    """Pass 3: lanes equal in j hold accumulators of their own token rows;
    row_ror:8 (D 64), permlane16_swap (D <= 128) and permlane32_swap (all)
    leave every lane with the sum over all TPL rows."""
    LPT, TPL = D // 8, 64 // (D // 8)
    rng = np.random.default_rng(D)
    x = rng.integers(-100, 100, size=64)
    y = x.copy()
    if TPL >= 8:
        y = y + dpp("ror8", y)
    if TPL >= 4:
        a, b = permlane_swap(16, y, y)
        y = a + b
    a, b = permlane_swap(32, y, y)
    y = a + b
    want = np.array([x[np.arange(64) % LPT == ln % LPT].sum() for ln in range(64)])
    assert np.array_equal(y, want)


def test_planted_stage_coordinate_fails():
    ok, _ = run_wave(256, 8, np.random.default_rng(5), planted=True)
    assert not ok
