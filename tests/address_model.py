"""CPU address model of the device writes of the paged-kernel path.

Test infrastructure (like oracle/): it restates, in numpy, the index
arithmetic by which each kernel of nanopd_amd/csrc/ chooses its work item and
the addresses it stores to, and checks every store (and the LDS / work-list
indices) against the sizes of the buffers the host passes. It executes
nothing on a GPU; the kernels' arithmetic is not computed, only where it
goes. Cited lines are those of the kernel sources.

Kernels covered (the FP8 and 2-byte pools share their addressing):
- qk_norm_rope_store_kernel (qk_norm_rope.hip:55-111): q_out rows, cache rows
  by slot;
- pack_metadata_kernel (metadata.hip:24-98): its output arrays;
- decode_fast_kernel (head dims 64, 128, 256) with its inline work list or
  decode_schedule_kernel's, decode_fast_item's output, partial, group-slot,
  (m, l) and counter stores, merge_unit_fast's reads and stores, and the
  dynamic LDS of pass 1-3;
- prefill_kernel's work list / fixed grid (prefill_attention.hip:164-288),
  its zero rows, partial records, counters and output rows (:290-660);
- copy_blocks_kernel (copy_blocks.hip:15-29).
Host-side choices (partition, grid, workspace layout) are restated from the
entry points (decode_attention.hip:1192-1512, prefill_attention.hip:686-851);
the workspace sizes are asked of the built library itself.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

K_COUNTER_BYTES = 1 << 20
K_MAX_COUNTERS = K_COUNTER_BYTES // 4

# decode_attention.hip constants
FAST_MAX_PARTITION = 2048
FAST_MAX_SCORES = 4096
FAST_MIN_ITEMS = 1280
FAST_MIN_ITEMS_ACTUAL = 1024
INLINE_SCHED_MAX = 64
SCHED_MAX_SEQS = 4096
MERGE_GROUP = 16
RING = 2


V_ROW = 128 + 16   # elements per row of the MFMA P.V steps' V tile in LDS (kVRow)


WIDE_GROUP = 16    # kWideGroup: heads of a decode_wide_item unit
WIDE_MIN_G_2B = 5  # kWideMinG2B: 2-byte groups of 5-8 heads run as decode_wide_item units


def wide_item(fp8: bool, g: int, d: int = 128) -> bool:
    """wide_item: at head dim 128, 16-head units, every FP8 group, and 2-byte
    groups of 5-8 heads."""
    return d == 128 and g <= WIDE_GROUP and (fp8 or g >= WIDE_MIN_G_2B)


K_ROW = 128 + 8        # kKRow: elements per row of the K tile in LDS
WIDE_K_LDS_FROM = 12   # kWideKLdsFrom: 2-byte units of more heads stage K through LDS


def wide_k_lds(fp8: bool, g: int) -> bool:
    """decode_wide_item's kKLds for a unit of g heads."""
    return not fp8 and g > WIDE_K_LDS_FROM


WIDE_LDS_BYTES = max(16 * V_ROW * 2 + 16 * K_ROW * 2, (WIDE_GROUP * 128 + WIDE_GROUP) * 4,
                     64 * WIDE_GROUP * 4)
"""kWideLdsBytes: V and K tiles, then O hand-off + 1/l, then merge weights, each from byte 0."""
WIDE_RING_2B = 2   # NPD_WIDE_RING_2B: steps of K and V in flight, 16-head units
WIDE_RING_FP8 = 4  # NPD_WIDE_RING_FP8


def wide_ring(fp8: bool) -> int:
    """decode_attention.hip wide_ring."""
    return WIDE_RING_FP8 if fp8 else WIDE_RING_2B


def ring_of(D: int, G: int = 1, fp8: bool = False) -> int:
    """decode_attention.hip ring_of (wide_ring for decode_wide_item units): steps in flight."""
    if wide_item(fp8, G, D):
        return wide_ring(fp8)
    return 2 * RING if D == 64 else RING

# prefill_attention.hip constants
KT = 64
SPLIT_STEPS = 16
MAX_SPLITS = 8
MAX_BLOCKS_LDS = 16384
REC_ML = 2 * 64 * 2


def rec_o(d: int) -> int:
    """Floats of one wave's partial O record at head dim d (rec_o)."""
    return d // 8 * 2 * 64 * 2
WAVE_ROWS = 32


class OutOfBounds(AssertionError):
    pass


@dataclass
class Buf:
    """A device buffer as the host passes it: its size in bytes."""
    name: str
    nbytes: int


@dataclass
class Writes:
    """Byte ranges [lo, hi) stored to, per buffer; check() raises on any range
    outside its buffer. Reads that must stay inside a buffer go through
    read()."""
    ranges: dict = field(default_factory=dict)
    errors: list = field(default_factory=list)
    count: int = 0

    def add(self, buf: Buf, lo, hi, what: str) -> None:
        lo = np.asarray(lo, dtype=np.int64).ravel()
        hi = np.asarray(hi, dtype=np.int64).ravel()
        if lo.size == 0:
            return
        self.count += lo.size
        bad = (lo < 0) | (hi > buf.nbytes) | (hi < lo)
        if bad.any():
            i = int(np.argmax(bad))
            self.errors.append(f"{what}: [{lo[i]}, {hi[i]}) outside {buf.name} of "
                               f"{buf.nbytes} bytes ({int(bad.sum())} ranges)")
        r = self.ranges.setdefault(buf.name, [buf.nbytes, np.iinfo(np.int64).max, -1])
        r[1] = min(r[1], int(lo.min()))
        r[2] = max(r[2], int(hi.max()))

    def read(self, buf: Buf, lo, hi, what: str) -> None:
        self.add(buf, lo, hi, "read " + what)

    def index(self, idx, limit: int, what: str) -> None:
        """Indices into an array of `limit` entries (LDS, counters)."""
        idx = np.asarray(idx, dtype=np.int64).ravel()
        if idx.size and ((idx < 0) | (idx >= limit)).any():
            bad = idx[(idx < 0) | (idx >= limit)]
            self.errors.append(f"{what}: index {int(bad[0])} outside [0, {limit})")

    def check(self) -> None:
        if self.errors:
            raise OutOfBounds("; ".join(self.errors[:8]))


def _ceil(a, b):
    return -(-a // b)


def pow2ceil(x: int) -> int:
    p = 1
    while p < x:
        p *= 2
    return p


# ---------------------------------------------------------------------------
# Fused prologue (qk_norm_rope.hip:55-111)
# ---------------------------------------------------------------------------

def prologue(W: Writes, q_out: Buf, k_cache: Buf, v_cache: Buf, slots: np.ndarray, T: int, H: int,
             KV: int, num_blocks: int, bs: int, q_stride: int, fp8: bool, D: int = 128) -> None:
    """One wave per (token, head) row; q rows to q_out, k / v rows by slot."""
    if T == 0:
        return
    t = np.arange(T, dtype=np.int64)
    hh = np.arange(H, dtype=np.int64)
    lo = ((t[:, None] * q_stride + hh[None, :] * D) * 2)
    W.add(q_out, lo, lo + 2 * D, "prologue q_out")
    slot = np.asarray(slots[:T], dtype=np.int64)
    store = (slot >= 0) & (slot < num_blocks * bs)
    blk = np.where(store, slot // bs, 0)
    off = np.where(store, slot - blk * bs, 0)
    elt = 1 if fp8 else 2
    kh = np.arange(KV, dtype=np.int64)
    e = ((blk[store][:, None] * KV + kh[None, :]) * bs + off[store][:, None]) * D
    for buf in (k_cache, v_cache):
        W.add(buf, e * elt, (e + D) * elt, "prologue cache row")


# ---------------------------------------------------------------------------
# Ragged metadata (metadata.hip:24-98)
# ---------------------------------------------------------------------------

def pack_metadata(W: Writes, out: dict, desc: np.ndarray, num_seqs: int, total_q: int,
                  max_bps: int) -> None:
    """out: Bufs cu, seq_lens, tables, positions, slots, token_seq."""
    ql = np.maximum(desc[0::3][:num_seqs], 0)
    nq = min(int(ql.sum()), total_q)
    W.add(out["cu"], 0, 4 * (num_seqs + 1), "metadata cu_seqlens")
    if num_seqs:
        W.add(out["seq_lens"], 0, 4 * num_seqs, "metadata seq_lens")
        W.add(out["tables"], 0, 4 * num_seqs * max_bps, "metadata tables")
    if nq:
        for k in ("positions", "slots", "token_seq"):
            W.add(out[k], 0, 4 * nq, f"metadata {k}")


# ---------------------------------------------------------------------------
# Decode attention, fast path
# ---------------------------------------------------------------------------

def use_fast_path(D: int, bs: int, S: int) -> bool:
    """decode_attention.hip use_fast_path."""
    if S > SCHED_MAX_SEQS:
        return False
    if D == 128:
        return bs % 16 == 0 and bs <= 256 and (bs & (bs - 1)) == 0
    return D in (64, 256) and bs in (16, 32)


def choose_partition(S, H, KV, D, bs, max_ctx, fp8) -> int:
    """decode_attention.hip:1201-1219."""
    units = S * KV
    if use_fast_path(D, bs, S):
        gp = pow2ceil(H // KV)
        wide = wide_item(fp8, H // KV, D)
        ps = FAST_MAX_PARTITION
        while ps >= 64:
            if ps <= bs:
                return bs
            if (ps * gp <= FAST_MAX_SCORES or wide) and units * _ceil(max_ctx, ps) >= FAST_MIN_ITEMS:
                return ps
            ps >>= 1
        return bs if bs > 64 else 64
    return 512 if units * _ceil(max_ctx, 512) >= 4096 else 256


def fast_min_partition(ps: int, bs: int) -> int:
    """decode_attention.hip fast_min_partition."""
    lo = max(ps // 4, 64)
    lo = max(lo, bs)
    return min(lo, ps)


def kv_split_of(H: int, KV: int, D: int = 128, bs: int = 16, S: int = 1) -> int:
    """decode_attention.hip kv_split_of: at head dim 128 with blocks of 16 or
    32 (the fast path) a group of more than 8 heads runs as the fewest equal
    units of at most 16 heads; other groups of more than 8 query heads as the
    smallest number of equal groups of at most 8."""
    g = H // KV
    cap = WIDE_GROUP if g > 8 and D == 128 and bs in (16, 32) and use_fast_path(D, bs, S) else 8
    k = 1
    while k < g and (g // k > cap or g % k):
        k += 1
    return k


def merge_groups(units: int, parts: int) -> int:
    """decode_attention.hip:1346-1349 (fast path)."""
    ng = _ceil(parts, MERGE_GROUP)
    return ng if parts > MERGE_GROUP and units * (1 + ng) <= K_MAX_COUNTERS else 0


@dataclass
class DecodeLaunch:
    S: int
    H: int
    KV: int                 # kv heads of the work units (pool kv heads * kv_split)
    bs: int
    max_bps: int
    fp8: bool
    kv_split: int = 1
    partition: int = 0
    min_partition: int = 0
    max_parts: int = 0
    max_groups: int = 0
    grid: int = 0
    part_off: int = 0       # bytes: partial accumulators
    ml_off: int = 0         # bytes: (m, l)
    items_off: int = K_COUNTER_BYTES + 16
    lds_floats: int = 0     # dynamic LDS of the launch, floats

    @property
    def G(self) -> int:
        return self.H // self.KV

    @property
    def units(self) -> int:
        return self.S * self.KV


def decode_host(S, H, KV, bs, max_bps, fp8, D=128) -> DecodeLaunch:
    """The host choices of attention_impl (decode_attention.hip:1441-1511)."""
    assert use_fast_path(D, bs, S), "model covers the fast path"
    split = kv_split_of(H, KV, D, bs, S)
    KV *= split
    L = DecodeLaunch(S, H, KV, bs, max_bps, fp8, split)
    max_ctx = bs * max_bps
    L.partition = choose_partition(S, H, KV, D, bs, max_ctx, fp8)
    L.min_partition = fast_min_partition(L.partition, bs)
    L.max_parts = _ceil(max_ctx, L.min_partition)
    units = S * KV
    L.part_off = _ceil(K_COUNTER_BYTES + 16 + units * L.max_parts * 8, 256) * 256
    L.max_groups = merge_groups(units, L.max_parts)
    G = H // KV
    L.ml_off = L.part_off + units * (L.max_parts + L.max_groups) * G * D * 4
    n = units * _ceil(max_ctx, L.partition)
    if L.min_partition < L.partition:
        h = min(units * L.max_parts, 2 * FAST_MIN_ITEMS_ACTUAL)
        n = max(n, h)
    if split > 1 and S <= INLINE_SCHED_MAX:
        n = _ceil(n, 8 * split) * 8 * split
    L.grid = n
    gp = pow2ceil(G)
    t = L.partition + 16 * ring_of(D, G, fp8)
    if wide_item(fp8, G, D):
        L.lds_floats = WIDE_LDS_BYTES // 4
    else:
        L.lds_floats = t * gp
    return L


def _nth(mask: np.ndarray, k: np.ndarray) -> np.ndarray:
    """Lane of the k-th set bit of a 64-lane mask; -1 where there is none (the
    kernel's count-trailing-zeros of an empty ballot)."""
    lanes = np.flatnonzero(mask)
    out = np.full(k.shape, -1, dtype=np.int64)
    ok = k < lanes.size
    out[ok] = lanes[k[ok]]
    return out


def decode_items(L: DecodeLaunch, seq_lens: np.ndarray):
    """(unit, part, ps) of every workgroup that runs an item, as the kernel
    derives them (decode_attention.hip:1010-1095; more than 64 sequences: the
    list decode_schedule_kernel writes, :1105-1172). Returns arrays and the
    work-list length."""
    S, KV = L.S, L.KV
    cap = L.max_bps * L.bs
    c = np.minimum(np.asarray(seq_lens[:S], dtype=np.int64), cap)
    if S > INLINE_SCHED_MAX:
        ps = L.partition
        np_ = np.where(c <= 0, 1, _ceil(c, ps))
        order = sorted(range(S), key=lambda s: -min(int(np_[s]), 1023))   # bins, stable enough
        units, parts = [], []
        for s in order:
            for kh in range(KV):
                units.extend([s * KV + kh] * int(np_[s]))
                parts.extend(range(int(np_[s])))
        n = len(units)
        units = np.asarray(units, dtype=np.int64)[: L.grid]
        parts = np.asarray(parts, dtype=np.int64)[: L.grid]
        return units, parts, np.full(units.shape, ps), n
    valid = np.ones(S, dtype=bool)
    ps = L.min_partition
    p = L.partition
    while p > L.min_partition:
        n = np.where(c > 0, _ceil(c, p), 1)
        if int(n.sum()) * KV >= FAST_MIN_ITEMS_ACTUAL:
            ps = p
            break
        p >>= 1
    full = np.where(c > 0, (c - 1) // ps, 0)
    bucket = np.where(c > 0, (c - full * ps + 15) >> 4, 0)
    maxfull = int(full.max()) if S else 0
    before = np.array([int(np.minimum(full, q).sum()) * KV for q in range(maxfull + 1)],
                      dtype=np.int64)
    nfull = int(before[maxfull]) if S else 0
    ids = np.arange(L.grid, dtype=np.int64)
    # blockIdx -> item id: every other full round of 256 reversed within each XCD
    xcd, pos = ids & 7, ids >> 3
    rnd = pos >> 5
    snake = ((rnd & 1) == 1) & ((rnd + 1) * 256 <= L.grid)
    ids = np.where(snake, ((rnd * 32 + (31 - (pos & 31))) << 3) | xcd, ids)
    assert np.array_equal(np.sort(ids), np.arange(L.grid)), "not a permutation"
    if L.kv_split > 1:
        # blockIdx -> item id: the units of one pool kv head 8 blockIdx apart
        span = 8 * L.kv_split
        q, rem = ids // span, ids % span
        ids = q * span + (rem & 7) * L.kv_split + (rem >> 3)
        assert np.array_equal(np.sort(ids), np.arange(L.grid)), "not a permutation"
    unit = np.full(ids.shape, -2, dtype=np.int64)   # -2: exits
    part = np.zeros(ids.shape, dtype=np.int64)
    # A: full partitions, level by level
    a = ids < nfull
    if a.any():
        lo = np.searchsorted(before[:maxfull], ids[a], side="right") - 1
        idl = ids[a] - before[lo]
        seq = np.empty(lo.shape, dtype=np.int64)
        for lv in np.unique(lo):
            sel = lo == lv
            seq[sel] = _nth(full > lv, idl[sel] // KV)
        unit[a] = np.where(seq >= 0, seq * KV + idl % KV, -1)
        part[a] = lo
    # B: last partitions by 16-token bucket, longest first
    b = ~a
    idb = ids[b] - nfull
    frm = np.array([int((valid & (bucket >= q)).sum()) * KV for q in range((ps >> 4) + 2)],
                   dtype=np.int64)
    run = idb < frm[0]
    ub = np.full(idb.shape, -2, dtype=np.int64)
    pb = np.zeros(idb.shape, dtype=np.int64)
    if run.any():
        x = idb[run]
        # largest q in [0, ps >> 4] with frm[q] > x (frm is non-increasing)
        lo = np.array([int(np.flatnonzero(frm[: (ps >> 4) + 1] > v).max()) for v in x],
                      dtype=np.int64) if x.size < 4096 else \
            np.sum(frm[None, : (ps >> 4) + 1] > x[:, None], axis=1) - 1
        x2 = x - frm[lo + 1]
        seq = np.empty(lo.shape, dtype=np.int64)
        for lv in np.unique(lo):
            sel = lo == lv
            seq[sel] = _nth(valid & (bucket == lv), x2[sel] // KV)
        ub[run] = np.where(seq >= 0, seq * KV + x2 % KV, -1)
        pb[run] = np.where(seq >= 0, full[np.maximum(seq, 0)], 0)
    unit[b] = ub
    part[b] = pb
    keep = unit != -2
    nitems = int(keep.sum())
    return unit[keep], part[keep], np.full(int(keep.sum()), ps), nitems


def decode(W: Writes, L: DecodeLaunch, out: Buf, ws: Buf, seq_lens: np.ndarray,
           out_stride_seq: int, out_stride_head: int, D: int = 128) -> None:
    """Every store of one decode launch (fast path)."""
    S, KV, G = L.S, L.KV, L.G
    units_total = L.units
    cap = L.max_bps * L.bs
    gp = pow2ceil(G)
    W.index([L.units - 1], K_MAX_COUNTERS, "decode unit counters")
    if S > INLINE_SCHED_MAX:
        # the schedule kernel: counters zeroed, item count, work list
        W.index([units_total * (1 + L.max_groups) - 1], K_MAX_COUNTERS, "decode schedule counters")
    unit, part, ps, nitems = decode_items(L, seq_lens)
    if S > INLINE_SCHED_MAX:
        W.add(ws, K_COUNTER_BYTES, K_COUNTER_BYTES + 8, "decode item count")
        W.add(ws, L.items_off, L.items_off + 8 * nitems, "decode work list")
        if nitems > L.grid:
            W.errors.append(f"decode: {nitems} items for a grid of {L.grid}")
    if (unit == -1).any():
        W.errors.append("decode: a workgroup derived no sequence (empty ballot)")
        return
    s = unit // KV
    kh = unit - s * KV
    W.index(s, S, "decode sequence of an item")
    ctx = np.minimum(np.asarray(seq_lens, dtype=np.int64)[s], cap)
    h = np.arange(G, dtype=np.int64)

    def out_rows(sel, what):
        lo = (s[sel][:, None] * out_stride_seq + (kh[sel][:, None] * G + h[None, :]) * out_stride_head) * 2
        W.add(out, lo, lo + 2 * D, what)

    empty = ctx <= 0
    out_rows(empty & (part == 0), "decode zero rows")
    nparts = np.where(empty, 0, _ceil(np.maximum(ctx, 1), ps))
    run = ~empty & (part < nparts)
    if ((~empty) & (part >= nparts)).any():
        pass   # such items return at once (decode_attention.hip:646)
    single = run & (nparts == 1)
    out_rows(single, "decode output rows")
    # LDS of the item: decode_fast_item's scores s_p[tl * GP + h];
    # decode_wide_item's V tile, O hand-off, 1/l and merge weights
    ntok = np.minimum(ctx - part * ps, ps)   # ps: per item
    ring = ring_of(D, L.G, L.fp8)
    nsteps = _ceil(_ceil(np.maximum(ntok, 0), 16), ring) * ring
    if run.any():
        tpad = L.partition + 16 * ring
        if wide_item(L.fp8, L.G, D):
            # one pass: the V tile s_vt[row * V_ROW + col] (2 bytes), then from
            # byte 0 the O hand-off s_o[h * D + d] (all 16 MFMA columns) and
            # 1/l s_il[n16] (4 bytes), then the merge weights s_w[lane * GP + h]
            W.index([2 * (15 * V_ROW + 127) + 1, 4 * (WIDE_GROUP * D + WIDE_GROUP - 1) + 3,
                     4 * (63 * gp + L.G - 1) + 3],
                    L.lds_floats * 4, "decode LDS V tile, O hand-off, 1/l, merge weights (bytes)")
            # the transposing reads: lane (g4, n16) at row 4*g4 + n16/4, col
            # nb*16 + 4*(n16%4) .. +3 (8 bytes)
            lane = np.arange(64)
            tr = 2 * (((lane >> 4) * 4 + ((lane & 15) >> 2)) * V_ROW + 4 * (lane & 3))
            W.index(tr[:, None] + 2 * 16 * np.arange(D // 16)[None, :] + 7, L.lds_floats * 4,
                    "decode LDS transposing V reads (bytes)")
            if wide_k_lds(L.fp8, L.G):
                # K tile after the V tile: writes of load i by lane (r, j) at
                # row i*TPL + r, chunk j; operand reads of S MFMA c by lane
                # (g4, n16) at row n16, chunk 4c + g4 (16 bytes each)
                k0 = 2 * 16 * V_ROW
                lpt = D // 8
                wr = (np.arange(4)[:, None] * (64 // lpt) + lane[None, :] // lpt) * K_ROW + 8 * (lane % lpt)
                rd = (lane[None, :] & 15) * K_ROW + 8 * (4 * np.arange(4)[:, None] + (lane[None, :] >> 4))
                assert (wr >= 0).all() and wr.max() // K_ROW == 15
                for x, what in ((wr, "writes"), (rd, "operand reads")):
                    W.index(k0 + 2 * x + 15, L.lds_floats * 4, f"decode LDS K tile {what} (bytes)")
                # every element of the 16 x 128 tile is written before it is read
                cover = np.zeros((16, K_ROW), dtype=bool)
                for row, col in zip((wr // K_ROW).ravel(), (wr % K_ROW).ravel()):
                    cover[row, col:col + 8] = True
                assert cover[:, :D].all() and not cover[:, D:].any()
        else:
            W.index(nsteps[run] * 16 * gp - 1, L.partition * gp + 16 * ring * gp, "decode LDS scores")
        nb = _ceil(ntok[run], L.bs)
        W.index(nb - 1, 128, "decode block ids per lane")
        # block-table reads of the partition
        b0 = part[run] * ps[run] // L.bs
        W.index(b0 + nb - 1, L.max_bps, "decode block-table column")
    multi = run & (nparts > 1)
    if not multi.any():
        return
    u = unit[multi]
    p = part[multi]
    n = nparts[multi]
    ubase = u * L.max_parts
    grouped = (L.max_groups > 0) & (n > MERGE_GROUP)
    ngroups = _ceil(n, MERGE_GROUP)
    g = p // MERGE_GROUP
    gsize = np.minimum(MERGE_GROUP, n - g * MERGE_GROUP)
    gbase = S * KV * L.max_parts + u * L.max_groups
    base = np.where(grouped & (gsize == 1), gbase + g, ubase + p)
    W.index(p, L.max_parts, "decode partition slot")
    acc_row = L.part_off + ((base[:, None] * G + h[None, :]) * D) * 4
    W.add(ws, acc_row, acc_row + 4 * D, "decode partial accumulators")
    ml = L.ml_off + ((base[:, None] * G + h[None, :]) * 2) * 4
    W.add(ws, ml, ml + 8, "decode partial (m, l)")
    # counters and merges (every item is taken to be the last to arrive)
    first_lvl = grouped & (gsize > 1)
    cidx = np.where(first_lvl, S * KV + u * L.max_groups + g, u)
    W.index(cidx, K_MAX_COUNTERS, "decode merge counter")
    slot0 = np.where(first_lvl, ubase + g * MERGE_GROUP, np.where(grouped, gbase, ubase))
    cnt = np.where(first_lvl, gsize, np.where(grouped, ngroups, n))
    last = slot0 + cnt - 1
    for sl, what in ((slot0, "first"), (last, "last")):
        r = L.part_off + sl * G * D * 4
        W.read(ws, r, r + G * D * 4, f"decode merge {what} partial")
        r = L.ml_off + sl * G * 2 * 4
        W.read(ws, r, r + G * 8, f"decode merge {what} (m, l)")
    W.index([64 * gp - 1], (L.partition + 16 * ring) * gp, "decode merge weights in LDS")
    dst = gbase + g
    if first_lvl.any():
        r = L.part_off + ((dst[first_lvl][:, None] * G + h[None, :]) * D) * 4
        W.add(ws, r, r + 4 * D, "decode group result")
        r = L.ml_off + ((dst[first_lvl][:, None] * G + h[None, :]) * 2) * 4
        W.add(ws, r, r + 8, "decode group (m, l)")
        # second level: every group result of the unit
        r = L.part_off + (gbase[first_lvl] + ngroups[first_lvl] - 1) * G * D * 4
        W.read(ws, r, r + G * D * 4, "decode second-level partial")
    lo = (s[multi][:, None] * out_stride_seq + (kh[multi][:, None] * G + h[None, :]) * out_stride_head) * 2
    W.add(out, lo, lo + 2 * D, "decode merged output rows")


# ---------------------------------------------------------------------------
# Chunked prefill (prefill_attention.hip)
# ---------------------------------------------------------------------------

@dataclass
class PrefillLaunch:
    S: int
    H: int
    KV: int
    bs: int
    max_bps: int
    max_q_len: int
    max_ctx: int
    hw: int = 4
    rt: int = 1
    tiles: int = 0
    hgroups: int = 0
    splits: int = 1
    ks_steps: int = SPLIT_STEPS
    o_off: int = 0
    ml_off: int = 0
    total: int = 0
    grid: int = 0
    groups: int = 0
    subtiles: int = 0
    num_cus: int = 256


def prefill_host(S, H, KV, bs, max_bps, max_q_len, max_ctx, num_cus=256,
                 D: int = 128) -> PrefillLaunch:
    """prefill_layout and prefill_impl (prefill_attention.hip), head dims 64
    and 128 (prefill_kernel)."""
    assert D in (64, 128)
    L = PrefillLaunch(S, H, KV, bs, max_bps, max_q_len, max_ctx, num_cus=num_cus)
    g = H // KV
    L.hw = 4 if g % 4 == 0 else (2 if g % 2 == 0 else 1)
    if max_ctx > 0:
        steps = _ceil(max_ctx, KT)
        ks = max(_ceil(steps, MAX_SPLITS), SPLIT_STEPS)
        L.ks_steps = ks
        L.splits = _ceil(steps, ks)
    if L.splits <= 1 or S <= 0 or H <= 0 or max_q_len <= 0:
        L.splits = 1
    else:
        t32 = _ceil(max_q_len, WAVE_ROWS) + 7
        nrec = S * t32 * H * L.splits
        L.o_off = K_COUNTER_BYTES
        L.ml_off = L.o_off + nrec * rec_o(D) * 4
        L.total = L.ml_off + nrec * REC_ML * 4
    L.rt = 4 // L.hw
    L.tiles = _ceil(max_q_len, 64 * L.rt)
    L.hgroups = g // L.hw
    L.groups = L.splits * S * KV
    L.grid = _ceil(L.groups, 8) * 8 * L.tiles * L.hgroups
    L.subtiles = L.tiles * L.rt * 2
    return L


def prefill_items(L: PrefillLaunch, cu: np.ndarray, ctx_lens: np.ndarray):
    """(s, t, j, kh, hg, q0, qlen, ctx, ks, eq) per running workgroup
    (prefill_attention.hip:170-288)."""
    TR = 64 * L.rt
    cap = L.max_bps * L.bs
    items = []
    if L.S * L.tiles <= 64:
        lane = np.arange(64)
        ls, lt = lane // L.tiles, lane % L.tiles
        valid = ls < L.S
        c0 = np.zeros(64, np.int64)
        ql = np.zeros(64, np.int64)
        cx = np.zeros(64, np.int64)
        n = np.zeros(64, np.int64)
        for i in np.flatnonzero(valid):
            c0[i] = cu[ls[i]]
            ql[i] = cu[ls[i] + 1] - c0[i]
            if lt[i] * TR < ql[i]:
                cx[i] = min(max(int(ctx_lens[ls[i]]), 0), cap)
                rw = min(ql[i] - lt[i] * TR, TR)
                nk = max(0, cx[i] - ql[i] + lt[i] * TR + rw)
                n[i] = _ceil(nk, KT)
            else:
                valid[i] = False
        per_item = L.KV * L.hgroups
        tot, nmax = int(n.sum()), int(n.max())
        avg = _ceil(tot * per_item, L.num_cus)
        parts = max(nmax // avg if avg > 0 else 1, 1)
        ks = max(_ceil(nmax, parts), L.ks_steps)
        # near-equal parts per tile; items by part length (longest first),
        # then tile, part, (kv-head, head group)
        nsp = np.where(valid, np.clip(_ceil(n, ks), 1, L.splits), 0)
        ln = np.where(valid, _ceil(n, np.maximum(nsp, 1)), -1)
        lenmax = int(ln.max())
        frm = [int(nsp[ln >= b].sum()) * per_item for b in range(lenmax + 2)]
        for bid in range(L.grid):
            idv = bid
            if idv >= frm[0]:
                continue
            lo = max(b for b in range(lenmax + 1) if frm[b] > idv)
            idv -= frm[lo + 1]
            lanes = np.flatnonzero(ln == lo)
            if len(lanes) == 0:
                items.append(None)
                continue
            sel = int(lanes[0])
            for k, l in enumerate(lanes):
                sel = int(l)
                c = int(nsp[l]) * per_item
                if idv < c or k == len(lanes) - 1:
                    break
                idv -= c
            j = idv // per_item
            rem = idv - j * per_item
            kh, hg = rem % L.KV, rem // L.KV
            items.append((sel // L.tiles, sel % L.tiles, j, kh, hg, int(c0[sel]), int(ql[sel]),
                          int(cx[sel]), ks, True))
        return items
    gunits = L.tiles * L.hgroups
    for bid in range(L.grid):
        xcd, p = bid & 7, bid >> 3
        gi = (p // gunits) * 8 + xcd
        if gi >= L.groups:
            continue
        u = p - (p // gunits) * gunits
        t = L.tiles - 1 - u // L.hgroups
        hg = u - (u // L.hgroups) * L.hgroups
        kh = gi % L.KV
        js = gi // L.KV
        s = js % L.S
        j = js // L.S
        q0 = int(cu[s])
        qlen = int(cu[s + 1]) - q0
        if t * TR >= qlen:
            continue
        ctx = min(max(int(ctx_lens[s]), 0), cap)
        items.append((s, t, j, kh, hg, q0, qlen, ctx, L.ks_steps, False))
    return items


def prefill(W: Writes, L: PrefillLaunch, out: Buf, ws: Buf, cu: np.ndarray, ctx_lens: np.ndarray,
            out_stride_token: int, out_stride_head: int, D: int = 128) -> None:
    TR = 64 * L.rt
    G = L.H // L.KV
    for it in prefill_items(L, cu, ctx_lens):
        if it is None:
            W.errors.append("prefill: a workgroup derived no tile (empty ballot)")
            continue
        s, t, j, kh, hg, q0, qlen, ctx, ks, eq = it
        W.index([s], L.S, "prefill sequence")
        prefix = ctx - qlen
        rows = min(qlen - t * TR, TR)
        pos0 = prefix + t * TR
        nkeys = max(pos0 + rows, 0)
        nsteps = _ceil(nkeys, KT)
        nsp = min(max(_ceil(nsteps, ks), 1), L.splits)
        if j >= nsp:
            continue
        if eq:   # near-equal parts, the first nsteps % nsp one step longer
            base, rm = divmod(nsteps, nsp)
            st0 = j * base + min(j, rm)
            st1 = st0 + base + (1 if j < rm else 0)
        else:
            st0 = j * ks
            st1 = nsteps if j == nsp - 1 else st0 + ks
        kbeg = st0 * KT
        kend = min(st1 * KT, nkeys)
        blk0 = kbeg // L.bs
        nblk = _ceil(kend, L.bs) - blk0 if kend > kbeg else 0
        W.index([nblk - 1] if nblk else [], MAX_BLOCKS_LDS, "prefill block ids in LDS")
        W.index([blk0 + nblk - 1] if nblk else [], L.max_bps, "prefill block-table column")
        for wave in range(8):
            pair, half = wave >> 1, wave & 1
            wr = pair // L.hw
            h = kh * G + hg * L.hw + (pair - wr * L.hw)
            wsub = (t * L.rt + wr) * 2 + half
            wrow0 = wsub * WAVE_ROWS
            r = np.arange(WAVE_ROWS) + wrow0
            r = r[r < qlen]
            lo = ((q0 + r) * out_stride_token + h * out_stride_head) * 2
            W.add(out, lo, lo + 2 * D, "prefill output rows")
            if st0 >= st1 or nsp <= 1:
                continue
            rec = ((s * L.subtiles + wsub) * L.H + h) * L.splits
            W.index([wsub], L.subtiles, "prefill subtile")
            for jj in (j, 0, nsp - 1):
                o = L.o_off + (rec + jj) * rec_o(D) * 4
                W.add(ws, o, o + rec_o(D) * 4, "prefill partial O")
                o = L.ml_off + (rec + jj) * REC_ML * 4
                W.add(ws, o, o + REC_ML * 4, "prefill partial (m, l)")
            cidx = ((s * L.tiles + t) * L.KV + kh) * L.hgroups + hg
            W.index([cidx], K_MAX_COUNTERS, "prefill merge counter")


def prefill_generic_units(S: int, H: int, KV: int, max_q_len: int, ctx_lens, cap: int):
    """(blockIdx, sequence, tile, head) of every workgroup of
    prefill_generic_kernel's grid that does not exit at once (prefill_attention.hip, the blockIdx
    mapping of prefill_generic_kernel and its grid in prefill_impl). Up to 64
    sequences go longest context first (ties: lower index first)."""
    tiles = _ceil(max_q_len, 64)
    G = H // KV
    per = tiles * G
    grid = _ceil(S * KV, 8) * 8 * per
    if S <= 64:
        n = [min(max(int(c), 0), cap) for c in ctx_lens[:S]]
        order = sorted(range(S), key=lambda i: (-n[i], i))
    else:
        order = list(range(S))
    out = []
    for bid in range(grid):
        xcd, p = bid & 7, bid >> 3
        gi = (p // per) * 8 + xcd
        if gi >= S * KV:
            continue
        u = p % per
        s = order[gi // KV]
        t = tiles - 1 - u // G
        h = (gi % KV) * G + u % G
        out.append((bid, s, t, h))
    return out


def prefill_generic(W: Writes, S: int, H: int, KV: int, bs: int, max_bps: int, num_blocks: int,
                    max_q_len: int, out: Buf, cu: np.ndarray, ctx_lens: np.ndarray,
                    out_stride_token: int, out_stride_head: int, tables: np.ndarray,
                    D: int) -> None:
    """prefill_generic_kernel (head dim 256): one workgroup per
    (sequence, head, 64-row tile), grouped by (sequence, kv head) on one XCD;
    every K/V row it reads and every output row it writes."""
    tiles = _ceil(max_q_len, 64)
    cap = max_bps * bs
    G = H // KV
    for _, s, t, h in prefill_generic_units(S, H, KV, max_q_len, ctx_lens, cap):
        q0 = int(cu[s])
        qlen = int(cu[s + 1]) - q0
        if t * 64 >= qlen:
            continue
        ctx = min(max(int(ctx_lens[s]), 0), cap)
        prefix = ctx - qlen
        rows = min(qlen - t * 64, 64)
        nkeys = max(prefix + t * 64 + rows, 0)
        if nkeys:
            tok = np.arange(nkeys)
            lb = tok // bs
            W.index(lb, max_bps, "prefill_generic block-table column")
            blk = np.clip(tables[s, lb], 0, num_blocks - 1)
            ri = (blk * KV + h // G) * bs + (tok - lb * bs)
            W.index(ri, num_blocks * KV * bs, "prefill_generic K/V row")
        r = np.arange(t * 64, t * 64 + 64)
        r = r[r < qlen]
        lo = ((q0 + r) * out_stride_token + h * out_stride_head) * 2
        W.add(out, lo, lo + 2 * D, "prefill_generic output rows")


# ---------------------------------------------------------------------------
# Block copy (copy_blocks.hip:15-29)
# ---------------------------------------------------------------------------

def copy_blocks(W: Writes, k_cache: Buf, v_cache: Buf, pairs: np.ndarray, num_blocks: int,
                block_bytes: int) -> None:
    pairs = np.asarray(pairs, dtype=np.int64).reshape(-1, 2)
    ok = (pairs >= 0).all(1) & (pairs < num_blocks).all(1)
    d = pairs[ok, 1]
    for buf in (k_cache, v_cache):
        W.add(buf, d * block_bytes, (d + 1) * block_bytes, "copy_blocks destination")
