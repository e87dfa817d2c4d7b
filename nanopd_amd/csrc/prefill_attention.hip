// Chunked-prefill attention over a paged prefix plus the new chunk (MFMA).
//
// Reference: the prefill branch of ModelRunner.paged_forward
// (nanoPD/engine/model_runner.py:152-168) runs F.scaled_dot_product_attention
// over the chunk's own K/V with a block-diagonal causal mask and never reads
// the prefix already in the pool. This op computes what that code means for a
// chunk on a prefix: query row i of sequence s, at position
// p = context_lens[s] - q_len + i, attends causally to keys 0..p of the paged
// cache (the chunk's K/V are stored before the call, as the reference stores
// them before attending, model_runner.py:146). For an empty prefix both agree.
//
// MI355X design (gfx950, v_mfma_f32_16x16x32_{bf16,f16}, wave64):
//   head dim D = 64 or 128 (prefill_kernel<.., D, ..>; the other multiples
//   of 32 up to 256 run prefill_generic_kernel below);
//   workgroup = 8 waves = one (sequence, kv-head, head group, 64-row query
//   tile, key split); wave w owns one query head and 32 query rows. Two waves
//   per SIMD, 256 VGPRs each (MFMA operands stay in VGPRs). HW = gcd(G, 4)
//   heads per workgroup, 4 / HW row tiles of 64 (G = 4: 4 heads x 64 rows).
//   The 64-key K/V tile the workgroup gathers from the pool into LDS is read
//   by all 8 waves (GQA and row reuse).
//   per step of 64 keys, each wave:
//     S^T = K . Q^T   -- A = K rows from LDS, B = the wave's query rows, kept
//                        in registers for the whole key loop;
//     softmax          -- lane l holds 16 keys of query (mb*16 + l%16) of each
//                        16-row block; the rest are in lanes l^16, l^32 (row
//                        max / sum with v_permlane16/32_swap). Scale and max
//                        subtraction are one FMA before exp2; the row sum is a
//                        v_dot2 of the rounded P pair with (1, 1). The running
//                        max is only moved (and O rescaled) when a row's new
//                        max exceeds it by more than 2^kTau: P entries then
//                        stay <= 2^kTau, exact in fp32 accumulation, and the
//                        rescale is rare after the first step;
//     O^T += V^T . P^T -- P^T is the S^T accumulator, already in B-operand
//                        layout (packed with v_cvt_pk_bf16_f32); V stays
//                        row-major in LDS like K, and the V^T A operand is two
//                        ds_read_b64_tr_b16 (gfx950 transposing LDS read: in a
//                        group of 16 lanes, lane j receives element j%4 of the
//                        8-byte chunks addressed by lanes 4e + j/4, e = 0..3).
//   The two waves of a SIMD are phase-shifted (one runs PV of the previous
//   step before QK, the other after softmax), so one's softmax VALU work can
//   run under the other's MFMAs. K/V loads run three steps ahead through a
//   register ring, are copied into LDS (2 K, 3 V buffers) one step ahead, and
//   keys past the visible range are clamped to the last visible key (a real,
//   finite context row) and masked.
//   Operand layouts of v_mfma_f32_16x16x32 (checked on the hardware):
//     A[m = lane%16][k = 8*(lane/16) + e], B[k = 8*(lane/16) + e][n = lane%16],
//     D[m = 4*(lane/16) + i][n = lane%16].
//
// Key splits: a query tile whose key range is longer than ks_steps steps of 64
// keys is cut into nsp <= splits_max ranges run by separate workgroups (the
// tiles of a long prefix would otherwise run many times longer than the rest):
// near-equal parts when the work list orders the items (at most 64 tiles),
// else at multiples of ks_steps.
// Each split publishes its unnormalised O, running max and row sum with
// device-coherent stores, then takes a ticket from a per-tile counter; the last
// of the nsp to arrive merges the others into its registers
//   M = max_j m_j,  L = sum_j l_j 2^(m_j - M),  O = sum_j O_j 2^(m_j - M) / L
// writes the output and resets the counter to 0.
#include <type_traits>

#include "common.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 8;        // waves per workgroup: 2 per SIMD
constexpr int kThreads = 64 * kWaves;
constexpr int kPairs = kWaves / 2;   // (head, 64-row tile) pairs, two 32-row waves each
constexpr int kWaveRows = 32;    // query rows per wave
constexpr int kKT = 64;          // keys per step
constexpr int kDepth = 3;        // K/V tiles in flight per workgroup
// LDS row of the K and V tiles (elements) at head dim d: 72 dwords at 128,
// 40 at 64 -- an 8-bank shift per row either way, so 16 rows of K read at one
// column and 4 rows x 32 bytes of a transposing V read both hit distinct banks
constexpr int lds_row(int d) { return d + 16; }
constexpr int kMaxBlocksLds = 16384;  // block ids of one workgroup's key range kept in LDS (64 KB)
constexpr int kSplitSteps = 16;       // a key range longer than this many steps is split
constexpr int kMaxSplits = 8;
constexpr float kTau = 8.f;           // lazy-rescale threshold, log2 units
constexpr float kLog2e = 1.4426950408889634f;
// partial record of one wave (32 rows of one head, one split) at head dim d,
// floats: [nb*2 + mb][half][lane][2], nb < d / 16
constexpr int rec_o(int d) { return d / 8 * 2 * 64 * 2; }
constexpr int kRecML = 2 * 64 * 2;       // [mb][lane][m, l]

struct PrefillArgs {
  uint16_t* out;
  const uint16_t* q;
  const u32x4* k_cache;
  const u32x4* v_cache;
  const int32_t* block_tables;
  const int32_t* cu_seqlens_q;
  const int32_t* context_lens;
  int* counters;
  float* part_o;
  float* part_ml;
  const float* k_scale;   // FP8 pools: per-kv-head scales (element = e4m3 byte * scale)
  const float* v_scale;
  int num_seqs, num_kv_heads, group, hgroups, block_size, bs_shift, num_blocks, max_bps;
  int tiles_max, subtiles, splits_max;   // subtiles: 32-row subtiles per sequence
  int ks_steps, num_groups;              // key steps per split; (split, seq, kv-head) groups
  int num_cus;                           // compute units of the device (work-list sizing)
  float scale_log2;
  int64_t q_stride_token, q_stride_head, out_stride_token, out_stride_head;
};

template <class TT>
struct Mfma;
template <>
struct Mfma<npd::BF16> {
  typedef bf16x8 V8;
  static __device__ __forceinline__ f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(V8, a),
                                                   __builtin_bit_cast(V8, b), c, 0, 0, 0);
  }
};
template <>
struct Mfma<npd::F16> {
  typedef f16x8 V8;
  static __device__ __forceinline__ f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(V8, a),
                                                  __builtin_bit_cast(V8, b), c, 0, 0, 0);
  }
};

// Max / sum over the 4 key groups of a query row (lanes l, l^16, l^32, l^48).
using npd::row_max4;
using npd::row_sum4;

typedef short s16x4 __attribute__((ext_vector_type(4)));
// ds_read_b64_tr_b16 on an LDS address given as a generic pointer to __shared__
__device__ __forceinline__ u32x2 lds_read_tr(const uint16_t* p) {
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p)));
}

// The work item of this workgroup (every wave derives the same one): the
// sequence s, its query tile t of TR rows, key split j of split length ks
// steps, kv head kh and head group hg, and the sequence's first query row,
// chunk length and context. eq: the tile's nsp = ceil(steps / ks) splits are
// near-equal parts (the first steps % nsp one step longer) instead of ks-step
// splits and a shorter last one. false: no item, the workgroup exits.
struct Item {
  int s, t, j, kh, hg, ks, q0, qlen, ctx;
  bool eq;
};
template <int TR>
__device__ __forceinline__ bool prefill_item(const PrefillArgs& a, int lane, Item& it) {
  int s, t, j, kh, hg, ks = a.ks_steps;
  int q0, qlen, ctx;
  const int cap = a.max_bps * a.block_size;
  if (a.num_seqs * a.tiles_max <= 64) {
    // Work list in longest-processing-time order, derived by every wave from
    // the sequence lengths. Lane i stands for (sequence i / tiles_max, tile
    // i % tiles_max) with n_i key steps. The split length ks is chosen so that
    // the longest key range falls into equal parts no shorter than the
    // average work per compute unit (and no shorter than the host's split,
    // which sized the workspace); each tile's splits are near-equal parts. The
    // kv-head is the fastest-varying index and every count is a multiple of
    // the kv-head count, so with 8 kv-heads each XCD (workgroups go to XCDs
    // round-robin by blockIdx) serves one kv-head and its K/V stays in that
    // XCD's L2.
    const int ls = lane / a.tiles_max, lt = lane - ls * a.tiles_max;
    bool valid = ls < a.num_seqs;
    int n = 0, c0 = 0, ql = 0, cx = 0;
    if (valid) {
      c0 = a.cu_seqlens_q[ls];
      ql = a.cu_seqlens_q[ls + 1] - c0;
      valid = lt * TR < ql;
      if (valid) {
        cx = a.context_lens[ls];
        cx = cx < 0 ? 0 : (cx < cap ? cx : cap);
        const int rw = (ql - lt * TR) < TR ? (ql - lt * TR) : TR;
        int nk = cx - ql + lt * TR + rw;
        nk = nk < 0 ? 0 : nk;
        n = (nk + kKT - 1) / kKT;
      }
    }
    const int per_item = a.num_kv_heads * a.hgroups;   // workgroups per (sequence, tile, split)
    const int tot = npd::wave_sum_i(n), nmax = npd::wave_max_i(n);   // DPP, wave-uniform
    const int avg = (int)(((int64_t)tot * per_item + a.num_cus - 1) / a.num_cus);
    int parts = avg > 0 ? nmax / avg : 1;
    parts = parts < 1 ? 1 : parts;
    const int ksd = __builtin_amdgcn_readfirstlane((nmax + parts - 1) / parts);
    ks = ksd > ks ? ksd : ks;
    // a tile of n steps runs as nsp = ceil(n / ks) near-equal parts: no short
    // tail part that would pay a whole item's prologue and merge for a few
    // steps. Items in longest-processing-time order: by part length (bucket
    // len = ceil(n / nsp)), longest first; within a bucket by tile, part and
    // then (kv-head, head group).
    int nsp = (n + ks - 1) / ks;
    nsp = nsp < 1 ? 1 : (nsp > a.splits_max ? a.splits_max : nsp);
    if (!valid) nsp = 0;
    const int len = valid ? (n + nsp - 1) / nsp : -1;
    const int lenmax = npd::wave_max_i(len);
    // items in buckets >= b, non-increasing in b; item id is in the last
    // bucket b with from(b) > id (binary search over DPP wave sums)
    auto from = [&](int b) -> int { return npd::wave_sum_i(len >= b ? nsp : 0) * per_item; };
    int id = blockIdx.x;
    if (id >= from(0)) return false;   // past the last item
    int lo = 0, hi = lenmax;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (from(mid) > id) lo = mid; else hi = mid - 1;
    }
    id -= from(lo + 1);
    // the tile of the bucket holding item id: walk the bucket's tiles (a
    // wave-uniform loop over at most 64 lanes)
    uint64_t m = __ballot(len == lo);
    int sel = __builtin_ctzll(m);
    for (;;) {
      const int c = __builtin_amdgcn_readlane(nsp, sel) * per_item;
      if (id < c || (m & (m - 1)) == 0) break;
      id -= c;
      m &= m - 1;
      sel = __builtin_ctzll(m);
    }
    j = id / per_item;
    id -= j * per_item;
    const int rem = id;
    kh = rem % a.num_kv_heads;
    hg = rem / a.num_kv_heads;
    s = __builtin_amdgcn_readfirstlane(sel / a.tiles_max);
    t = __builtin_amdgcn_readfirstlane(sel - s * a.tiles_max);
    j = __builtin_amdgcn_readfirstlane(j);
    q0 = __builtin_amdgcn_readlane(c0, sel);
    qlen = __builtin_amdgcn_readlane(ql, sel);
    ctx = __builtin_amdgcn_readlane(cx, sel);
  } else {
    // Unit = (split j, sequence, kv-head; tile t, head group). The units of
    // one (j, s, kv-head) read the same K/V key range: they form a group that
    // runs on one XCD at the same time (workgroups go to XCDs round-robin by
    // blockIdx, so the group's blockIdx values are 8 apart and consecutive in
    // that XCD's order), so K/V tiles come from that XCD's L2 after the first
    // read. Within a group the last tile (the most keys) comes first.
    const int gunits = a.tiles_max * a.hgroups;
    const int xcd = blockIdx.x & 7, p = blockIdx.x >> 3;
    const int gi = (p / gunits) * 8 + xcd;
    if (gi >= a.num_groups) return false;
    const int u = p - (p / gunits) * gunits;
    t = a.tiles_max - 1 - u / a.hgroups;
    hg = u - (u / a.hgroups) * a.hgroups;
    kh = gi % a.num_kv_heads;
    const int js = gi / a.num_kv_heads;
    s = js % a.num_seqs;
    j = js / a.num_seqs;
    q0 = a.cu_seqlens_q[s];
    qlen = a.cu_seqlens_q[s + 1] - q0;
    if (t * TR >= qlen) return false;
    ctx = a.context_lens[s];
    ctx = ctx < 0 ? 0 : (ctx < cap ? ctx : cap);
  }

  it = Item{s, t, j, kh, hg, ks, q0, qlen, ctx, a.num_seqs * a.tiles_max <= 64};
  return true;
}

// kOff32: every K/V element of the pool lies within 4 GiB of the cache base,
// so gather offsets are 32-bit. kF8: the pool holds OCP e4m3 bytes; a K/V
// chunk is 8 bytes, converted exactly to four TT pairs when copied into LDS,
// and the per-kv-head scales go into the score scale and the output.
template <class TT, int D, int HW, bool kOff32, bool kF8>
__global__ __launch_bounds__(kThreads) void prefill_kernel(PrefillArgs a) {
  static_assert(D == 64 || D == 128, "head dims of this kernel");
  constexpr int RT = kPairs / HW;                      // row tiles of 64 per workgroup
  constexpr int TR = 64 * RT;                          // query rows per workgroup
  constexpr int MB = kWaveRows / 16;                   // 16-row query blocks per wave
  constexpr int NC = D / 32;                           // head-dim chunks of QK
  constexpr int NB = D / 16;                           // 16-dim blocks of O
  constexpr int kRow = lds_row(D);
  constexpr int kRecO = rec_o(D);
  __shared__ __attribute__((aligned(16))) uint16_t s_k[2][kKT * kRow];
  __shared__ __attribute__((aligned(16))) uint16_t s_v[3][kKT * kRow];
  __shared__ int s_blk[kMaxBlocksLds];
  __shared__ int s_ticket;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, r = lane & 15;

  Item it;
  if (!prefill_item<TR>(a, lane, it)) return;
  const int s = it.s, t = it.t, j = it.j, kh = it.kh, hg = it.hg, ks = it.ks;
  const int q0 = it.q0, qlen = it.qlen, ctx = it.ctx;

  const int prefix = ctx - qlen;                       // position of query row 0
  const int rows = (qlen - t * TR) < TR ? (qlen - t * TR) : TR;
  const int pos0 = prefix + t * TR;                    // position of the tile's first row
  int nkeys = pos0 + rows;                             // keys 0 .. last row's position
  nkeys = nkeys < 0 ? 0 : nkeys;
  const int nsteps = (nkeys + kKT - 1) / kKT;
  // grid order: split j covers steps [j*ks, (j+1)*ks) -- the same keys for
  // every tile of the sequence -- the last split runs to the end of the
  // tile's range; work list: near-equal parts
  int nsp = (nsteps + ks - 1) / ks;
  nsp = nsp < 1 ? 1 : (nsp > a.splits_max ? a.splits_max : nsp);
  if (j >= nsp) return;
  int st0, st1;
  if (it.eq) {   // near-equal parts, the first nsteps % nsp one step longer
    const int base = nsteps / nsp, rem = nsteps - base * nsp;
    st0 = j * base + (j < rem ? j : rem);
    st1 = st0 + base + (j < rem ? 1 : 0);
  } else {
    st0 = j * ks;
    st1 = j == nsp - 1 ? nsteps : st0 + ks;
  }

  // wave -> (head of the group, row tile, half of the row tile)
  const int pair = wave >> 1, half = wave & 1;
  const int wr = pair / HW;
  const int h = kh * a.group + hg * HW + (pair - wr * HW);
  const int wsub = (t * RT + wr) * 2 + half;           // 32-row subtile index in the sequence
  const int wrow0 = wsub * kWaveRows;                  // this wave's first row
  const int wpos0 = prefix + wrow0;
  const int bs = a.block_size;
  const int kbeg = st0 * kKT;
  const int kend = st1 * kKT < nkeys ? st1 * kKT : nkeys;
  const int blk0 = kbeg / bs;
  const int nblk = kend > kbeg ? (kend + bs - 1) / bs - blk0 : 0;

  if (st0 >= st1) {
    // no key at all (every row of the tile sits before position 0): zero rows
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int row = wrow0 + mb * 16 + r;
      if (row >= qlen) continue;
      uint16_t* op = a.out + (int64_t)(q0 + row) * a.out_stride_token + (int64_t)h * a.out_stride_head;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) *reinterpret_cast<u32x2*>(op + nb * 16 + g * 4) = u32x2{0, 0};
    }
    return;
  }

  // block ids of the split's key range -> LDS (clamped into the pool); the
  // host guarantees max_bps <= kMaxBlocksLds, so the whole range fits
  for (int e = tid; e < nblk; e += kThreads) {
    int bid = a.block_tables[(int64_t)s * a.max_bps + blk0 + e];
    s_blk[e] = bid < 0 ? 0 : (bid >= a.num_blocks ? a.num_blocks - 1 : bid);
  }

  // the wave's query rows as B operands: qb[mb][c] = Q[row mb*16 + r][c*32 + 8g .. +8].
  // Rows past the chunk read its last row (their outputs are never stored):
  // unconditional loads keep the compiler's count of loads in flight exact.
  u32x4 qb[MB][NC];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    int row = wrow0 + mb * 16 + r;
    row = row < qlen ? row : qlen - 1;
    const uint16_t* qp = a.q + (int64_t)(q0 + row) * a.q_stride_token +
                         (int64_t)h * a.q_stride_head + g * 8;
#pragma unroll
    for (int c = 0; c < NC; ++c) qb[mb][c] = *reinterpret_cast<const u32x4*>(qp + c * 32);
  }
  __syncthreads();

  // K/V tile loaders: chunk tid + 512e (8 elements) of the 64-key tile, i.e.
  // key tid / CPR + KPP * e, column chunk tid % CPR. Loads run kDepth steps
  // ahead through a register ring (slot = step % kDepth): one tile in flight
  // per CU leaves a step waiting on memory latency.
  constexpr int CPR = D / 8;                           // 8-element chunks per row
  constexpr int KPP = kThreads / CPR;                  // keys per load pass
  constexpr int kPer = kKT / KPP;                      // 2 at D 128, 1 at D 64
  static_assert(kPer * KPP == kKT, "tile shape");
  typedef typename std::conditional<kF8, u32x2, u32x4>::type raw_t;   // 8 elements
  raw_t kst[kDepth][kPer], vst[kDepth][kPer];
  const int col = tid % CPR;
  // Every fetch issues the same loads, so the compiler's count of loads in
  // flight stays exact and its waits cover only the slot being used: tokens
  // past the split's range are clamped to its last key. Such keys only occur
  // past the tile's last row (the causal mask removes them) and hold real
  // context rows, so their V is finite and P = 0 cancels it.
  auto fetch = [&](int step, raw_t* ks, raw_t* vs) {
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      int tok = step * kKT + tid / CPR + KPP * e;
      tok = tok < kend ? tok : kend - 1;
      const int lb = a.bs_shift >= 0 ? tok >> a.bs_shift : tok / bs;
      const int blk = s_blk[lb - blk0];
      const int row = (blk * a.num_kv_heads + kh) * bs + (tok - lb * bs);   // < 2^31 (host check)
      if constexpr (kF8) {   // D-byte rows, 8-byte chunks
        const char* kb = reinterpret_cast<const char*>(a.k_cache);
        const char* vb = reinterpret_cast<const char*>(a.v_cache);
        if (kOff32) {
          const uint32_t off = (uint32_t)row * (uint32_t)D + (uint32_t)col * 8u;
          ks[e] = *reinterpret_cast<const u32x2*>(kb + off);
          vs[e] = *reinterpret_cast<const u32x2*>(vb + off);
        } else {
          const int64_t off = (int64_t)row * D + col * 8;
          ks[e] = *reinterpret_cast<const u32x2*>(kb + off);
          vs[e] = *reinterpret_cast<const u32x2*>(vb + off);
        }
      } else if (kOff32) {
        const uint32_t off = (uint32_t)row * (uint32_t)(2 * D) + (uint32_t)col * 16u;
        ks[e] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(a.k_cache) + off);
        vs[e] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(a.v_cache) + off);
      } else {
        const int64_t idx = (int64_t)row * CPR + col;
        ks[e] = a.k_cache[idx];
        vs[e] = a.v_cache[idx];
      }
    }
  };
  auto pairs = [](raw_t w) -> u32x4 {
    if constexpr (kF8)
      return u32x4{npd::e4m3x2_to<TT, false>(w.x), npd::e4m3x2_to<TT, true>(w.x),
                   npd::e4m3x2_to<TT, false>(w.y), npd::e4m3x2_to<TT, true>(w.y)};
    else
      return w;
  };
  auto stash = [&](int kbuf, int vbuf, const raw_t* ks, const raw_t* vs) {
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      const int kk = tid / CPR + KPP * e;
      *reinterpret_cast<u32x4*>(&s_k[kbuf][kk * kRow + col * 8]) = pairs(ks[e]);
      *reinterpret_cast<u32x4*>(&s_v[vbuf][kk * kRow + col * 8]) = pairs(vs[e]);
    }
  };

  f32x4 oacc[NB][MB];   // O^T[d = nb*16 + 4g + i][q = mb*16 + r]
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) oacc[nb][mb] = f32x4{0, 0, 0, 0};
  float mrow[MB], nmref[MB], lrow[MB];   // running max (log2 units), -max or 0, row sum
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    mrow[mb] = -INFINITY;
    nmref[mb] = 0.f;
    lrow[mb] = 0.f;
  }
  const float c2 = kF8 ? a.scale_log2 * a.k_scale[kh] : a.scale_log2;
  const float oscale = kF8 ? a.v_scale[kh] : 1.f;

#pragma unroll
  for (int d = 0; d < kDepth; ++d) fetch(st0 + d, kst[d], vst[d]);
  stash(0, 0, kst[0], vst[0]);
  __syncthreads();

  // Step pieces. qk: S^T of step `step` from K buffer kbuf; softmax: P of
  // that step into pb (moves the running max and rescales O when needed);
  // pv: O^T += V^T . P^T from V buffer vbuf.
  f32x4 sacc[4][MB];   // S^T[key = n*16 + 4g + i][q = mb*16 + r]
  auto qk = [&](int kbuf) {
    const uint16_t* kt = s_k[kbuf];
    // S^T = K . Q^T
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) sacc[n][mb] = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const u32x4 ka = *reinterpret_cast<const u32x4*>(&kt[(n * 16 + r) * kRow + c * 32 + g * 8]);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) sacc[n][mb] = Mfma<TT>::mma(ka, qb[mb][c], sacc[n][mb]);
      }
    }
  };
  auto softmax = [&](int step, u32x4 (&pb)[2][MB]) {
    const int key0 = step * kKT;
    // causal mask, lazy-max softmax
    const bool diag = key0 + kKT - 1 > wpos0;   // some key here is after some row
    float v[MB][16];
    float mxs[MB];
    bool need = false;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i) v[mb][n * 4 + i] = sacc[n][mb][i];
    }
    if (diag) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        // key n*16 + 4g + i of this step is visible to the row iff n*16 + i <= lim
        const int lim = wpos0 + mb * 16 + r - key0 - 4 * g;
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (n * 16 + i > lim) v[mb][n * 4 + i] = -INFINITY;
      }
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      // a chain of three-operand maxima (v_max3_f32: two values per instruction)
      float mx = fmaxf(fmaxf(v[mb][0], v[mb][1]), v[mb][2]);
#pragma unroll
      for (int e = 3; e < 15; e += 2) mx = fmaxf(fmaxf(mx, v[mb][e]), v[mb][e + 1]);
      mx = row_max4(fmaxf(mx, v[mb][15]));
      mxs[mb] = mx * c2;
      need = need || (mxs[mb] > mrow[mb] + kTau);
    }
    if (__ballot(need) != 0) {
      // a row whose max moved past the threshold takes the new max as its
      // reference; alpha = 0 from the initial -inf (O and l are still 0)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const bool nd = mxs[mb] > mrow[mb] + kTau;
        const float mnew = nd ? mxs[mb] : mrow[mb];
        const float alpha = nd ? __builtin_amdgcn_exp2f(mrow[mb] - mnew) : 1.f;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) oacc[nb][mb] *= alpha;
        lrow[mb] *= alpha;
        mrow[mb] = mnew;
        nmref[mb] = mnew == -INFINITY ? 0.f : -mnew;
      }
    }
    // P = 2^(s*c - m), packed; pb[kc][mb] is the B operand of keys kc*32 .. +32:
    // slots e<4 -> key kc*32 + 4g + e, e>=4 -> kc*32 + 16 + 4g + e - 4
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      uint32_t packed[8];
#pragma unroll
      for (int e = 0; e < 16; e += 2) {
        const float p0 = __builtin_amdgcn_exp2f(fmaf(v[mb][e], c2, nmref[mb]));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(v[mb][e + 1], c2, nmref[mb]));
        const uint32_t u = TT::pack2(p0, p1);
        lrow[mb] = TT::dot2(u, TT::kOne2, lrow[mb]);
        packed[e / 2] = u;
      }
      pb[0][mb] = u32x4{packed[0], packed[1], packed[2], packed[3]};
      pb[1][mb] = u32x4{packed[4], packed[5], packed[6], packed[7]};
    }
  };
  auto pv = [&](int vbuf, const u32x4 (&pb)[2][MB]) {
    // O^T += V^T . P^T ; A = V^T[d = nb*16 + r][keys kc*32 + {4g..4g+3, 16+4g..16+4g+3}]
    // transposing reads: lane r of group g addresses key (.. + 4g + r/4),
    // dims nb*16 + 4*(r%4) .. +3, and receives dim nb*16 + r of keys +0..3
    const uint16_t* vlane = s_v[vbuf] + (g * 4 + (r >> 2)) * kRow + 4 * (r & 3);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const u32x2 lo = lds_read_tr(vlane + (kc * 32) * kRow + nb * 16);
        const u32x2 hi = lds_read_tr(vlane + (kc * 32 + 16) * kRow + nb * 16);
        const u32x4 va = u32x4{lo.x, lo.y, hi.x, hi.y};
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) oacc[nb][mb] = Mfma<TT>::mma(va, pb[kc][mb], oacc[nb][mb]);
      }
    }
  };

  // Two waves share each SIMD (waves w and w + 4). Group A (waves 0-3) runs
  // a step as QK -> softmax -> PV; group B (waves 4-7) runs the PV of the
  // previous step first, then QK -> softmax, so that one wave's softmax (VALU)
  // runs while the other's MFMAs do. K tiles use two LDS buffers; V tiles
  // three, because group B still reads step j - 1's V in step j.
  // Register ring slot SL holds this step's tile (already in LDS); it is
  // refilled with step + kDepth, and slot SL + 1 (the next step's tile) is
  // copied into LDS at the end of the step.
  const bool late = wave >= kWaves / 2;
  u32x4 pb[2][MB];
  bool pending = false;   // group B: pb holds the P of a step whose PV is due
  auto step_body = [&](int step, auto slot) {
    constexpr int SL = decltype(slot)::value;
    constexpr int SN = (SL + 1) % kDepth;
    const int rel = step - st0;
    fetch(step + kDepth, kst[SL], vst[SL]);   // past st1: clamped, never used
    // some row of the wave sees a key here (always so with one row tile)
    const bool active = RT == 1 || step * kKT <= wpos0 + kWaveRows - 1;
    if (!late) {
      if (active) {
        qk(rel & 1);
        softmax(step, pb);
        pv(rel % 3, pb);
      }
    } else {
      if (pending) pv((rel + 2) % 3, pb);
      pending = active;
      if (active) {
        qk(rel & 1);
        softmax(step, pb);
      }
    }
    // K buffer (rel + 1) & 1 and V buffer (rel + 1) % 3 were last read in
    // step - 1 (group B's PV of step - 2 included), which every wave finished
    // before that step's barrier. Written even after the last step (nobody
    // reads it then): an unconditional copy keeps the compiler's load
    // accounting exact on every path.
    stash((rel + 1) & 1, (rel + 1) % 3, kst[SN], vst[SN]);
    __syncthreads();
  };
  // full rounds of the ring in the loop; the 0-2 remaining steps after it, so
  // that every path back to the loop head has run all three slots
  static_assert(kDepth == 3, "the unrolled ring below has three slots");
  int step = st0;
  for (; step + kDepth <= st1; step += kDepth) {
    step_body(step, std::integral_constant<int, 0>{});
    step_body(step + 1, std::integral_constant<int, 1>{});
    step_body(step + 2, std::integral_constant<int, 2>{});
  }
  if (step < st1) step_body(step, std::integral_constant<int, 0>{});
  if (step + 1 < st1) step_body(step + 1, std::integral_constant<int, 1>{});
  if (late && pending) pv((st1 - 1 - st0) % 3, pb);

  // row sums over the 4 lanes of a row
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) lrow[mb] = row_sum4(lrow[mb]);

  if (nsp > 1) {
    // publish this split's partial (register order: every store is 512
    // contiguous bytes), then the last split of the tile to arrive merges
    const int H = a.num_kv_heads * a.group;
    const int64_t rec = (((int64_t)s * a.subtiles + wsub) * H + h) * a.splits_max;
    {
      float* po = a.part_o + (rec + j) * kRecO + lane * 2;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const int idx = nb * MB + mb;
          npd::st_coherent2(po + (idx * 2) * 128, oacc[nb][mb][0], oacc[nb][mb][1]);
          npd::st_coherent2(po + (idx * 2 + 1) * 128, oacc[nb][mb][2], oacc[nb][mb][3]);
        }
      float* pm = a.part_ml + (rec + j) * kRecML + lane * 2;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) npd::st_coherent2(pm + mb * 128, mrow[mb], lrow[mb]);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);   // every store of this wave has completed
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    const int64_t cidx = (((int64_t)s * a.tiles_max + t) * a.num_kv_heads + kh) * a.hgroups + hg;
    if (tid == 0)
      s_ticket = __hip_atomic_fetch_add(a.counters + cidx, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_ticket != nsp - 1) return;
    for (int jj = 0; jj < nsp; ++jj) {
      if (jj == j) continue;
      const float* pm = a.part_ml + (rec + jj) * kRecML + lane * 2;
      float wa[MB], wb[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        float mp, lp;
        npd::ld_coherent2(pm + mb * 128, mp, lp);
        const float mm = fmaxf(mrow[mb], mp);
        wa[mb] = mrow[mb] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mrow[mb] - mm);
        wb[mb] = mp == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mp - mm);
        lrow[mb] = lrow[mb] * wa[mb] + lp * wb[mb];
        mrow[mb] = mm;
      }
      const float* po = a.part_o + (rec + jj) * kRecO + lane * 2;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const int idx = nb * MB + mb;
          float x0, x1, x2, x3;
          npd::ld_coherent2(po + (idx * 2) * 128, x0, x1);
          npd::ld_coherent2(po + (idx * 2 + 1) * 128, x2, x3);
          oacc[nb][mb] = oacc[nb][mb] * wa[mb] + f32x4{x0, x1, x2, x3} * wb[mb];
        }
    }
    if (tid == 0) __hip_atomic_store(a.counters + cidx, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // normalise and store: lane writes d = nb*16 + 4g .. +3 of query row mb*16 + r
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int row = wrow0 + mb * 16 + r;
    if (row >= qlen) continue;
    const float l = lrow[mb];
    const float inv = (l > 0.f && wpos0 + mb * 16 + r >= 0) ? oscale / l : 0.f;
    uint16_t* op = a.out + (int64_t)(q0 + row) * a.out_stride_token + (int64_t)h * a.out_stride_head;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const f32x4 o = oacc[nb][mb];
      u32x2 w;
      w.x = TT::pack2(o[0] * inv, o[1] * inv);
      w.y = TT::pack2(o[2] * inv, o[3] * inv);
      *reinterpret_cast<u32x2*>(op + nb * 16 + g * 4) = w;
    }
  }
}

// Every head dim but 64 and 128 (multiples of 32 from 32 to 256): at 256 the
// tiles and register ring of prefill_kernel would need about 174 KB of LDS
// and 336 VGPRs. One workgroup of 4 waves per
// (sequence, query head, 64-row query tile); wave w owns query rows
// 16w .. 16w + 15 of the tile. Per step of 64 keys the workgroup copies the kv
// head's K and V rows into LDS (keys past the visible range clamped to the
// last visible key, as in prefill_kernel), then every wave computes
//   S^T = K . Q^T     (v_mfma_f32_16x16x32, D/32 chunks of the head dim x
//                      4 blocks of 16 keys; Q rows held in registers),
//   a causal mask and an online softmax in fp32 (log2 units; O and the row
//   sum rescaled whenever a row's running max grows),
//   O^T += V^T . P^T  (D/16 blocks of 16 dims x 2 chunks of 32 keys; V^T via
//                      the transposing LDS read, P^T from the S^T layout).
// The operand layouts, the P packing and the normalisation (the row sum adds
// the rounded P values) are those of prefill_kernel. The next step's K/V
// chunks load into registers during the step (two workgroups per CU at 254
// VGPRs); the workgroups of one (sequence, kv head) share K/V through one
// XCD's L2 rather than one LDS tile, and there are no key splits. Rows with no
// visible key are written as zeros.
template <class TT, int D, bool kF8>
__global__ __launch_bounds__(256, 2) void prefill_generic_kernel(PrefillArgs a) {
  constexpr int kGT = 256;                      // threads
  constexpr int RW = D + 16;                    // LDS row (elements); 16-byte multiple
  constexpr int CPR = D / 8;                    // 8-element chunks per K/V row
  constexpr int NPASS = kKT * CPR / kGT;        // chunks of the 64-key tile per thread
  constexpr int NC = D / 32;                    // head-dim chunks of QK
  constexpr int NB = D / 16;                    // 16-dim blocks of O
  static_assert(D % 32 == 0 && D >= 32 && D <= 256, "head dims of this kernel");
  static_assert(NPASS * kGT == kKT * CPR && RW % 8 == 0, "tile shape");
  __shared__ __attribute__((aligned(16))) uint16_t s_k[kKT * RW];
  __shared__ __attribute__((aligned(16))) uint16_t s_v[kKT * RW];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, r = lane & 15;
  // Every workgroup of one (sequence, kv head) reads the same keys from 0 up:
  // they all run on one XCD (workgroups go to XCDs round-robin by blockIdx),
  // one after another in that XCD's order, so the K/V rows come from its L2
  // after the first read. Groups go longest context first (up to 64
  // sequences; more keep their order); within a group the last tile (the
  // most keys) first, the group's query heads of a tile together.
  const int per = a.tiles_max * a.group;        // workgroups per (sequence, kv head)
  const int xcd = (int)(blockIdx.x & 7u), p = (int)(blockIdx.x >> 3);
  const int gi = (p / per) * 8 + xcd;           // (sequence rank, kv head) index
  if (gi >= a.num_seqs * a.num_kv_heads) return;
  const int u = p - (p / per) * per;
  const int rank = gi / a.num_kv_heads;
  const int t = a.tiles_max - 1 - u / a.group;
  const int h = (gi - rank * a.num_kv_heads) * a.group + (u - (u / a.group) * a.group);
  const int cap = a.max_bps * a.block_size;
  int s = rank;
  if (a.num_seqs <= 64) {
    // lane i stands for sequence i; its rank counts the sequences with a
    // longer context (ties: the lower index first)
    int n = -1;
    if (lane < a.num_seqs) {
      n = a.context_lens[lane];
      n = n < 0 ? 0 : (n < cap ? n : cap);
    }
    int rk = 0;
    for (int i = 0; i < a.num_seqs; ++i) {
      const int ni = __builtin_amdgcn_readlane(n, i);
      rk += (ni > n || (ni == n && i < lane)) ? 1 : 0;
    }
    const uint64_t m = __ballot(lane < a.num_seqs && rk == rank);
    s = __builtin_amdgcn_readfirstlane(__builtin_ctzll(m));
  }
  const int q0 = a.cu_seqlens_q[s];
  const int qlen = a.cu_seqlens_q[s + 1] - q0;
  if (t * 64 >= qlen) return;
  int ctx = a.context_lens[s];
  ctx = ctx < 0 ? 0 : (ctx < cap ? ctx : cap);
  const int kh = h / a.group;
  const int prefix = ctx - qlen;                 // position of query row 0
  const int rows = (qlen - t * 64) < 64 ? (qlen - t * 64) : 64;
  int nkeys = prefix + t * 64 + rows;            // keys 0 .. the tile's last position
  nkeys = nkeys < 0 ? 0 : nkeys;
  const int nsteps = (nkeys + kKT - 1) / kKT;
  const int bs = a.block_size;
  const int row = t * 64 + wave * 16 + r;        // this lane's query row (S^T column r)
  const int pos = prefix + row;

  u32x4 qb[NC];   // B operand: Q[row][c*32 + 8g .. +8]; rows past the chunk read its last row
  {
    const int rq = row < qlen ? row : qlen - 1;
    const uint16_t* qp = a.q + (int64_t)(q0 + rq) * a.q_stride_token +
                         (int64_t)h * a.q_stride_head + g * 8;
#pragma unroll
    for (int c = 0; c < NC; ++c) qb[c] = *reinterpret_cast<const u32x4*>(qp + c * 32);
  }
  f32x4 oacc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) oacc[nb] = f32x4{0, 0, 0, 0};
  float m = -INFINITY, l = 0.f;
  const float c2 = kF8 ? a.scale_log2 * a.k_scale[kh] : a.scale_log2;
  const float oscale = kF8 ? a.v_scale[kh] : 1.f;

  // K/V of the step's tile: raw chunks loaded into registers one step ahead
  // (in flight during the previous step's MFMAs), converted and copied into
  // LDS at the step's start. Keys past the visible range are clamped to the
  // last visible key (a real, finite row; the causal mask removes them).
  // Chunk tid + 256e of the tile (e < NPASS) is chunk col_of(e) of key
  // key_of(e): every thread moves whole 16-byte chunks, also when D / 8 is
  // not a power of two.
  typedef typename std::conditional<kF8, u32x2, u32x4>::type raw_t;   // 8 elements
  raw_t kr[NPASS], vr[NPASS];
  auto key_of = [&](int e) { return (tid + kGT * e) / CPR; };
  auto col_of = [&](int e) { return (tid + kGT * e) % CPR; };
  auto fetch = [&](int step) {
#pragma unroll
    for (int e = 0; e < NPASS; ++e) {
      const int col = col_of(e);
      int tok = step * kKT + key_of(e);
      tok = tok < nkeys ? tok : nkeys - 1;
      const int lb = a.bs_shift >= 0 ? tok >> a.bs_shift : tok / bs;
      int blk = a.block_tables[(int64_t)s * a.max_bps + lb];
      blk = blk < 0 ? 0 : (blk >= a.num_blocks ? a.num_blocks - 1 : blk);
      const int64_t ri = ((int64_t)blk * a.num_kv_heads + kh) * bs + (tok - lb * bs);
      if constexpr (kF8) {   // D-byte rows, 8-byte chunks
        kr[e] = *reinterpret_cast<const u32x2*>(reinterpret_cast<const char*>(a.k_cache) + ri * D + col * 8);
        vr[e] = *reinterpret_cast<const u32x2*>(reinterpret_cast<const char*>(a.v_cache) + ri * D + col * 8);
      } else {
        const int64_t idx = ri * CPR + col;   // 16-byte units
        kr[e] = a.k_cache[idx];
        vr[e] = a.v_cache[idx];
      }
    }
  };
  auto pairs = [](raw_t w) -> u32x4 {
    if constexpr (kF8)
      return u32x4{npd::e4m3x2_to<TT, false>(w.x), npd::e4m3x2_to<TT, true>(w.x),
                   npd::e4m3x2_to<TT, false>(w.y), npd::e4m3x2_to<TT, true>(w.y)};
    else
      return w;
  };
  if (nsteps > 0) fetch(0);
  for (int step = 0; step < nsteps; ++step) {
    __syncthreads();   // every wave is done with the previous tile
#pragma unroll
    for (int e = 0; e < NPASS; ++e) {
      const int kk = key_of(e), col = col_of(e);
      *reinterpret_cast<u32x4*>(&s_k[kk * RW + col * 8]) = pairs(kr[e]);
      *reinterpret_cast<u32x4*>(&s_v[kk * RW + col * 8]) = pairs(vr[e]);
    }
    __syncthreads();
    if (step + 1 < nsteps) fetch(step + 1);

    // S^T[key n*16 + 4g + i][query r]
    f32x4 sacc[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) sacc[n] = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const u32x4 ka = *reinterpret_cast<const u32x4*>(&s_k[(n * 16 + r) * RW + c * 32 + g * 8]);
        sacc[n] = Mfma<TT>::mma(ka, qb[c], sacc[n]);
      }
    const int key0 = step * kKT;
    float v[16];
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = key0 + n * 16 + 4 * g + i;
        v[n * 4 + i] = key <= pos ? sacc[n][i] : -INFINITY;
      }
    float mx = v[0];
#pragma unroll
    for (int e = 1; e < 16; ++e) mx = fmaxf(mx, v[e]);
    mx = row_max4(mx);
    const float mnew = fmaxf(m, mx * c2);
    const float mref = mnew == -INFINITY ? 0.f : mnew;
    const float alpha = __builtin_amdgcn_exp2f(m - mref);   // 0 from the initial -inf
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) oacc[nb] *= alpha;
    l *= alpha;
    m = mnew;
    uint32_t packed[8];
#pragma unroll
    for (int e = 0; e < 16; e += 2) {
      const float p0 = __builtin_amdgcn_exp2f(fmaf(v[e], c2, -mref));
      const float p1 = __builtin_amdgcn_exp2f(fmaf(v[e + 1], c2, -mref));
      const uint32_t u = TT::pack2(p0, p1);
      l = TT::dot2(u, TT::kOne2, l);
      packed[e / 2] = u;
    }
    // B operand of keys kc*32 .. +32: slots e < 4 -> key 4g + e, e >= 4 -> 16 + 4g + e - 4
    const u32x4 pb[2] = {u32x4{packed[0], packed[1], packed[2], packed[3]},
                         u32x4{packed[4], packed[5], packed[6], packed[7]}};
    const uint16_t* vlane = s_v + (g * 4 + (r >> 2)) * RW + 4 * (r & 3);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const u32x2 lo = lds_read_tr(vlane + (kc * 32) * RW + nb * 16);
        const u32x2 hi = lds_read_tr(vlane + (kc * 32 + 16) * RW + nb * 16);
        oacc[nb] = Mfma<TT>::mma(u32x4{lo.x, lo.y, hi.x, hi.y}, pb[kc], oacc[nb]);
      }
  }
  l = row_sum4(l);
  if (row >= qlen) return;
  const float inv = (l > 0.f && pos >= 0) ? oscale / l : 0.f;
  uint16_t* op = a.out + (int64_t)(q0 + row) * a.out_stride_token + (int64_t)h * a.out_stride_head;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const f32x4 o = oacc[nb];
    u32x2 w;
    w.x = TT::pack2(o[0] * inv, o[1] * inv);
    w.y = TT::pack2(o[2] * inv, o[3] * inv);
    *reinterpret_cast<u32x2*>(op + nb * 16 + g * 4) = w;
  }
}

template <class TT, bool kF8>
int launch_generic(int64_t head_dim, const PrefillArgs& a, int64_t grid, hipStream_t st,
                   const char* name) {
  const dim3 g((unsigned)grid), b(256);
  switch (head_dim) {
    case 32: hipLaunchKernelGGL((prefill_generic_kernel<TT, 32, kF8>), g, b, 0, st, a); break;
    case 96: hipLaunchKernelGGL((prefill_generic_kernel<TT, 96, kF8>), g, b, 0, st, a); break;
    case 160: hipLaunchKernelGGL((prefill_generic_kernel<TT, 160, kF8>), g, b, 0, st, a); break;
    case 192: hipLaunchKernelGGL((prefill_generic_kernel<TT, 192, kF8>), g, b, 0, st, a); break;
    case 224: hipLaunchKernelGGL((prefill_generic_kernel<TT, 224, kF8>), g, b, 0, st, a); break;
    case 256: hipLaunchKernelGGL((prefill_generic_kernel<TT, 256, kF8>), g, b, 0, st, a); break;
    default: return npd::fail(NPD_E_INVALID, "%s: head_dim %lld", name, (long long)head_dim);
  }
  return npd::check_launch(name);
}

template <class TT, int D, bool kOff32, bool kF8>
int launch(int hw, const PrefillArgs& a, int64_t grid, hipStream_t st, const char* name) {
  switch (hw) {
    case 1: hipLaunchKernelGGL((prefill_kernel<TT, D, 1, kOff32, kF8>), dim3((unsigned)grid), dim3(kThreads), 0, st, a); break;
    case 2: hipLaunchKernelGGL((prefill_kernel<TT, D, 2, kOff32, kF8>), dim3((unsigned)grid), dim3(kThreads), 0, st, a); break;
    case 4: hipLaunchKernelGGL((prefill_kernel<TT, D, 4, kOff32, kF8>), dim3((unsigned)grid), dim3(kThreads), 0, st, a); break;
    default: return npd::fail(NPD_E_INVALID, "%s: heads per workgroup %d", name, hw);
  }
  return npd::check_launch(name);
}

template <class TT, bool kF8>
int launch_dt(int64_t head_dim, bool off32, int hw, const PrefillArgs& a, int64_t grid,
              hipStream_t st, const char* name) {
  if (head_dim == 64)
    return off32 ? launch<TT, 64, true, kF8>(hw, a, grid, st, name)
                 : launch<TT, 64, false, kF8>(hw, a, grid, st, name);
  return off32 ? launch<TT, 128, true, kF8>(hw, a, grid, st, name)
               : launch<TT, 128, false, kF8>(hw, a, grid, st, name);
}

// Workspace: [counter region (kCounterBytes) | O partials | (m, l) partials].
// Sized for the most records any head group / row tiling of these shapes can
// address: a sequence has tiles_max * (4 / HW) * 2 <= ceil(max_q_len / 32) + 7
// subtiles of 32 rows.
struct Layout {
  int splits, ks_steps;
  int64_t o_off, ml_off, total;
};

Layout prefill_layout(int64_t num_seqs, int64_t num_heads, int64_t head_dim, int64_t max_q_len,
                      int64_t max_context_len) {
  Layout L{1, kSplitSteps, 0, 0, 0};
  if (max_context_len > 0) {
    // splits of kSplitSteps steps, longer ones when that would exceed kMaxSplits
    const int64_t steps = (max_context_len + kKT - 1) / kKT;
    int64_t ks = (steps + kMaxSplits - 1) / kMaxSplits;
    ks = ks < kSplitSteps ? kSplitSteps : ks;
    L.ks_steps = (int)ks;
    L.splits = (int)((steps + ks - 1) / ks);
  }
  if (L.splits <= 1 || num_seqs <= 0 || num_heads <= 0 || max_q_len <= 0) {
    L.splits = 1;
    return L;
  }
  const int64_t t32 = (max_q_len + kWaveRows - 1) / kWaveRows + 7;
  const int64_t units = num_seqs * t32 * num_heads;
  const int64_t nrec = units * L.splits;
  L.o_off = npd::kCounterBytes;
  L.ml_off = L.o_off + nrec * rec_o((int)head_dim) * 4;
  L.total = L.ml_off + nrec * kRecML * 4;
  return L;
}

}  // namespace

extern "C" int64_t npd_paged_prefill_workspace_size(int64_t num_seqs, int64_t total_q,
                                                    int64_t num_heads, int64_t head_dim,
                                                    int64_t max_q_len, int64_t max_context_len) {
  (void)total_q;
  // head dims other than 64 and 128 (prefill_generic_kernel) need no workspace
  if (head_dim != 64 && head_dim != 128) return 0;
  return prefill_layout(num_seqs, num_heads, head_dim, max_q_len, max_context_len).total;
}

namespace {

// Shared by the 2-byte and the FP8 entry points: k_scale / v_scale are null
// for 2-byte pools.
int prefill_impl(void* out, const void* query, const void* key_cache, const void* value_cache,
                 const int32_t* block_tables, const int32_t* cu_seqlens_q,
                 const int32_t* context_lens, const float* k_scale, const float* v_scale,
                 int64_t num_seqs, int64_t total_q, int64_t num_heads, int64_t num_kv_heads,
                 int64_t head_dim, int64_t num_blocks, int64_t block_size,
                 int64_t max_blocks_per_seq, int64_t max_q_len, int64_t max_context_len,
                 float scale, int64_t q_stride_token, int64_t q_stride_head,
                 int64_t out_stride_token, int64_t out_stride_head, void* workspace,
                 int64_t workspace_bytes, int32_t dtype, void* stream, bool fp8,
                 const char* name) {
  using namespace npd;
  if (dtype != NPD_DTYPE_F16 && dtype != NPD_DTYPE_BF16)
    return fail(NPD_E_DTYPE, "%s: unsupported dtype code %d (fp16/bf16 only)", name, dtype);
  if (num_seqs < 0 || total_q < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_blocks <= 0 ||
      block_size <= 0 || max_blocks_per_seq <= 0 || max_q_len < 0)
    return fail(NPD_E_INVALID, "%s: bad sizes", name);
  if (head_dim < 32 || head_dim > 256 || head_dim % 32 != 0)
    return fail(NPD_E_INVALID, "%s: head_dim %lld is not a multiple of 32 in [32, 256]", name,
                (long long)head_dim);
  // head dims 64 and 128: prefill_kernel (key splits, shared K/V tiles);
  // every other one: prefill_generic_kernel
  const bool generic = head_dim != 64 && head_dim != 128;
  if (num_heads % num_kv_heads != 0)
    return fail(NPD_E_INVALID, "%s: num_heads %lld is not a multiple of num_kv_heads %lld", name,
                (long long)num_heads, (long long)num_kv_heads);
  const int64_t g = num_heads / num_kv_heads;
  const int hw = (g % 4 == 0) ? 4 : (g % 2 == 0 ? 2 : 1);   // gcd(g, 4)
  if (num_blocks * block_size * num_kv_heads > INT32_MAX || max_blocks_per_seq * block_size > INT32_MAX)
    return fail(NPD_E_INVALID, "%s: pool exceeds int32 row indexing", name);
  if (!generic && max_blocks_per_seq > kMaxBlocksLds)
    return fail(NPD_E_INVALID, "%s: block tables wider than %d blocks are not supported", name,
                kMaxBlocksLds);
  if (q_stride_token % 8 || q_stride_head % 8 || out_stride_token % 4 || out_stride_head % 4 ||
      q_stride_token < 0 || q_stride_head < 0 || out_stride_token < 0 || out_stride_head < 0)
    return fail(NPD_E_ALIGN, "%s: query strides must be multiples of 8 elements, out strides of 4",
                name);
  if (!(scale > 0.f) || scale == INFINITY)   // the row maxima are taken before scaling
    return fail(NPD_E_INVALID, "%s: scale must be positive and finite", name);
  if (num_seqs == 0 || total_q == 0 || max_q_len == 0) return NPD_OK;
  if (!out || !query || !key_cache || !value_cache || !block_tables || !cu_seqlens_q || !context_lens)
    return fail(NPD_E_INVALID, "%s: null pointer", name);
  if (fp8 && (!k_scale || !v_scale)) return fail(NPD_E_INVALID, "%s: null scale pointer", name);
  const uintptr_t cache_align = fp8 ? 7u : 15u;   // FP8 chunks are 8 bytes
  if (!aligned16(query) || (reinterpret_cast<uintptr_t>(key_cache) & cache_align) != 0 ||
      (reinterpret_cast<uintptr_t>(value_cache) & cache_align) != 0 ||
      (reinterpret_cast<uintptr_t>(out) & 7u) != 0)
    return fail(NPD_E_ALIGN, "%s: query pointer must be 16-byte aligned, caches %d-byte, out 8-byte",
                name, fp8 ? 8 : 16);
  if (generic) {
    const int64_t tiles = (max_q_len + 63) / 64;
    const int64_t grid = (num_seqs * num_kv_heads + 7) / 8 * 8 * tiles * g;
    if (grid > INT32_MAX) return fail(NPD_E_INVALID, "%s: too many tiles", name);
    PrefillArgs a{};
    a.out = static_cast<uint16_t*>(out);
    a.q = static_cast<const uint16_t*>(query);
    a.k_cache = static_cast<const u32x4*>(key_cache);
    a.v_cache = static_cast<const u32x4*>(value_cache);
    a.block_tables = block_tables;
    a.cu_seqlens_q = cu_seqlens_q;
    a.context_lens = context_lens;
    a.k_scale = k_scale;
    a.v_scale = v_scale;
    a.num_seqs = (int)num_seqs;
    a.num_kv_heads = (int)num_kv_heads;
    a.group = (int)g;
    a.block_size = (int)block_size;
    a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctzll((unsigned long long)block_size) : -1;
    a.num_blocks = (int)num_blocks;
    a.max_bps = (int)max_blocks_per_seq;
    a.tiles_max = (int)tiles;
    a.scale_log2 = scale * kLog2e;
    a.q_stride_token = q_stride_token;
    a.q_stride_head = q_stride_head;
    a.out_stride_token = out_stride_token;
    a.out_stride_head = out_stride_head;
    hipStream_t st = as_stream(stream);
    if (dtype == NPD_DTYPE_BF16)
      return fp8 ? launch_generic<BF16, true>(head_dim, a, grid, st, name)
                 : launch_generic<BF16, false>(head_dim, a, grid, st, name);
    return fp8 ? launch_generic<F16, true>(head_dim, a, grid, st, name)
               : launch_generic<F16, false>(head_dim, a, grid, st, name);
  }
  const Layout L = prefill_layout(num_seqs, num_heads, head_dim, max_q_len, max_context_len);
  if (L.total > 0) {
    if (!workspace || workspace_bytes < L.total)
      return fail(NPD_E_WORKSPACE, "%s: workspace of %lld bytes needed, %lld given", name,
                  (long long)L.total, (long long)workspace_bytes);
    if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
      return fail(NPD_E_ALIGN, "%s: workspace must be 256-byte aligned", name);
  }
  const int rt = kPairs / hw;
  const int64_t tiles = (max_q_len + 64LL * rt - 1) / (64LL * rt);
  const int64_t hgroups = g / hw;
  if (L.total > 0 && num_seqs * tiles * num_kv_heads * (g / hw) > kMaxCounters)
    return fail(NPD_E_INVALID, "%s: too many query tiles for the %lld merge counters", name,
                (long long)kMaxCounters);
  const int64_t groups = (int64_t)L.splits * num_seqs * num_kv_heads;
  const int64_t grid = (groups + 7) / 8 * 8 * tiles * hgroups;
  if (grid > INT32_MAX) return fail(NPD_E_INVALID, "%s: too many tiles", name);

  PrefillArgs a;
  a.out = static_cast<uint16_t*>(out);
  a.q = static_cast<const uint16_t*>(query);
  a.k_cache = static_cast<const u32x4*>(key_cache);
  a.v_cache = static_cast<const u32x4*>(value_cache);
  a.block_tables = block_tables;
  a.cu_seqlens_q = cu_seqlens_q;
  a.context_lens = context_lens;
  char* ws = static_cast<char*>(workspace);
  a.counters = L.total > 0 ? reinterpret_cast<int*>(ws) : nullptr;
  a.part_o = L.total > 0 ? reinterpret_cast<float*>(ws + L.o_off) : nullptr;
  a.part_ml = L.total > 0 ? reinterpret_cast<float*>(ws + L.ml_off) : nullptr;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.num_seqs = (int)num_seqs;
  a.num_kv_heads = (int)num_kv_heads;
  a.group = (int)g;
  a.hgroups = (int)hgroups;
  a.block_size = (int)block_size;
  a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctzll((unsigned long long)block_size) : -1;
  a.num_blocks = (int)num_blocks;
  a.max_bps = (int)max_blocks_per_seq;
  a.tiles_max = (int)tiles;
  a.subtiles = (int)(tiles * rt * 2);
  a.splits_max = L.splits;
  a.ks_steps = L.ks_steps;
  a.num_groups = (int)groups;
  a.num_cus = device_cus();
  a.scale_log2 = scale * kLog2e;
  a.q_stride_token = q_stride_token;
  a.q_stride_head = q_stride_head;
  a.out_stride_token = out_stride_token;
  a.out_stride_head = out_stride_head;
  hipStream_t st = as_stream(stream);
  const int64_t elt = fp8 ? 1 : 2;
  const bool off32 = num_blocks * num_kv_heads * block_size * head_dim * elt <= (int64_t)UINT32_MAX;
  if (dtype == NPD_DTYPE_BF16)
    return fp8 ? launch_dt<BF16, true>(head_dim, off32, hw, a, grid, st, name)
               : launch_dt<BF16, false>(head_dim, off32, hw, a, grid, st, name);
  return fp8 ? launch_dt<F16, true>(head_dim, off32, hw, a, grid, st, name)
             : launch_dt<F16, false>(head_dim, off32, hw, a, grid, st, name);
}

}  // namespace

extern "C" int npd_paged_prefill_attention(
    void* out, const void* query, const void* key_cache, const void* value_cache,
    const int32_t* block_tables, const int32_t* cu_seqlens_q, const int32_t* context_lens,
    int64_t num_seqs, int64_t total_q, int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
    int64_t num_blocks, int64_t block_size, int64_t max_blocks_per_seq, int64_t max_q_len,
    int64_t max_context_len, float scale, int64_t q_stride_token, int64_t q_stride_head,
    int64_t out_stride_token, int64_t out_stride_head, void* workspace, int64_t workspace_bytes,
    int32_t dtype, void* stream) {
  return prefill_impl(out, query, key_cache, value_cache, block_tables, cu_seqlens_q,
                      context_lens, nullptr, nullptr, num_seqs, total_q, num_heads, num_kv_heads,
                      head_dim, num_blocks, block_size, max_blocks_per_seq, max_q_len,
                      max_context_len, scale, q_stride_token, q_stride_head, out_stride_token,
                      out_stride_head, workspace, workspace_bytes, dtype, stream, false,
                      "npd_paged_prefill_attention");
}

extern "C" int npd_paged_prefill_attention_fp8(
    void* out, const void* query, const void* key_cache, const void* value_cache,
    const int32_t* block_tables, const int32_t* cu_seqlens_q, const int32_t* context_lens,
    const float* k_scale, const float* v_scale, int64_t num_seqs, int64_t total_q,
    int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, int64_t num_blocks,
    int64_t block_size, int64_t max_blocks_per_seq, int64_t max_q_len, int64_t max_context_len,
    float scale, int64_t q_stride_token, int64_t q_stride_head, int64_t out_stride_token,
    int64_t out_stride_head, void* workspace, int64_t workspace_bytes, int32_t dtype,
    void* stream) {
  return prefill_impl(out, query, key_cache, value_cache, block_tables, cu_seqlens_q,
                      context_lens, k_scale, v_scale, num_seqs, total_q, num_heads, num_kv_heads,
                      head_dim, num_blocks, block_size, max_blocks_per_seq, max_q_len,
                      max_context_len, scale, q_stride_token, q_stride_head, out_stride_token,
                      out_stride_head, workspace, workspace_bytes, dtype, stream, true,
                      "npd_paged_prefill_attention_fp8");
}
