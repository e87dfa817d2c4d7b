// Paged decode attention (one query token per sequence), GQA, split-context.
//
// Reference computation: PA/csrc/attention/paged_attention_kernel.cu:39-151
// (one 128-thread block per (seq, q-head), scores and probabilities rounded to
// the storage type) with host wrapper PA/csrc/attention/paged_attention_ops.cu:7-59;
// the split-context math (partials plus a log-sum-exp merge) follows the
// unbuilt PA/csrc/paged_attention_optimized/paged_attention_optimized.cu:66-219.
//
// MI355X design. The work unit is one wave64 per (sequence, kv-head, context
// partition of PS tokens); the wave serves all G = H / kvh query heads of the
// group, so every K/V row is read from HBM once, not G times.
//   lanes:  a head row of D 2-byte elements is D/8 lanes x 16 bytes (LPT lanes);
//           the wave covers TPL = 64 / LPT tokens per dwordx4 load and a step is
//           16 tokens (NL = 16 / TPL loads of K, later NL loads of V).
//   pass 1: K rows -> q.k with v_dot2_f32_{bf16,f16} (fp32 accumulate), then a
//           butterfly reduce-scatter across the LPT lanes of each token so that
//           each lane ends with its own (token, head) scores; scores go to LDS.
//   pass 2: exact softmax statistics over the partition in LDS (max, exp2, sum),
//           reduced across lanes with shuffles; probabilities stay in fp32.
//   pass 3: V rows -> acc[h][8 dims] += p * v in fp32; rows of the wave are
//           combined with shuffles at the end.
// A sequence that fits in one partition writes its output directly; longer
// ones write fp32 partials (acc, max, sum) and merge_partitions_kernel
// combines them (log-sum-exp merge). 2-byte pools with up to 4 heads per
// group use no MFMA: at one query row per sequence the op is HBM-bound; with
// 5-8 heads pass 3's fp32 products no longer keep up, and it runs on
// v_mfma_f32_16x16x16 (the probabilities rounded to the pool type in place).
// At head dim 128, groups of 5-16 heads (2-byte pools; larger groups as
// units of at most 16) and every group of an FP8 pool run as decode_wide_item
// units instead: one pass per partition with S^T = K.Q^T on
// v_mfma_f32_16x16x32 (K read straight into the operand layout, or staged
// through LDS for 2-byte units of 13-16 heads; the heads padded to 16) and
// O^T += V^T.P^T on v_mfma_f32_16x16x16 (V staged in LDS), probabilities
// formed against a per-head reference that moves only by more than 2^8, and
// no score buffer.
#include <type_traits>

#include "common.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

// O^T += V^T . P^T of the MFMA P.V steps on v_mfma_f32_16x16x16_{bf16,f16}:
// A[m = lane%16][k = 4*(lane/16) + e], B[k = 4*(lane/16) + e][n = lane%16],
// D[m = 4*(lane/16) + i][n = lane%16].
template <class TT>
struct Mfma16;
template <>
struct Mfma16<npd::BF16> {
  static __device__ __forceinline__ f32x4 mma(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                     __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
  }
};
template <>
struct Mfma16<npd::F16> {
  static __device__ __forceinline__ f32x4 mma(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                                 __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
  }
};
// S^T = K . Q^T of decode_wide_item units on v_mfma_f32_16x16x32_{bf16,f16}:
// A[m = lane%16][k = 8*(lane/16) + e], B[k = 8*(lane/16) + e][n = lane%16],
// D[m = 4*(lane/16) + i][n = lane%16].
template <class TT>
struct MfmaK32;
template <>
struct MfmaK32<npd::BF16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b),
                                                   c, 0, 0, 0);
  }
};
template <>
struct MfmaK32<npd::F16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b),
                                                  c, 0, 0, 0);
  }
};
// ds_read_b64_tr_b16 on an LDS address given as a generic pointer to LDS: in
// a group of 16 lanes, lane j receives element j%4 of the 8-byte chunks
// addressed by lanes 4e + j/4, e = 0..3
__device__ __forceinline__ u32x2 lds_read_tr(const uint16_t* p) {
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p)));
}
// LDS row (elements) of the 16-token V tile of the MFMA P.V steps: an 8-bank
// shift per row, so the 4 rows x 32 bytes of a transposing read hit distinct
// banks
constexpr int kVRow = 128 + 16;

constexpr int kMaxPartition = 512;   // tokens per partition, upper bound (LDS sizing)
constexpr int kStep = 16;            // tokens per step
#ifndef NPD_DECODE_RING
#define NPD_DECODE_RING 2
#endif
#ifndef NPD_DECODE_NT
#define NPD_DECODE_NT 1
#endif
constexpr int kRing = NPD_DECODE_RING;   // fast path: K/V steps in flight per wave
// head dim 64: rows of 128 bytes, half the bytes per step; twice the steps in
// flight keep the same bytes in flight (and the same ring registers)
constexpr int ring_of(int d) { return d == 64 ? 2 * kRing : kRing; }
// decode_wide_item units: steps of K and V in flight per wave. FP8 rows are
// half the bytes, so twice the steps keep the same bytes in flight (three
// waves per SIMD); the FP8 form for many units (kHiOcc) keeps two steps and
// four waves per SIMD instead.
#ifndef NPD_WIDE_RING_2B
#define NPD_WIDE_RING_2B 2
#endif
#ifndef NPD_WIDE_RING_FP8
#define NPD_WIDE_RING_FP8 4
#endif
constexpr int wide_ring(bool fp8, bool hi_occ = false) {
  return fp8 ? (hi_occ ? 2 : NPD_WIDE_RING_FP8) : NPD_WIDE_RING_2B;
}
// FP8 pools with up to 8 heads per group: launches of at least this many work
// units ((sequence, kv-head) pairs) take the four-wave form. Config 2 (512
// units): 43.8 against 46.0 us at 4 heads, 43.1 against 44.4 at 1, 46.0
// against 46.5 at 8; config 4 (80 units of 8k-32k tokens, every wave a long
// stream): 87.5 against 74.3 us, so few units keep the deeper ring.
constexpr int64_t kFp8HiOccUnits = 256;

#ifndef NPD_FAST_MAX_PARTITION
#define NPD_FAST_MAX_PARTITION 2048
#endif
constexpr int kFastMaxPartition = NPD_FAST_MAX_PARTITION;   // fast path: tokens per wave, max
// fast path: at most this many scores (tokens x padded heads) per wave: a
// wave's scores then take at most 16.5 KB of LDS, and 9 such waves fit a CU
// (2304 resident on 256 CUs, above kFastMinItems)
constexpr int kFastMaxScores = 4096;
// fast path: the partition is chosen to give at least this many work items
// at the longest context (5 per CU of a 256-CU device)
constexpr int64_t kFastMinItems = 1280;
// fast path, at most 64 sequences: the kernel halves the host's partition
// (down to a quarter of it) while the actual contexts give fewer items
constexpr int kFastMinItemsActual = 1024;
#ifndef NPD_DECODE_INLINE_SCHED_MAX
#define NPD_DECODE_INLINE_SCHED_MAX 64
#endif
constexpr int kInlineSchedMax = NPD_DECODE_INLINE_SCHED_MAX;   // at most 64 (one per lane)
constexpr float kLog2e = 1.4426950408889634f;

constexpr int ilog2(int x) { return x <= 1 ? 0 : 1 + ilog2(x >> 1); }
constexpr int pow2ceil(int x) { return x <= 1 ? 1 : 2 * pow2ceil((x + 1) / 2); }
constexpr int cmin(int a, int b) { return a < b ? a : b; }

__device__ __forceinline__ float shfl_xor(float v, int mask) { return __shfl_xor(v, mask, 64); }

template <class TT>
__device__ __forceinline__ void store_row8(uint16_t* dst, const float* v, float inv) {
  u32x4 w;
  w.x = TT::from_float(v[0] * inv) | (TT::from_float(v[1] * inv) << 16);
  w.y = TT::from_float(v[2] * inv) | (TT::from_float(v[3] * inv) << 16);
  w.z = TT::from_float(v[4] * inv) | (TT::from_float(v[5] * inv) << 16);
  w.w = TT::from_float(v[6] * inv) | (TT::from_float(v[7] * inv) << 16);
  *reinterpret_cast<u32x4*>(dst) = w;
}

struct DecodeArgs {
  uint16_t* out;
  const uint16_t* q;
  const u32x4* k_cache;
  const u32x4* v_cache;
  const int32_t* block_tables;
  const int32_t* seq_lens;
  float* part_acc;   // [S*kvh, max_parts, G, D], then [S*kvh, max_groups, G, D]
  float* part_ml;    // the same slots' (m, l): [..., G, 2]
  int* counters;     // [S*kvh] arrival counters of the fused merge, then
                     // [S*kvh, max_groups] those of its merge groups
  int* sched;        // fast path, more than 64 sequences: [1] number of work items
  const float* k_scale;   // fp8 pool: per-kv-head scales (element = e4m3 byte * scale)
  const float* v_scale;
  int num_seqs;
  int2* items;       // fast path: (unit, partition) work list
  int num_kv_heads;  // kv heads of the work units: pool_kv_heads * kv_split
  int kv_split;      // work units per pool kv head: a group of G > 8 query
                     // heads is served as kv_split groups of G / kv_split
  int pool_kv_heads; // kv heads of the cache layout
  int block_size;
  int num_blocks;
  int max_bps;
  int partition;     // PS, multiple of kStep, <= kMaxPartition (fast path: kFastMaxPartition)
  int min_partition; // fast path, <= 64 sequences: the kernel may halve PS down to this
  int max_parts;
  int max_groups;    // fast path: merge groups per unit (0: one-level merge)
  int head_dim;      // D (the generic path reads it at run time)
  float scale_log2;  // softmax scale * log2(e)
  int64_t q_stride_seq, q_stride_head, out_stride_seq, out_stride_head;
};

// Log-sum-exp merge of the partitions of one (sequence, kv-head) (formula of
// PA/csrc/paged_attention_optimized/paged_attention_optimized.cu:185-217, in
// the log2 domain used by the partition kernels):
//   M = max_p m_p;  L = sum_p l_p 2^(m_p - M);  out = sum_p acc_p 2^(m_p - M) / L
// Threads tid, tid+nthreads, ... each own one (head, 8-dim chunk).
// kCoherent: the partials were written by other waves of the running kernel;
// read them with agent-scope atomic loads (they bypass this XCD's L2).
template <bool kCoherent>
__device__ __forceinline__ float ld_part(const float* p) {
  if constexpr (kCoherent)
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    return *p;
}

template <class TT, int G, bool kCoherent = false>
__device__ __forceinline__ void merge_unit(const DecodeArgs& a, int unit, int s, int kh, int nparts,
                                           int tid, int nthreads) {
  const int64_t base = (int64_t)unit * a.max_parts;
  const int D = a.head_dim;
  const int CH = D / 8;  // 8-dim chunks per head
  for (int idx = tid; idx < G * CH; idx += nthreads) {
    const int h = idx / CH, c = idx % CH;
    float M = -INFINITY;
    for (int p = 0; p < nparts; ++p) M = fmaxf(M, ld_part<kCoherent>(a.part_ml + ((base + p) * G + h) * 2));
    float L = 0.f;
    float o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int p = 0; p < nparts; ++p) {
      const float mp = ld_part<kCoherent>(a.part_ml + ((base + p) * G + h) * 2);
      const float lp = ld_part<kCoherent>(a.part_ml + ((base + p) * G + h) * 2 + 1);
      const float w = __builtin_amdgcn_exp2f(mp - M);
      L = fmaf(lp, w, L);
      const float* src = a.part_acc + (((base + p) * G + h) * D + c * 8);
#pragma unroll
      for (int d = 0; d < 8; ++d) o[d] = fmaf(ld_part<kCoherent>(src + d), w, o[d]);
    }
    store_row8<TT>(a.out + s * a.out_stride_seq + (kh * G + h) * a.out_stride_head + c * 8, o,
                   1.f / L);
  }
}

// Reduce-scatter of decode_partition_kernel's partial dot products over the
// LPT lanes of a token row, stage STEP (partner lane ^ LPT >> (STEP + 1)):
// the first NH stages halve the values a lane holds (it keeps one half and
// adds its partner's copy of it), the rest are plain xor-sums. Stages are
// instantiated one by one, so every index into v is a constant: a loop over
// them was not unrolled, and its run-time indices into v compiled to
// compare-and-select chains over the whole array.
template <int NV, int LPT, int NH, int STEP>
__device__ __forceinline__ void partition_butterfly(float (&v)[NV], int j) {
  if constexpr ((LPT >> (STEP + 1)) >= 1) {
    constexpr int m = LPT >> (STEP + 1);
    if constexpr (STEP < NH) {
      constexpr int half = NV >> (STEP + 1);
      const bool upper = (j & m) != 0;
#pragma unroll
      for (int k = 0; k < half; ++k) {
        const float send = upper ? v[k] : v[k + half];
        const float keep = upper ? v[k + half] : v[k];
        v[k] = keep + shfl_xor(send, m);
      }
    } else {
      v[0] += shfl_xor(v[0], m);
    }
    partition_butterfly<NV, LPT, NH, STEP + 1>(v, j);
  }
}

// LPT: lanes per token row, a power of two >= the row's CPR = D / 8 16-byte
// chunks (D at run time, a multiple of 8 from 32 to 256); lanes j >= CPR of a
// row hold a zero query and load its last chunk (an address inside the row),
// so they add nothing to the dot products and store nothing.
template <class TT, int LPT, int G>
__global__ __launch_bounds__(64) void decode_partition_kernel(DecodeArgs a) {
  static_assert(LPT == 4 || LPT == 8 || LPT == 16 || LPT == 32, "lanes per token row");
  constexpr int TPL = 64 / LPT;          // tokens per load
  constexpr int NL = kStep / TPL;        // loads per step
  constexpr int GP = pow2ceil(G);        // heads padded to a power of two
  constexpr int NV = NL * GP;            // partial dot products per lane per step
  constexpr int LOG_LPT = ilog2(LPT);
  constexpr int NH = cmin(LOG_LPT, ilog2(NV));  // halving steps of the reduce-scatter
  constexpr int HELD = NV >> NH;                 // values a lane keeps
  static_assert(TPL * NL == kStep, "step shape");

  __shared__ float s_p[kMaxPartition * GP];      // scores, then probabilities
  __shared__ int s_blk[kMaxPartition + 1];       // block ids of the partition
  __shared__ float s_ml[2 * GP];                 // per-head max and sum

  const int lane = threadIdx.x;
  const int r = lane / LPT;   // token row within a load
  const int j = lane % LPT;   // 16-byte chunk of the head row
  const int cpr = a.head_dim / 8;          // chunks per head row
  const bool live = j < cpr;               // a chunk of the row (else padding)
  const int jc = live ? j : cpr - 1;       // the chunk this lane loads
  const int unit = blockIdx.x;
  const int s = unit / a.num_kv_heads;
  const int kh = unit - s * a.num_kv_heads;
  const int part = blockIdx.y;

  int ctx = a.seq_lens[s];
  const int cap = a.max_bps * a.block_size;
  ctx = ctx < cap ? ctx : cap;
  if (ctx <= 0) {
    if (part == 0 && lane < LPT && live) {
      const float z[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (int h = 0; h < G; ++h)
        store_row8<TT>(a.out + s * a.out_stride_seq + (kh * G + h) * a.out_stride_head + j * 8, z, 0.f);
    }
    return;
  }
  const int nparts = (ctx + a.partition - 1) / a.partition;
  if (part >= nparts) return;
  const int t0 = part * a.partition;
  const int ntok = (ctx - t0) < a.partition ? (ctx - t0) : a.partition;
  const int nsteps = (ntok + kStep - 1) / kStep;
  const int bs = a.block_size;
  const int b0 = t0 / bs;
  const int nb = (t0 + ntok - 1) / bs - b0 + 1;

  // Block ids of this partition -> LDS, clamped into the pool.
  const int32_t* bt_row = a.block_tables + (int64_t)s * a.max_bps;
  for (int e = lane; e < nb; e += 64) {
    int b = bt_row[b0 + e];
    b = b < 0 ? 0 : (b >= a.num_blocks ? a.num_blocks - 1 : b);
    s_blk[e] = b;
  }

  // Query chunk j of each head in the group, as packed pairs (zero on
  // padding lanes).
  u32x4 qv[G];
  const uint16_t* qbase = a.q + s * a.q_stride_seq + (kh * G) * a.q_stride_head + jc * 8;
#pragma unroll
  for (int h = 0; h < G; ++h) {
    qv[h] = *reinterpret_cast<const u32x4*>(qbase + h * a.q_stride_head);
    if (!live) qv[h] = u32x4{0, 0, 0, 0};
  }
  __syncthreads();

  // rows of the unit's pool kv head inside a block
  const int64_t head_off = (int64_t)(kh / a.kv_split) * bs;
  // power-of-two block sizes (wave-uniform) take a shift, not a division
  const bool bs_pow2 = (bs & (bs - 1)) == 0;
  const int bs_log2 = __builtin_ctz(bs);
  auto row_index = [&](int tl) -> int64_t {
    // 16-byte index of chunk j of token tl (clamped to the last valid token)
    const int t = t0 + (tl < ntok ? tl : ntok - 1);
    const int lb = bs_pow2 ? t >> bs_log2 : t / bs;
    const int off = t - lb * bs;
    const int blk = s_blk[lb - b0];
    return (((int64_t)blk * a.pool_kv_heads * bs) + head_off + off) * cpr + jc;
  };
  // K (pass 1) and V (pass 3) rows run R steps ahead in a register ring
  // (two steps where a step's loads take 32 registers). bench.py, config 2's
  // contexts, ring of 3 -> 4: D 96 126.7 -> 109.5 us, D 128 with blocks of 8
  // 129.4 -> 117.1; a ring of 6 at D 64 with blocks of 8 gained nothing.
  constexpr int R = NL <= 4 ? 4 : 2;
  auto load_rows = [&](const u32x4* __restrict__ pool, u32x4* buf, int st) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NL; ++i) buf[i] = pool[row_index(st * kStep + i * TPL + r)];
  };

  // ---------------- pass 1: scores ----------------
  u32x4 kb[R][NL];
#pragma unroll
  for (int b = 0; b < R; ++b)
    if (b < nsteps) load_rows(a.k_cache, kb[b], b);
  auto score_step = [&](const u32x4* kcur, int st) __attribute__((always_inline)) {
    float v[NV];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
#pragma unroll
      for (int h = 0; h < GP; ++h) {
        float d = 0.f;
        if (h < G) {
          d = TT::dot2(kcur[i].x, qv[h].x, d);
          d = TT::dot2(kcur[i].y, qv[h].y, d);
          d = TT::dot2(kcur[i].z, qv[h].z, d);
          d = TT::dot2(kcur[i].w, qv[h].w, d);
        }
        v[i * GP + h] = d;
      }
    }
    partition_butterfly<NV, LPT, NH, 0>(v, j);
    const int prefix = j >> (LOG_LPT - NH);
#pragma unroll
    for (int e = 0; e < HELD; ++e) {
      const int k = prefix * HELD + e;
      const int i = k / GP, h = k % GP;
      const int tl = st * kStep + i * TPL + r;
      if (h < G) s_p[tl * GP + h] = (tl < ntok) ? v[e] * a.scale_log2 : -INFINITY;
    }
  };
  for (int st0 = 0; st0 < nsteps; st0 += R) {
#pragma unroll
    for (int b = 0; b < R; ++b) {
      const int st = st0 + b;
      if (st < nsteps) {
        score_step(kb[b], st);
        if (st + R < nsteps) load_rows(a.k_cache, kb[b], st + R);
      }
    }
  }

  // Issue the first V loads before the softmax pass so they are in flight.
  u32x4 vb[R][NL];
#pragma unroll
  for (int b = 0; b < R; ++b)
    if (b < nsteps) load_rows(a.v_cache, vb[b], b);
  __syncthreads();

  // ---------------- pass 2: softmax over the partition ----------------
  {
    const int n = nsteps * kStep * GP;
    float m = -INFINITY;
    for (int idx = lane; idx < n; idx += 64) m = fmaxf(m, s_p[idx]);
#pragma unroll
    for (int mask = GP; mask < 64; mask <<= 1) m = fmaxf(m, shfl_xor(m, mask));
    float l = 0.f;
    for (int idx = lane; idx < n; idx += 64) {
      const float p = exp2f(s_p[idx] - m);
      s_p[idx] = p;
      l += p;
    }
#pragma unroll
    for (int mask = GP; mask < 64; mask <<= 1) l += shfl_xor(l, mask);
    if (lane < GP) {
      s_ml[lane] = m;
      s_ml[GP + lane] = l;
    }
  }
  __syncthreads();

  // ---------------- pass 3: probabilities x V ----------------
  // (units of more than 8 heads keep O only in the MFMA accumulators and
  // hand it over through LDS at the end: acc is for groups of up to 8)
  constexpr int GA = G <= 8 ? G : 1;
  float acc[GA][8];
#pragma unroll
  for (int h = 0; h < GA; ++h)
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[h][d] = 0.f;
  auto pv_step = [&](const u32x4* vcur, int st) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int tl = st * kStep + i * TPL + r;
      float p[GP];
#pragma unroll
      for (int h4 = 0; h4 < GP; h4 += 4) {
        if constexpr (GP >= 4) {
          const f32x4 pv = *reinterpret_cast<const f32x4*>(&s_p[tl * GP + h4]);
          p[h4] = pv.x; p[h4 + 1] = pv.y; p[h4 + 2] = pv.z; p[h4 + 3] = pv.w;
        }
      }
      if constexpr (GP < 4) {
#pragma unroll
        for (int h = 0; h < GP; ++h) p[h] = s_p[tl * GP + h];
      }
      const uint32_t w[4] = {vcur[i].x, vcur[i].y, vcur[i].z, vcur[i].w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float f0 = TT::lo(w[c]), f1 = TT::hi(w[c]);
#pragma unroll
        for (int h = 0; h < GA; ++h) {
          acc[h][2 * c] = fmaf(p[h], f0, acc[h][2 * c]);
          acc[h][2 * c + 1] = fmaf(p[h], f1, acc[h][2 * c + 1]);
        }
      }
    }
  };
  for (int st0 = 0; st0 < nsteps; st0 += R) {
#pragma unroll
    for (int b = 0; b < R; ++b) {
      const int st = st0 + b;
      if (st < nsteps) {
        pv_step(vb[b], st);
        if (st + R < nsteps) load_rows(a.v_cache, vb[b], st + R);
      }
    }
  }
  // Combine the TPL token rows of the wave.
#pragma unroll
  for (int mask = LPT; mask < 64; mask <<= 1)
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int d = 0; d < 8; ++d) acc[h][d] += shfl_xor(acc[h][d], mask);

  if (lane >= LPT || !live) return;
  const int D = a.head_dim;
  if (nparts == 1) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float l = s_ml[GP + h];
      store_row8<TT>(a.out + s * a.out_stride_seq + (kh * G + h) * a.out_stride_head + j * 8,
                     acc[h], 1.f / l);
    }
  } else {
    const int64_t base = (int64_t)unit * a.max_parts + part;
#pragma unroll
    for (int h = 0; h < G; ++h) {
      f32x4* dst = reinterpret_cast<f32x4*>(a.part_acc + ((base * G + h) * D + j * 8));
      dst[0] = f32x4{acc[h][0], acc[h][1], acc[h][2], acc[h][3]};
      dst[1] = f32x4{acc[h][4], acc[h][5], acc[h][6], acc[h][7]};
    }
    // (m, l) of every head: the row's live lanes take heads j, j + cpr, ...
    // (cpr may be below G at small head dims)
    for (int h = j; h < G; h += cpr) {
      a.part_ml[(base * G + h) * 2] = s_ml[h];
      a.part_ml[(base * G + h) * 2 + 1] = s_ml[GP + h];
    }
  }
}

// ---------------------------------------------------------------------------
// Fast path: head_dim 128 (any power-of-two block size from 16 to 256) and
// head_dim 64 or 256 (block sizes 16 and 32).
//
// Same work unit and passes as decode_partition_kernel, with the per-step
// cost cut down:
//   * a step is 16 tokens inside one block, so the block id is one readlane
//     per step and every lane's load offsets are loop constants;
//   * the reduce-scatter of the q.k partial sums over the LPT = D/8 lanes of
//     a token row uses DPP: for D 128 the partners are lane^8 (row_ror:8),
//     lane^7 (row_half_mirror), lane^2 and lane^1 (quad_perm); D 64 (8 lanes)
//     takes the last three stages; D 256 (32 lanes) adds lane^16 with
//     v_permlane16_swap (which hands each lane its kept value and its
//     partner's sent one, no select). A lane's partial sums are indexed
//     k = head_slot * NL + token_slot. Stages on head bits need no selects: q
//     slot h of a lane holds head h ^ hmask(lane), chosen so that at every such
//     stage the half a lane keeps is its lower half (one v_add_f32_dpp per
//     value). Stages on token bits pick the kept half with v_cndmask, so the K
//     loads stay the coalesced layout of the V loads.
// ---------------------------------------------------------------------------

using npd::dpp;
using npd::kDppHalfMirror;
using npd::kDppMirror;
using npd::kDppRor8;
using npd::kDppXor1;
using npd::kDppXor2;
using npd::lane_f;
using npd::row_max4;
using npd::row_sum4;
using npd::uniform_f;
using npd::wave_max_f;
using npd::wave_max_i;
using npd::wave_sum_f;
using npd::wave_sum_i;

// Coordinates of lane j (0..15) in the basis of the stage partner masks
// m = (8, 7, 2, 1) of GF(2)^4: j = a1*8 ^ a2*7 ^ a3*2 ^ a4*1, so a1 = j3,
// a2 = j2, a3 = j1 ^ j2, a4 = j0 ^ j2. At stage s the partner lane differs from
// lane j in coordinate a_s only.
__device__ __forceinline__ int bfly_coord(int j, int s) {
  const int j2 = (j >> 2) & 1;
  switch (s) {
    case 1: return (j >> 3) & 1;
    case 2: return j2;
    case 3: return ((j >> 1) & 1) ^ j2;
    default: return (j & 1) ^ j2;
  }
}

__device__ __forceinline__ u32x4 ld_stream(const u32x4* p) {
#if NPD_DECODE_NT
  return __builtin_nontemporal_load(p);
#else
  return *p;
#endif
}

// One reduce-scatter stage over `cnt` values (cnt == 1: plain all-reduce).
// kFree: the kept half is the lower one on every lane (head stages); else
// `upper` picks it (token stages).
template <int CNT, int CTRL, bool kFree>
__device__ __forceinline__ void bfly_stage(float* v, bool upper) {
  if constexpr (CNT >= 2) {
    constexpr int HALF = CNT / 2;
#pragma unroll
    for (int p = 0; p < HALF; ++p) {
      if constexpr (kFree) {
        v[p] += dpp<CTRL>(v[p + HALF]);
      } else {
        const float send = upper ? v[p] : v[p + HALF];
        const float keep = upper ? v[p + HALF] : v[p];
        v[p] = keep + dpp<CTRL>(send);
      }
    }
  } else {
    v[0] += dpp<CTRL>(v[0]);
  }
}

// The lane^16 stage of D 256 (rows of 32 lanes): v_permlane16_swap(A, B)
// exchanges A of the odd 16-lane rows with B of the even ones. With A = v[p]
// and B = v[p + HALF], an even-row lane (keeping the lower half) ends with its
// own v[p] and its partner's v[p], an odd-row lane with its partner's
// v[p + HALF] and its own v[p + HALF]: their sum is kept + received either way.
template <int CNT>
__device__ __forceinline__ void bfly_swap16(float* v) {
  constexpr int HALF = CNT >= 2 ? CNT / 2 : 1;
#pragma unroll
  for (int p = 0; p < HALF; ++p) {
    const uint32_t lo = __float_as_uint(v[p]);
    const uint32_t hi = __float_as_uint(CNT >= 2 ? v[p + HALF] : v[p]);
    const auto sw = __builtin_amdgcn_permlane16_swap(lo, hi, false, false);
    v[p] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
}

// Stage k (0-based) of the reduce-scatter over the D/8 lanes of a token row:
// the coordinate of lane j in that stage's basis direction (which half it
// keeps), and the DPP control of its partner.
template <int D>
__device__ __forceinline__ int stage_coord(int j, int k) {
  if constexpr (D == 64) return bfly_coord(j, k + 2);
  else if constexpr (D == 128) return bfly_coord(j, k + 1);
  else return k < 4 ? bfly_coord(j & 15, k + 1) : (j >> 4) & 1;
}
template <int D>
constexpr int stage_ctrl(int k) {
  return D == 64 ? (k == 0 ? kDppHalfMirror : (k == 1 ? kDppXor2 : kDppXor1))
                 : (k == 0 ? kDppRor8 : (k == 1 ? kDppHalfMirror : (k == 2 ? kDppXor2 : kDppXor1)));
}
// Stage K over NV values (halving while two or more remain, then all-reduce);
// stages below LGP split head bits (free), the rest select by `upper`.
template <int D, int NV, int LGP, int K>
__device__ __forceinline__ void rs_stage(float* v, int j) {
  constexpr int CNT = (NV >> K) >= 2 ? (NV >> K) : 1;
  if constexpr (D == 256 && K == 4) {
    bfly_swap16<CNT>(v);
  } else {
    bfly_stage<CNT, stage_ctrl<D>(K), (K < LGP)>(v, stage_coord<D>(j, K) != 0);
  }
}

using npd::ld_coherent2;
using npd::st_coherent2;

// Merge of one (sequence, kv-head) by a single wave (fast path), the
// same log-sum-exp merge as merge_unit but latency-bound work done in parallel:
//   A: up to 64 partitions, lane p loads (m, l) of partition p for every head,
//      a wave reduction gives M, and the weights 2^(m_p - M) go to LDS (0 past
//      the last partition); the first batch of partial rows is requested at
//      the same time, and the (m, l) registers die before B. More partitions
//      (a second-level merge of over 64 groups): M from a loop over them, no
//      batch in flight meanwhile;
//   B: each lane accumulates its (head, 8-dim chunk) pairs one after the
//      other (one accumulator live), with kMergeFlight partitions of loads in
//      flight. The loads are unconditional (clamped to the chunk's last
//      partition, weight 0), so each wait covers exactly one batch. With more
//      than 64 partitions the weights of each chunk of 64 are read again per
//      chunk and pair (L summed with the first pair).
// This keeps the merge's registers below those of the passes' loops, which
// it would otherwise set for 5-8 heads per group.
// The partials merged are the nparts consecutive slots from slot0. dst >= 0
// (wave-uniform): the result is itself a partial (accumulator and (m, l)
// relative to the merged max, not normalised), written to slot dst; else the
// normalised rows of (sequence s, kv-head kh) go to the output.
constexpr int kMergeFlight = 4;
// decode_wide_item units: a head's probability reference moves only when a step's max
// exceeds it by more than this (log2 units), so probabilities stay <= 2^8
constexpr float kTauDecode = 8.f;
constexpr int kMergeGroup = 16;   // partitions per first-level merge (long contexts)
template <class TT, int D, int G>
__device__ __forceinline__ void merge_unit_fast(const DecodeArgs& a, int64_t slot0, int nparts,
                                                int64_t dst, int s, int kh, int lane, float* s_w,
                                                float oscale) {
  constexpr int GP = pow2ceil(G), CH = D / 8;
  constexpr int OWN = (G * CH + 63) / 64;   // (head, chunk) pairs per lane
  auto slot = [&](int p) -> int64_t { return slot0 + p; };
  // the lane's first (head, chunk) pair, whose first batch of partial rows
  // does not depend on the (m, l) values
  const bool pair0 = lane < G * CH;
  const int h0 = pair0 ? lane / CH : 0, c0 = lane % CH;
  float x[kMergeFlight][8];
  auto load_batch = [&](int p0, int n, int q0, int h, int c) {
#pragma unroll
    for (int q = 0; q < kMergeFlight; ++q) {
      const int pq = p0 + (q0 + q < n ? q0 + q : n - 1);
      const float* src = a.part_acc + (slot(pq) * G + h) * D + c * 2;
#pragma unroll
      for (int k2 = 0; k2 < 4; ++k2) ld_coherent2(src + k2 * (2 * CH), x[q][2 * k2], x[q][2 * k2 + 1]);
    }
  };
  float M[G], L[G];   // wave-uniform (held in scalar registers)
#pragma unroll
  for (int h = 0; h < G; ++h) L[h] = 0.f;
  if (nparts <= 64) {
    // the first batch of partial rows is requested with the (m, l) values;
    // the weights come from the registers, which die here rather than living
    // through the accumulation below
    load_batch(0, nparts, 0, h0, c0);
    float m0[G], l0[G];   // partition `lane`
#pragma unroll
    for (int h = 0; h < G; ++h) { m0[h] = -INFINITY; l0[h] = 0.f; }
    if (lane < nparts) {
#pragma unroll
      for (int h = 0; h < G; ++h) ld_coherent2(a.part_ml + (slot(lane) * G + h) * 2, m0[h], l0[h]);
    }
#pragma unroll
    for (int h = 0; h < G; ++h) M[h] = uniform_f(wave_max_f(m0[h]));
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float w = 0.f, lw = 0.f;
      if (lane < nparts) {
        w = __builtin_amdgcn_exp2f(m0[h] - M[h]);
        lw = l0[h] * w;
      }
      s_w[lane * GP + h] = w;
      L[h] = uniform_f(L[h] + wave_sum_f(lw));
    }
  } else {
    // more than 64 partitions (a second-level merge of over 64 groups): no
    // batch in flight while the maxima are read, so that this rare branch
    // does not set the register peak
#pragma unroll
    for (int h = 0; h < G; ++h) M[h] = -INFINITY;
    for (int p = lane; p < nparts; p += 64) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float mp, lp;
        ld_coherent2(a.part_ml + (slot(p) * G + h) * 2, mp, lp);
        M[h] = fmaxf(M[h], mp);
      }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) M[h] = uniform_f(wave_max_f(M[h]));
  }
  // one (head, chunk) pair of the lane at a time: its accumulator is the
  // only one live (with more than 64 partitions the weights are recomputed
  // per pair; L is summed with the first)
#pragma unroll
  for (int k = 0; k < OWN; ++k) {
    const int idx = lane + 64 * k;
    const bool own = idx < G * CH;
    const int h = own ? idx / CH : 0, c = idx % CH;
    float o[8];
#pragma unroll
    for (int d = 0; d < 8; ++d) o[d] = 0.f;
    for (int p0 = 0; p0 < nparts; p0 += 64) {
      if (nparts > 64) {   // weights of this chunk of 64 partitions
        __syncthreads();   // every lane has read the previous ones
        const int p = p0 + lane;
#pragma unroll
        for (int hh = 0; hh < G; ++hh) {
          float w = 0.f, lw = 0.f;
          if (p < nparts) {
            float mp, lp;
            ld_coherent2(a.part_ml + (slot(p) * G + hh) * 2, mp, lp);
            w = __builtin_amdgcn_exp2f(mp - M[hh]);
            lw = lp * w;
          }
          s_w[lane * GP + hh] = w;
          if (k == 0) L[hh] = uniform_f(L[hh] + wave_sum_f(lw));
        }
      }
      __syncthreads();
      const int n = nparts - p0 < 64 ? nparts - p0 : 64;
      if (own) {
        for (int q0 = 0; q0 < n; q0 += kMergeFlight) {
          if (p0 > 0 || k > 0 || q0 > 0 || nparts > 64) load_batch(p0, n, q0, h, c);
#pragma unroll
          for (int q = 0; q < kMergeFlight; ++q) {
            const float w = s_w[(q0 + q) * GP + h];   // 0 past the chunk's last partition
#pragma unroll
            for (int d = 0; d < 8; ++d) o[d] = fmaf(x[q][d], w, o[d]);
          }
        }
      }
    }
    if (own) {
      if (dst >= 0) {
        // same layout as a published partition: [dim pair][chunk][2]
        float* row = a.part_acc + (dst * G + h) * D + c * 2;
#pragma unroll
        for (int k2 = 0; k2 < 4; ++k2) st_coherent2(row + k2 * (2 * CH), o[2 * k2], o[2 * k2 + 1]);
      } else {
        store_row8<TT>(a.out + s * a.out_stride_seq + (kh * G + h) * a.out_stride_head + c * 8,
                       o, oscale / L[h]);
      }
    }
  }
  __syncthreads();   // s_w is read no more
  if (dst >= 0 && lane == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) st_coherent2(a.part_ml + (dst * G + h) * 2, M[h], L[h]);
  }
}

// decode_wide_item units (head dim 128): S and P.V on the matrix cores, whose
// 16-wide tiles serve 16 heads as cheaply as 8. Groups of up to 16 heads
// (larger ones as the fewest equal units of at most 16) read the kv head's
// K/V rows once instead of once per 8-head sub-group. FP8 pools run every
// group this way (padded to 16
// columns): its 16-byte loads cover whole rows, and at config 2 it beats the
// LDS-staged two-pass form for every group size (48.0 against 51.0 us with 4
// heads, 51.4 against 63.5 with 8). 2-byte pools from 5 heads on (88.0
// against 91.8 us with 6 heads, 90.0 against 93.2 with 8, where the VALU
// kernel ran pass 3 on the matrix cores); with up to 4 heads the VALU kernel
// keeps up with HBM (84.3 against 85.4 us).
constexpr int kWideGroup = 16;
constexpr int kWideMinG2B = 5;
__host__ __device__ constexpr bool wide_item(bool fp8, int g, int d) {
  return d == 128 && g <= kWideGroup && (fp8 || g >= kWideMinG2B);
}
__host__ __device__ constexpr int cmax(int a, int b) { return a > b ? a : b; }

// FP8 (e4m3) element pairs: 8 bytes -> 4 pairs of TT, exact, by
// v_cvt_scalef32_pk_*_fp8 with scale 1 (the per-head scales are applied in
// fp32: to the scores and to the output).
template <class TT>
__device__ __forceinline__ u32x4 e4m3x8_to(u32x2 w) {
  return u32x4{npd::e4m3x2_to<TT, false>(w.x), npd::e4m3x2_to<TT, true>(w.x),
               npd::e4m3x2_to<TT, false>(w.y), npd::e4m3x2_to<TT, true>(w.y)};
}

// Slot of partition `part`'s partial: its own slot, or its merge group's
// result slot when long contexts merge in groups and its group has only it.
__device__ __forceinline__ int64_t partial_slot(const DecodeArgs& a, int unit, int part, int nparts) {
  const int64_t ubase = (int64_t)unit * a.max_parts;
  const bool grouped = a.max_groups > 0 && nparts > kMergeGroup;
  const int g = part / kMergeGroup;
  const int gsize = min(kMergeGroup, nparts - g * kMergeGroup);
  const int64_t gbase =
      (int64_t)a.num_seqs * a.num_kv_heads * a.max_parts + (int64_t)unit * a.max_groups;
  return grouped && gsize == 1 ? gbase + g : ubase + part;
}

// After a wave has issued the stores of its partial (partial_slot): waits for
// them, takes the merge ticket of its partition and, when it is the last of
// the unit's partitions (or of its merge group) to arrive, merges them (then
// the group results, when its group completes them) and resets the counter.
// s_w: the merge's [64][GP] weights in LDS.
template <class TT, int D, int G>
__device__ __forceinline__ void merge_tail(const DecodeArgs& a, int unit, int part, int nparts,
                                           int s, int kh, int lane, float* s_w, float out_scale) {
  const int64_t ubase = (int64_t)unit * a.max_parts;
  const bool grouped = a.max_groups > 0 && nparts > kMergeGroup;
  const int ngroups = (nparts + kMergeGroup - 1) / kMergeGroup;
  const int g = part / kMergeGroup;
  const int gsize = min(kMergeGroup, nparts - g * kMergeGroup);
  const int64_t gbase =
      (int64_t)a.num_seqs * a.num_kv_heads * a.max_parts + (int64_t)unit * a.max_groups;
  auto ticket_of = [&](int* counter) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);   // every store of this wave has completed
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    int t = 0;
    if (lane == 0) t = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return __shfl(t, 0, 64);
  };
  // one merge call site, so that its registers are allocated once
  int* counter = a.counters + unit;
  int64_t slot0 = ubase, dst = -1;
  int n = nparts;
  if (grouped) {
    if (gsize > 1) {   // first level: this partition's group
      counter = a.counters + a.num_seqs * a.num_kv_heads + unit * a.max_groups + g;
      slot0 = ubase + g * kMergeGroup;
      n = gsize;
      dst = gbase + g;
    } else {
      slot0 = gbase;
      n = ngroups;
    }
  }
  for (;;) {
    if (ticket_of(counter) != n - 1) return;
    merge_unit_fast<TT, D, G>(a, slot0, n, dst, s, kh, lane, s_w, dst >= 0 ? 1.f : out_scale);
    if (lane == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (dst < 0) return;
    // second level: the group results
    counter = a.counters + unit;
    slot0 = gbase;
    n = ngroups;
    dst = -1;
  }
}

template <class TT, int D, int G, int SPB>
__device__ __forceinline__ void decode_fast_item(const DecodeArgs& a, int unit, int part,
                                                 int ps, float* s_p) {
  typedef u32x4 raw_t;
  static_assert(D == 64 || D == 128 || D == 256, "head dims of the fast path");
  constexpr int LPT = D / 8;            // lanes per token row (16-byte chunks)
  constexpr int TPL = 64 / LPT;         // token rows per load
  constexpr int NL = 16 / TPL;          // loads per 16-token step (token slots)
  constexpr int NLB = ilog2(NL);
  constexpr int NS = ilog2(LPT);        // reduce-scatter stages
  constexpr int GP = pow2ceil(G);
  constexpr int LGP = ilog2(GP);
  constexpr int NV = NL * GP;           // NL token slots x GP head slots
  constexpr int NB = ilog2(NV);
  constexpr int NH = NB < NS ? NB : NS; // halving stages
  constexpr int HELD = NV >> NH;
  constexpr int NTS = NH > LGP ? NH - LGP : 0;   // token bits split by stages
  constexpr int BS = 16 * SPB;
  constexpr int NBUF = ring_of(D);   // steps in flight per pass
  static_assert(G <= 8 && !wide_item(false, G, D), "group sizes of decode_fast_item (else decode_wide_item)");
  const int lane = threadIdx.x;
  const int r = lane / LPT, j = lane % LPT;
  const int s = unit / a.num_kv_heads;
  const int kh = unit - s * a.num_kv_heads;

  int ctx = a.seq_lens[s];
  const int cap = a.max_bps * BS;
  ctx = ctx < cap ? ctx : cap;
  if (ctx <= 0) {
    if (part == 0 && lane < LPT) {
      const float z[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (int h = 0; h < G; ++h)
        store_row8<TT>(a.out + s * a.out_stride_seq + (kh * G + h) * a.out_stride_head + j * 8, z, 0.f);
    }
    return;
  }
  const int nparts = (ctx + ps - 1) / ps;
  if (part >= nparts) return;
  const int t0 = part * ps;
  const int ntok = (ctx - t0) < ps ? (ctx - t0) : ps;
  // steps rounded up to the ring size; steps past the context read block 0
  // of the pool (always present) and are masked out
  const int nsteps = (((ntok + 15) >> 4) + NBUF - 1) / NBUF * NBUF;
  const int b0 = t0 / BS;

  // stages 0..LGP-1 split head bits (q slots permuted by hmask), the next
  // NTS split token bits, high to low (selects); see stage_coord
  int hmask = 0;
#pragma unroll
  for (int k = 0; k < LGP && k < NS; ++k) hmask |= stage_coord<D>(j, k) << (LGP - 1 - k);
  const int headmask = hmask;
  int tokhi = 0;   // the token-slot bits this lane keeps (the low NLB - NTS bits are held)
#pragma unroll
  for (int t = 0; t < NTS; ++t) tokhi |= stage_coord<D>(j, LGP + t) << (NLB - 1 - t);

  // q slot h holds head h ^ headmask of the group (zeros for padding heads)
  u32x4 qv[GP];
  {
    const uint16_t* qb = a.q + s * a.q_stride_seq + (kh * G) * a.q_stride_head + j * 8;
#pragma unroll
    for (int h = 0; h < GP; ++h) {
      const int hh = h ^ headmask;
      qv[h] = hh < G ? *reinterpret_cast<const u32x4*>(qb + hh * a.q_stride_head) : u32x4{0, 0, 0, 0};
    }
  }
  // lane e holds the block ids of blocks e and 64 + e of the partition
  // (clamped; at most 128 blocks: kFastMaxPartition / 16); entries past the
  // partition hold block 0
  static_assert(kFastMaxPartition / 16 <= 128, "two block ids per lane");
  int myblk0 = 0, myblk1 = 0;
  {
    const int nb = (ntok + BS - 1) / BS;
    const int32_t* row = a.block_tables + (int64_t)s * a.max_bps + b0;
    auto clamp_blk = [&](int b) { return b < 0 ? 0 : (b >= a.num_blocks ? a.num_blocks - 1 : b); };
    if (lane < nb) myblk0 = clamp_blk(row[lane]);
    if (lane + 64 < nb) myblk1 = clamp_blk(row[lane + 64]);
  }
  const int voff = lane;   // offset (in lane chunks) of the lane's chunk r * LPT + j: slot i is token i*TPL + r
  const int pkh = kh / a.kv_split;   // the unit's kv head in the pool
  const float score_scale = a.scale_log2;   // scores in log2 units
  constexpr float out_scale = 1.f;

  const int64_t head_rows = (int64_t)pkh * BS;            // rows of head pkh in a block
  const int64_t blk_rows = (int64_t)a.pool_kv_heads * BS; // rows per block
  auto step_base = [&](int st) -> int64_t {              // chunk index of the step's first row
    const int bi = st / SPB;   // wave-uniform
    const int blk = __builtin_amdgcn_readlane(bi < 64 ? myblk0 : myblk1, bi & 63);
    return ((int64_t)blk * blk_rows + head_rows + (st % SPB) * 16) * LPT;
  };
  // K/V rows are read once per call: nontemporal loads keep them from
  // displacing reusable lines in L2
  auto load_k = [&](raw_t* buf, int st) {
    const int64_t b = step_base(st) + voff;
#pragma unroll
    for (int i = 0; i < NL; ++i) buf[i] = ld_stream(static_cast<const u32x4*>(a.k_cache) + b + i * 64);
  };
  auto load_v = [&](raw_t* buf, int st) {
    const int64_t b = step_base(st) + voff;
#pragma unroll
    for (int i = 0; i < NL; ++i) buf[i] = ld_stream(static_cast<const u32x4*>(a.v_cache) + b + i * 64);
  };

  // ---------------- pass 1: scores ----------------
  float runmax = -INFINITY;   // max of the scores this lane stored (its head: headmask)
  auto score_step = [&](const raw_t* kraw, int st) {
    float v[NV];   // v[h * NL + i]: q slot h . token slot i
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const u32x4 kbi = kraw[i];
#pragma unroll
      for (int h = 0; h < GP; ++h) {
        float d = TT::dot2(kbi.x, qv[h].x, 0.f);
        d = TT::dot2(kbi.y, qv[h].y, d);
        d = TT::dot2(kbi.z, qv[h].z, d);
        d = TT::dot2(kbi.w, qv[h].w, d);
        v[h * NL + i] = d;
      }
    }
    // head stages (free), then token stages (select), then all-reduce
    rs_stage<D, NV, LGP, 0>(v, j);
    rs_stage<D, NV, LGP, 1>(v, j);
    rs_stage<D, NV, LGP, 2>(v, j);
    if constexpr (NS >= 4) rs_stage<D, NV, LGP, 3>(v, j);
    if constexpr (NS >= 5) rs_stage<D, NV, LGP, 4>(v, j);
    // held: head hmask, token slot tokhi | e
#pragma unroll
    for (int e = 0; e < HELD; ++e) {
      const int h = headmask;
      const int ti = tokhi | e;
      const int tl = st * 16 + ti * TPL + r;
      if (h < G) {
        const float sv = (tl < ntok) ? v[e] * score_scale : -INFINITY;
        s_p[tl * GP + h] = sv;
        runmax = fmaxf(runmax, sv);
      }
    }
  };
  {
    // ring of NBUF steps in flight; the last round is peeled so the steady
    // loop has no branches and each wait leaves the newer loads pending
    raw_t kb[NBUF][NL];
#pragma unroll
    for (int b = 0; b < NBUF; ++b) load_k(kb[b], b);
    auto round = [&](int st0) {
#pragma unroll
      for (int b = 0; b < NBUF; ++b) {
        score_step(kb[b], st0 + b);
        load_k(kb[b], st0 + NBUF + b);
      }
    };
    int st0 = 0;
    for (; st0 + NBUF < nsteps; st0 += NBUF) round(st0);
#pragma unroll
    for (int b = 0; b < NBUF; ++b) score_step(kb[b], st0 + b);
  }

  raw_t vb[NBUF][NL];
#pragma unroll
  for (int b = 0; b < NBUF; ++b) load_v(vb[b], b);
  __syncthreads();

  // ---------------- pass 2: softmax statistics over the partition ----------------
  // the maxima come from pass 1's running maxima (DPP wave reductions, one
  // per head over the lanes that stored that head's scores)
  float m[GP], l[GP];
#pragma unroll
  for (int h = 0; h < GP; ++h) {
    m[h] = h < G ? wave_max_f(headmask == h ? runmax : -INFINITY) : -INFINITY;
    l[h] = 0.f;
  }
  const int ntl = nsteps * 16;
  for (int t = lane; t < ntl; t += 64) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float p = __builtin_amdgcn_exp2f(s_p[t * GP + h] - m[h]);
      s_p[t * GP + h] = p;
      l[h] += p;
    }
  }
#pragma unroll
  for (int h = 0; h < G; ++h) l[h] = wave_sum_f(l[h]);
  __syncthreads();

  // ---------------- pass 3: probabilities x V ----------------
  constexpr int GA = G;
  float acc[GA][8];
#pragma unroll
  for (int h = 0; h < GA; ++h)
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[h][d] = 0.f;
  auto pv_step = [&](const raw_t* vraw, int st) {
    u32x4 vbuf[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) vbuf[i] = vraw[i];
    if (st * 16 + 16 > ntok) {   // tail step: rows past the context may hold anything
#pragma unroll
      for (int i = 0; i < NL; ++i)
        if (st * 16 + i * TPL + r >= ntok) vbuf[i] = u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int tl = st * 16 + i * TPL + r;
      float p[GP];
      if constexpr (GP >= 4) {
#pragma unroll
        for (int h4 = 0; h4 < GP; h4 += 4) {
          const f32x4 pv = *reinterpret_cast<const f32x4*>(&s_p[tl * GP + h4]);
          p[h4] = pv.x; p[h4 + 1] = pv.y; p[h4 + 2] = pv.z; p[h4 + 3] = pv.w;
        }
      } else {
#pragma unroll
        for (int h = 0; h < GP; ++h) p[h] = s_p[tl * GP + h];
      }
      const uint32_t w[4] = {vbuf[i].x, vbuf[i].y, vbuf[i].z, vbuf[i].w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float f0 = TT::lo(w[c]), f1 = TT::hi(w[c]);
#pragma unroll
        for (int h = 0; h < GA; ++h) {
          acc[h][2 * c] = fmaf(p[h], f0, acc[h][2 * c]);
          acc[h][2 * c + 1] = fmaf(p[h], f1, acc[h][2 * c + 1]);
        }
      }
    }
  };
  {
    auto round = [&](int st0) {
#pragma unroll
      for (int b = 0; b < NBUF; ++b) {
        pv_step(vb[b], st0 + b);
        load_v(vb[b], st0 + NBUF + b);
      }
    };
    int st0 = 0;
    for (; st0 + NBUF < nsteps; st0 += NBUF) round(st0);
#pragma unroll
    for (int b = 0; b < NBUF; ++b) pv_step(vb[b], st0 + b);
  }
  // sum over the TPL rows of the wave (lanes equal in j): lane ^ 8 by DPP
  // (D 64), then the gfx950 row swaps: v_permlane16_swap / v_permlane32_swap
  // with both operands x hand every lane {x, x of lane ^ 16} (^ 32) in some
  // order
#pragma unroll
  for (int h = 0; h < GA; ++h)
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      float y = acc[h][d];
      if constexpr (TPL >= 8) y += dpp<kDppRor8>(y);
      if constexpr (TPL >= 4) {
        const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y),
                                                          false, false);
        y = __uint_as_float(p16[0]) + __uint_as_float(p16[1]);
      }
      const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y),
                                                        false, false);
      acc[h][d] = __uint_as_float(p32[0]) + __uint_as_float(p32[1]);
    }

  if (nparts == 1) {
    if (lane < LPT) {
#pragma unroll
      for (int h = 0; h < GA; ++h)
        store_row8<TT>(a.out + s * a.out_stride_seq + (kh * G + h) * a.out_stride_head + j * 8,
                       acc[h], out_scale / l[h]);
    }
    return;
  }
  // Several partitions: publish this one's partial, then the last wave of the
  // (sequence, kv-head) to arrive merges them all and resets the counter.
  // Partials go out as agent-scope atomic stores (written through to the
  // device-coherent level) and are read back with agent-scope atomic loads, so
  // no L2 writeback or invalidate is needed; the store completion wait orders
  // them before the counter update.
  // Partial rows are stored transposed, [dim pair k][chunk j][2], so that the
  // LPT lanes of a row write 8 * LPT contiguous bytes per store; after the row
  // reduction every row of the wave holds the sums, so row r stores heads
  // r, r + TPL, ...
  //
  // Long contexts (merge groups on) merge in two levels. The last of each
  // group of kMergeGroup partitions to arrive merges the group into the
  // group's result slot (a partition that is a group of one publishes there
  // directly); the last group to finish merges the group results into the
  // output. Group merges run as groups complete, so the merge left after the
  // last partition covers one group and the group results, not every
  // partition. Group result slots follow the partition slots of all units.
  const int64_t base = partial_slot(a, unit, part, nparts);
#pragma unroll
  for (int h = 0; h < GA; ++h) {
    if ((h % TPL) != r) continue;
    float* dst = a.part_acc + (base * G + h) * D + j * 2;
#pragma unroll
    for (int k = 0; k < 4; ++k) st_coherent2(dst + k * (2 * LPT), acc[h][2 * k], acc[h][2 * k + 1]);
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) st_coherent2(a.part_ml + (base * G + h) * 2, m[h], l[h]);
  }
  merge_tail<TT, D, G>(a, unit, part, nparts, s, kh, lane, s_p, out_scale);
}


// Units of more than kWideKLdsFrom heads over a 2-byte pool stage K through
// LDS: coalesced loads (4 rows x 256 B per load), rows of kKRow elements (one
// 16-byte pad, so the 16 rows a read covers start in different banks). bench.py
// A/B, config 2's contexts, 8 kv heads (direct -> staged, us): 13 heads
// 96.6 -> 94.5, 14 97.6 -> 95.7, 16 98.6 -> 95.9, 32 (two 16-head units)
// 126.6 -> 123.1; but 10 heads 93.5 -> 97.1, 12 94.6 -> 98.1, 6 88.3 -> 90.0,
// 8 90.0 -> 89.5, so smaller units read K straight into the MFMA operand.
constexpr int kWideKLdsFrom = 12;
constexpr int kKRow = 128 + 8;

// LDS of a decode_wide_item unit: the 16 x kVRow V tile and the 16 x kKRow K
// tile, then the 16 x D floats of the O hand-off (every MFMA column) and 16
// (1/l) values after it, then the merge's [64][GP] weights, each from byte 0
// once the one before is no longer read. Independent of the partition.
constexpr int kWideLdsBytes = cmax(cmax(16 * kVRow * 2 + 16 * kKRow * 2, (kWideGroup * 128 + kWideGroup) * 4),
                                   64 * kWideGroup * 4);

// Units of 5-16 heads of a 2-byte pool, and any group of an FP8 pool (padded
// to 16 with zero queries), D = 128: one pass over the partition. Per 16-token
// step of the unit's kv head:
//   S^T = K . Q^T on v_mfma_f32_16x16x32 (4 chunks of 32 dims). Its A
//     operand comes straight from the pool: lane (g4, n16) loads 16 bytes of
//     token n16's row (see load_k), so each load covers 64 contiguous bytes of
//     every row of the step; units of more than kWideKLdsFrom heads over a
//     2-byte pool load K coalesced and read the operand from LDS instead.
//     Lane (g4, n16) ends with the scores of tokens 4*g4 + i of head n16.
//   The head's step max (its 4 scores, then the 4 rows by v_permlane16/32_swap)
//     moves the head's reference only when it exceeds it by more than
//     2^kTauDecode, so probabilities stay <= 2^kTauDecode; a move rescales the
//     head's O accumulators, which the same lanes hold (O^T column n16).
//   The 4 probabilities, rounded to TT, are the B operand of O^T += V^T . P^T
//     on v_mfma_f32_16x16x16 as they stand; the V tile goes through LDS for
//     the transposing reads (ds_read_b64_tr_b16) of the A operand.
// No probability or score buffer: LDS is the V (and K) tile and the hand-off, so the
// partition is as long as the 2-byte path's and many waves fit a CU. K and V
// loads run NBUF steps ahead in a register ring.
template <class TT, int G, int SPB, bool kF8, bool kHiOcc = false, bool kL2 = false>
__device__ __forceinline__ void decode_wide_item(const DecodeArgs& a, int unit, int part, int ps,
                                                 float* s_lds) {
  constexpr int D = 128;
  static_assert(G <= kWideGroup, "a unit's heads fill at most the 16 MFMA columns");
  constexpr int LPT = D / 8;        // 16-byte chunks (FP8: 8-byte) per row
  constexpr int TPL = 64 / LPT;     // rows per coalesced load
  constexpr int NL = 16 / TPL;      // coalesced V loads per step
  constexpr int NKC = D / 32;       // S MFMAs (32-dim chunks) per step
  constexpr int NKL = kF8 ? 2 : 4;  // 16-byte K loads per lane and step
  constexpr int NVL = kF8 ? 2 : NL; // 16-byte V loads per lane and step
  constexpr int NOB = D / 16;       // 16-dim blocks of O^T
  constexpr int BS = 16 * SPB;
  constexpr int NBUF = wide_ring(kF8, kHiOcc);
  constexpr bool kKLds = !kF8 && G > kWideKLdsFrom;   // K staged through LDS
  const int lane = threadIdx.x;
  const int r = lane / LPT, j = lane % LPT;
  const int g4 = lane >> 4, n16 = lane & 15;
  const int s = unit / a.num_kv_heads;
  const int kh = unit - s * a.num_kv_heads;

  int ctx = a.seq_lens[s];
  const int cap = a.max_bps * BS;
  ctx = ctx < cap ? ctx : cap;
  if (ctx <= 0) {
    if (part == 0) {
      const float z[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (int h = r; h < G; h += TPL)
        store_row8<TT>(a.out + s * a.out_stride_seq + (kh * G + h) * a.out_stride_head + j * 8, z, 0.f);
    }
    return;
  }
  const int nparts = (ctx + ps - 1) / ps;
  if (part >= nparts) return;
  const int t0 = part * ps;
  const int ntok = (ctx - t0) < ps ? (ctx - t0) : ps;
  // steps rounded up to the ring size; steps past the context read a block of
  // the pool (clamped ids) and are masked out
  const int nsteps = (((ntok + 15) >> 4) + NBUF - 1) / NBUF * NBUF;
  const int b0 = t0 / BS;
  // lane e holds the block ids of blocks e and 64 + e of the partition
  // (clamped; at most 128 blocks: kFastMaxPartition / 16)
  static_assert(kFastMaxPartition / 16 <= 128, "two block ids per lane");
  int myblk0 = 0, myblk1 = 0;
  {
    const int nb = (ntok + BS - 1) / BS;
    const int32_t* row = a.block_tables + (int64_t)s * a.max_bps + b0;
    auto clamp_blk = [&](int b) { return b < 0 ? 0 : (b >= a.num_blocks ? a.num_blocks - 1 : b); };
    if (lane < nb) myblk0 = clamp_blk(row[lane]);
    if (lane + 64 < nb) myblk1 = clamp_blk(row[lane + 64]);
  }
  const int pkh = kh / a.kv_split;   // the unit's kv head in the pool
  const float score_scale = kF8 ? a.scale_log2 * a.k_scale[pkh] : a.scale_log2;
  const float out_scale = kF8 ? a.v_scale[pkh] : 1.f;
  const int64_t head_rows = (int64_t)pkh * BS;            // rows of head pkh in a block
  const int64_t blk_rows = (int64_t)a.pool_kv_heads * BS; // rows per block
  auto step_base = [&](int st) -> int64_t {              // chunk index of the step's first row
    const int bi = st / SPB;   // wave-uniform
    const int blk = __builtin_amdgcn_readlane(bi < 64 ? myblk0 : myblk1, bi & 63);
    return ((int64_t)blk * blk_rows + head_rows + (st % SPB) * 16) * LPT;
  };
  // K in the MFMA layout, 16-byte loads: load c of lane (g4, n16) = row n16,
  // 16-byte chunk 4c + g4 of the row, so each load covers 64 contiguous bytes
  // of every row of the step. 2-byte pools: dims 32c + 8*g4 .. +7, the A
  // operand of S MFMA c. FP8 (rows of 128 bytes, two loads): dims
  // 64c + 16*g4 .. +15, converted in two halves, the A operands of S MFMAs
  // 2c and 2c + 1 (the head dims are summed in another order; Q follows it)
  // 2-byte pools: nontemporal loads (98.6 us, against 107.3 with plain loads,
  // config 2 with 128 q heads), except where several units read one kv
  // head's rows (kL2: groups above 16 heads; the units' items sit on one XCD,
  // and plain loads let the later ones find the rows in its L2: 256 q heads
  // 154.6 -> 126.3 us, 384 223.2 -> 158.5); FP8 pools: plain loads (46.6 us,
  // against 47.3 with nontemporal ones, config 2)
  auto ld_kv = [](const u32x4* p) -> u32x4 {
    if constexpr (kF8 || kL2) return *p;
    else return ld_stream(p);
  };
  // (kKLds: coalesced like V, load i of lane (r, j) = row i*TPL + r, chunk j)
  auto load_k = [&](u32x4* buf, int st) {
    if constexpr (kKLds) {
      const int64_t b = step_base(st) + lane;
#pragma unroll
      for (int i = 0; i < NKL; ++i) buf[i] = ld_kv(static_cast<const u32x4*>(a.k_cache) + b + i * 64);
    } else {
      const int64_t b = (kF8 ? step_base(st) / 2 + n16 * (LPT / 2) : step_base(st) + n16 * LPT) + g4;
#pragma unroll
      for (int c = 0; c < NKL; ++c) buf[c] = ld_kv(static_cast<const u32x4*>(a.k_cache) + b + 4 * c);
    }
  };
  // V coalesced, 16-byte loads: 2-byte pools: load i of lane (r, j) = row
  // i*TPL + r, chunk j (8 dims); FP8: load i of lane (r8, j8) = row 8i + r8,
  // 16-byte chunk j8 (16 dims), 1 KB contiguous per load
  auto load_v = [&](u32x4* buf, int st) {
    const int64_t b = (kF8 ? step_base(st) / 2 : step_base(st)) + lane;
#pragma unroll
    for (int i = 0; i < NVL; ++i) buf[i] = ld_kv(static_cast<const u32x4*>(a.v_cache) + b + i * 64);
  };
  // Q^T as the B operand of S MFMA c: lane (g4, n16) = head n16, the dims of
  // the K operand (2-byte pools: 32c + 8*g4 .. +7; FP8: 64(c/2) + 16*g4 +
  // 8(c%2) .. +7)
  u32x4 qb[NKC];
  {
    const uint16_t* qrow = a.q + s * a.q_stride_seq + (kh * G + n16) * a.q_stride_head;
#pragma unroll
    for (int c = 0; c < NKC; ++c)   // zeros past the group
      qb[c] = n16 < G ? *reinterpret_cast<const u32x4*>(
                            qrow + (kF8 ? 64 * (c / 2) + 16 * g4 + 8 * (c % 2) : 32 * c + 8 * g4))
                      : u32x4{0, 0, 0, 0};
  }
  uint16_t* s_vt = reinterpret_cast<uint16_t*>(s_lds);
  uint16_t* s_kt = s_vt + 16 * kVRow;   // kKLds: the step's K rows
  // A of the P.V MFMA: V^T[dim nb*16 + n16][tokens 4*g4 .. +3] by transposing
  // reads (lane (g4, n16) addresses token 4*g4 + n16/4, dims nb*16 + 4*(n16%4) .. +3)
  const uint16_t* vl = s_vt + (g4 * 4 + (n16 >> 2)) * kVRow + 4 * (n16 & 3);
  f32x4 oacc[NOB];
#pragma unroll
  for (int nb = 0; nb < NOB; ++nb) oacc[nb] = f32x4{0, 0, 0, 0};
  float mref = -INFINITY;   // head n16's reference (uniform over the 4 rows)
  float lp = 0.f;           // this lane's sum of head n16's rounded probabilities

  auto step = [&](const u32x4* kraw, const u32x4* vraw, int st) {
    // the step's V rows into LDS first (row = token of the step, TT
    // elements), so the writes complete under the S MFMAs and the softmax
    // (the previous step's transposing reads were issued before them); in a
    // tail step rows past the context may hold anything (0 x NaN): zeros
    const bool tail = st * 16 + 16 > ntok;
    if constexpr (kF8) {
#pragma unroll
      for (int i = 0; i < NVL; ++i) {
        const int row = 8 * i + (lane >> 3), c16 = lane & 7;
        u32x4 v0 = e4m3x8_to<TT>(u32x2{vraw[i].x, vraw[i].y});
        u32x4 v1 = e4m3x8_to<TT>(u32x2{vraw[i].z, vraw[i].w});
        if (tail && st * 16 + row >= ntok) v0 = v1 = u32x4{0, 0, 0, 0};
        *reinterpret_cast<u32x4*>(&s_vt[row * kVRow + c16 * 16]) = v0;
        *reinterpret_cast<u32x4*>(&s_vt[row * kVRow + c16 * 16 + 8]) = v1;
      }
    } else {
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        u32x4 v = vraw[i];
        if (tail && st * 16 + i * TPL + r >= ntok) v = u32x4{0, 0, 0, 0};
        *reinterpret_cast<u32x4*>(&s_vt[(i * TPL + r) * kVRow + j * 8]) = v;
      }
    }
    if constexpr (kKLds) {   // rows past the context are masked from the scores below
#pragma unroll
      for (int i = 0; i < NKL; ++i)
        *reinterpret_cast<u32x4*>(&s_kt[(i * TPL + r) * kKRow + j * 8]) = kraw[i];
    }
    // S^T for the step's 16 tokens
    f32x4 sacc = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < NKL; ++c) {
      if constexpr (kF8) {
        sacc = MfmaK32<TT>::mma(e4m3x8_to<TT>(u32x2{kraw[c].x, kraw[c].y}), qb[2 * c], sacc);
        sacc = MfmaK32<TT>::mma(e4m3x8_to<TT>(u32x2{kraw[c].z, kraw[c].w}), qb[2 * c + 1], sacc);
      } else if constexpr (kKLds) {   // row n16, dims 32c + 8*g4 .. +7
        sacc = MfmaK32<TT>::mma(*reinterpret_cast<const u32x4*>(&s_kt[n16 * kKRow + (4 * c + g4) * 8]),
                                qb[c], sacc);
      } else {
        sacc = MfmaK32<TT>::mma(kraw[c], qb[c], sacc);
      }
    }
    float sv[4];
    const int tl = st * 16 + 4 * g4;
#pragma unroll
    for (int i = 0; i < 4; ++i)   // rows past the context may hold anything: select, not scale
      sv[i] = (tl + i < ntok) ? sacc[i] * score_scale : -INFINITY;
    const float x = row_max4(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])));
    float f = 1.f;
    if (x > mref + kTauDecode) {
      f = mref == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mref - x);
      mref = x;
    }
    if (__ballot(f != 1.f) != 0) {   // the first step, then rarely
      lp *= f;
#pragma unroll
      for (int nb = 0; nb < NOB; ++nb) oacc[nb] *= f;
    }
    const float ref = mref == -INFINITY ? 0.f : mref;
    const uint32_t p01 = TT::pack2(__builtin_amdgcn_exp2f(sv[0] - ref), __builtin_amdgcn_exp2f(sv[1] - ref));
    const uint32_t p23 = TT::pack2(__builtin_amdgcn_exp2f(sv[2] - ref), __builtin_amdgcn_exp2f(sv[3] - ref));
    lp += (TT::lo(p01) + TT::hi(p01)) + (TT::lo(p23) + TT::hi(p23));
    const u32x2 pbv = u32x2{p01, p23};
#pragma unroll
    for (int nb = 0; nb < NOB; ++nb) oacc[nb] = Mfma16<TT>::mma(lds_read_tr(vl + nb * 16), pbv, oacc[nb]);
  };
  {
    // ring of NBUF steps in flight; the last round is peeled so the steady
    // loop has no branches and each wait leaves the newer loads pending
    u32x4 kb[NBUF][NKL];
    u32x4 vb[NBUF][NVL];
#pragma unroll
    for (int b = 0; b < NBUF; ++b) {
      load_k(kb[b], b);
      load_v(vb[b], b);
    }
    auto round = [&](int st0) {
#pragma unroll
      for (int b = 0; b < NBUF; ++b) {
        step(kb[b], vb[b], st0 + b);
        load_k(kb[b], st0 + NBUF + b);
        load_v(vb[b], st0 + NBUF + b);
      }
    };
    int st0 = 0;
    for (; st0 + NBUF < nsteps; st0 += NBUF) round(st0);
#pragma unroll
    for (int b = 0; b < NBUF; ++b) step(kb[b], vb[b], st0 + b);
  }
  const float lsum = row_sum4(lp);   // head n16's l (every row)

  // O^T blocks (lane (g4, n16): dims nb*16 + 4*g4 .. +3 of head n16) ->
  // s_o[h][D] and 1/l -> s_il[h], read back per (head, 8-dim chunk). The V
  // and K tiles are no longer read: the last MFMAs, which consume them, feed
  // these stores.
  float* s_o = s_lds;
  float* s_il = s_lds + kWideGroup * D;   // past all 16 columns' rows
#pragma unroll
  for (int nb = 0; nb < NOB; ++nb) *reinterpret_cast<f32x4*>(&s_o[n16 * D + nb * 16 + 4 * g4]) = oacc[nb];
  if (g4 == 0) s_il[n16] = out_scale / lsum;
  const int64_t base = nparts == 1 ? -1 : partial_slot(a, unit, part, nparts);
  // row r of the wave (TPL rows of LPT lanes) writes heads r, r + TPL, ...
#pragma unroll
  for (int h = 0; h < G; ++h) {
    if ((h % TPL) != r) continue;
    const f32x4 lo = *reinterpret_cast<const f32x4*>(&s_o[h * D + j * 8]);
    const f32x4 hi = *reinterpret_cast<const f32x4*>(&s_o[h * D + j * 8 + 4]);
    const float o[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    if (base < 0) {
      store_row8<TT>(a.out + s * a.out_stride_seq + (kh * G + h) * a.out_stride_head + j * 8, o,
                     s_il[h]);
    } else {
      float* dst = a.part_acc + (base * G + h) * D + j * 2;
#pragma unroll
      for (int k = 0; k < 4; ++k) st_coherent2(dst + k * (2 * LPT), o[2 * k], o[2 * k + 1]);
    }
  }
  if (base < 0) return;
  if (g4 == 0 && n16 < G) st_coherent2(a.part_ml + (base * G + n16) * 2, mref, lsum);
  merge_tail<TT, D, G>(a, unit, part, nparts, s, kh, lane, s_lds, out_scale);
}


// Fast-path kernel: workgroup i (one wave) takes item i of the work list that
// decode_schedule_kernel built -- longest sequences first, a unit's partitions
// consecutive -- so long units start together, finish and merge early, and the
// short ones fill the tail. The grid is sized for the most items possible;
// workgroups past the list (all at the end of the grid) exit at once.
// LDS is dynamic, sized for the launch's partition (fast_lds_bytes).
template <class TT, int D, int G, int SPB, bool kF8, bool kHiOcc = false, bool kL2 = false>
// decode_wide_item units: at most 256 VGPRs; they take 149 (2-byte) and 163
// (FP8), three waves per SIMD (four, at 128, ran 5% slower at 16 heads); the
// FP8 four-wave form (kHiOcc, a ring of two steps) takes 118.
__global__ __launch_bounds__(64)
__attribute__((amdgpu_waves_per_eu(wide_item(kF8, G, D) ? (kHiOcc ? 4 : 2) : 1)))
void decode_fast_kernel(DecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) float s_dyn[];
  int unit, part, ps = a.partition;
  if (a.num_seqs <= kInlineSchedMax) {
    // Small batch: every workgroup derives its item from seq_lens alone, in
    // longest-processing-time order:
    //   A. the full partitions (PS tokens) of every sequence but its last,
    //      level by level (partition 0 of every unit, then partition 1, ...);
    //      the level of an item is found by binary search over the counts of
    //      items before each level (DPP wave sums);
    //   B. the last partition of every sequence (PS tokens or fewer; an empty
    //      context has one item that writes zeros), longest first, in 16-token
    //      buckets (binary search over ballot counts).
    // Items past the resident capacity of the GPU start as earlier ones end,
    // so the ones dispatched last are the shortest.
    // The partition is the host's (chosen from the table width) or, when
    // the actual contexts give fewer than kFastMinItemsActual items at that
    // length, the longest of its halves down to a.min_partition that does.
    const int lane = threadIdx.x;
    const int cap = a.max_bps * a.block_size;
    const int kvh = a.num_kv_heads;
    const bool valid = lane < a.num_seqs;
    int c = valid ? a.seq_lens[lane] : 0;
    c = c < cap ? c : cap;
    ps = a.min_partition;
    for (int p = a.partition; p > a.min_partition; p >>= 1) {
      const int sh = __builtin_ctz(p);   // partitions are powers of two
      const int n = valid ? (c > 0 ? (c + p - 1) >> sh : 1) : 0;
      if (wave_sum_i(n) * kvh >= kFastMinItemsActual) {
        ps = p;
        break;
      }
    }
    int full = 0, bucket = 0;   // full partitions before the last; last one's length in 16s
    if (valid && c > 0) {
      full = (c - 1) / ps;
      bucket = (c - full * ps + 15) >> 4;
    }
    // sequence = the k-th set bit of m
    auto nth = [&](uint64_t m, int k) -> int {
      const int rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                 __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
      return __builtin_ctzll(__ballot(((m >> lane) & 1) && rank == k));
    };
    // items before level p: kvh * sum over sequences of min(full, p)
    auto before = [&](int p) -> int { return wave_sum_i(full < p ? full : p) * kvh; };
    const int maxfull = wave_max_i(full);
    int id = blockIdx.x, seq = -1;
    {
      // Workgroups go to the 8 XCDs round-robin (blockIdx % 8) and, within
      // an XCD, to its 32 CUs in turn, so in longest-first order the same
      // CUs would take the longest item of every round of 256. Every other
      // full round is reversed within each XCD (a "snake"), so each CU's
      // items pair long with short. Only full rounds are permuted: the map
      // stays a bijection of [0, grid).
      const int xcd = id & 7, pos = id >> 3, rnd = pos >> 5;
      if ((rnd & 1) != 0 && (rnd + 1) * 256 <= (int)gridDim.x)
        id = ((rnd * 32 + (31 - (pos & 31))) << 3) | xcd;
    }
    if (a.kv_split > 1) {
      // The kv_split units of one pool kv head have consecutive item ids
      // (every level and bucket starts at a multiple of the unit count).
      // Their blockIdx values are made 8 apart -- the same XCD, as
      // workgroups go to the 8 XCDs round-robin -- so the K/V rows the first
      // unit reads are in that XCD's L2 for the others. The grid is a
      // multiple of 8 * kv_split, so this permutes [0, grid).
      const int span = 8 * a.kv_split, q = id / span, rem = id - q * span;
      id = q * span + (rem & 7) * a.kv_split + (rem >> 3);
    }
    part = 0;
    const int nfull = before(maxfull);
    if (id < nfull) {
      // level of item id: the last p with before(p) <= id (binary search)
      int lo = 0, hi = maxfull - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (before(mid) <= id) lo = mid; else hi = mid - 1;
      }
      id -= before(lo);
      seq = nth(__ballot(full > lo), id / kvh);
      unit = seq * kvh + id % kvh;
      part = lo;
    } else {
      id -= nfull;
    }
    if (seq < 0) {
      // items in buckets >= b, non-increasing in b; item id is in the last
      // bucket b with from(b) > id (binary search)
      auto from = [&](int b) -> int { return __popcll(__ballot(valid && bucket >= b)) * kvh; };
      if (id >= from(0)) return;   // past the last item
      int lo = 0, hi = ps >> 4;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (from(mid) > id) lo = mid; else hi = mid - 1;
      }
      id -= from(lo + 1);
      seq = nth(__ballot(valid && bucket == lo), id / kvh);
      unit = seq * kvh + id % kvh;
      part = __builtin_amdgcn_readlane(full, seq);
    }
  } else {
    if ((int)blockIdx.x >= a.sched[1]) return;
    const int2 it = a.items[blockIdx.x];
    unit = it.x;
    part = it.y;
  }
  if constexpr (wide_item(kF8, G, D))
    decode_wide_item<TT, G, SPB, kF8, kHiOcc, kL2>(a, unit, part, ps, s_dyn);
  else
    decode_fast_item<TT, D, G, SPB>(a, unit, part, ps, s_dyn);
}

// Builds the work list of decode_fast_kernel (one workgroup):
//   - zeroes the merge counters (per unit and per merge group);
//   - counting-sorts the sequences by partition count, descending;
//   - lists the items of each sequence in that order, unit by unit
//     (item = (unit, partition)); a sequence with no context gets one item,
//     which writes zeros.
constexpr int kSchedThreads = 1024;
constexpr int kSchedMaxSeqs = 4096;
constexpr int kSchedBins = 1024;

__global__ __launch_bounds__(kSchedThreads) void decode_schedule_kernel(DecodeArgs a, int num_seqs) {
  __shared__ int s_np[kSchedMaxSeqs];      // partitions per sequence
  __shared__ int s_order[kSchedMaxSeqs];   // sequences, most partitions first
  __shared__ int s_offs[kSchedMaxSeqs];    // first item of each sorted sequence
  __shared__ int s_hist[kSchedBins];
  __shared__ int s_wsum[kSchedThreads / 64];
  __shared__ int s_carry;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int kvh = a.num_kv_heads;
  const int cap = a.max_bps * a.block_size;
  const int units = num_seqs * kvh;
  auto bin_of = [](int np) { return kSchedBins - 1 - (np < kSchedBins ? np : kSchedBins - 1); };
  // block-wide exclusive scan of one value per thread (chunk of kSchedThreads)
  auto block_scan = [&](int c, int carry_in) {
    int inc = c;
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(inc, o, 64);
      if (lane >= o) inc += v;
    }
    if (lane == 63) s_wsum[wid] = inc;
    __syncthreads();
    int pre = carry_in;
    for (int w = 0; w < wid; ++w) pre += s_wsum[w];
    __syncthreads();
    return pre + inc - c;   // exclusive prefix; pre + inc is the inclusive one
  };
  for (int u = tid; u < units * (1 + a.max_groups); u += kSchedThreads) a.counters[u] = 0;
  s_hist[tid] = 0;
  __syncthreads();
  for (int sq = tid; sq < num_seqs; sq += kSchedThreads) {
    int c = a.seq_lens[sq];
    c = c < cap ? c : cap;
    const int np = c <= 0 ? 1 : (c + a.partition - 1) / a.partition;
    s_np[sq] = np;
    atomicAdd(&s_hist[bin_of(np)], 1);
  }
  __syncthreads();
  static_assert(kSchedBins == kSchedThreads, "one bin per thread");
  const int start = block_scan(s_hist[tid], 0);
  s_hist[tid] = start;
  __syncthreads();
  for (int sq = tid; sq < num_seqs; sq += kSchedThreads)
    s_order[atomicAdd(&s_hist[bin_of(s_np[sq])], 1)] = sq;
  __syncthreads();
  int carry = 0;
  for (int base = 0; base < num_seqs; base += kSchedThreads) {
    const int k = base + tid;
    const int cnt = k < num_seqs ? kvh * s_np[s_order[k]] : 0;
    const int ex = block_scan(cnt, carry);
    if (k < num_seqs) s_offs[k] = ex;
    if (tid == kSchedThreads - 1) s_carry = ex + cnt;
    __syncthreads();
    carry = s_carry;
    __syncthreads();
  }
  if (tid == 0) a.sched[1] = carry;
  // items of sorted sequence k: (unit kh, partition p) for kh < kvh, p < np,
  // unit by unit; one wave per sequence
  for (int k = wid; k < num_seqs; k += kSchedThreads / 64) {
    const int sq = s_order[k], np = s_np[sq], n = kvh * np, o = s_offs[k];
    for (int e = lane; e < n; e += 64) {
      const int kh = e / np;
      a.items[o + e] = make_int2(sq * kvh + kh, e - kh * np);
    }
  }
}

// Merge kernel for the generic path: one workgroup per (sequence, kv-head).
template <class TT, int G>
__global__ __launch_bounds__(256) void merge_partitions_kernel(DecodeArgs a) {
  const int unit = blockIdx.x;
  const int s = unit / a.num_kv_heads;
  const int kh = unit - s * a.num_kv_heads;
  int ctx = a.seq_lens[s];
  const int cap = a.max_bps * a.block_size;
  ctx = ctx < cap ? ctx : cap;
  if (ctx <= 0) return;
  const int nparts = (ctx + a.partition - 1) / a.partition;
  if (nparts <= 1) return;
  merge_unit<TT, G>(a, unit, s, kh, nparts, threadIdx.x, blockDim.x);
}

bool use_fast_path(int64_t head_dim, int64_t block_size, int64_t num_seqs) {
  if (num_seqs > kSchedMaxSeqs) return false;
  if (head_dim == 128)
    return block_size % 16 == 0 && block_size <= 256 && (block_size & (block_size - 1)) == 0;
  return (head_dim == 64 || head_dim == 256) && (block_size == 16 || block_size == 32);
}

// Partition length (tokens per wave). The fast path takes the longest of
// 2048 / 1024 / ... / 64 tokens (at most kFastMaxScores / GP) that gives
// kFastMinItems work items at the longest context, never below the block
// size. Long partitions cost less per token: each work item pays a fixed
// latency (work-list lookup, q load, the softmax pass over LDS, publishing
// its partial) that the streaming loops of other waves hide only in part,
// and 1280 waves with two 16-token steps in flight each still keep HBM busy.
// decode_wide_item units (16 heads; every FP8 group) have no score buffer,
// so no score limit: for FP8 pools the 2-byte rules beat shorter partitions
// (57.6 against 72 us at 256 tokens and 4096 items, config 2 with 128 q
// heads; 88 against 94 us at 1024 tokens with 256 q heads). The generic path
// uses 512 or 256. The workspace is sized with the same rule.
int choose_partition(int64_t num_seqs, int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                     int64_t block_size, int64_t max_ctx, bool fp8) {
  const int64_t units = num_seqs * num_kv_heads;
  if (use_fast_path(head_dim, block_size, num_seqs)) {
#ifdef NPD_DECODE_PARTITION
    if (NPD_DECODE_PARTITION >= block_size) return NPD_DECODE_PARTITION;
#endif
    const int gp = pow2ceil((int)(num_heads / num_kv_heads));
    const bool wide = wide_item(fp8, (int)(num_heads / num_kv_heads), (int)head_dim);
    for (int ps = kFastMaxPartition; ps >= 64; ps >>= 1) {
      if (ps <= block_size) return (int)block_size;
      if (ps * gp > kFastMaxScores && !wide) continue;
      if (units * ((max_ctx + ps - 1) / ps) >= kFastMinItems) return ps;
    }
    return block_size > 64 ? (int)block_size : 64;
  }
  return units * ((max_ctx + 511) / 512) >= 4096 ? 512 : 256;
}

// Shortest partition the fast path's kernel may take for a host partition ps
// (down to ps / 4, never below 64 tokens or the block); the workspace and the
// grid are sized for it.
int fast_min_partition(int ps, int64_t block_size) {
  int lo = ps / 4;
  lo = lo < 64 ? 64 : lo;
  lo = lo < block_size ? (int)block_size : lo;
  return lo < ps ? lo : ps;
}

// Grid of the fast path: the items at the host's partition or, when the
// kernel may halve it, at most 2 * kFastMinItemsActual - 2 (it halves only
// while a length gives fewer than kFastMinItemsActual items, and halving at
// most doubles the count), within the slots the workspace holds.
int64_t fast_grid(const DecodeArgs& a, int64_t units) {
  const int64_t max_ctx = (int64_t)a.max_bps * a.block_size;
  int64_t n = units * ((max_ctx + a.partition - 1) / a.partition);
  if (a.min_partition < a.partition) {
    int64_t h = units * a.max_parts;
    h = h < 2 * kFastMinItemsActual ? h : 2 * kFastMinItemsActual;
    n = n > h ? n : h;
  }
  if (a.kv_split > 1 && a.num_seqs <= kInlineSchedMax) {   // whole spans of the XCD permutation
    const int64_t span = 8 * a.kv_split;
    n = (n + span - 1) / span * span;
  }
  return n;
}

// Dynamic LDS of decode_fast_kernel for a partition: scores (fp32) of every
// token of the partition plus the ring padding (decode_fast_item; see
// fast_score_floats), or kWideLdsBytes for decode_wide_item units, for any
// partition.
int64_t fast_lds_bytes(int partition, int g, bool fp8, int d) {
  if (wide_item(fp8, g, d)) return kWideLdsBytes;
  const int t = partition + 16 * ring_of(d);
  return (int64_t)t * pow2ceil(g) * 4;
}

template <class TT, int D, int G, int SPB, bool kF8 = false, bool kHiOcc = false, bool kL2 = false>
int launch_fast_bs(const DecodeArgs& a, int num_seqs, int64_t max_items, hipStream_t st) {
  if (num_seqs > kInlineSchedMax)
    hipLaunchKernelGGL(decode_schedule_kernel, dim3(1), dim3(kSchedThreads), 0, st, a, num_seqs);
  hipLaunchKernelGGL((decode_fast_kernel<TT, D, G, SPB, kF8, kHiOcc, kL2>), dim3((unsigned)max_items), dim3(64),
                     (unsigned)fast_lds_bytes(a.partition, G, kF8, D), st, a);
  return NPD_OK;
}

template <class TT, int D, int G>
int launch_fast(const DecodeArgs& a, int num_seqs, int64_t max_items, hipStream_t st) {
  if constexpr (D != 128 || G > 8) {   // block sizes 16 and 32 (use_fast_path, kv_split_of)
    if constexpr (D == 128 && G > 8) {
      if (a.kv_split > 1) {   // several units per kv head: plain loads (kL2)
        if (a.block_size == 16) return launch_fast_bs<TT, D, G, 1, false, false, true>(a, num_seqs, max_items, st);
        return launch_fast_bs<TT, D, G, 2, false, false, true>(a, num_seqs, max_items, st);
      }
    }
    if (a.block_size == 16) return launch_fast_bs<TT, D, G, 1>(a, num_seqs, max_items, st);
    return launch_fast_bs<TT, D, G, 2>(a, num_seqs, max_items, st);
  } else {
    switch (a.block_size) {
      case 16: return launch_fast_bs<TT, D, G, 1>(a, num_seqs, max_items, st);
      case 32: return launch_fast_bs<TT, D, G, 2>(a, num_seqs, max_items, st);
      case 64: return launch_fast_bs<TT, D, G, 4>(a, num_seqs, max_items, st);
      case 128: return launch_fast_bs<TT, D, G, 8>(a, num_seqs, max_items, st);
      default: return launch_fast_bs<TT, D, G, 16>(a, num_seqs, max_items, st);
    }
  }
}

// FP8 pools: the fast path only, head_dim 128, block sizes 16 and 32; with up
// to 8 heads per group and at least kFp8HiOccUnits units, the four-wave form
template <class TT, int G>
int launch_fast_fp8(const DecodeArgs& a, int num_seqs, int64_t max_items, hipStream_t st) {
  if constexpr (G <= 8) {
    if ((int64_t)num_seqs * a.num_kv_heads >= kFp8HiOccUnits) {
      if (a.block_size == 16) return launch_fast_bs<TT, 128, G, 1, true, true>(a, num_seqs, max_items, st);
      return launch_fast_bs<TT, 128, G, 2, true, true>(a, num_seqs, max_items, st);
    }
  }
  if (a.block_size == 16) return launch_fast_bs<TT, 128, G, 1, true>(a, num_seqs, max_items, st);
  return launch_fast_bs<TT, 128, G, 2, true>(a, num_seqs, max_items, st);
}

template <class TT>
int dispatch_fp8(int g, const DecodeArgs& a, int64_t units, hipStream_t st) {
  const int ns = (int)(units / a.num_kv_heads);
  const int64_t mi = fast_grid(a, units);
  switch (g) {
    case 1: launch_fast_fp8<TT, 1>(a, ns, mi, st); break;
    case 2: launch_fast_fp8<TT, 2>(a, ns, mi, st); break;
    case 3: launch_fast_fp8<TT, 3>(a, ns, mi, st); break;
    case 4: launch_fast_fp8<TT, 4>(a, ns, mi, st); break;
    case 5: launch_fast_fp8<TT, 5>(a, ns, mi, st); break;
    case 6: launch_fast_fp8<TT, 6>(a, ns, mi, st); break;
    case 7: launch_fast_fp8<TT, 7>(a, ns, mi, st); break;
    case 9: launch_fast_fp8<TT, 9>(a, ns, mi, st); break;
    case 10: launch_fast_fp8<TT, 10>(a, ns, mi, st); break;
    case 11: launch_fast_fp8<TT, 11>(a, ns, mi, st); break;
    case 12: launch_fast_fp8<TT, 12>(a, ns, mi, st); break;
    case 13: launch_fast_fp8<TT, 13>(a, ns, mi, st); break;
    case 14: launch_fast_fp8<TT, 14>(a, ns, mi, st); break;
    case 15: launch_fast_fp8<TT, 15>(a, ns, mi, st); break;
    case kWideGroup: launch_fast_fp8<TT, kWideGroup>(a, ns, mi, st); break;
    default: launch_fast_fp8<TT, 8>(a, ns, mi, st); break;
  }
  return npd::check_launch("npd_paged_attention_fp8");
}

// Generic path: any head dim (a multiple of 8 from 32 to 256), block size and
// batch; a wave's lanes per token row are the next power of two above D / 8.
template <class TT, int G>
int launch_generic(const DecodeArgs& a, int64_t units, hipStream_t st) {
  const dim3 grid((unsigned)units, (unsigned)a.max_parts);
  const int cpr = a.head_dim / 8;
  if (cpr <= 4)
    hipLaunchKernelGGL((decode_partition_kernel<TT, 4, G>), grid, dim3(64), 0, st, a);
  else if (cpr <= 8)
    hipLaunchKernelGGL((decode_partition_kernel<TT, 8, G>), grid, dim3(64), 0, st, a);
  else if (cpr <= 16)
    hipLaunchKernelGGL((decode_partition_kernel<TT, 16, G>), grid, dim3(64), 0, st, a);
  else
    hipLaunchKernelGGL((decode_partition_kernel<TT, 32, G>), grid, dim3(64), 0, st, a);
  if (a.max_parts > 1)
    hipLaunchKernelGGL((merge_partitions_kernel<TT, G>), dim3((unsigned)units), dim3(256), 0, st, a);
  return npd::check_launch("npd_paged_attention");
}

template <class TT, int D, int G>
int launch_decode(const DecodeArgs& a, int64_t units, hipStream_t st) {
  if (use_fast_path(D, a.block_size, units / a.num_kv_heads)) {
    const int rc = launch_fast<TT, D, G>(a, (int)(units / a.num_kv_heads), fast_grid(a, units), st);
    if (rc != NPD_OK) return rc;
    return npd::check_launch("npd_paged_attention");
  }
  if constexpr (G > 8)   // kv_split_of forms units of 9-16 heads on the fast path only
    return npd::fail(NPD_E_INVALID, "npd_paged_attention: no kernel for %d-head units here", G);
  else
    return launch_generic<TT, G>(a, units, st);
}

template <class TT, int D>
int dispatch_g(int g, const DecodeArgs& a, int64_t units, hipStream_t st) {
  if constexpr (D == 128) {
    switch (g) {   // one-pass units of 9-16 heads (kv_split_of: blocks of 16 or 32)
      case 9: return launch_decode<TT, 128, 9>(a, units, st);
      case 10: return launch_decode<TT, 128, 10>(a, units, st);
      case 11: return launch_decode<TT, 128, 11>(a, units, st);
      case 12: return launch_decode<TT, 128, 12>(a, units, st);
      case 13: return launch_decode<TT, 128, 13>(a, units, st);
      case 14: return launch_decode<TT, 128, 14>(a, units, st);
      case 15: return launch_decode<TT, 128, 15>(a, units, st);
      case kWideGroup: return launch_decode<TT, 128, kWideGroup>(a, units, st);
      default: break;
    }
  }
  switch (g) {
    case 1: return launch_decode<TT, D, 1>(a, units, st);
    case 2: return launch_decode<TT, D, 2>(a, units, st);
    case 3: return launch_decode<TT, D, 3>(a, units, st);
    case 4: return launch_decode<TT, D, 4>(a, units, st);
    case 5: return launch_decode<TT, D, 5>(a, units, st);
    case 6: return launch_decode<TT, D, 6>(a, units, st);
    case 7: return launch_decode<TT, D, 7>(a, units, st);
    default: return launch_decode<TT, D, 8>(a, units, st);
  }
}

template <class TT>
int dispatch_generic_g(int g, const DecodeArgs& a, int64_t units, hipStream_t st) {
  switch (g) {
    case 1: return launch_generic<TT, 1>(a, units, st);
    case 2: return launch_generic<TT, 2>(a, units, st);
    case 3: return launch_generic<TT, 3>(a, units, st);
    case 4: return launch_generic<TT, 4>(a, units, st);
    case 5: return launch_generic<TT, 5>(a, units, st);
    case 6: return launch_generic<TT, 6>(a, units, st);
    case 7: return launch_generic<TT, 7>(a, units, st);
    default: return launch_generic<TT, 8>(a, units, st);
  }
}

template <class TT>
int dispatch_d(int64_t d, int g, const DecodeArgs& a, int64_t units, hipStream_t st) {
  switch (d) {
    case 64: return dispatch_g<TT, 64>(g, a, units, st);
    case 128: return dispatch_g<TT, 128>(g, a, units, st);
    case 256: return dispatch_g<TT, 256>(g, a, units, st);
    default: return dispatch_generic_g<TT>(g, a, units, st);
  }
}

// Work units per pool kv head. At head dim 128 with blocks of 16 or 32 (the
// fast path) the one-pass units serve up to 16 heads in their MFMA columns, so
// a group of more than 8 heads runs as the fewest equal units of at most 16
// heads (one for 9-16, two of 12 for 24, two of 16 for 32), each reading the
// kv head's K/V rows once. Otherwise the kernels keep a group's queries and
// accumulators in registers for at most 8 query heads: a larger group is
// served as kv_split equal groups of at most 8 heads (the smallest such
// split), each reading the kv head's K/V.
int kv_split_of(int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, int64_t block_size,
                int64_t num_seqs) {
  const int64_t g = num_kv_heads > 0 ? num_heads / num_kv_heads : 1;
  const int64_t cap = g > 8 && head_dim == 128 && (block_size == 16 || block_size == 32) &&
                              use_fast_path(head_dim, block_size, num_seqs)
                          ? kWideGroup : 8;
  int64_t k = 1;
  while (k < g && (g / k > cap || g % k != 0)) ++k;
  return (int)k;
}

// Merge groups per unit of the fast path's two-level merge (0: one level):
// used when a unit has more than one group of partitions and the counter
// region holds a counter per unit and per group.
int64_t merge_groups(bool fast, int64_t units, int64_t parts) {
  const int64_t ng = (parts + kMergeGroup - 1) / kMergeGroup;
  return fast && parts > kMergeGroup && units * (1 + ng) <= npd::kMaxCounters ? ng : 0;
}

}  // namespace

extern "C" int64_t npd_paged_attention_workspace_size(int64_t num_seqs, int64_t num_heads,
                                                      int64_t num_kv_heads, int64_t head_dim,
                                                      int64_t block_size,
                                                      int64_t max_blocks_per_seq) {
  if (num_seqs <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
      max_blocks_per_seq <= 0)
    return 0;
  num_kv_heads *= kv_split_of(num_heads, num_kv_heads, head_dim, block_size, num_seqs);   // units' kv heads
  const int64_t max_ctx = block_size * max_blocks_per_seq;
  if (!use_fast_path(head_dim, block_size, num_seqs)) {
    const int ps =
        choose_partition(num_seqs, num_heads, num_kv_heads, head_dim, block_size, max_ctx, false);
    const int64_t parts = (max_ctx + ps - 1) / ps;
    if (parts <= 1) return 0;
    return npd::kCounterBytes + num_seqs * num_heads * parts * (head_dim + 2) * (int64_t)sizeof(float);
  }
  // fast path: counter region, item count (16 B), work list, partials of the
  // partitions and of the merge groups; enough for a 2-byte pool and, for the
  // block sizes the FP8 entry point takes, an FP8 pool (whose partitions may
  // differ: no score limit)
  const int64_t units = num_seqs * num_kv_heads;
  auto need = [&](bool fp8) {
    const int ps = fast_min_partition(
        choose_partition(num_seqs, num_heads, num_kv_heads, head_dim, block_size, max_ctx, fp8),
        block_size);
    const int64_t parts = (max_ctx + ps - 1) / ps;
    const int64_t slots = parts + merge_groups(true, units, parts);
    return (npd::kCounterBytes + 16 + units * parts * 8 + 255) / 256 * 256 +
           num_seqs * num_heads * slots * (head_dim + 2) * (int64_t)sizeof(float);
  };
  const int64_t n = need(false);
  if (block_size != 16 && block_size != 32) return n;
  const int64_t n8 = need(true);
  return n8 > n ? n8 : n;
}

namespace {

// Argument checks of every decode entry point (everything but the workspace),
// before any launch: NPD_OK or the error code, with the message set.
int attention_check(const void* out, const void* query, const void* key_cache,
                    const void* value_cache, const int32_t* block_tables, const int32_t* seq_lens,
                    int64_t num_seqs, int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                    int64_t num_blocks, int64_t block_size, int64_t max_blocks_per_seq,
                    int64_t q_stride_seq, int64_t q_stride_head, int64_t out_stride_seq,
                    int64_t out_stride_head, const float* k_scale, const float* v_scale,
                    int32_t dtype, bool fp8, const char* name) {
  using namespace npd;
  if (dtype != NPD_DTYPE_F16 && dtype != NPD_DTYPE_BF16)
    return fail(NPD_E_DTYPE, "%s: unsupported dtype code %d (fp16/bf16 only)", name, dtype);
  if (num_seqs < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_blocks <= 0 ||
      block_size <= 0 || max_blocks_per_seq <= 0)
    return fail(NPD_E_INVALID,
                "%s: bad sizes (seqs %lld, heads %lld, kv heads %lld, blocks %lld, block %lld, "
                "max blocks/seq %lld)", name, (long long)num_seqs, (long long)num_heads,
                (long long)num_kv_heads, (long long)num_blocks, (long long)block_size,
                (long long)max_blocks_per_seq);
  if (num_heads % num_kv_heads != 0)
    return fail(NPD_E_INVALID, "%s: num_heads %lld is not a multiple of num_kv_heads %lld", name,
                (long long)num_heads, (long long)num_kv_heads);
  // the work units' kv heads and group size (groups above 8 heads are split)
  const int split = kv_split_of(num_heads, num_kv_heads, head_dim, block_size, num_seqs);
  const int64_t pool_kv_heads = num_kv_heads;
  num_kv_heads *= split;
  if (head_dim < 32 || head_dim > 256 || head_dim % 8 != 0)
    return fail(NPD_E_INVALID, "%s: head_dim %lld is not a multiple of 8 in [32, 256]", name,
                (long long)head_dim);
  if (num_blocks * block_size * pool_kv_heads > INT32_MAX ||
      max_blocks_per_seq * block_size > INT32_MAX)
    return fail(NPD_E_INVALID, "%s: pool exceeds int32 row indexing", name);
  if (num_seqs * num_kv_heads > 0x7fffffff)
    return fail(NPD_E_INVALID, "%s: too many (seq, kv-head) units", name);
  if (q_stride_seq % 8 || q_stride_head % 8 || out_stride_seq % 8 || out_stride_head % 8 ||
      q_stride_seq < 0 || q_stride_head < 0 || out_stride_seq < 0 || out_stride_head < 0)
    return fail(NPD_E_ALIGN, "%s: query/out strides must be non-negative multiples of 8 elements",
                name);
  if (fp8 && (head_dim != 128 || (block_size != 16 && block_size != 32) ||
              !use_fast_path(head_dim, block_size, num_seqs)))
    return fail(NPD_E_INVALID, "%s: fp8 pools need head_dim 128, block_size 16 or 32 and at most "
                "%d sequences", name, kSchedMaxSeqs);
  if (num_seqs == 0) return NPD_OK;
  if (!out || !query || !key_cache || !value_cache || !block_tables || !seq_lens ||
      (fp8 && (!k_scale || !v_scale)))
    return fail(NPD_E_INVALID, "%s: null pointer", name);
  const uintptr_t cache_align = fp8 ? 7u : 15u;
  if (!aligned16(out) || !aligned16(query) ||
      (reinterpret_cast<uintptr_t>(key_cache) & cache_align) ||
      (reinterpret_cast<uintptr_t>(value_cache) & cache_align))
    return fail(NPD_E_ALIGN, "%s: out/query pointers must be 16-byte aligned, caches %d-byte", name,
                fp8 ? 8 : 16);
  const int64_t max_ctx = block_size * max_blocks_per_seq;
  const int partition =
      choose_partition(num_seqs, num_heads, num_kv_heads, head_dim, block_size, max_ctx, fp8);
  const bool fast = use_fast_path(head_dim, block_size, num_seqs);
  const int limit = fast ? kFastMaxPartition : kMaxPartition;
  if (partition > limit)
    return fail(NPD_E_INVALID, "%s: block_size %lld is above %d", name, (long long)block_size,
                limit);
  const int min_partition = fast ? fast_min_partition(partition, block_size) : partition;
  if ((max_ctx + min_partition - 1) / min_partition > 65535)
    return fail(NPD_E_INVALID, "%s: context too long", name);
  if (num_seqs * num_kv_heads > kMaxCounters)
    return fail(NPD_E_INVALID, "%s: %lld (sequence, kv-head) units exceed the %lld merge counters",
                name, (long long)(num_seqs * num_kv_heads), (long long)kMaxCounters);
  return NPD_OK;
}

// Shared by the 2-byte and the fp8 entry points: k_scale / v_scale are null
// for 2-byte pools.
int attention_impl(void* out, const void* query, const void* key_cache, const void* value_cache,
                   const int32_t* block_tables, const int32_t* seq_lens, int64_t num_seqs,
                   int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, int64_t num_blocks,
                   int64_t block_size, int64_t max_blocks_per_seq, float scale,
                   int64_t q_stride_seq, int64_t q_stride_head, int64_t out_stride_seq,
                   int64_t out_stride_head, const float* k_scale, const float* v_scale,
                   void* workspace, int64_t workspace_bytes, int32_t dtype, void* stream,
                   bool fp8, const char* name) {
  using namespace npd;
  {
    const int rc = attention_check(out, query, key_cache, value_cache, block_tables, seq_lens,
                                   num_seqs, num_heads, num_kv_heads, head_dim, num_blocks,
                                   block_size, max_blocks_per_seq, q_stride_seq, q_stride_head,
                                   out_stride_seq, out_stride_head, k_scale, v_scale, dtype, fp8,
                                   name);
    if (rc != NPD_OK || num_seqs == 0) return rc;
  }
  const int split = kv_split_of(num_heads, num_kv_heads, head_dim, block_size, num_seqs);
  const int64_t pool_kv_heads = num_kv_heads;
  num_kv_heads *= split;
  const int64_t g = num_heads / num_kv_heads;
  const int64_t max_ctx = block_size * max_blocks_per_seq;
  const int partition =
      choose_partition(num_seqs, num_heads, num_kv_heads, head_dim, block_size, max_ctx, fp8);
  const bool fast = use_fast_path(head_dim, block_size, num_seqs);
  const int min_partition = fast ? fast_min_partition(partition, block_size) : partition;
  // partial slots per unit: for the shortest partition the kernel may take
  const int64_t max_parts = (max_ctx + min_partition - 1) / min_partition;
  const int64_t need = npd_paged_attention_workspace_size(num_seqs, num_heads, pool_kv_heads,
                                                          head_dim, block_size, max_blocks_per_seq);
  if (need > 0) {
    if (!workspace || workspace_bytes < need)
      return fail(NPD_E_WORKSPACE, "%s: workspace of %lld bytes needed, %lld given", name,
                  (long long)need, (long long)workspace_bytes);
    if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
      return fail(NPD_E_ALIGN, "%s: workspace must be 256-byte aligned", name);
  }

  DecodeArgs a;
  a.out = static_cast<uint16_t*>(out);
  a.q = static_cast<const uint16_t*>(query);
  a.k_cache = static_cast<const u32x4*>(key_cache);
  a.v_cache = static_cast<const u32x4*>(value_cache);
  a.block_tables = block_tables;
  a.seq_lens = seq_lens;
  const int64_t units = num_seqs * num_kv_heads;
  // [counters | item count | work list | partial acc | partial (m, l)]
  char* wsb = static_cast<char*>(workspace);
  const bool fast_ws = use_fast_path(head_dim, block_size, num_seqs);
  const int64_t part_off =
      fast_ws ? (kCounterBytes + 16 + units * max_parts * 8 + 255) / 256 * 256 : kCounterBytes;
  a.counters = wsb ? reinterpret_cast<int*>(wsb) : nullptr;
  a.sched = wsb ? reinterpret_cast<int*>(wsb + kCounterBytes) : nullptr;
  a.items = wsb ? reinterpret_cast<int2*>(wsb + kCounterBytes + 16) : nullptr;
  a.part_acc = wsb ? reinterpret_cast<float*>(wsb + part_off) : nullptr;
  a.max_groups = (int)merge_groups(fast_ws, units, max_parts);
  a.part_ml = wsb ? a.part_acc + units * (max_parts + a.max_groups) * g * head_dim : nullptr;
  a.num_kv_heads = (int)num_kv_heads;
  a.kv_split = split;
  a.pool_kv_heads = (int)pool_kv_heads;
  a.num_seqs = (int)num_seqs;
  a.block_size = (int)block_size;
  a.num_blocks = (int)num_blocks;
  a.max_bps = (int)max_blocks_per_seq;
  a.partition = partition;
  a.min_partition = min_partition;
  a.max_parts = (int)max_parts;
  a.head_dim = (int)head_dim;
  a.scale_log2 = scale * kLog2e;
  a.q_stride_seq = q_stride_seq;
  a.q_stride_head = q_stride_head;
  a.out_stride_seq = out_stride_seq;
  a.out_stride_head = out_stride_head;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  hipStream_t st = as_stream(stream);
  if (fp8) {
    if (dtype == NPD_DTYPE_BF16) return dispatch_fp8<BF16>((int)g, a, units, st);
    return dispatch_fp8<F16>((int)g, a, units, st);
  }
  if (dtype == NPD_DTYPE_BF16) return dispatch_d<BF16>(head_dim, (int)g, a, units, st);
  return dispatch_d<F16>(head_dim, (int)g, a, units, st);
}

}  // namespace

extern "C" int npd_paged_attention(void* out, const void* query, const void* key_cache,
                                   const void* value_cache, const int32_t* block_tables,
                                   const int32_t* seq_lens, int64_t num_seqs, int64_t num_heads,
                                   int64_t num_kv_heads, int64_t head_dim, int64_t num_blocks,
                                   int64_t block_size, int64_t max_blocks_per_seq, float scale,
                                   int64_t q_stride_seq, int64_t q_stride_head,
                                   int64_t out_stride_seq, int64_t out_stride_head,
                                   void* workspace, int64_t workspace_bytes, int32_t dtype,
                                   void* stream) {
  return attention_impl(out, query, key_cache, value_cache, block_tables, seq_lens, num_seqs,
                        num_heads, num_kv_heads, head_dim, num_blocks, block_size,
                        max_blocks_per_seq, scale, q_stride_seq, q_stride_head, out_stride_seq,
                        out_stride_head, nullptr, nullptr, workspace, workspace_bytes, dtype,
                        stream, false, "npd_paged_attention");
}

extern "C" int npd_paged_attention_fp8(void* out, const void* query, const void* key_cache,
                                       const void* value_cache, const int32_t* block_tables,
                                       const int32_t* seq_lens, const float* k_scale,
                                       const float* v_scale, int64_t num_seqs,
                                       int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                                       int64_t num_blocks, int64_t block_size,
                                       int64_t max_blocks_per_seq, float scale,
                                       int64_t q_stride_seq, int64_t q_stride_head,
                                       int64_t out_stride_seq, int64_t out_stride_head,
                                       void* workspace, int64_t workspace_bytes, int32_t dtype,
                                       void* stream) {
  return attention_impl(out, query, key_cache, value_cache, block_tables, seq_lens, num_seqs,
                        num_heads, num_kv_heads, head_dim, num_blocks, block_size,
                        max_blocks_per_seq, scale, q_stride_seq, q_stride_head, out_stride_seq,
                        out_stride_head, k_scale, v_scale, workspace, workspace_bytes, dtype,
                        stream, true, "npd_paged_attention_fp8");
}

// ---------------------------------------------------------------------------
// No-allocation variant of npd_paged_attention: the workspace is `scratch`, a
// static device array that every GPU the library runs on holds until the
// process ends. Calls on one GPU share it (calls that overlap on one GPU
// race); every call leaves its merge counters at zero, as with a caller's
// workspace, and the counter region is cleared once per device at set-up.
// ---------------------------------------------------------------------------
#include <mutex>

namespace {

constexpr int64_t kScratchBytes = NPD_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices];   // device address of `scratch`, per device

__global__ __launch_bounds__(256) void clear_counters_kernel(u32x4* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = u32x4{0, 0, 0, 0};
}

// The device a stream's work runs on: the stream's own device for a created
// stream; the null stream and the per-thread / legacy handles belong to the
// calling thread's current device. -1 on failure.
int stream_device(hipStream_t st) {
  if (st == nullptr || st == hipStreamPerThread || st == hipStreamLegacy) {
    int dev = -1;
    return hipGetDevice(&dev) == hipSuccess ? dev : -1;
  }
  hipDevice_t dev = -1;
  return hipStreamGetDevice(st, &dev) == hipSuccess ? (int)dev : -1;
}

// Makes `dev` the calling thread's current device for its lifetime and
// restores the previous one after (a new host thread starts on device 0,
// whatever device the stream it is handed belongs to).
struct DeviceGuard {
  int prev = -1;
  bool ok = false;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) return;
    ok = prev == dev || hipSetDevice(dev) == hipSuccess;
  }
  ~DeviceGuard() {
    if (ok && prev >= 0) (void)hipSetDevice(prev);
  }
};

// The device address of device `dev`'s `scratch` (nullptr and an error
// message on failure); `dev` must be the current device. The first call on a
// device looks the address up and enqueues the clear of its counter region on
// `st`, ahead of the caller's kernels.
void* scratch_of_device(int dev, hipStream_t st, const char* name) {
  if (dev < 0 || dev >= kScratchDevices) {
    npd::fail(NPD_E_LAUNCH, "%s: no usable device for the stream (%d)", name, dev);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev]) return g_scratch_ptr[dev];
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !ptr) {
    npd::fail(NPD_E_LAUNCH, "%s: hipGetSymbolAddress(scratch): %s", name, hipGetErrorString(e));
    return nullptr;
  }
  const int64_t n = npd::kCounterBytes / 16;
  hipLaunchKernelGGL(clear_counters_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     static_cast<u32x4*>(ptr), n);
  if (npd::check_launch(name) != NPD_OK) return nullptr;
  g_scratch_ptr[dev] = ptr;
  return ptr;
}

}  // namespace

extern "C" int npd_paged_attention_noalloc(void* out, const void* query, const void* key_cache,
                                           const void* value_cache, const int32_t* block_tables,
                                           const int32_t* seq_lens, int64_t num_seqs,
                                           int64_t num_heads, int64_t num_kv_heads,
                                           int64_t head_dim, int64_t num_blocks,
                                           int64_t block_size, int64_t max_blocks_per_seq,
                                           float scale, int64_t q_stride_seq,
                                           int64_t q_stride_head, int64_t out_stride_seq,
                                           int64_t out_stride_head, int32_t dtype, void* stream) {
  const char* name = "npd_paged_attention_noalloc";
  // the same argument checks as npd_paged_attention, before the scratch is
  // touched: invalid calls get the same codes and launch nothing
  const int rc = attention_check(out, query, key_cache, value_cache, block_tables, seq_lens,
                                 num_seqs, num_heads, num_kv_heads, head_dim, num_blocks,
                                 block_size, max_blocks_per_seq, q_stride_seq, q_stride_head,
                                 out_stride_seq, out_stride_head, nullptr, nullptr, dtype, false,
                                 name);
  if (rc != NPD_OK || num_seqs == 0) return rc;
  const int64_t need = npd_paged_attention_workspace_size(num_seqs, num_heads, num_kv_heads,
                                                          head_dim, block_size, max_blocks_per_seq);
  if (need > kScratchBytes)
    return npd::fail(NPD_E_WORKSPACE,
                     "%s: these shapes need %lld bytes of workspace, above the %lld-byte static "
                     "scratch; call npd_paged_attention with a workspace", name, (long long)need,
                     (long long)kScratchBytes);
  // the scratch of the stream's device, looked up (and the launches made)
  // with that device current
  const hipStream_t st = npd::as_stream(stream);
  const int dev = stream_device(st);
  if (dev < 0) return npd::fail(NPD_E_LAUNCH, "%s: cannot tell the stream's device", name);
  DeviceGuard guard(dev);
  if (!guard.ok) return npd::fail(NPD_E_LAUNCH, "%s: cannot make device %d current", name, dev);
  void* ws = nullptr;
  if (need > 0) {
    ws = scratch_of_device(dev, st, name);
    if (!ws) return NPD_E_LAUNCH;
  }
  return attention_impl(out, query, key_cache, value_cache, block_tables, seq_lens, num_seqs,
                        num_heads, num_kv_heads, head_dim, num_blocks, block_size,
                        max_blocks_per_seq, scale, q_stride_seq, q_stride_head, out_stride_seq,
                        out_stride_head, nullptr, nullptr, ws, ws ? kScratchBytes : 0, dtype,
                        stream, false, name);
}
