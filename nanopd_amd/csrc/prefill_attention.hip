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
//   workgroup = one (sequence, kv-head, tile of 64 query positions) with 2*G
//   waves: wave w serves query head kv*G + w/2 and the 32 query rows
//   (w%2)*32 .. +32 of the tile. Each 64-key K/V tile is gathered from the
//   pool once into LDS and used by all 2*G waves (GQA reuse); two waves per
//   SIMD let one wave's softmax (VALU) run under the other's MFMAs.
//   per step of 64 keys, each wave:
//     S^T = K . Q^T   -- A = K rows from LDS, B = the wave's query rows, kept
//                        in registers for the whole key loop;
//     online softmax  -- lane l owns query (mb*16 + l%16) of each 16-row block:
//                        16 of its 64 scores per step are in-lane, the rest in
//                        lanes l^16, l^32; the O rescale is skipped when no
//                        row maximum moved;
//     O^T += V^T . P^T -- P^T is the S^T accumulator, already in B-operand
//                        layout (packed with v_cvt_pk_bf16_f32); V stays
//                        row-major in LDS like K, and the V^T A operand is two
//                        ds_read_b64_tr_b16 (gfx950 transposing LDS read: in a
//                        group of 16 lanes, lane j receives element j%4 of the
//                        8-byte chunks addressed by lanes 4e + j/4, e = 0..3).
//   Operand layouts of v_mfma_f32_16x16x32 (checked on the hardware):
//     A[m = lane%16][k = 8*(lane/16) + e], B[k = 8*(lane/16) + e][n = lane%16],
//     D[m = 4*(lane/16) + i][n = lane%16].
//   K/V tiles are double-buffered in LDS: the next tile's global loads are in
//   flight while the current one is multiplied. Keys past the visible range
//   are written as zeros and masked, so no NaN from stale pool memory leaks in.
#include "common.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kD = 128;          // head_dim of this kernel
constexpr int kQT = 64;          // query positions per workgroup
constexpr int kQW = 32;          // query rows per wave
constexpr int kKT = 64;          // keys per step
// LDS row of the K and V tiles (elements): 72 dwords, an 8-bank shift per row,
// so 16 rows of K read at one column and 4 rows x 32 bytes of a transposing
// V read both hit distinct banks
constexpr int kRow = kD + 16;
constexpr int kMaxBlocksLds = 1024;   // block ids of one workgroup's key range kept in LDS
constexpr float kLog2e = 1.4426950408889634f;

struct PrefillArgs {
  uint16_t* out;
  const uint16_t* q;
  const u32x4* k_cache;
  const u32x4* v_cache;
  const int32_t* block_tables;
  const int32_t* cu_seqlens_q;
  const int32_t* context_lens;
  int num_seqs, num_kv_heads, block_size, num_blocks, max_bps, tiles_max;
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

__device__ __forceinline__ float shfl_xor(float v, int m) { return __shfl_xor(v, m, 64); }

typedef short s16x4 __attribute__((ext_vector_type(4)));
// ds_read_b64_tr_b16 on an LDS address given as a generic pointer to __shared__
__device__ __forceinline__ u32x2 lds_read_tr(const uint16_t* p) {
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p)));
}

template <class TT, int G>
__global__ __launch_bounds__(128 * G) void prefill_kernel(PrefillArgs a) {
  constexpr int NT = 128 * G;                          // threads
  constexpr int MB = kQW / 16;                         // 16-row query blocks per wave
  __shared__ __attribute__((aligned(16))) uint16_t s_k[2][kKT * kRow];
  __shared__ __attribute__((aligned(16))) uint16_t s_v[2][kKT * kRow];
  __shared__ int s_blk[kMaxBlocksLds];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, r = lane & 15;

  // item: tiles of a sequence are visited last-tile first (they see the most keys)
  const int per_seq = a.num_kv_heads * a.tiles_max;
  const int s = blockIdx.x / per_seq;
  const int rem = blockIdx.x - s * per_seq;
  const int kh = rem / a.tiles_max;
  const int t = a.tiles_max - 1 - (rem - kh * a.tiles_max);

  const int q0 = a.cu_seqlens_q[s], q1 = a.cu_seqlens_q[s + 1];
  const int qlen = q1 - q0;
  if (t * kQT >= qlen) return;
  const int cap = a.max_bps * a.block_size;
  int ctx = a.context_lens[s];
  ctx = ctx < cap ? ctx : cap;
  const int prefix = ctx - qlen;                       // position of query row 0
  const int rows = (qlen - t * kQT) < kQT ? (qlen - t * kQT) : kQT;
  const int pos0 = prefix + t * kQT;                   // position of the tile's first row
  int nkeys = pos0 + rows;                             // keys 0 .. last row's position
  nkeys = nkeys < 0 ? 0 : nkeys;
  const int h = kh * G + (wave >> 1);
  const int wrow0 = (wave & 1) * kQW;                  // this wave's first row in the tile
  const int wpos0 = pos0 + wrow0;
  const int nsteps = (nkeys + kKT - 1) / kKT;
  const int bs = a.block_size;
  const int nblk = (nkeys + bs - 1) / bs;

  // block ids of the key range -> LDS (clamped into the pool)
  for (int e = tid; e < nblk && e < kMaxBlocksLds; e += NT) {
    int b = a.block_tables[(int64_t)s * a.max_bps + e];
    s_blk[e] = b < 0 ? 0 : (b >= a.num_blocks ? a.num_blocks - 1 : b);
  }

  // the wave's query rows as B operands: qb[mb][c] = Q[row mb*16 + r][c*32 + 8g .. +8]
  u32x4 qb[MB][4];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int row = t * kQT + wrow0 + mb * 16 + r;
    const bool ok = row < qlen;
    const uint16_t* qp = a.q + (int64_t)(q0 + (ok ? row : 0)) * a.q_stride_token +
                         (int64_t)h * a.q_stride_head + g * 8;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      qb[mb][c] = ok ? *reinterpret_cast<const u32x4*>(qp + c * 32) : u32x4{0, 0, 0, 0};
  }
  __syncthreads();

  // K/V tile loaders: chunk ch (16 bytes) of the 64 x 256-byte tile
  constexpr int kChunks = kKT * kD / 8;                // 1024
  constexpr int kPer = (kChunks + NT - 1) / NT;
  u32x4 kst[kPer], vst[kPer];
  auto fetch = [&](int step) {
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      const int ch = tid + e * NT;
      kst[e] = u32x4{0, 0, 0, 0};
      vst[e] = u32x4{0, 0, 0, 0};
      if (ch < kChunks) {
        const int kk = ch >> 4, col = ch & 15;
        const int tok = step * kKT + kk;
        if (tok < nkeys) {
          const int lb = tok / bs;
          int blk;
          if (lb < kMaxBlocksLds) {
            blk = s_blk[lb];
          } else {
            blk = a.block_tables[(int64_t)s * a.max_bps + lb];
            blk = blk < 0 ? 0 : (blk >= a.num_blocks ? a.num_blocks - 1 : blk);
          }
          const int64_t idx = (((int64_t)blk * a.num_kv_heads + kh) * bs + (tok - lb * bs)) * 16 + col;
          kst[e] = a.k_cache[idx];
          vst[e] = a.v_cache[idx];
        }
      }
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      const int ch = tid + e * NT;
      if (ch < kChunks) {
        const int kk = ch >> 4, col = ch & 15;
        *reinterpret_cast<u32x4*>(&s_k[buf][kk * kRow + col * 8]) = kst[e];
        *reinterpret_cast<u32x4*>(&s_v[buf][kk * kRow + col * 8]) = vst[e];
      }
    }
  };

  f32x4 oacc[8][MB];   // O^T[d = nb*16 + 4g + i][q = mb*16 + r]
#pragma unroll
  for (int nb = 0; nb < 8; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) oacc[nb][mb] = f32x4{0, 0, 0, 0};
  float mrow[MB], lrow[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) { mrow[mb] = -INFINITY; lrow[mb] = 0.f; }

  if (nsteps > 0) {
    fetch(0);
    stash(0);
  }
  __syncthreads();
  for (int step = 0; step < nsteps; ++step) {
    const int buf = step & 1;
    if (step + 1 < nsteps) fetch(step + 1);
    const uint16_t* kt = s_k[buf];
    const uint16_t* vt = s_v[buf];

    // S^T = K . Q^T : sacc[n][mb] holds S^T[key = n*16 + 4g + i][q = mb*16 + r]
    f32x4 sacc[4][MB];
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) sacc[n][mb] = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const u32x4 ka = *reinterpret_cast<const u32x4*>(&kt[(n * 16 + r) * kRow + c * 32 + g * 8]);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) sacc[n][mb] = Mfma<TT>::mma(ka, qb[mb][c], sacc[n][mb]);
      }
    }
    // scale, causal mask, online softmax (log2 domain); pb[kc][mb] is the
    // B operand of keys kc*32 .. +32: slots e<4 -> key kc*32 + 4g + e,
    // e>=4 -> kc*32 + 16 + 4g + e - 4
    const int key0 = step * kKT;
    const bool diag = key0 + kKT - 1 > wpos0;   // some key here is after some row
    u32x4 pb[2][MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int qpos = wpos0 + mb * 16 + r;
      float v[16];
#pragma unroll
      for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float x = sacc[n][mb][i] * a.scale_log2;
          if (diag && key0 + n * 16 + g * 4 + i > qpos) x = -INFINITY;
          v[n * 4 + i] = x;
        }
      float mx = v[0];
#pragma unroll
      for (int e = 1; e < 16; ++e) mx = fmaxf(mx, v[e]);
      mx = fmaxf(mx, shfl_xor(mx, 16));
      mx = fmaxf(mx, shfl_xor(mx, 32));
      const float mnew = fmaxf(mrow[mb], mx);
      // a row that has seen only masked keys keeps m = -inf: use 0 as the
      // reference so exp2 gives 0, not NaN
      const float mref = mnew == -INFINITY ? 0.f : mnew;
      const float alpha = __builtin_amdgcn_exp2f(mrow[mb] - mref);
      float ls = 0.f;
      uint32_t packed[8];
#pragma unroll
      for (int e = 0; e < 16; e += 2) {
        const float p0 = __builtin_amdgcn_exp2f(v[e] - mref);
        const float p1 = __builtin_amdgcn_exp2f(v[e + 1] - mref);
        const uint32_t u = TT::pack2(p0, p1);
        ls += TT::lo(u) + TT::hi(u);
        packed[e / 2] = u;
      }
      lrow[mb] = lrow[mb] * alpha + ls;
      mrow[mb] = mnew;
      // packed[n*2 + i/2] holds keys n*16 + 4g + i, i in pairs
      pb[0][mb] = u32x4{packed[0], packed[1], packed[2], packed[3]};
      pb[1][mb] = u32x4{packed[4], packed[5], packed[6], packed[7]};
      if (__ballot(alpha != 1.f) != 0) {
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) oacc[nb][mb] *= alpha;
      }
    }
    // O^T += V^T . P^T ; A = V^T[d = nb*16 + r][keys kc*32 + {4g..4g+3, 16+4g..16+4g+3}]
    // transposing reads: lane r of group g addresses key (.. + 4g + r/4),
    // dims nb*16 + 4*(r%4) .. +3, and receives dim nb*16 + r of keys +0..3
    const uint16_t* vlane = vt + (g * 4 + (r >> 2)) * kRow + 4 * (r & 3);
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const u32x2 lo = lds_read_tr(vlane + (kc * 32) * kRow + nb * 16);
        const u32x2 hi = lds_read_tr(vlane + (kc * 32 + 16) * kRow + nb * 16);
        const u32x4 va = u32x4{lo.x, lo.y, hi.x, hi.y};
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) oacc[nb][mb] = Mfma<TT>::mma(va, pb[kc][mb], oacc[nb][mb]);
      }
    }
    // buf ^ 1 was last read in the previous step, which every wave finished
    // before that step's barrier
    if (step + 1 < nsteps) stash(buf ^ 1);
    __syncthreads();
  }

  // normalise and store: lane writes d = nb*16 + 4g .. +3 of query row mb*16 + r
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    float l = lrow[mb];
    l += shfl_xor(l, 16);
    l += shfl_xor(l, 32);
    const int row = t * kQT + wrow0 + mb * 16 + r;
    if (row >= qlen) continue;
    const float inv = (l > 0.f && wpos0 + mb * 16 + r >= 0) ? 1.f / l : 0.f;
    uint16_t* op = a.out + (int64_t)(q0 + row) * a.out_stride_token + (int64_t)h * a.out_stride_head;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      const f32x4 o = oacc[nb][mb];
      u32x2 w;
      w.x = TT::pack2(o[0] * inv, o[1] * inv);
      w.y = TT::pack2(o[2] * inv, o[3] * inv);
      *reinterpret_cast<u32x2*>(op + nb * 16 + g * 4) = w;
    }
  }
}

template <class TT>
int launch(int g, const PrefillArgs& a, int64_t grid, hipStream_t st) {
  switch (g) {
    case 1: hipLaunchKernelGGL((prefill_kernel<TT, 1>), dim3((unsigned)grid), dim3(128), 0, st, a); break;
    case 2: hipLaunchKernelGGL((prefill_kernel<TT, 2>), dim3((unsigned)grid), dim3(256), 0, st, a); break;
    case 4: hipLaunchKernelGGL((prefill_kernel<TT, 4>), dim3((unsigned)grid), dim3(512), 0, st, a); break;
    case 6: hipLaunchKernelGGL((prefill_kernel<TT, 6>), dim3((unsigned)grid), dim3(768), 0, st, a); break;
    case 8: hipLaunchKernelGGL((prefill_kernel<TT, 8>), dim3((unsigned)grid), dim3(1024), 0, st, a); break;
    default: return npd::fail(NPD_E_INVALID, "npd_paged_prefill_attention: group size %d", g);
  }
  return npd::check_launch("npd_paged_prefill_attention");
}

}  // namespace

extern "C" int64_t npd_paged_prefill_workspace_size(int64_t, int64_t, int64_t, int64_t, int64_t,
                                                    int64_t) {
  return 0;
}

extern "C" int npd_paged_prefill_attention(
    void* out, const void* query, const void* key_cache, const void* value_cache,
    const int32_t* block_tables, const int32_t* cu_seqlens_q, const int32_t* context_lens,
    int64_t num_seqs, int64_t total_q, int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
    int64_t num_blocks, int64_t block_size, int64_t max_blocks_per_seq, int64_t max_q_len,
    int64_t max_context_len, float scale, int64_t q_stride_token, int64_t q_stride_head,
    int64_t out_stride_token, int64_t out_stride_head, void* workspace, int64_t workspace_bytes,
    int32_t dtype, void* stream) {
  using namespace npd;
  (void)workspace;
  (void)workspace_bytes;
  (void)max_context_len;
  const char* name = "npd_paged_prefill_attention";
  if (dtype != NPD_DTYPE_F16 && dtype != NPD_DTYPE_BF16)
    return fail(NPD_E_DTYPE, "%s: unsupported dtype code %d (fp16/bf16 only)", name, dtype);
  if (num_seqs < 0 || total_q < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_blocks <= 0 ||
      block_size <= 0 || max_blocks_per_seq <= 0 || max_q_len < 0)
    return fail(NPD_E_INVALID, "%s: bad sizes", name);
  if (head_dim != kD)
    return fail(NPD_E_INVALID, "%s: head_dim %lld not supported (128 only)", name,
                (long long)head_dim);
  if (num_heads % num_kv_heads != 0)
    return fail(NPD_E_INVALID, "%s: num_heads %lld is not a multiple of num_kv_heads %lld", name,
                (long long)num_heads, (long long)num_kv_heads);
  const int64_t g = num_heads / num_kv_heads;
  if (g != 1 && g != 2 && g != 4 && g != 6 && g != 8)
    return fail(NPD_E_INVALID, "%s: query heads per kv head %lld not in {1, 2, 4, 6, 8}", name,
                (long long)g);
  if (num_blocks * block_size * num_kv_heads > INT32_MAX || max_blocks_per_seq * block_size > INT32_MAX)
    return fail(NPD_E_INVALID, "%s: pool exceeds int32 row indexing", name);
  if (q_stride_token % 8 || q_stride_head % 8 || out_stride_token % 4 || out_stride_head % 4 ||
      q_stride_token < 0 || q_stride_head < 0 || out_stride_token < 0 || out_stride_head < 0)
    return fail(NPD_E_ALIGN, "%s: query strides must be multiples of 8 elements, out strides of 4",
                name);
  if (num_seqs == 0 || total_q == 0 || max_q_len == 0) return NPD_OK;
  if (!out || !query || !key_cache || !value_cache || !block_tables || !cu_seqlens_q || !context_lens)
    return fail(NPD_E_INVALID, "%s: null pointer", name);
  if (!aligned16(query) || !aligned16(key_cache) || !aligned16(value_cache) ||
      (reinterpret_cast<uintptr_t>(out) & 7u) != 0)
    return fail(NPD_E_ALIGN, "%s: query/cache pointers must be 16-byte aligned, out 8-byte", name);
  const int64_t tiles = (max_q_len + kQT - 1) / kQT;
  const int64_t grid = num_seqs * num_kv_heads * tiles;
  if (grid > INT32_MAX) return fail(NPD_E_INVALID, "%s: too many tiles", name);

  PrefillArgs a;
  a.out = static_cast<uint16_t*>(out);
  a.q = static_cast<const uint16_t*>(query);
  a.k_cache = static_cast<const u32x4*>(key_cache);
  a.v_cache = static_cast<const u32x4*>(value_cache);
  a.block_tables = block_tables;
  a.cu_seqlens_q = cu_seqlens_q;
  a.context_lens = context_lens;
  a.num_seqs = (int)num_seqs;
  a.num_kv_heads = (int)num_kv_heads;
  a.block_size = (int)block_size;
  a.num_blocks = (int)num_blocks;
  a.max_bps = (int)max_blocks_per_seq;
  a.tiles_max = (int)tiles;
  a.scale_log2 = scale * kLog2e;
  a.q_stride_token = q_stride_token;
  a.q_stride_head = q_stride_head;
  a.out_stride_token = out_stride_token;
  a.out_stride_head = out_stride_head;
  hipStream_t st = as_stream(stream);
  if (dtype == NPD_DTYPE_BF16) return launch<BF16>((int)g, a, grid, st);
  return launch<F16>((int)g, a, grid, st);
}
