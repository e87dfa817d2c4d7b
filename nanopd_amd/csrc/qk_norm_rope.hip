// Fused attention prologue for Qwen3-style layers: per-head RMSNorm of q and k
// (q_norm / k_norm), rotate-half RoPE at each token's position, and the paged
// KV store of the rotated k and of v by slot -- one launch per layer, reading
// the fused QKV projection output as it is. Without norm weights (null
// pointers) the same launch serves Qwen2 / Llama layers, whose attention has
// no q / k norm (the reference applies them only when the module has them,
// nanoPD/engine/model_runner.py:101-104): RoPE of q and k as projected.
//
// Reference: per layer, paged_forward runs HF Qwen3Attention's q_norm / k_norm
// and apply_rotary_pos_emb (nanoPD/engine/model_runner.py:97-115), transposes
// and copies k / v (.contiguous(), :142-143, :191-192) and calls
// paged_kv_store (:146, :189): about a dozen elementwise launches plus the
// copies. Here a group of lanes handles one (token, head) row of the QKV
// output:
//   rows [0, H)           q heads: normalise, rotate, write q_out
//   rows [H, H + KV)      k heads: normalise, rotate, store to k_cache[slot]
//   rows [H + KV, H + 2KV) v heads: store to v_cache[slot]
// A row of D elements takes LW = min(D / 2, 64) lanes (head dims 64, 128,
// 256: 32, 64, 64 lanes; a wave holds two rows of 64). Lane l holds the
// rotate-half pairs (i, i + D/2) for i = l, l + LW, ... (one pair for D 64 and
// 128, two for D 256), so RoPE needs no data exchange; the RMS statistic is
// a reduction over the row's LW lanes.
// RMSNorm rounds as HF Qwen3RMSNorm does (transformers modeling_qwen3):
// n = half(half(x * rsqrt(mean(x^2) + eps)) * w), with the mean in fp32.
// RoPE then rotates n in fp32 with cos / sin of pos * inv_freq[l] (inv_freq
// from the caller, fp32) and rounds once. The reference's HF
// apply_rotary_pos_emb rounds cos / sin and each product to the model dtype
// first; the fp32 rotation here is the more accurate of the two and differs
// from it by a few half-precision ulps at most.
// FP8 pools (kF8): the rotated k and the raw v, rounded to the 2-byte type as
// above, are stored as e4m3 bytes of value / scale[kv head] (the rounding of
// npd_paged_kv_store_slots_fp8, so both paths write the same bytes).
#include "common.h"

namespace {

constexpr int kThreads = 256;   // 4 waves per workgroup

struct RopeArgs {
  uint16_t* q_out;
  void* k_cache;   // 2-byte elements, or e4m3 bytes (kF8)
  void* v_cache;
  const float* k_scale;   // kF8: per-kv-head scales
  const float* v_scale;
  const uint16_t* qkv;
  const int32_t* slots;
  const int32_t* positions;
  const float* inv_freq;
  const uint16_t* q_w;
  const uint16_t* k_w;
  int64_t rows;               // tokens * (H + 2 KV)
  int heads, kv_heads, block_size, num_blocks;
  int64_t qkv_stride, q_stride;
  float eps;
};

// Sum over aligned groups of LW lanes (the lanes of one row).
template <int LW>
__device__ __forceinline__ float group_sum(float x) {
#pragma unroll
  for (int m = LW / 2; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
  return x;
}

template <class TT>
__device__ __forceinline__ float ld(const uint16_t* p) {
  return TT::lo((uint32_t)*p);
}

template <class TT, bool kF8, int D>
__global__ __launch_bounds__(kThreads) void qk_norm_rope_store_kernel(RopeArgs a) {
  constexpr int HALF = D / 2;
  constexpr int LW = HALF < 64 ? HALF : 64;   // lanes per row
  constexpr int P = HALF / LW;                // rotate-half pairs per lane
  constexpr int RPW = 64 / LW;                // rows per wave
  const int lane = threadIdx.x & 63;
  const int64_t row =
      ((int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6)) * RPW + lane / LW;
  if (row >= a.rows) return;
  const int l = lane % LW;
  const int per = a.heads + 2 * a.kv_heads;
  const int64_t t = row / per;
  const int hh = (int)(row - t * per);
  const uint16_t* src = a.qkv + t * a.qkv_stride + (int64_t)hh * D;
  float x0[P], x1[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    x0[p] = ld<TT>(src + l + p * LW);
    x1[p] = ld<TT>(src + l + p * LW + HALF);
  }

  const int slot = a.slots[t];
  const bool store = slot >= 0 && slot < a.num_blocks * a.block_size;
  const int64_t blk = store ? slot / a.block_size : 0;
  const int off = store ? slot - (int)blk * a.block_size : 0;

  if (hh >= a.heads + a.kv_heads) {   // v: plain store
    if (!store) return;
    const int kh = hh - a.heads - a.kv_heads;
    const int64_t e = ((blk * a.kv_heads + kh) * a.block_size + off) * D;
    if constexpr (kF8) {
      uint8_t* dst = static_cast<uint8_t*>(a.v_cache) + e;
      const float sc = a.v_scale[kh];
#pragma unroll
      for (int p = 0; p < P; ++p) {
        dst[l + p * LW] = (uint8_t)npd::e4m3_byte(x0[p], sc);
        dst[l + p * LW + HALF] = (uint8_t)npd::e4m3_byte(x1[p], sc);
      }
    } else {
      uint16_t* dst = static_cast<uint16_t*>(a.v_cache) + e;
#pragma unroll
      for (int p = 0; p < P; ++p) {
        dst[l + p * LW] = src[l + p * LW];
        dst[l + p * LW + HALF] = src[l + p * LW + HALF];
      }
    }
    return;
  }
  const bool is_q = hh < a.heads;
  const uint16_t* w = is_q ? a.q_w : a.k_w;
  // no norm weight (Qwen2 / Llama layers): RoPE of the projection output as
  // it is. The choice is uniform over a row's lanes, so the row reduction
  // below runs on every lane it exchanges with.
  const bool norm = w != nullptr;
  float r = 1.f;
  if (norm) {
    float ss = 0.f;
#pragma unroll
    for (int p = 0; p < P; ++p) ss += x0[p] * x0[p] + x1[p] * x1[p];
    r = rsqrtf(group_sum<LW>(ss) * (1.f / D) + a.eps);
  }
  const float pos = (float)a.positions[t];
  uint16_t y0[P], y1[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int i = l + p * LW;
    float n0 = x0[p], n1 = x1[p];
    if (norm) {
      n0 = TT::lo(TT::from_float(TT::lo(TT::from_float(x0[p] * r)) * ld<TT>(w + i)));
      n1 = TT::lo(TT::from_float(TT::lo(TT::from_float(x1[p] * r)) * ld<TT>(w + i + HALF)));
    }
    float s, c;
    sincosf(pos * a.inv_freq[i], &s, &c);
    y0[p] = (uint16_t)TT::from_float(n0 * c - n1 * s);
    y1[p] = (uint16_t)TT::from_float(n1 * c + n0 * s);
  }
  uint16_t* dst;
  if (is_q) {
    dst = a.q_out + t * a.q_stride + (int64_t)hh * D;
  } else {
    if (!store) return;
    const int kh = hh - a.heads;
    const int64_t e = ((blk * a.kv_heads + kh) * a.block_size + off) * D;
    if constexpr (kF8) {
      uint8_t* d8 = static_cast<uint8_t*>(a.k_cache) + e;
      const float sc = a.k_scale[kh];
#pragma unroll
      for (int p = 0; p < P; ++p) {
        d8[l + p * LW] = (uint8_t)npd::e4m3_byte(TT::lo(y0[p]), sc);
        d8[l + p * LW + HALF] = (uint8_t)npd::e4m3_byte(TT::lo(y1[p]), sc);
      }
      return;
    }
    dst = static_cast<uint16_t*>(a.k_cache) + e;
  }
#pragma unroll
  for (int p = 0; p < P; ++p) {
    dst[l + p * LW] = y0[p];
    dst[l + p * LW + HALF] = y1[p];
  }
}

template <class TT, bool kF8>
void launch_rope(int64_t head_dim, int64_t grid, hipStream_t st, const RopeArgs& a) {
  switch (head_dim) {
    case 64:
      hipLaunchKernelGGL((qk_norm_rope_store_kernel<TT, kF8, 64>), dim3((unsigned)grid),
                         dim3(kThreads), 0, st, a);
      break;
    case 128:
      hipLaunchKernelGGL((qk_norm_rope_store_kernel<TT, kF8, 128>), dim3((unsigned)grid),
                         dim3(kThreads), 0, st, a);
      break;
    default:
      hipLaunchKernelGGL((qk_norm_rope_store_kernel<TT, kF8, 256>), dim3((unsigned)grid),
                         dim3(kThreads), 0, st, a);
      break;
  }
}

}  // namespace

namespace {

// Shared by the 2-byte and the FP8 entry points (k_scale / v_scale null for
// 2-byte pools).
int rope_impl(void* q_out, void* k_cache, void* v_cache, const void* qkv,
              const int32_t* slot_mapping, const int32_t* positions, const float* inv_freq,
              const void* q_norm_weight, const void* k_norm_weight, const float* k_scale,
              const float* v_scale, int64_t num_tokens, int64_t num_heads, int64_t num_kv_heads,
              int64_t head_dim, int64_t num_blocks, int64_t block_size, int64_t qkv_stride_token,
              int64_t q_stride_token, float eps, int32_t dtype, void* stream, bool fp8,
              const char* name) {
  using namespace npd;
  if (dtype != NPD_DTYPE_F16 && dtype != NPD_DTYPE_BF16)
    return fail(NPD_E_DTYPE, "%s: unsupported dtype code %d (fp16/bf16 only)", name, dtype);
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(NPD_E_INVALID, "%s: head_dim %lld not in {64, 128, 256}", name,
                (long long)head_dim);
  if (num_tokens < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_blocks <= 0 || block_size <= 0)
    return fail(NPD_E_INVALID, "%s: bad sizes", name);
  if (num_blocks * block_size > INT32_MAX)
    return fail(NPD_E_INVALID, "%s: pool exceeds int32 slot indexing", name);
  if (qkv_stride_token < (num_heads + 2 * num_kv_heads) * head_dim || q_stride_token < num_heads * head_dim)
    return fail(NPD_E_INVALID, "%s: token strides shorter than a token's heads", name);
  if (!(eps >= 0.f))
    return fail(NPD_E_INVALID, "%s: eps must be non-negative", name);
  if (num_tokens == 0) return NPD_OK;
  if (!q_out || !k_cache || !v_cache || !qkv || !slot_mapping || !positions || !inv_freq ||
      (fp8 && (!k_scale || !v_scale)))
    return fail(NPD_E_INVALID, "%s: null pointer", name);
  if ((q_norm_weight == nullptr) != (k_norm_weight == nullptr))
    return fail(NPD_E_INVALID, "%s: pass both norm weights (Qwen3) or neither (Qwen2 / Llama)",
                name);
  const int64_t rows = num_tokens * (num_heads + 2 * num_kv_heads);
  const int64_t rows_per_block = (kThreads / 64) * (head_dim == 64 ? 2 : 1);
  const int64_t grid = (rows + rows_per_block - 1) / rows_per_block;
  if (grid > INT32_MAX) return fail(NPD_E_INVALID, "%s: too many rows", name);
  RopeArgs a;
  a.q_out = static_cast<uint16_t*>(q_out);
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.qkv = static_cast<const uint16_t*>(qkv);
  a.slots = slot_mapping;
  a.positions = positions;
  a.inv_freq = inv_freq;
  a.q_w = static_cast<const uint16_t*>(q_norm_weight);
  a.k_w = static_cast<const uint16_t*>(k_norm_weight);
  a.rows = rows;
  a.heads = (int)num_heads;
  a.kv_heads = (int)num_kv_heads;
  a.block_size = (int)block_size;
  a.num_blocks = (int)num_blocks;
  a.qkv_stride = qkv_stride_token;
  a.q_stride = q_stride_token;
  a.eps = eps;
  hipStream_t st = as_stream(stream);
  if (dtype == NPD_DTYPE_BF16) {
    if (fp8) launch_rope<BF16, true>(head_dim, grid, st, a);
    else launch_rope<BF16, false>(head_dim, grid, st, a);
  } else {
    if (fp8) launch_rope<F16, true>(head_dim, grid, st, a);
    else launch_rope<F16, false>(head_dim, grid, st, a);
  }
  return check_launch(name);
}

}  // namespace

extern "C" int npd_qk_norm_rope_store(void* q_out, void* k_cache, void* v_cache, const void* qkv,
                                      const int32_t* slot_mapping, const int32_t* positions,
                                      const float* inv_freq, const void* q_norm_weight,
                                      const void* k_norm_weight, int64_t num_tokens,
                                      int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                                      int64_t num_blocks, int64_t block_size,
                                      int64_t qkv_stride_token, int64_t q_stride_token, float eps,
                                      int32_t dtype, void* stream) {
  return rope_impl(q_out, k_cache, v_cache, qkv, slot_mapping, positions, inv_freq, q_norm_weight,
                   k_norm_weight, nullptr, nullptr, num_tokens, num_heads, num_kv_heads, head_dim,
                   num_blocks, block_size, qkv_stride_token, q_stride_token, eps, dtype, stream,
                   false, "npd_qk_norm_rope_store");
}

extern "C" int npd_qk_norm_rope_store_fp8(void* q_out, void* k_cache, void* v_cache,
                                          const void* qkv, const int32_t* slot_mapping,
                                          const int32_t* positions, const float* inv_freq,
                                          const void* q_norm_weight, const void* k_norm_weight,
                                          const float* k_scale, const float* v_scale,
                                          int64_t num_tokens, int64_t num_heads,
                                          int64_t num_kv_heads, int64_t head_dim,
                                          int64_t num_blocks, int64_t block_size,
                                          int64_t qkv_stride_token, int64_t q_stride_token,
                                          float eps, int32_t dtype, void* stream) {
  return rope_impl(q_out, k_cache, v_cache, qkv, slot_mapping, positions, inv_freq, q_norm_weight,
                   k_norm_weight, k_scale, v_scale, num_tokens, num_heads, num_kv_heads, head_dim,
                   num_blocks, block_size, qkv_stride_token, q_stride_token, eps, dtype, stream,
                   true, "npd_qk_norm_rope_store_fp8");
}
