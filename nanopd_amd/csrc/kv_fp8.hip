// FP8 (OCP e4m3) paged KV pool: the store side.
//
// No counterpart in the reference (its caches are fp16 only,
// nanoPD/engine/model_runner.py:24-31); this is the next format after the
// 2-byte pool. A pool element is one e4m3 byte with a per-kv-head fp32 scale:
// value = e4m3(byte) * scale[head]. Storing rounds x / scale[head] (an IEEE
// fp32 division) to the nearest e4m3 value, ties to even, after clamping to
// the format's range [-448, 448]; NaN stays NaN. The pool layout is the
// 2-byte one with 1-byte elements: [num_blocks, num_kv_heads, block_size,
// head_dim], so a (block, kv-head) tile of Qwen3-8B shapes is 2 KiB.
//
// One thread converts 8 elements: a 16-byte source load, 8 fp32 divisions,
// four v_cvt_pk_fp8_f32, one 8-byte store; a wave writes 4 head rows of K and
// 4 of V (D = 128) as 512-byte bursts.
#include "common.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
constexpr int kThreads = 256;

__device__ __forceinline__ float clamp8(float x) { return npd::e4m3_clamp(x); }

// 8 source elements (4 packed pairs) / scale -> 8 e4m3 bytes
template <class TT>
__device__ __forceinline__ u32x2 to_e4m3(u32x4 w, float scale) {
  const uint32_t in[4] = {w.x, w.y, w.z, w.w};
  uint32_t out[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    int acc = 0;
    acc = __builtin_amdgcn_cvt_pk_fp8_f32(clamp8(TT::lo(in[2 * p]) / scale),
                                          clamp8(TT::hi(in[2 * p]) / scale), acc, false);
    acc = __builtin_amdgcn_cvt_pk_fp8_f32(clamp8(TT::lo(in[2 * p + 1]) / scale),
                                          clamp8(TT::hi(in[2 * p + 1]) / scale), acc, true);
    out[p] = (uint32_t)acc;
  }
  return u32x2{out[0], out[1]};
}

// LPR = 8-element chunks per head row (head_dim / 8); 0: a runtime count
// `lpr` (head dims other than 64, 128 and 256).
template <class TT, int LPR>
__global__ __launch_bounds__(kThreads) void kv_store_fp8_kernel(
    u32x2* __restrict__ k_cache, u32x2* __restrict__ v_cache, const u32x4* __restrict__ k_src,
    const u32x4* __restrict__ v_src, const int32_t* __restrict__ slots,
    const float* __restrict__ k_scale, const float* __restrict__ v_scale, int64_t total,
    int num_kv_heads, int block_size, int num_blocks, int64_t stride_head_v,
    int64_t stride_token_v, int lpr) {
  const int64_t gid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (gid >= total) return;
  const int lanes = LPR > 0 ? LPR : lpr;
  const int64_t row = LPR > 0 ? gid / LPR : gid / lanes;
  const int c = (int)(gid - row * lanes);
  const int t = (int)(row / num_kv_heads);
  const int h = (int)(row - (int64_t)t * num_kv_heads);
  const int slot = slots[t];
  if (slot < 0 || slot >= num_blocks * block_size) return;
  const int blk = slot / block_size;
  const int off = slot - blk * block_size;
  const int64_t src = (int64_t)h * stride_head_v + (int64_t)t * stride_token_v + c;
  const int64_t dst = (((int64_t)blk * num_kv_heads + h) * block_size + off) * lanes + c;
  k_cache[dst] = to_e4m3<TT>(k_src[src], k_scale[h]);
  v_cache[dst] = to_e4m3<TT>(v_src[src], v_scale[h]);
}

}  // namespace

extern "C" int npd_paged_kv_store_slots_fp8(void* k_cache, void* v_cache, const void* k_src,
                                            const void* v_src, const int32_t* slot_mapping,
                                            const float* k_scale, const float* v_scale,
                                            int64_t num_tokens, int64_t num_kv_heads,
                                            int64_t head_dim, int64_t num_blocks,
                                            int64_t block_size, int64_t src_stride_head,
                                            int64_t src_stride_token, int32_t src_dtype,
                                            void* stream) {
  using namespace npd;
  const char* name = "npd_paged_kv_store_slots_fp8";
  if (src_dtype != NPD_DTYPE_F16 && src_dtype != NPD_DTYPE_BF16)
    return fail(NPD_E_DTYPE, "%s: unsupported source dtype code %d (fp16/bf16 only)", name,
                src_dtype);
  if (num_tokens < 0 || num_kv_heads <= 0 || block_size <= 0 || num_blocks <= 0)
    return fail(NPD_E_INVALID, "%s: bad sizes (tokens %lld, kv heads %lld, block %lld, blocks %lld)",
                name, (long long)num_tokens, (long long)num_kv_heads, (long long)block_size,
                (long long)num_blocks);
  if (head_dim <= 0 || head_dim % 8 != 0 || head_dim > 4096)
    return fail(NPD_E_INVALID, "%s: head_dim %lld is not a positive multiple of 8 (at most 4096)",
                name, (long long)head_dim);
  if (num_blocks * block_size > INT32_MAX || num_tokens > INT32_MAX)
    return fail(NPD_E_INVALID, "%s: pool or token count exceeds int32 indexing", name);
  if (num_tokens == 0) return NPD_OK;
  if (!k_cache || !v_cache || !k_src || !v_src || !slot_mapping || !k_scale || !v_scale)
    return fail(NPD_E_INVALID, "%s: null pointer", name);
  if ((reinterpret_cast<uintptr_t>(k_cache) & 7u) || (reinterpret_cast<uintptr_t>(v_cache) & 7u) ||
      !aligned16(k_src) || !aligned16(v_src))
    return fail(NPD_E_ALIGN, "%s: caches must be 8-byte aligned, sources 16-byte aligned", name);
  if ((src_stride_head % 8) != 0 || (src_stride_token % 8) != 0 || src_stride_head < 0 ||
      src_stride_token < 0)
    return fail(NPD_E_ALIGN, "%s: source strides must be non-negative multiples of 8 elements",
                name);
  const int lpr = (int)(head_dim / 8);
  const int64_t total = num_tokens * num_kv_heads * lpr;
  const int64_t grid = (total + kThreads - 1) / kThreads;
  hipStream_t st = as_stream(stream);
  auto* kc = static_cast<u32x2*>(k_cache);
  auto* vc = static_cast<u32x2*>(v_cache);
  auto* ks = static_cast<const u32x4*>(k_src);
  auto* vs = static_cast<const u32x4*>(v_src);
  const int64_t sh = src_stride_head / 8, stt = src_stride_token / 8;
#define NPD_FP8_LAUNCH(T, L)                                                                   \
  hipLaunchKernelGGL((kv_store_fp8_kernel<T, L>), dim3((unsigned)grid), dim3(kThreads), 0, st, \
                     kc, vc, ks, vs, slot_mapping, k_scale, v_scale, total, (int)num_kv_heads, \
                     (int)block_size, (int)num_blocks, sh, stt, lpr)
  const bool bf = src_dtype == NPD_DTYPE_BF16;
  switch (lpr) {
    case 8: if (bf) NPD_FP8_LAUNCH(BF16, 8); else NPD_FP8_LAUNCH(F16, 8); break;
    case 16: if (bf) NPD_FP8_LAUNCH(BF16, 16); else NPD_FP8_LAUNCH(F16, 16); break;
    case 32: if (bf) NPD_FP8_LAUNCH(BF16, 32); else NPD_FP8_LAUNCH(F16, 32); break;
    default: if (bf) NPD_FP8_LAUNCH(BF16, 0); else NPD_FP8_LAUNCH(F16, 0); break;
  }
#undef NPD_FP8_LAUNCH
  return check_launch(name);
}
