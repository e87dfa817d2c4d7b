// Paged KV store: scatter new K/V rows into the block pool.
//
// Reference: PA/csrc/kvstore/paged_kv_store_kernel.cu:16-58 (one 32-thread
// block per (token, head) moving 8 bytes per thread) and its host wrapper
// PA/csrc/kvstore/paged_kv_store_ops.cu:7-50.
//
// Here one thread moves 16 bytes (a dwordx4) of K and 16 bytes of V, a
// head row of D 2-byte elements takes D/8 lanes, so one wave64 writes 4 (D=128)
// rows of K and 4 of V as fully coalesced 1 KiB bursts. The grid is flat over
// (token, head, 16-byte chunk); every launch shape divides evenly. At
// configuration 3's size (2096 tokens, 17.2 MB moved) a launch takes 3.84 us
// back to back (4.32 us in a rocprofv3 trace), against 2.8 us for a one-token
// store: the fixed cost of a launch, not HBM, bounds it. Measured and dropped
// at that size: 2 or 4 chunks per thread (3.8 / 4.7 us against 3.4 us on that
// box), 64- or 512-thread workgroups (same or slower), non-temporal loads and
// stores (2.99 us on one box, 3.97 on another).
// Head dims 64, 128 and 256 have compile-time lane counts; any other multiple
// of 8 runs the same kernel with a runtime count, and a head dim of 4 mod 8
// moves 8-byte vectors (the reference's float2 granularity, any head_dim % 4
// == 0, paged_kv_store_ops.cu:25-26).
#include "common.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;

// LPR = vector lanes per head row: head_dim / 8 for 16-byte vectors (V =
// u32x4), head_dim / 4 for 8-byte ones (u32x2). LPR 0: a runtime lane count
// `lpr` (head dims other than 64, 128 and 256).
template <int LPR, bool kSlots, class V = u32x4>
__global__ __launch_bounds__(kThreads) void kv_store_kernel(
    V* __restrict__ k_cache, V* __restrict__ v_cache,
    const V* __restrict__ k_src, const V* __restrict__ v_src,
    const int32_t* __restrict__ block_tables, const int32_t* __restrict__ index,
    int64_t total, int num_kv_heads, int block_size, int num_blocks, int max_bps,
    int64_t stride_head_v, int64_t stride_token_v, int lpr) {
  const int64_t gid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (gid >= total) return;
  const int lanes = LPR > 0 ? LPR : lpr;
  const int64_t row = LPR > 0 ? gid / LPR : gid / lanes;
  const int c = (int)(gid - row * lanes);
  const int t = (int)(row / num_kv_heads);
  const int h = (int)(row - (int64_t)t * num_kv_heads);

  int blk, off;
  if constexpr (kSlots) {
    const int slot = index[t];
    if (slot < 0 || slot >= num_blocks * block_size) return;
    blk = slot / block_size;
    off = slot - blk * block_size;
  } else {
    const int pos = index[t];
    if (pos < 0) return;
    const int lb = pos / block_size;
    if (lb >= max_bps) return;
    blk = block_tables[(int64_t)t * max_bps + lb];
    if (blk < 0 || blk >= num_blocks) return;
    off = pos - lb * block_size;
  }
  const int64_t src = (int64_t)h * stride_head_v + (int64_t)t * stride_token_v + c;
  const int64_t dst = (((int64_t)blk * num_kv_heads + h) * block_size + off) * lanes + c;
  const V kv = k_src[src];
  const V vv = v_src[src];
  k_cache[dst] = kv;
  v_cache[dst] = vv;
}

int launch_store(bool slots, void* k_cache, void* v_cache, const void* k_src,
                 const void* v_src, const int32_t* block_tables, const int32_t* index,
                 int64_t num_tokens, int64_t num_kv_heads, int64_t head_dim,
                 int64_t num_blocks, int64_t block_size, int64_t max_bps,
                 int64_t stride_head, int64_t stride_token, int32_t dtype, void* stream,
                 const char* name) {
  using namespace npd;
  if (dtype != NPD_DTYPE_F16 && dtype != NPD_DTYPE_BF16)
    return fail(NPD_E_DTYPE, "%s: unsupported dtype code %d (fp16/bf16 only)", name, dtype);
  if (num_tokens < 0 || num_kv_heads <= 0 || block_size <= 0 || num_blocks <= 0)
    return fail(NPD_E_INVALID, "%s: bad sizes (tokens %lld, kv heads %lld, block %lld, blocks %lld)",
                name, (long long)num_tokens, (long long)num_kv_heads, (long long)block_size,
                (long long)num_blocks);
  if (head_dim <= 0 || head_dim % 4 != 0 || head_dim > 4096)
    return fail(NPD_E_INVALID, "%s: head_dim %lld is not a positive multiple of 4 (at most 4096)",
                name, (long long)head_dim);
  if (!slots && max_bps <= 0)
    return fail(NPD_E_INVALID, "%s: max_blocks_per_seq must be positive", name);
  if (num_blocks * block_size > INT32_MAX || num_tokens > INT32_MAX)
    return fail(NPD_E_INVALID, "%s: pool or token count exceeds int32 indexing", name);
  if (num_tokens == 0) return NPD_OK;
  if (!k_cache || !v_cache || !k_src || !v_src || !index || (!slots && !block_tables))
    return fail(NPD_E_INVALID, "%s: null pointer", name);
  // 16-byte vectors when head rows are whole 16-byte units, else 8-byte ones
  // (head_dim % 8 == 4, rows of 8-byte units as the reference moves them)
  const bool v16 = head_dim % 8 == 0;
  const int vb = v16 ? 16 : 8;   // vector bytes
  const uintptr_t am = (uintptr_t)vb - 1;
  if (((uintptr_t)k_cache & am) || ((uintptr_t)v_cache & am) || ((uintptr_t)k_src & am) ||
      ((uintptr_t)v_src & am))
    return fail(NPD_E_ALIGN, "%s: cache and source pointers must be %d-byte aligned", name, vb);
  const int64_t ve = vb / 2;     // elements per vector
  if ((stride_head % ve) != 0 || (stride_token % ve) != 0 || stride_head < 0 || stride_token < 0)
    return fail(NPD_E_ALIGN, "%s: source strides (%lld, %lld) must be non-negative multiples of %lld elements",
                name, (long long)stride_head, (long long)stride_token, (long long)ve);

  const int lpr = (int)(head_dim / ve);
  const int64_t total = num_tokens * num_kv_heads * lpr;
  const int64_t grid = (total + kThreads - 1) / kThreads;
  hipStream_t st = as_stream(stream);
  const int64_t sh = stride_head / ve, stt = stride_token / ve;
  const int nkv = (int)num_kv_heads, bsz = (int)block_size, nbk = (int)num_blocks, mbs = (int)max_bps;
#define NPD_STORE_LAUNCH(L, V)                                                                   \
  do {                                                                                           \
    auto* kc = static_cast<V*>(k_cache);                                                         \
    auto* vc = static_cast<V*>(v_cache);                                                         \
    auto* ks = static_cast<const V*>(k_src);                                                     \
    auto* vs = static_cast<const V*>(v_src);                                                     \
    if (slots)                                                                                   \
      hipLaunchKernelGGL((kv_store_kernel<L, true, V>), dim3((unsigned)grid), dim3(kThreads), 0, \
                         st, kc, vc, ks, vs, block_tables, index, total, nkv, bsz, nbk, mbs, sh, \
                         stt, lpr);                                                              \
    else                                                                                         \
      hipLaunchKernelGGL((kv_store_kernel<L, false, V>), dim3((unsigned)grid), dim3(kThreads), 0, \
                         st, kc, vc, ks, vs, block_tables, index, total, nkv, bsz, nbk, mbs, sh, \
                         stt, lpr);                                                              \
  } while (0)
  if (!v16) {
    NPD_STORE_LAUNCH(0, u32x2);
  } else {
    switch (lpr) {
      case 8: NPD_STORE_LAUNCH(8, u32x4); break;
      case 16: NPD_STORE_LAUNCH(16, u32x4); break;
      case 32: NPD_STORE_LAUNCH(32, u32x4); break;
      default: NPD_STORE_LAUNCH(0, u32x4); break;
    }
  }
#undef NPD_STORE_LAUNCH
  return check_launch(name);
}

}  // namespace

extern "C" int npd_paged_kv_store(void* k_cache, void* v_cache, const void* k_src,
                                  const void* v_src, const int32_t* block_tables,
                                  const int32_t* positions, int64_t num_tokens,
                                  int64_t num_kv_heads, int64_t head_dim, int64_t num_blocks,
                                  int64_t block_size, int64_t max_blocks_per_seq,
                                  int64_t src_stride_head, int64_t src_stride_token,
                                  int32_t dtype, void* stream) {
  return launch_store(false, k_cache, v_cache, k_src, v_src, block_tables, positions,
                      num_tokens, num_kv_heads, head_dim, num_blocks, block_size,
                      max_blocks_per_seq, src_stride_head, src_stride_token, dtype, stream,
                      "npd_paged_kv_store");
}

extern "C" int npd_paged_kv_store_slots(void* k_cache, void* v_cache, const void* k_src,
                                        const void* v_src, const int32_t* slot_mapping,
                                        int64_t num_tokens, int64_t num_kv_heads,
                                        int64_t head_dim, int64_t num_blocks,
                                        int64_t block_size, int64_t src_stride_head,
                                        int64_t src_stride_token, int32_t dtype,
                                        void* stream) {
  return launch_store(true, k_cache, v_cache, k_src, v_src, nullptr, slot_mapping, num_tokens,
                      num_kv_heads, head_dim, num_blocks, block_size, 0, src_stride_head,
                      src_stride_token, dtype, stream, "npd_paged_kv_store_slots");
}
