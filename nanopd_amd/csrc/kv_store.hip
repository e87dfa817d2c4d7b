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
// configuration 3's size (2096 tokens, 17.2 MB moved) a launch takes 3.4 us
// back to back, against 2.8 us for a one-token store: the fixed cost of a
// launch, not HBM, bounds it. Measured and dropped at that size: 2 or 4
// chunks per thread (3.8 / 4.7 us), 64- or 512-thread workgroups (same or
// slower), non-temporal loads and stores (2.99 us on one box, 3.97 on another).
#include "common.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;

// LPR = 16-byte lanes per head row (head_dim / 8).
template <int LPR, bool kSlots>
__global__ __launch_bounds__(kThreads) void kv_store_kernel(
    u32x4* __restrict__ k_cache, u32x4* __restrict__ v_cache,
    const u32x4* __restrict__ k_src, const u32x4* __restrict__ v_src,
    const int32_t* __restrict__ block_tables, const int32_t* __restrict__ index,
    int64_t total, int num_kv_heads, int block_size, int num_blocks, int max_bps,
    int64_t stride_head_v, int64_t stride_token_v) {
  const int64_t gid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (gid >= total) return;
  const int c = (int)(gid & (LPR - 1));
  const int64_t row = gid / LPR;
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
  const int64_t dst = (((int64_t)blk * num_kv_heads + h) * block_size + off) * LPR + c;
  const u32x4 kv = k_src[src];
  const u32x4 vv = v_src[src];
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
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(NPD_E_INVALID, "%s: head_dim %lld not in {64, 128, 256}", name, (long long)head_dim);
  if (!slots && max_bps <= 0)
    return fail(NPD_E_INVALID, "%s: max_blocks_per_seq must be positive", name);
  if (num_blocks * block_size > INT32_MAX || num_tokens > INT32_MAX)
    return fail(NPD_E_INVALID, "%s: pool or token count exceeds int32 indexing", name);
  if (num_tokens == 0) return NPD_OK;
  if (!k_cache || !v_cache || !k_src || !v_src || !index || (!slots && !block_tables))
    return fail(NPD_E_INVALID, "%s: null pointer", name);
  if (!aligned16(k_cache) || !aligned16(v_cache) || !aligned16(k_src) || !aligned16(v_src))
    return fail(NPD_E_ALIGN, "%s: cache and source pointers must be 16-byte aligned", name);
  if ((stride_head % 8) != 0 || (stride_token % 8) != 0 || stride_head < 0 || stride_token < 0)
    return fail(NPD_E_ALIGN, "%s: source strides (%lld, %lld) must be non-negative multiples of 8 elements",
                name, (long long)stride_head, (long long)stride_token);

  const int lpr = (int)(head_dim / 8);
  const int64_t total = num_tokens * num_kv_heads * lpr;
  const int64_t grid = (total + kThreads - 1) / kThreads;
  hipStream_t st = as_stream(stream);
  auto* kc = static_cast<u32x4*>(k_cache);
  auto* vc = static_cast<u32x4*>(v_cache);
  auto* ks = static_cast<const u32x4*>(k_src);
  auto* vs = static_cast<const u32x4*>(v_src);
  const int64_t sh = stride_head / 8, stt = stride_token / 8;
#define NPD_STORE_LAUNCH(L)                                                                    \
  do {                                                                                         \
    if (slots)                                                                                 \
      hipLaunchKernelGGL((kv_store_kernel<L, true>), dim3((unsigned)grid), dim3(kThreads), 0, \
                         st, kc, vc, ks, vs, block_tables, index, total, (int)num_kv_heads,    \
                         (int)block_size, (int)num_blocks, (int)max_bps, sh, stt);             \
    else                                                                                       \
      hipLaunchKernelGGL((kv_store_kernel<L, false>), dim3((unsigned)grid), dim3(kThreads), 0, \
                         st, kc, vc, ks, vs, block_tables, index, total, (int)num_kv_heads,    \
                         (int)block_size, (int)num_blocks, (int)max_bps, sh, stt);             \
  } while (0)
  switch (lpr) {
    case 8: NPD_STORE_LAUNCH(8); break;
    case 16: NPD_STORE_LAUNCH(16); break;
    default: NPD_STORE_LAUNCH(32); break;
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
