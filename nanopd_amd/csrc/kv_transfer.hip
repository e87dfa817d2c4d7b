// Block-list pack / unpack of the paged KV pool: the single-GPU half of KV
// transfer for prefill/decode disaggregation.
//
// The reference moves a sequence's KV between GPUs block by block:
// extract_kv_to_pinned / load_kv_from_pinned copy k_cache[:, bid] (every
// layer of one block) into / out of a buffer laid out [layers, n, kv heads,
// block size, head dim], one torch copy per block and tensor
// (nanoPD/workers/kv_transfer.py:45-69), and the P2P path does the same per
// block between devices (:72-82). Here one launch gathers every (layer, block)
// of a block list into that wire layout (or scatters it back into a pool at
// another block list), so the cross-device step is a single contiguous copy
// of the buffer (hipMemcpyPeerAsync, or an RCCL send/recv over xGMI).
//
// Work unit: one workgroup moves up to kChunk bytes of one (layer, block) of
// K and the same of V as 16-byte non-temporal loads and stores (each byte is
// touched once). Element type does not matter: blocks are moved as bytes.
#include "common.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
constexpr int kUnroll = 4;
constexpr int64_t kChunk = (int64_t)kThreads * kUnroll * 16;   // bytes per workgroup and tensor

// grid: x = chunk of a block, y = list entry i, z = layer.
// kGather: pool[layer, ids[i]] -> wire[layer, i]; else wire -> pool.
template <bool kGather>
__global__ __launch_bounds__(kThreads) void kv_blocks_kernel(
    u32x4* __restrict__ k_pool, u32x4* __restrict__ v_pool, u32x4* __restrict__ k_wire,
    u32x4* __restrict__ v_wire, const int32_t* __restrict__ ids, int64_t n, int64_t num_blocks,
    int64_t vecs_per_block) {
  const int64_t i = blockIdx.y, layer = blockIdx.z;
  const int bid = ids[i];
  const bool valid = bid >= 0 && bid < num_blocks;
  if (!kGather && !valid) return;   // never write outside the pool
  const int64_t pool0 = (layer * num_blocks + (valid ? bid : 0)) * vecs_per_block;
  const int64_t wire0 = (layer * n + i) * vecs_per_block;
  const int64_t v0 = (int64_t)blockIdx.x * (kThreads * kUnroll) + threadIdx.x;
  u32x4 kv[kUnroll], vv[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t e = v0 + (int64_t)u * kThreads;
    if (e < vecs_per_block) {
      if (kGather) {
        kv[u] = valid ? __builtin_nontemporal_load(k_pool + pool0 + e) : u32x4{0, 0, 0, 0};
        vv[u] = valid ? __builtin_nontemporal_load(v_pool + pool0 + e) : u32x4{0, 0, 0, 0};
      } else {
        kv[u] = __builtin_nontemporal_load(k_wire + wire0 + e);
        vv[u] = __builtin_nontemporal_load(v_wire + wire0 + e);
      }
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t e = v0 + (int64_t)u * kThreads;
    if (e < vecs_per_block) {
      if (kGather) {
        __builtin_nontemporal_store(kv[u], k_wire + wire0 + e);
        __builtin_nontemporal_store(vv[u], v_wire + wire0 + e);
      } else {
        __builtin_nontemporal_store(kv[u], k_pool + pool0 + e);
        __builtin_nontemporal_store(vv[u], v_pool + pool0 + e);
      }
    }
  }
}

int launch(bool gather, void* k_pool, void* v_pool, void* k_wire, void* v_wire,
           const int32_t* ids, int64_t n, int64_t num_layers, int64_t num_blocks,
           int64_t block_bytes, void* stream, const char* name) {
  using namespace npd;
  if (n < 0 || num_layers <= 0 || num_blocks <= 0 || block_bytes <= 0)
    return fail(NPD_E_INVALID, "%s: bad sizes (n %lld, layers %lld, blocks %lld, block bytes %lld)",
                name, (long long)n, (long long)num_layers, (long long)num_blocks,
                (long long)block_bytes);
  if (block_bytes % 16 != 0)
    return fail(NPD_E_ALIGN, "%s: block of %lld bytes is not a multiple of 16", name,
                (long long)block_bytes);
  if (n > 65535 || num_layers > 65535)
    return fail(NPD_E_INVALID, "%s: at most 65535 blocks and layers per call", name);
  if (n == 0) return NPD_OK;
  if (!k_pool || !v_pool || !k_wire || !v_wire || !ids)
    return fail(NPD_E_INVALID, "%s: null pointer", name);
  if (!aligned16(k_pool) || !aligned16(v_pool) || !aligned16(k_wire) || !aligned16(v_wire))
    return fail(NPD_E_ALIGN, "%s: pool and wire pointers must be 16-byte aligned", name);
  const int64_t vecs = block_bytes / 16;
  const dim3 grid((unsigned)((block_bytes + kChunk - 1) / kChunk), (unsigned)n, (unsigned)num_layers);
  auto* kp = static_cast<u32x4*>(k_pool);
  auto* vp = static_cast<u32x4*>(v_pool);
  auto* kw = static_cast<u32x4*>(k_wire);
  auto* vw = static_cast<u32x4*>(v_wire);
  if (gather)
    hipLaunchKernelGGL(kv_blocks_kernel<true>, grid, dim3(kThreads), 0, as_stream(stream), kp, vp,
                       kw, vw, ids, n, num_blocks, vecs);
  else
    hipLaunchKernelGGL(kv_blocks_kernel<false>, grid, dim3(kThreads), 0, as_stream(stream), kp,
                       vp, kw, vw, ids, n, num_blocks, vecs);
  return check_launch(name);
}

}  // namespace

extern "C" int npd_kv_gather_blocks(const void* k_cache, const void* v_cache, int64_t num_layers,
                                    int64_t num_blocks, int64_t block_bytes,
                                    const int32_t* block_ids, int64_t num_ids, void* wire_k,
                                    void* wire_v, void* stream) {
  return launch(true, const_cast<void*>(k_cache), const_cast<void*>(v_cache), wire_k, wire_v,
                block_ids, num_ids, num_layers, num_blocks, block_bytes, stream,
                "npd_kv_gather_blocks");
}

extern "C" int npd_kv_scatter_blocks(void* k_cache, void* v_cache, int64_t num_layers,
                                     int64_t num_blocks, int64_t block_bytes,
                                     const int32_t* block_ids, int64_t num_ids,
                                     const void* wire_k, const void* wire_v, void* stream) {
  return launch(false, k_cache, v_cache, const_cast<void*>(wire_k), const_cast<void*>(wire_v),
                block_ids, num_ids, num_layers, num_blocks, block_bytes, stream,
                "npd_kv_scatter_blocks");
}
