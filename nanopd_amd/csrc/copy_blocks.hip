// Copy-on-write block copy: duplicate whole pool blocks of K and V.
//
// The reference computes the (src, dst) pair in BlockSpaceManager.append_slot
// (nanoPD/block_manager/block_manager.py:91-96) but never copies; this is the
// missing op. Each block is num_kv_heads*block_size*head_dim 2-byte elements
// (64 KiB of K+V for Qwen3-8B shapes), moved as 16-byte vectors.
#include "common.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;

// grid.x strides over one block's vectors, grid.y = pair index.
__global__ __launch_bounds__(kThreads) void copy_blocks_kernel(
    u32x4* __restrict__ k_cache, u32x4* __restrict__ v_cache,
    const int32_t* __restrict__ pairs, int num_blocks, int64_t vecs_per_block) {
  const int src = pairs[2 * blockIdx.y];
  const int dst = pairs[2 * blockIdx.y + 1];
  if (src < 0 || src >= num_blocks || dst < 0 || dst >= num_blocks) return;
  const int64_t s0 = (int64_t)src * vecs_per_block, d0 = (int64_t)dst * vecs_per_block;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < vecs_per_block;
       i += (int64_t)gridDim.x * kThreads) {
    const u32x4 kv = k_cache[s0 + i];
    const u32x4 vv = v_cache[s0 + i];
    k_cache[d0 + i] = kv;
    v_cache[d0 + i] = vv;
  }
}

}  // namespace

extern "C" int npd_copy_blocks(void* k_cache, void* v_cache, const int32_t* pairs,
                               int64_t num_pairs, int64_t num_blocks, int64_t block_elems,
                               int32_t dtype, void* stream) {
  using namespace npd;
  const char* name = "npd_copy_blocks";
  if (dtype != NPD_DTYPE_F16 && dtype != NPD_DTYPE_BF16)
    return fail(NPD_E_DTYPE, "%s: unsupported dtype code %d (fp16/bf16 only)", name, dtype);
  if (num_pairs < 0 || num_blocks <= 0 || block_elems <= 0 || num_blocks > INT32_MAX)
    return fail(NPD_E_INVALID, "%s: bad sizes (pairs %lld, blocks %lld, block elems %lld)", name,
                (long long)num_pairs, (long long)num_blocks, (long long)block_elems);
  if (num_pairs > 65535)
    return fail(NPD_E_INVALID, "%s: at most 65535 pairs per call (got %lld)", name,
                (long long)num_pairs);
  if (block_elems % 8 != 0)
    return fail(NPD_E_ALIGN, "%s: block of %lld elements is not a multiple of 16 bytes", name,
                (long long)block_elems);
  if (num_pairs == 0) return NPD_OK;
  if (!k_cache || !v_cache || !pairs) return fail(NPD_E_INVALID, "%s: null pointer", name);
  if (!aligned16(k_cache) || !aligned16(v_cache))
    return fail(NPD_E_ALIGN, "%s: cache pointers must be 16-byte aligned", name);
  const int64_t vecs = block_elems / 8;
  const int64_t gx = (vecs + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(copy_blocks_kernel, dim3((unsigned)(gx < 1024 ? gx : 1024), (unsigned)num_pairs),
                     dim3(kThreads), 0, as_stream(stream), static_cast<u32x4*>(k_cache),
                     static_cast<u32x4*>(v_cache), pairs, (int)num_blocks, vecs);
  return check_launch(name);
}
