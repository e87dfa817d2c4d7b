/*
 * nanopd.h -- C ABI of libnanopd_hip.so, the MI355X (gfx950) implementation of
 * nanoPD's `paged_kernels` extension: the paged KV store and paged attention
 * that ModelRunner.paged_forward calls once per attention layer.
 *
 * Conventions (all entry points):
 *   - Every pointer is a device pointer unless stated otherwise; the caller owns
 *     all memory. The library keeps no pointer after a call returns.
 *   - Caches are the reference layout [num_blocks, num_kv_heads, block_size,
 *     head_dim], contiguous (nanoPD/engine/model_runner.py:24-31).
 *   - dtype: NPD_DTYPE_F16 or NPD_DTYPE_BF16 (elements of 2 bytes).
 *   - stream: a hipStream_t passed as void* (NULL = the null stream). Work is
 *     enqueued on it; no call synchronises the host.
 *   - Return value: 0 on success, a negative NPD_E* code on failure. Nothing is
 *     launched when validation fails. npd_last_error() gives a message for the
 *     last failure on the calling thread. No C++ exception crosses the ABI, and
 *     the process is never terminated (the reference calls exit(), see
 *     PA/csrc/utils/cuda_utils.h:18-29).
 *   - Index contents are checked in the kernels, not on the host (that would
 *     need a device-to-host sync): a token whose slot or block falls outside the
 *     pool is skipped by the stores, and attention clamps block ids into the
 *     pool so that no access leaves it.
 *   - Thread-safe and reentrant: no mutable global state beyond the per-thread
 *     error message, except the static scratch of npd_paged_attention_noalloc
 *     (one per device, set up once under a lock; see there).
 * Citations are relative to the reference tree; PA/ = nanoPD/paged_attention/.
 */
#ifndef NANOPD_H
#define NANOPD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NPD_DTYPE_F16  0
#define NPD_DTYPE_BF16 1

#define NPD_OK              0
#define NPD_E_INVALID      -1  /* bad shape, size, stride or argument */
#define NPD_E_DTYPE        -2  /* unsupported element type */
#define NPD_E_ALIGN        -3  /* pointer or stride not 16-byte aligned */
#define NPD_E_WORKSPACE    -4  /* workspace missing or too small */
#define NPD_E_LAUNCH       -5  /* the HIP runtime reported an error */

/* Message for the last failed call on this thread ("" if none). */
const char* npd_last_error(void);

/* Library version, e.g. 100 for 0.1.0. */
int npd_version(void);

/*
 * Paged KV store, per-token block tables.
 * Replaces paged_kv_store (PA/csrc/kvstore/paged_kv_store.h:23-27,
 * PA/csrc/kvstore/paged_kv_store_ops.cu:7-50, kernel
 * PA/csrc/kvstore/paged_kv_store_kernel.cu:16-58).
 * For token t < num_tokens and head h < num_kv_heads:
 *   pos = positions[t];  blk = block_tables[t * max_blocks_per_seq + pos / block_size]
 *   k_cache[blk, h, pos % block_size, :] = k_src[h * src_stride_head + t * src_stride_token + :]
 *   (same for v). Strides are in elements; the reference passes k_src
 *   [kvh, T, D] contiguous, i.e. src_stride_head = T*D, src_stride_token = D.
 * Tokens with pos < 0, pos / block_size >= max_blocks_per_seq or blk outside
 * [0, num_blocks) are skipped.
 * head_dim: any positive multiple of 4 up to 4096, as the reference's
 * (PA/csrc/kvstore/paged_kv_store_ops.cu:25-26 moves 8-byte pieces). Caches
 * and sources 16-byte aligned with strides in multiples of 8 elements, or, when
 * head_dim % 8 == 4, 8-byte aligned with strides in multiples of 4.
 */
int npd_paged_kv_store(void* k_cache, void* v_cache,
                       const void* k_src, const void* v_src,
                       const int32_t* block_tables, const int32_t* positions,
                       int64_t num_tokens, int64_t num_kv_heads, int64_t head_dim,
                       int64_t num_blocks, int64_t block_size,
                       int64_t max_blocks_per_seq,
                       int64_t src_stride_head, int64_t src_stride_token,
                       int32_t dtype, void* stream);

/*
 * Paged KV store driven by a flat slot mapping (no reference counterpart; the
 * reference builds a [T, max_bps] table per prefill sequence per layer for it,
 * nanoPD/engine/model_runner.py:132-150):
 *   slot = slot_mapping[t]; if slot < 0 or slot >= num_blocks*block_size: skip
 *   k_cache[slot / block_size, h, slot % block_size, :] = k_src[t*src_stride_token + h*src_stride_head + :]
 * Accepts token-major sources ([T, kvh, D] straight from k_proj) without a copy.
 * head_dim, alignment and strides as npd_paged_kv_store.
 */
int npd_paged_kv_store_slots(void* k_cache, void* v_cache,
                             const void* k_src, const void* v_src,
                             const int32_t* slot_mapping,
                             int64_t num_tokens, int64_t num_kv_heads, int64_t head_dim,
                             int64_t num_blocks, int64_t block_size,
                             int64_t src_stride_head, int64_t src_stride_token,
                             int32_t dtype, void* stream);

/*
 * FP8 (OCP e4m3) pool variant of npd_paged_kv_store_slots (no reference
 * counterpart: the reference's caches are fp16, nanoPD/engine/model_runner.py:
 * 24-31). Caches hold one e4m3 byte per element, same [num_blocks, kvh,
 * block_size, head_dim] layout; k_scale / v_scale: fp32 [num_kv_heads].
 *   byte = e4m3_rne(clamp(x / scale[h], -448, 448))   (IEEE fp32 division;
 *   NaN stays NaN), so that element = e4m3(byte) * scale[h].
 * Sources are fp16 or bf16 (src_dtype), as in npd_paged_kv_store_slots.
 * Caches 8-byte aligned, sources 16-byte aligned; head_dim a positive multiple
 * of 8 up to 4096.
 */
int npd_paged_kv_store_slots_fp8(void* k_cache, void* v_cache,
                                 const void* k_src, const void* v_src,
                                 const int32_t* slot_mapping,
                                 const float* k_scale, const float* v_scale,
                                 int64_t num_tokens, int64_t num_kv_heads, int64_t head_dim,
                                 int64_t num_blocks, int64_t block_size,
                                 int64_t src_stride_head, int64_t src_stride_token,
                                 int32_t src_dtype, void* stream);

/*
 * Bytes of device workspace npd_paged_attention needs for these shapes (merge
 * counter region, work list, split-context partials). 0 means no workspace is
 * needed.
 */
int64_t npd_paged_attention_workspace_size(int64_t num_seqs, int64_t num_heads,
                                           int64_t num_kv_heads, int64_t head_dim,
                                           int64_t block_size, int64_t max_blocks_per_seq);

/*
 * Paged decode attention (one query token per sequence).
 * Replaces paged_attention_forward (PA/csrc/attention/paged_attention.h:24-34,
 * PA/csrc/attention/paged_attention_ops.cu:7-59, kernel
 * PA/csrc/attention/paged_attention_kernel.cu:39-151):
 *   out[s, h, :] = softmax(scale * q[s,h] . K[s, h / (H/kvh)]^T) . V[s, h / (H/kvh)]
 * over the first seq_lens[s] tokens, gathered through block_tables[s, :].
 * query/out strides are in elements (head_dim contiguous). seq_lens[s] <= 0
 * gives zeros; seq_lens[s] is clamped to max_blocks_per_seq * block_size.
 * Every output element is written: out need not be zeroed.
 * head_dim: a multiple of 8 from 32 to 256 (64, 128 and 256 have tuned
 * kernels; the reference takes multiples of 32 up to 1024,
 * PA/csrc/attention/paged_attention_kernel.cu:16-20).
 * workspace: at least npd_paged_attention_workspace_size(...) bytes, 256-byte
 * aligned (may be NULL when that size is 0), zero-filled before its first
 * use. Layout: a fixed 1 MiB region of merge counters (at most 262144
 * (sequence, kv-head) units) that every call leaves at zero, then the work
 * list and split-context partials. Partials never overlap the counter region,
 * so one workspace (large enough for each call) serves calls of any shape,
 * and npd_paged_prefill_attention calls too, if they are stream-ordered.
 */
int npd_paged_attention(void* out, const void* query,
                        const void* key_cache, const void* value_cache,
                        const int32_t* block_tables, const int32_t* seq_lens,
                        int64_t num_seqs, int64_t num_heads, int64_t num_kv_heads,
                        int64_t head_dim, int64_t num_blocks, int64_t block_size,
                        int64_t max_blocks_per_seq, float scale,
                        int64_t q_stride_seq, int64_t q_stride_head,
                        int64_t out_stride_seq, int64_t out_stride_head,
                        void* workspace, int64_t workspace_bytes,
                        int32_t dtype, void* stream);

/* Size of the static device scratch of npd_paged_attention_noalloc (64 MiB). */
#define NPD_NOALLOC_SCRATCH_BYTES (64LL << 20)

/*
 * npd_paged_attention without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, serving loops that forbid
 * hipMalloc). No counterpart in the reference (its decode op allocates
 * nothing because it has no split-context path).
 * Same arguments, semantics and results as npd_paged_attention; it calls no
 * hipMalloc / hipFree. Its workspace is a static device array of
 * NPD_NOALLOC_SCRATCH_BYTES that each GPU the library runs on holds until the
 * process ends; shapes whose npd_paged_attention_workspace_size exceeds it
 * fail with NPD_E_WORKSPACE (e.g. 64 sequences of up to 4096 tokens need
 * 17.3 MiB, 8 of up to 32768 need 18.3 MiB). Arguments are checked first, as
 * by npd_paged_attention (same error codes; nothing is launched on failure).
 * The device is the stream's (hipStreamGetDevice; the null stream's is the
 * calling thread's current device): the call makes it current while it looks
 * up that device's array and launches, then restores the caller's device. The
 * first call on a device looks up the array's address and enqueues the clear
 * of its counter region on `stream`. All calls on one GPU share the array: calls that overlap on one
 * GPU (concurrent streams or threads) race and must be serialised by the
 * caller; stream-ordered calls are safe, since every call leaves the counters
 * at zero.
 */
int npd_paged_attention_noalloc(void* out, const void* query,
                                const void* key_cache, const void* value_cache,
                                const int32_t* block_tables, const int32_t* seq_lens,
                                int64_t num_seqs, int64_t num_heads, int64_t num_kv_heads,
                                int64_t head_dim, int64_t num_blocks, int64_t block_size,
                                int64_t max_blocks_per_seq, float scale,
                                int64_t q_stride_seq, int64_t q_stride_head,
                                int64_t out_stride_seq, int64_t out_stride_head,
                                int32_t dtype, void* stream);

/*
 * Bytes of device workspace npd_paged_prefill_attention needs.
 */
int64_t npd_paged_prefill_workspace_size(int64_t num_seqs, int64_t total_q,
                                         int64_t num_heads, int64_t head_dim,
                                         int64_t max_q_len, int64_t max_context_len);

/*
 * Chunked-prefill attention over a paged prefix plus the new chunk (varlen).
 * Replaces the prefill branch of paged_forward, which runs
 * F.scaled_dot_product_attention over the chunk alone with a block-diagonal
 * causal mask (nanoPD/engine/model_runner.py:152-168); this op also reads the
 * prefix already in the pool, which the reference ignores.
 * Sequence s owns query rows cu_seqlens_q[s] .. cu_seqlens_q[s+1]-1 of query
 * [total_q, H, D]; its chunk K/V must already be stored in the pool;
 * context_lens[s] counts prefix + chunk tokens. Query row i of s sits at
 * position p = context_lens[s] - q_len_s + i and attends to keys 0..p.
 * Rows with p < 0 (context shorter than the chunk) get zeros. scale must be
 * positive and finite.
 * max_q_len: host-known upper bound on the chunk lengths (grid size).
 * head_dim: a multiple of 32 from 32 to 256 (64 and 128 have the tuned
 * kernel; the reference's SDPA takes any, nanoPD/engine/model_runner.py:166-168).
 * max_context_len: host-known upper bound on context_lens; at head dims 64
 * and 128 key ranges longer than 1024 keys are split over up to 8 workgroups
 * when it allows (<= 0: no split; other head dims never split). It sizes the
 * workspace: npd_paged_prefill_workspace_size(...) bytes,
 * 256-byte aligned, zero-filled before first use, with the same fixed 1 MiB
 * counter region as npd_paged_attention's (every call leaves its counters at
 * zero; partials follow the region), so any stream-ordered sequence of calls
 * of either op may share one workspace that is large enough for each.
 */
int npd_paged_prefill_attention(void* out, const void* query,
                                const void* key_cache, const void* value_cache,
                                const int32_t* block_tables,
                                const int32_t* cu_seqlens_q,
                                const int32_t* context_lens,
                                int64_t num_seqs, int64_t total_q,
                                int64_t num_heads, int64_t num_kv_heads,
                                int64_t head_dim, int64_t num_blocks,
                                int64_t block_size, int64_t max_blocks_per_seq,
                                int64_t max_q_len, int64_t max_context_len,
                                float scale,
                                int64_t q_stride_token, int64_t q_stride_head,
                                int64_t out_stride_token, int64_t out_stride_head,
                                void* workspace, int64_t workspace_bytes,
                                int32_t dtype, void* stream);

/*
 * npd_paged_prefill_attention over an FP8 (e4m3) pool written by
 * npd_paged_kv_store_slots_fp8 (no reference counterpart; the reference's
 * prefill, nanoPD/engine/model_runner.py:152-168, reads fp16 K/V). K and V
 * elements are e4m3(byte) * k_scale[kv head] (v_scale for V), converted
 * exactly to the query's type (fp16/bf16, dtype) before the MFMAs; arithmetic
 * and workspace as in npd_paged_prefill_attention. head_dim as there;
 * caches 8-byte aligned.
 */
int npd_paged_prefill_attention_fp8(void* out, const void* query,
                                    const void* key_cache, const void* value_cache,
                                    const int32_t* block_tables,
                                    const int32_t* cu_seqlens_q,
                                    const int32_t* context_lens,
                                    const float* k_scale, const float* v_scale,
                                    int64_t num_seqs, int64_t total_q,
                                    int64_t num_heads, int64_t num_kv_heads,
                                    int64_t head_dim, int64_t num_blocks,
                                    int64_t block_size, int64_t max_blocks_per_seq,
                                    int64_t max_q_len, int64_t max_context_len,
                                    float scale,
                                    int64_t q_stride_token, int64_t q_stride_head,
                                    int64_t out_stride_token, int64_t out_stride_head,
                                    void* workspace, int64_t workspace_bytes,
                                    int32_t dtype, void* stream);

/*
 * npd_paged_attention over an FP8 (e4m3) pool written by
 * npd_paged_kv_store_slots_fp8 (no reference counterpart). K and V elements
 * are e4m3(byte) * k_scale[kv head] (v_scale for V); query/out are fp16 or
 * bf16 (dtype), arithmetic as in npd_paged_attention. head_dim 128, block_size
 * 16 or 32, at most 4096 sequences; caches 8-byte aligned. The workspace is
 * sized by npd_paged_attention_workspace_size with the same arguments.
 */
int npd_paged_attention_fp8(void* out, const void* query,
                            const void* key_cache, const void* value_cache,
                            const int32_t* block_tables, const int32_t* seq_lens,
                            const float* k_scale, const float* v_scale,
                            int64_t num_seqs, int64_t num_heads, int64_t num_kv_heads,
                            int64_t head_dim, int64_t num_blocks, int64_t block_size,
                            int64_t max_blocks_per_seq, float scale,
                            int64_t q_stride_seq, int64_t q_stride_head,
                            int64_t out_stride_seq, int64_t out_stride_head,
                            void* workspace, int64_t workspace_bytes,
                            int32_t dtype, void* stream);

/*
 * Copy-on-write block copy (no reference counterpart: the reference returns
 * the (src, dst) pair from BlockSpaceManager.append_slot,
 * nanoPD/block_manager/block_manager.py:91-96, and never copies).
 * For each pair i: k_cache[pairs[2i+1]] = k_cache[pairs[2i]], same for v;
 * a whole block is num_kv_heads * block_size * head_dim elements.
 * Pairs with an index outside [0, num_blocks) are skipped.
 */
int npd_copy_blocks(void* k_cache, void* v_cache, const int32_t* pairs,
                    int64_t num_pairs, int64_t num_blocks,
                    int64_t block_elems, int32_t dtype, void* stream);

/*
 * Block-list pack of a multi-layer KV pool into the transfer ("wire") layout,
 * replacing the per-block copies of extract_kv_to_pinned
 * (nanoPD/workers/kv_transfer.py:45-53):
 *   wire_k[l, i, :] = k_cache[l, block_ids[i], :]   (same for v)
 * for l < num_layers, i < num_ids. Pool: [num_layers, num_blocks,
 * block_bytes] bytes per tensor (a block is num_kv_heads * block_size *
 * head_dim elements of any type); wire: [num_layers, num_ids, block_bytes].
 * An id outside [0, num_blocks) gives zero bytes in the wire.
 * block_bytes a multiple of 16, 16-byte aligned pointers.
 */
int npd_kv_gather_blocks(const void* k_cache, const void* v_cache, int64_t num_layers,
                         int64_t num_blocks, int64_t block_bytes,
                         const int32_t* block_ids, int64_t num_ids,
                         void* wire_k, void* wire_v, void* stream);

/*
 * The inverse, replacing load_kv_from_pinned (kv_transfer.py:56-69):
 *   k_cache[l, block_ids[i], :] = wire_k[l, i, :]   (same for v).
 * Ids outside [0, num_blocks) are skipped. Same layouts and limits as
 * npd_kv_gather_blocks.
 */
int npd_kv_scatter_blocks(void* k_cache, void* v_cache, int64_t num_layers,
                          int64_t num_blocks, int64_t block_bytes,
                          const int32_t* block_ids, int64_t num_ids,
                          const void* wire_k, const void* wire_v, void* stream);

/*
 * Fused attention prologue of a Qwen3-, Qwen2- or Llama-style layer (replaces
 * the per-layer q_norm / k_norm, rotary embedding, K/V transpose copies and
 * paged_kv_store calls of nanoPD/engine/model_runner.py:97-115, :142-146,
 * :189-192).
 * qkv: [num_tokens, (num_heads + 2 num_kv_heads) * head_dim] token rows
 * (q heads, then k heads, then v heads) with token stride qkv_stride_token
 * elements -- the fused QKV projection output as it is.
 * For each token t, at position positions[t]:
 *   q_out[t, h, :]        = rope(rmsnorm(q[t, h, :], q_norm_weight))
 *   k_cache[slot, kh, :]  = rope(rmsnorm(k[t, kh, :], k_norm_weight))
 *   v_cache[slot, kh, :]  = v[t, kh, :]
 * with slot = slot_mapping[t] (block * block_size + offset, pool layout
 * [num_blocks, num_kv_heads, block_size, head_dim]); tokens whose slot is
 * negative or outside the pool are not stored (q_out is still written).
 * rmsnorm(x, w) = half(half(x * rsqrt(mean(x^2) + eps)) * w) as HF
 * Qwen3RMSNorm; with both norm weights NULL (layers without q / k norms,
 * which the reference skips, model_runner.py:101-104) rmsnorm(x, .) = x.
 * rope is rotate-half with angle positions[t] * inv_freq[i]
 * (inv_freq: fp32 [head_dim / 2]), computed in fp32 and rounded once.
 * q_out token stride is q_stride_token elements (heads contiguous).
 * head_dim 64, 128 or 256; dtype fp16 or bf16 for every 2-byte tensor.
 */
int npd_qk_norm_rope_store(void* q_out, void* k_cache, void* v_cache,
                           const void* qkv, const int32_t* slot_mapping,
                           const int32_t* positions, const float* inv_freq,
                           const void* q_norm_weight, const void* k_norm_weight,
                           int64_t num_tokens, int64_t num_heads,
                           int64_t num_kv_heads, int64_t head_dim,
                           int64_t num_blocks, int64_t block_size,
                           int64_t qkv_stride_token, int64_t q_stride_token,
                           float eps, int32_t dtype, void* stream);

/*
 * npd_qk_norm_rope_store into an FP8 (e4m3) pool (no reference counterpart;
 * the reference's caches are fp16, nanoPD/engine/model_runner.py:24-31):
 * q_out as above; the rotated k and the raw v, rounded to dtype as above, are
 * stored as the e4m3 bytes of value / k_scale[kv head] (v_scale for v) with
 * the rounding of npd_paged_kv_store_slots_fp8, so both paths write the same
 * bytes. Caches are [num_blocks, num_kv_heads, block_size, head_dim] bytes.
 */
int npd_qk_norm_rope_store_fp8(void* q_out, void* k_cache, void* v_cache,
                               const void* qkv, const int32_t* slot_mapping,
                               const int32_t* positions, const float* inv_freq,
                               const void* q_norm_weight, const void* k_norm_weight,
                               const float* k_scale, const float* v_scale,
                               int64_t num_tokens, int64_t num_heads,
                               int64_t num_kv_heads, int64_t head_dim,
                               int64_t num_blocks, int64_t block_size,
                               int64_t qkv_stride_token, int64_t q_stride_token,
                               float eps, int32_t dtype, void* stream);

/*
 * Ragged-batch metadata packing on the GPU (no reference counterpart: the
 * reference re-tensorises its context dict per layer with host loops,
 * nanoPD/engine/model_runner.py:129-187, from nanoPD/engine/engine.py:45-90).
 * Input, one compact upload: seq_desc[s] = {q_len, ctx_before, table_len} for
 * s < num_seqs (prefill chunks and decodes alike, in batch order) and the
 * concatenation of every sequence's block table, table_len entries each.
 * Outputs (device, caller-allocated):
 *   cu_seqlens_q[num_seqs+1]  prefix sums of q_len
 *   seq_lens[num_seqs]        ctx_before + q_len (context after the step)
 *   block_tables[num_seqs, max_blocks_per_seq]  zero-padded rows
 *   positions[total_q]        ctx_before + i for the i-th new token
 *   slot_mapping[total_q]     table[pos / block_size] * block_size + pos % block_size,
 *                             or -1 when pos / block_size >= table_len
 *   token_seq[total_q]        owning sequence of each token
 * total_q must equal the sum of q_len (checked by the kernel: entries past
 * the true total are left untouched). num_seqs <= 4096.
 */
int npd_pack_metadata(const int32_t* seq_desc, const int32_t* flat_tables,
                      int64_t num_seqs, int64_t total_q, int64_t flat_len,
                      int64_t max_blocks_per_seq, int64_t block_size,
                      int32_t* cu_seqlens_q, int32_t* seq_lens,
                      int32_t* block_tables, int32_t* positions,
                      int32_t* slot_mapping, int32_t* token_seq,
                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NANOPD_H */
