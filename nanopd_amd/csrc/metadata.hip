// Ragged-batch metadata packing on the GPU.
//
// The reference builds this per attention layer from a Python dict with host
// loops and one host-to-device copy per sequence (nanoPD/engine/model_runner.py:
// 129-150 for prefills, :177-187 for decodes; the dict comes from
// nanoPD/engine/engine.py:45-90). Here the host uploads one compact int32
// buffer per step and a single workgroup expands it:
//   pass A: prefix sums of q_len (cu_seqlens_q) and of table_len (offsets into
//           the flat tables) with a workgroup scan, kept in LDS;
//   pass B: every thread fills table rows and per-token entries; a token finds
//           its sequence by binary search over cu_seqlens_q in LDS.
// Positions follow the reference: a chunk of n tokens starting at ctx_before
// gets positions ctx_before .. ctx_before+n-1 (model_runner.py:133-137), a
// decode token gets position ctx_before (engine.py:55-60), seq_lens is the
// position after the last new token (model_runner.py:183), and the slot is
// table[pos / bs] * bs + pos % bs (paged_kv_store_kernel.cu:45-51).
#include "common.h"

namespace {

constexpr int kThreads = 1024;
constexpr int kMaxSeqs = 4096;

__global__ __launch_bounds__(kThreads) void pack_metadata_kernel(
    const int32_t* __restrict__ desc, const int32_t* __restrict__ flat, int num_seqs,
    int total_q, int64_t flat_len, int max_bps, int bs, int32_t* __restrict__ cu_seqlens,
    int32_t* __restrict__ seq_lens, int32_t* __restrict__ tables, int32_t* __restrict__ positions,
    int32_t* __restrict__ slots, int32_t* __restrict__ token_seq) {
  __shared__ int s_cu[kMaxSeqs + 1];
  __shared__ int s_toff[kMaxSeqs + 1];
  __shared__ int s_wsum[2][kThreads / 64];
  __shared__ int s_carry[2];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  if (tid == 0) { s_carry[0] = 0; s_carry[1] = 0; }
  __syncthreads();
  // pass A: chunked exclusive scans of q_len and table_len
  for (int base = 0; base < num_seqs; base += kThreads) {
    const int s = base + tid;
    int ql = 0, tl = 0;
    if (s < num_seqs) {
      ql = desc[3 * s] > 0 ? desc[3 * s] : 0;
      tl = desc[3 * s + 2] > 0 ? desc[3 * s + 2] : 0;
    }
    int iq = ql, it = tl;  // inclusive wave scans
    for (int o = 1; o < 64; o <<= 1) {
      const int a = __shfl_up(iq, o, 64), b = __shfl_up(it, o, 64);
      if (lane >= o) { iq += a; it += b; }
    }
    if (lane == 63) { s_wsum[0][wid] = iq; s_wsum[1][wid] = it; }
    __syncthreads();
    int pq = s_carry[0], pt = s_carry[1];
    for (int w = 0; w < wid; ++w) { pq += s_wsum[0][w]; pt += s_wsum[1][w]; }
    if (s < num_seqs) {
      s_cu[s] = pq + iq - ql;
      s_toff[s] = pt + it - tl;
    }
    __syncthreads();
    if (tid == kThreads - 1) { s_carry[0] = pq + iq; s_carry[1] = pt + it; }
    __syncthreads();
  }
  if (tid == 0) { s_cu[num_seqs] = s_carry[0]; s_toff[num_seqs] = s_carry[1]; }
  __syncthreads();

  // pass B1: per-sequence outputs and padded tables
  for (int s = tid; s <= num_seqs; s += kThreads) cu_seqlens[s] = s_cu[s];
  for (int s = tid; s < num_seqs; s += kThreads) {
    const int ql = desc[3 * s] > 0 ? desc[3 * s] : 0;
    seq_lens[s] = desc[3 * s + 1] + ql;
  }
  const int64_t nt = (int64_t)num_seqs * max_bps;
  for (int64_t e = tid; e < nt; e += kThreads) {
    const int s = (int)(e / max_bps), b = (int)(e - (int64_t)s * max_bps);
    const int tl = s_toff[s + 1] - s_toff[s];
    const int64_t src = (int64_t)s_toff[s] + b;
    tables[e] = (b < tl && src < flat_len) ? flat[src] : 0;
  }
  // pass B2: per-token outputs
  const int nq = s_cu[num_seqs] < total_q ? s_cu[num_seqs] : total_q;
  for (int t = tid; t < nq; t += kThreads) {
    int lo = 0, hi = num_seqs - 1;  // last s with s_cu[s] <= t
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_cu[mid] <= t) lo = mid; else hi = mid - 1;
    }
    const int s = lo;
    const int pos = desc[3 * s + 1] + (t - s_cu[s]);
    const int tl = s_toff[s + 1] - s_toff[s];
    const int lb = pos >= 0 ? pos / bs : -1;
    int slot = -1;
    if (lb >= 0 && lb < tl && (int64_t)s_toff[s] + lb < flat_len)
      slot = flat[s_toff[s] + lb] * bs + (pos - lb * bs);
    positions[t] = pos;
    slots[t] = slot;
    token_seq[t] = s;
  }
}

}  // namespace

extern "C" int npd_pack_metadata(const int32_t* seq_desc, const int32_t* flat_tables,
                                 int64_t num_seqs, int64_t total_q, int64_t flat_len,
                                 int64_t max_blocks_per_seq, int64_t block_size,
                                 int32_t* cu_seqlens_q, int32_t* seq_lens, int32_t* block_tables,
                                 int32_t* positions, int32_t* slot_mapping, int32_t* token_seq,
                                 void* stream) {
  using namespace npd;
  const char* name = "npd_pack_metadata";
  if (num_seqs < 0 || num_seqs > kMaxSeqs)
    return fail(NPD_E_INVALID, "%s: num_seqs %lld outside [0, %d]", name, (long long)num_seqs,
                kMaxSeqs);
  if (total_q < 0 || total_q > INT32_MAX || flat_len < 0 || max_blocks_per_seq <= 0 ||
      block_size <= 0 || num_seqs * max_blocks_per_seq > INT32_MAX)
    return fail(NPD_E_INVALID, "%s: bad sizes (total_q %lld, flat %lld, max blocks %lld, block %lld)",
                name, (long long)total_q, (long long)flat_len, (long long)max_blocks_per_seq,
                (long long)block_size);
  if (num_seqs == 0 && total_q != 0)
    return fail(NPD_E_INVALID, "%s: tokens without sequences", name);
  if (!seq_desc || !cu_seqlens_q || (num_seqs > 0 && (!seq_lens || !block_tables)) ||
      (total_q > 0 && (!positions || !slot_mapping || !token_seq)) || (flat_len > 0 && !flat_tables))
    return fail(NPD_E_INVALID, "%s: null pointer", name);
  hipLaunchKernelGGL(pack_metadata_kernel, dim3(1), dim3(kThreads), 0, as_stream(stream), seq_desc,
                     flat_tables, (int)num_seqs, (int)total_q, flat_len, (int)max_blocks_per_seq,
                     (int)block_size, cu_seqlens_q, seq_lens, block_tables, positions, slot_mapping,
                     token_seq);
  return check_launch(name);
}
