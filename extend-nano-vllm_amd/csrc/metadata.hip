// Verify-batch metadata on the device: the per-token loops of the
// reference's prepare_prefill (nanovllm/engine/model_runner.py:761-800)
// derived from per-sequence (first position, query length) and the block
// tables, so a step uploads O(sequences) values instead of O(tokens).
//
// One workgroup: the sequence prefix sums are a block-wide scan in LDS, then
// every thread derives the positions and slots of a strided set of tokens
// (sequence found by binary search over the scanned offsets).  The work is
// a few thousand integers; the point is removing host work, not bandwidth.
//
// The commit form derives the same metadata for the draft's replay of the
// committed tails (model_runner.py:1216-1249, the per-token contexts of
// :1127-1156): sequence i commits accept_len[i] + 1 rows (its accepted
// drafts, then the bonus token) taken from its verify rows i * q_stride ..,
// so the query lengths come from the accept scan's output on the device,
// and each commit row also gets its verify row, its token (the verify
// argmax of that row, which an accepted draft equals) and each sequence its
// last commit row, whose draft states seed the next proposal.
//
// Draft slot convention.  The draft forms (commit and draft steps) take a
// slot offset: the K/V of RoPE position p goes to the slot of position
// p + slot_offset, and that row sees p + slot_offset + 1 keys.  Offset 0
// stores position p at slot p, as the reference's draft prefill does
// (model_runner.py:1379-1390); offset 1 is the reference's decode and
// commit convention (slot len + step, context len + step + 1,
// model_runner.py:1087-1096; slot start + 1 + i, context start + 2 + i,
// :1143-1149).
#include "common.h"

namespace nva {
namespace {

constexpr int kMetaThreads = 256;
constexpr int kMaxMetaSeqs = 2048;

// inclusive block scan of one value per thread (kMetaThreads values)
__device__ int block_scan(int v, int* sh) {
  const int tid = threadIdx.x;
  sh[tid] = v;
  __syncthreads();
  for (int d = 1; d < kMetaThreads; d <<= 1) {
    const int u = tid >= d ? sh[tid - d] : 0;
    __syncthreads();
    sh[tid] += u;
    __syncthreads();
  }
  const int r = sh[tid];
  __syncthreads();
  return r;
}

// Commit-form inputs and outputs (unused by the verify form).
struct CommitArgs {
  int32_t q_stride;                 // verify rows per sequence
  const int32_t* verify_argmax;     // [num_verify_rows]
  int32_t num_verify_rows;
  int32_t* verify_rows;             // [num_tokens]
  int64_t* token_ids;               // [num_tokens]
  int64_t* last_rows;               // [num_seqs]
};

// COMMIT: q_lens holds accept lengths; sequence i has min(max(a_i, 0) + 1,
// q_stride) rows.
template <bool COMMIT>
__global__ void __launch_bounds__(kMetaThreads)
verify_metadata_kernel(const int32_t* __restrict__ start_pos, const int32_t* __restrict__ q_lens,
                       int32_t num_seqs, const int32_t* __restrict__ block_tables,
                       int64_t bt_stride, int32_t max_blocks, int32_t block_size,
                       int32_t slot_offset, int32_t* __restrict__ cu_q_out,
                       int32_t* __restrict__ cu_k_out, int64_t* __restrict__ positions,
                       int32_t* __restrict__ slots, int32_t num_tokens, CommitArgs ca) {
  __shared__ int cu_q[kMaxMetaSeqs + 1];
  __shared__ int cu_k[kMaxMetaSeqs + 1];
  __shared__ int scan[kMetaThreads];
  const int tid = threadIdx.x;
  if (tid == 0) {
    cu_q[0] = 0;
    cu_k[0] = 0;
  }
  // every thread reads cu_q[0] below, also when there is no sequence (and
  // so no barrier inside the scan loop)
  __syncthreads();
  int carry_q = 0, carry_k = 0;
  for (int base = 0; base < num_seqs; base += kMetaThreads) {
    const int i = base + tid;
    int q = i < num_seqs ? q_lens[i] : 0;
    if (COMMIT && i < num_seqs) {
      q = (q < 0 ? 0 : q) + 1;
      q = q < ca.q_stride ? q : ca.q_stride;
    }
    const int k = i < num_seqs ? start_pos[i] + q + slot_offset : 0;
    const int iq = block_scan(q, scan) + carry_q;
    const int ik = block_scan(k, scan) + carry_k;
    if (i < num_seqs) {
      cu_q[i + 1] = iq;
      cu_k[i + 1] = ik;
    }
    __syncthreads();
    const int last = (num_seqs - base < kMetaThreads ? num_seqs - base : kMetaThreads);
    carry_q = cu_q[base + last];
    carry_k = cu_k[base + last];
    __syncthreads();
  }
  for (int i = tid; i <= num_seqs; i += kMetaThreads) {
    cu_q_out[i] = cu_q[i];
    cu_k_out[i] = cu_k[i];
    if (COMMIT && i < num_seqs) ca.last_rows[i] = static_cast<int64_t>(cu_q[i + 1]) - 1;
  }
  const int total = cu_q[num_seqs];
  for (int t = tid; t < num_tokens; t += kMetaThreads) {
    int64_t pos = 0;
    int32_t slot = -1;
    int32_t vrow = -1;
    if (t < total) {
      // sequence s with cu_q[s] <= t < cu_q[s + 1] (empty sequences skipped)
      int lo = 0, hi = num_seqs;
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (cu_q[mid] <= t) lo = mid; else hi = mid;
      }
      const int p = start_pos[lo] + (t - cu_q[lo]);
      pos = p;
      const int ps = p + slot_offset;      // the position whose slot holds p's K/V
      const int b = ps / block_size;
      if (ps >= 0 && b < max_blocks) {
        const int32_t id = block_tables[static_cast<int64_t>(lo) * bt_stride + b];
        if (id >= 0) slot = id * block_size + ps % block_size;
      }
      if (COMMIT) vrow = lo * ca.q_stride + (t - cu_q[lo]);
    }
    positions[t] = pos;
    slots[t] = slot;
    if (COMMIT) {
      // rows past the committed ones read verify row 0 (never attended)
      const int32_t src = vrow >= 0 && vrow < ca.num_verify_rows ? vrow : 0;
      ca.verify_rows[t] = vrow;
      ca.token_ids[t] = ca.num_verify_rows > 0 ? ca.verify_argmax[src] : 0;
    }
  }
}

}  // namespace
}  // namespace nva

using namespace nva;

extern "C" int nva_verify_metadata(const int32_t* start_pos, const int32_t* q_lens,
                                   int32_t num_seqs, const int32_t* block_tables,
                                   int64_t block_table_stride, int32_t max_blocks_per_seq,
                                   int32_t block_size, int32_t* cu_seqlens_q,
                                   int32_t* cu_seqlens_k, int64_t* positions,
                                   int32_t* slot_mapping, int32_t num_tokens, void* stream) {
  if (num_seqs < 0 || num_tokens < 0 || block_size <= 0 || max_blocks_per_seq < 0) return NVA_ERR_ARG;
  if (num_seqs > kMaxMetaSeqs) return NVA_ERR_UNSUPPORTED;
  if (block_table_stride < max_blocks_per_seq) return NVA_ERR_ARG;
  if (!cu_seqlens_q || !cu_seqlens_k || (num_tokens > 0 && (!positions || !slot_mapping)))
    return NVA_ERR_ARG;
  if (num_seqs > 0 && (!start_pos || !q_lens || (max_blocks_per_seq > 0 && !block_tables)))
    return NVA_ERR_ARG;
  verify_metadata_kernel<false><<<1, kMetaThreads, 0, static_cast<hipStream_t>(stream)>>>(
      start_pos, q_lens, num_seqs, block_tables, block_table_stride, max_blocks_per_seq, block_size,
      0, cu_seqlens_q, cu_seqlens_k, positions, slot_mapping, num_tokens, CommitArgs{});
  return launch_status();
}

extern "C" int nva_commit_metadata(const int32_t* start_pos, const int32_t* accept_len,
                                   int32_t num_seqs, int32_t q_stride,
                                   const int32_t* verify_argmax, int32_t num_verify_rows,
                                   const int32_t* block_tables, int64_t block_table_stride,
                                   int32_t max_blocks_per_seq, int32_t block_size,
                                   int32_t slot_offset, int32_t* cu_seqlens_q,
                                   int32_t* cu_seqlens_k, int64_t* positions,
                                   int32_t* slot_mapping, int32_t* verify_rows, int64_t* token_ids,
                                   int64_t* last_rows, int32_t num_tokens, void* stream) {
  if (num_seqs < 0 || num_tokens < 0 || block_size <= 0 || max_blocks_per_seq < 0 ||
      q_stride <= 0 || num_verify_rows < 0 || (slot_offset != 0 && slot_offset != 1))
    return NVA_ERR_ARG;
  if (num_seqs > kMaxMetaSeqs) return NVA_ERR_UNSUPPORTED;
  if (block_table_stride < max_blocks_per_seq) return NVA_ERR_ARG;
  if (!cu_seqlens_q || !cu_seqlens_k) return NVA_ERR_ARG;
  if (num_tokens > 0 && (!positions || !slot_mapping || !verify_rows || !token_ids))
    return NVA_ERR_ARG;
  if (num_tokens > 0 && num_verify_rows > 0 && !verify_argmax) return NVA_ERR_ARG;
  if (num_seqs > 0 && (!start_pos || !accept_len || !last_rows ||
                       (max_blocks_per_seq > 0 && !block_tables)))
    return NVA_ERR_ARG;
  const CommitArgs ca{q_stride, verify_argmax, num_verify_rows, verify_rows, token_ids, last_rows};
  verify_metadata_kernel<true><<<1, kMetaThreads, 0, static_cast<hipStream_t>(stream)>>>(
      start_pos, accept_len, num_seqs, block_tables, block_table_stride, max_blocks_per_seq,
      block_size, slot_offset, cu_seqlens_q, cu_seqlens_k, positions, slot_mapping, num_tokens, ca);
  return launch_status();
}

// Draft-step metadata for a draft queued right behind a verify: column i of
// bs (i < num_seqs a sequence, the rest padding), row s of steps.  One
// thread per (s, i); each reads its sequence's accepted count from the
// verify's accept output, so the draft's lengths follow the verified step
// without the host.  Step s of a sequence of length L is at RoPE position
// p = L - 1 + s; its K/V go to the slot of position p + slot_offset and it
// sees p + slot_offset + 1 keys.
__global__ void __launch_bounds__(kMetaThreads)
draft_metadata_kernel(const int64_t* __restrict__ lens, const int64_t* __restrict__ verify_row,
                      const int32_t* __restrict__ accept_len, int32_t num_seqs, int32_t bs,
                      int32_t steps, const int32_t* __restrict__ block_tables,
                      int64_t bt_stride, int32_t max_blocks, int32_t block_size,
                      int32_t slot_offset, int64_t* __restrict__ positions,
                      int32_t* __restrict__ slot_mapping, int32_t* __restrict__ context_lens) {
  const int idx = blockIdx.x * kMetaThreads + threadIdx.x;
  if (idx >= steps * bs) return;
  const int s = idx / bs, i = idx % bs;
  int64_t pos = 0;
  int32_t slot = -1;
  int32_t keys = 1;
  if (i < num_seqs) {
    const int64_t len = lens[i] + accept_len[verify_row[i]] + 1;
    pos = len - 1 + s;
    const int64_t ps = pos + slot_offset;   // the position whose slot holds pos's K/V
    const int64_t blk = ps / block_size;
    const int32_t id = ps >= 0 && blk < max_blocks
                           ? block_tables[static_cast<int64_t>(i) * bt_stride + blk] : -1;
    if (id >= 0) slot = static_cast<int32_t>(static_cast<int64_t>(id) * block_size + ps % block_size);
    keys = static_cast<int32_t>(ps + 1);
  }
  positions[idx] = pos;
  slot_mapping[idx] = slot;
  context_lens[idx] = keys;
}

extern "C" int nva_draft_metadata(const int64_t* lens, const int64_t* verify_row,
                                  const int32_t* accept_len, int32_t num_seqs, int32_t bs,
                                  int32_t steps, const int32_t* block_tables,
                                  int64_t block_table_stride, int32_t max_blocks_per_seq,
                                  int32_t block_size, int32_t slot_offset, int64_t* positions,
                                  int32_t* slot_mapping, int32_t* context_lens, void* stream) {
  if (num_seqs < 0 || bs < num_seqs || steps < 0 || block_size <= 0 || max_blocks_per_seq < 0 ||
      block_table_stride < max_blocks_per_seq || (slot_offset != 0 && slot_offset != 1))
    return NVA_ERR_ARG;
  if (steps == 0 || bs == 0) return NVA_OK;
  if (!positions || !slot_mapping || !context_lens) return NVA_ERR_ARG;
  if (num_seqs > 0 && (!lens || !verify_row || !accept_len ||
                       (max_blocks_per_seq > 0 && !block_tables)))
    return NVA_ERR_ARG;
  const int n = steps * bs;
  draft_metadata_kernel<<<(n + kMetaThreads - 1) / kMetaThreads, kMetaThreads, 0,
                          static_cast<hipStream_t>(stream)>>>(
      lens, verify_row, accept_len, num_seqs, bs, steps, block_tables, block_table_stride,
      max_blocks_per_seq, block_size, slot_offset, positions, slot_mapping, context_lens);
  return launch_status();
}

// ---------------------------------------------------------------- verify input ids

// One thread per verify row t = p * q + j: row 0 of each sequence is its last
// committed token, rows 1..q-1 its proposals, read from the draft's output
// [q-1][proposal_stride] at the sequence's column order[p]; a column outside
// [0, proposal_stride) marks padding (ids 0), so no read leaves the output.
// compose[0] == 0 leaves ids as they are (the host wrote them), so one
// captured graph serves both callers.
__global__ void __launch_bounds__(kMetaThreads)
verify_input_ids_kernel(const int32_t* __restrict__ compose, const int32_t* __restrict__ last_tokens,
                        const int32_t* __restrict__ order, const int64_t* __restrict__ proposals,
                        int64_t proposal_stride, int32_t num_rows, int32_t q,
                        int64_t* __restrict__ ids) {
  const int t = blockIdx.x * kMetaThreads + threadIdx.x;
  if (t >= num_rows * q || compose[0] == 0) return;
  const int p = t / q, j = t % q;
  const int32_t col = order[p];
  int64_t id = 0;
  if (col >= 0 && col < proposal_stride)
    id = j == 0 ? static_cast<int64_t>(last_tokens[p]) : proposals[(j - 1) * proposal_stride + col];
  ids[t] = id;
}

extern "C" int nva_verify_input_ids(const int32_t* compose, const int32_t* last_tokens,
                                    const int32_t* order, const int64_t* proposals,
                                    int64_t proposal_stride, int32_t num_rows, int32_t q,
                                    int64_t* ids, void* stream) {
  if (num_rows < 0 || q < 1 || proposal_stride < 1) return NVA_ERR_ARG;
  if (num_rows == 0) return NVA_OK;
  if (!compose || !last_tokens || !order || !ids || (q > 1 && !proposals)) return NVA_ERR_ARG;
  if (static_cast<int64_t>(num_rows) * q > INT32_MAX) return NVA_ERR_ARG;
  const int n = num_rows * q;
  verify_input_ids_kernel<<<(n + kMetaThreads - 1) / kMetaThreads, kMetaThreads, 0,
                            static_cast<hipStream_t>(stream)>>>(
      compose, last_tokens, order, proposals, proposal_stride, num_rows, q, ids);
  return launch_status();
}
