// K4: vocab argmax fused with the greedy accepted-prefix / bonus scan.
//
// Grid (chunks_per_row, rows), 256 threads.  Each block scans one vocab chunk
// of one row with 16-byte loads and reduces (value, index) pairs packed into
// one 64-bit key:
//     key = ord16(value) << 32 | (0xFFFFFFFF - index)
// where ord16 maps bf16 bit patterns to unsigned integers in numeric order
// (-0 folded onto +0, every NaN above +inf).  The maximum key is then the
// first index of the maximum, with NaN as the maximum -- torch.argmax's rule.
// The last block of a row (device-scope counter) merges the chunk keys; the
// last row of a sequence (second counter) runs the accept scan.  Both counters
// reset themselves and the merged partials are cleared, so the workspace is
// zero-filled again after every call, whatever its shape, and the kernel is
// safe to replay from a HIP graph.
#include "common.h"

namespace nva {
namespace {

constexpr int kThreads = 256;
constexpr int kTargetBlocks = 2048;   // ~8 blocks per CU on 256 CUs
constexpr int kMinChunk = 4096;       // elements; two 16-byte loads per thread

__device__ __forceinline__ uint64_t make_key(uint32_t b, uint32_t idx) {
  const uint32_t mag = b & 0x7FFFu;
  uint32_t ord;
  if (mag > 0x7F80u)
    ord = 0xFFFFu;
  else if (mag == 0)
    ord = 0x8000u;
  else
    ord = (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
  return (static_cast<uint64_t>(ord) << 32) | (0xFFFFFFFFu - idx);
}

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), m, kWave);
  const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), m, kWave);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

__device__ __forceinline__ uint64_t block_max(uint64_t v, uint64_t* red) {
#pragma unroll
  for (int m = kWave / 2; m >= 1; m >>= 1) v = umax64(v, shfl_xor64(v, m));
  const int w = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) red[w] = v;
  __syncthreads();
  uint64_t r = red[0];
#pragma unroll
  for (int i = 1; i < kThreads / kWave; ++i) r = umax64(r, red[i]);
  __syncthreads();
  return r;
}

__device__ __forceinline__ uint64_t scan_vec(uint4 w, uint32_t base, uint64_t best) {
  const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t b = (d[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
    best = umax64(best, make_key(b, base + e));
  }
  return best;
}

template <bool ACCEPT, bool OUT64>
__global__ void __launch_bounds__(kThreads)
argmax_kernel(const uint16_t* __restrict__ logits, int64_t row_stride, int32_t vocab,
              int32_t chunk_elems, int32_t chunks, int32_t num_rows, bool vec,
              const int32_t* __restrict__ cu_q, int32_t num_seqs,
              const int64_t* __restrict__ input_ids, const int64_t* __restrict__ index_map,
              int32_t* __restrict__ argmax32, int64_t* __restrict__ out64,
              int32_t* __restrict__ accept_len, int32_t* __restrict__ bonus,
              uint64_t* __restrict__ partials, uint32_t* __restrict__ row_cnt,
              uint32_t* __restrict__ seq_cnt) {
  __shared__ uint64_t red[kThreads / kWave];
  __shared__ int flag;
  const int32_t row = blockIdx.y;
  const int32_t chunk = blockIdx.x;

  if (ACCEPT && row == 0 && chunk == 0) {
    for (int32_t s = threadIdx.x; s < num_seqs; s += kThreads) {
      if (cu_q[s + 1] - cu_q[s] <= 0) {
        accept_len[s] = 0;
        bonus[s] = -1;
      }
    }
  }

  const int32_t begin = chunk * chunk_elems;
  int32_t end = begin + chunk_elems;
  end = end > vocab ? vocab : end;
  const uint16_t* rp = logits + static_cast<int64_t>(row) * row_stride;
  uint64_t best = 0;
  if (vec) {
    const int32_t nvec = (end - begin) / 8;
    const uint4* vp = reinterpret_cast<const uint4*>(rp + begin);
#pragma unroll 4
    for (int32_t v = threadIdx.x; v < nvec; v += kThreads)
      best = scan_vec(vp[v], static_cast<uint32_t>(begin + v * 8), best);
    for (int32_t c = begin + nvec * 8 + threadIdx.x; c < end; c += kThreads)
      best = umax64(best, make_key(rp[c], static_cast<uint32_t>(c)));
  } else {
    for (int32_t c = begin + threadIdx.x; c < end; c += kThreads)
      best = umax64(best, make_key(rp[c], static_cast<uint32_t>(c)));
  }
  uint64_t key = block_max(best, red);

  if (chunks > 1) {
    if (threadIdx.x == 0) {
      store_relaxed_agent(partials + static_cast<int64_t>(row) * chunks + chunk, key);
      __threadfence();
      const uint32_t old = atomicAdd(row_cnt + row, 1u);
      flag = (old == static_cast<uint32_t>(chunks - 1));
    }
    __syncthreads();
    if (!flag) return;
    __threadfence();
    uint64_t k = 0;
    for (int32_t c = threadIdx.x; c < chunks; c += kThreads) {
      uint64_t* slot = partials + static_cast<int64_t>(row) * chunks + c;
      k = umax64(k, load_relaxed_agent(slot));
      // leave the whole workspace zero-filled: a later call with another
      // shape may place its counters where these partials were
      store_relaxed_agent(slot, static_cast<uint64_t>(0));
    }
    key = block_max(k, red);
    if (threadIdx.x == 0) store_relaxed_agent(row_cnt + row, 0u);
  }
  if (threadIdx.x != 0) return;

  const uint32_t idx = 0xFFFFFFFFu - static_cast<uint32_t>(key);
  if constexpr (OUT64) {
    out64[row] = static_cast<int64_t>(idx) + (index_map ? index_map[idx] : 0);
  } else {
    argmax32[row] = static_cast<int32_t>(idx);
  }
  if constexpr (ACCEPT) {
    // sequence owning this row: largest s with cu_q[s] <= row
    int32_t lo = 0, hi = num_seqs;  // invariant: cu_q[lo] <= row < cu_q[hi]
    if (row < cu_q[0] || row >= cu_q[num_seqs]) return;
    while (hi - lo > 1) {
      const int32_t mid = (lo + hi) >> 1;
      if (cu_q[mid] <= row) lo = mid; else hi = mid;
    }
    const int32_t s = lo;
    const int32_t start = cu_q[s];
    const int32_t stop = cu_q[s + 1] < num_rows ? cu_q[s + 1] : num_rows;
    const int32_t q = stop - start;
    __threadfence();
    const uint32_t old = atomicAdd(seq_cnt + s, 1u);
    if (old != static_cast<uint32_t>(q - 1)) return;
    store_relaxed_agent(seq_cnt + s, 0u);
    __threadfence();
    int32_t a = 0;
    int32_t target = load_acquire_agent(argmax32 + start);
    while (a < q - 1 && input_ids[start + 1 + a] == static_cast<int64_t>(target)) {
      ++a;
      target = load_acquire_agent(argmax32 + start + a);
    }
    accept_len[s] = a;
    bonus[s] = target;
  }
}

void choose_chunks(int32_t rows, int32_t vocab, int32_t* chunk_elems, int32_t* chunks) {
  const int32_t rows1 = rows > 0 ? rows : 1;
  int32_t by_target = (kTargetBlocks + rows1 - 1) / rows1;
  int32_t by_size = (vocab + kMinChunk - 1) / kMinChunk;
  if (by_size < 1) by_size = 1;
  int32_t c = by_target < by_size ? by_target : by_size;
  if (c < 1) c = 1;
  int32_t ce = (vocab + c - 1) / c;
  ce = (ce + 8 * kThreads - 1) / (8 * kThreads) * (8 * kThreads);
  *chunk_elems = ce;
  *chunks = (vocab + ce - 1) / ce;
}

size_t workspace_bytes(int32_t rows, int32_t seqs, int32_t vocab) {
  int32_t ce, c;
  choose_chunks(rows, vocab, &ce, &c);
  size_t partial = c > 1 ? static_cast<size_t>(rows) * c * sizeof(uint64_t) : 0;
  return partial + static_cast<size_t>(rows) * 4 + static_cast<size_t>(seqs) * 4 + 16;
}

template <bool ACCEPT, bool OUT64>
int launch(const void* logits, int64_t row_stride, int32_t vocab, int32_t rows,
           const int32_t* cu_q, int32_t seqs, const int64_t* input_ids,
           const int64_t* index_map, int32_t* argmax32, int64_t* out64, int32_t* accept_len,
           int32_t* bonus, void* ws, size_t ws_bytes, hipStream_t stream) {
  int32_t ce, c;
  choose_chunks(rows, vocab, &ce, &c);
  if (ws_bytes < workspace_bytes(rows, seqs, vocab) || (!ws && c > 1)) return NVA_ERR_WORKSPACE;
  if (ACCEPT && !ws) return NVA_ERR_WORKSPACE;
  char* p = static_cast<char*>(ws);
  uint64_t* partials = reinterpret_cast<uint64_t*>(p);
  size_t off = c > 1 ? static_cast<size_t>(rows) * c * sizeof(uint64_t) : 0;
  uint32_t* row_cnt = reinterpret_cast<uint32_t*>(p + off);
  uint32_t* seq_cnt = reinterpret_cast<uint32_t*>(p + off + static_cast<size_t>(rows) * 4);
  const bool vec = aligned16(logits) && (row_stride % 8 == 0);
  dim3 grid(c, rows);
  argmax_kernel<ACCEPT, OUT64><<<grid, kThreads, 0, stream>>>(
      static_cast<const uint16_t*>(logits), row_stride, vocab, ce, c, rows, vec, cu_q, seqs,
      input_ids, index_map, argmax32, out64, accept_len, bonus, partials, row_cnt, seq_cnt);
  return launch_status();
}

}  // namespace
}  // namespace nva

using namespace nva;

extern "C" size_t nva_argmax_workspace_size(int32_t num_rows, int32_t num_seqs, int32_t vocab) {
  if (num_rows < 0 || num_seqs < 0 || vocab <= 0) return 0;
  return workspace_bytes(num_rows, num_seqs, vocab);
}

extern "C" int nva_argmax_accept(const void* logits, int64_t row_stride, int32_t vocab,
                                 const int32_t* cu_seqlens_q, int32_t num_seqs,
                                 int32_t num_tokens, const int64_t* input_ids, int32_t* argmax,
                                 int32_t* accept_len, int32_t* bonus, void* workspace,
                                 size_t workspace_bytes_, void* stream) {
  if (vocab <= 0 || num_seqs < 0 || num_tokens < 0 || row_stride < vocab) return NVA_ERR_ARG;
  if (num_seqs == 0 && num_tokens == 0) return NVA_OK;
  if (!cu_seqlens_q || !accept_len || !bonus || (num_tokens > 0 && (!logits || !input_ids || !argmax)))
    return NVA_ERR_ARG;
  if (num_tokens == 0) return NVA_ERR_ARG;  // sequences without rows: nothing to verify
  return launch<true, false>(logits, row_stride, vocab, num_tokens, cu_seqlens_q, num_seqs,
                             input_ids, nullptr, argmax, nullptr, accept_len, bonus, workspace,
                             workspace_bytes_, static_cast<hipStream_t>(stream));
}

extern "C" int nva_argmax_rows(const void* logits, int64_t row_stride, int32_t vocab,
                               int32_t num_rows, const int64_t* index_map, int64_t* out,
                               void* workspace, size_t workspace_bytes_, void* stream) {
  if (vocab <= 0 || num_rows < 0 || row_stride < vocab) return NVA_ERR_ARG;
  if (num_rows == 0) return NVA_OK;
  if (!logits || !out) return NVA_ERR_ARG;
  return launch<false, true>(logits, row_stride, vocab, num_rows, nullptr, 0, nullptr, index_map,
                             nullptr, out, nullptr, nullptr, workspace, workspace_bytes_,
                             static_cast<hipStream_t>(stream));
}
