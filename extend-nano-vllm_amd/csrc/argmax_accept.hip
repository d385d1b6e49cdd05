// K4: vocab argmax fused with the greedy accepted-prefix / bonus scan.
//
// Two launches, no cross-workgroup synchronisation (device-scope fences are
// L2 write-backs on a multi-XCD part, far too costly per block):
//   1. argmax_partial_kernel, grid (chunks_per_row, rows), 256 threads: each
//      block scans one vocab chunk of one row with 16-byte loads.  Each thread
//      walks its elements in increasing index order keeping (ord, index) of
//      the first maximum; the block merges the threads' results as 64-bit keys
//          key = ord16(value) << 32 | (0xFFFFFFFF - index)
//      where ord16 maps bf16 bit patterns to unsigned integers in numeric
//      order (-0 folded onto +0, every NaN above +inf), so the maximum key is
//      the first index of the maximum with NaN as the maximum -- the rule of
//      torch.argmax.  The block's key goes to partials[row][chunk].
//   2. argmax_finalize_kernel, one wave per sequence (or per row group when
//      there is no accept scan): merges each row's chunk keys, writes the
//      argmax, then lane 0 runs the accept scan of speculative.py:11-30.
#include "common.h"

namespace nva {
namespace {

constexpr int kThreads = 256;
constexpr int kTargetBlocks = 2048;   // ~8 blocks per CU on 256 CUs
constexpr int kMinChunk = 4096;       // elements; two 16-byte loads per thread
constexpr int kRowsPerFinalizeWave = 4;

__device__ __forceinline__ uint32_t ord16(uint32_t b) {
  const uint32_t mag = b & 0x7FFFu;
  const uint32_t o = (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
  return mag > 0x7F80u ? 0xFFFFu : (mag == 0 ? 0x8000u : o);
}

__device__ __forceinline__ uint64_t make_key(uint32_t ord, uint32_t idx) {
  return (static_cast<uint64_t>(ord) << 32) | (0xFFFFFFFFu - idx);
}

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), m, kWave);
  const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), m, kWave);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

__device__ __forceinline__ uint64_t wave_max(uint64_t v) {
#pragma unroll
  for (int m = kWave / 2; m >= 1; m >>= 1) v = umax64(v, shfl_xor64(v, m));
  return v;
}

// strictly greater keeps the earlier index: elements arrive in index order
__device__ __forceinline__ void take(uint32_t b, uint32_t idx, uint32_t& best_ord,
                                     uint32_t& best_idx) {
  const uint32_t o = ord16(b);
  const bool gt = o > best_ord;
  best_ord = gt ? o : best_ord;
  best_idx = gt ? idx : best_idx;
}

__global__ void __launch_bounds__(kThreads)
argmax_partial_kernel(const uint16_t* __restrict__ logits, int64_t row_stride, int32_t vocab,
                      int32_t chunk_elems, int32_t chunks, bool vec,
                      uint64_t* __restrict__ partials) {
  __shared__ uint64_t red[kThreads / kWave];
  const int32_t row = blockIdx.y;
  const int32_t chunk = blockIdx.x;
  const int32_t begin = chunk * chunk_elems;
  int32_t end = begin + chunk_elems;
  end = end > vocab ? vocab : end;
  const uint16_t* rp = logits + static_cast<int64_t>(row) * row_stride;
  uint32_t best_ord = 0, best_idx = 0xFFFFFFFFu;
  if (vec) {
    // thread t owns vectors t, t+256, ...: within a thread indices increase
    const int32_t nvec = (end - begin) / 8;
    const uint4* vp = reinterpret_cast<const uint4*>(rp + begin);
#pragma unroll 4
    for (int32_t v = threadIdx.x; v < nvec; v += kThreads) {
      const uint4 w = vp[v];
      const uint32_t base = static_cast<uint32_t>(begin + v * 8);
      const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) take((d[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu, base + e, best_ord, best_idx);
    }
    for (int32_t c = begin + nvec * 8 + threadIdx.x; c < end; c += kThreads)
      take(rp[c], static_cast<uint32_t>(c), best_ord, best_idx);
  } else {
    for (int32_t c = begin + threadIdx.x; c < end; c += kThreads)
      take(rp[c], static_cast<uint32_t>(c), best_ord, best_idx);
  }
  // threads that saw nothing keep key 0, below every real key
  uint64_t key = best_idx == 0xFFFFFFFFu ? 0 : make_key(best_ord, best_idx);
  key = wave_max(key);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = key;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t k = red[0];
#pragma unroll
    for (int i = 1; i < kThreads / kWave; ++i) k = umax64(k, red[i]);
    partials[static_cast<int64_t>(row) * chunks + chunk] = k;
  }
}

// merge one row's chunk keys across the wave -> argmax index
__device__ __forceinline__ uint32_t merge_row(const uint64_t* __restrict__ partials, int32_t row,
                                              int32_t chunks) {
  uint64_t k = 0;
  for (int32_t c = wave_lane(); c < chunks; c += kWave)
    k = umax64(k, partials[static_cast<int64_t>(row) * chunks + c]);
  k = wave_max(k);
  return 0xFFFFFFFFu - static_cast<uint32_t>(k);
}

// one wave per sequence: argmax of its rows, then the accept scan
__global__ void __launch_bounds__(kWave)
argmax_accept_finalize_kernel(const uint64_t* __restrict__ partials, int32_t chunks,
                              int32_t num_rows, const int32_t* __restrict__ cu_q, int32_t num_seqs,
                              const int64_t* __restrict__ input_ids, int32_t* __restrict__ argmax32,
                              int32_t* __restrict__ accept_len, int32_t* __restrict__ bonus) {
  const int32_t s = blockIdx.x;
  if (s >= num_seqs) return;
  int32_t start = cu_q[s];
  int32_t stop = cu_q[s + 1];
  start = start < 0 ? 0 : start;
  stop = stop > num_rows ? num_rows : stop;
  const int32_t q = stop - start;
  if (q <= 0) {
    if (wave_lane() == 0) {
      accept_len[s] = 0;
      bonus[s] = -1;
    }
    return;
  }
  // lane 0 tracks the scan while rows are merged in order
  int32_t a = 0;
  bool open = true;
  int32_t bonus_tok = -1;
  for (int32_t j = 0; j < q; ++j) {
    const uint32_t idx = merge_row(partials, start + j, chunks);
    if (wave_lane() == 0) {
      argmax32[start + j] = static_cast<int32_t>(idx);
      if (open) {
        if (j < q - 1 && input_ids[start + 1 + j] == static_cast<int64_t>(idx)) {
          ++a;
        } else {
          open = false;
          bonus_tok = static_cast<int32_t>(idx);
        }
      }
    }
  }
  if (wave_lane() == 0) {
    accept_len[s] = a;
    bonus[s] = bonus_tok;
  }
}

// rows without an accept scan: each wave finalises kRowsPerFinalizeWave rows
__global__ void __launch_bounds__(kWave)
argmax_rows_finalize_kernel(const uint64_t* __restrict__ partials, int32_t chunks,
                            int32_t num_rows, const int64_t* __restrict__ index_map,
                            int64_t* __restrict__ out64) {
  for (int32_t i = 0; i < kRowsPerFinalizeWave; ++i) {
    const int32_t row = blockIdx.x * kRowsPerFinalizeWave + i;
    if (row >= num_rows) return;
    const uint32_t idx = merge_row(partials, row, chunks);
    if (wave_lane() == 0)
      out64[row] = static_cast<int64_t>(idx) + (index_map ? index_map[idx] : 0);
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

size_t workspace_bytes(int32_t rows, int32_t vocab) {
  int32_t ce, c;
  choose_chunks(rows, vocab, &ce, &c);
  return static_cast<size_t>(rows) * c * sizeof(uint64_t) + 16;
}

int launch_partials(const void* logits, int64_t row_stride, int32_t vocab, int32_t rows,
                    void* ws, size_t ws_bytes, hipStream_t stream, int32_t* chunks_out) {
  int32_t ce, c;
  choose_chunks(rows, vocab, &ce, &c);
  if (!ws || ws_bytes < workspace_bytes(rows, vocab) || (reinterpret_cast<uintptr_t>(ws) & 7u))
    return NVA_ERR_WORKSPACE;
  const bool vec = aligned16(logits) && (row_stride % 8 == 0);
  dim3 grid(c, rows);
  argmax_partial_kernel<<<grid, kThreads, 0, stream>>>(static_cast<const uint16_t*>(logits),
                                                       row_stride, vocab, ce, c, vec,
                                                       static_cast<uint64_t*>(ws));
  *chunks_out = c;
  return launch_status();
}

}  // namespace
}  // namespace nva

using namespace nva;

extern "C" size_t nva_argmax_workspace_size(int32_t num_rows, int32_t num_seqs, int32_t vocab) {
  if (num_rows < 0 || num_seqs < 0 || vocab <= 0) return 0;
  return workspace_bytes(num_rows, vocab);
}

extern "C" int nva_argmax_accept(const void* logits, int64_t row_stride, int32_t vocab,
                                 const int32_t* cu_seqlens_q, int32_t num_seqs,
                                 int32_t num_tokens, const int64_t* input_ids, int32_t* argmax,
                                 int32_t* accept_len, int32_t* bonus, void* workspace,
                                 size_t workspace_bytes_, void* stream) {
  if (vocab <= 0 || num_seqs < 0 || num_tokens < 0 || row_stride < vocab) return NVA_ERR_ARG;
  if (num_seqs == 0) return NVA_OK;
  if (!cu_seqlens_q || !accept_len || !bonus) return NVA_ERR_ARG;
  if (num_tokens > 0 && (!logits || !input_ids || !argmax)) return NVA_ERR_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int32_t chunks = 1;
  if (num_tokens > 0) {
    const int st = launch_partials(logits, row_stride, vocab, num_tokens, workspace,
                                   workspace_bytes_, s, &chunks);
    if (st != NVA_OK) return st;
  }
  argmax_accept_finalize_kernel<<<num_seqs, kWave, 0, s>>>(
      static_cast<const uint64_t*>(workspace), chunks, num_tokens, cu_seqlens_q, num_seqs,
      input_ids, argmax, accept_len, bonus);
  return launch_status();
}

extern "C" int nva_argmax_rows(const void* logits, int64_t row_stride, int32_t vocab,
                               int32_t num_rows, const int64_t* index_map, int64_t* out,
                               void* workspace, size_t workspace_bytes_, void* stream) {
  if (vocab <= 0 || num_rows < 0 || row_stride < vocab) return NVA_ERR_ARG;
  if (num_rows == 0) return NVA_OK;
  if (!logits || !out) return NVA_ERR_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int32_t chunks = 1;
  const int st = launch_partials(logits, row_stride, vocab, num_rows, workspace, workspace_bytes_,
                                 s, &chunks);
  if (st != NVA_OK) return st;
  const int32_t waves = (num_rows + kRowsPerFinalizeWave - 1) / kRowsPerFinalizeWave;
  argmax_rows_finalize_kernel<<<waves, kWave, 0, s>>>(static_cast<const uint64_t*>(workspace),
                                                      chunks, num_rows, index_map, out);
  return launch_status();
}
