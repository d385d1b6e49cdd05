// K4: vocab argmax fused with the greedy accepted-prefix / bonus scan.
//
// Two launches, no cross-workgroup synchronisation (device-scope fences are
// L2 write-backs on a multi-XCD part, far too costly per block):
//   1. argmax_partial_kernel, grid (chunks_per_row, rows), 256 threads: each
//      block reduces one 16384-element vocab chunk of one row to the 64-bit
//      key
//          key = ord16(value) << 32 | (0xFFFFFFFF - index)
//      of its first maximum, where ord16 maps bf16 bit patterns to unsigned
//      integers in numeric order (-0 and +0 equal, every NaN above +inf), so
//      the maximum key over a row is its first maximum with NaN as the
//      maximum -- the rule of torch.argmax.  The block's key goes to
//      partials[row][chunk].  Each thread holds eight 16-byte vectors in
//      registers and maps them to ord16 with packed 16-bit operations (two
//      elements per instruction), keeping only the running maximum; after
//      the block's maximum is known, the threads holding it scan their
//      registers for its first index.  A chunk with a NaN, an odd-length
//      tail or unaligned rows takes an element-by-element loop instead.
//   2. the merge: each row's chunk keys give its argmax, then the accept
//      scan of speculative.py:11-30 runs per sequence.  Up to 8192 keys and
//      2048 rows, one workgroup issues every load at once and passes the
//      row results to the scans through LDS (one memory latency); beyond
//      that, one wave per sequence (or per row group when there is no accept
//      scan) loads the sequence's offsets, then all of its chunk keys and
//      next input ids at once (one per lane).
#include <atomic>
#include <mutex>

#include "common.h"

namespace nva {
namespace {

constexpr int kThreads = 256;
constexpr int kVecsPerThread = 8;                               // 16-byte vectors in registers
constexpr int kChunkElems = kThreads * kVecsPerThread * 8;      // 16384 elements per block

typedef __attribute__((ext_vector_type(2))) unsigned short u16x2_t;
typedef __attribute__((ext_vector_type(2))) short s16x2_t;

// ord16: 0x8000 + magnitude for non-negative values, 0x8000 - magnitude for
// negative ones (so -0 == +0 and -inf = 0x0080), every NaN 0xFFFF.  Every
// element's key is therefore above 0, which stands for "no element".
__device__ __forceinline__ uint32_t ord16(uint32_t b) {
  const uint32_t mag = b & 0x7FFFu;
  if (mag > 0x7F80u) return 0xFFFFu;
  return (b & 0x8000u) ? 0x8000u - mag : 0x8000u + mag;
}

// ord16 of the two bf16 values of a 32-bit word, without the NaN rule (the
// caller routes chunks holding a NaN to the exact loop); also raises
// mag_max to the word's magnitudes.  Packed 16-bit ops: sign mask s, then
// (mag ^ s) - s is +-mag, and ^ 0x8000 adds 0x8000 modulo 2^16.
__device__ __forceinline__ uint32_t ord16x2(uint32_t w, u16x2_t& mag_max) {
  const u16x2_t s = __builtin_bit_cast(u16x2_t, __builtin_bit_cast(s16x2_t, w) >> 15);
  const u16x2_t m = __builtin_bit_cast(u16x2_t, w & 0x7FFF7FFFu);
  mag_max = __builtin_elementwise_max(mag_max, m);
  return __builtin_bit_cast(uint32_t, (m ^ s) - s) ^ 0x80008000u;
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

// block-wide maximum of a 64-bit key (every thread gets it)
__device__ __forceinline__ uint64_t block_max64(uint64_t v, uint64_t* red) {
  v = wave_max(v);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  uint64_t r = red[0];
#pragma unroll
  for (int i = 1; i < kThreads / kWave; ++i) r = umax64(r, red[i]);
  __syncthreads();
  return r;
}

// strictly greater keeps the earlier index: elements arrive in index order
__device__ __forceinline__ void take(uint32_t b, uint32_t idx, uint32_t& best_ord,
                                     uint32_t& best_idx) {
  const uint32_t o = ord16(b);
  const bool gt = o > best_ord;
  best_ord = gt ? o : best_ord;
  best_idx = gt ? idx : best_idx;
}

// exact element-by-element reduction of rp[begin, end): thread t visits
// t, t + 256, ... in increasing order
__device__ uint64_t chunk_exact(const uint16_t* __restrict__ rp, int32_t begin, int32_t end,
                                uint64_t* red) {
  uint32_t best_ord = 0, best_idx = 0xFFFFFFFFu;
  for (int32_t c = begin + static_cast<int32_t>(threadIdx.x); c < end; c += kThreads)
    take(rp[c], static_cast<uint32_t>(c), best_ord, best_idx);
  // threads that saw nothing keep key 0, below every real key
  return block_max64(best_idx == 0xFFFFFFFFu ? 0 : make_key(best_ord, best_idx), red);
}

__global__ void __launch_bounds__(kThreads)
argmax_partial_kernel(const uint16_t* __restrict__ logits, int64_t row_stride, int32_t vocab,
                      int32_t chunks, bool vec, uint64_t* __restrict__ partials) {
  __shared__ uint64_t red[kThreads / kWave];
  const int32_t row = blockIdx.y;
  const int32_t chunk = blockIdx.x;
  const int32_t begin = chunk * kChunkElems;
  const int32_t end = begin + kChunkElems < vocab ? begin + kChunkElems : vocab;
  const uint16_t* rp = logits + static_cast<int64_t>(row) * row_stride;
  const int tid = static_cast<int>(threadIdx.x);
  uint64_t key;
  if (!vec || ((end - begin) & 7) != 0) {
    key = chunk_exact(rp, begin, end, red);
  } else {
    // ---- phase 1: the chunk's vectors into registers as packed ord16
    // keys (vector tid + 256 i of the chunk in o[i]); loads past the
    // chunk's vectors read zeros and are set to key 0 below
    const int32_t nvec = (end - begin) >> 3;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(rp + begin, nvec * 16);
    uint32_t o[kVecsPerThread][4];
    u16x2_t mag_max = {0, 0};
#pragma unroll
    for (int i = 0; i < kVecsPerThread; ++i) {
      const uint4 w = __builtin_bit_cast(
          uint4,
          __builtin_amdgcn_raw_buffer_load_b128(rs, (tid + kThreads * i) * 16, 0, kLoadStreamed));
      o[i][0] = ord16x2(w.x, mag_max);
      o[i][1] = ord16x2(w.y, mag_max);
      o[i][2] = ord16x2(w.z, mag_max);
      o[i][3] = ord16x2(w.w, mag_max);
    }
    if (nvec < kThreads * kVecsPerThread) {
#pragma unroll
      for (int i = 0; i < kVecsPerThread; ++i)
        if (tid + kThreads * i >= nvec) o[i][0] = o[i][1] = o[i][2] = o[i][3] = 0;
    }
    u16x2_t omax = {0, 0};
#pragma unroll
    for (int i = 0; i < kVecsPerThread; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) omax = __builtin_elementwise_max(omax, __builtin_bit_cast(u16x2_t, o[i][j]));
    const uint32_t lmax = omax.x > omax.y ? omax.x : omax.y;
    const uint32_t lmag = mag_max.x > mag_max.y ? mag_max.x : mag_max.y;
    // ---- the block's maximum key and largest magnitude in one reduction
    const uint64_t both = block_max64((static_cast<uint64_t>(lmag > 0x7F80u) << 32) | lmax, red);
    if (both >> 32) {
      key = chunk_exact(rp, begin, end, red);   // a NaN: the exact loop applies its rule
    } else {
      const uint32_t M = static_cast<uint32_t>(both);
      // ---- phase 2: the first index holding M (threads that hold it scan
      // their registers from the last element back, so the first match wins)
      uint32_t first = 0xFFFFFFFFu;
      if (lmax == M) {
#pragma unroll
        for (int i = kVecsPerThread - 1; i >= 0; --i) {
#pragma unroll
          for (int j = 3; j >= 0; --j) {
            const uint32_t at = static_cast<uint32_t>(begin + (tid + kThreads * i) * 8 + 2 * j);
            first = (o[i][j] >> 16) == M ? at + 1 : first;
            first = (o[i][j] & 0xFFFFu) == M ? at : first;
          }
        }
      }
      // the smallest index is the largest (0xFFFFFFFF - index)
      key = block_max64(first == 0xFFFFFFFFu ? 0 : make_key(M, first), red);
    }
  }
  if (tid == 0) partials[static_cast<int64_t>(row) * chunks + chunk] = key;
}

// One pass of a wave over rows r0 .. r0 + rn - 1 of a contiguous run of
// rows whose chunk keys start at `keys`: lane l holds key l of the pass
// (row l / chunks) when a pass covers whole rows, else the lane-strided
// maximum of one row's keys.  Returns the lane's key and sets its row.
__device__ __forceinline__ uint64_t pass_keys(const uint64_t* __restrict__ keys, int32_t chunks,
                                              int32_t r0, int32_t rn, int32_t& my_row) {
  const int lane = wave_lane();
  uint64_t mine = 0;
  my_row = -1;
  if (chunks <= kWave) {
    if (lane < rn * chunks) {
      mine = keys[static_cast<int64_t>(r0) * chunks + lane];
      my_row = lane / chunks;
    }
  } else {
    for (int32_t c = lane; c < chunks; c += kWave)
      mine = umax64(mine, keys[static_cast<int64_t>(r0) * chunks + c]);
    my_row = 0;
  }
  return mine;
}

__host__ __device__ __forceinline__ int32_t rows_per_pass(int32_t chunks) {
  return chunks <= kWave ? kWave / chunks : 1;
}

// one wave per sequence: argmax of its rows, then the accept scan.  The
// sequence's rows are contiguous, so its chunk keys are one contiguous run;
// each pass loads the keys of as many rows as the lanes hold and those
// rows' next input ids together, so a verify sequence (q <= 64 / chunks
// rows) waits for memory once instead of once per row.
__global__ void __launch_bounds__(kWave)
argmax_accept_finalize_kernel(const uint64_t* __restrict__ partials, int32_t chunks,
                              int32_t num_rows, const int32_t* __restrict__ cu_q, int32_t num_seqs,
                              const int64_t* __restrict__ input_ids, int32_t* __restrict__ argmax32,
                              int32_t* __restrict__ accept_len, int32_t* __restrict__ bonus) {
  const int32_t s = blockIdx.x;
  if (s >= num_seqs) return;
  const int lane = wave_lane();
  int32_t start = cu_q[s];
  int32_t stop = cu_q[s + 1];
  start = start < 0 ? 0 : start;
  stop = stop > num_rows ? num_rows : stop;
  const int32_t q = stop - start;
  if (q <= 0) {
    if (lane == 0) {
      accept_len[s] = 0;
      bonus[s] = -1;
    }
    return;
  }
  const uint64_t* keys = partials + static_cast<int64_t>(start) * chunks;
  int32_t a = 0, bonus_tok = -1;
  bool open = true;
  const int32_t per_pass = rows_per_pass(chunks);
  for (int32_t r0 = 0; r0 < q; r0 += per_pass) {
    const int32_t rn = q - r0 < per_pass ? q - r0 : per_pass;
    // lane j < rn holds the input token that row r0 + j's argmax must match
    const int64_t next = (lane < rn && r0 + lane < q - 1) ? input_ids[start + 1 + r0 + lane] : -1;
    int32_t my_row;
    const uint64_t mine = pass_keys(keys, chunks, r0, rn, my_row);
    for (int32_t j = 0; j < rn; ++j) {
      const uint64_t k = wave_max(my_row == j ? mine : 0);
      const uint32_t idx = 0xFFFFFFFFu - static_cast<uint32_t>(k);
      const int32_t row = r0 + j;
      if (lane == 0) argmax32[start + row] = static_cast<int32_t>(idx);
      if (open) {
        const int64_t want = __shfl(next, j, kWave);
        if (row < q - 1 && want == static_cast<int64_t>(idx)) {
          ++a;
        } else {
          open = false;
          bonus_tok = static_cast<int32_t>(idx);
        }
      }
    }
  }
  if (lane == 0) {
    accept_len[s] = a;
    bonus[s] = bonus_tok;
  }
}

// Small batches (a verify step's few hundred rows): one workgroup issues all
// of its global loads at once -- every chunk key (coalesced), every row's
// next input id and the sequence offsets -- so the merge waits for memory
// once, where the wave-per-sequence kernel waits twice (offsets, then keys).
// Row argmaxes and "equals the next input id" flags go through LDS to the
// per-sequence scans.  Covers num_rows * chunks <= kSmallKeys, num_rows <=
// kSmallRows and num_seqs + 1 <= kSmallRows; every row in [0, num_rows) gets
// its argmax written.  Partials + merge for [384, 151936] (64 sequences of 6
// rows): 22.3-22.5 us with the wave-per-sequence merge, 20.8 us with this
// one; [40, 151936]: 8.2 -> 7.0 us.
constexpr int kSmallThreads = 1024;
constexpr int kSmallKeys = 8 * kSmallThreads;
constexpr int kSmallRows = 2 * kSmallThreads;

__global__ void __launch_bounds__(kSmallThreads)
argmax_accept_finalize_small_kernel(const uint64_t* __restrict__ partials, int32_t chunks,
                                    int32_t num_rows, const int32_t* __restrict__ cu_q,
                                    int32_t num_seqs, const int64_t* __restrict__ input_ids,
                                    int32_t* __restrict__ argmax32, int32_t* __restrict__ accept_len,
                                    int32_t* __restrict__ bonus) {
  __shared__ uint64_t keys[kSmallKeys];
  __shared__ int32_t amax[kSmallRows];
  __shared__ int32_t cu[kSmallRows];
  __shared__ uint8_t match[kSmallRows];
  const int tid = static_cast<int>(threadIdx.x);
  const int32_t nkeys = num_rows * chunks;
  // ---- every global load first (fixed trip counts: nothing waits between them)
  uint64_t kv[kSmallKeys / kSmallThreads];
#pragma unroll
  for (int i = 0; i < kSmallKeys / kSmallThreads; ++i) {
    const int32_t at = tid + i * kSmallThreads;
    kv[i] = at < nkeys ? partials[at] : 0;
  }
  int64_t next[kSmallRows / kSmallThreads];
  int32_t off[kSmallRows / kSmallThreads];
#pragma unroll
  for (int i = 0; i < kSmallRows / kSmallThreads; ++i) {
    const int32_t r = tid + i * kSmallThreads;
    next[i] = r + 1 < num_rows ? input_ids[r + 1] : -1;
    off[i] = r <= num_seqs ? cu_q[r] : 0;
  }
#pragma unroll
  for (int i = 0; i < kSmallKeys / kSmallThreads; ++i) {
    const int32_t at = tid + i * kSmallThreads;
    if (at < nkeys) keys[at] = kv[i];
  }
#pragma unroll
  for (int i = 0; i < kSmallRows / kSmallThreads; ++i) cu[tid + i * kSmallThreads] = off[i];
  __syncthreads();
  // ---- row argmaxes (the largest key's index) and their match flags
#pragma unroll
  for (int i = 0; i < kSmallRows / kSmallThreads; ++i) {
    const int32_t r = tid + i * kSmallThreads;
    if (r < num_rows) {
      uint64_t best = 0;
      for (int32_t c = 0; c < chunks; ++c) best = umax64(best, keys[r * chunks + c]);
      const uint32_t idx = 0xFFFFFFFFu - static_cast<uint32_t>(best);
      argmax32[r] = static_cast<int32_t>(idx);
      amax[r] = static_cast<int32_t>(idx);
      match[r] = next[i] == static_cast<int64_t>(idx) ? 1 : 0;
    }
  }
  __syncthreads();
  // ---- accept scan per sequence (speculative.py:11-30)
  for (int32_t s = tid; s < num_seqs; s += kSmallThreads) {
    int32_t start = cu[s];
    int32_t stop = cu[s + 1];
    start = start < 0 ? 0 : start;
    stop = stop > num_rows ? num_rows : stop;
    const int32_t q = stop - start;
    if (q <= 0) {
      accept_len[s] = 0;
      bonus[s] = -1;
      continue;
    }
    int32_t a = 0;
    while (a < q - 1 && match[start + a]) ++a;
    accept_len[s] = a;
    bonus[s] = amax[start + a];
  }
}

bool small_finalize(int32_t num_rows, int32_t chunks, int32_t num_seqs) {
  return static_cast<int64_t>(num_rows) * chunks <= kSmallKeys && num_rows <= kSmallRows &&
         num_seqs + 1 <= kSmallRows;
}

// rows without an accept scan: each wave finalises one pass of rows
// (rows_per_pass(chunks) rows, their keys loaded together)
__global__ void __launch_bounds__(kWave)
argmax_rows_finalize_kernel(const uint64_t* __restrict__ partials, int32_t chunks,
                            int32_t num_rows, const int64_t* __restrict__ index_map,
                            int64_t* __restrict__ out64) {
  const int32_t per_pass = rows_per_pass(chunks);
  const int32_t r0 = blockIdx.x * per_pass;
  if (r0 >= num_rows) return;
  const int32_t rn = num_rows - r0 < per_pass ? num_rows - r0 : per_pass;
  int32_t my_row;
  const uint64_t mine = pass_keys(partials, chunks, r0, rn, my_row);
  // lane j keeps row j's index, so the index-map lookups of the pass are
  // one vector load (one memory latency) and the stores one vector store
  const int lane = wave_lane();
  uint32_t row_idx = 0;
  for (int32_t j = 0; j < rn; ++j) {
    const uint64_t k = wave_max(my_row == j ? mine : 0);
    if (lane == j) row_idx = 0xFFFFFFFFu - static_cast<uint32_t>(k);
  }
  if (lane < rn)
    out64[r0 + lane] = static_cast<int64_t>(row_idx) + (index_map ? index_map[row_idx] : 0);
}

// Chunks of kChunkElems elements per row.
int32_t row_chunks(int32_t vocab) { return vocab > 0 ? (vocab + kChunkElems - 1) / kChunkElems : 1; }

// ---- static scratch of the allocation-free entry point
//
// The chunk keys of nva_argmax_accept_static live in this array instead of a
// caller workspace.  Each GPU the library runs on holds its own copy until
// the process ends.  Host code never passes `scratch` itself to a kernel
// (on the host that name is a stand-in, not a device address): the device
// address comes from hipGetSymbolAddress, looked up once per device with
// that device current, and is kept in g_scratch_ptr.
// Two keys beyond the limit: the workspace check asks for 16 bytes of slack.
static __device__ __align__(256) uint64_t scratch[NVA_ARGMAX_STATIC_KEYS + 2];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device (looked up on the first
// call per device).  The stream must belong to that device.
int static_scratch(hipStream_t stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return NVA_ERR_LAUNCH;
  if (stream) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess) return NVA_ERR_ARG;
    if (sdev != dev) return NVA_ERR_ARG;
  }
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
        (void)hipGetLastError();   // do not leave the error for the next launch check
        return NVA_ERR_LAUNCH;
      }
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return NVA_OK;
}

size_t workspace_bytes(int32_t rows, int32_t vocab) {
  return static_cast<size_t>(rows) * row_chunks(vocab) * sizeof(uint64_t) + 16;
}

int launch_partials(const void* logits, int64_t row_stride, int32_t vocab, int32_t rows,
                    void* ws, size_t ws_bytes, hipStream_t stream, int32_t* chunks_out) {
  const int32_t c = row_chunks(vocab);
  if (!ws || ws_bytes < workspace_bytes(rows, vocab) || (reinterpret_cast<uintptr_t>(ws) & 7u))
    return NVA_ERR_WORKSPACE;
  const bool vec = aligned16(logits) && (row_stride % 8 == 0);
  dim3 grid(c, rows);
  argmax_partial_kernel<<<grid, kThreads, 0, stream>>>(static_cast<const uint16_t*>(logits),
                                                       row_stride, vocab, c, vec,
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

namespace {

int check_accept_args(const void* logits, int64_t row_stride, int32_t vocab,
                      const int32_t* cu_seqlens_q, int32_t num_seqs, int32_t num_tokens,
                      const int64_t* input_ids, const int32_t* argmax, const int32_t* accept_len,
                      const int32_t* bonus) {
  if (vocab <= 0 || num_seqs < 0 || num_tokens < 0 || row_stride < vocab) return NVA_ERR_ARG;
  if (num_seqs == 0) return NVA_OK;
  if (!cu_seqlens_q || !accept_len || !bonus) return NVA_ERR_ARG;
  if (num_tokens > 0 && (!logits || !input_ids || !argmax)) return NVA_ERR_ARG;
  return NVA_OK;
}

// The two launches of nva_argmax_accept over the given chunk-key buffer
// (arguments already checked, num_seqs > 0).
int argmax_accept_launch(const void* logits, int64_t row_stride, int32_t vocab,
                         const int32_t* cu_seqlens_q, int32_t num_seqs, int32_t num_tokens,
                         const int64_t* input_ids, int32_t* argmax, int32_t* accept_len,
                         int32_t* bonus, void* workspace, size_t workspace_bytes_,
                         hipStream_t s) {
  int32_t chunks = 1;
  if (num_tokens > 0) {
    const int st = launch_partials(logits, row_stride, vocab, num_tokens, workspace,
                                   workspace_bytes_, s, &chunks);
    if (st != NVA_OK) return st;
  }
  if (small_finalize(num_tokens, chunks, num_seqs))
    argmax_accept_finalize_small_kernel<<<1, kSmallThreads, 0, s>>>(
        static_cast<const uint64_t*>(workspace), chunks, num_tokens, cu_seqlens_q, num_seqs,
        input_ids, argmax, accept_len, bonus);
  else
    argmax_accept_finalize_kernel<<<num_seqs, kWave, 0, s>>>(
        static_cast<const uint64_t*>(workspace), chunks, num_tokens, cu_seqlens_q, num_seqs,
        input_ids, argmax, accept_len, bonus);
  return launch_status();
}

}  // namespace

extern "C" int nva_argmax_accept(const void* logits, int64_t row_stride, int32_t vocab,
                                 const int32_t* cu_seqlens_q, int32_t num_seqs,
                                 int32_t num_tokens, const int64_t* input_ids, int32_t* argmax,
                                 int32_t* accept_len, int32_t* bonus, void* workspace,
                                 size_t workspace_bytes_, void* stream) {
  const int st = check_accept_args(logits, row_stride, vocab, cu_seqlens_q, num_seqs,
                                   num_tokens, input_ids, argmax, accept_len, bonus);
  if (st != NVA_OK || num_seqs == 0) return st;
  return argmax_accept_launch(logits, row_stride, vocab, cu_seqlens_q, num_seqs, num_tokens,
                              input_ids, argmax, accept_len, bonus, workspace, workspace_bytes_,
                              static_cast<hipStream_t>(stream));
}

extern "C" int nva_argmax_accept_static(const void* logits, int64_t row_stride, int32_t vocab,
                                        const int32_t* cu_seqlens_q, int32_t num_seqs,
                                        int32_t num_tokens, const int64_t* input_ids,
                                        int32_t* argmax, int32_t* accept_len, int32_t* bonus,
                                        void* stream) {
  int st = check_accept_args(logits, row_stride, vocab, cu_seqlens_q, num_seqs, num_tokens,
                             input_ids, argmax, accept_len, bonus);
  if (st != NVA_OK || num_seqs == 0) return st;
  if (static_cast<int64_t>(num_tokens) * row_chunks(vocab) > NVA_ARGMAX_STATIC_KEYS)
    return NVA_ERR_CAPACITY;
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  st = static_scratch(s, &ws);
  if (st != NVA_OK) return st;
  // every chunk key the merge reads is written by this call's first launch,
  // so the array needs no clearing between calls
  return argmax_accept_launch(logits, row_stride, vocab, cu_seqlens_q, num_seqs, num_tokens,
                              input_ids, argmax, accept_len, bonus, ws,
                              sizeof(uint64_t) * (NVA_ARGMAX_STATIC_KEYS + 2), s);
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
  const int32_t per_pass = rows_per_pass(chunks);
  const int32_t waves = (num_rows + per_pass - 1) / per_pass;
  argmax_rows_finalize_kernel<<<waves, kWave, 0, s>>>(static_cast<const uint64_t*>(workspace),
                                                      chunks, num_rows, index_map, out);
  return launch_status();
}
