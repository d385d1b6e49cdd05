// K1: paged verify attention for gfx950 (MFMA 16x16x32 bf16).
//
// Unit of work: one wave (64 threads) runs a *segment* -- one query tile of
// one sequence against a contiguous key range, for one kv head.  A query
// tile is up to 64/G consecutive query positions of a sequence times the G
// query heads that share the kv head (G = Hq / Hkv), padded to NT*16 columns
// (NT = 1, 2, 4); a verify step (k+1 positions) is a single tile, a prefill
// is many.  Each tile only walks the keys its last row can see.  Segments
// come from one of two decompositions:
//   * stream (single-tile sequences of at most 32 rows over an FP8 cache):
//     per kv head the key chunks of all sequences are laid end to end and
//     cut into one equal range per SIMD of the device, so every wave streams
//     the same number of keys whatever the length mix;
//   * fixed (everything else): one workgroup per (kv head, sequence, query
//     tile, key split).  For bf16 tiles of up to 32 rows eight waves share a
//     2816-key split (wave w takes chunks w, w+8, ...) and fold their
//     softmax states together in LDS; for single-tile 17-32-row tiles whose
//     segments fill every CU once or twice, four waves share a whole
//     sequence instead and the grid pairs a long sequence with a short one
//     on each CU (paired mode, see paired_mode); bf16 tiles of 33-64 rows run on four
//     waves that share each chunk through LDS, one wave per 16 query
//     columns (paged_attention_tile_kernel); FP8 tiles of more than 32 rows
//     run one wave per 3072-key split (the lengths follow the batch, see
//     choose_split).
// A sequence covered by one segment gets bf16 output directly; otherwise
// each segment writes a normalised fp32 partial plus its log-sum-exp and
// combine_kernel merges them.
//
// Per 32-key chunk a wave computes S^T = K . Q^T (two 16-key tiles, MFMA with
// keys as M, query rows as N, head_dim as K in four 32-wide slices) and
// O^T += V^T . P^T (head_dim as M in eight 16-row tiles, keys as K).
//   * The MFMA sums over K in any order, so K and Q operands only have to
//     agree on which head_dim element sits in which lane slot: lane l holds
//     row (l % 16) and elements 32*s + 8*(l/16) .. +7 of slice s, a 16-byte
//     load straight from the paged cache, or (FP8 caches, and bf16 segments
//     shared by several waves) a 16-byte read of a wave-private LDS tile
//     that the K rows were staged into (XOR-swizzled 16-byte columns, see
//     kst_slot), so that K too loads whole 128-byte lines with the
//     non-temporal hint, as V does.  The Q operands
//     are parked in LDS in that order and re-read per chunk, so they hold no
//     registers.
//   * The S^T accumulator layout (lane l: query column l % 16, keys
//     4*(l/16) + i) is exactly the B-operand layout of the P^T operand once
//     the 8 lane slots are mapped to keys {4g..4g+3, 16+4g..16+4g+3}; V^T uses
//     the same key mapping.  V is therefore staged through a wave-private LDS
//     tile (row pitch 68 dwords: conflict-free for the column reads) and read
//     back two head_dim elements per dword, feeding an even and an odd d-tile;
//     the shared-tile kernel instead reads its V^T operands with the LDS
//     transpose load from 72-dword rows (v_operand_tr).
//   * K/V loads are raw buffer loads from a per-chunk descriptor (uniform
//     base, loop-invariant lane offsets, record count ending at the last
//     visible key so that rows past it read as zeros).  Where a SIMD holds
//     a single wave (64-row tiles) or dequantisation lengthens the math
//     (FP8), they are issued one chunk ahead into a second register buffer.
// FP8 caches are dequantised to bf16 on load with the hardware conversion
// (exact: every e4m3 value is a bf16 value).  At the end each lane writes,
// straight from its accumulators, 8 consecutive head_dim values of one query
// column per 32-column group (16-byte bf16 stores; fp32 partials when the
// keys are split); waves sharing a segment first park their states in LDS
// and each finishes a quarter of head_dim.
#include <stdio.h>
#include <stdlib.h>

#include "common.h"

namespace nva {
namespace {

constexpr int kD = 128;
constexpr int kCombineWaves = 4;
constexpr int kCombineThreads = kCombineWaves * kWave;
constexpr int kChunk = 32;
constexpr int kVPitch = 68;                          // dwords per staged V row
constexpr int kVStage = kChunk * kVPitch;            // dwords of the wave's V stage
constexpr int kSplitKeys = 3072;       // fixed decomposition, one wave per split
constexpr int kKeysPerSharedWave = 352; // fixed decomposition, several waves per split
constexpr int kMinSplit = 128;
constexpr int64_t kMinWaves = 1024;
// a split spans at most kWave - 2 blocks; blocks hold at least kChunk tokens
constexpr int kMaxSeqGroups = 8;        // stream mode: up to 8 * 64 sequences
constexpr int kMinRangeChunks = 4;      // stream mode: at least 128 keys per range
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleSlack = 8.0f;   // log2 headroom before the running max moves

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(2))) float f32x2_t;

struct AttnParams {
  const uint16_t* q;
  int64_t q_row_stride, q_head_stride;
  const uint8_t* k_cache;
  const uint8_t* v_cache;
  int64_t blk_stride, tok_stride, head_stride;       // elements
  int32_t num_blocks, block_size;
  const int32_t* cu_q;                                // null: row i is sequence i
  const int32_t* cu_k;                                // non-null: L_i = cu_k[i+1]-cu_k[i]
  const int32_t* seqlens;                             // otherwise L_i = seqlens[i]
  const int32_t* block_tables;
  int64_t bt_stride;
  int32_t bt_cols;
  int32_t num_seqs, num_tokens, max_q, max_k;
  int32_t hq, hkv, group;
  float scale_log2;
  const float* k_scale;
  const float* v_scale;
  uint16_t* out;
  int64_t out_row_stride, out_head_stride;
  float* ws_o;
  float* ws_lse;
  int32_t split_len, max_splits;
  int32_t qtile, n_qtiles;                            // query positions per workgroup
  // stream decomposition (one query tile per sequence)
  int32_t min_range_chunks, max_range_chunks;
  int32_t* row_nsplit;                                // [num_tokens] split count per query row
  // paired mode: grid rows y >= pair_rows take the sequences from the last
  // one backwards (0: row y is sequence y)
  int32_t pair_rows;
};

__device__ __forceinline__ float exp2f_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Reductions over the lane pairs (l, l ^ 16) and (l, l ^ 32), every lane
// receiving the pair's result.  gfx950's v_permlane16_swap /
// v_permlane32_swap with both operands x leave the pair's two values, the
// lower lane's first, in the two results of every lane of the pair: a
// VALU exchange.  __shfl_xor compiles to ds_bpermute, which goes through
// the LDS unit and makes the next use wait for every outstanding LDS
// operation of the wave (in the key loop: the V rows just staged).  Both
// lanes combine the same two values in the same order, and max and + are
// commutative, so the results equal the shuffle forms' bit for bit.  The
// two results are read into integers before the bit cast: a bit cast of
// the second element of the builtin's result vector compiles to the first
// element (ROCm 7.2 clang).
__device__ __forceinline__ float max_xor16(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const uint32_t lo = r[0], hi = r[1];
  return fmaxf(__builtin_bit_cast(float, lo), __builtin_bit_cast(float, hi));
}
__device__ __forceinline__ float max_xor32(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const uint32_t lo = r[0], hi = r[1];
  return fmaxf(__builtin_bit_cast(float, lo), __builtin_bit_cast(float, hi));
}
__device__ __forceinline__ float sum_xor16(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const uint32_t lo = r[0], hi = r[1];
  return __builtin_bit_cast(float, lo) + __builtin_bit_cast(float, hi);
}
__device__ __forceinline__ float sum_xor32(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const uint32_t lo = r[0], hi = r[1];
  return __builtin_bit_cast(float, lo) + __builtin_bit_cast(float, hi);
}

// Orders a wave's own LDS writes and reads: LDS executes one wave's
// operations in issue order, so the compiler must only keep program order
// and wait for outstanding LDS operations.
__device__ __forceinline__ void lds_wave_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

typedef __attribute__((ext_vector_type(4))) short s16x4_t;
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

// The V^T operand of the O^T += V^T . P^T product for head_dim tile (pp, hf),
// read from a staged chunk (32 key rows of `pitch` dwords, bf16) with gfx950's
// LDS transpose load.  ds_read_b64_tr_b16 hands lane l element e of the
// 8-byte piece that lane 16 (l / 16) + 4 e + (l % 16) / 4 addressed, at that
// piece's position (l % 16) % 4.  Lane l addresses key row
// 4 (l / 16) + (l % 16) / 4 (+ 16 for the second load), head_dim
// 32 pp + 8 (l % 4) + 4 hf, so lane (g, m16) receives
//   A row m16 <-> d = 32 pp + 8 (m16 / 4) + 4 hf + m16 % 4,
//   k-slot 8 g + 4 r + e <-> key 16 r + 4 g + e   (the P^T operand's order),
// and the accumulator tile (pp, hf) holds d = 32 pp + 8 g + 4 hf + i in
// element i of lane (g, m16): the two tiles of pair pp give the lane eight
// consecutive head_dim values.  With a row pitch of 72 dwords the 16 lanes
// one LDS cycle serves fall on at most two addresses per bank (at 68 dwords,
// four).
__device__ __forceinline__ bf16x8_t v_operand_tr(const uint32_t* rows, int pitch, int lane, int pp,
                                                 int hf) {
  const int row = 4 * (lane >> 4) + ((lane & 15) >> 2);
  uint32_t* p0 = const_cast<uint32_t*>(rows) + row * pitch + 16 * pp + 4 * (lane & 3) + 2 * hf;
  const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(p0));
  const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(p0 + 16 * pitch));
  return bf16x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

__device__ __forceinline__ f32x4_t mfma(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
}

// 8 fp8 (OCP e4m3fn) bytes -> 8 bf16, exact: v_cvt_scalef32_pk_bf16_fp8 with
// scale 1.0 converts two bytes of the selected 16-bit half (every e4m3 value,
// subnormals included, is a bf16 value; 0x7F / 0xFF give NaN).  The kernel
// applies k_scale / v_scale in fp32 elsewhere.
__device__ __forceinline__ bf16x8_t fp8x8_to_bf16(uint2 w) {
  const bf16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.x, 1.0f, false);
  const bf16x2_t b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.x, 1.0f, true);
  const bf16x2_t c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.y, 1.0f, false);
  const bf16x2_t d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.y, 1.0f, true);
  const uint4 r = make_uint4(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                            __builtin_bit_cast(uint32_t, c), __builtin_bit_cast(uint32_t, d));
  return __builtin_bit_cast(bf16x8_t, r);
}

// Query rows and keys of sequence seq (any lane's own sequence).  The end
// of the key range is one load from a selected pointer (cu_k + 1 or
// seqlens), issued with the others before any value is used, so the
// geometry costs one memory latency.
// q_rows_raw (optional) receives the sequence's row count before the
// max_seqlen_q clip (bounded by num_tokens the same way).  A sequence
// clipped to its first max_q rows also drops the keys of its clipped rows
// (L shrinks by the rows cut), so each kept row j still sees keys
// [0, L - q_raw + j], its unclipped causal window.
__device__ __forceinline__ void seq_geometry(const AttnParams& p, int seq, int& q_start, int& q_len,
                                             int& L, int* q_rows_raw = nullptr) {
  int q0 = seq, q1 = seq + 1, k0 = 0;
  const int k1 = (p.cu_k ? p.cu_k + 1 : p.seqlens)[seq];
  if (p.cu_q) {
    q0 = p.cu_q[seq];
    q1 = p.cu_q[seq + 1];
  }
  if (p.cu_k) k0 = p.cu_k[seq];
  q_start = q0;
  int raw = q1 - q0;
  if (q_start < 0 || q_start >= p.num_tokens) raw = 0;
  else if (raw > p.num_tokens - q_start) raw = p.num_tokens - q_start;
  q_len = raw > p.max_q ? p.max_q : raw;
  if (q_rows_raw) *q_rows_raw = raw;
  L = k1 - k0 - (raw - q_len);
  L = L > p.max_k ? p.max_k : L;
}

// seq_geometry for a wave-uniform seq: readfirstlane states the values'
// uniformity, which the compiler cannot see through the pointer select, so
// that they stay in scalar registers (a buffer descriptor built from them
// would otherwise need a waterfall loop per load).
__device__ __forceinline__ void seq_geometry_uniform(const AttnParams& p, int seq, int& q_start,
                                                     int& q_len, int& L,
                                                     int* q_rows_raw = nullptr) {
  seq_geometry(p, seq, q_start, q_len, L, q_rows_raw);
  q_start = __builtin_amdgcn_readfirstlane(q_start);
  q_len = __builtin_amdgcn_readfirstlane(q_len);
  L = __builtin_amdgcn_readfirstlane(L);
  if (q_rows_raw) *q_rows_raw = __builtin_amdgcn_readfirstlane(*q_rows_raw);
}

// Block ids of the split that starts at key kv_begin, one per lane: lane i
// holds logical block kv_begin / block_size + i (the host keeps a split
// within kWave - 2 blocks; lanes past the split hold ids nobody reads).
// Needs no sequence geometry, so the fixed kernel issues it together with
// the geometry loads instead of after them.
__device__ __forceinline__ int split_block_ids(const AttnParams& p, int seq, int kv_begin) {
  const int col = kv_begin / p.block_size + static_cast<int>(threadIdx.x & (kWave - 1));
  return col < p.bt_cols ? p.block_tables[static_cast<int64_t>(seq) * p.bt_stride + col] : -1;
}

// Segments over an FP8 cache, and shared segments over a bf16 cache
// (several waves, one chunk buffer), also stage K through a wave-private
// LDS tile: the K rows then load like the V rows, whole 128-byte lines per
// instruction with the non-temporal hint (FP8 rows dequantised to bf16 on
// the way in, as V's), and the MFMA operands are read back in the order
// the registers held them.
// NVA_K_STAGE=0 at build time keeps K in registers (half lines, default
// policy) for comparison.
#ifndef NVA_K_STAGE
#define NVA_K_STAGE 1
#endif
// Dword offset of 16-byte column c (0..15) of K row r in a K stage: rows of
// 64 dwords, the column XORed with the row's low four bits, so that the
// 16 rows of an operand read (one column) and the 16 columns of a staging
// write (one row) each fall on 16 different 16-byte bank groups.  With the
// V stage's 68-dword pitch instead, the operand reads conflicted (626 k
// conflict cycles per config-3 call, 10.5 M per FP8 config-4 call; 0 with
// the swizzle, the call times unchanged).
__device__ __forceinline__ int kst_slot(int r, int c) { return r * 64 + ((c ^ (r & 15)) << 2); }
constexpr bool k_staged(bool fp8, bool pipe, int wps) {
  return NVA_K_STAGE && (fp8 || (!pipe && wps > 1));
}

// One segment of work: the query tile qt of sequence seq (all its rows
// for kv head kvh; the sequence's rows start at q_start, it has q_len query
// rows and L keys) against keys [kv_begin, kv_end), which is split `split`
// of the `nsplit` splits covering the keys the tile can see.  lane_blk is
// split_block_ids(p, seq, kv_begin).  A single split
// writes the bf16 output; otherwise a normalised fp32 partial and its
// log-sum-exp go to the workspace for combine_kernel.
//
// WPS > 1 waves (one workgroup) share a segment: wave w takes chunks w,
// w + WPS, ...; their softmax states are merged through LDS at the end and
// wave 0 writes the result.  `vst` then holds WPS stages.
template <int NT, bool FP8, bool PIPE, int WPS>
__device__ __forceinline__ void attend_segment(const AttnParams& p, uint32_t* vst, bf16x8_t* qst,
                                               const int kvh, const int seq, const int qt,
                                               const int q_start, const int q_len, const int L,
                                               const int kv_begin, const int kv_end,
                                               const int split, const int nsplit,
                                               const int lane_blk) {
  static_assert(WPS == 1 || !PIPE, "shared segments use the single-buffer loop");
  static_assert(WPS == 1 || (NT <= 2 && (8 * kWave * 4 + 2 * kWave) <= kVStage),
                "a wave's parked state must fit one V stage per column tile");
  constexpr bool KST = k_staged(FP8, PIPE, WPS);
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = WPS > 1 ? __builtin_amdgcn_readfirstlane(threadIdx.x / kWave) : 0;
  const int g = lane >> 4;
  const int m16 = lane & 15;
  uint32_t* const stage = vst + wv * kVStage;           // this wave's V stage
  uint32_t* const kstage = KST ? vst + (WPS + wv) * kVStage : stage;  // its K stage

  // this tile's query positions: j0 .. j0 + jn - 1 of the sequence
  const int j0 = qt * p.qtile;
  const int jn = (q_len - j0 < p.qtile) ? q_len - j0 : p.qtile;
  const int rows = jn * p.group;
  // keys any row of the tile can see (bottom-right causal)
  const int kv_limit = L - q_len + j0 + jn;

  float kscale = 1.0f, vscale = 1.0f;
  if (FP8) {
    kscale = p.k_scale ? *p.k_scale : 1.0f;
    vscale = p.v_scale ? *p.v_scale : 1.0f;
  }
  const float sl2 = p.scale_log2 * kscale;

  // ---- query operands, loaded here and parked in LDS (in operand order:
  // entry (nt, s) is one 16-byte vector per lane, read back conflict-free
  // for every chunk so that they hold no registers across the loop) once
  // the first chunk's K/V loads are in flight; and the causal limits
  // Padding columns (n >= rows) load row 0 and are zeroed when parked, so
  // the loads are unconditional and nothing waits for them before the K/V
  // loads go out.
  int lim[NT];
  bf16x8_t qv[NT][4];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int n = nt * 16 + m16;
    const int nn = n < rows ? n : 0;
    const int j = j0 + nn / p.group, hh = nn % p.group;
    const uint16_t* qp = p.q + static_cast<int64_t>(q_start + j) * p.q_row_stride +
                         static_cast<int64_t>(kvh * p.group + hh) * p.q_head_stride;
#pragma unroll
    for (int s = 0; s < 4; ++s) qv[nt][s] = *reinterpret_cast<const bf16x8_t*>(qp + 32 * s + 8 * g);
    const int c = L - q_len + j;
    lim[nt] = n < rows ? (c < L - 1 ? c : L - 1) : -1;
  }

  float m_run[NT], l_run[NT];
  f32x4_t acc[NT][8];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    m_run[nt] = -INFINITY;
    l_run[nt] = 0.0f;
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[nt][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  const int nchunks = (kv_end - kv_begin + kChunk - 1) / kChunk;
  constexpr int64_t esz = FP8 ? 1 : 2;

  // lane i of lane_blk holds the id of logical block first_blk + i: one
  // load for the split instead of a dependent load per chunk
  const int first_blk = kv_begin / p.block_size;

  // Raw K/V registers of one 32-key chunk (bf16: K 2x4 and V 8 16-byte
  // vectors per lane; FP8: K 2x4 8-byte and V 4 16-byte vectors).
  struct Chunk {
    uint4 k[2][4];
    uint4 v[8];
    int kb;        // first key of the chunk
    bool valid;    // block id in range; otherwise the chunk's keys are masked
  };

  // Loop-invariant byte offsets of this lane's loads inside one (block, kv
  // head) tile of 32 tokens; a chunk only builds two buffer descriptors
  // (uniform), so no per-chunk address arithmetic runs on the vector ALUs.
  //   K: key (16*kt + m16), d 32*s + 8*g .. +7   (s through the immediate offset)
  //   V: bf16 row (4*i + g), d 8*m16 .. +7; FP8 row (8*i + lane/8), bytes 16*(lane%8)
  const uint32_t tokb = static_cast<uint32_t>(p.tok_stride * esz);
  uint32_t koff[2], voff[8];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) koff[kt] = (kt * 16 + m16) * tokb + 8 * g * esz;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    voff[i] = FP8 ? (8 * i + (lane >> 3)) * tokb + (lane & 7) * 16 : (4 * i + g) * tokb + m16 * 16;

  // Issue the loads of chunk c (no waits: the data is consumed by
  // compute_chunk one chunk later, so each load's latency overlaps the
  // previous chunk's math).  The descriptors' record count ends at the last
  // visible key, so rows past the sequence end (and every row of an invalid
  // block) read as zeros instead of stale cache contents.  V loads (whole
  // 128-byte lines per instruction) carry the non-temporal hint.  K loaded
  // straight into operand order reads half lines per instruction (the
  // other half one instruction later), where the hint costs time: measured
  // on the Qwen3-8B bench shapes, no hint 63.5 us per call, both 61.3, K
  // only 63.7, V only 59.3; FP8 config 4: 486 -> 442 us.  Staged K (KST)
  // loads as V does, whole lines with the hint: config 3 56.4 -> 55.2 us,
  // FP8 config 4 430.6 -> 414 us.  Issuing the next chunk's loads as soon
  // as the staging frees the registers (before this chunk's math) ran
  // slower, 55.2 -> 56.1 us: more requests in flight per CU, less DRAM
  // efficiency.
  auto load_chunk = [&](int c, Chunk& ch) {
    const int kb = kv_begin + c * kChunk;
    ch.kb = kb;
    // the host keeps a split within kWave blocks, so the id is always in a lane
    const int raw = __builtin_amdgcn_readlane(lane_blk, kb / p.block_size - first_blk);
    ch.valid = raw >= 0 && raw < p.num_blocks;
    const int pblk = ch.valid ? raw : 0;
    const int visible = kv_limit - kb < kChunk ? kv_limit - kb : kChunk;
    const int nrec = ch.valid ? visible * static_cast<int>(tokb) : 0;
    const int64_t tile = (static_cast<int64_t>(pblk) * p.blk_stride +
                          static_cast<int64_t>(kvh) * p.head_stride +
                          static_cast<int64_t>(kb % p.block_size) * p.tok_stride) * esz;
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(p.k_cache + tile, nrec);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(p.v_cache + tile, nrec);
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        if (KST && FP8) {
          // whole lines, as V: FP8 row 8 s + lane / 8, bytes 16 (lane % 8) .. +15
          if (kt == 0)
            ch.k[0][s] = __builtin_bit_cast(
                uint4, __builtin_amdgcn_raw_buffer_load_b128(kr, voff[s], 0, kLoadStreamed));
        } else if (FP8) {
          const uint2 w = __builtin_bit_cast(
              uint2,
              __builtin_amdgcn_raw_buffer_load_b64(kr, koff[kt] + 32 * s, 0, 0));
          ch.k[kt][s] = make_uint4(w.x, w.y, 0, 0);
        } else if (KST) {
          // whole lines, as V: row 4 (4 kt + s) + g, bytes 16 m16 .. +15
          ch.k[kt][s] = __builtin_bit_cast(
              uint4,
              __builtin_amdgcn_raw_buffer_load_b128(kr, voff[4 * kt + s], 0, kLoadStreamed));
        } else {
          ch.k[kt][s] = __builtin_bit_cast(
              uint4,
              __builtin_amdgcn_raw_buffer_load_b128(kr, koff[kt] + 64 * s, 0, 0));
        }
      }
    }
#pragma unroll
    for (int i = 0; i < (FP8 ? 4 : 8); ++i)
      ch.v[i] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(vr, voff[i], 0, kLoadStreamed));
  };

  auto compute_chunk = [&](const Chunk& ch) {
    if (!ch.valid) return;
    const int kb = ch.kb;
    // ---- V rows into the wave's LDS stage.  The stage belongs to this wave
    // alone and LDS executes a wave's operations in order, so a compiler
    // barrier plus an LDS wait (before the first read) orders them.
    if (FP8) {
      // Lane l stages 16 values of row 8 i + l / 8 as two 16-byte halves
      // at dwords 8 (l % 8) and + 4.  A 16-byte LDS store serves eight
      // lanes per cycle over 32 four-byte banks, so if every lane stored
      // its first half first, lanes l and l + 4 would share a bank group
      // (2-way conflicts on every store).  Lanes 4-7 of each eight store
      // their second half first: each store's eight lanes then cover all
      // 32 banks.
      const bool swap = (lane >> 2) & 1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 8 * i + (lane >> 3);
        uint32_t* dst = stage + row * kVPitch + (lane & 7) * 8;
        const uint2 lo = make_uint2(ch.v[i].x, ch.v[i].y), hi = make_uint2(ch.v[i].z, ch.v[i].w);
        *reinterpret_cast<bf16x8_t*>(dst + (swap ? 4 : 0)) = fp8x8_to_bf16(swap ? hi : lo);
        *reinterpret_cast<bf16x8_t*>(dst + (swap ? 0 : 4)) = fp8x8_to_bf16(swap ? lo : hi);
      }
      if (KST) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = 8 * i + (lane >> 3);
          const int c0 = 2 * (lane & 7);
          const uint4 k = ch.k[0][i];
          const uint2 lo = make_uint2(k.x, k.y), hi = make_uint2(k.z, k.w);
          *reinterpret_cast<bf16x8_t*>(kstage + kst_slot(row, c0 + (swap ? 1 : 0))) =
              fp8x8_to_bf16(swap ? hi : lo);
          *reinterpret_cast<bf16x8_t*>(kstage + kst_slot(row, c0 + (swap ? 0 : 1))) =
              fp8x8_to_bf16(swap ? lo : hi);
        }
        lds_wave_sync();
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        *reinterpret_cast<uint4*>(stage + (4 * i + g) * kVPitch + m16 * 4) = ch.v[i];
      if (KST) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          *reinterpret_cast<uint4*>(kstage + kst_slot(4 * i + g, m16)) = ch.k[i / 4][i % 4];
        lds_wave_sync();
      }
    }

    // ---- S^T = K . Q^T: per head_dim slice s, every (key tile, query
    // tile) pair; the query operands come from LDS one slice at a time
    f32x4_t sacc[2][NT];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) sacc[kt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      bf16x8_t kop[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        if (KST)  // key 16 kt + m16, head_dim 32 s + 8 g .. +7 (the Q operands' order)
          kop[kt] = *reinterpret_cast<const bf16x8_t*>(kstage + kst_slot(16 * kt + m16, 4 * s + g));
        else
          kop[kt] = FP8 ? fp8x8_to_bf16(make_uint2(ch.k[kt][s].x, ch.k[kt][s].y))
                        : __builtin_bit_cast(bf16x8_t, ch.k[kt][s]);
      }
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const bf16x8_t qo = qst[(nt * 4 + s) * kWave + lane];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) sacc[kt][nt] = mfma(kop[kt], qo, sacc[kt][nt]);
      }
    }

    // ---- online softmax (per query column; lanes l, l^16, l^32, l^48 share one).
    // Scores stay raw (the scale is folded into the exp2 argument); the
    // running max m_run (scaled, log2 domain) is only raised when a column's
    // new max exceeds it by more than kRescaleSlack, so the accumulator
    // rescale is skipped for most chunks: probabilities stay <= 2^kRescaleSlack.
    // Only a chunk that reaches past some column's causal limit (or the
    // sequence end) is masked, behind a uniform branch: written as a select
    // per score, the compare and select ran on every chunk (40 VALU
    // instructions of ~170 per chunk).
    const bool full = kb + kChunk - 1 <= L - q_len + j0 && kb + kChunk <= kv_limit;
    if (!full) {
      const int rel = kb + 4 * g;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (rel + kt * 16 + i > lim[nt]) sacc[kt][nt][i] = -INFINITY;
    }
    bf16x8_t pb[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      float sv[8];
      float cmax = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v = sacc[kt][nt][i];
          sv[kt * 4 + i] = v;
          cmax = fmaxf(cmax, v);
        }
      }
      cmax = max_xor16(cmax);
      cmax = max_xor32(cmax);
      cmax *= sl2;
      const bool need = cmax > m_run[nt] + kRescaleSlack;
      if (__any(need)) {
        const float m_new = need ? cmax : m_run[nt];
        const float alpha = need ? exp2f_fast(m_run[nt] - m_new) : 1.0f;
        l_run[nt] *= alpha;
        m_run[nt] = m_new;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[nt][t][i] *= alpha;
        }
      }
      const float msub = m_run[nt] == -INFINITY ? 0.0f : m_run[nt];
      float psum = 0.0f;
      f32x2_t pv[4];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float e = exp2f_fast(__builtin_fmaf(sv[k], sl2, -msub));
        pv[k >> 1][k & 1] = e;
        psum += e;
      }
      l_run[nt] += psum;
      uint4 pk;
      pk.x = __builtin_bit_cast(uint32_t, __builtin_convertvector(pv[0], bf16x2_t));
      pk.y = __builtin_bit_cast(uint32_t, __builtin_convertvector(pv[1], bf16x2_t));
      pk.z = __builtin_bit_cast(uint32_t, __builtin_convertvector(pv[2], bf16x2_t));
      pk.w = __builtin_bit_cast(uint32_t, __builtin_convertvector(pv[3], bf16x2_t));
      pb[nt] = __builtin_bit_cast(bf16x8_t, pk);
    }

    lds_wave_sync();

    // ---- O^T += V^T . P^T ; pair pp covers d = 32*pp + 2*m + {0 (even tile), 1 (odd tile)}
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      uint32_t w[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int key = (j < 4) ? (4 * g + j) : (16 + 4 * g + (j - 4));
        w[j] = stage[key * kVPitch + 16 * pp + m16];
      }
      uint4 ev, od;
      ev.x = __builtin_amdgcn_perm(w[1], w[0], 0x05040100u);
      ev.y = __builtin_amdgcn_perm(w[3], w[2], 0x05040100u);
      ev.z = __builtin_amdgcn_perm(w[5], w[4], 0x05040100u);
      ev.w = __builtin_amdgcn_perm(w[7], w[6], 0x05040100u);
      od.x = __builtin_amdgcn_perm(w[1], w[0], 0x07060302u);
      od.y = __builtin_amdgcn_perm(w[3], w[2], 0x07060302u);
      od.z = __builtin_amdgcn_perm(w[5], w[4], 0x07060302u);
      od.w = __builtin_amdgcn_perm(w[7], w[6], 0x07060302u);
      const bf16x8_t ea = __builtin_bit_cast(bf16x8_t, ev);
      const bf16x8_t oa = __builtin_bit_cast(bf16x8_t, od);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        acc[nt][2 * pp] = mfma(ea, pb[nt], acc[nt][2 * pp]);
        acc[nt][2 * pp + 1] = mfma(oa, pb[nt], acc[nt][2 * pp + 1]);
      }
    }
    // the next chunk overwrites the stage: its reads must be done first
    lds_wave_sync();
  };

  // The wave's first chunk is requested before the query operands are
  // parked, so its latency overlaps the parking and the barrier (a barrier
  // waits for LDS operations only, not for outstanding loads).
  Chunk ca;
  if (PIPE || wv < nchunks) load_chunk(PIPE ? 0 : wv, ca);
  __builtin_amdgcn_sched_barrier(0);
  if (wv == 0) {
    const bf16x8_t zero = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int s = 0; s < 4; ++s) qst[(nt * 4 + s) * kWave + lane] = nt * 16 + m16 < rows ? qv[nt][s] : zero;
  }
  if constexpr (WPS > 1) __syncthreads(); else lds_wave_sync();

  // Two register buffers, unrolled by two so that no buffer is copied: the
  // loads of chunk c+1 are issued before chunk c is computed.  The
  // scheduling barriers keep the compiler from sinking them to their use.
  // Every load is unconditional (past the end the last chunk is loaded
  // again, from L2) so the compiler's wait counts only ever wait for the
  // older buffer.
  if constexpr (PIPE) {
    Chunk cb;
    const int last = nchunks - 1;
    int c = 0;
    for (; c < last; c += 2) {
      load_chunk(c + 1, cb);
      __builtin_amdgcn_sched_barrier(0);
      compute_chunk(ca);
      load_chunk(c + 2 < last ? c + 2 : last, ca);
      __builtin_amdgcn_sched_barrier(0);
      compute_chunk(cb);
    }
    if (c == last) compute_chunk(ca);
  } else {
    // one buffer: other resident waves on the SIMD hide the latency
    for (int c = wv; c < nchunks; c += WPS) {
      compute_chunk(ca);
      if (c + WPS < nchunks) load_chunk(c + WPS, ca);
    }
  }

  if constexpr (WPS > 1) {
    // ---- shared segment: every wave parks its (max, sum, accumulator)
    // state, half per column tile: tile 0 in its own V stage (free once its
    // loop is done), tile 1 in a second bank of WPS stages that no loop
    // touches, so no barrier is needed before parking.  After one barrier
    // the NT * 4 items (column tile nt, head_dim columns 32 pp .. 32 pp + 31)
    // are dealt to the waves in turn; each folds the WPS states of its item
    // in wave order (deterministic) and writes them straight from registers:
    // lane (g, m16) holds 8 consecutive values of query column m16.
    constexpr int kAccWords = 8 * kWave * 4;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      float* mine = reinterpret_cast<float*>(vst + (nt * WPS + wv) * kVStage);
#pragma unroll
      for (int t = 0; t < 8; ++t) reinterpret_cast<f32x4_t*>(mine)[t * kWave + lane] = acc[nt][t];
      mine[kAccWords + lane] = m_run[nt];
      mine[kAccWords + kWave + lane] = l_run[nt];
    }
    __syncthreads();
    // NT * 4 (column tile, 32-wide head_dim group) items, one per wave
    // where there are enough waves
    for (int it = wv; it < NT * 4; it += WPS) {
      const int nt = it / 4, pp = it % 4;
      const float* st[WPS];
      float fw[WPS];
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < WPS; ++w) {
        st[w] = reinterpret_cast<const float*>(vst + (nt * WPS + w) * kVStage);
        fw[w] = st[w][kAccWords + lane];
        M = fmaxf(M, fw[w]);
      }
      float lsum = 0.0f;
#pragma unroll
      for (int w = 0; w < WPS; ++w) {
        fw[w] = fw[w] == -INFINITY ? 0.0f : exp2f_fast(fw[w] - M);
        lsum += fw[w] * st[w][kAccWords + kWave + lane];
      }
      lsum = sum_xor16(lsum);
      lsum = sum_xor32(lsum);
      const float inv = lsum > 0.0f ? vscale / lsum : 0.0f;
      const int n = nt * 16 + m16;
      if (n < rows) {
        const int j = j0 + n / p.group, hh = n % p.group;
        const int tok = q_start + j;
        const int h = kvh * p.group + hh;
        const int64_t slot = (static_cast<int64_t>(tok) * p.hq + h) * p.max_splits + split;
        // tiles 2 pp (even d) and 2 pp + 1 (odd d): d = 32 pp + 8 g + 2 i + e
        float o[8];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          f32x4_t sum = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int w = 0; w < WPS; ++w) {
            const f32x4_t a = reinterpret_cast<const f32x4_t*>(st[w])[(2 * pp + e) * kWave + lane];
#pragma unroll
            for (int i = 0; i < 4; ++i) sum[i] += fw[w] * a[i];
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) o[2 * i + e] = sum[i] * inv;
        }
        const int d0 = 32 * pp + 8 * g;
        if (nsplit == 1) {
          uint16_t* op = p.out + static_cast<int64_t>(tok) * p.out_row_stride +
                         static_cast<int64_t>(h) * p.out_head_stride + d0;
          *reinterpret_cast<uint4*>(op) = make_uint4(pack_bf16(o[0], o[1]), pack_bf16(o[2], o[3]),
                                                     pack_bf16(o[4], o[5]), pack_bf16(o[6], o[7]));
        } else {
          float* wo = p.ws_o + slot * kD + d0;
          *reinterpret_cast<float4*>(wo) = make_float4(o[0], o[1], o[2], o[3]);
          *reinterpret_cast<float4*>(wo + 4) = make_float4(o[4], o[5], o[6], o[7]);
          // log-sum-exp (log2 domain) of the column for combine_kernel
          if (pp == 0 && g == 0) p.ws_lse[slot] = lsum > 0.0f ? M + __log2f(lsum) : -INFINITY;
        }
      }
    }
    return;
  }

  // ---- finish (one wave): per column sum, then straight from registers:
  // lane (g, m16) holds d = 32 pp + 8 g + 0..7 of query column m16 in the
  // tiles 2 pp (even d) and 2 pp + 1 (odd d)
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    float lsum = l_run[nt];
    lsum = sum_xor16(lsum);
    lsum = sum_xor32(lsum);
    const float inv = lsum > 0.0f ? vscale / lsum : 0.0f;
    const int n = nt * 16 + m16;
    if (n < rows) {
      const int j = j0 + n / p.group, hh = n % p.group;
      const int tok = q_start + j;
      const int h = kvh * p.group + hh;
      const int64_t slot = (static_cast<int64_t>(tok) * p.hq + h) * p.max_splits + split;
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        float o[8];
#pragma unroll
        for (int e = 0; e < 2; ++e)
#pragma unroll
          for (int i = 0; i < 4; ++i) o[2 * i + e] = acc[nt][2 * pp + e][i] * inv;
        const int d0 = 32 * pp + 8 * g;
        if (nsplit == 1) {
          uint16_t* op = p.out + static_cast<int64_t>(tok) * p.out_row_stride +
                         static_cast<int64_t>(h) * p.out_head_stride + d0;
          *reinterpret_cast<uint4*>(op) = make_uint4(pack_bf16(o[0], o[1]), pack_bf16(o[2], o[3]),
                                                     pack_bf16(o[4], o[5]), pack_bf16(o[6], o[7]));
        } else {
          float* wo = p.ws_o + slot * kD + d0;
          *reinterpret_cast<float4*>(wo) = make_float4(o[0], o[1], o[2], o[3]);
          *reinterpret_cast<float4*>(wo + 4) = make_float4(o[4], o[5], o[6], o[7]);
        }
      }
      // log-sum-exp (log2 domain) of the column for combine_kernel
      if (nsplit > 1 && g == 0) p.ws_lse[slot] = lsum > 0.0f ? m_run[nt] + __log2f(lsum) : -INFINITY;
    }
  }
}

// zero the output rows of a query tile that sees no keys
__device__ __forceinline__ void zero_tile(const AttnParams& p, int kvh, int seq, int qt) {
  int q_start, q_len, L;
  seq_geometry(p, seq, q_start, q_len, L);
  const int j0 = qt * p.qtile;
  const int jn = (q_len - j0 < p.qtile) ? q_len - j0 : p.qtile;
  for (int idx = threadIdx.x; idx < jn * p.group * (kD / 8); idx += blockDim.x) {
    const int n = idx / (kD / 8), dv = idx % (kD / 8);
    const int j = j0 + n / p.group, hh = n % p.group;
    uint16_t* o = p.out + static_cast<int64_t>(q_start + j) * p.out_row_stride +
                  static_cast<int64_t>(kvh * p.group + hh) * p.out_head_stride + dv * 8;
    *reinterpret_cast<uint4*>(o) = make_uint4(0, 0, 0, 0);
  }
}

// record the split count of a query tile's rows for combine_kernel (one
// writer per tile: the kv-head-0 workgroup that also owns split 0)
__device__ __forceinline__ void note_rows(const AttnParams& p, int seq, int qt, int nsplit) {
  int q_start, q_len, L;
  seq_geometry(p, seq, q_start, q_len, L);
  const int j0 = qt * p.qtile;
  const int jn = (q_len - j0 < p.qtile) ? q_len - j0 : p.qtile;
  for (int j = threadIdx.x; j < jn; j += blockDim.x) p.row_nsplit[q_start + j0 + j] = nsplit;
}

// Rows q_start + q_len .. q_start + q_raw - 1 of a sequence clipped to
// max_seqlen_q (cu_seqlens_q gave it more rows than the bound the grid was
// sized for) get zero output and split count 0, so that combine_kernel
// leaves them alone instead of merging a stale count left in the workspace
// by an earlier call.  Threads tid, tid + nthreads, ... share the stores.
__device__ void clear_clipped_rows(const AttnParams& p, int q_start, int q_len, int q_raw, int tid,
                                   int nthreads) {
  const int per_row = p.hq * (kD / 8);
  for (int t = q_start + q_len; t < q_start + q_raw; ++t) {
    uint16_t* row = p.out + static_cast<int64_t>(t) * p.out_row_stride;
    for (int i = tid; i < per_row; i += nthreads) {
      const int h = i / (kD / 8), c = i % (kD / 8);
      *reinterpret_cast<uint4*>(row + static_cast<int64_t>(h) * p.out_head_stride + c * 8) =
          make_uint4(0, 0, 0, 0);
    }
    if (p.row_nsplit && tid == 0) p.row_nsplit[t] = 0;
  }
}

// keys the single query tile of a sequence sees, in 32-key chunks (stream mode)
__device__ __forceinline__ int stream_chunks(const AttnParams& p, int seq) {
  int q_start, q_len, L;
  seq_geometry(p, seq, q_start, q_len, L);
  return (q_len > 0 && L > 0) ? (L + kChunk - 1) / kChunk : 0;
}

// Fixed decomposition, one wave per (kv head, sequence, query tile, split):
// used when a sequence has several query tiles (prefill).
// Dispatch order (x fastest): kv head, sequence, then (query tile, split)
// slowest, so every full split is dispatched before the shorter trailing
// splits and the empty splits that pad the grid come last.
// Two waves per SIMD fit the register budget of tiles up to 32 columns;
// 64-column tiles (NT = 4) need the full register file of one wave.
template <int NT, bool FP8, bool PIPE, int WPS>
__global__ void __launch_bounds__(kWave * WPS, NT >= 4 ? 1 : 2)
paged_attention_kernel(AttnParams p) {
  // WPS V stages, then WPS K stages where K is staged; shared segments park
  // their states in NT banks of WPS stages (the second bank is the K stages)
  __shared__ __attribute__((aligned(16))) uint32_t
      vst[kVStage * WPS * (k_staged(FP8, PIPE, WPS) ? 2 : (WPS > 1 && NT > 1 ? NT : 1))];
  __shared__ bf16x8_t qst[NT * 4 * kWave];
  const int kvh = blockIdx.x;
  const int row = blockIdx.y;
  const int seq = (p.pair_rows > 0 && row >= p.pair_rows) ? p.num_seqs - 1 - (row - p.pair_rows) : row;
  const int split = blockIdx.z % p.max_splits;
  const int qt = blockIdx.z / p.max_splits;
  const int kv_begin = split * p.split_len;
  const int lane_blk = split_block_ids(p, seq, kv_begin);
  int q_start, q_len, L, q_raw;
  seq_geometry_uniform(p, seq, q_start, q_len, L, &q_raw);
  const int j0 = qt * p.qtile;
  const int jn = (q_len - j0 < p.qtile) ? q_len - j0 : p.qtile;
  const int kv_limit = L - q_len + j0 + jn;  // meaningful when jn > 0
  const int nsplit = kv_limit > 0 ? (kv_limit + p.split_len - 1) / p.split_len : 0;
  const bool note = kvh == 0 && split == 0 && p.row_nsplit;
  // rows past max_seqlen_q, if any, are cleared by one workgroup
  const bool clip_owner = kvh == 0 && split == 0 && qt == p.n_qtiles - 1 && q_raw > q_len;
  // one branch on the whole geometry, so every geometry load is issued
  // before the first wait
  if (jn <= 0 || kv_begin >= kv_limit) {
    if (jn > 0) {
      if (note) note_rows(p, seq, qt, nsplit);
      if (kv_limit <= 0 && split == 0) zero_tile(p, kvh, seq, qt);
    }
    if (clip_owner) clear_clipped_rows(p, q_start, q_len, q_raw, threadIdx.x, blockDim.x);
    return;
  }
  if (note) note_rows(p, seq, qt, nsplit);
  const int kv_end = kv_begin + p.split_len < kv_limit ? kv_begin + p.split_len : kv_limit;
  attend_segment<NT, FP8, PIPE, WPS>(p, vst, qst, kvh, seq, qt, q_start, q_len, L, kv_begin, kv_end,
                                     split, nsplit, lane_blk);
  if (clip_owner) clear_clipped_rows(p, q_start, q_len, q_raw, threadIdx.x, blockDim.x);
}

// ---------------------------------------------------------------- shared-tile kernel
// Tiles of 33-64 rows (64-row verify tiles of GQA group 8 with k = 7, and the
// prefill tiles of every geometry): WPT waves share one segment (kv head,
// sequence, query tile, key split), wave w owning the NTW = 4 / WPT column
// tiles 16 NTW w .. of the 64 query columns over every key of the split,
// so each wave finishes its own columns and nothing is merged.
//   * The workgroup loads each 32-key chunk once, cooperatively: thread t
//     takes the 16-byte granules t, t + WPT * 64, ... of the chunk's 8 KiB
//     of K rows and 8 KiB of V rows (eight lanes cover a 128-byte line), D
//     chunks ahead of the one being computed, into registers.  That keeps
//     D * 16 KiB in flight per workgroup where one wave per SIMD holding
//     all 64 columns' accumulators had room for one chunk ahead.
//   * A chunk's registers are written to one of two LDS slots (K rows of 68
//     dwords, conflict-free for the 16-byte writes and K operand reads, then
//     V rows of 72 dwords for the transpose loads), and one barrier per
//     chunk publishes it and frees the other slot.
//   * The query operands stay in registers (NTW column tiles per wave); the
//     S^T, softmax and O^T steps are attend_segment's, per wave.
// The loads of chunks past the end use an empty descriptor (zeros, no
// memory traffic), so every step of the D-unrolled loop issues the same
// loads and the compiler's waits only ever wait for the oldest buffer.
template <int WPT, int D>
__global__ void __launch_bounds__(kWave * WPT, 2)
paged_attention_tile_kernel(AttnParams p) {
  constexpr int NTW = 4 / WPT;
  constexpr int kThreads = kWave * WPT;
  constexpr int kRowGran = kD * 2 / 16;                  // 16-byte granules per K or V row
  constexpr int kHalf = kChunk * kRowGran / kThreads;    // per thread per chunk, of K (and of V)
  constexpr int kTileVPitch = 72;                        // dwords per staged V row (transpose loads)
  constexpr int kSlot = kChunk * (kVPitch + kTileVPitch); // dwords: K rows, then V rows
  static_assert(WPT == 2 || WPT == 4, "two or four waves per 64-row tile");
  __shared__ __attribute__((aligned(16))) uint32_t slots[2 * kSlot];

  const int kvh = blockIdx.x;
  const int seq = blockIdx.y;
  const int split = blockIdx.z % p.max_splits;
  const int qt = blockIdx.z / p.max_splits;
  const int kv_begin = split * p.split_len;
  const int lane_blk = split_block_ids(p, seq, kv_begin);
  int q_start, q_len, L, q_raw;
  seq_geometry_uniform(p, seq, q_start, q_len, L, &q_raw);
  const int j0 = qt * p.qtile;
  const int jn = (q_len - j0 < p.qtile) ? q_len - j0 : p.qtile;
  const int kv_limit = L - q_len + j0 + jn;  // meaningful when jn > 0
  const int nsplit = kv_limit > 0 ? (kv_limit + p.split_len - 1) / p.split_len : 0;
  const bool note = kvh == 0 && split == 0 && p.row_nsplit;
  const bool clip_owner = kvh == 0 && split == 0 && qt == p.n_qtiles - 1 && q_raw > q_len;
  if (jn <= 0 || kv_begin >= kv_limit) {
    if (jn > 0) {
      if (note) note_rows(p, seq, qt, nsplit);
      if (kv_limit <= 0 && split == 0) zero_tile(p, kvh, seq, qt);
    }
    if (clip_owner) clear_clipped_rows(p, q_start, q_len, q_raw, threadIdx.x, blockDim.x);
    return;
  }
  if (note) note_rows(p, seq, qt, nsplit);
  const int kv_end = kv_begin + p.split_len < kv_limit ? kv_begin + p.split_len : kv_limit;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wv = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int g = lane >> 4;
  const int m16 = lane & 15;
  const int rows = jn * p.group;
  const float sl2 = p.scale_log2;

  // ---- this wave's query operands (padding columns zero) and causal limits
  int lim[NTW];
  bf16x8_t qv[NTW][4];
#pragma unroll
  for (int nt = 0; nt < NTW; ++nt) {
    const int n = (wv * NTW + nt) * 16 + m16;
    const int nn = n < rows ? n : 0;
    const int j = j0 + nn / p.group, hh = nn % p.group;
    const uint16_t* qp = p.q + static_cast<int64_t>(q_start + j) * p.q_row_stride +
                         static_cast<int64_t>(kvh * p.group + hh) * p.q_head_stride;
#pragma unroll
    for (int s = 0; s < 4; ++s) qv[nt][s] = *reinterpret_cast<const bf16x8_t*>(qp + 32 * s + 8 * g);
    const int c = L - q_len + j;
    lim[nt] = n < rows ? (c < L - 1 ? c : L - 1) : -1;
  }

  const int nchunks = (kv_end - kv_begin + kChunk - 1) / kChunk;
  const int first_blk = kv_begin / p.block_size;
  const uint32_t tokb = static_cast<uint32_t>(p.tok_stride * 2);
  // granule i of this thread: row (tid + i * kThreads) / 16, column % 16
  uint32_t goff[kHalf], loff[kHalf], vloff[kHalf];
#pragma unroll
  for (int i = 0; i < kHalf; ++i) {
    const int gi = tid + i * kThreads;
    goff[i] = static_cast<uint32_t>(gi / kRowGran) * tokb + (gi % kRowGran) * 16;
    loff[i] = static_cast<uint32_t>(gi / kRowGran) * kVPitch + (gi % kRowGran) * 4;
    vloff[i] = static_cast<uint32_t>(gi / kRowGran) * kTileVPitch + (gi % kRowGran) * 4;
  }

  // chunk c's block id (uniform), in range or not
  auto chunk_block = [&](int c) {
    const int kb = kv_begin + c * kChunk;
    return __builtin_amdgcn_readlane(lane_blk, kb / p.block_size - first_blk);
  };
  auto load_chunk = [&](int c, uint4 (&r)[2 * kHalf]) {
    const bool live = c < nchunks;
    const int cc = live ? c : nchunks - 1;
    const int kb = kv_begin + cc * kChunk;
    const int raw = chunk_block(cc);
    const bool valid = live && raw >= 0 && raw < p.num_blocks;
    const int visible = kv_limit - kb < kChunk ? kv_limit - kb : kChunk;
    const int nrec = valid ? visible * static_cast<int>(tokb) : 0;
    const int64_t tile = (static_cast<int64_t>(valid ? raw : 0) * p.blk_stride +
                          static_cast<int64_t>(kvh) * p.head_stride +
                          static_cast<int64_t>(kb % p.block_size) * p.tok_stride) * 2;
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(p.k_cache + tile, nrec);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(p.v_cache + tile, nrec);
#pragma unroll
    for (int i = 0; i < kHalf; ++i)
      r[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(kr, goff[i], 0,
                                                                             kLoadStreamed));
#pragma unroll
    for (int i = 0; i < kHalf; ++i)
      r[kHalf + i] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(vr, goff[i], 0, kLoadStreamed));
  };
  auto stage = [&](const uint4 (&r)[2 * kHalf], int slot) {
    uint32_t* kst = slots + slot * kSlot;
#pragma unroll
    for (int i = 0; i < kHalf; ++i) *reinterpret_cast<uint4*>(kst + loff[i]) = r[i];
#pragma unroll
    for (int i = 0; i < kHalf; ++i)
      *reinterpret_cast<uint4*>(kst + kChunk * kVPitch + vloff[i]) = r[kHalf + i];
  };

  float m_run[NTW], l_run[NTW];
  f32x4_t acc[NTW][8];
#pragma unroll
  for (int nt = 0; nt < NTW; ++nt) {
    m_run[nt] = -INFINITY;
    l_run[nt] = 0.0f;
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[nt][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  auto compute = [&](int c, int slot) {
    const int raw = chunk_block(c);
    if (raw < 0 || raw >= p.num_blocks) return;       // invalid block: its keys are masked
    const int kb = kv_begin + c * kChunk;
    const uint32_t* kst = slots + slot * kSlot;
    const uint32_t* vst = kst + kChunk * kVPitch;
    f32x4_t sacc[2][NTW];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) sacc[kt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      bf16x8_t kop[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
        kop[kt] = *reinterpret_cast<const bf16x8_t*>(kst + (16 * kt + m16) * kVPitch + 16 * s + 4 * g);
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) sacc[kt][nt] = mfma(kop[kt], qv[nt][s], sacc[kt][nt]);
    }
    // masked only past a causal limit, behind a uniform branch (as above)
    const bool full = kb + kChunk - 1 <= L - q_len + j0 && kb + kChunk <= kv_limit;
    if (!full) {
      const int rel = kb + 4 * g;
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (rel + kt * 16 + i > lim[nt]) sacc[kt][nt][i] = -INFINITY;
    }
    bf16x8_t pb[NTW];
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) {
      float sv[8];
      float cmax = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v = sacc[kt][nt][i];
          sv[kt * 4 + i] = v;
          cmax = fmaxf(cmax, v);
        }
      }
      cmax = max_xor16(cmax);
      cmax = max_xor32(cmax);
      cmax *= sl2;
      const bool need = cmax > m_run[nt] + kRescaleSlack;
      if (__any(need)) {
        const float m_new = need ? cmax : m_run[nt];
        const float alpha = need ? exp2f_fast(m_run[nt] - m_new) : 1.0f;
        l_run[nt] *= alpha;
        m_run[nt] = m_new;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[nt][t][i] *= alpha;
        }
      }
      const float msub = m_run[nt] == -INFINITY ? 0.0f : m_run[nt];
      float psum = 0.0f;
      f32x2_t pv[4];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float e = exp2f_fast(__builtin_fmaf(sv[k], sl2, -msub));
        pv[k >> 1][k & 1] = e;
        psum += e;
      }
      l_run[nt] += psum;
      uint4 pk;
      pk.x = __builtin_bit_cast(uint32_t, __builtin_convertvector(pv[0], bf16x2_t));
      pk.y = __builtin_bit_cast(uint32_t, __builtin_convertvector(pv[1], bf16x2_t));
      pk.z = __builtin_bit_cast(uint32_t, __builtin_convertvector(pv[2], bf16x2_t));
      pk.w = __builtin_bit_cast(uint32_t, __builtin_convertvector(pv[3], bf16x2_t));
      pb[nt] = __builtin_bit_cast(bf16x8_t, pk);
    }
    // O^T += V^T . P^T through the LDS transpose load (v_operand_tr): tile
    // (pp, hf) covers d = 32 pp + 8 (m / 4) + 4 hf + m % 4.  Against four
    // 4-byte reads and eight byte permutes per tile pair (the one-wave
    // segments' form), this removes 32 of the chunk's ~87 VALU instructions
    // per wave: config 5 417 -> 407 us per call, output bits unchanged.
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const bf16x8_t va = v_operand_tr(vst, kTileVPitch, lane, pp, hf);
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) acc[nt][2 * pp + hf] = mfma(va, pb[nt], acc[nt][2 * pp + hf]);
      }
    }
  };

  // ---- D chunks in flight in registers, two LDS slots: step c computes
  // chunk c from slot c & 1, stages chunk c + 1 (loaded D steps ago) into
  // the other slot, refills its registers with chunk c + 1 + D, and one
  // barrier publishes the staged chunk and frees slot c & 1.
  uint4 buf[D][2 * kHalf];
#pragma unroll
  for (int d = 0; d < D; ++d) load_chunk(d, buf[d]);
  stage(buf[0], 0);
  load_chunk(D, buf[0]);
  __syncthreads();
  for (int cb = 0; cb < nchunks; cb += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int c = cb + d;
      if (c < nchunks) compute(c, c & 1);
      const int nb = (d + 1) % D;          // a constant once the loop is unrolled
      stage(buf[nb], (c + 1) & 1);
      load_chunk(c + 1 + D, buf[nb]);
      __syncthreads();
    }
  }

  // ---- finish: this wave's columns, straight from registers (lane (g, m16)
  // holds d = 32 pp + 8 g + 0..7 of query column m16: d .. d + 3 in tile
  // 2 pp, d + 4 .. d + 7 in tile 2 pp + 1)
#pragma unroll
  for (int nt = 0; nt < NTW; ++nt) {
    float lsum = l_run[nt];
    lsum = sum_xor16(lsum);
    lsum = sum_xor32(lsum);
    const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    const int n = (wv * NTW + nt) * 16 + m16;
    if (n < rows) {
      const int j = j0 + n / p.group, hh = n % p.group;
      const int tok = q_start + j;
      const int h = kvh * p.group + hh;
      const int64_t slot = (static_cast<int64_t>(tok) * p.hq + h) * p.max_splits + split;
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        float o[8];
#pragma unroll
        for (int e = 0; e < 2; ++e)
#pragma unroll
          for (int i = 0; i < 4; ++i) o[4 * e + i] = acc[nt][2 * pp + e][i] * inv;
        const int d0 = 32 * pp + 8 * g;
        if (nsplit == 1) {
          uint16_t* op = p.out + static_cast<int64_t>(tok) * p.out_row_stride +
                         static_cast<int64_t>(h) * p.out_head_stride + d0;
          *reinterpret_cast<uint4*>(op) = make_uint4(pack_bf16(o[0], o[1]), pack_bf16(o[2], o[3]),
                                                     pack_bf16(o[4], o[5]), pack_bf16(o[6], o[7]));
        } else {
          float* wo = p.ws_o + slot * kD + d0;
          *reinterpret_cast<float4*>(wo) = make_float4(o[0], o[1], o[2], o[3]);
          *reinterpret_cast<float4*>(wo + 4) = make_float4(o[4], o[5], o[6], o[7]);
        }
      }
      if (nsplit > 1 && g == 0) p.ws_lse[slot] = lsum > 0.0f ? m_run[nt] + __log2f(lsum) : -INFINITY;
    }
  }
  if (clip_owner) clear_clipped_rows(p, q_start, q_len, q_raw, threadIdx.x, blockDim.x);
}

// Balanced ("stream") decomposition for one query tile per sequence (verify
// and decode).  For each kv head, the chunks of all sequences are laid end
// to end and cut into equal ranges of rc chunks; workgroup (kvh, r) takes
// ranges r, r + gridDim.y, ...  A range may cover the tail of one sequence
// and the head of the next, so every workgroup streams the same number of
// keys whatever the length mix, and no wave waits behind a long sequence.
// Sequence s's split index is its range index minus that of its first chunk.
template <int NT, bool FP8, bool PIPE>
__global__ void __launch_bounds__(kWave, PIPE ? 1 : 2)
paged_attention_stream_kernel(AttnParams p) {
  __shared__ __attribute__((aligned(16))) uint32_t vst[kVStage * (k_staged(FP8, PIPE, 1) ? 2 : 1)];
  __shared__ bf16x8_t qst[NT * 4 * kWave];
  __shared__ int pre[kMaxSeqGroups * kWave + 1];          // pre[s]: chunks of sequences < s
  const int kvh = blockIdx.x;
  const int lane = threadIdx.x;

  // exclusive prefix of the per-sequence chunk counts, one 64-sequence group
  // at a time (wave-wide inclusive scan plus the running carry)
  int carry = 0;
  if (lane == 0) pre[0] = 0;
  for (int base = 0; base < p.num_seqs; base += kWave) {
    int v = base + lane < p.num_seqs ? stream_chunks(p, base + lane) : 0;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int u = __shfl_up(v, d, kWave);
      if (lane >= d) v += u;
    }
    if (base + lane < p.num_seqs) pre[base + lane + 1] = carry + v;
    carry += __shfl(v, kWave - 1, kWave);
  }
  lds_wave_sync();
  // Every value that places a range is wave-uniform (a shuffle of one lane,
  // LDS entries read at one address); readfirstlane says so, so that the
  // K/V buffer descriptors built from them stay in scalar registers instead
  // of needing a waterfall loop around every load.
  const int total = __builtin_amdgcn_readfirstlane(carry);
  auto incl_of = [&](int s) { return __builtin_amdgcn_readfirstlane(pre[s + 1]); };
  const int rc_even = (total + static_cast<int>(gridDim.y) - 1) / static_cast<int>(gridDim.y);
  int rc = rc_even > p.min_range_chunks ? rc_even : p.min_range_chunks;
  rc = rc < p.max_range_chunks ? rc : p.max_range_chunks;

  if (blockIdx.y == 0) {
    // split count of every row for combine_kernel (one writer: kv head 0),
    // one sequence per lane
    if (kvh == 0 && p.row_nsplit) {
      for (int s = lane; s < p.num_seqs; s += kWave) {
        const int hi = pre[s + 1], lo = pre[s];
        const int ns = hi > lo ? (hi - 1) / rc - lo / rc + 1 : 0;
        int q_start, q_len, L, q_raw;
        seq_geometry(p, s, q_start, q_len, L, &q_raw);
        for (int j = 0; j < q_len; ++j) p.row_nsplit[q_start + j] = ns;
        // rows past max_seqlen_q: this lane alone clears them
        if (q_raw > q_len) clear_clipped_rows(p, q_start, q_len, q_raw, 0, 1);
      }
    }
    // sequences with no visible key get zero rows
    for (int s = 0; s < p.num_seqs; ++s) {
      if (pre[s + 1] != pre[s]) continue;
      int q_start, q_len, L;
      seq_geometry(p, s, q_start, q_len, L);
      if (q_len > 0) zero_tile(p, kvh, s, 0);
    }
  }

  for (int r = blockIdx.y; r * rc < total; r += gridDim.y) {
    const int start = r * rc;
    const int end = start + rc < total ? start + rc : total;
    // first sequence whose chunks reach past `start` (binary search on the
    // monotone prefix)
    int s = 0, hi_s = p.num_seqs - 1;
    while (s < hi_s) {
      const int mid = (s + hi_s) >> 1;
      if (incl_of(mid) <= start) s = mid + 1; else hi_s = mid;
    }
    for (; s < p.num_seqs; ++s) {
      const int hi = incl_of(s);
      const int lo = s > 0 ? incl_of(s - 1) : 0;
      if (lo >= end) break;
      if (hi <= start) continue;
      const int c0 = (start > lo ? start : lo) - lo;
      const int c1 = (end < hi ? end : hi) - lo;
      int q_start, q_len, L;
      seq_geometry_uniform(p, s, q_start, q_len, L);
      const int kv_limit = L;
      const int kv_begin = c0 * kChunk;
      const int kv_end = c1 * kChunk < kv_limit ? c1 * kChunk : kv_limit;
      const int split = r - lo / rc;
      const int nsplit = (hi - 1) / rc - lo / rc + 1;
      attend_segment<NT, FP8, PIPE, 1>(p, vst, qst, kvh, s, 0, q_start, q_len, L, kv_begin, kv_end,
                                       split, nsplit, split_block_ids(p, s, kv_begin));
    }
  }
}

// Merge split partials.  Workgroup (t, y) merges, for token row t, the
// 256 (head, 4-element) slices y*256 .. of the row; each thread owns one
// slice.  The attention kernel recorded each row's split count, so a row
// costs one dependent load before its partials; every thread issues the
// loads of up to kCombineBatch splits at once (partials are laid out
// [row][head][split][d]) and merges batches with a running log-sum-exp.
constexpr int kCombineBatch = 8;
__global__ void __launch_bounds__(kCombineThreads)
combine_kernel(AttnParams p) {
  const int t = blockIdx.x;
  const int tid = threadIdx.x;
  if (t >= p.num_tokens) return;
  // rows outside the batch's query range were not written by this call
  const int lo = p.cu_q ? p.cu_q[0] : 0;
  const int hi = p.cu_q ? p.cu_q[p.num_seqs] : p.num_seqs;
  int nsplit = p.row_nsplit[t];
  if (t < lo || t >= hi || nsplit <= 1) return;
  nsplit = nsplit < p.max_splits ? nsplit : p.max_splits;
  const int idx = blockIdx.y * kCombineThreads + tid;
  if (idx >= p.hq * (kD / 4)) return;
  const int h = idx / (kD / 4), d4 = idx % (kD / 4);
  const int64_t base = (static_cast<int64_t>(t) * p.hq + h) * p.max_splits;
  float M = -INFINITY, wsum = 0.0f;
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = 0; s0 < nsplit; s0 += kCombineBatch) {
    float lse[kCombineBatch];
    float4 v[kCombineBatch];
#pragma unroll
    for (int u = 0; u < kCombineBatch; ++u) {
      const bool in = s0 + u < nsplit;
      lse[u] = in ? p.ws_lse[base + s0 + u] : -INFINITY;
      v[u] = in ? *reinterpret_cast<const float4*>(p.ws_o + (base + s0 + u) * kD + 4 * d4)
                : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float mb = M;
#pragma unroll
    for (int u = 0; u < kCombineBatch; ++u) mb = fmaxf(mb, lse[u]);
    if (mb == -INFINITY) continue;
    const float r = M == -INFINITY ? 0.0f : exp2f_fast(M - mb);
    wsum *= r;
    o.x *= r; o.y *= r; o.z *= r; o.w *= r;
#pragma unroll
    for (int u = 0; u < kCombineBatch; ++u) {
      const float w = lse[u] == -INFINITY ? 0.0f : exp2f_fast(lse[u] - mb);
      wsum += w;
      o.x += w * v[u].x; o.y += w * v[u].y; o.z += w * v[u].z; o.w += w * v[u].w;
    }
    M = mb;
  }
  const float inv = wsum > 0.0f ? 1.0f / wsum : 0.0f;
  uint16_t* op = p.out + static_cast<int64_t>(t) * p.out_row_stride +
                 static_cast<int64_t>(h) * p.out_head_stride + 4 * d4;
  *reinterpret_cast<uint2*>(op) = make_uint2(pack_bf16(o.x * inv, o.y * inv), pack_bf16(o.z * inv, o.w * inv));
}

// query positions per workgroup: as many as fit 64 tile rows (>= 1)
int32_t choose_qtile(int32_t max_q, int32_t group) {
  int32_t qtile = group > 0 ? 64 / group : 1;
  qtile = qtile < 1 ? 1 : qtile;
  return max_q < qtile ? (max_q > 0 ? max_q : 1) : qtile;
}

// Compute units of the current device (cached per device; 256 when the
// query fails).
int32_t device_cus() {
  static int32_t cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

// Split length of the fixed decomposition.  A segment is one (sequence, kv
// head, query tile); `waves` waves share each split.
//   * Eight waves per split (bf16 tiles of up to 32 rows): 352 keys per
//     wave, 2816 per split; when the batch has at least four segments per
//     CU (several rounds of workgroups, which the dispatcher balances), one
//     split covers the whole sequence instead (no fp32 partials, no
//     combine, each workgroup streams longer).
//   * One wave per split (64-row tiles, FP8 tiles off the stream path):
//     3072 keys; with at least one segment per SIMD, about three quarters of
//     the longest sequence (a multiple of 1024), so that only the longest
//     sequences split in two: fewer, longer waves, while the trailing
//     splits still fill in behind the first round.
// Measured on MI355X (bench.py --kernels, NVA_ATTN_SPLIT_KEYS sweeps in one
// run): Qwen3-32B verify (64-row tiles, keys 2-8k) 521 us at 3072, 545 at
// 4096, 484-487 at 6144, 590 at 8192 (one round of unequal waves); Qwen3-32B
// draft decode (8-row tiles, 1024 segments) 431 us at 3072, 414 whole;
// Qwen3-0.6B verify (256 segments, one round, keys 512-4096) 58.0-58.3 us
// at 2688, 58.4-58.5 at 2816, 59.6 at 2560, 60.1-60.9 at 3072, 61.5-62.4 at
// 2304, 64.4 at 2048, 64.3 whole: in one round the split balances the
// longest first splits against a short sequence plus the longest second
// split, each workgroup's start-up worth ~340 keys of streaming.  With K
// staged through LDS (two alternating sweeps on one box): 55.2-55.3 at
// 2816, 55.6-55.7 at 2944, 55.8-55.9 at 2688, 56.5 at 2560 and at 3072,
// 56.6 at 2432.  The length shrinks in 128-key steps (to a 128-key
// minimum) only while fewer than kMinWaves waves would be launched, and is
// capped so that a split spans at most kWave - 2 blocks of block_size tokens
// (the kernel holds one block id per lane); block_size 0 (unknown: the
// workspace query) assumes the smallest block, kChunk tokens, which bounds
// the split count from above.
void choose_split(int32_t num_seqs, int32_t num_kv_heads, int32_t n_qtiles, int32_t max_k,
                  int32_t waves, int32_t block_size, int32_t* split_len, int32_t* max_splits) {
  const int64_t segs = static_cast<int64_t>(num_seqs > 0 ? num_seqs : 1) *
                       (num_kv_heads > 0 ? num_kv_heads : 1) * (n_qtiles > 0 ? n_qtiles : 1);
  const int64_t base = segs * (waves > 0 ? waves : 1);
  const int32_t mk = max_k > 1 ? max_k : 1;
  const int32_t cus = device_cus();
  int32_t len;
  if (waves > 1) {
    len = kKeysPerSharedWave * waves;
    const int32_t whole = (mk + kMinSplit - 1) / kMinSplit * kMinSplit;
    if (segs >= 4 * static_cast<int64_t>(cus) && whole > len) len = whole;
  } else {
    len = kSplitKeys;
    const int32_t most = 3 * (mk / 4) / 1024 * 1024;
    if (segs >= 4 * static_cast<int64_t>(cus) && most > len) len = most;
  }
  const int32_t span = (kWave - 2) * (block_size > 0 ? block_size : kChunk);
  if (len > span) len = span / kMinSplit * kMinSplit;
  while (len > kMinSplit && base * ((mk + len - 1) / len) < kMinWaves) len -= kMinSplit;
  // NVA_ATTN_SPLIT_KEYS (a multiple of 128) fixes the split length for tuning
  static const int32_t forced = [] {
    const char* v = getenv("NVA_ATTN_SPLIT_KEYS");
    const int32_t f = v ? atoi(v) : 0;
    return (f > 0 && f % kMinSplit == 0) ? f : 0;
  }();
  if (forced) len = forced;
  *split_len = len;
  *max_splits = (mk + len - 1) / len;
}

// Stream decomposition applies when every sequence is a single query tile
// of at most 32 rows (64-row tiles need the whole register file for the
// fixed decomposition's state already).
// Decomposition and pipelining per tile shape, from measurements on MI355X
// (Qwen3-0.6B/8B/32B verify and draft-decode shapes, longest-first batches):
//   * up to 32 rows, bf16: fixed decomposition, one chunk buffer, eight waves
//     per workgroup sharing each split (their states merged in LDS), two
//     waves per SIMD hiding each other's latency.  This beat the stream
//     decomposition for 4- and 10-row tiles too (draft decode 80.8 -> 70.7
//     us, Qwen3-0.6B verify 74.4 -> 65.1 us).  Single tiles of 17-32 rows
//     at one to two segments per CU run paired mode instead (paired_mode);
//   * single-tile sequences of up to 32 rows, FP8: stream decomposition with
//     the chunk loads issued one chunk ahead (502 us against 573 us fixed);
//   * bf16 64-row tiles: the shared-tile kernel, four waves per tile with
//     every chunk loaded once per workgroup and four chunks in flight
//     (Qwen3-32B verify, config 5's shapes: 425-428 us against 477 us for
//     one wave per SIMD holding all 64 columns and one chunk ahead, when
//     three chunks were in flight; four then took 441 us at 171 VGPRs, two
//     waves per SIMD instead of three; with V through the LDS transpose
//     load the kernel holds 151 / 160 VGPRs at three / four chunks, three
//     waves per SIMD either way, and four chunks run 404-405 against 407 us;
//     two waves per tile 432 us);
//   * FP8 64-row tiles: fixed decomposition with the loads one chunk ahead
//     (one wave per SIMD for 64 rows: no room for a second).
// NVA_ATTN_STREAM=0/1 (1: also bf16 tiles of up to 16 rows) and
// NVA_ATTN_PIPE=0/1 override the choices (tuning).
int env_choice(const char* name) {
  const char* v = getenv(name);
  return v ? (atoi(v) != 0) : -1;
}

bool stream_mode(int32_t num_seqs, int32_t max_q, int32_t qtile, int32_t group, bool fp8) {
  static const int forced = env_choice("NVA_ATTN_STREAM");
  if (forced == 0 || max_q > qtile || num_seqs > kMaxSeqGroups * kWave) return false;
  if (forced == 1) return max_q * group <= (fp8 ? 32 : 16);
  return fp8 && max_q * group <= 32;
}

bool pipelined(int nt, bool fp8) {
  static const int forced = env_choice("NVA_ATTN_PIPE");
  return forced >= 0 ? forced == 1 : (nt >= 4 || fp8);
}

// Waves sharing one split of the fixed decomposition.  Eight for bf16 tiles
// of up to 32 rows without the one-chunk-ahead loads (two waves per SIMD;
// the eight parked states fill most of the CU's LDS; four in paired mode);
// one otherwise.
// NVA_ATTN_WPS=1/2/4/8 overrides it for those tiles (tuning).
int segment_waves(int nt, bool fp8) {
  if (fp8 || nt >= 4 || pipelined(nt, fp8)) return 1;
  static const int forced = [] {
    const char* v = getenv("NVA_ATTN_WPS");
    const int f = v ? atoi(v) : 0;
    return (f == 1 || f == 2 || f == 4 || f == 8) ? f : 0;
  }();
  return forced ? forced : 8;
}

int tile_mfmas(int32_t tile_rows) { return tile_rows <= 16 ? 1 : tile_rows <= 32 ? 2 : 4; }

// Paired mode, for bf16 single-tile sequences of 17-32 rows (the verify of
// a GQA group of 4 with k = 4..7) whose segments number more than one and at
// most two per CU: four waves share a whole sequence (no split, no fp32
// partials), two such workgroups fit a CU at once (186 VGPRs, 76 KiB of
// LDS), so every segment is resident from the start, and the grid pairs
// them: the dispatcher gives workgroup i and workgroup i + CUs the same CU,
// so grid rows past CUs / Hkv take the sequences from the last one
// backwards.  With the batch longest first (the engine's verify order)
// each CU then holds a long and a short sequence, about the same keys per
// CU, and one workgroup's fold overlaps the other's loads.  With eight
// waves per split (one workgroup per CU, two rounds) a CU streams nothing
// while a workgroup folds its eight states and the next one starts.
// Measured on config 3's shapes (B64 q6 32/8, keys U[256, 2304], 300-launch
// graph bursts, alternating runs on one box): 56.6 against 58.0 us with
// eight waves per 2688-key split (56.0-56.2 against 57.2-57.4 on another
// box); without the pairing (rows in batch order) 61.6 us; the same mode
// for 4- and 10-row tiles: no gain (53.1 against 53.0 us) and a loss
// (62-66 against 56.1 us, 256 segments).
// Up to kPairedMaxKeys keys per sequence (the shapes measured);
// NVA_ATTN_PAIRED=0/1 overrides the choice (tuning).
constexpr int32_t kPairedMaxKeys = 3072;
bool paired_mode(int32_t num_seqs, int32_t hkv, int32_t n_qtiles, int32_t max_k, int nt, bool fp8) {
  static const int forced = env_choice("NVA_ATTN_PAIRED");
  if (forced == 0 || fp8 || nt != 2 || n_qtiles != 1 || pipelined(nt, fp8)) return false;
  if (max_k > kPairedMaxKeys) return false;
  const int64_t segs = static_cast<int64_t>(num_seqs) * hkv;
  const int64_t cus = device_cus();
  return segs > (forced == 1 ? 0 : cus) && segs <= 2 * cus;
}

// Upper bound on a sequence's split count in stream mode: a range holds at
// least kMinRangeChunks chunks, and a sequence may start mid-range.
int32_t stream_max_splits(int32_t max_k) {
  const int32_t chunks = (max_k + kChunk - 1) / kChunk;
  return (chunks + kMinRangeChunks - 1) / kMinRangeChunks + 1;
}

// Stream workgroups per kv head: one wave per SIMD of the device.
int32_t stream_ranges_per_head(int32_t hkv) {
  static const int per_simd = [] {
    const char* v = getenv("NVA_ATTN_STREAM_WAVES");
    return v && atoi(v) > 0 ? atoi(v) : 1;
  }();
  const int32_t simds = device_cus() * 4 * per_simd;
  const int32_t h = hkv > 0 ? hkv : 1;
  return (simds + h - 1) / h;
}

// Workspace for either KV dtype (the size query does not name one): the
// larger of the stream and fixed layouts that could apply to either.
size_t workspace_bytes(int32_t num_seqs, int32_t num_tokens, int32_t hq, int32_t hkv, int32_t max_q,
                       int32_t max_k) {
  const int32_t qtile = choose_qtile(max_q, hkv > 0 ? hq / hkv : 1);
  const int32_t group = hkv > 0 ? hq / hkv : 1;
  size_t bytes = 0;
  if (stream_mode(num_seqs, max_q, qtile, group, false) ||
      stream_mode(num_seqs, max_q, qtile, group, true)) {
    const size_t slots = static_cast<size_t>(num_tokens) * hq * stream_max_splits(max_k);
    bytes = slots * kD * sizeof(float) + slots * sizeof(float) +
            static_cast<size_t>(num_tokens) * sizeof(int32_t) + 512;
  }
  const int32_t n_qtiles = (max_q + qtile - 1) / qtile;
  const int nt = tile_mfmas(qtile * (hkv > 0 ? hq / hkv : 1));
  // either KV dtype: the larger split count of the two wave choices
  int32_t len, ms, ms_fp8;
  choose_split(num_seqs, hkv, n_qtiles, max_k, segment_waves(nt, false), 0, &len, &ms);
  choose_split(num_seqs, hkv, n_qtiles, max_k, segment_waves(nt, true), 0, &len, &ms_fp8);
  ms = ms_fp8 > ms ? ms_fp8 : ms;
  if (ms > 1) {
    const size_t slots = static_cast<size_t>(num_tokens) * hq * ms;
    const size_t fixed = slots * kD * sizeof(float) + slots * sizeof(float) +
                         static_cast<size_t>(num_tokens) * sizeof(int32_t) + 256;
    bytes = fixed > bytes ? fixed : bytes;
  }
  return bytes;
}

// Shared-tile kernel for bf16 64-row tiles: waves per tile and chunks in
// flight.  NVA_ATTN_TILE=0 selects the one-wave kernel instead; "W,D"
// (W = 2 or 4, D = 2..4) picks a variant (tuning).
struct TileChoice {
  int wpt, depth;
};
TileChoice tile_choice() {
  static const TileChoice c = [] {
    TileChoice t{4, 4};
    const char* v = getenv("NVA_ATTN_TILE");
    if (v) {
      int w = 0, d = 0;
      if (atoi(v) == 0) return TileChoice{0, 0};
      // two waves per tile hold 32 columns' accumulators each: only two
      // chunks in flight fit their registers without spilling
      if (sscanf(v, "%d,%d", &w, &d) == 2 && ((w == 2 && d == 2) || (w == 4 && d >= 2 && d <= 4)))
        t = TileChoice{w, d};
    }
    return t;
  }();
  return c;
}

template <int WPT>
void launch_tile(const AttnParams& p, int depth, dim3 grid, hipStream_t s) {
  if constexpr (WPT == 2) {
    paged_attention_tile_kernel<2, 2><<<grid, kWave * 2, 0, s>>>(p);
  } else {
    switch (depth) {
      case 3:
        paged_attention_tile_kernel<WPT, 3><<<grid, kWave * WPT, 0, s>>>(p);
        return;
      case 4:
        paged_attention_tile_kernel<WPT, 4><<<grid, kWave * WPT, 0, s>>>(p);
        return;
      default:
        paged_attention_tile_kernel<WPT, 2><<<grid, kWave * WPT, 0, s>>>(p);
        return;
    }
  }
}

template <int NT>
void launch_nt(const AttnParams& p, bool fp8, bool stream, int wps, dim3 grid, hipStream_t s) {
  if constexpr (NT == 4) {
    const TileChoice t = tile_choice();
    if (!fp8 && t.wpt == 2) {
      launch_tile<2>(p, t.depth, grid, s);
      return;
    }
    if (!fp8 && t.wpt == 4) {
      launch_tile<4>(p, t.depth, grid, s);
      return;
    }
  }
  const bool pipe = pipelined(NT, fp8);
  if constexpr (NT < 4) {
    if (stream) {
      if (fp8) {
        if (pipe)
          paged_attention_stream_kernel<NT, true, true><<<grid, kWave, 0, s>>>(p);
        else
          paged_attention_stream_kernel<NT, true, false><<<grid, kWave, 0, s>>>(p);
      } else {
        if (pipe)
          paged_attention_stream_kernel<NT, false, true><<<grid, kWave, 0, s>>>(p);
        else
          paged_attention_stream_kernel<NT, false, false><<<grid, kWave, 0, s>>>(p);
      }
      return;
    }
  }
  if (pipe) {
    if (fp8)
      paged_attention_kernel<NT, true, true, 1><<<grid, kWave, 0, s>>>(p);
    else
      paged_attention_kernel<NT, false, true, 1><<<grid, kWave, 0, s>>>(p);
    return;
  }
  if constexpr (NT < 4) {
    switch (fp8 ? 1 : wps) {
      case 2:
        paged_attention_kernel<NT, false, false, 2><<<grid, 2 * kWave, 0, s>>>(p);
        return;
      case 4:
        paged_attention_kernel<NT, false, false, 4><<<grid, 4 * kWave, 0, s>>>(p);
        return;
      case 8:
        paged_attention_kernel<NT, false, false, 8><<<grid, 8 * kWave, 0, s>>>(p);
        return;
      default:
        break;
    }
  }
  if (fp8)
    paged_attention_kernel<NT, true, false, 1><<<grid, kWave, 0, s>>>(p);
  else
    paged_attention_kernel<NT, false, false, 1><<<grid, kWave, 0, s>>>(p);
}

int run_attention(AttnParams& p, int kv_dtype, void* workspace, size_t workspace_bytes_, hipStream_t s) {
  if (p.hq <= 0 || p.hkv <= 0 || p.hq % p.hkv != 0) return NVA_ERR_ARG;
  if (kv_dtype != NVA_KV_BF16 && kv_dtype != NVA_KV_FP8_E4M3) return NVA_ERR_ARG;
  if (p.num_seqs < 0 || p.num_tokens < 0 || p.max_q < 0 || p.max_k < 0) return NVA_ERR_ARG;
  if (p.num_seqs == 0 || p.num_tokens == 0 || p.max_q == 0) return NVA_OK;
  if (!p.q || !p.k_cache || !p.v_cache || !p.block_tables || !p.out) return NVA_ERR_ARG;
  if (p.block_size <= 0 || p.block_size % kChunk != 0 || p.num_blocks <= 0) return NVA_ERR_UNSUPPORTED;
  if (p.bt_cols < 0 || p.bt_stride < p.bt_cols) return NVA_ERR_ARG;
  p.group = p.hq / p.hkv;
  if (p.group > 64) return NVA_ERR_UNSUPPORTED;
  p.qtile = choose_qtile(p.max_q, p.group);
  p.n_qtiles = (p.max_q + p.qtile - 1) / p.qtile;
  const int tile_rows = p.qtile * p.group;
  // alignment of 16-byte vector accesses
  const int64_t vec_elems = kv_dtype == NVA_KV_BF16 ? 8 : 16;
  if (!aligned16(p.q) || !aligned16(p.out) || !aligned16(p.k_cache) || !aligned16(p.v_cache) ||
      p.q_row_stride % 8 || p.q_head_stride % 8 || p.out_row_stride % 8 || p.out_head_stride % 8 ||
      p.blk_stride % vec_elems || p.tok_stride % vec_elems || p.head_stride % vec_elems)
    return NVA_ERR_UNSUPPORTED;
  const bool fp8 = kv_dtype == NVA_KV_FP8_E4M3;
  const bool stream = stream_mode(p.num_seqs, p.max_q, p.qtile, p.group, fp8);
  const int nt = tile_mfmas(tile_rows);
  // paired mode's whole-sequence split must fit the kernel's block ids
  const int32_t mk = p.max_k > 1 ? p.max_k : 1;
  const int32_t whole = (mk + kMinSplit - 1) / kMinSplit * kMinSplit;
  const bool paired = !stream && paired_mode(p.num_seqs, p.hkv, p.n_qtiles, p.max_k, nt, fp8) &&
                      whole / p.block_size + 2 <= kWave;
  int wps = segment_waves(nt, fp8);
  dim3 grid;
  p.row_nsplit = nullptr;
  p.pair_rows = 0;
  if (stream) {
    // a range may span at most kWave - 2 whole blocks (one block id per lane)
    p.min_range_chunks = kMinRangeChunks;
    p.max_range_chunks = (kWave - 2) * p.block_size / kChunk;
    p.max_splits = stream_max_splits(p.max_k);
    p.split_len = 0;
    grid = dim3(p.hkv, stream_ranges_per_head(p.hkv), 1);
  } else if (paired) {
    // one split per sequence (a multiple of 128 keys covering max_k)
    wps = 4;
    p.split_len = whole;
    p.max_splits = 1;
    p.pair_rows = device_cus() / p.hkv;
    grid = dim3(p.hkv, p.num_seqs, p.n_qtiles);
  } else {
    choose_split(p.num_seqs, p.hkv, p.n_qtiles, p.max_k, wps, p.block_size, &p.split_len,
                 &p.max_splits);
    // the kernel keeps one block id per lane: a split may touch at most kWave blocks
    if (p.split_len / p.block_size + 2 > kWave) return NVA_ERR_UNSUPPORTED;
    grid = dim3(p.hkv, p.num_seqs, p.max_splits * p.n_qtiles);
  }
  if (stream || p.max_splits > 1) {
    const size_t need = workspace_bytes(p.num_seqs, p.num_tokens, p.hq, p.hkv, p.max_q, p.max_k);
    const size_t slots = static_cast<size_t>(p.num_tokens) * p.hq * p.max_splits;
    // the layout this launch writes: partials, log-sum-exps, split counts
    const size_t used = slots * kD * sizeof(float) + slots * sizeof(float) +
                        static_cast<size_t>(p.num_tokens) * sizeof(int32_t);
    if (!workspace || workspace_bytes_ < need || workspace_bytes_ < used || !aligned16(workspace))
      return NVA_ERR_WORKSPACE;
    p.ws_o = static_cast<float*>(workspace);
    p.ws_lse = p.ws_o + slots * kD;
    p.row_nsplit = reinterpret_cast<int32_t*>(p.ws_lse + slots);
  } else {
    p.ws_o = nullptr;
    p.ws_lse = nullptr;
  }
  if (nt <= 1)
    launch_nt<1>(p, fp8, stream, wps, grid, s);
  else if (nt == 2)
    launch_nt<2>(p, fp8, stream, wps, grid, s);
  else
    launch_nt<4>(p, fp8, stream, wps, grid, s);
  if (hipGetLastError() != hipSuccess) return NVA_ERR_LAUNCH;
  if (stream || p.max_splits > 1) {
    const int slices = p.hq * (kD / 4);
    combine_kernel<<<dim3(p.num_tokens, (slices + kCombineThreads - 1) / kCombineThreads),
                     kCombineThreads, 0, s>>>(p);
  }
  return launch_status();
}

}  // namespace
}  // namespace nva

using namespace nva;

extern "C" size_t nva_paged_attention_workspace_size(int32_t num_seqs, int32_t num_tokens,
                                                     int32_t num_q_heads, int32_t num_kv_heads,
                                                     int32_t head_dim, int32_t max_seqlen_q,
                                                     int32_t max_seqlen_k) {
  if (num_seqs <= 0 || num_tokens <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim != kD ||
      max_seqlen_q <= 0)
    return 0;
  return workspace_bytes(num_seqs, num_tokens, num_q_heads, num_kv_heads, max_seqlen_q,
                         max_seqlen_k);
}

extern "C" int nva_paged_attention_varlen(
    const void* q, int64_t q_row_stride, int64_t q_head_stride, const void* k_cache,
    const void* v_cache, int kv_dtype, int64_t cache_block_stride, int64_t cache_token_stride,
    int64_t cache_head_stride, int32_t num_blocks, int32_t block_size,
    const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, const int32_t* block_tables,
    int64_t block_table_stride, int32_t max_blocks_per_seq, int32_t num_seqs, int32_t num_tokens, int32_t max_seqlen_q,
    int32_t max_seqlen_k, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    float softmax_scale, const float* k_scale, const float* v_scale, void* out,
    int64_t out_row_stride, int64_t out_head_stride, void* workspace, size_t workspace_bytes_,
    void* stream) {
  if (head_dim != kD) return NVA_ERR_UNSUPPORTED;
  if (!cu_seqlens_q || !cu_seqlens_k) return NVA_ERR_ARG;
  AttnParams p = {};
  p.q = static_cast<const uint16_t*>(q);
  p.q_row_stride = q_row_stride;
  p.q_head_stride = q_head_stride;
  p.k_cache = static_cast<const uint8_t*>(k_cache);
  p.v_cache = static_cast<const uint8_t*>(v_cache);
  p.blk_stride = cache_block_stride;
  p.tok_stride = cache_token_stride;
  p.head_stride = cache_head_stride;
  p.num_blocks = num_blocks;
  p.block_size = block_size;
  p.cu_q = cu_seqlens_q;
  p.cu_k = cu_seqlens_k;
  p.seqlens = nullptr;
  p.block_tables = block_tables;
  p.bt_stride = block_table_stride;
  p.bt_cols = max_blocks_per_seq;
  p.num_seqs = num_seqs;
  p.num_tokens = num_tokens;
  p.max_q = max_seqlen_q;
  p.max_k = max_seqlen_k;
  p.hq = num_q_heads;
  p.hkv = num_kv_heads;
  p.scale_log2 = softmax_scale * kLog2e;
  p.k_scale = k_scale;
  p.v_scale = v_scale;
  p.out = static_cast<uint16_t*>(out);
  p.out_row_stride = out_row_stride;
  p.out_head_stride = out_head_stride;
  return run_attention(p, kv_dtype, workspace, workspace_bytes_, static_cast<hipStream_t>(stream));
}

extern "C" int nva_paged_attention_decode(
    const void* q, int64_t q_row_stride, int64_t q_head_stride, const void* k_cache,
    const void* v_cache, int kv_dtype, int64_t cache_block_stride, int64_t cache_token_stride,
    int64_t cache_head_stride, int32_t num_blocks, int32_t block_size,
    const int32_t* cache_seqlens, const int32_t* block_tables, int64_t block_table_stride,
    int32_t max_blocks_per_seq, int32_t num_seqs, int32_t max_seqlen_k, int32_t num_q_heads, int32_t num_kv_heads,
    int32_t head_dim, float softmax_scale, const float* k_scale, const float* v_scale, void* out,
    int64_t out_row_stride, int64_t out_head_stride, void* workspace, size_t workspace_bytes_,
    void* stream) {
  if (head_dim != kD) return NVA_ERR_UNSUPPORTED;
  if (!cache_seqlens) return NVA_ERR_ARG;
  AttnParams p = {};
  p.q = static_cast<const uint16_t*>(q);
  p.q_row_stride = q_row_stride;
  p.q_head_stride = q_head_stride;
  p.k_cache = static_cast<const uint8_t*>(k_cache);
  p.v_cache = static_cast<const uint8_t*>(v_cache);
  p.blk_stride = cache_block_stride;
  p.tok_stride = cache_token_stride;
  p.head_stride = cache_head_stride;
  p.num_blocks = num_blocks;
  p.block_size = block_size;
  p.cu_q = nullptr;
  p.cu_k = nullptr;
  p.seqlens = cache_seqlens;
  p.block_tables = block_tables;
  p.bt_stride = block_table_stride;
  p.bt_cols = max_blocks_per_seq;
  p.num_seqs = num_seqs;
  p.num_tokens = num_seqs;
  p.max_q = 1;
  p.max_k = max_seqlen_k;
  p.hq = num_q_heads;
  p.hkv = num_kv_heads;
  p.scale_log2 = softmax_scale * kLog2e;
  p.k_scale = k_scale;
  p.v_scale = v_scale;
  p.out = static_cast<uint16_t*>(out);
  p.out_row_stride = out_row_stride;
  p.out_head_stride = out_head_stride;
  return run_attention(p, kv_dtype, workspace, workspace_bytes_, static_cast<hipStream_t>(stream));
}
