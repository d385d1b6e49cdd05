/*
 * nanovllm_amd.h -- C ABI of the MI355X (gfx950) EAGLE3 speculative-step
 * kernels.  Built into libnanovllm_amd.so from extend-nano-vllm_amd/csrc/.
 *
 * Reference: kagami4243/extend-nano-vLLM (package `nanovllm`).  Each entry
 * point names the reference call it replaces (file:line).  The reference's
 * kernels are Python-callable Triton / FlashAttention-2 functions taking torch
 * tensors; here the same operations take raw device pointers, element strides
 * and sizes.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers unless stated otherwise.  The caller owns
 *     every buffer; nothing is allocated or freed inside the library.
 *   - Strides are in ELEMENTS of the pointed-to type.
 *   - `stream` is a hipStream_t (passed as void*); work is enqueued on it with
 *     no host synchronisation, so every call may be captured in a HIP graph.
 *   - bf16 tensors are passed as their 16-bit storage; KV caches are bf16
 *     (NVA_KV_BF16) or OCP float8_e4m3fn (NVA_KV_FP8_E4M3).
 *   - The return value is an nva_status; argument errors are detected on the
 *     host before anything is launched.  Device-resident metadata (slots,
 *     block ids, lengths) is bounds-checked inside the kernels: an
 *     out-of-range slot or block id is skipped, never dereferenced.
 *   - Calls on one stream are ordered; calls that share a workspace must not
 *     run concurrently on different streams.
 */
#ifndef NANOVLLM_AMD_H
#define NANOVLLM_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum nva_status {
  NVA_OK = 0,
  NVA_ERR_ARG = 1,          /* null pointer, bad size/stride/shape */
  NVA_ERR_WORKSPACE = 2,    /* workspace missing or smaller than required */
  NVA_ERR_UNSUPPORTED = 3,  /* valid but unsupported (e.g. head_dim != 128) */
  NVA_ERR_LAUNCH = 4,       /* the HIP runtime rejected a launch */
  NVA_ERR_CAPACITY = 5      /* input larger than a static scratch array holds */
};

enum nva_kv_dtype { NVA_KV_BF16 = 0, NVA_KV_FP8_E4M3 = 1 };

/* Human-readable name of a status code (static string). */
const char *nva_status_string(int status);

/* Library version string (static). */
const char *nva_version(void);

/* ---------------------------------------------------------------------
 * K2a  KV-cache slot write.
 * Replaces store_kvcache / store_kvcache_kernel
 *   (nanovllm/layers/attention.py:189-217, kernel :14-43).
 * key/value: bf16 [num_tokens, num_kv_heads, head_dim], head stride ==
 *   head_dim, row strides key_row_stride / value_row_stride (views into a
 *   fused QKV output are allowed).
 * k_cache/v_cache: [num_slots, num_kv_heads * head_dim] contiguous (the
 *   reference's [num_blocks, block_size, Hkv, D] layer view flattened),
 *   slot = block_id * block_size + offset.
 * Token t is written to slot_mapping[t]; negative slots (the reference's -1)
 *   and slots >= num_slots are skipped.
 * FP8: each element is stored as e4m3(x / scale), round-to-nearest-even,
 *   saturating to +-448; k_scale / v_scale are device fp32 scalars (NULL =
 *   1.0).  bf16 caches ignore the scales, as the reference does.
 * ------------------------------------------------------------------- */
int nva_store_kvcache(const void *key, int64_t key_row_stride,
                      const void *value, int64_t value_row_stride,
                      void *k_cache, void *v_cache, int kv_dtype,
                      const int32_t *slot_mapping, int32_t num_tokens,
                      int32_t num_kv_heads, int32_t head_dim, int64_t num_slots,
                      const float *k_scale, const float *v_scale, void *stream);

/* The same slot write into a cache addressed by strides, for layouts other
 * than contiguous token rows.  Replaces the same reference call
 *   (nanovllm/layers/attention.py:189-217); the reference asserts the
 *   token-major layout (:198-203), which is the case
 *   cache_token_stride == num_kv_heads * head_dim, cache_head_stride ==
 *   head_dim.
 * k_cache/v_cache: [num_blocks, block_size, num_kv_heads, head_dim] in
 *   element strides cache_block_stride, cache_token_stride,
 *   cache_head_stride (unit stride over head_dim), e.g. the head-major pages
 *   [num_blocks, num_kv_heads, block_size, head_dim] seen as
 *   (Hkv*bs*D, D, bs*D).  Slot s is token s % block_size of block
 *   s / block_size; slots outside [0, num_blocks * block_size) are skipped.
 * Everything else as nva_store_kvcache. */
int nva_store_kvcache_paged(const void *key, int64_t key_row_stride,
                            const void *value, int64_t value_row_stride,
                            void *k_cache, void *v_cache, int kv_dtype,
                            int64_t cache_block_stride, int64_t cache_token_stride,
                            int64_t cache_head_stride, int32_t num_blocks,
                            int32_t block_size, const int32_t *slot_mapping,
                            int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
                            const float *k_scale, const float *v_scale, void *stream);

/* ---------------------------------------------------------------------
 * K2b  Rollback of rejected draft rows.
 * Device mirror of the reference's logical rollback after greedy
 *   verification: Sequence.truncate_tokens + BlockManager.truncate
 *   (nanovllm/engine/scheduler.py:165-170, block_manager.py:197-205,
 *   sequence.py:84-91).  Rows j > accept_len[i] of sequence i (verify rows
 *   [cu_seqlens_q[i], cu_seqlens_q[i+1])) are rejected: their slot_mapping
 *   entry becomes -1 and seqlens_k[i] drops by the number of rejected rows,
 *   so later attention never reads them.  accept_len is clamped to
 *   [0, q_i - 1].
 * With poison != 0 the rejected slots are zeroed in num_layers layers of the
 *   caches (k_cache / v_cache point at layer 0; layer l is at
 *   + l * layer_stride elements; each slot row has row_elems elements).
 *   With poison == 0 the caches may be NULL.
 * ------------------------------------------------------------------- */
int nva_rollback(const int32_t *cu_seqlens_q, const int32_t *accept_len, int32_t num_seqs,
                 int32_t *slot_mapping, int32_t *seqlens_k,
                 void *k_cache, void *v_cache, int kv_dtype, int32_t num_layers,
                 int64_t layer_stride, int32_t row_elems, int64_t num_slots, int poison,
                 void *stream);

/* ---------------------------------------------------------------------
 * K3  EAGLE3 auxiliary hidden-state add + concat + row gather.
 * Replaces `hidden_states + residual` at the aux layers, torch.cat(aux, -1)
 *   (nanovllm/models/qwen3.py:284-289) and the per-sequence row slicing that
 *   feeds the draft fc (nanovllm/engine/model_runner.py:1073, :1236-1242;
 *   nanovllm/engine/llm_engine.py:170).
 * hidden / residual: HOST arrays of num_layers (1..4) device pointers, each a
 *   bf16 [rows, hidden_size] matrix with row stride in_row_stride.
 * out[r, l*hidden_size + c] = bf16(f32(hidden[l][src_rows[r], c]) +
 *                                 f32(residual[l][src_rows[r], c]))
 *   rounded to nearest even; out has row stride out_row_stride.
 * src_rows entries outside [0, num_in_rows) produce zero rows.
 * ------------------------------------------------------------------- */
int nva_aux_gather(const void *const *hidden, const void *const *residual, int32_t num_layers,
                   int64_t in_row_stride, int32_t hidden_size, int32_t num_in_rows,
                   const int32_t *src_rows, int32_t num_rows,
                   void *out, int64_t out_row_stride, void *stream);

/* ---------------------------------------------------------------------
 * K4a  Vocab argmax fused with the greedy accepted-prefix / bonus scan.
 * Replaces the per-sequence `target_logits[start:end].argmax(dim=-1).tolist()`
 *   of verify_eagle3_batch (nanovllm/engine/model_runner.py:1066-1074) and
 *   verify_greedy_proposals (nanovllm/engine/speculative.py:11-30).
 * logits: bf16 [num_tokens, vocab], row stride row_stride.
 * cu_seqlens_q: [num_seqs + 1] verify row offsets (device).
 * input_ids: the verify input tokens [num_tokens] (int64, device): proposal j
 *   of sequence i is input_ids[cu_seqlens_q[i] + 1 + j], j < q_i - 1 (row 0
 *   of each sequence is the previous target token).
 * Outputs: argmax[num_tokens] (torch.argmax semantics on bf16: first index of
 *   the maximum, NaN is the maximum, -0 == +0); accept_len[num_seqs] = first
 *   j with proposal_j != argmax[row j], else q_i - 1; bonus[num_seqs] =
 *   argmax[row accept_len] (the replacement or bonus token).  A sequence with
 *   q_i == 0 gets accept_len 0 and bonus -1.
 * workspace: nva_argmax_workspace_size(num_tokens, num_seqs, vocab) bytes,
 *   8-byte aligned, no initialisation needed (per-chunk partial maxima).
 * Two kernels are enqueued (chunk partials, then the merge and accept scan).
 * ------------------------------------------------------------------- */
size_t nva_argmax_workspace_size(int32_t num_rows, int32_t num_seqs, int32_t vocab);

int nva_argmax_accept(const void *logits, int64_t row_stride, int32_t vocab,
                      const int32_t *cu_seqlens_q, int32_t num_seqs, int32_t num_tokens,
                      const int64_t *input_ids,
                      int32_t *argmax, int32_t *accept_len, int32_t *bonus,
                      void *workspace, size_t workspace_bytes, void *stream);

/* Allocation-free variant of nva_argmax_accept.  No counterpart in the
 *   reference: it is for callers that cannot allocate device memory (code
 *   under HIP graph capture, tight serving loops, harnesses that forbid
 *   hipMalloc).  Same arguments, outputs and launches as nva_argmax_accept,
 *   without the workspace: the chunk keys go to a static device array of
 *   NVA_ARGMAX_STATIC_KEYS 64-bit keys (512 KiB) that each GPU holds until
 *   the process ends.  Its address is looked up once per device
 *   (hipGetSymbolAddress) on the first call made with that device current.
 *   A caller that records the call into a HIP graph makes one ordinary
 *   (uncaptured) call on that device first, so that the lookup, a runtime
 *   call, happens outside the capture; captured calls and their replays then
 *   only launch kernels.
 * Limit: num_tokens * ceil(vocab / 16384) <= NVA_ARGMAX_STATIC_KEYS (6553
 *   rows of a 151936-token vocabulary); larger inputs return
 *   NVA_ERR_CAPACITY and launch nothing.  The stream must belong to the
 *   current device (NVA_ERR_ARG otherwise).
 * Nothing is allocated, freed or cleared: every key the merge reads is
 *   written earlier in the same call.  All calls on one GPU share the array,
 *   so calls that overlap on one GPU (other streams, other host threads) race
 *   and must be serialised by the caller. */
#define NVA_ARGMAX_STATIC_KEYS 65536

int nva_argmax_accept_static(const void *logits, int64_t row_stride, int32_t vocab,
                             const int32_t *cu_seqlens_q, int32_t num_seqs, int32_t num_tokens,
                             const int64_t *input_ids,
                             int32_t *argmax, int32_t *accept_len, int32_t *bonus,
                             void *stream);

/* ---------------------------------------------------------------------
 * K4b  Row argmax with an optional index map (greedy sampling).
 * Replaces Eagle3ForCausalLM.sample_greedy's argmax + d2t lookup
 *   (nanovllm/models/eagle3.py:294-296) and the greedy branch of Sampler
 *   (nanovllm/layers/sampler.py:10-19, temperature 0).
 * out[r] = idx + (index_map ? index_map[idx] : 0), idx = argmax of row r
 *   (same semantics as nva_argmax_accept); out is int64 [num_rows].
 * workspace: as for nva_argmax_accept (num_seqs = 0).
 * ------------------------------------------------------------------- */
int nva_argmax_rows(const void *logits, int64_t row_stride, int32_t vocab, int32_t num_rows,
                    const int64_t *index_map, int64_t *out,
                    void *workspace, size_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------------
 * K1  Paged verify attention.
 *
 * Shared arguments:
 *   q: bf16 [rows, num_q_heads, head_dim] with strides q_row_stride,
 *      q_head_stride (d contiguous).  out: bf16, same shape, strides
 *      out_row_stride, out_head_stride.
 *   k_cache / v_cache: one layer, [num_blocks, block_size, num_kv_heads,
 *      head_dim] addressed by cache_block_stride / cache_token_stride /
 *      cache_head_stride (d contiguous), kv_dtype bf16 or fp8 e4m3.
 *   block_tables: int32 [num_seqs, max_blocks_per_seq], row stride
 *      block_table_stride; key n of sequence i is at block
 *      block_tables[i][n / block_size], offset n % block_size.  Keys beyond
 *      max_blocks_per_seq * block_size and block ids outside [0, num_blocks)
 *      are treated as empty (masked), never dereferenced.
 *   Query rows at or beyond num_tokens (from inconsistent cu_seqlens_q) are
 *      skipped.
 *   softmax_scale multiplies q.k; for FP8 caches the scores are also
 *      multiplied by *k_scale and the output by *v_scale (NULL = 1.0), as in
 *      the reference's FP8 decode kernel; bf16 caches ignore the scales.
 *   GQA: query head h reads kv head h / (num_q_heads / num_kv_heads).
 *   head_dim must be 128, block_size a multiple of 32 and
 *      num_q_heads / num_kv_heads <= 64; any query length is accepted.
 *   workspace: nva_paged_attention_workspace_size(...) bytes (split-KV
 *      partial results; needs no initialisation).
 * ------------------------------------------------------------------- */

/* Replaces flash_attn_varlen_func(q, k_cache, v_cache, max_seqlen_q,
 *   cu_seqlens_q, max_seqlen_k, cu_seqlens_k, softmax_scale, causal=True,
 *   block_table) -- the EAGLE3 verify attention (nanovllm/layers/
 *   attention.py:385-395).  Sequence i has q_i = cu_seqlens_q[i+1] -
 *   cu_seqlens_q[i] query rows and L_i = cu_seqlens_k[i+1] - cu_seqlens_k[i]
 *   keys including its new rows; causality is bottom-right aligned: query row
 *   j sees keys [0, L_i - q_i + j].  max_seqlen_q / max_seqlen_k bound q_i and
 *   L_i: they size the grid, and the lengths live on the device, where the
 *   host cannot check them.  A longer sequence is clipped, not refused:
 *   rows past max_seqlen_q are written as zeros, while the kept rows j <
 *   max_seqlen_q still see exactly keys [0, L_i - q_i + j]; and when the keys
 *   those rows see run past max_seqlen_k, only the first max_seqlen_k keys
 *   are attended (row j's range then ends at max_seqlen_k - q' + j, q' the
 *   kept rows).  Pass the true maxima (the reference's prepare_prefill does,
 *   model_runner.py:776-781) or safe upper bounds. */
size_t nva_paged_attention_workspace_size(int32_t num_seqs, int32_t num_tokens,
                                          int32_t num_q_heads, int32_t num_kv_heads,
                                          int32_t head_dim, int32_t max_seqlen_q,
                                          int32_t max_seqlen_k);

int nva_paged_attention_varlen(const void *q, int64_t q_row_stride, int64_t q_head_stride,
                               const void *k_cache, const void *v_cache, int kv_dtype,
                               int64_t cache_block_stride, int64_t cache_token_stride,
                               int64_t cache_head_stride, int32_t num_blocks, int32_t block_size,
                               const int32_t *cu_seqlens_q, const int32_t *cu_seqlens_k,
                               const int32_t *block_tables, int64_t block_table_stride,
                               int32_t max_blocks_per_seq, int32_t num_seqs, int32_t num_tokens,
                               int32_t max_seqlen_q, int32_t max_seqlen_k,
                               int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                               float softmax_scale, const float *k_scale, const float *v_scale,
                               void *out, int64_t out_row_stride, int64_t out_head_stride,
                               void *workspace, size_t workspace_bytes, void *stream);

/* Replaces flash_attn_with_kvcache(q[:, None], k_cache, v_cache,
 *   cache_seqlens, block_table, softmax_scale, causal=True) -- the one-query
 *   decode used by the draft (nanovllm/layers/attention.py:396-399) -- and
 *   fp8_paged_decode_attention(q, k_cache, v_cache, context_lens,
 *   block_tables, scale, k_scale, v_scale) (nanovllm/layers/
 *   attention.py:249-293).  Row r (of num_seqs) is one query that sees keys
 *   [0, cache_seqlens[r]) through block_tables row r. */
int nva_paged_attention_decode(const void *q, int64_t q_row_stride, int64_t q_head_stride,
                               const void *k_cache, const void *v_cache, int kv_dtype,
                               int64_t cache_block_stride, int64_t cache_token_stride,
                               int64_t cache_head_stride, int32_t num_blocks, int32_t block_size,
                               const int32_t *cache_seqlens,
                               const int32_t *block_tables, int64_t block_table_stride,
                               int32_t max_blocks_per_seq, int32_t num_seqs, int32_t max_seqlen_k,
                               int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                               float softmax_scale, const float *k_scale, const float *v_scale,
                               void *out, int64_t out_row_stride, int64_t out_head_stride,
                               void *workspace, size_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------------
 * Supporting per-token kernels of the target / draft forward (between the
 * projection GEMMs, which stay on hipBLASLt through torch).  bf16 in/out,
 * fp32 math; rounding follows the reference's eager formulas.
 * ------------------------------------------------------------------- */

/* RMSNorm.forward without residual (nanovllm/layers/layernorm.py:70-89):
 *   out = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * weight), per row. */
int nva_rms_norm(const void *x, int64_t x_row_stride, const void *weight, void *out,
                 int64_t out_row_stride, int32_t rows, int32_t hidden, float eps, void *stream);

/* RMSNorm.forward with residual (add_rms_forward, layernorm.py:91-107):
 *   s = f32(x) + f32(residual); residual_out = bf16(s);
 *   out = bf16(bf16(s * rsqrt(mean(s^2) + eps)) * weight). */
int nva_add_rms_norm(const void *x, int64_t x_row_stride, const void *residual,
                     int64_t residual_row_stride, const void *weight, void *out,
                     int64_t out_row_stride, void *residual_out, int64_t residual_out_row_stride,
                     int32_t rows, int32_t hidden, float eps, void *stream);

/* A bf16 tensor add followed by RMSNorm.forward without residual, as the
 *   EAGLE3 draft layer composes them (nanovllm/models/eagle3.py:141-146, and
 *   the final norm of forward_with_cache, :256-258):
 *   sum_out = bf16(f32(x) + f32(residual));
 *   out = bf16(bf16(sum_out * rsqrt(mean(sum_out^2) + eps)) * weight).
 *   Differs from nva_add_rms_norm only in normalising the bf16-rounded sum.
 *   sum_out must not be x or residual. */
int nva_add_then_rms_norm(const void *x, int64_t x_row_stride, const void *residual,
                          int64_t residual_row_stride, const void *weight, void *out,
                          int64_t out_row_stride, void *sum_out, int64_t sum_out_row_stride,
                          int32_t rows, int32_t hidden, float eps, void *stream);

/* Qwen3Attention.project_qkv after the QKV GEMM (nanovllm/models/qwen3.py:
 *   77-98): per-head q/k RMSNorm (skipped when both norm weights are NULL,
 *   the EAGLE3 draft layer) then neox rotary embedding
 *   (nanovllm/layers/rotary_embedding.py:6-48) with cos_sin a float32
 *   [max_position, head_dim] table (cos | sin halves).  qkv rows hold
 *   [q heads | k heads | v heads]; q_out [T, Hq, D] and k_out [T, Hkv, D] are
 *   contiguous.  head_dim must be 128. */
int nva_qk_norm_rope(const void *qkv, int64_t row_stride, const int64_t *positions,
                     const void *q_norm_weight, const void *k_norm_weight, const float *cos_sin,
                     int32_t max_position, int32_t num_tokens, int32_t num_q_heads,
                     int32_t num_kv_heads, int32_t head_dim, float eps, void *q_out, void *k_out,
                     void *stream);

/* nva_qk_norm_rope followed by the paged K/V write of the layer
 *   (nanovllm/models/qwen3.py:77-98 then store_kvcache,
 *   nanovllm/layers/attention.py:189-217), in one launch: q_out as above;
 *   the rotated key heads (rounded to bf16) and the value heads of qkv go to
 *   the caches at slot_mapping[t] exactly as nva_store_kvcache_paged writes
 *   them (same strides, kv_dtype, scales; a negative or out-of-range slot is
 *   skipped).  No key tensor is produced. */
int nva_qk_norm_rope_store(const void *qkv, int64_t row_stride, const int64_t *positions,
                           const void *q_norm_weight, const void *k_norm_weight,
                           const float *cos_sin, int32_t max_position, int32_t num_tokens,
                           int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, float eps,
                           void *q_out, void *k_cache, void *v_cache, int kv_dtype,
                           int64_t cache_block_stride, int64_t cache_token_stride,
                           int64_t cache_head_stride, int32_t num_blocks, int32_t block_size,
                           const int32_t *slot_mapping, const float *k_scale,
                           const float *v_scale, void *stream);

/* ---------------------------------------------------------------------
 * Verify-batch metadata on the device.
 * Replaces the per-token loops of prepare_prefill for the verify rows
 *   (nanovllm/engine/model_runner.py:761-800, block tables :755-759).
 * Sequence i contributes q_lens[i] rows at positions start_pos[i] ..
 *   start_pos[i] + q_lens[i] - 1 and sees start_pos[i] + q_lens[i] keys:
 *   cu_seqlens_q[i+1] = cu_seqlens_q[i] + q_lens[i];
 *   cu_seqlens_k[i+1] = cu_seqlens_k[i] + start_pos[i] + q_lens[i];
 *   positions[t] = start_pos[i] + (t - cu_seqlens_q[i]);
 *   slot_mapping[t] = block_tables[i][p / block_size] * block_size + p % block_size
 *   for p = positions[t], or -1 when that block id is negative or past
 *   max_blocks_per_seq (the reference pads block tables with -1).
 * Rows t >= cu_seqlens_q[num_seqs] (up to num_tokens) get position 0 and
 *   slot -1.  All arrays are device memory; num_seqs <= 2048.
 * ------------------------------------------------------------------- */
int nva_verify_metadata(const int32_t *start_pos, const int32_t *q_lens, int32_t num_seqs,
                        const int32_t *block_tables, int64_t block_table_stride,
                        int32_t max_blocks_per_seq, int32_t block_size, int32_t *cu_seqlens_q,
                        int32_t *cu_seqlens_k, int64_t *positions, int32_t *slot_mapping,
                        int32_t num_tokens, void *stream);

/* ---------------------------------------------------------------------
 * Commit metadata: the draft's replay of the committed tails, derived on
 * the device from the accept scan's results.
 * Replaces what commit_eagle3 builds per sequence on the host -- the
 *   output token ids, their positions, the verify rows whose aux states
 *   feed the fc, the per-token paged contexts and the last row that seeds
 *   the draft state (nanovllm/engine/model_runner.py:1216-1249, contexts
 *   :1127-1156) -- for a whole verify batch at once.
 * Sequence i commits q_i = min(max(accept_len[i], 0) + 1, q_stride) rows
 *   (its accepted drafts, then the bonus token) from its verify rows
 *   i * q_stride .. i * q_stride + q_i - 1; cu_seqlens_q / cu_seqlens_k /
 *   positions / slot_mapping are nva_verify_metadata's outputs for
 *   (start_pos, q_i).  Per commit row t of sequence i:
 *   verify_rows[t] = i * q_stride + (t - cu_seqlens_q[i]);
 *   token_ids[t] = verify_argmax[verify_rows[t]] (int64; an accepted draft
 *   equals the argmax of its row);
 *   rows t >= cu_seqlens_q[num_seqs] get verify row -1, token
 *   verify_argmax[0], position 0 and slot -1.
 * last_rows[i] = cu_seqlens_q[i+1] - 1 (int64).  num_seqs <= 2048; every
 *   array is device memory.
 * Draft slot convention (slot_offset, 0 or 1; anything else is
 *   NVA_ERR_ARG): the K/V of commit row t (RoPE position p = positions[t])
 *   go to the slot of position p + slot_offset, and sequence i sees
 *   cu_seqlens_k[i+1] - cu_seqlens_k[i] = start_pos[i] + q_i + slot_offset
 *   keys, so row j of it sees the keys up to and including its own slot.
 *   slot_offset = 1 is the reference's commit convention: token i of the
 *   tail is written at slot start + 1 + i with context start + 2 + i
 *   (nanovllm/engine/model_runner.py:1143-1149, _set_eagle3_commit_context
 *   called from :1127-1156).  slot_offset = 0 writes position p at slot p,
 *   as the reference's draft prefill does (:1379-1390) and this build's
 *   engine does throughout.  A binder replacing the reference's commit loop
 *   with this entry must use the same offset in nva_draft_metadata (or in
 *   its own draft loop): the draft steps read the slots the commit wrote.
 * ------------------------------------------------------------------- */
int nva_commit_metadata(const int32_t *start_pos, const int32_t *accept_len, int32_t num_seqs,
                        int32_t q_stride, const int32_t *verify_argmax, int32_t num_verify_rows,
                        const int32_t *block_tables, int64_t block_table_stride,
                        int32_t max_blocks_per_seq, int32_t block_size, int32_t slot_offset,
                        int32_t *cu_seqlens_q, int32_t *cu_seqlens_k, int64_t *positions,
                        int32_t *slot_mapping, int32_t *verify_rows, int64_t *token_ids,
                        int64_t *last_rows, int32_t num_tokens, void *stream);

/* Draft-step metadata for a draft queued right behind a verify, before the
 *   host has read its results.  Replaces the host loop that builds each
 *   draft step's position, slot and context length
 *   (nanovllm/engine/model_runner.py:1087-1096, :1159-1213) for the step
 *   that follows a verify: sequence i (columns i < num_seqs of bs; the rest
 *   are padding) has length L_i = lens[i] + accept_len[verify_row[i]] + 1
 *   after the verified step (accept_len is the accept scan's output, indexed
 *   by the sequence's row in the verify batch), and its draft step s <
 *   steps is at RoPE position p = L_i - 1 + s: positions[s * bs + i] = p,
 *   and with P = p + slot_offset, context_lens[...] = P + 1 and
 *   slot_mapping[...] = block id * block_size + P % block_size through
 *   block_tables row i (-1 where the block id is negative or P is past
 *   max_blocks_per_seq pages).  Padding columns get position 0, context 1
 *   and slot -1.  Every array is device memory.
 * Draft slot convention (slot_offset, 0 or 1; anything else is
 *   NVA_ERR_ARG): slot_offset = 1 is the reference's decode convention,
 *   slot len(seq) + step and context len(seq) + step + 1 for the query at
 *   RoPE position len(seq) - 1 + step (_set_eagle3_decode_context,
 *   nanovllm/engine/model_runner.py:1087-1096).  slot_offset = 0 writes
 *   position p at slot p with context p + 1, the convention of this
 *   build's engine and of the reference's draft prefill (:1379-1390).  The
 *   decode and commit loops of one engine must use the same offset
 *   (nva_commit_metadata). */
int nva_draft_metadata(const int64_t *lens, const int64_t *verify_row, const int32_t *accept_len,
                       int32_t num_seqs, int32_t bs, int32_t steps, const int32_t *block_tables,
                       int64_t block_table_stride, int32_t max_blocks_per_seq,
                       int32_t block_size, int32_t slot_offset, int64_t *positions,
                       int32_t *slot_mapping, int32_t *context_lens, void *stream);

/* Verify input ids composed on the device from the draft's proposals.
 *   Replaces the reference's verify input, each sequence's last
 *   num_scheduled_tokens tokens after its proposals were appended
 *   (nanovllm/engine/llm_engine.py:129-141 appends them,
 *   nanovllm/engine/model_runner.py:770-774 reads them): for verify row
 *   t = p * q + j of sequence p (num_rows sequences of q rows),
 *   ids[t] = last_tokens[p] for j == 0 and
 *   proposals[(j - 1) * proposal_stride + order[p]] for j >= 1, the draft's
 *   output laid out [q-1][proposal_stride] with the sequence in column
 *   order[p].  A row whose order[p] is outside [0, proposal_stride) is
 *   padding: its q ids are 0.  When compose[0] == 0 nothing is written
 *   (ids keep what the host uploaded), so a captured graph can hold the
 *   launch for both uses.  Every array is device memory. */
int nva_verify_input_ids(const int32_t *compose, const int32_t *last_tokens, const int32_t *order,
                         const int64_t *proposals, int64_t proposal_stride, int32_t num_rows,
                         int32_t q, int64_t *ids, void *stream);

/* SiluAndMul (nanovllm/layers/activation.py:11-14): x rows [a | b] of
 *   2*intermediate elements -> out = bf16(bf16(silu(a)) * b). */
int nva_silu_mul(const void *x, int64_t x_row_stride, void *out, int64_t out_row_stride,
                 int32_t rows, int32_t intermediate, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* NANOVLLM_AMD_H */
