/*
 * CPU oracle for the EAGLE3 speculative-decoding step.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker.
 * The product path (extend-nano-vllm_amd/) never calls it and fails loudly
 * when its HIP library is missing.
 *
 * Each function restates one piece of the reference algorithm
 * (kagami4243/extend-nano-vLLM, package `nanovllm`) in plain scalar C and
 * cites the file:line it follows.  Floating-point attention is accumulated in
 * double so that it is a tighter reference than any GPU kernel under test.
 *
 * How each function is pinned (checked independently of its own formula) is
 * listed in tests/test_oracle.py; summary:
 *   oracle_argmax_bf16        torch CPU argmax (first max, NaN is max), brute force
 *   oracle_accept             hand-worked vectors in tests/golden/, the
 *                             Python restatement of speculative.py
 *   oracle_f32_to_e4m3 /      torch CPU float8_e4m3fn casts on every bf16 bit
 *   oracle_e4m3_to_f32          pattern and all 256 fp8 codes
 *   oracle_f32_to_bf16        torch CPU bf16 casts on random and special floats
 *   oracle_store_kv           round trip gather(store(x)) == x, slot == -1 skip
 *   oracle_aux_gather         torch CPU bf16 add + cat + index_select
 *   oracle_paged_attention    numpy dense attention with an explicit mask over
 *                             pages gathered through the block table, and
 *                             closed forms (one visible key, equal scores)
 *   oracle_fp8_paged_decode   oracle_paged_attention within 2e-3 (the
 *                             reference's own bound, tests/test_fp8_kv_cache.py:81)
 *   oracle_rollback           closed form on hand-worked cases
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* scalar format conversions                                           */
/* ------------------------------------------------------------------ */

float oracle_bf16_to_f32(uint16_t b)
{
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Round-to-nearest-even float -> bfloat16; NaN becomes 0x7FC0.  This is the
 * conversion torch applies when a float result is stored as bfloat16. */
uint16_t oracle_f32_to_bf16(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    if (isnan(f))
        return 0x7FC0;
    uint32_t bias = ((u >> 16) & 1u) + 0x7FFFu;
    return (uint16_t)((u + bias) >> 16);
}

/* float8_e4m3fn (OCP): 1 sign, 4 exponent (bias 7), 3 mantissa bits, no
 * infinities, 0x7F/0xFF are NaN, largest finite 448. */
float oracle_e4m3_to_f32(uint8_t b)
{
    int sign = b >> 7;
    int e = (b >> 3) & 0xF;
    int m = b & 7;
    float v;
    if (e == 0xF && m == 7)
        return NAN;
    if (e == 0)
        v = ldexpf((float)m, -9);            /* subnormal: m/8 * 2^-6 */
    else
        v = ldexpf(1.0f + m / 8.0f, e - 7);
    return sign ? -v : v;
}

/* float -> float8_e4m3fn, round to nearest even, saturating to +-448 for
 * finite and infinite magnitudes beyond the format, NaN -> 0x7F (sign kept).
 *
 * The reference stores through Triton's fp32 -> fp8e4nv conversion
 * (layers/attention.py:39-43, store of a float tensor into a float8 pointer),
 * which on NVIDIA lowers to the saturating round-to-nearest conversion.  For
 * |x| <= 448 this equals torch's `.to(torch.float8_e4m3fn)`; beyond it torch
 * produces NaN while the reference saturates, and this oracle follows the
 * reference. */
uint8_t oracle_f32_to_e4m3(float x)
{
    uint32_t u;
    memcpy(&u, &x, 4);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80);
    if (isnan(x))
        return (uint8_t)(sign | 0x7F);
    double a = fabs((double)x);
    if (a >= 464.0)              /* 464 is the tie between 448 and 480: RNE -> 448 */
        return (uint8_t)(sign | 0x7E);
    /* Scan the 127 non-negative finite codes for the nearest; ties go to the
     * even code (mantissa LSB 0).  Exhaustive and obviously correct. */
    int best = 0;
    double best_err = INFINITY;
    for (int c = 0; c <= 0x7E; ++c) {
        double v = (double)oracle_e4m3_to_f32((uint8_t)c);
        double err = fabs(v - a);
        if (err < best_err || (err == best_err && (c & 1) == 0 && (best & 1) == 1)) {
            best = c;
            best_err = err;
        }
    }
    return (uint8_t)(sign | best);
}

/* ------------------------------------------------------------------ */
/* K4: row argmax + greedy accepted-prefix / bonus scan                */
/* ------------------------------------------------------------------ */

/* torch.argmax(dim=-1) on bfloat16 rows, as called on the verify logits in
 * engine/model_runner.py:1071-1073: the first index of the maximum; any NaN
 * counts as larger than every number (first NaN wins); -0 equals +0. */
void oracle_argmax_bf16(const uint16_t *logits, int64_t rows, int64_t vocab,
                        int64_t row_stride, int32_t *out)
{
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t *row = logits + r * row_stride;
        int64_t best = 0;
        float bv = oracle_bf16_to_f32(row[0]);
        if (!isnan(bv)) {
            for (int64_t c = 1; c < vocab; ++c) {
                float v = oracle_bf16_to_f32(row[c]);
                if (isnan(v)) {
                    best = c;
                    break;
                }
                if (v > bv) {
                    bv = v;
                    best = c;
                }
            }
        }
        out[r] = (int32_t)best;
    }
}

/* verify_greedy_proposals (engine/speculative.py:11-30) for a whole verify
 * batch.  Sequence i owns verify rows [cu_q[i], cu_q[i+1]); row j is the
 * target token at input position base-1+j (llm_engine.py:130-137), so the
 * proposal checked against row j is the verify input token of row j+1
 * (model_runner.py:770-771 builds input_ids = seq[base-1 : base+k]).
 * accept_len[i] = first j with proposal_j != argmax[row j] (else q_i-1);
 * bonus[i] = argmax[row accept_len[i]] (the replacement or bonus token,
 * speculative.py:22-29).  An empty sequence (q_i == 0) gives 0 and -1. */
void oracle_accept(const int32_t *cu_q, int32_t num_seqs, const int32_t *argmax,
                   const int64_t *input_ids, int32_t *accept_len, int32_t *bonus)
{
    for (int32_t i = 0; i < num_seqs; ++i) {
        int32_t start = cu_q[i], q = cu_q[i + 1] - cu_q[i];
        if (q <= 0) {
            accept_len[i] = 0;
            bonus[i] = -1;
            continue;
        }
        int32_t a = 0;
        while (a < q - 1 && input_ids[start + 1 + a] == (int64_t)argmax[start + a])
            ++a;
        accept_len[i] = a;
        bonus[i] = argmax[start + a];
    }
}

/* ------------------------------------------------------------------ */
/* K2: store_kvcache and rollback                                      */
/* ------------------------------------------------------------------ */

/* store_kvcache (layers/attention.py:14-43, wrapper :189-217): for each token
 * row t with a valid slot, cache row `slot` (Hkv*D contiguous elements) gets
 * key[t] and value[t].  kv_dtype 0 = bfloat16 (byte copy), 1 = float8_e4m3fn
 * (x / scale, then oracle_f32_to_e4m3).  The reference skips slot == -1; this
 * restatement skips every negative slot and every slot >= num_slots. */
void oracle_store_kv(const uint16_t *key, int64_t key_row_stride,
                     const uint16_t *value, int64_t value_row_stride,
                     void *k_cache, void *v_cache, int32_t kv_dtype,
                     const int32_t *slot_mapping, int32_t num_tokens,
                     int32_t row_elems, int64_t num_slots,
                     float k_scale, float v_scale)
{
    for (int32_t t = 0; t < num_tokens; ++t) {
        int64_t slot = slot_mapping[t];
        if (slot < 0 || slot >= num_slots)
            continue;
        const uint16_t *k = key + (int64_t)t * key_row_stride;
        const uint16_t *v = value + (int64_t)t * value_row_stride;
        if (kv_dtype == 0) {
            memcpy((uint16_t *)k_cache + slot * row_elems, k, (size_t)row_elems * 2);
            memcpy((uint16_t *)v_cache + slot * row_elems, v, (size_t)row_elems * 2);
        } else {
            uint8_t *kc = (uint8_t *)k_cache + slot * row_elems;
            uint8_t *vc = (uint8_t *)v_cache + slot * row_elems;
            for (int32_t e = 0; e < row_elems; ++e) {
                kc[e] = oracle_f32_to_e4m3(oracle_bf16_to_f32(k[e]) / k_scale);
                vc[e] = oracle_f32_to_e4m3(oracle_bf16_to_f32(v[e]) / v_scale);
            }
        }
    }
}

/* Rollback of rejected draft rows after acceptance.  The reference's rollback
 * is logical (scheduler.py:165-170 truncates the token list,
 * block_manager.py:197-205 frees tail blocks); rejected K/V bytes stay in the
 * cache unread because the context length no longer covers them.  The device
 * mirror: rows j > accept_len[i] of sequence i are rejected, their slot is set
 * to -1 and the sequence's key count drops by the number of rejected rows.
 * With poison != 0 the rejected cache rows are also zeroed. */
void oracle_rollback(const int32_t *cu_q, const int32_t *accept_len, int32_t num_seqs,
                     int32_t *slot_mapping, int32_t *seqlens_k,
                     void *k_cache, void *v_cache, int32_t kv_dtype,
                     int32_t row_elems, int64_t num_slots, int32_t poison)
{
    size_t esz = kv_dtype == 0 ? 2 : 1;
    for (int32_t i = 0; i < num_seqs; ++i) {
        int32_t start = cu_q[i], q = cu_q[i + 1] - cu_q[i];
        int32_t a = accept_len[i];
        if (a < 0)
            a = 0;
        if (a > q - 1)
            a = q - 1;
        int32_t rejected = 0;
        for (int32_t j = a + 1; j < q; ++j) {
            int64_t slot = slot_mapping[start + j];
            if (poison && slot >= 0 && slot < num_slots) {
                memset((char *)k_cache + slot * row_elems * esz, 0, row_elems * esz);
                memset((char *)v_cache + slot * row_elems * esz, 0, row_elems * esz);
            }
            slot_mapping[start + j] = -1;
            ++rejected;
        }
        seqlens_k[i] -= rejected;
    }
}

/* ------------------------------------------------------------------ */
/* K3: EAGLE3 aux hidden-state add + concat + row gather               */
/* ------------------------------------------------------------------ */

/* models/qwen3.py:284-289 appends bf16(hidden + residual) after each aux
 * layer and concatenates them on the last dim; model_runner.py:1073 and
 * :1236-1242 then slice the rows each sequence commits.  Closed form:
 * out[r, l*H + c] = bf16(f32(h_l[src[r], c]) + f32(res_l[src[r], c])). */
void oracle_aux_gather(const uint16_t *const *hidden, const uint16_t *const *residual,
                       int32_t num_layers, int64_t row_stride, int32_t hidden_size,
                       const int32_t *src_rows, int32_t num_rows,
                       uint16_t *out, int64_t out_row_stride)
{
    for (int32_t r = 0; r < num_rows; ++r) {
        int64_t s = src_rows[r];
        for (int32_t l = 0; l < num_layers; ++l) {
            const uint16_t *h = hidden[l] + s * row_stride;
            const uint16_t *res = residual[l] + s * row_stride;
            uint16_t *o = out + (int64_t)r * out_row_stride + (int64_t)l * hidden_size;
            for (int32_t c = 0; c < hidden_size; ++c)
                o[c] = oracle_f32_to_bf16(oracle_bf16_to_f32(h[c]) + oracle_bf16_to_f32(res[c]));
        }
    }
}

/* ------------------------------------------------------------------ */
/* K1: paged verify attention                                          */
/* ------------------------------------------------------------------ */

static double cache_elem(const void *cache, int32_t kv_dtype, int64_t idx)
{
    if (kv_dtype == 0)
        return (double)oracle_bf16_to_f32(((const uint16_t *)cache)[idx]);
    return (double)oracle_e4m3_to_f32(((const uint8_t *)cache)[idx]);
}

/* Textbook attention over a paged cache, the operation the reference hands to
 * flash_attn_varlen_func(q, k_cache, v_cache, cu_seqlens_q, cu_seqlens_k, ...,
 * causal=True, block_table) in layers/attention.py:385-395 (and to
 * flash_attn_with_kvcache for one query row, :396-399).
 * Sequence i has q_i = cu_q[i+1]-cu_q[i] query rows and L_i = seqlens_k[i]
 * keys (the new rows included).  Causality is bottom-right aligned: query row
 * j sees keys [0, L_i - q_i + j].  Key n of sequence i lives in physical block
 * block_tables[i*bt_stride + n/block_size], offset n%block_size.  GQA: query
 * head h reads kv head h / (Hq/Hkv).
 *   out = softmax(q.K^T * scale * k_scale) . V * v_scale
 * accumulated in double; a row with no visible key produces zeros.
 * q strides and cache strides are in elements; out is [T, Hq, D] float. */
void oracle_paged_attention(const uint16_t *q, int64_t q_row_stride, int64_t q_head_stride,
                            const void *k_cache, const void *v_cache, int32_t kv_dtype,
                            int64_t blk_stride, int64_t tok_stride, int64_t head_stride,
                            const int32_t *cu_q, const int32_t *seqlens_k,
                            const int32_t *block_tables, int64_t bt_stride,
                            int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                            int32_t head_dim, int32_t block_size, double softmax_scale,
                            double k_scale, double v_scale, float *out)
{
    int32_t group = num_q_heads / num_kv_heads;
    for (int32_t i = 0; i < num_seqs; ++i) {
        int32_t qn = cu_q[i + 1] - cu_q[i];
        int32_t L = seqlens_k[i];
        const int32_t *bt = block_tables + (int64_t)i * bt_stride;
        for (int32_t j = 0; j < qn; ++j) {
            int64_t t = cu_q[i] + j;
            int32_t visible = L - qn + j + 1;
            if (visible > L)
                visible = L;
            for (int32_t h = 0; h < num_q_heads; ++h) {
                float *o = out + (t * num_q_heads + h) * head_dim;
                const uint16_t *qr = q + t * q_row_stride + (int64_t)h * q_head_stride;
                int32_t kvh = h / group;
                if (visible <= 0) {
                    for (int32_t d = 0; d < head_dim; ++d)
                        o[d] = 0.0f;
                    continue;
                }
                double m = -INFINITY;
                for (int32_t n = 0; n < visible; ++n) {
                    int64_t base = (int64_t)bt[n / block_size] * blk_stride +
                                   (int64_t)(n % block_size) * tok_stride + (int64_t)kvh * head_stride;
                    double s = 0.0;
                    for (int32_t d = 0; d < head_dim; ++d)
                        s += (double)oracle_bf16_to_f32(qr[d]) * cache_elem(k_cache, kv_dtype, base + d);
                    s *= softmax_scale * k_scale;
                    if (s > m)
                        m = s;
                }
                double denom = 0.0;
                double acc[1024];
                for (int32_t d = 0; d < head_dim; ++d)
                    acc[d] = 0.0;
                for (int32_t n = 0; n < visible; ++n) {
                    int64_t base = (int64_t)bt[n / block_size] * blk_stride +
                                   (int64_t)(n % block_size) * tok_stride + (int64_t)kvh * head_stride;
                    double s = 0.0;
                    for (int32_t d = 0; d < head_dim; ++d)
                        s += (double)oracle_bf16_to_f32(qr[d]) * cache_elem(k_cache, kv_dtype, base + d);
                    s *= softmax_scale * k_scale;
                    double p = exp(s - m);
                    denom += p;
                    for (int32_t d = 0; d < head_dim; ++d)
                        acc[d] += p * cache_elem(v_cache, kv_dtype, base + d);
                }
                for (int32_t d = 0; d < head_dim; ++d)
                    o[d] = (float)(acc[d] / denom * v_scale);
            }
        }
    }
}

/* Restatement of the reference's FP8 paged decode kernel
 * (layers/attention.py:85-182, launched by :249-293): one (row, q-head) at a
 * time, fp32 online softmax over 64-key tiles read through the row's block
 * table; scores = sum(q * k) * (scale * k_scale), keys >= context_len masked,
 * out = acc / sum * v_scale.  Sums inside a tile run in index order (Triton's
 * tl.sum order is unspecified), so agreement with the reference is to fp32
 * rounding, not bitwise.  Caches are float8_e4m3fn. */
void oracle_fp8_paged_decode(const uint16_t *q, int64_t q_row_stride, int64_t q_head_stride,
                             const uint8_t *k_cache, const uint8_t *v_cache,
                             int64_t blk_stride, int64_t tok_stride, int64_t head_stride,
                             const int32_t *context_lens, const int32_t *block_tables,
                             int64_t bt_stride, int32_t num_rows, int32_t num_q_heads,
                             int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                             float softmax_scale, float k_scale, float v_scale, float *out)
{
    enum { BLOCK_N = 64 };
    int32_t group = num_q_heads / num_kv_heads;
    for (int32_t t = 0; t < num_rows; ++t) {
        const int32_t *bt = block_tables + (int64_t)t * bt_stride;
        int32_t ctx = context_lens[t];
        for (int32_t h = 0; h < num_q_heads; ++h) {
            int32_t kvh = h / group;
            const uint16_t *qr = q + (int64_t)t * q_row_stride + (int64_t)h * q_head_stride;
            float running_max = -INFINITY, running_sum = 0.0f;
            float acc[1024];
            for (int32_t d = 0; d < head_dim; ++d)
                acc[d] = 0.0f;
            for (int32_t start = 0; start < ctx; start += BLOCK_N) {
                float scores[BLOCK_N];
                float tile_max = -INFINITY;
                for (int32_t n = 0; n < BLOCK_N; ++n) {
                    int32_t pos = start + n;
                    if (pos >= ctx) {
                        scores[n] = -INFINITY;
                        continue;
                    }
                    int64_t base = (int64_t)bt[pos / block_size] * blk_stride +
                                   (int64_t)(pos % block_size) * tok_stride + (int64_t)kvh * head_stride;
                    float s = 0.0f;
                    for (int32_t d = 0; d < head_dim; ++d)
                        s += oracle_bf16_to_f32(qr[d]) * oracle_e4m3_to_f32(k_cache[base + d]);
                    s = s * (softmax_scale * k_scale);
                    scores[n] = s;
                    if (s > tile_max)
                        tile_max = s;
                }
                float next_max = running_max > tile_max ? running_max : tile_max;
                float prev_scale = expf(running_max - next_max);
                float wsum = 0.0f;
                for (int32_t d = 0; d < head_dim; ++d)
                    acc[d] *= prev_scale;
                for (int32_t n = 0; n < BLOCK_N; ++n) {
                    int32_t pos = start + n;
                    float w = expf(scores[n] - next_max);
                    wsum += w;
                    if (pos >= ctx)
                        continue;
                    int64_t base = (int64_t)bt[pos / block_size] * blk_stride +
                                   (int64_t)(pos % block_size) * tok_stride + (int64_t)kvh * head_stride;
                    for (int32_t d = 0; d < head_dim; ++d)
                        acc[d] += oracle_e4m3_to_f32(v_cache[base + d]) * w;
                }
                running_sum = running_sum * prev_scale + wsum;
                running_max = next_max;
            }
            float *o = out + ((int64_t)t * num_q_heads + h) * head_dim;
            for (int32_t d = 0; d < head_dim; ++d)
                o[d] = acc[d] / running_sum * v_scale;
        }
    }
}
