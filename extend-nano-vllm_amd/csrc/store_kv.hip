// K2: KV-cache slot write (store_kvcache) and rollback of rejected draft rows.
//
// Store: one 256-thread block per token; each thread moves 16-byte vectors
// (8 bf16) of the key and value rows, head by head, to the token's place in
// the paged cache.  The cache is addressed through its block, token and
// head strides, so both the token-major layout [blocks, block_size, Hkv, D]
// and a head-major one ([blocks, Hkv, block_size, D] seen through a permuted
// view) are written in place.  This is an HBM copy: per token it reads
// 2 * Hkv * D * 2 bytes and writes the same (half for fp8).
// Rollback: one block per sequence; thread j handles verify row j.
#include "common.h"

namespace nva {
namespace {

constexpr int kStoreThreads = 256;

struct CacheGeometry {
  int64_t blk_stride, tok_stride, head_stride;  // elements
  int32_t block_size;
  int64_t num_slots;                            // num_blocks * block_size
};

template <bool FP8>
__global__ void __launch_bounds__(kStoreThreads)
store_kvcache_kernel(const uint16_t* __restrict__ key, int64_t key_row_stride,
                     const uint16_t* __restrict__ value, int64_t value_row_stride,
                     void* __restrict__ k_cache, void* __restrict__ v_cache,
                     const int32_t* __restrict__ slot_mapping, int32_t num_tokens,
                     int32_t num_heads, int32_t head_dim, CacheGeometry geo, bool vec,
                     const float* __restrict__ k_scale_p, const float* __restrict__ v_scale_p) {
  const int32_t t = blockIdx.x;
  if (t >= num_tokens) return;
  const int64_t slot = slot_mapping[t];
  if (slot < 0 || slot >= geo.num_slots) return;
  const int64_t base = (slot / geo.block_size) * geo.blk_stride + (slot % geo.block_size) * geo.tok_stride;
  const uint16_t* k = key + static_cast<int64_t>(t) * key_row_stride;
  const uint16_t* v = value + static_cast<int64_t>(t) * value_row_stride;
  float ks = 1.0f, vs = 1.0f;
  if constexpr (FP8) {
    ks = k_scale_p ? *k_scale_p : 1.0f;
    vs = v_scale_p ? *v_scale_p : 1.0f;
  }
  if (vec) {
    // element e = 8 * i of the row: head e / D, offset e % D (D % 8 == 0)
    const int vpr = head_dim / 8;
    for (int i = threadIdx.x; i < num_heads * vpr; i += kStoreThreads) {
      const int h = i / vpr, j = i % vpr;
      const int64_t dst = base + h * geo.head_stride + 8 * j;
      const uint4 kw = reinterpret_cast<const uint4*>(k)[i];
      const uint4 vw = reinterpret_cast<const uint4*>(v)[i];
      if constexpr (!FP8) {
        store_streamed(reinterpret_cast<uint4*>(static_cast<uint16_t*>(k_cache) + dst), kw);
        store_streamed(reinterpret_cast<uint4*>(static_cast<uint16_t*>(v_cache) + dst), vw);
      } else {
        const uint32_t kin[4] = {kw.x, kw.y, kw.z, kw.w};
        const uint32_t vin[4] = {vw.x, vw.y, vw.z, vw.w};
        uint32_t ko[2] = {0, 0}, vo[2] = {0, 0};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t kb = (kin[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
          const uint32_t vb = (vin[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
          ko[e >> 2] |= f32_to_e4m3(bf16_to_f32(kb) / ks) << ((e & 3) * 8);
          vo[e >> 2] |= f32_to_e4m3(bf16_to_f32(vb) / vs) << ((e & 3) * 8);
        }
        *reinterpret_cast<uint2*>(static_cast<uint8_t*>(k_cache) + dst) = make_uint2(ko[0], ko[1]);
        *reinterpret_cast<uint2*>(static_cast<uint8_t*>(v_cache) + dst) = make_uint2(vo[0], vo[1]);
      }
    }
  } else {
    for (int i = threadIdx.x; i < num_heads * head_dim; i += kStoreThreads) {
      const int64_t dst = base + (i / head_dim) * geo.head_stride + i % head_dim;
      if constexpr (!FP8) {
        static_cast<uint16_t*>(k_cache)[dst] = k[i];
        static_cast<uint16_t*>(v_cache)[dst] = v[i];
      } else {
        static_cast<uint8_t*>(k_cache)[dst] = static_cast<uint8_t>(f32_to_e4m3(bf16_to_f32(k[i]) / ks));
        static_cast<uint8_t*>(v_cache)[dst] = static_cast<uint8_t>(f32_to_e4m3(bf16_to_f32(v[i]) / vs));
      }
    }
  }
}

__global__ void __launch_bounds__(256)
rollback_kernel(const int32_t* __restrict__ cu_q, const int32_t* __restrict__ accept_len,
                int32_t num_seqs, int32_t* __restrict__ slot_mapping, int32_t* __restrict__ seqlens_k,
                uint8_t* __restrict__ k_cache, uint8_t* __restrict__ v_cache, int32_t num_layers,
                int64_t layer_stride_bytes, int64_t row_bytes, int64_t num_slots, int poison) {
  const int32_t i = blockIdx.x;
  if (i >= num_seqs) return;
  const int32_t start = cu_q[i];
  const int32_t q = cu_q[i + 1] - start;
  int32_t a = accept_len[i];
  a = a < 0 ? 0 : a;
  a = a > q - 1 ? q - 1 : a;
  const int32_t rejected = q - 1 - a;
  if (rejected <= 0) return;
  // Poison first (reads the slots before they are cleared below).
  if (poison) {
    for (int32_t j = a + 1; j < q; ++j) {
      const int64_t slot = slot_mapping[start + j];
      if (slot < 0 || slot >= num_slots) continue;
      for (int32_t l = 0; l < num_layers; ++l) {
        uint8_t* kr = k_cache + l * layer_stride_bytes + slot * row_bytes;
        uint8_t* vr = v_cache + l * layer_stride_bytes + slot * row_bytes;
        for (int64_t b = threadIdx.x; b < row_bytes; b += blockDim.x) {
          kr[b] = 0;
          vr[b] = 0;
        }
      }
    }
    __syncthreads();
  }
  for (int32_t j = a + 1 + threadIdx.x; j < q; j += blockDim.x) slot_mapping[start + j] = -1;
  if (threadIdx.x == 0) seqlens_k[i] -= rejected;
}

int launch_store(const void* key, int64_t key_row_stride, const void* value,
                 int64_t value_row_stride, void* k_cache, void* v_cache, int kv_dtype,
                 const int32_t* slot_mapping, int32_t num_tokens, int32_t num_kv_heads,
                 int32_t head_dim, const CacheGeometry& geo, const float* k_scale,
                 const float* v_scale, hipStream_t s) {
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || geo.num_slots < 0) return NVA_ERR_ARG;
  if (kv_dtype != NVA_KV_BF16 && kv_dtype != NVA_KV_FP8_E4M3) return NVA_ERR_ARG;
  if (num_tokens == 0) return NVA_OK;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping) return NVA_ERR_ARG;
  const int32_t row_elems = num_kv_heads * head_dim;
  if (key_row_stride < row_elems || value_row_stride < row_elems) return NVA_ERR_ARG;
  // 16-byte source vectors; destination vectors of 8 elements (16 B bf16,
  // 8 B fp8) at every (block, token, head) start
  const int64_t dst_align = kv_dtype == NVA_KV_BF16 ? 16 : 8;
  const int64_t esz = kv_dtype == NVA_KV_BF16 ? 2 : 1;
  const bool vec = head_dim % 8 == 0 && key_row_stride % 8 == 0 && value_row_stride % 8 == 0 &&
                   aligned16(key) && aligned16(value) &&
                   reinterpret_cast<uintptr_t>(k_cache) % dst_align == 0 &&
                   reinterpret_cast<uintptr_t>(v_cache) % dst_align == 0 &&
                   (geo.blk_stride * esz) % dst_align == 0 && (geo.tok_stride * esz) % dst_align == 0 &&
                   (geo.head_stride * esz) % dst_align == 0;
  dim3 grid(num_tokens);
  if (kv_dtype == NVA_KV_BF16) {
    store_kvcache_kernel<false><<<grid, kStoreThreads, 0, s>>>(
        static_cast<const uint16_t*>(key), key_row_stride, static_cast<const uint16_t*>(value),
        value_row_stride, k_cache, v_cache, slot_mapping, num_tokens, num_kv_heads, head_dim, geo,
        vec, k_scale, v_scale);
  } else {
    store_kvcache_kernel<true><<<grid, kStoreThreads, 0, s>>>(
        static_cast<const uint16_t*>(key), key_row_stride, static_cast<const uint16_t*>(value),
        value_row_stride, k_cache, v_cache, slot_mapping, num_tokens, num_kv_heads, head_dim, geo,
        vec, k_scale, v_scale);
  }
  return launch_status();
}

}  // namespace
}  // namespace nva

using namespace nva;

extern "C" int nva_store_kvcache(const void* key, int64_t key_row_stride, const void* value,
                                 int64_t value_row_stride, void* k_cache, void* v_cache,
                                 int kv_dtype, const int32_t* slot_mapping, int32_t num_tokens,
                                 int32_t num_kv_heads, int32_t head_dim, int64_t num_slots,
                                 const float* k_scale, const float* v_scale, void* stream) {
  // token-major rows: slot s starts at s * Hkv * D, head h at h * D
  const int64_t row = static_cast<int64_t>(num_kv_heads) * head_dim;
  const CacheGeometry geo{row, row, head_dim, 1, num_slots};
  return launch_store(key, key_row_stride, value, value_row_stride, k_cache, v_cache, kv_dtype,
                      slot_mapping, num_tokens, num_kv_heads, head_dim, geo, k_scale, v_scale,
                      static_cast<hipStream_t>(stream));
}

extern "C" int nva_store_kvcache_paged(const void* key, int64_t key_row_stride, const void* value,
                                       int64_t value_row_stride, void* k_cache, void* v_cache,
                                       int kv_dtype, int64_t cache_block_stride,
                                       int64_t cache_token_stride, int64_t cache_head_stride,
                                       int32_t num_blocks, int32_t block_size,
                                       const int32_t* slot_mapping, int32_t num_tokens,
                                       int32_t num_kv_heads, int32_t head_dim,
                                       const float* k_scale, const float* v_scale, void* stream) {
  if (num_blocks < 0 || block_size <= 0 || cache_block_stride < 0 || cache_token_stride < 0 ||
      cache_head_stride < 0)
    return NVA_ERR_ARG;
  const CacheGeometry geo{cache_block_stride, cache_token_stride, cache_head_stride, block_size,
                          static_cast<int64_t>(num_blocks) * block_size};
  return launch_store(key, key_row_stride, value, value_row_stride, k_cache, v_cache, kv_dtype,
                      slot_mapping, num_tokens, num_kv_heads, head_dim, geo, k_scale, v_scale,
                      static_cast<hipStream_t>(stream));
}

extern "C" int nva_rollback(const int32_t* cu_seqlens_q, const int32_t* accept_len,
                            int32_t num_seqs, int32_t* slot_mapping, int32_t* seqlens_k,
                            void* k_cache, void* v_cache, int kv_dtype, int32_t num_layers,
                            int64_t layer_stride, int32_t row_elems, int64_t num_slots, int poison,
                            void* stream) {
  if (num_seqs < 0) return NVA_ERR_ARG;
  if (num_seqs == 0) return NVA_OK;
  if (!cu_seqlens_q || !accept_len || !slot_mapping || !seqlens_k) return NVA_ERR_ARG;
  if (kv_dtype != NVA_KV_BF16 && kv_dtype != NVA_KV_FP8_E4M3) return NVA_ERR_ARG;
  const int64_t esz = kv_dtype == NVA_KV_BF16 ? 2 : 1;
  if (poison) {
    if (!k_cache || !v_cache || num_layers <= 0 || row_elems <= 0 || num_slots < 0 ||
        layer_stride < static_cast<int64_t>(row_elems) * num_slots)
      return NVA_ERR_ARG;
  }
  rollback_kernel<<<num_seqs, 256, 0, static_cast<hipStream_t>(stream)>>>(
      cu_seqlens_q, accept_len, num_seqs, slot_mapping, seqlens_k,
      static_cast<uint8_t*>(k_cache), static_cast<uint8_t*>(v_cache), num_layers,
      layer_stride * esz, static_cast<int64_t>(row_elems) * esz, num_slots, poison);
  return launch_status();
}
