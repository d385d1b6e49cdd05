// Supporting per-token kernels of the target/draft forward that sit between
// the projection GEMMs: RMSNorm (optionally fused with the residual add),
// per-head q/k RMSNorm fused with neox RoPE, and SiLU-and-mul.  They are
// memory bound and replace chains of small eager torch ops; rounding follows
// the reference's eager formulas step by step (see each kernel).
#include "common.h"

namespace nva {
namespace {

constexpr int kNormThreads = 256;
constexpr int kMaxHidden = 1 << 20;
constexpr int kRowVecs = 4;    // 16-byte vectors per thread a register-resident row may use

__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int m = kWave / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormThreads / kWave; ++i) s += red[i];
  __syncthreads();
  return s;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = kWave / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

// RMSNorm of one row, optionally after adding a residual row:
//   s = f32(x) (+ f32(residual));  residual_out = bf16(s)
//   out = bf16( bf16(s * rsqrt(mean(s^2) + eps)) * weight )
// (nanovllm/layers/layernorm.py:70-82 and :91-107: the fp32 sum is normalised,
// rounded to bf16, then multiplied by the bf16 weight in bf16.)  ROUND
// normalises the bf16-rounded sum instead: a bf16 tensor add followed by
// RMSNorm without residual (the EAGLE3 draft layer, eagle3.py:141-146).
template <bool ADD, bool ROUND = false>
__global__ void __launch_bounds__(kNormThreads)
rms_norm_kernel(const uint16_t* __restrict__ x, int64_t x_stride,
                const uint16_t* __restrict__ residual, int64_t res_stride,
                const uint16_t* __restrict__ weight, uint16_t* __restrict__ out,
                int64_t out_stride, uint16_t* __restrict__ residual_out, int64_t res_out_stride,
                int32_t hidden, float eps, bool vec) {
  __shared__ float red[kNormThreads / kWave];
  const int64_t r = blockIdx.x;
  const uint16_t* xr = x + r * x_stride;
  const uint16_t* rr = ADD ? residual + r * res_stride : nullptr;
  uint16_t* o = out + r * out_stride;
  uint16_t* ro = ADD ? residual_out + r * res_out_stride : nullptr;
  float ss = 0.0f;
  if (vec && hidden <= 8 * kNormThreads * kRowVecs) {
    // Rows of up to 8 * kNormThreads * kRowVecs elements stay in registers:
    // every load (x, residual, weight) is issued up front and the second
    // pass normalises the values held, instead of re-reading them after the
    // reduction.  The per-thread sums run in the same order as the loop
    // below, so the result is bit-identical to it.
    float s[kRowVecs][8];
    uint4 w[kRowVecs];
#pragma unroll
    for (int i = 0; i < kRowVecs; ++i) {
      const int v = threadIdx.x + i * kNormThreads;
      if (v < hidden / 8) {
        const uint4 a = reinterpret_cast<const uint4*>(xr)[v];
        uint4 b = make_uint4(0, 0, 0, 0);
        if (ADD) b = reinterpret_cast<const uint4*>(rr)[v];
        w[i] = reinterpret_cast<const uint4*>(weight)[v];
        const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
        uint32_t so[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float lo = bf16_to_f32(aw[e] & 0xFFFFu), hi = bf16_to_f32(aw[e] >> 16);
          if (ADD) {
            lo += bf16_to_f32(bw[e] & 0xFFFFu);
            hi += bf16_to_f32(bw[e] >> 16);
            so[e] = static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
            if (ROUND) {
              lo = bf16_to_f32(so[e] & 0xFFFFu);
              hi = bf16_to_f32(so[e] >> 16);
            }
          }
          s[i][2 * e] = lo;
          s[i][2 * e + 1] = hi;
          ss += lo * lo + hi * hi;
        }
        if (ADD) reinterpret_cast<uint4*>(ro)[v] = make_uint4(so[0], so[1], so[2], so[3]);
      }
    }
    const float inv = rsqrtf(block_sum(ss, red) / static_cast<float>(hidden) + eps);
#pragma unroll
    for (int i = 0; i < kRowVecs; ++i) {
      const int v = threadIdx.x + i * kNormThreads;
      if (v < hidden / 8) {
        const uint32_t ww[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
        uint32_t ov[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float nl = bf16_to_f32(f32_to_bf16(s[i][2 * e] * inv)) * bf16_to_f32(ww[e] & 0xFFFFu);
          const float nh = bf16_to_f32(f32_to_bf16(s[i][2 * e + 1] * inv)) * bf16_to_f32(ww[e] >> 16);
          ov[e] = static_cast<uint32_t>(f32_to_bf16(nl)) | (static_cast<uint32_t>(f32_to_bf16(nh)) << 16);
        }
        reinterpret_cast<uint4*>(o)[v] = make_uint4(ov[0], ov[1], ov[2], ov[3]);
      }
    }
    return;
  }
  // pass 1: sum of squares of the fp32 (residual-added) row
  if (vec) {
    for (int v = threadIdx.x; v < hidden / 8; v += kNormThreads) {
      const uint4 a = reinterpret_cast<const uint4*>(xr)[v];
      uint4 b = make_uint4(0, 0, 0, 0);
      if (ADD) b = reinterpret_cast<const uint4*>(rr)[v];
      const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
      uint32_t so[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float lo = bf16_to_f32(aw[e] & 0xFFFFu), hi = bf16_to_f32(aw[e] >> 16);
        if (ADD) {
          lo += bf16_to_f32(bw[e] & 0xFFFFu);
          hi += bf16_to_f32(bw[e] >> 16);
          so[e] = static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
          if (ROUND) {
            lo = bf16_to_f32(so[e] & 0xFFFFu);
            hi = bf16_to_f32(so[e] >> 16);
          }
        }
        ss += lo * lo + hi * hi;
      }
      if (ADD) reinterpret_cast<uint4*>(ro)[v] = make_uint4(so[0], so[1], so[2], so[3]);
    }
  } else {
    for (int c = threadIdx.x; c < hidden; c += kNormThreads) {
      float v = bf16_to_f32(xr[c]);
      if (ADD) {
        v += bf16_to_f32(rr[c]);
        ro[c] = f32_to_bf16(v);
        if (ROUND) v = bf16_to_f32(f32_to_bf16(v));
      }
      ss += v * v;
    }
  }
  const float inv = rsqrtf(block_sum(ss, red) / static_cast<float>(hidden) + eps);
  // pass 2: recompute the fp32 row (exactly the same sums) and normalise
  if (vec) {
    for (int v = threadIdx.x; v < hidden / 8; v += kNormThreads) {
      const uint4 a = reinterpret_cast<const uint4*>(xr)[v];
      uint4 b = make_uint4(0, 0, 0, 0);
      if (ADD) b = reinterpret_cast<const uint4*>(rr)[v];
      const uint4 w = reinterpret_cast<const uint4*>(weight)[v];
      const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
      uint32_t ov[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float lo = bf16_to_f32(aw[e] & 0xFFFFu), hi = bf16_to_f32(aw[e] >> 16);
        if (ADD) {
          lo += bf16_to_f32(bw[e] & 0xFFFFu);
          hi += bf16_to_f32(bw[e] >> 16);
          if (ROUND) {
            lo = bf16_to_f32(f32_to_bf16(lo));
            hi = bf16_to_f32(f32_to_bf16(hi));
          }
        }
        const float nl = bf16_to_f32(f32_to_bf16(lo * inv)) * bf16_to_f32(ww[e] & 0xFFFFu);
        const float nh = bf16_to_f32(f32_to_bf16(hi * inv)) * bf16_to_f32(ww[e] >> 16);
        ov[e] = static_cast<uint32_t>(f32_to_bf16(nl)) | (static_cast<uint32_t>(f32_to_bf16(nh)) << 16);
      }
      reinterpret_cast<uint4*>(o)[v] = make_uint4(ov[0], ov[1], ov[2], ov[3]);
    }
  } else {
    for (int c = threadIdx.x; c < hidden; c += kNormThreads) {
      float v = bf16_to_f32(xr[c]);
      if (ADD) v += bf16_to_f32(rr[c]);
      if (ROUND) v = bf16_to_f32(f32_to_bf16(v));
      const float n = bf16_to_f32(f32_to_bf16(v * inv));
      o[c] = f32_to_bf16(n * bf16_to_f32(weight[c]));
    }
  }
}

// Per-head RMSNorm (optional) + neox rotary embedding for the q and k heads
// of a fused QKV row; one wave per head, lane l owns elements l and l + 64
// (the two halves the rotation pairs).
//   norm:  x = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w)   (qwen3.py:87-96)
//   rope:  y1 = x1*cos - x2*sin, y2 = x2*cos + x1*sin in fp32, rounded to bf16
//          with cos/sin = cos_sin[pos][i], cos_sin[pos][64 + i]
//          (rotary_embedding.py:6-48)
__global__ void __launch_bounds__(kNormThreads)
qk_norm_rope_kernel(const uint16_t* __restrict__ qkv, int64_t row_stride,
                    const int64_t* __restrict__ positions, const uint16_t* __restrict__ q_w,
                    const uint16_t* __restrict__ k_w, const float* __restrict__ cos_sin,
                    int32_t max_pos, int32_t num_tokens, int32_t hq, int32_t hkv, float eps,
                    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_out) {
  const int t = blockIdx.y;
  const int head = blockIdx.x * (kNormThreads / kWave) + threadIdx.x / kWave;
  const int lane = wave_lane();
  if (t >= num_tokens || head >= hq + hkv) return;
  const bool is_q = head < hq;
  const uint16_t* src = qkv + static_cast<int64_t>(t) * row_stride + static_cast<int64_t>(head) * 128;
  // every load is issued before the first use (the position's cos/sin row
  // behind the position itself, both ahead of the norm's reduction)
  int64_t pos = positions[t];
  float x1 = bf16_to_f32(src[lane]);
  float x2 = bf16_to_f32(src[lane + 64]);
  const uint16_t* w = is_q ? q_w : k_w;
  const float w1 = w ? bf16_to_f32(w[lane]) : 1.0f;
  const float w2 = w ? bf16_to_f32(w[lane + 64]) : 1.0f;
  pos = pos < 0 ? 0 : (pos >= max_pos ? max_pos - 1 : pos);
  const float c = cos_sin[pos * 128 + lane];
  const float s = cos_sin[pos * 128 + 64 + lane];
  if (w) {
    const float inv = rsqrtf(wave_sum(x1 * x1 + x2 * x2) / 128.0f + eps);
    x1 = bf16_to_f32(f32_to_bf16(bf16_to_f32(f32_to_bf16(x1 * inv)) * w1));
    x2 = bf16_to_f32(f32_to_bf16(bf16_to_f32(f32_to_bf16(x2 * inv)) * w2));
  }
  const float y1 = x1 * c - x2 * s;
  const float y2 = x2 * c + x1 * s;
  uint16_t* dst = is_q ? q_out + (static_cast<int64_t>(t) * hq + head) * 128
                       : k_out + (static_cast<int64_t>(t) * hkv + (head - hq)) * 128;
  dst[lane] = f32_to_bf16(y1);
  dst[lane + 64] = f32_to_bf16(y2);
}

// qk_norm_rope_kernel and store_kvcache in one launch: waves [0, hq) take
// the query heads (normalised, rotated, written to q_out), waves [hq, hq +
// hkv) the key heads (normalised, rotated, rounded to bf16, then written to
// the paged cache at the token's slot, e4m3(bf16 / k_scale) for FP8) and
// waves [hq + hkv, hq + 2 hkv) the value heads (copied to the cache, e4m3(
// bf16 / v_scale) for FP8).  Every value written is the one the two separate
// kernels write; a slot that is negative or past the cache is skipped.
struct SlotPages {
  int64_t blk_stride, tok_stride, head_stride;  // elements
  int32_t block_size;
  int64_t num_slots;
};

template <bool FP8>
__device__ __forceinline__ void put_cache_pair(void* cache, int64_t dst, int lane, uint16_t a,
                                               uint16_t b, float scale) {
  if constexpr (FP8) {
    uint8_t* c = static_cast<uint8_t*>(cache) + dst;
    c[lane] = static_cast<uint8_t>(f32_to_e4m3(bf16_to_f32(a) / scale));
    c[lane + 64] = static_cast<uint8_t>(f32_to_e4m3(bf16_to_f32(b) / scale));
  } else {
    // one full 128-byte line per instruction (64 lanes x 2 bytes)
    uint16_t* c = static_cast<uint16_t*>(cache) + dst;
    store_streamed(c + lane, a);
    store_streamed(c + lane + 64, b);
  }
}

template <bool FP8>
__global__ void __launch_bounds__(kNormThreads)
qk_norm_rope_store_kernel(const uint16_t* __restrict__ qkv, int64_t row_stride,
                          const int64_t* __restrict__ positions, const uint16_t* __restrict__ q_w,
                          const uint16_t* __restrict__ k_w, const float* __restrict__ cos_sin,
                          int32_t max_pos, int32_t num_tokens, int32_t hq, int32_t hkv, float eps,
                          uint16_t* __restrict__ q_out, void* __restrict__ k_cache,
                          void* __restrict__ v_cache, SlotPages pages,
                          const int32_t* __restrict__ slot_mapping,
                          const float* __restrict__ k_scale_p, const float* __restrict__ v_scale_p) {
  const int t = blockIdx.y;
  const int head = blockIdx.x * (kNormThreads / kWave) + threadIdx.x / kWave;
  const int lane = wave_lane();
  if (t >= num_tokens || head >= hq + 2 * hkv) return;
  const uint16_t* src = qkv + static_cast<int64_t>(t) * row_stride + static_cast<int64_t>(head) * 128;
  int64_t dst = 0;
  if (head >= hq) {
    const int64_t slot = slot_mapping[t];
    if (slot < 0 || slot >= pages.num_slots) return;
    const int kvh = (head - hq) % hkv;
    dst = (slot / pages.block_size) * pages.blk_stride + (slot % pages.block_size) * pages.tok_stride +
          kvh * pages.head_stride;
  }
  if (head >= hq + hkv) {
    put_cache_pair<FP8>(v_cache, dst, lane, src[lane], src[lane + 64],
                        FP8 && v_scale_p ? *v_scale_p : 1.0f);
    return;
  }
  const bool is_q = head < hq;
  int64_t pos = positions[t];
  float x1 = bf16_to_f32(src[lane]);
  float x2 = bf16_to_f32(src[lane + 64]);
  const uint16_t* w = is_q ? q_w : k_w;
  const float w1 = w ? bf16_to_f32(w[lane]) : 1.0f;
  const float w2 = w ? bf16_to_f32(w[lane + 64]) : 1.0f;
  pos = pos < 0 ? 0 : (pos >= max_pos ? max_pos - 1 : pos);
  const float c = cos_sin[pos * 128 + lane];
  const float s = cos_sin[pos * 128 + 64 + lane];
  if (w) {
    const float inv = rsqrtf(wave_sum(x1 * x1 + x2 * x2) / 128.0f + eps);
    x1 = bf16_to_f32(f32_to_bf16(bf16_to_f32(f32_to_bf16(x1 * inv)) * w1));
    x2 = bf16_to_f32(f32_to_bf16(bf16_to_f32(f32_to_bf16(x2 * inv)) * w2));
  }
  const uint16_t y1 = f32_to_bf16(x1 * c - x2 * s);
  const uint16_t y2 = f32_to_bf16(x2 * c + x1 * s);
  if (is_q) {
    uint16_t* qd = q_out + (static_cast<int64_t>(t) * hq + head) * 128;
    store_streamed(qd + lane, y1);
    store_streamed(qd + lane + 64, y2);
  } else {
    put_cache_pair<FP8>(k_cache, dst, lane, y1, y2, FP8 && k_scale_p ? *k_scale_p : 1.0f);
  }
}

// out = bf16( bf16(silu(a)) * b ) for a row [a | b] (activation.py:11-14:
// F.silu in bf16, then a bf16 product).  The division stays IEEE: with the
// hardware reciprocal in its place silu(a)'s bf16 rounding flips next to
// rounding midpoints, and the product's second rounding then leaves the
// one-ulp bound against torch.
__device__ __forceinline__ uint16_t silu_mul_one(uint16_t a, uint16_t b) {
  const float av = bf16_to_f32(a);
  const float sv = bf16_to_f32(f32_to_bf16(av / (1.0f + __expf(-av))));
  return f32_to_bf16(sv * bf16_to_f32(b));
}

// vec: 16-byte vectors of 8 elements (rows and strides multiples of 8,
// 16-byte aligned); grid.x covers a row in kNormThreads * 8 elements
__global__ void __launch_bounds__(kNormThreads)
silu_mul_kernel(const uint16_t* __restrict__ x, int64_t x_stride, uint16_t* __restrict__ out,
                int64_t out_stride, int32_t inter, bool vec) {
  const int64_t r = blockIdx.y;
  const uint16_t* a = x + r * x_stride;
  const uint16_t* b = a + inter;
  uint16_t* o = out + r * out_stride;
  if (vec) {
    const int v = blockIdx.x * kNormThreads + threadIdx.x;
    if (v >= inter / 8) return;
    const uint4 av = reinterpret_cast<const uint4*>(a)[v];
    const uint4 bv = reinterpret_cast<const uint4*>(b)[v];
    const uint32_t aw[4] = {av.x, av.y, av.z, av.w}, bw[4] = {bv.x, bv.y, bv.z, bv.w};
    uint32_t ow[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      ow[e] = static_cast<uint32_t>(silu_mul_one(aw[e] & 0xFFFFu, bw[e] & 0xFFFFu)) |
              (static_cast<uint32_t>(silu_mul_one(aw[e] >> 16, bw[e] >> 16)) << 16);
    reinterpret_cast<uint4*>(o)[v] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    return;
  }
  for (int c = blockIdx.x * kNormThreads + threadIdx.x; c < inter; c += gridDim.x * kNormThreads)
    o[c] = silu_mul_one(a[c], b[c]);
}

}  // namespace
}  // namespace nva

using namespace nva;

extern "C" int nva_rms_norm(const void* x, int64_t x_row_stride, const void* weight, void* out,
                            int64_t out_row_stride, int32_t rows, int32_t hidden, float eps,
                            void* stream) {
  if (rows < 0 || hidden <= 0 || hidden > kMaxHidden) return NVA_ERR_ARG;
  if (rows == 0) return NVA_OK;
  if (!x || !weight || !out || x_row_stride < hidden || out_row_stride < hidden) return NVA_ERR_ARG;
  const bool vec = hidden % 8 == 0 && x_row_stride % 8 == 0 && out_row_stride % 8 == 0 &&
                   aligned16(x) && aligned16(weight) && aligned16(out);
  rms_norm_kernel<false><<<rows, kNormThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(x), x_row_stride, nullptr, 0,
      static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(out), out_row_stride, nullptr,
      0, hidden, eps, vec);
  return launch_status();
}

namespace {

template <bool ROUND>
int launch_add_rms_norm(const void* x, int64_t x_row_stride, const void* residual,
                        int64_t residual_row_stride, const void* weight, void* out,
                        int64_t out_row_stride, void* residual_out,
                        int64_t residual_out_row_stride, int32_t rows, int32_t hidden, float eps,
                        void* stream) {
  if (rows < 0 || hidden <= 0 || hidden > kMaxHidden) return NVA_ERR_ARG;
  if (rows == 0) return NVA_OK;
  if (!x || !residual || !weight || !out || !residual_out || x_row_stride < hidden ||
      residual_row_stride < hidden || out_row_stride < hidden || residual_out_row_stride < hidden)
    return NVA_ERR_ARG;
  // pass 2 re-reads x and residual: residual_out must not overwrite them
  if (residual_out == x || residual_out == residual) return NVA_ERR_ARG;
  const bool vec = hidden % 8 == 0 && x_row_stride % 8 == 0 && residual_row_stride % 8 == 0 &&
                   out_row_stride % 8 == 0 && residual_out_row_stride % 8 == 0 && aligned16(x) &&
                   aligned16(residual) && aligned16(weight) && aligned16(out) &&
                   aligned16(residual_out);
  rms_norm_kernel<true, ROUND><<<rows, kNormThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(x), x_row_stride, static_cast<const uint16_t*>(residual),
      residual_row_stride, static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(out),
      out_row_stride, static_cast<uint16_t*>(residual_out), residual_out_row_stride, hidden, eps,
      vec);
  return launch_status();
}

}  // namespace

extern "C" int nva_add_rms_norm(const void* x, int64_t x_row_stride, const void* residual,
                                int64_t residual_row_stride, const void* weight, void* out,
                                int64_t out_row_stride, void* residual_out,
                                int64_t residual_out_row_stride, int32_t rows, int32_t hidden,
                                float eps, void* stream) {
  return launch_add_rms_norm<false>(x, x_row_stride, residual, residual_row_stride, weight, out,
                                    out_row_stride, residual_out, residual_out_row_stride, rows,
                                    hidden, eps, stream);
}

extern "C" int nva_add_then_rms_norm(const void* x, int64_t x_row_stride, const void* residual,
                                     int64_t residual_row_stride, const void* weight, void* out,
                                     int64_t out_row_stride, void* sum_out,
                                     int64_t sum_out_row_stride, int32_t rows, int32_t hidden,
                                     float eps, void* stream) {
  return launch_add_rms_norm<true>(x, x_row_stride, residual, residual_row_stride, weight, out,
                                   out_row_stride, sum_out, sum_out_row_stride, rows, hidden, eps,
                                   stream);
}

extern "C" int nva_qk_norm_rope(const void* qkv, int64_t row_stride, const int64_t* positions,
                                const void* q_norm_weight, const void* k_norm_weight,
                                const float* cos_sin, int32_t max_position, int32_t num_tokens,
                                int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                float eps, void* q_out, void* k_out, void* stream) {
  if (head_dim != 128) return NVA_ERR_UNSUPPORTED;
  if (num_tokens < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || max_position <= 0)
    return NVA_ERR_ARG;
  if (num_tokens == 0) return NVA_OK;
  if (!qkv || !positions || !cos_sin || !q_out || !k_out ||
      row_stride < static_cast<int64_t>(num_q_heads + num_kv_heads) * head_dim)
    return NVA_ERR_ARG;
  if ((q_norm_weight == nullptr) != (k_norm_weight == nullptr)) return NVA_ERR_ARG;
  const int heads_per_block = kNormThreads / kWave;
  dim3 grid((num_q_heads + num_kv_heads + heads_per_block - 1) / heads_per_block, num_tokens);
  qk_norm_rope_kernel<<<grid, kNormThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(qkv), row_stride, positions,
      static_cast<const uint16_t*>(q_norm_weight), static_cast<const uint16_t*>(k_norm_weight),
      cos_sin, max_position, num_tokens, num_q_heads, num_kv_heads, eps,
      static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_out));
  return launch_status();
}

extern "C" int nva_qk_norm_rope_store(
    const void* qkv, int64_t row_stride, const int64_t* positions, const void* q_norm_weight,
    const void* k_norm_weight, const float* cos_sin, int32_t max_position, int32_t num_tokens,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, float eps, void* q_out,
    void* k_cache, void* v_cache, int kv_dtype, int64_t cache_block_stride,
    int64_t cache_token_stride, int64_t cache_head_stride, int32_t num_blocks, int32_t block_size,
    const int32_t* slot_mapping, const float* k_scale, const float* v_scale, void* stream) {
  if (head_dim != 128) return NVA_ERR_UNSUPPORTED;
  if (num_tokens < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || max_position <= 0 ||
      num_blocks < 0 || block_size <= 0 || cache_block_stride < 0 || cache_token_stride < 0 ||
      cache_head_stride < 0)
    return NVA_ERR_ARG;
  if (kv_dtype != NVA_KV_BF16 && kv_dtype != NVA_KV_FP8_E4M3) return NVA_ERR_ARG;
  if (num_tokens == 0) return NVA_OK;
  if (!qkv || !positions || !cos_sin || !q_out || !k_cache || !v_cache || !slot_mapping ||
      row_stride < static_cast<int64_t>(num_q_heads + 2 * num_kv_heads) * head_dim)
    return NVA_ERR_ARG;
  if ((q_norm_weight == nullptr) != (k_norm_weight == nullptr)) return NVA_ERR_ARG;
  const SlotPages pages{cache_block_stride, cache_token_stride, cache_head_stride, block_size,
                        static_cast<int64_t>(num_blocks) * block_size};
  const int heads_per_block = kNormThreads / kWave;
  dim3 grid((num_q_heads + 2 * num_kv_heads + heads_per_block - 1) / heads_per_block, num_tokens);
  auto* kern = kv_dtype == NVA_KV_BF16 ? qk_norm_rope_store_kernel<false>
                                       : qk_norm_rope_store_kernel<true>;
  kern<<<grid, kNormThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(qkv), row_stride, positions,
      static_cast<const uint16_t*>(q_norm_weight), static_cast<const uint16_t*>(k_norm_weight),
      cos_sin, max_position, num_tokens, num_q_heads, num_kv_heads, eps,
      static_cast<uint16_t*>(q_out), k_cache, v_cache, pages, slot_mapping, k_scale, v_scale);
  return launch_status();
}

extern "C" int nva_silu_mul(const void* x, int64_t x_row_stride, void* out, int64_t out_row_stride,
                            int32_t rows, int32_t intermediate, void* stream) {
  if (rows < 0 || intermediate <= 0) return NVA_ERR_ARG;
  if (rows == 0) return NVA_OK;
  if (!x || !out || x_row_stride < 2 * static_cast<int64_t>(intermediate) ||
      out_row_stride < intermediate)
    return NVA_ERR_ARG;
  const bool vec = intermediate % 8 == 0 && x_row_stride % 8 == 0 && out_row_stride % 8 == 0 &&
                   aligned16(x) && aligned16(out);
  const int per_block = kNormThreads * (vec ? 8 : 4);
  dim3 grid((intermediate + per_block - 1) / per_block, rows);
  silu_mul_kernel<<<grid, kNormThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(x), x_row_stride, static_cast<uint16_t*>(out), out_row_stride,
      intermediate, vec);
  return launch_status();
}
