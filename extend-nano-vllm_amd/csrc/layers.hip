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
// rounded to bf16, then multiplied by the bf16 weight in bf16.)
template <bool ADD>
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
  float x1 = bf16_to_f32(src[lane]);
  float x2 = bf16_to_f32(src[lane + 64]);
  const uint16_t* w = is_q ? q_w : k_w;
  if (w) {
    const float inv = rsqrtf(wave_sum(x1 * x1 + x2 * x2) / 128.0f + eps);
    x1 = bf16_to_f32(f32_to_bf16(bf16_to_f32(f32_to_bf16(x1 * inv)) * bf16_to_f32(w[lane])));
    x2 = bf16_to_f32(f32_to_bf16(bf16_to_f32(f32_to_bf16(x2 * inv)) * bf16_to_f32(w[lane + 64])));
  }
  int64_t pos = positions[t];
  pos = pos < 0 ? 0 : (pos >= max_pos ? max_pos - 1 : pos);
  const float c = cos_sin[pos * 128 + lane];
  const float s = cos_sin[pos * 128 + 64 + lane];
  const float y1 = x1 * c - x2 * s;
  const float y2 = x2 * c + x1 * s;
  uint16_t* dst = is_q ? q_out + (static_cast<int64_t>(t) * hq + head) * 128
                       : k_out + (static_cast<int64_t>(t) * hkv + (head - hq)) * 128;
  dst[lane] = f32_to_bf16(y1);
  dst[lane + 64] = f32_to_bf16(y2);
}

// out = bf16( bf16(silu(a)) * b ) for a row [a | b] (activation.py:11-14:
// F.silu in bf16, then a bf16 product)
__global__ void __launch_bounds__(kNormThreads)
silu_mul_kernel(const uint16_t* __restrict__ x, int64_t x_stride, uint16_t* __restrict__ out,
                int64_t out_stride, int32_t inter) {
  const int64_t r = blockIdx.y;
  const uint16_t* a = x + r * x_stride;
  const uint16_t* b = a + inter;
  uint16_t* o = out + r * out_stride;
  for (int c = blockIdx.x * kNormThreads + threadIdx.x; c < inter; c += gridDim.x * kNormThreads) {
    const float av = bf16_to_f32(a[c]);
    const float sv = bf16_to_f32(f32_to_bf16(av / (1.0f + __expf(-av))));
    o[c] = f32_to_bf16(sv * bf16_to_f32(b[c]));
  }
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

extern "C" int nva_add_rms_norm(const void* x, int64_t x_row_stride, const void* residual,
                                int64_t residual_row_stride, const void* weight, void* out,
                                int64_t out_row_stride, void* residual_out,
                                int64_t residual_out_row_stride, int32_t rows, int32_t hidden,
                                float eps, void* stream) {
  if (rows < 0 || hidden <= 0 || hidden > kMaxHidden) return NVA_ERR_ARG;
  if (rows == 0) return NVA_OK;
  if (!x || !residual || !weight || !out || !residual_out || x_row_stride < hidden ||
      residual_row_stride < hidden || out_row_stride < hidden || residual_out_row_stride < hidden)
    return NVA_ERR_ARG;
  const bool vec = hidden % 8 == 0 && x_row_stride % 8 == 0 && residual_row_stride % 8 == 0 &&
                   out_row_stride % 8 == 0 && residual_out_row_stride % 8 == 0 && aligned16(x) &&
                   aligned16(residual) && aligned16(weight) && aligned16(out) &&
                   aligned16(residual_out);
  rms_norm_kernel<true><<<rows, kNormThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(x), x_row_stride, static_cast<const uint16_t*>(residual),
      residual_row_stride, static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(out),
      out_row_stride, static_cast<uint16_t*>(residual_out), residual_out_row_stride, hidden, eps,
      vec);
  return launch_status();
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

extern "C" int nva_silu_mul(const void* x, int64_t x_row_stride, void* out, int64_t out_row_stride,
                            int32_t rows, int32_t intermediate, void* stream) {
  if (rows < 0 || intermediate <= 0) return NVA_ERR_ARG;
  if (rows == 0) return NVA_OK;
  if (!x || !out || x_row_stride < 2 * static_cast<int64_t>(intermediate) ||
      out_row_stride < intermediate)
    return NVA_ERR_ARG;
  const int bx = (intermediate + kNormThreads * 4 - 1) / (kNormThreads * 4);
  dim3 grid(bx, rows);
  silu_mul_kernel<<<grid, kNormThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(x), x_row_stride, static_cast<uint16_t*>(out), out_row_stride,
      intermediate);
  return launch_status();
}
