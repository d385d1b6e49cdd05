// K3: EAGLE3 auxiliary hidden-state add + concat + row gather.
//
// Grid (num_rows, num_layers); each block adds one aux layer's hidden and
// residual row (bf16, in float, rounded to nearest even) and writes it into
// its column slice of the concatenated [R, L*H] output.  HBM bound: per
// output row it reads 2*L*H*2 bytes and writes L*H*2 bytes.
#include "common.h"

namespace nva {
namespace {

constexpr int kMaxAuxLayers = 4;
constexpr int kAuxThreads = 256;

struct AuxPtrs {
  const uint16_t* hidden[kMaxAuxLayers];
  const uint16_t* residual[kMaxAuxLayers];
};

__device__ __forceinline__ uint32_t add_pair(uint32_t a, uint32_t b) {
  const uint32_t lo = f32_to_bf16(bf16_to_f32(a & 0xFFFFu) + bf16_to_f32(b & 0xFFFFu));
  const uint32_t hi = f32_to_bf16(bf16_to_f32(a >> 16) + bf16_to_f32(b >> 16));
  return lo | (hi << 16);
}

__global__ void __launch_bounds__(kAuxThreads)
aux_gather_kernel(AuxPtrs p, int64_t in_row_stride, int32_t hidden_size, int32_t num_in_rows,
                  const int32_t* __restrict__ src_rows, int32_t num_rows,
                  uint16_t* __restrict__ out, int64_t out_row_stride, bool vec) {
  const int32_t r = blockIdx.x;
  const int32_t l = blockIdx.y;
  if (r >= num_rows) return;
  const int64_t src = src_rows[r];
  uint16_t* o = out + static_cast<int64_t>(r) * out_row_stride + static_cast<int64_t>(l) * hidden_size;
  if (src < 0 || src >= num_in_rows) {
    for (int c = threadIdx.x; c < hidden_size; c += kAuxThreads) o[c] = 0;
    return;
  }
  const uint16_t* h = p.hidden[l] + src * in_row_stride;
  const uint16_t* res = p.residual[l] + src * in_row_stride;
  if (vec) {
    const int nvec = hidden_size / 8;
    for (int i = threadIdx.x; i < nvec; i += kAuxThreads) {
      const uint4 a = reinterpret_cast<const uint4*>(h)[i];
      const uint4 b = reinterpret_cast<const uint4*>(res)[i];
      uint4 s;
      s.x = add_pair(a.x, b.x);
      s.y = add_pair(a.y, b.y);
      s.z = add_pair(a.z, b.z);
      s.w = add_pair(a.w, b.w);
      reinterpret_cast<uint4*>(o)[i] = s;
    }
  } else {
    for (int c = threadIdx.x; c < hidden_size; c += kAuxThreads)
      o[c] = f32_to_bf16(bf16_to_f32(h[c]) + bf16_to_f32(res[c]));
  }
}

}  // namespace
}  // namespace nva

using namespace nva;

extern "C" int nva_aux_gather(const void* const* hidden, const void* const* residual,
                              int32_t num_layers, int64_t in_row_stride, int32_t hidden_size,
                              int32_t num_in_rows, const int32_t* src_rows, int32_t num_rows, void* out,
                              int64_t out_row_stride, void* stream) {
  if (num_layers < 1 || num_layers > kMaxAuxLayers || hidden_size <= 0 || num_rows < 0 ||
      num_in_rows < 0)
    return NVA_ERR_ARG;
  if (num_rows == 0) return NVA_OK;
  if (!hidden || !residual || !src_rows || !out) return NVA_ERR_ARG;
  if (in_row_stride < hidden_size || out_row_stride < static_cast<int64_t>(num_layers) * hidden_size)
    return NVA_ERR_ARG;
  AuxPtrs p = {};
  bool vec = (hidden_size % 8 == 0) && (in_row_stride % 8 == 0) && (out_row_stride % 8 == 0) &&
             aligned16(out);
  for (int l = 0; l < num_layers; ++l) {
    if (!hidden[l] || !residual[l]) return NVA_ERR_ARG;
    p.hidden[l] = static_cast<const uint16_t*>(hidden[l]);
    p.residual[l] = static_cast<const uint16_t*>(residual[l]);
    vec = vec && aligned16(hidden[l]) && aligned16(residual[l]);
  }
  dim3 grid(num_rows, num_layers);
  aux_gather_kernel<<<grid, kAuxThreads, 0, static_cast<hipStream_t>(stream)>>>(
      p, in_row_stride, hidden_size, num_in_rows, src_rows, num_rows, static_cast<uint16_t*>(out),
      out_row_stride, vec);
  return launch_status();
}
