// Shared device helpers for the EAGLE3 speculative-step kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nanovllm_amd.h"

namespace nva {

typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short bf16x4_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

constexpr int kWave = 64;

// ---------------------------------------------------------------- bf16

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even float -> bf16, NaN -> 0x7FC0 (the conversion torch
// applies when it stores a float result as bfloat16).  gfx950's
// v_cvt_pk_bf16_f32 rounds to nearest even, subnormals included (the
// kernels run with f32 denormals preserved); only a NaN's payload differs
// from torch's, hence the select.  Three instructions against the integer
// rounding's seven.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const uint16_t r = __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
  return f != f ? static_cast<uint16_t>(0x7FC0) : r;
}

// ---------------------------------------------------------------- fp8 e4m3fn

// OCP float8_e4m3fn -> float.  The byte shifted left by 7 is an IEEE half with
// the same sign/mantissa and an exponent bias of 15 instead of 7, so the half
// value times 2^8 is exact for normals and subnormals alike.  0x7F/0xFF are NaN.
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
  uint32_t em = b & 0x7Fu;
  uint16_t hbits = static_cast<uint16_t>(((b & 0x80u) << 8) | (em << 7));
  _Float16 h = __builtin_bit_cast(_Float16, hbits);
  float v = static_cast<float>(h) * 256.0f;
  return em == 0x7Fu ? __builtin_nanf("") : v;
}

// float -> float8_e4m3fn, round to nearest even, magnitudes >= 464 (including
// infinities) saturate to +-448, NaN -> 0x7F with the sign kept.
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
  uint32_t u = __float_as_uint(x);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign | 0x7Fu;
  float af = __uint_as_float(a);
  if (af >= 464.0f) return sign | 0x7Eu;
  if (af < 0.015625f) {                       // below the smallest normal 2^-6
    // subnormal codes are m * 2^-9, m = 0..7; m == 8 is the code of 2^-6
    uint32_t m = static_cast<uint32_t>(__builtin_rintf(af * 512.0f));
    return sign | m;
  }
  int32_t e = static_cast<int32_t>(a >> 23) - 127;   // -6 .. 8
  uint32_t mant = a & 0x7FFFFFu;
  uint32_t keep = mant >> 20;
  uint32_t low = mant & 0xFFFFFu;
  if (low > 0x80000u || (low == 0x80000u && (keep & 1u))) ++keep;
  if (keep == 8u) { keep = 0; ++e; }
  return sign | (static_cast<uint32_t>(e + 7) << 3) | keep;
}

// ---------------------------------------------------------------- misc

__device__ __forceinline__ int wave_lane() { return threadIdx.x & (kWave - 1); }

template <typename T>
__device__ __forceinline__ T load_acquire_agent(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T load_relaxed_agent(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void store_relaxed_agent(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

inline int launch_status() {
  return hipGetLastError() == hipSuccess ? NVA_OK : NVA_ERR_LAUNCH;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Cache-policy operand of a buffer load that reads whole lines exactly once
// (V pages, logits): the nt (non-temporal) bit, so streamed lines leave the
// caches early and do not displace lines that are still to be re-read.
constexpr int kLoadStreamed = 2;

// Streaming (non-temporal) stores for rows that no kernel re-reads soon
// from a cache: new KV-cache rows (read next by the attention, from HBM)
// and the fused kernel's query rows.  Each call site writes whole 128-byte
// lines per instruction.  The scattered cache rows of the verify step
// (6144 rows of 256 bytes at 64 KiB strides) otherwise linger dirty and
// drain while the next kernel streams its reads: the verify attention that
// follows the fused norm/RoPE/store launch took 59.3 us per call against
// 58.2-58.5 us with these stores streamed (Qwen3-8B bench shapes, kernel
// trace; 57.0-57.9 us with no store before it).
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void store_streamed(uint16_t* p, uint16_t v) {
  __builtin_nontemporal_store(v, p);
}
__device__ __forceinline__ void store_streamed(uint4* p, uint4 v) {
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, v), reinterpret_cast<u32x4_t*>(p));
}

// Raw buffer descriptor over num_records bytes at base: loads at offsets
// past the end return zeros (dword 3: 32-bit data format, no swizzle).
constexpr int kRsrcWord3 = 0x00020000;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int num_records) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), num_records,
                                           kRsrcWord3);
}

}  // namespace nva
