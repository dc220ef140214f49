// SPDX-License-Identifier: Apache-2.0
// Shared device helpers for the MI355X (gfx950) quantized-KV kernels.
//
// Everything here is plain HIP for CDNA4: wave64, 16-byte global accesses,
// explicit round-to-nearest-even conversions.  The fp32 quantize/dequantize
// helpers rely on this library being compiled with -ffp-contract=off and
// HIP's default correctly rounded fp32 division, so each operation rounds
// exactly once, as IEEE (and the reference's torch CPU ops) do.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kvq_hip.h"

namespace kvq {

// 16-bit storage types.  bf16 is kept as raw bits; fp16 uses _Float16.
struct bf16 {
  uint16_t bits;
};
using f16 = _Float16;

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(f16 v) { return static_cast<float>(v); }
__device__ __forceinline__ float to_f32(bf16 v) {
  return __uint_as_float(static_cast<uint32_t>(v.bits) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

template <typename T>
__device__ __forceinline__ T from_f32(float f);
template <>
__device__ __forceinline__ float from_f32<float>(float f) { return f; }
template <>
__device__ __forceinline__ f16 from_f32<f16>(float f) { return static_cast<f16>(f); }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float f) { return bf16{f32_to_bf16_bits(f)}; }

// Round an fp32 value to the precision of T and widen it back.
template <typename T>
__device__ __forceinline__ float round_to(float f) { return to_f32(from_f32<T>(f)); }

// Load 8 consecutive elements of T as fp32 (16 B for 16-bit types).
__device__ __forceinline__ void load8(const float* p, float (&x)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
  x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}
__device__ __forceinline__ void load8(const bf16* p, float (&x)[8]) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = __uint_as_float(w[i] << 16);
    x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ void load8(const f16* p, float (&x)[8]) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  const h8 v = *reinterpret_cast<const h8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = static_cast<float>(v[i]);
}

// Store 8 fp32 values as T (RNE for 16-bit types).
__device__ __forceinline__ void store8(float* p, const float (&x)[8]) {
  *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(x[4], x[5], x[6], x[7]);
}
__device__ __forceinline__ void store8(bf16* p, const float (&x)[8]) {
  uint4 v;
  v.x = f32_to_bf16_bits(x[0]) | (static_cast<uint32_t>(f32_to_bf16_bits(x[1])) << 16);
  v.y = f32_to_bf16_bits(x[2]) | (static_cast<uint32_t>(f32_to_bf16_bits(x[3])) << 16);
  v.z = f32_to_bf16_bits(x[4]) | (static_cast<uint32_t>(f32_to_bf16_bits(x[5])) << 16);
  v.w = f32_to_bf16_bits(x[6]) | (static_cast<uint32_t>(f32_to_bf16_bits(x[7])) << 16);
  *reinterpret_cast<uint4*>(p) = v;
}
__device__ __forceinline__ void store8(f16* p, const float (&x)[8]) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  h8 v;
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = static_cast<_Float16>(x[i]);
  *reinterpret_cast<h8*>(p) = v;
}

// KIVI group scale: max((mx - mn) / 15, 1e-6); the floor applies to the scale.
__device__ __forceinline__ float kivi_group_scale(float mn, float mx) {
  const float s = (mx - mn) / 15.0f;
  return s < 1.0e-6f ? 1.0e-6f : s;
}

// KIVI code: clamp(floor((x - mn) / scale + 0.5), 0, 15); ties round up.
__device__ __forceinline__ uint32_t kivi_quantize(float x, float mn, float scale) {
  float t = (x - mn) / scale;
  t = t + 0.5f;
  t = floorf(t);
  t = t < 0.0f ? 0.0f : t;
  t = t > 15.0f ? 15.0f : t;
  return static_cast<uint32_t>(t);
}

// KIVI dequant: q * scale, then + mn, as two separate fp32 roundings.
__device__ __forceinline__ float kivi_dequant(uint32_t q, float scale, float mn) {
  return __fadd_rn(__fmul_rn(static_cast<float>(q), scale), mn);
}

__device__ __forceinline__ float fmin_ordered(float a, float b) { return b < a ? b : a; }
__device__ __forceinline__ float fmax_ordered(float a, float b) { return b > a ? b : a; }

template <typename I>
__device__ __forceinline__ int64_t ld_index(const I* p, int64_t i) {
  return static_cast<int64_t>(p[i]);
}

}  // namespace kvq

// Dispatch helpers for the C-ABI layer.
#define KVQ_DISPATCH_FLOAT(code, T, ...)                      \
  switch (code) {                                             \
    case KVQ_DTYPE_F32: { using T = float; __VA_ARGS__; break; } \
    case KVQ_DTYPE_F16: { using T = kvq::f16; __VA_ARGS__; break; } \
    case KVQ_DTYPE_BF16: { using T = kvq::bf16; __VA_ARGS__; break; } \
    default: return KVQ_ERR_INVALID;                          \
  }

#define KVQ_DISPATCH_INDEX(code, I, ...)                       \
  switch (code) {                                              \
    case KVQ_INDEX_I32: { using I = int32_t; __VA_ARGS__; break; } \
    case KVQ_INDEX_I64: { using I = int64_t; __VA_ARGS__; break; } \
    default: return KVQ_ERR_INVALID;                           \
  }

#define KVQ_LAUNCH_CHECK()                                     \
  do {                                                         \
    hipError_t _e = hipGetLastError();                         \
    if (_e != hipSuccess) return static_cast<int>(_e);         \
  } while (0)
