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

#include <atomic>

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
// bf16 pairs through v_cvt_pk_bf16_f32 (round to nearest even, the same bits
// as f32_to_bf16_bits for every non-NaN input).
__device__ __forceinline__ uint32_t bf16x2_bits(float lo, float hi) {
  typedef float f2v __attribute__((ext_vector_type(2)));
  typedef __bf16 b2v __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2v{lo, hi}), b2v));
}
__device__ __forceinline__ void store8(bf16* p, const float (&x)[8]) {
  uint4 v;
  v.x = bf16x2_bits(x[0], x[1]);
  v.y = bf16x2_bits(x[2], x[3]);
  v.z = bf16x2_bits(x[4], x[5]);
  v.w = bf16x2_bits(x[6], x[7]);
  *reinterpret_cast<uint4*>(p) = v;
}
__device__ __forceinline__ void store8(f16* p, const float (&x)[8]) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  h8 v;
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = static_cast<_Float16>(x[i]);
  *reinterpret_cast<h8*>(p) = v;
}

// Streaming stores for dense outputs nobody re-reads soon (gathered K/V):
// nontemporal global stores (the `nt` bit) do not allocate in L2 on the way
// out.  The config-4 gather writes 335 MB of bf16 K/V; with plain stores it
// ran at 3.7 TB/s, with these at 5.8 TB/s.
typedef uint32_t kvq_u4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void store16_nt(void* p, kvq_u4v v) {
  __builtin_nontemporal_store(v, reinterpret_cast<kvq_u4v*>(p));
}
__device__ __forceinline__ void store8_nt(float* p, const float (&x)[8]) {
  store16_nt(p, kvq_u4v{__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]),
                        __float_as_uint(x[3])});
  store16_nt(p + 4, kvq_u4v{__float_as_uint(x[4]), __float_as_uint(x[5]), __float_as_uint(x[6]),
                            __float_as_uint(x[7])});
}
__device__ __forceinline__ void store8_nt(bf16* p, const float (&x)[8]) {
  store16_nt(p, kvq_u4v{bf16x2_bits(x[0], x[1]), bf16x2_bits(x[2], x[3]),
                        bf16x2_bits(x[4], x[5]), bf16x2_bits(x[6], x[7])});
}
__device__ __forceinline__ void store8_nt(f16* p, const float (&x)[8]) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  h8 v;
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = static_cast<_Float16>(x[i]);
  store16_nt(p, __builtin_bit_cast(kvq_u4v, v));
}

// KIVI group scale: max((mx - mn) / 15, 1e-6); the floor applies to the scale.
// The quotient is correctly rounded without a division: q0 = x * RN(1/15),
// then one remainder step r = fma(-q0, 15, x) (exact), q = fma(r, RN(1/15), q0).
// Checked against IEEE x / 15 for every mantissa of a binade; every step scales
// by powers of two, so that covers every normal x, and an x small enough for
// subnormal steps gives a quotient far under the 1e-6 floor either way.
__device__ __forceinline__ float kivi_group_scale(float mn, float mx) {
  constexpr float kRcp15 = 1.0f / 15.0f;
  const float x = mx - mn;
  const float q0 = x * kRcp15;
  const float s = __builtin_fmaf(__builtin_fmaf(-q0, 15.0f, x), kRcp15, q0);
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

// One packed word (8 codes, code i at bits 4i) with the codes of
// kivi_quantize, exactly, with no division and no branch.
//
// With d = x - mn (rounded as there) and q = RN(d / scale), the reference's
// code floor(RN(q + 0.5)) is k or k + 1 for k = floor(q).  RN(q + 0.5) is exact
// for k >= 1, so the code is k + 1 iff q >= k + 0.5; for k = 0 the sum rounds
// to 1 already at q = pred(0.5) = 0.5 - 2^-25 (1 - 2^-25 is a tie, to even).
// With T_k = k + 0.5 (k >= 1) or pred(0.5) (k = 0):
//
//   q >= T_k  <=>  d / scale >= T_k - ulp(T_k) / 2  <=>  y >= 0,
//   y = fma(scale * 2^-24, 2^e(T_k), fma(-scale, T_k, d))
//
// (round to nearest moves a quotient onto T_k from above the midpoint below
// it; at the midpoint itself ties go to T_k for k >= 1, whose last mantissa
// bit is 0, and d = scale * midpoint has no solution for k = 0).  2^e(T) is T
// with its mantissa cleared, so the outer product is scale * ulp(T) / 2,
// exact.  The inner fma is exact near the threshold: d and scale * T are
// multiples of ulp(scale) / 2 for k >= 1 and of ulp(scale) * 2^-25 for k = 0,
// so a difference of a few scale * ulp(T) fits in 24 bits; further away
// |d - scale * T| dwarfs the outer term and rounding keeps its sign.  Either
// way y has the sign of the exact d - scale * (T_k - ulp(T_k) / 2).
//
// k comes from v = d * rcp(scale) (v_rcp_f32, 1 ulp): v is within 5e-6 of q,
// so floor(v) is floor(q) or one off it next to an integer, where the test
// above, made against the neighbouring T, gives the same code.  T_k is one
// add: k + pred(0.5) rounds to k + 0.5 for k >= 1.  v >= 0 and q < 15.5 keep
// the codes in 0..15 with no clamp.  v_cvt_pk_u8_f32 drops each code into a
// byte (even codes of the word in one register, odd codes in another) and a
// single shift-or interleaves the nibbles.  The choice between k and k + 1
// is folded into that conversion, which rounds to nearest even: it converts
// t + 0.25 when y >= 0 and t - 0.25 otherwise (t = k + 0.5, or pred(0.5) at
// k = 0, so the two round to k + 1 and k).  y is never -0: its outer product
// is positive, so an exact cancellation rounds to +0.
__device__ __forceinline__ uint32_t kivi_pack_word(const float (&x)[8], float mn, float scale) {
  const float rcp = __builtin_amdgcn_rcpf(scale);
  const float s24 = scale * 0x1p-24f;
  uint32_t ev = 0, od = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float d = x[i] - mn;
    const float k = __builtin_floorf(d * rcp);
    const float t = k + 0x1.fffffep-2f;
    const float e = __int_as_float(__float_as_int(t) & 0x7f800000);
    const float y = __builtin_fmaf(s24, e, __builtin_fmaf(-scale, t, d));
    // +-0.25 with y's sign: (y & sign) | bits(0.25)
    const float step = __uint_as_float((__float_as_uint(y) & 0x80000000u) | 0x3e800000u);
    const float r = t + step;
    if (i % 2 == 0)
      ev = __builtin_amdgcn_cvt_pk_u8_f32(r, i / 2, ev);
    else
      od = __builtin_amdgcn_cvt_pk_u8_f32(r, i / 2, od);
  }
  return ev | (od << 4);
}

// The 8 nibbles of a packed word as floats (nibble i -> c[i]): one mask per
// parity, then v_cvt_f32_ubyte{0..3} on each byte (the compiler would
// extract every nibble on its own).
template <int B>
__device__ __forceinline__ float ubyte_f32(uint32_t v) {
  float r;
  if (B == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
  if (B == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
  if (B == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
  if (B == 3) asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
  return r;
}
__device__ __forceinline__ void nibbles_f32(uint32_t w, float (&c)[8]) {
  const uint32_t ev = w & 0x0f0f0f0fu;         // nibbles 0, 2, 4, 6 in bytes 0..3
  const uint32_t od = (w >> 4) & 0x0f0f0f0fu;  // nibbles 1, 3, 5, 7
  c[0] = ubyte_f32<0>(ev);
  c[1] = ubyte_f32<0>(od);
  c[2] = ubyte_f32<1>(ev);
  c[3] = ubyte_f32<1>(od);
  c[4] = ubyte_f32<2>(ev);
  c[5] = ubyte_f32<2>(od);
  c[6] = ubyte_f32<3>(ev);
  c[7] = ubyte_f32<3>(od);
}

// KIVI dequant: q * scale, then + mn, as two separate fp32 roundings.
__device__ __forceinline__ float kivi_dequant(uint32_t q, float scale, float mn) {
  return __fadd_rn(__fmul_rn(static_cast<float>(q), scale), mn);
}

// Maximum over lanes l, l ^ 16, l ^ 32 and l ^ 48 (one value from each of
// the wave's four 16-lane rows), with gfx950's row-swap permutes: VALU only.
// (__shfl_xor goes through ds_bpermute: an LDS round trip plus address
// arithmetic per step.)  permlane32_swap(u, u) returns [lo, lo] and [hi, hi]
// (the wave's 32-lane halves), permlane16_swap(v, v) rows [0, 0, 2, 2] and
// [1, 1, 3, 3]; the max of each pair covers the lanes the next step needs.
__device__ __forceinline__ float max_rows4(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  // med3(a, b, FLT_MAX) is max(a, b) for every a, b <= FLT_MAX (-inf
  // included), without the canonicalizing moves fmaxf puts in front of
  // values the compiler cannot vouch for (with +inf as the third operand the
  // compiler turns it back into fmaxf)
  constexpr float kBig = 0x1.fffffep127f;
  const float m = __builtin_amdgcn_fmed3f(__uint_as_float(a[0]), __uint_as_float(a[1]), kBig);
  const uint32_t v = __float_as_uint(m);  // lanes l, l ^ 32
  const auto b = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return __builtin_amdgcn_fmed3f(__uint_as_float(b[0]), __uint_as_float(b[1]), kBig);  // and l ^ 16
}

// max_rows4 of two values in three swaps instead of four: the first swap
// trades x's lanes 32-63 for y's lanes 0-31, so one register carries x's
// reduction in lanes 0-31 and y's in lanes 32-63 until the last swap hands
// each half to every lane.
__device__ __forceinline__ void max_rows4_pair(float& x, float& y) {
  constexpr float kBig = 0x1.fffffep127f;
  // a[0] = (x lanes 0-31, y lanes 0-31), a[1] = (x lanes 32-63, y lanes 32-63)
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  const uint32_t z = __float_as_uint(
      __builtin_amdgcn_fmed3f(__uint_as_float(a[0]), __uint_as_float(a[1]), kBig));
  const auto b = __builtin_amdgcn_permlane16_swap(z, z, false, false);
  const uint32_t w = __float_as_uint(
      __builtin_amdgcn_fmed3f(__uint_as_float(b[0]), __uint_as_float(b[1]), kBig));
  const auto c = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  x = __uint_as_float(c[0]);
  y = __uint_as_float(c[1]);
}

// Sum over the same four lanes, rows paired first (l ^ 16), then halves
// (l ^ 32): lane for lane the additions of v += shfl_xor(v, 16); v +=
// shfl_xor(v, 32), so the result is bit-identical to that form.
__device__ __forceinline__ float sum_rows4(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float s = __uint_as_float(a[0]) + __uint_as_float(a[1]);  // lanes l, l ^ 16
  const uint32_t v = __float_as_uint(s);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);          // and l ^ 32
}

// Whole-wave reductions without LDS: DPP inside each 16-lane row (quad
// swaps, then the half-row and row mirrors, which pair the quads and halves
// already reduced), then the row swaps above.  Every lane ends with the same
// value (each step adds or maxes equal operand pairs in either order).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
constexpr int kDppQuadXor1 = 0xB1;  // quad_perm [1, 0, 3, 2]
constexpr int kDppQuadXor2 = 0x4E;  // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
__device__ __forceinline__ float max_wave64(float x) {
  x = fmaxf(x, dpp_f32<kDppQuadXor1>(x));
  x = fmaxf(x, dpp_f32<kDppQuadXor2>(x));
  x = fmaxf(x, dpp_f32<kDppHalfMirror>(x));
  x = fmaxf(x, dpp_f32<kDppRowMirror>(x));
  return max_rows4(x);
}
__device__ __forceinline__ float sum_wave64(float x) {
  x += dpp_f32<kDppQuadXor1>(x);
  x += dpp_f32<kDppQuadXor2>(x);
  x += dpp_f32<kDppHalfMirror>(x);
  x += dpp_f32<kDppRowMirror>(x);
  return sum_rows4(x);
}

__device__ __forceinline__ float fmin_ordered(float a, float b) { return b < a ? b : a; }
__device__ __forceinline__ float fmax_ordered(float a, float b) { return b > a ? b : a; }

template <typename I>
__device__ __forceinline__ int64_t ld_index(const I* p, int64_t i) {
  return static_cast<int64_t>(p[i]);
}

// Value of lane (lane ^ MASK) in the wave: DPP quad permutes for masks 1 and
// 2, ds_swizzle's xor mode inside 32-lane halves, ds_bpermute across them.
template <int MASK>
__device__ __forceinline__ float lane_xor(float v) {
  static_assert(MASK > 0 && MASK < 64 && (MASK & (MASK - 1)) == 0, "power-of-two mask");
  const int b = __float_as_int(v);
  int r;
  if (MASK == 1)
    r = __builtin_amdgcn_update_dpp(b, b, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  else if (MASK == 2)
    r = __builtin_amdgcn_update_dpp(b, b, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  else if (MASK < 32)
    r = __builtin_amdgcn_ds_swizzle(b, (MASK << 10) | 0x1F);  // and 0x1f, or 0, xor MASK
  else
    r = __builtin_amdgcn_ds_bpermute(static_cast<int>((threadIdx.x ^ MASK) & 63) << 2, b);
  return __int_as_float(r);
}

// Division by a launch constant d >= 1 for 0 <= n < 2^31 (Granlund-Montgomery):
// n / d = (umulhi(n, m) + n) >> s with s = ceil(log2 d) and
// m = floor(2^32 (2^s - d) / d) + 1, computed on the host.
struct FastDiv {
  uint32_t d, m, s;
  static FastDiv make(uint32_t d) {
    uint32_t s = 0;
    while ((1ull << s) < d) ++s;
    const uint64_t m = ((1ull << 32) * ((1ull << s) - d)) / d + 1;
    return FastDiv{d, static_cast<uint32_t>(m), s};
  }
  __device__ __forceinline__ uint32_t div(uint32_t n) const {
    return (__umulhi(n, m) + n) >> s;
  }
};

// Eight consecutive elements kept in their storage type (loaded early, widened
// to fp32 when used).
template <typename T>
struct Raw8;
template <>
struct Raw8<float> {
  float4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = *reinterpret_cast<const float4*>(p);
    b = *reinterpret_cast<const float4*>(p + 4);
  }
  __device__ __forceinline__ void get(float (&x)[8]) const {
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  }
};
template <>
struct Raw8<bf16> {
  uint4 v;
  __device__ __forceinline__ void load(const bf16* p) { v = *reinterpret_cast<const uint4*>(p); }
  __device__ __forceinline__ void get(float (&x)[8]) const {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(w[i] << 16);
      x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
};
template <>
struct Raw8<f16> {
  uint4 v;
  __device__ __forceinline__ void load(const f16* p) { v = *reinterpret_cast<const uint4*>(p); }
  __device__ __forceinline__ void get(float (&x)[8]) const {
    typedef _Float16 h8v __attribute__((ext_vector_type(8)));
    const h8v h = __builtin_bit_cast(h8v, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = static_cast<float>(h[i]);
  }
};

// ---- LDS DMA -------------------------------------------------------------
// global_load_lds: every lane reads `size` bytes at its own global address and
// the wave writes them to LDS at base + size * lane (base must be uniform).
typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ void dma16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)(lds), 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)(lds), 4, 0, 0);
}

// s_waitcnt vmcnt(N) with lgkmcnt/expcnt left alone (gfx9 encoding: vmcnt
// bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("" ::: "memory");
}

// LDS one workgroup may use on the current device, cached per device (the
// attribute query is host work that a decode step should not repeat).
inline int device_lds_max(int64_t* out) {
  static std::atomic<int64_t> cache[64];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= 64) {
    *out = 0;
    return KVQ_OK;
  }
  int64_t v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    int vmax = 0;
    e = hipDeviceGetAttribute(&vmax, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
    if (e != hipSuccess) return static_cast<int>(e);
    v = vmax;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  *out = v;
  return KVQ_OK;
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
