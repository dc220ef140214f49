// SPDX-License-Identifier: Apache-2.0
// fp8_per_token_head: OCP E4M3 (e4m3fn) codes with one fp32 scale per
// (token, kv head), stored into and read back from the paged byte layout.
//
// Reference semantics (pkg/methods/fp8_per_token_head/semantics.py:52-68):
//   scale = max(amax(|x|) / 448, 1e-6)            per (token, head), fp32
//   code  = e4m3fn(clamp(x / scale, -448, 448))    round to nearest even
//   x_hat = float(code) * scale
// and the store kernel it anchors (pkg/ops/triton/per_token_head_store.py:
// 141-220): one (token, head) row per program, negative slots skipped, data
// [NB, Bs, KVH, D] bytes and scales [NB, Bs, KVH] fp32.
//
// The quotient is IEEE x / scale (this library builds with correctly rounded
// fp32 division and no contraction), then v_cvt_pk_fp8_f32 -- gfx950's
// conversion to OCP e4m3fn, round to nearest even -- packs four codes a word.
// Every code the clamp admits is finite, so the conversion never saturates.
//
// Store: a group of GS lanes holds one (token, head) row of keys and values,
// VEC elements per lane (16-byte bf16 loads, 8-byte code stores for D % 8 ==
// 0); amax is a butterfly inside the group.  HBM-bound: 2 B of bf16 in and
// 1 B of code out per element, plus 4 B of scale per row.
// Gather: one thread per VEC codes of one (position, head) row, into dense
// TND rows of the activation dtype (code * scale in fp32, then RNE).
#include "kvq_common.h"

namespace {

using namespace kvq;

constexpr float kE4M3Max = 448.0f;
constexpr float kScaleFloor = 1.0e-6f;  // the fp32 rounding of the literal 1e-6

// Four codes (element i in byte i), round to nearest even.
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return static_cast<uint32_t>(w);
}

// The four codes of a word as fp32 (exact).
__device__ __forceinline__ void e4m3x4_f32(uint32_t w, float (&x)[4]) {
  typedef float f2v __attribute__((ext_vector_type(2)));
  const f2v lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), false);
  const f2v hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), true);
  x[0] = lo.x;
  x[1] = lo.y;
  x[2] = hi.x;
  x[3] = hi.y;
}

// VEC consecutive elements of T as fp32.
template <int VEC, typename T>
__device__ __forceinline__ void load_vec(const T* p, float (&x)[VEC]) {
  if constexpr (VEC == 8) {
    load8(p, x);
  } else if constexpr (sizeof(T) == 4) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
  } else {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    const T* h = reinterpret_cast<const T*>(&v);
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = to_f32(h[i]);
  }
}

template <int VEC, typename T>
__device__ __forceinline__ void store_vec_nt(T* p, const float (&x)[VEC]) {
  if constexpr (VEC == 8) {
    store8_nt(p, x);
  } else if constexpr (sizeof(T) == 4) {
    store16_nt(p, kvq_u4v{__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]),
                          __float_as_uint(x[3])});
  } else {
    T h[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) h[i] = from_f32<T>(x[i]);
    *reinterpret_cast<uint2*>(p) = *reinterpret_cast<const uint2*>(h);
  }
}

template <int GS>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (GS >= 2) v = fmaxf(v, lane_xor<1>(v));
  if constexpr (GS >= 4) v = fmaxf(v, lane_xor<2>(v));
  if constexpr (GS >= 8) v = fmaxf(v, lane_xor<4>(v));
  if constexpr (GS >= 16) v = fmaxf(v, lane_xor<8>(v));
  if constexpr (GS >= 32) v = fmaxf(v, lane_xor<16>(v));
  if constexpr (GS >= 64) v = fmaxf(v, lane_xor<32>(v));
  return v;
}

// Quantize one side's row slice held by this lane; returns the row scale.
template <int VEC, int GS>
__device__ __forceinline__ float quantize_row(const float (&x)[VEC], bool active,
                                              uint32_t (&codes)[VEC / 4]) {
  float a = 0.0f;
  if (active) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) a = fmaxf(a, fabsf(x[i]));
  }
  const float amax = group_max<GS>(a);
  float scale = amax / kE4M3Max;
  scale = scale < kScaleFloor ? kScaleFloor : scale;
  float q[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    float t = x[i] / scale;
    t = t < -kE4M3Max ? -kE4M3Max : t;
    t = t > kE4M3Max ? kE4M3Max : t;
    q[i] = t;
  }
#pragma unroll
  for (int w = 0; w < VEC / 4; ++w) codes[w] = e4m3x4(q[4 * w], q[4 * w + 1], q[4 * w + 2],
                                                      q[4 * w + 3]);
  return scale;
}

template <typename T, typename I, int VEC, int GS>
__global__ void __launch_bounds__(256)
fp8_pth_store_kernel(const T* __restrict__ key, const T* __restrict__ value,
                     const I* __restrict__ slots, int64_t rows, int kvh, int d, int64_t num_slots,
                     uint8_t* __restrict__ k_data, float* __restrict__ k_scale,
                     uint8_t* __restrict__ v_data, float* __restrict__ v_scale) {
  constexpr int kRowsPerBlock = 256 / GS;
  const int lane = threadIdx.x % GS;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / GS;
  if (row >= rows) return;  // whole groups leave together
  const int64_t tok = row / kvh;
  const int h = static_cast<int>(row - tok * kvh);
  const int64_t slot = ld_index(slots, tok);
  if (slot < 0 || slot >= num_slots) return;  // padding (negative) or outside the cache
  const int c0 = lane * VEC;
  const bool active = c0 < d;
  float xk[VEC], xv[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) xk[i] = xv[i] = 0.0f;
  if (active) {
    load_vec<VEC>(key + row * d + c0, xk);
    load_vec<VEC>(value + row * d + c0, xv);
  }
  uint32_t ck[VEC / 4], cv[VEC / 4];
  const float sk = quantize_row<VEC, GS>(xk, active, ck);
  const float sv = quantize_row<VEC, GS>(xv, active, cv);
  const int64_t dst = slot * kvh + h;
  if (active) {
    if constexpr (VEC == 8) {
      *reinterpret_cast<uint2*>(k_data + dst * d + c0) = make_uint2(ck[0], ck[1]);
      *reinterpret_cast<uint2*>(v_data + dst * d + c0) = make_uint2(cv[0], cv[1]);
    } else {
      *reinterpret_cast<uint32_t*>(k_data + dst * d + c0) = ck[0];
      *reinterpret_cast<uint32_t*>(v_data + dst * d + c0) = cv[0];
    }
  }
  if (lane == 0) {
    k_scale[dst] = sk;
    v_scale[dst] = sv;
  }
}

template <typename TO, typename TB, int VEC>
__global__ void __launch_bounds__(256)
fp8_pth_gather_kernel(const uint8_t* __restrict__ k_data, const float* __restrict__ k_scale,
                      const uint8_t* __restrict__ v_data, const float* __restrict__ v_scale,
                      int bs, int kvh, int d, int64_t nb, const TB* __restrict__ block_table,
                      int64_t maxb, const int64_t* __restrict__ cu, TO* __restrict__ out_k,
                      TO* __restrict__ out_v) {
  const int b = blockIdx.y;
  const int64_t row0 = cu[b];
  const int64_t len = cu[b + 1] - row0;
  const int per_head = d / VEC;
  const int64_t per_pos = static_cast<int64_t>(kvh) * per_head;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= len * per_pos) return;
  const int64_t p = gid / per_pos;
  if (p >= maxb * bs) return;  // a length the table does not cover reads nothing past it
  const int rem = static_cast<int>(gid - p * per_pos);
  const int h = rem / per_head;
  const int c0 = (rem - h * per_head) * VEC;
  int64_t blk = static_cast<int64_t>(block_table[static_cast<int64_t>(b) * maxb + p / bs]);
  blk = blk < 0 ? 0 : (blk >= nb ? nb - 1 : blk);  // unallocated ids read page 0
  const int64_t src = (blk * bs + p % bs) * kvh + h;
  const float sk = k_scale[src];
  const float sv = v_scale[src];
  uint32_t kw[VEC / 4], vw[VEC / 4];
  if constexpr (VEC == 8) {
    const uint2 a = *reinterpret_cast<const uint2*>(k_data + src * d + c0);
    const uint2 c = *reinterpret_cast<const uint2*>(v_data + src * d + c0);
    kw[0] = a.x; kw[1] = a.y;
    vw[0] = c.x; vw[1] = c.y;
  } else {
    kw[0] = *reinterpret_cast<const uint32_t*>(k_data + src * d + c0);
    vw[0] = *reinterpret_cast<const uint32_t*>(v_data + src * d + c0);
  }
  float xk[VEC], xv[VEC];
#pragma unroll
  for (int w = 0; w < VEC / 4; ++w) {
    float a[4], c[4];
    e4m3x4_f32(kw[w], a);
    e4m3x4_f32(vw[w], c);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      xk[4 * w + i] = __fmul_rn(a[i], sk);
      xv[4 * w + i] = __fmul_rn(c[i], sv);
    }
  }
  const int64_t o = (row0 + p) * kvh * d + static_cast<int64_t>(h) * d + c0;
  store_vec_nt<VEC>(out_k + o, xk);
  store_vec_nt<VEC>(out_v + o, xv);
}

template <typename T, typename I, int VEC>
int launch_store(const void* key, const void* value, const void* slots, int64_t rows, int kvh,
                 int d, int64_t num_slots, uint8_t* kd, float* ks, uint8_t* vd, float* vs,
                 hipStream_t s) {
  const int lanes = d / VEC;
  int gs = 1;
  while (gs < lanes) gs *= 2;
#define KVQ_FP8_STORE(GS)                                                                    \
  case GS: {                                                                                 \
    const int64_t blocks = (rows + (256 / GS) - 1) / (256 / GS);                             \
    if (blocks > 0x7fffffff) return KVQ_ERR_INVALID;                                         \
    hipLaunchKernelGGL((fp8_pth_store_kernel<T, I, VEC, GS>), dim3(static_cast<unsigned>(blocks)), \
                       dim3(256), 0, s, static_cast<const T*>(key), static_cast<const T*>(value), \
                       static_cast<const I*>(slots), rows, kvh, d, num_slots, kd, ks, vd, vs); \
    break;                                                                                   \
  }
  switch (gs) {
    KVQ_FP8_STORE(1)
    KVQ_FP8_STORE(2)
    KVQ_FP8_STORE(4)
    KVQ_FP8_STORE(8)
    KVQ_FP8_STORE(16)
    KVQ_FP8_STORE(32)
    KVQ_FP8_STORE(64)
    default:
      return KVQ_ERR_GEOMETRY;
  }
#undef KVQ_FP8_STORE
  return KVQ_OK;
}

}  // namespace

extern "C" int kvq_fp8_pth_store(const void* key, const void* value, int dtype,
                                 const void* slot_mapping, int slot_index_type,
                                 int64_t num_tokens, int num_kv_heads, int head_size,
                                 uint8_t* k_data, float* k_scale, uint8_t* v_data,
                                 float* v_scale, int64_t num_blocks, int block_size,
                                 void* stream) {
  if (num_tokens == 0) return KVQ_OK;
  if (!key || !value || !slot_mapping || !k_data || !k_scale || !v_data || !v_scale ||
      num_tokens < 0 || num_blocks <= 0 || block_size <= 0 || num_kv_heads <= 0)
    return KVQ_ERR_INVALID;
  if (head_size <= 0 || head_size % 4) return KVQ_ERR_GEOMETRY;
  const bool vec8 = head_size % 8 == 0;
  if (head_size > (vec8 ? 8 : 4) * 64) return KVQ_ERR_GEOMETRY;
  const int64_t rows = num_tokens * num_kv_heads;
  const int64_t num_slots = num_blocks * static_cast<int64_t>(block_size);
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = KVQ_OK;
  KVQ_DISPATCH_FLOAT(dtype, T,
    KVQ_DISPATCH_INDEX(slot_index_type, I,
      rc = vec8 ? launch_store<T, I, 8>(key, value, slot_mapping, rows, num_kv_heads, head_size,
                                        num_slots, k_data, k_scale, v_data, v_scale, s)
                : launch_store<T, I, 4>(key, value, slot_mapping, rows, num_kv_heads, head_size,
                                        num_slots, k_data, k_scale, v_data, v_scale, s)));
  if (rc != KVQ_OK) return rc;
  KVQ_LAUNCH_CHECK();
  return KVQ_OK;
}

extern "C" int kvq_fp8_pth_gather(const uint8_t* k_data, const float* k_scale,
                                  const uint8_t* v_data, const float* v_scale,
                                  int64_t num_blocks, int block_size, int num_kv_heads,
                                  int head_size, const void* block_table, int block_index_type,
                                  int64_t max_blocks, const int64_t* cu_seqlens, int64_t batch,
                                  void* out_k, void* out_v, int out_dtype, void* stream) {
  if (batch == 0 || max_blocks == 0) return KVQ_OK;
  if (!k_data || !k_scale || !v_data || !v_scale || !block_table || !cu_seqlens || !out_k ||
      !out_v || batch < 0 || max_blocks < 0 || num_blocks <= 0 || block_size <= 0 ||
      num_kv_heads <= 0 || batch > 65535)
    return KVQ_ERR_INVALID;
  if (head_size <= 0 || head_size % 4) return KVQ_ERR_GEOMETRY;
  const bool vec8 = head_size % 8 == 0;
  const int vec = vec8 ? 8 : 4;
  // grid.x covers the longest request the table can describe
  const int64_t per_pos = static_cast<int64_t>(num_kv_heads) * (head_size / vec);
  const int64_t blocks = (max_blocks * block_size * per_pos + 255) / 256;
  if (blocks > 0x7fffffff) return KVQ_ERR_INVALID;
  const dim3 grid(static_cast<unsigned>(blocks), static_cast<unsigned>(batch));
  hipStream_t s = static_cast<hipStream_t>(stream);
  KVQ_DISPATCH_FLOAT(out_dtype, TO,
    KVQ_DISPATCH_INDEX(block_index_type, TB,
      if (vec8)
        hipLaunchKernelGGL((fp8_pth_gather_kernel<TO, TB, 8>), grid, dim3(256), 0, s, k_data,
                           k_scale, v_data, v_scale, block_size, num_kv_heads, head_size,
                           num_blocks, static_cast<const TB*>(block_table), max_blocks,
                           cu_seqlens, static_cast<TO*>(out_k), static_cast<TO*>(out_v));
      else
        hipLaunchKernelGGL((fp8_pth_gather_kernel<TO, TB, 4>), grid, dim3(256), 0, s, k_data,
                           k_scale, v_data, v_scale, block_size, num_kv_heads, head_size,
                           num_blocks, static_cast<const TB*>(block_table), max_blocks,
                           cu_seqlens, static_cast<TO*>(out_k), static_cast<TO*>(out_v))));
  KVQ_LAUNCH_CHECK();
  return KVQ_OK;
}
