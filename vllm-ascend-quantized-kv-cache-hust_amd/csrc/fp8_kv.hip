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
// The codes are those of the IEEE quotient x / scale; quantize_codes reaches
// them through one reciprocal per row and an exactness window, falling back to
// the division only next to a code boundary.  v_cvt_pk_fp8_f32 -- gfx950's
// conversion to OCP e4m3fn, round to nearest even -- packs four codes a word.
// Every value the clamp admits is finite, so the conversion never saturates.
//
// Store: a group of GS lanes holds one (token, head) row of keys and values;
// each lane holds NCH chunks of W elements, chunk j at lane * W + j * D / NCH
// (W = 8, NCH = 2 when D % 16 == 0), so every load and store instruction of
// a group covers contiguous bytes; amax is a butterfly inside the group.  HBM-bound: 2 B of bf16 in and
// 1 B of code out per element, plus 4 B of scale per row.
// Gather: one thread per NCH chunks of W codes of one (position, head) row,
// laid out as in the store, into dense TND rows of the activation dtype
// (code * scale in fp32, then RNE).
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

// The sign bits of four fp32 values at bit 7 of bytes 0..3.
__device__ __forceinline__ uint32_t sign_bytes(float a, float b, float c, float d) {
  // v_perm: bytes {a.b3, b.b3, 0, 0} and {0, 0, c.b3, d.b3}
  const uint32_t lo = __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x0c0c0703u);
  const uint32_t hi = __builtin_amdgcn_perm(__float_as_uint(d), __float_as_uint(c), 0x07030c0cu);
  return (lo | hi) & 0x80808080u;
}

// Codes of e4m3fn(clamp(x / scale, -448, 448)), four elements a word.
//
// The IEEE quotient is needed only where it decides a code.  With
// y = RN(1/scale), t = RN(|x| * y) is within (2^-23 + 2^-48) |q| of the exact
// quotient q = |x| / scale, and RN(q) within 2^-24 |q| of q, so RN(q) lies
// within 3.03 * 2^-24 |q| of t: fewer than 7 steps of the fp32 bit pattern,
// also when a binade boundary between them halves the step.  Rounding to E4M3
// (like the clamp) is monotone, so when t - 8 steps and t + 8 steps give the
// same code as t, every value between them does, RN(q) included.  Otherwise
// (a code boundary within 8 steps: about 1 element in 60,000) the word is
// recomputed from the IEEE quotient.  The sign is applied to the magnitude's
// code, as round-to-nearest and the clamp are symmetric (-0 gives 0x80).
template <int VEC>
__device__ __forceinline__ void quantize_codes(const float (&x)[VEC], float scale,
                                               uint32_t (&codes)[VEC / 4]) {
  const float y = __fdiv_rn(1.0f, scale);
#pragma unroll
  for (int w = 0; w < VEC / 4; ++w) {
    float t[4], lo[4], hi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      t[i] = fminf(fabsf(x[4 * w + i]) * y, kE4M3Max);
      const uint32_t b = __float_as_uint(t[i]);
      lo[i] = __uint_as_float(__builtin_elementwise_sub_sat(b, 8u));
      hi[i] = fminf(__uint_as_float(b + 8u), kE4M3Max);
    }
    uint32_t c = e4m3x4(t[0], t[1], t[2], t[3]);
    const uint32_t cl = e4m3x4(lo[0], lo[1], lo[2], lo[3]);
    const uint32_t ch = e4m3x4(hi[0], hi[1], hi[2], hi[3]);
    if (cl != c || ch != c) {
#pragma unroll
      for (int i = 0; i < 4; ++i) t[i] = fminf(__fdiv_rn(fabsf(x[4 * w + i]), scale), kE4M3Max);
      c = e4m3x4(t[0], t[1], t[2], t[3]);
    }
    codes[w] = c | sign_bytes(x[4 * w], x[4 * w + 1], x[4 * w + 2], x[4 * w + 3]);
  }
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
  float scale = __fdiv_rn(amax, kE4M3Max);
  scale = scale < kScaleFloor ? kScaleFloor : scale;
  quantize_codes<VEC>(x, scale, codes);
  return scale;
}

template <typename T, typename I, int W, int NCH, int GS>
__global__ void __launch_bounds__(256)
fp8_pth_store_kernel(const T* __restrict__ key, const T* __restrict__ value,
                     const I* __restrict__ slots, uint32_t rows, FastDiv kvh, int d,
                     int64_t num_slots, uint8_t* __restrict__ k_data,
                     float* __restrict__ k_scale, uint8_t* __restrict__ v_data,
                     float* __restrict__ v_scale) {
  constexpr int VEC = W * NCH;
  constexpr int kRowsPerBlock = 256 / GS;
  const int lane = threadIdx.x % GS;
  const uint32_t row = blockIdx.x * kRowsPerBlock + threadIdx.x / GS;
  if (row >= rows) return;  // whole groups leave together
  const uint32_t tok = kvh.div(row);
  const int h = static_cast<int>(row - tok * kvh.d);
  const int64_t slot = ld_index(slots, tok);
  if (slot < 0 || slot >= num_slots) return;  // padding (negative) or outside the cache
  // chunk j of this lane: W elements at lane * W + j * (d / NCH)
  const int c0 = lane * W;
  const int half = d / NCH;
  const bool active = c0 < half;
  float xk[VEC], xv[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) xk[i] = xv[i] = 0.0f;
  if (active) {
    const int64_t base = static_cast<int64_t>(row) * d + c0;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      float a[W], b[W];
      load_vec<W>(key + base + j * half, a);
      load_vec<W>(value + base + j * half, b);
#pragma unroll
      for (int i = 0; i < W; ++i) {
        xk[j * W + i] = a[i];
        xv[j * W + i] = b[i];
      }
    }
  }
  uint32_t ck[VEC / 4], cv[VEC / 4];
  const float sk = quantize_row<VEC, GS>(xk, active, ck);
  const float sv = quantize_row<VEC, GS>(xv, active, cv);
  const int64_t dst = slot * kvh.d + h;
  if (active) {
    uint8_t* kp = k_data + dst * d + c0;
    uint8_t* vp = v_data + dst * d + c0;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      if constexpr (W == 8) {
        *reinterpret_cast<uint2*>(kp + j * half) = make_uint2(ck[2 * j], ck[2 * j + 1]);
        *reinterpret_cast<uint2*>(vp + j * half) = make_uint2(cv[2 * j], cv[2 * j + 1]);
      } else {
        *reinterpret_cast<uint32_t*>(kp + j * half) = ck[j];
        *reinterpret_cast<uint32_t*>(vp + j * half) = cv[j];
      }
    }
  }
  if (lane == 0) {
    k_scale[dst] = sk;
    v_scale[dst] = sv;
  }
}

template <typename TO, typename TB, int W, int NCH>
__global__ void __launch_bounds__(256)
fp8_pth_gather_kernel(const uint8_t* __restrict__ k_data, const float* __restrict__ k_scale,
                      const uint8_t* __restrict__ v_data, const float* __restrict__ v_scale,
                      FastDiv bs, int kvh, int d, int64_t nb, const TB* __restrict__ block_table,
                      int64_t maxb, const int64_t* __restrict__ cu, FastDiv per_pos,
                      FastDiv per_head, TO* __restrict__ out_k, TO* __restrict__ out_v) {
  const int b = blockIdx.y;
  const int64_t row0 = cu[b];
  const int64_t len = cu[b + 1] - row0;
  const int half = d / NCH;
  // gid < 2^31 (the grid is checked on the host), so 32-bit division suffices
  const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
  if (static_cast<int64_t>(gid) >= len * per_pos.d) return;
  const uint32_t p = per_pos.div(gid);
  const uint32_t pb = bs.div(p);
  if (pb >= maxb) return;  // a length the table does not cover reads nothing past it
  const uint32_t rem = gid - p * per_pos.d;
  const uint32_t h = per_head.div(rem);
  const int c0 = static_cast<int>(rem - h * per_head.d) * W;  // chunk j at c0 + j * half
  int64_t blk = static_cast<int64_t>(block_table[static_cast<int64_t>(b) * maxb + pb]);
  blk = blk < 0 ? 0 : (blk >= nb ? nb - 1 : blk);  // unallocated ids read page 0
  const int64_t src = (blk * bs.d + (p - pb * bs.d)) * kvh + h;
  const float sk = k_scale[src];
  const float sv = v_scale[src];
  uint32_t kw[NCH][W / 4], vw[NCH][W / 4];
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const uint8_t* kp = k_data + src * d + c0 + j * half;
    const uint8_t* vp = v_data + src * d + c0 + j * half;
    if constexpr (W == 8) {
      const uint2 a = *reinterpret_cast<const uint2*>(kp);
      const uint2 c = *reinterpret_cast<const uint2*>(vp);
      kw[j][0] = a.x; kw[j][1] = a.y;
      vw[j][0] = c.x; vw[j][1] = c.y;
    } else {
      kw[j][0] = *reinterpret_cast<const uint32_t*>(kp);
      vw[j][0] = *reinterpret_cast<const uint32_t*>(vp);
    }
  }
  const int64_t o = (row0 + p) * kvh * d + static_cast<int64_t>(h) * d + c0;  // TND row
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    float xk[W], xv[W];
#pragma unroll
    for (int w = 0; w < W / 4; ++w) {
      float a[4], c[4];
      e4m3x4_f32(kw[j][w], a);
      e4m3x4_f32(vw[j][w], c);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xk[4 * w + i] = __fmul_rn(a[i], sk);
        xv[4 * w + i] = __fmul_rn(c[i], sv);
      }
    }
    store_vec_nt<W>(out_k + o + j * half, xk);
    store_vec_nt<W>(out_v + o + j * half, xv);
  }
}

template <typename T, typename I, int W, int NCH>
int launch_store(const void* key, const void* value, const void* slots, int64_t rows, int kvh,
                 int d, int64_t num_slots, uint8_t* kd, float* ks, uint8_t* vd, float* vs,
                 hipStream_t s) {
  const FastDiv kvh_div = FastDiv::make(static_cast<uint32_t>(kvh));
  const int lanes = d / (W * NCH);
  int gs = 1;
  while (gs < lanes) gs *= 2;
#define KVQ_FP8_STORE(GS)                                                                    \
  case GS: {                                                                                 \
    const int64_t blocks = (rows + (256 / GS) - 1) / (256 / GS);                             \
    if (blocks > 0x7fffffff) return KVQ_ERR_INVALID;                                         \
    hipLaunchKernelGGL((fp8_pth_store_kernel<T, I, W, NCH, GS>), dim3(static_cast<unsigned>(blocks)), \
                       dim3(256), 0, s, static_cast<const T*>(key), static_cast<const T*>(value), \
                       static_cast<const I*>(slots), static_cast<uint32_t>(rows), kvh_div, d, \
                       num_slots, kd, ks, vd, vs);                                            \
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
  const int vec = head_size % 16 == 0 ? 16 : (head_size % 8 == 0 ? 8 : 4);
  if (head_size > vec * 64) return KVQ_ERR_GEOMETRY;
  const int64_t rows = num_tokens * num_kv_heads;
  if (rows > 0x7fffffff) return KVQ_ERR_INVALID;
  const int64_t num_slots = num_blocks * static_cast<int64_t>(block_size);
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = KVQ_OK;
  KVQ_DISPATCH_FLOAT(dtype, T,
    KVQ_DISPATCH_INDEX(slot_index_type, I,
      rc = vec == 16 ? launch_store<T, I, 8, 2>(key, value, slot_mapping, rows, num_kv_heads,
                                                head_size, num_slots, k_data, k_scale, v_data,
                                                v_scale, s)
         : vec == 8 ? launch_store<T, I, 8, 1>(key, value, slot_mapping, rows, num_kv_heads,
                                               head_size, num_slots, k_data, k_scale, v_data,
                                               v_scale, s)
                    : launch_store<T, I, 4, 1>(key, value, slot_mapping, rows, num_kv_heads,
                                               head_size, num_slots, k_data, k_scale, v_data,
                                               v_scale, s)));
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
  const int vec = head_size % 16 == 0 ? 16 : (head_size % 8 == 0 ? 8 : 4);
  // grid.x covers the longest request the table can describe
  const int64_t per_pos = static_cast<int64_t>(num_kv_heads) * (head_size / vec);
  const int64_t threads = max_blocks * block_size * per_pos;
  if (threads > 0x7fffffff - 255) return KVQ_ERR_INVALID;
  const dim3 grid(static_cast<unsigned>((threads + 255) / 256), static_cast<unsigned>(batch));
  const FastDiv bs_div = FastDiv::make(static_cast<uint32_t>(block_size));
  const FastDiv pos_div = FastDiv::make(static_cast<uint32_t>(per_pos));
  const FastDiv head_div = FastDiv::make(static_cast<uint32_t>(head_size / vec));
  hipStream_t s = static_cast<hipStream_t>(stream);
#define KVQ_FP8_GATHER(W, NCH)                                                               \
  hipLaunchKernelGGL((fp8_pth_gather_kernel<TO, TB, W, NCH>), grid, dim3(256), 0, s, k_data, \
                     k_scale, v_data, v_scale, bs_div, num_kv_heads, head_size, num_blocks,  \
                     static_cast<const TB*>(block_table), max_blocks, cu_seqlens, pos_div,   \
                     head_div, static_cast<TO*>(out_k), static_cast<TO*>(out_v))
  KVQ_DISPATCH_FLOAT(out_dtype, TO,
    KVQ_DISPATCH_INDEX(block_index_type, TB,
      if (vec == 16)
        KVQ_FP8_GATHER(8, 2);
      else if (vec == 8)
        KVQ_FP8_GATHER(8, 1);
      else
        KVQ_FP8_GATHER(4, 1)));
#undef KVQ_FP8_GATHER
  KVQ_LAUNCH_CHECK();
  return KVQ_OK;
}
