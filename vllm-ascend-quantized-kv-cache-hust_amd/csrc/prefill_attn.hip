// SPDX-License-Identifier: Apache-2.0
// Causal (or full) attention over dense TND K/V on MFMA, for prefill and the
// prompt rows of a chunked batch.
//
// Replaces the NPU fused-attention calls with input_layout "TND":
// pkg/methods/kivi_int4/attention_backend.py:1248-1262 (PrefillNoCache),
// :1320-1334 (chunked prompt rows), the dense fallback :1341-1392, and the
// INT8 prefill paths pkg/methods/int8_dynamic/attention_backend.py:282-296,
// 350-364.  Query row i of a request with lq queries and lk keys sits at
// position lk - lq + i; with `causal`, key positions past it are masked
// (pkg/methods/kivi_int4/semantics.py:285-299).
//
// One workgroup = 4 waves = 64 query rows of one query head; each wave owns
// 16 rows.  Keys/values stream through LDS in 32-token blocks.
//   S^T = K * Q^T   (v_mfma_f32_16x16x32_{bf16,f16}): A = K rows from LDS
//                   (16-byte reads), B = Q^T from registers (loaded once).
//   O^T += V^T * P^T: B = P^T straight from the S^T result registers (each
//                   lane already holds its query row's 8 probabilities);
//                   A = V^T read from the LDS block.
// Online softmax in the log2 domain, fp32 accumulation, output in the input
// dtype (fp32 inputs run through bf16 operands).
#include "kvq_common.h"

namespace {

using namespace kvq;

typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef uint16_t u8v __attribute__((ext_vector_type(8)));

constexpr int kRowsPerWave = 16;
constexpr int kWaves = 4;
constexpr int kKvBlock = 32;

// Operand element type of the MFMA for an input type.
template <typename T> struct Op { using type = bf16; };
template <> struct Op<f16> { using type = f16; };

__device__ __forceinline__ uint16_t op_bits(float x, bf16) { return f32_to_bf16_bits(x); }
__device__ __forceinline__ uint16_t op_bits(float x, f16) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}
template <typename T>
__device__ __forceinline__ uint16_t raw_bits(T v) {
  return op_bits(to_f32(v), typename Op<T>::type{});
}
template <>
__device__ __forceinline__ uint16_t raw_bits<bf16>(bf16 v) { return v.bits; }
template <>
__device__ __forceinline__ uint16_t raw_bits<f16>(f16 v) { return __builtin_bit_cast(uint16_t, v); }

__device__ __forceinline__ float op_to_f32(uint16_t bits, bf16) {
  return __uint_as_float(static_cast<uint32_t>(bits) << 16);
}
__device__ __forceinline__ float op_to_f32(uint16_t bits, f16) {
  return static_cast<float>(__builtin_bit_cast(_Float16, bits));
}

__device__ __forceinline__ f4 mfma16(u8v a, u8v b, f4 c, bf16) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8, a), __builtin_bit_cast(b8, b),
                                                 c, 0, 0, 0);
}
__device__ __forceinline__ f4 mfma16(u8v a, u8v b, f4 c, f16) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a), __builtin_bit_cast(h8, b),
                                                c, 0, 0, 0);
}

// Eight consecutive elements as operand bits (one 16-byte load for 16-bit types).
template <typename T>
__device__ __forceinline__ u8v load_op8(const T* p) {
  u8v r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = raw_bits(p[i]);
  return r;
}
template <>
__device__ __forceinline__ u8v load_op8<bf16>(const bf16* p) {
  return *reinterpret_cast<const u8v*>(p);
}
template <>
__device__ __forceinline__ u8v load_op8<f16>(const f16* p) {
  return *reinterpret_cast<const u8v*>(p);
}

template <typename T, int D>
__global__ void __launch_bounds__(256)
prefill_attn_kernel(const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
                    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k, int hq,
                    int kvh, float qscale, int causal, T* __restrict__ out) {
  using O = typename Op<T>::type;
  constexpr int KS = D / 32;   // k-steps of the score MFMA
  constexpr int DB = D / 16;   // 16-dim output blocks
  __shared__ uint16_t s_k[kKvBlock * D];
  __shared__ uint16_t s_v[kKvBlock * D];

  const int b = blockIdx.z;
  const int head = blockIdx.y;
  const int kvhead = head / (hq / kvh);
  const int q_start = cu_q[b];
  const int lq = cu_q[b + 1] - q_start;
  const int k_start = cu_k[b];
  const int lk = cu_k[b + 1] - k_start;
  const int row0 = blockIdx.x * (kRowsPerWave * kWaves);
  if (row0 >= lq) return;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int n = lane & 15;
  const int kg = lane >> 4;
  const int wrow0 = row0 + wave * kRowsPerWave;
  const int my_row = wrow0 + n;           // query row of the lane's column
  const bool row_live = my_row < lq;
  const int my_pos = lk - lq + my_row;    // its kv position
  // kv range the workgroup needs
  const int last_row = min(row0 + kRowsPerWave * kWaves, lq) - 1;
  const int kv_end = causal ? min(lk, lk - lq + last_row + 1) : lk;

  // Q^T operand: lane (col n = query row, k-group kg) holds dims 32*s + 8*kg + i
  u8v qop[KS];
  {
    const T* qrow = q + (static_cast<int64_t>(q_start + (row_live ? my_row : 0)) * hq + head) * D;
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int i = 0; i < 8; ++i)  // unscaled: exact in the operand type
        qop[s][i] = row_live ? raw_bits(qrow[32 * s + 8 * kg + i]) : uint16_t(0);
  }

  float m_run = -INFINITY, l_run = 0.0f;
  f4 o[DB];
#pragma unroll
  for (int j = 0; j < DB; ++j) o[j] = f4{0.f, 0.f, 0.f, 0.f};

  for (int kb = 0; kb < kv_end; kb += kKvBlock) {
    __syncthreads();
    // stage K and V rows [kb, kb + 32) of this kv head (16-byte loads)
    constexpr int QPR = D / 8;  // 8-element pieces per row
    for (int e = tid; e < kKvBlock * QPR; e += 256) {
      const int t = e / QPR;
      const int c = (e - t * QPR) * 8;
      const int pos = kb + t;
      u8v kvv, vvv;
      if (pos < lk) {
        const int64_t src = (static_cast<int64_t>(k_start + pos) * kvh + kvhead) * D + c;
        kvv = load_op8(k + src);
        vvv = load_op8(v + src);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          kvv[i] = 0;
          vvv[i] = 0;
        }
      }
      *reinterpret_cast<u8v*>(s_k + t * D + c) = kvv;
      *reinterpret_cast<u8v*>(s_v + t * D + c) = vvv;
    }
    __syncthreads();
    // waves whose rows are all before this block under the causal mask skip it
    const int wave_last_pos = lk - lq + min(wrow0 + kRowsPerWave, lq) - 1;
    if (wrow0 >= lq || (causal && kb > wave_last_pos)) continue;

    // scores: two 16-token halves; lane holds query row n, tokens 4*kg + r (+16)
    f4 s0 = f4{0.f, 0.f, 0.f, 0.f}, s1 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u8v a0 = *reinterpret_cast<const u8v*>(s_k + n * D + 32 * s + 8 * kg);
      const u8v a1 = *reinterpret_cast<const u8v*>(s_k + (16 + n) * D + 32 * s + 8 * kg);
      s0 = mfma16(a0, qop[s], s0, O{});
      s1 = mfma16(a1, qop[s], s1, O{});
    }
    float sc[8];
    float tmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int p0 = kb + 4 * kg + r;
      const int p1 = p0 + 16;
      const bool ok0 = p0 < lk && (!causal || p0 <= my_pos);
      const bool ok1 = p1 < lk && (!causal || p1 <= my_pos);
      sc[r] = ok0 ? s0[r] * qscale : -INFINITY;
      sc[4 + r] = ok1 ? s1[r] * qscale : -INFINITY;
      tmax = fmaxf(tmax, fmaxf(sc[r], sc[4 + r]));
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = m_run == -INFINITY ? (m_new == -INFINITY ? 1.0f : 0.0f)
                                           : exp2f(m_run - m_new);
    float psum = 0.0f;
    u8v pop;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float p = m_new == -INFINITY ? 0.0f : exp2f(sc[i] - m_new);
      pop[i] = op_bits(p, O{});
      // normalise by the probabilities the MFMA actually sees
      psum += op_to_f32(pop[i], O{});
    }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;
    // PV: A = V^T rows (dims), 8 tokens {4*kg + r, 16 + 4*kg + r}
#pragma unroll
    for (int j = 0; j < DB; ++j) {
      const int dim = 16 * j + n;
      u8v a;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        a[r] = s_v[(4 * kg + r) * D + dim];
        a[4 + r] = s_v[(16 + 4 * kg + r) * D + dim];
      }
      o[j] *= alpha;
      o[j] = mfma16(a, pop, o[j], O{});
    }
  }
  if (!row_live) return;
  // o[j][r] = O^T[dim 16*j + 4*kg + r][row n]
  const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
  T* orow = out + (static_cast<int64_t>(q_start + my_row) * hq + head) * D;
#pragma unroll
  for (int j = 0; j < DB; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) orow[16 * j + 4 * kg + r] = from_f32<T>(o[j][r] * inv);
}

}  // namespace

extern "C" int kvq_prefill_attn(const void* query, const void* key, const void* value, int dtype,
                                const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                int64_t batch, int64_t max_q_len, int num_heads,
                                int num_kv_heads, int head_size, float scale, int causal,
                                void* out, void* stream) {
  if (batch == 0 || max_q_len == 0) return KVQ_OK;
  if (!query || !key || !value || !cu_seqlens_q || !cu_seqlens_k || !out || batch < 0 ||
      max_q_len < 0 || batch > 65535 || num_heads > 65535)
    return KVQ_ERR_INVALID;
  if (num_kv_heads <= 0 || num_heads % num_kv_heads) return KVQ_ERR_GEOMETRY;
  if (head_size != 64 && head_size != 128 && head_size != 256 && head_size != 32)
    return KVQ_ERR_GEOMETRY;
  const int64_t qblocks = (max_q_len + 63) / 64;
  if (qblocks > 0x7fffffff) return KVQ_ERR_INVALID;
  const dim3 grid(static_cast<unsigned>(qblocks), num_heads, static_cast<unsigned>(batch));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const float qscale = scale * 1.4426950408889634f;
#define KVQ_PREFILL(DD)                                                                  \
  KVQ_DISPATCH_FLOAT(dtype, T,                                                           \
    hipLaunchKernelGGL((prefill_attn_kernel<T, DD>), grid, dim3(256), 0, s,              \
                       static_cast<const T*>(query), static_cast<const T*>(key),          \
                       static_cast<const T*>(value), cu_seqlens_q, cu_seqlens_k,          \
                       num_heads, num_kv_heads, qscale, causal, static_cast<T*>(out)))
  switch (head_size) {
    case 32: KVQ_PREFILL(32); break;
    case 64: KVQ_PREFILL(64); break;
    case 128: KVQ_PREFILL(128); break;
    default: KVQ_PREFILL(256); break;
  }
#undef KVQ_PREFILL
  KVQ_LAUNCH_CHECK();
  return KVQ_OK;
}
