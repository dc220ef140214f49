// SPDX-License-Identifier: Apache-2.0
// INT8 dynamic per-channel KV cache kernels for MI355X (gfx950).
//
// Reference: pkg/methods/int8_dynamic/attention_backend.py (i8ab) and
// pkg/methods/int8_dynamic/semantics.py.
//   * scales     -- i8ab:130-150: amax over tokens per (head, dim), computed in
//                   the activation dtype, inv = (1/amax)*127, aq = 1/inv;
//   * quantize   -- i8ab:152-171 fused with the scatter the host's
//                   reshape_and_cache performs (i8ab:86-88);
//   * dequant    -- i8ab:370-404 (paged int8 -> dense TND);
//   * decode     -- i8ab:173-205 (fused attention with per-channel antiquant).
// Every arithmetic step of scales/quantize/dequant rounds to the activation
// dtype exactly where torch does, so codes and scales are bit-exact.
#include <algorithm>

#include "kvq_common.h"
#include "kvq_decode.h"

namespace {

using namespace kvq;

// ---- scales ----------------------------------------------------------------

// amax over tokens, per channel and side.  A workgroup takes a slice of the
// tokens for up to 2048 channels (blockIdx.y picks the 2048): thread (r, ph)
// keeps the max of channels [8r, 8r + 8) over tokens t0 + ph, t0 + ph +
// phases, ... with four rows in flight per step; the phases meet in LDS and
// one integer atomicMax per channel and workgroup folds the slice in (|x| bits
// order like the floats, and the max does not depend on the order).
template <typename T>
__global__ void __launch_bounds__(256)
int8_amax_kernel(const T* __restrict__ key, const T* __restrict__ value, int64_t tokens,
                 int64_t channels, int64_t tokens_per_block, uint32_t* __restrict__ amax) {
  __shared__ float part[256 * 8];
  const int side = blockIdx.z;
  const int64_t cbase = static_cast<int64_t>(blockIdx.y) * 2048;
  const int cn = static_cast<int>(channels - cbase < 2048 ? channels - cbase : 2048);
  const int rt = cn / 8;         // threads per token row, <= 256
  const int phases = 256 / rt;   // >= 1
  const int tid = threadIdx.x;
  const int r = tid % rt;
  const int ph = tid / rt;
  const T* x = (side == 0 ? key : value) + cbase + 8 * r;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * tokens_per_block;
  const int64_t t1 = t0 + tokens_per_block < tokens ? t0 + tokens_per_block : tokens;
  float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (ph < phases) {
    int64_t t = t0 + ph;
    for (; t + 3 * phases < t1; t += 4 * phases) {
      float v0[8], v1[8], v2[8], v3[8];
      load8(x + t * channels, v0);
      load8(x + (t + phases) * channels, v1);
      load8(x + (t + 2 * phases) * channels, v2);
      load8(x + (t + 3 * phases) * channels, v3);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        a[i] = fmaxf(a[i], fmaxf(fmaxf(fabsf(v0[i]), fabsf(v1[i])),
                                 fmaxf(fabsf(v2[i]), fabsf(v3[i]))));
    }
    for (; t < t1; t += phases) {
      float v[8];
      load8(x + t * channels, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) a[i] = fmaxf(a[i], fabsf(v[i]));
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) part[tid * 8 + i] = a[i];
  __syncthreads();
  if (tid < rt) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float m = part[tid * 8 + i];
      for (int q = 1; q < phases; ++q) m = fmaxf(m, part[(q * rt + tid) * 8 + i]);
      atomicMax(amax + side * channels + cbase + 8 * tid + i, __float_as_uint(m));
    }
  }
}

__global__ void zero_u32_kernel(uint32_t* p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

template <typename T>
__global__ void __launch_bounds__(256)
int8_finalize_scales_kernel(const uint32_t* __restrict__ amax, int64_t channels,
                            T* __restrict__ k_inv, T* __restrict__ v_inv, T* __restrict__ k_aq,
                            T* __restrict__ v_aq) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= 2 * channels) return;
  const int side = i >= channels;
  const int64_t c = i - side * channels;
  float a = __uint_as_float(amax[i]);            // exact value of the dtype
  if (a < 1.0e-12f) a = round_to<T>(1.0e-12f);   // clamp(min=1e-12) in the dtype
  const float r = round_to<T>(1.0f / a);         // reciprocal()
  const float inv = round_to<T>(r * 127.0f);     // * 127.0
  const float aq = round_to<T>(1.0f / inv);      // 1.0 / inv
  (side ? v_inv : k_inv)[c] = from_f32<T>(inv);
  (side ? v_aq : k_aq)[c] = from_f32<T>(aq);
}

// ---- quantize + scatter ----------------------------------------------------

template <typename T>
__device__ __forceinline__ int8_t int8_code(float x, float inv) {
  const float p = round_to<T>(x * inv);  // x * inv (+ 0) in the activation dtype
  float r = rintf(p);                    // torch.round: half to even
  r = r < -128.0f ? -128.0f : (r > 127.0f ? 127.0f : r);
  return static_cast<int8_t>(r);
}

template <typename T, typename I>
__global__ void __launch_bounds__(256)
int8_quant_scatter_kernel(const T* __restrict__ key, const T* __restrict__ value,
                          const T* __restrict__ k_inv, const T* __restrict__ v_inv,
                          const I* __restrict__ slots, int64_t tokens, int64_t channels,
                          int8_t* __restrict__ kc, int8_t* __restrict__ vc) {
  const int64_t per_row = channels / 8;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= tokens * per_row) return;
  const int64_t t = gid / per_row;
  const int64_t c8 = (gid - t * per_row) * 8;
  const int64_t slot = ld_index(slots, t);
  if (slot < 0) return;
  float xk[8], xv[8], ik[8], iv[8];
  load8(key + t * channels + c8, xk);
  load8(value + t * channels + c8, xv);
  load8(k_inv + c8, ik);
  load8(v_inv + c8, iv);
  uint32_t k_lo = 0, k_hi = 0, v_lo = 0, v_hi = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    k_lo |= (static_cast<uint32_t>(static_cast<uint8_t>(int8_code<T>(xk[i], ik[i])))) << (8 * i);
    k_hi |= (static_cast<uint32_t>(static_cast<uint8_t>(int8_code<T>(xk[i + 4], ik[i + 4])))) << (8 * i);
    v_lo |= (static_cast<uint32_t>(static_cast<uint8_t>(int8_code<T>(xv[i], iv[i])))) << (8 * i);
    v_hi |= (static_cast<uint32_t>(static_cast<uint8_t>(int8_code<T>(xv[i + 4], iv[i + 4])))) << (8 * i);
  }
  // [NB, Bs, KVH, D] with slot = blk*Bs + off is row `slot` of [NB*Bs, KVH*D]
  *reinterpret_cast<uint2*>(kc + slot * channels + c8) = make_uint2(k_lo, k_hi);
  *reinterpret_cast<uint2*>(vc + slot * channels + c8) = make_uint2(v_lo, v_hi);
}

// ---- paged dequant to dense ------------------------------------------------

template <typename T>
__global__ void __launch_bounds__(256)
int8_dequant_gather_kernel(const int8_t* __restrict__ kc, const int8_t* __restrict__ vc, int bs,
                           int64_t channels, const T* __restrict__ k_aq,
                           const T* __restrict__ v_aq, const int32_t* __restrict__ block_table,
                           int64_t maxb, const int64_t* __restrict__ cu, T* __restrict__ out_k,
                           T* __restrict__ out_v) {
  const int b = blockIdx.y;
  const int64_t row0 = cu[b];
  const int64_t len = cu[b + 1] - row0;
  const int64_t per_row = channels / 8;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= len * per_row) return;
  const int64_t p = gid / per_row;
  const int64_t c8 = (gid - p * per_row) * 8;
  const int64_t blk = block_table[static_cast<int64_t>(b) * maxb + p / bs];
  const int64_t src = (blk * bs + p % bs) * channels + c8;
  const uint2 kw = *reinterpret_cast<const uint2*>(kc + src);
  const uint2 vw = *reinterpret_cast<const uint2*>(vc + src);
  float ak[8], av[8], xk[8], xv[8];
  load8(k_aq + c8, ak);
  load8(v_aq + c8, av);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t kword = i < 4 ? kw.x : kw.y;
    const uint32_t vword = i < 4 ? vw.x : vw.y;
    const float kq = static_cast<float>(static_cast<int8_t>((kword >> (8 * (i & 3))) & 0xffu));
    const float vq = static_cast<float>(static_cast<int8_t>((vword >> (8 * (i & 3))) & 0xffu));
    xk[i] = round_to<T>(kq * ak[i]);  // (x.to(dtype) - 0) * (1/inv) in the dtype
    xv[i] = round_to<T>(vq * av[i]);
  }
  store8_nt(out_k + (row0 + p) * channels + c8, xk);
  store8_nt(out_v + (row0 + p) * channels + c8, xv);
}

// ---- decode (generic wave-per-item kernel) ---------------------------------

constexpr int kMaxRep = 16;
constexpr int kMaxDpl = 4;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <typename T>
__global__ void __launch_bounds__(64)
int8_decode_generic_kernel(const T* __restrict__ query, int hq, int kvh, int d, float qscale,
                           const int8_t* __restrict__ kc, const int8_t* __restrict__ vc, int bs,
                           const T* __restrict__ k_aq, const T* __restrict__ v_aq,
                           const int32_t* __restrict__ block_table, int64_t maxb,
                           const int32_t* __restrict__ work, float* __restrict__ ws_o,
                           float* __restrict__ ws_ml) {
  const int wi = blockIdx.x;
  const int h = blockIdx.y;
  const int lane = threadIdx.x;
  const int32_t* wk = work + 4 * static_cast<int64_t>(wi);
  const int b = wk[0], pb = wk[1], pe = wk[2];
  const int rep = hq / kvh;
  const int dpl = (d + 63) / 64;
  const int64_t channels = static_cast<int64_t>(kvh) * d;
  const int32_t* bt = block_table + static_cast<int64_t>(b) * maxb;

  __shared__ float s_q[kMaxRep * 256];
  __shared__ float s_p[kMaxRep * 64];
  for (int i = lane; i < rep * d; i += 64) {
    const int r = i / d;
    const int c = i - r * d;
    // fold the key antiquant scale into q: q.(x*aq) = (q*aq).x
    s_q[i] = to_f32(query[(static_cast<int64_t>(b) * hq + h * rep + r) * d + c]) * qscale *
             to_f32(k_aq[h * d + c]);
  }
  __syncthreads();
  float m[kMaxRep], l[kMaxRep], acc[kMaxRep][kMaxDpl];
#pragma unroll
  for (int r = 0; r < kMaxRep; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.0f;
#pragma unroll
    for (int k = 0; k < kMaxDpl; ++k) acc[r][k] = 0.0f;
  }
  for (int p0 = pb; p0 < pe; p0 += 64) {
    const int p = p0 + lane;
    const bool live = p < pe;
    float s[kMaxRep];
#pragma unroll
    for (int r = 0; r < kMaxRep; ++r) s[r] = 0.0f;
    if (live) {
      const int64_t blk = bt[p / bs];
      const int8_t* krow = kc + (blk * bs + p % bs) * channels + static_cast<int64_t>(h) * d;
      for (int c = 0; c < d; ++c) {
        const float kv = static_cast<float>(krow[c]);
#pragma unroll
        for (int r = 0; r < kMaxRep; ++r)
          if (r < rep) s[r] += s_q[r * d + c] * kv;
      }
    }
#pragma unroll
    for (int r = 0; r < kMaxRep; ++r) {
      if (r >= rep) continue;
      const float sr = live ? s[r] : -INFINITY;
      const float m_new = fmaxf(m[r], wave_max(sr));
      const float alpha = (m[r] == -INFINITY) ? 0.0f : exp2f(m[r] - m_new);
      const float pr = live ? exp2f(sr - m_new) : 0.0f;
      l[r] = l[r] * alpha + wave_sum(pr);
#pragma unroll
      for (int k = 0; k < kMaxDpl; ++k) acc[r][k] *= alpha;
      m[r] = m_new;
      s_p[r * 64 + lane] = pr;
    }
    __syncthreads();
    const int n = (pe - p0) < 64 ? (pe - p0) : 64;
    for (int i = 0; i < n; ++i) {
      const int pp = p0 + i;
      const int64_t blk = bt[pp / bs];
      const int8_t* vrow = vc + (blk * bs + pp % bs) * channels + static_cast<int64_t>(h) * d;
#pragma unroll
      for (int k = 0; k < kMaxDpl; ++k) {
        const int c = lane + 64 * k;
        if (k >= dpl || c >= d) continue;
        const float v = static_cast<float>(vrow[c]);
#pragma unroll
        for (int r = 0; r < kMaxRep; ++r)
          if (r < rep) acc[r][k] += s_p[r * 64 + i] * v;
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int r = 0; r < kMaxRep; ++r) {
    if (r >= rep) continue;
    const int64_t hh = static_cast<int64_t>(wi) * hq + h * rep + r;
    if (lane == 0) {
      ws_ml[2 * hh] = m[r];
      ws_ml[2 * hh + 1] = l[r];
    }
#pragma unroll
    for (int k = 0; k < kMaxDpl; ++k) {
      const int c = lane + 64 * k;
      // the value antiquant scale is per output channel: apply it once here
      if (k < dpl && c < d) ws_o[hh * d + c] = acc[r][k] * to_f32(v_aq[h * d + c]);
    }
  }
}

}  // namespace

extern "C" int kvq_int8_calc_scales(const void* key, const void* value, int dtype,
                                    int64_t num_tokens, int64_t channels, uint32_t* amax_ws,
                                    void* k_inv, void* v_inv, void* k_aq, void* v_aq,
                                    void* stream) {
  if (!key || !value || !amax_ws || !k_inv || !v_inv || !k_aq || !v_aq || num_tokens < 0 ||
      channels <= 0 || channels % 8)
    return KVQ_ERR_INVALID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t n = 2 * channels;
  hipLaunchKernelGGL(zero_u32_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     s, amax_ws, n);
  KVQ_LAUNCH_CHECK();
  if (num_tokens > 0) {
    // about 256 token slices per side (at least 1024 tokens each): enough
    // workgroups to fill the chip, few atomics per channel
    const int64_t cblocks = (channels + 2047) / 2048;
    const int64_t tpb = std::max<int64_t>(1024, (num_tokens + 255) / 256);
    const int64_t tblocks = (num_tokens + tpb - 1) / tpb;
    if (tblocks > 0x7fffffff || cblocks > 65535) return KVQ_ERR_INVALID;
    const dim3 grid(static_cast<unsigned>(tblocks), static_cast<unsigned>(cblocks), 2);
    KVQ_DISPATCH_FLOAT(dtype, T,
      hipLaunchKernelGGL((int8_amax_kernel<T>), grid, dim3(256), 0, s,
                         static_cast<const T*>(key), static_cast<const T*>(value), num_tokens,
                         channels, tpb, amax_ws));
    KVQ_LAUNCH_CHECK();
  }
  KVQ_DISPATCH_FLOAT(dtype, T,
    hipLaunchKernelGGL((int8_finalize_scales_kernel<T>), dim3(static_cast<unsigned>((n + 255) / 256)),
                       dim3(256), 0, s, amax_ws, channels, static_cast<T*>(k_inv),
                       static_cast<T*>(v_inv), static_cast<T*>(k_aq), static_cast<T*>(v_aq)));
  KVQ_LAUNCH_CHECK();
  return KVQ_OK;
}

extern "C" int kvq_int8_quant_scatter(const void* key, const void* value, int dtype,
                                      const void* k_inv, const void* v_inv,
                                      const void* slot_mapping, int slot_index_type,
                                      int64_t num_tokens, int64_t channels, int8_t* key_cache,
                                      int8_t* value_cache, int64_t num_blocks, int block_size,
                                      void* stream) {
  if (num_tokens == 0) return KVQ_OK;
  if (!key || !value || !k_inv || !v_inv || !slot_mapping || !key_cache || !value_cache ||
      num_tokens < 0 || channels <= 0 || channels % 8 || num_blocks <= 0 || block_size <= 0)
    return KVQ_ERR_INVALID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t total = num_tokens * (channels / 8);
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7fffffff) return KVQ_ERR_INVALID;
  KVQ_DISPATCH_FLOAT(dtype, T,
    KVQ_DISPATCH_INDEX(slot_index_type, I,
      hipLaunchKernelGGL((int8_quant_scatter_kernel<T, I>), dim3(static_cast<unsigned>(blocks)),
                         dim3(256), 0, s, static_cast<const T*>(key),
                         static_cast<const T*>(value), static_cast<const T*>(k_inv),
                         static_cast<const T*>(v_inv), static_cast<const I*>(slot_mapping),
                         num_tokens, channels, key_cache, value_cache)));
  KVQ_LAUNCH_CHECK();
  return KVQ_OK;
}

extern "C" int kvq_int8_dequant_gather(const int8_t* key_cache, const int8_t* value_cache,
                                       int64_t num_blocks, int block_size, int num_kv_heads,
                                       int head_size, const void* k_aq, const void* v_aq,
                                       int dtype, const int32_t* block_table,
                                       int64_t max_blocks, const int64_t* cu_seqlens,
                                       int64_t batch, void* out_k, void* out_v, void* stream) {
  if (batch == 0) return KVQ_OK;
  if (!key_cache || !value_cache || !k_aq || !v_aq || !block_table || !cu_seqlens || !out_k ||
      !out_v || batch < 0 || num_blocks <= 0 || block_size <= 0 || head_size % 8 ||
      num_kv_heads <= 0 || batch > 65535)
    return KVQ_ERR_INVALID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t channels = static_cast<int64_t>(num_kv_heads) * head_size;
  // grid.x covers the longest request: max_blocks * block_size rows
  const int64_t rows = max_blocks * block_size;
  const int64_t blocks = (rows * (channels / 8) + 255) / 256;
  if (blocks > 0x7fffffff) return KVQ_ERR_INVALID;
  const dim3 grid(static_cast<unsigned>(blocks), static_cast<unsigned>(batch));
  KVQ_DISPATCH_FLOAT(dtype, T,
    hipLaunchKernelGGL((int8_dequant_gather_kernel<T>), grid, dim3(256), 0, s, key_cache,
                       value_cache, block_size, channels, static_cast<const T*>(k_aq),
                       static_cast<const T*>(v_aq), block_table, max_blocks, cu_seqlens,
                       static_cast<T*>(out_k), static_cast<T*>(out_v)));
  KVQ_LAUNCH_CHECK();
  return KVQ_OK;
}

extern "C" int64_t kvq_int8_decode_workspace_bytes(int64_t num_work, int num_heads,
                                                   int head_size) {
  return kvq::decode_workspace_bytes(num_work, num_heads, head_size);
}

extern "C" int kvq_int8_decode_attn(const void* query, int dtype, int64_t batch, int num_heads,
                                    int num_kv_heads, int head_size, float scale,
                                    const int8_t* key_cache, const int8_t* value_cache,
                                    int64_t num_blocks, int block_size, const void* k_aq,
                                    const void* v_aq, const int32_t* block_table,
                                    int64_t max_blocks, const int32_t* seq_meta,
                                    const int32_t* work, int64_t num_work, void* workspace,
                                    void* out, void* stream) {
  if (batch == 0) return KVQ_OK;
  if (!query || !key_cache || !value_cache || !k_aq || !v_aq || !block_table || !seq_meta ||
      !work || !workspace || !out || batch < 0 || num_work <= 0 || num_blocks <= 0 ||
      block_size <= 0)
    return KVQ_ERR_INVALID;
  if (num_kv_heads <= 0 || num_heads % num_kv_heads || head_size % 8 || head_size > 256 ||
      num_heads / num_kv_heads > kMaxRep)
    return KVQ_ERR_GEOMETRY;
  if (num_work > 0x7fffffff || batch > 0x7fffffff || num_heads > 65535) return KVQ_ERR_INVALID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* ws_o = static_cast<float*>(workspace);
  float* ws_ml = ws_o + num_work * num_heads * head_size;
  const float qscale = scale * 1.4426950408889634f;
  bool mfma = false;
  int rc = kvq::launch_int8_decode_mfma(query, dtype, num_heads, num_kv_heads, head_size, qscale,
                                       key_cache, value_cache, block_size, num_blocks,
                                       k_aq, v_aq,
                                       block_table, max_blocks, work, num_work, ws_o, ws_ml, s,
                                       &mfma);
  if (rc != KVQ_OK) return rc;
  if (!mfma) {  // the MFMA kernel covers every item (empty ones included) when it runs
    const dim3 grid(static_cast<unsigned>(num_work), num_kv_heads);
    KVQ_DISPATCH_FLOAT(dtype, T,
      hipLaunchKernelGGL((int8_decode_generic_kernel<T>), grid, dim3(64), 0, s,
                         static_cast<const T*>(query), num_heads, num_kv_heads, head_size,
                         qscale, key_cache, value_cache, block_size,
                         static_cast<const T*>(k_aq), static_cast<const T*>(v_aq), block_table,
                         max_blocks, work, ws_o, ws_ml));
    KVQ_LAUNCH_CHECK();
  }
  return kvq::launch_decode_combine(dtype, batch, num_heads, head_size, seq_meta, 4, 1, ws_o,
                                    ws_ml, out, s);
}
