// SPDX-License-Identifier: Apache-2.0
// Fused KIVI INT4 decode attention for MI355X (gfx950): split-K over a work
// list, log-sum-exp combine.
//
// The reference gathers the whole int4 history into a dense bf16 tensor and
// calls the NPU fused-attention op (pkg/methods/kivi_int4/attention_backend.py:
// 849-935, 1193-1230).  Here the history is dequantized in registers inside
// the attention kernel; positions past a side's int4 history read that
// side's residual ring directly, so nothing dense is ever materialized.
//
// Work items (built by the host from the request lengths, no device sync):
//   kind 0: a range where keys and values both come from int4 pages -- the
//           MFMA kernel of decode_mfma.hip;
//   kind 1: tails where one side is already in the ring -- the tail path of
//           decode_tail.h, run by the same launch in a second pass of its
//           grid (after every kind-0 wave), or by the standalone tail kernel
//           when the int4 kernel does not apply.
// Everything runs on the caller's stream.  Geometries neither MFMA path
// covers go to the generic kernel below: one wave per (work item, kv head),
// the QK dot products lane-per-position, the PV accumulation lane-per-dim.
// Each work item leaves (m, l, o[D]) per query head in the workspace (m in
// the log2 domain); the combine kernel merges a request's items.
#include <mutex>

#include "kvq_common.h"
#include "kvq_decode.h"

namespace {

using namespace kvq;

constexpr int kMaxRep = 16;   // query heads per kv head handled by the generic kernel
constexpr int kMaxDpl = 4;    // dims per lane (head_size <= 256)

__device__ __forceinline__ float wave_max(float v) { return max_wave64(v); }
__device__ __forceinline__ float wave_sum(float v) { return sum_wave64(v); }

// Staging of the K or V rows of positions [p0, p0 + n) (n <= 64) of one kv
// head into LDS as fp32 [64][d + 1].  Positions below `hist` come from the
// int4 pages (dequantized exactly: q*scale then +mn), the rest from the
// residual ring.  Every path issues its loads in independent batches before
// using them, so a wave waits for a few memory round trips, not one per load.

constexpr int kBatch = 8;

__device__ __forceinline__ int64_t clamp_page(const int32_t* __restrict__ bt, int p, int bs,
                                              int64_t nb) {
  const int64_t blk = bt[p / bs];
  return blk < 0 ? 0 : (blk >= nb ? nb - 1 : blk);  // never leave the cache
}

// Ring rows of positions [p0 + i0, p0 + n): task = (position, 8-dim chunk).
template <typename TR>
__device__ __forceinline__ void stage_ring(float* __restrict__ dst, int p0, int i0, int n,
                                           int hist, int kvh, int h, int d,
                                           const TR* __restrict__ ring, int64_t ring_row0,
                                           int ring_first, int ring_len, int lane) {
  const int ndv = d / 8;
  const int pitch = d + 1;
  const int tasks = (n - i0) * ndv;
  for (int t0 = 0; t0 < tasks; t0 += 64 * kBatch) {
    float x[kBatch][8];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int tk = t0 + 64 * k + lane;
      const int t = tk < tasks ? tk : tasks - 1;  // clamped: unconditional load
      const int pi = i0 + t / ndv;
      const int dv = t % ndv;
      const int rl = (ring_first + (p0 + pi - hist)) % ring_len;
      load8(ring + ((ring_row0 + rl) * kvh + h) * d + dv * 8, x[k]);
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int t = t0 + 64 * k + lane;
      if (t < tasks) {
        const int pi = i0 + t / ndv;
        const int dv = t % ndv;
#pragma unroll
        for (int i = 0; i < 8; ++i) dst[pi * pitch + dv * 8 + i] = x[k][i];
      }
    }
  }
}

// Int4 keys of positions [p0, p0 + m): lane = dim; the <= 9 words holding the
// m tokens of that dim (and their group scale/min) load in one batch.
__device__ __forceinline__ void stage_int4_keys(float* __restrict__ dst, int p0, int m,
                                                const int32_t* __restrict__ bt, int64_t nb,
                                                int bs, int kvh, int h, int d, int g,
                                                const uint32_t* __restrict__ kq,
                                                const float* __restrict__ ks,
                                                const float* __restrict__ km, int lane) {
  constexpr int kMaxWords = 9;  // 64 tokens starting anywhere inside a word
  const int pitch = d + 1;
  const int gpb = bs / g;
  const int wpd = bs / 8;
  const int first = p0 & ~7;
  for (int c = lane; c < d; c += 64) {
    uint32_t w[kMaxWords];
    float sc[kMaxWords], mn[kMaxWords];
#pragma unroll
    for (int k = 0; k < kMaxWords; ++k) {
      // clamped into [p0, p0 + m): every load is valid and unconditional
      const int p = first + 8 * k;
      const int pp = p < p0 ? p0 : (p < p0 + m ? p : p0 + m - 1);
      const int64_t blk = clamp_page(bt, pp, bs, nb);
      const int off = pp % bs;
      const int64_t row = (blk * kvh + h) * static_cast<int64_t>(d) + c;
      w[k] = kq[row * wpd + off / 8];
      sc[k] = ks[row * gpb + off / g];
      mn[k] = km[row * gpb + off / g];
    }
#pragma unroll
    for (int k = 0; k < kMaxWords; ++k) {
      const int p = first + 8 * k;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int pi = p + j - p0;
        if (pi >= 0 && pi < m) dst[pi * pitch + c] = kivi_dequant((w[k] >> (4 * j)) & 0xfu, sc[k], mn[k]);
      }
    }
  }
}

// Int4 values of positions [p0, p0 + m): task = (position, word of 8 dims).
__device__ __forceinline__ void stage_int4_values(float* __restrict__ dst, int p0, int m,
                                                  const int32_t* __restrict__ bt, int64_t nb,
                                                  int bs, int kvh, int h, int d, int g,
                                                  const uint32_t* __restrict__ vq,
                                                  const float* __restrict__ vs,
                                                  const float* __restrict__ vm, int lane) {
  const int ndv = d / 8;
  const int pitch = d + 1;
  const int tasks = m * ndv;
  for (int t0 = 0; t0 < tasks; t0 += 64 * kBatch) {
    uint32_t w[kBatch];
    float sc[kBatch], mn[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int tk = t0 + 64 * k + lane;
      const int t = tk < tasks ? tk : tasks - 1;  // clamped: unconditional load
      const int pi = t / ndv;
      const int dv = t % ndv;
      const int p = p0 + pi;
      const int64_t vrow = (clamp_page(bt, p, bs, nb) * bs + p % bs) * kvh + h;
      w[k] = vq[vrow * ndv + dv];
      sc[k] = vs[vrow * (d / g) + (dv * 8) / g];
      mn[k] = vm[vrow * (d / g) + (dv * 8) / g];
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int t = t0 + 64 * k + lane;
      if (t < tasks) {
        const int pi = t / ndv;
        const int dv = t % ndv;
#pragma unroll
        for (int i = 0; i < 8; ++i)
          dst[pi * pitch + dv * 8 + i] = kivi_dequant((w[k] >> (4 * i)) & 0xfu, sc[k], mn[k]);
      }
    }
  }
}

template <typename TQ, typename TR>
__global__ void __launch_bounds__(64)
kivi_decode_generic_kernel(const TQ* __restrict__ query, int hq, int kvh, int d, float qscale,
                           const int32_t* __restrict__ kq, const float* __restrict__ ks,
                           const float* __restrict__ km, const int32_t* __restrict__ vq,
                           const float* __restrict__ vs, const float* __restrict__ vm, int bs,
                           int g, int64_t nb, const int32_t* __restrict__ block_table,
                           int64_t maxb, const int32_t* __restrict__ seq_meta,
                           const int32_t* __restrict__ work, const TR* __restrict__ ring_k,
                           const TR* __restrict__ ring_v, int ring_len,
                           float* __restrict__ ws_o, float* __restrict__ ws_ml,
                           int skip_kind0, int skip_kind1) {
  const int wi = blockIdx.x;
  const int h = blockIdx.y;
  const int lane = threadIdx.x;
  const int32_t* wk = work + 4 * static_cast<int64_t>(wi);
  // the MFMA kernels own these (kinds 0, 2, 3: int4 ranges; kind 1: tail)
  if ((skip_kind0 && wk[3] != 1) || (skip_kind1 && wk[3] == 1)) return;
  const int b = wk[0];
  const int pb = wk[1];
  const int pe = wk[2];
  // kind 2 / 3: only the even / odd 64-position chunks of [pb, pe)
  const int half = wk[3] >= 2 ? wk[3] - 2 : -1;
  const int32_t* sm = seq_meta + 8 * static_cast<int64_t>(b);
  const int khist = sm[1], vhist = sm[2], row = sm[3], kfirst = sm[4], vfirst = sm[5];
  const int rep = hq / kvh;
  const int dpl = (d + 63) / 64;
  const int pitch = d + 1;
  const int32_t* bt = block_table + static_cast<int64_t>(b) * maxb;
  const uint32_t* kqu = reinterpret_cast<const uint32_t*>(kq);
  const uint32_t* vqu = reinterpret_cast<const uint32_t*>(vq);

  extern __shared__ float lds_f[];
  float* s_rows = lds_f;                 // [64][d + 1]
  float* s_q = s_rows + 64 * pitch;      // [rep][d]
  float* s_p = s_q + rep * d;            // [rep][64]
  for (int i = lane; i < rep * d; i += 64) {
    const int r = i / d;
    const int c = i - r * d;
    s_q[i] = to_f32(query[(static_cast<int64_t>(b) * hq + h * rep + r) * d + c]) * qscale;
  }

  float m[kMaxRep], l[kMaxRep], acc[kMaxRep][kMaxDpl];
#pragma unroll
  for (int r = 0; r < kMaxRep; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.0f;
#pragma unroll
    for (int k = 0; k < kMaxDpl; ++k) acc[r][k] = 0.0f;
  }

  for (int p0 = pb + (half == 1 ? 64 : 0); p0 < pe; p0 += (half >= 0 ? 128 : 64)) {
    const int n = (pe - p0) < 64 ? (pe - p0) : 64;
    {
      const int m = khist - p0 < 0 ? 0 : (khist - p0 < n ? khist - p0 : n);  // int4 keys
      if (m > 0) stage_int4_keys(s_rows, p0, m, bt, nb, bs, kvh, h, d, g, kqu, ks, km, lane);
      if (m < n)
        stage_ring(s_rows, p0, m, n, khist, kvh, h, d, ring_k,
                   static_cast<int64_t>(row) * ring_len, kfirst, ring_len, lane);
    }
    __syncthreads();
    const bool live = lane < n;
    float s[kMaxRep];
#pragma unroll
    for (int r = 0; r < kMaxRep; ++r) s[r] = 0.0f;
    if (live) {
      const float* krow = s_rows + lane * pitch;
      for (int c = 0; c < d; ++c) {
        const float kv = krow[c];
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
    {
      const int m = vhist - p0 < 0 ? 0 : (vhist - p0 < n ? vhist - p0 : n);  // int4 values
      if (m > 0) stage_int4_values(s_rows, p0, m, bt, nb, bs, kvh, h, d, g, vqu, vs, vm, lane);
      if (m < n)
        stage_ring(s_rows, p0, m, n, vhist, kvh, h, d, ring_v,
                   static_cast<int64_t>(row) * ring_len, vfirst, ring_len, lane);
    }
    __syncthreads();
    for (int i = 0; i < n; ++i) {
      const float* vrow = s_rows + i * pitch;
#pragma unroll
      for (int k = 0; k < kMaxDpl; ++k) {
        const int c = lane + 64 * k;
        if (k >= dpl || c >= d) continue;
        const float v = vrow[c];
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
      if (k < dpl && c < d) ws_o[hh * d + c] = acc[r][k];
    }
  }
}

}  // namespace

namespace kvq {

// Log-sum-exp combine of a request's work items: one wave per (request, query
// head), four heads per workgroup.  Lane s holds item s's (m, l) of the current
// chunk of 64 items; the weights 2^(m_s - max) go to every lane through
// readlane, and each lane accumulates columns lane + 64*k of sum_s w_s * o_s.
// The o rows of the first kPre items are loaded before the (m, l) pass, so a
// request with up to kPre items costs one round trip to memory instead of one
// per few items.  Items with m = -inf (no position) carry weight 0 and their o
// never reaches the sum (selected out, so stale bytes cannot turn it NaN).
template <typename TO, int KD>
__global__ void __launch_bounds__(256)
decode_combine_kernel(int hq, int d, const int32_t* __restrict__ seq_meta, int meta_stride,
                      int first_col, const float* __restrict__ ws_o,
                      const float* __restrict__ ws_ml, TO* __restrict__ out) {
  constexpr int kPre = 16;
  const int lane = threadIdx.x & 63;
  const int hh = blockIdx.y * 4 + (threadIdx.x >> 6);
  if (hh >= hq) return;  // whole wave: no workgroup barrier below
  const int b = blockIdx.x;
  const int32_t* sm = seq_meta + static_cast<int64_t>(meta_stride) * b;
  const int fw = sm[first_col];
  const int nw = sm[first_col + 1];
  TO* orow = out + (static_cast<int64_t>(b) * hq + hh) * d;
  if (nw <= 0) {  // no items: the empty sum, as the loops below would leave it
#pragma unroll
    for (int k = 0; k < KD; ++k) {
      const int c = lane + 64 * k;
      if (c < d) orow[c] = from_f32<TO>(0.0f);
    }
    return;
  }
  const int64_t stride = static_cast<int64_t>(hq) * d;
  const float* rows = ws_o + (static_cast<int64_t>(fw) * hq + hh) * d;
  float pre[kPre][KD];
#pragma unroll
  for (int j = 0; j < kPre; ++j)
#pragma unroll
    for (int k = 0; k < KD; ++k) {
      const int c = lane + 64 * k;
      // rows past the request or columns past d are read in bounds (item 0,
      // column 0) and never used
      pre[j][k] = rows[(j < nw ? j * stride : 0) + (c < d ? c : 0)];
    }
  // (m, l) of the first 64 items in one 8-byte load per lane, kept for the
  // weights below: one round trip to memory for the whole combine when the
  // request has at most 64 items
  float m0 = -INFINITY, l0 = 0.0f;
  if (lane < nw) {
    const float2 ml = *reinterpret_cast<const float2*>(
        ws_ml + 2 * (static_cast<int64_t>(fw + lane) * hq + hh));
    m0 = ml.x;
    l0 = ml.y;
  }
  float mx = m0;
  for (int s0 = 64; s0 < nw; s0 += 64) {
    const int s = s0 + lane;
    if (s < nw) mx = fmaxf(mx, ws_ml[2 * (static_cast<int64_t>(fw + s) * hq + hh)]);
  }
  mx = max_wave64(mx);
  float acc[KD];
#pragma unroll
  for (int k = 0; k < KD; ++k) acc[k] = 0.0f;
  float wsum = 0.0f;
  for (int s0 = 0; s0 < nw; s0 += 64) {
    const int s = s0 + lane;
    float wgt = 0.0f;
    if (s < nw) {
      float ms = m0, ls = l0;
      if (s0 > 0) {
        const int64_t idx = static_cast<int64_t>(fw + s) * hq + hh;
        ms = ws_ml[2 * idx];
        ls = ws_ml[2 * idx + 1];
      }
      if (ms != -INFINITY) {
        wgt = exp2f(ms - mx);
        wsum += wgt * ls;
      }
    }
    const int cnt = nw - s0 < 64 ? nw - s0 : 64;
    int j0 = 0;
    if (s0 == 0) {
#pragma unroll
      for (int j = 0; j < kPre; ++j) {
        const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wgt), j));
#pragma unroll
        for (int k = 0; k < KD; ++k) acc[k] += wj != 0.0f ? wj * pre[j][k] : 0.0f;
      }
      j0 = kPre;
    }
    const float* row0 = rows + s0 * stride;
#pragma unroll 4
    for (int j = j0; j < cnt; ++j) {
      const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wgt), j));
      const float* row = row0 + j * stride;
#pragma unroll
      for (int k = 0; k < KD; ++k) {
        const int c = lane + 64 * k;
        const float x = row[c < d ? c : 0];  // columns past d are read in bounds, unused
        acc[k] += wj != 0.0f ? wj * x : 0.0f;
      }
    }
  }
  wsum = sum_wave64(wsum);
  const float inv = wsum > 0.0f ? 1.0f / wsum : 0.0f;
#pragma unroll
  for (int k = 0; k < KD; ++k) {
    const int c = lane + 64 * k;
    if (c < d) orow[c] = from_f32<TO>(acc[k] * inv);
  }
}

int launch_decode_combine(int dtype, int64_t batch, int hq, int d, const int32_t* seq_meta,
                          int meta_stride, int first_col, const float* ws_o,
                          const float* ws_ml, void* out, hipStream_t s) {
  if (d <= 0 || d > 256) return KVQ_ERR_GEOMETRY;
  const dim3 grid(static_cast<unsigned>(batch), (hq + 3) / 4);
  const int kd = (d + 63) / 64;
#define KVQ_LAUNCH_COMBINE(KD)                                                              \
  KVQ_DISPATCH_FLOAT(dtype, TO,                                                             \
    hipLaunchKernelGGL((decode_combine_kernel<TO, KD>), grid, dim3(256), 0, s, hq, d,       \
                       seq_meta, meta_stride, first_col, ws_o, ws_ml, static_cast<TO*>(out)))
  switch (kd) {
    case 1: KVQ_LAUNCH_COMBINE(1); break;
    case 2: KVQ_LAUNCH_COMBINE(2); break;
    case 3: KVQ_LAUNCH_COMBINE(3); break;
    default: KVQ_LAUNCH_COMBINE(4); break;
  }
#undef KVQ_LAUNCH_COMBINE
  KVQ_LAUNCH_CHECK();
  return KVQ_OK;
}

}  // namespace kvq

extern "C" int64_t kvq_kivi_decode_workspace_bytes(int64_t num_work, int num_heads,
                                                   int head_size) {
  return kvq::decode_workspace_bytes(num_work, num_heads, head_size);
}

extern "C" int kvq_kivi_decode_attn(const void* query, int q_dtype, int64_t batch, int num_heads,
                                    int num_kv_heads, int head_size, float scale,
                                    const int32_t* k_quant, const float* k_scale,
                                    const float* k_mn, const int32_t* v_quant,
                                    const float* v_scale, const float* v_mn, int64_t num_blocks,
                                    int block_size, int group_size, const int32_t* block_table,
                                    int64_t max_blocks, const int32_t* seq_meta,
                                    const int32_t* work, int64_t num_work,
                                    const int32_t* pieces, int64_t num_pieces, const void* ring_k,
                                    const void* ring_v, int ring_dtype, int ring_len,
                                    void* workspace, void* out, void* stream) {
  if (batch == 0) return KVQ_OK;
  if (!query || !k_quant || !k_scale || !k_mn || !v_quant || !v_scale || !v_mn ||
      !block_table || !seq_meta || !work || !workspace || !out || batch < 0 || num_work <= 0 ||
      num_blocks <= 0 || ring_len <= 0 || !ring_k || !ring_v)
    return KVQ_ERR_INVALID;
  if (num_kv_heads <= 0 || num_heads % num_kv_heads || group_size <= 0 || group_size % 8 ||
      head_size % 8 || head_size % group_size || block_size % group_size || head_size > 256)
    return KVQ_ERR_GEOMETRY;
  if (num_heads / num_kv_heads > kMaxRep) return KVQ_ERR_GEOMETRY;
  if (num_work > 0x7fffffff || batch > 0x7fffffff || num_heads > 65535) return KVQ_ERR_INVALID;
  if (num_pieces < 0 || num_pieces > num_work) return KVQ_ERR_INVALID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* ws_o = static_cast<float*>(workspace);
  float* ws_ml = ws_o + num_work * num_heads * head_size;
  const float qscale = scale * 1.4426950408889634f;  // fold log2(e): exp2 in the kernels

  // int4 items (kind 0), and the tail items (kind 1) in a second pass of the
  // same grid where the tail path applies
  bool mfma = false, tail = false;
  int rc = kvq::launch_kivi_decode_mfma(query, q_dtype, num_heads, num_kv_heads, head_size,
                                       qscale, k_quant, k_scale, k_mn, v_quant, v_scale, v_mn,
                                       block_size, group_size, num_blocks, block_table,
                                       max_blocks, seq_meta, work, num_work, pieces,
                                       num_pieces, ring_k, ring_v, ring_dtype, ring_len, ws_o,
                                       ws_ml, s, &mfma, &tail);
  if (rc != KVQ_OK) return rc;
  if (!tail) {
    rc = kvq::launch_kivi_decode_tail_mfma(query, q_dtype, num_heads, num_kv_heads, head_size,
                                           qscale, k_quant, k_scale, k_mn, v_quant, v_scale,
                                           v_mn, block_size, group_size, num_blocks,
                                           block_table, max_blocks, seq_meta, work, num_work,
                                           ring_k, ring_v, ring_dtype, ring_len, ws_o, ws_ml, s,
                                           &tail);
    if (rc != KVQ_OK) return rc;
  }
  if (!mfma || !tail) {
    const dim3 grid(static_cast<unsigned>(num_work), num_kv_heads);
    const int rep = num_heads / num_kv_heads;
    const size_t lds = sizeof(float) * (64 * (head_size + 1) + rep * head_size + rep * 64);
    KVQ_DISPATCH_FLOAT(q_dtype, TQ,
      KVQ_DISPATCH_FLOAT(ring_dtype, TR,
        hipLaunchKernelGGL((kivi_decode_generic_kernel<TQ, TR>), grid, dim3(64), lds, s,
                           static_cast<const TQ*>(query), num_heads, num_kv_heads, head_size,
                           qscale, k_quant, k_scale, k_mn, v_quant, v_scale, v_mn, block_size,
                           group_size, num_blocks, block_table, max_blocks, seq_meta, work,
                           static_cast<const TR*>(ring_k), static_cast<const TR*>(ring_v),
                           ring_len, ws_o, ws_ml, mfma ? 1 : 0, tail ? 1 : 0)));
    KVQ_LAUNCH_CHECK();
  }
  return kvq::launch_decode_combine(q_dtype, batch, num_heads, head_size, seq_meta, 8, 6, ws_o,
                                    ws_ml, out, s);
}

// ---- allocation-free decode --------------------------------------------------
// kvq_kivi_decode_attn_noalloc keeps its split-K partials in a file-scope
// device array instead of a caller workspace.  Each device holds its own copy
// at its own address from module load until the process ends.  Host code must
// never pass `scratch` itself to a kernel (its host-side name is a stand-in,
// not a device address): it uses the address hipGetSymbolAddress returns,
// resolved once per device with that device current.

namespace {

__device__ __align__(256) float scratch[KVQ_DECODE_SCRATCH_BYTES / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// This device's address of `scratch` (the calling thread's current device).
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return KVQ_ERR_INVALID;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return static_cast<int>(e);
    if (!p) return KVQ_ERR_INVALID;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return KVQ_OK;
}

}  // namespace

extern "C" int kvq_kivi_decode_attn_noalloc(
    const void* query, int q_dtype, int64_t batch, int num_heads, int num_kv_heads,
    int head_size, float scale, const int32_t* k_quant, const float* k_scale, const float* k_mn,
    const int32_t* v_quant, const float* v_scale, const float* v_mn, int64_t num_blocks,
    int block_size, int group_size, const int32_t* block_table, int64_t max_blocks,
    const int32_t* seq_meta, const int32_t* work, int64_t num_work, const int32_t* pieces,
    int64_t num_pieces, const void* ring_k, const void* ring_v, int ring_dtype, int ring_len,
    void* out, void* stream) {
  if (batch == 0) return KVQ_OK;
  if (num_work <= 0 || num_heads <= 0 || head_size <= 0) return KVQ_ERR_INVALID;
  // every partial (m, l, o) of the work list must fit the static array
  if (num_work > KVQ_DECODE_SCRATCH_BYTES ||
      kvq::decode_workspace_bytes(num_work, num_heads, head_size) > KVQ_DECODE_SCRATCH_BYTES)
    return KVQ_ERR_SCRATCH;
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != KVQ_OK) return rc;
  return kvq_kivi_decode_attn(query, q_dtype, batch, num_heads, num_kv_heads, head_size, scale,
                              k_quant, k_scale, k_mn, v_quant, v_scale, v_mn, num_blocks,
                              block_size, group_size, block_table, max_blocks, seq_meta, work,
                              num_work, pieces, num_pieces, ring_k, ring_v, ring_dtype, ring_len,
                              ws, out, stream);
}
