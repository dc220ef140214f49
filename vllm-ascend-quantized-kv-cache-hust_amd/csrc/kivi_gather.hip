// SPDX-License-Identifier: Apache-2.0
// KIVI INT4 paged gather-dequant to dense TND, with the residual-tail overlay
// fused in (reference: pkg/ops/kivi_gather.py:36-156 and the overlay loop of
// pkg/methods/kivi_int4/attention_backend.py:889-935).
//
// One workgroup per (request, page, kv head); pages past the request's
// length exit at once.  The op is store-bound: 0.56 B of int4 + scales in,
// 2 B of bf16 out per element.
//
// Keys: the page's words ([D][Bs/8], one word = 8 tokens of one dim) are
// staged in LDS transposed to [Bs/8][D] so that thread (chunk, dim8) reads its
// 8 words with two 16-byte LDS reads and emits 8 token rows of 8 dims as
// 16-byte stores; lanes with consecutive dim8 cover a head row contiguously.
// Values: one thread per packed word (8 dims of one token) -> one 16-byte
// store.  Rows in the request's residual tail are copied from the ring.
#include "kvq_common.h"

namespace {

using namespace kvq;

template <typename R>
__device__ __forceinline__ void load_ring8(const R* p, float (&x)[8]) {
  load8(p, x);
}

template <typename TO, typename TR, typename TB>
__global__ void __launch_bounds__(256)
kivi_gather_kernel(const int32_t* __restrict__ kq, const float* __restrict__ ks,
                   const float* __restrict__ km, const int32_t* __restrict__ vq,
                   const float* __restrict__ vs, const float* __restrict__ vm, int bs, int kvh,
                   int d, int g, const TB* __restrict__ block_table, int64_t maxb,
                   const int64_t* __restrict__ cu, const int32_t* __restrict__ ring_meta,
                   const TR* __restrict__ ring_k, const TR* __restrict__ ring_v, int ring_len,
                   TO* __restrict__ out_k, TO* __restrict__ out_v) {
  const int j = blockIdx.x;
  const int b = blockIdx.y;
  const int h = blockIdx.z;
  const int64_t row0 = cu[b];
  const int64_t len = cu[b + 1] - row0;
  const int64_t p0 = static_cast<int64_t>(j) * bs;
  if (p0 >= len) return;
  int64_t blk = static_cast<int64_t>(block_table[static_cast<int64_t>(b) * maxb + j]);
  if (blk < 0) blk = 0;

  int ring_row = 0, k_first = 0, k_tail = 0, v_first = 0, v_tail = 0;
  if (ring_meta != nullptr) {
    const int32_t* m = ring_meta + 5 * b;
    ring_row = m[0];
    k_first = m[1];
    k_tail = m[2];
    v_first = m[3];
    v_tail = m[4];
  }
  const int64_t k_tail_start = len - k_tail;
  const int64_t v_tail_start = len - v_tail;
  const int64_t hd = static_cast<int64_t>(kvh) * d;

  extern __shared__ uint32_t lds[];
  const int nchunk = bs / 8;
  const int pitch = d + 4;  // padded row of the transposed word tile
  uint32_t* s_words = lds;                                            // [nchunk][pitch]
  float* s_scale = reinterpret_cast<float*>(s_words + nchunk * pitch);  // [d][bs/g]
  float* s_min = s_scale + d * (bs / g);

  const int tid = threadIdx.x;
  const int nthreads = blockDim.x;

  // ---- keys -------------------------------------------------------------
  const int64_t kbase = (blk * kvh + h) * static_cast<int64_t>(d);
  {
    const uint32_t* src = reinterpret_cast<const uint32_t*>(kq) + kbase * nchunk;
    for (int i = tid; i < d * nchunk; i += nthreads) {
      const int c = i / nchunk;
      const int w = i - c * nchunk;
      s_words[w * pitch + c] = src[i];
    }
    const int spb = d * (bs / g);
    for (int i = tid; i < spb; i += nthreads) {
      s_scale[i] = ks[kbase * (bs / g) + i];
      s_min[i] = km[kbase * (bs / g) + i];
    }
  }
  __syncthreads();
  {
    const int ndv = d / 8;
    for (int tile = tid; tile < nchunk * ndv; tile += nthreads) {
      const int dv = tile % ndv;
      const int tc = tile / ndv;
      uint32_t w[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) w[i] = s_words[tc * pitch + dv * 8 + i];
      const int grp = (tc * 8) / g;
      float sc[8], mn[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        sc[i] = s_scale[(dv * 8 + i) * (bs / g) + grp];
        mn[i] = s_min[(dv * 8 + i) * (bs / g) + grp];
      }
#pragma unroll
      for (int l = 0; l < 8; ++l) {
        const int64_t p = p0 + tc * 8 + l;
        if (p >= len) break;
        float x[8];
        if (p >= k_tail_start) {
          const int lane = static_cast<int>((k_first + (p - k_tail_start)) % ring_len);
          load_ring8(ring_k + ((static_cast<int64_t>(ring_row) * ring_len + lane) * kvh + h) * d +
                         dv * 8,
                     x);
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) x[i] = kivi_dequant((w[i] >> (4 * l)) & 0xfu, sc[i], mn[i]);
        }
        store8_nt(out_k + (row0 + p) * hd + h * d + dv * 8, x);
      }
    }
  }

  // ---- values -----------------------------------------------------------
  {
    const int words = d / 8;
    const int ng = d / g;
    const int64_t rows = (len - p0) < bs ? (len - p0) : bs;
    const uint32_t* src = reinterpret_cast<const uint32_t*>(vq);
    for (int i = tid; i < rows * words; i += nthreads) {
      const int off = i / words;
      const int w = i - off * words;
      const int64_t p = p0 + off;
      float x[8];
      if (p >= v_tail_start) {
        const int lane = static_cast<int>((v_first + (p - v_tail_start)) % ring_len);
        load_ring8(ring_v + ((static_cast<int64_t>(ring_row) * ring_len + lane) * kvh + h) * d +
                       w * 8,
                   x);
      } else {
        const int64_t vrow = (blk * bs + off) * kvh + h;
        const uint32_t word = src[vrow * words + w];
        const int gi = (w * 8) / g;
        const float sc = vs[vrow * ng + gi];
        const float mn = vm[vrow * ng + gi];
        nibbles_f32(word, x);
#pragma unroll
        for (int l = 0; l < 8; ++l) x[l] = __fadd_rn(__fmul_rn(x[l], sc), mn);
      }
      store8_nt(out_v + (row0 + p) * hd + h * d + w * 8, x);
    }
  }
}

// Head size 128, G in {64, 128}, block size a multiple of 32 up to 128:
// every global load of a (page, head) goes out first -- the key words 16
// bytes a lane, the value words, scales and minima one per lane -- so the
// page's 18 KB are in flight together instead of in dependent phases; then
// the key words go through LDS transposed and both sides are dequantized and
// stored.  Every store instruction writes whole 256-byte head rows (16 lanes
// of 16 bytes): nontemporal stores that cover a line only in part run far
// slower.
template <typename TO, typename TR, typename TB, int G>
__global__ void __launch_bounds__(256)
kivi_gather_d128_kernel(const int32_t* __restrict__ kq, const float* __restrict__ ks,
                        const float* __restrict__ km, const int32_t* __restrict__ vq,
                        const float* __restrict__ vs, const float* __restrict__ vm, int bs,
                        int kvh, const TB* __restrict__ block_table, int64_t maxb,
                        int64_t npages, const int64_t* __restrict__ cu,
                        const int32_t* __restrict__ ring_meta,
                        const TR* __restrict__ ring_k, const TR* __restrict__ ring_v,
                        int ring_len, TO* __restrict__ out_k, TO* __restrict__ out_v) {
  constexpr int D = 128;
  constexpr int WPR = D / 8;  // words per value row
  // 1-D grid: workgroup ids go to the 8 XCDs in turn; the kv heads of one
  // page take ids 8 apart, so they run on one XCD close together (they share
  // the page's value rows and write whole token rows between them)
  const int xcd = static_cast<int>(blockIdx.x % 8);
  const int64_t sidx = blockIdx.x / 8;
  const int h = static_cast<int>(sidx % kvh);
  const int64_t pg = (sidx / kvh) * 8 + xcd;  // page index b * maxb + j
  if (pg >= npages) return;
  const int b = static_cast<int>(pg / maxb);
  const int j = static_cast<int>(pg - static_cast<int64_t>(b) * maxb);
  const int64_t row0 = cu[b];
  const int64_t len = cu[b + 1] - row0;
  const int64_t p0 = static_cast<int64_t>(j) * bs;
  if (p0 >= len) return;
  int64_t blk = static_cast<int64_t>(block_table[static_cast<int64_t>(b) * maxb + j]);
  if (blk < 0) blk = 0;

  int ring_row = 0, k_first = 0, k_tail = 0, v_first = 0, v_tail = 0;
  if (ring_meta != nullptr) {
    const int32_t* m = ring_meta + 5 * b;
    ring_row = m[0];
    k_first = m[1];
    k_tail = m[2];
    v_first = m[3];
    v_tail = m[4];
  }
  const int64_t k_tail_start = len - k_tail;
  const int64_t v_tail_start = len - v_tail;
  const int64_t hd = static_cast<int64_t>(kvh) * D;

  extern __shared__ uint32_t lds[];
  const int nchunk = bs / 8;
  const int pitch = D + 4;  // padded row of the transposed word tile
  uint32_t* s_words = lds;                                              // [nchunk][pitch]
  float* s_scale = reinterpret_cast<float*>(s_words + nchunk * pitch);  // [D][bs/G]
  float* s_min = s_scale + D * (bs / G);
  const int tid = threadIdx.x;

  // ---- every global load first ------------------------------------------
  const int64_t kbase = (blk * kvh + h) * static_cast<int64_t>(D);
  const int kquads = D * nchunk / 4;  // 16-byte runs of the page's key words
  const int spb = D * (bs / G);       // key scales of the page and head
  const int rows = static_cast<int>((len - p0) < bs ? (len - p0) : bs);
  const int vitems = rows * WPR;  // (row, word) pairs
  const uint4* ksrc = reinterpret_cast<const uint4*>(kq + kbase * nchunk);
  uint4 kw[2];
  float ksc = 0.0f, kmn = 0.0f;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int i = tid + 256 * k;
    if (i < kquads) kw[k] = ksrc[i];
  }
  if (tid < spb) {
    ksc = ks[kbase * (bs / G) + tid];
    kmn = km[kbase * (bs / G) + tid];
  }
  // value item i = tid + 256 k: row i / 16, word i % 16 (bs * 16 <= 2048 items)
  uint32_t vw[8];
  float vsc[8], vmn[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int i = tid + 256 * k;
    vw[k] = 0;
    vsc[k] = vmn[k] = 0.0f;
    if (i < vitems) {
      const int r = i / WPR;
      const int w = i - r * WPR;
      const int64_t vrow = (blk * bs + r) * kvh + h;
      vw[k] = reinterpret_cast<const uint32_t*>(vq)[vrow * WPR + w];
      vsc[k] = vs[vrow * (D / G) + (w * 8) / G];
      vmn[k] = vm[vrow * (D / G) + (w * 8) / G];
    }
  }

  // ---- values -------------------------------------------------------------
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int i = tid + 256 * k;
    if (i < vitems) {
      const int r = i / WPR;
      const int w = i - r * WPR;
      const int64_t p = p0 + r;
      float x[8];
      if (p >= v_tail_start) {
        const int lane = static_cast<int>((v_first + (p - v_tail_start)) % ring_len);
        load_ring8(ring_v + ((static_cast<int64_t>(ring_row) * ring_len + lane) * kvh + h) * D +
                       w * 8,
                   x);
      } else {
        nibbles_f32(vw[k], x);
#pragma unroll
        for (int l = 0; l < 8; ++l) x[l] = __fadd_rn(__fmul_rn(x[l], vsc[k]), vmn[k]);
      }
      store8_nt(out_v + (row0 + p) * hd + h * D + w * 8, x);
    }
  }

  // ---- keys: words to LDS transposed ([chunk][dim]), then dequantize ----
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int i = tid + 256 * k;
    if (i < kquads) {
      const uint32_t w4[4] = {kw[k].x, kw[k].y, kw[k].z, kw[k].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int n = 4 * i + e;  // word n: dim n / nchunk, chunk n % nchunk
        const int c = n / nchunk;
        s_words[(n - c * nchunk) * pitch + c] = w4[e];
      }
    }
  }
  if (tid < spb) {
    s_scale[tid] = ksc;
    s_min[tid] = kmn;
  }
  __syncthreads();
  {
    constexpr int ndv = D / 8;
    const int tile = tid;
    if (tile < nchunk * ndv) {
      const int dv = tile % ndv;
      const int tc = tile / ndv;
      uint32_t w[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) w[i] = s_words[tc * pitch + dv * 8 + i];
      const int grp = (tc * 8) / G;
      float sc[8], mn[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        sc[i] = s_scale[(dv * 8 + i) * (bs / G) + grp];
        mn[i] = s_min[(dv * 8 + i) * (bs / G) + grp];
      }
#pragma unroll
      for (int l = 0; l < 8; ++l) {
        const int64_t p = p0 + tc * 8 + l;
        if (p >= len) break;
        float x[8];
        if (p >= k_tail_start) {
          const int lane = static_cast<int>((k_first + (p - k_tail_start)) % ring_len);
          load_ring8(ring_k + ((static_cast<int64_t>(ring_row) * ring_len + lane) * kvh + h) * D +
                         dv * 8,
                     x);
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) x[i] = kivi_dequant((w[i] >> (4 * l)) & 0xfu, sc[i], mn[i]);
        }
        store8_nt(out_k + (row0 + p) * hd + h * D + dv * 8, x);
      }
    }
  }
}

}  // namespace

extern "C" int kvq_kivi_gather_dequant(const int32_t* k_quant, const float* k_scale,
                                       const float* k_mn, const int32_t* v_quant,
                                       const float* v_scale, const float* v_mn,
                                       int64_t num_blocks, int block_size, int num_kv_heads,
                                       int head_size, int group_size, const void* block_table,
                                       int block_index_type, int64_t max_blocks,
                                       const int64_t* cu_seqlens, int64_t batch,
                                       const int32_t* ring_meta, const void* ring_k,
                                       const void* ring_v, int ring_dtype, int ring_len,
                                       void* out_k, void* out_v, int out_dtype, void* stream) {
  if (batch == 0 || max_blocks == 0) return KVQ_OK;
  if (!k_quant || !k_scale || !k_mn || !v_quant || !v_scale || !v_mn || !block_table ||
      !cu_seqlens || !out_k || !out_v || batch < 0 || max_blocks < 0 || num_blocks <= 0)
    return KVQ_ERR_INVALID;
  if (group_size <= 0 || group_size % 8 || head_size % 8 || head_size % group_size ||
      block_size % group_size || num_kv_heads <= 0)
    return KVQ_ERR_GEOMETRY;
  if (ring_meta && (!ring_k || !ring_v || ring_len <= 0)) return KVQ_ERR_INVALID;
  if (batch > 65535 || num_kv_heads > 65535 || max_blocks > 0x7fffffff) return KVQ_ERR_INVALID;
  const size_t lds = sizeof(uint32_t) * (block_size / 8) * (head_size + 4) +
                     2 * sizeof(float) * head_size * (block_size / group_size);
  if (lds > 160 * 1024) return KVQ_ERR_GEOMETRY;
  const dim3 grid(static_cast<unsigned>(max_blocks), static_cast<unsigned>(batch),
                  num_kv_heads);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int rdt = ring_meta ? ring_dtype : out_dtype;
  if (head_size == 128 && (group_size == 64 || group_size == 128) && block_size % 32 == 0 &&
      block_size <= 128) {
    const int64_t npages = batch * max_blocks;
    const int64_t grid1 = (npages + 7) / 8 * 8 * num_kv_heads;
    if (grid1 > 0x7fffffff) return KVQ_ERR_INVALID;
#define KVQ_LAUNCH_GATHER_D128(GG)                                                            \
    KVQ_DISPATCH_FLOAT(out_dtype, TO,                                                       \
      KVQ_DISPATCH_FLOAT(rdt, TR,                                                           \
        KVQ_DISPATCH_INDEX(block_index_type, TB,                                            \
          hipLaunchKernelGGL((kivi_gather_d128_kernel<TO, TR, TB, GG>), dim3(static_cast<unsigned>(grid1)), dim3(256), \
                             lds, s, k_quant, k_scale, k_mn, v_quant, v_scale, v_mn,         \
                             block_size, num_kv_heads, static_cast<const TB*>(block_table),  \
                             max_blocks, npages, cu_seqlens, ring_meta,                      \
                             static_cast<const TR*>(ring_k),                                 \
                             static_cast<const TR*>(ring_v), ring_len > 0 ? ring_len : 1,    \
                             static_cast<TO*>(out_k), static_cast<TO*>(out_v)))))
    if (group_size == 128) {
      KVQ_LAUNCH_GATHER_D128(128);
    } else {
      KVQ_LAUNCH_GATHER_D128(64);
    }
#undef KVQ_LAUNCH_GATHER_D128
    KVQ_LAUNCH_CHECK();
    return KVQ_OK;
  }
  KVQ_DISPATCH_FLOAT(out_dtype, TO,
    KVQ_DISPATCH_FLOAT(rdt, TR,
      KVQ_DISPATCH_INDEX(block_index_type, TB,
        hipLaunchKernelGGL((kivi_gather_kernel<TO, TR, TB>), grid, dim3(256), lds, s, k_quant,
                           k_scale, k_mn, v_quant, v_scale, v_mn, block_size, num_kv_heads,
                           head_size, group_size, static_cast<const TB*>(block_table),
                           max_blocks, cu_seqlens, ring_meta, static_cast<const TR*>(ring_k),
                           static_cast<const TR*>(ring_v), ring_len > 0 ? ring_len : 1,
                           static_cast<TO*>(out_k), static_cast<TO*>(out_v)))));
  KVQ_LAUNCH_CHECK();
  return KVQ_OK;
}
