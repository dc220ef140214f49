// SPDX-License-Identifier: Apache-2.0
// KIVI INT4 pack kernels for MI355X (gfx950).
//
// Head size 128 with G in {64, 128} and 16-bit input, both per-side entry
// points (kvq_kivi_pack_key / kvq_kivi_pack_value) run on the one-launch
// store's LDS-staged kernel (below) with the other side empty.  The forms
// described next serve the other geometries, and inputs past that kernel's
// int32 source-row range.
//
// Key pack  (reference: pkg/ops/triton/kivi_pack.py:134-226)
//   Head size 128 with G in {64, 128} and 16-bit input: the register form
//   below (kivi_pack_key_wave_kernel), one wave per group, head and quarter
//   (G = 128) or half (G = 64) of the dims.  Other geometries: one workgroup per (token group, kv head).
//   Thread (tc, dv) owns an 8x8
//   tile: 8 consecutive tokens x 8 consecutive dims, read as 8 16-byte rows
//   (16 lanes cover one 256-byte head row, fully coalesced).  Per-dim min/max
//   over the group's tokens go through LDS; each thread then quantizes its
//   tile into 8 words (8 tokens of one dim per word) which are staged in LDS
//   as [dim][chunk] and written back in address order.
//
// Value pack (reference: pkg/ops/triton/kivi_pack.py:61-131)
//   One lane per output word (8 consecutive dims of one token-head row, a
//   16-byte load); waves walk units of 64 lanes, four at a time with the next
//   four in flight.  The head-dim group's min/max is a butterfly over the
//   group's G/8 adjacent lanes (DPP quad permutes and ds_swizzle).  Head sizes
//   whose rows do not tile a wave keep the one-thread-per-word kernel.
//
// One-launch store (kvq_kivi_store, the mixin's store batches: both packs and
// the ring-row writes of a step or a chunk)
//   kivi_pack_lds_kernel: 8 KB units staged by LDS DMA, each lane holding one
//   quantization group's 64 values after the read-back, two units in flight
//   per wave (layout notes at the kernel).  Packing a prefill chunk's keys and
//   values this way takes one launch.
//
// All quantize with kivi_pack_word: a reciprocal per group, a floor per
// element, and two fmas that decide exactly, with no division and no branch,
// whether the reference's rounded quotient reaches the next code.
#include <mutex>

#include "kvq_common.h"

namespace {

using namespace kvq;

template <typename T>
__device__ __forceinline__ const T* src_row(const T* a, int64_t n_a, const T* b, int64_t row,
                                             int64_t row_elems) {
  return row < n_a ? a + row * row_elems : b + (row - n_a) * row_elems;
}

template <typename T, typename I>
__global__ void __launch_bounds__(1024)
kivi_pack_key_kernel(const T* __restrict__ src_a, int64_t n_a, const T* __restrict__ src_b,
                     const int64_t* __restrict__ src_index, const I* __restrict__ slots,
                     int kvh, int d, int g, int bs, int32_t* __restrict__ kq,
                     float* __restrict__ ks, float* __restrict__ km) {
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * g;
  const int h = blockIdx.y;
  const int64_t first = ld_index(slots, t0);
  if (first < 0) return;  // uniform across the workgroup
  const int64_t blk = first / bs;
  const int off = static_cast<int>(first - blk * bs);
  const int nchunk = g / 8;
  const int ndv = d / 8;
  const int tiles = nchunk * ndv;

  extern __shared__ float smem[];
  float* s_mn = smem;                   // [nchunk][d]
  float* s_mx = s_mn + nchunk * d;      // [nchunk][d]
  float* s_scale = s_mx + nchunk * d;   // [d]
  float* s_min = s_scale + d;           // [d]
  uint32_t* s_words = reinterpret_cast<uint32_t*>(s_min + d);  // [d][nchunk]

  const int tid = threadIdx.x;
  const bool active = tid < tiles;
  const int dv = active ? tid % ndv : 0;
  const int tc = active ? tid / ndv : 0;
  const int64_t row_elems = static_cast<int64_t>(kvh) * d;

  float x[8][8];
  if (active) {
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      const int64_t t = t0 + tc * 8 + l;
      const int64_t row = src_index ? src_index[t] : t;
      load8(src_row(src_a, n_a, src_b, row, row_elems) + h * d + dv * 8, x[l]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float mn = x[0][j], mx = x[0][j];
#pragma unroll
      for (int l = 1; l < 8; ++l) {
        mn = fmin_ordered(mn, x[l][j]);
        mx = fmax_ordered(mx, x[l][j]);
      }
      s_mn[tc * d + dv * 8 + j] = mn;
      s_mx[tc * d + dv * 8 + j] = mx;
    }
  }
  __syncthreads();

  const int64_t row_base = (blk * kvh + h) * static_cast<int64_t>(d);
  const int groups_per_block = bs / g;
  for (int c = tid; c < d; c += blockDim.x) {
    float mn = s_mn[c], mx = s_mx[c];
    for (int k = 1; k < nchunk; ++k) {
      mn = fmin_ordered(mn, s_mn[k * d + c]);
      mx = fmax_ordered(mx, s_mx[k * d + c]);
    }
    const float sc = kivi_group_scale(mn, mx);
    s_scale[c] = sc;
    s_min[c] = mn;
    const int64_t sidx = (row_base + c) * groups_per_block + off / g;
    ks[sidx] = sc;
    km[sidx] = mn;
  }
  __syncthreads();

  if (active) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = dv * 8 + j;
      float col[8];
#pragma unroll
      for (int l = 0; l < 8; ++l) col[l] = x[l][j];
      s_words[c * nchunk + tc] = kivi_pack_word(col, s_min[c], s_scale[c]);
    }
  }
  __syncthreads();

  const int words_per_dim = bs / 8;
  const int total_words = d * nchunk;
  uint32_t* out = reinterpret_cast<uint32_t*>(kq);
  for (int i = tid; i < total_words; i += blockDim.x) {
    const int c = i / nchunk;
    const int w = i - c * nchunk;
    out[(row_base + c) * words_per_dim + off / 8 + w] = s_words[i];
  }
}

// Key pack, register form (head size 128, G in {64, 128}, 16-bit input): one
// wave per (token group, kv head, part of the head dims).  Lane (tg, dl) holds
// consecutive tokens (token group tg) x 8 consecutive dims (dl) as raw 16-byte
// rows -- each load instruction reads whole 64- or 128-byte row parts -- so
// the per-dim min/max is a register pass plus a butterfly over tg, and every
// output word (8 consecutive tokens of one dim) is built from one lane's own
// registers.  No LDS, no barrier; the wave's share of the group stays in
// registers.  Quarters at G = 128 give each lane 8 rows instead of 16: twice
// the waves, so a SIMD's waves reach their arithmetic at staggered times
// instead of all waiting on 16 loads.
template <typename T>
__device__ __forceinline__ void unpack8(const uint4& v, float (&x)[8]);
template <>
__device__ __forceinline__ void unpack8<bf16>(const uint4& v, float (&x)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = __uint_as_float(w[i] << 16);
    x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
template <>
__device__ __forceinline__ void unpack8<f16>(const uint4& v, float (&x)[8]) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  const h8 h = __builtin_bit_cast(h8, v);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = static_cast<float>(h[i]);
}

// Unit u = ((group * kvh) + head) * P + part, P = 16 / DL parts of 8 * DL dims
// each; the whole wave calls it.  Lane (tg, dl) holds 8 dims of G * DL / 64
// tokens: DL = 8 gives halves of the head (16 rows per lane at G = 128), DL = 4
// quarters (8 rows per lane), twice the waves with half the loads each.
template <typename T, typename I, int G, int DL = 8>
__device__ __forceinline__ void key_pack_wave(const T* src_a, int64_t n_a, const T* src_b,
                                              const int64_t* __restrict__ src_index,
                                              const I* __restrict__ slots, int64_t u, int lane,
                                              int kvh, int bs, int32_t* __restrict__ kq,
                                              float* __restrict__ ks, float* __restrict__ km) {
  constexpr int D = 128;
  constexpr int P = 16 / DL;
  constexpr int TPL = G * DL / 64;  // tokens per lane
  static_assert((DL == 4 || DL == 8) && TPL % 8 == 0, "whole words per lane");
  const int part = static_cast<int>(u % P);
  const int h = static_cast<int>((u / P) % kvh);
  const int64_t t0 = (u / P) / kvh * G;
  const int64_t first = ld_index(slots, t0);
  if (first < 0) return;  // uniform across the wave
  const int64_t blk = first / bs;
  const int off = static_cast<int>(first - blk * bs);
  const int dl = lane % DL;
  const int tg = lane / DL;
  const int64_t row_elems = static_cast<int64_t>(kvh) * D;
  const int col = h * D + part * (8 * DL) + 8 * dl;

  uint4 raw[TPL];
#pragma unroll
  for (int k = 0; k < TPL; ++k) {
    const int64_t t = t0 + TPL * tg + k;
    const int64_t row = src_index ? src_index[t] : t;
    raw[k] = *reinterpret_cast<const uint4*>(src_row(src_a, n_a, src_b, row, row_elems) + col);
  }
  float mn[8], mx[8];
  {
    float x[8];
    unpack8<T>(raw[0], x);
#pragma unroll
    for (int j = 0; j < 8; ++j) mn[j] = mx[j] = x[j];
#pragma unroll
    for (int k = 1; k < TPL; ++k) {
      unpack8<T>(raw[k], x);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        mn[j] = fmin_ordered(mn[j], x[j]);
        mx[j] = fmax_ordered(mx[j], x[j]);
      }
    }
  }
  // the token groups of a dim are lanes dl + DL*tg: combine over tg
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if constexpr (DL == 4) {
      mn[j] = fmin_ordered(mn[j], lane_xor<4>(mn[j]));
      mx[j] = fmax_ordered(mx[j], lane_xor<4>(mx[j]));
    }
    mn[j] = fmin_ordered(mn[j], lane_xor<8>(mn[j]));
    mx[j] = fmax_ordered(mx[j], lane_xor<8>(mx[j]));
    mn[j] = fmin_ordered(mn[j], lane_xor<16>(mn[j]));
    mx[j] = fmax_ordered(mx[j], lane_xor<16>(mx[j]));
    mn[j] = fmin_ordered(mn[j], lane_xor<32>(mn[j]));
    mx[j] = fmax_ordered(mx[j], lane_xor<32>(mx[j]));
  }
  float sc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) sc[j] = kivi_group_scale(mn[j], mx[j]);

  const int64_t row_base = (blk * kvh + h) * static_cast<int64_t>(D) + part * (8 * DL) + 8 * dl;
  const int wpd = bs / 8;
  uint32_t* out = reinterpret_cast<uint32_t*>(kq);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    uint32_t wd[TPL / 8];
#pragma unroll
    for (int c = 0; c < TPL / 8; ++c) {
      float col8[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float x[8];
        unpack8<T>(raw[8 * c + i], x);
        col8[i] = x[j];
      }
      wd[c] = kivi_pack_word(col8, mn[j], sc[j]);
    }
    // streaming (nontemporal) stores: the packed pages are not re-read soon
    uint32_t* dst = out + (row_base + j) * wpd + off / 8 + (TPL / 8) * tg;
    if constexpr (TPL / 8 == 2) {
      typedef uint32_t u2v __attribute__((ext_vector_type(2)));
      __builtin_nontemporal_store(u2v{wd[0], wd[1]}, reinterpret_cast<u2v*>(dst));
    } else {
      __builtin_nontemporal_store(wd[0], dst);
    }
  }
  if (tg == 0) {
    const int gpb = bs / G;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t sidx = (row_base + j) * gpb + off / G;
      ks[sidx] = sc[j];
      km[sidx] = mn[j];
    }
  }
}

template <typename T, typename I, int G, int DL>
__global__ void __launch_bounds__(256)
kivi_pack_key_wave_kernel(const T* __restrict__ src_a, int64_t n_a, const T* __restrict__ src_b,
                          const int64_t* __restrict__ src_index, const I* __restrict__ slots,
                          int64_t units, int kvh, int bs, int32_t* __restrict__ kq,
                          float* __restrict__ ks, float* __restrict__ km) {
  const int64_t u = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (u >= units) return;  // whole wave
  key_pack_wave<T, I, G, DL>(src_a, n_a, src_b, src_index, slots, u, threadIdx.x & 63, kvh, bs,
                             kq, ks, km);
}

template <typename T, typename I>
__global__ void __launch_bounds__(256)
kivi_pack_value_kernel(const T* __restrict__ src_a, int64_t n_a, const T* __restrict__ src_b,
                       const int64_t* __restrict__ src_index, const I* __restrict__ slots,
                       int64_t num_tokens, int kvh, int d, int g, int bs,
                       int32_t* __restrict__ vq, float* __restrict__ vs,
                       float* __restrict__ vm) {
  const int words = d / 8;
  const int gw = g / 8;  // lanes per head-dim group
  const int64_t total = num_tokens * kvh * words;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const bool valid = gid < total;
  const int64_t r = valid ? gid / words : 0;
  const int w = static_cast<int>(gid - r * words);
  const int64_t t = r / kvh;
  const int h = static_cast<int>(r - t * kvh);
  const int64_t row_elems = static_cast<int64_t>(kvh) * d;
  const int64_t row = valid ? (src_index ? src_index[t] : t) : 0;
  const T* base = src_row(src_a, n_a, src_b, row, row_elems) + h * d;

  float x[8];
  float mn = 0.0f, mx = 0.0f;
  if (valid) {
    load8(base + w * 8, x);
    mn = x[0];
    mx = x[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) {
      mn = fmin_ordered(mn, x[i]);
      mx = fmax_ordered(mx, x[i]);
    }
  }
  if ((gw & (gw - 1)) == 0 && gw <= 64) {
    // groups are gw adjacent, gw-aligned lanes (d % g == 0 keeps rows aligned)
    for (int o = 1; o < gw; o <<= 1) {
      mn = fmin_ordered(mn, __shfl_xor(mn, o, 64));
      mx = fmax_ordered(mx, __shfl_xor(mx, o, 64));
    }
  } else if (valid) {
    // uneven group width: every lane of the group scans the whole group
    const int g0 = (w / gw) * g;
    float y[8];
    load8(base + g0, y);
    mn = y[0];
    mx = y[0];
    for (int k = 0; k < g; k += 8) {
      load8(base + g0 + k, y);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        mn = fmin_ordered(mn, y[i]);
        mx = fmax_ordered(mx, y[i]);
      }
    }
  }
  if (!valid) return;
  const int64_t slot = ld_index(slots, t);
  if (slot < 0) return;
  const float sc = kivi_group_scale(mn, mx);
  const uint32_t word = kivi_pack_word(x, mn, sc);
  const int64_t blk = slot / bs;
  const int64_t off = slot - blk * bs;
  const int64_t orow = (blk * bs + off) * kvh + h;
  reinterpret_cast<uint32_t*>(vq)[orow * words + w] = word;
  if (w % gw == 0) {
    const int64_t sidx = orow * (d / g) + w / gw;
    vs[sidx] = sc;
    vm[sidx] = mn;
  }
}


// Residual ring write: row dst_rows[i] of the ring takes source row
// src_rows[i] (or i), converted to the ring dtype; 8 elements per thread.
template <typename TS, typename TD>
__global__ void __launch_bounds__(256)
ring_write_kernel(const TS* __restrict__ src, const int64_t* __restrict__ src_rows,
                  const int64_t* __restrict__ dst_rows, int64_t n, int row_elems,
                  TD* __restrict__ ring) {
  const int per_row = row_elems / 8;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= n * per_row) return;
  const int64_t i = gid / per_row;
  const int c = static_cast<int>(gid - i * per_row) * 8;
  const int64_t sr = src_rows ? src_rows[i] : i;
  float x[8];
  load8(src + sr * row_elems + c, x);
  store8(ring + dst_rows[i] * row_elems + c, x);
}

// One value word: the lane's 8 dims x (word w of a row of head h, stored at
// page slot `slot`).  The head-dim group's min/max is a butterfly over its gw
// adjacent lanes; every lane of the wave runs it (lanes of rows past the end
// included), then only valid lanes with a slot store.
template <int WPR>
__device__ __forceinline__ void value_pack_word(const float (&x)[8], int w, bool valid,
                                                int64_t slot, int h, int kvh, int gw, int ng,
                                                int32_t* __restrict__ vq, float* __restrict__ vs,
                                                float* __restrict__ vm) {
  float mn = x[0], mx = x[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) {
    mn = fminf(mn, x[i]);
    mx = fmaxf(mx, x[i]);
  }
  // every step runs; steps at or past gw keep the lane's value (a uniform
  // select, no branch)
#define KVQ_GROUP_STEP(O)                                               \
  {                                                                     \
    const float pn = fminf(mn, lane_xor<O>(mn));                        \
    const float px = fmaxf(mx, lane_xor<O>(mx));                        \
    mn = gw > O ? pn : mn;                                              \
    mx = gw > O ? px : mx;                                              \
  }
  if (WPR > 1) KVQ_GROUP_STEP(1)
  if (WPR > 2) KVQ_GROUP_STEP(2)
  if (WPR > 4) KVQ_GROUP_STEP(4)
  if (WPR > 8) KVQ_GROUP_STEP(8)
  if (WPR > 16) KVQ_GROUP_STEP(16)
  if (WPR > 32) KVQ_GROUP_STEP(32)
#undef KVQ_GROUP_STEP
  if (!valid || slot < 0) return;
  const float sc = kivi_group_scale(mn, mx);
  const uint32_t word = kivi_pack_word(x, mn, sc);
  const int64_t orow = slot * kvh + h;  // page row (blk * bs + off) of head h
  __builtin_nontemporal_store(word, reinterpret_cast<uint32_t*>(vq) + orow * WPR + w);
  if (w % gw == 0) {
    const int64_t sidx = orow * ng + w / gw;
    vs[sidx] = sc;
    vm[sidx] = mn;
  }
}

// ---- wave-pipelined value pack ---------------------------------------------
// Waves walk their units with a register double buffer: the next units'
// source rows are in flight while the current ones are reduced, quantized and
// stored, so loads overlap the arithmetic instead of every wave of the chip
// loading, then computing, then storing in lockstep.

// Value pack: the flat (token-head row, word) index space in units of one
// wave (64 lanes = 64 / WPR rows, WPR = head_size / 8 words per row).  Each
// wave takes U consecutive units per step and keeps the next step's U units
// in flight; the head-dim group min/max is a butterfly over its g / 8 adjacent
// lanes.  row -> token goes through a host-built FastDiv (no 64-bit division).
template <typename T, typename I, int WPR>
__global__ void __launch_bounds__(256)
kivi_pack_value_wave_kernel(const T* __restrict__ src_a, int64_t n_a, const T* __restrict__ src_b,
                            const int64_t* __restrict__ src_index, const I* __restrict__ slots,
                            int32_t rows, FastDiv kvh_div, int g, int bs,
                            int32_t* __restrict__ vq, float* __restrict__ vs,
                            float* __restrict__ vm) {
  constexpr int RPU = 64 / WPR;  // rows per unit
  constexpr int U = 4;           // units per step
  constexpr int D = 8 * WPR;
  const int lane = threadIdx.x & 63;
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * (blockDim.x / 64) + (threadIdx.x >> 6);
  const int64_t nw = static_cast<int64_t>(gridDim.x) * (blockDim.x / 64);
  const int kvh = static_cast<int>(kvh_div.d);
  const int gw = g / 8;
  const int ng = D / g;
  const int w = lane % WPR;
  const int64_t row_elems = static_cast<int64_t>(kvh) * D;
  const int64_t units = (static_cast<int64_t>(rows) + RPU - 1) / RPU;

  struct Buf {
    Raw8<T> x[U];
    int64_t slot[U];
  };
  auto load = [&](Buf& b, int64_t u0) {
#pragma unroll
    for (int k = 0; k < U; ++k) {
      int32_t r = static_cast<int32_t>((u0 + k) * RPU) + lane / WPR;
      r = r < rows ? r : rows - 1;  // rows past the end read the last row, store nothing
      const uint32_t t = kvh_div.div(static_cast<uint32_t>(r));
      if (src_index) {
        const int h = r - static_cast<int32_t>(t) * kvh;
        b.x[k].load(src_row(src_a, n_a, src_b, src_index[t], row_elems) + h * D + w * 8);
      } else {
        // rows of src_a are the (token, head) rows in order: row r starts at r * D
        b.x[k].load(src_a + static_cast<int64_t>(r) * D + w * 8);
      }
      b.slot[k] = ld_index(slots, static_cast<int64_t>(t));
    }
  };
  auto compute = [&](const Buf& b, int64_t u0) {
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int64_t r = (u0 + k) * RPU + lane / WPR;
      float x[8];
      b.x[k].get(x);
      const uint32_t t = kvh_div.div(static_cast<uint32_t>(r < rows ? r : rows - 1));
      const int h = static_cast<int>(r < rows ? r : rows - 1) - static_cast<int>(t) * kvh;
      value_pack_word<WPR>(x, w, r < rows, b.slot[k], h, kvh, gw, ng, vq, vs, vm);
    }
  };

  Buf ba, bb;
  int64_t u = wave * U;
  const int64_t step = nw * U;
  if (u < units) load(ba, u);
  for (; u < units; u += 2 * step) {
    if (u + step < units) load(bb, u + step);
    compute(ba, u);
    if (u + step >= units) break;
    if (u + 2 * step < units) load(ba, u + 2 * step);
    compute(bb, u + step);
  }
}

// ---- LDS-staged pack (head size 128, G in {64, 128}, 16-bit input) ---------
// The work is cut into units of 8 KB of source rows.  A key unit is one token
// group of one head and part of its dims: G = 128 -> 128 tokens x 32 dims (a
// quarter of the head), G = 64 -> 64 tokens x 64 dims (a half).  A value unit
// is 32 (token, head) rows.  Each wave takes up to four units and walks them
// with two wave-private LDS stages: a unit's rows arrive by LDS DMA (16 bytes
// a lane, the 16-byte chunks of a row XOR-swizzled), are copied to registers,
// and the stage is refilled with the unit after next while the copy is
// quantized and stored, so two units stay in flight.  Read back, every lane
// holds 64 values of one quantization group:
//   key unit: 64 tokens of one dim, gathered with ds_read_b64_tr_b16.  Lane
//     l of each 16-lane group receives element l % 4 of the 8-byte runs that
//     lanes l / 4 + 4k address (k = 0..3, in that order): lane a pointing at
//     token T + a / 4, dims 4m..4m+3 hands lane 4q + r tokens T..T+3 of dim
//     4m + r;
//   value unit: half a row (64 dims), by 16-byte LDS reads.
// The group min/max is a lane-local scan plus at most one exchange with the
// lane holding the group's other half (G = 128), and every lane writes its 8
// packed words as one 32-byte run; scales and minima go out as consecutive
// 4-byte lanes.  The swizzles keep the transposing reads and the row reads
// free of bank conflicts within each half wave.  Each unit's source rows and
// page slots are read once, up front, into a small LDS table, so the loop
// itself issues no vector loads but the DMAs.  The loop is not unrolled and
// keys and values share one quantize body: the kernel stays well inside the
// instruction cache.
namespace lp {

constexpr int kUnit = 8192;  // source bytes per unit
constexpr int kWaves = 4;    // waves per workgroup
constexpr int kUnitsPerWave = 4;
constexpr int kStages = 2;   // LDS stages per wave (units in flight)
constexpr int kMeta = 512;   // per unit: 128 int32 source rows (keys) or 32 (values)
constexpr int kLds = kStages * kUnit * kWaves + kMeta * kUnitsPerWave * kWaves;
constexpr int kD = 128;

typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s* lds_v4s_ptr;
typedef uint32_t u2v __attribute__((ext_vector_type(2)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));

// LDS DMA of 16 bytes a lane into stage + 16 * lane, written as inline asm so
// that the compiler's wait-count pass does not track it: with stores in
// flight that pass can only wait for every outstanding access (vmcnt(0)),
// where the loop below waits for exactly the DMA it needs.  The stage
// address goes to M0 through an operand constraint; the nop keeps the M0
// write and the DMA apart.
__device__ __forceinline__ void dma16_counted(const void* g, const char* stage) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)(stage))));
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "{m0}"(m0) : "memory");
}

// s_waitcnt lgkmcnt(0), vmcnt and expcnt left alone.
__device__ __forceinline__ void wait_lgkm0() {
  __builtin_amdgcn_s_waitcnt(0xF | (7 << 4) | (0 << 8) | (3 << 14));
  asm volatile("" ::: "memory");
}

// One side of a pack: token t reads row index[t] (or t) of a, rows past n_a
// continuing into b, and goes to page slot slots[t] (negative: not stored).
// Source row numbers stay below 2^31.
template <typename T, typename I>
struct Side {
  const T* a;
  int64_t n_a;
  const T* b;
  const int64_t* index;
  const I* slots;
  int64_t count;  // tokens
};

template <typename T, typename I>
struct Ctx {
  Side<T, I> k, v;
  int kvh, bs;
  FastDiv kdiv;  // division by kvh
  int32_t* kq;
  float* ks;
  float* km;
  int32_t* vq;
  float* vs;
  float* vm;
};

template <typename T>
__device__ __forceinline__ void unpack2(uint32_t w, float& lo, float& hi);
template <>
__device__ __forceinline__ void unpack2<bf16>(uint32_t w, float& lo, float& hi) {
  lo = __uint_as_float(w << 16);
  hi = __uint_as_float(w & 0xffff0000u);
}
template <>
__device__ __forceinline__ void unpack2<f16>(uint32_t w, float& lo, float& hi) {
  lo = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w)));
  hi = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
}

// 64 values (32 words of two) -> group min, scale and 8 packed words of 8
// consecutive values each.  The min/max is exchanged first with the lane
// holding the group's other half: XOR 1 with the next lane (a value row at
// G = 128), XOR 8 within the 16-lane row (a key dim at G = 128), or none.
template <typename T>
__device__ __forceinline__ void quantize64(const uint32_t (&e)[32], int partner,
                                           uint32_t (&word)[8], float& mn_out, float& sc_out) {
  float mn, mx;
  {
    float a, b;
    unpack2<T>(e[0], a, b);
    mn = fmin_ordered(a, b);
    mx = fmax_ordered(a, b);
  }
#pragma unroll
  for (int i = 1; i < 32; ++i) {
    float a, b;
    unpack2<T>(e[i], a, b);
    mn = fmin_ordered(fmin_ordered(mn, a), b);
    mx = fmax_ordered(fmax_ordered(mx, a), b);
  }
  if (partner == 1) {
    mn = fmin_ordered(mn, lane_xor<1>(mn));
    mx = fmax_ordered(mx, lane_xor<1>(mx));
  } else if (partner == 8) {
    // rotating a 16-lane row by 8 swaps its halves: lane ^ 8
    mn = fmin_ordered(mn, __int_as_float(__builtin_amdgcn_update_dpp(
                              0, __float_as_int(mn), 0x128, 0xF, 0xF, false)));
    mx = fmax_ordered(mx, __int_as_float(__builtin_amdgcn_update_dpp(
                              0, __float_as_int(mx), 0x128, 0xF, 0xF, false)));
  }
  const float sc = kivi_group_scale(mn, mx);
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) unpack2<T>(e[4 * w + i], x[2 * i], x[2 * i + 1]);
    word[w] = kivi_pack_word(x, mn, sc);
  }
  mn_out = mn;
  sc_out = sc;
}

// Unit u's source-row table, for a side read through an index.  Key: the
// rows of its G tokens (int32).  Value: for each of its 32 (token, head) rows
// the source head row row * kvh + h (int32; the last row for rows past the
// end).  A side without an index needs no table.
template <typename T, typename I, int G>
__device__ __forceinline__ void load_table(const Ctx<T, I>& c, int64_t nk, int64_t u, char* meta,
                                           int lane) {
  int32_t* rows = reinterpret_cast<int32_t*>(meta);
  if (u < nk) {
    if (!c.k.index) return;
    constexpr int P = G == 128 ? 4 : 2;
    const int64_t t0 = u / P / c.kvh * G;
#pragma unroll
    for (int i = 0; i < G / 64; ++i) rows[64 * i + lane] = static_cast<int32_t>(c.k.index[t0 + 64 * i + lane]);
  } else if (c.v.index && lane < 32) {
    const int64_t nrows = c.v.count * c.kvh;
    const int64_t r = (u - nk) * 32 + lane;
    const int64_t rc = r < nrows ? r : nrows - 1;
    const uint32_t t = c.kdiv.div(static_cast<uint32_t>(rc));
    const int h = static_cast<int>(rc) - static_cast<int>(t) * c.kvh;
    rows[lane] = static_cast<int32_t>(c.v.index[t] * c.kvh + h);
  }
}

// Page slot of token t, read through the scalar cache (t is uniform), so the
// load is counted apart from the DMAs.
template <typename I>
__device__ __forceinline__ int64_t slot_of(const I* slots, int64_t t) {
  typedef const __attribute__((address_space(4))) I* const_ptr;
  return static_cast<int64_t>(((const_ptr)(reinterpret_cast<uintptr_t>(slots)))[t]);
}

// Unit u's 8 DMAs into stage.  Every unit issues exactly 8 (a key group with
// no slot is loaded too, then not stored): the loop's counted waits rely on it.
// A source address is base + row * row_bytes, the base chosen by whether the
// row lies in a or in b and holding the lane's column.
template <typename T, typename I, int G>
__device__ __forceinline__ void issue(const Ctx<T, I>& c, int64_t nk, int64_t u, const char* meta,
                                      const char* stage, int lane) {
  const int32_t* rows = reinterpret_cast<const int32_t*>(meta);
  uint64_t addr[8];
  if (u < nk) {
    constexpr int P = G == 128 ? 4 : 2;
    const int part = static_cast<int>(u % P);
    const int h = static_cast<int>((u / P) % c.kvh);
    const uint32_t rb = static_cast<uint32_t>(c.kvh * kD * sizeof(T));
    const uint64_t a0 = reinterpret_cast<uintptr_t>(c.k.a);
    const uint64_t b0 = reinterpret_cast<uintptr_t>(c.k.b) - static_cast<uint64_t>(c.k.n_a) * rb;
    // the lane's column: G = 128 -> 16-byte chunk (lane % 4) ^ 2 (d >= 4)
    // of the quarter; G = 64 -> chunk (lane % 8) ^ (4 ((lane / 8) >> 1 & 1))
    int col0, col1;
    if constexpr (G == 128) {
      col0 = part * 32 + 8 * (lane % 4);
      col1 = part * 32 + 8 * ((lane % 4) ^ 2);
    } else {
      col0 = col1 = part * 64 + 8 * ((lane % 8) ^ (4 * (((lane / 8) >> 1) & 1)));
    }
    const uint32_t off0 = static_cast<uint32_t>((h * kD + col0) * sizeof(T));
    const uint32_t off1 = static_cast<uint32_t>((h * kD + col1) * sizeof(T));
    const int64_t t0 = u / P / c.kvh * G;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const int tok = G == 128 ? 16 * d + lane / 4 : 8 * d + lane / 8;
      const int32_t row = c.k.index ? rows[tok] : static_cast<int32_t>(t0 + tok);
      const uint64_t base = (row < c.k.n_a ? a0 : b0) + (G == 128 && d >= 4 ? off1 : off0);
      addr[d] = base + static_cast<uint64_t>(static_cast<uint32_t>(row)) * rb;
    }
  } else {
    // DMA d: row 4d + lane / 16 of the unit, 16-byte chunk
    // (lane % 16) ^ (row % 8) = (lane % 16) ^ (lane / 16 + 4 (d % 2))
    const uint32_t hb = static_cast<uint32_t>(kD * sizeof(T));
    const int64_t split = c.v.n_a * c.kvh;
    const uint64_t a0 = reinterpret_cast<uintptr_t>(c.v.a);
    const uint64_t b0 = reinterpret_cast<uintptr_t>(c.v.b) - static_cast<uint64_t>(split) * hb;
    const uint32_t off0 = 16u * static_cast<uint32_t>((lane % 16) ^ (lane / 16));
    const uint32_t off1 = 16u * static_cast<uint32_t>((lane % 16) ^ (lane / 16 + 4));
    const int64_t nrows = c.v.count * c.kvh;
    const int64_t r0 = (u - nk) * 32;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const int64_t r = r0 + 4 * d + lane / 16;
      const int32_t f = c.v.index ? rows[4 * d + lane / 16]
                                  : static_cast<int32_t>(r < nrows ? r : nrows - 1);
      const uint64_t base = (f < split ? a0 : b0) + (d % 2 ? off1 : off0);
      addr[d] = base + static_cast<uint64_t>(static_cast<uint32_t>(f)) * hb;
    }
  }
#pragma unroll
  for (int d = 0; d < 8; ++d)
    dma16_counted(reinterpret_cast<const void*>(addr[d]), stage + d * 1024);
}

// Read a landed stage into registers: 64 values of one group per lane, in
// order (see the layout notes above).
template <int G>
__device__ __forceinline__ void read_stage(bool key, const char* stage, int lane,
                                           uint32_t (&e)[32]) {
  if (key) {
    const int a = lane % 16;
    const int g = lane / 16;
    int base, step;
    if constexpr (G == 128) {
      base = 64 * (64 * ((a % 4) >> 1) + a / 4) + 16 * (g ^ (2 * ((a % 4) >> 1))) +
             8 * ((a % 4) & 1);
      step = 256;
    } else {
      base = 128 * (a / 4) + 16 * ((2 * g + ((a % 4) >> 1)) ^ (4 * (((a / 4) >> 1) & 1))) +
             8 * ((a % 4) & 1);
      step = 512;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const u2v r = __builtin_bit_cast(
          u2v, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_ptr)(stage + base + step * i)));
      e[2 * i] = r.x;
      e[2 * i + 1] = r.y;
    }
  } else {
    const int rho = lane / 2;
    const int hh = lane % 2;
    const int s = rho % 8;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const u4v q = *reinterpret_cast<const u4v*>(stage + rho * 256 + 16 * (8 * hh + (j ^ s)));
      e[4 * j] = q.x;
      e[4 * j + 1] = q.y;
      e[4 * j + 2] = q.z;
      e[4 * j + 3] = q.w;
    }
  }
}

// Quantize unit u (held in registers) and store its words, scales and minima.
template <typename T, typename I, int G>
__device__ __forceinline__ void finish(const Ctx<T, I>& c, int64_t nk, int64_t u, const char* meta,
                                       const uint32_t (&e)[32], int lane) {
  const bool key = u < nk;
  const int a = lane % 16;
  int64_t slot;
  int64_t orow = 0;
  if (key) {
    constexpr int P = G == 128 ? 4 : 2;
    slot = slot_of(c.k.slots, u / P / c.kvh * G);
    if (slot < 0) return;  // uniform: the group is not stored
  } else {
    // the unit's rows span tokens tf..tl: their slots come through the
    // scalar cache and each lane picks its own
    const int64_t nrows = c.v.count * c.kvh;
    const int64_t r0 = (u - nk) * 32;
    const int64_t r = r0 + lane / 2;
    const int64_t rl = r0 + 31 < nrows ? r0 + 31 : nrows - 1;
    const int64_t tf = c.kdiv.div(static_cast<uint32_t>(r0));
    const int64_t tl = c.kdiv.div(static_cast<uint32_t>(rl));
    const int64_t t = c.kdiv.div(static_cast<uint32_t>(r < nrows ? r : nrows - 1));
    slot = -1;
    for (int64_t tt = tf; tt <= tl; ++tt) {
      const int64_t st = slot_of(c.v.slots, tt);
      slot = t == tt ? st : slot;
    }
    if (r >= nrows) slot = -1;
    orow = slot * c.kvh + (static_cast<int>(r < nrows ? r : nrows - 1) - static_cast<int>(t) * c.kvh);
  }
  uint32_t word[8];
  float mn, sc;
  quantize64<T>(e, G == 128 ? (key ? 8 : 1) : 0, word, mn, sc);
  if (slot < 0) return;  // a value row past the end, or a token with no slot
  const u4v lo{word[0], word[1], word[2], word[3]};
  const u4v hi{word[4], word[5], word[6], word[7]};
  if (key) {
    constexpr int P = G == 128 ? 4 : 2;
    const int part = static_cast<int>(u % P);
    const int h = static_cast<int>((u / P) % c.kvh);
    const int g = lane / 16;
    const int dim = G == 128 ? part * 32 + 4 * (2 * g + ((a / 4) & 1)) + a % 4 : part * 64 + lane;
    const int hh = G == 128 ? (a / 4) >> 1 : 0;  // token half of a G = 128 group
    const int64_t blk = slot / c.bs;
    const int off = static_cast<int>(slot - blk * c.bs);
    const int64_t drow = (blk * c.kvh + h) * kD + dim;
    if (hh == 0) {
      const int64_t sidx = drow * (c.bs / G) + off / G;
      c.ks[sidx] = sc;
      c.km[sidx] = mn;
    }
    u4v* dst = reinterpret_cast<u4v*>(c.kq + drow * (c.bs / 8) + off / 8 + 8 * hh);
    __builtin_nontemporal_store(lo, dst);
    __builtin_nontemporal_store(hi, dst + 1);
  } else {
    const int hh = lane % 2;
    if (G == 64 || hh == 0) {
      const int64_t sidx = orow * (kD / G) + (G == 64 ? hh : 0);
      c.vs[sidx] = sc;
      c.vm[sidx] = mn;
    }
    u4v* dst = reinterpret_cast<u4v*>(c.vq + orow * (kD / 8) + 8 * hh);
    __builtin_nontemporal_store(lo, dst);
    __builtin_nontemporal_store(hi, dst + 1);
  }
}

}  // namespace lp

// One-launch store.  A store batch (key pack groups, value pack rows,
// ring-row writes of both sides) whose ring writes overwrite no row that the
// same batch packs has no order inside it, so it runs as one grid:
// workgroups [0, pack_blocks) take the key units then the value units (unit
// w + k * (pack_blocks * 4) for wave w, k < 4), the blocks after them copy
// ring rows (16 bytes a thread, same dtype).  Pack sources index [ring rows ;
// input rows].  The ring is read (pack sources) and written (ring rows) by
// the same grid, so its pointers are not restrict-qualified.  PLANNED reads
// the pack and ring counts from counts[0..3] (capped by the side counts given,
// which are then capacities), so one captured launch serves every step;
// waves past a count exit at once.
template <typename T, typename I, int G, bool PLANNED>
__global__ void __launch_bounds__(256)
kivi_pack_lds_kernel(lp::Ctx<T, I> c, int64_t pack_blocks, const int64_t* __restrict__ counts,
                     T* ring_k, T* ring_v, const T* __restrict__ in_k,
                     const T* __restrict__ in_v, const int64_t* __restrict__ kr_src,
                     const int64_t* __restrict__ kr_dst, const int64_t* __restrict__ vr_src,
                     const int64_t* __restrict__ vr_dst, int64_t nkr, int64_t nvr) {
  __shared__ __attribute__((aligned(16))) char lds[lp::kLds];
  if constexpr (PLANNED) {
    c.k.count = min(counts[0], c.k.count);
    c.v.count = min(counts[1], c.v.count);
    nkr = min(counts[2], nkr);
    nvr = min(counts[3], nvr);
  }
  if (blockIdx.x >= pack_blocks) {
    // ring rows: 16 bytes a thread, same dtype
    const int per_row = c.kvh * (lp::kD / 8);
    const int64_t i0 = (static_cast<int64_t>(blockIdx.x) - pack_blocks) * 256 + threadIdx.x;
    const int64_t i = i0 / per_row;
    if (i >= nkr + nvr) return;
    const int64_t e = (i0 - i * per_row) * 8;
    const int64_t row_elems = static_cast<int64_t>(c.kvh) * lp::kD;
    const bool key = i < nkr;
    const int64_t j = key ? i : i - nkr;
    const T* src = (key ? in_k : in_v) + (key ? kr_src : vr_src)[j] * row_elems + e;
    T* dst = (key ? ring_k : ring_v) + (key ? kr_dst : vr_dst)[j] * row_elems + e;
    *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
    return;
  }
  constexpr int P = G == 128 ? 4 : 2;
  const int64_t nk = c.k.count / G * c.kvh * P;
  const int64_t nu = nk + (c.v.count * c.kvh + 31) / 32;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t nw = pack_blocks * lp::kWaves;
  const int64_t w = static_cast<int64_t>(blockIdx.x) * lp::kWaves + wave;
  int n = 0;
#pragma unroll
  for (int k = 0; k < lp::kUnitsPerWave; ++k) n += w + k * nw < nu ? 1 : 0;
  if (n == 0) return;
  constexpr int S = lp::kStages;
  char* stage = lds + wave * S * lp::kUnit;
  char* meta = lds + lp::kWaves * S * lp::kUnit + wave * lp::kUnitsPerWave * lp::kMeta;
  if (c.k.index || c.v.index) {
    for (int k = 0; k < n; ++k)
      lp::load_table<T, I, G>(c, nk, w + k * nw, meta + k * lp::kMeta, lane);
    wait_vmcnt<0>();  // the tables are written before any DMA goes out
    lp::wait_lgkm0();
  }
#pragma unroll
  for (int k = 0; k < S; ++k)
    if (k < n) lp::issue<T, I, G>(c, nk, w + k * nw, meta + k * lp::kMeta, stage + k * lp::kUnit, lane);
  // Step k: unit k's rows were DMA'd into stage k % S S steps ago, unit
  // k + 1's (two stages) one step ago.  Loads complete in issue order, so with
  // at most 8 vector-memory operations outstanding -- the 8 DMAs of unit
  // k + 1 -- unit k has landed, whatever the stores in between do.
#pragma clang loop unroll(disable)
  for (int k = 0; k < n; ++k) {
    const int64_t u = w + k * nw;
    char* cur = stage + (k % S) * lp::kUnit;
    if (S == 2 && k + 1 < n)
      wait_vmcnt<8>();
    else
      wait_vmcnt<0>();
    uint32_t e[32];
    lp::read_stage<G>(u < nk, cur, lane, e);
    lp::wait_lgkm0();  // the stage is read before the next DMA overwrites it
    if (k + S < n) lp::issue<T, I, G>(c, nk, u + S * nw, meta + (k + S) * lp::kMeta, cur, lane);
    lp::finish<T, I, G>(c, nk, u, meta + k * lp::kMeta, e, lane);
  }
}

// Workgroups of `kernel` that fit the device at once (CUs x occupancy),
// cached per kernel and device; 0 on error.
template <typename K>
int64_t resident_blocks(K* kernel, int threads) {
  static std::mutex mu;
  static int64_t cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  std::lock_guard<std::mutex> lock(mu);
  if (cache[dev] == 0) {
    int cus = 0, per = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, reinterpret_cast<const void*>(kernel),
                                                     threads, 0) != hipSuccess)
      return 0;
    cache[dev] = static_cast<int64_t>(cus) * (per > 0 ? per : 1);
  }
  return cache[dev];
}

// Launch kivi_pack_lds_kernel: pack workgroups of 4 waves taking 1 to 4
// units each (as few as lets the resident waves hold all the work at once),
// then the ring-row blocks.  Side counts are token counts (capacities when
// counts != null).
template <typename T, typename I, int G>
int launch_pack_lds(const lp::Ctx<T, I>& c, const int64_t* counts, T* ring_k, T* ring_v,
                    const T* in_k, const T* in_v, const int64_t* kr_src, const int64_t* kr_dst,
                    const int64_t* vr_src, const int64_t* vr_dst, int64_t nkr, int64_t nvr,
                    hipStream_t s) {
  constexpr int P = G == 128 ? 4 : 2;
  if (c.v.count * c.kvh >= 0x7fffffff) return KVQ_ERR_INVALID;
  const int64_t units = c.k.count / G * c.kvh * P + (c.v.count * c.kvh + 31) / 32;
  const bool planned = counts != nullptr;
  auto* kern = planned ? kivi_pack_lds_kernel<T, I, G, true> : kivi_pack_lds_kernel<T, I, G, false>;
  // units per wave: enough that the resident waves cover the work at once,
  // at most kUnitsPerWave (the kernel takes u, u + nw, ... while below units)
  const int64_t fit = resident_blocks(kern, 256);
  if (fit <= 0) return KVQ_ERR_INVALID;
  const int64_t resident_waves = fit * lp::kWaves;
  int64_t upw = (units + resident_waves - 1) / resident_waves;
  upw = upw < 1 ? 1 : (upw > lp::kUnitsPerWave ? lp::kUnitsPerWave : upw);
  const int64_t per_block = lp::kWaves * upw;
  const int64_t pack_blocks = (units + per_block - 1) / per_block;
  const int64_t rchunks = (nkr + nvr) * c.kvh * (lp::kD / 8);
  const int64_t blocks = pack_blocks + (rchunks + 255) / 256;
  if (blocks == 0) return KVQ_OK;
  if (blocks > 0x7fffffff) return KVQ_ERR_INVALID;
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, c, pack_blocks,
                     counts, ring_k, ring_v, in_k, in_v, kr_src, kr_dst, vr_src, vr_dst, nkr, nvr);
  KVQ_LAUNCH_CHECK();
  return KVQ_OK;
}

// The store's job sections on the LDS-staged pack: c0..c3 are the section
// sizes (capacities when counts != null).
template <typename T>
int launch_store_lds(const void* key_input, const void* value_input, void* ring_k, void* ring_v,
                     int64_t ring_rows, int kvh, int g, int bs, const int64_t* sections,
                     const int64_t* counts, int64_t c0, int64_t c1, int64_t c2, int64_t c3,
                     int32_t* kq, float* ks, float* km, int32_t* vq, float* vs, float* vm,
                     hipStream_t s) {
  const int64_t* kp_src = sections;
  const int64_t* kp_slot = kp_src + c0;
  const int64_t* vp_src = kp_slot + c0;
  const int64_t* vp_slot = vp_src + c1;
  const int64_t* kr_src = vp_slot + c1;
  const int64_t* kr_dst = kr_src + c2;
  const int64_t* vr_src = kr_dst + c2;
  const int64_t* vr_dst = vr_src + c3;
  T* rk = static_cast<T*>(ring_k);
  T* rv = static_cast<T*>(ring_v);
  const T* ik = static_cast<const T*>(key_input);
  const T* iv = static_cast<const T*>(value_input);
  lp::Ctx<T, int64_t> c{};
  c.k = lp::Side<T, int64_t>{rk, ring_rows, ik, kp_src, kp_slot, c0};
  c.v = lp::Side<T, int64_t>{rv, ring_rows, iv, vp_src, vp_slot, c1};
  c.kvh = kvh;
  c.bs = bs;
  c.kdiv = FastDiv::make(static_cast<uint32_t>(kvh));
  c.kq = kq;
  c.ks = ks;
  c.km = km;
  c.vq = vq;
  c.vs = vs;
  c.vm = vm;
  if (g == 128)
    return launch_pack_lds<T, int64_t, 128>(c, counts, rk, rv, ik, iv, kr_src, kr_dst, vr_src,
                                            vr_dst, c2, c3, s);
  return launch_pack_lds<T, int64_t, 64>(c, counts, rk, rv, ik, iv, kr_src, kr_dst, vr_src,
                                         vr_dst, c2, c3, s);
}

// One side of a pack on the LDS-staged kernel (the other side empty, no ring
// rows): the per-side entry points' path where the kernel applies, so every
// pack writes its scales and minima as consecutive runs (a per-row scale
// written alone covers a 4-byte piece of a line, which the memory side turns
// into a read of the line).
template <typename T, typename I>
int pack_side_lds(bool key, const void* src_a, int64_t n_a, const void* src_b,
                  const int64_t* src_index, const void* slot_mapping, int64_t num_tokens,
                  int kvh, int g, int bs, int32_t* quant, float* scale, float* mn,
                  hipStream_t s) {
  const lp::Side<T, I> side{static_cast<const T*>(src_a), n_a, static_cast<const T*>(src_b),
                            src_index, static_cast<const I*>(slot_mapping), num_tokens};
  const lp::Side<T, I> none{nullptr, 0, nullptr, nullptr, nullptr, 0};
  lp::Ctx<T, I> c{};
  c.k = key ? side : none;
  c.v = key ? none : side;
  c.kvh = kvh;
  c.bs = bs;
  c.kdiv = FastDiv::make(static_cast<uint32_t>(kvh));
  c.kq = key ? quant : nullptr;
  c.ks = key ? scale : nullptr;
  c.km = key ? mn : nullptr;
  c.vq = key ? nullptr : quant;
  c.vs = key ? nullptr : scale;
  c.vm = key ? nullptr : mn;
  if (g == 128)
    return launch_pack_lds<T, I, 128>(c, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                      nullptr, nullptr, nullptr, 0, 0, s);
  return launch_pack_lds<T, I, 64>(c, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                   nullptr, nullptr, nullptr, 0, 0, s);
}

bool pack_lds_applies(int src_dtype, int head_size, int group_size, int64_t num_tokens,
                      int kvh) {
  return head_size == 128 && (group_size == 64 || group_size == 128) &&
         (src_dtype == KVQ_DTYPE_BF16 || src_dtype == KVQ_DTYPE_F16) &&
         num_tokens * kvh < 0x7fffffff;  // source rows are int32 in the kernel
}

template <typename I>
int pack_side_lds_dispatch(bool key, int src_dtype, const void* src_a, int64_t n_a,
                           const void* src_b, const int64_t* src_index, const void* slot_mapping,
                           int64_t num_tokens, int kvh, int g, int bs, int32_t* quant,
                           float* scale, float* mn, hipStream_t s) {
  if (src_dtype == KVQ_DTYPE_BF16)
    return pack_side_lds<bf16, I>(key, src_a, n_a, src_b, src_index, slot_mapping, num_tokens,
                                  kvh, g, bs, quant, scale, mn, s);
  return pack_side_lds<f16, I>(key, src_a, n_a, src_b, src_index, slot_mapping, num_tokens, kvh,
                               g, bs, quant, scale, mn, s);
}

int pack_side(bool key, int src_dtype, const void* src_a, int64_t n_a, const void* src_b,
              const int64_t* src_index, const void* slot_mapping, int slot_index_type,
              int64_t num_tokens, int kvh, int g, int bs, int32_t* quant, float* scale,
              float* mn, hipStream_t s) {
  if (slot_index_type == KVQ_INDEX_I64)
    return pack_side_lds_dispatch<int64_t>(key, src_dtype, src_a, n_a, src_b, src_index,
                                           slot_mapping, num_tokens, kvh, g, bs, quant, scale,
                                           mn, s);
  return pack_side_lds_dispatch<int32_t>(key, src_dtype, src_a, n_a, src_b, src_index,
                                         slot_mapping, num_tokens, kvh, g, bs, quant, scale, mn,
                                         s);
}

bool kivi_geometry_ok(int kvh, int d, int g, int bs) {
  return kvh > 0 && d > 0 && g > 0 && bs > 0 && g % 8 == 0 && d % 8 == 0 && d % g == 0 &&
         bs % g == 0;
}

}  // namespace

extern "C" int kvq_abi_version(void) { return 1; }

extern "C" int kvq_kivi_pack_key(const void* src_a, int64_t n_a, const void* src_b,
                                 const int64_t* src_index, int src_dtype,
                                 const void* slot_mapping, int slot_index_type,
                                 int64_t num_tokens, int num_kv_heads, int head_size,
                                 int group_size, int block_size, int32_t* k_quant,
                                 float* k_scale, float* k_mn, void* stream) {
  if (num_tokens == 0) return KVQ_OK;
  if (!src_a || !slot_mapping || !k_quant || !k_scale || !k_mn || num_tokens < 0)
    return KVQ_ERR_INVALID;
  if (!kivi_geometry_ok(num_kv_heads, head_size, group_size, block_size))
    return KVQ_ERR_GEOMETRY;
  if (num_tokens % group_size) return KVQ_ERR_INVALID;
  if (!src_index && n_a < num_tokens) return KVQ_ERR_INVALID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (pack_lds_applies(src_dtype, head_size, group_size, num_tokens, num_kv_heads) &&
      (slot_index_type == KVQ_INDEX_I32 || slot_index_type == KVQ_INDEX_I64))
    return pack_side(true, src_dtype, src_a, n_a, src_b, src_index, slot_mapping,
                     slot_index_type, num_tokens, num_kv_heads, group_size, block_size, k_quant,
                     k_scale, k_mn, s);
  if (head_size == 128 && (group_size == 64 || group_size == 128) &&
      (src_dtype == KVQ_DTYPE_BF16 || src_dtype == KVQ_DTYPE_F16)) {
    // register form: one wave per (token group, head, part of the dims):
    // quarters at G = 128 (8 rows per lane), halves at G = 64
    const int parts = group_size == 128 ? 4 : 2;
    const int64_t units = num_tokens / group_size * num_kv_heads * parts;
    const int64_t blocks = (units + 3) / 4;
    if (blocks > 0x7fffffff) return KVQ_ERR_INVALID;
#define KVQ_LAUNCH_KEY_WAVE(T, GG)                                                            \
  KVQ_DISPATCH_INDEX(slot_index_type, I,                                                      \
    hipLaunchKernelGGL((kivi_pack_key_wave_kernel<T, I, GG, GG == 128 ? 4 : 8>),               \
                       dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s,                  \
                       static_cast<const T*>(src_a), n_a, static_cast<const T*>(src_b),       \
                       src_index, static_cast<const I*>(slot_mapping), units, num_kv_heads,   \
                       block_size, k_quant, k_scale, k_mn))
    if (src_dtype == KVQ_DTYPE_BF16) {
      if (group_size == 128) { KVQ_LAUNCH_KEY_WAVE(bf16, 128); } else { KVQ_LAUNCH_KEY_WAVE(bf16, 64); }
    } else {
      if (group_size == 128) { KVQ_LAUNCH_KEY_WAVE(f16, 128); } else { KVQ_LAUNCH_KEY_WAVE(f16, 64); }
    }
#undef KVQ_LAUNCH_KEY_WAVE
    KVQ_LAUNCH_CHECK();
    return KVQ_OK;
  }
  const int tiles = (group_size / 8) * (head_size / 8);
  if (tiles > 1024) return KVQ_ERR_GEOMETRY;
  const int threads = ((tiles + 63) / 64) * 64;
  const size_t lds = sizeof(float) * (3 * (group_size / 8) * head_size + 2 * head_size);
  if (lds > 160 * 1024) return KVQ_ERR_GEOMETRY;
  const dim3 grid(static_cast<unsigned>(num_tokens / group_size), num_kv_heads);
  KVQ_DISPATCH_FLOAT(src_dtype, T,
    KVQ_DISPATCH_INDEX(slot_index_type, I,
      hipLaunchKernelGGL((kivi_pack_key_kernel<T, I>), grid, dim3(threads), lds, s,
                         static_cast<const T*>(src_a), n_a, static_cast<const T*>(src_b),
                         src_index, static_cast<const I*>(slot_mapping), num_kv_heads,
                         head_size, group_size, block_size, k_quant, k_scale, k_mn)));
  KVQ_LAUNCH_CHECK();
  return KVQ_OK;
}

extern "C" int kvq_kivi_pack_value(const void* src_a, int64_t n_a, const void* src_b,
                                   const int64_t* src_index, int src_dtype,
                                   const void* slot_mapping, int slot_index_type,
                                   int64_t num_tokens, int num_kv_heads, int head_size,
                                   int group_size, int block_size, int32_t* v_quant,
                                   float* v_scale, float* v_mn, void* stream) {
  if (num_tokens == 0) return KVQ_OK;
  if (!src_a || !slot_mapping || !v_quant || !v_scale || !v_mn || num_tokens < 0)
    return KVQ_ERR_INVALID;
  if (!kivi_geometry_ok(num_kv_heads, head_size, group_size, block_size))
    return KVQ_ERR_GEOMETRY;
  if (!src_index && n_a < num_tokens) return KVQ_ERR_INVALID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (pack_lds_applies(src_dtype, head_size, group_size, num_tokens, num_kv_heads) &&
      (slot_index_type == KVQ_INDEX_I32 || slot_index_type == KVQ_INDEX_I64))
    return pack_side(false, src_dtype, src_a, n_a, src_b, src_index, slot_mapping,
                     slot_index_type, num_tokens, num_kv_heads, group_size, block_size, v_quant,
                     v_scale, v_mn, s);
  const int wpr = head_size / 8;
  const int gw = group_size / 8;
  const int64_t rows = num_tokens * num_kv_heads;
  if (64 % wpr == 0 && (gw & (gw - 1)) == 0 && rows < 0x7fffffff) {
    // wave-pipelined kernel over units of 64 / wpr rows, 4 units per step
    const int64_t units = (rows + (64 / wpr) - 1) / (64 / wpr);
    const int64_t steps = (units + 3) / 4;
    const int64_t want = (steps + 3) / 4;  // workgroups of 4 waves, one step each
    const FastDiv kdiv = FastDiv::make(static_cast<uint32_t>(num_kv_heads));
#define KVQ_LAUNCH_VALUE_WAVE(WPR)                                                            \
    KVQ_DISPATCH_FLOAT(src_dtype, T,                                                        \
      KVQ_DISPATCH_INDEX(slot_index_type, I,                                                \
        const int64_t fit = resident_blocks(kivi_pack_value_wave_kernel<T, I, WPR>, 256);   \
        if (fit <= 0) return KVQ_ERR_INVALID;                                               \
        const int64_t blocks = want < fit ? want : fit;                                     \
        hipLaunchKernelGGL((kivi_pack_value_wave_kernel<T, I, WPR>),                        \
                           dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s,             \
                           static_cast<const T*>(src_a), n_a, static_cast<const T*>(src_b),  \
                           src_index, static_cast<const I*>(slot_mapping),                   \
                           static_cast<int32_t>(rows), kdiv, group_size, block_size,         \
                           v_quant, v_scale, v_mn)))
    switch (wpr) {
      case 1: KVQ_LAUNCH_VALUE_WAVE(1); break;
      case 2: KVQ_LAUNCH_VALUE_WAVE(2); break;
      case 4: KVQ_LAUNCH_VALUE_WAVE(4); break;
      case 8: KVQ_LAUNCH_VALUE_WAVE(8); break;
      case 16: KVQ_LAUNCH_VALUE_WAVE(16); break;
      case 32: KVQ_LAUNCH_VALUE_WAVE(32); break;
      default: KVQ_LAUNCH_VALUE_WAVE(64); break;
    }
#undef KVQ_LAUNCH_VALUE_WAVE
    KVQ_LAUNCH_CHECK();
    return KVQ_OK;
  }
  const int64_t total = num_tokens * num_kv_heads * (head_size / 8);
  const int threads = 256;
  const int64_t blocks = (total + threads - 1) / threads;
  if (blocks > 0x7fffffff) return KVQ_ERR_INVALID;
  KVQ_DISPATCH_FLOAT(src_dtype, T,
    KVQ_DISPATCH_INDEX(slot_index_type, I,
      hipLaunchKernelGGL((kivi_pack_value_kernel<T, I>), dim3(static_cast<unsigned>(blocks)),
                         dim3(threads), 0, s, static_cast<const T*>(src_a), n_a,
                         static_cast<const T*>(src_b), src_index,
                         static_cast<const I*>(slot_mapping), num_tokens, num_kv_heads,
                         head_size, group_size, block_size, v_quant, v_scale, v_mn)));
  KVQ_LAUNCH_CHECK();
  return KVQ_OK;
}

extern "C" int kvq_kivi_ring_write(const void* src, int src_dtype, const int64_t* src_rows,
                                   const int64_t* dst_rows, int64_t num_rows, int row_elems,
                                   void* ring, int ring_dtype, void* stream) {
  if (num_rows == 0) return KVQ_OK;
  if (!src || !dst_rows || !ring || num_rows < 0 || row_elems <= 0 || row_elems % 8)
    return KVQ_ERR_INVALID;
  const int64_t total = num_rows * (row_elems / 8);
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7fffffff) return KVQ_ERR_INVALID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  KVQ_DISPATCH_FLOAT(src_dtype, TS,
    KVQ_DISPATCH_FLOAT(ring_dtype, TD,
      hipLaunchKernelGGL((ring_write_kernel<TS, TD>), dim3(static_cast<unsigned>(blocks)),
                         dim3(256), 0, s, static_cast<const TS*>(src), src_rows, dst_rows,
                         num_rows, row_elems, static_cast<TD*>(ring))));
  KVQ_LAUNCH_CHECK();
  return KVQ_OK;
}

extern "C" int kvq_kivi_store(const void* key_input, const void* value_input, void* ring_k,
                              void* ring_v, int64_t ring_rows, int dtype, int num_kv_heads,
                              int head_size, int group_size, int block_size, const int64_t* jobs,
                              int64_t n_key_pack, int64_t n_value_pack, int64_t n_key_ring,
                              int64_t n_value_ring, int32_t* k_quant, float* k_scale,
                              float* k_mn, int32_t* v_quant, float* v_scale, float* v_mn,
                              void* stream) {
  if (n_key_pack < 0 || n_value_pack < 0 || n_key_ring < 0 || n_value_ring < 0 ||
      ring_rows < 0)
    return KVQ_ERR_INVALID;
  if (n_key_pack + n_value_pack + n_key_ring + n_value_ring == 0) return KVQ_OK;
  if (!jobs || !ring_k || !ring_v) return KVQ_ERR_INVALID;
  if ((n_key_pack || n_key_ring) && !key_input) return KVQ_ERR_INVALID;
  if ((n_value_pack || n_value_ring) && !value_input) return KVQ_ERR_INVALID;
  if (n_key_pack && (!k_quant || !k_scale || !k_mn)) return KVQ_ERR_INVALID;
  if (n_value_pack && (!v_quant || !v_scale || !v_mn)) return KVQ_ERR_INVALID;
  if (!kivi_geometry_ok(num_kv_heads, head_size, group_size, block_size))
    return KVQ_ERR_GEOMETRY;
  // the register key pack's geometry; callers fall back to the separate
  // pack and ring-write entry points elsewhere
  if (head_size != 128 || (group_size != 64 && group_size != 128) ||
      (dtype != KVQ_DTYPE_BF16 && dtype != KVQ_DTYPE_F16))
    return KVQ_ERR_GEOMETRY;
  if (n_key_pack % group_size) return KVQ_ERR_INVALID;
  if (n_value_pack * num_kv_heads >= 0x7fffffff) return KVQ_ERR_INVALID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == KVQ_DTYPE_BF16)
    return launch_store_lds<bf16>(key_input, value_input, ring_k, ring_v, ring_rows, num_kv_heads,
                                  group_size, block_size, jobs, nullptr, n_key_pack, n_value_pack,
                                  n_key_ring, n_value_ring, k_quant, k_scale, k_mn, v_quant,
                                  v_scale, v_mn, s);
  return launch_store_lds<f16>(key_input, value_input, ring_k, ring_v, ring_rows, num_kv_heads,
                               group_size, block_size, jobs, nullptr, n_key_pack, n_value_pack,
                               n_key_ring, n_value_ring, k_quant, k_scale, k_mn, v_quant, v_scale,
                               v_mn, s);
}

extern "C" int kvq_kivi_store_planned(const void* key_input, const void* value_input,
                                      void* ring_k, void* ring_v, int64_t ring_rows, int dtype,
                                      int num_kv_heads, int head_size, int group_size,
                                      int block_size, const int64_t* plan,
                                      int64_t cap_key_pack, int64_t cap_value_pack,
                                      int64_t cap_ring, int32_t* k_quant, float* k_scale,
                                      float* k_mn, int32_t* v_quant, float* v_scale,
                                      float* v_mn, void* stream) {
  if (cap_key_pack < 0 || cap_value_pack < 0 || cap_ring < 0 || ring_rows < 0)
    return KVQ_ERR_INVALID;
  if (!plan || !ring_k || !ring_v || !key_input || !value_input || !k_quant || !k_scale ||
      !k_mn || !v_quant || !v_scale || !v_mn)
    return KVQ_ERR_INVALID;
  if (!kivi_geometry_ok(num_kv_heads, head_size, group_size, block_size))
    return KVQ_ERR_GEOMETRY;
  if (head_size != 128 || (group_size != 64 && group_size != 128) ||
      (dtype != KVQ_DTYPE_BF16 && dtype != KVQ_DTYPE_F16))
    return KVQ_ERR_GEOMETRY;
  if (cap_key_pack % group_size) return KVQ_ERR_INVALID;
  if (cap_value_pack * num_kv_heads >= 0x7fffffff) return KVQ_ERR_INVALID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // plan: the four counts, then the job sections at capacity offsets
  if (dtype == KVQ_DTYPE_BF16)
    return launch_store_lds<bf16>(key_input, value_input, ring_k, ring_v, ring_rows, num_kv_heads,
                                  group_size, block_size, plan + 4, plan, cap_key_pack,
                                  cap_value_pack, cap_ring, cap_ring, k_quant, k_scale, k_mn,
                                  v_quant, v_scale, v_mn, s);
  return launch_store_lds<f16>(key_input, value_input, ring_k, ring_v, ring_rows, num_kv_heads,
                               group_size, block_size, plan + 4, plan, cap_key_pack,
                               cap_value_pack, cap_ring, cap_ring, k_quant, k_scale, k_mn, v_quant,
                               v_scale, v_mn, s);
}
