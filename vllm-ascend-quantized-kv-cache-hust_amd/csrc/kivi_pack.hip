// SPDX-License-Identifier: Apache-2.0
// KIVI INT4 pack kernels for MI355X (gfx950).
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
// Both quantize with kivi_pack_word: a reciprocal per group, a floor per
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

// ---- one-launch store -------------------------------------------------------
// A store batch (key pack groups, value pack rows, ring-row writes of both
// sides) whose ring writes overwrite no row that the same batch packs has no
// order inside it, so it runs as one grid of 4-wave workgroups split into
// [key pack | value pack | ring rows].  Pack sources index [ring rows ; input
// rows]; ring writes copy input rows to ring rows (same dtype, 16 bytes per
// thread).  jobs (int64): key pack src | key pack slot | value pack src |
// value pack slot | key ring src | key ring dst | value ring src | value ring
// dst.  The ring is read (pack sources) and written (ring rows) by the same
// grid, so its pointers are not restrict-qualified.
//
// PLANNED: the grid and the job sections are sized by capacities (c0..c3) and
// the actual counts are read from the device (jobs[0..3], sections from
// jobs + 4 at capacity offsets), so one captured launch serves every step;
// waves past a count exit at once.
template <typename T, int G, bool PLANNED>
__global__ void __launch_bounds__(256)
kivi_store_kernel(T* ring_k, T* ring_v, int64_t n_ring, const T* __restrict__ in_k,
                  const T* __restrict__ in_v, const int64_t* __restrict__ jobs, int64_t c0,
                  int64_t c1, int64_t c2, int64_t c3, int64_t kblocks, int64_t vblocks,
                  FastDiv kvh_div, int bs, int32_t* __restrict__ kq, float* __restrict__ ks,
                  float* __restrict__ km, int32_t* __restrict__ vq, float* __restrict__ vs,
                  float* __restrict__ vm) {
  constexpr int D = 128;
  constexpr int WPR = D / 8;
  const int kvh = static_cast<int>(kvh_div.d);
  const int64_t row_elems = static_cast<int64_t>(kvh) * D;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  // counts and the eight job sections
  int64_t nkp = c0, nvp = c1, nkr = c2, nvr = c3;
  const int64_t* kp_src = jobs;
  if constexpr (PLANNED) {
    nkp = min(jobs[0], c0);
    nvp = min(jobs[1], c1);
    nkr = min(jobs[2], c2);
    nvr = min(jobs[3], c3);
    kp_src = jobs + 4;
  }
  const int64_t* kp_slot = kp_src + c0;
  const int64_t* vp_src = kp_slot + c0;
  const int64_t* vp_slot = vp_src + c1;
  const int64_t* kr_src = vp_slot + c1;
  const int64_t* kr_dst = kr_src + c2;
  const int64_t* vr_src = kr_dst + c2;
  const int64_t* vr_dst = vr_src + c3;
  int64_t b = blockIdx.x;
  if (b < kblocks) {
    const int64_t u = b * 4 + wave;
    if (u < nkp / G * kvh * 2)
      key_pack_wave<T, int64_t, G>(ring_k, n_ring, in_k, kp_src, kp_slot, u, lane, kvh, bs, kq,
                                   ks, km);
    return;
  }
  b -= kblocks;
  if (b < vblocks) {
    const int64_t* vsrc = vp_src;
    const int64_t* vslot = vp_slot;
    const int64_t rows = nvp * kvh;  // the host keeps this below 2^31
    // a wave whose first row is past the end has nothing to store (uniform)
    if ((b * 4 + wave) * (64 / WPR) >= rows) return;
    const int64_t r = (b * 4 + wave) * (64 / WPR) + lane / WPR;
    const int64_t rc = r < rows ? r : rows - 1;  // past the end: read the last row, store nothing
    const uint32_t t = kvh_div.div(static_cast<uint32_t>(rc));
    const int h = static_cast<int>(rc) - static_cast<int>(t) * kvh;
    const int w = lane % WPR;
    float x[8];
    load8(src_row<T>(ring_v, n_ring, in_v, vsrc[t], row_elems) + h * D + w * 8, x);
    value_pack_word<WPR>(x, w, r < rows, vslot[t], h, kvh, G / 8, D / G, vq, vs, vm);
    return;
  }
  b -= vblocks;
  const int per_row = kvh * (D / 8);
  const int64_t c = b * 256 + threadIdx.x;
  const int64_t i = c / per_row;
  if (i >= nkr + nvr) return;
  const int64_t e = (c - i * per_row) * 8;
  const bool key = i < nkr;
  const int64_t j = key ? i : i - nkr;
  const T* src = (key ? in_k : in_v) + (key ? kr_src : vr_src)[j] * row_elems + e;
  T* dst = (key ? ring_k : ring_v) + (key ? kr_dst : vr_dst)[j] * row_elems + e;
  *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
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
  const int64_t kunits = n_key_pack / group_size * num_kv_heads * 2;
  const int64_t kblocks = (kunits + 3) / 4;
  const int64_t vunits = (n_value_pack * num_kv_heads + 3) / 4;  // 4 rows per wave
  const int64_t vblocks = (vunits + 3) / 4;
  const int64_t rchunks = (n_key_ring + n_value_ring) * num_kv_heads * (head_size / 8);
  const int64_t rblocks = (rchunks + 255) / 256;
  const int64_t blocks = kblocks + vblocks + rblocks;
  if (blocks > 0x7fffffff) return KVQ_ERR_INVALID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const FastDiv kdiv = FastDiv::make(static_cast<uint32_t>(num_kv_heads));
#define KVQ_LAUNCH_STORE(T, GG)                                                               \
  hipLaunchKernelGGL((kivi_store_kernel<T, GG, false>), dim3(static_cast<unsigned>(blocks)),  \
                     dim3(256), 0, s, static_cast<T*>(ring_k), static_cast<T*>(ring_v),        \
                     ring_rows, static_cast<const T*>(key_input),                              \
                     static_cast<const T*>(value_input), jobs, n_key_pack, n_value_pack,       \
                     n_key_ring, n_value_ring, kblocks, vblocks, kdiv, block_size, k_quant,    \
                     k_scale, k_mn, v_quant, v_scale, v_mn)
  if (dtype == KVQ_DTYPE_BF16) {
    if (group_size == 128) { KVQ_LAUNCH_STORE(bf16, 128); } else { KVQ_LAUNCH_STORE(bf16, 64); }
  } else {
    if (group_size == 128) { KVQ_LAUNCH_STORE(f16, 128); } else { KVQ_LAUNCH_STORE(f16, 64); }
  }
#undef KVQ_LAUNCH_STORE
  KVQ_LAUNCH_CHECK();
  return KVQ_OK;
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
  const int64_t kunits = cap_key_pack / group_size * num_kv_heads * 2;
  const int64_t kblocks = (kunits + 3) / 4;
  const int64_t vunits = (cap_value_pack * num_kv_heads + 3) / 4;  // 4 rows per wave
  const int64_t vblocks = (vunits + 3) / 4;
  const int64_t rchunks = 2 * cap_ring * num_kv_heads * (head_size / 8);
  const int64_t rblocks = (rchunks + 255) / 256;
  const int64_t blocks = kblocks + vblocks + rblocks;
  if (blocks == 0) return KVQ_OK;
  if (blocks > 0x7fffffff) return KVQ_ERR_INVALID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const FastDiv kdiv = FastDiv::make(static_cast<uint32_t>(num_kv_heads));
#define KVQ_LAUNCH_STORE(T, GG)                                                               \
  hipLaunchKernelGGL((kivi_store_kernel<T, GG, true>), dim3(static_cast<unsigned>(blocks)),   \
                     dim3(256), 0, s, static_cast<T*>(ring_k), static_cast<T*>(ring_v),        \
                     ring_rows, static_cast<const T*>(key_input),                              \
                     static_cast<const T*>(value_input), plan, cap_key_pack, cap_value_pack,   \
                     cap_ring, cap_ring, kblocks, vblocks, kdiv, block_size, k_quant, k_scale, \
                     k_mn, v_quant, v_scale, v_mn)
  if (dtype == KVQ_DTYPE_BF16) {
    if (group_size == 128) { KVQ_LAUNCH_STORE(bf16, 128); } else { KVQ_LAUNCH_STORE(bf16, 64); }
  } else {
    if (group_size == 128) { KVQ_LAUNCH_STORE(f16, 128); } else { KVQ_LAUNCH_STORE(f16, 64); }
  }
#undef KVQ_LAUNCH_STORE
  KVQ_LAUNCH_CHECK();
  return KVQ_OK;
}
