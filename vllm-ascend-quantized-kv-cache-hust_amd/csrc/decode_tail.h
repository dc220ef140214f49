// SPDX-License-Identifier: Apache-2.0
// Decode attention over the mixed-source tail of one request (a kind-1 work
// item), for one kv head, on one wave: the tail path of the int4 decode kernel.
//
// A request's tail is the positions past min(k_hist, v_hist): keys there are
// int4 (below k_hist) or residual-ring rows, values int4 (below v_hist) or
// ring rows.  The wave walks its item in sub-tiles of kTT = 32 positions:
//   * stages the sub-tile's K as [token][dim] in the activation dtype T: int4
//     history is dequantized (q*scale then +mn in fp32, the reference's gather
//     arithmetic, pkg/methods/kivi_int4/attention_backend.py:849-935) and kept
//     as two T parts, hi = T(k) and lo = T(k - hi); ring rows are copied with
//     lo = 0.  A key rounded to bf16 alone moves the score of an outlier
//     channel (key scale ~20) by ~1e-2, which the softmax carries into the
//     output, while hi + lo keeps ~16 bits;
//   * S^T = (K_hi + K_lo) * Q^T with v_mfma_f32_16x16x32_{bf16,f16} on the raw
//     query (exact products, fp32 accumulation; the softmax scale and log2(e)
//     are applied to the fp32 scores);
//   * then stages V as rows over the same LDS (the keys are consumed by then)
//     and computes O = P * V with P split into two T parts (hi + lo), so p
//     keeps ~16 bits, the V operand gathered by transposing LDS reads;
//   * leaves (m, l, o) per head in the split-K workspace for the combine.
// The int4 key words and the ring value rows of the next sub-tile are loaded
// into registers while the current one computes.
// LDS: 2 * kTT * kKP * 2 bytes = 17 KiB, inside the int4 path's 19-20 KiB per wave.
// Two waves may share an item: wave `half` of `nhalf` takes every nhalf-th
// sub-tile, and the halves' partial results merge through LDS (merge_halves).
#pragma once

#include "kvq_common.h"
#include "kvq_decode.h"

#include <type_traits>

namespace kvq {
namespace tail {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef uint16_t u8v __attribute__((ext_vector_type(8)));
typedef uint16_t u4s __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4 mfma16(u8v a, u8v b, f4 c, bf16) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8, a),
                                                 __builtin_bit_cast(b8, b), c, 0, 0, 0);
}
__device__ __forceinline__ f4 mfma16(u8v a, u8v b, f4 c, f16) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a),
                                                __builtin_bit_cast(h8, b), c, 0, 0, 0);
}

template <typename T>
__device__ __forceinline__ uint16_t bits_of(float x) {
  const T v = from_f32<T>(x);
  return __builtin_bit_cast(uint16_t, v);
}

// Two values as T, round to nearest even, in one register (a in the low half):
// one hardware pair conversion instead of two software roundings.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float a, float b);
template <>
__device__ __forceinline__ uint32_t pack2<bf16>(float a, float b) { return bf16x2_bits(a, b); }
template <>
__device__ __forceinline__ uint32_t pack2<f16>(float a, float b) {
  typedef float f2v __attribute__((ext_vector_type(2)));
  typedef _Float16 h2v __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2v{a, b}), h2v));
}
// The low / high T half of a pair, widened to fp32 (exact).
template <typename T>
__device__ __forceinline__ float half_f32(uint32_t w, int hi);
template <>
__device__ __forceinline__ float half_f32<bf16>(uint32_t w, int hi) {
  return __uint_as_float(hi ? (w & 0xffff0000u) : (w << 16));
}
template <>
__device__ __forceinline__ float half_f32<f16>(uint32_t w, int hi) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(hi ? w >> 16 : w)));
}

__device__ __forceinline__ float sum_kg(float v) { return sum_rows4(v); }  // over the 4 lane groups of 16
__device__ __forceinline__ float max_kg(float v) { return max_rows4(v); }

__device__ __forceinline__ int64_t clamp_page(const int32_t* __restrict__ bt, int p, int bsh,
                                              int64_t nb) {
  const int64_t blk = bt[p >> bsh];
  return blk < 0 ? 0 : (blk >= nb ? nb - 1 : blk);  // never leave the cache
}

// Ring lane of window entry x = first + (p - hist): first < ring_len and the
// window is shorter than the ring, so one conditional subtract replaces the
// modulo; the clamp keeps a malformed entry inside the ring.
__device__ __forceinline__ int ring_lane(int x, int ring_len) {
  x = x >= ring_len ? x - ring_len : x;
  return x < ring_len ? (x < 0 ? 0 : x) : ring_len - 1;
}

// One wave's partial attention result for one work item and kv head, in the
// lane layout of the path that produced it: o[q][r] belongs to query head
// 4*kg + r of the GQA group and one head dim fixed by (q, lane); m and l are
// the log2-domain running max and sum of head n = lane % 16.
struct Partial {
  f4 o[8];
  float m, l;
};

// Two waves of a workgroup (half 0 and half 1) split an item's positions; the
// half-1 wave hands its partial to its half-0 partner through `xfer` (LDS of
// at least 34 * 64 floats that only the half-1 wave writes), and the half-0
// wave folds it into its own, as the split-K combine would.  Every wave of the
// workgroup calls this, under workgroup-uniform control flow: two barriers.
__device__ __forceinline__ void merge_halves(Partial& p, float* __restrict__ xfer, int half,
                                             int lane) {
  f4* xo = reinterpret_cast<f4*>(xfer);
  if (half == 1) {
#pragma unroll
    for (int q = 0; q < 8; ++q) xo[q * 64 + lane] = p.o[q];
    xfer[32 * 64 + lane] = p.m;
    xfer[33 * 64 + lane] = p.l;
  }
  __syncthreads();
  if (half == 0) {
    const float mb = xfer[32 * 64 + lane];
    const float lb = xfer[33 * 64 + lane];
    const float mx = fmaxf(p.m, mb);
    // an empty half has m = -inf, l = 0, o = 0: weight 0 (and no inf - inf)
    const float sa = p.m == -INFINITY ? 0.0f : exp2f(p.m - mx);
    const float sb = mb == -INFINITY ? 0.0f : exp2f(mb - mx);
    const int kg = lane >> 4;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float ar = __shfl(sa, 4 * kg + r, 64);
      const float br = __shfl(sb, 4 * kg + r, 64);
#pragma unroll
      for (int q = 0; q < 8; ++q) p.o[q][r] = p.o[q][r] * ar + xo[q * 64 + lane][r] * br;
    }
    p.l = p.l * sa + lb * sb;
    p.m = mx;
  }
  __syncthreads();  // the partner's region is free again
}

constexpr int kD = 128;
constexpr int kTT = 32;           // positions per sub-tile
constexpr int kKP = kD + 8;       // K row pitch (elements): rows stay 16-byte aligned
constexpr int kKW = kTT / 8 + 1;  // key words of one dim covering a sub-tile (8-aligned start)
constexpr int kLdsBytes = 2 * kTT * kKP * 2;
static_assert(kTT * kD * 2 <= kLdsBytes, "the V rows fit the key region they reuse");

typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s* lds_v4s_ptr;

// One sub-tile's int4 key operands for the lane's dims 2*lane and 2*lane + 1:
// the kKW words covering the sub-tile, and the scale and minimum of the (at
// most two: g >= 32) key groups they fall in, [dim][group].
struct KeyWords {
  uint32_t w[2][kKW];
  float sc[2][2], mn[2][2];
};

// Eight 16-byte pieces of ring rows, as loaded by one lane (vector types, so
// the pieces stay in registers: uint4 copies become byte copies that keep
// a loop-carried array in scratch memory).
typedef uint32_t w4 __attribute__((ext_vector_type(4)));
struct Rows8 {
  w4 r[8];
};

// Work item wi (kind 1) for kv head h: the partial over sub-tiles half,
// half + nhalf, ... of the item.  lds_raw: at least kLdsBytes, the wave's own.
//
// Most global loads of a sub-tile are issued into registers while the
// previous sub-tile computes, so that the wave waits for memory less often:
//   int4 key words    issued after the scores, staged at the next sub-tile's start;
//   ring value rows   issued after the PV step, staged after the next scores;
//   block-table rows  two sub-tiles ahead, so no load waits on another;
//   ring key rows     issued at the sub-tile's start, in flight while its int4
//                     keys are staged (a sub-tile ahead they would need 32 more
//                     registers, which the int4 path sharing the kernel's
//                     allocation cannot spare).
// Values go to LDS as rows ([token][dim], 16-byte chunk c of row r at chunk
// c ^ 2 (r % 4)) and reach the PV MFMAs through transposing reads.  Int4 values
// inside a tail (a value side without a window) are loaded and dequantized
// where they are staged.
template <typename T>
__device__ __forceinline__ Partial tail_item(char* __restrict__ lds_raw, const T* __restrict__ query,
                                          int hq, int kvh, float qscale,
                                          const uint32_t* __restrict__ kq,
                                          const float* __restrict__ ks,
                                          const float* __restrict__ km,
                                          const uint32_t* __restrict__ vq,
                                          const float* __restrict__ vs,
                                          const float* __restrict__ vm, int bs, int g, int64_t nb,
                                          const int32_t* __restrict__ block_table, int64_t maxb,
                                          const int32_t* __restrict__ seq_meta,
                                          const int32_t* __restrict__ wk, int wi, int h,
                                          const T* __restrict__ ring_k,
                                          const T* __restrict__ ring_v, int ring_len,
                                          int half, int nhalf) {
  constexpr int D = kD;
  uint16_t* sk = reinterpret_cast<uint16_t*>(lds_raw);  // [kTT][kKP] int4 key hi parts
  uint16_t* skl = sk + kTT * kKP;                        // [kTT][kKP] int4 key lo parts
  char* sv = lds_raw;                                    // [kTT][D] value rows, after the scores
  // opaque to the optimizer: the lane-dependent set-up below is recomputed per
  // item instead of being hoisted out of the caller's item loop, where it
  // would stay live (in registers) across the int4 path as well
  int lane = threadIdx.x & 63;
  asm volatile("" : "+v"(lane));
  const int b = wk[0];
  const int pb = wk[1];
  const int pe = wk[2];
  const int32_t* sm = seq_meta + 8 * static_cast<int64_t>(b);
  const int khist = sm[1], vhist = sm[2], row = sm[3], kfirst = sm[4], vfirst = sm[5];
  const int rep = hq / kvh;
  const int n = lane & 15;
  const int kg = lane >> 4;
  // bs and g are powers of two: positions split into page and offset, and
  // offsets into key groups, with shifts and masks, not integer divisions
  const int bsh = __builtin_ctz(static_cast<unsigned>(bs));
  const int gsh = __builtin_ctz(static_cast<unsigned>(g));
  const int gpb = bs >> gsh;
  const int wpd = bs >> 3;
  const int32_t* bt = block_table + static_cast<int64_t>(b) * maxb;
  const int64_t ring_row0 = static_cast<int64_t>(row) * ring_len;
  const int c0 = 2 * lane;  // the int4 key dims this lane stages
  // lane 0 of the request's ring row for head h; lanes lie 32-bit byte offsets
  // past it (a ring row of all heads is under 4 GiB), a uniform base plus a
  // lane offset per load
  const char* rk_base = reinterpret_cast<const char*>(ring_k + (ring_row0 * kvh + h) * D);
  const char* rv_base = reinterpret_cast<const char*>(ring_v + (ring_row0 * kvh + h) * D);

  // B operand of QK: q[head n][32*s4 + 8*kg + i], raw (the scale is applied in fp32)
  u8v qb[4];
  {
    const bool live = n < rep;
    const T* qrow = query + (static_cast<int64_t>(b) * hq + h * rep + (live ? n : 0)) * D;
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      const uint4 v = *reinterpret_cast<const uint4*>(qrow + 32 * s4 + 8 * kg);
      qb[s4] = __builtin_bit_cast(u8v, live ? v : make_uint4(0, 0, 0, 0));
    }
  }

  // positions of the sub-tile at p: nt in the item, the first mk with int4
  // keys, the first mv with int4 values
  auto count = [&](int p, int hist) {
    const int nt = (pe - p) < kTT ? (pe - p) : kTT;
    return hist - p < 0 ? 0 : (hist - p < nt ? hist - p : nt);
  };
  // lane j: the block-table entry of the sub-tile's page j (pages past its
  // last repeat the last); only sub-tiles with int4 data look pages up
  auto load_pages = [&](int p) -> int32_t {
    if (p >= pe || (p >= khist && p >= vhist)) return 0;  // uniform
    const int last = ((pe - p < kTT ? pe : p + kTT) - 1) >> bsh;
    const int idx = (p >> bsh) + lane;
    return bt[idx < last ? idx : last];
  };
  // the page of position q of the sub-tile at p (all lanes take part)
  auto page_of = [&](int32_t pg, int p, int q) -> int64_t {
    const int64_t blk = __shfl(pg, (q >> bsh) - (p >> bsh), 64);
    return blk < 0 ? 0 : (blk >= nb ? nb - 1 : blk);  // never leave the cache
  };
  // the same for a position the whole wave shares: a scalar
  auto page_uniform = [&](int32_t pg, int p, int q) -> int64_t {
    const int64_t blk = __builtin_amdgcn_readlane(pg, (q >> bsh) - (p >> bsh));
    return blk < 0 ? 0 : (blk >= nb ? nb - 1 : blk);
  };
  // int4 key words, scales and minima of positions [p, p + mk): the kKW words
  // of each of the lane's two dims (clamped into the range: every load valid)
  auto load_key_words = [&](int p, int32_t pg, KeyWords& kw) {
    const int mk = count(p, khist);
    if (mk == 0) return;  // uniform
    const int first = p & ~7;
    // every position here is the whole wave's: pages and offsets are scalars,
    // and the lane's dims c0 and c0 + 1 add byte offsets to a scalar base
    const uint32_t wo = static_cast<uint32_t>(c0 * wpd * 4);
    const uint32_t so = static_cast<uint32_t>(c0 * gpb * 4);
#pragma unroll
    for (int k = 0; k < kKW; ++k) {
      const int q = first + 8 * k;
      const int qq = q < p ? p : (q < p + mk ? q : p + mk - 1);
      const int64_t r = (page_uniform(pg, p, qq) * kvh + h) * D;
      const char* wb = reinterpret_cast<const char*>(kq + r * wpd + ((qq & (bs - 1)) >> 3));
      kw.w[0][k] = *reinterpret_cast<const uint32_t*>(wb + wo);
      kw.w[1][k] = *reinterpret_cast<const uint32_t*>(wb + wo + 4 * wpd);
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {  // the groups of positions p and p + mk - 1
      const int qq = s ? p + mk - 1 : p;
      const int64_t r = (page_uniform(pg, p, qq) * kvh + h) * D * gpb + ((qq & (bs - 1)) >> gsh);
      const char* sb = reinterpret_cast<const char*>(ks + r);
      const char* mb = reinterpret_cast<const char*>(km + r);
      kw.sc[0][s] = *reinterpret_cast<const float*>(sb + so);
      kw.sc[1][s] = *reinterpret_cast<const float*>(sb + so + 4 * gpb);
      kw.mn[0][s] = *reinterpret_cast<const float*>(mb + so);
      kw.mn[1][s] = *reinterpret_cast<const float*>(mb + so + 4 * gpb);
    }
  };
  // ring key rows: slot 4*jm + s4 holds row 16*jm + n of the sub-tile, dims
  // 32*s4 + 8*kg .. + 7; rows outside [mk, nt) read a row in the ring and are
  // not staged
  auto load_ring_keys = [&](int p) {
    const int nt = (pe - p) < kTT ? (pe - p) : kTT;
    const int mk = count(p, khist);
    Rows8 kr;
#pragma unroll
    for (int jm = 0; jm < 2; ++jm) {
      const int pi = 16 * jm + n;
      const int pc = pi < mk ? mk : (pi < nt ? pi : nt - 1);
      const int rl = ring_lane(kfirst + (p + pc - khist), ring_len);
      const uint32_t off = static_cast<uint32_t>((rl * kvh * D + 8 * kg) * 2);
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
        kr.r[4 * jm + s4] = *reinterpret_cast<const w4*>(rk_base + off + 64 * s4);
    }
    return kr;
  };
  // ring value rows: slot k holds row (lane / 16) + 4k, chunk lane % 16
  auto load_ring_values = [&](int p) {
    const int nt = (pe - p) < kTT ? (pe - p) : kTT;
    const int mv = count(p, vhist);
    Rows8 vr;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int pi = kg + 4 * k;
      const int pc = pi < mv ? mv : (pi < nt ? pi : nt - 1);
      const int rl = ring_lane(vfirst + (p + pc - vhist), ring_len);
      vr.r[k] = *reinterpret_cast<const w4*>(rv_base + static_cast<uint32_t>((rl * kvh * D + 8 * n) * 2));
    }
    return vr;
  };

  float m_run = -INFINITY;
  float l_run = 0.0f;
  f4 o_acc[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) o_acc[q] = f4{0.f, 0.f, 0.f, 0.f};

  const int step = kTT * nhalf;
  const int p_first = pb + kTT * half;
  KeyWords kw;
  Rows8 vr;
  int32_t pg_cur = load_pages(p_first);
  if (p_first < pe) {  // uniform
    load_key_words(p_first, pg_cur, kw);
    vr = load_ring_values(p_first);
  }
  int32_t pg_next = load_pages(p_first + step);

  // PV operand reads: lane s of a 16-lane group addresses value row base + s / 4,
  // dims 16q + 4 (s % 4) .. + 3, so that lane n receives V[base + k][16q + n]
  const int tr_row = n >> 2;
  const int tr_chunk = (n & 3) >> 1;
  const int tr_half = 8 * (n & 1);

  for (int p0 = p_first; p0 < pe; p0 += step) {
    // wave-uniform (scalar registers: the branches on them are scalar branches)
    const int nt = __builtin_amdgcn_readfirstlane((pe - p0) < kTT ? (pe - p0) : kTT);
    const int mk = __builtin_amdgcn_readfirstlane(count(p0, khist));
    const int mv = __builtin_amdgcn_readfirstlane(count(p0, vhist));
    const int p1 = p0 + step;
    // the ring key rows, in flight while the int4 keys are staged
    const Rows8 kr = load_ring_keys(p0);
    // one wave: its LDS accesses take effect in program order, so the previous
    // sub-tile's reads are done before these writes
    // ---- key rows: int4 rows [0, mk) as hi and lo parts, ring rows [mk, nt)
    // as they are (their lo parts zero, read only when the sub-tile has int4 rows)
    if (mk > 0) {
      // words realigned to the sub-tile (word k: positions p0 + 8k .. + 7), so
      // that row t = 8k + j is nibble j of word k and no row needs a test:
      // rows past mk are overwritten by the ring rows below or masked
      const int sh = 4 * (p0 & 7);
      // rows from tb on fall in the next key group (g >= 32: at most one boundary)
      const int tb = (((p0 >> gsh) + 1) << gsh) - p0;
#pragma unroll
      for (int k = 0; k < kTT / 8; ++k) {
        const uint32_t a0 = __builtin_amdgcn_alignbit(kw.w[0][k + 1], kw.w[0][k], sh);
        const uint32_t a1 = __builtin_amdgcn_alignbit(kw.w[1][k + 1], kw.w[1][k], sh);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int t = 8 * k + j;
          const bool gb = t >= tb;  // selects, not an index: registers
          const float x0 = kivi_dequant((a0 >> (4 * j)) & 0xfu, gb ? kw.sc[0][1] : kw.sc[0][0],
                                        gb ? kw.mn[0][1] : kw.mn[0][0]);
          const float x1 = kivi_dequant((a1 >> (4 * j)) & 0xfu, gb ? kw.sc[1][1] : kw.sc[1][0],
                                        gb ? kw.mn[1][1] : kw.mn[1][0]);
          const uint32_t hi = pack2<T>(x0, x1);
          *reinterpret_cast<uint32_t*>(sk + t * kKP + c0) = hi;
          *reinterpret_cast<uint32_t*>(skl + t * kKP + c0) =
              pack2<T>(x0 - half_f32<T>(hi, 0), x1 - half_f32<T>(hi, 1));
        }
      }
    }
    const bool ring0 = n >= mk && n < nt;            // row n is a ring key
    const bool ring1 = 16 + n >= mk && 16 + n < nt;  // row 16 + n
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int o = (16 * (i >> 2) + n) * kKP + 32 * (i & 3) + 8 * kg;
      if (i < 4 ? ring0 : ring1) *reinterpret_cast<w4*>(sk + o) = kr.r[i];
    }
    if (mk > 0) {  // uniform
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int o = (16 * (i >> 2) + n) * kKP + 32 * (i & 3) + 8 * kg;
        if (i < 4 ? ring0 : ring1) *reinterpret_cast<w4*>(skl + o) = w4{0, 0, 0, 0};
      }
    }
    // ---- scores: S^T[token][head] for kTT/16 x 16 tokens ------------------------
    f4 sacc[kTT / 16];
    // the key lo parts exist only for int4 keys: one uniform branch for the block
    auto scores = [&](auto with_lo) {
#pragma unroll
      for (int jm = 0; jm < kTT / 16; ++jm) {
        sacc[jm] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
          const int o = (16 * jm + n) * kKP + 32 * s4 + 8 * kg;
          const u8v a = *reinterpret_cast<const u8v*>(sk + o);
          sacc[jm] = mfma16(a, qb[s4], sacc[jm], T{});
          if constexpr (decltype(with_lo)::value) {
            const u8v al = *reinterpret_cast<const u8v*>(skl + o);
            sacc[jm] = mfma16(al, qb[s4], sacc[jm], T{});
          }
        }
      }
    };
    if (mk > 0)
      scores(std::true_type{});
    else
      scores(std::false_type{});
    if (p1 < pe) load_key_words(p1, pg_next, kw);  // uniform: the next sub-tile's int4 keys
    float tmax = -INFINITY;
#pragma unroll
    for (int jm = 0; jm < kTT / 16; ++jm) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int pos = p0 + 16 * jm + 4 * kg + r;
        const float sv_ = pos < pe ? sacc[jm][r] * qscale : -INFINITY;
        sacc[jm][r] = sv_;
        tmax = fmaxf(tmax, sv_);
      }
    }
    tmax = max_kg(tmax);
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = m_run == -INFINITY ? 0.0f : exp2f(m_run - m_new);
    float psum = 0.0f;
#pragma unroll
    for (int jm = 0; jm < kTT / 16; ++jm) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pr = exp2f(sacc[jm][r] - m_new);
        sacc[jm][r] = pr;
        psum += pr;
      }
    }
    l_run = l_run * alpha + sum_kg(psum);
    m_run = m_new;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float ar = __shfl(alpha, 4 * kg + r, 64);
#pragma unroll
      for (int q = 0; q < 8; ++q) o_acc[q][r] *= ar;
    }

    // ---- value rows into LDS (over the consumed key rows) -----------------------
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int pi = kg + 4 * k;
      // positions past the item: p = 0 there, and zero V keeps 0 * V exact
      const w4 x = pi < nt ? vr.r[k] : w4{0, 0, 0, 0};
      *reinterpret_cast<w4*>(sv + pi * (2 * D) + 16 * (n ^ (2 * (pi & 3)))) = x;
    }
    if (mv > 0) {  // uniform: int4 values (rare), loaded and dequantized over their rows
#pragma unroll 1
      for (int k = 0; k < 8; ++k) {
        const int pi = kg + 4 * k;
        const int64_t blk = page_of(pg_cur, p0, p0 + (pi < mv ? pi : 0));
        if (pi < mv) {
          const int p = p0 + pi;
          const int64_t vrow = ((blk << bsh) + (p & (bs - 1))) * kvh + h;
          const uint32_t w = vq[vrow * (D / 8) + n];
          const float sc = vs[vrow * (D >> gsh) + ((8 * n) >> gsh)];
          const float mn = vm[vrow * (D >> gsh) + ((8 * n) >> gsh)];
          uint32_t q[4];
#pragma unroll
          for (int i = 0; i < 4; ++i)
            q[i] = pack2<T>(kivi_dequant((w >> (8 * i)) & 0xfu, sc, mn),
                            kivi_dequant((w >> (8 * i + 4)) & 0xfu, sc, mn));
          *reinterpret_cast<w4*>(sv + pi * (2 * D) + 16 * (n ^ (2 * (pi & 3)))) =
              w4{q[0], q[1], q[2], q[3]};
        }
      }
    }

    // ---- O += P V: slot i of lane group kg is token 32*st + 16*(i/4) + 4*kg + i%4
#pragma unroll
    for (int st = 0; st < kTT / 32; ++st) {
      u8v ahi, alo;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float p = sacc[2 * st + i / 4][i % 4];
        const float hi = to_f32(from_f32<T>(p));
        ahi[i] = bits_of<T>(p);
        alo[i] = bits_of<T>(p - hi);
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        v4s part[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int r = 32 * st + 16 * hh + 4 * kg + tr_row;
          const int pos = (2 * q + tr_chunk) ^ (2 * tr_row);
          part[hh] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_v4s_ptr)(sv + r * (2 * D) + 16 * pos + tr_half));
        }
        const u8v bv = {static_cast<uint16_t>(part[0][0]), static_cast<uint16_t>(part[0][1]),
                        static_cast<uint16_t>(part[0][2]), static_cast<uint16_t>(part[0][3]),
                        static_cast<uint16_t>(part[1][0]), static_cast<uint16_t>(part[1][1]),
                        static_cast<uint16_t>(part[1][2]), static_cast<uint16_t>(part[1][3])};
        o_acc[q] = mfma16(ahi, bv, o_acc[q], T{});
        o_acc[q] = mfma16(alo, bv, o_acc[q], T{});
      }
    }
    // the next sub-tile's values, then the block-table rows of the one after
    if (p1 < pe) vr = load_ring_values(p1);
    pg_cur = pg_next;
    pg_next = load_pages(p1 + step);
  }

  Partial res;
#pragma unroll
  for (int q = 0; q < 8; ++q) res.o[q] = o_acc[q];
  res.m = m_run;
  res.l = l_run;
  return res;
}

// Writes a tail partial for heads 0..rep-1 of kv head h's group: o[q][r] is
// O[head 4*kg + r][dim 16*q + n].
__device__ __forceinline__ void tail_store(const Partial& p, int wi, int hq, int h, int rep,
                                           int lane, float* __restrict__ ws_o,
                                           float* __restrict__ ws_ml) {
  const int n = lane & 15;
  const int kg = lane >> 4;
  const int64_t head0 = static_cast<int64_t>(wi) * hq + h * rep;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int hh = 4 * kg + r;
    if (hh < rep) {
#pragma unroll
      for (int q = 0; q < 8; ++q) ws_o[(head0 + hh) * kD + 16 * q + n] = p.o[q][r];
    }
  }
  if (kg == 0 && n < rep) {
    ws_ml[2 * (head0 + n)] = p.m;
    ws_ml[2 * (head0 + n) + 1] = p.l;
  }
}

}  // namespace tail
}  // namespace kvq
