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
//   * then stages V transposed as [dim][token] over the same LDS (the keys are
//     consumed by then) and computes O = P * V with P split into two T parts
//     (hi + lo), so p keeps ~16 bits;
//   * leaves (m, l, o) per head in the split-K workspace for the combine.
// LDS: 2 * kTT * kKP * 2 bytes = 17 KiB, inside the int4 path's 19-20 KiB per wave.
// Two waves may share an item: wave `half` of `nhalf` takes every nhalf-th
// sub-tile, and the halves' partial results merge through LDS (merge_halves).
#pragma once

#include "kvq_common.h"
#include "kvq_decode.h"

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

__device__ __forceinline__ float sum_kg(float v) {  // over the 4 lane groups of 16
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}
__device__ __forceinline__ float max_kg(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  v = fmaxf(v, __shfl_xor(v, 32, 64));
  return v;
}

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
constexpr int kTT = 32;          // positions per sub-tile
constexpr int kKP = kD + 8;      // K row pitch (elements): rows stay 16-byte aligned
constexpr int kVP = kTT + 4;     // V^T row pitch (elements): 8-byte aligned token quads
constexpr int kKW = kTT / 8 + 1;  // key words of one dim covering a sub-tile (8-aligned start)
constexpr int kLdsBytes = 2 * kTT * kKP * 2;
static_assert(kD * kVP <= 2 * kTT * kKP, "V^T fits the key region it reuses");

// Work item wi (kind 1) for kv head h: the partial over sub-tiles half,
// half + nhalf, ... of the item.  lds_raw: at least kLdsBytes, the wave's own.
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
  uint16_t* sk = reinterpret_cast<uint16_t*>(lds_raw);  // [kTT][kKP] key hi parts
  uint16_t* skl = sk + kTT * kKP;                        // [kTT][kKP] key lo parts
  uint16_t* svt = sk;                                    // [D][kVP], after the scores
  const int lane = threadIdx.x & 63;
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

  float m_run = -INFINITY;
  float l_run = 0.0f;
  f4 o_acc[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) o_acc[q] = f4{0.f, 0.f, 0.f, 0.f};

  for (int p0 = pb + kTT * half; p0 < pe; p0 += kTT * nhalf) {
    const int nt = (pe - p0) < kTT ? (pe - p0) : kTT;
    const int mk = khist - p0 < 0 ? 0 : (khist - p0 < nt ? khist - p0 : nt);  // int4 keys
    // one wave: its LDS accesses take effect in program order, so the previous
    // sub-tile's reads are done before these writes
    // ---- K rows -------------------------------------------------------------
    {
      if (mk > 0) {
        // lane: dims 2*lane and 2*lane + 1, the <= kKW words of each covering
        // positions [p0, p0+mk); the two dims of a token go out as one pair
        const int first = p0 & ~7;
        const int c0 = 2 * lane;
        uint32_t w[2][kKW];
        float sc[2][kKW], mn[2][kKW];
#pragma unroll
        for (int k = 0; k < kKW; ++k) {
          // clamped into [p0, p0 + mk): every load is valid and unconditional
          const int p = first + 8 * k;
          const int pp = p < p0 ? p0 : (p < p0 + mk ? p : p0 + mk - 1);
          const int64_t r = (clamp_page(bt, pp, bsh, nb) * kvh + h) * D + c0;
          const int off = pp & (bs - 1);
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            w[e][k] = kq[(r + e) * wpd + (off >> 3)];
            sc[e][k] = ks[(r + e) * gpb + (off >> gsh)];
            mn[e][k] = km[(r + e) * gpb + (off >> gsh)];
          }
        }
#pragma unroll
        for (int k = 0; k < kKW; ++k) {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int t = first + 8 * k + j - p0;
            if (t >= 0 && t < mk) {
              const float x0 = kivi_dequant((w[0][k] >> (4 * j)) & 0xfu, sc[0][k], mn[0][k]);
              const float x1 = kivi_dequant((w[1][k] >> (4 * j)) & 0xfu, sc[1][k], mn[1][k]);
              const uint32_t hi = pack2<T>(x0, x1);
              *reinterpret_cast<uint32_t*>(sk + t * kKP + c0) = hi;
              *reinterpret_cast<uint32_t*>(skl + t * kKP + c0) =
                  pack2<T>(x0 - half_f32<T>(hi, 0), x1 - half_f32<T>(hi, 1));
            }
          }
        }
      }
      // ring keys: task = (position, 16-byte chunk), copied as is; their lo
      // parts are zero and only read when the sub-tile also holds int4 keys
      const int tasks = (nt - mk) * (D / 8);
      for (int t0 = 0; t0 < tasks; t0 += 64 * 4) {
        uint4 x[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int t0k = t0 + 64 * k + lane;
          const int t = t0k < tasks ? t0k : tasks - 1;  // clamped: unconditional load
          const int pi = mk + t / (D / 8);
          const int rl = ring_lane(kfirst + (p0 + pi - khist), ring_len);
          x[k] = *reinterpret_cast<const uint4*>(ring_k + ((ring_row0 + rl) * kvh + h) * D +
                                                 8 * (t % (D / 8)));
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int t = t0 + 64 * k + lane;
          if (t < tasks) {
            const int pi = mk + t / (D / 8);
            *reinterpret_cast<uint4*>(sk + pi * kKP + 8 * (t % (D / 8))) = x[k];
            if (mk > 0)
              *reinterpret_cast<uint4*>(skl + pi * kKP + 8 * (t % (D / 8))) = make_uint4(0, 0, 0, 0);
          }
        }
      }
    }
    // ---- scores: S^T[token][head] for kTT/16 x 16 tokens ------------------------
    f4 sacc[kTT / 16];
#pragma unroll
    for (int jm = 0; jm < kTT / 16; ++jm) {
      sacc[jm] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const int o = (16 * jm + n) * kKP + 32 * s4 + 8 * kg;
        const u8v a = *reinterpret_cast<const u8v*>(sk + o);
        sacc[jm] = mfma16(a, qb[s4], sacc[jm], T{});
        if (mk > 0) {  // uniform: key lo parts exist only for int4 keys
          const u8v al = *reinterpret_cast<const u8v*>(skl + o);
          sacc[jm] = mfma16(al, qb[s4], sacc[jm], T{});
        }
      }
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int jm = 0; jm < kTT / 16; ++jm) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int pos = p0 + 16 * jm + 4 * kg + r;
        const float sv = pos < pe ? sacc[jm][r] * qscale : -INFINITY;
        sacc[jm][r] = sv;
        tmax = fmaxf(tmax, sv);
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

    // ---- V rows, stored transposed ----------------------------------------------
    // lane task = (token pair, 8-dim word): both tokens' 8 values as T pairs
    // (int4 words dequantized, ring rows as they are), then for every dim one
    // 32-bit store of the two tokens, which are adjacent in the [dim][token] rows
    {
      const int mv = vhist - p0 < 0 ? 0 : (vhist - p0 < nt ? vhist - p0 : nt);  // int4 values
      const int nd = D / 8;
      const int tasks = ((nt + 1) / 2) * nd;
      for (int t0 = 0; t0 < tasks; t0 += 64 * 2) {
        uint4 x[2][2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const int t0k = t0 + 64 * k + lane;
          const int t = t0k < tasks ? t0k : tasks - 1;  // clamped: unconditional loads
          const int dv = t % nd;
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            int pi = 2 * (t / nd) + e;
            pi = pi < nt ? pi : nt - 1;  // an odd sub-tile's last pair: zeroed below
            if (pi < mv) {
              const int p = p0 + pi;
              const int64_t vrow =
                  ((clamp_page(bt, p, bsh, nb) << bsh) + (p & (bs - 1))) * kvh + h;
              const uint32_t w = vq[vrow * nd + dv];
              const float sc = vs[vrow * (D >> gsh) + ((8 * dv) >> gsh)];
              const float mn = vm[vrow * (D >> gsh) + ((8 * dv) >> gsh)];
              uint32_t q[4];
#pragma unroll
              for (int i = 0; i < 4; ++i)
                q[i] = pack2<T>(kivi_dequant((w >> (8 * i)) & 0xfu, sc, mn),
                                kivi_dequant((w >> (8 * i + 4)) & 0xfu, sc, mn));
              x[k][e] = make_uint4(q[0], q[1], q[2], q[3]);
            } else {
              const int rl = ring_lane(vfirst + (p0 + pi - vhist), ring_len);
              x[k][e] = *reinterpret_cast<const uint4*>(
                  ring_v + ((ring_row0 + rl) * kvh + h) * D + 8 * dv);
            }
          }
        }
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const int t = t0 + 64 * k + lane;
          if (t < tasks) {
            const int pi0 = 2 * (t / nd);
            const int dv = t % nd;
            const bool past = pi0 + 1 >= nt;
            const uint32_t a[4] = {x[k][0].x, x[k][0].y, x[k][0].z, x[k][0].w};
            const uint32_t b[4] = {x[k][1].x, x[k][1].y, x[k][1].z, x[k][1].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const uint32_t bb = past ? 0u : b[i];
              // dim 8 dv + 2 i: the low halves; dim 8 dv + 2 i + 1: the high halves
              *reinterpret_cast<uint32_t*>(svt + (8 * dv + 2 * i) * kVP + pi0) =
                  __builtin_amdgcn_perm(bb, a[i], 0x05040100u);
              *reinterpret_cast<uint32_t*>(svt + (8 * dv + 2 * i + 1) * kVP + pi0) =
                  __builtin_amdgcn_perm(bb, a[i], 0x07060302u);
            }
          }
        }
      }
      // positions past the item: p = 0 there, and zero V keeps 0 * V exact
      for (int e = lane; e < (kTT - nt) * D; e += 64) {
        const int d = e / (kTT - nt);
        const int pi = nt + e % (kTT - nt);
        svt[d * kVP + pi] = 0;
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
        const uint16_t* vrow = svt + (16 * q + n) * kVP + 32 * st + 4 * kg;
        const u4s v0 = *reinterpret_cast<const u4s*>(vrow);
        const u4s v1 = *reinterpret_cast<const u4s*>(vrow + 16);
        const u8v bv = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
        o_acc[q] = mfma16(ahi, bv, o_acc[q], T{});
        o_acc[q] = mfma16(alo, bv, o_acc[q], T{});
      }
    }
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
