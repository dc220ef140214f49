// SPDX-License-Identifier: Apache-2.0
// The int4 tile of the MFMA decode for 64-token tiles (key groups of 64 or
// more): codes reach the MFMA operands through transposing LDS reads.
//
// ds_read_b64_tr_b4 (gfx950): within each 16-lane group, lane n receives
// nibble n of the 8-byte runs the group's 16 lanes address -- nibble k of its
// result from lane k's run, a 16 x 16 nibble transpose done by the read.
// (Pinned on the device by kvq_selftest_tr4.)
//   * A key run is 16 tokens of one dim.  The 16 lanes of a group name 16
//     dims, so lane n gets 16 dims of token n: two k-steps of the score MFMA
//     S^T = K * Q' (row = token, k = dim), with no lane shuffle and no
//     per-code select.
//   * A value run is 16 dims of one token.  The lanes name 16 tokens, so lane
//     n gets dim n of each: two k-steps of the PV operand (k = token,
//     column = dim).
// One dword of a result (8 codes) becomes four fp16 pairs, each one
// v_and_or_b32 against the 1024 magic, after one shift for the upper two:
//     slot i   0  1  2   3   4  5  6   7
//     nibble   0  4  1'  5'  2  6  3'  7'     (' = read in place as 16c)
// Primed slots (i & 2) hold 1024 + 16c, the others 1024 + c; the other
// operand of the MFMA carries 1/16 at the primed slots.  The offset:
//   keys    the unprimed pairs drop it with one packed subtract (exact c); the
//           primed pairs keep it, and the group's constant
//           sum_primed 1024 * Q'/16 = 64 * sum_primed Q' leaves the scores in
//           fp32 (its ratio to the signal is 64/c, small enough for the fp32
//           accumulation);
//   values  all slots keep it; a constant-B MFMA (1024 in every slot) over the
//           same P' removes it (1024 * P' and 64 * P' at the primed slots).
#pragma once

#include <type_traits>

#include "kvq_common.h"

namespace kvq {
namespace tr {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i* lds_v2i_ptr;

constexpr uint32_t kMagic = 0x64006400u;  // fp16 1024.0 in both halves

// nibble of slot i: 4*(i & 1) + (i >> 1)
__host__ __device__ constexpr int slot_nib(int i) { return 4 * (i & 1) + (i >> 1); }
__host__ __device__ constexpr bool slot_primed(int i) { return (i & 2) != 0; }

__device__ __forceinline__ h8 as_h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  u4v v = {a, b, c, d};
  return __builtin_bit_cast(h8, v);
}

// The three constants of the conversion, held in VGPRs: v_and_or_b32 is a
// VOP3 instruction, which on gfx950 takes no literal and at most one scalar
// operand, so with the constants as literals the compiler splits each pair
// into v_and_b32 + v_or_b32.  (The empty asm only hides the values; the
// and/or itself stays ordinary code, so the compiler's hazard tracking sees
// every VALU write that feeds an MFMA operand.)
struct Consts {
  uint32_t magic, lo, hi;
  __device__ __forceinline__ Consts() : magic(kMagic), lo(0x000f000fu), hi(0x00f000f0u) {
    asm volatile("" : "+v"(magic), "+v"(lo), "+v"(hi));
  }
};

__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
  return (a & m) | o;
}

// The eight fp16 slots of the 8 codes in w (the slot table above).
__device__ __forceinline__ h8 codes(uint32_t w, const Consts& c) {
  const uint32_t w8 = w >> 8;
  return as_h8(and_or(w, c.lo, c.magic), and_or(w, c.hi, c.magic), and_or(w8, c.lo, c.magic),
               and_or(w8, c.hi, c.magic));
}
// ... with the 1024 removed from the unprimed slots (pairs 0 and 2)
__device__ __forceinline__ h8 key_codes(uint32_t w, const Consts& c) {
  const uint32_t w8 = w >> 8;
  const h2 off = h2{1024.0f16, 1024.0f16};
  const uint32_t p0 =
      __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, and_or(w, c.lo, c.magic)) - off);
  const uint32_t p2 =
      __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, and_or(w8, c.lo, c.magic)) - off);
  return as_h8(p0, and_or(w, c.hi, c.magic), p2, and_or(w8, c.hi, c.magic));
}

__device__ __forceinline__ uint32_t lds_off(const void* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)(p)));
}
__device__ __forceinline__ v2i read_tr4(uint32_t off) {
  return __builtin_amdgcn_ds_read_tr4_b64_v2i32((lds_v2i_ptr)(uintptr_t)(off));
}

// Tile layout in 32-bit words (a wave's buffer is 64-byte aligned).
//   KW  key words in 16-byte slots: dim d's 32-token half h (two 16-token
//       runs) at slot 2d + (h ^ ((d >> 2) & 1)).  A score read names 16
//       consecutive dims at one run offset; the xor puts them on 8 different
//       16-byte bank offsets.
//   KS, KM  the key group's scale and minimum per dim, dim order.
//   VW  value words: token t's 16-byte chunk c at slot 4t + (c ^ pi(t)),
//       pi(t) = ((t >> 4) & 3) ^ ((t >> 1) & 1); a PV read names the 16
//       tokens of a lane group (t = 16 jm + 4 g + r), which pi spreads over 8
//       bank offsets.
//   VS, VM  [vg][s][g][i]: scale / min of value group vg of token
//       tau(g, 8 s + slot_nib(i)), the token of PV slot i in k-step s for
//       lane group g (tau(g, j) = 16 (j >> 2) + 4 g + (j & 3)).
template <int NVG, bool KSV>
struct Tile {
  static constexpr int D = 128;
  static constexpr int GT = 64;
  static constexpr int KW = 0;
  static constexpr int KS = KW + 1024;
  static constexpr int KM = KS + 128;
  static constexpr int VW = KM + 128;
  static constexpr int VS = VW + 1024;
  static constexpr int VM = VS + 64 * NVG;
  static constexpr int WORDS = VM + 64 * NVG;
  static constexpr int BYTES = 4 * WORDS;
  static_assert(BYTES % 64 == 0 && (4 * VW) % 64 == 0, "swizzle alignment");
  // DMA instructions per tile (the waits count them)
  static constexpr int KW_INST = 4;                  // 16-byte lanes
  static constexpr int VW_INST = 4;                  // 16-byte lanes
  static constexpr int KS_DMA = KSV ? 1 : 4;         // scale + min
  static constexpr int VS_DMA = 2 * NVG;             // 4-byte lanes, scale + min
  static constexpr int NINST = KW_INST + VW_INST + KS_DMA + VS_DMA;
  static constexpr int NINST_CONT = NINST - KS_DMA;  // same key group as the previous tile
  static_assert(NINST < 64, "vmcnt range");
};

__device__ __forceinline__ int tau(int g, int j) { return 16 * (j >> 2) + 4 * g + (j & 3); }

// Lane parts of the DMA byte offsets (the instruction parts are uniform).
struct LaneDma {
  uint32_t k;   // key words: dim (lane >> 1) of the instruction's 32, half
                // (lane & 1) ^ ((lane >> 3) & 1)
  uint32_t v;   // value words: token (lane >> 2) of the instruction's 16 (row part)
  uint32_t vc;  // value words: chunk (lane & 3) ^ ((lane >> 3) & 1), before the
                // instruction's xor
  uint32_t ks;  // key scales
  uint32_t vs;  // value scales: token of entry `lane`
};

__device__ __forceinline__ LaneDma lane_dma(int lane, int wpd, int kvh, int gpb, int ng, bool ksv) {
  LaneDma ld;
  ld.k = static_cast<uint32_t>(4 * ((lane >> 1) * wpd + 4 * ((lane & 1) ^ ((lane >> 3) & 1))));
  ld.v = static_cast<uint32_t>(4 * ((lane >> 2) * kvh * 16));
  ld.vc = static_cast<uint32_t>((lane & 3) ^ ((lane >> 3) & 1));
  ld.ks = static_cast<uint32_t>(ksv ? 16 * (lane & 31) : 4 * lane * gpb);
  const int s = lane >> 5, g = (lane >> 3) & 3, i = lane & 7;
  ld.vs = static_cast<uint32_t>(4 * tau(g, 8 * s + slot_nib(i)) * kvh * ng);
  return ld;
}

// DMA of one tile into `buf`.  kq_t, ks_t, km_t: the tile's first key word /
// scale of its page row (kv head h, dim 0); vq_t, vs_t, vm_t: the tile's first
// token's value word / scale of head h.  Every address stays inside the
// tile's rows of its page.
template <int NVG, bool KSV>
__device__ __forceinline__ void issue_tile(char* buf, const LaneDma& ld, const uint32_t* kq_t,
                                           int wpd, const float* ks_t, const float* km_t,
                                           int gpb, const uint32_t* vq_t, int kvh,
                                           const float* vs_t, const float* vm_t, bool with_ks) {
  using T = Tile<NVG, KSV>;
  const char* kb = reinterpret_cast<const char*>(kq_t);
#pragma unroll
  for (int i = 0; i < T::KW_INST; ++i)
    dma16(kb + 4 * (32 * i * wpd) + ld.k, buf + 4 * T::KW + 1024 * i);
  if (with_ks) {  // uniform
    const char* sb = reinterpret_cast<const char*>(ks_t);
    const char* mb = reinterpret_cast<const char*>(km_t);
    if constexpr (KSV) {
      // KM follows KS: lanes 32..63 (the minima) land right after the scales
      dma16((threadIdx.x & 32 ? mb : sb) + ld.ks, buf + 4 * T::KS);
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        dma4(sb + 4 * 64 * i * gpb + ld.ks, buf + 4 * (T::KS + 64 * i));
        dma4(mb + 4 * 64 * i * gpb + ld.ks, buf + 4 * (T::KM + 64 * i));
      }
    }
  }
  const char* vb = reinterpret_cast<const char*>(vq_t);
#pragma unroll
  for (int i = 0; i < T::VW_INST; ++i)
    dma16(vb + 4 * (16 * i * kvh * 16) + ld.v + 16 * (ld.vc ^ static_cast<uint32_t>(i)),
          buf + 4 * T::VW + 1024 * i);
  const char* vsb = reinterpret_cast<const char*>(vs_t);
  const char* vmb = reinterpret_cast<const char*>(vm_t);
#pragma unroll
  for (int vg = 0; vg < NVG; ++vg) {
    dma4(vsb + 4 * vg + ld.vs, buf + 4 * (T::VS + 64 * vg));
    dma4(vmb + 4 * vg + ld.vs, buf + 4 * (T::VM + 64 * vg));
  }
}

// The lane's query values: head n of the GQA group (n & 7 when folded),
// dims 64 P + 16 kg + 8 e + slot_nib(i) in k-step s = 2 P + e, slot i, with
// the primed slots scaled by 1/16 (exact).  16-bit inputs stay packed as slot
// pairs (16 VGPRs instead of 32 across the item) and widen where a key group
// is prepared; bf16 pairs are pre-scaled (a bf16 exponent change is exact),
// fp16 pairs scale in the widening fma.  Lanes past the group hold 0.
template <typename TQ>
struct QLane {
  uint32_t w[4][4];  // pair p of k-step s: slots 2p (low half) and 2p + 1
  __device__ __forceinline__ f2 get(int s, int p) const;
};
template <>
__device__ __forceinline__ f2 QLane<bf16>::get(int s, int p) const {
  float lo, hi;
  asm volatile("v_lshlrev_b32 %0, 16, %1" : "=v"(lo) : "v"(w[s][p]));
  asm volatile("v_and_b32 %0, 0xffff0000, %1" : "=v"(hi) : "v"(w[s][p]));
  return f2{lo, hi};
}
template <>
__device__ __forceinline__ f2 QLane<f16>::get(int s, int p) const {
  // fp16 -> fp32 times 1 or 1/16, exact: x * c + 0 in the mixed-precision fma
  const float c = (p & 1) ? 0.0625f : 1.0f;
  float lo, hi;
  asm volatile("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "=v"(lo) : "v"(w[s][p]), "v"(c));
  asm volatile("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
               : "=v"(hi)
               : "v"(w[s][p]), "v"(c));
  return f2{lo, hi};
}
template <>
struct QLane<float> {
  float q[4][8];
  __device__ __forceinline__ f2 get(int s, int p) const { return f2{q[s][2 * p], q[s][2 * p + 1]}; }
};

template <typename TQ>
__device__ __forceinline__ uint16_t bits16(TQ x) {
  return __builtin_bit_cast(uint16_t, x);
}

template <typename TQ>
__device__ __forceinline__ QLane<TQ> load_q(const TQ* __restrict__ query, int b, int hq, int h,
                                            int rep, int n, int kg, bool fold) {
  QLane<TQ> ql;
  const int hn = fold ? (n & 7) : n;
  const bool live = hn < rep;
  const TQ* qrow = query + (static_cast<int64_t>(b) * hq + h * rep + (live ? hn : 0)) * 128;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    float x[8];
    load8(qrow + 64 * (s >> 1) + 16 * kg + 8 * (s & 1), x);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      float a = live ? x[slot_nib(2 * p)] : 0.0f;
      float c = live ? x[slot_nib(2 * p + 1)] : 0.0f;
      if constexpr (std::is_same<TQ, float>::value) {
        ql.q[s][2 * p] = (p & 1) ? a * 0.0625f : a;
        ql.q[s][2 * p + 1] = (p & 1) ? c * 0.0625f : c;
      } else {
        if constexpr (std::is_same<TQ, bf16>::value) {
          if (p & 1) {  // exact: the widened input times a power of two
            a *= 0.0625f;
            c *= 0.0625f;
          }
        }
        ql.w[s][p] = static_cast<uint32_t>(bits16(from_f32<TQ>(a))) |
                     (static_cast<uint32_t>(bits16(from_f32<TQ>(c))) << 16);
      }
    }
  }
  return ql;
}

// B operands of one key group: Q' = q * key_scale as fp16 hi + lo parts (the
// products stay exact, Q' keeps about 22 bits), and
//   kb = (sum_d q * mn - 64 * sum_primed Q') * qscale
// added to every fp32 score (the key minima, and the primed slots' offset).
// Folded (GQA groups of at most 8 heads): column n < 8 carries head n's hi
// part and column n + 8 its lo part, so one MFMA per k-step gives both, and
// a rotate-by-8 add sums them.
struct QGroup {
  h8 bq[4], bl[4];
  float kb;
};

// x - sel * (fp16 half of `pair`), exact in fp32: sel is 1 or 0.
template <int HALF>
__device__ __forceinline__ float sub_half_sel(float x, uint32_t pair, float nsel) {
  float r;
  if (HALF == 0)
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(pair), "v"(nsel), "v"(x));
  else
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
        : "=v"(r)
        : "v"(pair), "v"(nsel), "v"(x));
  return r;
}

__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{lo, hi}), h2));
}

__device__ __forceinline__ float sum_kg(float v) { return sum_rows4(v); }  // over the 4 lane groups of 16

// x + (x of lane n ^ 8 in the same 16-lane row): v_add_f32 with a DPP
// row_ror:8 operand.
__device__ __forceinline__ float add_ror8(float x) {
  const int y = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, false);
  return x + __int_as_float(y);
}

template <typename TQ, int NVG, bool KSV, bool FOLD>
__device__ __forceinline__ void prepare_group(const uint32_t* W, int n, int kg,
                                              const QLane<TQ>& ql, float qscale, QGroup& qg) {
#pragma clang fp contract(fast)
  using T = Tile<NVG, KSV>;
  const float* ksf = reinterpret_cast<const float*>(W + T::KS);
  const float* kmf = reinterpret_cast<const float*>(W + T::KM);
  // the lane's 32 scales and minima (dims 64 P + 16 kg + 8 e + 0..7), all
  // read before any is used
  f4 sc[4][2], mn[4][2];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int base = 64 * (s >> 1) + 16 * kg + 8 * (s & 1);
    sc[s][0] = *reinterpret_cast<const f4*>(ksf + base);
    sc[s][1] = *reinterpret_cast<const f4*>(ksf + base + 4);
    mn[s][0] = *reinterpret_cast<const f4*>(kmf + base);
    mn[s][1] = *reinterpret_cast<const f4*>(kmf + base + 4);
  }
  // folded: lo lanes (n >= 8) take x - hi, hi lanes x - 0
  const float nsel = (FOLD && n >= 8) ? -1.0f : 0.0f;
  const h2 one2 = h2{1.0f16, 1.0f16};
  // one partial sum per k-step: four short chains instead of one long one
  float kb_u[4], kb_p[4], off[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    kb_u[s] = kb_p[s] = off[s] = 0.0f;
    uint32_t ph[4], pl[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int d0 = slot_nib(2 * p), d1 = slot_nib(2 * p + 1);
      const f2 q = ql.get(s, p);
      const float s0 = sc[s][d0 >> 2][d0 & 3], s1 = sc[s][d1 >> 2][d1 & 3];
      const float m0 = mn[s][d0 >> 2][d0 & 3], m1 = mn[s][d1 >> 2][d1 & 3];
      const float x0 = q[0] * s0;
      const float x1 = q[1] * s1;
      if (p & 1)
        kb_p[s] += q[0] * m0 + q[1] * m1;
      else
        kb_u[s] += q[0] * m0 + q[1] * m1;
      const uint32_t hi = pack_h2(x0, x1);
      if (FOLD) {
        ph[p] = pack_h2(sub_half_sel<0>(x0, hi, nsel), sub_half_sel<1>(x1, hi, nsel));
        if (p & 1) off[s] = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, ph[p]), one2, off[s], false);
      } else {
        ph[p] = hi;
        pl[p] = pack_h2(sub_half_sel<0>(x0, hi, -1.0f), sub_half_sel<1>(x1, hi, -1.0f));
        if (p & 1) {
          off[s] = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, ph[p]), one2, off[s], false);
          off[s] = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, pl[p]), one2, off[s], false);
        }
      }
    }
    qg.bq[s] = as_h8(ph[0], ph[1], ph[2], ph[3]);
    if (!FOLD) qg.bl[s] = as_h8(pl[0], pl[1], pl[2], pl[3]);
  }
  // primed q are q / 16: their minima term is 16 * kb_p
  const float kb = sum_kg((kb_u[0] + kb_u[1]) + (kb_u[2] + kb_u[3]) +
                          16.0f * ((kb_p[0] + kb_p[1]) + (kb_p[2] + kb_p[3])));
  float offs = sum_kg((off[0] + off[1]) + (off[2] + off[3]));
  if (FOLD) offs = add_ror8(offs);  // hi column + lo column of the head
  qg.kb = (kb - 1024.0f * offs) * qscale;
}

// Running state of one wave: softmax max / sum (log2 domain), the PV
// accumulators o_acc[v] (dims 16 v + column), the constant-B MFMA sums that
// remove the 1024 offset (one per value group), and the value-minima term.
template <int NVG>
struct Acc {
  float m_run, l_run;
  f4 o_acc[8];
  f4 c_acc[NVG];
  float bias_v[NVG];
  __device__ __forceinline__ void init() {
    m_run = -INFINITY;
    l_run = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; ++q) o_acc[q] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int v = 0; v < NVG; ++v) {
      c_acc[v] = f4{0.f, 0.f, 0.f, 0.f};
      bias_v[v] = 0.0f;
    }
  }
};

// LDS byte offsets of one lane's transposing reads in a buffer at `buf_off`.
// Key read (k-step pair P, 32-token half h, run jm & 1): the lane names dim
// 64 P + 16 kg + n.  Value read (dims 16 v .. 16 v + 15): the lane names token
// tau(kg, n).
__device__ __forceinline__ uint32_t key_read_base(uint32_t buf_off, int n, int kg) {
  return buf_off + 4 * Tile<1, false>::KW + 32 * (16 * kg + n) + 16 * ((n >> 2) & 1);
}
__device__ __forceinline__ uint32_t val_read_base(uint32_t buf_off, int n, int kg) {
  const int t = tau(kg, n);
  const int pi = ((t >> 4) & 3) ^ ((t >> 1) & 1);
  return buf_off + 4 * Tile<1, false>::VW + 64 * t + 16 * pi;
}

// One tile: scores, softmax update and PV.  FULL: every token < pe.
// Order: all eight key reads, the score MFMAs (the second k-step pair's reads
// land behind the first pair's MFMAs), then all eight value reads, which land
// behind the softmax; the PV MFMAs run k-step outer, so consecutive MFMAs
// write different accumulators.
template <int NVG, bool KSV, bool FOLD, bool FULL>
__device__ __forceinline__ void compute_tile(const uint32_t* W, uint32_t buf_off, int p0, int pe,
                                             int n, int kg, const QGroup& qg, float qscale,
                                             Acc<NVG>& acc) {
#pragma clang fp contract(fast)
  using T = Tile<NVG, KSV>;
  static_assert(Tile<NVG, KSV>::KW == Tile<1, false>::KW && Tile<NVG, KSV>::VW == Tile<1, false>::VW,
                "read bases assume the common word offsets");
  const Consts cst;
  // ---- scores: S^T[token 16 jm + row][head] over k-steps s = 2P + e ----------------
  const uint32_t kbase = key_read_base(buf_off, n, kg);
  v2i rk[2][4];
#pragma unroll
  for (int P = 0; P < 2; ++P)
#pragma unroll
    for (int jm = 0; jm < 4; ++jm)
      rk[P][jm] = read_tr4(((kbase + 2048u * P) ^ (16u * (jm >> 1))) + 8u * (jm & 1));
  f4 sacc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) sacc[j] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int P = 0; P < 2; ++P)
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int jm = 0; jm < 4; ++jm) {
        const h8 a = key_codes(static_cast<uint32_t>(rk[P][jm][e]), cst);
        sacc[jm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qg.bq[2 * P + e], sacc[jm], 0, 0, 0);
        if (!FOLD)
          sacc[jm] =
              __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qg.bl[2 * P + e], sacc[jm], 0, 0, 0);
      }
  // the value reads go out now and land while the softmax runs
  const uint32_t vbase = val_read_base(buf_off, n, kg);
  v2i rv[8];
#pragma unroll
  for (int v = 0; v < 8; ++v) rv[v] = read_tr4((vbase ^ (16u * (v >> 1))) + 8u * (v & 1));
  __builtin_amdgcn_sched_barrier(0);
  if (FOLD) {
#pragma unroll
    for (int jm = 0; jm < 4; ++jm)
#pragma unroll
      for (int r = 0; r < 4; ++r) sacc[jm][r] = add_ror8(sacc[jm][r]);
  }
  // lane (kg, n) holds head n (n & 7 folded) at tokens 16 jm + 4 kg + r
  const float kb = qg.kb;
  float tm[4];
#pragma unroll
  for (int jm = 0; jm < 4; ++jm) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float sv = sacc[jm][r] * qscale + kb;
      if (!FULL) sv = p0 + 16 * jm + 4 * kg + r < pe ? sv : -INFINITY;
      sacc[jm][r] = sv;
    }
    tm[jm] = fmaxf(fmaxf(sacc[jm][0], sacc[jm][1]), fmaxf(sacc[jm][2], sacc[jm][3]));
  }
  float tmax = fmaxf(fmaxf(tm[0], tm[1]), fmaxf(tm[2], tm[3]));
  tmax = max_rows4(tmax);
  const float m_new = fmaxf(acc.m_run, tmax);
  const float alpha = acc.m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(acc.m_run - m_new);
  float ps[4];
#pragma unroll
  for (int jm = 0; jm < 4; ++jm) {
#pragma unroll
    for (int r = 0; r < 4; ++r) sacc[jm][r] = __builtin_amdgcn_exp2f(sacc[jm][r] - m_new);
    ps[jm] = (sacc[jm][0] + sacc[jm][1]) + (sacc[jm][2] + sacc[jm][3]);
  }
  acc.l_run = acc.l_run * alpha + sum_kg((ps[0] + ps[1]) + (ps[2] + ps[3]));
  acc.m_run = m_new;
  // once the running max settles most tiles leave it alone (alpha == 1 on
  // every lane): the rescale is skipped as a whole (multiplying by 1 is exact)
  if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float ar = __shfl(alpha, 4 * kg + r, 64);
#pragma unroll
      for (int q = 0; q < 8; ++q) acc.o_acc[q][r] *= ar;
#pragma unroll
      for (int v = 0; v < NVG; ++v) acc.c_acc[v][r] *= ar;
    }
#pragma unroll
    for (int v = 0; v < NVG; ++v) acc.bias_v[v] *= alpha;
  }
  // ---- PV: O[head][dim 16 v + col] += P'[head][token] * V[token][dim] -------------
  const h8 ones_b = as_h8(kMagic, kMagic, kMagic, kMagic);
  const float* vsf = reinterpret_cast<const float*>(W + T::VS) + 8 * kg;
  const float* vmf = reinterpret_cast<const float*>(W + T::VM) + 8 * kg;
  const h2 sixteenth = h2{0.0625f16, 0.0625f16};
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    // P' of k-step s, value group vg: slot i holds token tau(kg, 8 s + slot_nib(i)),
    // whose p is sacc[2 s + (i & 1)][i >> 1]
    h8 pa[NVG];
#pragma unroll
    for (int vg = 0; vg < NVG; ++vg) {
      const f4 s0 = *reinterpret_cast<const f4*>(vsf + 64 * vg + 32 * s);
      const f4 s1 = *reinterpret_cast<const f4*>(vsf + 64 * vg + 32 * s + 4);
      const f4 m0 = *reinterpret_cast<const f4*>(vmf + 64 * vg + 32 * s);
      const f4 m1 = *reinterpret_cast<const f4*>(vmf + 64 * vg + 32 * s + 4);
      float pp[8], bsum[2] = {0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float p = sacc[2 * s + (i & 1)][i >> 1];
        float sv = i < 4 ? s0[i] : s1[i - 4];
        float mv = i < 4 ? m0[i] : m1[i - 4];
        if (!FULL) {
          // past the range p = 0, but the scale/min bytes are unwritten:
          // select zeros so a stale NaN cannot reach the sums
          const bool live = p0 + tau(kg, 8 * s + slot_nib(i)) < pe;
          sv = live ? sv : 0.0f;
          mv = live ? mv : 0.0f;
        }
        pp[i] = p * sv;
        bsum[i & 1] += p * mv;
      }
      acc.bias_v[vg] += bsum[0] + bsum[1];
      // primed slots (pairs 1 and 3) carry 1/16: their codes read as 16c
      const uint32_t a1 = __builtin_bit_cast(
          uint32_t, __builtin_bit_cast(h2, pack_h2(pp[2], pp[3])) * sixteenth);
      const uint32_t a3 = __builtin_bit_cast(
          uint32_t, __builtin_bit_cast(h2, pack_h2(pp[6], pp[7])) * sixteenth);
      pa[vg] = as_h8(pack_h2(pp[0], pp[1]), a1, pack_h2(pp[4], pp[5]), a3);
    }
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const int vg = NVG == 1 ? 0 : v / 4;
      acc.o_acc[v] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          pa[vg], codes(static_cast<uint32_t>(rv[v][s]), cst), acc.o_acc[v], 0, 0, 0);
    }
#pragma unroll
    for (int vg = 0; vg < NVG; ++vg)
      acc.c_acc[vg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[vg], ones_b, acc.c_acc[vg], 0, 0, 0);
  }
}

// Partial of the item for heads 4 kg + r (rows 8..15 repeat heads 0..7 when
// folded and are not stored): o - offset + minima term.
template <int NVG>
__device__ __forceinline__ void finish(Acc<NVG>& acc, int kg, f4 (&o)[8]) {
#pragma unroll
  for (int v = 0; v < NVG; ++v) acc.bias_v[v] = sum_kg(acc.bias_v[v]);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int hh = 4 * kg + r;
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const int vg = NVG == 1 ? 0 : v / 4;
      const float bv = __shfl(acc.bias_v[vg], hh, 64);
      o[v][r] = acc.o_acc[v][r] - acc.c_acc[vg][r] + bv;
    }
  }
}

// Writes heads 0..rep-1 of kv head h's group: o[v][r] is head 4 kg + r, dim 16 v + n.
__device__ __forceinline__ void store_partial(const f4 (&o)[8], float m, float l, int wi, int hq,
                                              int h, int rep, int n, int kg,
                                              float* __restrict__ ws_o, float* __restrict__ ws_ml) {
  const int64_t head0 = static_cast<int64_t>(wi) * hq + h * rep;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int hh = 4 * kg + r;
    if (hh < rep && hh < 16) {
#pragma unroll
      for (int v = 0; v < 8; ++v) ws_o[(head0 + hh) * 128 + 16 * v + n] = o[v][r];
    }
  }
  if (kg == 0 && n < rep) {
    ws_ml[2 * (head0 + n)] = m;
    ws_ml[2 * (head0 + n) + 1] = l;
  }
}

}  // namespace tr
}  // namespace kvq
