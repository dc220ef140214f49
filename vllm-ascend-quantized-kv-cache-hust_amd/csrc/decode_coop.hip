// SPDX-License-Identifier: Apache-2.0
// Page-streaming KIVI INT4 decode for MI355X (gfx950): two workgroups of four
// waves per piece of the decode plan, one per half of the 8 kv heads (a wave
// per kv head), each streaming whole pages for its heads through a four-slot
// LDS ring.
//
// Why: an int4 page of one request holds, per side, all kv heads' codes and
// scales in a few contiguous runs -- keys [head][dim][128 tokens] (64 KiB),
// values [token][head][128 dims] (64 KiB), and the scale/min regions.  A wave
// per (item, kv head) reads only its head's share: half of each key line per
// 64-token tile, half of each value line (the other half is the next head's),
// and 4 bytes of every 32- or 64-byte value scale row.  Those lines are
// requested again by other waves later, after the XCD's L2 may have dropped
// them (config 3 fetched 1.23x, config 5 1.48x the algorithmic bytes), and
// each wave issues about twice the line requests its bytes need.  Here a
// workgroup streams its half of each page once, every line whole, in four
// stages:
//   K0  key codes of dims 0..63 (4 heads x 64 dims x 64 B = 16 KiB, a
//       contiguous 4 KiB run per head) + their scales / minima;
//   K1  dims 64..127;
//   V0  value codes of tokens 0..63 (64 tokens x 4 heads x 64 B = 16 KiB, a
//       256-byte run of each 512-byte token row) + their scales / minima;
//   V1  tokens 64..127.
// Each wave issues 5 LDS-DMA instructions per stage (16-byte lanes; its head's
// key run, or 16 tokens of the value runs, plus a slice of the scales), 20 a
// stage per workgroup.  Both workgroups of a piece run on one XCD, where the
// two halves of a value line or a value scale line meet in its L2.  The ring
// keeps three stages in flight while one is computed; one barrier per stage
// both publishes the stage and frees the slot the next DMA refills.
//
// Compute per wave (its kv head h, the GQA group's query heads as MFMA
// columns) uses the transposing-read operands of decode_tr.h: scores for the
// page's 128 tokens accumulate over K0 and K1 (S^T = K * Q', k = dim), the
// online softmax runs on 128 tokens after K1, and PV runs over V0 and V1
// (O = P' * V, k = token).
//
// Work: the plan's pieces (kvq_plan_kivi_decode, KVQ_PLAN_PIECES, cut on page
// bounds).  A piece's int4 items (kind 0: positions where both sides are
// int4) stream as one continuous stage sequence, so the ring stays full across
// item bounds; positions of a page outside the item are masked.  Its tail
// items (kind 1, residual-window positions) run afterwards, one wave per kv
// head, through decode_tail.h.  Each item leaves (m, l, o) per query head in
// the split-K workspace for the combine kernel.
//
// The stage DMAs are inline asm, so the compiler's wait-count pass does not
// track them: every wait for a stage is explicit (vector memory operations
// complete in order, so "at most N outstanding" means every DMA issued before
// the last N has landed).  The query loads of an item go out, also as asm,
// right before the DMAs of the item's first stage, so the wait for that stage
// covers them.
#include "decode_tail.h"
#include "decode_tr.h"
#include "kvq_common.h"
#include "kvq_decode.h"

namespace {

using namespace kvq;
using tr::f4;
using tr::h2;
using tr::h8;
using tr::v2i;

constexpr int kKvHeads = 8;  // kv heads of the layer
constexpr int kWaves = 4;    // kv heads per workgroup, one wave each: two workgroups a piece
constexpr int kPage = 128;   // positions per page (block size)
constexpr int kD = 128;      // head size
constexpr int kStages = 4;   // stages per page: K0, K1, V0, V1
constexpr int kSlots = 4;    // LDS ring slots
constexpr int kNI = 5;       // DMA instructions per wave per stage

// LDS ring geometry for key group size G (64 or 128).
template <int G>
struct Ring {
  static constexpr int NG = kD / G;     // value groups per head row
  static constexpr int GPB = kPage / G; // key groups per page
  static constexpr int CODES = 16384;   // code bytes of a stage (both kinds), 4 heads
  // scales + minima of a stage: keys 4 heads x 64 dims x GPB, values 64
  // tokens x 4 heads x NG (equal)
  static constexpr int KS_ONE = 64 * GPB * 4;           // one head's scales (or minima), K stage
  static constexpr int KS_HALF = kWaves * KS_ONE;       // the minima follow all heads' scales
  static constexpr int SCALES = 2 * KS_HALF;            // 2 KiB (G 128) / 4 KiB (G 64)
  static_assert(SCALES == 2 * 64 * kWaves * NG * 4, "key and value stages hold equal scales");
  static constexpr int SLOT = CODES + SCALES;
  static constexpr int BYTES = kSlots * SLOT;           // 72 / 80 KiB: two workgroups a CU
  static constexpr int VS_LANES = SCALES / kWaves / 16;  // 16-byte DMA lanes per wave: 32 / 64
};

// One counted LDS DMA: 16 bytes per active lane from base + voff + IMM (base
// uniform, voff the lane's byte offset) to LDS byte address m0 + IMM + 16 *
// lane (m0 uniform): the instruction offset moves both addresses.  The s_nop
// covers the M0-write hazard.
template <int IMM>
__device__ __forceinline__ void cdma16(const char* base, uint32_t voff, uint32_t m0) {
  static_assert(IMM >= 0 && IMM < 4096, "instruction offset range");
  m0 = __builtin_amdgcn_readfirstlane(m0);
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 offset:%2"
               :
               : "v"(voff), "s"(base), "i"(IMM), "{m0}"(m0)
               : "memory");
}

// 16-byte load into registers, not tracked by the compiler's wait counts.
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u4 cload16(const void* g) {
  u4 r;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(g) : "memory");
  return r;
}

// The plan's tables (pieces, work items, block table) are read-only for the
// kernel's lifetime; read through the constant address space, their uniform
// reads become scalar loads.  As ordinary global reads they would be vector
// loads (the memory-clobbering DMA statements stop the compiler from proving
// them invariant), and the compiler's wait for each would drain every stage
// DMA in flight.
typedef const __attribute__((address_space(4))) int32_t cint32;
__device__ __forceinline__ cint32* as_const(const int32_t* p) { return (cint32*)(p); }

// s_waitcnt vmcnt(N) lgkmcnt(0): at most N vector memory operations of this
// wave in flight, and none of its LDS reads (those of the stage computed last
// are done before the barrier that lets another wave refill their slot).
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (0 << 8));
  asm volatile("" ::: "memory");
}

// The lane's 32 query values (dims 16 kg + 0..15 and 64 + 16 kg + 0..15 of
// query head hn) as four 16-byte loads, in flight until the item's first
// stage has landed.
struct QRaw {
  u4 r[4];
};

template <typename TQ>
__device__ __forceinline__ QRaw issue_q(const TQ* __restrict__ query, int b, int hq, int h,
                                        int rep, int n, int kg, bool fold) {
  static_assert(sizeof(TQ) == 2, "16-bit queries");
  const int hn = fold ? (n & 7) : n;
  const int head = h * rep + (hn < rep ? hn : 0);  // lanes past the group read a valid row
  const TQ* row = query + (static_cast<int64_t>(b) * hq + head) * kD;
  QRaw q;
  q.r[0] = cload16(row + 16 * kg);
  q.r[1] = cload16(row + 16 * kg + 8);
  q.r[2] = cload16(row + 64 + 16 * kg);
  q.r[3] = cload16(row + 64 + 16 * kg + 8);
  return q;
}

// The loaded query as fp32 slot pairs (tr::QLane<float>: k-step s = dims
// 64 (s >> 1) + 16 kg + 8 (s & 1) .. + 7; pair p = slots 2p, 2p + 1 = dims p
// and p + 4), the primed pairs (p odd) times 1/16 (exact), zero for lanes past
// the group.  Unpacked once per item: every key group of every page reuses it.
template <typename TQ>
__device__ __forceinline__ float half_to_f32(uint32_t dword, int half) {
  const uint32_t bits = half ? (dword >> 16) : (dword & 0xffffu);
  if constexpr (std::is_same<TQ, bf16>::value) {
    return __uint_as_float(bits << 16);
  } else {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
  }
}

template <typename TQ>
__device__ __forceinline__ tr::QLane<float> unpack_q(const QRaw& q, bool live) {
  tr::QLane<float> ql;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const u4 v = q.r[s];  // dims 8 s' + 0..7 of the run: dword k = dims 2k, 2k + 1
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      // dim p (dword p >> 1, half p & 1) and dim p + 4 (dword 2 + (p >> 1))
      const float f = (p & 1) ? 0.0625f : 1.0f;
      const float a = half_to_f32<TQ>(v[p >> 1], p & 1) * f;
      const float c = half_to_f32<TQ>(v[2 + (p >> 1)], p & 1) * f;
      ql.q[s][2 * p] = live ? a : 0.0f;
      ql.q[s][2 * p + 1] = live ? c : 0.0f;
    }
  }
  return ql;
}

// B operands of one K stage (dims 64 P .. 64 P + 63; k-steps 2P, 2P + 1 as
// e = 0, 1) for key group grp of the page, and the stage's share of the
// group's minima / offset term (summed over both K stages, then scaled).
struct KHalf {
  h8 bq[2], bl[2];
  float kb;  // sum_d q * mn - 1024 * sum_d Q' over this stage's dims (unscaled)
};

template <int G, bool FOLD, int P>
__device__ __forceinline__ void prepare_half(const float* ksf, const float* kmf, int grp, int n,
                                             int kg, const tr::QLane<float>& ql, KHalf& kh) {
#pragma clang fp contract(fast)
  constexpr int GPB = Ring<G>::GPB;
  // ksf / kmf: [64 dims x GPB] scales / minima of this head and stage
  const float nsel = (FOLD && n >= 8) ? -1.0f : 0.0f;
  const h2 one2 = h2{1.0f16, 1.0f16};
  float kb_u[2], kb_p[2], off[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int s = 2 * P + e;
    const int base = 16 * kg + 8 * e;  // dim within the stage
    float sc[8], mn[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      sc[k] = ksf[(base + k) * GPB + grp];
      mn[k] = kmf[(base + k) * GPB + grp];
    }
    kb_u[e] = kb_p[e] = off[e] = 0.0f;
    uint32_t ph[4], pl[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int d0 = tr::slot_nib(2 * p), d1 = tr::slot_nib(2 * p + 1);
      const tr::f2 q = ql.get(s, p);
      const float x0 = q[0] * sc[d0];
      const float x1 = q[1] * sc[d1];
      float& kbs = (p & 1) ? kb_p[e] : kb_u[e];
      kbs = __builtin_fmaf(q[1], mn[d1], __builtin_fmaf(q[0], mn[d0], kbs));
      const uint32_t hi = tr::pack_h2(x0, x1);
      if (FOLD) {
        ph[p] = tr::pack_h2(tr::sub_half_sel<0>(x0, hi, nsel), tr::sub_half_sel<1>(x1, hi, nsel));
        off[e] = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, ph[p]), one2, off[e], false);
      } else {
        ph[p] = hi;
        pl[p] = tr::pack_h2(tr::sub_half_sel<0>(x0, hi, -1.0f), tr::sub_half_sel<1>(x1, hi, -1.0f));
        off[e] = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, ph[p]), one2, off[e], false);
        off[e] = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, pl[p]), one2, off[e], false);
      }
    }
    kh.bq[e] = tr::as_h8(ph[0], ph[1], ph[2], ph[3]);
    if (!FOLD) kh.bl[e] = tr::as_h8(pl[0], pl[1], pl[2], pl[3]);
  }
  // primed q are q / 16: their minima term is 16 * kb_p
  const float kb = tr::sum_kg((kb_u[0] + kb_u[1]) + 16.0f * (kb_p[0] + kb_p[1]));
  // every code slot holds 1024 + c (primed: 1024 + 16 c against Q' / 16): the
  // MFMA sums carry 1024 * sum Q', removed here rather than per code
  float offs = tr::sum_kg(off[0] + off[1]);
  if (FOLD) offs = tr::add_ror8(offs);  // hi column + lo column of the head
  kh.kb = kb - 1024.0f * offs;
}

// Per-wave running state of the item being computed.
template <int G, bool FOLD>
struct WaveState {
  static constexpr int NG = Ring<G>::NG;
  static constexpr int GPB = Ring<G>::GPB;
  tr::Acc<NG> acc;
  f4 sacc[8];       // scores of the page's 128 tokens (row 4 kg + r of block jm)
  float kb[GPB];    // the page's key-group constants, summed over K0 and K1
};

template <int G, bool FOLD, int P>
__device__ __forceinline__ void key_stage(const char* slot, int w, int n, int kg,
                                          const tr::QLane<float>& ql, WaveState<G, FOLD>& st) {
#pragma clang fp contract(fast)
  constexpr int GPB = Ring<G>::GPB;
  const tr::Consts cst;
  const uint32_t base = tr::lds_off(slot);
  // keys of the workgroup's head w: [dim 0..63][64 B], 16-byte chunk c of dim d
  // at c ^ ((d >> 1) & 3)
  const int d = 16 * kg + n;
  const uint32_t krel = 4096u * w + 64u * d + 16u * ((d >> 1) & 3);
  v2i rk[8];
#pragma unroll
  for (int jm = 0; jm < 8; ++jm)
    rk[jm] = tr::read_tr4(base + (krel ^ (16u * (jm >> 1))) + 8u * (jm & 1));
  // [scales: head x 64 dims x GPB][minima: same]
  const float* ksf = reinterpret_cast<const float*>(slot + Ring<G>::CODES + Ring<G>::KS_ONE * w);
  const float* kmf = ksf + Ring<G>::KS_HALF / 4;
  if (P == 0) {
#pragma unroll
    for (int jm = 0; jm < 8; ++jm) st.sacc[jm] = f4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int grp = 0; grp < GPB; ++grp) {
    KHalf kh;
    prepare_half<G, FOLD, P>(ksf, kmf, grp, n, kg, ql, kh);
    st.kb[grp] = P == 0 ? kh.kb : st.kb[grp] + kh.kb;
    // the token blocks of key group grp: jm in [grp * 8 / GPB, (grp + 1) * 8 / GPB)
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int j = 0; j < 8 / GPB; ++j) {
        const int jm = grp * (8 / GPB) + j;
        const h8 a = tr::codes(static_cast<uint32_t>(rk[jm][e]), cst);
        st.sacc[jm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, kh.bq[e], st.sacc[jm], 0, 0, 0);
        if (!FOLD)
          st.sacc[jm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, kh.bl[e], st.sacc[jm], 0, 0, 0);
      }
  }
}

// Softmax of the page's 128 scores (after K1); qscale > 0.  FULL: every
// position of the page is in [pb, pe), so nothing is masked, the maximum is
// taken on the raw MFMA sums per key group (s = qscale (sum + kb) keeps their
// order) and each score is one fma into the exponent.  Otherwise positions
// outside [pb, pe) are masked.  Leaves p in sacc and updates (m, l),
// rescaling the accumulators.
template <int G, bool FOLD, bool FULL>
__device__ __forceinline__ void page_softmax(int page_pos, int pb, int pe, int kg, float qscale,
                                             WaveState<G, FOLD>& st) {
#pragma clang fp contract(fast)
  constexpr int NG = Ring<G>::NG;
  constexpr int GPB = Ring<G>::GPB;
  constexpr int JPG = 8 / GPB;  // token blocks per key group
  if (FOLD) {
#pragma unroll
    for (int jm = 0; jm < 8; ++jm)
#pragma unroll
      for (int r = 0; r < 4; ++r) st.sacc[jm][r] = tr::add_ror8(st.sacc[jm][r]);
  }
  float tmax = -INFINITY;
  float bias[GPB];  // qscale * kb of each group
#pragma unroll
  for (int grp = 0; grp < GPB; ++grp) bias[grp] = st.kb[grp] * qscale;
  if (FULL) {
#pragma unroll
    for (int grp = 0; grp < GPB; ++grp) {
      float rm = -INFINITY;
#pragma unroll
      for (int j = 0; j < JPG; ++j) {
        const f4& v = st.sacc[grp * JPG + j];
        rm = fmaxf(rm, fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])));
      }
      tmax = fmaxf(tmax, rm * qscale + bias[grp]);
    }
  } else {
#pragma unroll
    for (int jm = 0; jm < 8; ++jm) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int pos = page_pos + 16 * jm + 4 * kg + r;
        const float sv = st.sacc[jm][r] * qscale + bias[jm / JPG];
        st.sacc[jm][r] = pos >= pb && pos < pe ? sv : -INFINITY;
      }
      tmax = fmaxf(tmax, fmaxf(fmaxf(st.sacc[jm][0], st.sacc[jm][1]),
                               fmaxf(st.sacc[jm][2], st.sacc[jm][3])));
    }
  }
  tmax = max_rows4(tmax);
  tr::Acc<NG>& acc = st.acc;
  const float m_new = fmaxf(acc.m_run, tmax);
  // m_new is finite: every page of an item holds at least one of its positions
  const float alpha = acc.m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(acc.m_run - m_new);
  float ps[8];
#pragma unroll
  for (int jm = 0; jm < 8; ++jm) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float x = FULL ? st.sacc[jm][r] * qscale + (bias[jm / JPG] - m_new)
                           : st.sacc[jm][r] - m_new;
      st.sacc[jm][r] = __builtin_amdgcn_exp2f(x);
    }
    ps[jm] = (st.sacc[jm][0] + st.sacc[jm][1]) + (st.sacc[jm][2] + st.sacc[jm][3]);
  }
  const float psum = ((ps[0] + ps[1]) + (ps[2] + ps[3])) + ((ps[4] + ps[5]) + (ps[6] + ps[7]));
  acc.l_run = acc.l_run * alpha + tr::sum_kg(psum);
  acc.m_run = m_new;
  if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float ar = __shfl(alpha, 4 * kg + r, 64);
#pragma unroll
      for (int q = 0; q < 8; ++q) acc.o_acc[q][r] *= ar;
#pragma unroll
      for (int v = 0; v < NG; ++v) acc.c_acc[v][r] *= ar;
    }
#pragma unroll
    for (int v = 0; v < NG; ++v) acc.bias_v[v] *= alpha;
  }
}

// PV over the stage's 64 tokens (U = 0: tokens 0..63 of the page, 1: 64..127).
// FULL: all 64 positions are in [pb, pe).
template <int G, bool FOLD, int U, bool FULL>
__device__ __forceinline__ void value_stage(const char* slot, int w, int n, int kg, int page_pos,
                                            int pb, int pe, WaveState<G, FOLD>& st) {
#pragma clang fp contract(fast)
  constexpr int NG = Ring<G>::NG;
  const tr::Consts cst;
  const uint32_t base = tr::lds_off(slot);
  // values: 256-byte token rows (the workgroup's 4 heads x 64 B); token t's
  // 16-byte chunk q (= 4 head + dim block / 2) at q ^ psi(t), psi(t) = (t & 3) |
  // (((t >> 4) & 3) << 2); lane (kg, n) names token tau(kg, n), whose psi is n,
  // so a lane group's 16 reads land on 16 different chunks of a row
  const int t = tr::tau(kg, n);
  const uint32_t lane_base = base + 256u * t;
  v2i rv[8];
#pragma unroll
  for (int v = 0; v < 8; ++v)
    rv[v] = tr::read_tr4(lane_base + 16u * ((4u * w + (v >> 1)) ^ n) + 8u * (v & 1));
  // value scales / minima: [token 0..63][head 0..3][NG] floats
  const float* vsf = reinterpret_cast<const float*>(slot + Ring<G>::CODES);
  const float* vmf = vsf + 64 * kWaves * NG;
  const h8 ones_b = tr::as_h8(tr::kMagic, tr::kMagic, tr::kMagic, tr::kMagic);
  const h2 sixteenth = h2{0.0625f16, 0.0625f16};
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    h8 pa[NG];
    float bsum[NG];
#pragma unroll
    for (int vg = 0; vg < NG; ++vg) bsum[vg] = 0.0f;
    float pp[NG][8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int tt = tr::tau(kg, 8 * s + tr::slot_nib(i));  // token within the stage
      const float p = st.sacc[4 * U + 2 * s + (i & 1)][i >> 1];
      const bool live = FULL || (page_pos + 64 * U + tt >= pb && page_pos + 64 * U + tt < pe);
#pragma unroll
      for (int vg = 0; vg < NG; ++vg) {
        // past the item p = 0, but the bytes may be unwritten: select zeros so a
        // stale NaN cannot reach the sums
        const float sv0 = vsf[(tt * kWaves + w) * NG + vg];
        const float mv0 = vmf[(tt * kWaves + w) * NG + vg];
        const float sv = live ? sv0 : 0.0f;
        const float mv = live ? mv0 : 0.0f;
        pp[vg][i] = p * sv;
        bsum[vg] += p * mv;
      }
    }
#pragma unroll
    for (int vg = 0; vg < NG; ++vg) {
      st.acc.bias_v[vg] += bsum[vg];
      const uint32_t a1 = __builtin_bit_cast(
          uint32_t, __builtin_bit_cast(h2, tr::pack_h2(pp[vg][2], pp[vg][3])) * sixteenth);
      const uint32_t a3 = __builtin_bit_cast(
          uint32_t, __builtin_bit_cast(h2, tr::pack_h2(pp[vg][6], pp[vg][7])) * sixteenth);
      pa[vg] = tr::as_h8(tr::pack_h2(pp[vg][0], pp[vg][1]), a1, tr::pack_h2(pp[vg][4], pp[vg][5]),
                         a3);
    }
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const int vg = NG == 1 ? 0 : v / 4;
      st.acc.o_acc[v] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          pa[vg], tr::codes(static_cast<uint32_t>(rv[v][s]), cst), st.acc.o_acc[v], 0, 0, 0);
    }
#pragma unroll
    for (int vg = 0; vg < NG; ++vg)
      st.acc.c_acc[vg] =
          __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[vg], ones_b, st.acc.c_acc[vg], 0, 0, 0);
  }
}

// Walks the int4 items of a piece: (item, page, stage) in order, skipping tail
// items.  All fields are workgroup-uniform.  FETCH (the DMA cursor): the
// page's block id is read as the cursor reaches the page, one stage before
// the DMAs that use it, so the read's latency hides behind a stage's compute.
template <bool FETCH>
struct Cursor {
  cint32* work;
  cint32* table;
  int64_t maxb, nb;
  int it, it_end;      // current item, end of the piece
  int b, pb, pe;       // the item's request and positions
  int pg, pg_end;      // current page (absolute page index of the request), end
  int stage;           // 0..3 within the page
  int64_t blk;         // FETCH: block id of page pg, clamped into the cache
  __device__ __forceinline__ void fetch() {
    if (FETCH) {
      const int64_t v = table[static_cast<int64_t>(b) * maxb + pg];
      blk = v < 0 ? 0 : (v >= nb ? nb - 1 : v);  // never leave the cache
    }
  }
  __device__ __forceinline__ bool load_item() {  // first int4 item at or after `it`
    for (; it < it_end; ++it) {
      cint32* w = work + 4 * static_cast<int64_t>(it);
      if (w[3] == 0 && w[2] > w[1]) {
        b = w[0];
        pb = w[1];
        pe = w[2];
        pg = pb / kPage;
        pg_end = (pe + kPage - 1) / kPage;
        stage = 0;
        fetch();
        return true;
      }
    }
    return false;
  }
  __device__ __forceinline__ void advance() {
    if (++stage < kStages) return;
    stage = 0;
    if (++pg < pg_end) {
      fetch();
      return;
    }
    ++it;
    load_item();
  }
  __device__ __forceinline__ void next_page() {
    stage = kStages - 1;
    advance();
  }
  __device__ __forceinline__ bool item_first() const { return stage == 0 && pg == pb / kPage; }
  __device__ __forceinline__ bool item_last() const { return stage == kStages - 1 && pg == pg_end - 1; }
};

template <typename TQ, int G, bool FOLD>
__global__ void __launch_bounds__(64 * kWaves, 2)
kivi_decode_coop_kernel(const TQ* __restrict__ query, int hq, float qscale,
                        const uint32_t* __restrict__ kq, const float* __restrict__ ks,
                        const float* __restrict__ km, const uint32_t* __restrict__ vq,
                        const float* __restrict__ vs, const float* __restrict__ vm, int64_t nb,
                        const int32_t* __restrict__ block_table, int64_t maxb,
                        const int32_t* __restrict__ seq_meta, const int32_t* __restrict__ work,
                        const int32_t* __restrict__ pieces, int64_t num_pieces,
                        const TQ* __restrict__ ring_k, const TQ* __restrict__ ring_v,
                        int ring_len, float* __restrict__ ws_o, float* __restrict__ ws_ml) {
  using R = Ring<G>;
  extern __shared__ __align__(16) char lds_raw[];
  // Workgroup b runs half (b >> 3) & 1 of the kv heads of piece ((b >> 4) << 3)
  // | (b & 7): the two halves of a piece get the same b % 8, which places them
  // on one XCD, where the value scale lines they share meet in its L2.
  const int bx = blockIdx.x;
  const int half = (bx >> 3) & 1;
  const int64_t k = (static_cast<int64_t>(bx >> 4) << 3) | (bx & 7);
  if (k >= num_pieces) return;  // workgroup-uniform
  const int lane0 = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // the wave's head of the half
  const int hb = kWaves * half;                                     // the half's first kv head
  const int h = hb + w;                                             // the wave's kv head
  const int rep = hq / kKvHeads;
  const int wpd = kPage / 8;           // key words per (page, head, dim) row
  cint32* cwork = as_const(work);
  cint32* ctable = as_const(block_table);
  const int it0 = as_const(pieces)[k], it1 = as_const(pieces)[k + 1];
  const uint32_t ring0 = tr::lds_off(lds_raw);
  // Lane-dependent values are derived afresh in every stage from a copy of the
  // lane index the compiler cannot see through: hoisted out of the stage loop,
  // the dozens of per-lane LDS and global offsets would stay live across it and
  // push the stage state out of registers.
  auto fresh_lane = [&]() {
    int ln = lane0;
    asm volatile("" : "+v"(ln));
    return ln;
  };

  // Stage DMAs of wave w (kv head h = hb + w): a uniform base plus lane offsets
  // fixed for the kernel, so a stage costs no vector arithmetic.  The
  // instruction offset moves the global and the LDS address alike.
  //   K stage, instruction i (0..3): dim 16 i + (lane >> 2) of head h's run,
  //     chunk (lane & 3) ^ ((lane >> 3) & 3) of its 64-byte row;
  //   K scales: waves 0, 1 copy the scales of heads hb + 2 w', hb + 2 w' + 1
  //     (w' = w & 1), waves 2, 3 their minima (two runs of 64 GPB floats, 128
  //     GPB floats apart);
  //   V stage, instruction i: token 16 w + 4 i + (lane >> 4) of the stage, the
  //     half's 256 bytes of the token row, chunk (lane & 15) ^ psi(token), psi =
  //     (lane >> 4) | (w << 2) for all four instructions;
  //   V scales: waves 0, 1 copy the scales of tokens 32 w' .. 32 w' + 31 (the
  //     half's 4 NG floats of each), waves 2, 3 their minima.
  constexpr int HALF = R::KS_ONE / 16;  // lanes per head run of K scales: 16 / 32
  static_assert(2 * HALF <= 64 && R::VS_LANES <= 64, "one DMA instruction per scale run");
  constexpr int VARR = 64 * kWaves * R::NG * 4;  // bytes per value scale (or minimum) run
  static_assert(2 * 16 * R::VS_LANES == VARR, "two waves cover each value scale run");
  const uint32_t k_lane = 64u * (lane0 >> 2) + 16u * ((lane0 & 3) ^ ((lane0 >> 3) & 3));
  const uint32_t ks_lane =
      16u * (lane0 % HALF) + (lane0 >= HALF ? static_cast<uint32_t>(2 * R::KS_ONE) : 0u);
  uint32_t v_lane[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = 16 * w + 4 * i + (lane0 >> 4);  // token within the stage
    const int psi = (t & 3) | (((t >> 4) & 3) << 2);
    v_lane[i] = 512u * static_cast<uint32_t>(t) + 256u * static_cast<uint32_t>(half) +
                16u * static_cast<uint32_t>((lane0 & 15) ^ psi);
  }
  const int wp = w & 1;  // K scales: the head pair hb + 2 wp, + 1; V scales: the token half
  // V scales: token 32 wp + lane / NG, its 16-byte part lane % NG
  const uint32_t vs_lane = static_cast<uint32_t>(
      32 * R::NG * (32 * wp + lane0 / R::NG) + 16 * (lane0 % R::NG));
  const float* k_arr = w < 2 ? ks : km;
  const float* v_arr = w < 2 ? vs : vm;
  auto issue_stage = [&](const Cursor<true>& c, int slot) {
    const int64_t blk = c.blk;
    const uint32_t sbase = ring0 + static_cast<uint32_t>(slot * R::SLOT);
    if (c.stage < 2) {  // K0 / K1: head h's dims 64 P .. 64 P + 63
      const int P = c.stage;
      const int64_t row = (blk * kKvHeads + h) * kD + 64 * P;  // (page, head, dim) row
      const char* src = reinterpret_cast<const char*>(kq + row * wpd);
      const uint32_t dst = sbase + 4096u * w;
      cdma16<0>(src, k_lane, dst);
      cdma16<1024>(src, k_lane, dst);
      cdma16<2048>(src, k_lane, dst);
      cdma16<3072>(src, k_lane, dst);
      // scales (or minima) of heads hb + 2 wp, + 1, dims 64 P .. 64 P + 63
      const int64_t srow = ((blk * kKvHeads + hb + 2 * wp) * kD + 64 * P) * R::GPB;
      if (lane0 < 2 * HALF)
        cdma16<0>(reinterpret_cast<const char*>(k_arr + srow), ks_lane,
                  sbase + R::CODES + (w < 2 ? 0u : static_cast<uint32_t>(R::KS_HALF)) +
                      static_cast<uint32_t>(2 * R::KS_ONE * wp));
    } else {  // V0 / V1: tokens 64 U .. 64 U + 63, waves take 16 tokens each
      const int U = c.stage - 2;
      const int64_t tok0 = blk * kPage + 64 * U;  // first token of the stage
      const char* src = reinterpret_cast<const char*>(vq + tok0 * kKvHeads * 16);
      const uint32_t dst = sbase + 4096u * w;
      cdma16<0>(src, v_lane[0], dst);
      cdma16<0>(src, v_lane[1], dst + 1024u);
      cdma16<0>(src, v_lane[2], dst + 2048u);
      cdma16<0>(src, v_lane[3], dst + 3072u);
      // [scale: 64 tok x 4 heads x NG][min: same]: wave w's token half of one run
      if (lane0 < R::VS_LANES)
        cdma16<0>(reinterpret_cast<const char*>(v_arr + (tok0 * kKvHeads + hb) * R::NG),
                  vs_lane,
                  sbase + R::CODES + (w < 2 ? 0u : static_cast<uint32_t>(VARR)) +
                      static_cast<uint32_t>(16 * R::VS_LANES * wp));
    }
  };

  // ---- phase 1: the piece's int4 items, streamed ---------------------------------
  int total = 0;  // stages of the piece
  for (int it = it0; it < it1; ++it) {
    cint32* w = cwork + 4 * static_cast<int64_t>(it);
    if (w[3] == 0 && w[2] > w[1]) total += kStages * ((w[2] + kPage - 1) / kPage - w[1] / kPage);
  }
  if (total > 0) {
    Cursor<true> ic{cwork, ctable, maxb, nb, it0, it1, 0, 0, 0, 0, 0, 0, 0};
    ic.load_item();
    Cursor<false> cc{cwork, ctable, maxb, nb, ic.it, it1, ic.b, ic.pb, ic.pe, ic.pg, ic.pg_end,
                     0, 0};
    QRaw q_next = issue_q<TQ>(query, ic.b, hq, h, rep, lane0 & 15, lane0 >> 4, FOLD);
    for (int j = 0; j < 3 && j < total; ++j) {
      if (j > 0 && ic.item_first())
        q_next = issue_q<TQ>(query, ic.b, hq, h, rep, lane0 & 15, lane0 >> 4, FOLD);
      issue_stage(ic, j);
      ic.advance();
    }
    tr::QLane<float> ql;
    WaveState<G, FOLD> st;
    // Stage i of the piece: wait until it has landed for every wave (the last
    // stages drain the ring), then refill the slot of stage i - 1, which every
    // wave has finished reading, with stage i + 3.  Returns the lane index.
    auto begin_stage = [&](int i) -> int {
      if (i + 2 < total)
        vm_wait<2 * kNI>();
      else if (i + 1 < total)
        vm_wait<kNI>();
      else
        vm_wait<0>();
      __builtin_amdgcn_s_barrier();
      const int ln = fresh_lane();
      if (i + 3 < total) {
        if (ic.item_first()) q_next = issue_q<TQ>(query, ic.b, hq, h, rep, ln & 15, ln >> 4, FOLD);
        issue_stage(ic, (i + 3) & 3);
        ic.advance();
      }
      return ln;
    };
    // every read of a stage's slot precedes the next refill
    auto end_stage = [] { asm volatile("" ::: "memory"); };
    // Pages in order; a page's stage k sits in ring slot k (4 stages a page).
    for (int i0 = 0; i0 < total; i0 += kStages) {
      const int page_pos = cc.pg * kPage;
      const int pb = cc.pb, pe = cc.pe;
      // K0: key dims 0..63
      int ln = begin_stage(i0);
      int n = ln & 15, kg = ln >> 4;
      if (cc.pg == pb / kPage) {
        // the item's query landed with its first stage: only now may the
        // compiler read the registers the untracked loads fill
        asm volatile("" : "+v"(q_next.r[0]), "+v"(q_next.r[1]), "+v"(q_next.r[2]),
                     "+v"(q_next.r[3]));
        ql = unpack_q<TQ>(q_next, (FOLD ? (n & 7) : n) < rep);
        st.acc.init();
      }
      key_stage<G, FOLD, 0>(lds_raw, w, n, kg, ql, st);
      end_stage();
      // K1: dims 64..127, then the page's softmax
      ln = begin_stage(i0 + 1);
      n = ln & 15;
      kg = ln >> 4;
      key_stage<G, FOLD, 1>(lds_raw + R::SLOT, w, n, kg, ql, st);
      if (page_pos >= pb && page_pos + kPage <= pe)  // uniform
        page_softmax<G, FOLD, true>(page_pos, pb, pe, kg, qscale, st);
      else
        page_softmax<G, FOLD, false>(page_pos, pb, pe, kg, qscale, st);
      end_stage();
      // V0: tokens 0..63
      ln = begin_stage(i0 + 2);
      n = ln & 15;
      kg = ln >> 4;
      if (page_pos >= pb && page_pos + 64 <= pe)
        value_stage<G, FOLD, 0, true>(lds_raw + 2 * R::SLOT, w, n, kg, page_pos, pb, pe, st);
      else
        value_stage<G, FOLD, 0, false>(lds_raw + 2 * R::SLOT, w, n, kg, page_pos, pb, pe, st);
      end_stage();
      // V1: tokens 64..127
      ln = begin_stage(i0 + 3);
      n = ln & 15;
      kg = ln >> 4;
      if (page_pos + 64 >= pb && page_pos + kPage <= pe)
        value_stage<G, FOLD, 1, true>(lds_raw + 3 * R::SLOT, w, n, kg, page_pos, pb, pe, st);
      else
        value_stage<G, FOLD, 1, false>(lds_raw + 3 * R::SLOT, w, n, kg, page_pos, pb, pe, st);
      end_stage();
      if (cc.pg == cc.pg_end - 1) {  // the item's last page
        tr::Acc<Ring<G>::NG>& acc = st.acc;
        f4 o[8];
        tr::finish<Ring<G>::NG>(acc, kg, o);
        tr::store_partial(o, acc.m_run, acc.l_run, cc.it, hq, h, rep, n, kg, ws_o, ws_ml);
      }
      cc.next_page();
    }
    __builtin_amdgcn_s_barrier();  // the ring is free: the tail items reuse it
  }

  // ---- phase 2: the piece's tail items, one wave per kv head ----------------------
  char* my_lds = lds_raw + w * tail::kLdsBytes;
  for (int wi = it0; wi < it1; ++wi) {
    const int32_t* wk = work + 4 * static_cast<int64_t>(wi);
    if (wk[3] == 0 && wk[2] > wk[1]) continue;  // int4 items ran above
    tail::Partial tp = tail::tail_item<TQ>(my_lds, query, hq, kKvHeads, qscale, kq, ks, km, vq,
                                           vs, vm, kPage, G, nb, block_table, maxb, seq_meta,
                                           wk, wi, h, ring_k, ring_v, ring_len, 0, 1);
    tail::tail_store(tp, wi, hq, h, rep, lane0, ws_o, ws_ml);
  }
}

}  // namespace

namespace kvq {

bool coop_decode_applies(int q_dtype, int hq, int kvh, int d, int ring_dtype, int bs, int g) {
  return kvh == kKvHeads && d == kD && bs == kPage && (g == 64 || g == 128) &&
         hq % kvh == 0 && hq / kvh <= 16 && tail_path_applies(q_dtype, hq, kvh, d, ring_dtype, bs);
}

int launch_kivi_decode_coop(const void* query, int q_dtype, int hq, int kvh, int d, float qscale,
                            const int32_t* kq, const float* ks, const float* km,
                            const int32_t* vq, const float* vs, const float* vm, int bs, int g,
                            int64_t nb, const int32_t* block_table, int64_t maxb,
                            const int32_t* seq_meta, const int32_t* work, int64_t num_work,
                            const int32_t* pieces, int64_t num_pieces, const void* ring_k,
                            const void* ring_v, int ring_dtype, int ring_len, float* ws_o,
                            float* ws_ml, hipStream_t s, bool* launched) {
  *launched = false;
  if (!pieces || num_pieces <= 0 || !coop_decode_applies(q_dtype, hq, kvh, d, ring_dtype, bs, g))
    return KVQ_OK;
  // the page softmax orders raw scores, which a positive scale keeps
  if (!(qscale > 0.0f) || qscale == INFINITY) return KVQ_OK;
  int64_t lds_max = 0;
  const int lrc = device_lds_max(&lds_max);
  if (lrc != KVQ_OK) return lrc;
  const int ring = g == 64 ? Ring<64>::BYTES : Ring<128>::BYTES;
  static_assert(kWaves * tail::kLdsBytes <= Ring<128>::BYTES, "the tail items fit the ring");
  if (ring > lds_max) return KVQ_OK;  // not this device: the per-wave kernels run
  if (num_pieces > (int64_t{1} << 26)) return KVQ_ERR_INVALID;
  // two workgroups (kv head halves) a piece, in groups of 8 pieces
  const dim3 grid(static_cast<unsigned>(16 * ((num_pieces + 7) / 8)));
  const dim3 block(64 * kWaves);
  const bool fold = hq / kvh <= 8;
  const uint32_t* kqu = reinterpret_cast<const uint32_t*>(kq);
  const uint32_t* vqu = reinterpret_cast<const uint32_t*>(vq);
#define KVQ_LAUNCH_COOP(TQ, G, F)                                                             \
  hipLaunchKernelGGL((kivi_decode_coop_kernel<TQ, G, F>), grid, block, Ring<G>::BYTES, s,      \
                     static_cast<const TQ*>(query), hq, qscale, kqu, ks, km, vqu, vs, vm, nb,  \
                     block_table, maxb, seq_meta, work, pieces, num_pieces,                    \
                     static_cast<const TQ*>(ring_k), static_cast<const TQ*>(ring_v), ring_len, \
                     ws_o, ws_ml)
#define KVQ_LAUNCH_COOP_G(TQ)                                                                 \
  if (g == 64) {                                                                              \
    if (fold) KVQ_LAUNCH_COOP(TQ, 64, true); else KVQ_LAUNCH_COOP(TQ, 64, false);            \
  } else {                                                                                    \
    if (fold) KVQ_LAUNCH_COOP(TQ, 128, true); else KVQ_LAUNCH_COOP(TQ, 128, false);          \
  }
  if (q_dtype == KVQ_DTYPE_BF16) {
    KVQ_LAUNCH_COOP_G(bf16);
  } else {
    KVQ_LAUNCH_COOP_G(f16);
  }
#undef KVQ_LAUNCH_COOP_G
#undef KVQ_LAUNCH_COOP
  KVQ_LAUNCH_CHECK();
  (void)num_work;
  *launched = true;
  return KVQ_OK;
}

}  // namespace kvq
