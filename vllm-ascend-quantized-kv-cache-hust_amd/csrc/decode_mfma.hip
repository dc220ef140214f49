// SPDX-License-Identifier: Apache-2.0
// MFMA decode attention over KIVI int4 pages (kind-0, -2 and -3 work items)
// for gfx950, with the tail (kind-1) items through decode_tail.h.
//
// One wave per (work item, kv head), or per (piece, kv head) walking a piece's
// items.  An int4 item is a range of positions, starting on a multiple of 64,
// whose keys and values are both in int4 pages (kinds 2 / 3: only its even /
// odd 64-position chunks); the wave walks it in "group tiles" of GT = 8*CPG
// tokens (CPG = 8 for G >= 64, 4 for G = 32), each inside one page and one
// key-scale group.
//
// Tiles are double-buffered in the wave's LDS: while tile i is computed, the
// DMA loads of tile i+1 (global_load_lds, 16-byte and 4-byte lanes, written
// straight into LDS without passing through registers) are in flight.  Each
// wave owns its two buffers, so there is no workgroup barrier; a wave waits
// only on its own vector-memory counter.
//
// QK^T (v_mfma_f32_16x16x32_f16, S^T = K * Q'^T):
//   A = key codes, row m = token, 8 head dims per lane.  A key word packs 8
//       tokens of one dim, so a lane reads 8 words (8 dims x 8 tokens of its
//       chunk) and builds each register from one nibble of two words with
//       v_perm_b32 + v_and_or_b32 as the fp16 value 1024 + code, then one
//       packed fp16 subtract leaves the exact code (0..15).
//   B = Q' = q * softmax_scale * log2(e) * key_scale(dim, group), column n =
//       query head of the GQA group, split into two fp16 parts hi + lo
//       (hi = fp16(Q'), lo = fp16(Q' - hi)) and applied with two MFMAs: the
//       products are exact and Q' keeps ~22 bits, so outlier key channels
//       (large key_scale) do not turn fp16 rounding into score error.
//   The per-group key minimum adds sum_d q*mn (fp32) to every score.
// PV (O = P' * V):
//   A = P' = p * value_scale(token, group), fp16, row = query head; the lane
//       already holds the p of its tokens from the QK output layout.
//   B = value codes (1024 + code) built the same way from value words (a word
//       packs 8 dims of one token), column = head dim; MFMA columns are chosen
//       so that all 16 lie in one value group.
//   The 1024 offset again goes through a constant-B MFMA, and sum_t p*mn
//   (value minima) is accumulated in fp32 and added at the end.
// Online softmax in the log2 domain; each work item leaves (m, l, o) per head
// for the log-sum-exp combine.
#include "decode_tail.h"
#include "decode_tr.h"
#include "kvq_common.h"
#include "kvq_decode.h"

namespace {

using namespace kvq;

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));

constexpr uint32_t kMagic = 0x64006400u;  // fp16 1024.0 in both halves
constexpr uint32_t kZeroSel = 0x0c0c0c0cu;

__device__ __forceinline__ h8 as_h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  u4v v = {a, b, c, d};
  return __builtin_bit_cast(h8, v);
}

typedef float f2 __attribute__((ext_vector_type(2)));

// x - (fp16 half of `pair`), exact in fp32: one v_fma_mix_f32 reading the
// half directly (the compiler would convert and subtract in two steps).
template <int HALF>
__device__ __forceinline__ float sub_half(float x, uint32_t pair) {
  float r;
  if (HALF == 0)
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(pair), "v"(x));
  else
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
        : "=v"(r)
        : "v"(pair), "v"(x));
  return r;
}

// (hi, lo) fp16 pairs of x: hi = fp16(x), lo = fp16(x - hi), both round to
// nearest; two lanes per v_cvt_pk_f16_f32.
__device__ __forceinline__ void split_h2(f2 x, uint32_t& hi, uint32_t& lo) {
  hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(x, h2));
  const f2 r = f2{sub_half<0>(x[0], hi), sub_half<1>(x[1], hi)};
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, h2));
}

__device__ __forceinline__ uint32_t h2_bits(_Float16 a, _Float16 b) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, a)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, b)) << 16);
}

// fp16 pair (lo, hi), round to nearest.
__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{lo, hi}), h2));
}

// Selector putting byte u of `lo` in byte 0 and byte u of `hi` in byte 2.
__device__ __forceinline__ uint32_t pair_sel(uint32_t u) {
  return (kZeroSel & 0xff00ff00u) | u | ((4u + u) << 16);
}

// fp16 pair (1024 + nibble j of lo, 1024 + nibble j of hi).
__device__ __forceinline__ uint32_t code_pair(uint32_t lo, uint32_t hi, uint32_t j) {
  uint32_t x = __builtin_amdgcn_perm(hi, lo, pair_sel(j >> 1));
  x >>= (j & 1u) * 4u;
  return (x & 0x000f000fu) | kMagic;
}

// fp16 pair (nibble j of lo, nibble j of hi): the exact codes (1024 + c - 1024).
__device__ __forceinline__ uint32_t code_pair_exact(uint32_t lo, uint32_t hi, uint32_t j) {
  const h2 v = __builtin_bit_cast(h2, code_pair(lo, hi, j)) - h2{1024.0f16, 1024.0f16};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float sum_kg(float v) { return sum_rows4(v); }  // over the 4 lane groups of 16
__device__ __forceinline__ float max_kg(float v) {
  return max_rows4(v);
}

// ---- tile layout -------------------------------------------------------------
// One wave's tile buffer.  Key and value words arrive with 16-byte DMA lanes in
// their page order; the small scale/min regions are gathered with 4-byte lanes
// so that what one lane needs for one MFMA step is 8 consecutive floats:
//   KW [dim][chunk]          key word (dim, 8-token chunk), CPG words per dim
//   VW [token][word]         value words, 16 per token
//   KS, KM [s4][kg][ii]      key scale / min of dim 32*s4 + 4*ii + kg
//   VS, VM [st][v][kg][i]    value scale / min of token tk(st, kg, i), group of v
// A lane reads its 8 key words (dims 4 apart) and 8 value words (tokens 8
// apart) as pairs with ds_read2_b32.  tk(st, kg, i) is the token of PV slot
// 8*kg + i in k-step st: the token whose p the lane already holds from the
// score layout.
// VG1: one value group spans the whole head (G >= 128 at CPG 8), so every PV
// column group shares the token's value scale and min: they are gathered and
// applied once per PV k-step instead of once per column group.
// KSV: the key scales of a group are one contiguous run per head (one group
// per page, bs == g): one 16-byte-lane DMA brings both the scales (lanes
// 0-31) and the minima (lanes 32-63) in dim order, instead of four 4-byte
// gathers in the permuted order prepare_group reads.
template <int CPG, bool VG1 = false, bool KSV = false>
struct Tile {
  static_assert(!VG1 || CPG == 8, "VG1 needs 64-token tiles");
  static constexpr int D = 128;
  static constexpr int GT = 8 * CPG;    // tokens per tile
  static constexpr int NJ = CPG / 2;    // score MFMAs per k-step (16 tokens each)
  static constexpr int SUB = 16 / CPG;  // tokens of one chunk inside one score MFMA
  static constexpr int NVG = 16 / CPG;  // PV column groups (one value group each)
  static constexpr int NJJ = CPG / 2;   // PV MFMAs per column group (NVG * NJJ == 8)
  static constexpr int PVS = CPG / 4;   // PV k-steps (32 tokens) per tile
  static constexpr int NVS = VG1 ? 1 : NVG;  // value scale/min groups per PV k-step
  static constexpr int KW = 0;
  static constexpr int KS = KW + D * CPG;
  static constexpr int KM = KS + D;
  static constexpr int KEY_WORDS = KM + D;  // the key part: a wave's own region
  static constexpr int VW = KEY_WORDS;
  static constexpr int VS = VW + GT * 16;
  static constexpr int VM = VS + PVS * NVS * 32;
  static constexpr int WORDS = VM + PVS * NVS * 32;
  static constexpr int BYTES = 4 * WORDS;
  // DMA instructions per tile; the waits rely on this number
  static constexpr int KW_INST = D * CPG * 4 / 1024;  // 16-byte lanes
  static constexpr int VW_INST = GT * 64 / 1024;      // 16-byte lanes
  static constexpr int KS_INST = D / 64;              // 4-byte lanes (per array)
  static constexpr int KS_DMA = KSV ? 1 : 2 * KS_INST; // key scale + min DMA instructions
  static constexpr int VS_INST = PVS * NVS * 32 / 64; // 4-byte lanes
  static constexpr int NINST = KW_INST + VW_INST + KS_DMA + 2 * VS_INST;
  // a tile that continues the previous tile's key group skips the key
  // scale/min DMA (prepare_group reads them only at a group's first tile)
  static constexpr int NINST_CONT = NINST - KS_DMA;
  static_assert(NINST < 64, "vmcnt range");
};

// tk = tile_token(st, kg, i): the token of PV slot 8*kg + i in k-step st, the
// one whose p the lane already holds from the score layout (score row
// mr = 4*kg + i%4 of MFMA jm = 2*st + i/4 is token 8*(mr % CPG) + jm*SUB +
// mr / CPG).  With i%4 < 4 <= CPG the row splits into a lane part and a
// constant part, so LDS reads at tk take one lane base and immediate offsets.
template <int CPG>
__device__ __forceinline__ int tile_token_lane(int kg) {
  return 8 * ((4 * kg) % CPG) + (4 * kg) / CPG;
}
template <int CPG>
__device__ __forceinline__ constexpr int tile_token_const(int st, int i) {
  return 8 * (i % 4) + (2 * st + i / 4) * (16 / CPG);
}
template <int CPG>
__device__ __forceinline__ int tile_token(int st, int kg, int i) {
  return tile_token_lane<CPG>(kg) + tile_token_const<CPG>(st, i);
}

// Offsets of DMA lane e = 64*i + lane for the gathered scale/min regions.
// Every field of e used below is a bit field and the maps are linear in
// them, so off(64*i + lane) == off(64*i) + off(lane): the lane part is
// computed once per wave, the instruction part folds to a uniform value.
template <int CPG>
__device__ __forceinline__ int key_scale_off(int e, int gpb) {
  const int ii = e % 8, kg = (e / 8) % 4, s4 = e / 32;
  return (32 * s4 + 4 * ii + kg) * gpb;
}
template <int CPG, bool VG1>
__device__ __forceinline__ int value_scale_off(int e, int kvh, int ng, int g) {
  constexpr int NVS = Tile<CPG, VG1>::NVS;
  const int i8 = e % 8, kg = (e / 8) % 4, v = (e / 32) % NVS, st = e / (32 * NVS);
  return tile_token<CPG>(st, kg, i8) * kvh * ng + (8 * CPG * v) / g;
}

struct LaneDma {
  uint32_t k, v, ks, vs;  // byte offsets of this lane's DMA data (lane part)
};

template <int CPG, bool VG1, bool KSV>
__device__ __forceinline__ LaneDma lane_dma(int lane, int wpd, int kvh, int gpb, int ng, int g) {
  constexpr int LPR = CPG / 4;  // 16-byte lanes per key dim row (CPG words)
  LaneDma ld;
  ld.k = static_cast<uint32_t>(4 * ((lane / LPR) * wpd + 4 * (lane % LPR)));
  ld.v = static_cast<uint32_t>(4 * ((lane / 4) * kvh * 16 + 4 * (lane % 4)));
  ld.ks = static_cast<uint32_t>(KSV ? 16 * (lane & 31) : 4 * key_scale_off<CPG>(lane, gpb));
  ld.vs = static_cast<uint32_t>(4 * value_scale_off<CPG, VG1>(lane, kvh, ng, g));
  return ld;
}

// DMA of one tile's key words and key scale/min for kv head h into the
// wave's key region `buf`.  kq_t, ks_t, km_t point at the tile's first word /
// scale (page blk, token offset off0, key group grp); every lane address stays
// inside the tile's rows of that page.
template <int CPG, bool KSV>
__device__ __forceinline__ void issue_keys(char* buf, const LaneDma& ld, const uint32_t* kq_t,
                                           int wpd, const float* ks_t, const float* km_t,
                                           int gpb, bool with_ks) {
  using T = Tile<CPG, false, KSV>;
  constexpr int LPR = CPG / 4;
  constexpr int DPI = 64 / LPR;  // key dim rows per instruction
  const char* kb = reinterpret_cast<const char*>(kq_t);
  const char* sb = reinterpret_cast<const char*>(ks_t);
  const char* mb = reinterpret_cast<const char*>(km_t);
#pragma unroll
  for (int i = 0; i < T::KW_INST; ++i)
    dma16(kb + 4 * (i * DPI * wpd) + ld.k, buf + 4 * T::KW + 1024 * i);
  if (!with_ks) return;  // uniform
  if constexpr (KSV) {
    // KM follows KS in the tile, so lane l lands at KS + 16 l either way
    dma16((threadIdx.x & 32 ? mb : sb) + ld.ks, buf + 4 * T::KS);
    return;
  }
#pragma unroll
  for (int i = 0; i < T::KS_INST; ++i) {
    const int o = 4 * key_scale_off<CPG>(64 * i, gpb);
    dma4(sb + o + ld.ks, buf + 4 * (T::KS + 64 * i));
    dma4(mb + o + ld.ks, buf + 4 * (T::KM + 64 * i));
  }
}

// DMA of one whole tile (keys and the gathered value operands) for kv head h
// into the wave's tile buffer; vq_t, vs_t, vm_t point at the tile's first value
// word / scale of head h.
template <int CPG, bool VG1, bool KSV>
__device__ __forceinline__ void issue_tile(char* buf, const LaneDma& ld, const uint32_t* kq_t,
                                           int wpd, const uint32_t* vq_t, int kvh,
                                           const float* ks_t, const float* km_t, int gpb,
                                           const float* vs_t, const float* vm_t, int ng, int g,
                                           bool with_ks) {
  using T = Tile<CPG, VG1, KSV>;
  issue_keys<CPG, KSV>(buf, ld, kq_t, wpd, ks_t, km_t, gpb, with_ks);
  const char* vb = reinterpret_cast<const char*>(vq_t);
  const char* vsb = reinterpret_cast<const char*>(vs_t);
  const char* vmb = reinterpret_cast<const char*>(vm_t);
#pragma unroll
  for (int i = 0; i < T::VW_INST; ++i)
    dma16(vb + 4 * (16 * i * kvh * 16) + ld.v, buf + 4 * T::VW + 1024 * i);
#pragma unroll
  for (int i = 0; i < T::VS_INST; ++i) {
    const int o = 4 * value_scale_off<CPG, VG1>(64 * i, kvh, ng, g);
    dma4(vsb + o + ld.vs, buf + 4 * (T::VS + 64 * i));
    dma4(vmb + o + ld.vs, buf + 4 * (T::VM + 64 * i));
  }
}

__device__ __forceinline__ void read8(const uint32_t* p, uint32_t (&w)[8]) {
  const uint4 a = *reinterpret_cast<const uint4*>(p);
  const uint4 b = *reinterpret_cast<const uint4*>(p + 4);
  w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
}
__device__ __forceinline__ void read8f(const uint32_t* p, float (&f)[8]) {
  uint32_t w[8];
  read8(p, w);
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = __uint_as_float(w[i]);
}

// The value operands of one tile as the PV step reads them: the wave's
// gathered copy (VW [token][16 words]; VS, VM in PV-slot order, 8 consecutive
// floats per lane and step), resolved to the lane (kg, chunk) once so that
// each read is a base plus an immediate offset.
template <int CPG, bool VG1>
struct WaveValues {
  const uint32_t* vw;  // VW + 16 * tile_token_lane(kg) + chunk
  const uint32_t* sm;  // the tile + 8 * kg
  __device__ __forceinline__ WaveValues(const uint32_t* W, int kg, int chunk)
      : vw(W + Tile<CPG, VG1>::VW + 16 * tile_token_lane<CPG>(kg) + chunk), sm(W + 8 * kg) {}
  __device__ __forceinline__ void scales(int st, int v, float (&sc)[8], float (&mn)[8]) const {
    using T = Tile<CPG, VG1>;
    const int base = (st * T::NVS + (VG1 ? 0 : v)) * 32;
    read8f(sm + T::VS + base, sc);
    read8f(sm + T::VM + base, mn);
  }
  __device__ __forceinline__ void words(int st, int v, uint32_t (&w)[8]) const {
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = vw[16 * tile_token_const<CPG>(st, i) + CPG * v];
  }
};


// fp16 pair of nibbles from two words: byte `sel` of lo and of hi, the nibble
// picked by `mask` (0x000f000f: low nibble -> 1024 + c; 0x00f000f0: high
// nibble -> 1024 + 16c, exact as well).
__device__ __forceinline__ uint32_t nib_pair(uint32_t lo, uint32_t hi, uint32_t sel,
                                             uint32_t mask) {
  return (__builtin_amdgcn_perm(hi, lo, sel) & mask) | kMagic;
}
// ... with the 1024 removed exactly: c or 16c.
__device__ __forceinline__ uint32_t nib_pair_exact(uint32_t lo, uint32_t hi, uint32_t sel,
                                                   uint32_t mask) {
  const h2 v = __builtin_bit_cast(h2, nib_pair(lo, hi, sel, mask)) - h2{1024.0f16, 1024.0f16};
  return __builtin_bit_cast(uint32_t, v);
}

// Per-lane constants of the nibble selection (lanes of odd nibble parity read
// codes as 16c; their score rows / output columns are scaled back by 1/16).
template <int CPG>
struct LaneNib {
  uint32_t selk[CPG / 2];  // byte selectors of the score MFMAs (per jm)
  uint32_t selv[CPG / 2];  // byte selectors of the PV MFMAs (per jj)
  uint32_t maskk, maskv;
  float row_scale;         // score rows held by this lane: 1 or 1/16
  float col_scale;         // output column held by this lane: 1 or 1/16
  __device__ __forceinline__ LaneNib(int n, int kg) {
    constexpr int SUB = 16 / CPG;
    const int sub = n / CPG;
    // (jm*SUB + sub) >> 1 with SUB even: jm*SUB/2 + sub/2 (sub/2 == 0 for CPG 8)
#pragma unroll
    for (int jm = 0; jm < CPG / 2; ++jm) {
      selk[jm] = pair_sel(static_cast<uint32_t>(jm * (SUB / 2) + (sub >> 1)));
      selv[jm] = selk[jm];
    }
    const bool odd = (sub & 1) != 0;  // SUB is even, so the parity is sub's
    maskk = maskv = odd ? 0x00f000f0u : 0x000f000fu;
    const int row_sub = (4 * kg) / CPG;  // score rows 4*kg + r all share it
    row_scale = (row_sub & 1) ? 0.0625f : 1.0f;
    col_scale = odd ? 0.0625f : 1.0f;
  }
};

// The lane's 32 query values (dims 32*s4 + 4*ii + kg) kept as 16 packed
// pairs for 16-bit inputs (pair 4*s4 + p = elements 2p, 2p+1 of k-step s4).
// The widening is volatile asm: it stays where the values are used (once per
// key group) instead of being hoisted out of the tile loop as 32 live fp32
// registers.
template <typename TQ>
struct QRegs {
  uint32_t w[16];
  __device__ __forceinline__ void set(int i, TQ lo, TQ hi) {
    w[i] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, lo)) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, hi)) << 16);
  }
  __device__ __forceinline__ float lo(int i) const;
  __device__ __forceinline__ float hi(int i) const;
};
template <>
__device__ __forceinline__ float QRegs<bf16>::lo(int i) const {
  float r;
  asm volatile("v_lshlrev_b32 %0, 16, %1" : "=v"(r) : "v"(w[i]));
  return r;
}
template <>
__device__ __forceinline__ float QRegs<bf16>::hi(int i) const {
  float r;
  asm volatile("v_and_b32 %0, 0xffff0000, %1" : "=v"(r) : "v"(w[i]));
  return r;
}
template <>
__device__ __forceinline__ float QRegs<f16>::lo(int i) const {
  float r;  // fp16 -> fp32 is exact: x * 1.0 + 0.0 in the mixed-precision fma
  asm volatile("v_fma_mix_f32 %0, %1, 1.0, 0 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w[i]));
  return r;
}
template <>
__device__ __forceinline__ float QRegs<f16>::hi(int i) const {
  float r;
  asm volatile("v_fma_mix_f32 %0, %1, 1.0, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
               : "=v"(r)
               : "v"(w[i]));
  return r;
}
template <>
struct QRegs<float> {
  float w[32];
  __device__ __forceinline__ void set(int i, float lo, float hi) {
    w[2 * i] = lo;
    w[2 * i + 1] = hi;
  }
  __device__ __forceinline__ float lo(int i) const { return w[2 * i]; }
  __device__ __forceinline__ float hi(int i) const { return w[2 * i + 1]; }
};

// B operands of one key group: Q' = q * key_scale(dim, group) as hi/lo fp16
// pairs for the 4 k-steps, and the minima term kb = sum_d q * mn (times the
// softmax scale).  Shared by the group's tiles (two 64-token tiles at G = 128).
//
// Folded form (GQA groups of at most 8 heads): columns n and n + 8 both carry
// head n % 8, column n < 8 with the hi part and column n + 8 with the lo part
// in bq, so one MFMA per k-step gives both partial scores and a rotate-by-8
// add within each 16-lane row sums them (bl unused).
struct QGroup {
  h8 bq[4], bl[4];
  float kb;
};

template <typename TQ, int CPG, bool FOLD, bool KSV>
__device__ __forceinline__ void prepare_group(const uint32_t* W, int n, int kg,
                                              const QRegs<TQ>& qv, float qscale, QGroup& qg) {
#pragma clang fp contract(fast)
  using T = Tile<CPG>;
  float kb = 0.0f;
#pragma unroll
  for (int s4 = 0; s4 < 4; ++s4) {
    float sc[8], mn[8];
    if constexpr (KSV) {  // dim order: dims 32*s4 + 4*ii + kg, 16 bytes apart
      const float* ksf = reinterpret_cast<const float*>(W + T::KS) + 32 * s4 + kg;
      const float* kmf = reinterpret_cast<const float*>(W + T::KM) + 32 * s4 + kg;
#pragma unroll
      for (int ii = 0; ii < 8; ++ii) {
        sc[ii] = ksf[4 * ii];
        mn[ii] = kmf[4 * ii];
      }
    } else {
      read8f(W + T::KS + (s4 * 4 + kg) * 8, sc);
      read8f(W + T::KM + (s4 * 4 + kg) * 8, mn);
    }
    uint32_t qh[4], ql[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const float q0 = qv.lo(4 * s4 + p);  // exact widening of the input
      const float q1 = qv.hi(4 * s4 + p);
      split_h2(f2{q0 * sc[2 * p], q1 * sc[2 * p + 1]}, qh[p], ql[p]);
      kb += q0 * mn[2 * p] + q1 * mn[2 * p + 1];
    }
    if (FOLD) {
      const bool lo_col = n >= 8;
      qg.bq[s4] = as_h8(lo_col ? ql[0] : qh[0], lo_col ? ql[1] : qh[1], lo_col ? ql[2] : qh[2],
                        lo_col ? ql[3] : qh[3]);
    } else {
      qg.bq[s4] = as_h8(qh[0], qh[1], qh[2], qh[3]);
      qg.bl[s4] = as_h8(ql[0], ql[1], ql[2], ql[3]);
    }
  }
  qg.kb = sum_kg(kb) * qscale;
}

// x + (x of lane n ^ 8 in the same 16-lane row): v_add_f32 with a DPP
// row_ror:8 operand.
__device__ __forceinline__ float add_ror8(float x) {
  const int y = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, false);
  return x + __int_as_float(y);
}

// One tile of scores, softmax update and PV.  FULL: every token < pe.  W is
// the wave's key region; `vals` reads the tile's value operands.
template <typename TQ, int CPG, bool VG1, bool FULL, bool FOLD, typename VALS>
__device__ __forceinline__ void compute_tile(const uint32_t* W, const VALS& vals, int p0, int pe, int n, int kg,
                                             const QGroup& qg, float qscale,
                                             const LaneNib<CPG>& ln, float& m_run, float& l_run, f4 (&o_acc)[8],
                                             f4 (&c_acc)[16 / CPG], float (&bias_v)[16 / CPG]) {
  // attention math is tolerance-checked: let mul+add fuse here (the library
  // builds with -ffp-contract=off for the bit-exact pack/dequant paths)
#pragma clang fp contract(fast)
  using T = Tile<CPG, VG1>;
  const int chunk = n % CPG;
  const h8 ones_b = as_h8(kMagic, kMagic, kMagic, kMagic);
  // ---- scores ----------------------------------------------------------------
  f4 sacc[T::NJ];
#pragma unroll
  for (int j = 0; j < T::NJ; ++j) sacc[j] = f4{0.f, 0.f, 0.f, 0.f};
  // key words of k-step s4: dims 32*s4 + 4*ii + kg of chunk `chunk`, pairs 32
  // words apart; each k-step's words are read while the previous one computes
  uint32_t wkb[2][8];
  auto load_keys = [&](int s4, uint32_t (&w)[8]) {
    const uint32_t* kw = W + T::KW + (32 * s4 + kg) * CPG + chunk;
#pragma unroll
    for (int ii = 0; ii < 8; ++ii) w[ii] = kw[4 * ii * CPG];
  };
  load_keys(0, wkb[0]);
#pragma unroll
  for (int s4 = 0; s4 < 4; ++s4) {
    if (s4 < 3) load_keys(s4 + 1, wkb[(s4 + 1) & 1]);
    const uint32_t(&w)[8] = wkb[s4 & 1];
#pragma unroll
    for (int jm = 0; jm < T::NJ; ++jm) {
      const uint32_t sel = ln.selk[jm];
      const h8 a = as_h8(nib_pair_exact(w[0], w[1], sel, ln.maskk),
                         nib_pair_exact(w[2], w[3], sel, ln.maskk),
                         nib_pair_exact(w[4], w[5], sel, ln.maskk),
                         nib_pair_exact(w[6], w[7], sel, ln.maskk));
      sacc[jm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qg.bq[s4], sacc[jm], 0, 0, 0);
      if (!FOLD)
        sacc[jm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qg.bl[s4], sacc[jm], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the k-steps' live ranges apart
  }
  if (FOLD) {
#pragma unroll
    for (int jm = 0; jm < T::NJ; ++jm)
#pragma unroll
      for (int r = 0; r < 4; ++r) sacc[jm][r] = add_ror8(sacc[jm][r]);
  }
  const float kb = qg.kb;
  // softmax scale * log2(e), and 1/16 on the rows read as 16c
  const float rs = qscale * ln.row_scale;
  // lane holds head n, rows m' = 4*kg + r: token tk = tile_token(jm/2, kg, 4*(jm%2) + r)
  float tmax = -INFINITY;
#pragma unroll
  for (int jm = 0; jm < T::NJ; ++jm) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float sv = sacc[jm][r] * rs + kb;
      if (!FULL) {
        const int pos = p0 + tile_token<CPG>(jm / 2, kg, 4 * (jm % 2) + r);
        sv = pos < pe ? sv : -INFINITY;
      }
      sacc[jm][r] = sv;
      tmax = fmaxf(tmax, sv);
    }
  }
  tmax = max_kg(tmax);
  const float m_new = fmaxf(m_run, tmax);
  const float alpha = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
  float psum = 0.0f;
#pragma unroll
  for (int jm = 0; jm < T::NJ; ++jm) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float pr = __builtin_amdgcn_exp2f(sacc[jm][r] - m_new);  // v_exp_f32
      sacc[jm][r] = pr;
      psum += pr;
    }
  }
  l_run = l_run * alpha + sum_kg(psum);
  m_run = m_new;
  // once the running max settles most tiles leave it alone (alpha == 1 on
  // every lane): the rescale is skipped as a whole (multiplying by 1 is exact)
  if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float ar = __shfl(alpha, 4 * kg + r, 64);
#pragma unroll
      for (int q = 0; q < 8; ++q) o_acc[q][r] *= ar;
#pragma unroll
      for (int v = 0; v < T::NVS; ++v) c_acc[v][r] *= ar;
    }
#pragma unroll
    for (int v = 0; v < T::NVS; ++v) bias_v[v] *= alpha;
  }

  // ---- PV ----------------------------------------------------------------------
#pragma unroll
  for (int st = 0; st < T::PVS; ++st) {
    float pv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) pv[i] = sacc[2 * st + i / 4][i % 4];
    h8 a;  // P' of the k-step for column group v (VG1: for all of them)
#pragma unroll
    for (int v = 0; v < T::NVG; ++v) {
      if (!VG1 || v == 0) {
        float sc[8], mn[8];
        vals.scales(st, v, sc, mn);
        float pp[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float s_ = sc[i], m_ = mn[i];
          if (!FULL) {
            // past the range p = 0, but the scale/min bytes are unwritten:
            // select zeros so a stale NaN cannot reach the sums
            const bool live = p0 + tile_token<CPG>(st, kg, i) < pe;
            s_ = live ? s_ : 0.0f;
            m_ = live ? m_ : 0.0f;
          }
          pp[i] = pv[i] * s_;
          bias_v[v] += pv[i] * m_;
        }
        a = as_h8(pack_h2(pp[0], pp[1]), pack_h2(pp[2], pp[3]), pack_h2(pp[4], pp[5]),
                  pack_h2(pp[6], pp[7]));
        c_acc[v] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ones_b, c_acc[v], 0, 0, 0);
      }
      uint32_t w[8];  // word chunk + CPG*v of tokens tk(st, kg, i)
      vals.words(st, v, w);
#pragma unroll
      for (int jj = 0; jj < T::NJJ; ++jj) {
        const uint32_t sel = ln.selv[jj];
        const h8 bv = as_h8(nib_pair(w[0], w[1], sel, ln.maskv), nib_pair(w[2], w[3], sel, ln.maskv),
                            nib_pair(w[4], w[5], sel, ln.maskv), nib_pair(w[6], w[7], sel, ln.maskv));
        o_acc[v * T::NJJ + jj] =
            __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bv, o_acc[v * T::NJJ + jj], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// q of head n (n % 8 when folded) of kv head h's GQA group for dims 32*s4 + 4*ii + kg, in the
// input dtype (the softmax scale is applied to the fp32 scores).  Lanes past
// the group read head 0's row (always valid) and zero it.
template <typename TQ, bool FOLD>
__device__ __forceinline__ QRegs<TQ> load_q(const TQ* __restrict__ query, int b, int hq, int h,
                                            int rep, int n, int kg) {
  constexpr int D = 128;
  QRegs<TQ> qv;
  const int hn = FOLD ? (n & 7) : n;  // folded: columns n and n + 8 carry head n % 8
  const bool live = hn < rep;
  const TQ* qrow = query + (static_cast<int64_t>(b) * hq + h * rep + (live ? hn : 0)) * D;
  const TQ zero = from_f32<TQ>(0.0f);
#pragma unroll
  for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const TQ lo = qrow[32 * s4 + 8 * p + kg];
      const TQ hi = qrow[32 * s4 + 8 * p + 4 + kg];
      qv.set(4 * s4 + p, live ? lo : zero, live ? hi : zero);
    }
  return qv;
}

// The item's page ids, one per lane (lane i: page pg0 + i), loaded once per
// 64 pages rather than read from the table in front of every tile's DMA.  Page
// ids are clamped into [0, nb): the host validates live ids, the clamp only
// guarantees that no DMA can leave the cache whatever the table holds.
struct PageIds {
  const int32_t* bt;
  int64_t maxb, nb;
  int bsh, pg0, pg_last, lane, vec;  // bs = 1 << bsh
  __device__ __forceinline__ PageIds(const int32_t* bt_, int64_t maxb_, int64_t nb_, int bsh_,
                                     int pb, int pe, int lane_)
      : bt(bt_), maxb(maxb_), nb(nb_), bsh(bsh_), pg0(pb >> bsh_), pg_last((pe - 1) >> bsh_),
        lane(lane_), vec(0) {
    if (pb < pe) vec = load();
  }
  __device__ __forceinline__ int load() const {
    const int pg = pg0 + lane;
    const int64_t b0 = pg <= pg_last && pg < maxb ? bt[pg] : 0;
    return static_cast<int>(b0 < 0 ? 0 : (b0 >= nb ? nb - 1 : b0));
  }
  // page of position p; positions only move forward, one tile (<= one page)
  // at a time
  __device__ __forceinline__ int64_t page(int p) {
    if ((p >> bsh) - pg0 >= 64) {  // uniform; only items longer than 64 pages get here
      pg0 += 64;
      vec = load();
    }
    return __builtin_amdgcn_readlane(vec, (p >> bsh) - pg0);
  }
};

// Running state of one wave: softmax max / sum (log2 domain), the PV
// accumulators (codes read as 1024 + c or 1024 + 16c), the constant-B MFMA
// sums that remove the 1024 offset, and the value-minima term per column group.
template <int CPG, bool VG1>
struct WaveAcc {
  static constexpr int NVG = 16 / CPG;
  static constexpr int NVS = Tile<CPG, VG1>::NVS;  // c_acc / bias_v entries in use
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
  // Epilogue: remove the PV offset, undo the 16x columns and add the minima;
  // o[v*NJJ + jj][r] of the result is O[head 4*kg + r][dim_of(v, jj)].
  __device__ __forceinline__ tail::Partial finish(const LaneNib<CPG>& ln, int kg) {
    constexpr int NJJ = CPG / 2;
#pragma unroll
    for (int v = 0; v < NVS; ++v) bias_v[v] = sum_kg(bias_v[v]);
    tail::Partial p;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int hh = 4 * kg + r;
#pragma unroll
      for (int v = 0; v < NVG; ++v) {
        const int vs_ = VG1 ? 0 : v;
        const float bv = __shfl(bias_v[vs_], hh, 64);
#pragma unroll
        for (int jj = 0; jj < NJJ; ++jj)
          p.o[v * NJJ + jj][r] = (o_acc[v * NJJ + jj][r] - c_acc[vs_][r]) * ln.col_scale + bv;
      }
    }
    p.m = m_run;
    p.l = l_run;
    return p;
  }
};

// Writes an int4-path partial for heads 0..rep-1 of kv head h's group.
template <int CPG>
__device__ __forceinline__ void store_partial(const tail::Partial& p, int wi, int hq, int h,
                                              int rep, int n, int kg, float* __restrict__ ws_o,
                                              float* __restrict__ ws_ml) {
  constexpr int D = 128;
  constexpr int NJJ = CPG / 2;
  constexpr int SUB = 16 / CPG;
  const int64_t head0 = static_cast<int64_t>(wi) * hq + h * rep;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int hh = 4 * kg + r;
#pragma unroll
    for (int v = 0; v < 16 / CPG; ++v)
#pragma unroll
      for (int jj = 0; jj < NJJ; ++jj) {
        const int dim = 8 * (n % CPG + CPG * v) + jj * SUB + n / CPG;
        if (hh < rep) ws_o[(head0 + hh) * D + dim] = p.o[v * NJJ + jj][r];
      }
  }
  if (kg == 0 && n < rep) {
    ws_ml[2 * (head0 + n)] = p.m;
    ws_ml[2 * (head0 + n) + 1] = p.l;
  }
}

// One int4 work item (kinds 0, 2, 3) of kv head h on the transposing-read
// tile (CPG 8: 64-token tiles, key groups of 64 or more): the same walk as the
// general loop of the kernel below -- windows of 64-position chunks, one
// barrier per window, a double buffer per wave filled by LDS DMA -- with
// decode_tr.h's tile layout and compute.
template <typename TQ, int NVG, bool KSV, bool FOLD>
__device__ __forceinline__ void tr_item(
    const TQ* __restrict__ query, int hq, int kvh, int h, int rep, float qscale,
    const uint32_t* __restrict__ kq, const float* __restrict__ ks, const float* __restrict__ km,
    const uint32_t* __restrict__ vq, const float* __restrict__ vs, const float* __restrict__ vm,
    int bs, int g, int64_t nb, const int32_t* __restrict__ block_table, int64_t maxb, int b,
    int pb, int pe, int kind, int wi, char* my_lds, float* xfer, int half, int npair, int lane,
    int n, int kg, int gpb, int ng, int wpd, bool pieces, float* __restrict__ ws_o,
    float* __restrict__ ws_ml) {
  using T = tr::Tile<NVG, KSV>;
  constexpr int D = T::D;
  constexpr int GT = T::GT;
  const tr::QLane<TQ> ql = tr::load_q<TQ>(query, b, hq, h, rep, n, kg, FOLD);
  const tr::LaneDma ld = tr::lane_dma(lane, wpd, kvh, gpb, ng, KSV);
  tr::Acc<NVG> acc;
  acc.init();
  const int bsh = __builtin_ctz(static_cast<unsigned>(bs));
  const int gsh = __builtin_ctz(static_cast<unsigned>(g));
  PageIds pages(block_table + static_cast<int64_t>(b) * maxb, maxb, nb, bsh, pb, pe, lane);
  auto issue = [&](char* buf, int p, bool with_ks) {
    const int64_t blk = pages.page(p);
    const int off0 = p & (bs - 1);
    const int64_t krow = (blk * kvh + h) * D;
    const int64_t vtok = ((blk << bsh) + off0) * kvh + h;
    tr::issue_tile<NVG, KSV>(buf, ld, kq + krow * wpd + (off0 >> 3), wpd,
                             ks + krow * gpb + (off0 >> gsh), km + krow * gpb + (off0 >> gsh), gpb,
                             vq + vtok * 16, kvh, vs + vtok * ng, vm + vtok * ng, with_ks);
  };
  const int hs = kind >= 2 ? kind - 2 : -1;
  const int cb = hs < 0 ? (pb & ~(64 * npair - 1)) : pb + 64 * hs;
  const int cs = 64 * npair * (hs < 0 ? 1 : 2);
  const int nwin = (pe - cb + cs - 1) / cs;
  int p_first = cb + (cs / npair) * half;
  if (p_first < pb) p_first += cs;
  auto next_tile = [&](int p) {
    p += GT;
    if ((p & 63) == 0) p += cs - 64;
    return p;
  };
  tr::QGroup qg;
  auto step = [&](const char* __restrict__ cur, char* __restrict__ nxt, int p0, bool new_group) {
    const int p1 = next_tile(p0);
    if (p1 < pe) {
      if ((p1 >> gsh) != (p0 >> gsh)) {
        issue(nxt, p1, true);
        wait_vmcnt<T::NINST>();
      } else {
        issue(nxt, p1, false);
        wait_vmcnt<T::NINST_CONT>();
      }
    } else {
      wait_vmcnt<0>();
    }
    const uint32_t* W = reinterpret_cast<const uint32_t*>(cur);
    if (new_group) tr::prepare_group<TQ, NVG, KSV, FOLD>(W, n, kg, ql, qscale, qg);
    if (pieces) __builtin_amdgcn_s_setprio(1);
    const uint32_t off = tr::lds_off(cur);
    if (p0 + GT <= pe)
      tr::compute_tile<NVG, KSV, FOLD, true>(W, off, p0, pe, n, kg, qg, qscale, acc);
    else
      tr::compute_tile<NVG, KSV, FOLD, false>(W, off, p0, pe, n, kg, qg, qscale, acc);
    if (pieces) __builtin_amdgcn_s_setprio(0);
  };
  if (p_first < pe) issue(my_lds, p_first, true);  // prologue: tile 0 into buffer 0
  int cur = 0;
  int p = p_first;
  int g_prev = -1;
  for (int k = 0; k < nwin; ++k) {
    __builtin_amdgcn_s_barrier();  // the workgroup's waves enter window k together
    const int wend = cb + cs * (k + 1);
    while (p < pe && p < wend) {
      step(my_lds + cur * T::BYTES, my_lds + (cur ^ 1) * T::BYTES, p, (p >> gsh) != g_prev);
      asm volatile("" ::: "memory");
      cur ^= 1;
      g_prev = p >> gsh;
      p = next_tile(p);
    }
  }
  tail::Partial part;
  tr::finish<NVG>(acc, kg, part.o);
  part.m = acc.m_run;
  part.l = acc.l_run;
  if (npair == 2) tail::merge_halves(part, xfer, half, lane);
  if (half == 0) tr::store_partial(part.o, part.m, part.l, wi, hq, h, rep, n, kg, ws_o, ws_ml);
}

// LDS of one wave: its two tile buffers, or the tail path's staging.
template <int CPG, bool VG1, bool KSV>
__host__ __device__ constexpr int tile_bytes() {
  return CPG == 8 ? tr::Tile<VG1 ? 1 : 2, KSV>::BYTES : Tile<CPG, VG1, KSV>::BYTES;
}
template <int CPG, bool VG1, bool KSV, bool TAIL>
__host__ __device__ constexpr int wave_lds_bytes() {
  return TAIL && tail::kLdsBytes > 2 * tile_bytes<CPG, VG1, KSV>()
             ? tail::kLdsBytes
             : 2 * tile_bytes<CPG, VG1, KSV>();
}

// A workgroup holds npair * hpw waves: kv heads q*hpw .. q*hpw + hpw - 1 of
// its items, npair (1 or 2) waves per head.  With two, wave `half` 0 / 1 takes
// the first / second 64-position chunk of every 128-position window of an
// int4 item (the two halves of a 128-token page, whose key rows it thereby
// fetches whole and at the same moment), and every other 32-position sub-tile
// of a tail item; the halves' partials merge through LDS at the item's end.
// A barrier per window keeps the workgroup's waves in step, so that the heads
// sharing a value line (and a scale line) request it together as well.
// (Measured on config-3 and config-5 decode, in-step groups cut the HBM
// fetch by up to 17% but wait at the barriers for longer than that saves:
// the launcher runs one wave per (kv head, item) in a workgroup of its own.
// The general form stays: with npair and hpw as run-time values the kernel
// allocates 233 VGPRs and spills nothing, while a one-wave-only copy of the
// same loop spills.)
// Without pieces (TAIL): the grid covers the work items twice; the first pass
// takes the int4 (kind-0) items, the second the tail (kind-1) items, so every
// tail wave is dispatched after every int4 wave and runs in the slots the
// shorter int4 items free, with no second stream or event between the two.
// With pieces (TAIL only): one workgroup per (piece, head group) walks the
// piece's items [pieces[k], pieces[k+1]) in order, int4 and tail alike; the
// host cuts the pieces to about equal cost, so every workgroup of the single
// pass ends at about the same time.
template <typename TQ, int CPG, bool VG1, bool KSV, bool FOLD, bool TAIL>
__global__ void __launch_bounds__(512, 2)
kivi_decode_mfma_kernel(const TQ* __restrict__ query, int hq, int kvh, int hpw, int npair,
                        float qscale,
                        const uint32_t* __restrict__ kq, const float* __restrict__ ks,
                        const float* __restrict__ km, const uint32_t* __restrict__ vq,
                        const float* __restrict__ vs, const float* __restrict__ vm, int bs,
                        int g, int64_t nb, const int32_t* __restrict__ block_table,
                        int64_t maxb, const int32_t* __restrict__ seq_meta,
                        const int32_t* __restrict__ work, int64_t num_work,
                        const int32_t* __restrict__ pieces_arg, int64_t num_pieces,
                        const TQ* __restrict__ ring_k, const TQ* __restrict__ ring_v,
                        int ring_len, float* __restrict__ ws_o, float* __restrict__ ws_ml) {
  using T = Tile<CPG, VG1, KSV>;
  constexpr int D = T::D;
  constexpr int GT = T::GT;
  constexpr int WAVE_LDS = wave_lds_bytes<CPG, VG1, KSV, TAIL>();

  extern __shared__ __align__(16) char lds_raw[];
  const int32_t* pieces = TAIL ? pieces_arg : nullptr;
  const int lane0 = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int hw = wave % hpw;    // head within the workgroup's group
  const int half = wave / hpw;  // < npair
  char* const my_lds = lds_raw + wave * WAVE_LDS;
  // the half-1 partner of this wave's head hands its partial over here
  float* const xfer = reinterpret_cast<float*>(lds_raw + (hw + hpw) * WAVE_LDS);
  const int nq = kvh / hpw;
  int it0, it1, qh, pass = 0;
  if (pieces) {
    int k;
    if (!xcd_item_head(blockIdx.x, nq, num_pieces, k, qh)) return;  // workgroup-uniform
    it0 = pieces[k];
    it1 = pieces[k + 1];
  } else {
    const int64_t pass_len = xcd_grid_size(num_work, nq);
    pass = TAIL && blockIdx.x >= pass_len ? 1 : 0;
    if (!xcd_item_head(blockIdx.x - pass * pass_len, nq, num_work, it0, qh)) return;
    it1 = it0 + 1;
  }
  const int h = qh * hpw + hw;
  const int rep = hq / kvh;
  // every branch below depends on the work item only: workgroup-uniform, so
  // every wave meets the same barriers
  for (int wi = it0; wi < it1; ++wi) {
  const int32_t* wk = work + 4 * static_cast<int64_t>(wi);
  const int kind = wk[3];
  // without pieces the other pass (or the tail kernel) owns it;
  // kinds 0, 2 and 3 are int4 ranges, kind 1 the tail
  if (!pieces && (kind == 1 ? 1 : 0) != pass) continue;
  if constexpr (TAIL) {
    if (kind == 1) {
      tail::Partial tp = tail::tail_item<TQ>(my_lds, query, hq, kvh, qscale, kq, ks, km, vq, vs,
                                             vm, bs, g, nb, block_table, maxb, seq_meta, wk, wi,
                                             h, ring_k, ring_v, ring_len, half, npair);
      if (npair == 2) tail::merge_halves(tp, xfer, half, lane0);
      if (half == 0) tail::tail_store(tp, wi, hq, h, rep, lane0, ws_o, ws_ml);
      continue;
    }
  }
  // lane-dependent set-up per item (not hoisted out of the item loop)
  int lane = lane0;
  asm volatile("" : "+v"(lane));
  const int n = lane & 15;
  const int kg = lane >> 4;
  const int b = wk[0];
  const int pb = wk[1];
  const int pe = wk[2];
  const int gpb = bs / g;
  const int ng = D / g;
  const int wpd = bs / 8;
  if constexpr (CPG == 8) {
    tr_item<TQ, VG1 ? 1 : 2, KSV, FOLD>(query, hq, kvh, h, rep, qscale, kq, ks, km, vq, vs, vm,
                                        bs, g, nb, block_table, maxb, b, pb, pe, kind, wi,
                                        my_lds, xfer, half, npair, lane, n, kg, gpb, ng, wpd,
                                        pieces != nullptr, ws_o, ws_ml);
  } else {

  const QRegs<TQ> qv = load_q<TQ, FOLD>(query, b, hq, h, rep, n, kg);
  const LaneNib<CPG> ln(n, kg);
  const LaneDma ld = lane_dma<CPG, VG1, KSV>(lane, wpd, kvh, gpb, ng, g);

  WaveAcc<CPG, VG1> acc;
  acc.init();
  // bs and g are powers of two (the launcher checks): page, offset and key
  // group come from shifts and masks, not integer divisions
  const int bsh = __builtin_ctz(static_cast<unsigned>(bs));
  const int gsh = __builtin_ctz(static_cast<unsigned>(g));
  PageIds pages(block_table + static_cast<int64_t>(b) * maxb, maxb, nb, bsh, pb, pe, lane);
  auto issue = [&](char* buf, int p, bool with_ks) {
    const int64_t blk = pages.page(p);
    const int off0 = p & (bs - 1);
    const int64_t krow = (blk * kvh + h) * D;
    const int64_t vtok = ((blk << bsh) + off0) * kvh + h;
    issue_tile<CPG, VG1, KSV>(buf, ld, kq + krow * wpd + (off0 >> 3), wpd, vq + vtok * 16, kvh,
                         ks + krow * gpb + (off0 >> gsh), km + krow * gpb + (off0 >> gsh), gpb,
                         vs + vtok * ng, vm + vtok * ng, ng, g, with_ks);
  };
  // 64-position chunks: window k holds chunk cb + cs*k + (cs/npair)*half of
  // each half.  Kind 0: the (64*npair)-aligned windows over [pb, pe); kind 2 /
  // 3 (only the even / odd chunks of [pb, pe)): npair of its chunks.  Items
  // start on multiples of 64, so chunks are 64-aligned and hold whole tiles.
  const int hs = kind >= 2 ? kind - 2 : -1;
  const int cb = hs < 0 ? (pb & ~(64 * npair - 1)) : pb + 64 * hs;
  const int cs = 64 * npair * (hs < 0 ? 1 : 2);
  const int nwin = (pe - cb + cs - 1) / cs;
  int p_first = cb + (cs / npair) * half;
  if (p_first < pb) p_first += cs;  // kind 0 from an odd chunk: half 0 starts a window later
  // the wave's tile after p: the next tile of its chunk, else its next chunk
  auto next_tile = [&](int p) {
    p += GT;
    if ((p & 63) == 0) p += cs - 64;
    return p;
  };
  // One tile step: DMA of the wave's next tile into `nxt`, then compute tile
  // p0 from `cur`.  Both buffers are __restrict__ within the step, which tells the
  // compiler's wait-count pass that the reads of `cur` cannot alias the DMA
  // in flight into `nxt`: without it the pass puts vmcnt(0) -- a wait for the
  // next tile -- in front of the first LDS read and the double buffer never
  // overlaps.  The wait for tile p0 itself is explicit.
  QGroup qg;
  auto step = [&](const char* __restrict__ cur, char* __restrict__ nxt, int p0, bool new_group) {
    const int p1 = next_tile(p0);
    if (p1 < pe) {
      // a tile needs the key scales exactly when its key group differs from
      // the wave's previous tile's
      if ((p1 >> gsh) != (p0 >> gsh)) {
        issue(nxt, p1, true);
        wait_vmcnt<T::NINST>();
      } else {
        issue(nxt, p1, false);
        wait_vmcnt<T::NINST_CONT>();
      }
    } else {
      wait_vmcnt<0>();
    }
    const uint32_t* W = reinterpret_cast<const uint32_t*>(cur);
    // tiles are GT-aligned and GT divides g: the wave's first tile, or one in
    // another key group than its previous tile, prepares the group's Q'
    if (new_group) prepare_group<TQ, CPG, FOLD, KSV>(W, n, kg, qv, qscale, qg);
    // single-round piece plans: raised wave priority over the tile's compute,
    // so a SIMD's arbiter finishes one wave's tile while the other's DMA is in
    // flight (config 3: 94.4 -> 93.5 us; over the many rounds of a split plan
    // it starves the waves that would issue the next DMA: config 5 2.58 ->
    // 2.94 ms, so those keep the default)
    if (pieces) __builtin_amdgcn_s_setprio(1);
    const WaveValues<CPG, VG1> vals(W, kg, n % CPG);
    if (p0 + GT <= pe)
      compute_tile<TQ, CPG, VG1, true, FOLD>(W, vals, p0, pe, n, kg, qg, qscale, ln, acc.m_run,
                                             acc.l_run, acc.o_acc, acc.c_acc, acc.bias_v);
    else
      compute_tile<TQ, CPG, VG1, false, FOLD>(W, vals, p0, pe, n, kg, qg, qscale, ln, acc.m_run,
                                              acc.l_run, acc.o_acc, acc.c_acc, acc.bias_v);
    if (pieces) __builtin_amdgcn_s_setprio(0);
  };
  if (p_first < pe) issue(my_lds, p_first, true);  // prologue: tile 0 into buffer 0
  int cur = 0;
  int p = p_first;
  int g_prev = -1;  // key group of the wave's previous tile
  for (int k = 0; k < nwin; ++k) {
    __builtin_amdgcn_s_barrier();  // the workgroup's waves enter window k together
    const int wend = cb + cs * (k + 1);
    while (p < pe && p < wend) {
      step(my_lds + cur * T::BYTES, my_lds + (cur ^ 1) * T::BYTES, p, (p >> gsh) != g_prev);
      // every LDS read of this buffer has been consumed before the next
      // iteration's DMA may overwrite it
      asm volatile("" ::: "memory");
      cur ^= 1;
      g_prev = p >> gsh;
      p = next_tile(p);
    }
  }
  tail::Partial part = acc.finish(ln, kg);
  if (npair == 2) tail::merge_halves(part, xfer, half, lane);
  if (half == 0) store_partial<CPG>(part, wi, hq, h, rep, n, kg, ws_o, ws_ml);
  }  // CPG 4
  }  // items
}

// Copies 1 KiB with 16-byte DMA lanes and 256 B with 4-byte DMA lanes through
// LDS and writes the LDS image back, so a test can pin the lane -> LDS address
// mapping the decode kernel's tile layout relies on.
__global__ void lds_dma_probe_kernel(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst) {
  extern __shared__ __align__(16) char lds_raw[];
  const int lane = threadIdx.x;
  dma16(src + 4 * lane, lds_raw);
  dma4(src + 256 + lane, lds_raw + 1024);
  wait_vmcnt<0>();
  const uint32_t* l = reinterpret_cast<const uint32_t*>(lds_raw);
#pragma unroll
  for (int i = 0; i < 5; ++i) dst[64 * i + lane] = l[64 * i + lane];
}

// The cross-lane reductions the kernels use (kvq_common.h), on 16 rounds of
// 64 values: dst[4 (64 t + l) + {0, 1, 2, 3}] = max_rows4, sum_rows4,
// max_wave64, sum_wave64 of lane l's value src[64 t + l].
__global__ void lane_reduction_probe_kernel(const float* __restrict__ src, float* __restrict__ dst) {
  const int lane = threadIdx.x;
  for (int t = 0; t < 16; ++t) {
    const float x = src[64 * t + lane];
    float* o = dst + 6 * (64 * t + lane);
    o[0] = max_rows4(x);
    o[1] = sum_rows4(x);
    o[2] = max_wave64(x);
    o[3] = sum_wave64(x);
    float px = x, py = src[64 * ((t + 1) % 16) + lane];
    max_rows4_pair(px, py);
    o[4] = px;
    o[5] = py;
  }
}

// 16x32 (A) times 32x16 (B) through the same intrinsic and operand mapping the
// decode kernels rely on: lane l holds A[l%16][8*(l/16)+i] and B[8*(l/16)+i][l%16];
// the result lands as D[4*(l/16)+r][l%16].
__global__ void mfma_layout_probe_kernel(const _Float16* __restrict__ a,
                                         const _Float16* __restrict__ b, float* __restrict__ d) {
  const int l = threadIdx.x;
  h8 av, bv;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    av[i] = a[(l % 16) * 32 + 8 * (l / 16) + i];
    bv[i] = b[(8 * (l / 16) + i) * 16 + l % 16];
  }
  f4 acc = f4{0.f, 0.f, 0.f, 0.f};
  acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc, 0, 0, 0);
#pragma unroll
  for (int r = 0; r < 4; ++r) d[(4 * (l / 16) + r) * 16 + l % 16] = acc[r];
}

}  // namespace

namespace kvq {

// Waves per (kv head, item) and kv heads per workgroup of the INT4 decode.
// (kivi_plan.cpp counts 8 / kDecodeWavesPerHead (kv head, piece) slots per CU.)
constexpr int kDecodeWavesPerHead = 1;
constexpr int kDecodeHeadsPerWg = 1;

// LDS per wave of the kernel instance these parameters select.
template <bool TAIL>
int64_t wave_lds_of(int cpg, bool vg1, bool ksv) {
  if (cpg != 8) return wave_lds_bytes<4, false, false, TAIL>();
  if (ksv) return wave_lds_bytes<8, true, true, TAIL>();
  return vg1 ? wave_lds_bytes<8, true, false, TAIL>() : wave_lds_bytes<8, false, false, TAIL>();
}

int launch_kivi_decode_mfma(const void* query, int q_dtype, int hq, int kvh, int d, float qscale,
                            const int32_t* kq, const float* ks, const float* km,
                            const int32_t* vq, const float* vs, const float* vm, int bs, int g,
                            int64_t nb, const int32_t* block_table, int64_t maxb,
                            const int32_t* seq_meta, const int32_t* work, int64_t num_work,
                            const int32_t* pieces, int64_t num_pieces,
                            const void* ring_k, const void* ring_v, int ring_dtype, int ring_len,
                            float* ws_o, float* ws_ml, hipStream_t s, bool* launched,
                            bool* tail_done) {
  *launched = false;
  *tail_done = false;
  if (d != 128 || hq / kvh > 16 || g % 8 || d % g || g < 32 || g > 128) return KVQ_OK;
  if (bs <= 0 || (bs & (bs - 1))) return KVQ_OK;  // power-of-two pages (shift arithmetic)
  // tiles of 64 tokens (32 for G = 32): inside one key group and one page
  const int cpg = g >= 64 ? 8 : 4;
  if (bs % (8 * cpg)) return KVQ_OK;
  const uint32_t* kqu = reinterpret_cast<const uint32_t*>(kq);
  const uint32_t* vqu = reinterpret_cast<const uint32_t*>(vq);
  const bool tail = tail_path_applies(q_dtype, hq, kvh, d, ring_dtype, bs);
  // pieces need the tail path (a piece mixes int4 and tail items)
  const bool use_pieces = tail && pieces && num_pieces > 0;
  // GQA groups of at most 8 heads fold the hi/lo score parts into one MFMA
  const bool fold = hq / kvh <= 8;
  // one value group per head row: value scales gathered once per PV k-step
  const bool vg1 = cpg == 8 && g >= 128;
  // a key group per page: its scales are contiguous per head
  const bool ksv = vg1 && bs == g;
  if (use_pieces) {
    // whole pages for all kv heads per workgroup where the geometry allows
    bool coop = false;
    const int crc = launch_kivi_decode_coop(query, q_dtype, hq, kvh, d, qscale, kq, ks, km, vq,
                                            vs, vm, bs, g, nb, block_table, maxb, seq_meta, work,
                                            num_work, pieces, num_pieces, ring_k, ring_v,
                                            ring_dtype, ring_len, ws_o, ws_ml, s, &coop);
    if (crc != KVQ_OK) return crc;
    if (coop) {
      *launched = true;
      *tail_done = true;
      return KVQ_OK;
    }
  }
  const int64_t wave_lds = tail ? wave_lds_of<true>(cpg, vg1, ksv) : wave_lds_of<false>(cpg, vg1, ksv);
  int64_t lds_max = 0;  // LDS one workgroup may use on this device
  const int lrc = device_lds_max(&lds_max);
  if (lrc != KVQ_OK) return lrc;
  // waves per kv head, and kv heads per workgroup: as many as the heads and
  // the LDS allow, up to kDecodeHeadsPerWg
  const int npair = kDecodeWavesPerHead;
  int hpw = kDecodeHeadsPerWg;
  while (hpw > 1 && (kvh % hpw || npair * hpw * wave_lds > lds_max)) hpw /= 2;
  if (npair * wave_lds > lds_max) return KVQ_OK;  // not this device: the portable kernels run
  const int nq = kvh / hpw;
  const int64_t pass_len = xcd_grid_size(num_work, nq);
  const int64_t blocks =
      use_pieces ? xcd_grid_size(num_pieces, nq) : (tail ? 2 : 1) * pass_len;
  if (blocks > 0x7fffffff) return KVQ_ERR_INVALID;
  const int32_t* pieces_k = use_pieces ? pieces : nullptr;
  const dim3 grid(static_cast<unsigned>(blocks));
  const dim3 block(64 * npair * hpw);
  const size_t lds = static_cast<size_t>(npair * hpw * wave_lds);
#define KVQ_LAUNCH_MFMA(TQ, C, V, KV, F, TL)                                                  \
  hipLaunchKernelGGL((kivi_decode_mfma_kernel<TQ, C, V, KV, F, TL>), grid, block, lds, s,    \
                     static_cast<const TQ*>(query), hq, kvh, hpw, npair, qscale, kqu, ks, km, \
                     vqu, vs, vm,                                                             \
                     bs, g, nb, block_table, maxb, seq_meta, work, num_work, pieces_k,       \
                     num_pieces, static_cast<const TQ*>(ring_k), static_cast<const TQ*>(ring_v),\
                     ring_len, ws_o, ws_ml)
#define KVQ_LAUNCH_MFMA_F(TQ, C, V, KV, TL)                                                   \
  if (fold) KVQ_LAUNCH_MFMA(TQ, C, V, KV, true, TL); else KVQ_LAUNCH_MFMA(TQ, C, V, KV, false, TL);
#define KVQ_LAUNCH_MFMA_CF(TQ, TL)                                                            \
  if (cpg == 8) {                                                                             \
    if (ksv) { KVQ_LAUNCH_MFMA_F(TQ, 8, true, true, TL) }                                     \
    else if (vg1) { KVQ_LAUNCH_MFMA_F(TQ, 8, true, false, TL) }                               \
    else { KVQ_LAUNCH_MFMA_F(TQ, 8, false, false, TL) }                                       \
  } else {                                                                                    \
    KVQ_LAUNCH_MFMA_F(TQ, 4, false, false, TL)                                                \
  }
  if (tail && q_dtype == KVQ_DTYPE_BF16) {
    KVQ_LAUNCH_MFMA_CF(bf16, true);
  } else if (tail) {
    KVQ_LAUNCH_MFMA_CF(f16, true);
  } else {
    // without the tail pass the ring pointers are never read; they fill the
    // parameters in the query dtype
    KVQ_DISPATCH_FLOAT(q_dtype, TQ, KVQ_LAUNCH_MFMA_CF(TQ, false));
  }
#undef KVQ_LAUNCH_MFMA_CF
#undef KVQ_LAUNCH_MFMA_F
#undef KVQ_LAUNCH_MFMA
  KVQ_LAUNCH_CHECK();
  *launched = true;
  *tail_done = tail;
  return KVQ_OK;
}

}  // namespace kvq

extern "C" int kvq_selftest_mfma_f16(const void* a, const void* b, float* d, void* stream) {
  if (!a || !b || !d) return KVQ_ERR_INVALID;
  hipLaunchKernelGGL(mfma_layout_probe_kernel, dim3(1), dim3(64), 0,
                     static_cast<hipStream_t>(stream), static_cast<const _Float16*>(a),
                     static_cast<const _Float16*>(b), d);
  KVQ_LAUNCH_CHECK();
  return KVQ_OK;
}

extern "C" int kvq_selftest_lane_reductions(const float* src, float* dst, void* stream) {
  if (!src || !dst) return KVQ_ERR_INVALID;
  hipLaunchKernelGGL(lane_reduction_probe_kernel, dim3(1), dim3(64), 0,
                     static_cast<hipStream_t>(stream), src, dst);
  KVQ_LAUNCH_CHECK();
  return KVQ_OK;
}

extern "C" int kvq_selftest_lds_dma(const void* src, void* dst, void* stream) {
  if (!src || !dst) return KVQ_ERR_INVALID;
  hipLaunchKernelGGL(lds_dma_probe_kernel, dim3(1), dim3(64), 1280,
                     static_cast<hipStream_t>(stream), static_cast<const uint32_t*>(src),
                     static_cast<uint32_t*>(dst));
  KVQ_LAUNCH_CHECK();
  return KVQ_OK;
}
