// SPDX-License-Identifier: Apache-2.0
// MFMA decode attention over KIVI int4 pages (kind-0 work items) for gfx950.
//
// One wave per (work item, kv head).  A work item is a 128-aligned range of
// positions whose keys and values are both in int4 pages; the wave walks it in
// "group tiles" of GT = 8*CPG tokens (CPG = 8 for G >= 64, 4 for G = 32), each
// inside one page and one key-scale group.
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

// (hi, lo) fp16 parts of x: hi = fp16(x), lo = fp16(x - hi).
__device__ __forceinline__ void split_h(float x, _Float16& hi, _Float16& lo) {
  hi = static_cast<_Float16>(x);
  lo = static_cast<_Float16>(x - static_cast<float>(hi));
}

__device__ __forceinline__ uint32_t h2_bits(_Float16 a, _Float16 b) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, a)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, b)) << 16);
}

__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  const _Float16 a = static_cast<_Float16>(lo);
  const _Float16 b = static_cast<_Float16>(hi);
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, a)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, b)) << 16);
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

// ---- LDS DMA -------------------------------------------------------------
// global_load_lds: every lane reads `size` bytes at its own global address and
// the wave writes them to LDS at base + size * lane (base must be uniform).

typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ void dma16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)(lds), 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)(lds), 4, 0, 0);
}

// s_waitcnt vmcnt(N) with lgkmcnt/expcnt left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("" ::: "memory");
}

// Tile buffer layout (bytes) for one wave.
template <int CPG>
struct TileLayout {
  static constexpr int D = 128;
  static constexpr int GT = 8 * CPG;
  static constexpr int NVG = 16 / CPG;
  static constexpr int KW = 0;                      // key words  [d][CPG] u32
  static constexpr int VW = KW + D * CPG * 4;       // value words [t][16] u32
  static constexpr int KS = VW + GT * 64;           // key scale   [d] f32
  static constexpr int KM = KS + D * 4;             // key min     [d] f32
  static constexpr int VS = KM + D * 4;             // value scale [t][NVG] f32
  static constexpr int VM = VS + GT * NVG * 4;      // value min   [t][NVG] f32
  static constexpr int BYTES = VM + GT * NVG * 4;
  // DMA instructions per tile: the wait counts below rely on this number
  static constexpr int KW_INST = D * CPG * 4 / 1024;
  static constexpr int VW_INST = GT * 64 / 1024;
  static constexpr int NINST = KW_INST + VW_INST + 2 * (D / 64) + 2 * (GT * NVG / 64);
};

// Issue the DMA loads of one tile (page blk, offsets [off0, off0 + GT), key
// group grp) of kv head h into `buf`.  Every load is in bounds: the tile lies
// inside page blk, which the caller has checked is a live block id.
template <int CPG>
__device__ __forceinline__ void issue_tile(char* buf, int lane, int64_t blk, int off0, int grp,
                                           int h, int kvh, int bs, int gpb, int ng,
                                           const uint32_t* __restrict__ kq,
                                           const float* __restrict__ ks,
                                           const float* __restrict__ km,
                                           const uint32_t* __restrict__ vq,
                                           const float* __restrict__ vs,
                                           const float* __restrict__ vm) {
  using L = TileLayout<CPG>;
  constexpr int D = L::D;
  constexpr int LPR = CPG / 4;   // 16-byte lanes per key dim row (CPG words)
  constexpr int DPI = 64 / LPR;  // key dim rows per instruction
  const int wpd = bs / 8;
  const int64_t krow0 = (blk * kvh + h) * D;
#pragma unroll
  for (int i = 0; i < L::KW_INST; ++i) {
    const int d = i * DPI + lane / LPR;
    const int part = lane % LPR;
    dma16(kq + (krow0 + d) * wpd + off0 / 8 + 4 * part, buf + L::KW + i * 1024);
  }
#pragma unroll
  for (int i = 0; i < L::VW_INST; ++i) {
    const int t = 16 * i + lane / 4;
    const int part = lane % 4;
    dma16(vq + ((blk * bs + off0 + t) * kvh + h) * 16 + 4 * part, buf + L::VW + i * 1024);
  }
#pragma unroll
  for (int i = 0; i < D / 64; ++i) {
    const int d = 64 * i + lane;
    dma4(ks + (krow0 + d) * gpb + grp, buf + L::KS + i * 256);
    dma4(km + (krow0 + d) * gpb + grp, buf + L::KM + i * 256);
  }
#pragma unroll
  for (int i = 0; i < L::GT * L::NVG / 64; ++i) {
    const int e = 64 * i + lane;
    const int t = e / L::NVG;
    int vg = e % L::NVG;
    vg = vg < ng ? vg : 0;  // slots past the tile's groups load a duplicate (never read)
    const int64_t idx = ((blk * bs + off0 + t) * kvh + h) * ng + vg;
    dma4(vs + idx, buf + L::VS + i * 256);
    dma4(vm + idx, buf + L::VM + i * 256);
  }
}

template <typename TQ, int CPG>
__global__ void __launch_bounds__(64, 2)
kivi_decode_mfma_kernel(const TQ* __restrict__ query, int hq, int kvh, float qscale,
                        const uint32_t* __restrict__ kq, const float* __restrict__ ks,
                        const float* __restrict__ km, const uint32_t* __restrict__ vq,
                        const float* __restrict__ vs, const float* __restrict__ vm, int bs,
                        int g, int64_t nb, const int32_t* __restrict__ block_table,
                        int64_t maxb, const int32_t* __restrict__ work,
                        float* __restrict__ ws_o, float* __restrict__ ws_ml) {
  using L = TileLayout<CPG>;
  constexpr int D = L::D;
  constexpr int GT = L::GT;      // tokens per tile
  constexpr int NJ = CPG / 2;    // score MFMAs per k-step (16 tokens each)
  constexpr int SUB = 16 / CPG;  // tokens of one chunk inside one score MFMA
  constexpr int NVG = L::NVG;    // PV column groups (one value group each)
  constexpr int NJJ = CPG / 2;   // PV MFMAs per column group (NVG * NJJ == 8)
  constexpr int PVS = CPG / 4;   // PV k-steps (32 tokens) per tile

  extern __shared__ __align__(16) char lds_raw[];
  const int wi = blockIdx.x;
  const int h = blockIdx.y;
  const int lane = threadIdx.x;
  const int32_t* wk = work + 4 * static_cast<int64_t>(wi);
  if (wk[3] != 0) return;  // kind-1 items belong to the generic kernel (uniform)
  const int b = wk[0];
  const int pb = wk[1];
  const int pe = wk[2];
  const int rep = hq / kvh;
  const int n = lane & 15;
  const int kg = lane >> 4;
  const int gpb = bs / g;
  const int ng = D / g;
  const int32_t* bt = block_table + static_cast<int64_t>(b) * maxb;

  // q of head n for the lane's dims d = 32*s + 4*i + kg, in the input dtype.
  // Lanes past the GQA group read head 0's row (always valid) and zero it, so
  // the 32 loads issue back to back instead of behind per-lane branches.
  TQ qv[32];
  {
    const bool live = n < rep;
    const TQ* qrow = query + (static_cast<int64_t>(b) * hq + h * rep + (live ? n : 0)) * D;
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
      for (int i = 0; i < 8; ++i) qv[8 * s4 + i] = qrow[32 * s4 + 4 * i + kg];
    if (!live) {
#pragma unroll
      for (int i = 0; i < 32; ++i) qv[i] = from_f32<TQ>(0.0f);
    }
  }
  const h8 ones_a = as_h8(kMagic, kMagic, kMagic, kMagic);

  float m_run = -INFINITY;
  float l_run = 0.0f;
  f4 o_acc[8];
  f4 c_acc[NVG];
  float bias_v[NVG];
#pragma unroll
  for (int q = 0; q < 8; ++q) o_acc[q] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int v = 0; v < NVG; ++v) {
    c_acc[v] = f4{0.f, 0.f, 0.f, 0.f};
    bias_v[v] = 0.0f;
  }

  // page ids are clamped into [0, nb): the host validates live ids, the clamp
  // only guarantees that no DMA can leave the cache whatever the table holds
  auto page = [&](int p) -> int64_t {
    const int64_t blk = bt[p / bs];
    return blk < 0 ? 0 : (blk >= nb ? nb - 1 : blk);
  };
  // prologue: tile 0 into buffer 0
  {
    const int64_t blk = page(pb);
    issue_tile<CPG>(lds_raw, lane, blk, pb % bs, (pb % bs) / g, h, kvh, bs, gpb, ng, kq, ks, km,
                    vq, vs, vm);
  }
  int cur = 0;
  for (int p0 = pb; p0 < pe; p0 += GT) {
    // prefetch tile p0 + GT into the other buffer, then wait for this tile only
    const int p1 = p0 + GT;
    if (p1 < pe) {
      const int64_t blk1 = page(p1);
      issue_tile<CPG>(lds_raw + (cur ^ 1) * L::BYTES, lane, blk1, p1 % bs, (p1 % bs) / g, h,
                      kvh, bs, gpb, ng, kq, ks, km, vq, vs, vm);
      wait_vmcnt<L::NINST>();
    } else {
      wait_vmcnt<0>();
    }
    const char* buf = lds_raw + cur * L::BYTES;
    const float* sks = reinterpret_cast<const float*>(buf + L::KS);
    const float* skm = reinterpret_cast<const float*>(buf + L::KM);
    const uint32_t* skw = reinterpret_cast<const uint32_t*>(buf + L::KW);
    const uint32_t* svw = reinterpret_cast<const uint32_t*>(buf + L::VW);
    const float* svs = reinterpret_cast<const float*>(buf + L::VS);
    const float* svm = reinterpret_cast<const float*>(buf + L::VM);

    // ---- scores ------------------------------------------------------------
    const int chunk = n % CPG;
    const int sub = n / CPG;
    float kb = 0.0f;
    f4 sacc[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) sacc[j] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      uint32_t qh[4], ql[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const int d0 = 32 * s4 + 8 * p + kg;  // element 2p
        const int d1 = d0 + 4;                // element 2p + 1
        const float q0 = to_f32(qv[8 * s4 + 2 * p]) * qscale;
        const float q1 = to_f32(qv[8 * s4 + 2 * p + 1]) * qscale;
        _Float16 h0, l0, h1, l1;
        split_h(q0 * sks[d0], h0, l0);
        split_h(q1 * sks[d1], h1, l1);
        qh[p] = h2_bits(h0, h1);
        ql[p] = h2_bits(l0, l1);
        kb += q0 * skm[d0] + q1 * skm[d1];
      }
      uint32_t w[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) w[i] = skw[(32 * s4 + 4 * i + kg) * CPG + chunk];
      const h8 bq = as_h8(qh[0], qh[1], qh[2], qh[3]);
      const h8 bl = as_h8(ql[0], ql[1], ql[2], ql[3]);
#pragma unroll
      for (int jm = 0; jm < NJ; ++jm) {
        const uint32_t j = static_cast<uint32_t>(jm * SUB + sub);
        const h8 a = as_h8(code_pair_exact(w[0], w[1], j), code_pair_exact(w[2], w[3], j),
                           code_pair_exact(w[4], w[5], j), code_pair_exact(w[6], w[7], j));
        sacc[jm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bq, sacc[jm], 0, 0, 0);
        sacc[jm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bl, sacc[jm], 0, 0, 0);
      }
    }
    kb = sum_kg(kb);
    // lane holds head n, rows m' = 4*kg + r: token 8*(m' % CPG) + jm*SUB + m'/CPG
    float tmax = -INFINITY;
#pragma unroll
    for (int jm = 0; jm < NJ; ++jm) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int mr = 4 * kg + r;
        const int pos = p0 + 8 * (mr % CPG) + jm * SUB + mr / CPG;
        const float sv = pos < pe ? sacc[jm][r] + kb : -INFINITY;
        sacc[jm][r] = sv;
        tmax = fmaxf(tmax, sv);
      }
    }
    tmax = max_kg(tmax);
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = m_run == -INFINITY ? 0.0f : exp2f(m_run - m_new);
    float psum = 0.0f;
#pragma unroll
    for (int jm = 0; jm < NJ; ++jm) {
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
#pragma unroll
      for (int v = 0; v < NVG; ++v) c_acc[v][r] *= ar;
    }
#pragma unroll
    for (int v = 0; v < NVG; ++v) bias_v[v] *= alpha;

    // ---- PV ------------------------------------------------------------------
#pragma unroll
    for (int st = 0; st < PVS; ++st) {
      int tk[8];
      float pv[8];
      bool live[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int jm = 2 * st + i / 4;
        const int mr = 4 * kg + (i % 4);
        tk[i] = 8 * (mr % CPG) + jm * SUB + mr / CPG;
        pv[i] = sacc[jm][i % 4];
        live[i] = p0 + tk[i] < pe;
      }
#pragma unroll
      for (int v = 0; v < NVG; ++v) {
        const int vgrp = (8 * CPG * v) / g;
        float pp[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          // tokens past the range have p = 0 but unwritten scale/min bytes:
          // select zeros so a stale NaN cannot leak into the sums (the reads
          // stay inside the tile buffer, so they are unconditional)
          const float sc_raw = svs[tk[i] * NVG + vgrp];
          const float mn_raw = svm[tk[i] * NVG + vgrp];
          const float sc = live[i] ? sc_raw : 0.0f;
          const float mn = live[i] ? mn_raw : 0.0f;
          pp[i] = pv[i] * sc;
          bias_v[v] += pv[i] * mn;
        }
        const h8 a = as_h8(pack_h2(pp[0], pp[1]), pack_h2(pp[2], pp[3]), pack_h2(pp[4], pp[5]),
                           pack_h2(pp[6], pp[7]));
        c_acc[v] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ones_a, c_acc[v], 0, 0, 0);
        const int vchunk = n % CPG + CPG * v;
        uint32_t w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = svw[tk[i] * 16 + vchunk];
#pragma unroll
        for (int jj = 0; jj < NJJ; ++jj) {
          const uint32_t nib = static_cast<uint32_t>(jj * SUB + n / CPG);
          const h8 bv = as_h8(code_pair(w[0], w[1], nib), code_pair(w[2], w[3], nib),
                              code_pair(w[4], w[5], nib), code_pair(w[6], w[7], nib));
          o_acc[v * NJJ + jj] =
              __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bv, o_acc[v * NJJ + jj], 0, 0, 0);
        }
      }
    }
    // every LDS read of this buffer has been consumed before the next
    // iteration's DMA may overwrite it
    asm volatile("" ::: "memory");
    cur ^= 1;
  }

  // ---- epilogue: remove the PV offset, add the value-minimum term --------
#pragma unroll
  for (int v = 0; v < NVG; ++v) bias_v[v] = sum_kg(bias_v[v]);
  const int64_t head0 = static_cast<int64_t>(wi) * hq + h * rep;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int hh = 4 * kg + r;
#pragma unroll
    for (int v = 0; v < NVG; ++v) {
      const float bv = __shfl(bias_v[v], hh, 64) - c_acc[v][r];
#pragma unroll
      for (int jj = 0; jj < NJJ; ++jj) {
        const int dim = 8 * (n % CPG + CPG * v) + jj * SUB + n / CPG;
        if (hh < rep) ws_o[(head0 + hh) * D + dim] = o_acc[v * NJJ + jj][r] + bv;
      }
    }
  }
  if (kg == 0 && n < rep) {
    ws_ml[2 * (head0 + n)] = m_run;
    ws_ml[2 * (head0 + n) + 1] = l_run;
  }
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

int launch_kivi_decode_mfma(const void* query, int q_dtype, int hq, int kvh, int d, float qscale,
                            const int32_t* kq, const float* ks, const float* km,
                            const int32_t* vq, const float* vs, const float* vm, int bs, int g,
                            int64_t nb, const int32_t* block_table, int64_t maxb,
                            const int32_t* seq_meta,
                            const int32_t* work, int64_t num_work, float* ws_o, float* ws_ml,
                            hipStream_t s, bool* launched) {
  (void)seq_meta;
  *launched = false;
  if (d != 128 || hq / kvh > 16 || g % 8 || d % g || g < 32 || g > 128) return KVQ_OK;
  // tiles of 64 tokens (32 for G = 32): inside one key group and one page
  const int cpg = g >= 64 ? 8 : 4;
  if (bs % (8 * cpg)) return KVQ_OK;
  const dim3 grid(static_cast<unsigned>(num_work), kvh);
  const dim3 block(64);
  const uint32_t* kqu = reinterpret_cast<const uint32_t*>(kq);
  const uint32_t* vqu = reinterpret_cast<const uint32_t*>(vq);
#define KVQ_LAUNCH_MFMA(C)                                                                   \
  KVQ_DISPATCH_FLOAT(q_dtype, TQ,                                                           \
    hipLaunchKernelGGL((kivi_decode_mfma_kernel<TQ, C>), grid, block,                       \
                       2 * TileLayout<C>::BYTES, s, static_cast<const TQ*>(query), hq, kvh, \
                       qscale, kqu, ks, km, vqu, vs, vm, bs, g, nb, block_table, maxb, work,\
                       ws_o, ws_ml))
  if (cpg == 8) {
    KVQ_LAUNCH_MFMA(8);
  } else {
    KVQ_LAUNCH_MFMA(4);
  }
#undef KVQ_LAUNCH_MFMA
  KVQ_LAUNCH_CHECK();
  *launched = true;
  return KVQ_OK;
}

int launch_int8_decode_mfma(const void*, int, int, int, int, float, const int8_t*, const int8_t*,
                            int, const void*, const void*, const int32_t*, int64_t,
                            const int32_t*, int64_t, float*, float*, hipStream_t,
                            bool* launched) {
  *launched = false;
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

extern "C" int kvq_selftest_lds_dma(const void* src, void* dst, void* stream) {
  if (!src || !dst) return KVQ_ERR_INVALID;
  hipLaunchKernelGGL(lds_dma_probe_kernel, dim3(1), dim3(64), 1280,
                     static_cast<hipStream_t>(stream), static_cast<const uint32_t*>(src),
                     static_cast<uint32_t*>(dst));
  KVQ_LAUNCH_CHECK();
  return KVQ_OK;
}
