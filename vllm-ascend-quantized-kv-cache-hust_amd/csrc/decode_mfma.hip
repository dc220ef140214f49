// SPDX-License-Identifier: Apache-2.0
// MFMA decode attention over KIVI int4 pages (kind-0 work items) for gfx950.
//
// One workgroup per work item, one wave per kv head.  A work item is a range
// of positions whose keys and values are both in int4 pages; the range is cut
// into "group tiles" of GT = 8*CPG tokens (CPG = min(16, G/8) 8-token chunks),
// each inside one page and one key-scale group.
//
// QK^T (v_mfma_f32_16x16x32_f16, S^T = K * Q'^T):
//   A = key codes, row m = token, 8 head dims per lane.  A key word packs 8
//       tokens of one dim, so a lane loads 8 words (8 dims x 8 tokens of its
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

constexpr int kHeadsPerWg = 4;  // waves (kv heads) per workgroup

template <typename TQ, int CPG>
__global__ void __launch_bounds__(256, 2)
kivi_decode_mfma_kernel(const TQ* __restrict__ query, int hq, int kvh, float qscale,
                        const uint32_t* __restrict__ kq, const float* __restrict__ ks,
                        const float* __restrict__ km, const uint32_t* __restrict__ vq,
                        const float* __restrict__ vs, const float* __restrict__ vm, int bs,
                        int g, const int32_t* __restrict__ block_table, int64_t maxb,
                        const int32_t* __restrict__ work, float* __restrict__ ws_o,
                        float* __restrict__ ws_ml) {
  constexpr int D = 128;
  constexpr int GT = 8 * CPG;    // tokens per group tile
  constexpr int NJ = CPG / 2;    // score MFMAs per k-step (16 tokens each)
  constexpr int SUB = 16 / CPG;  // tokens of one chunk inside one score MFMA
  constexpr int NVG = 16 / CPG;  // PV column groups (one value group each)
  constexpr int NJJ = CPG / 2;   // PV MFMAs per column group (NVG * NJJ == 8)
  constexpr int PVS = CPG / 4;   // PV k-steps (32 tokens) per group tile
  constexpr int HW = kHeadsPerWg;

  __shared__ uint32_t s_kw[HW * D * CPG];       // key words   [hl][d][chunk]
  __shared__ uint32_t s_vw[HW * GT * 16];       // value words [hl][t][word]
  __shared__ float s_ks[HW * D], s_km[HW * D];  // key scale/min of the tile's group
  __shared__ float s_vs[GT * HW * NVG], s_vm[GT * HW * NVG];  // value scale/min [t][hl][vg]

  const int wi = blockIdx.x;
  const int h0 = blockIdx.y * HW;
  const int tid = threadIdx.x;
  const int hl = tid >> 6;
  const int h = h0 + hl;
  const int lane = tid & 63;
  const int32_t* wk = work + 4 * static_cast<int64_t>(wi);
  if (wk[3] != 0) return;  // kind-1 items belong to the generic kernel (uniform)
  const int heads = (kvh - h0) < HW ? (kvh - h0) : HW;
  const bool wave_live = hl < heads;
  const int b = wk[0];
  const int pb = wk[1];
  const int pe = wk[2];
  const int rep = hq / kvh;
  const int n = lane & 15;
  const int kg = lane >> 4;
  const int gpb = bs / g;
  const int wpd = bs / 8;
  const int ng = D / g;  // == NVG: the kernel runs only for 8*CPG == G <= 128
  const int32_t* bt = block_table + static_cast<int64_t>(b) * maxb;

  // q of head n for the lane's dims d = 32*s + 4*i + kg, kept in the input
  // dtype (two 16-bit values per VGPR); softmax scale * log2(e) applies on use
  TQ qv[32];
  {
    const bool live = wave_live && n < rep;
    const TQ* qrow = query + (static_cast<int64_t>(b) * hq + (live ? h * rep + n : 0)) * D;
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        qv[8 * s4 + i] = live ? qrow[32 * s4 + 4 * i + kg] : from_f32<TQ>(0.0f);
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

  for (int p0 = pb; p0 < pe; p0 += GT) {
    const int64_t blk = bt[p0 / bs];
    const int off0 = p0 % bs;
    const int grp = off0 / g;
    __syncthreads();  // the previous tile's LDS reads are done
    // ---- stage the tile: every load 16 B and coalesced -------------------
    {
      // key words: row (hl, d) holds CPG words at kq[((blk*kvh + h)*D + d)*wpd + off0/8]
      constexpr int QPR = CPG / 4;  // 16-byte pieces per row
      for (int e = tid; e < heads * D * QPR; e += 64 * HW) {
        const int row = e / QPR;
        const int q4 = e - row * QPR;
        const int rh = row / D;
        const int d = row - rh * D;
        const uint4 w = *reinterpret_cast<const uint4*>(
            kq + ((blk * kvh + h0 + rh) * D + d) * wpd + off0 / 8 + 4 * q4);
        *reinterpret_cast<uint4*>(s_kw + row * CPG + 4 * q4) = w;
      }
      // value words: token t, head hl -> 16 words (64 B)
      for (int e = tid; e < GT * heads * 4; e += 64 * HW) {
        const int q4 = e & 3;
        const int th = e >> 2;
        const int t = th / heads;
        const int rh = th - t * heads;
        const uint4 w = *reinterpret_cast<const uint4*>(
            vq + ((blk * bs + off0 + t) * kvh + h0 + rh) * 16 + 4 * q4);
        *reinterpret_cast<uint4*>(s_vw + (rh * GT + t) * 16 + 4 * q4) = w;
      }
      for (int e = tid; e < heads * D; e += 64 * HW) {
        const int rh = e / D;
        const int d = e - rh * D;
        const int64_t idx = ((blk * kvh + h0 + rh) * D + d) * gpb + grp;
        s_ks[e] = ks[idx];
        s_km[e] = km[idx];
      }
      for (int e = tid; e < GT * heads * ng; e += 64 * HW) {
        const int vg = e % ng;
        const int th = e / ng;
        const int t = th / heads;
        const int rh = th - t * heads;
        // positions past the range keep p = 0; zeroing their scale/min keeps
        // p*scale and p*min exact zeros without a branch (the bytes past the
        // sequence end are not written history and may hold anything)
        const bool live_t = p0 + t < pe;
        const int64_t idx = ((blk * bs + off0 + t) * kvh + h0 + rh) * ng + vg;
        s_vs[(t * HW + rh) * NVG + vg] = live_t ? vs[idx] : 0.0f;
        s_vm[(t * HW + rh) * NVG + vg] = live_t ? vm[idx] : 0.0f;
      }
    }
    __syncthreads();
    if (!wave_live) continue;

    // ---- scores: per k-step, Q' for this key group then the MFMAs -------
    const float* sks = s_ks + hl * D;
    const float* skm = s_km + hl * D;
    const uint32_t* skw = s_kw + hl * D * CPG;
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
      __builtin_amdgcn_sched_barrier(0);
    }
    kb = sum_kg(kb);
    // lane holds head n, rows m' = 4*kg + r: token 8*(m' % CPG) + jm*SUB + m'/CPG
    const float kcorr = kb;
    float tmax = -INFINITY;
#pragma unroll
    for (int jm = 0; jm < NJ; ++jm) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int mr = 4 * kg + r;
        const int pos = p0 + 8 * (mr % CPG) + jm * SUB + mr / CPG;
        const float sv = pos < pe ? sacc[jm][r] + kcorr : -INFINITY;
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

    // ---- PV ----------------------------------------------------------------
    const uint32_t* svw = s_vw + hl * GT * 16;
#pragma unroll
    for (int st = 0; st < PVS; ++st) {
      int tk[8];
      float pv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int jm = 2 * st + i / 4;
        const int mr = 4 * kg + (i % 4);
        tk[i] = 8 * (mr % CPG) + jm * SUB + mr / CPG;
        pv[i] = sacc[jm][i % 4];
      }
#pragma unroll
      for (int v = 0; v < NVG; ++v) {
        const int vgrp = (8 * CPG * v) / g;
        float pp[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float sc = s_vs[(tk[i] * HW + hl) * NVG + vgrp];
          const float mn = s_vm[(tk[i] * HW + hl) * NVG + vgrp];
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
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (!wave_live) return;

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
                            const int32_t* block_table, int64_t maxb, const int32_t* seq_meta,
                            const int32_t* work, int64_t num_work, float* ws_o, float* ws_ml,
                            hipStream_t s, bool* launched) {
  (void)seq_meta;
  *launched = false;
  if (d != 128 || hq / kvh > 16 || g < 32 || g % 8 || d % g) return KVQ_OK;
  const int cpg = g / 8 >= 16 ? 16 : g / 8;
  if (cpg != 16 && cpg != 8 && cpg != 4) return KVQ_OK;
  if (g > 128) return KVQ_OK;  // one value group per 16 MFMA columns needs G <= 128
  const dim3 grid(static_cast<unsigned>(num_work), (kvh + kHeadsPerWg - 1) / kHeadsPerWg);
  const dim3 block(64 * kHeadsPerWg);
  const uint32_t* kqu = reinterpret_cast<const uint32_t*>(kq);
  const uint32_t* vqu = reinterpret_cast<const uint32_t*>(vq);
#define KVQ_LAUNCH_MFMA(C)                                                                   \
  KVQ_DISPATCH_FLOAT(q_dtype, TQ,                                                           \
    hipLaunchKernelGGL((kivi_decode_mfma_kernel<TQ, C>), grid, block, 0, s,                 \
                       static_cast<const TQ*>(query), hq, kvh, qscale, kqu, ks, km, vqu, vs, \
                       vm, bs, g, block_table, maxb, work, ws_o, ws_ml))
  if (cpg == 16) {
    KVQ_LAUNCH_MFMA(16);
  } else if (cpg == 8) {
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
