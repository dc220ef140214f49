// SPDX-License-Identifier: Apache-2.0
// MFMA decode attention over INT8 per-channel pages (kind-0 work items) for
// gfx950.
//
// Reference: the fused decode with per-channel antiquant of
// pkg/methods/int8_dynamic/attention_backend.py:173-205 (antiquant_mode 0,
// offset 0): K = code * k_aq, V = code * v_aq per (kv head, dim), softmax in
// fp32.  Cache layout [NB, Bs, KVH, D] int8: one token of one kv head is a
// 128-byte row, the rows of a token's heads are adjacent.
//
// One wave per (work item, kv head), 32-token tiles double-buffered in the
// wave's 16 KB of LDS: global_load_lds DMA with 16-byte lanes brings whole
// 128-byte rows (one cache line each) while the previous tile computes.  On
// config 2 this ran 117 us against 126 us for register tiles loaded 32 bytes
// a lane (two requests per line), at 118 instead of 232 VGPRs.
//
// QK^T (v_mfma_f32_16x16x32_f16, S^T = K * Q'^T), per 16-token group j:
//   A = key codes, row = token, k = dim.  Lane (g, n) = (lane / 16, lane % 16)
//       reads the 32 contiguous bytes [32g, 32g + 32) of token row n and
//       takes dims 32g + 8s + i at k-step s.  A byte b becomes the exact fp16
//       code: v_perm places (b ^ 0x80) under the exponent byte 0x64 (fp16
//       1024 + b + 128) and one packed subtract of 1152 leaves b.
//   B = Q' = q * k_aq (exact in fp32 for bf16 / fp16 activations) scaled by a
//       power of two per head into fp16 range, split into hi + lo fp16 parts
//       (~22 bits): two MFMAs, or with GQA groups of at most 8 heads one MFMA
//       whose columns n and n + 8 carry the two parts (FOLD).  The softmax
//       scale * log2(e) and the inverse power of two multiply the fp32 scores.
// PV (O = P * V), one 32-token k-step per tile:
//   A = P (fp16), row = query head, k = token: lane (g, n) already holds p of
//       tokens 16j + 4g + r (j = 0, 1; r = 0..3) for head n from the QK
//       output layout, and uses exactly those tokens as its 8 k-values.
//   B = value codes, column n of tile t = dim 8n + t: the lane reads bytes
//       [8n, 8n + 8) of its 8 token rows and builds code pairs from byte t of
//       two rows (v_perm + or + packed subtract, exact).
//   v_aq multiplies the output per dim at the end.
// Online softmax in the log2 domain; each item leaves (m, l, o) per query head
// for the log-sum-exp combine.
//
// Tiles start on the 16-aligned position at or below the item's start, so
// with block_size % 16 == 0 every 16-token group lies in one page (one
// uniform page lookup per group).  Positions outside [start, end) are masked;
// their addresses are clamped to the group holding end - 1 and page ids to
// [0, num_blocks), so every load stays inside the cache and the table row.
#include "kvq_common.h"
#include "kvq_decode.h"

namespace {

using namespace kvq;

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));

constexpr int kD = 128;
constexpr int kTile = 32;  // tokens per tile: two groups of 16
constexpr uint32_t kExp64 = 0x64646464u;  // 0x64: high byte of fp16 1024 + u, u < 256
constexpr uint32_t kFlip = 0x80808080u;   // int8 code -> excess-128 byte

__device__ __forceinline__ h8 as_h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  u4v v = {a, b, c, d};
  return __builtin_bit_cast(h8, v);
}

__device__ __forceinline__ uint32_t minus1152(uint32_t pair) {
  const h2 v = __builtin_bit_cast(h2, pair) - h2{1152.0f16, 1152.0f16};
  return __builtin_bit_cast(uint32_t, v);
}

// Exact fp16 codes (bytes 2u, 2u + 1 of the excess-128 word x).
template <int U>
__device__ __forceinline__ uint32_t key_pair(uint32_t x) {
  // byte0 = x.b[2U], byte1 = 0x64, byte2 = x.b[2U + 1], byte3 = 0x64
  constexpr uint32_t sel = (2u * U) | (4u << 8) | ((2u * U + 1u) << 16) | (4u << 24);
  return minus1152(__builtin_amdgcn_perm(kExp64, x, sel));
}

// Exact fp16 codes (byte K of excess-128 word lo, byte K of word hi).
template <int K>
__device__ __forceinline__ uint32_t value_pair(uint32_t lo, uint32_t hi) {
  // byte0 = lo.b[K], byte1 = 0, byte2 = hi.b[K], byte3 = 0
  constexpr uint32_t sel = 0x0c000c00u | K | ((4u + K) << 16);
  return minus1152(__builtin_amdgcn_perm(hi, lo, sel) | 0x64006400u);
}

__device__ __forceinline__ uint32_t h2_bits(_Float16 a, _Float16 b) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, a)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, b)) << 16);
}

// One tile's codes in registers.  k[j][w]: word w of bytes [32g, 32g + 32) of
// token 16j + n; v[j][r]: bytes [8n, 8n + 8) of token 16j + 4g + r.
struct TileRegs {
  uint4 k[2][2];
  uint2 v[2][4];
};

struct WaveCtx {
  const int8_t* kc;
  const int8_t* vc;
  const int32_t* bt;  // this request's table row
  int64_t nb;
  int bs, kvh, h, g, n;
  int last_group;     // 16-aligned start of the group holding end - 1
};

// ---- LDS-staged tiles -------------------------------------------------------
// The tile's 32 key rows and 32 value rows (128 bytes each: one cache line per
// row) arrive by DMA in the wave's LDS, 16-byte lanes, eight lanes per row, so
// every request is a whole line.  Chunk c of row t (16 bytes) sits at position
// c ^ (t % 8): the operand reads of 16 rows spread over the banks.  The
// operand registers are then filled from LDS in the layout compute_tile reads.
constexpr int kTileBytes = 2 * kTile * kD;  // key rows, then value rows

__device__ __forceinline__ void issue_tile_dma(char* buf, const WaveCtx& c, int p, int lane) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    int gt = p + 16 * j;
    gt = gt < c.last_group ? gt : c.last_group;
    const int64_t b0 = c.bt[gt / c.bs];
    const int64_t blk = b0 < 0 ? 0 : (b0 >= c.nb ? c.nb - 1 : b0);
    const int64_t row0 = blk * c.bs + gt % c.bs;  // first token row of the group
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int r = 8 * half + lane / 8;           // row of the group
      const int chunk = (lane % 8) ^ (r % 8);      // global chunk for LDS position lane % 8
      const int64_t off = ((row0 + r) * c.kvh + c.h) * kD + 16 * chunk;
      char* dst = buf + (16 * j + 8 * half) * kD;  // the DMA adds 16 * lane
      dma16(c.kc + off, dst);
      dma16(c.vc + off, dst + kTile * kD);
    }
  }
}

__device__ __forceinline__ void read_tile_lds(TileRegs& t, const char* buf, int g, int n) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const char* kr = buf + (16 * j + n) * kD;  // row % 8 == n % 8
    t.k[j][0] = *reinterpret_cast<const uint4*>(kr + 16 * ((2 * g) ^ (n % 8)));
    t.k[j][1] = *reinterpret_cast<const uint4*>(kr + 16 * ((2 * g + 1) ^ (n % 8)));
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int vrow = 16 * j + 4 * g + r;
      const char* vr = buf + kTile * kD + vrow * kD;
      t.v[j][r] =
          *reinterpret_cast<const uint2*>(vr + 16 * ((n / 2) ^ (vrow % 8)) + 8 * (n % 2));
    }
  }
}

struct SoftmaxState {
  float m;    // running max of head n (log2 domain), same in the 4 lane groups
  float l;    // this lane's partial sum of p
  f4 o[8];    // o[t][r]: head 4g + r, dim 8n + t
};

// x + (x of lane n ^ 8 in the same 16-lane row): v_add_f32 with a DPP
// row_ror:8 operand.
__device__ __forceinline__ float add_ror8(float x) {
  const int y = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, false);
  return x + __int_as_float(y);
}

// FOLD (GQA groups of at most 8 heads): qh carries the hi part of head n in
// columns n < 8 and the lo part of head n - 8 in columns n >= 8, so one MFMA
// per k-step gives both partial scores and a rotate-by-8 add sums them (both
// lanes then hold head n % 8's score; ql unused).
template <bool FOLD>
__device__ __forceinline__ void compute_tile(const TileRegs& t, int p, int pb, int pe,
                                             const h8 (&qh)[4], const h8 (&ql)[4], float sc,
                                             int g, SoftmaxState& st) {
  // ---- S^T = K * Q'^T: 2 groups of 16 tokens ----
  f4 s[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    s[j] = f4{0.f, 0.f, 0.f, 0.f};
    const uint32_t w[8] = {t.k[j][0].x ^ kFlip, t.k[j][0].y ^ kFlip, t.k[j][0].z ^ kFlip,
                           t.k[j][0].w ^ kFlip, t.k[j][1].x ^ kFlip, t.k[j][1].y ^ kFlip,
                           t.k[j][1].z ^ kFlip, t.k[j][1].w ^ kFlip};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const h8 a = as_h8(key_pair<0>(w[2 * ks]), key_pair<1>(w[2 * ks]),
                         key_pair<0>(w[2 * ks + 1]), key_pair<1>(w[2 * ks + 1]));
      s[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qh[ks], s[j], 0, 0, 0);
      if (!FOLD) s[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ql[ks], s[j], 0, 0, 0);
    }
  }
  if (FOLD) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) s[j][r] = add_ror8(s[j][r]);
  }
  // ---- online softmax for head n over tokens 16j + 4g + r ----
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tok = p + 16 * j + 4 * g + r;
      const float v = (tok >= pb && tok < pe) ? s[j][r] * sc : -INFINITY;
      s[j][r] = v;
      mx = fmaxf(mx, v);
    }
  mx = max_rows4(mx);
  const float m_new = fmaxf(st.m, mx);
  // a fully masked prefix keeps m = -inf: nothing to rescale, p = 0
  const float m_use = m_new == -INFINITY ? 0.0f : m_new;
  const float alpha = st.m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(st.m - m_use);
  st.m = m_new;
  float psum = 0.0f;
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float pv = __builtin_amdgcn_exp2f(s[j][r] - m_use);  // exp2(-inf) = 0
      s[j][r] = pv;
      psum += pv;
    }
  st.l = st.l * alpha + psum;
  // o rows are heads 4g + r: their alphas live in lanes 4g + r
  if (__any(alpha != 1.0f)) {
    float a[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) a[r] = __shfl(alpha, 4 * g + r, 64);
#pragma unroll
    for (int tt = 0; tt < 8; ++tt)
#pragma unroll
      for (int r = 0; r < 4; ++r) st.o[tt][r] *= a[r];
  }
  // ---- O += P * V: one k-step of 32 tokens ----
  {
    const h8 a = as_h8(h2_bits(static_cast<_Float16>(s[0][0]), static_cast<_Float16>(s[0][1])),
                       h2_bits(static_cast<_Float16>(s[0][2]), static_cast<_Float16>(s[0][3])),
                       h2_bits(static_cast<_Float16>(s[1][0]), static_cast<_Float16>(s[1][1])),
                       h2_bits(static_cast<_Float16>(s[1][2]), static_cast<_Float16>(s[1][3])));
    // the lane's 8 tokens (i = 4j + r), bytes of dims 8n .. 8n + 7
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint2 x = t.v[i / 4][i % 4];
      lo[i] = x.x ^ kFlip;
      hi[i] = x.y ^ kFlip;
    }
#define KVQ_PV_TILE(TT, W, K)                                                                \
  {                                                                                          \
    const h8 b = as_h8(value_pair<K>(W[0], W[1]), value_pair<K>(W[2], W[3]),                 \
                       value_pair<K>(W[4], W[5]), value_pair<K>(W[6], W[7]));                \
    st.o[TT] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, st.o[TT], 0, 0, 0);            \
  }
    KVQ_PV_TILE(0, lo, 0)
    KVQ_PV_TILE(1, lo, 1)
    KVQ_PV_TILE(2, lo, 2)
    KVQ_PV_TILE(3, lo, 3)
    KVQ_PV_TILE(4, hi, 0)
    KVQ_PV_TILE(5, hi, 1)
    KVQ_PV_TILE(6, hi, 2)
    KVQ_PV_TILE(7, hi, 3)
#undef KVQ_PV_TILE
  }
}

// A workgroup holds hpw waves: kv heads q*hpw .. q*hpw + hpw - 1 of one work
// item, one wave per head, each with its own two tile buffers.  With hpw = kvh
// (the launcher's choice whenever the LDS allows) a barrier after every tile
// keeps the item's heads in step, so that the rows of one token, which the
// heads' K and V lines interleave in HBM, are requested together: the DRAM
// pages open once for all heads instead of once per head (config-2 decode
// 111.5 -> 101 us, one 8-wave workgroup per CU).
template <typename TQ, bool FOLD>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
int8_decode_mfma_kernel(const TQ* __restrict__ query, int hq, int kvh, int hpw, float qscale,
                        const int8_t* __restrict__ kc, const int8_t* __restrict__ vc, int bs,
                        int64_t nb, const TQ* __restrict__ k_aq, const TQ* __restrict__ v_aq,
                        const int32_t* __restrict__ block_table, int64_t maxb,
                        const int32_t* __restrict__ work, float* __restrict__ ws_o,
                        float* __restrict__ ws_ml) {
  const int groups = kvh / hpw;
  const int wi = blockIdx.x / groups;
  // wave-uniform; saying so keeps the DMA destinations in scalar registers
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = (blockIdx.x - wi * groups) * hpw + wave;
  const int lane = threadIdx.x & 63;
  const int32_t* wk = work + 4 * static_cast<int64_t>(wi);
  const int b = wk[0];
  const int pb = wk[1];
  const int pe = wk[2];
  const int rep = hq / kvh;
  const int n = lane & 15;
  const int g = lane >> 4;
  if (wk[3] != 0) {
    // an empty request's item: m = -inf, l = 0 (the combine gives it weight 0
    // and writes zeros when a request has nothing else)
    if (lane < rep) {
      const int64_t hh = static_cast<int64_t>(wi) * hq + static_cast<int64_t>(h) * rep + lane;
      ws_ml[2 * hh] = -INFINITY;
      ws_ml[2 * hh + 1] = 0.0f;
    }
    return;
  }

  // ---- Q' = q * k_aq for head n, dims 32g + 8s + i, scaled by 2^e ----
  float qf[32];
  float amax = 0.0f;
  {
    const int hn = FOLD ? (n & 7) : n;  // folded: columns n and n + 8 carry head n % 8
    const bool live = hn < rep;
    const TQ* qrow = query + (static_cast<int64_t>(b) * hq + h * rep + (live ? hn : 0)) * kD;
    const TQ* arow = k_aq + static_cast<int64_t>(h) * kD;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const int dim = 32 * g + i;
      const float x = to_f32(qrow[dim]) * to_f32(arow[dim]);
      qf[i] = live ? x : 0.0f;
      amax = fmaxf(amax, fabsf(qf[i]));
    }
  }
  amax = max_rows4(amax);
  int ex = 0;
  if (amax > 0.0f) (void)frexpf(amax, &ex);
  const int e = amax > 0.0f ? 15 - ex : 0;  // max |Q' * 2^e| in [2^14, 2^15)
  h8 qh[4], ql[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      _Float16 hh[2], ll[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const float x = ldexpf(qf[8 * ks + 2 * u + k], e);
        hh[k] = static_cast<_Float16>(x);
        ll[k] = static_cast<_Float16>(x - static_cast<float>(hh[k]));
      }
      hw[u] = h2_bits(hh[0], hh[1]);
      lw[u] = h2_bits(ll[0], ll[1]);
    }
    if (FOLD) {
      const bool lo_col = n >= 8;
      qh[ks] = as_h8(lo_col ? lw[0] : hw[0], lo_col ? lw[1] : hw[1], lo_col ? lw[2] : hw[2],
                     lo_col ? lw[3] : hw[3]);
    } else {
      qh[ks] = as_h8(hw[0], hw[1], hw[2], hw[3]);
      ql[ks] = as_h8(lw[0], lw[1], lw[2], lw[3]);
    }
  }
  const float sc = ldexpf(qscale, -e);

  WaveCtx c;
  c.kc = kc;
  c.vc = vc;
  c.bt = block_table + static_cast<int64_t>(b) * maxb;
  c.nb = nb;
  c.bs = bs;
  c.kvh = kvh;
  c.h = h;
  c.g = g;
  c.n = n;
  c.last_group = (pe - 1) & ~15;

  SoftmaxState st;
  st.m = -INFINITY;
  st.l = 0.0f;
#pragma unroll
  for (int tt = 0; tt < 8; ++tt) st.o[tt] = f4{0.f, 0.f, 0.f, 0.f};

  // two LDS buffers: tile i + 1's DMA is in flight while tile i computes.
  // Both are __restrict__ within a step, so the compiler's wait-count pass
  // knows the reads of `cur` cannot alias the DMA into `nxt`; the wait for
  // tile i itself is explicit.
  const int p0 = pb & ~15;
  extern __shared__ __align__(16) char lds_wg[];
  char* const lds_i8 = lds_wg + wave * 2 * kTileBytes;  // this wave's two tile buffers
  auto step = [&](const char* __restrict__ cur, char* __restrict__ nxt, int p) {
    if (p + kTile < pe) {
      issue_tile_dma(nxt, c, p + kTile, lane);
      wait_vmcnt<8>();  // the 8 DMA instructions of tile i + 1 may stay in flight
    } else {
      wait_vmcnt<0>();
    }
    TileRegs t;
    read_tile_lds(t, cur, g, n);
    compute_tile<FOLD>(t, p, pb, pe, qh, ql, sc, g, st);
  };
  if (p0 < pe) issue_tile_dma(lds_i8, c, p0, lane);  // an empty range leaves m = -inf, l = 0
  int cur = 0;
  for (int p = p0; p < pe; p += kTile) {
    step(lds_i8 + cur * kTileBytes, lds_i8 + (cur ^ 1) * kTileBytes, p);
    // every LDS read of this buffer is consumed before the next DMA into it
    asm volatile("" ::: "memory");
    cur ^= 1;
    if (hpw > 1) __syncthreads();  // uniform: the workgroup's heads share the item
  }

  // ---- epilogue ----
  float l = st.l;
  l = sum_rows4(l);
  float va[8];
#pragma unroll
  for (int tt = 0; tt < 8; ++tt) va[tt] = to_f32(v_aq[static_cast<int64_t>(h) * kD + 8 * n + tt]);
  const int64_t head0 = static_cast<int64_t>(wi) * hq + static_cast<int64_t>(h) * rep;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int hh = 4 * g + r;
    if (hh < rep) {
      float* dst = ws_o + (head0 + hh) * kD + 8 * n;
      float4 lo4, hi4;
      lo4.x = st.o[0][r] * va[0];
      lo4.y = st.o[1][r] * va[1];
      lo4.z = st.o[2][r] * va[2];
      lo4.w = st.o[3][r] * va[3];
      hi4.x = st.o[4][r] * va[4];
      hi4.y = st.o[5][r] * va[5];
      hi4.z = st.o[6][r] * va[6];
      hi4.w = st.o[7][r] * va[7];
      *reinterpret_cast<float4*>(dst) = lo4;
      *reinterpret_cast<float4*>(dst + 4) = hi4;
    }
  }
  if (g == 0 && n < rep) {
    ws_ml[2 * (head0 + n)] = st.m;
    ws_ml[2 * (head0 + n) + 1] = l;
  }
}

}  // namespace

namespace kvq {

int launch_int8_decode_mfma(const void* query, int dtype, int hq, int kvh, int d, float qscale,
                            const int8_t* kc, const int8_t* vc, int bs, int64_t nb,
                            const void* k_aq, const void* v_aq, const int32_t* block_table,
                            int64_t maxb, const int32_t* work, int64_t num_work, float* ws_o,
                            float* ws_ml, hipStream_t s, bool* launched) {
  *launched = false;
  if (d != kD || hq / kvh > 16 || bs % 16) return KVQ_OK;
  if (num_work * kvh > 0x7fffffff) return KVQ_ERR_INVALID;
  // all kv heads of an item in one workgroup when they fit (at most 8 waves
  // and their tile buffers in the workgroup's LDS), else one wave per head
  int64_t lds_max = 0;
  const int lrc = device_lds_max(&lds_max);
  if (lrc != KVQ_OK) return lrc;
  const int hpw = kvh <= 8 && kvh * 2 * kTileBytes <= lds_max ? kvh : 1;
  const dim3 grid(static_cast<unsigned>(num_work * (kvh / hpw)));
  // GQA groups of at most 8 heads fold the hi/lo score parts into one MFMA
  const bool fold = hq / kvh <= 8;
#define KVQ_LAUNCH_I8(TQ, F)                                                                  \
  hipLaunchKernelGGL((int8_decode_mfma_kernel<TQ, F>), grid, dim3(64 * hpw),                 \
                     hpw * 2 * kTileBytes, s, static_cast<const TQ*>(query), hq, kvh, hpw,   \
                     qscale, kc, vc, bs, nb,                                                 \
                     static_cast<const TQ*>(k_aq), static_cast<const TQ*>(v_aq), block_table,\
                     maxb, work, ws_o, ws_ml)
  KVQ_DISPATCH_FLOAT(dtype, TQ,
    if (fold) KVQ_LAUNCH_I8(TQ, true); else KVQ_LAUNCH_I8(TQ, false));
#undef KVQ_LAUNCH_I8
  KVQ_LAUNCH_CHECK();
  *launched = true;
  return KVQ_OK;
}

}  // namespace kvq
