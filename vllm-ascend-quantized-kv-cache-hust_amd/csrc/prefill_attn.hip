// SPDX-License-Identifier: Apache-2.0
// Causal (or full) attention over dense TND K/V on MFMA, for prefill and the
// prompt rows of a chunked batch.
//
// Replaces the NPU fused-attention calls with input_layout "TND":
// pkg/methods/kivi_int4/attention_backend.py:1248-1262 (PrefillNoCache),
// :1320-1334 (chunked prompt rows), the dense fallback :1341-1392, and the
// INT8 prefill paths pkg/methods/int8_dynamic/attention_backend.py:282-296,
// 350-364.  Query row i of a request with lq queries and lk keys sits at
// position lk - lq + i; with `causal`, key positions past it are masked
// (pkg/methods/kivi_int4/semantics.py:285-299).
//
// bf16/fp16 inputs with head_size 64 or 128 run prefill_attn_fa_kernel
// (64-key blocks, DMA-staged K, transposed V, described at the kernel).  The
// kernel below covers the rest (fp32 inputs, head_size 32 and 256):
// one workgroup = 4 waves = 64 query rows of one query head; each wave owns
// 16 rows.  Keys/values stream through LDS in 32-token blocks.
//   S^T = K * Q^T   (v_mfma_f32_16x16x32_{bf16,f16}): A = K rows from LDS
//                   (16-byte reads), B = Q^T from registers (loaded once).
//   O^T += V^T * P^T: B = P^T straight from the S^T result registers (each
//                   lane already holds its query row's 8 probabilities);
//                   A = V^T read from the LDS block.
// Online softmax in the log2 domain, fp32 accumulation, output in the input
// dtype (fp32 inputs run through bf16 operands).
#include "kvq_common.h"

namespace {

using namespace kvq;

typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef uint16_t u8v __attribute__((ext_vector_type(8)));

constexpr int kRowsPerWave = 16;
constexpr int kWaves = 4;
constexpr int kKvBlock = 32;

// Operand element type of the MFMA for an input type.
template <typename T> struct Op { using type = bf16; };
template <> struct Op<f16> { using type = f16; };

__device__ __forceinline__ uint16_t op_bits(float x, bf16) { return f32_to_bf16_bits(x); }
__device__ __forceinline__ uint16_t op_bits(float x, f16) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}
template <typename T>
__device__ __forceinline__ uint16_t raw_bits(T v) {
  return op_bits(to_f32(v), typename Op<T>::type{});
}
template <>
__device__ __forceinline__ uint16_t raw_bits<bf16>(bf16 v) { return v.bits; }
template <>
__device__ __forceinline__ uint16_t raw_bits<f16>(f16 v) { return __builtin_bit_cast(uint16_t, v); }

__device__ __forceinline__ float op_to_f32(uint16_t bits, bf16) {
  return __uint_as_float(static_cast<uint32_t>(bits) << 16);
}
__device__ __forceinline__ float op_to_f32(uint16_t bits, f16) {
  return static_cast<float>(__builtin_bit_cast(_Float16, bits));
}

// Two fp32 values as an operand pair (round to nearest even), and back.
__device__ __forceinline__ uint32_t pack_op2(float lo, float hi, bf16) { return bf16x2_bits(lo, hi); }
__device__ __forceinline__ uint32_t pack_op2(float lo, float hi, f16) {
  typedef float f2v __attribute__((ext_vector_type(2)));
  typedef _Float16 h2v __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2v{lo, hi}), h2v));
}
__device__ __forceinline__ float op_lo_f32(uint32_t w, bf16) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float op_hi_f32(uint32_t w, bf16) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float op_lo_f32(uint32_t w, f16) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w)));
}
__device__ __forceinline__ float op_hi_f32(uint32_t w, f16) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
}

__device__ __forceinline__ f4 mfma16(u8v a, u8v b, f4 c, bf16) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8, a), __builtin_bit_cast(b8, b),
                                                 c, 0, 0, 0);
}
__device__ __forceinline__ f4 mfma16(u8v a, u8v b, f4 c, f16) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a), __builtin_bit_cast(h8, b),
                                                c, 0, 0, 0);
}

// Eight consecutive elements as operand bits (one 16-byte load for 16-bit types).
template <typename T>
__device__ __forceinline__ u8v load_op8(const T* p) {
  u8v r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = raw_bits(p[i]);
  return r;
}
template <>
__device__ __forceinline__ u8v load_op8<bf16>(const bf16* p) {
  return *reinterpret_cast<const u8v*>(p);
}
template <>
__device__ __forceinline__ u8v load_op8<f16>(const f16* p) {
  return *reinterpret_cast<const u8v*>(p);
}

template <typename T, int D>
__global__ void __launch_bounds__(256)
prefill_attn_kernel(const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
                    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k, int hq,
                    int kvh, float qscale, int causal, T* __restrict__ out) {
  using O = typename Op<T>::type;
  constexpr int KS = D / 32;   // k-steps of the score MFMA
  constexpr int DB = D / 16;   // 16-dim output blocks
  __shared__ uint16_t s_k[kKvBlock * D];
  __shared__ uint16_t s_v[kKvBlock * D];

  const int b = blockIdx.z;
  const int head = blockIdx.y;
  const int kvhead = head / (hq / kvh);
  const int q_start = cu_q[b];
  const int lq = cu_q[b + 1] - q_start;
  const int k_start = cu_k[b];
  const int lk = cu_k[b + 1] - k_start;
  const int row0 = blockIdx.x * (kRowsPerWave * kWaves);
  if (row0 >= lq) return;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int n = lane & 15;
  const int kg = lane >> 4;
  const int wrow0 = row0 + wave * kRowsPerWave;
  const int my_row = wrow0 + n;           // query row of the lane's column
  const bool row_live = my_row < lq;
  const int my_pos = lk - lq + my_row;    // its kv position
  // kv range the workgroup needs
  const int last_row = min(row0 + kRowsPerWave * kWaves, lq) - 1;
  const int kv_end = causal ? min(lk, lk - lq + last_row + 1) : lk;

  // Q^T operand: lane (col n = query row, k-group kg) holds dims 32*s + 8*kg + i
  u8v qop[KS];
  {
    const T* qrow = q + (static_cast<int64_t>(q_start + (row_live ? my_row : 0)) * hq + head) * D;
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int i = 0; i < 8; ++i)  // unscaled: exact in the operand type
        qop[s][i] = row_live ? raw_bits(qrow[32 * s + 8 * kg + i]) : uint16_t(0);
  }

  float m_run = -INFINITY, l_run = 0.0f;
  f4 o[DB];
#pragma unroll
  for (int j = 0; j < DB; ++j) o[j] = f4{0.f, 0.f, 0.f, 0.f};

  for (int kb = 0; kb < kv_end; kb += kKvBlock) {
    __syncthreads();
    // stage K and V rows [kb, kb + 32) of this kv head (16-byte loads)
    constexpr int QPR = D / 8;  // 8-element pieces per row
    for (int e = tid; e < kKvBlock * QPR; e += 256) {
      const int t = e / QPR;
      const int c = (e - t * QPR) * 8;
      const int pos = kb + t;
      u8v kvv, vvv;
      if (pos < lk) {
        const int64_t src = (static_cast<int64_t>(k_start + pos) * kvh + kvhead) * D + c;
        kvv = load_op8(k + src);
        vvv = load_op8(v + src);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          kvv[i] = 0;
          vvv[i] = 0;
        }
      }
      *reinterpret_cast<u8v*>(s_k + t * D + c) = kvv;
      *reinterpret_cast<u8v*>(s_v + t * D + c) = vvv;
    }
    __syncthreads();
    // waves whose rows are all before this block under the causal mask skip it
    const int wave_last_pos = lk - lq + min(wrow0 + kRowsPerWave, lq) - 1;
    if (wrow0 >= lq || (causal && kb > wave_last_pos)) continue;

    // scores: two 16-token halves; lane holds query row n, tokens 4*kg + r (+16)
    f4 s0 = f4{0.f, 0.f, 0.f, 0.f}, s1 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u8v a0 = *reinterpret_cast<const u8v*>(s_k + n * D + 32 * s + 8 * kg);
      const u8v a1 = *reinterpret_cast<const u8v*>(s_k + (16 + n) * D + 32 * s + 8 * kg);
      s0 = mfma16(a0, qop[s], s0, O{});
      s1 = mfma16(a1, qop[s], s1, O{});
    }
    float sc[8];
    float tmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int p0 = kb + 4 * kg + r;
      const int p1 = p0 + 16;
      const bool ok0 = p0 < lk && (!causal || p0 <= my_pos);
      const bool ok1 = p1 < lk && (!causal || p1 <= my_pos);
      sc[r] = ok0 ? s0[r] * qscale : -INFINITY;
      sc[4 + r] = ok1 ? s1[r] * qscale : -INFINITY;
      tmax = fmaxf(tmax, fmaxf(sc[r], sc[4 + r]));
    }
    tmax = max_rows4(tmax);
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = m_run == -INFINITY ? (m_new == -INFINITY ? 1.0f : 0.0f)
                                           : exp2f(m_run - m_new);
    float psum = 0.0f;
    u8v pop;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float p = m_new == -INFINITY ? 0.0f : exp2f(sc[i] - m_new);
      pop[i] = op_bits(p, O{});
      // normalise by the probabilities the MFMA actually sees
      psum += op_to_f32(pop[i], O{});
    }
    psum = sum_rows4(psum);
    l_run = l_run * alpha + psum;
    m_run = m_new;
    // PV: A = V^T rows (dims), 8 tokens {4*kg + r, 16 + 4*kg + r}
#pragma unroll
    for (int j = 0; j < DB; ++j) {
      const int dim = 16 * j + n;
      u8v a;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        a[r] = s_v[(4 * kg + r) * D + dim];
        a[4 + r] = s_v[(16 + 4 * kg + r) * D + dim];
      }
      o[j] *= alpha;
      o[j] = mfma16(a, pop, o[j], O{});
    }
  }
  if (!row_live) return;
  // o[j][r] = O^T[dim 16*j + 4*kg + r][row n]
  const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
  T* orow = out + (static_cast<int64_t>(q_start + my_row) * hq + head) * D;
#pragma unroll
  for (int j = 0; j < DB; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) orow[16 * j + 4 * kg + r] = from_f32<T>(o[j][r] * inv);
}

// ---- 64-key-block kernel for 16-bit inputs, D in {64, 128} ------------------
// One workgroup = 4 waves x 32 query rows (two 16-row MFMA column groups) of one
// query head; key/value blocks of 64 tokens, double-buffered in LDS with one
// barrier per block:
//   K  [64][D]    written by global_load_lds (16-byte lanes); the 16-byte
//                 column of each row is XOR-swizzled by the row so that the
//                 16 rows one score MFMA reads sit in different banks;
//   V  [64][D]    written by global_load_lds too, row-major; 16-byte column
//                 c of row r stored at c ^ (2*(r % 4) + 8*((r / 4) % 2)) (the
//                 second term at D = 128), so that the rows the transposing
//                 reads of one LDS cycle cover sit in different banks.
// Keys run one block ahead of values: the step of block i computes block i's
// softmax and PV and block i+1's scores, whose MFMAs interleave with block
// i's exponentials (independent work, one basic block); block i+2's keys and
// block i+1's values are in flight (DMA) meanwhile.
//   S^T = K * Q^T: A = 16 keys x 32 dims (one 16-byte read per lane), B = the
//                  wave's Q^T (registers), each A feeding both column groups.
//   O^T += V^T * P^T: B = P^T straight from the S^T registers (the lane's
//                  keys 16*(2ks + i/4) + 4*kg + i%4 of its query column),
//                  A = the same 8 keys of one dim, gathered out of the
//                  row-major V by two transposing LDS reads
//                  (ds_read_b64_tr_b16: within each 16-lane group, lane l gets
//                  element l % 4 of the 8-byte runs that lanes l / 4 + 4k
//                  address, k = 0..3).
// The rescale needs no shuffles: S^T and O^T both put the lane's query in
// its column.
// The common step's softmax is the row maxima, one compare per column, and an
// fma and exp2 per score; the offset bookkeeping (new offset, rescale factor)
// sits in the branch that the lazy offset rarely takes.

constexpr int kFaGroupRows = 128;  // query rows per workgroup
constexpr int kFaXcds = 8;         // XCDs workgroup ids are dealt over
constexpr int kFaBlock = 64;  // keys per block
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s* lds_v4s_ptr;

// LDS DMA of 16 bytes per lane from base + voff (base uniform, in SGPRs;
// voff the lane's 32-bit byte offset) to LDS bytes m0 + 16 * lane (m0
// uniform), so no 64-bit address is formed per lane.  The s_nop covers the
// M0-write hazard.  Inline asm, outside the compiler's wait counting: the
// kernel waits for every block's DMA explicitly (wait_vmcnt<0> before the
// barrier that publishes it).
__device__ __forceinline__ void dma16_so(const char* base, uint32_t voff, uint32_t m0) {
  m0 = __builtin_amdgcn_readfirstlane(m0);
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(base), "{m0}"(m0)
               : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)(p)));
}

template <int D>
struct FaLds {
  static constexpr int K_BYTES = kFaBlock * D * 2;
  static constexpr int V_BYTES = kFaBlock * D * 2;
  static constexpr int BUF = K_BYTES + V_BYTES;
  static constexpr int BYTES = 2 * BUF;
};

// NG 16-row query column groups per wave; the workgroup's 8 / NG waves cover
// 128 rows and share the LDS blocks.  The launcher uses NG = 2 (4 waves of 32
// rows, 2 waves per SIMD): each LDS operand feeds two MFMAs.  NG = 1 (8 waves
// of 16 rows, 4 per SIMD) measured 26% slower on config 4 (twice the LDS reads
// per MFMA, and spills at the 128-VGPR limit of 4 waves per SIMD).
template <typename T, int D, int NG>
__global__ void __launch_bounds__(64 * (8 / NG))
__attribute__((amdgpu_waves_per_eu(4 / NG, 4 / NG)))
prefill_attn_fa_kernel(const T* __restrict__ q, const T* __restrict__ k,
                       const T* __restrict__ v, const int32_t* __restrict__ cu_q,
                       const int32_t* __restrict__ cu_k, int hq, int kvh, float qscale,
                       int causal, int qblocks, int batch, T* __restrict__ out) {
  using O = typename Op<T>::type;
  using L = FaLds<D>;
  constexpr int kFaWaves = 8 / NG;
  constexpr int kFaRows = 16 * NG;  // query rows per wave
  constexpr int KS = D / 32;      // score k-steps
  constexpr int DB = D / 16;      // output dim blocks
  constexpr int PPR = D / 8;      // 16-byte pieces per row
  constexpr int RPI = 64 / PPR;   // K rows per DMA instruction
  constexpr int KINST = kFaBlock / RPI / kFaWaves;  // DMA instructions per wave per block
  static_assert(KINST >= 1 && kFaBlock % (RPI * kFaWaves) == 0, "K / V DMA split");
  static_assert(PPR >= 8, "V swizzle 2 * (r % 4) stays inside the row");
  // V's 16-byte column c of row r sits at c ^ vswz(r): 2 (r % 4) spreads the
  // four rows one transposing read covers over the banks, and with 16 columns
  // a row (D = 128) 8 ((r / 4) % 2) also parts the rows 4 apart that the two
  // 16-lane groups of one LDS cycle read
  auto vswz = [](int r) { return 2 * (r % 4) + (PPR >= 16 ? 8 * ((r / 4) % 2) : 0); };
  extern __shared__ __align__(16) char lds[];
  const uint32_t lds0 = lds_addr(lds);  // LDS byte address of the buffers (DMA M0)

  // Workgroup ids go to the XCDs round-robin.  The rep * qblocks workgroups
  // that stream one (request, kv head)'s K/V run on one XCD, one such pair
  // after another, so that XCD's L2 keeps the pair's blocks between them;
  // inside a pair the heavy query blocks (more keys under the causal mask)
  // come first, the pair's query heads interleaved.
  const int rep = hq / kvh;
  const int per_pair = rep * qblocks;
  const int xcd = static_cast<int>(blockIdx.x) % kFaXcds;
  const int xj = static_cast<int>(blockIdx.x) / kFaXcds;
  const int pair = xcd + kFaXcds * (xj / per_pair);
  if (pair >= batch * kvh) return;  // padding of the last round
  const int w = xj % per_pair;
  const int b = pair / kvh;
  const int kvhead = pair - b * kvh;
  const int head = kvhead * rep + w % rep;
  const int qb = qblocks - 1 - w / rep;
  const int q_start = cu_q[b];
  const int lq = cu_q[b + 1] - q_start;
  const int k_start = cu_k[b];
  const int lk = cu_k[b + 1] - k_start;
  const int row0 = qb * (kFaRows * kFaWaves);
  if (row0 >= lq || lk <= 0) return;  // uniform over the workgroup
  const int tid = threadIdx.x;
  // wave-uniform; saying so keeps the DMA destinations in scalar registers
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int n = lane & 15;
  const int kg = lane >> 4;
  const int wrow0 = row0 + wave * kFaRows;
  const int last_row = min(row0 + kFaRows * kFaWaves, lq) - 1;
  const int kv_end = causal ? min(lk, lk - lq + last_row + 1) : lk;
  const int nblk = (kv_end + kFaBlock - 1) / kFaBlock;
  const int wave_last = min(wrow0 + kFaRows, lq) - 1;  // < wrow0 when the wave has no rows
  const int wave_last_pos = lk - lq + wave_last;

  // Q^T operands: group g2, k-step s: query row wrow0 + 16*g2 + n, dims 32s + 8kg + i
  // (unscaled: exact in the operand type)
  u8v qop[NG][KS];
  int my_pos[NG];
  bool live[NG];
#pragma unroll
  for (int g2 = 0; g2 < NG; ++g2) {
    const int row = wrow0 + 16 * g2 + n;
    live[g2] = row < lq;
    my_pos[g2] = lk - lq + row;
    const T* qrow = q + (static_cast<int64_t>(q_start + (live[g2] ? row : 0)) * hq + head) * D;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      u8v x = load_op8(qrow + 32 * s + 8 * kg);
      if (!live[g2]) x = u8v{0, 0, 0, 0, 0, 0, 0, 0};
      qop[g2][s] = x;
    }
  }

  // ---- staging ----
  const T* kbase = k + (static_cast<int64_t>(k_start) * kvh + kvhead) * D;
  const T* vbase = v + (static_cast<int64_t>(k_start) * kvh + kvhead) * D;
  const int64_t row_stride = static_cast<int64_t>(kvh) * D;
  // per-lane byte offsets of the K and V rows this lane moves (row r of the
  // block, swizzled piece), relative to the block's first row: 32-bit, so
  // that every DMA is a uniform base plus a lane offset
  uint32_t koff[KINST], voff[KINST];
  int krow[KINST];
#pragma unroll
  for (int i = 0; i < KINST; ++i) {
    const int inst = wave * KINST + i;
    const int r = inst * RPI + lane / PPR;  // block row of this lane
    krow[i] = r;
    koff[i] = static_cast<uint32_t>((r * row_stride + 8 * ((lane % PPR) ^ (r % PPR))) * 2);
    voff[i] = static_cast<uint32_t>((r * row_stride + 8 * ((lane % PPR) ^ vswz(r))) * 2);
  }
  // DMA of block rows kb .. kb + 63 of `base` into `dst` with the lane
  // offsets `off`; in the last block rows past the end read the last row
  // (masked later)
  auto issue_rows = [&](const T* base, const uint32_t (&off)[KINST], char* dst, int kb) {
    const char* gb = reinterpret_cast<const char*>(base + static_cast<int64_t>(kb) * row_stride);
    if (kb + kFaBlock <= lk) {  // uniform: only the last block clamps
#pragma unroll
      for (int i = 0; i < KINST; ++i)
        dma16_so(gb, off[i], lds0 + static_cast<uint32_t>(dst - lds) + 1024u * (wave * KINST + i));
    } else {
#pragma unroll
      for (int i = 0; i < KINST; ++i) {
        // rows past the end step back to row lk - 1 - kb of the block (>= 0),
        // so the offset from the block's first row stays non-negative
        const int back = kb + krow[i] >= lk ? kb + krow[i] - (lk - 1) : 0;
        dma16_so(gb, off[i] - static_cast<uint32_t>(back) * static_cast<uint32_t>(row_stride * 2),
                 lds0 + static_cast<uint32_t>(dst - lds) + 1024u * (wave * KINST + i));
      }
    }
  };
  // PV operand reads: lane s of a 16-lane group addresses V row keybase + s / 4,
  // dims 16j + 4 (s % 4) .. + 3 (swizzled 16-byte column), so that lane n of
  // the group receives V[keybase + k][16j + n], k = 0..3
  const int tr_row = lane % 16 / 4;
  const int tr_chunk = (lane % 4) / 2;  // + 2j
  const int tr_half = 8 * (lane % 2);   // byte offset inside the 16-byte column

  // Per query column: m_run, the raw score the exponent offset stands for
  // (-inf before the first finite score); m_off = -qscale * m_run (0 while
  // m_run is -inf), so p = 2^(qscale * s + m_off); m_thr = m_run + 8 / qscale,
  // the raw score past which the offset moves (lazy offset, below).
  const float lazy_thr = 8.0f / qscale;  // qscale > 0
  float m_run[NG], m_off[NG], m_thr[NG];
#pragma unroll
  for (int g2 = 0; g2 < NG; ++g2) {
    m_run[g2] = -INFINITY;
    m_off[g2] = 0.0f;
    m_thr[g2] = -INFINITY;
  }
  // l_acc[g2]: every row holds the running sum of the (rounded) P of query
  // column n, accumulated by an MFMA with an all-ones A, so it is the exact sum
  // of what the PV MFMAs saw and rescales together with o
  f4 l_acc[NG];
  f4 o[DB][NG];
#pragma unroll
  for (int g2 = 0; g2 < NG; ++g2) {
    l_acc[g2] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < DB; ++j) o[j][g2] = f4{0.f, 0.f, 0.f, 0.f};
  }
  const uint16_t one = op_bits(1.0f, O{});
  const u8v ones = u8v{one, one, one, one, one, one, one, one};

  // LDS: two key buffers and two value buffers.  Keys run one block ahead of
  // values: step i computes block i's softmax and PV and block i + 1's scores
  // (the score MFMAs interleaved with the softmax's exponentials, which do not
  // depend on them), while block i + 2's keys and block i + 1's values arrive.
  char* const kbuf0 = lds;
  char* const kbuf1 = lds + L::K_BYTES;
  char* const vbuf0 = lds + 2 * L::K_BYTES;
  char* const vbuf1 = lds + 2 * L::K_BYTES + L::V_BYTES;
  // waves whose rows all precede block i under the causal mask skip it (and
  // every later block)
  auto active = [&](int i) {
    return wrow0 <= wave_last && !(causal && i * kFaBlock > wave_last_pos);
  };
  // the K operands of 16-key group kb2 of the block at `sk`
  auto k_reads = [&](const uint16_t* sk, int kb2, u8v (&a)[KS]) {
    const int r = 16 * kb2 + n;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int piece = (4 * s + kg) ^ (r % PPR);
      a[s] = *reinterpret_cast<const u8v*>(sk + r * D + 8 * piece);
    }
  };
  auto k_mfmas = [&](const u8v (&a)[KS], f4 (&acc)[NG]) {
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int g2 = 0; g2 < NG; ++g2) acc[g2] = mfma16(a[s], qop[g2][s], acc[g2], O{});
  };

  // prologue: keys of blocks 0 and 1, values of block 0; scores of block 0
  issue_rows(kbase, koff, kbuf0, 0);
  if (nblk > 1) issue_rows(kbase, koff, kbuf1, kFaBlock);
  issue_rows(vbase, voff, vbuf0, 0);
  wait_vmcnt<0>();  // landed in LDS
  __syncthreads();
  f4 sacc[4][NG];
#pragma unroll
  for (int kb2 = 0; kb2 < 4; ++kb2)
#pragma unroll
    for (int g2 = 0; g2 < NG; ++g2) sacc[kb2][g2] = f4{0.f, 0.f, 0.f, 0.f};
  if (active(0)) {
#pragma unroll
    for (int kb2 = 0; kb2 < 4; ++kb2) {
      u8v a[KS];
      k_reads(reinterpret_cast<const uint16_t*>(kbuf0), kb2, a);
      k_mfmas(a, sacc[kb2]);
    }
  }
  __syncthreads();  // block 0's keys are read before block 2's overwrite them

  // One block step.  The four buffers are __restrict__ within the step, so
  // the compiler's wait-count pass knows that the LDS reads of `kn` (block
  // i + 1's keys) and `vc` (block i's values) cannot alias the DMA in flight
  // into `kd` and `vd` (otherwise it waits for that DMA before the first read).
  auto step = [&](const char* __restrict__ kn, const char* __restrict__ vc,
                  char* __restrict__ kd, char* __restrict__ vd, int i) {
    const int kb = i * kFaBlock;
    if (i + 2 < nblk) issue_rows(kbase, koff, kd, kb + 2 * kFaBlock);
    if (i + 1 < nblk) issue_rows(vbase, voff, vd, kb + kFaBlock);
    if (active(i)) {
      // ---- online softmax of block i per query column ----
      // the max runs over raw scores (qscale > 0), the exponent is one fma:
      // p = 2^(qscale * s + m_off)
      const bool full = kb + kFaBlock <= lk && (!causal || kb + kFaBlock - 1 <= lk - lq + wrow0);
      if (!full) {  // uniform: one branch, then a compare per score
#pragma unroll
        for (int g2 = 0; g2 < NG; ++g2) {
          // key kb + 16 kb2 + 4 kg + r is live when 16 kb2 + r <= rel
          const int rel = (causal ? min(lk - 1, my_pos[g2]) : lk - 1) - kb - 4 * kg;
#pragma unroll
          for (int e = 0; e < 16; ++e)
            sacc[e / 4][g2][e % 4] = 16 * (e / 4) + e % 4 <= rel ? sacc[e / 4][g2][e % 4] : -INFINITY;
        }
      }
      float tmax[NG];
      // row maxima: two chains per column group, the groups side by side,
      // then the cross-row steps of both groups together
#pragma unroll
      for (int g2 = 0; g2 < NG; ++g2) {
        // med3(a, b, FLT_MAX) = max(a, b) for scores (never +inf or NaN),
        // without the canonicalizing moves a two-operand fmaxf gets
        constexpr float kBig = 0x1.fffffep127f;
        float ta = __builtin_amdgcn_fmed3f(sacc[0][g2][0], sacc[0][g2][1], kBig);
        float tb = __builtin_amdgcn_fmed3f(sacc[2][g2][0], sacc[2][g2][1], kBig);
#pragma unroll
        for (int e = 2; e < 8; ++e) {
          ta = fmaxf(ta, sacc[e / 4][g2][e % 4]);
          tb = fmaxf(tb, sacc[2 + e / 4][g2][e % 4]);
        }
        tmax[g2] = fmaxf(ta, tb);
      }
      if constexpr (NG == 2) {
        max_rows4_pair(tmax[0], tmax[1]);
      } else {
#pragma unroll
        for (int g2 = 0; g2 < NG; ++g2) tmax[g2] = max_rows4(tmax[g2]);
      }
      // lazy offset: a column's offset moves only when its max grows past
      // m_run by more than 8 (log2 units), so p <= 2^8 and most blocks skip
      // the branch (o, l and the offsets stay); the normalisation by l makes
      // the result the same softmax whatever offset the column settled on
      bool grow[NG], rescale = false;
#pragma unroll
      for (int g2 = 0; g2 < NG; ++g2) {
        grow[g2] = tmax[g2] > m_thr[g2];
        rescale = rescale || grow[g2];
      }
      if (__any(rescale)) {
#pragma unroll
        for (int g2 = 0; g2 < NG; ++g2) {
          const float m_new = grow[g2] ? tmax[g2] : m_run[g2];
          // the first finite max finds o and l still zero
          const float alpha =
              !grow[g2] ? 1.0f
                        : (m_run[g2] == -INFINITY
                               ? 0.0f
                               : __builtin_amdgcn_exp2f(qscale * (m_run[g2] - m_new)));
          l_acc[g2] *= alpha;
#pragma unroll
          for (int j = 0; j < DB; ++j) o[j][g2] *= alpha;
          m_run[g2] = m_new;
          m_off[g2] = m_new == -INFINITY ? 0.0f : -qscale * m_new;
          m_thr[g2] = m_new + lazy_thr;
        }
      }
      // raised wave priority from here to the end of the PV MFMAs: the SIMD's
      // arbiter then issues this wave's MFMAs first and fills their cycles
      // with the other wave's row maxima, which pulls the two waves into
      // alternating phases (+1-3% on config-4 attention)
      __builtin_amdgcn_s_setprio(1);
      // ---- P of block i, with block i + 1's score MFMAs in between ----------
      // 16-key group c: its exponentials (pop[g2][c / 2], half c % 2) beside
      // the score MFMAs of the next block's group c
      // (the last step computes scores of stale keys it never uses: one
      // branch-free block keeps the MFMAs and the exponentials interleavable)
      f4 snext[4][NG];
#pragma unroll
      for (int kb2 = 0; kb2 < 4; ++kb2)
#pragma unroll
        for (int g2 = 0; g2 < NG; ++g2) snext[kb2][g2] = f4{0.f, 0.f, 0.f, 0.f};
      uint32_t pw[NG][2][4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        u8v a[KS];
        k_reads(reinterpret_cast<const uint16_t*>(kn), c, a);
#pragma unroll
        for (int g2 = 0; g2 < NG; ++g2)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(qscale, sacc[c][g2][2 * h], m_off[g2]));
            const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(qscale, sacc[c][g2][2 * h + 1], m_off[g2]));
            pw[g2][c / 2][2 * (c % 2) + h] = pack_op2(p0, p1, O{});
          }
        k_mfmas(a, snext[c]);
      }
      u8v pop[NG][2];  // [g2][ks]
#pragma unroll
      for (int g2 = 0; g2 < NG; ++g2)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          pop[g2][ks] = __builtin_bit_cast(u8v, make_uint4(pw[g2][ks][0], pw[g2][ks][1],
                                                           pw[g2][ks][2], pw[g2][ks][3]));
      // ---- O^T += V^T * P^T ----
      const char* sv_base = vc;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int jh = 0; jh < 2; ++jh) {
        u8v a[DB / 2];  // half the dim blocks' V^T operands of this k-step, then the MFMAs
#pragma unroll
        for (int jj = 0; jj < DB / 2; ++jj) {
          const int j = jh * (DB / 2) + jj;
          v4s part[2];
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            // keys 32 ks + 16 hh + 4 kg + k, k = 0..3
            const int r = 32 * ks + 16 * hh + 4 * kg + tr_row;
            const int pos = (2 * j + tr_chunk) ^ vswz(r);
            part[hh] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_v4s_ptr)(sv_base + r * (2 * D) + 16 * pos + tr_half));
          }
          a[jj] = u8v{static_cast<uint16_t>(part[0][0]), static_cast<uint16_t>(part[0][1]),
                      static_cast<uint16_t>(part[0][2]), static_cast<uint16_t>(part[0][3]),
                      static_cast<uint16_t>(part[1][0]), static_cast<uint16_t>(part[1][1]),
                      static_cast<uint16_t>(part[1][2]), static_cast<uint16_t>(part[1][3])};
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs
#pragma unroll
        for (int jj = 0; jj < DB / 2; ++jj)
#pragma unroll
          for (int g2 = 0; g2 < NG; ++g2)
            o[jh * (DB / 2) + jj][g2] = mfma16(a[jj], pop[g2][ks], o[jh * (DB / 2) + jj][g2], O{});
        if (jh == 1) {
#pragma unroll
          for (int g2 = 0; g2 < NG; ++g2) l_acc[g2] = mfma16(ones, pop[g2][ks], l_acc[g2], O{});
        }
      }
      __builtin_amdgcn_s_setprio(0);
#pragma unroll
      for (int kb2 = 0; kb2 < 4; ++kb2)
#pragma unroll
        for (int g2 = 0; g2 < NG; ++g2) sacc[kb2][g2] = snext[kb2][g2];
    }
    if (i + 1 < nblk) wait_vmcnt<0>();  // block i + 2's keys and i + 1's values landed
  };
  // two steps per iteration, so that each step's buffers are compile-time
  // LDS offsets (folded into the reads' immediates instead of per-read adds)
  int i = 0;
  for (; i + 1 < nblk; i += 2) {
    step(kbuf1, vbuf0, kbuf0, vbuf1, i);
    __syncthreads();
    step(kbuf0, vbuf1, kbuf1, vbuf0, i + 1);
    __syncthreads();
  }
  if (i < nblk) {
    step(kbuf1, vbuf0, kbuf0, vbuf1, i);
    __syncthreads();
  }

  // o[j][g2][r] = O^T[dim 16j + 4kg + r][query 16*g2 + n]
#pragma unroll
  for (int g2 = 0; g2 < NG; ++g2) {
    if (!live[g2]) continue;
    const float l = l_acc[g2][0];
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    T* orow = out + (static_cast<int64_t>(q_start + wrow0 + 16 * g2 + n) * hq + head) * D;
#pragma unroll
    for (int j = 0; j < DB; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) orow[16 * j + 4 * kg + r] = from_f32<T>(o[j][g2][r] * inv);
  }
}

}  // namespace

extern "C" int kvq_prefill_attn(const void* query, const void* key, const void* value, int dtype,
                                const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                int64_t batch, int64_t max_q_len, int num_heads,
                                int num_kv_heads, int head_size, float scale, int causal,
                                void* out, void* stream) {
  if (batch == 0 || max_q_len == 0) return KVQ_OK;
  if (!query || !key || !value || !cu_seqlens_q || !cu_seqlens_k || !out || batch < 0 ||
      max_q_len < 0 || batch > 65535 || num_heads > 65535)
    return KVQ_ERR_INVALID;
  if (num_kv_heads <= 0 || num_heads % num_kv_heads) return KVQ_ERR_GEOMETRY;
  if (head_size != 64 && head_size != 128 && head_size != 256 && head_size != 32)
    return KVQ_ERR_GEOMETRY;
  if (!(scale > 0.0f)) return KVQ_ERR_INVALID;  // the softmax max runs over raw scores
  hipStream_t s = static_cast<hipStream_t>(stream);
  const float qscale = scale * 1.4426950408889634f;
  int64_t lds_max = 0;  // LDS one workgroup may use on this device
  const int lrc = device_lds_max(&lds_max);
  if (lrc != KVQ_OK) return lrc;
  const int64_t fa_lds = head_size == 64 ? FaLds<64>::BYTES : FaLds<128>::BYTES;
  constexpr int kFaNG = 2;
  if ((dtype == KVQ_DTYPE_BF16 || dtype == KVQ_DTYPE_F16) &&
      (head_size == 64 || head_size == 128) && fa_lds <= lds_max) {
    const int64_t fab = (max_q_len + kFaGroupRows - 1) / kFaGroupRows;
    const int64_t pairs = batch * num_kv_heads;
    const int64_t wgs = (pairs + kFaXcds - 1) / kFaXcds * kFaXcds * (num_heads / num_kv_heads) * fab;
    if (wgs > 0x7fffffff) return KVQ_ERR_INVALID;
    const dim3 fgrid(static_cast<unsigned>(wgs));
#define KVQ_PREFILL_FA(TT, DD)                                                              \
    hipLaunchKernelGGL((prefill_attn_fa_kernel<TT, DD, kFaNG>), fgrid, dim3(64 * (8 / kFaNG)), \
                       FaLds<DD>::BYTES, s, static_cast<const TT*>(query),                 \
                       static_cast<const TT*>(key), static_cast<const TT*>(value),         \
                       cu_seqlens_q, cu_seqlens_k, num_heads, num_kv_heads, qscale, causal, \
                       static_cast<int>(fab), static_cast<int>(batch), static_cast<TT*>(out))
    if (dtype == KVQ_DTYPE_BF16) {
      if (head_size == 64) KVQ_PREFILL_FA(kvq::bf16, 64);
      else KVQ_PREFILL_FA(kvq::bf16, 128);
    } else {
      if (head_size == 64) KVQ_PREFILL_FA(kvq::f16, 64);
      else KVQ_PREFILL_FA(kvq::f16, 128);
    }
#undef KVQ_PREFILL_FA
    KVQ_LAUNCH_CHECK();
    return KVQ_OK;
  }
  const int64_t qblocks = (max_q_len + 63) / 64;
  if (qblocks > 0x7fffffff) return KVQ_ERR_INVALID;
  const dim3 grid(static_cast<unsigned>(qblocks), num_heads, static_cast<unsigned>(batch));
#define KVQ_PREFILL(DD)                                                                  \
  KVQ_DISPATCH_FLOAT(dtype, T,                                                           \
    hipLaunchKernelGGL((prefill_attn_kernel<T, DD>), grid, dim3(256), 0, s,              \
                       static_cast<const T*>(query), static_cast<const T*>(key),          \
                       static_cast<const T*>(value), cu_seqlens_q, cu_seqlens_k,          \
                       num_heads, num_kv_heads, qscale, causal, static_cast<T*>(out)))
  switch (head_size) {
    case 32: KVQ_PREFILL(32); break;
    case 64: KVQ_PREFILL(64); break;
    case 128: KVQ_PREFILL(128); break;
    default: KVQ_PREFILL(256); break;
  }
#undef KVQ_PREFILL
  KVQ_LAUNCH_CHECK();
  return KVQ_OK;
}
