// SPDX-License-Identifier: Apache-2.0
// Internal interfaces shared by the decode-attention translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kvq_hip.h"

namespace kvq {

// ---- XCD-aware grid mapping ------------------------------------------------
// Workgroups are handed to the 8 XCDs round-robin (id % 8).  The kv heads of
// one work item share HBM lines: a token's value words and value scales/mins
// of all heads are contiguous.  Items are also taken in pairs (2P, 2P+1): a
// paired int4 range's two halves (its even and its odd 64-position tiles)
// read the two halves of the same key lines.  Mapping id -> (item, head) so
// that every head of both items of a pair lands on XCD P % 8, dispatched back
// to back, lets that XCD's L2 serve each of those lines once.
constexpr int kXcds = 8;

__host__ __device__ __forceinline__ int64_t xcd_grid_size(int64_t num_work, int kvh) {
  return (num_work + 2 * kXcds - 1) / (2 * kXcds) * (2 * kXcds) * kvh;
}

__device__ __forceinline__ bool xcd_item_head(int64_t id, int kvh, int64_t num_work, int& item,
                                              int& head) {
  const int64_t j = id / kXcds;
  const int64_t pair = id % kXcds + kXcds * (j / (2 * kvh));
  const int64_t it = 2 * pair + (j / kvh) % 2;
  head = static_cast<int>(j % kvh);
  item = static_cast<int>(it);
  return it < num_work;
}

// Workspace: o [num_work, num_heads, D] fp32, then (m, l) [num_work, num_heads, 2].
inline int64_t decode_workspace_bytes(int64_t num_work, int num_heads, int head_size) {
  return num_work * num_heads * (static_cast<int64_t>(head_size) + 2) *
         static_cast<int64_t>(sizeof(float));
}

// The MFMA tail path (kind-1 items) applies: D = 128, GQA group <= 16, query
// and ring in the same 16-bit dtype, and a power-of-two block size (its
// position arithmetic is shifts and masks).
inline bool tail_path_applies(int q_dtype, int hq, int kvh, int d, int ring_dtype, int bs) {
  return d == 128 && hq / kvh <= 16 && ring_dtype == q_dtype && bs > 0 && (bs & (bs - 1)) == 0 &&
         (q_dtype == KVQ_DTYPE_BF16 || q_dtype == KVQ_DTYPE_F16);
}

// Launch the MFMA kernel for the kind-0 work items when the geometry is one it
// covers, taking the kind-1 items too when the tail path applies: in a second
// pass of the same grid, or, given pieces, in one pass of one wave per (piece,
// kv head).  *launched / *tail_done tell the caller which kinds still need
// another kernel.
int launch_kivi_decode_mfma(const void* query, int q_dtype, int hq, int kvh, int d, float qscale,
                            const int32_t* kq, const float* ks, const float* km,
                            const int32_t* vq, const float* vs, const float* vm, int bs, int g,
                            int64_t nb, const int32_t* block_table, int64_t maxb,
                            const int32_t* seq_meta, const int32_t* work, int64_t num_work,
                            const int32_t* pieces, int64_t num_pieces, const void* ring_k, const void* ring_v, int ring_dtype, int ring_len,
                            float* ws_o, float* ws_ml, hipStream_t s, bool* launched,
                            bool* tail_done);

// The page-streaming decode (decode_coop.hip): given pieces, one workgroup of
// kvh waves per piece streams whole pages of the piece's int4 items for all kv
// heads, then runs its tail items.  Applies at kvh 8, head size 128, block
// size 128, group 64 or 128, GQA groups of at most 16 heads, 16-bit query and
// ring, a positive finite scale and a device with the ring's LDS; *launched
// tells the caller whether it ran (every kind then done).
bool coop_decode_applies(int q_dtype, int hq, int kvh, int d, int ring_dtype, int bs, int g);
int launch_kivi_decode_coop(const void* query, int q_dtype, int hq, int kvh, int d, float qscale,
                            const int32_t* kq, const float* ks, const float* km,
                            const int32_t* vq, const float* vs, const float* vm, int bs, int g,
                            int64_t nb, const int32_t* block_table, int64_t maxb,
                            const int32_t* seq_meta, const int32_t* work, int64_t num_work,
                            const int32_t* pieces, int64_t num_pieces, const void* ring_k,
                            const void* ring_v, int ring_dtype, int ring_len, float* ws_o,
                            float* ws_ml, hipStream_t s, bool* launched);

// Standalone MFMA tail kernel for the kind-1 items, for geometries the int4
// kernel does not cover.  *launched tells the caller whether kind-1 items still
// need the generic kernel.
int launch_kivi_decode_tail_mfma(const void* query, int q_dtype, int hq, int kvh, int d,
                                 float qscale, const int32_t* kq, const float* ks,
                                 const float* km, const int32_t* vq, const float* vs,
                                 const float* vm, int bs, int g, int64_t nb,
                                 const int32_t* block_table, int64_t maxb,
                                 const int32_t* seq_meta, const int32_t* work, int64_t num_work,
                                 const void* ring_k, const void* ring_v, int ring_dtype,
                                 int ring_len, float* ws_o, float* ws_ml, hipStream_t s,
                                 bool* launched);

// INT8 counterpart: kind-0 items (all positions in int8 pages) on MFMA.
int launch_int8_decode_mfma(const void* query, int dtype, int hq, int kvh, int d, float qscale,
                            const int8_t* kc, const int8_t* vc, int bs, int64_t nb,
                            const void* k_aq,
                            const void* v_aq, const int32_t* block_table, int64_t maxb,
                            const int32_t* work, int64_t num_work, float* ws_o, float* ws_ml,
                            hipStream_t s, bool* launched);

// Merge each request's work items: out = sum_s 2^(m_s-M) o_s / sum_s 2^(m_s-M) l_s.
// seq_meta row b holds (first_work, num_work) at columns first_col, first_col+1.
int launch_decode_combine(int dtype, int64_t batch, int hq, int d, const int32_t* seq_meta,
                          int meta_stride, int first_col, const float* ws_o, const float* ws_ml,
                          void* out, hipStream_t s);

}  // namespace kvq
