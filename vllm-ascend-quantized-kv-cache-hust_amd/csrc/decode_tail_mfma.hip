// SPDX-License-Identifier: Apache-2.0
// Standalone launch of the tail path (kind-1 work items) for geometries where
// the int4 decode kernel -- which otherwise runs the tail items itself, in a
// second pass of its grid -- does not apply.  The tail arithmetic lives in
// decode_tail.h.
#include "decode_tail.h"

namespace {

using namespace kvq;

template <typename T>
__global__ void __launch_bounds__(64, 2)
kivi_decode_tail_mfma_kernel(const T* __restrict__ query, int hq, int kvh, float qscale,
                             const uint32_t* __restrict__ kq, const float* __restrict__ ks,
                             const float* __restrict__ km, const uint32_t* __restrict__ vq,
                             const float* __restrict__ vs, const float* __restrict__ vm, int bs,
                             int g, int64_t nb, const int32_t* __restrict__ block_table,
                             int64_t maxb, const int32_t* __restrict__ seq_meta,
                             const int32_t* __restrict__ work, const T* __restrict__ ring_k,
                             const T* __restrict__ ring_v, int ring_len, int64_t num_work,
                             float* __restrict__ ws_o, float* __restrict__ ws_ml) {
  extern __shared__ __align__(16) char lds_raw[];
  int wi, h;
  if (!xcd_item_head(blockIdx.x, kvh, num_work, wi, h)) return;
  const int32_t* wk = work + 4 * static_cast<int64_t>(wi);
  if (wk[3] != 1) return;  // kind-0 items belong to the int4 kernels (uniform)
  const tail::Partial p =
      tail::tail_item<T>(lds_raw, query, hq, kvh, qscale, kq, ks, km, vq, vs, vm, bs, g, nb,
                         block_table, maxb, seq_meta, wk, wi, h, ring_k, ring_v, ring_len, 0, 1);
  tail::tail_store(p, wi, hq, h, hq / kvh, threadIdx.x & 63, ws_o, ws_ml);
}

}  // namespace

namespace kvq {

int launch_kivi_decode_tail_mfma(const void* query, int q_dtype, int hq, int kvh, int d,
                                 float qscale, const int32_t* kq, const float* ks,
                                 const float* km, const int32_t* vq, const float* vs,
                                 const float* vm, int bs, int g, int64_t nb,
                                 const int32_t* block_table, int64_t maxb,
                                 const int32_t* seq_meta, const int32_t* work, int64_t num_work,
                                 const void* ring_k, const void* ring_v, int ring_dtype,
                                 int ring_len, float* ws_o, float* ws_ml, hipStream_t s,
                                 bool* launched) {
  *launched = false;
  if (!tail_path_applies(q_dtype, hq, kvh, d, ring_dtype, bs)) return KVQ_OK;
  const dim3 grid(static_cast<unsigned>(xcd_grid_size(num_work, kvh)));
  const size_t lds = tail::kLdsBytes;
  const uint32_t* kqu = reinterpret_cast<const uint32_t*>(kq);
  const uint32_t* vqu = reinterpret_cast<const uint32_t*>(vq);
  if (q_dtype == KVQ_DTYPE_BF16) {
    hipLaunchKernelGGL((kivi_decode_tail_mfma_kernel<bf16>), grid, dim3(64), lds, s,
                       static_cast<const bf16*>(query), hq, kvh, qscale, kqu, ks, km, vqu, vs, vm,
                       bs, g, nb, block_table, maxb, seq_meta, work,
                       static_cast<const bf16*>(ring_k), static_cast<const bf16*>(ring_v),
                       ring_len, num_work, ws_o, ws_ml);
  } else {
    hipLaunchKernelGGL((kivi_decode_tail_mfma_kernel<f16>), grid, dim3(64), lds, s,
                       static_cast<const f16*>(query), hq, kvh, qscale, kqu, ks, km, vqu, vs, vm,
                       bs, g, nb, block_table, maxb, seq_meta, work,
                       static_cast<const f16*>(ring_k), static_cast<const f16*>(ring_v),
                       ring_len, num_work, ws_o, ws_ml);
  }
  KVQ_LAUNCH_CHECK();
  *launched = true;
  return KVQ_OK;
}

}  // namespace kvq
