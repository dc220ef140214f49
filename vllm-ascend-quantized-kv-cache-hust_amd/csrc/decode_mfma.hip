// SPDX-License-Identifier: Apache-2.0
// MFMA decode-attention kernels (kind-0 work items).  Until they land, every
// work item is served by the generic kernels.
#include "kvq_common.h"
#include "kvq_decode.h"

namespace kvq {

int launch_kivi_decode_mfma(const void*, int, int, int, int, float, const int32_t*, const float*,
                            const float*, const int32_t*, const float*, const float*, int, int,
                            const int32_t*, int64_t, const int32_t*, const int32_t*, int64_t,
                            float*, float*, hipStream_t, bool* launched) {
  *launched = false;
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
