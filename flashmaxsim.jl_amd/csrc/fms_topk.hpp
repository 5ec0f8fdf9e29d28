// fms_topk.hpp -- host launcher of the per-row top-k kernel (fms_topk.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fms {

// Largest k the kernel sorts in LDS (8 KB of (key, index) pairs).
constexpr int kTopkMaxK = 1024;

// Caller guarantees 1 <= k <= min(ncols, kTopkMaxK), ncols <= INT32_MAX,
// nrows <= UINT32_MAX, S/vals/idx device pointers of nrows*ncols / nrows*k.
hipError_t topk_rows(const float* S, int64_t nrows, int64_t ncols, int k, float* vals,
                     int32_t* idx, hipStream_t stream);

}  // namespace fms
