// fms_topk.hpp -- host launcher of the per-row top-k kernel (fms_topk.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fms {

// Largest k the kernel sorts in LDS (8 KB of (key, index) pairs).
constexpr int kTopkMaxK = 1024;
// Most rows per call: one 1024-thread workgroup per row, grid below 2^32 work-items.
constexpr int64_t kTopkMaxRows = ((int64_t)1 << 32) / 1024 - 1;

// Caller guarantees 1 <= k <= min(ncols, kTopkMaxK), ncols <= INT32_MAX,
// 1 <= nrows <= kTopkMaxRows, S/vals/idx device pointers of nrows*ncols / nrows*k.
hipError_t topk_rows(const float* S, int64_t nrows, int64_t ncols, int k, float* vals,
                     int32_t* idx, hipStream_t stream);

}  // namespace fms
