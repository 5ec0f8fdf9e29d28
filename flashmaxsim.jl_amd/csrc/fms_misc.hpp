// fms_misc.hpp -- host launchers of the small kernels in fms_misc.hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fms {

// X (ntok, dim) of fp32, or of fp16 when `half`; scales of the same type.
hipError_t quantize_int8(bool half, const void* X, int8_t* codes, void* scales, int dim,
                         int64_t ntok, hipStream_t stream);
hipError_t int8_dots(int32_t* out, const int8_t* qc, const int8_t* dc, int dim, int Tq, int Td,
                     bool vec, hipStream_t stream);
hipError_t length_normalize(float* scores, const uint8_t* qmask, int64_t Tq, int64_t nrows,
                            int64_t ncols, const void* idx, int idx64, int64_t N, float neg,
                            hipStream_t stream);
hipError_t varlen_normalize(float* scores, const int32_t* cu_q, int64_t N, hipStream_t stream);
hipError_t mfma_layout_probe(float* out, int op, hipStream_t stream);
hipError_t cross_lane_probe(float* out, hipStream_t stream);
hipError_t read_bandwidth(const void* p, int64_t bytes, uint32_t* out, int blocks,
                          hipStream_t stream);
hipError_t gather_bandwidth(const void* g, int64_t gallery_bytes, int64_t doc_bytes,
                            const int32_t* docs, int64_t ndocs, uint32_t* out, hipStream_t stream);

}  // namespace fms
