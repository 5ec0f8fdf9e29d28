// fms_inbatch_split.hpp -- launcher of the split-K InBatch() kernel (the
// feature dim taken a K slice at a time): 16-bit features with dims the
// register-resident kernel does not take, and fp32 features.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fms {

struct InBatchSplitArgs {
  const char* Q;      // (Bq, Tq, dim) features
  const char* D;      // (Bd, Td, dim)
  const uint8_t* qm;  // (Bq, Tq) nullable
  const uint8_t* dm;  // (Bd, Td) nullable
  float* S;           // (Bq, Bd): S[i*Bd + j] = MaxSim(Q_i, D_j)
  int32_t* args;      // (Bq, Bd, Tq) nullable
  int Bq, Bd, Tq, Td;
  int rowbytes;       // dim * element bytes (a multiple of 16)
  int norm = 0;
  // filled by the launcher: query rows are 32-token tiles, ntq per query
  // (scored into St (Bq * ntq, Bd) and summed into S when ntq > 1); nqg
  // groups of 8 query rows per document
  int ntq = 1, nqg = 1;
  float* St = nullptr;
  // filled by the launcher: the plan words (valid rows of every 32-row
  // document chunk, then valid tokens of every query row) and the number of
  // block-order slots (nqg x 8 x ceil(Bd / 8), some past Bd)
  const uint32_t* plan = nullptr;
  int nslots = 0;
};

// Element bytes 2 or 4; rows a multiple of 16 bytes; 16-byte aligned bases.
bool inbatch_split_supported(int esz, int64_t dim, int64_t Tq, int64_t Td, int64_t Bq,
                             int64_t Bd, const void* Q, const void* D);
// dtype: 0 fp32, 1 fp16, 2 bf16 (the C ABI's codes).
hipError_t launch_inbatch_split(int32_t dtype, const InBatchSplitArgs& args, hipStream_t stream);

}  // namespace fms
