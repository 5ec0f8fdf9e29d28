// fms_inbatch.hpp -- launcher of the MFMA-tiled InBatch() kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fms {

struct InBatchArgs {
  const char* Q;       // (Bq, Tq, dim) 16-bit features
  const char* D;       // (Bd, Td, dim)
  const uint8_t* qm;   // (Bq, Tq) nullable
  const uint8_t* dm;   // (Bd, Td) nullable
  float* S;            // (Bq, Bd): S[i*Bd + j] = MaxSim(Q_i, D_j)
  int32_t* args;       // (Bq, Bd, Tq) nullable
  int Bq, Bd, Tq, Td;
  int nqb, ndb, db;    // filled by the launcher
};

// dim == 128, 1 <= Tq <= 32, 16-byte aligned features.
bool inbatch_mfma_supported(int64_t dim, int64_t Tq, int64_t Td, const void* Q, const void* D);
hipError_t launch_inbatch_mfma(int dtype_bf16, const InBatchArgs& args, hipStream_t stream);

}  // namespace fms
