// fms_inbatch.hpp -- launcher of the MFMA-tiled InBatch() kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fms {

struct InBatchArgs {
  const char* Q;       // (Bq, Tq, dim) 16-bit features
  const char* D;       // (Bd, Td, dim)
  const uint8_t* qm;   // (Bq, Tq) nullable
  const uint8_t* dm;   // (Bd, Td) nullable (in-batch only)
  const int32_t* cu = nullptr;  // packed documents: (Bd + 1,) 1-based CSR over D (ntok
                                // rows); nullptr = the in-batch layout.  Td is then max_len.
  int64_t ntok = 0;
  float* S;            // (Bq, Bd): S[i*Bd + j] = MaxSim(Q_i, D_j)
  int32_t* args;       // (Bq, Bd, Tq) nullable
  int Bq, Bd, Tq, Td;
  int dim = 128;       // 32, 64, 96 or 128
  int norm = 0;
  // filled by the launcher for Tq > 32: query rows of the kernel are tiles of
  // 32 tokens, ntq per query, scored into St (Bq * ntq, Bd) and summed into S
  int ntq = 1;
  float* St = nullptr;        // S *= 1 / max(valid tokens of query i, 1)
  // filled by the launcher
  int nqb, ndb;        // query blocks, document blocks
  int db;              // most documents of a block (uniform partition: ranges of floor or ceil of Bd/ndb)
  int dbcap;           // most documents a block can hold
  int balance;         // 1: partition documents by chunk count (Bd <= kIbBalanceMaxDocs)
  int tilt;            // 1: balanced one-round grid of two blocks per CU, first half of
                       //    the document ranges weighted 22 : 18 against the second
  const uint32_t* cmask;  // (Bd, nch) valid rows per chunk (plan kernel)
  const int32_t* dcount;  // (Bd,) chunks with a valid row
  const int32_t* dfirst;  // (Bd,) first valid token, -1 = none
};

// dim in {32, 64, 96, 128}, 1 <= Tq <= 4096, 16-byte aligned features.
bool inbatch_mfma_supported(int64_t dim, int64_t Tq, int64_t Td, const void* Q, const void* D);
// Runs the plan kernel (per-document chunk masks, in a workspace from the
// library pool) and the in-batch kernel on `stream`.  With args.cu set the
// documents are PackedSeq token ranges (every row valid, no dmask): the
// multi-query packed scan.
hipError_t launch_inbatch_mfma(int dtype_bf16, const InBatchArgs& args, hipStream_t stream);

}  // namespace fms
