// fms_layouts.hpp -- how each reference layout maps a linear pair id p to
// one (query, document) pair.  Output cells are always p-major: the tape /
// partial of pair p occupy [p*rows, (p+1)*rows) and its score is scores[p],
// which is exactly the reference's column-major (Tq, C, B) / (Tq, B) /
// (Tq, Bd, Bq) / (max_q, N) layouts.
#pragma once

#include <stdint.h>

#include "fms_device.hpp"

namespace fms {

// One (query, document) pair as a wave sees it.  All fields are uniform.
struct PairView {
  const char* q;      // first query token (features or int8 codes)
  const uint8_t* qm;  // query mask of that query (nullable = all true)
  const float* qs;    // int8 query scales (nullable for float features)
  int tq;             // query tokens that exist for this pair
  const char* d;      // first document token
  const uint8_t* dm;  // document mask (nullable = all true)
  const float* ds;    // int8 document scales
  int td;             // document tokens (0 = empty / invalid)
  bool valid;         // false only for an out-of-range candidate index
};

__device__ __forceinline__ int64_t clamp64(int64_t v, int64_t lo, int64_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

// Longest ragged sequence (in tokens) whose bytes fit one buffer resource.
__device__ __forceinline__ int64_t max_seq_tokens(int64_t rowbytes) {
  return rowbytes > 0 ? (int64_t)0x7fffffff / rowbytes : (int64_t)0x7fffffff;
}

// paired_tile_kernel! (kernels_forward.jl:195-269): pair b = (Q_b, D_b).
// The single pair layout is B = 1.
struct LayPaired {
  const char* Q; const char* D;
  const uint8_t* qm; const uint8_t* dm;
  const float* Qs; const float* Ds;
  int64_t qbytes, dbytes;  // bytes of one query / one document
  int Tq, Td;
  __device__ PairView get(int64_t b) const {
    PairView v;
    v.q = Q + b * qbytes; v.qm = qm ? qm + b * Tq : nullptr; v.qs = Qs ? Qs + b * Tq : nullptr;
    v.tq = Tq;
    v.d = D + b * dbytes; v.dm = dm ? dm + b * Td : nullptr; v.ds = Ds ? Ds + b * Td : nullptr;
    v.td = Td; v.valid = true;
    return v;
  }
};

// candidates_tile_kernel! (kernels_forward.jl:271-356): pair p = c + C*b
// scores Q_b against gallery[:, :, idx[c,b]]; 1 <= idx <= N else invalid.
struct LayCand {
  const char* Q; const char* G; const void* idx;
  const uint8_t* qm; const uint8_t* dm;
  const float* Qs; const float* Gs;
  int64_t qbytes, dbytes, N, C;
  int Tq, Td, idx64;
  __device__ PairView get(int64_t p) const {
    const int64_t b = p / C;
    const int64_t j = idx64 ? static_cast<const int64_t*>(idx)[p]
                            : (int64_t) static_cast<const int32_t*>(idx)[p];
    PairView v;
    v.q = Q + b * qbytes; v.qm = qm ? qm + b * Tq : nullptr; v.qs = Qs ? Qs + b * Tq : nullptr;
    v.tq = Tq;
    v.valid = (j >= 1 && j <= N);
    const int64_t jj = v.valid ? j - 1 : 0;
    v.d = G + jj * dbytes; v.dm = dm ? dm + jj * Td : nullptr; v.ds = Gs ? Gs + jj * Td : nullptr;
    v.td = v.valid ? Td : 0;
    return v;
  }
};

// In-batch: pair p = j + Bd*i scores Q_i against D_j (S[j,i], args[t,j,i]).
struct LayInBatch {
  const char* Q; const char* D;
  const uint8_t* qm; const uint8_t* dm;
  int64_t qbytes, dbytes, Bd;
  int Tq, Td;
  __device__ PairView get(int64_t p) const {
    const int64_t j = p % Bd, i = p / Bd;
    PairView v;
    v.q = Q + i * qbytes; v.qm = qm ? qm + i * Tq : nullptr; v.qs = nullptr; v.tq = Tq;
    v.d = D + j * dbytes; v.dm = dm ? dm + j * Td : nullptr; v.ds = nullptr; v.td = Td;
    v.valid = true;
    return v;
  }
};

// packed_tile_kernel! (kernels_packed.jl:35-114): one query against
// document b = tokens[:, cu[b]:cu[b+1]-1]; cu is clamped into the token
// range so a malformed device cu cannot read out of bounds.
struct LayPacked {
  const char* q; const char* tok; const int32_t* cu; const uint8_t* qm;
  int64_t ntok, rowbytes;
  int Tq;
  __device__ PairView get(int64_t b) const {
    const int64_t a = clamp64((int64_t)cu[b] - 1, 0, ntok);
    const int64_t z = clamp64(clamp64((int64_t)cu[b + 1] - 1, a, ntok), a,
                              a + max_seq_tokens(rowbytes));
    PairView v;
    v.q = q; v.qm = qm; v.qs = nullptr; v.tq = Tq;
    v.d = tok + a * rowbytes; v.dm = nullptr; v.ds = nullptr; v.td = (int)(z - a);
    v.valid = true;
    return v;
  }
};

// varlen_tile_kernel! (kernels_packed.jl:145-227): pair n = (Q tokens
// cu_q[n]:cu_q[n+1]-1, D tokens cu_d[n]:cu_d[n+1]-1); no masks.
struct LayVarlen {
  const char* Qt; const char* Dt; const int32_t* cu_q; const int32_t* cu_d;
  int64_t nq, nd, rowbytes;
  int max_q;
  __device__ PairView get(int64_t n) const {
    const int64_t qa = clamp64((int64_t)cu_q[n] - 1, 0, nq);
    const int64_t qz = clamp64(clamp64((int64_t)cu_q[n + 1] - 1, qa, nq), qa, qa + max_seq_tokens(rowbytes));
    const int64_t da = clamp64((int64_t)cu_d[n] - 1, 0, nd);
    const int64_t dz = clamp64(clamp64((int64_t)cu_d[n + 1] - 1, da, nd), da, da + max_seq_tokens(rowbytes));
    PairView v;
    v.q = Qt + qa * rowbytes; v.qm = nullptr; v.qs = nullptr;
    v.tq = (int)((qz - qa) < max_q ? (qz - qa) : max_q);
    v.d = Dt + da * rowbytes; v.dm = nullptr; v.ds = nullptr; v.td = (int)(dz - da);
    v.valid = true;
    return v;
  }
};

}  // namespace fms
