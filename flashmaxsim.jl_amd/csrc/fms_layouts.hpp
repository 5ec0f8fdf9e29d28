// fms_layouts.hpp -- how each reference layout maps a scan position k to
// one (query, document) pair and its output slot.  Output cells are always
// pair-major: the tape / partial of output slot o occupy [o*rows,
// (o+1)*rows) and its score is scores[o], which is exactly the reference's
// column-major (Tq, C, B) / (Tq, B) / (Tq, Bd, Bq) / (max_q, N) layouts.
// Every layout but LayCandSorted scans in output order (o = k).
#pragma once

#include <stdint.h>

#include "fms_device.hpp"
#include "fms_group.hpp"

namespace fms {

// One (query, document) pair as a wave sees it.  All fields are uniform.
struct PairView {
  const char* q;      // first query token (features or int8 codes)
  const uint8_t* qm;  // query mask of that query (nullable = all true)
  const char* qs;     // int8 query scales (nullable for float features)
  int qs_half;        // 1: the query scales are fp16, 0: fp32
  int tq;             // query tokens that exist for this pair
  const char* d;      // first document token
  const uint8_t* dm;  // document mask (nullable = all true)
  const char* ds;     // int8 document scales (fp16 / fp32 per the scan's Op)
  int td;             // document tokens (0 = empty / invalid)
  bool valid;         // false only for an out-of-range candidate index
  int64_t out;        // output slot (pair id) of this pair
};

// Read-only element at a wave-uniform index through the constant address
// space, so the backend reads it with a scalar load.  A vector load here
// would be followed by a full vmcnt drain of the wave's chunk prefetch.
template <class T>
__device__ __forceinline__ T sload(const T* p, int64_t i) {
  typedef __attribute__((address_space(4))) const T* cptr;
  return ((cptr)p)[i];
}

// The same view with every field moved to scalar registers.  A view is a
// function of uniform values only, but the compiler cannot always prove
// that after it has been carried through a loop; a buffer resource built
// from a pointer it believes divergent becomes a per-lane waterfall loop
// around every load.
template <class T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
  return reinterpret_cast<T*>(rfl64(reinterpret_cast<uint64_t>(p)));
}

__device__ __forceinline__ PairView uniform_view(const PairView& v) {
  PairView u;
  u.q = uniform_ptr(v.q);
  u.qm = uniform_ptr(v.qm);
  u.qs = uniform_ptr(v.qs);
  u.qs_half = (int)rfl32((uint32_t)v.qs_half);
  u.tq = (int)rfl32((uint32_t)v.tq);
  u.d = uniform_ptr(v.d);
  u.dm = uniform_ptr(v.dm);
  u.ds = uniform_ptr(v.ds);
  u.td = (int)rfl32((uint32_t)v.td);
  u.valid = rfl32(v.valid ? 1u : 0u) != 0u;
  u.out = (int64_t)rfl64((uint64_t)v.out);
  return u;
}

__device__ __forceinline__ int64_t clamp64(int64_t v, int64_t lo, int64_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

// Longest ragged sequence (in tokens) whose bytes fit one buffer resource.
__device__ __forceinline__ int64_t max_seq_tokens(int64_t rowbytes) {
  return rowbytes > 0 ? (int64_t)0x7fffffff / rowbytes : (int64_t)0x7fffffff;
}

// paired_tile_kernel! (kernels_forward.jl:195-269): pair b = (Q_b, D_b).
// The single pair layout is B = 1.
// INT8 scales are addressed in bytes: qs_esz / ds_esz are 2 (fp16) or 4 (fp32).
struct LayPaired {
  const char* Q; const char* D;
  const uint8_t* qm; const uint8_t* dm;
  const char* Qs; const char* Ds;
  int64_t qbytes, dbytes;  // bytes of one query / one document
  int Tq, Td;
  int qs_esz = 4, ds_esz = 4;
  __device__ PairView get(int64_t b) const {
    PairView v;
    v.q = Q + b * qbytes; v.qm = qm ? qm + b * Tq : nullptr;
    v.qs = Qs ? Qs + b * Tq * qs_esz : nullptr; v.qs_half = qs_esz == 2;
    v.tq = Tq;
    v.d = D + b * dbytes; v.dm = dm ? dm + b * Td : nullptr;
    v.ds = Ds ? Ds + b * Td * ds_esz : nullptr;
    v.td = Td; v.valid = true; v.out = b;
    return v;
  }
};

// candidates_tile_kernel! (kernels_forward.jl:271-356): pair p = c + C*b
// scores Q_b against gallery[:, :, idx[c,b]]; 1 <= idx <= N else invalid.
struct LayCand {
  const char* Q; const char* G; const void* idx;
  const uint8_t* qm; const uint8_t* dm;
  const char* Qs; const char* Gs;
  int64_t qbytes, dbytes, N, C;
  int Tq, Td, idx64;
  int qs_esz = 4, ds_esz = 4;
  __device__ PairView get(int64_t p) const {
    const int64_t b = p / C;
    const int64_t j = idx64 ? sload(static_cast<const int64_t*>(idx), p)
                            : (int64_t)sload(static_cast<const int32_t*>(idx), p);
    PairView v;
    v.q = Q + b * qbytes; v.qm = qm ? qm + b * Tq : nullptr;
    v.qs = Qs ? Qs + b * Tq * qs_esz : nullptr; v.qs_half = qs_esz == 2;
    v.tq = Tq;
    v.valid = (j >= 1 && j <= N);
    const int64_t jj = v.valid ? j - 1 : 0;
    v.d = G + jj * dbytes; v.dm = dm ? dm + jj * Td : nullptr;
    v.ds = Gs ? Gs + jj * Td * ds_esz : nullptr;
    v.td = v.valid ? Td : 0;
    v.out = p;
    return v;
  }
};

// The candidate layout scanned in document order (group_pairs_by_document):
// position k is pair order[k].p, so the pairs that share a document are
// adjacent and the waves that score them read it together.
struct LayCandSorted {
  LayCand c;
  const PairRef* order;
  __device__ PairView get(int64_t k) const {
    PairRef r;
    r.p = sload(&order[k].p, 0);
    r.j = sload(&order[k].j, 0);
    const int64_t p = r.p, b = p / c.C;
    PairView v;
    v.q = c.Q + b * c.qbytes; v.qm = c.qm ? c.qm + b * c.Tq : nullptr;
    v.qs = c.Qs ? c.Qs + b * c.Tq * c.qs_esz : nullptr; v.qs_half = c.qs_esz == 2;
    v.tq = c.Tq;
    v.valid = r.j >= 0;
    const int64_t jj = v.valid ? r.j : 0;
    v.d = c.G + jj * c.dbytes; v.dm = c.dm ? c.dm + jj * c.Td : nullptr;
    v.ds = c.Gs ? c.Gs + jj * c.Td * c.ds_esz : nullptr;
    v.td = v.valid ? c.Td : 0;
    v.out = p;
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
    v.q = Q + i * qbytes; v.qm = qm ? qm + i * Tq : nullptr; v.qs = nullptr; v.qs_half = 0;
    v.tq = Tq;
    v.d = D + j * dbytes; v.dm = dm ? dm + j * Td : nullptr; v.ds = nullptr; v.td = Td;
    v.valid = true; v.out = p;
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
    const int64_t a = clamp64((int64_t)sload(cu, b) - 1, 0, ntok);
    const int64_t z = clamp64(clamp64((int64_t)sload(cu, b + 1) - 1, a, ntok), a,
                              a + max_seq_tokens(rowbytes));
    PairView v;
    v.q = q; v.qm = qm; v.qs = nullptr; v.qs_half = 0; v.tq = Tq;
    v.d = tok + a * rowbytes; v.dm = nullptr; v.ds = nullptr; v.td = (int)(z - a);
    v.valid = true; v.out = b;
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
    const int64_t qa = clamp64((int64_t)sload(cu_q, n) - 1, 0, nq);
    const int64_t qz = clamp64(clamp64((int64_t)sload(cu_q, n + 1) - 1, qa, nq), qa, qa + max_seq_tokens(rowbytes));
    const int64_t da = clamp64((int64_t)sload(cu_d, n) - 1, 0, nd);
    const int64_t dz = clamp64(clamp64((int64_t)sload(cu_d, n + 1) - 1, da, nd), da, da + max_seq_tokens(rowbytes));
    PairView v;
    v.q = Qt + qa * rowbytes; v.qm = nullptr; v.qs = nullptr; v.qs_half = 0;
    v.tq = (int)((qz - qa) < max_q ? (qz - qa) : max_q);
    v.d = Dt + da * rowbytes; v.dm = nullptr; v.ds = nullptr; v.td = (int)(dz - da);
    v.valid = true; v.out = n;
    return v;
  }
};

}  // namespace fms
