// fms_backward.hpp -- backward of the fused MaxSim forward on its argmax tape.
//
// For every pair p (one query against one document, as the forward layouts
// enumerate them) and every query token t with qmask and a valid tape entry
// u = args[t, p] (1-based):
//     dQ[:, t of p's query] += delta_p * D[:, u of p's document]
//     dD[:, u of p's document] += delta_p * Q[:, t of p's query]
// with delta_p = Delta[p] * inv_n[query of p] (inv_n NULL = 1).  Pairs come
// in groups of G consecutive pairs that share one query (paired / varlen:
// G = 1; candidates: C; in-batch: Bd; packed: all B pairs share the single
// query).  dQ and dD are written in full (rows no source reaches are 0),
// in the feature type; all sums run in fp32.
//
// dQ is a gather: one wave per (query group, token) sums its pairs in pair
// order (deterministic).  dD is destination-owned: the sources are counted
// per destination row, prefix-summed into a CSR and filled (atomic slot per
// source), then one wave per destination row sums its sources.  The order
// of sources within a row is the fill order, so dD may differ between runs
// in the last bits, as the reference's device CSR does (src/invgrid.jl:10-14).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fms_layouts.hpp"

namespace fms {

struct PullbackArgs {
  int dtype;                 // FMS_F32 / FMS_F16 / FMS_BF16 (feature type of everything below)
  char* dQ;                  // same layout as the query features
  char* dD;                  // same layout as the document features (nd_rows rows)
  const char* Qbase;         // the query features the layout points into
  const char* Dbase;         // the document features the layout points into
  const int32_t* args;       // (rows, npairs) tape, pair-major
  const void* Delta;         // (npairs,) cotangent, feature type
  const void* inv_n;         // (npairs / G,) feature type, nullable = 1
  int64_t npairs, G;         // pairs; pairs per query group
  int64_t nq_rows, nd_rows;  // rows of dQ / dD
  int rows;                  // tape rows per pair (Tq, or max_q for varlen)
  int dim;
  bool zero_dq;              // dQ rows may belong to no group (varlen): clear dQ first
};

// Runs the pullback on `stream` (workspace from the library pool).
template <class L>
hipError_t launch_pullback(const L& lay, const PullbackArgs& a, hipStream_t stream);

}  // namespace fms
