// fms_group.hpp -- grouping of candidate pairs by document.
//
// A candidate call scores C*B pairs (c, b) against documents idx[c, b] of a
// gallery of N.  When documents repeat (C*B comparable to N, or re-ranking
// lists shared between queries), scanning the pairs in document order lets
// the waves that score one document read it together, so it leaves HBM once
// instead of once per pair.  The order is a counting sort on the document
// index; pairs with an out-of-range index sort last.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace fms {

// One entry of the document order: pair id p = c + C*b and its 0-based
// document (-1 for an index outside 1..N).
struct PairRef {
  int32_t p;
  int32_t j;
};

// Device bytes group_pairs_by_document needs for npairs pairs over N
// documents (order, per-document counters, scan partials).
size_t group_workspace_bytes(int64_t npairs, int64_t N);

// Fills `*order` (inside `workspace`) with all npairs pair ids, grouped by
// document in ascending document order, out-of-range indices last.  The
// order of the pairs of one document is unspecified (LDS-atomic scatter);
// each pair's result does not depend on it.  Requires npairs, N < 2^31.
hipError_t group_pairs_by_document(const void* idx, int idx64, int64_t npairs, int64_t N,
                                   void* workspace, const PairRef** order, hipStream_t stream);
// The same, also returning doc_end (N + 1 counters in `workspace`): the pairs of
// document j are order[j > 0 ? doc_end[j-1] : 0 .. doc_end[j]).
hipError_t group_pairs_by_document(const void* idx, int idx64, int64_t npairs, int64_t N,
                                   void* workspace, const PairRef** order,
                                   const uint32_t** doc_end, hipStream_t stream);

// In-place exclusive prefix sum of n counters on `stream`; `sums` holds
// scan_workspace_bytes(n) bytes.
size_t scan_workspace_bytes(int64_t n);
hipError_t exclusive_scan_u32(uint32_t* counts, int64_t n, uint32_t* sums, hipStream_t stream);

// The device a stream belongs to (the current device for the null stream).
hipError_t stream_device(hipStream_t stream, int* dev);

// Stream-ordered workspace from a library-owned memory pool of the stream's
// device (created on first use, kept for the life of the process so repeated
// calls do not return memory to the driver between synchronisations).
hipError_t workspace_alloc(void** ptr, size_t bytes, hipStream_t stream);
// Number of workspace_alloc calls so far in this process (a test probe).
uint64_t workspace_alloc_count();
hipError_t workspace_free(void* ptr, hipStream_t stream);

}  // namespace fms
