// fms_inbatch.hip -- InBatch() MaxSim as an MFMA-bound tiled contraction.
//
// S[j, i] = sum_t max_u <Q_i[t], D_j[u]> for all (i, j) of Bq queries x Bd
// documents (the reference materialises D'Q chunks and then runs an atomic
// argmax-accumulate, forward_layouts.jl:202-225; here nothing but S and the
// tape leaves the chip).
//
// Two launches.  A plan kernel reads the document masks once per call: the
// valid rows of every 32-token chunk, each document's count of chunks with a
// valid row and its first valid token.  The in-batch kernel then runs two
// workgroups per CU (at C3 a single round of the grid):
//
// Workgroup = 4 waves (one per SIMD), 16 queries x a range of documents.
//   * document ranges split the documents by work (chunk steps plus one per
//     document, from the plan), so the workgroups finish together; every
//     workgroup checks the split against the per-block document limit and
//     all fall back to an even split otherwise;
//   * every wave keeps 4 query tiles (32 tokens x d=128 fp16/bf16) in
//     registers for the whole workgroup lifetime, so each LDS fragment read
//     feeds 4 MFMAs; the four waves share one chunk stream (a barrier per
//     step), and the two waves of a SIMD belong to different workgroups;
//     issue priority falls as a step progresses, so the wave that is behind
//     issues first and neither workgroup runs ahead (the SIMD otherwise
//     favours the older wave, and the younger workgroup would finish alone);
//   * the workgroup streams its documents in 32-row chunks (in the in-batch
//     layout, chunks of two 16-row units, so a document's last unit and the
//     next document's first share a chunk, folded as two register halves
//     with the first document's close between them): each chunk
//     (8 KB) is fetched ONCE from L2/HBM straight into LDS (buffer_load ...
//     lds, one 16-byte load per thread, no registers), in MFMA fragment
//     order: the 64 lanes of one fragment read cover 1 KB contiguously (no
//     bank conflicts) and a lane's 8 reads are one address plus immediates;
//   * masked rows (dmask = 0, and rows past Td in a document's last chunk)
//     are replaced AT LOAD TIME by a copy of the document's first valid
//     token f.  A copy scores exactly what f scores, so the maximum is
//     unchanged, and with first-occurrence tie breaking a copy can only win
//     where f ties it: a winning copy maps back to f when the document is
//     closed.  The fold therefore needs no row masks at all;
//   * software pipeline over three LDS buffers: chunk c+2 is requested while
//     chunk c is multiplied, and one barrier per step (after each wave's
//     own load of chunk c+1 has landed) publishes the next chunk.  Loads
//     are unconditional (the stream is padded to whole rounds of the
//     buffers and stops at its last entry, so loads past the end re-read
//     it), so the in-order vmcnt accounting waits for exactly one chunk;
//   * per chunk and wave: 8 LDS fragment reads feed 4 x 8 MFMA 32x32x16 in
//     two phases of two independent accumulation chains (a dependent
//     32x32x16 MFMA issues at about half the rate of an independent one).
//     Each phase's MFMAs overlap the running max/argmax update of the two
//     tiles multiplied before them: phase 1 multiplies tiles 0,1 while tiles
//     2,3 of the previous chunk fold, phase 2 multiplies tiles 2,3 while
//     tiles 0,1 fold.  The fold is cut into pieces (fold_piece, fold_piece8,
//     the closes of a split entry) and each MFMA is followed by its share,
//     fenced by sched_barrier, with the pad-free reverse scan (first_equal3);
//   * the document close (merge of the wave halves, score) uses v_permlane32
//     and DPP, not LDS shuffles, and no branches;
//   * per-document tape (int16, Td <= 2048) / score go to LDS and leave in
//     one coalesced pass at the end of the block;
//   * with args null (scores only, kTape = false) the fold is the v_max3
//     tree alone, with the running maximum as its root's third input, and
//     the close merges the halves by a max: no argmax, no tape.
// Block -> (query block, document range) is XCD-aware: the query blocks of
// one document range run together on one XCD, so its L2 serves the range's
// chunks to all of them.
#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>
#include <stdint.h>
#include <type_traits>

#include "fms_device.hpp"
#include "fms_group.hpp"
#include "fms_inbatch.hpp"

namespace fms {

namespace {

constexpr int kIbWaves = 4;
constexpr int kIbQpw = 4;                          // query tiles per wave
static_assert(kIbQpw == 4, "the step is written for two phases of two query tiles");
constexpr int kIbQueries = kIbWaves * kIbQpw;      // queries per block
constexpr int kIbMaxNkb = 8;                       // k-blocks of 16 features: dim <= 128
constexpr int kIbMaxTq = 4096;                     // query tokens (tiles of 32 past 32)
constexpr int kIbBufs = 3;                         // LDS chunk buffers (kIbBufs - 1 chunks in flight)
static_assert(kIbBufs == 3 || kIbBufs == 4, "the step loop rotates 3 or 4 buffers");
constexpr int kXcds = 8;
constexpr int kIbMaxChunkMasks = 512;            // documents x chunks per block
constexpr int kIbMaxDocs = 40;                   // documents per block
constexpr int kIbMaxChunks = 64;                 // chunks per document (Td <= 2048)
constexpr int kIbMaxList = (kIbMaxChunkMasks + kIbBufs - 1) / kIbBufs * kIbBufs;  // padded stream
constexpr int kIbBlocksPerCu = 2;                // occupancy the launch bounds ask for
constexpr int kIbBalanceMaxDocs = 6144;          // partition weights fit the result area
// List entry: chunk (6 bits) | document in block (6) | last chunk of its
// document (1) | first valid token + 1 (19).
constexpr int kInfoDocShift = 6, kInfoLastBit = 12, kInfoFirstShift = 13;
constexpr uint32_t kInfoDocMask = 63u, kInfoFirstMask = 0x7ffffu;
// Plan value of a document's first valid token: the token (-1 = none), with
// kPlanNfBit set when its feature row holds an Inf or NaN.
constexpr int kPlanNfBit = 30;
constexpr int kPlanTooLong = -2;  // packed document longer than max_len
static_assert(kIbMaxDocs <= (int)kInfoDocMask + 1, "document index fits its field");
// In-batch layout: the stream is made of 16-row units (rows 16u .. 16u+15 of
// a document), two per list entry, so a document's last unit and the next
// document's first share a chunk.  Entry: unit of the chunk's first half
// (7 bits) | unit of its second half (7) | their documents (6 + 6) | split:
// the halves belong to different documents, the first closes after its half
// (1) | last: the second half's document closes after the chunk (1).  A
// separate word holds the two documents' first valid tokens (16 + 16 bits).
constexpr int kHU1Shift = 7, kHDoc0Shift = 14, kHDoc1Shift = 20, kHSplitBit = 26, kHLastBit = 27;
constexpr uint32_t kHUMask = 127u;
static_assert(2 * kIbMaxChunks <= (int)kHUMask + 1, "unit index fits its field");

}  // namespace

// This lane's index, computed where it is used (volatile: not hoisted out of
// a loop, so it does not hold a register across it).
__device__ __forceinline__ int lane_id_here() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// Workgroup barrier that does not drain in-flight global loads: wait only
// for this wave's LDS accesses (lgkmcnt(0)), then s_barrier.
// __syncthreads() would add a release fence, i.e. s_waitcnt vmcnt(0), and
// stall on the chunk loads that are deliberately kept in flight across the
// barrier.  The empty asm statements stop the compiler from moving LDS
// accesses across.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt / expcnt unconstrained
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Workgroup barrier after this wave's LDS accesses AND all but its last
// kVm buffer loads have completed: the loads of the chunk the next step
// reads (each wave's own share of it) are in LDS before any wave passes.
template <int kVm>
__device__ __forceinline__ void dma_barrier() {
  static_assert(kVm >= 0 && kVm < 16, "vmcnt field");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0070 | kVm);  // vmcnt(kVm) lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Whether any 16-bit element of a fragment word pair is Inf or NaN.
template <class Op>
__device__ __forceinline__ bool frag_nonfinite(const u32x4& w) {
  constexpr uint32_t e = std::is_same<Op, OpBF16>::value ? 0x7f80u : 0x7c00u;
  bool nf = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) nf |= ((w[i] & e) == e) | ((w[i] & (e << 16)) == (e << 16));
  return nf;
}


// Whether the feature row of rb <= 256 bytes at `row` (16-bit elements, bf16
// or fp16) holds an Inf or NaN: one dword per lane, wave ballot.  Uniform
// result.
__device__ __forceinline__ bool row_nonfinite(const char* row, int bf16, int rb) {
  const int lane = threadIdx.x & 63;
  const uint32_t w = lane * 4 < rb ? *reinterpret_cast<const uint32_t*>(row + lane * 4) : 0u;
  const uint32_t e = bf16 ? 0x7f807f80u : 0x7c007c00u;
  const bool nf = ((w & (e & 0xffffu)) == (e & 0xffffu)) | ((w & (e & 0xffff0000u)) == (e & 0xffff0000u));
  return __ballot(nf) != 0ull;
}

// Per-document chunk plan, computed once per call rather than once per query
// block: one wave per document, lane = chunk (nch <= 64).  cmask[j*nch + ch]
// holds the valid rows of chunk ch of document j (rows past Td clear),
// dcount[j] the chunks with a valid row, dfirst[j] the first valid token
// (-1 = none) with kPlanNfBit set when that token's row is not finite.
__global__ void __launch_bounds__(256) inbatch_plan_kernel(const uint8_t* dm, const char* D,
                                                           int bf16, int rb, int Bd, int Td, int nch,
                                                           uint32_t* cmask, int32_t* dcount,
                                                           int32_t* dfirst) {
  const int lane = threadIdx.x & 63;
  const int j = blockIdx.x * 4 + uniform(threadIdx.x >> 6);
  if (j >= Bd) return;
  const int rows = Td - lane * kTile;
  uint32_t m = rows >= kTile ? 0xffffffffu : (rows > 0 ? (1u << rows) - 1u : 0u);
  if (dm) {
    // 32 byte loads per lane, all in flight; bytes past the document read 0.
    const rsrc_t r = make_rsrc(dm + (int64_t)j * Td, (uint32_t)Td);
    uint32_t b[kTile];
#pragma unroll
    for (int t = 0; t < kTile; ++t) b[t] = buf_load1(r, lane * kTile + t);
    uint32_t bits = 0u;
#pragma unroll
    for (int t = 0; t < kTile; ++t) bits |= (b[t] & 0xffu) ? (1u << t) : 0u;
    m &= bits;
  }
  if (lane < nch) cmask[(int64_t)j * nch + lane] = m;
  const uint64_t nz = __ballot(m != 0u);
  int f = -1;
  if (nz != 0u) {
    const int k = __builtin_ctzll(nz);
    f = k * kTile + __builtin_ctz((uint32_t)__builtin_amdgcn_readlane((int)m, k));
    if (row_nonfinite(D + ((int64_t)j * Td + f) * rb, bf16, rb)) f |= 1 << kPlanNfBit;
  }
  if (lane == 0) {
    dcount[j] = __builtin_popcountll(nz);
    dfirst[j] = f;
  }
}

// The same plan for PackedSeq documents: document j is token rows
// [cu[j]-1, cu[j+1]-1) (clamped into the token range, as the packed scans
// clamp a malformed device cu); every row is valid.  A document longer than
// Td = max_len rows does not fit the plan: it gets no chunks and the plan
// value kPlanTooLong, and the scan writes NaN scores for it rather than
// scoring a truncated document.
__global__ void __launch_bounds__(256) packed_plan_kernel(const int32_t* cu, const char* tokens,
                                                          int bf16, int rb, int64_t ntok, int Bd, int Td,
                                                          int nch, uint32_t* cmask,
                                                          int32_t* dcount, int32_t* dfirst) {
  const int lane = threadIdx.x & 63;
  const int j = blockIdx.x * 4 + uniform(threadIdx.x >> 6);
  if (j >= Bd) return;
  const int64_t a = std::min<int64_t>(std::max<int64_t>((int64_t)cu[j] - 1, 0), ntok);
  const int64_t z = std::min<int64_t>(std::max<int64_t>((int64_t)cu[j + 1] - 1, a), ntok);
  const bool too_long = z - a > Td;
  const int len = too_long ? 0 : (int)(z - a);
  const int rows = len - lane * kTile;
  const uint32_t m = rows >= kTile ? 0xffffffffu : (rows > 0 ? (1u << rows) - 1u : 0u);
  if (lane < nch) cmask[(int64_t)j * nch + lane] = m;
  int f = too_long ? kPlanTooLong : -1;
  if (len > 0) f = row_nonfinite(tokens + a * rb, bf16, rb) ? (1 << kPlanNfBit) : 0;
  if (lane == 0) {
    dcount[j] = (len + kTile - 1) / kTile;
    dfirst[j] = f;
  }
}

// Exclusive scan over the 64 * kIbWaves threads of a block; every thread
// must call it.  *total receives the block sum.
__device__ int block_exclusive_scan_i32(int v, int* total) {
  __shared__ int wsum[kIbWaves];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) wsum[wave] = x;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kIbWaves; ++w) {
    const int sw = wsum[w];
    before += w < wave ? sw : 0;
    all += sw;
  }
  __syncthreads();
  *total = all;
  return before + x - v;
}

// kPacked: documents are PackedSeq token ranges (A.cu), not Td-row slabs.
// kT24 (Tq == 24): a wave's 4 queries are 96 consecutive query tokens, which
// fill 3 tiles of 32 exactly (instead of 4 tiles three-quarters full); a step
// is then one phase -- three MFMA chains over the chunk while the previous
// chunk's three tiles fold -- and a document's close sums each query over
// the lanes (and tiles) that hold its tokens.
// kNkb: k-blocks of 16 features per token (dim = 16 * kNkb, 2..8).  A chunk
// is kNkb k-blocks of 1 KB; wave w copies k-block w mod kNkb of every chunk
// (with fewer k-blocks than waves, two waves copy the same bytes to the same
// place, so every wave issues the same loads per step).
// kTape = false: args is null (scores only, as the reference's maxsim keeps
// them, dispatch.jl:124): the fold keeps the running maximum alone.
template <class Op, bool kPacked, bool kT24, int kNkb, bool kTape>
__global__ void __launch_bounds__(64 * kIbWaves, kIbBlocksPerCu) inbatch_mfma(const InBatchArgs A) {
  typedef typename Op::Acc Acc;
  typedef typename Op::Frag Frag;
  static_assert(kNkb >= 1 && kNkb <= kIbMaxNkb, "query tiles of dim <= 128 stay in registers");
  // The in-batch layout streams 16-row units; the packed layouts (long
  // documents, little tail to save) stream whole 32-row document chunks.
  constexpr bool kHalf = !kPacked && !kT24;
  constexpr int kIbNkb = kNkb;
  constexpr int kIbRowBytes = kNkb * 32;                                // bytes per token row
  constexpr int kIbFrags = kNkb * 64;                                   // 16-byte fragments per chunk
  constexpr int kIbKbPerWave = (kNkb + kIbWaves - 1) / kIbWaves;        // copies per wave per chunk
  // Chunk buffers, in MFMA fragment order: fragment (kb, lane) at
  // [kb * 64 + lane].  Four separate arrays, so the compiler can tell which
  // buffer each load-to-LDS writes.
  __shared__ u32x4 cbuf0[kIbFrags], cbuf1[kIbFrags], cbuf2[kIbFrags];
  __shared__ u32x4 cbuf3[kIbBufs == 4 ? kIbFrags : 1];
  __shared__ uint32_t chunk_mask[kIbMaxChunkMasks];  // valid rows per (doc, chunk)
  __shared__ int32_t doc_first[kIbMaxDocs];          // plan value: first valid token | flag
  __shared__ uint32_t lst_mask[kIbMaxList];          // compacted chunk list
  __shared__ uint32_t lst_info[kIbMaxList];
  __shared__ int32_t lst_row0[kPacked ? kIbMaxList : 1];  // packed: document's first row
  __shared__ uint32_t lst_first[kHalf ? kIbMaxList : 1];  // units: first valid tokens
  __shared__ int unit_start[kHalf ? kIbMaxDocs + 1 : 1];  // units: a document's first entry unit
  __shared__ int unit_first[kHalf ? kIbMaxDocs : 1];      //   and its first unit
  __shared__ int32_t doc_row0[kPacked ? kIbMaxDocs + 1 : 1];
  __shared__ int lst_count;
  __shared__ int any_nf;  // some document's first valid row is not finite
  __shared__ int16_t res_tape[kIbWaves][kIbQpw][kIbMaxDocs][kTile];  // Td <= 2048
  // Scores per (wave, query tile, document), then (units) 64 sink floats
  // for the branch-free close: lane 31 stores the score, the other lanes
  // store to the sink.  One array, so the compiler can tell the store from
  // the chunk buffers the loads to LDS write (a store through a pointer
  // that may point into either of two arrays made it wait for every load
  // in flight at each close).
  constexpr int kScoreWords = kIbWaves * kIbQpw * kIbMaxDocs;
  __shared__ float score_buf[kScoreWords + (kHalf ? 64 : 0)];
  float (&res_score)[kIbWaves][kIbQpw][kIbMaxDocs] =
      *reinterpret_cast<float(*)[kIbWaves][kIbQpw][kIbMaxDocs]>(score_buf);

  const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
  const int r32 = lane & 31, h = lane >> 5;

  // XCD-aware block mapping.  Blocks are dealt round-robin to the 8 XCDs
  // (XCD = id % 8); in each XCD's own order k = id / 8 the query block runs
  // fastest, so the nqb blocks of one document range are dispatched together
  // on one XCD and stream the range's chunks through that XCD's L2 at about
  // the same time: HBM delivers each range about once, not once per query
  // block.  Document range db = (k / nqb) * 8 + XCD (the grid is padded to
  // whole rows of 8 ranges).
  const int nqb = A.nqb, ndb = A.ndb;
  const int id = blockIdx.x;
  const int xcd = id % kXcds, kx = id / kXcds;
  const int qb = kx % nqb;
  const int db = (kx / nqb) * kXcds + xcd;
  if (db >= ndb) return;

  // ---- this block's documents -------------------------------------------------
  // Uniform: block b takes documents [b*Bd/ndb, (b+1)*Bd/ndb) (at most A.db).
  // Balanced (A.balance): the document blocks split the documents by weight
  // dcount + 1 (chunk steps plus the close), block b taking the documents
  // whose weight prefix lies in [b, b+1) * total / ndb; every block checks
  // that no block would exceed A.dbcap documents and falls back to the
  // uniform split otherwise, so all blocks agree.
  __shared__ int part_j0, part_j1, part_bad;
  int j0 = (int)((int64_t)db * A.Bd / ndb), j1 = (int)((int64_t)(db + 1) * A.Bd / ndb);
  if (A.balance) {
    int32_t* const wpre = reinterpret_cast<int32_t*>(&res_tape[0][0][0][0]);  // (Bd + 1,)
    const int Bd = A.Bd;
    const int per = (Bd + 64 * kIbWaves - 1) / (64 * kIbWaves);  // documents per thread
    const int jb = tid * per, je = jb + per < Bd ? jb + per : Bd;
    int local = 0;
    for (int j = jb; j < je; ++j) local += A.dcount[j] + 1;
    if (tid == 0) { part_j0 = Bd; part_j1 = Bd; part_bad = 0; }
    int total;
    int run = block_exclusive_scan_i32(local, &total);
    for (int j = jb; j < je; ++j) {
      wpre[j] = run;
      run += A.dcount[j] + 1;
    }
    __syncthreads();
    const int ndbk = A.ndb, cap = A.dbcap;
    // Tilted (A.tilt): the dispatcher fills one slot of every CU before the
    // second, so in a one-round grid the blocks of the first half of the
    // document ranges are the older block of their CU, which the SIMDs favour
    // (measured: the younger ran ~10% slower at equal work).  Those ranges get
    // 22 parts of the weight, the second half 18.
    const int64_t half = ndbk / 2, wo = 22, wy = 18;
    auto bucket = [&](int j) {
      if (!A.tilt) return (int)(((int64_t)wpre[j] * ndbk) / total);
      const int64_t x = ((int64_t)wpre[j] * half * (wo + wy)) / total;
      return (int)(x < half * wo ? x / wo : half + (x - half * wo) / wy);
    };
    for (int j = tid; j < Bd; j += 64 * kIbWaves) {
      const int bj = bucket(j);
      const int bp = j > 0 ? bucket(j - 1) : -1;
      if (bj >= db && bp < db) part_j0 = j;
      if (bj >= db + 1 && bp < db + 1) part_j1 = j;
      if (j + cap < Bd && bucket(j + cap) == bj) part_bad = 1;
    }
    __syncthreads();
    if (!part_bad) {  // (LDS values: made wave-uniform for the buffer descriptors)
      j0 = uniform(part_j0);
      j1 = uniform(part_j1);
    }
    __syncthreads();  // partition scratch (result area) free again
  }
  const int ndoc = j1 - j0;
  const int Tq = A.Tq, Td = A.Td;
  // Packed: the block's documents are token rows [row(j0), row(j1)); doc_row0
  // holds each one's first row relative to row(j0) (cu clamped into the
  // token range, as the packed scans clamp it).
  int64_t prow0 = 0;
  if constexpr (kPacked) {
    if (tid <= ndoc) {
      const int64_t a = std::min<int64_t>(std::max<int64_t>((int64_t)A.cu[j0 + tid] - 1, 0), A.ntok);
      doc_row0[tid] = (int32_t)std::min<int64_t>(a, (int64_t)0x7fffffff);
    }
    __syncthreads();
    prow0 = uniform(doc_row0[0]);
    __syncthreads();
    if (tid <= ndoc) doc_row0[tid] -= (int32_t)prow0;
  }
  const int nch = Td > 0 ? (Td + kTile - 1) / kTile : 1;  // <= 64
  const int nall = ndoc * nch;

  // ---- this block's chunk masks and first tokens, from the plan ------------------
  // (issued before the query loads, so waiting for them leaves those in flight)
  uint32_t cm[kIbMaxChunkMasks / (64 * kIbWaves)];
#pragma unroll
  for (int k = 0; k < kIbMaxChunkMasks / (64 * kIbWaves); ++k) {
    const int c = tid + k * 64 * kIbWaves;
    cm[k] = c < nall ? A.cmask[(int64_t)j0 * nch + c] : 0u;
  }
  const int dfv = tid < ndoc ? A.dfirst[j0 + tid] : -1;

  // ---- resident query tiles --------------------------------------------------
  // Query masks are loaded unconditionally (an empty resource when absent
  // reads 0) and tested only when a document closes.
  // Query rows of the kernel: with A.ntq > 1 tiles per query (Tq > 32), row
  // v is tokens 32 * (v % ntq) .. + 31 of query v / ntq (qrow, qt0, qtn: that
  // query, first token and token count); else row v is query v.
  Frag qf[kIbQpw][kIbNkb];
  uint32_t qmb[kIbQpw];  // per query (kT24: per tile, this lane's token)
  bool qlive[kIbQpw];
  int qi[kIbQpw], qrow[kIbQpw], qt0[kIbQpw], qtn[kIbQpw];
  const int ntq = A.ntq, nqv = A.Bq * ntq;
#pragma unroll
  for (int q = 0; q < kIbQpw; ++q) {
    qi[q] = qb * kIbQueries + wave * kIbQpw + q;
    qlive[q] = qi[q] < nqv;
    qrow[q] = qi[q] / ntq;
    qt0[q] = (qi[q] - qrow[q] * ntq) * kTile;
    qtn[q] = std::min(kTile, Tq - qt0[q]);
  }
  if constexpr (!kT24) {
#pragma unroll
    for (int q = 0; q < kIbQpw; ++q) {
      const bool live = qlive[q];
      const int64_t tok0 = live ? (int64_t)qrow[q] * Tq + qt0[q] : 0;
      const rsrc_t rq = make_rsrc(A.Q + tok0 * kIbRowBytes, live ? (uint32_t)qtn[q] * kIbRowBytes : 0u);
      const int base = r32 * kIbRowBytes + h * 16;
#pragma unroll
      for (int kb = 0; kb < kIbNkb; ++kb) qf[q][kb] = Op::load(rq, base + kb * 32);
      qmb[q] = buf_load1(make_rsrc(A.qm ? (const void*)(A.qm + tok0) : (const void*)A.Q,
                                   (A.qm && live) ? (uint32_t)qtn[q] : 0u), r32);
    }
  } else {
    // The wave's live queries are consecutive rows of Q: tile t, lane r32 holds
    // token 32t + r32 of the 96 (rows past the live queries read 0).
    const int nlive = std::max(0, std::min(kIbQpw, A.Bq - qi[0]));
    const rsrc_t rq = make_rsrc(A.Q + (int64_t)qi[0] * 24 * kIbRowBytes,
                                (uint32_t)(nlive * 24 * kIbRowBytes));
    const rsrc_t rm = make_rsrc(A.qm ? (const void*)(A.qm + (int64_t)qi[0] * 24) : (const void*)A.Q,
                                A.qm ? (uint32_t)(nlive * 24) : 0u);
#pragma unroll
    for (int t = 0; t < 3; ++t) {
      const int base = (32 * t + r32) * kIbRowBytes + h * 16;
#pragma unroll
      for (int kb = 0; kb < kIbNkb; ++kb) qf[t][kb] = Op::load(rq, base + kb * 32);
      qmb[t] = buf_load1(rm, 32 * t + r32);
    }
  }
  const bool has_qm = A.qm != nullptr;
  auto token_valid = [&](int q) {
    return qlive[q] && r32 < qtn[q] && (!has_qm || qmb[q] != 0u);
  };
  // kT24: the query (0..3 in the wave) and token (0..23) of this lane in tile t,
  // and whether that token is valid.
  auto t24_query = [&](int t) { return (32 * t + r32) / 24; };
  auto t24_token = [&](int t) { return (32 * t + r32) % 24; };
  auto t24_valid = [&](int t) {
    const int qq = t24_query(t);
    const bool live = qq == 0 ? qlive[0] : qq == 1 ? qlive[1] : qq == 2 ? qlive[2] : qlive[3];
    return live && (!has_qm || qmb[t] != 0u);
  };
#pragma unroll
  for (int k = 0; k < kIbMaxChunkMasks / (64 * kIbWaves); ++k) {
    const int c = tid + k * 64 * kIbWaves;
    if (c < nall) chunk_mask[c] = cm[k];
  }
  if (tid < ndoc) doc_first[tid] = dfv;
  if (tid == 0) any_nf = 0;

  // ---- defaults of the results --------------------------------------------------
  // A document without a valid token never closes: score 0, tape 0.
  static_assert(sizeof(res_tape) % (16 * 64 * kIbWaves) == 0, "whole 16-byte stores");
  if constexpr (kTape) {
#pragma unroll
    for (int k = 0; k < (int)(sizeof(res_tape) / (16 * 64 * kIbWaves)); ++k)
      reinterpret_cast<u32x4*>(&res_tape[0][0][0][0])[tid + k * 64 * kIbWaves] = u32x4{0u, 0u, 0u, 0u};
  }
  for (int e = tid; e < kIbWaves * kIbQpw * kIbMaxDocs; e += 64 * kIbWaves)
    (&res_score[0][0][0])[e] = 0.0f;
  __syncthreads();  // chunk_mask, doc_first complete
  if (tid < ndoc && dfv >= 0 && ((dfv >> kPlanNfBit) & 1)) any_nf = 1;
  if (tid < ndoc && dfv == kPlanTooLong) {  // packed document longer than max_len: NaN
    for (int w = 0; w < kIbWaves; ++w)
      for (int q = 0; q < kIbQpw; ++q)
        res_score[w][q][tid] = __builtin_bit_cast(float, 0x7fc00000u);
  }

  // ---- compacted chunk list ------------------------------------------------------
  if constexpr (kHalf) {
    // Unit stream.  A document's units run from its first unit with a valid
    // row to its last (masked rows in between are substituted at load time),
    // documents follow each other in the block's order, and entry e holds
    // units 2e and 2e+1 (the last entry's second half, when the count is
    // odd, is the next unit of its first half's document, all rows masked).
    // Entry e: row validity lst_mask[e] (bits 0-15 the first half's rows,
    // 16-31 the second's), lst_info[e] as the kH* constants describe,
    // lst_first[e] the two documents' first valid tokens.
    if (wave == 0) {
      int fu = -1, lu = -1;
      if (lane < ndoc) {
        for (int c = 0; c < nch; ++c) {
          const uint32_t m = chunk_mask[lane * nch + c];
          if (m & 0xffffu) {
            fu = fu < 0 ? 2 * c : fu;
            lu = 2 * c;
          }
          if (m >> 16) {
            fu = fu < 0 ? 2 * c + 1 : fu;
            lu = 2 * c + 1;
          }
        }
      }
      const int n = fu < 0 ? 0 : lu - fu + 1;
      int incl = n;  // inclusive prefix over the lanes (documents), lanes >= ndoc add 0
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(incl, o);
        incl += lane >= o ? v : 0;
      }
      if (lane <= ndoc) unit_start[lane] = incl - n;  // unit_start[ndoc] = total
      if (lane < ndoc) unit_first[lane] = fu;
      if (lane == 63) lst_count = incl;
    }
    __syncthreads();
    const int nunit = lst_count;
    const int nent = (nunit + 1) >> 1;
    // document of unit k: the last document whose first unit is <= k (a
    // document without units starts where the next one does)
    auto doc_of = [&](int k) {
      int lo = 0, hi = ndoc - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (unit_start[mid] <= k) lo = mid;
        else hi = mid - 1;
      }
      return lo;
    };
    auto unit_bits = [&](int jj, int u) {
      return (chunk_mask[jj * nch + (u >> 1)] >> ((u & 1) * 16)) & 0xffffu;
    };
    for (int e = tid; e < nent; e += 64 * kIbWaves) {
      const int k0 = 2 * e, k1 = k0 + 1;
      const int d0 = doc_of(k0), u0 = unit_first[d0] + (k0 - unit_start[d0]);
      const bool has1 = k1 < nunit;
      const int d1 = has1 ? doc_of(k1) : d0;
      const int u1 = has1 ? unit_first[d1] + (k1 - unit_start[d1]) : u0 + 1;
      const bool split = d1 != d0;
      const bool lastu = !has1 || k1 + 1 == unit_start[d1 + 1];
      lst_mask[e] = unit_bits(d0, u0) | (has1 ? unit_bits(d1, u1) << 16 : 0u);
      lst_info[e] = (uint32_t)u0 | ((uint32_t)u1 << kHU1Shift) | ((uint32_t)d0 << kHDoc0Shift) |
                    ((uint32_t)d1 << kHDoc1Shift) | ((uint32_t)split << kHSplitBit) |
                    ((uint32_t)lastu << kHLastBit);
      lst_first[e] = (uint32_t)(doc_first[d0] & 0xffff) | ((uint32_t)(doc_first[d1] & 0xffff) << 16);
    }
    if (tid == 0) lst_count = nent;
    __syncthreads();
  } else {
    // Only chunks with at least one valid row are streamed and multiplied (a
    // document's fully masked tail costs nothing).  Entry i: row validity
    // lst_mask[i]; lst_info[i] packs (chunk, document, last chunk of its
    // document, first valid token + 1) as the kInfo* constants describe.
    if (wave == 0) {
      int base = 0;
      for (int c0 = 0; c0 < nall; c0 += 64) {
        const int c = c0 + lane;
        const uint32_t m = c < nall ? chunk_mask[c] : 0u;
        const uint64_t bal = __ballot(m != 0u);
        if (m != 0u) {
          const int pos = base + __builtin_popcountll(bal & ((1ull << lane) - 1ull));
          const int jj = c / nch, ch = c - jj * nch;
          lst_mask[pos] = m;
          const int df = doc_first[jj];
          const uint32_t f1 = df < 0 ? 0u : (uint32_t)(df & ~(1 << kPlanNfBit)) + 1u;
          lst_info[pos] = (uint32_t)ch | ((uint32_t)jj << kInfoDocShift) | (f1 << kInfoFirstShift);
          if constexpr (kPacked) lst_row0[pos] = doc_row0[jj];
        }
        base += __builtin_popcountll(bal);
      }
      if (lane == 0) lst_count = base;
    }
    __syncthreads();
    const int nst = uniform(lst_count);
    bool last[kIbMaxChunkMasks / (64 * kIbWaves)];
  #pragma unroll
    for (int k = 0; k < kIbMaxChunkMasks / (64 * kIbWaves); ++k) {
      const int i = tid + k * 64 * kIbWaves;
      last[k] = i < nst && (i + 1 == nst ||
                               ((lst_info[i + 1] >> kInfoDocShift) & kInfoDocMask) !=
                                   ((lst_info[i] >> kInfoDocShift) & kInfoDocMask));
    }
    __syncthreads();
  #pragma unroll
    for (int k = 0; k < kIbMaxChunkMasks / (64 * kIbWaves); ++k)
      if (last[k]) lst_info[tid + k * 64 * kIbWaves] |= 1u << kInfoLastBit;
    __syncthreads();
  }
  const int nsteps = uniform(lst_count);
  // Pad the stream to whole rounds of the kIbBufs buffers with repeats of
  // its last entry, close (and split) bits cleared: folding a chunk again
  // changes no result (a running max only moves on a strictly greater score,
  // and after the document's close nothing reads it).  The lists hold
  // kIbMaxList.
  const int nsteps_pad = (nsteps + kIbBufs - 1) / kIbBufs * kIbBufs;
  static_assert(kIbBufs <= 64 * kIbWaves, "one thread per padding entry");
  if (tid < nsteps_pad - nsteps) {
    lst_mask[nsteps + tid] = lst_mask[nsteps - 1];
    lst_info[nsteps + tid] = lst_info[nsteps - 1] & (kHalf ? ~((1u << kHSplitBit) | (1u << kHLastBit))
                                                           : ~(1u << kInfoLastBit));
    if constexpr (kPacked) lst_row0[nsteps + tid] = lst_row0[nsteps - 1];
    if constexpr (kHalf) lst_first[nsteps + tid] = lst_first[nsteps - 1];
  }
  __syncthreads();

  // ---- chunk stream -------------------------------------------------------------
  // One buffer resource spans the block's documents [j0, j1) (contiguous in
  // D).  A chunk goes HBM/L2 -> LDS with no registers in between: wave w
  // fills k-blocks kb = kIbKbPerWave*w + k, one 16-byte load per lane: lane
  // l loads units 2kb + l/32 of chunk row l%32 (a masked row loads the
  // document's first valid token instead) into fragment slot kb*64 + l.
  // The stream position stops at the last (padded) entry, so loads issued
  // past the end re-read it.
  // (packed: the block's rows run to the end of the token array, at most
  // 2^24 - 1 rows past row(j0) so the range fits the resource's 32 bits)
  const rsrc_t rd = kPacked
      ? make_rsrc_u(A.D + prow0 * kIbRowBytes,
                    (uint32_t)std::min<int64_t>(A.ntok - prow0, 0xffffff) * kIbRowBytes)
      : make_rsrc(A.D + (int64_t)j0 * Td * kIbRowBytes, (uint32_t)(ndoc * Td * kIbRowBytes));
  int ld_i = 0;  // next list entry to request
  // (units: `row0` is the entry's first-token word; row r32 of the chunk is
  // row r32 % 16 of the unit of half r32 / 16)
  auto chunk_load = [&](u32x4* buf, uint32_t m, uint32_t info, int row0) {
    int voff;
    if constexpr (kHalf) {
      // Every per-lane term is recomputed here from the lane id (an asm the
      // compiler cannot hoist) and selects between uniform values, so no
      // lane constant stays live across the step loop.
      // The half of the entry is picked by per-lane shift amounts and the
      // row by a multiply, not by selects: selects between uniform values
      // on a lane condition became exec-masked branches.
      const int ln = lane_id_here();
      const uint32_t hi = ((uint32_t)ln >> 4) & 1u;  // chunk rows 16..31: the second half
      const int ux = (int)((info >> (hi * kHU1Shift)) & kHUMask);
      const int jx = (int)((info >> (kHDoc0Shift + hi * (kHDoc1Shift - kHDoc0Shift))) & kInfoDocMask);
      const int fx = (int)(((uint32_t)row0 >> (hi << 4)) & 0xffffu);
      const int real = (int)((m >> (ln & 31)) & 1u);
      const int src = fx + real * (16 * ux + (ln & 15) - fx);
      voff = (jx * Td + src) * kIbRowBytes + ((ln >> 5) << 4);
    } else {
      const int ch = info & 63u, jj = (info >> kInfoDocShift) & kInfoDocMask;
      const int f = (int)((info >> kInfoFirstShift) & kInfoFirstMask) - 1;
      const int fsrc = f < 0 ? 0 : f;  // (never: listed chunks have a valid row)
      const int real = (int)((m >> r32) & 1u);  // (a multiply, not a select: see above)
      const int src = fsrc + real * (ch * kTile + r32 - fsrc);
      voff = ((kPacked ? row0 : jj * Td) + src) * kIbRowBytes + h * 16;
    }
#pragma unroll
    for (int k = 0; k < kIbKbPerWave; ++k) {
      const int kb = (kIbKbPerWave * wave + k) % kIbNkb;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rd, (lds_ptr_t)(buf + kb * 64), 16,
                                               voff + kb * 32, 0, 0, 0);
    }
    if (ld_i + 1 < nsteps_pad) ++ld_i;
  };

  // Running maxima and their slots.  Slots hold the chunk row base plus the
  // register's row offset (kRowSlots of the folds): unit stream, 16 (v + 1)
  // where chunk row 0 is document row 16 v; 32-row chunks, 32 x chunk.  The
  // 1-based token is then slot + tok_off(), and kNoSlot (nothing taken)
  // gives a token below 1.  (tok_off is recomputed from the lane id where it
  // is used: one more register live across the step loop made it spill.)
  constexpr int kNoSlot = -(1 << 24);
  auto tok_off = [&]() { return ((lane_id_here() >> 3) & 4) + (kHalf ? -15 : 1); };
  float mx[kIbQpw];
  int slot[kIbQpw];
#pragma unroll
  for (int q = 0; q < kIbQpw; ++q) { mx[q] = -INFINITY; slot[q] = kNoSlot; }

  // Close query q's document jj: merge the wave halves, map a winning
  // substituted row back to the first valid token f, reduce the score,
  // stage tape and score in LDS, reset the running max.  (A document whose
  // scores are all -Inf closes on f with -Inf, as the reference's first-token
  // rule gives; the NaN case of that rule is settled after the loop.)
  auto close = [&](int q, int jj, int f) {
    if constexpr (!kTape) {
      // scores only: the maximum of both halves, summed as below
      const float m = merge_halves_max(mx[q]);
      const float score = half_sum_in_lanes(token_valid(q) ? m : 0.0f);
      if constexpr (kHalf) score_buf[lane == 31 ? (wave * kIbQpw + q) * kIbMaxDocs + jj : kScoreWords + lane] = score;
      else if (lane == 31) res_score[wave][q][jj] = score;
      mx[q] = -INFINITY;
      return;
    }
    int tok = slot[q] + tok_off();
    float m = mx[q];
    merge_halves_all(m, tok);  // the folds here never take a NaN
    // Map a winning copy back to f.  The winner is the lowest row that
    // reaches the maximum, and every copy scores exactly what f scores, so
    // a copy after f never wins (f reaches the same maximum first): only a
    // masked row before f can, or none (tok 0, all scores -Inf or NaN).
    // Both are the tokens below f + 1.  After the mapping tok >= 1.
    tok = tok > f + 1 ? tok : f + 1;
    const bool tv = token_valid(q);
    // the score, left in lanes 16-31 (and 48-63): lane 31 stores it
    const float score = half_sum_in_lanes(tv ? m : 0.0f);
    if constexpr (kHalf) {
      // without branches: both halves hold the merged token and store it to
      // the same place; lanes other than 31 store the score to a sink
      res_tape[wave][q][jj][r32] = (int16_t)(tv ? tok : 0);
      score_buf[lane == 31 ? (wave * kIbQpw + q) * kIbMaxDocs + jj : kScoreWords + lane] = score;
    } else {
      if (h == 0) res_tape[wave][q][jj][r32] = (int16_t)(tv ? tok : 0);
      if (lane == 31) res_score[wave][q][jj] = score;
    }
    mx[q] = -INFINITY;
    slot[q] = kNoSlot;
  };

  // Fold one query tile's chunk scores into its running max/argmax, and
  // close the document when `inf` is its last chunk.
  auto fold_close = [&](int q, const Acc& ac, uint32_t inf) {
    float sc[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) sc[r] = ac[r];
    if constexpr (kTape) fold_tree<false, true>(sc, (int)(inf & 63u) * kTile, mx[q], slot[q]);
    else fold_max(sc, mx[q]);
  };
  auto close_if_last = [&](int q0, int q1, uint32_t inf) {
    if (inf & (1u << kInfoLastBit)) {
      const int jj = (inf >> kInfoDocShift) & kInfoDocMask;
      const int f = (int)((inf >> kInfoFirstShift) & kInfoFirstMask) - 1;
      close(q0, jj, f);
      close(q1, jj, f);
    }
  };

  // kT24: close the three tiles of the document of entry `inf` together when
  // it was the document's last chunk.  Each tile merges and maps back as
  // `close` does; query sums then split tile t at lane 24, 16 and 8 (query
  // q's 24 tokens are tokens 24q..24q+23 of the wave's 96), each part summed
  // in the order half_sum uses.
  auto close24_if_last = [&](uint32_t inf) {
    if (inf & (1u << kInfoLastBit)) {
      const int jj = (inf >> kInfoDocShift) & kInfoDocMask;
      const int f = (int)((inf >> kInfoFirstShift) & kInfoFirstMask) - 1;
      float part[3];
#pragma unroll
      for (int t = 0; t < 3; ++t) {
        if constexpr (kTape) {
          int tok = slot[t] + tok_off();
          float m = mx[t];
          merge_halves_all(m, tok);
          tok = tok > f + 1 ? tok : f + 1;  // a winning copy maps back to f, as in `close`
          const bool tv = t24_valid(t);
          part[t] = tv ? m : 0.0f;
          if (h == 0) res_tape[wave][t24_query(t)][jj][t24_token(t)] = (int16_t)(tv ? tok : 0);
        } else {
          part[t] = t24_valid(t) ? merge_halves_max(mx[t]) : 0.0f;
        }
        mx[t] = -INFINITY;
        slot[t] = kNoSlot;
      }
      const float l0 = half_sum(r32 < 24 ? part[0] : 0.0f), u0 = half_sum(r32 < 24 ? 0.0f : part[0]);
      const float l1 = half_sum(r32 < 16 ? part[1] : 0.0f), u1 = half_sum(r32 < 16 ? 0.0f : part[1]);
      const float l2 = half_sum(r32 < 8 ? part[2] : 0.0f), u2 = half_sum(r32 < 8 ? 0.0f : part[2]);
      if (lane == 0) {
        res_score[wave][0][jj] = l0;
        res_score[wave][1][jj] = u0 + l1;
        res_score[wave][2][jj] = u1 + l2;
        res_score[wave][3][jj] = u2;
      }
    }
  };

  // Tiles (qa, qb) x a chunk (fragments `a`) as two MFMA chains, and after
  // each MFMA one eighth of the fold of tiles fa and fb (scores x0, x1 of
  // an entry whose first slot is slot0), fenced so that every MFMA has its
  // share of VALU work beside it and the fold's compares need no wait-state
  // padding (fold_piece).
  auto mma_fold_pinned = [&](const Frag (&a)[kIbNkb], Acc& na, Acc& nb, int qa, int qb,
                             const Acc& x0, const Acc& x1, int fa, int fb, int slot0) {
    float s0[16], s1[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) { s0[r] = x0[r]; s1[r] = x1[r]; }
    na = Acc{};
    nb = Acc{};
    FoldPieces pa, pb;
    MaxPieces xa, xb;  // (scores only)
    constexpr int kM = 2 * kIbNkb;  // MFMAs of the phase
    static_for<0, kM>([&](auto kc) {
      constexpr int k = decltype(kc)::value;
      if constexpr (k % 2 == 0) na = Op::mma(a[k / 2], qf[qa][k / 2], na);
      else nb = Op::mma(a[k / 2], qf[qb][k / 2], nb);
      static_for<(16 * k + kM - 1) / kM, (16 * (k + 1) + kM - 1) / kM>([&](auto pc) {
        constexpr int p = decltype(pc)::value;
        if constexpr (!kTape) {
          if constexpr (p < 8) fold_max_piece<p>(xa, s0, mx[fa]);
          else fold_max_piece<p - 8>(xb, s1, mx[fb]);
        } else if constexpr (p < 8) {
          fold_piece<p, true>(pa, s0, slot0, mx[fa], slot[fa]);
        } else {
          fold_piece<p - 8, true>(pb, s1, slot0, mx[fb], slot[fb]);
        }
      });
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // One step: entry i+1 register -> LDS, refill that register stage with
  // entry i+3, read the list info for the next step, then two phases of 16
  // MFMAs (two independent accumulation chains each):
  //   phase 1: tiles 0,1 x entry i  while tiles 2,3 of entry i-1 are folded;
  //   phase 2: tiles 2,3 x entry i  while tiles 0,1 of entry i are folded.
  // Every phase's VALU work is independent of its MFMAs, so the two overlap
  // within the wave, and only 4 accumulator tiles are ever live.
  uint32_t ld_m = 0u, ld_info = 0u;  // list entry ld_i, read one step ahead
  int ld_r0 = 0;
  uint32_t cur_info = 0u;            // list entry i
  uint32_t prev_info = 0u;           // list entry i-1 (no close bit before step 0)
  Acc lag2, lag3;                    // tiles 2,3 of entry i-1
#pragma unroll
  for (int r = 0; r < 16; ++r) { lag2[r] = -INFINITY; lag3[r] = -INFINITY; }
  // Step i multiplies buffer `cur` (entry i) and requests entry
  // i + kIbBufs - 1 into buffer `ahead` (the one entry i-1 used).
  auto step = [&](int i, const u32x4* cur, u32x4* ahead) {
    chunk_load(ahead, (uint32_t)uniform((int)ld_m), (uint32_t)uniform((int)ld_info), uniform(ld_r0));
    // Issue priority falls as the step progresses (3, 2, 1): of the two waves
    // on a SIMD (one from each of the CU's two blocks) the one further behind
    // in its step issues first, so neither block runs ahead of the other.
    __builtin_amdgcn_s_setprio(3);
    // List entries for the next step, read now so the LDS latency hides
    // behind this step's MFMAs instead of stalling before the barrier.
    ld_m = lst_mask[ld_i];
    ld_info = lst_info[ld_i];
    if constexpr (kPacked) ld_r0 = lst_row0[ld_i];
    const uint32_t next_info = lst_info[i + 1 < nsteps_pad ? i + 1 : i];
    const uint32_t info = (uint32_t)uniform((int)cur_info);
    const uint32_t pinfo = (uint32_t)uniform((int)prev_info);
    Frag a[kIbNkb];
#pragma unroll
    for (int kb = 0; kb < kIbNkb; ++kb) a[kb] = cur[kb * 64 + lane];
    Acc n0, n1, n2, n3;
    mma_fold_pinned(a, n0, n1, 0, 1, lag2, lag3, 2, 3, (int)(pinfo & 63u) * kTile);
    close_if_last(2, 3, pinfo);
    __builtin_amdgcn_s_setprio(2);
    mma_fold_pinned(a, n2, n3, 2, 3, n0, n1, 0, 1, (int)(info & 63u) * kTile);
    close_if_last(0, 1, info);
    __builtin_amdgcn_s_setprio(1);
    lag2 = n2;
    lag3 = n3;
    prev_info = info;
    cur_info = next_info;
    // Entry i+1's loads were issued before those of entries i+2 .. i+kIbBufs-1,
    // which alone may remain.
    dma_barrier<(kIbBufs - 2) * kIbKbPerWave>();
  };

  // Unit-stream folds (kHalf).  An entry whose halves hold one document
  // folds all 16 registers at once; a split entry folds registers 0..7 into
  // the first document, closes it, and starts the second document with
  // registers 8..15 (the close is branch-free, so the whole phase stays one
  // block for the scheduler to interleave with its MFMAs).  Slots are
  // (v + 1) * 16 + the register's row offset, where chunk row 0 is document
  // row 16 v (the upper half's registers 8..15 start at row offset 16).
  auto fold_units = [&](int q0, int q1, const Acc& x0, const Acc& x1, uint32_t inf, auto split) {
    float s0[16], s1[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) { s0[r] = x0[r]; s1[r] = x1[r]; }
    const int v0 = (int)(inf & kHUMask);
    if constexpr (!kTape) {
      if constexpr (decltype(split)::value) {
        const int jj = (int)((inf >> kHDoc0Shift) & kInfoDocMask);
        fold_max8<false>(s0, mx[q0]);
        fold_max8<false>(s1, mx[q1]);
        close(q0, jj, 0);
        close(q1, jj, 0);
        fold_max8<true>(s0, mx[q0]);
        fold_max8<true>(s1, mx[q1]);
      } else {
        fold_max(s0, mx[q0]);
        fold_max(s1, mx[q1]);
      }
    } else if constexpr (decltype(split)::value) {
      const int v1 = (int)((inf >> kHU1Shift) & kHUMask) - 1;
      const int jj = (int)((inf >> kHDoc0Shift) & kInfoDocMask);
      const int f = uniform(doc_first[jj]) & 0xffff;
      fold_tree8<false, true>(s0, (v0 + 1) * 16, mx[q0], slot[q0]);
      fold_tree8<false, true>(s1, (v0 + 1) * 16, mx[q1], slot[q1]);
      close(q0, jj, f);
      close(q1, jj, f);
      fold_tree8<true, true>(s0, (v1 + 1) * 16 + 16, mx[q0], slot[q0]);
      fold_tree8<true, true>(s1, (v1 + 1) * 16 + 16, mx[q1], slot[q1]);
    } else {
      fold_tree<false, true>(s0, (v0 + 1) * 16, mx[q0], slot[q0]);
      fold_tree<false, true>(s1, (v0 + 1) * 16, mx[q1], slot[q1]);
    }
  };
  // After a phase: the entry's last bit closes its second half's document.
  auto close_units = [&](int q0, int q1, uint32_t inf) {
    if (inf & (1u << kHLastBit)) {
      const int jj = (int)((inf >> kHDoc1Shift) & kInfoDocMask);
      const int f = uniform(doc_first[jj]) & 0xffff;
      close(q0, jj, f);
      close(q1, jj, f);
    }
  };
  // A phase whose folded entry is split: tiles (qa, qb) x the chunk as two
  // MFMA chains and beside them, fenced, 18 units in fold_units' order: the
  // lower halves of tiles fa and fb (four pieces each), the closes of their
  // first document, the upper halves (four pieces each).  Without the fences
  // the scheduler issued all MFMAs first and the fold after them.
  auto mma_fold_split_pinned = [&](const Frag (&a)[kIbNkb], Acc& na, Acc& nb, int qa, int qb,
                                   const Acc& x0, const Acc& x1, int fa, int fb, uint32_t inf) {
    float s0[16], s1[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) { s0[r] = x0[r]; s1[r] = x1[r]; }
    const int v0 = (int)(inf & kHUMask);
    const int v1 = (int)((inf >> kHU1Shift) & kHUMask) - 1;
    const int jj = (int)((inf >> kHDoc0Shift) & kInfoDocMask);
    const int f = uniform(doc_first[jj]) & 0xffff;
    const int lo0 = (v0 + 1) * 16, hi0 = (v1 + 1) * 16 + 16;
    na = Acc{};
    nb = Acc{};
    FoldPieces8 la, lb, ua, ub;
    MaxPieces8 xla, xlb, xua, xub;  // (scores only)
    constexpr int kM = 2 * kIbNkb, kU = 18;
    static_for<0, kM>([&](auto kc) {
      constexpr int k = decltype(kc)::value;
      if constexpr (k % 2 == 0) na = Op::mma(a[k / 2], qf[qa][k / 2], na);
      else nb = Op::mma(a[k / 2], qf[qb][k / 2], nb);
      static_for<(kU * k + kM - 1) / kM, (kU * (k + 1) + kM - 1) / kM>([&](auto uc) {
        constexpr int u = decltype(uc)::value;
        if constexpr (u == 8) close(fa, jj, f);
        else if constexpr (u == 9) close(fb, jj, f);
        else if constexpr (!kTape) {
          if constexpr (u < 4) fold_max_piece8<u, false>(xla, s0, mx[fa]);
          else if constexpr (u < 8) fold_max_piece8<u - 4, false>(xlb, s1, mx[fb]);
          else if constexpr (u < 14) fold_max_piece8<u - 10, true>(xua, s0, mx[fa]);
          else fold_max_piece8<u - 14, true>(xub, s1, mx[fb]);
        } else if constexpr (u < 4) {
          fold_piece8<u, false>(la, s0, lo0, mx[fa], slot[fa]);
        } else if constexpr (u < 8) {
          fold_piece8<u - 4, false>(lb, s1, lo0, mx[fb], slot[fb]);
        } else if constexpr (u < 14) {
          fold_piece8<u - 10, true>(ua, s0, hi0, mx[fa], slot[fa]);
        } else {
          fold_piece8<u - 14, true>(ub, s1, hi0, mx[fb], slot[fb]);
        }
      });
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  // The step of `step` over the unit stream: each phase is written out for
  // both kinds of entry it folds (split or not), with its MFMAs, so the
  // multiplies and the fold stay interleaved in one block either way.
  auto step_units = [&](int i, const u32x4* cur, u32x4* ahead) {
    chunk_load(ahead, (uint32_t)uniform((int)ld_m), (uint32_t)uniform((int)ld_info), uniform(ld_r0));
    __builtin_amdgcn_s_setprio(3);
    ld_m = lst_mask[ld_i];
    ld_info = lst_info[ld_i];
    ld_r0 = (int)lst_first[ld_i];
    const uint32_t next_info = lst_info[i + 1 < nsteps_pad ? i + 1 : i];
    const uint32_t info = (uint32_t)uniform((int)cur_info);
    const uint32_t pinfo = (uint32_t)uniform((int)prev_info);
    Frag a[kIbNkb];
#pragma unroll
    for (int kb = 0; kb < kIbNkb; ++kb) a[kb] = cur[kb * 64 + lane];
    Acc n0, n1, n2, n3;
    auto phase1 = [&](auto split) {
      if constexpr (!decltype(split)::value) {
        mma_fold_pinned(a, n0, n1, 0, 1, lag2, lag3, 2, 3, ((int)(pinfo & kHUMask) + 1) * 16);
        return;
      }
      mma_fold_split_pinned(a, n0, n1, 0, 1, lag2, lag3, 2, 3, pinfo);
    };
    if (pinfo & (1u << kHSplitBit)) phase1(std::true_type());
    else phase1(std::false_type());
    close_units(2, 3, pinfo);
    __builtin_amdgcn_s_setprio(2);
    auto phase2 = [&](auto split) {
      if constexpr (!decltype(split)::value) {
        mma_fold_pinned(a, n2, n3, 2, 3, n0, n1, 0, 1, ((int)(info & kHUMask) + 1) * 16);
        return;
      }
      mma_fold_split_pinned(a, n2, n3, 2, 3, n0, n1, 0, 1, info);
    };
    if (info & (1u << kHSplitBit)) phase2(std::true_type());
    else phase2(std::false_type());
    close_units(0, 1, info);
    __builtin_amdgcn_s_setprio(1);
    lag2 = n2;
    lag3 = n3;
    prev_info = info;
    cur_info = next_info;
    dma_barrier<(kIbBufs - 2) * kIbKbPerWave>();
  };

  // kT24 step: entry i's chunk times the three tiles (three independent MFMA
  // chains) while the three tiles of entry i-1 fold (pinned, one fold piece
  // per MFMA); one phase, closes after the fold.  Loads, list reads and the
  // barrier as in `step`.
  Acc lagt[3];
#pragma unroll
  for (int t = 0; t < 3; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) lagt[t][r] = -INFINITY;
  auto step24 = [&](int i, const u32x4* cur, u32x4* ahead) {
    chunk_load(ahead, (uint32_t)uniform((int)ld_m), (uint32_t)uniform((int)ld_info), uniform(ld_r0));
    ld_m = lst_mask[ld_i];
    ld_info = lst_info[ld_i];
    if constexpr (kPacked) ld_r0 = lst_row0[ld_i];
    const uint32_t next_info = lst_info[i + 1 < nsteps_pad ? i + 1 : i];
    const uint32_t info = (uint32_t)uniform((int)cur_info);
    const uint32_t pinfo = (uint32_t)uniform((int)prev_info);
    Frag a[kIbNkb];
#pragma unroll
    for (int kb = 0; kb < kIbNkb; ++kb) a[kb] = cur[kb * 64 + lane];
    // The three MFMA chains, each MFMA followed by one eighth of the fold of
    // a tile of entry i-1 (24 pieces over the 3 x kIbNkb MFMAs), fenced as
    // in mma_fold_pinned.
    Acc n[3];
    {
      const int slot0 = (int)(pinfo & 63u) * kTile;
      float s[3][16];
#pragma unroll
      for (int t = 0; t < 3; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[t][r] = lagt[t][r];
      n[0] = n[1] = n[2] = Acc{};
      FoldPieces pc[3];
      MaxPieces xc[3];  // (scores only)
      constexpr int kM = 3 * kIbNkb;
      static_for<0, kM>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        n[k % 3] = Op::mma(a[k / 3], qf[k % 3][k / 3], n[k % 3]);
        static_for<(24 * k + kM - 1) / kM, (24 * (k + 1) + kM - 1) / kM>([&](auto pcc) {
          constexpr int p = decltype(pcc)::value;
          if constexpr (kTape) fold_piece<p % 8, true>(pc[p / 8], s[p / 8], slot0, mx[p / 8], slot[p / 8]);
          else fold_max_piece<p % 8>(xc[p / 8], s[p / 8], mx[p / 8]);
        });
        __builtin_amdgcn_sched_barrier(0);
      });
    }
    close24_if_last(pinfo);
    lagt[0] = n[0];
    lagt[1] = n[1];
    lagt[2] = n[2];
    prev_info = info;
    cur_info = next_info;
    dma_barrier<(kIbBufs - 2) * kIbKbPerWave>();
  };

  if (nsteps_pad > 0) {
    auto row0_at = [&](int i) {
      return kPacked ? uniform(lst_row0[i]) : kHalf ? uniform((int)lst_first[i]) : 0;
    };
    chunk_load(cbuf0, lst_mask[0], lst_info[0], row0_at(0));                // entry 0
    chunk_load(cbuf1, lst_mask[ld_i], lst_info[ld_i], row0_at(ld_i));       // entry 1
    if constexpr (kIbBufs == 4)
      chunk_load(cbuf2, lst_mask[ld_i], lst_info[ld_i], row0_at(ld_i));     // entry 2
    ld_m = lst_mask[ld_i];
    ld_info = lst_info[ld_i];
    if constexpr (kPacked) ld_r0 = lst_row0[ld_i];
    if constexpr (kHalf) ld_r0 = (int)lst_first[ld_i];
    cur_info = lst_info[0];
    dma_barrier<(kIbBufs - 2) * kIbKbPerWave>();  // entry 0 in LDS
    // Every load is unconditional and the buffers rotate statically.
    for (int i = 0; i < nsteps_pad; i += kIbBufs) {
      if constexpr (kT24) {
        static_assert(kIbBufs == 3, "the kT24 loop rotates 3 buffers");
        step24(i, cbuf0, cbuf2);
        step24(i + 1, cbuf1, cbuf0);
        step24(i + 2, cbuf2, cbuf1);
      } else if constexpr (kHalf) {
        static_assert(kIbBufs == 3, "the unit-stream loop rotates 3 buffers");
        step_units(i, cbuf0, cbuf2);
        step_units(i + 1, cbuf1, cbuf0);
        step_units(i + 2, cbuf2, cbuf1);
      } else if constexpr (kIbBufs == 4) {
        step(i, cbuf0, cbuf3);
        step(i + 1, cbuf1, cbuf0);
        step(i + 2, cbuf2, cbuf1);
        step(i + 3, cbuf3, cbuf2);
      } else {
        step(i, cbuf0, cbuf2);
        step(i + 1, cbuf1, cbuf0);
        step(i + 2, cbuf2, cbuf1);
      }
    }
    // No load into LDS may outlive the workgroup.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    const uint32_t pinfo = (uint32_t)uniform((int)prev_info);
    if constexpr (kT24) {  // the three tiles of the last entry
      fold_close(0, lagt[0], pinfo);
      fold_close(1, lagt[1], pinfo);
      fold_close(2, lagt[2], pinfo);
      close24_if_last(pinfo);
    } else if constexpr (kHalf) {  // tiles 2,3 of the last entry
      if (pinfo & (1u << kHSplitBit)) fold_units(2, 3, lag2, lag3, pinfo, std::true_type());
      else fold_units(2, 3, lag2, lag3, pinfo, std::false_type());
      close_units(2, 3, pinfo);
    } else {  // tiles 2,3 of the last entry
      fold_close(2, lag2, pinfo);
      fold_close(3, lag3, pinfo);
      close_if_last(2, 3, pinfo);
    }
  }

  // ---- first-token rule for NaN scores -------------------------------------------
  // The reference keeps (NaN, f) when the first valid token f of a document
  // scores NaN (`arg == 0 || s > mx`, kernels_forward.jl:49-52); the fold
  // skipped that NaN like any other.  score(f) can be NaN only when the query
  // token or f's feature row holds an Inf or NaN (plan flag kPlanNfBit), so
  // only those (query, document) pairs are examined, after the loop, on the
  // staged results: score(f) is recomputed by the same MFMAs (row f as every
  // row of the A operand), and where it is NaN the token's tape becomes f
  // and the document's score NaN.  Finite features never enter this branch.
  if constexpr (kT24) {
    // The same rule with the packed tiles: tile t's lanes hold tokens of
    // queries t24_query(t); a tile is examined when one of its valid tokens
    // or the document's first row is not finite.
    uint32_t tnf = 0u;  // bit t: some valid token of tile t is not finite
#pragma unroll
    for (int t = 0; t < 3; ++t) {
      bool nf = false;
#pragma unroll
      for (int kb = 0; kb < kIbNkb; ++kb) nf |= frag_nonfinite<Op>(qf[t][kb]);
      nf = ((uint32_t)nf | lane_xor32((uint32_t)nf, h)) != 0u;
      tnf |= __ballot(nf & t24_valid(t)) != 0ull ? (1u << t) : 0u;
    }
    if (tnf != 0u || uniform(any_nf) != 0) {
      for (int jj = 0; jj < ndoc; ++jj) {
        const int df = uniform(doc_first[jj]);
        if (df < 0) continue;  // no valid token: the document never closed
        const int f = df & ~(1 << kPlanNfBit);
        const bool dnf = ((df >> kPlanNfBit) & 1) != 0;
        const int rowoff = ((kPacked ? doc_row0[jj] : jj * Td) + f) * kIbRowBytes;
        Frag a[kIbNkb];
#pragma unroll
        for (int kb = 0; kb < kIbNkb; ++kb) a[kb] = Op::load(rd, rowoff + kb * 32 + h * 16);
#pragma unroll
        for (int t = 0; t < 3; ++t) {
          if (!dnf && !((tnf >> t) & 1u)) continue;
          Acc acc = Acc{};
#pragma unroll
          for (int kb = 0; kb < kIbNkb; ++kb) acc = Op::mma(a[kb], qf[t][kb], acc);
          const float s0 = acc[0];  // every row is f: <f, this lane's query token>
          const bool fix = t24_valid(t) && is_nan_bits(s0);
          if (__ballot(fix) == 0ull) continue;
          if (kTape && (fix & (h == 0))) res_tape[wave][t24_query(t)][jj][t24_token(t)] = (int16_t)(f + 1);
          const int qa = (32 * t) / 24;  // the tile's first query; the other is qa + 1
          const bool fa = __ballot(fix && t24_query(t) == qa) != 0ull;
          const bool fb = __ballot(fix && t24_query(t) == qa + 1) != 0ull;
          if (lane == 0 && fa) res_score[wave][qa][jj] = __builtin_bit_cast(float, 0x7fc00000u);
          if (lane == 0 && fb) res_score[wave][qa + 1][jj] = __builtin_bit_cast(float, 0x7fc00000u);
        }
      }
    }
  } else {
    uint32_t qnf = 0u;  // bit q: some valid token of query q is not finite
#pragma unroll
    for (int q = 0; q < kIbQpw; ++q) {
      bool nf = false;
#pragma unroll
      for (int kb = 0; kb < kIbNkb; ++kb) nf |= frag_nonfinite<Op>(qf[q][kb]);
      nf = ((uint32_t)nf | lane_xor32((uint32_t)nf, h)) != 0u;
      qnf |= __ballot(nf & token_valid(q)) != 0ull ? (1u << q) : 0u;
    }
    if (qnf != 0u || uniform(any_nf) != 0) {
      for (int jj = 0; jj < ndoc; ++jj) {
        const int df = uniform(doc_first[jj]);
        if (df < 0) continue;  // no valid token: the document never closed
        const int f = df & ~(1 << kPlanNfBit);
        const bool dnf = ((df >> kPlanNfBit) & 1) != 0;
        const int rowoff = ((kPacked ? doc_row0[jj] : jj * Td) + f) * kIbRowBytes;
        Frag a[kIbNkb];
#pragma unroll
        for (int kb = 0; kb < kIbNkb; ++kb) a[kb] = Op::load(rd, rowoff + kb * 32 + h * 16);
#pragma unroll
        for (int q = 0; q < kIbQpw; ++q) {
          if (!dnf && !((qnf >> q) & 1u)) continue;
          Acc acc = Acc{};
#pragma unroll
          for (int kb = 0; kb < kIbNkb; ++kb) acc = Op::mma(a[kb], qf[q][kb], acc);
          const float s0 = acc[0];  // every row is f: <f, q token lane%32>
          const bool fix = token_valid(q) && is_nan_bits(s0);
          if (__ballot(fix) == 0ull) continue;
          if (kTape && (fix & (h == 0))) res_tape[wave][q][jj][r32] = (int16_t)(f + 1);
          if (lane == 0) res_score[wave][q][jj] = __builtin_bit_cast(float, 0x7fc00000u);
        }
      }
    }
  }
  __syncthreads();  // results of every wave staged

  // ---- write the block's tape and scores (coalesced) ------------------------------
  // Query row qi's tape for documents j0..j1-1 is ndoc runs of its qtn tokens
  // (one contiguous run of ndoc * Tq int32 when a row is a whole query); its
  // scores are ndoc contiguous floats in A.S (A.St, unnormalised, for tiles).
#pragma unroll
  for (int q = 0; q < kIbQpw; ++q) {
    if (!qlive[q]) continue;
    const int64_t p0 = (int64_t)qrow[q] * A.Bd + j0;
    if (kTape && A.args) {
      int32_t* const out = A.args + p0 * Tq + qt0[q];
      const int tn = qtn[q], n = ndoc * tn;
      const int16_t* const src = &res_tape[wave][q][0][0];
      if (tn == kTile && Tq == kTile && ((reinterpret_cast<uintptr_t>(out) & 15u) == 0u)) {
        // whole 32-token query rows (16-byte aligned output): the staged tape
        // and the output run are both one contiguous run of n entries (n a
        // multiple of 32), 4 per lane per pass: an 8-byte LDS read and a
        // 16-byte store
        for (int e = lane * 4; e < n; e += 256) {
          const uint2 w = *reinterpret_cast<const uint2*>(src + e);
          const i32x4 v = {(int32_t)(int16_t)(w.x & 0xffffu), (int32_t)(int16_t)(w.x >> 16),
                           (int32_t)(int16_t)(w.y & 0xffffu), (int32_t)(int16_t)(w.y >> 16)};
          *reinterpret_cast<i32x4*>(out + e) = v;
        }
      } else {
        // e / tn as (e * ceil(2^32 / tn)) >> 32, exact for e < 2^27 (the
        // factor is 2^32 itself for tn = 1, hence 64 bits)
        const uint64_t mg = ((uint64_t)1 << 32) / (uint64_t)tn + (((uint64_t)1 << 32) % (uint64_t)tn != 0);
#pragma unroll 4
        for (int e = lane; e < n; e += 64) {
          const int jj = (int)(((uint64_t)(uint32_t)e * mg) >> 32), t = e - jj * tn;
          out[jj * Tq + t] = src[jj * kTile + t];
        }
      }
    }
    if (ntq > 1) {
      if (lane < ndoc) A.St[(int64_t)qi[q] * A.Bd + j0 + lane] = res_score[wave][q][lane];
      continue;
    }
    // normalize epilogue: 1 / max(valid query tokens, 1) in fp32 (normalize.jl:4-10)
    float inv = 1.0f;
    if (A.norm) {
      float nf;
      if constexpr (kT24) {
        int c = 0;
#pragma unroll
        for (int t = 0; t < 3; ++t)
          c += __builtin_popcountll(__ballot(h == 0 && t24_query(t) == q && t24_valid(t)));
        nf = (float)c;
      } else {
        nf = (float)__builtin_popcountll(__ballot(h == 0 && token_valid(q)));
      }
      inv = 1.0f / (nf > 1.0f ? nf : 1.0f);
    }
    if (lane < ndoc) {
      const float sc = res_score[wave][q][lane];
      A.S[p0 + lane] = A.norm ? sc * inv : sc;
    }
  }
}

// S[i, j] = sum over tiles tb (in order) of St[i * ntq + tb, j], times
// 1 / max(valid tokens of query i, 1) when normalising (the kernel's epilogue
// rule, over all Tq tokens).  Grid (document blocks, query stride).
__global__ void __launch_bounds__(256) inbatch_tile_sum_kernel(const float* St, int ntq, int Bq,
                                                               int Bd, const uint8_t* qm, int Tq,
                                                               int norm, float* S) {
  __shared__ int cnt;
  for (int i = blockIdx.y; i < Bq; i += gridDim.y) {
    float inv = 1.0f;
    if (norm) {
      if (threadIdx.x == 0) cnt = 0;
      __syncthreads();
      int c = 0;
      for (int t = threadIdx.x; t < Tq; t += 256) c += qm ? (qm[(int64_t)i * Tq + t] != 0) : 1;
      atomicAdd(&cnt, c);
      __syncthreads();
      const float nf = (float)cnt;
      inv = 1.0f / (nf > 1.0f ? nf : 1.0f);
      __syncthreads();  // cnt read by every thread before the next query resets it
    }
    for (int j = blockIdx.x * 256 + threadIdx.x; j < Bd; j += gridDim.x * 256) {
      float s = 0.0f;
      for (int tb = 0; tb < ntq; ++tb) s += St[((int64_t)i * ntq + tb) * Bd + j];
      S[(int64_t)i * Bd + j] = norm ? s * inv : s;
    }
  }
}

hipError_t launch_inbatch_mfma(int dtype_bf16, const InBatchArgs& args_in, hipStream_t stream) {
  InBatchArgs A = args_in;
  A.ntq = A.Tq > kTile ? (A.Tq + kTile - 1) / kTile : 1;
  A.nqb = (int)(((int64_t)A.Bq * A.ntq + kIbQueries - 1) / kIbQueries);
  // Documents per block: the grid should be a whole number of rounds of the
  // resident block slots (kIbBlocksPerCu per CU) -- a last round that
  // fills only part of the GPU idles the rest -- as few blocks as that
  // allows (each block pays one set-up), and the block's chunk list within
  // kIbMaxChunkMasks.
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus < 1)
    cus = 256;
  const int64_t slots = (int64_t)cus * kIbBlocksPerCu;
  const int nch = A.Td > 0 ? (A.Td + kTile - 1) / kTile : 1;
  const int db_cap = std::min(kIbMaxDocs, std::max(1, kIbMaxChunkMasks / nch));
  // With the balanced split (blocks of equal work) one round is enough; the
  // uniform split keeps two, so the dispatcher can even out lengths.
  const int balance = A.Bd <= kIbBalanceMaxDocs ? 1 : 0;
  // The document ranges split Bd evenly (fractional bounds: ranges of
  // floor or ceil of Bd/ndb documents), so ndb can be exactly what fills the
  // rounds: nqb * ndb <= rounds * slots.
  int64_t ndb = (A.Bd + db_cap - 1) / db_cap;  // (fallback: the smallest grid that fits)
  for (int64_t rounds = balance ? 1 : 2; rounds <= 64; ++rounds) {
    const int64_t ndb_want = std::max<int64_t>(1, rounds * slots / A.nqb);
    if (ndb_want >= A.Bd) {
      ndb = std::max<int64_t>(1, A.Bd);
      break;
    }
    if ((A.Bd + ndb_want - 1) / ndb_want <= db_cap) {
      ndb = ndb_want;
      break;
    }
  }
  A.ndb = (int)ndb;
  A.db = (int)((A.Bd + ndb - 1) / ndb);  // most documents of a range
  A.dbcap = db_cap;
  A.balance = balance;
  A.tilt = balance && kIbBlocksPerCu == 2 && (int64_t)A.nqb * ndb == slots && ndb % 2 == 0 ? 1 : 0;

  // Plan workspace: chunk masks, chunk counts, first tokens.
  auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
  const size_t mask_bytes = al((size_t)A.Bd * nch * 4), vec_bytes = al((size_t)A.Bd * 4);
  const size_t tile_bytes = A.ntq > 1 ? al((size_t)A.Bq * A.ntq * A.Bd * 4) : 0;
  void* ws = nullptr;
  hipError_t e = workspace_alloc(&ws, mask_bytes + 2 * vec_bytes + tile_bytes, stream);
  if (e != hipSuccess) return e;
  char* w = static_cast<char*>(ws);
  uint32_t* cmask = reinterpret_cast<uint32_t*>(w);
  int32_t* dcount = reinterpret_cast<int32_t*>(w + mask_bytes);
  int32_t* dfirst = reinterpret_cast<int32_t*>(w + mask_bytes + vec_bytes);
  A.St = A.ntq > 1 ? reinterpret_cast<float*>(w + mask_bytes + 2 * vec_bytes) : nullptr;
  A.cmask = cmask;
  A.dcount = dcount;
  A.dfirst = dfirst;
  const int rb = A.dim * 2;
  if (A.cu)
    hipLaunchKernelGGL(packed_plan_kernel, dim3((unsigned)((A.Bd + 3) / 4)), dim3(256), 0, stream,
                       A.cu, A.D, dtype_bf16, rb, A.ntok, A.Bd, A.Td, nch, cmask, dcount, dfirst);
  else
    hipLaunchKernelGGL(inbatch_plan_kernel, dim3((unsigned)((A.Bd + 3) / 4)), dim3(256), 0, stream,
                       A.dm, A.D, dtype_bf16, rb, A.Bd, A.Td, nch, cmask, dcount, dfirst);
  e = hipGetLastError();
  if (e == hipSuccess) {
    const dim3 grid((unsigned)(A.nqb * ((A.ndb + kXcds - 1) / kXcds) * kXcds)), block(64 * kIbWaves);
    // Tq == 24: four queries fill three tiles (kT24)
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, block, 0, stream, A); };
    // args null: the scores-only kernels (running maximum, no argmax)
    auto by_nkb = [&](auto op, auto packed, auto t24, auto tape) {
      typedef decltype(op) O;
      constexpr bool P = decltype(packed)::value, T = decltype(t24)::value;
      constexpr bool K = decltype(tape)::value;
      switch (A.dim / 16) {
        case 2: go(inbatch_mfma<O, P, T, 2, K>); break;
        case 4: go(inbatch_mfma<O, P, T, 4, K>); break;
        case 6: go(inbatch_mfma<O, P, T, 6, K>); break;
        default: go(inbatch_mfma<O, P, T, 8, K>); break;
      }
    };
    auto by_tape = [&](auto op, auto packed, auto t24) {
      if (A.args) by_nkb(op, packed, t24, std::true_type());
      else by_nkb(op, packed, t24, std::false_type());
    };
    auto by_t24 = [&](auto op, auto packed) {
      if (A.Tq == 24) by_tape(op, packed, std::true_type());
      else by_tape(op, packed, std::false_type());
    };
    auto by_packed = [&](auto op) {
      if (A.cu) by_t24(op, std::true_type());
      else by_t24(op, std::false_type());
    };
    if (dtype_bf16) by_packed(OpBF16());
    else by_packed(OpF16());
    if (A.ntq > 1)
      hipLaunchKernelGGL(inbatch_tile_sum_kernel,
                         dim3((unsigned)std::min((A.Bd + 255) / 256, 64), (unsigned)std::min(A.Bq, 65535)),
                         dim3(256), 0, stream, A.St, A.ntq, A.Bq, A.Bd, A.qm, A.Tq, A.norm, A.S);
    e = hipGetLastError();
  }
  const hipError_t ef = workspace_free(ws, stream);
  return e != hipSuccess ? e : ef;
}

// A block's documents span one buffer resource: ndoc * Td * dim * 2 bytes <=
// kIbMaxChunkMasks * 32 * 256 = 8 MB.  Tape entries are staged as int16.
bool inbatch_mfma_supported(int64_t dim, int64_t Tq, int64_t Td, const void* Q, const void* D) {
  const bool al = ((reinterpret_cast<uintptr_t>(Q) | reinterpret_cast<uintptr_t>(D)) & 15u) == 0;
  const bool dim_ok = dim == 32 || dim == 64 || dim == 96 || dim == 128;
  return dim_ok && Tq >= 1 && Tq <= kIbMaxTq && Td >= 0 && (Td + kTile - 1) / kTile <= kIbMaxChunks && al;
}

}  // namespace fms
