// fms_inbatch.hip -- InBatch() MaxSim as an MFMA-bound tiled contraction.
//
// S[j, i] = sum_t max_u <Q_i[t], D_j[u]> for all (i, j) of Bq queries x Bd
// documents (the reference materialises D'Q chunks and then runs an atomic
// argmax-accumulate, forward_layouts.jl:202-225; here nothing but S and the
// tape leaves the chip).
//
// Workgroup = 4 waves (one per SIMD), two workgroups per CU, 16 queries x a
// block of DB documents.
//   * every wave keeps 4 query tiles (32 tokens x d=128 fp16/bf16) in
//     registers for the whole workgroup lifetime, so each LDS fragment read
//     feeds 4 MFMAs;
//   * the workgroup streams its documents in 32-token chunks: each chunk
//     (8 KB) is fetched ONCE from L2/HBM (two coalesced 16-byte loads per
//     thread) and stored to one of two LDS buffers with 272-byte rows, so the
//     MFMA-layout ds_read_b128s of consecutive lanes hit distinct banks;
//   * masked rows (dmask = 0, and rows past Td in a document's last chunk)
//     are replaced AT LOAD TIME by a copy of the document's first valid
//     token f.  A copy scores exactly what f scores, so the maximum is
//     unchanged, and with first-occurrence tie breaking a copy can only win
//     where f ties it: a winning copy maps back to f when the document is
//     closed.  The fold therefore needs no row masks at all;
//   * software pipeline: chunk c+3 is requested while chunk c is multiplied
//     (chunks c+2 and c+3 in flight), chunk c+1 moves register -> LDS at the
//     start of step c, and one barrier per step publishes it.  Loads are
//     unconditional (the stream position stops at the last chunk, so loads
//     issued past the end re-read it) and the loop has no global stores, so
//     the compiler's in-order vmcnt accounting waits for exactly one chunk;
//   * per chunk and wave: 8 LDS fragment reads feed 4 x 8 MFMA 32x32x16
//     issued k-block by k-block across the 4 query tiles, i.e. 4 independent
//     accumulation chains (a dependent 32x32x16 MFMA issues at about half the
//     rate of an independent one), then each tile's running max/argmax
//     update (fold_tree); the two workgroups on a CU have independent
//     barriers, so one's folds overlap the other's MFMAs on each SIMD;
//   * the document close (merge of the wave halves, score) uses v_permlane32
//     and DPP, not LDS shuffles, and no branches;
//   * per-document tape (int16, Td <= 2048) / score go to LDS and leave in
//     one coalesced pass at the end of the block.
// Documents per block are chosen so the grid is a whole number (>= 2) of
// rounds of the resident block slots.  Block -> (query block, document
// block) is XCD-aware: consecutive block ids go to different XCDs, so each
// XCD's blocks share one slice of documents (its L2) and iterate over all
// query blocks.
#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>
#include <stdint.h>

#include "fms_device.hpp"
#include "fms_inbatch.hpp"

namespace fms {

namespace {

constexpr int kIbWaves = 4;
constexpr int kIbQpw = 4;                          // query tiles per wave
constexpr int kIbQueries = kIbWaves * kIbQpw;      // queries per block
constexpr int kIbNkb = 8;                          // dim == 128
constexpr int kIbRowBytes = kIbNkb * 32;           // 256 B per token
constexpr int kIbLdsRow = kIbRowBytes + 16;        // padded LDS row (272 B)
constexpr int kIbLdsChunk = kTile * kIbLdsRow;     // one LDS chunk buffer
constexpr int kIbUnits = kTile * kIbRowBytes / 16 / (64 * kIbWaves);  // 16-byte units per thread
constexpr int kXcds = 8;
constexpr int kIbMaxChunkMasks = 512;            // documents x chunks per block
constexpr int kIbMaxDocs = 24;                   // documents per block
constexpr int kIbMaxChunks = 64;                 // chunks per document (Td <= 2048)
constexpr int kIbBlocksPerCu = 2;                // occupancy the launch bounds ask for
// List entry: chunk (6 bits) | document in block (5) | last chunk of its
// document (1) | first valid token + 1 (20).
constexpr int kInfoDocShift = 6, kInfoLastBit = 11, kInfoFirstShift = 12;
constexpr uint32_t kInfoDocMask = 31u;

// LDS byte offset of 16-byte unit `u` (0..15) of chunk row `row` (0..31).
// Rows are padded to 272 bytes: the MFMA-layout reads of consecutive lanes
// (consecutive rows, same unit) start 68 banks apart, i.e. on distinct
// 16-byte bank groups for 8 (32-bank) or 16 (64-bank) lanes per pass, the
// staging writes of 16 lanes cover one contiguous row, and the 8 fragment
// reads of a lane are one base address plus immediate offsets.
__device__ __forceinline__ int lds_off(int row, int u) { return row * kIbLdsRow + (u << 4); }

}  // namespace

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

template <class Op>
__global__ void __launch_bounds__(64 * kIbWaves, kIbBlocksPerCu) inbatch_mfma(const InBatchArgs A) {
  typedef typename Op::Acc Acc;
  typedef typename Op::Frag Frag;
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][kIbLdsChunk];
  __shared__ uint32_t chunk_mask[kIbMaxChunkMasks];  // valid rows per (doc, chunk)
  __shared__ int32_t doc_first[kIbMaxDocs];          // first valid token, -1 = none
  __shared__ uint32_t lst_mask[kIbMaxChunkMasks];    // compacted chunk list
  __shared__ uint32_t lst_info[kIbMaxChunkMasks];
  __shared__ int lst_count;
  __shared__ int16_t res_tape[kIbWaves][kIbQpw][kIbMaxDocs][kTile];  // Td <= 2048
  __shared__ float res_score[kIbWaves][kIbQpw][kIbMaxDocs];

  const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
  const int r32 = lane & 31, h = lane >> 5;

  // XCD-aware block mapping (blocks are dealt round-robin to the 8 XCDs).
  const int nqb = A.nqb, ndb = A.ndb;
  const int id = blockIdx.x;
  int qb, db;
  if (ndb % kXcds == 0) {
    const int per = ndb / kXcds, xcd = id % kXcds, k = id / kXcds;
    db = xcd * per + k % per;
    qb = k / per;
  } else {
    db = id % ndb;
    qb = id / ndb;
  }
  if (qb >= nqb) return;
  const int j0 = db * A.db, j1 = (j0 + A.db < A.Bd) ? j0 + A.db : A.Bd;
  const int ndoc = j1 - j0;
  const int Tq = A.Tq, Td = A.Td;
  const int nch = Td > 0 ? (Td + kTile - 1) / kTile : 1;  // <= 64
  const int nall = ndoc * nch;

  // ---- row validity of this block's chunks (one ballot each) ----------------
  for (int c = wave; c < nall; c += kIbWaves) {
    const int j = uniform(j0 + c / nch), ch = uniform(c % nch);
    uint32_t mb = 1u;
    if (A.dm) mb = buf_load1(make_rsrc(A.dm + (int64_t)j * Td, (uint32_t)Td), ch * kTile + r32);
    const uint32_t m = (uint32_t)__ballot((ch * kTile + r32 < Td) && mb != 0u);
    if (lane == 0) chunk_mask[c] = m;
  }

  // ---- resident query tiles --------------------------------------------------
  Frag qf[kIbQpw][kIbNkb];
  bool tvalid[kIbQpw];
  int qi[kIbQpw];
#pragma unroll
  for (int q = 0; q < kIbQpw; ++q) {
    qi[q] = qb * kIbQueries + wave * kIbQpw + q;
    const bool live = qi[q] < A.Bq;
    const int iq = live ? qi[q] : 0;
    const rsrc_t rq = make_rsrc(A.Q + (int64_t)iq * Tq * kIbRowBytes,
                                live ? (uint32_t)Tq * kIbRowBytes : 0u);
    const int base = r32 * kIbRowBytes + h * 16;
#pragma unroll
    for (int kb = 0; kb < kIbNkb; ++kb) qf[q][kb] = Op::load(rq, base + kb * 32);
    uint32_t mb = 1u;
    if (A.qm) mb = buf_load1(make_rsrc(A.qm + (int64_t)iq * Tq, live ? (uint32_t)Tq : 0u), r32);
    tvalid[q] = live && r32 < Tq && mb != 0u;
  }

  __syncthreads();  // chunk_mask complete
  // ---- first valid token of each document; defaults of the results ----------
  for (int jj = wave; jj < ndoc; jj += kIbWaves) {
    const uint32_t m = lane < nch ? chunk_mask[jj * nch + lane] : 0u;
    const uint64_t nz = __ballot(m != 0u);
    int f = -1;
    if (nz != 0u) {
      const int k = uniform(__builtin_ctzll(nz));
      f = k * kTile + __builtin_ctz((uint32_t)uniform((int)chunk_mask[jj * nch + k]));
    }
    if (lane == 0) doc_first[jj] = f;
  }
  // A document without a valid token never closes: score 0, tape 0.
  for (int e = tid; e < kIbWaves * kIbQpw * kIbMaxDocs * kTile; e += 64 * kIbWaves)
    (&res_tape[0][0][0][0])[e] = 0;
  for (int e = tid; e < kIbWaves * kIbQpw * kIbMaxDocs; e += 64 * kIbWaves)
    (&res_score[0][0][0])[e] = 0.0f;
  __syncthreads();  // doc_first complete

  // ---- compacted chunk list ------------------------------------------------------
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
        lst_info[pos] = (uint32_t)(ch | (jj << kInfoDocShift) |
                                   ((doc_first[jj] + 1) << kInfoFirstShift));
      }
      base += __builtin_popcountll(bal);
    }
    if (lane == 0) lst_count = base;
  }
  __syncthreads();
  const int nsteps = uniform(lst_count);
  bool last[kIbMaxChunkMasks / (64 * kIbWaves)];
#pragma unroll
  for (int k = 0; k < kIbMaxChunkMasks / (64 * kIbWaves); ++k) {
    const int i = tid + k * 64 * kIbWaves;
    last[k] = i < nsteps && (i + 1 == nsteps ||
                             ((lst_info[i + 1] >> kInfoDocShift) & kInfoDocMask) !=
                                 ((lst_info[i] >> kInfoDocShift) & kInfoDocMask));
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kIbMaxChunkMasks / (64 * kIbWaves); ++k)
    if (last[k]) lst_info[tid + k * 64 * kIbWaves] |= 1u << kInfoLastBit;
  __syncthreads();

  // ---- chunk stream -------------------------------------------------------------
  // One buffer resource spans the block's documents [j0, j1) (contiguous in
  // D).  Thread tid moves kIbUnits 16-byte units of every chunk: unit
  // tid + i*256 is row (tid>>4) + 16*i, column tid&15; a masked row loads
  // the document's first valid token instead.  The stream position stops at
  // the last list entry, so loads issued past the end re-read it.
  const rsrc_t rd = make_rsrc(A.D + (int64_t)j0 * Td * kIbRowBytes, (uint32_t)(ndoc * Td * kIbRowBytes));
  const int urow = tid >> 4, ucol = tid & 15;
  typedef u32x4 Stage[kIbUnits];
  int ld_i = 0;  // next list entry to request
  auto chunk_load = [&](Stage& g, uint32_t m, uint32_t info) {
    const int ch = info & 63u, jj = (info >> kInfoDocShift) & kInfoDocMask;
    const int f = (int)(info >> kInfoFirstShift) - 1;
    const int fsrc = f < 0 ? 0 : f;  // (never: listed chunks have a valid row)
#pragma unroll
    for (int i = 0; i < kIbUnits; ++i) {
      const int row = urow + 16 * i;
      const int src = ((m >> row) & 1u) ? ch * kTile + row : fsrc;
      g[i] = buf_load16(rd, (jj * Td + src) * kIbRowBytes + ucol * 16);
    }
    if (ld_i + 1 < nsteps) ++ld_i;
  };
  auto lds_store = [&](int i, const Stage& g) {
#pragma unroll
    for (int u = 0; u < kIbUnits; ++u)
      *reinterpret_cast<u32x4*>(&lds[i & 1][lds_off(urow + 16 * u, ucol)]) = g[u];
  };

  float mx[kIbQpw];
  int slot[kIbQpw];
#pragma unroll
  for (int q = 0; q < kIbQpw; ++q) { mx[q] = -INFINITY; slot[q] = -1; }

  // Close query q's document jj: merge the wave halves, map a winning
  // substituted row back to the first valid token f, reduce the score,
  // stage tape and score in LDS, reset the running max.
  auto close = [&](int q, int jj, int f) {
    int tok = slot_to_token(slot[q], h);
    float m = mx[q];
    merge_halves(m, tok, h);
    // Branch-free: the mask word is read for every lane (t0 is always a
    // valid token index of the document).
    const int t0 = tok > 0 ? tok - 1 : 0;
    const uint32_t mw = chunk_mask[jj * nch + (t0 >> 5)];
    const bool real = (tok > 0) & (((mw >> (t0 & 31)) & 1u) != 0u);
    tok = real ? tok : f + 1;
    const float part = (tvalid[q] & (tok != 0)) ? m : 0.0f;
    const float score = half_sum(part);
    if (h == 0) res_tape[wave][q][jj][r32] = (int16_t)(tvalid[q] ? tok : 0);
    if (lane == 0) res_score[wave][q][jj] = score;
    mx[q] = -INFINITY;
    slot[q] = -1;
  };

  // One step: entry i+1 register -> LDS, refill that register stage with
  // entry i+3, multiply entry i (LDS buffer i%2) query by query with the
  // previous query's fold interleaved, close the document after its last
  // entry, read the list info for the next step, publish.
  uint32_t ld_m = 0u, ld_info = 0u;  // list entry ld_i, read one step ahead
  uint32_t cur_info = 0u;            // list entry i
  auto step = [&](int i, Stage& g_next) {
    lds_store(i + 1, g_next);
    chunk_load(g_next, (uint32_t)uniform((int)ld_m), (uint32_t)uniform((int)ld_info));
    // List entries for the next step, read now so the LDS latency hides
    // behind this step's MFMAs instead of stalling before the barrier.
    ld_m = lst_mask[ld_i];
    ld_info = lst_info[ld_i];
    const uint32_t next_info = lst_info[i + 1 < nsteps ? i + 1 : i];
    const uint32_t info = (uint32_t)uniform((int)cur_info);
    const int ch = info & 63u;
    Frag a[kIbNkb];
#pragma unroll
    for (int kb = 0; kb < kIbNkb; ++kb)
      a[kb] = *reinterpret_cast<const Frag*>(&lds[i & 1][lds_off(r32, 2 * kb + h)]);
    Acc acc[kIbQpw];
    // The query tiles' accumulations interleave k-block by k-block:
    // kIbQpw independent MFMA chains, so no MFMA waits for the result of
    // the one issued just before it (a dependent 32x32x16 MFMA issues at
    // about half the rate of independent ones).
#pragma unroll
    for (int q = 0; q < kIbQpw; ++q) acc[q] = Acc{};
#pragma unroll
    for (int kb = 0; kb < kIbNkb; ++kb)
#pragma unroll
      for (int q = 0; q < kIbQpw; ++q) acc[q] = Op::mma(a[kb], qf[q][kb], acc[q]);
#pragma unroll
    for (int q = 0; q < kIbQpw; ++q) {
      float s[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = acc[q][r];
      fold_tree(s, ch * 16, mx[q], slot[q]);
    }
    if (info & (1u << kInfoLastBit)) {
      const int jj = (info >> kInfoDocShift) & kInfoDocMask;
      const int f = (int)(info >> kInfoFirstShift) - 1;
#pragma unroll
      for (int q = 0; q < kIbQpw; ++q) close(q, jj, f);
    }
    cur_info = next_info;
    lds_barrier();
  };

  if (nsteps > 0) {
    Stage g0, g1;
    chunk_load(g0, lst_mask[0], lst_info[0]);           // entry 0
    chunk_load(g1, lst_mask[ld_i], lst_info[ld_i]);     // entry 1
    lds_store(0, g0);
    chunk_load(g0, lst_mask[ld_i], lst_info[ld_i]);     // entry 2
    ld_m = lst_mask[ld_i];
    ld_info = lst_info[ld_i];
    cur_info = lst_info[0];
    lds_barrier();
    int i = 0;
    for (; i + 1 < nsteps; i += 2) {  // both steps unconditional: exact vmcnt waits
      step(i, g1);      // g1 held entry i+1, now requests i+3
      step(i + 1, g0);  // g0 held entry i+2, now requests i+4
    }
    if (i < nsteps) step(i, g1);
  }
  __syncthreads();  // results of every wave staged

  // ---- write the block's tape and scores (coalesced) ------------------------------
#pragma unroll
  for (int q = 0; q < kIbQpw; ++q) {
    if (qi[q] >= A.Bq) continue;
    for (int jj = 0; jj < ndoc; ++jj) {
      const int64_t p = (int64_t)qi[q] * A.Bd + (j0 + jj);
      if (A.args && h == 0 && r32 < Tq) A.args[p * Tq + r32] = res_tape[wave][q][jj][r32];
      if (lane == 0) A.S[p] = res_score[wave][q][jj];
    }
  }
}

hipError_t launch_inbatch_mfma(int dtype_bf16, const InBatchArgs& args_in, hipStream_t stream) {
  InBatchArgs A = args_in;
  A.nqb = (A.Bq + kIbQueries - 1) / kIbQueries;
  // Documents per block: the grid should be a whole number of rounds of the
  // resident block slots (kIbBlocksPerCu per CU) -- a last round that
  // fills only part of the GPU idles the rest -- with at least two rounds
  // for balance, as few blocks as that allows (each block pays one set-up),
  // and the block's chunk list within kIbMaxChunkMasks.
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus < 1)
    cus = 256;
  const int64_t slots = (int64_t)cus * kIbBlocksPerCu;
  const int nch = A.Td > 0 ? (A.Td + kTile - 1) / kTile : 1;
  const int db_cap = std::min(kIbMaxDocs, std::max(1, kIbMaxChunkMasks / nch));
  int db = 1;
  for (int64_t rounds = 2; rounds <= 64; ++rounds) {
    const int64_t ndb_want = (rounds * slots + A.nqb - 1) / A.nqb;
    db = (int)std::max<int64_t>(1, (A.Bd + ndb_want - 1) / ndb_want);
    if (db <= db_cap) break;
  }
  db = std::min(db, db_cap);
  A.db = db;
  A.ndb = (A.Bd + db - 1) / db;
  const dim3 grid((unsigned)(A.nqb * A.ndb)), block(64 * kIbWaves);
  if (dtype_bf16)
    hipLaunchKernelGGL((inbatch_mfma<OpBF16>), grid, block, 0, stream, A);
  else
    hipLaunchKernelGGL((inbatch_mfma<OpF16>), grid, block, 0, stream, A);
  return hipGetLastError();
}

// A block's documents span one buffer resource: ndoc * Td * 256 bytes <=
// kIbMaxChunkMasks * 32 * 256 = 4 MB.  Tape entries are staged as int16.
bool inbatch_mfma_supported(int64_t dim, int64_t Tq, int64_t Td, const void* Q, const void* D) {
  const bool al = ((reinterpret_cast<uintptr_t>(Q) | reinterpret_cast<uintptr_t>(D)) & 15u) == 0;
  return dim == kIbNkb * 16 && Tq >= 1 && Tq <= kTile && Td >= 0 &&
         (Td + kTile - 1) / kTile <= kIbMaxChunks && al;
}

}  // namespace fms
