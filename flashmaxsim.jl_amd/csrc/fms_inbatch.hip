// fms_inbatch.hip -- InBatch() MaxSim as an MFMA-bound tiled contraction.
//
// S[j, i] = sum_t max_u <Q_i[t], D_j[u]> for all (i, j) of Bq queries x Bd
// documents (the reference materialises D'Q chunks and then runs an atomic
// argmax-accumulate, forward_layouts.jl:202-225; here nothing but S and the
// tape leaves the chip).
//
// Workgroup = 4 waves (one per SIMD), two workgroups per CU, 16 queries x a
// block of DB documents.
//   * every wave keeps QPW = 4 query tiles (32 tokens x d=128 fp16/bf16) in
//     registers for the whole workgroup lifetime, so each LDS fragment read
//     feeds 4 MFMAs;
//   * the workgroup streams its documents in 32-token chunks: each chunk
//     (8 KB) is fetched ONCE from L2/HBM (one coalesced 16-byte load per
//     thread) and stored to one of two LDS buffers, XOR-swizzled so that the
//     MFMA-layout ds_read_b128s of 8 consecutive lanes hit distinct banks;
//   * software pipeline: chunk c+3 is requested while chunk c is multiplied
//     (chunks c+2 and c+3 in flight), chunk c+1 moves register -> LDS at the
//     start of step c, and one barrier per step publishes it.  Loads are
//     unconditional (past the end a zero-size buffer resource returns zeros
//     without touching memory) and the loop has no global stores, so the
//     compiler's in-order vmcnt accounting waits for exactly one chunk;
//   * per chunk and wave: 8 LDS fragment reads feed 4 x 8 MFMA 32x32x16,
//     then the per-lane running max/argmax update (the scans' epilogue,
//     ~0.75x the MFMA time); the two workgroups on a CU have independent
//     barriers, so one's epilogue co-executes with the other's MFMAs on each
//     SIMD; fully masked chunks skip both;
//   * per-document tape / score go to LDS and leave in one coalesced pass at
//     the end of the block.
// Block -> (query block, document block) is XCD-aware: consecutive block ids
// go to different XCDs, so each XCD's blocks share one slice of documents
// (<= 4 MB, its L2) and iterate over all query blocks.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "fms_device.hpp"
#include "fms_inbatch.hpp"

namespace fms {

namespace {

constexpr int kIbWaves = 4;
constexpr int kIbQpw = 4;
constexpr int kIbNkb = 8;                          // dim == 128
constexpr int kIbRowBytes = kIbNkb * 32;           // 256 B per token
constexpr int kIbChunkBytes = kTile * kIbRowBytes;  // 8 KB per chunk
constexpr int kIbQueries = kIbWaves * kIbQpw;       // 16 queries per block
constexpr int kIbUnits = kIbChunkBytes / 16 / (64 * kIbWaves);  // 16-byte units per thread
constexpr int kXcds = 8;
constexpr int kIbMaxChunkMasks = 1024;           // DB * nch per block
constexpr int kIbMaxDocs = 16;                   // documents per block

// LDS byte offset of 16-byte unit `u` (0..15) of chunk row `row` (0..31).
__device__ __forceinline__ int lds_off(int row, int u) {
  return row * kIbRowBytes + ((u ^ (row & 7)) << 4);
}

}  // namespace

// Workgroup barrier that does not drain in-flight global loads: wait only
// for this wave's LDS writes (lgkmcnt(0)), then s_barrier.  __syncthreads()
// would add a release fence, i.e. s_waitcnt vmcnt(0), and stall on the
// chunk loads that are deliberately kept in flight across the barrier.  The
// empty asm statements stop the compiler from moving LDS accesses across.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt / expcnt unconstrained
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <class Op>
__global__ void __launch_bounds__(64 * kIbWaves, 2) inbatch_mfma(const InBatchArgs A) {
  typedef typename Op::Acc Acc;
  typedef typename Op::Frag Frag;
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][kIbChunkBytes];
  __shared__ uint32_t chunk_mask[kIbMaxChunkMasks];  // ballot of valid rows per (doc, chunk)
  __shared__ int32_t res_tape[kIbWaves][kIbQpw][kIbMaxDocs][kTile];
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
  const int Tq = A.Tq, Td = A.Td;
  const int nch = Td > 0 ? (Td + kTile - 1) / kTile : 1;
  const int nsteps = (j1 - j0) * nch;

  // ---- chunk validity masks of this block's documents (one ballot each) -----
  for (int c = wave; c < nsteps; c += kIbWaves) {
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

  // ---- chunk stream -------------------------------------------------------------
  // Thread tid moves kIbUnits 16-byte units of every chunk: unit
  // tid + i*256 is row (tid>>4) + 16*i, column tid&15.
  const int urow = tid >> 4, ucol = tid & 15;
  typedef u32x4 Stage[kIbUnits];
  auto chunk_load = [&](int c, Stage& g) {
    const bool in = c < nsteps;
    const int cc = in ? c : 0;
    const int j = uniform(j0 + cc / nch), ch = uniform(cc % nch);
    const rsrc_t rd = make_rsrc(A.D + (int64_t)j * Td * kIbRowBytes,
                                in ? (uint32_t)Td * kIbRowBytes : 0u);
#pragma unroll
    for (int i = 0; i < kIbUnits; ++i)
      g[i] = buf_load16(rd, (ch * kTile + urow + 16 * i) * kIbRowBytes + ucol * 16);
  };
  auto lds_store = [&](int c, const Stage& g) {
#pragma unroll
    for (int i = 0; i < kIbUnits; ++i)
      *reinterpret_cast<u32x4*>(&lds[c & 1][lds_off(urow + 16 * i, ucol)]) = g[i];
  };

  float mx[kIbQpw];
  int slot[kIbQpw];
#pragma unroll
  for (int q = 0; q < kIbQpw; ++q) { mx[q] = -INFINITY; slot[q] = -1; }

  // One step: chunk c+1 register -> LDS, refill that register stage with
  // chunk c+3, multiply chunk c (LDS buffer c%2) against the wave's query
  // tiles, fold it into the running max, close its document after its last
  // chunk.  Fully masked chunks skip the MFMAs and the fold.
  auto step = [&](int c, Stage& g_next) {
    lds_store(c + 1, g_next);
    chunk_load(c + 3, g_next);
    const int jj = uniform(c / nch), ch = uniform(c % nch);
    const uint32_t m32 = (uint32_t)uniform((int)chunk_mask[c]);
    if (m32 != 0u) {
      Acc acc[kIbQpw];
#pragma unroll
      for (int q = 0; q < kIbQpw; ++q) acc[q] = Acc{};
#pragma unroll
      for (int kb = 0; kb < kIbNkb; ++kb) {
        const Frag a = *reinterpret_cast<const Frag*>(&lds[c & 1][lds_off(r32, 2 * kb + h)]);
#pragma unroll
        for (int q = 0; q < kIbQpw; ++q) acc[q] = Op::mma(a, qf[q][kb], acc[q]);
      }
#pragma unroll
      for (int q = 0; q < kIbQpw; ++q) {
        float s[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = acc[q][r];
        if (m32 == 0xffffffffu) {
          running_max<true>(s, 0u, ch * 16, mx[q], slot[q]);
        } else {
          running_max<false>(s, m32 >> (4 * h), ch * 16, mx[q], slot[q]);
        }
      }
    }
    if (ch == nch - 1) {  // document done: stage tape + score in LDS
#pragma unroll
      for (int q = 0; q < kIbQpw; ++q) {
        int tok = slot_to_token(slot[q], h);
        float m = mx[q];
        merge_halves(m, tok);
        const float part = (tvalid[q] && tok != 0) ? m : 0.0f;
        const float score = half_sum(part);
        if (h == 0) res_tape[wave][q][jj][r32] = tvalid[q] ? tok : 0;
        if (lane == 0) res_score[wave][q][jj] = score;
        mx[q] = -INFINITY;
        slot[q] = -1;
      }
    }
    lds_barrier();
  };

  if (nsteps > 0) {
    Stage g0, g1;
    chunk_load(0, g0);
    chunk_load(1, g1);
    lds_store(0, g0);
    chunk_load(2, g0);
    lds_barrier();  // also publishes chunk_mask
    int c = 0;
    for (; c + 1 < nsteps; c += 2) {  // both steps unconditional: exact vmcnt waits
      step(c, g1);      // g1 held chunk c+1, now requests c+3
      step(c + 1, g0);  // g0 held chunk c+2, now requests c+4
    }
    if (c < nsteps) step(c, g1);
  }

  // ---- write the block's tape and scores (coalesced) ------------------------------
  const int ndoc = j1 - j0;
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
  // documents per block: enough blocks to fill 256 CUs several times over
  int db = kIbMaxDocs;
  while (db > 1 && (int64_t)A.nqb * ((A.Bd + db - 1) / db) < 2048) db >>= 1;
  A.db = db;
  A.ndb = (A.Bd + db - 1) / db;
  const dim3 grid((unsigned)(A.nqb * A.ndb)), block(64 * kIbWaves);
  if (dtype_bf16)
    hipLaunchKernelGGL(inbatch_mfma<OpBF16>, grid, block, 0, stream, A);
  else
    hipLaunchKernelGGL(inbatch_mfma<OpF16>, grid, block, 0, stream, A);
  return hipGetLastError();
}

bool inbatch_mfma_supported(int64_t dim, int64_t Tq, int64_t Td, const void* Q, const void* D) {
  const bool al = ((reinterpret_cast<uintptr_t>(Q) | reinterpret_cast<uintptr_t>(D)) & 15u) == 0;
  return dim == kIbNkb * 16 && Tq >= 1 && Tq <= kTile && Td >= 0 &&
         (Td + kTile - 1) / kTile <= kIbMaxChunkMasks / kIbMaxDocs &&
         Td * kIbRowBytes < ((int64_t)1 << 31) && al;
}

}  // namespace fms
