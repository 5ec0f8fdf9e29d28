// fms_runs.hpp -- the candidate scan over document batches.
//
// After the counting sort by document (group_pairs_by_document), the pairs of
// each document form a run of consecutive positions.  Every run is cut into
// batches of at most KQ pairs starting at the run start, so the batch
// structure is a function of the sort alone: batch starts are run starts plus
// multiples of KQ.  A wave owns the batches that START in its range of ppw
// positions (a batch may run past that range's end; the next wave skips it),
// and per batch it
//   * loads the KQ query tiles into registers (pairs missing from a short
//     batch read an empty resource: zeros, no traffic),
//   * streams the document once, chunk by chunk, with the next chunk -- also
//     across batch boundaries -- prefetched into a second register buffer,
//   * multiplies every chunk by each of the batch's query tiles (KQ
//     independent MFMA chains) and folds each into that pair's running
//     max / argmax, exactly as scan_fast does for one pair,
//   * closes every pair at the document's last chunk.
// So each document leaves HBM once per batch instead of once per pair; a
// run longer than KQ costs one read per KQ pairs.  Results are identical to
// scan_fast (the same per-pair arithmetic in the same order).
#pragma once

#include "fms_scan.hpp"

namespace fms {

struct RunArgs : ScanArgs<LayCand> {
  const PairRef* order;     // pair ids grouped by document, invalid indices last
  const uint32_t* doc_end;  // (N + 1,): document j's pairs end at doc_end[j]
};

// [start, end) of the run of 0-based document j (j < 0: the invalid pairs,
// sorted after document N - 1).
__device__ __forceinline__ void run_bounds(const RunArgs& A, int j, int64_t& rs, int64_t& re) {
  const int64_t jj = j < 0 ? A.lay.N : (int64_t)j;
  rs = jj > 0 ? (int64_t)sload(A.doc_end, jj - 1) : 0;
  re = (int64_t)sload(A.doc_end, jj);
}

// The view of the document of run j (td = 0 and invalid for j < 0).
__device__ __forceinline__ void doc_view(const RunArgs& A, int j, PairView& v) {
  const LayCand& c = A.lay;
  v.valid = j >= 0;
  const int64_t jj = v.valid ? j : 0;
  v.d = c.G + jj * c.dbytes;
  v.dm = c.dm ? c.dm + jj * c.Td : nullptr;
  v.ds = c.Gs ? c.Gs + jj * c.Td * c.ds_esz : nullptr;
  v.td = v.valid ? c.Td : 0;
}

// The query side of pair p (output slot p = c + C * b); p < 0: an empty slot.
__device__ __forceinline__ void query_view(const RunArgs& A, int p, PairView& v) {
  const LayCand& c = A.lay;
  const int64_t b = p >= 0 ? (int64_t)((uint32_t)p / (uint32_t)c.C) : 0;
  v.q = c.Q + b * c.qbytes;
  v.qm = c.qm ? c.qm + b * c.Tq : nullptr;
  v.qs = c.Qs ? c.Qs + b * c.Tq * c.qs_esz : nullptr;
  v.qs_half = c.qs_esz == 2;
  v.tq = p >= 0 ? c.Tq : 0;
  v.out = p;
}

template <class Op, int NKB, int KQ>
__global__ void __launch_bounds__(64 * kWaves) scan_runs(const RunArgs A) {
  typedef typename Op::Acc Acc;
  const int lane = threadIdx.x & 63, r32 = lane & 31, h = lane >> 5;
  const int64_t P = A.npairs;
  const int64_t w = (int64_t)blockIdx.x * kWaves + uniform((int)(threadIdx.x >> 6));
  const int64_t s0 = w * A.ppw;
  if (s0 >= P) return;
  const int64_t e0 = s0 + A.ppw < P ? s0 + A.ppw : P;

  // First batch start at or after s0.
  int64_t k;
  {
    int64_t rs, re;
    run_bounds(A, sload(&A.order[s0].j, 0), rs, re);
    const int64_t off = s0 - rs;
    k = (off % KQ == 0) ? s0 : rs + (off / KQ + 1) * KQ;
    if (k > re) k = re;
  }
  if (k >= e0) return;

  const int rowbytes = A.dim * Op::kEsz;
  const int lane_off = r32 * rowbytes + h * Op::kEpl * Op::kEsz;
  const int nkb = A.nkb;

  // Batch at position k: its run's document j and kb pairs (kb <= KQ).  The
  // pair ids are re-read from the order where they are used (scalar cache)
  // rather than carried through the loop in scalar registers.
  auto batch_at = [&](int64_t pos, int& j, int& kb) {
    j = sload(&A.order[pos].j, 0);
    int64_t rs, re;
    run_bounds(A, j, rs, re);
    kb = (int)(re - pos < KQ ? re - pos : KQ);
  };

  // wave cursor: batch (k, j, kb), query tile qt, chunk ch of nch
  int j, kb;
  batch_at(k, j, kb);
  auto pair_id = [&](int i) { return i < kb ? sload(&A.order[k + i].p, 0) : -1; };
  PairView dv;
  doc_view(A, j, dv);
  dv = uniform_view(dv);
  int nch = dv.td > 0 ? (dv.td + kTile - 1) / kTile : 1;
  int qt = 0, ch = 0;

  Chunk<Op, NKB> bufA, bufB;
  QTile<Op, NKB> q[KQ];
  float mx[KQ], score[KQ];
  int slot[KQ];
#pragma unroll
  for (int i = 0; i < KQ; ++i) { mx[i] = -INFINITY; slot[i] = -1; score[i] = 0.0f; }

  load_chunk<Op, NKB>(bufA, dv, 0, nkb, rowbytes, lane_off, r32);

  // The batch's query tiles for query tile qt.  The first batch loads them
  // here; every later batch's are requested right after the previous batch's
  // last MFMAs, so they are in flight with the prefetched chunk.
  auto load_queries = [&]() {
#pragma unroll
    for (int i = 0; i < KQ; ++i) {
      PairView qv = dv;
      query_view(A, pair_id(i), qv);
      load_qtile<Op, NKB>(q[i], uniform_view(qv), qt, nkb, rowbytes, lane_off, r32);
    }
  };
  load_queries();

  auto step = [&](Chunk<Op, NKB>& cur, Chunk<Op, NKB>& nxt) -> bool {
    const uint32_t m32 = chunk_rows_valid(dv, ch, r32, cur.mbyte);
    // advance a copy of the cursor and prefetch its chunk
    int64_t nk = k;
    int nj = j, nkbn = kb;
    int nqt_i = qt, nch_i = ch + 1, nnch = nch;
    PairView ndv = dv;
    bool more = true;
    if (nch_i >= nch) {
      nch_i = 0;
      if (++nqt_i >= A.nqt) {
        nqt_i = 0;
        nk = k + kb;
        more = nk < e0;
        if (more) {
          batch_at(nk, nj, nkbn);
          doc_view(A, nj, ndv);
          ndv = uniform_view(ndv);
          nnch = ndv.td > 0 ? (ndv.td + kTile - 1) / kTile : 1;
        }
      }
    }
    // Unconditional (after the wave's last chunk it re-reads the current one).
    load_chunk<Op, NKB>(nxt, more ? ndv : dv, more ? nch_i : ch, nkb, rowbytes, lane_off, r32);
    __builtin_amdgcn_sched_barrier(0);

#pragma unroll
    for (int i = 0; i < KQ; ++i) {
      if (i < kb) {
        Acc acc = {};
#pragma unroll
        for (int kk = 0; kk < NKB; ++kk) acc = Op::mma(cur.a[kk], q[i].f[kk], acc);
        float s[16];
        acc_to_scores<Op>(acc, q[i].qscale, cur.ds, h, s);
        take_first_row(s, m32, h, ch, mx[i], slot[i]);
        update_chunk(s, m32, h, ch, mx[i], slot[i]);
      }
    }

    if (ch == nch - 1) {
#pragma unroll
      for (int i = 0; i < KQ; ++i) {
        if (i < kb) {
          PairView pv = dv;
          query_view(A, pair_id(i), pv);
          pv = uniform_view(pv);
          uint32_t qmb = q[i].mbyte;
          asm volatile("" : "+v"(qmb));
          const bool tvalid = q[i].t < pv.tq && mask_ok(pv.qm, qmb);
          score[i] += finish_tile(A, pv.out, qt, r32, h, tvalid, mx[i], slot[i]);
          mx[i] = -INFINITY;
          slot[i] = -1;
          if (qt == A.nqt - 1) {
            write_score(A, pv, score[i], lane);
            score[i] = 0.0f;
          }
        }
      }
    }
    const bool new_tiles = more && nch_i == 0;  // the next step starts a (batch, tile)
    k = nk; j = nj; kb = nkbn;
    qt = nqt_i; ch = nch_i; nch = nnch; dv = ndv;
    if (new_tiles) load_queries();
    return more;
  };

  while (step(bufA, bufB) && step(bufB, bufA)) {
  }
}

// Pairs per wave of the batch kernel: about 8 batches per wave, so a call of
// 256k pairs makes ~12k waves (several rounds of 8 resident per CU).
inline int run_ppw(int64_t npairs, int kq) {
  int64_t ppw = npairs / 16384;
  if (ppw < kq) ppw = kq;
  if (ppw > 64) ppw = 64;
  return (int)ppw;
}

// Whether the batch kernel serves this Op and dim (the fast kernel's dims).
template <class Op>
inline bool runs_supported(int dim, bool vec) {
  if (Op::kEsz == 4 || !vec || dim <= 0 || dim % Op::kKb != 0) return false;
  return fast_nkb<Op>(dim / Op::kKb) != 0;
}

template <class Op>
hipError_t launch_runs(const RunArgs& A_in, hipStream_t stream);

}  // namespace fms
