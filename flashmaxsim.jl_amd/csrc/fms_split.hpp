// fms_split.hpp -- the split-d scan kernel, built in its own translation
// units (fms_split_<type>.hip) with MFMA accumulators in ordinary VGPRs:
// it carries two accumulation chains across loop iterations, which in AGPRs
// would be copied back and forth every step.  The launcher in fms_scan.hpp
// dispatches to it for dims that are whole batches and whose query tile
// does not fit in registers.
#pragma once

#include "fms_scan.hpp"

namespace fms {

// scan_split<Op, L, KBAT>: dim == nbat * KBAT * KB exactly (16-byte aligned
// rows), for dims whose query tile does not fit in registers (and fp32).
// One step multiplies one batch of KBAT k-blocks of one (pair, query tile,
// chunk): the batch's document AND query fragments are loaded the step
// before (the query tile is re-read per chunk from L1/L2), so every step
// issues the same loads and the MFMAs wait only for the batch they use.
// Even and odd k-blocks accumulate into two independent chains, added when
// the chunk's last batch is done.

// Layouts whose positions all score the same query (a packed call scores
// one query against every document): the split kernel stages that query in
// LDS once per workgroup, in MFMA fragment order, instead of re-reading it
// from L1/L2 for every chunk.  Fragment (qt, kb, lane) sits at
// (qt * nkb + kb) * 64 + lane.
template <class L>
struct shared_query { static constexpr bool value = false; };
template <>
struct shared_query<LayPacked> { static constexpr bool value = true; };

constexpr int kSplitLdsQBytes = 64 * 1024;  // largest staged query (nqt * nkb KB)

template <class Op, int KBAT>
struct SplitBatch {
  typename Op::Frag a[KBAT];     // document fragments
  typename Op::Frag b[KBAT];     // query fragments
  uint32_t mbyte;                // raw document mask byte of row lane%32
  uint32_t qmbyte;               // raw query mask byte of token lane%32
  float qscale;                  // int8 query scale of token lane%32
  float ds[1];                   // int8 document scale of chunk row lane%32
};

template <class Op, int KBAT, bool kLdsQ>
__device__ __forceinline__ void load_split(SplitBatch<Op, KBAT>& c, const PairView& v, int qt,
                                           int ch, int bi, int rowbytes, int h, int r32,
                                           const u32x4* qlds, int nkb) {
  const int kofs = (bi * KBAT * Op::kKb + h * Op::kEpl) * Op::kEsz;
  const rsrc_t rd = make_rsrc_u(v.d, (uint32_t)v.td * (uint32_t)rowbytes);
  const rsrc_t rq = make_rsrc_u(v.q, (uint32_t)v.tq * (uint32_t)rowbytes);
  const int dbase = (ch * kTile + r32) * rowbytes + kofs;
  const int qbase = (qt * kTile + r32) * rowbytes + kofs;
#pragma unroll
  for (int k = 0; k < KBAT; ++k) {
    c.a[k] = Op::load(rd, dbase + k * Op::kKb * Op::kEsz);
    if constexpr (kLdsQ)
      c.b[k] = qlds[(qt * nkb + bi * KBAT + k) * 64 + h * 32 + r32];
    else
      c.b[k] = Op::load(rq, qbase + k * Op::kKb * Op::kEsz);
  }
  // Masks read unconditionally (zero-size resource when absent, see mask_ok).
  const bool has_dm = v.dm != nullptr, has_qm = v.qm != nullptr;
  c.mbyte = buf_load1(make_rsrc_u(has_dm ? (const void*)v.dm : (const void*)v.d,
                                  has_dm ? (uint32_t)v.td : 0u),
                      ch * kTile + r32);
  c.qmbyte = buf_load1(make_rsrc_u(has_qm ? (const void*)v.qm : (const void*)v.q,
                                   has_qm ? (uint32_t)v.tq : 0u),
                       qt * kTile + r32);
  c.qscale = 0.0f;
  if constexpr (Op::kInt) c.qscale = load_qscale(v, qt * kTile + r32);
  load_ds<Op>(c.ds, v, ch, r32);
}

template <class Op, class L, int KBAT, bool kLdsQ>
__global__ void __launch_bounds__(64 * kWaves) scan_split(const ScanArgs<L> A) {
  typedef typename Op::Acc Acc;
  const int lane = threadIdx.x & 63, r32 = lane & 31, h = lane >> 5;
  extern __shared__ u32x4 qlds[];  // kLdsQ: the shared query, nqt * nkb * 64 fragments
  if constexpr (kLdsQ) {
    // Every thread of the block takes part (before any wave may leave):
    // fragment (qt, kb, lane) = 16 bytes of query row qt*32 + lane%32 at
    // element kb*KB + (lane/32)*kEpl; rows past tq read 0.
    const PairView v0 = uniform_view(A.lay.get(0));
    const int rb = A.dim * Op::kEsz;
    const rsrc_t rq = make_rsrc_u(v0.q, (uint32_t)v0.tq * (uint32_t)rb);
    const int nfrag = A.nqt * A.nkb * 64;
    constexpr int kBatch = 8;  // loads in flight per thread
    for (int u0 = threadIdx.x; u0 < nfrag; u0 += kBatch * 64 * kWaves) {
      typename Op::Frag f[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int u = u0 + j * 64 * kWaves;
        const int fl = u & 63, kb = (u >> 6) % A.nkb, qt = (u >> 6) / A.nkb;
        // (u past nfrag: qt == A.nqt, a row past tq, which reads 0 and is not stored)
        f[j] = Op::load(rq, (qt * kTile + (fl & 31)) * rb + (kb * Op::kKb + (fl >> 5) * Op::kEpl) * Op::kEsz);
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j)
        if (u0 + j * 64 * kWaves < nfrag) qlds[u0 + j * 64 * kWaves] = f[j];
    }
    __syncthreads();
  }
  int64_t first, stride;
  int cnt;
  wave_positions(A, first, stride, cnt);
  if (cnt <= 0) return;
  const int rowbytes = A.dim * Op::kEsz;
  const int nbat = A.nkb / KBAT;

  // wave cursor: position index pi (view v), query tile qt, chunk ch of
  // nch, batch bi of nbat
  int pi = 0, qt = 0, ch = 0, bi = 0;
  PairView v = uniform_view(A.lay.get(first));
  int nch = v.td > 0 ? (v.td + kTile - 1) / kTile : 1;

  SplitBatch<Op, KBAT> bufA, bufB;
  Acc acc0 = {}, acc1 = {};
  float mx = -INFINITY, score = 0.0f;
  int slot = -1;

  load_split<Op, KBAT, kLdsQ>(bufA, v, 0, 0, 0, rowbytes, h, r32, qlds, A.nkb);

  auto step = [&](SplitBatch<Op, KBAT>& cur, SplitBatch<Op, KBAT>& nxt) -> bool {
    // advance a copy of the cursor and prefetch its batch
    int npi = pi, nqt_i = qt, nch_i = ch, nbi = bi + 1, nnch = nch;
    PairView nv = v;
    if (nbi >= nbat) {
      nbi = 0;
      if (++nch_i >= nch) {
        nch_i = 0;
        if (++nqt_i >= A.nqt) {
          nqt_i = 0;
          ++npi;
          const int64_t kpos = first + (int64_t)(npi < cnt ? npi : pi) * stride;
          if (npi < cnt) {
            nv = uniform_view(A.lay.get(kpos));
            nnch = nv.td > 0 ? (nv.td + kTile - 1) / kTile : 1;
          }
        }
      }
    }
    const bool more = npi < cnt;
    // One call on a selected cursor (after the wave's last batch it re-reads
    // the current one): two calls under `if (more)` get merged with their
    // arguments as divergent phis, and the loads become waterfall loops.
    load_split<Op, KBAT, kLdsQ>(nxt, more ? nv : v, more ? nqt_i : qt, more ? nch_i : ch,
                                more ? nbi : bi, rowbytes, h, r32, qlds, A.nkb);
    __builtin_amdgcn_sched_barrier(0);

#pragma unroll
    for (int k = 0; k < KBAT; ++k) {
      if (k & 1)
        acc1 = Op::mma(cur.a[k], cur.b[k], acc1);
      else
        acc0 = Op::mma(cur.a[k], cur.b[k], acc0);
    }

    if (bi == nbat - 1) {  // chunk complete: fold it
      Acc acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = acc0[r] + acc1[r];
      acc0 = Acc{};
      acc1 = Acc{};
      float s[16];
      acc_to_scores<Op>(acc, cur.qscale, cur.ds, h, s);
      const uint32_t m32 = chunk_rows_valid(v, ch, r32, cur.mbyte);
      take_first_row(s, m32, h, ch, mx, slot);
      update_chunk(s, m32, h, ch, mx, slot);
      if (ch == nch - 1) {
        uint32_t qmb = cur.qmbyte;
        asm volatile("" : "+v"(qmb));
        const bool tvalid = (qt * kTile + r32) < v.tq && mask_ok(v.qm, qmb);
        score += finish_tile(A, v.out, qt, r32, h, tvalid, mx, slot);
        mx = -INFINITY;
        slot = -1;
          if (qt == A.nqt - 1) {
          write_score(A, v, score, lane);
          score = 0.0f;
        }
      }
    }
    pi = npi; qt = nqt_i; ch = nch_i; bi = nbi; nch = nnch; v = nv;
    return more;
  };

  while (step(bufA, bufB) && step(bufB, bufA)) {
  }
}

template <class Op, class L>
hipError_t launch_split(const ScanArgs<L>& A, dim3 grid, dim3 block, hipStream_t stream) {
  if constexpr (shared_query<L>::value && Op::kEsz == 2) {
    const size_t qbytes = (size_t)A.nqt * A.nkb * 64 * 16;
    if (A.npairs > 0 && qbytes <= (size_t)kSplitLdsQBytes) {
      hipLaunchKernelGGL((scan_split<Op, L, split_kbat<Op>(), true>), grid, block, qbytes, stream, A);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((scan_split<Op, L, split_kbat<Op>(), false>), grid, block, 0, stream, A);
  return hipGetLastError();
}

}  // namespace fms
