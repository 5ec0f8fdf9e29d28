// fms_scan.hpp -- fused MaxSim scan kernels (pair / paired / candidates /
// in-batch-by-pair / packed / varlen), fp16 / bf16 / fp32 / int8.
//
// One wave owns a contiguous run of pairs and processes them one after the
// other (candidate pairs p = c + C*b of one query b are consecutive, so the
// query tile stays in registers across them).  Per pair and 32-token query
// tile, the document streams through in 32-token chunks; each chunk is one
// MFMA per k-block and one running max/argmax update per accumulator
// register.  Nothing of size Tq x Td ever reaches HBM.
//
// Two kernel shapes:
//   scan_fast<Op, L, NKB>: dim == NKB' * KB for NKB' <= NKB, 16-byte aligned
//     rows.  The query tile is register resident (NKB fragments), the next
//     chunk (possibly of the next pair) is prefetched into a second register
//     buffer while the current one is multiplied.
//   scan_generic<Op, L, VEC>: any dim (split-d: the query fragment is
//     re-read per k-block from L1/L2) and, with VEC = false, rows that are
//     not 16-byte multiples (element-wise guarded loads).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "fms_device.hpp"
#include "fms_layouts.hpp"

namespace fms {

template <class L>
struct ScanArgs {
  L lay;
  int dim;        // feature dimension
  int nkb;        // k-blocks = ceil(dim / KB)
  int rows;       // tape rows per pair (Tq, or max_q for varlen)
  int nqt;        // query tiles per pair = max(1, ceil(rows / 32))
  int ppw;        // pairs per wave
  int ds_vec;     // int8: document scale rows are 16-byte aligned (Td % 4 == 0)
  int64_t npairs;
  int32_t* args;    // (rows, npairs) nullable
  float* partial;   // (rows, npairs) nullable
  float* scores;    // (npairs,) nullable
  float neg;
};

template <class Op, int NKB>
struct Chunk {
  typename Op::Frag a[NKB];
  uint32_t mbyte;                 // document mask byte of row lane%32
  float ds[Op::kInt ? 16 : 1];    // int8: document scale of each accumulator row
};

// Per-lane query state for one (pair, query tile).
template <class Op, int NKB>
struct QTile {
  typename Op::Frag f[NKB];
  float qscale;   // int8 query scale of this lane's token
  bool tvalid;    // this lane's query token exists and is unmasked
};

// ---- shared pieces ---------------------------------------------------------------

// Validity of this lane's chunk row (row lane%32 of chunk ch) -> wave ballot.
__device__ __forceinline__ uint32_t chunk_rows_valid(const PairView& v, int ch, int r32,
                                                     uint32_t mbyte) {
  const bool ok = (ch * kTile + r32 < v.td) && (mbyte != 0u);
  return (uint32_t)__ballot(ok);
}

template <class Op>
__device__ __forceinline__ void load_ds(float (&ds)[Op::kInt ? 16 : 1], const PairView& v, int ch,
                                        int h, bool vec) {
  if constexpr (Op::kInt) {
    const rsrc_t rs = make_rsrc(v.ds, (uint32_t)v.td * 4u);
    if (vec) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 w = buf_load16f(rs, (ch * kTile + 8 * g + 4 * h) * 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) ds[4 * g + i] = w[i];
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        ds[r] = __builtin_bit_cast(float, buf_load4(rs, (ch * kTile + acc_row(r, h)) * 4));
    }
  }
}

// Accumulator -> fp32 scores.  int8: s = (qs[t] * ds[u]) * Float32(acc)
// evaluated left to right (quant.jl:113, kernels_int8.jl:25).
template <class Op>
__device__ __forceinline__ void acc_to_scores(const typename Op::Acc& acc, float qscale,
                                              const float (&ds)[Op::kInt ? 16 : 1],
                                              float (&s)[16]) {
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    if constexpr (Op::kInt) {
      const float sc = qscale * ds[r];
      s[r] = sc * (float)acc[r];
    } else {
      s[r] = acc[r];
    }
  }
}

__device__ __forceinline__ void update_chunk(const float (&s)[16], uint32_t m32, int h, int ch,
                                             float& mx, int& slot) {
  if (m32 == 0xffffffffu)
    running_max_seq<false>(s, 0u, ch * 16, mx, slot);
  else if (m32 != 0u)
    running_max_seq<true>(s, m32 >> (4 * h), ch * 16, mx, slot);
}

// Close one (pair, query tile): merge halves, write tape / partial, return
// this tile's contribution to the pair score (same value in every lane).
template <class L>
__device__ __forceinline__ float finish_tile(const ScanArgs<L>& A, int64_t p, int qt, int r32,
                                             int h, bool tvalid, float mx, int slot) {
  int tok = slot_to_token(slot, h);
  merge_halves(mx, tok);
  const float part = (tvalid && tok != 0) ? mx : 0.0f;
  const int arg = tvalid ? tok : 0;
  const int t = qt * kTile + r32;
  if (h == 0 && t < A.rows) {
    const int64_t o = p * (int64_t)A.rows + t;
    if (A.args) A.args[o] = arg;
    if (A.partial) A.partial[o] = part;
  }
  return half_sum(part);
}

template <class L>
__device__ __forceinline__ void write_score(const ScanArgs<L>& A, int64_t p, bool valid,
                                            float score, int lane) {
  if (A.scores && lane == 0) A.scores[p] = valid ? score : A.neg;
}

// ---- fast kernel ------------------------------------------------------------------

template <class Op, int NKB>
__device__ __forceinline__ void load_chunk(Chunk<Op, NKB>& c, const PairView& v, int ch, int nkb,
                                           int rowbytes, int lane_off, int r32, int h,
                                           bool ds_vec) {
  const rsrc_t rd = make_rsrc(v.d, (uint32_t)v.td * (uint32_t)rowbytes);
  const int base = ch * kTile * rowbytes + lane_off;
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
    if (kb < nkb) c.a[kb] = Op::load(rd, base + kb * Op::kKb * Op::kEsz);
  if (v.dm) {
    const rsrc_t rm = make_rsrc(v.dm, (uint32_t)v.td);
    c.mbyte = buf_load1(rm, ch * kTile + r32);
  } else {
    c.mbyte = 1u;
  }
  load_ds<Op>(c.ds, v, ch, h, ds_vec);
}

template <class Op, int NKB>
__device__ __forceinline__ void load_qtile(QTile<Op, NKB>& q, const PairView& v, int qt, int nkb,
                                           int rowbytes, int lane_off, int r32) {
  const rsrc_t rq = make_rsrc(v.q, (uint32_t)v.tq * (uint32_t)rowbytes);
  const int base = qt * kTile * rowbytes + lane_off;
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
    q.f[kb] = (kb < nkb) ? Op::load(rq, base + kb * Op::kKb * Op::kEsz) : Op::zero();
  const int t = qt * kTile + r32;
  uint32_t mb = 1u;
  if (v.qm) mb = buf_load1(make_rsrc(v.qm, (uint32_t)v.tq), t);
  q.tvalid = (t < v.tq) && (mb != 0u);
  q.qscale = 0.0f;
  if constexpr (Op::kInt) q.qscale = __builtin_bit_cast(float, buf_load4(make_rsrc(v.qs, (uint32_t)v.tq * 4u), t * 4));
}

template <class Op, class L, int NKB>
__global__ void __launch_bounds__(64 * kWaves) scan_fast(const ScanArgs<L> A) {
  typedef typename Op::Acc Acc;
  const int lane = threadIdx.x & 63, r32 = lane & 31, h = lane >> 5;
  const int wave = uniform((int)(blockIdx.x * kWaves + (threadIdx.x >> 6)));
  const int64_t p0 = (int64_t)wave * A.ppw;
  if (p0 >= A.npairs) return;
  const int64_t p1 = (p0 + A.ppw < A.npairs) ? p0 + A.ppw : A.npairs;
  const int rowbytes = A.dim * Op::kEsz;
  const int lane_off = r32 * rowbytes + h * Op::kEpl * Op::kEsz;
  const int nkb = A.nkb;
  const bool ds_vec = A.ds_vec != 0;

  // wave cursor: pair p, query tile qt, chunk ch of nch
  int64_t p = p0;
  int qt = 0, ch = 0;
  PairView v = A.lay.get(p);
  int nch = v.td > 0 ? (v.td + kTile - 1) / kTile : 1;

  Chunk<Op, NKB> bufA, bufB;
  QTile<Op, NKB> q;
  const char* q_src = nullptr;
  int q_qt = -1;
  float mx = -INFINITY, score = 0.0f;
  int slot = -1;

  load_chunk<Op, NKB>(bufA, v, 0, nkb, rowbytes, lane_off, r32, h, ds_vec);

  // One step: make sure the query tile is resident, prefetch the next chunk
  // into `nxt`, multiply `cur`, fold it into the running max, and close the
  // tile / pair when this was its last chunk.  Returns false after the
  // wave's final chunk.
  auto step = [&](Chunk<Op, NKB>& cur, Chunk<Op, NKB>& nxt) -> bool {
    if (ch == 0 && (v.q != q_src || qt != q_qt)) {
      load_qtile<Op, NKB>(q, v, qt, nkb, rowbytes, lane_off, r32);
      q_src = v.q;
      q_qt = qt;
    }
    // advance a copy of the cursor and prefetch its chunk
    int64_t np = p;
    int nqt_i = qt, nch_i = ch + 1, nnch = nch;
    PairView nv = v;
    if (nch_i >= nch) {
      nch_i = 0;
      if (++nqt_i >= A.nqt) {
        nqt_i = 0;
        ++np;
        if (np < p1) {
          nv = A.lay.get(np);
          nnch = nv.td > 0 ? (nv.td + kTile - 1) / kTile : 1;
        }
      }
    }
    const bool more = np < p1;
    if (more) load_chunk<Op, NKB>(nxt, nv, nch_i, nkb, rowbytes, lane_off, r32, h, ds_vec);

    Acc acc = {};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
      if (kb < nkb) acc = Op::mma(cur.a[kb], q.f[kb], acc);
    float s[16];
    acc_to_scores<Op>(acc, q.qscale, cur.ds, s);
    const uint32_t m32 = chunk_rows_valid(v, ch, r32, cur.mbyte);
    update_chunk(s, m32, h, ch, mx, slot);

    if (ch == nch - 1) {
      score += finish_tile(A, p, qt, r32, h, q.tvalid, mx, slot);
      mx = -INFINITY;
      slot = -1;
      if (qt == A.nqt - 1) {
        write_score(A, p, v.valid, score, lane);
        score = 0.0f;
      }
    }
    p = np; qt = nqt_i; ch = nch_i; nch = nnch; v = nv;
    return more;
  };

  while (step(bufA, bufB) && step(bufB, bufA)) {
  }
}

// ---- generic kernel ---------------------------------------------------------------

template <class Op, bool VEC>
__device__ __forceinline__ typename Op::Frag load_frag(rsrc_t r, int row, int rowbytes, int kb,
                                                        int h, int dim) {
  const int k0 = kb * Op::kKb + h * Op::kEpl;
  const int voff = row * rowbytes + k0 * Op::kEsz;
  if constexpr (VEC) {
    return (k0 < dim) ? Op::load(r, voff) : Op::zero();
  } else {
    return Op::load_guarded(r, voff, k0, dim);
  }
}

template <class Op, class L, bool VEC>
__global__ void __launch_bounds__(64 * kWaves) scan_generic(const ScanArgs<L> A) {
  typedef typename Op::Acc Acc;
  const int lane = threadIdx.x & 63, r32 = lane & 31, h = lane >> 5;
  const int wave = uniform((int)(blockIdx.x * kWaves + (threadIdx.x >> 6)));
  const int64_t p0 = (int64_t)wave * A.ppw;
  if (p0 >= A.npairs) return;
  const int64_t p1 = (p0 + A.ppw < A.npairs) ? p0 + A.ppw : A.npairs;
  const int dim = A.dim;
  const int rowbytes = dim * Op::kEsz;

  for (int64_t p = p0; p < p1; ++p) {
    const PairView v = A.lay.get(p);
    const int nch = v.td > 0 ? (v.td + kTile - 1) / kTile : 1;
    const rsrc_t rq = make_rsrc(v.q, (uint32_t)v.tq * (uint32_t)rowbytes);
    const rsrc_t rd = make_rsrc(v.d, (uint32_t)v.td * (uint32_t)rowbytes);
    float score = 0.0f;
    for (int qt = 0; qt < A.nqt; ++qt) {
      const int t = qt * kTile + r32;
      uint32_t mb = 1u;
      if (v.qm) mb = buf_load1(make_rsrc(v.qm, (uint32_t)v.tq), t);
      const bool tvalid = (t < v.tq) && (mb != 0u);
      float qscale = 0.0f;
      if constexpr (Op::kInt) qscale = __builtin_bit_cast(float, buf_load4(make_rsrc(v.qs, (uint32_t)v.tq * 4u), t * 4));
      float mx = -INFINITY;
      int slot = -1;
      for (int ch = 0; ch < nch; ++ch) {
        Acc acc = {};
        const int row = ch * kTile + r32;
        // split-d: 8 k-blocks of document and query fragments in flight per
        // batch; blocks past nkb load as zero and add nothing.
        for (int kb0 = 0; kb0 < A.nkb; kb0 += 8) {
          typename Op::Frag a[8], b[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int kb = kb0 + i;
            a[i] = kb < A.nkb ? load_frag<Op, VEC>(rd, row, rowbytes, kb, h, dim) : Op::zero();
            b[i] = kb < A.nkb ? load_frag<Op, VEC>(rq, t, rowbytes, kb, h, dim) : Op::zero();
          }
#pragma unroll
          for (int i = 0; i < 8; ++i) acc = Op::mma(a[i], b[i], acc);
        }
        uint32_t mbyte = 1u;
        if (v.dm) mbyte = buf_load1(make_rsrc(v.dm, (uint32_t)v.td), row);
        float ds[Op::kInt ? 16 : 1];
        load_ds<Op>(ds, v, ch, h, false);
        float s[16];
        acc_to_scores<Op>(acc, qscale, ds, s);
        update_chunk(s, chunk_rows_valid(v, ch, r32, mbyte), h, ch, mx, slot);
      }
      score += finish_tile(A, p, qt, r32, h, tvalid, mx, slot);
    }
    write_score(A, p, v.valid, score, lane);
  }
}

// ---- host-side launcher -------------------------------------------------------------

// Fast-kernel bucket (register-resident k-blocks) for a given nkb; 0 = none.
template <class Op>
constexpr int fast_bucket(int nkb) {
  if (Op::kEsz == 4) return 0;  // fp32 uses the generic kernel
  const int b1 = (Op::kKb == 16) ? 8 : 4;   // dim <= 128
  const int b2 = 2 * b1;                    // dim <= 256
  return nkb <= b1 ? b1 : (nkb <= b2 ? b2 : 0);
}

inline int pairs_per_wave(int64_t npairs) {
  // Aim for ~32k waves (8 resident per SIMD over 1024 SIMDs, several rounds)
  // so that each wave keeps its query tile across a handful of pairs.
  int64_t ppw = npairs / 32768;
  if (ppw < 1) ppw = 1;
  if (ppw > 32) ppw = 32;
  return (int)ppw;
}

template <class Op, class L>
hipError_t launch_scan(const L& lay, int dim, int rows, int64_t npairs, int32_t* args,
                       float* partial, float* scores, float neg, bool vec, bool ds_vec,
                       hipStream_t stream) {
  ScanArgs<L> A;
  A.lay = lay;
  A.dim = dim;
  A.nkb = (dim + Op::kKb - 1) / Op::kKb;
  A.rows = rows;
  A.nqt = rows > 0 ? (rows + kTile - 1) / kTile : 1;
  A.ppw = pairs_per_wave(npairs);
  A.ds_vec = ds_vec ? 1 : 0;
  A.npairs = npairs;
  A.args = args;
  A.partial = partial;
  A.scores = scores;
  A.neg = neg;
  const int64_t waves = (npairs + A.ppw - 1) / A.ppw;
  const dim3 grid((unsigned)((waves + kWaves - 1) / kWaves));
  const dim3 block(64 * kWaves);
  const bool fast_ok = vec && (dim % Op::kKb == 0) && dim > 0;
  const int bucket = fast_ok ? fast_bucket<Op>(A.nkb) : 0;
  if constexpr (Op::kEsz != 4) {
    constexpr int b1 = (Op::kKb == 16) ? 8 : 4;
    if (bucket == b1) {
      hipLaunchKernelGGL((scan_fast<Op, L, b1>), grid, block, 0, stream, A);
      return hipGetLastError();
    }
    if (bucket == 2 * b1) {
      hipLaunchKernelGGL((scan_fast<Op, L, 2 * b1>), grid, block, 0, stream, A);
      return hipGetLastError();
    }
  }
  if (vec) {
    hipLaunchKernelGGL((scan_generic<Op, L, true>), grid, block, 0, stream, A);
  } else {
    hipLaunchKernelGGL((scan_generic<Op, L, false>), grid, block, 0, stream, A);
  }
  return hipGetLastError();
}

}  // namespace fms
