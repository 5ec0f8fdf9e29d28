// fms_scan.hpp -- fused MaxSim scan kernels (pair / paired / candidates /
// in-batch-by-pair / packed / varlen), fp16 / bf16 / fp32 / int8.
//
// One wave owns a run of scan positions and processes their pairs one after
// the other.  In output order (every layout but LayCandSorted) the run is
// contiguous: candidate pairs p = c + C*b of one query b are consecutive, so
// the query tile stays in registers across them.  In document order
// (LayCandSorted) the waves of a workgroup take interleaved positions, so
// the kWaves waves of a workgroup score kWaves consecutive entries of the
// document order at the same time: pairs that share a document read it
// together, through one L2, once.  Per pair and 32-token query
// tile, the document streams through in 32-token chunks; each chunk is one
// MFMA per k-block and one running max/argmax update per accumulator
// register.  Nothing of size Tq x Td ever reaches HBM.
//
// Three kernel shapes, tried in this order:
//   scan_fast<Op, L, NKB>: dim == NKB * KB exactly, 16-byte aligned rows.
//     The loads and MFMAs of a step are unconditional, so the compiler's
//     in-order vmcnt accounting waits for exactly the chunk it multiplies
//     and never drains the prefetch.  The query tile is register resident
//     (NKB fragments), the next
//     chunk (possibly of the next pair) is prefetched into a second register
//     buffer while the current one is multiplied.
//   scan_split<Op, L, KBAT> (fms_split.hpp): dims that are whole batches of
//     KBAT k-blocks but whose query tile does not fit in registers (and
//     fp32); document and query fragments stream one batch ahead.
//   scan_generic<Op, L, VEC>: any dim (split-d: the query fragment is
//     re-read per k-block from L1/L2) and, with VEC = false, rows that are
//     not 16-byte multiples (element-wise guarded loads).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "fms_device.hpp"
#include "fms_layouts.hpp"
#include "fms_scan_decl.hpp"

namespace fms {

// Layouts whose positions are interleaved across the waves of a workgroup.
template <class L>
struct interleaved { static constexpr bool value = false; };
template <>
struct interleaved<LayCandSorted> { static constexpr bool value = true; };

template <class L>
struct ScanArgs {
  L lay;
  int dim;        // feature dimension
  int nkb;        // k-blocks = ceil(dim / KB)
  int rows;       // tape rows per pair (Tq, or max_q for varlen)
  int nqt;        // query tiles per pair = max(1, ceil(rows / 32))
  int ppw;        // pairs per wave
  int64_t npairs;
  int32_t* args;    // (rows, npairs) nullable
  float* partial;   // (rows, npairs) nullable
  float* scores;    // (npairs,) nullable
  float neg;
  int norm;         // scores *= 1 / max(valid query tokens, 1) (valid pairs only)
};

template <class Op, int NKB>
struct Chunk {
  typename Op::Frag a[NKB];
  uint32_t mbyte;                 // document mask byte of row lane%32 (0 when the
                                  // pair has no mask: test with mask_ok)
  float ds[1];                    // int8: document scale of chunk row lane%32
};

// Per-lane query state for one (pair, query tile).
template <class Op, int NKB>
struct QTile {
  typename Op::Frag f[NKB];
  float qscale;    // int8 query scale of this lane's token
  uint32_t mbyte;  // query mask byte of this lane's token, raw (0 when there is
                   // no mask).  Tested only at tile close, so nothing waits for
                   // the load before the MFMAs.
  int t;           // this lane's query token
};

// ---- shared pieces ---------------------------------------------------------------

// Scan positions of this wave: first, first + stride, ... (cnt of them).
template <class L>
__device__ __forceinline__ void wave_positions(const ScanArgs<L>& A, int64_t& first,
                                               int64_t& stride, int& cnt) {
  const int wib = uniform((int)(threadIdx.x >> 6));
  int64_t rem;
  if constexpr (interleaved<L>::value) {
    first = (int64_t)blockIdx.x * kWaves * A.ppw + wib;
    stride = kWaves;
    rem = A.npairs > first ? (A.npairs - first + kWaves - 1) / kWaves : 0;
  } else {
    first = ((int64_t)blockIdx.x * kWaves + wib) * A.ppw;
    stride = 1;
    rem = A.npairs > first ? A.npairs - first : 0;
  }
  cnt = (int)(rem < A.ppw ? rem : A.ppw);
}

// A raw mask byte (read unconditionally from a zero-size resource when the
// mask pointer is NULL) and whether it marks a valid token.
__device__ __forceinline__ bool mask_ok(const void* mask, uint32_t raw) {
  return mask == nullptr || raw != 0u;
}

// Validity of this lane's chunk row (row lane%32 of chunk ch) -> wave ballot.
__device__ __forceinline__ uint32_t chunk_rows_valid(const PairView& v, int ch, int r32,
                                                     uint32_t mbyte) {
  const bool ok = (ch * kTile + r32 < v.td) && mask_ok(v.dm, mbyte);
  return (uint32_t)__ballot(ok);
}

// int8: each lane loads the document scale of chunk row lane%32 (rows past the
// document read 0 and are masked).  acc_to_scores fetches the 16 scales of its
// accumulator rows from the lanes that hold them, so a chunk buffer carries
// one scale register instead of sixteen.
// fp16 document scales (Op::kDsHalf) widen exactly to fp32.
template <class Op>
__device__ __forceinline__ void load_ds(float (&ds)[1], const PairView& v, int ch, int r32) {
  if constexpr (Op::kInt) {
    const int row = ch * kTile + r32;
    if constexpr (Op::kDsHalf) {
      const rsrc_t rs = make_rsrc_u(v.ds, (uint32_t)v.td * 2u);
      ds[0] = (float)__builtin_bit_cast(_Float16, (uint16_t)buf_load2(rs, row * 2));
    } else {
      const rsrc_t rs = make_rsrc_u(v.ds, (uint32_t)v.td * 4u);
      ds[0] = __builtin_bit_cast(float, buf_load4(rs, row * 4));
    }
  }
}

// int8 query scale of token t, fp32 or fp16 (v.qs_half, uniform) widened to
// fp32.  Both halves of the 4-byte word are read unconditionally (a
// conditional load would make the compiler drain the chunk prefetch); for
// fp16 scales the second read is the next token's scale or 0 past the end.
__device__ __forceinline__ float load_qscale(const PairView& v, int t) {
  const uint32_t esz = v.qs_half ? 2u : 4u;
  const rsrc_t r = make_rsrc_u(v.qs, (uint32_t)v.tq * esz);
  const uint32_t lo = buf_load2(r, t * (int)esz) & 0xffffu;
  const uint32_t hi = buf_load2(r, t * (int)esz + 2) & 0xffffu;
  const float h16 = (float)__builtin_bit_cast(_Float16, (uint16_t)lo);
  const float f32 = __builtin_bit_cast(float, lo | (hi << 16));
  return v.qs_half ? h16 : f32;
}

// Accumulator -> fp32 scores.  int8: s = (qs[t] * ds[u]) * Float32(acc)
// evaluated left to right (quant.jl:113, kernels_int8.jl:25).
template <class Op>
__device__ __forceinline__ void acc_to_scores(const typename Op::Acc& acc, float qscale,
                                              const float (&ds)[1], int h, float (&s)[16]) {
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    if constexpr (Op::kInt) {
      const float sc = qscale * __shfl(ds[0], acc_row(r, h), 64);
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
__device__ __forceinline__ float finish_tile(const ScanArgs<L>& A, int64_t out, int qt, int r32,
                                             int h, bool tvalid, float mx, int slot) {
  int tok = slot_to_token(slot, h);
  merge_halves(mx, tok, h);
  const float part = (tvalid && tok != 0) ? mx : 0.0f;
  const int arg = tvalid ? tok : 0;
  const int t = qt * kTile + r32;
  if (h == 0 && t < A.rows) {
    const int64_t o = out * (int64_t)A.rows + t;
    if (A.args) A.args[o] = arg;
    if (A.partial) A.partial[o] = part;
  }
  return half_sum(part);
}

// 1 / max(n, 1) in fp32, n = the pair's valid query tokens (its qmask count,
// or all tq tokens without a mask): inv_token_counts (normalize.jl:4-10) and
// varlen_inv_n_kernel! (kernels_packed.jl:277-282).  Wave-uniform control.
__device__ __forceinline__ float pair_inv_count(const PairView& v, int lane) {
  int n = 0;
  for (int t0 = 0; t0 < v.tq; t0 += 64) {
    const int t = t0 + lane;
    const bool ok = t < v.tq && (v.qm == nullptr || v.qm[t] != 0);
    n += __builtin_popcountll(__ballot(ok));
  }
  const float nf = (float)n;
  return 1.0f / (nf > 1.0f ? nf : 1.0f);
}

// The pair's score: Σ_t, then the normalize epilogue (length_normalize,
// normalize.jl:23-25) on valid pairs; an invalid candidate keeps neg
// (length_normalize_candidates, normalize.jl:37-46).
template <class L>
__device__ __forceinline__ void write_score(const ScanArgs<L>& A, const PairView& v, float score,
                                            int lane) {
  if (!A.scores) return;
  if (A.norm && v.valid) score *= pair_inv_count(v, lane);
  if (lane == 0) A.scores[v.out] = v.valid ? score : A.neg;
}

// ---- fast kernel ------------------------------------------------------------------

template <class Op, int NKB>
__device__ __forceinline__ void load_chunk(Chunk<Op, NKB>& c, const PairView& v, int ch, int nkb,
                                           int rowbytes, int lane_off, int r32) {
  const rsrc_t rd = make_rsrc_u(v.d, (uint32_t)v.td * (uint32_t)rowbytes);
  const int base = ch * kTile * rowbytes + lane_off;
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) c.a[kb] = Op::load(rd, base + kb * Op::kKb * Op::kEsz);
  // Unconditional load (a zero-size resource reads 0 when there is no
  // mask): conditional loads make the compiler's vmcnt count path
  // dependent, and it then drains the prefetch.
  const bool has_m = v.dm != nullptr;
  const uint32_t mraw = buf_load1(make_rsrc_u(has_m ? (const void*)v.dm : (const void*)v.d,
                                              has_m ? (uint32_t)v.td : 0u),
                                  ch * kTile + r32);
  c.mbyte = mraw;
  load_ds<Op>(c.ds, v, ch, r32);
}

template <class Op, int NKB>
__device__ __forceinline__ void load_qtile(QTile<Op, NKB>& q, const PairView& v, int qt, int nkb,
                                           int rowbytes, int lane_off, int r32) {
  const rsrc_t rq = make_rsrc_u(v.q, (uint32_t)v.tq * (uint32_t)rowbytes);
  const int base = qt * kTile * rowbytes + lane_off;
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) q.f[kb] = Op::load(rq, base + kb * Op::kKb * Op::kEsz);
  q.t = qt * kTile + r32;
  const bool has_m = v.qm != nullptr;
  const uint32_t mraw = buf_load1(make_rsrc_u(has_m ? (const void*)v.qm : (const void*)v.q,
                                              has_m ? (uint32_t)v.tq : 0u),
                                  q.t);
  q.mbyte = mraw;
  q.qscale = 0.0f;
  if constexpr (Op::kInt) q.qscale = load_qscale(v, q.t);
}

template <class Op, class L, int NKB>
__global__ void __launch_bounds__(64 * kWaves) scan_fast(const ScanArgs<L> A) {
  typedef typename Op::Acc Acc;
  const int lane = threadIdx.x & 63, r32 = lane & 31, h = lane >> 5;
  int64_t first, stride;
  int cnt;
  wave_positions(A, first, stride, cnt);
  if (cnt <= 0) return;
  const int rowbytes = A.dim * Op::kEsz;
  const int lane_off = r32 * rowbytes + h * Op::kEpl * Op::kEsz;
  const int nkb = A.nkb;

  // wave cursor: position index pi (pair view v), query tile qt, chunk ch of nch
  int pi = 0;
  int qt = 0, ch = 0;
  PairView v = uniform_view(A.lay.get(first));
  int nch = v.td > 0 ? (v.td + kTile - 1) / kTile : 1;

  Chunk<Op, NKB> bufA, bufB;
  QTile<Op, NKB> q;
  const char* q_src = nullptr;
  int q_qt = -1;
  float mx = -INFINITY, score = 0.0f;
  int slot = -1;

  load_chunk<Op, NKB>(bufA, v, 0, nkb, rowbytes, lane_off, r32);

  // One step: make sure the query tile is resident, prefetch the next chunk
  // into `nxt`, multiply `cur`, fold it into the running max, and close the
  // tile / pair when this was its last chunk.  Returns false after the
  // wave's final chunk.
  auto step = [&](Chunk<Op, NKB>& cur, Chunk<Op, NKB>& nxt) -> bool {
    // Row validity of `cur` first: its mask byte is the last load of the
    // previous step, so this waits for `cur` (needed next anyway) and for
    // nothing issued in this step.
    const uint32_t m32 = chunk_rows_valid(v, ch, r32, cur.mbyte);
    if (ch == 0 && (v.q != q_src || qt != q_qt)) {
      load_qtile<Op, NKB>(q, v, qt, nkb, rowbytes, lane_off, r32);
      q_src = v.q;
      q_qt = qt;
    }
    // advance a copy of the cursor and prefetch its chunk
    int npi = pi;
    int nqt_i = qt, nch_i = ch + 1, nnch = nch;
    PairView nv = v;
    if (nch_i >= nch) {
      nch_i = 0;
      if (++nqt_i >= A.nqt) {
        nqt_i = 0;
        ++npi;
        // The layouts read idx / order / cu with unchecked scalar loads; the
        // position stays valid even if such a load is speculated.
        const int64_t kpos = first + (int64_t)(npi < cnt ? npi : pi) * stride;
        if (npi < cnt) {
          nv = uniform_view(A.lay.get(kpos));
          nnch = nv.td > 0 ? (nv.td + kTile - 1) / kTile : 1;
        }
      }
    }
    const bool more = npi < cnt;
    // Unconditional: after the wave's last chunk it re-reads the current one
    // (an L2 hit), so every step issues the same loads and the MFMAs below
    // wait only for the chunk they multiply.
    load_chunk<Op, NKB>(nxt, more ? nv : v, more ? nch_i : ch, nkb, rowbytes, lane_off, r32);
    // Keep the prefetch ahead of the MFMAs: the scheduler would otherwise
    // sink the independent loads below them and nothing would overlap.
    __builtin_amdgcn_sched_barrier(0);

    Acc acc = {};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) acc = Op::mma(cur.a[kb], q.f[kb], acc);
    float s[16];
    acc_to_scores<Op>(acc, q.qscale, cur.ds, h, s);
    take_first_row(s, m32, h, ch, mx, slot);
    update_chunk(s, m32, h, ch, mx, slot);

    if (ch == nch - 1) {
      // The empty asm pins the query-mask test here: hoisted next to its
      // load, it would make the compiler wait for the whole prefetch.
      uint32_t qmb = q.mbyte;
      asm volatile("" : "+v"(qmb));
      const bool tvalid = q.t < v.tq && mask_ok(v.qm, qmb);
      score += finish_tile(A, v.out, qt, r32, h, tvalid, mx, slot);
      mx = -INFINITY;
      slot = -1;
      if (qt == A.nqt - 1) {
        write_score(A, v, score, lane);
        score = 0.0f;
      }
    }
    pi = npi; qt = nqt_i; ch = nch_i; nch = nnch; v = nv;
    return more;
  };

  while (step(bufA, bufB) && step(bufB, bufA)) {
  }
}

// ---- split-d kernel: fms_split.hpp (its own translation units) ----------------------

// k-blocks per split-d batch: 128 bytes of each operand per lane per step.
template <class Op>
constexpr int split_kbat() {
  return 128 / (Op::kEpl * Op::kEsz);
}

template <class Op, class L>
hipError_t launch_split(const ScanArgs<L>& A, dim3 grid, dim3 block, hipStream_t stream);

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
  int64_t first, stride;
  int cnt;
  wave_positions(A, first, stride, cnt);
  const int dim = A.dim;
  const int rowbytes = dim * Op::kEsz;

  for (int pi = 0; pi < cnt; ++pi) {
    const PairView v = uniform_view(A.lay.get(first + pi * stride));
    const int nch = v.td > 0 ? (v.td + kTile - 1) / kTile : 1;
    const rsrc_t rq = make_rsrc_u(v.q, (uint32_t)v.tq * (uint32_t)rowbytes);
    const rsrc_t rd = make_rsrc_u(v.d, (uint32_t)v.td * (uint32_t)rowbytes);
    float score = 0.0f;
    for (int qt = 0; qt < A.nqt; ++qt) {
      const int t = qt * kTile + r32;
      uint32_t mb = 1u;
      if (v.qm) mb = buf_load1(make_rsrc_u(v.qm, (uint32_t)v.tq), t);
      const bool tvalid = (t < v.tq) && (mb != 0u);
      float qscale = 0.0f;
      if constexpr (Op::kInt) qscale = load_qscale(v, t);
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
        if (v.dm) mbyte = buf_load1(make_rsrc_u(v.dm, (uint32_t)v.td), row);
        float ds[1];
        load_ds<Op>(ds, v, ch, r32);
        float s[16];
        acc_to_scores<Op>(acc, qscale, ds, h, s);
        const uint32_t m32 = chunk_rows_valid(v, ch, r32, mbyte);
        take_first_row(s, m32, h, ch, mx, slot);
        update_chunk(s, m32, h, ch, mx, slot);
      }
      score += finish_tile(A, v.out, qt, r32, h, tvalid, mx, slot);
    }
    write_score(A, v, score, lane);
  }
}

// ---- host-side launcher -------------------------------------------------------------

// Fast-kernel instantiation for a given nkb (k-blocks per token); 0 = none,
// use the generic kernel.  16-bit features: dim 64 / 128 / 256; int8: dim
// 64 / 128 / 256; fp32 always uses the generic kernel.
template <class Op>
constexpr int fast_nkb(int nkb) {
  if (Op::kEsz == 4) return 0;
  const int b = (Op::kKb == 16) ? 4 : 2;
  return (nkb == b || nkb == 2 * b || nkb == 4 * b) ? nkb : 0;
}



template <class Op, class L>
hipError_t launch_scan(const L& lay, int dim, int rows, int64_t npairs, int32_t* args,
                       float* partial, float* scores, float neg, bool norm, bool vec,
                       hipStream_t stream) {
  ScanArgs<L> A;
  A.lay = lay;
  A.dim = dim;
  A.nkb = (dim + Op::kKb - 1) / Op::kKb;
  A.rows = rows;
  A.nqt = rows > 0 ? (rows + kTile - 1) / kTile : 1;
  A.ppw = pairs_per_wave(npairs);
  A.npairs = npairs;
  A.args = args;
  A.partial = partial;
  A.scores = scores;
  A.neg = neg;
  A.norm = norm ? 1 : 0;
  const int64_t waves = (npairs + A.ppw - 1) / A.ppw;
  const dim3 grid((unsigned)((waves + kWaves - 1) / kWaves));
  const dim3 block(64 * kWaves);
  const bool fast_ok = vec && (dim % Op::kKb == 0) && dim > 0;
  const int nkb_fast = fast_ok ? fast_nkb<Op>(A.nkb) : 0;
  if constexpr (Op::kEsz != 4) {
    constexpr int b = (Op::kKb == 16) ? 4 : 2;
    if (nkb_fast == b) {
      hipLaunchKernelGGL((scan_fast<Op, L, b>), grid, block, 0, stream, A);
      return hipGetLastError();
    }
    if (nkb_fast == 2 * b) {
      hipLaunchKernelGGL((scan_fast<Op, L, 2 * b>), grid, block, 0, stream, A);
      return hipGetLastError();
    }
    if (nkb_fast == 4 * b) {
      hipLaunchKernelGGL((scan_fast<Op, L, 4 * b>), grid, block, 0, stream, A);
      return hipGetLastError();
    }
  }
  // Split-d: any dim that is a whole number of KBAT-k-block batches.
  constexpr int kbat = split_kbat<Op>();
  if (vec && dim > 0 && dim % (kbat * Op::kKb) == 0) return launch_split<Op, L>(A, grid, block, stream);
  if (vec) {
    hipLaunchKernelGGL((scan_generic<Op, L, true>), grid, block, 0, stream, A);
  } else {
    hipLaunchKernelGGL((scan_generic<Op, L, false>), grid, block, 0, stream, A);
  }
  return hipGetLastError();
}

}  // namespace fms
