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
  char* qfrag;              // scan_runs_lds: query tiles in fragment order (nullable)
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

// ---- the same scan with the chunk stream in LDS (16-bit features) -------------------
//
// scan_runs loads each chunk straight into MFMA fragment registers: one
// 16-byte load per lane and k-block, lane l reading row l%32, so every load
// instruction touches 32 cache lines (32 bytes of each), and the vector
// memory pipeline, not HBM, sets the pace.  scan_runs_lds instead copies
// every chunk HBM/L2 -> LDS by direct buffer-to-LDS loads that each read
// 1 KB of whole rows (R = 64/U consecutive rows of U 16-byte units: 8 cache
// lines), two steps ahead into one of two LDS slots per wave, so the chunks
// of steps i+1 and i+2 are in flight while step i multiplies.  A load lands
// lane-major (lane l's 16 bytes at l*16), so the unit a lane fetches is
// chosen to leave the slot row-major with each row's units XOR-swizzled:
// unit u of row r sits at r*U + (u ^ key(r)), key(r) = (r / (16/U)) % U.
// The fragment reads (lane L: row L%32, unit 2kb + L/32) then fall on 16
// distinct 16-byte bank groups for any 16 consecutive lanes (no LDS bank
// conflicts); each lane keeps its NKB read addresses in registers.  The
// rows' mask bytes follow as one byte load per lane (lane l: row l%32),
// which lands as a dword at lane*4 after the fragments.  Batches, pair
// arithmetic and fold are exactly scan_runs': the results are bit-identical.
//
// Waits.  The compiler does not order the copies against the slot reads, so
// the reads are inline asm that completes on return, after an explicit
// vmcnt wait that leaves only the most recent copy group (the next step's)
// in flight: loads complete in issue order, so that finds this step's copy
// in LDS whatever was issued between (stores of a closed tile, query tiles),
// which can only make it wait longer.  The slot is refilled after the read
// has completed.  The query tiles of a (batch, tile) are loaded after the
// previous tile's last MFMAs, outside the per-chunk loop, so only a tile's
// first step waits for them: the chunk loop carries no register load at all.

// Units of 16 bytes per row and the swizzle key of row r (16-bit features,
// NKB k-blocks of 32 bytes per row).
template <int NKB>
__device__ __forceinline__ constexpr int lds_units() {
  return 2 * NKB;
}
template <int NKB>
__device__ __forceinline__ int lds_key(int r) {
  constexpr int U = lds_units<NKB>();
  return (r / (16 / U)) % U;
}

// The NKB fragments (lane address addr[kb] + kOff) and the row mask dword
// (maddr + kOff) of one chunk slot, complete on return.
template <int NKB, int kOff>
__device__ __forceinline__ void lds_read_chunk(u32x4 (&a)[NKB], uint32_t& mrow,
                                               const uint32_t (&addr)[NKB], uint32_t maddr);

template <int kOff>
__device__ __forceinline__ void lds_read_chunk4(u32x4 (&a)[4], uint32_t& mrow,
                                                const uint32_t (&ad)[4], uint32_t maddr) {
  asm volatile(
      "ds_read_b128 %0, %5 offset:%10\n\t"
      "ds_read_b128 %1, %6 offset:%10\n\t"
      "ds_read_b128 %2, %7 offset:%10\n\t"
      "ds_read_b128 %3, %8 offset:%10\n\t"
      "ds_read_b32 %4, %9 offset:%10\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(a[0]), "=&v"(a[1]), "=&v"(a[2]), "=&v"(a[3]), "=&v"(mrow)
      : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3]), "v"(maddr), "n"(kOff)
      : "memory");
}

template <int kOff>
__device__ __forceinline__ void lds_read_chunk8(u32x4 (&a)[8], uint32_t& mrow,
                                                const uint32_t (&ad)[8], uint32_t maddr) {
  asm volatile(
      "ds_read_b128 %0, %9 offset:%18\n\t"
      "ds_read_b128 %1, %10 offset:%18\n\t"
      "ds_read_b128 %2, %11 offset:%18\n\t"
      "ds_read_b128 %3, %12 offset:%18\n\t"
      "ds_read_b128 %4, %13 offset:%18\n\t"
      "ds_read_b128 %5, %14 offset:%18\n\t"
      "ds_read_b128 %6, %15 offset:%18\n\t"
      "ds_read_b128 %7, %16 offset:%18\n\t"
      "ds_read_b32 %8, %17 offset:%18\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(a[0]), "=&v"(a[1]), "=&v"(a[2]), "=&v"(a[3]), "=&v"(a[4]), "=&v"(a[5]),
        "=&v"(a[6]), "=&v"(a[7]), "=&v"(mrow)
      : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3]), "v"(ad[4]), "v"(ad[5]), "v"(ad[6]),
        "v"(ad[7]), "v"(maddr), "n"(kOff)
      : "memory");
}

template <int NKB, int kOff>
__device__ __forceinline__ void lds_read_chunk(u32x4 (&a)[NKB], uint32_t& mrow,
                                               const uint32_t (&addr)[NKB], uint32_t maddr) {
  static_assert(NKB == 4 || NKB == 8, "d = 64 or 128");
  if constexpr (NKB == 4) lds_read_chunk4<kOff>(a, mrow, addr, maddr);
  else lds_read_chunk8<kOff>(a, mrow, addr, maddr);
}

// Wait until at most kVm of this wave's vector memory operations are
// outstanding.
template <int kVm>
__device__ __forceinline__ void vm_wait() {
  static_assert(kVm >= 0 && kVm < 64, "vmcnt field");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kVm) : "memory");
}

// Query tiles in MFMA fragment order (scan_runs_lds with RunArgs.qfrag):
// tile (b, qt) of query b is NKB blocks of 1 KB, block kb holding lane l's
// fragment -- token qt*32 + l%32, 16-byte unit 2kb + l/32 -- at l*16, tokens
// past Tq zero.  Loading a tile is then NKB loads of 1 KB each (8 cache
// lines) instead of NKB loads that each touch 32 token rows.  One thread per
// 16-byte unit; Q rows are 16-byte aligned (the fast dims).
template <int NKB>
__global__ void __launch_bounds__(256) query_frag_kernel(const char* Q, int Tq, int rowbytes,
                                                         int nqt, int64_t nunits, u32x4* out) {
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= nunits) return;
  const int lane = (int)(g & 63);
  const int kb = (int)((g >> 6) % NKB);
  const int64_t tile = (g >> 6) / NKB;
  const int64_t b = tile / nqt;
  const int qt = (int)(tile - b * nqt);
  const int t = qt * kTile + (lane & 31);
  u32x4 v = u32x4{0u, 0u, 0u, 0u};
  if (t < Tq)
    v = *reinterpret_cast<const u32x4*>(Q + (b * Tq + t) * (int64_t)rowbytes +
                                        (2 * kb + (lane >> 5)) * 16);
  out[g] = v;
}

// Bytes of the fragment-ordered query tiles of B queries (0 when the
// document-batch scan of this Op and dim does not stream through LDS).
template <class Op>
inline size_t runs_qfrag_bytes(int dim, int Tq, int64_t B) {
  if (Op::kInt || Op::kEsz != 2 || dim % Op::kKb != 0) return 0;
  const int nkb = dim / Op::kKb;
  if (nkb != 4 && nkb != 8) return 0;
  const int64_t nqt = Tq > 0 ? (Tq + kTile - 1) / kTile : 1;
  return (size_t)B * (size_t)nqt * (size_t)nkb * 1024u;
}

// One query tile of a pair from the fragment-ordered copy (`tile`, NKB KB;
// a pair without a query reads a zero-size resource: zeros), with the same
// token and mask state as load_qtile.
template <class Op, int NKB>
__device__ __forceinline__ void load_qtile_frag(QTile<Op, NKB>& q, const PairView& v,
                                                const char* tile, int qt, int lane, int r32) {
  const rsrc_t rq = make_rsrc_u(tile, v.tq > 0 ? (uint32_t)(NKB * 1024) : 0u);
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) q.f[kb] = Op::load(rq, kb * 1024 + lane * 16);
  q.t = qt * kTile + r32;
  const bool has_m = v.qm != nullptr;
  q.mbyte = buf_load1(make_rsrc_u(has_m ? (const void*)v.qm : (const void*)tile,
                                  has_m ? (uint32_t)v.tq : 0u),
                      q.t);
  q.qscale = 0.0f;
}

// A stream position of scan_runs_lds: batch (k, j, kb), query tile qt,
// chunk ch of nch, and the batch's document view.
struct RunCursor {
  int64_t k;
  int j, kb, qt, ch, nch;
  PairView dv;
};

// The byte offset, within a chunk, of the 16-byte unit that lane `lane`
// copies in load i of a chunk: row R*i + lane/U, the unit that lands at slot
// position lane%U of that row's swizzle.
template <int NKB>
__device__ __forceinline__ int lds_copy_offset(int i, int lane, int rowbytes) {
  constexpr int U = lds_units<NKB>(), R = 64 / U;
  const int row = R * i + lane / U;
  return row * rowbytes + ((lane % U) ^ lds_key<NKB>(row)) * 16;
}

// Copy the chunk at stream position c into the LDS slot at `base`: NKB
// loads of R whole rows each (lane offsets `off`, from lds_copy_offset,
// relative to a resource that starts at the chunk and ends with the
// document, so rows past it read 0), then the mask byte of chunk row l%32
// into the slot's mask dwords (base + NKB*64; a zero-size resource without
// a mask).  The fragment copies are non-temporal: every 128-byte line of
// the chunk is read by exactly one of them, and the query tiles the scan
// re-reads then stay in L2.  A device function rather than a lambda: a
// buffer resource local to a lambda keeps the host compile from emitting
// the kernel's launch stub.
template <class Op, int NKB>
__device__ __forceinline__ void copy_chunk_lds(const RunCursor& c, typename Op::Frag* base,
                                               const int* off, int rowbytes, int lane) {
  typedef __attribute__((address_space(3))) void* lds_void_t;
  const int chunk0 = c.ch * kTile;
  const int rows = c.dv.td - chunk0;
  const rsrc_t rd = make_rsrc(c.dv.d + (int64_t)chunk0 * rowbytes,
                              rows > 0 ? (uint32_t)rows * (uint32_t)rowbytes : 0u);
#pragma unroll
  for (int i = 0; i < NKB; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rd, (lds_void_t)(base + i * 64), 16, off[i], 0, 0,
                                             /*nt*/ 2);
  const bool has_m = c.dv.dm != nullptr;
  const rsrc_t rm = make_rsrc(has_m ? (const void*)c.dv.dm : (const void*)c.dv.d,
                              has_m ? (uint32_t)c.dv.td : 0u);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rm, (lds_void_t)(base + NKB * 64), 1,
                                           chunk0 + (lane & 31), 0, 0, 0);
}

template <class Op, int NKB, int KQ, bool kQF>
__global__ void __launch_bounds__(64 * kWaves, 2) scan_runs_lds(const RunArgs A) {
  typedef RunCursor Cur;
  typedef typename Op::Acc Acc;
  typedef typename Op::Frag Frag;
  static_assert(sizeof(Frag) == 16 && !Op::kInt, "16-bit feature fragments");
  constexpr int kFr = NKB * 64;                 // fragments per chunk
  constexpr int kSlot = kFr + 16;               // + 256 bytes of row mask dwords
  constexpr uint32_t kSlotBytes = kSlot * 16;
  constexpr int kGroup = NKB + 1;               // copies per chunk
  __shared__ Frag ring[kWaves][2][kSlot];

  const int lane = threadIdx.x & 63, r32 = lane & 31, h = lane >> 5;
  const int wib = uniform((int)(threadIdx.x >> 6));
  const int64_t P = A.npairs;
  const int64_t w = (int64_t)blockIdx.x * kWaves + wib;
  const int64_t s0 = w * A.ppw;
  if (s0 >= P) return;
  const int64_t e0 = s0 + A.ppw < P ? s0 + A.ppw : P;

  // First batch start at or after s0 (as scan_runs).
  int64_t k0;
  {
    int64_t rs, re;
    run_bounds(A, sload(&A.order[s0].j, 0), rs, re);
    const int64_t off = s0 - rs;
    k0 = (off % KQ == 0) ? s0 : rs + (off / KQ + 1) * KQ;
    if (k0 > re) k0 = re;
  }
  if (k0 >= e0) return;

  const int rowbytes = A.dim * Op::kEsz;
  const int lane_off = r32 * rowbytes + h * Op::kEpl * Op::kEsz;
  const int nkb = A.nkb;
  // This lane's fragment addresses in slot 0 (slot 1 is kSlotBytes further).
  const uint32_t lds_wave = (uint32_t)reinterpret_cast<uintptr_t>(
      (const __attribute__((address_space(3))) void*)&ring[wib][0][0]);
  uint32_t raddr[NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
    raddr[kb] = lds_wave +
                (uint32_t)(r32 * lds_units<NKB>() + ((2 * kb + h) ^ lds_key<NKB>(r32))) * 16u;
  const uint32_t lds_mask = lds_wave + (uint32_t)kFr * 16u + (uint32_t)lane * 4u;

  auto cur_at = [&](Cur& c, int64_t pos) {
    c.k = pos;
    c.j = sload(&A.order[pos].j, 0);
    int64_t rs, re;
    run_bounds(A, c.j, rs, re);
    c.kb = (int)(re - pos < KQ ? re - pos : KQ);
    doc_view(A, c.j, c.dv);
    c.dv = uniform_view(c.dv);
    c.nch = c.dv.td > 0 ? (c.dv.td + kTile - 1) / kTile : 1;
    c.qt = 0;
    c.ch = 0;
  };
  // The next step of the stream; false (and c unchanged) after the last.
  auto cur_next = [&](Cur& c) -> bool {
    if (c.ch + 1 < c.nch) {
      ++c.ch;
      return true;
    }
    if (c.qt + 1 < A.nqt) {
      ++c.qt;
      c.ch = 0;
      return true;
    }
    const int64_t nk = c.k + c.kb;
    if (nk >= e0) return false;
    cur_at(c, nk);
    return true;
  };
  Frag* const wave_ring = &ring[wib][0][0];
  int coff[NKB];  // this lane's copy offsets within a chunk
#pragma unroll
  for (int i = 0; i < NKB; ++i) coff[i] = lds_copy_offset<NKB>(i, lane, rowbytes);
  auto copy_chunk = [&](const Cur& c, Frag* base) {
    copy_chunk_lds<Op, NKB>(c, base, coff, rowbytes, lane);
  };

  Cur C, L;
  cur_at(C, k0);
  L = C;
  copy_chunk(L, wave_ring);
  bool lmore = cur_next(L);
  copy_chunk(L, wave_ring + kSlot);  // (re-reads the first chunk when the stream has one step)
  if (lmore) lmore = cur_next(L);

  auto pair_id = [&](int i) { return i < C.kb ? sload(&A.order[C.k + i].p, 0) : -1; };
  QTile<Op, NKB> q[KQ];
  float mx[KQ], score[KQ];
  int slot[KQ];
#pragma unroll
  for (int i = 0; i < KQ; ++i) { mx[i] = -INFINITY; slot[i] = -1; score[i] = 0.0f; }
  auto load_queries = [&]() {
#pragma unroll
    for (int i = 0; i < KQ; ++i) {
      const int p = pair_id(i);
      PairView qv = C.dv;
      query_view(A, p, qv);
      if constexpr (kQF) {
        const int64_t b = p >= 0 ? (int64_t)((uint32_t)p / (uint32_t)A.lay.C) : 0;
        const char* tile = A.qfrag + (b * A.nqt + C.qt) * (int64_t)(NKB * 1024);
        load_qtile_frag<Op, NKB>(q[i], uniform_view(qv), tile, C.qt, lane, r32);
      } else {
        load_qtile<Op, NKB>(q[i], uniform_view(qv), C.qt, nkb, rowbytes, lane_off, r32);
      }
    }
  };

  int par = 0;  // slot of the current step
  // One step: read the slot, refill it two steps ahead, multiply and fold
  // every pair of the batch, close the tile at its last chunk.  Returns
  // whether the stream has a next step (C then points at it).
  auto run_step = [&]() -> bool {
    vm_wait<kGroup>();  // this step's copy group has landed
    Frag a[NKB];
    uint32_t mbyte;
    if (par)
      lds_read_chunk<NKB, (int)kSlotBytes>(a, mbyte, raddr, lds_mask);
    else
      lds_read_chunk<NKB, 0>(a, mbyte, raddr, lds_mask);
    const uint32_t m32 = chunk_rows_valid(C.dv, C.ch, r32, mbyte);
    copy_chunk(L, wave_ring + par * kSlot);
    if (lmore) lmore = cur_next(L);
    __builtin_amdgcn_sched_barrier(0);

#pragma unroll
    for (int i = 0; i < KQ; ++i) {
      if (i < C.kb) {
        Acc acc = {};
#pragma unroll
        for (int kk = 0; kk < NKB; ++kk) acc = Op::mma(a[kk], q[i].f[kk], acc);
        float s[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = acc[r];
        take_first_row(s, m32, h, C.ch, mx[i], slot[i]);
        if (m32 == 0xffffffffu)
          fold_tree<true>(s, C.ch * 16, mx[i], slot[i]);
        else
          update_chunk(s, m32, h, C.ch, mx[i], slot[i]);
      }
    }
    if (C.ch == C.nch - 1) {
#pragma unroll
      for (int i = 0; i < KQ; ++i) {
        if (i < C.kb) {
          PairView pv = C.dv;
          query_view(A, pair_id(i), pv);
          pv = uniform_view(pv);
          uint32_t qmb = q[i].mbyte;
          asm volatile("" : "+v"(qmb));
          const bool tvalid = q[i].t < pv.tq && mask_ok(pv.qm, qmb);
          score[i] += finish_tile(A, pv.out, C.qt, r32, h, tvalid, mx[i], slot[i]);
          mx[i] = -INFINITY;
          slot[i] = -1;
          if (C.qt == A.nqt - 1) {
            write_score(A, pv, score[i], lane);
            score[i] = 0.0f;
          }
        }
      }
    }
    par ^= 1;
    return cur_next(C);
  };

  // Per (batch, query tile): its queries, its first step (which waits for
  // them), then its other chunks.
  for (;;) {
    load_queries();
    bool more = run_step();
    while (more && C.ch != 0) more = run_step();
    if (!more) break;
  }
  // No copy into LDS may outlive the wave.
  vm_wait<0>();
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
