// fms_inbatch_split.hip -- InBatch() MaxSim with the feature dimension split
// into K slices, for query tiles that do not fit in registers: 16-bit
// features of any dim that is a multiple of 8 other than 32, 64, 96, 128
// (those run the register-resident kernel of fms_inbatch.hip), and fp32
// features of any dim that is a multiple of 4.
//
// S[j, i] = sum_t max_u <Q_i[t], D_j[u]> (forward_layouts.jl:202-225, where
// the reference materialises D'Q chunks and runs an argmax-accumulate); the
// same fused scores and argmax tape as the other in-batch kernel.
//
// Work item = one document j x kRows query rows (a query row is a 32-token
// tile of a query: query v / ntq, tokens 32 (v % ntq) ..).  Blocks of 4
// waves, one per CU for 16-bit features and two for fp32, each walk their
// items in turn (a persistent grid).  An item's document chunks are taken
// kCg at a time (a chunk group: 6 chunks for 16-bit features, 3 for fp32);
// per group the block runs the whole K loop:
//   * K advances by a slice of 128 bytes of every row (64 features of a
//     16-bit type, 32 of fp32).  The document's slice (shared by the four
//     waves) goes HBM/L2 -> LDS with direct buffer-to-LDS loads (no
//     registers in between), in MFMA fragment order: 1 KB per (chunk, unit
//     pair m), lane l's 16 bytes at l * 16 = row l % 32, 16-byte unit
//     2m + l / 32 of the slice, so a fragment read is 1 KB contiguous over
//     the wave (no bank conflicts).  A wave's own query rows' fragments are
//     loaded straight into registers in the same order.  Rows past the
//     document or the query, and units past the row (the last slice of a
//     dim that is not a multiple of it) read zeros (buffer bounds);
//   * the block's slices (items, their groups, their K slices, in order)
//     form one stream with three stages: slice task p + 2 is requested
//     while task p is multiplied, across group and item boundaries, so an
//     item's first slices arrive while the previous item folds and closes;
//     one barrier per task (every wave's share of task p has landed, and
//     every wave is done with the stage task p - 1 used, which the request
//     of task p + 2 then refills);
//   * wave w holds the accumulators of query rows 2w, 2w + 1 for the whole
//     chunk group (2 x kCg 32x32 tiles): each query fragment read feeds kCg
//     MFMA chains and each document fragment read two;
//   * 16-bit: one v_mfma_f32_32x32x16 per unit pair.  fp32: the 16 bytes of
//     a unit pair are four k-blocks of v_mfma_f32_32x32x2f32; dword e of
//     the lanes of half h is feature 8m + 4h + e of the slice, the same
//     bijection for both operands, so the four MFMAs sum the 8 features of
//     the unit pair;
//   * after a group's last slice each accumulator tile is folded, chunk by
//     chunk in document order, into the running max / argmax exactly as the
//     scans fold (first valid row taken, then strictly greater; chunk valid
//     words from a plan kernel over dmask and Td), and the item's last group
//     closes the tiles: wave halves merged, tape rows and the score written
//     straight to global memory.
// Item -> (document, query group) is XCD-aware: each XCD takes every 8th
// document, in bands of kBand documents; within a band the document runs
// fastest, so the XCD's 32 CUs hold kBand documents x 32 / kBand query groups
// at a time, and the band's documents stay in that XCD's L2 while all query
// groups pass over them.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <algorithm>
#include <atomic>

#include "fms_device.hpp"
#include "fms_group.hpp"
#include "fms_inbatch_split.hpp"
#include "fms_scan.hpp"

namespace fms {

namespace {

constexpr int kSpWaves = 4;
constexpr int kRows = 2 * kSpWaves;     // query rows per block (two per wave)
constexpr int kSliceBytes = 128;        // bytes of every row per K step
constexpr int kPairs = kSliceBytes / 32;  // unit pairs per slice (4)
constexpr int kStages = 3;              // document slice stages in LDS (2 slices ahead)
static_assert(kTile == 8 * kSpWaves, "every wave copies 8 whole rows of each chunk");
constexpr int kQLoads = 2 * kPairs;     // query fragment loads per slice and wave

// The chunk group per element size.  kCg document chunks per group, kBlocks
// blocks per CU.  16-bit: six chunks, one block (a wave holds 12 accumulator
// tiles and its query fragments in about 424 registers).  fp32: three
// chunks, two blocks (256 registers): its MFMAs take 8 times as long per
// byte, so a second wave per SIMD covers the first one's per-slice work
// (measured at the C3 shape: 3.55 -> 3.39 ms), while for 16-bit features the
// halved reuse of each query fragment costs more than that (2.85 -> 3.71 ms).
template <int kEsz>
struct SplitShape {
  static constexpr int kCg = kEsz == 4 ? 3 : 6;
  static constexpr int kBlocks = kEsz == 4 ? 2 : 1;
  static constexpr int kDFrags = kCg * kPairs;  // 1 KB blocks of a document slice
  // Vector memory operations per slice and wave: kCg document copies into
  // LDS, then the query fragment loads into registers.
  static constexpr int kOpsPerSlice = kCg + kQLoads;
  // Issued after a slice's document copies by the time that slice is read:
  // its own query loads and the two slices requested since.
  static constexpr int kAfterCopies = kQLoads + (kStages - 2) * kOpsPerSlice;
  static_assert(kAfterCopies < 64, "vmcnt field");
};
constexpr int kMaxCg = SplitShape<2>::kCg;  // the largest group (range checks)
static_assert(SplitShape<4>::kCg <= kMaxCg, "range checks cover every shape");
constexpr int kSpXcds = 8;
constexpr int kBand = 8;  // documents an XCD keeps in flight together

// The block's waves have all landed their loads of the slice to be read next
// (each leaves only its kVm most recent loads in flight) and finished their
// LDS accesses; the asm statements keep the compiler from moving LDS
// accesses across.
template <int kVm>
__device__ __forceinline__ void slice_barrier() {
  static_assert(kVm >= 0 && kVm < 64, "vmcnt field");
  asm volatile("" ::: "memory");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(kVm) : "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// acc += the products of one unit pair (16 bytes per lane of each operand):
// kMmaPerPair MFMAs.
template <class Op>
__device__ __forceinline__ typename Op::Acc mma_pair(u32x4 a, u32x4 b, typename Op::Acc acc) {
  if constexpr (Op::kEsz == 4) {
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = Op::mma(a[e], b[e], acc);
    return acc;
  } else {
    return Op::mma(a, b, acc);
  }
}

// Valid-row words of the call, one launch before the scan: plan[j * nch + c]
// bit r = row 32c + r of document j is below Td and unmasked; plan[ndw + v]
// bit r = token 32 (v % ntq) + r of query v / ntq is below Tq and unmasked.
// The scan reads them with scalar loads (a wave-uniform word per chunk or
// query row), which leaves the vector-memory counter to the slice stream.
__global__ void __launch_bounds__(256) split_plan_kernel(const uint8_t* dm, const uint8_t* qm,
                                                         int Bd, int Td, int nch, int Bq, int Tq,
                                                         int ntq, uint32_t* plan) {
  const int64_t ndw = (int64_t)Bd * nch, total = ndw + (int64_t)Bq * ntq;
  const int lane = threadIdx.x & 63;
  // two words per wave and pass: lanes 0..31 word w, lanes 32..63 word w + 1
  for (int64_t w = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 2; w < total;
       w += (int64_t)gridDim.x * 8) {
    const int64_t wi = w + (lane >> 5);
    bool bit = false;
    if (wi < ndw) {
      const int64_t j = wi / nch;
      const int row = (int)(wi - j * nch) * kTile + (lane & 31);
      bit = row < Td && (dm == nullptr || dm[j * Td + row] != 0);
    } else if (wi < total) {
      const int64_t v = wi - ndw, i = v / ntq;
      const int t = (int)(v - i * ntq) * kTile + (lane & 31);
      bit = t < Tq && (qm == nullptr || qm[i * Tq + t] != 0);
    }
    const uint64_t b = __ballot(bit);
    if ((lane & 31) == 0 && wi < total) plan[wi] = (uint32_t)(b >> (lane & 32));
  }
}

// Slot x of the block order -> (document, query group).  Slots are dealt
// round-robin to the 8 XCDs (slot x runs on XCD x % 8: the grid is a multiple
// of 8 and each block walks slots blockIdx.x + n * gridDim.x); XCD x serves
// documents 8 dl + x, dl < ndx, in bands of kBand consecutive dl: inside a
// band dl runs fastest, then the query group.  A document index >= Bd marks
// a slot with no work (the last band when Bd is not a multiple of 8).
__device__ __forceinline__ int split_slot_doc(int x, int nqg, int ndx, int& qg) {
  const int xcd = x % kSpXcds, kx = x / kSpXcds;
  const int band = kx / (kBand * nqg);
  const int bsz = std::min(kBand, ndx - band * kBand);
  const int within = kx - band * kBand * nqg;
  qg = within / bsz;
  return (band * kBand + within % bsz) * kSpXcds + xcd;
}

// kWhole: rows are whole slices (rowbytes a multiple of kSliceBytes, as at
// d = 768 in 16 bits or d = 128 in fp32), so no unit lies past a row's end
// and the slice's byte offset goes to the loads' scalar offset.
template <class Op, bool kWhole>
__global__ void __launch_bounds__(64 * kSpWaves, SplitShape<Op::kEsz>::kBlocks)
    inbatch_split(const InBatchSplitArgs A) {
  typedef typename Op::Acc Acc;
  typedef SplitShape<Op::kEsz> Shape;
  constexpr int kCg = Shape::kCg, kDFrags = Shape::kDFrags, kAfterCopies = Shape::kAfterCopies;
  constexpr int kMmaPerPair = Op::kEsz == 4 ? 4 : 1;
  typedef __attribute__((address_space(3))) void* lds_void_t;
  __shared__ u32x4 dbuf[kStages][kDFrags * 64];

  const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
  const int r32 = lane & 31, h = lane >> 5;

  const int rowbytes = A.rowbytes, Tq = A.Tq, Td = A.Td, ntq = A.ntq, Bd = A.Bd, nqg = A.nqg;
  const int nslices = (rowbytes + kSliceBytes - 1) / kSliceBytes;
  const int nch = Td > 0 ? (Td + kTile - 1) / kTile : 0;
  const int ngroups = (nch + kCg - 1) / kCg;
  const int nqv = A.Bq * ntq;
  const int ndx = (Bd + kSpXcds - 1) / kSpXcds;
  const int G = gridDim.x;
  // The plan words are read through the constant address space: scalar
  // loads (wave-uniform words, lgkmcnt), nothing in the vector-memory count
  // that the slice waits rely on.  The kernel never writes them.
  typedef __attribute__((address_space(4))) const uint32_t* cword_ptr;
  const cword_ptr cmask = (cword_ptr)(uintptr_t)A.plan;
  const cword_ptr qmask = cmask + (int64_t)Bd * nch;

  // This block's slots with a document, in order.
  auto next_slot = [&](int x) {
    for (; x < A.nslots; x += G) {
      int qg;
      if (split_slot_doc(x, nqg, ndx, qg) < Bd) break;
    }
    return x;
  };

  // Query rows of a wave for query group qg: query, first token, token count.
  struct Rows {
    int qv[2], qi[2], qt0[2], qtn[2];
  };
  auto rows_of = [&](int qg) {
    Rows R;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int v = qg * kRows + 2 * wave + q;
      const bool live = v < nqv;
      R.qv[q] = live ? v : -1;
      R.qi[q] = live ? v / ntq : 0;
      R.qt0[q] = live ? (v - R.qi[q] * ntq) * kTile : 0;
      R.qtn[q] = live ? std::min(kTile, Tq - R.qt0[q]) : 0;
    }
    return R;
  };

  // ---- the load stream ---------------------------------------------------------
  // A block's work is one sequence of slice tasks: its slots (items) in order,
  // each item its chunk groups in order, each group its K slices.  The stream
  // requests task p + 2 while task p is multiplied, across group and item
  // boundaries, so a new item's first slices arrive while the previous item
  // folds and closes.  Per task and wave: kCg document copies into LDS (the
  // four waves together copy the whole slice), then this wave's own query
  // fragments (2 rows x kPairs unit pairs) into registers, lane l reading
  // row l % 32, unit 2m + l / 32 of the slice.  Rows past the document or
  // query and units past the row read out of range (zeros).  Past the last
  // task the resources are empty: the same operations, no memory traffic.
  // Document copies read whole rows: a wave's copy of chunk c is its rows
  // 8w .. 8w + 7 (1 KB, 8 cache lines), lane l taking row 8w + l / 8 and the
  // unit that leaves the chunk row-major with each row's 8 units
  // XOR-swizzled: unit u of row r at r * 8 + (u ^ key(r)), key(r) =
  // (r / 2) % 8.  The fragment reads (lane: row r32, unit 2m + h) then fall
  // on 16 distinct 16-byte bank groups for any 16 consecutive lanes.
  const int crow = 8 * wave + (lane >> 3);
  const int copy_off = ((lane & 7) ^ ((crow >> 1) & 7)) * 16;
  int roff[kPairs];  // fragment m of a chunk: u32x4 index in the chunk's 4 KB
#pragma unroll
  for (int m = 0; m < kPairs; ++m) roff[m] = r32 * 8 + ((2 * m + h) ^ ((r32 >> 1) & 7));
  int is_slot = next_slot(blockIdx.x), is_g = 0, is_s = 0;
  rsrc_t rdoc, rq[2];
  auto set_issue_item = [&]() {
    if (is_slot < A.nslots) {
      int qg;
      const int j = split_slot_doc(is_slot, nqg, ndx, qg);
      const Rows R = rows_of(qg);
      rdoc = make_rsrc_u(A.D + (int64_t)j * Td * rowbytes, (uint32_t)Td * (uint32_t)rowbytes);
#pragma unroll
      for (int q = 0; q < 2; ++q)
        rq[q] = make_rsrc_u(A.Q + ((int64_t)R.qi[q] * Tq + R.qt0[q]) * rowbytes,
                            (uint32_t)R.qtn[q] * (uint32_t)rowbytes);
    } else {
      rdoc = make_rsrc_u(A.D, 0u);
      rq[0] = rq[1] = make_rsrc_u(A.Q, 0u);
    }
  };
  set_issue_item();
  // Query fragments of kStages tasks in flight: set k holds tasks 3n + k.
  u32x4 qf[kStages][2][kPairs];
  auto issue = [&](auto SETc) {
    constexpr int kSet = decltype(SETc)::value;
    // A unit past the row end is pushed out of range with all low 31 bits set
    // (branch-free: a select here became divergent branches around the loads).
    if constexpr (kWhole) {
      const int so = is_s * kSliceBytes;  // uniform: the loads' scalar offset
#pragma unroll
      for (int c = 0; c < kCg; ++c) {
        const int row = (is_g * kCg + c) * kTile + crow;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rdoc, (lds_void_t)&dbuf[kSet][c * 256 + wave * 64],
                                                 16, row * rowbytes + copy_off, so, 0, 0);
      }
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int m = 0; m < kPairs; ++m)
          qf[kSet][q][m] = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq[q], r32 * rowbytes + (2 * m + h) * 16,
                                                           so, 0));
    } else {
      const int so = is_s * kSliceBytes + copy_off;
      const int dpast = -(int)(so >= rowbytes) & 0x7fffffff;
#pragma unroll
      for (int c = 0; c < kCg; ++c) {
        const int row = (is_g * kCg + c) * kTile + crow;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rdoc, (lds_void_t)&dbuf[kSet][c * 256 + wave * 64], 16, (row * rowbytes + so) | dpast,
            0, 0, 0);
      }
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int m = 0; m < kPairs; ++m) {
          const int o = is_s * kSliceBytes + (2 * m + h) * 16;
          const int qpast = -(int)(o >= rowbytes) & 0x7fffffff;
          qf[kSet][q][m] = buf_load16(rq[q], (r32 * rowbytes + o) | qpast);
        }
    }
    if (++is_s == nslices) {
      is_s = 0;
      if (++is_g == ngroups) {
        is_g = 0;
        is_slot = next_slot(is_slot + G);
        set_issue_item();
      }
    }
  };

  // ---- the compute side -----------------------------------------------------------
  int c_slot = next_slot(blockIdx.x), c_g = 0, c_s = 0;
  int j = 0;
  Rows R{};
  auto set_compute_item = [&]() {
    int qg = 0;
    j = c_slot < A.nslots ? split_slot_doc(c_slot, nqg, ndx, qg) : 0;
    R = rows_of(qg);
  };
  set_compute_item();
  float mx[2] = {-INFINITY, -INFINITY};
  int slot[2] = {-1, -1};

  // Close the item's document for both query rows: wave halves merged, tape
  // row and score written straight to global memory.  Both rows' running
  // max starts again for the block's next item, a row past the last query
  // (whose folds saw zeros) included.
  auto close_item = [&]() {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      if (R.qv[q] < 0) {
        mx[q] = -INFINITY;
        slot[q] = -1;
        continue;
      }
      const uint32_t qw = qmask[R.qv[q]];
      const bool tv = ((qw >> r32) & 1u) != 0u;
      int tok = slot_to_token(slot[q], h);
      float m = mx[q];
      merge_halves(m, tok, h);
      const float part = (tv && tok != 0) ? m : 0.0f;
      const int64_t p = (int64_t)R.qi[q] * Bd + j;
      if (A.args && h == 0 && r32 < R.qtn[q]) A.args[p * Tq + R.qt0[q] + r32] = tv ? tok : 0;
      const float score = half_sum(part);
      if (ntq > 1) {
        if (lane == 0) A.St[(int64_t)R.qv[q] * Bd + j] = score;
      } else {
        const float nf = (float)__builtin_popcount(qw);
        const float inv = 1.0f / (nf > 1.0f ? nf : 1.0f);
        if (lane == 0) A.S[p] = A.norm ? score * inv : score;
      }
      mx[q] = -INFINITY;
      slot[q] = -1;
    }
  };

  if (ngroups == 0) {  // Td = 0: every pair scores 0 with an all-zero tape
    for (; c_slot < A.nslots; c_slot = next_slot(c_slot + G)) {
      set_compute_item();
      close_item();
    }
    return;
  }

  int64_t ntasks = 0;  // (items x groups x slices can pass 2^31 at extreme shapes)
  for (int x = c_slot; x < A.nslots; x = next_slot(x + G)) ntasks += (int64_t)ngroups * nslices;
  if (ntasks == 0) return;

  Acc acc[kCg][2];
  uint32_t gmask[kCg];  // the group's chunk words (scalar loads at its first slice)

  // Task p: wait for its copies (exactly kAfterCopies vector operations were
  // issued after them: its own query loads and the whole of task p + 1), a
  // barrier makes every wave's share visible and frees the stage task p - 1
  // read, task p + 2 is requested into that stage and query set, and task p
  // is multiplied; after a group's last slice the group folds, after an
  // item's last group the item closes.  Chunks past the document read zeros:
  // their MFMAs run unguarded and their accumulators are never folded.
  auto step = [&](auto SETc) {
    constexpr int kSet = decltype(SETc)::value;
    slice_barrier<kAfterCopies>();
    issue(std::integral_constant<int, (kSet + 2) % kStages>());
    if (c_s == 0) {
#pragma unroll
      for (int c = 0; c < kCg; ++c) {
        const int ch = std::min(c_g * kCg + c, nch - 1);
        gmask[c] = cmask[(int64_t)j * nch + ch];
      }
    }
    // Document fragments of unit pair m + 1 are read while pair m's MFMAs run
    // (two register sets); a group's first slice starts its accumulators.
    auto multiply = [&](auto FIRSTc) {
      constexpr bool kFirst = decltype(FIRSTc)::value;
      const u32x4* B = &dbuf[kSet][0];
      u32x4 a[2][kCg];
#pragma unroll
      for (int c = 0; c < kCg; ++c) a[0][c] = B[c * 256 + roff[0]];
#pragma unroll
      for (int m = 0; m < kPairs; ++m) {
        if (m + 1 < kPairs) {
#pragma unroll
          for (int c = 0; c < kCg; ++c) a[(m + 1) & 1][c] = B[c * 256 + roff[m + 1]];
        }
#pragma unroll
        for (int c = 0; c < kCg; ++c)
#pragma unroll
          for (int q = 0; q < 2; ++q)
            acc[c][q] = mma_pair<Op>(a[m & 1][c], qf[kSet][q][m],
                                     (kFirst && m == 0) ? Acc{} : acc[c][q]);
      }
      // Schedule: the first pair's reads, then per chunk of each pair one read
      // of the next pair and the chunk's MFMAs (the compiler otherwise puts
      // every read right before its MFMAs and waits for it there).
      __builtin_amdgcn_sched_group_barrier(0x100, kCg, 0);
#pragma unroll
      for (int m = 0; m < kPairs; ++m)
#pragma unroll
        for (int c = 0; c < kCg; ++c) {
          if (m + 1 < kPairs) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 2 * kMmaPerPair, 0);
        }
    };
    if (c_s == 0) multiply(std::true_type());
    else multiply(std::false_type());

    if (++c_s == nslices) {
      c_s = 0;
      // fold the group's chunks in document order
#pragma unroll
      for (int c = 0; c < kCg; ++c) {
        const int ch = c_g * kCg + c;
        if (ch >= nch) continue;
        const uint32_t m32 = gmask[c];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          float s[16];
#pragma unroll
          for (int r = 0; r < 16; ++r) s[r] = acc[c][q][r];
          take_first_row(s, m32, h, ch, mx[q], slot[q]);
          if (m32 == 0xffffffffu)
            fold_tree<true>(s, ch * 16, mx[q], slot[q]);
          else
            update_chunk(s, m32, h, ch, mx[q], slot[q]);
        }
      }
      if (++c_g == ngroups) {
        c_g = 0;
        close_item();
        c_slot = next_slot(c_slot + G);
        set_compute_item();
      }
    }
  };

  issue(std::integral_constant<int, 0>());
  issue(std::integral_constant<int, 1>());
  // Whole rounds of three steps, then the one or two tasks left: no branch
  // around a step inside a round, so the compiler's wait counts see every
  // step's loads (a skip edge made it drain the loads of later tasks).
  static_assert(kStages == 3, "the task loop below is unrolled by three");
  int64_t p = 0;
  for (; p + kStages <= ntasks; p += kStages) {
    step(std::integral_constant<int, 0>());
    step(std::integral_constant<int, 1>());
    step(std::integral_constant<int, 2>());
  }
  if (p < ntasks) step(std::integral_constant<int, 0>());
  if (p + 1 < ntasks) step(std::integral_constant<int, 1>());
  slice_barrier<0>();  // the empty requests past the last task
}

// S[i, j] = sum over tiles tb (in order) of St[i * ntq + tb, j], times
// 1 / max(valid tokens of query i, 1) when normalising.
__global__ void __launch_bounds__(256) split_tile_sum_kernel(const float* St, int ntq, int Bq,
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
      __syncthreads();
    }
    for (int jj = blockIdx.x * 256 + threadIdx.x; jj < Bd; jj += gridDim.x * 256) {
      float s = 0.0f;
      for (int tb = 0; tb < ntq; ++tb) s += St[((int64_t)i * ntq + tb) * Bd + jj];
      S[(int64_t)i * Bd + jj] = norm ? s * inv : s;
    }
  }
}

}  // namespace

bool inbatch_split_supported(int esz, int64_t dim, int64_t Tq, int64_t Td, int64_t Bq,
                             int64_t Bd, const void* Q, const void* D) {
  const bool al = ((reinterpret_cast<uintptr_t>(Q) | reinterpret_cast<uintptr_t>(D)) & 15u) == 0;
  const int64_t rowbytes = dim * esz;
  const int64_t ntq = Tq > kTile ? (Tq + kTile - 1) / kTile : 1;
  const int64_t nqg = (Bq * ntq + kRows - 1) / kRows, ndx = (Bd + kSpXcds - 1) / kSpXcds;
  // 32-bit buffer offsets: a document's rows, a query tile's rows, the slot count
  const int64_t lim = ((int64_t)1 << 31) - 4096;
  return (esz == 2 || esz == 4) && dim > 0 && rowbytes % 16 == 0 && al && Tq >= 1 && Td >= 0 &&
         Bq >= 1 && Bd >= 1 && Bq * ntq <= ((int64_t)1 << 30) && Bd <= ((int64_t)1 << 26) &&
         (Td + kTile * kMaxCg) * rowbytes < lim && kTile * rowbytes < lim &&
         nqg <= lim / kSpXcds / ndx;
}

namespace {

// Compute units of the current device (cached per device; gfx950: 256).
int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < 64) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  if (dev < 64) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace

hipError_t launch_inbatch_split(int32_t dtype, const InBatchSplitArgs& args_in,
                                hipStream_t stream) {
  InBatchSplitArgs A = args_in;
  A.ntq = A.Tq > kTile ? (A.Tq + kTile - 1) / kTile : 1;
  A.nqg = (int)(((int64_t)A.Bq * A.ntq + kRows - 1) / kRows);
  const int ndx = (A.Bd + kSpXcds - 1) / kSpXcds;
  A.nslots = A.nqg * ndx * kSpXcds;
  // One workspace: the plan words (documents' chunk words, then query rows'
  // words), then, with several tiles per query, the tile scores St.
  const int nch = A.Td > 0 ? (A.Td + kTile - 1) / kTile : 0;
  const int64_t nwords = (int64_t)A.Bd * nch + (int64_t)A.Bq * A.ntq;
  const size_t plan_bytes = ((size_t)nwords * sizeof(uint32_t) + 255) / 256 * 256;
  const size_t st_bytes = A.ntq > 1 ? (size_t)A.Bq * A.ntq * A.Bd * sizeof(float) : 0;
  void* ws = nullptr;
  hipError_t e = workspace_alloc(&ws, plan_bytes + st_bytes, stream);
  if (e != hipSuccess) return e;
  A.plan = static_cast<uint32_t*>(ws);
  if (A.ntq > 1) A.St = reinterpret_cast<float*>(static_cast<char*>(ws) + plan_bytes);
  hipLaunchKernelGGL(split_plan_kernel, dim3((unsigned)std::min<int64_t>((nwords + 7) / 8, 1024)),
                     dim3(256), 0, stream, A.dm, A.qm, A.Bd, A.Td, nch, A.Bq, A.Tq, A.ntq,
                     static_cast<uint32_t*>(ws));
  e = hipGetLastError();
  // kBlocks blocks per CU (CUs a multiple of 8, so slot x stays on XCD
  // x % 8), each walking its slots.
  const int cus = std::max(kSpXcds, device_cus() / kSpXcds * kSpXcds);
  const int per_cu = dtype == 0 ? SplitShape<4>::kBlocks : SplitShape<2>::kBlocks;
  const dim3 grid((unsigned)std::min(A.nslots, cus * per_cu)), block(64 * kSpWaves);
  if (e == hipSuccess) {
    const bool whole = A.rowbytes % kSliceBytes == 0;
    switch (dtype) {
      case 1:
        if (whole) hipLaunchKernelGGL((inbatch_split<OpF16, true>), grid, block, 0, stream, A);
        else hipLaunchKernelGGL((inbatch_split<OpF16, false>), grid, block, 0, stream, A);
        break;
      case 2:
        if (whole) hipLaunchKernelGGL((inbatch_split<OpBF16, true>), grid, block, 0, stream, A);
        else hipLaunchKernelGGL((inbatch_split<OpBF16, false>), grid, block, 0, stream, A);
        break;
      default:
        if (whole) hipLaunchKernelGGL((inbatch_split<OpF32, true>), grid, block, 0, stream, A);
        else hipLaunchKernelGGL((inbatch_split<OpF32, false>), grid, block, 0, stream, A);
        break;
    }
    e = hipGetLastError();
  }
  if (e == hipSuccess && A.ntq > 1) {
    hipLaunchKernelGGL(split_tile_sum_kernel,
                       dim3((unsigned)std::min((A.Bd + 255) / 256, 64),
                            (unsigned)std::min(A.Bq, 65535)),
                       dim3(256), 0, stream, A.St, A.ntq, A.Bq, A.Bd, A.qm, A.Tq, A.norm, A.S);
    e = hipGetLastError();
  }
  const hipError_t ef = workspace_free(ws, stream);
  if (e == hipSuccess) e = ef;
  return e;
}

}  // namespace fms
