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
// Block = one document j x kRows query rows (a query row is a 32-token tile
// of a query: query v / ntq, tokens 32 (v % ntq) ..), 4 waves, one block per
// CU.  The document's chunks are taken kCg at a time (a chunk group); per
// group the block runs the whole K loop:
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
//   * three stages: slice s + 2 is requested while slice s is multiplied;
//     one barrier per slice (every wave's share of slice s has landed, and
//     every wave is done with the stage slice s - 1 used, which the request
//     of slice s + 2 then refills);
//   * wave w holds the accumulators of query rows 2w, 2w + 1 for the whole
//     chunk group (2 x kCg 32x32 tiles): each query fragment read feeds kCg
//     MFMA chains and each document fragment read two;
//   * 16-bit: one v_mfma_f32_32x32x16 per unit pair.  fp32: the 16 bytes of
//     a unit pair are four k-blocks of v_mfma_f32_32x32x2f32; dword e of
//     the lanes of half h is feature 8m + 4h + e of the slice, the same
//     bijection for both operands, so the four MFMAs sum the 8 features of
//     the unit pair;
//   * after the K loop each accumulator tile is folded, chunk by chunk in
//     document order, into the running max / argmax exactly as the scans
//     fold (first valid row taken, then strictly greater; chunk masks from
//     dmask and Td), and the last group closes the tiles: wave halves
//     merged, tape rows and the score written straight to global memory.
// Block -> (document, query group) is XCD-aware: each XCD takes every 8th
// document, in bands of kBand documents; within a band the document runs
// fastest, so the XCD's 32 CUs hold kBand documents x 32 / kBand query groups
// at a time, and the band's documents stay in that XCD's L2 while all query
// groups pass over them.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <algorithm>

#include "fms_device.hpp"
#include "fms_group.hpp"
#include "fms_inbatch_split.hpp"
#include "fms_scan.hpp"

namespace fms {

namespace {

constexpr int kSpWaves = 4;
constexpr int kRows = 2 * kSpWaves;     // query rows per block (two per wave)
constexpr int kCg = 6;                  // document chunks per group
constexpr int kSliceBytes = 128;        // bytes of every row per K step
constexpr int kPairs = kSliceBytes / 32;  // unit pairs per slice (4)
constexpr int kDFrags = kCg * kPairs;   // 1 KB blocks of a document slice
constexpr int kStages = 3;              // document slice buffers in LDS (2 slices ahead)
static_assert(kDFrags % kSpWaves == 0, "every wave copies unit pair m = wave of each chunk");
// Vector memory operations per slice and wave: kCg document copies into LDS,
// then 2 x kPairs query fragment loads into registers.
constexpr int kQLoads = 2 * kPairs;
constexpr int kOpsPerSlice = kCg + kQLoads;
// Issued after a slice's document copies by the time that slice is read: its
// own query loads and the two slices requested since.
constexpr int kAfterCopies = kQLoads + (kStages - 2) * kOpsPerSlice;
static_assert(kAfterCopies < 64, "vmcnt field");
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

template <class Op>
__global__ void __launch_bounds__(64 * kSpWaves, 1) inbatch_split(const InBatchSplitArgs A) {
  typedef typename Op::Acc Acc;
  constexpr int kMmaPerPair = Op::kEsz == 4 ? 4 : 1;
  typedef __attribute__((address_space(3))) void* lds_void_t;
  __shared__ u32x4 dbuf[kStages][kDFrags * 64];

  const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
  const int r32 = lane & 31, h = lane >> 5;

  // XCD-aware mapping: blocks are dealt round-robin to the 8 XCDs; XCD x
  // serves documents 8 dl + x, dl < ndx.  Its order k = id / 8 walks bands
  // of kBand consecutive dl: inside a band dl runs fastest, then the query
  // group.
  const int id = blockIdx.x, xcd = id % kSpXcds, kx = id / kSpXcds;
  const int ndx = (A.Bd + kSpXcds - 1) / kSpXcds;
  const int band = kx / (kBand * A.nqg);
  const int bsz = std::min(kBand, ndx - band * kBand);
  const int within = kx - band * kBand * A.nqg;
  const int qg = within / bsz;
  const int j = (band * kBand + within % bsz) * kSpXcds + xcd;
  if (j >= A.Bd) return;

  const int rowbytes = A.rowbytes, Tq = A.Tq, Td = A.Td, ntq = A.ntq;
  const int nslices = (rowbytes + kSliceBytes - 1) / kSliceBytes;
  const int nch = Td > 0 ? (Td + kTile - 1) / kTile : 0;
  const int nqv = A.Bq * ntq;

  // This wave's two query rows: query, first token, token count, liveness.
  int qi[2], qt0[2], qtn[2], qv[2];
  bool qlive[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    qv[q] = qg * kRows + 2 * wave + q;
    qlive[q] = qv[q] < nqv;
    qi[q] = qlive[q] ? qv[q] / ntq : 0;
    qt0[q] = (qv[q] - qi[q] * ntq) * kTile;
    qtn[q] = qlive[q] ? std::min(kTile, Tq - qt0[q]) : 0;
  }
  // Query token validity of this lane (token r32 of each row).
  bool tvalid[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const bool in = qlive[q] && r32 < qtn[q];
    tvalid[q] = in && (A.qm == nullptr || A.qm[(int64_t)qi[q] * Tq + qt0[q] + r32] != 0);
  }

  // Loads of this wave per slice: the document copies, unit pair m = wave of
  // every chunk of the group into LDS (the block's four waves together copy
  // the whole slice), and this wave's own query fragments, both rows x kPairs
  // unit pairs, into registers.  Lane l reads row l % 32, unit 2m + l / 32 of
  // the slice; a unit past the row reads out of range (zeros).
  const int copy_off = (2 * wave + h) * 16;
  const rsrc_t rdoc = make_rsrc_u(A.D + (int64_t)j * Td * rowbytes, (uint32_t)Td * (uint32_t)rowbytes);
  rsrc_t rq[2];
#pragma unroll
  for (int q = 0; q < 2; ++q)
    rq[q] = make_rsrc_u(A.Q + ((int64_t)qi[q] * Tq + qt0[q]) * rowbytes,
                        (uint32_t)qtn[q] * (uint32_t)rowbytes);
  // Query fragments of kStages slices in flight: set k holds slices
  // kStages * n + k.
  u32x4 qf[kStages][2][kPairs];

  // Slice s of group g: its document copies into stage s % kStages, its query
  // fragments into set s % kStages (kSet, a constant: the slice loop is
  // unrolled by kStages).  A slice index past the last re-reads the last
  // slice, so every step issues the same operations.
  auto issue = [&](auto SETc, int g, int s) {
    constexpr int kSet = decltype(SETc)::value;
    // Rows past the document or the query lie outside their resources; a unit
    // past the row end is pushed out of range with all low 31 bits set
    // (branch-free: a select here became divergent branches around the loads).
    const int sc = std::min(s, nslices - 1);
    const int so = sc * kSliceBytes + copy_off;
    const int dpast = -(int)(so >= rowbytes) & 0x7fffffff;
#pragma unroll
    for (int c = 0; c < kCg; ++c) {
      const int row = (g * kCg + c) * kTile + r32;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rdoc, (lds_void_t)&dbuf[kSet][(c * kPairs + wave) * 64], 16, (row * rowbytes + so) | dpast,
          0, 0, 0);
    }
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int m = 0; m < kPairs; ++m) {
        const int o = sc * kSliceBytes + (2 * m + h) * 16;
        const int qpast = -(int)(o >= rowbytes) & 0x7fffffff;
        qf[kSet][q][m] = buf_load16(rq[q], (r32 * rowbytes + o) | qpast);
      }
  };

  float mx[2] = {-INFINITY, -INFINITY};
  int slot[2] = {-1, -1};
  const int ngroups = nch > 0 ? (nch + kCg - 1) / kCg : 0;
  for (int g = 0; g < ngroups; ++g) {
    const int gc = std::min(kCg, nch - g * kCg);  // chunks in this group
    // chunk row validity (lane row r32 of each chunk), ballotted after the K loop
    uint32_t mbyte[kCg];
#pragma unroll
    for (int c = 0; c < kCg; ++c) {
      const int row = (g * kCg + c) * kTile + r32;
      mbyte[c] = (row < Td && (A.dm == nullptr || A.dm[(int64_t)j * Td + row] != 0)) ? 1u : 0u;
    }
    Acc acc[kCg][2];
#pragma unroll
    for (int c = 0; c < kCg; ++c) { acc[c][0] = Acc{}; acc[c][1] = Acc{}; }

    // Prologue: slices 0 and 1.  Step s then waits for its copies (exactly
    // kAfterCopies operations were issued after them), a barrier makes every
    // wave's share visible and frees the stage step s - 1 read, slice s + 2
    // is requested into that stage and query set, and slice s is multiplied.
    // Chunks past the document (the last group of a long one) read zeros:
    // their MFMAs run unguarded and their accumulators are never folded.
    issue(std::integral_constant<int, 0>(), g, 0);
    issue(std::integral_constant<int, 1>(), g, 1);
    auto step = [&](auto SETc, int s) {
      constexpr int kSet = decltype(SETc)::value;
      slice_barrier<kAfterCopies>();
      issue(std::integral_constant<int, (kSet + 2) % kStages>(), g, s + 2);
      // Document fragments of unit pair m + 1 are read while pair m's MFMAs
      // run (two register sets).
      const u32x4* B = &dbuf[kSet][lane];
      u32x4 a[2][kCg];
#pragma unroll
      for (int c = 0; c < kCg; ++c) a[0][c] = B[(c * kPairs) * 64];
#pragma unroll
      for (int m = 0; m < kPairs; ++m) {
        if (m + 1 < kPairs) {
#pragma unroll
          for (int c = 0; c < kCg; ++c) a[(m + 1) & 1][c] = B[(c * kPairs + m + 1) * 64];
        }
#pragma unroll
        for (int c = 0; c < kCg; ++c) {
          acc[c][0] = mma_pair<Op>(a[m & 1][c], qf[kSet][0][m], acc[c][0]);
          acc[c][1] = mma_pair<Op>(a[m & 1][c], qf[kSet][1][m], acc[c][1]);
        }
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
    // Whole rounds of three steps, then the one or two slices left: no branch
    // inside a round, so the compiler's wait counts see only the straight path
    // (a skip edge inside a round made it drain the loads of later slices).
    static_assert(kStages == 3, "the slice loop below is unrolled by three");
    int s0 = 0;
    for (; s0 + kStages <= nslices; s0 += kStages) {
      step(std::integral_constant<int, 0>(), s0);
      step(std::integral_constant<int, 1>(), s0 + 1);
      step(std::integral_constant<int, 2>(), s0 + 2);
    }
    if (s0 < nslices) step(std::integral_constant<int, 0>(), s0);
    if (s0 + 1 < nslices) step(std::integral_constant<int, 1>(), s0 + 1);
    slice_barrier<0>();  // no copy into LDS outlives the group (the next refills the stages)

    // fold the group's chunks in document order
#pragma unroll
    for (int c = 0; c < kCg; ++c) {
      if (c >= gc) continue;
      const int ch = g * kCg + c;
      const uint32_t m32 = (uint32_t)__ballot(mbyte[c] != 0u);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        float s[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = acc[c][q][r];
        take_first_row(s, m32, h, ch, mx[q], slot[q]);
        if (m32 == 0xffffffffu)
          fold_tree(s, ch * 16, mx[q], slot[q]);
        else
          update_chunk(s, m32, h, ch, mx[q], slot[q]);
      }
    }
  }

  // close the document for both query rows
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    if (!qlive[q]) continue;
    int tok = slot_to_token(slot[q], h);
    float m = mx[q];
    merge_halves(m, tok, h);
    const float part = (tvalid[q] && tok != 0) ? m : 0.0f;
    const int64_t p = (int64_t)qi[q] * A.Bd + j;
    if (A.args && h == 0 && r32 < qtn[q]) A.args[p * Tq + qt0[q] + r32] = tvalid[q] ? tok : 0;
    const float score = half_sum(part);
    if (ntq > 1) {
      if (lane == 0) A.St[(int64_t)qv[q] * A.Bd + j] = score;
    } else {
      float inv = 1.0f;
      if (A.norm) {
        const float nf = (float)__builtin_popcountll(__ballot(h == 0 && tvalid[q]));
        inv = 1.0f / (nf > 1.0f ? nf : 1.0f);
      }
      if (lane == 0) A.S[p] = A.norm ? score * inv : score;
    }
  }
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
  return (esz == 2 || esz == 4) && dim > 0 && rowbytes % 16 == 0 && al && Tq >= 1 && Td >= 0 &&
         Bq >= 1 && Bd >= 1 && Bq * ntq <= ((int64_t)1 << 30) && Bd <= ((int64_t)1 << 26);
}

hipError_t launch_inbatch_split(int32_t dtype, const InBatchSplitArgs& args_in,
                                hipStream_t stream) {
  InBatchSplitArgs A = args_in;
  A.ntq = A.Tq > kTile ? (A.Tq + kTile - 1) / kTile : 1;
  A.nqg = (int)(((int64_t)A.Bq * A.ntq + kRows - 1) / kRows);
  void* ws = nullptr;
  if (A.ntq > 1) {
    hipError_t e = workspace_alloc(&ws, (size_t)A.Bq * A.ntq * A.Bd * sizeof(float), stream);
    if (e != hipSuccess) return e;
    A.St = static_cast<float*>(ws);
  }
  const int64_t blocks = (int64_t)A.nqg * ((A.Bd + kSpXcds - 1) / kSpXcds) * kSpXcds;
  const dim3 grid((unsigned)blocks), block(64 * kSpWaves);
  switch (dtype) {
    case 1: hipLaunchKernelGGL(inbatch_split<OpF16>, grid, block, 0, stream, A); break;
    case 2: hipLaunchKernelGGL(inbatch_split<OpBF16>, grid, block, 0, stream, A); break;
    default: hipLaunchKernelGGL(inbatch_split<OpF32>, grid, block, 0, stream, A); break;
  }
  hipError_t e = hipGetLastError();
  if (e == hipSuccess && A.ntq > 1) {
    hipLaunchKernelGGL(split_tile_sum_kernel,
                       dim3((unsigned)std::min((A.Bd + 255) / 256, 64),
                            (unsigned)std::min(A.Bq, 65535)),
                       dim3(256), 0, stream, A.St, A.ntq, A.Bq, A.Bd, A.qm, A.Tq, A.norm, A.S);
    e = hipGetLastError();
  }
  if (ws) {
    const hipError_t ef = workspace_free(ws, stream);
    if (e == hipSuccess) e = ef;
  }
  return e;
}

}  // namespace fms
