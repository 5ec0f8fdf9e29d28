// fms_topk.hip -- the k best entries of every row of an fp32 score matrix.
//
// Retrieval callers keep the k best documents per query after a MaxSim scan
// (in the reference that is the caller's `partialsortperm(scores, 1:k;
// rev = true)`, README.md:132).  Row r of the (nrows, ncols) row-major matrix
// -- Julia's (ncols, nrows) column-major, one column per query -- yields
// vals[r, 0..k) in descending order and idx[r, 0..k) as 1-based column
// indices.  The order is total: larger score first (Julia's isless: every
// NaN above +Inf, -0.0 below +0.0), equal scores by smaller index -- what a
// stable reverse sort returns.
//
// One 1024-thread workgroup ranks a row (or a slice of one) in three phases:
//   1. radix select over the 32-bit order keys, 8 bits per pass from the top
//      (4 passes; LDS histogram of the entries still matching the prefix):
//      the k-th largest key T and how many entries lie strictly above it;
//   2. one ordered pass over the row (block-wide prefix counts per 1024-entry
//      tile, stopping once the picks are complete): every entry above T, and
//      the first (by index) entries equal to T until k are chosen;
//   3. a bitonic sort in LDS of the k picks on (key, ~index).
// Each pass reads the row from L2 (a row of 20,000 scores is 80 KB), so the
// cost is five row reads per workgroup.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cmath>

#include "fms_group.hpp"
#include "fms_topk.hpp"

namespace fms {

namespace {

constexpr int kTkThreads = 1024;
constexpr int kTkWaves = kTkThreads / 64;
constexpr int kTkBins = 256;
constexpr int64_t kTkMinSlice = 512;    // entries per slice of the two-stage split, at least
constexpr int64_t kTkMaxBlocks = 512;   // workgroups of the first stage (one round), at most
constexpr int64_t kTkSplitCols = 16384; // rows shorter than this are ranked in one stage

// Order-preserving key: unsigned order of keys = isless order of floats.
__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  if (f != f) return 0xffffffffu;  // every NaN ranks above +Inf
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Inclusive prefix sum over the wave's 64 lanes.
__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t w = __shfl_up(v, o, 64);
    if (lane >= o) v += w;
  }
  return v;
}

// Block b ranks slice b % nslices of row b / nslices: entries [c0, c1) of the
// row (ld apart), c0 = slice * ncols / nslices.  An entry's index is its
// column, or (kIdx) the 1-based index stored beside it in SI; ties go to the
// smaller index either way.  Out: k entries at vals/idx[b * k ...], 1-based.
template <bool kIdx>
__global__ void __launch_bounds__(kTkThreads) topk_rows_kernel(const float* __restrict__ S,
                                                               const int32_t* __restrict__ SI,
                                                               int64_t ld, int64_t ncols,
                                                               int nslices, int k, int kpow2,
                                                               float* __restrict__ vals,
                                                               int32_t* __restrict__ idx) {
  __shared__ uint32_t hist[kTkBins];
  __shared__ uint32_t sel_prefix, sel_need;
  __shared__ uint32_t wsum[kTkWaves];
  __shared__ uint64_t pick[kTopkMaxK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x / nslices, slice = blockIdx.x % nslices;
  const int64_t c0 = slice * ncols / nslices, n = (slice + 1) * ncols / nslices - c0;
  const float* const s = S + row * ld + c0;
  // 0-based index of entry i (i < n)
  auto index_of = [&](int64_t i) -> uint32_t {
    if constexpr (kIdx)
      return (uint32_t)SI[row * ld + c0 + i] - 1u;
    else
      return (uint32_t)(c0 + i);
  };

  // ---- 1. radix select: T = the k-th largest key ---------------------------------
  // Invariant: 1 <= need <= (entries whose key matches prefix under pmask); the
  // entries above the prefix group number k - need.
  uint32_t prefix = 0u, pmask = 0u, need = (uint32_t)k;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    for (int b = tid; b < kTkBins; b += kTkThreads) hist[b] = 0u;
    __syncthreads();
#pragma unroll 4
    for (int64_t i = tid; i < n; i += kTkThreads) {
      const uint32_t key = order_key(s[i]);
      if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 0xffu], 1u);
    }
    __syncthreads();
    if (wave == 0) {
      // lane l holds bins 255-4l .. 252-4l: lanes in descending digit order
      uint32_t c[4], tot = 0u;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        c[e] = hist[255 - 4 * lane - e];
        tot += c[e];
      }
      const uint32_t inc = wave_inclusive_sum(tot, lane), before = inc - tot;
      if (before < need && need <= inc) {  // exactly one lane
        uint32_t acc = before;
        int d = 255 - 4 * lane - 3;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (acc + c[e] >= need) {
            d = 255 - 4 * lane - e;
            break;
          }
          acc += c[e];
        }
        sel_prefix = prefix | ((uint32_t)d << shift);
        sel_need = need - acc;
      }
    }
    __syncthreads();
    prefix = sel_prefix;
    need = sel_need;
    pmask |= 0xffu << shift;
  }
  const uint32_t T = prefix;
  const uint32_t ngt = (uint32_t)k - need;  // entries strictly above T

  // ---- 2. ordered collection -------------------------------------------------------
  // pick = (key << 32) | ~index: descending order of pick is the output order.
  uint32_t base_gt = 0u, base_eq = 0u;
  for (int64_t t0 = 0; t0 < n; t0 += kTkThreads) {
    const int64_t i = t0 + tid;
    const uint32_t key = i < n ? order_key(s[i]) : 0u;
    const uint32_t gt = (i < n && key > T) ? 1u : 0u;
    const uint32_t eq = (i < n && key == T) ? 1u : 0u;
    const uint32_t v = gt | (eq << 16);  // (at most 1024 of each per tile)
    const uint32_t inc = wave_inclusive_sum(v, lane);
    if (lane == 63) wsum[wave] = inc;
    __syncthreads();
    uint32_t off = 0u, tot = 0u;
#pragma unroll
    for (int w = 0; w < kTkWaves; ++w) {
      const uint32_t x = wsum[w];
      off += w < wave ? x : 0u;
      tot += x;
    }
    const uint32_t ex = off + inc - v;
    const uint64_t p =
        ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - (i < n ? index_of(i) : 0u));
    if (gt) {  // exactly ngt entries lie above T (the guard holds for a row read unchanged)
      const uint32_t r = base_gt + (ex & 0xffffu);
      if (r < ngt) pick[r] = p;
    }
    if (eq) {
      const uint32_t r = base_eq + (ex >> 16);
      if (r < need) pick[ngt + r] = p;
    }
    base_gt += tot & 0xffffu;
    base_eq += tot >> 16;
    __syncthreads();  // wsum is rewritten by the next tile
    if (base_gt >= ngt && base_eq >= need) break;  // block-uniform
  }
  // pad to a power of two with entries below every real key (key 0 is never
  // produced: the only float that maps there, -NaN with all bits set, is
  // canonicalised)
  for (int e = k + tid; e < kpow2; e += kTkThreads) pick[e] = 0ull;

  // ---- 3. bitonic sort, descending -------------------------------------------------
  for (int size = 2; size <= kpow2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      __syncthreads();
      for (int t = tid; t < (kpow2 >> 1); t += kTkThreads) {
        const int lo = 2 * t - (t & (stride - 1)), hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const uint64_t a = pick[lo], b = pick[hi];
        if ((a < b) == desc) {
          pick[lo] = b;
          pick[hi] = a;
        }
      }
    }
  }
  __syncthreads();
  for (int e = tid; e < k; e += kTkThreads) {
    const uint64_t p = pick[e];
    vals[(int64_t)blockIdx.x * k + e] = key_value((uint32_t)(p >> 32));
    idx[(int64_t)blockIdx.x * k + e] = (int32_t)(0xffffffffu - (uint32_t)p) + 1;
  }
}

}  // namespace

hipError_t topk_rows(const float* S, int64_t nrows, int64_t ncols, int k, float* vals,
                     int32_t* idx, hipStream_t stream) {
  int kpow2 = 1;
  while (kpow2 < k) kpow2 <<= 1;
  // One workgroup ranks a row in time proportional to its length (LDS
  // histogram atomics), so rows of kTkSplitCols entries or more are first cut
  // into G slices, each ranked by its own workgroup (G ~ sqrt(ncols / k),
  // every slice at least max(k, kTkMinSlice) entries, one round of at most
  // kTkMaxBlocks workgroups; a second launch costs more than it saves on
  // shorter rows), and the
  // G * k survivors of a row -- slice-major, so equal scores stay in index
  // order -- are ranked again.  The global top-k lies within the union of the
  // slice top-ks under the same (score, index) order, so the result is exact.
  int64_t G = (int64_t)std::sqrt((double)ncols / (double)k);
  G = std::min<int64_t>(G, ncols / std::max<int64_t>(k, kTkMinSlice));
  G = std::min<int64_t>(G, std::max<int64_t>(1, kTkMaxBlocks / nrows));
  if (ncols < kTkSplitCols || G < 2) {
    hipLaunchKernelGGL(topk_rows_kernel<false>, dim3((unsigned)nrows), dim3(kTkThreads), 0,
                       stream, S, nullptr, ncols, ncols, 1, k, kpow2, vals, idx);
    return hipGetLastError();
  }
  void* ws = nullptr;
  const size_t nsurv = (size_t)(nrows * G * k);
  hipError_t e = workspace_alloc(&ws, nsurv * 8, stream);
  if (e != hipSuccess) return e;
  float* sv = static_cast<float*>(ws);
  int32_t* si = reinterpret_cast<int32_t*>(sv + nsurv);
  hipLaunchKernelGGL(topk_rows_kernel<false>, dim3((unsigned)(nrows * G)), dim3(kTkThreads), 0,
                     stream, S, nullptr, ncols, ncols, (int)G, k, kpow2, sv, si);
  e = hipGetLastError();
  if (e == hipSuccess) {
    hipLaunchKernelGGL(topk_rows_kernel<true>, dim3((unsigned)nrows), dim3(kTkThreads), 0,
                       stream, sv, si, G * k, G * k, 1, k, kpow2, vals, idx);
    e = hipGetLastError();
  }
  const hipError_t ef = workspace_free(ws, stream);
  return e != hipSuccess ? e : ef;
}

}  // namespace fms
