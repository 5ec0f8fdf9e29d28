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
// One 1024-thread workgroup per row, three phases, no workspace:
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

#include "fms_topk.hpp"

namespace fms {

namespace {

constexpr int kTkThreads = 1024;
constexpr int kTkWaves = kTkThreads / 64;
constexpr int kTkBins = 256;

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

__global__ void __launch_bounds__(kTkThreads) topk_rows_kernel(const float* __restrict__ S,
                                                               int64_t ncols, int k, int kpow2,
                                                               float* __restrict__ vals,
                                                               int32_t* __restrict__ idx) {
  __shared__ uint32_t hist[kTkBins];
  __shared__ uint32_t sel_prefix, sel_need;
  __shared__ uint32_t wsum[kTkWaves];
  __shared__ uint64_t pick[kTopkMaxK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  const float* const s = S + row * ncols;

  // ---- 1. radix select: T = the k-th largest key ---------------------------------
  // Invariant: 1 <= need <= (entries whose key matches prefix under pmask); the
  // entries above the prefix group number k - need.
  uint32_t prefix = 0u, pmask = 0u, need = (uint32_t)k;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    for (int b = tid; b < kTkBins; b += kTkThreads) hist[b] = 0u;
    __syncthreads();
#pragma unroll 4
    for (int64_t i = tid; i < ncols; i += kTkThreads) {
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
  for (int64_t t0 = 0; t0 < ncols; t0 += kTkThreads) {
    const int64_t i = t0 + tid;
    const uint32_t key = i < ncols ? order_key(s[i]) : 0u;
    const uint32_t gt = (i < ncols && key > T) ? 1u : 0u;
    const uint32_t eq = (i < ncols && key == T) ? 1u : 0u;
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
    const uint64_t p = ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
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
    vals[row * k + e] = key_value((uint32_t)(p >> 32));
    idx[row * k + e] = (int32_t)(0xffffffffu - (uint32_t)p) + 1;
  }
}

}  // namespace

hipError_t topk_rows(const float* S, int64_t nrows, int64_t ncols, int k, float* vals,
                     int32_t* idx, hipStream_t stream) {
  int kpow2 = 1;
  while (kpow2 < k) kpow2 <<= 1;
  hipLaunchKernelGGL(topk_rows_kernel, dim3((unsigned)nrows), dim3(kTkThreads), 0, stream, S,
                     ncols, k, kpow2, vals, idx);
  return hipGetLastError();
}

}  // namespace fms
