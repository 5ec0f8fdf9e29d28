// fms_backward.hip -- pullback of the fused MaxSim forward on its argmax tape
// (see fms_backward.hpp for the mathematics and the two halves).
//
// Launches per call: delta (delta_p = Delta[p] * inv_n[query of p], fp32),
// [clear dQ], dQ gather, count -> prefix sum -> fill of the destination CSR,
// dD per destination row.  A wave owns one output row in the two row
// kernels; lane l holds features l, l + 64, ... of it (KI per lane).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "fms_backward.hpp"
#include "fms_group.hpp"

namespace fms {

namespace {

constexpr int kBwdThreads = 256;            // 4 waves
constexpr int kBwdUnroll = 8;               // source rows in flight per wave

inline int64_t bcdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }
inline unsigned grid_for(int64_t waves) {
  const int64_t b = bcdiv(waves, kBwdThreads / 64);
  return (unsigned)(b < 1 ? 1 : (b > 1048576 ? 1048576 : b));
}

// Feature element <-> fp32.
struct EF32 {
  static constexpr int kSz = 4;
  __device__ static float ld(const char* p) { return *reinterpret_cast<const float*>(p); }
  __device__ static void st(char* p, float v) { *reinterpret_cast<float*>(p) = v; }
};
struct EF16 {
  static constexpr int kSz = 2;
  __device__ static float ld(const char* p) { return (float)*reinterpret_cast<const _Float16*>(p); }
  __device__ static void st(char* p, float v) { *reinterpret_cast<_Float16*>(p) = (_Float16)v; }
};
struct EBF16 {
  static constexpr int kSz = 2;
  __device__ static float ld(const char* p) {
    return __builtin_bit_cast(float, (uint32_t)*reinterpret_cast<const uint16_t*>(p) << 16);
  }
  __device__ static void st(char* p, float v) {  // round to nearest even
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const uint16_t r = (v != v) ? (uint16_t)0x7FC0u : (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
    *reinterpret_cast<uint16_t*>(p) = r;
  }
};

__device__ __forceinline__ int64_t uni64(int64_t v) { return (int64_t)rfl64((uint64_t)v); }

template <class E>
__global__ void __launch_bounds__(kBwdThreads) bwd_delta_kernel(const char* Delta, const char* inv_n,
                                                               int64_t P, int64_t G, float* delta) {
  const int64_t stride = (int64_t)gridDim.x * kBwdThreads;
  for (int64_t p = (int64_t)blockIdx.x * kBwdThreads + threadIdx.x; p < P; p += stride)
    delta[p] = E::ld(Delta + p * E::kSz) * (inv_n ? E::ld(inv_n + (p / G) * E::kSz) : 1.0f);
}

__global__ void __launch_bounds__(kBwdThreads) bwd_zero_kernel(uint32_t* w, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kBwdThreads;
  for (int64_t i = (int64_t)blockIdx.x * kBwdThreads + threadIdx.x; i < n; i += stride) w[i] = 0u;
}

__global__ void __launch_bounds__(kBwdThreads) bwd_zero16_kernel(uint16_t* w, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kBwdThreads;
  for (int64_t i = (int64_t)blockIdx.x * kBwdThreads + threadIdx.x; i < n; i += stride) w[i] = 0u;
}

// Sources of pair p: query tokens t < tq with qmask, a tape entry in 1..td,
// and a nonzero delta (a zero delta adds nothing, backward_pair.jl:21).
// kFill = false: count them per destination row; true: give each a slot in
// its row (off[r] runs from the row's start to its end) and record
// p * rows + t there.
template <class L, bool kFill>
__global__ void __launch_bounds__(kBwdThreads) bwd_csr_kernel(const L lay, const int32_t* args,
                                                             const float* delta, int64_t P,
                                                             int rows, const char* Dbase,
                                                             int64_t rb, uint32_t* cnt_or_off,
                                                             uint32_t* col) {
  const int lane = threadIdx.x & 63;
  const int64_t nw = (int64_t)gridDim.x * (kBwdThreads / 64);
  for (int64_t p = uni64((int64_t)blockIdx.x * (kBwdThreads / 64) + (threadIdx.x >> 6)); p < P;
       p += nw) {
    const PairView v = uniform_view(lay.get(p));
    const float dl = sload(delta, p);
    if (!v.valid || dl == 0.0f) continue;
    const int64_t r0 = (int64_t)(v.d - Dbase) / rb;
    for (int t = lane; t < v.tq; t += 64) {
      const int u = args[p * rows + t];
      const bool ok = (v.qm == nullptr || v.qm[t] != 0) && u >= 1 && u <= v.td;
      if (!ok) continue;
      if constexpr (kFill) {
        const uint32_t pos = atomicAdd(&cnt_or_off[r0 + u - 1], 1u);
        col[pos] = (uint32_t)(p * rows + t);
      } else {
        atomicAdd(&cnt_or_off[r0 + u - 1], 1u);
      }
    }
  }
}

// dD row r = sum over its sources s = p*rows + t of delta_p * Q[:, t of p].
template <class L, class E, int KI>
__global__ void __launch_bounds__(kBwdThreads) bwd_dd_kernel(const L lay, const float* delta,
                                                            const uint32_t* end, const uint32_t* col,
                                                            int64_t nrows, int rows, int dim,
                                                            int64_t rb, char* dD) {
  const int lane = threadIdx.x & 63;
  const int64_t nw = (int64_t)gridDim.x * (kBwdThreads / 64);
  for (int64_t r = uni64((int64_t)blockIdx.x * (kBwdThreads / 64) + (threadIdx.x >> 6)); r < nrows;
       r += nw) {
    const int64_t s0 = r > 0 ? (int64_t)sload(end, r - 1) : 0, s1 = (int64_t)sload(end, r);
    float acc[KI];
#pragma unroll
    for (int j = 0; j < KI; ++j) acc[j] = 0.0f;
    for (int64_t s = s0; s < s1; s += kBwdUnroll) {
      const char* qrow[kBwdUnroll];
      float dl[kBwdUnroll];
#pragma unroll
      for (int i = 0; i < kBwdUnroll; ++i) {
        const int64_t si = s + i < s1 ? s + i : s1 - 1;
        const uint32_t src = sload(col, si);
        const int64_t p = src / (uint32_t)rows, t = src % (uint32_t)rows;
        const PairView v = uniform_view(lay.get(p));
        qrow[i] = v.q + t * rb;
        dl[i] = s + i < s1 ? sload(delta, p) : 0.0f;
      }
      float x[kBwdUnroll][KI];
#pragma unroll
      for (int i = 0; i < kBwdUnroll; ++i)
#pragma unroll
        for (int j = 0; j < KI; ++j) {
          const int k = lane + 64 * j;
          x[i][j] = k < dim ? E::ld(qrow[i] + (int64_t)k * E::kSz) : 0.0f;
        }
#pragma unroll
      for (int i = 0; i < kBwdUnroll; ++i)
#pragma unroll
        for (int j = 0; j < KI; ++j) acc[j] += dl[i] * x[i][j];
    }
    char* out = dD + r * rb;
#pragma unroll
    for (int j = 0; j < KI; ++j) {
      const int k = lane + 64 * j;
      if (k < dim) E::st(out + (int64_t)k * E::kSz, acc[j]);
    }
  }
}

// dQ row (group g, token t) = sum over the group's pairs p, in pair order, of
// delta_p * D[:, args[t, p] of p's document] (valid sources only).
template <class L, class E, int KI>
__global__ void __launch_bounds__(kBwdThreads) bwd_dq_kernel(const L lay, const float* delta,
                                                            const int32_t* args, int64_t ngroups,
                                                            int64_t G, int rows, int dim, int64_t rb,
                                                            const char* Qbase, char* dQ) {
  const int lane = threadIdx.x & 63;
  const int64_t nw = (int64_t)gridDim.x * (kBwdThreads / 64), nall = ngroups * rows;
  for (int64_t w = uni64((int64_t)blockIdx.x * (kBwdThreads / 64) + (threadIdx.x >> 6)); w < nall;
       w += nw) {
    const int64_t g = w / rows;
    const int t = (int)(w - g * rows);
    const PairView v0 = uniform_view(lay.get(g * G));
    if (t >= v0.tq) continue;  // (varlen: past this query's tokens)
    const bool tvalid = v0.qm == nullptr || sload(v0.qm, t) != 0;
    float acc[KI];
#pragma unroll
    for (int j = 0; j < KI; ++j) acc[j] = 0.0f;
    if (tvalid) {
      for (int64_t p0 = g * G; p0 < (g + 1) * G; p0 += kBwdUnroll) {
        const char* drow[kBwdUnroll];
        float dl[kBwdUnroll];
#pragma unroll
        for (int i = 0; i < kBwdUnroll; ++i) {
          const int64_t p = p0 + i < (g + 1) * G ? p0 + i : (g + 1) * G - 1;
          const PairView v = uniform_view(lay.get(p));
          const int u = sload(args, p * rows + t);
          const bool ok = p0 + i < (g + 1) * G && v.valid && u >= 1 && u <= v.td;
          drow[i] = v.d + (int64_t)(ok ? u - 1 : 0) * rb;
          dl[i] = ok ? sload(delta, p) : 0.0f;
        }
        float x[kBwdUnroll][KI];
#pragma unroll
        for (int i = 0; i < kBwdUnroll; ++i)
#pragma unroll
          for (int j = 0; j < KI; ++j) {
            const int k = lane + 64 * j;
            x[i][j] = (k < dim && dl[i] != 0.0f) ? E::ld(drow[i] + (int64_t)k * E::kSz) : 0.0f;
          }
#pragma unroll
        for (int i = 0; i < kBwdUnroll; ++i)
#pragma unroll
          for (int j = 0; j < KI; ++j) acc[j] += dl[i] * x[i][j];
      }
    }
    char* out = dQ + (v0.q - Qbase) + (int64_t)t * rb;
#pragma unroll
    for (int j = 0; j < KI; ++j) {
      const int k = lane + 64 * j;
      if (k < dim) E::st(out + (int64_t)k * E::kSz, acc[j]);
    }
  }
}

template <class L, class E, int KI>
void launch_rows(const L& lay, const PullbackArgs& a, const float* delta, const uint32_t* end,
                 const uint32_t* col, int64_t rb, hipStream_t st) {
  const int64_t ngroups = a.npairs / a.G;
  hipLaunchKernelGGL((bwd_dq_kernel<L, E, KI>), dim3(grid_for(ngroups * a.rows)), dim3(kBwdThreads),
                     0, st, lay, delta, a.args, ngroups, a.G, a.rows, a.dim, rb, a.Qbase, a.dQ);
  hipLaunchKernelGGL((bwd_dd_kernel<L, E, KI>), dim3(grid_for(a.nd_rows)), dim3(kBwdThreads), 0, st,
                     lay, delta, end, col, a.nd_rows, a.rows, a.dim, rb, a.dD);
}

template <class L, class E>
void launch_rows_e(const L& lay, const PullbackArgs& a, const float* delta, const uint32_t* end,
                   const uint32_t* col, int64_t rb, hipStream_t st) {
  if (a.dim <= 64) launch_rows<L, E, 1>(lay, a, delta, end, col, rb, st);
  else if (a.dim <= 128) launch_rows<L, E, 2>(lay, a, delta, end, col, rb, st);
  else if (a.dim <= 512) launch_rows<L, E, 8>(lay, a, delta, end, col, rb, st);
  else launch_rows<L, E, 32>(lay, a, delta, end, col, rb, st);
}

}  // namespace

template <class L>
hipError_t launch_pullback(const L& lay, const PullbackArgs& a, hipStream_t st) {
  const int esz = a.dtype == 0 ? 4 : 2;
  const int64_t rb = (int64_t)a.dim * esz;
  // Both gradients are written in full; 2-byte units because a row of 2-byte
  // features need not be a dword multiple.
  auto clear = [&](char* p, int64_t nrows) {
    const int64_t nhalf = nrows * rb / 2;
    if (nhalf > 0)
      hipLaunchKernelGGL(bwd_zero16_kernel, dim3(grid_for(bcdiv(nhalf, 64))), dim3(kBwdThreads), 0, st,
                         reinterpret_cast<uint16_t*>(p), nhalf);
  };
  if (a.npairs == 0) {  // no pair: both gradients are zero
    clear(a.dQ, a.nq_rows);
    clear(a.dD, a.nd_rows);
    return hipGetLastError();
  }
  // workspace: delta (npairs f32), end offsets (nd_rows + 1), sources (npairs * rows), scan sums
  const int64_t nsrc = a.npairs * a.rows;
  const size_t b_delta = al256((size_t)a.npairs * 4), b_end = al256((size_t)(a.nd_rows + 1) * 4);
  const size_t b_col = al256((size_t)(nsrc > 0 ? nsrc : 1) * 4), b_sums = scan_workspace_bytes(a.nd_rows);
  void* ws = nullptr;
  hipError_t e = workspace_alloc(&ws, b_delta + b_end + b_col + b_sums, st);
  if (e != hipSuccess) return e;
  char* w = static_cast<char*>(ws);
  float* delta = reinterpret_cast<float*>(w);
  uint32_t* cnt = reinterpret_cast<uint32_t*>(w + b_delta);
  uint32_t* col = reinterpret_cast<uint32_t*>(w + b_delta + b_end);
  uint32_t* sums = reinterpret_cast<uint32_t*>(w + b_delta + b_end + b_col);
  const unsigned flat = (unsigned)std::min<int64_t>(65536, std::max<int64_t>(1, bcdiv(a.npairs, kBwdThreads)));
  const char* Dl = static_cast<const char*>(a.Delta);
  const char* Il = static_cast<const char*>(a.inv_n);
  if (a.dtype == 0)
    hipLaunchKernelGGL(bwd_delta_kernel<EF32>, dim3(flat), dim3(kBwdThreads), 0, st, Dl, Il, a.npairs, a.G, delta);
  else if (a.dtype == 1)
    hipLaunchKernelGGL(bwd_delta_kernel<EF16>, dim3(flat), dim3(kBwdThreads), 0, st, Dl, Il, a.npairs, a.G, delta);
  else
    hipLaunchKernelGGL(bwd_delta_kernel<EBF16>, dim3(flat), dim3(kBwdThreads), 0, st, Dl, Il, a.npairs, a.G, delta);
  if (a.zero_dq) clear(a.dQ, a.nq_rows);
  // destination CSR
  hipLaunchKernelGGL(bwd_zero_kernel, dim3(grid_for(bcdiv(a.nd_rows + 1, 64))), dim3(kBwdThreads), 0, st,
                     cnt, a.nd_rows + 1);
  hipLaunchKernelGGL((bwd_csr_kernel<L, false>), dim3(grid_for(a.npairs)), dim3(kBwdThreads), 0, st, lay,
                     a.args, delta, a.npairs, a.rows, a.Dbase, rb, cnt, col);
  e = exclusive_scan_u32(cnt, a.nd_rows, sums, st);
  if (e == hipSuccess) {
    hipLaunchKernelGGL((bwd_csr_kernel<L, true>), dim3(grid_for(a.npairs)), dim3(kBwdThreads), 0, st, lay,
                       a.args, delta, a.npairs, a.rows, a.Dbase, rb, cnt, col);
    if (a.dtype == 0) launch_rows_e<L, EF32>(lay, a, delta, cnt, col, rb, st);
    else if (a.dtype == 1) launch_rows_e<L, EF16>(lay, a, delta, cnt, col, rb, st);
    else launch_rows_e<L, EBF16>(lay, a, delta, cnt, col, rb, st);
    e = hipGetLastError();
  }
  const hipError_t ef = workspace_free(ws, st);
  return e != hipSuccess ? e : ef;
}

template hipError_t launch_pullback<LayPaired>(const LayPaired&, const PullbackArgs&, hipStream_t);
template hipError_t launch_pullback<LayCand>(const LayCand&, const PullbackArgs&, hipStream_t);
template hipError_t launch_pullback<LayInBatch>(const LayInBatch&, const PullbackArgs&, hipStream_t);
template hipError_t launch_pullback<LayPacked>(const LayPacked&, const PullbackArgs&, hipStream_t);
template hipError_t launch_pullback<LayVarlen>(const LayVarlen&, const PullbackArgs&, hipStream_t);

}  // namespace fms
