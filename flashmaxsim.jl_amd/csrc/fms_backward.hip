// fms_backward.hip -- pullback of the fused MaxSim forward on its argmax tape
// (the mathematics and the output contract are in fms_backward.hpp).
//
// Vector path (feature rows of 64..2048 bytes, a multiple of 16, buffers
// 16-byte aligned).  A row is read and written in 16-byte chunks; Lr lanes
// cover one row (Lr = the power of two >= chunks per row, at most 64, with
// two chunks per lane past 64), so one wave instruction moves 64 / Lr rows.
// Per call:
//   delta     delta_p = Delta[p] * inv_n[query of p], fp32.
//   dQ        bwd_dq_vec: a wave owns a block of tokens of one query group and
//             a share of the group's pairs; per pair it reads the tape block
//             once (one dword per lane), hands each lane its tokens' entries
//             by ds_bpermute, and gathers the chosen document rows.  The four
//             waves of a workgroup split the pairs and sum in LDS in a fixed
//             order; across workgroups (pair splits, split index = block
//             index mod nsplit, so split s runs on XCD s mod 8 and keeps its
//             share of the documents in that XCD's L2) fp32 partials are
//             summed in split order by bwd_dq_reduce.  Deterministic.
//   dD        bwd_doc_csr: a workgroup per document sorts the document's
//             sources (pair, token) by destination row in LDS (count, scan,
//             fill) and writes the row lists; bwd_dd_vec then sums each row's
//             source query rows in registers.  Rows of no document (and
//             documents of no pair) are written 0.  The order within a row
//             is the LDS fill order (not fixed).
// Other row sizes take the generic path: one wave per output row, features
// strided over the lanes, and a destination CSR built with global atomics.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <type_traits>

#include "fms_backward.hpp"
#include "fms_device.hpp"
#include "fms_group.hpp"

namespace fms {

namespace {

constexpr int kBwdThreads = 256;  // 4 waves
constexpr int kBwdUnroll = 8;     // source rows in flight per wave (generic kernels)
constexpr int kDocTile = 4096;    // destination rows per LDS tile of bwd_doc_csr
constexpr int kDocThreads = 1024; // threads of bwd_doc_csr (16 waves)
constexpr int kDocUnroll = 4;     // sources in flight per thread (bwd_doc_csr)
constexpr int kDocKeep = 16;      // sources a thread keeps in registers (bwd_doc_csr, one tape read)
constexpr int kDdUnroll = 8;      // sources in flight per row group (bwd_dd_vec)

inline int64_t bcdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }
inline unsigned grid_for(int64_t waves) {
  const int64_t b = bcdiv(waves, kBwdThreads / 64);
  return (unsigned)(b < 1 ? 1 : (b > 1048576 ? 1048576 : b));
}

// Feature element <-> fp32, one element (generic kernels) or one 16-byte
// chunk of kV elements (vector kernels).
struct EF32 {
  static constexpr int kSz = 4, kV = 4;
  __device__ static float ld(const char* p) { return *reinterpret_cast<const float*>(p); }
  __device__ static void st(char* p, float v) { *reinterpret_cast<float*>(p) = v; }
  __device__ static void unpack(const uint4& r, float* x) {
    x[0] = __uint_as_float(r.x);
    x[1] = __uint_as_float(r.y);
    x[2] = __uint_as_float(r.z);
    x[3] = __uint_as_float(r.w);
  }
  __device__ static uint4 pack(const float* x) {
    return make_uint4(__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]),
                      __float_as_uint(x[3]));
  }
  // acc[e] += d * chunk element e, one fused multiply-add each
  __device__ static void fma_chunk(const uint4& r, float d, float* acc) {
    acc[0] = __builtin_fmaf(d, __uint_as_float(r.x), acc[0]);
    acc[1] = __builtin_fmaf(d, __uint_as_float(r.y), acc[1]);
    acc[2] = __builtin_fmaf(d, __uint_as_float(r.z), acc[2]);
    acc[3] = __builtin_fmaf(d, __uint_as_float(r.w), acc[3]);
  }
};
struct EF16 {
  static constexpr int kSz = 2, kV = 8;
  __device__ static float ld(const char* p) { return (float)*reinterpret_cast<const _Float16*>(p); }
  __device__ static void st(char* p, float v) { *reinterpret_cast<_Float16*>(p) = (_Float16)v; }
  __device__ static float lo(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)w); }
  __device__ static float hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  }
  __device__ static uint32_t two(float a, float b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)a) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)b) << 16);
  }
  __device__ static void unpack(const uint4& r, float* x) {
    x[0] = lo(r.x); x[1] = hi(r.x); x[2] = lo(r.y); x[3] = hi(r.y);
    x[4] = lo(r.z); x[5] = hi(r.z); x[6] = lo(r.w); x[7] = hi(r.w);
  }
  __device__ static uint4 pack(const float* x) {
    return make_uint4(two(x[0], x[1]), two(x[2], x[3]), two(x[4], x[5]), two(x[6], x[7]));
  }
  // acc[e] += d * chunk element e; the half -> float widening folds into the
  // fused multiply-add (v_fma_mix_f32 reads either half of a register)
  __device__ static void fma_word(uint32_t w, float d, float& a0, float& a1) {
    a0 = __builtin_fmaf(d, lo(w), a0);
    a1 = __builtin_fmaf(d, hi(w), a1);
  }
  __device__ static void fma_chunk(const uint4& r, float d, float* acc) {
    fma_word(r.x, d, acc[0], acc[1]);
    fma_word(r.y, d, acc[2], acc[3]);
    fma_word(r.z, d, acc[4], acc[5]);
    fma_word(r.w, d, acc[6], acc[7]);
  }
};
struct EBF16 {
  static constexpr int kSz = 2, kV = 8;
  __device__ static float ld(const char* p) {
    return __builtin_bit_cast(float, (uint32_t)*reinterpret_cast<const uint16_t*>(p) << 16);
  }
  __device__ static uint16_t round(float v) {  // round to nearest even
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    return (v != v) ? (uint16_t)0x7FC0u : (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
  }
  __device__ static void st(char* p, float v) { *reinterpret_cast<uint16_t*>(p) = round(v); }
  __device__ static float lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
  __device__ static float hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xFFFF0000u); }
  __device__ static uint32_t two(float a, float b) {
    return (uint32_t)round(a) | ((uint32_t)round(b) << 16);
  }
  __device__ static void unpack(const uint4& r, float* x) {
    x[0] = lo(r.x); x[1] = hi(r.x); x[2] = lo(r.y); x[3] = hi(r.y);
    x[4] = lo(r.z); x[5] = hi(r.z); x[6] = lo(r.w); x[7] = hi(r.w);
  }
  __device__ static uint4 pack(const float* x) {
    return make_uint4(two(x[0], x[1]), two(x[2], x[3]), two(x[4], x[5]), two(x[6], x[7]));
  }
  __device__ static void fma_chunk(const uint4& r, float d, float* acc) {
    acc[0] = __builtin_fmaf(d, lo(r.x), acc[0]);
    acc[1] = __builtin_fmaf(d, hi(r.x), acc[1]);
    acc[2] = __builtin_fmaf(d, lo(r.y), acc[2]);
    acc[3] = __builtin_fmaf(d, hi(r.y), acc[3]);
    acc[4] = __builtin_fmaf(d, lo(r.z), acc[4]);
    acc[5] = __builtin_fmaf(d, hi(r.z), acc[5]);
    acc[6] = __builtin_fmaf(d, lo(r.w), acc[6]);
    acc[7] = __builtin_fmaf(d, hi(r.w), acc[7]);
  }
};

__device__ __forceinline__ int64_t uni64(int64_t v) { return (int64_t)rfl64((uint64_t)v); }
__device__ __forceinline__ float uniform_f(float v) { return __uint_as_float(rfl32(__float_as_uint(v))); }

__device__ __forceinline__ uint4 load16(const char* p) { return *reinterpret_cast<const uint4*>(p); }

// Row geometry of the vector kernels (uniform kernel argument).
struct RowGeo {
  int lg_lr;  // log2(lanes per row)
  int cpl;    // chunks per lane (1 or 2)
  int nch;    // 16-byte chunks per row
  int tpl;    // dQ: tokens per lane
  int tpw;    // dQ: tokens per wave (tpl * 64 / lanes per row, <= 64)
};

// ---- documents as the dD kernels see them -----------------------------------------
// A document owns a run of dD rows (found from the view of its first pair) and
// the pairs that score it; its sources are (pair k, query token t), numbered
// p * rows + t, with list slots from slot0(d) on; qrow0(p) is the first dQ /
// query row of p's query.  npairs / first / slot0 take a wave-uniform
// document; pair / qok / qrow0 take per-lane arguments.
struct DocsInBatch {  // document j: pairs p = j + Bd * i, i < Bq
  int64_t ndocs;
  uint32_t Bd, Bq;
  int rows, Tq;
  const uint8_t* qm;
  __device__ int64_t npairs(int64_t) const { return Bq; }
  __device__ int64_t first(int64_t d) const { return d; }
  __device__ int64_t pair(int64_t d, uint32_t k) const { return d + (int64_t)Bd * k; }
  __device__ int64_t slot0(int64_t d) const { return d * (int64_t)Bq * rows; }
  __device__ bool qok(uint32_t p, int t) const { return !qm || qm[(int64_t)(p / Bd) * Tq + t]; }
  __device__ int64_t qrow0(uint32_t p) const { return (int64_t)(p / Bd) * Tq; }
};
struct DocsPaired {  // document b: pair b
  int64_t ndocs;
  int rows, Tq;
  const uint8_t* qm;
  __device__ int64_t npairs(int64_t) const { return 1; }
  __device__ int64_t first(int64_t d) const { return d; }
  __device__ int64_t pair(int64_t d, uint32_t) const { return d; }
  __device__ int64_t slot0(int64_t d) const { return d * rows; }
  __device__ bool qok(uint32_t p, int t) const { return !qm || qm[(int64_t)p * Tq + t]; }
  __device__ int64_t qrow0(uint32_t p) const { return (int64_t)p * Tq; }
};
struct DocsCand {  // gallery document j: the pairs the document order lists for it
  int64_t ndocs;
  const uint32_t* end;
  const PairRef* order;
  uint32_t C;
  int rows, Tq;
  const uint8_t* qm;
  __device__ int64_t start(int64_t d) const { return d > 0 ? (int64_t)sload(end, d - 1) : 0; }
  __device__ int64_t npairs(int64_t d) const { return (int64_t)sload(end, d) - start(d); }
  __device__ int64_t first(int64_t d) const { return sload(&order[start(d)].p, 0); }
  __device__ int64_t pair(int64_t d, uint32_t k) const { return order[start(d) + k].p; }
  __device__ int64_t slot0(int64_t d) const { return start(d) * rows; }
  __device__ bool qok(uint32_t p, int t) const { return !qm || qm[(int64_t)(p / C) * Tq + t]; }
  __device__ int64_t qrow0(uint32_t p) const { return (int64_t)(p / C) * Tq; }
};
struct DocsPacked {  // document b: pair b; one shared query
  int64_t ndocs;
  int rows;
  const uint8_t* qm;
  __device__ int64_t npairs(int64_t) const { return 1; }
  __device__ int64_t first(int64_t d) const { return d; }
  __device__ int64_t pair(int64_t d, uint32_t) const { return d; }
  __device__ int64_t slot0(int64_t d) const { return d * rows; }
  __device__ bool qok(uint32_t, int t) const { return !qm || qm[t]; }
  __device__ int64_t qrow0(uint32_t) const { return 0; }
};
struct DocsVarlen {  // document segment n: pair n
  int64_t ndocs;
  int rows;
  const int32_t* cu_q;
  int64_t nq;
  __device__ int64_t npairs(int64_t) const { return 1; }
  __device__ int64_t first(int64_t d) const { return d; }
  __device__ int64_t pair(int64_t d, uint32_t) const { return d; }
  __device__ int64_t slot0(int64_t d) const { return d * rows; }
  __device__ bool qok(uint32_t, int) const { return true; }
  __device__ int64_t qrow0(uint32_t p) const { return clamp64((int64_t)cu_q[p] - 1, 0, nq); }
};

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

// ---- vector path: dQ --------------------------------------------------------------------

// Work item = (query group g, token block tb).  kWaveSplit: a workgroup owns
// one (item, split) and its four waves split the split's pairs (the pairs of
// split s of group g are g*G + [s*ps, (s+1)*ps)); otherwise each wave owns
// one item and all its pairs (nsplit == 1).  nsplit == 1 writes dQ in the
// feature type; nsplit > 1 writes fp32 partials part[s][query row][dim].
template <class L, class E, bool kWaveSplit>
__global__ void __launch_bounds__(kBwdThreads) bwd_dq_vec_kernel(
    const L lay, const float* delta, const int32_t* args, int64_t G, int rows, int ntb, int nsplit,
    int64_t nitems, RowGeo geo, int64_t rb, int dim, const char* Qbase, char* dQ, float* part,
    int64_t nq_rows) {
  constexpr int kV = E::kV, kSL = 64 / kV;  // 16-byte slots per lane (64 fp32 accumulators)
  const int lane = threadIdx.x & 63;
  const int w = uniform((int)(threadIdx.x >> 6));
  int64_t item;
  int split;
  if constexpr (kWaveSplit) {
    split = (int)(blockIdx.x % (unsigned)nsplit);
    item = (int64_t)(blockIdx.x / (unsigned)nsplit);
  } else {
    split = 0;
    item = (int64_t)blockIdx.x * 4 + w;
    if (item >= nitems) return;  // whole wave
  }
  const int64_t g = item / ntb;
  const int tb = (int)(item - g * ntb);
  const int64_t gend = (g + 1) * G;
  const int64_t ps = (G + nsplit - 1) / nsplit;
  int64_t pa = std::min(gend, g * G + (int64_t)split * ps);
  int64_t pb = std::min(gend, pa + ps);
  if constexpr (kWaveSplit) {
    const int64_t q = (pb - pa + 3) / 4;
    pa = std::min(pb, pa + w * q);
    pb = std::min(pb, pa + q);
  }
  const PairView v0 = uniform_view(lay.get(g * G));
  const int lg = geo.lg_lr, rpi = 64 >> lg;
  const int gid = lane >> lg, c0 = lane & ((1 << lg) - 1);
  const int t0 = tb * geo.tpw;
  const int tend = std::min(v0.tq, t0 + geo.tpw);
  // slot s of a lane: token t0 + srcl(s), 16-byte chunk ch(s) of the row
  const int cm = geo.cpl - 1, cs = geo.cpl - 1 == 0 ? 0 : 1;
  auto srcl = [&](int s) { return gid + rpi * (s >> cs); };
  auto choff = [&](int s) { return (c0 + ((s & cm) << lg)) * 16; };
  uint32_t actm = 0u, wrm = 0u;  // slot bits: accumulate / write
#pragma unroll
  for (int s = 0; s < kSL; ++s) {
    const int t = t0 + srcl(s);
    const bool wr = (s >> cs) < geo.tpl && t < tend && choff(s) < geo.nch * 16;
    wrm |= (uint32_t)wr << s;
    actm |= (uint32_t)(wr && (v0.qm == nullptr || v0.qm[t] != 0)) << s;
  }
  float acc[kSL][kV];
#pragma unroll
  for (int s = 0; s < kSL; ++s)
#pragma unroll
    for (int e = 0; e < kV; ++e) acc[s][e] = 0.0f;
  const bool tlane = lane < geo.tpw && t0 + lane < tend;
  // Software pipeline: the view, delta and tape block of pair p + 1 are
  // loaded while pair p's rows are gathered.
  PairView vnext;
  float dnext = 0.0f;
  int tnext = 0;
  // Items start at different pairs of their range (step k takes pair
  // pa + (rot + k) mod len), so the waves that share documents do not
  // request them in lockstep.
  const int64_t len = pb - pa;
  const int64_t rot = len > 0 ? (item * 2) % len : 0;
  auto pair_at = [&](int64_t k) {
    int64_t q = rot + k;
    if (q >= len) q -= len;
    return pa + q;
  };
  if (len > 0) {
    const int64_t p0 = pair_at(0);
    vnext = uniform_view(lay.get(p0));
    dnext = sload(delta, p0);
    tnext = tlane ? args[p0 * rows + t0 + lane] : 0;
  }
  for (int64_t k = 0; k < len; ++k) {
    const PairView v = vnext;
    const float dl = dnext;
    const int tv = tnext;
    if (k + 1 < len) {
      const int64_t pn = pair_at(k + 1);
      vnext = uniform_view(lay.get(pn));
      dnext = sload(delta, pn);
      if (tlane) tnext = args[pn * rows + t0 + lane];
    }
    if (!v.valid || dl == 0.0f) continue;
    uint4 raw[kSL];
#pragma unroll
    for (int s = 0; s < kSL; ++s) {
      const int u = __shfl(tv, srcl(s));
      raw[s] = (((actm >> s) & 1u) && u >= 1 && u <= v.td)
                   ? load16(v.d + (int64_t)(u - 1) * rb + choff(s))
                   : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int s = 0; s < kSL; ++s) {
      E::fma_chunk(raw[s], dl, acc[s]);
    }
  }
  if constexpr (kWaveSplit) {  // (w0 + w2) + (w1 + w3), element-major LDS rows of 64 lanes
    __shared__ float red[2][64 * 64];
    if (w >= 2) {
#pragma unroll
      for (int s = 0; s < kSL; ++s)
#pragma unroll
        for (int e = 0; e < kV; ++e) red[w - 2][(s * kV + e) * 64 + lane] = acc[s][e];
    }
    __syncthreads();
    if (w < 2) {
#pragma unroll
      for (int s = 0; s < kSL; ++s)
#pragma unroll
        for (int e = 0; e < kV; ++e) acc[s][e] += red[w][(s * kV + e) * 64 + lane];
    }
    __syncthreads();
    if (w == 1) {
#pragma unroll
      for (int s = 0; s < kSL; ++s)
#pragma unroll
        for (int e = 0; e < kV; ++e) red[0][(s * kV + e) * 64 + lane] = acc[s][e];
    }
    __syncthreads();
    if (w != 0) return;
#pragma unroll
    for (int s = 0; s < kSL; ++s)
#pragma unroll
      for (int e = 0; e < kV; ++e) acc[s][e] += red[0][(s * kV + e) * 64 + lane];
  }
  const int64_t qrow0 = (int64_t)(v0.q - Qbase) / rb;
#pragma unroll
  for (int s = 0; s < kSL; ++s) {
    if (!((wrm >> s) & 1u)) continue;
    const int t = t0 + srcl(s);
    if (nsplit == 1) {
      *reinterpret_cast<uint4*>(dQ + (qrow0 + t) * rb + choff(s)) = E::pack(acc[s]);
    } else {
      float* dst = part + ((int64_t)split * nq_rows + qrow0 + t) * dim + (choff(s) / 16) * kV;
#pragma unroll
      for (int e = 0; e < kV; e += 4)
        *reinterpret_cast<float4*>(dst + e) =
            make_float4(acc[s][e], acc[s][e + 1], acc[s][e + 2], acc[s][e + 3]);
    }
  }
}

// In-batch dQ with the documents staged in LDS.  A workgroup of 16 waves owns
// 16 work items (query i, token block) and document share s (documents
// [s*ps, (s+1)*ps), split index = block index mod nsplit as above); every
// document of the share is copied once into LDS by direct buffer-to-LDS
// loads and the 16 queries gather their chosen rows from there, so a
// document row leaves L2 once per workgroup instead of once per (query,
// token) that chose it.  Three LDS buffers: documents j + 1 and j + 2 are in
// flight while j is gathered (the copy latency is several gathers long).
constexpr int kIbThreads = 1024;
constexpr int kIbItems = kIbThreads / 64;
constexpr int kIbStagePer = 3;                                // copies per wave per document
constexpr int kIbStageChunks = kIbStagePer * kIbThreads;      // 48 KB per LDS buffer
constexpr int kIbBufs = 3;

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Wait until at most kVm of this wave's loads are outstanding (the
// buffer-to-LDS copies among them; loads complete in issue order), then meet
// the workgroup: every wave's finished copies are visible after.
template <int kVm>
__device__ __forceinline__ void dma_wait_barrier() {
  static_assert(kVm >= 0 && kVm < 16, "vmcnt field");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0070 | kVm);  // vmcnt(kVm) lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p);
}

// Four 16-byte LDS reads, complete on return.
__device__ __forceinline__ void lds_read4(uint4 (&r)[4], const uint32_t (&a)[4]) {
  asm volatile(
      "ds_read_b128 %0, %4\n\t"
      "ds_read_b128 %1, %5\n\t"
      "ds_read_b128 %2, %6\n\t"
      "ds_read_b128 %3, %7\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
      : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]));
}

template <class E, int kCPL>
__global__ void __launch_bounds__(kIbThreads) bwd_dq_ib_kernel(
    const LayInBatch lay, const float* delta, const int32_t* args, int rows, int ntb, int nsplit,
    int64_t nitems, RowGeo geo, int64_t rb, int dim, char* dQ, float* part, int64_t nq_rows) {
  constexpr int kV = E::kV, kSL = 64 / kV, kHalf = kSL / 2;
  constexpr int kOps = kIbStagePer + 2;  // loads a wave issues per document
  // Three separate arrays (not one indexed array): the compiler then sees that
  // a copy into one buffer cannot alias reads of another and does not wait
  // for the copy before each read.
  __shared__ uint4 dbuf0[kIbStageChunks], dbuf1[kIbStageChunks], dbuf2[kIbStageChunks];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int split = (int)(blockIdx.x % (unsigned)nsplit);
  const int64_t item = (int64_t)(blockIdx.x / (unsigned)nsplit) * kIbItems + w;
  const bool live = item < nitems;  // (a dead wave still copies and meets the barriers)
  const int64_t i = live ? item / ntb : 0;
  const int tb = live ? (int)(item - i * ntb) : 0;
  const int64_t Bd = lay.Bd;
  const int td = lay.Td, nch = geo.nch;
  const uint32_t stage_bytes = (uint32_t)(td * rb);
  const int64_t ps = (Bd + nsplit - 1) / nsplit;
  const int64_t ja = std::min<int64_t>(Bd, (int64_t)split * ps), jb = std::min<int64_t>(Bd, ja + ps);
  const int lg = geo.lg_lr, rpi = 64 >> lg;
  const int gid = lane >> lg, c0 = lane & ((1 << lg) - 1);
  const int t0 = tb * geo.tpw;
  const int tend = live ? std::min(lay.Tq, t0 + geo.tpw) : 0;
  const uint8_t* qm = lay.qm ? lay.qm + i * lay.Tq : nullptr;
  constexpr int cs = kCPL == 2 ? 1 : 0;
  auto srcl = [&](int s) { return gid + rpi * (s >> cs); };
  auto chunk = [&](int s) { return c0 + ((s & (kCPL - 1)) << lg); };
  uint32_t actm = 0u, wrm = 0u;
#pragma unroll
  for (int s = 0; s < kSL; ++s) {
    const int t = t0 + srcl(s);
    const bool wr = (s >> cs) < geo.tpl && t < tend && chunk(s) < nch;
    wrm |= (uint32_t)wr << s;
    actm |= (uint32_t)(wr && (qm == nullptr || qm[t] != 0)) << s;
  }
  float acc[kSL][kV];
#pragma unroll
  for (int s = 0; s < kSL; ++s)
#pragma unroll
    for (int e = 0; e < kV; ++e) acc[s][e] = 0.0f;
  const bool tlane = lane < geo.tpw && t0 + lane < tend;
  const int tcol = std::min(t0 + lane, rows - 1);  // in bounds for every lane
  // Document j -> LDS buffer b (wave w copies 16-byte chunks (k*16 + w)*64 +
  // lane; a copy past the document reads 0 from the resource's range check),
  // and the pair (i, j)'s delta and tape block.  Always exactly kOps loads.
  // Workgroups of one share start at different documents (step k reads
  // document ja + (rot + k) mod len), so the share's documents are requested
  // from HBM by many workgroups at once rather than in lockstep.
  const int64_t len = jb - ja;
  const int64_t rot = len > 0 ? ((int64_t)(blockIdx.x / (unsigned)nsplit) * 2) % len : 0;
  auto fetch = [&](int64_t k, uint4* buf, float& dl, int& tv) {
    int64_t j = rot + k;
    if (j >= len) j -= len;
    j += ja;
    const rsrc_t r = make_rsrc_u(lay.D + j * lay.dbytes, stage_bytes);
#pragma unroll
    for (int k = 0; k < kIbStagePer; ++k) {
      const int base = (k * kIbItems + w) * 64;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)(buf + base), 16, (base + lane) * 16,
                                               0, 0, 0);
    }
    const int64_t p = j + Bd * i;
    dl = delta[p];
    tv = args[p * rows + tcol];
  };
  // The LDS reads go through lds_read4: the compiler cannot tell which buffer
  // a copy targets once the rotation wraps, and would otherwise wait for the
  // copies in flight (the next two documents) before each read.  The step
  // barrier already orders them: document j's copy completed before step j.
  auto gather = [&](const uint4* rowbase, float dlv, int tvv) {
    const float dl = live ? uniform_f(dlv) : 0.0f;
    const int tv = tlane ? tvv : 0;
    if (dl == 0.0f) return;
    const uint32_t lbase = lds_addr(rowbase);
#pragma unroll
    for (int h = 0; h < kSL / 4; ++h) {
      uint32_t addr[4];
      bool ok[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int s = h * 4 + q;
        const int u = __shfl(tv, srcl(s));
        ok[q] = ((actm >> s) & 1u) && u >= 1 && u <= td;
        addr[q] = lbase + (uint32_t)(((ok[q] ? u - 1 : 0) * nch + chunk(s)) * 16);
      }
      uint4 raw[4];
      lds_read4(raw, addr);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        E::fma_chunk(raw[q], ok[q] ? dl : 0.0f, acc[h * 4 + q]);
      }
    }
  };
  // Steps 0, 1, 2, ... rotate through buffers 0, 1, 2 and register sets 0, 1,
  // 2 (delta and tape block, loaded two steps ahead).  Every step issues the
  // same loads (past the share's end it re-fetches the last step's document
  // into the buffer just retired), so each wait is one count.
  float d0 = 0.0f, d1 = 0.0f, d2 = 0.0f;
  int v0r = 0, v1r = 0, v2r = 0;
  if (len > 0) {
    fetch(0, dbuf0, d0, v0r);
    fetch(std::min<int64_t>(1, len - 1), dbuf1, d1, v1r);
  }
  dma_wait_barrier<kOps>();  // document ja ready
  // step k: gather from `rd` with (dc, tc) (nothing past the share's end);
  // fetch step k + 2's document into `wr` / (dn, tn).  The loop body is straight-line (the
  // last round pads with empty steps) so the compiler's own load counting
  // stays exact across the back edge.
  auto step = [&](int64_t k, const uint4* rd, uint4* wr, float& dc, int& tc, float& dn, int& tn) {
    const float dcur = k < len ? dc : 0.0f;
    const int tcur = tc;
    fetch(std::min(k + 2, len - 1), wr, dn, tn);  // `wr` was read at step k - 1
    gather(rd, dcur, tcur);
    dma_wait_barrier<kOps>();  // k + 1 ready; k + 2 may stay in flight
  };
  for (int64_t k = 0; k < len; k += 3) {
    step(k, dbuf0, dbuf2, d0, v0r, d2, v2r);
    step(k + 1, dbuf1, dbuf0, d1, v1r, d0, v0r);
    step(k + 2, dbuf2, dbuf1, d2, v2r, d1, v1r);
  }
  dma_wait_barrier<0>();  // no copy may land after the workgroup's LDS is released
  if (!live) return;
  const int64_t qrow0 = i * lay.Tq;
#pragma unroll
  for (int s = 0; s < kSL; ++s) {
    if (!((wrm >> s) & 1u)) continue;
    const int t = t0 + srcl(s);
    if (nsplit == 1) {
      *reinterpret_cast<uint4*>(dQ + (qrow0 + t) * rb + chunk(s) * 16) = E::pack(acc[s]);
    } else {
      float* dst = part + ((int64_t)split * nq_rows + qrow0 + t) * dim + chunk(s) * kV;
#pragma unroll
      for (int e = 0; e < kV; e += 4)
        *reinterpret_cast<float4*>(dst + e) =
            make_float4(acc[s][e], acc[s][e + 1], acc[s][e + 2], acc[s][e + 3]);
    }
  }
}

// dQ chunk c (16 bytes of the feature type) = sum over splits, in split order,
// of the fp32 partials.
template <class E>
__global__ void __launch_bounds__(kBwdThreads) bwd_dq_reduce_kernel(const float* part, int nsplit,
                                                                   int64_t nchunks, int64_t stride,
                                                                   char* dQ) {
  constexpr int kV = E::kV;
  const int64_t step = (int64_t)gridDim.x * kBwdThreads;
  for (int64_t c = (int64_t)blockIdx.x * kBwdThreads + threadIdx.x; c < nchunks; c += step) {
    float acc[kV];
#pragma unroll
    for (int e = 0; e < kV; ++e) acc[e] = 0.0f;
    for (int s = 0; s < nsplit; ++s) {
      const float* src = part + (int64_t)s * stride + c * kV;
#pragma unroll
      for (int e = 0; e < kV; e += 4) {
        const float4 x = *reinterpret_cast<const float4*>(src + e);
        acc[e] += x.x;
        acc[e + 1] += x.y;
        acc[e + 2] += x.z;
        acc[e + 3] += x.w;
      }
    }
    *reinterpret_cast<uint4*>(dQ + c * 16) = E::pack(acc);
  }
}

// ---- vector path: dD ---------------------------------------------------------------------

// Exclusive scan of cnt[0, n) (n <= kDocTile) into out[]; returns the total.
// Every thread of the (kDocThreads) block calls it.
__device__ uint32_t block_scan_tile(const uint32_t* cnt, uint32_t* out, int n) {
  constexpr int kWaves = kDocThreads / 64, kPer = kDocTile / kDocThreads;
  __shared__ uint32_t wsum[kWaves];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int i0 = tid * kPer;
  uint32_t loc[kPer];
  uint32_t sum = 0u;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    loc[j] = (i0 + j < n) ? cnt[i0 + j] : 0u;
    sum += loc[j];
  }
  uint32_t x = sum;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) wsum[w] = x;
  __syncthreads();
  uint32_t before = x - sum, total = 0u;
#pragma unroll
  for (int j = 0; j < kWaves; ++j) {
    if (j < w) before += wsum[j];
    total += wsum[j];
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    if (i0 + j < n) out[i0 + j] = before;
    before += loc[j];
  }
  __syncthreads();  // wsum and out are read by the caller / next call
  return total;
}

// Sources f = k * tq + t (pair k of the document, query token t) of one
// document, kDocUnroll per thread at a time: calls fn(p, t, u) for those with
// a nonzero delta, a true qmask and a tape entry u0 < u <= u0 + ut.
template <class Docs, class Fn>
__device__ __forceinline__ void for_doc_sources(const Docs& docs, int64_t d, uint32_t nsrc, int tq,
                                                const float* delta, const int32_t* args, int rows,
                                                int u0, int ut, Fn fn) {
  for (uint32_t f0 = 0; f0 < nsrc; f0 += kDocUnroll * kDocThreads) {
    int64_t p[kDocUnroll];
    int t[kDocUnroll], u[kDocUnroll];
    bool ok[kDocUnroll];
#pragma unroll
    for (int q = 0; q < kDocUnroll; ++q) {
      const uint32_t f = f0 + q * kDocThreads + threadIdx.x;
      ok[q] = f < nsrc;
      const uint32_t k = ok[q] ? f / (uint32_t)tq : 0u;
      t[q] = ok[q] ? (int)(f - k * (uint32_t)tq) : 0;
      p[q] = docs.pair(d, k);
      u[q] = ok[q] ? args[p[q] * rows + t[q]] : 0;
    }
#pragma unroll
    for (int q = 0; q < kDocUnroll; ++q) {
      if (ok[q] && u[q] > u0 && u[q] <= u0 + ut && delta[p[q]] != 0.0f &&
          docs.qok((uint32_t)p[q], t[q]))
        fn(p[q], t[q], u[q]);
    }
  }
}

// One workgroup per document (grid-stride): sources of the document with a
// nonzero delta, a true qmask and a tape entry 1 <= u <= td, sorted by u in
// LDS tiles of kDocTile rows; writes rstart/rcount of the document's rows and
// each source as (query row, delta bits) into list[slot0(d) ...].
template <class L, class Docs>
__global__ void __launch_bounds__(kDocThreads) bwd_doc_csr_kernel(const L lay, const Docs docs,
                                                                 const float* delta,
                                                                 const int32_t* args, int rows,
                                                                 const char* Dbase, int64_t rb,
                                                                 uint32_t* rstart, uint32_t* rcount,
                                                                 uint2* list) {
  __shared__ uint32_t cnt[kDocTile], cur[kDocTile];
  const int tid = threadIdx.x;
  for (int64_t d = blockIdx.x; d < docs.ndocs; d += gridDim.x) {
    const int64_t np = uni64(docs.npairs(d));
    if (np == 0) continue;
    const PairView v = uniform_view(lay.get(uni64(docs.first(d))));
    const int64_t r0 = (int64_t)(v.d - Dbase) / rb;
    const int td = v.td, tq = v.tq;
    const uint32_t nsrc = (uint32_t)(np * tq);
    int64_t slot = docs.slot0(d);
    if (nsrc <= (uint32_t)(kDocKeep * kDocThreads) && td <= kDocTile) {
      // One tape read: each thread keeps its sources (row, (query row, delta))
      // in registers between the count and the fill.
      uint32_t key[kDocKeep];
      uint2 val[kDocKeep];
#pragma unroll
      for (int q = 0; q < kDocKeep; ++q) {
        const uint32_t f = q * kDocThreads + tid;
        const bool in = f < nsrc;
        const uint32_t k = in ? f / (uint32_t)tq : 0u;
        const int t = in ? (int)(f - k * (uint32_t)tq) : 0;
        const int64_t p = docs.pair(d, k);
        const int u = in ? args[p * rows + t] : 0;
        const float dl = delta[p];
        const bool ok = in && u >= 1 && u <= td && dl != 0.0f && docs.qok((uint32_t)p, t);
        key[q] = ok ? (uint32_t)(u - 1) : 0xFFFFFFFFu;
        val[q] = make_uint2((uint32_t)(docs.qrow0((uint32_t)p) + t), __float_as_uint(dl));
      }
      for (int i = tid; i < td; i += kDocThreads) cnt[i] = 0u;
      __syncthreads();
#pragma unroll
      for (int q = 0; q < kDocKeep; ++q)
        if (key[q] != 0xFFFFFFFFu) atomicAdd(&cnt[key[q]], 1u);
      __syncthreads();
      block_scan_tile(cnt, cur, td);
      for (int i = tid; i < td; i += kDocThreads) {
        rstart[r0 + i] = (uint32_t)slot + cur[i];
        rcount[r0 + i] = cnt[i];
      }
      __syncthreads();  // every start read before the fill moves the cursors
#pragma unroll
      for (int q = 0; q < kDocKeep; ++q)
        if (key[q] != 0xFFFFFFFFu) list[slot + atomicAdd(&cur[key[q]], 1u)] = val[q];
      __syncthreads();
      continue;
    }
    for (int u0 = 0; u0 < td; u0 += kDocTile) {
      const int ut = std::min(kDocTile, td - u0);
      for (int i = tid; i < ut; i += kDocThreads) cnt[i] = 0u;
      __syncthreads();
      for_doc_sources(docs, d, nsrc, tq, delta, args, rows, u0, ut,
                      [&](int64_t, int, int u) { atomicAdd(&cnt[u - 1 - u0], 1u); });
      __syncthreads();
      const uint32_t total = block_scan_tile(cnt, cur, ut);
      for (int i = tid; i < ut; i += kDocThreads) {
        rstart[r0 + u0 + i] = (uint32_t)slot + cur[i];
        rcount[r0 + u0 + i] = cnt[i];
      }
      __syncthreads();  // every start read before the fill moves the cursors
      for_doc_sources(docs, d, nsrc, tq, delta, args, rows, u0, ut, [&](int64_t p, int t, int u) {
        const uint32_t pos = atomicAdd(&cur[u - 1 - u0], 1u);
        list[slot + pos] = make_uint2((uint32_t)(docs.qrow0((uint32_t)p) + t), __float_as_uint(delta[p]));
      });
      __syncthreads();
      slot += total;
    }
  }
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = std::max(v, (uint32_t)__shfl_xor((int)v, o));
  return v;
}

// dD row r = sum over its listed sources of delta_p * Q[query row].  A wave
// covers 64 / Lr consecutive rows, Lr lanes per row; every row of [0, nrows)
// is written.  Each lane of a row group reads one list entry of a batch of Lr
// (the next batch is loaded while this one is gathered); the group gathers
// the batch's query rows kDdUnroll at a time, taking row and delta by
// ds_bpermute.  Entries are checked against the list and the query rows, so
// a malformed tape or cu cannot send a read out of bounds.
template <class E, int kCPL>
__global__ void __launch_bounds__(kBwdThreads) bwd_dd_vec_kernel(
    const uint32_t* rstart, const uint32_t* rcount, const uint2* list, uint32_t nlist,
    int64_t nrows, RowGeo geo, int64_t rb, const char* Qbase, int64_t nq_rows, char* dD) {
  constexpr int kV = E::kV;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int lg = geo.lg_lr, lr = 1 << lg, rpi = 64 >> lg;
  const int gid = lane >> lg, c0 = lane & (lr - 1), gbase = gid << lg;
  const int64_t per_block = 4 * (int64_t)rpi;
  auto fetch = [&](uint32_t jj, uint32_t n, uint32_t base) {
    return (jj < n && base + jj < nlist) ? list[base + jj] : make_uint2(0u, 0u);
  };
  for (int64_t rb0 = (int64_t)blockIdx.x * per_block; rb0 < nrows; rb0 += (int64_t)gridDim.x * per_block) {
    const int64_t r = rb0 + w * rpi + gid;
    const bool rv = r < nrows;
    const uint32_t n = rv ? rcount[r] : 0u;
    const uint32_t base = n ? rstart[r] : 0u;
    const uint32_t nmax = wave_max_u32(n);
    float acc[kCPL][kV];
#pragma unroll
    for (int cc = 0; cc < kCPL; ++cc)
#pragma unroll
      for (int e = 0; e < kV; ++e) acc[cc][e] = 0.0f;
    uint2 ent = fetch(c0, n, base);
    for (uint32_t j = 0; j < nmax; j += lr) {
      const bool ok = ent.x < nq_rows;
      const float dlane = ok ? __uint_as_float(ent.y) : 0.0f;
      const int qlane = ok ? (int)ent.x : 0;
      ent = fetch(j + lr + c0, n, base);  // next batch
      const uint32_t nb = std::min<uint32_t>(lr, nmax - j);
      for (uint32_t i0 = 0; i0 < nb; i0 += kDdUnroll) {
        uint4 raw[kDdUnroll][kCPL];
        float dl[kDdUnroll];
#pragma unroll
        for (int i = 0; i < kDdUnroll; ++i) {
          const int sl = gbase + (int)((i0 + i) & (uint32_t)(lr - 1));
          dl[i] = (i0 + i < (uint32_t)lr) ? __shfl(dlane, sl) : 0.0f;
          const char* qa = Qbase + (int64_t)__shfl(qlane, sl) * rb;
#pragma unroll
          for (int cc = 0; cc < kCPL; ++cc) {
            const int ch = c0 + (cc << lg);
            raw[i][cc] = (dl[i] != 0.0f && cc < geo.cpl && ch < geo.nch) ? load16(qa + ch * 16)
                                                                        : make_uint4(0u, 0u, 0u, 0u);
          }
        }
#pragma unroll
        for (int i = 0; i < kDdUnroll; ++i)
#pragma unroll
          for (int cc = 0; cc < kCPL; ++cc) {
            E::fma_chunk(raw[i][cc], dl[i], acc[cc]);
          }
      }
    }
    if (rv) {
#pragma unroll
      for (int cc = 0; cc < kCPL; ++cc) {
        const int ch = c0 + (cc << lg);
        if (cc < geo.cpl && ch < geo.nch)
          *reinterpret_cast<uint4*>(dD + r * rb + ch * 16) = E::pack(acc[cc]);
      }
    }
  }
}

// ---- in-batch, 16-bit features: the feature-half path --------------------------------------
// The kernels above gather whole rows.  In-batch, that sends every XCD after
// all of Q for dD (Bq * Tq rows, about one XCD's L2) and leaves one fp32 dQ
// partial per XCD.  Here each workgroup works on one half of the feature row,
// h = XCD index & 1 (workgroups are dealt to the 8 XCDs round-robin by
// workgroup index), so an XCD reads one half of Q (dD) or one half of one
// quarter of D (dQ), a fraction of its L2:
//   bwd_ib_compact  the tape as one byte per source, document-major:
//                   ct[j][i][t] = u, or 0 where there is no source (masked
//                   token, entry outside 1..Td, delta 0); query rows of Tqp
//                   (Tq rounded up to 4) bytes, documents ct_stride bytes
//                   apart; and delta document-major, dT[j][i].
//   bwd_ib_dd       a workgroup per (document, half): counting sort of the
//                   document's sources by row in LDS (one counter set per
//                   wave), then each row's query half-rows summed in
//                   registers, in list order.  Every row is written.
//   bwd_ib_dq       a workgroup per (16 work items, half, document quarter):
//                   the quarter's half-rows staged through LDS as in
//                   bwd_dq_ib; one fp32 partial per quarter, summed in
//                   quarter order by bwd_dq_reduce.  Deterministic.
constexpr int kIbxMaxSrc = 32768;          // key bytes per document (Bq * Tqp)
constexpr int kIbxMaxBq = 4096;            // queries
constexpr int kIbxDdThreads = 512;         // bwd_ib_dd: 8 waves
constexpr int kIbxDdWaves = kIbxDdThreads / 64;
constexpr int kIbxKeep = kIbxMaxSrc / 16 / kIbxDdThreads;  // 16-byte key chunks a thread keeps
constexpr int kIbxDdUnroll = 8;            // query half-rows in flight per row group
constexpr int kIbxStage = 3 * kIbThreads;  // 16-byte chunks per LDS buffer of bwd_ib_dq (48 KB)
constexpr int kIbxQuarters = 4;            // document quarters of bwd_ib_dq
constexpr int kIbxDdLdsMax = 65536;        // dynamic LDS of bwd_ib_dd

struct IbxGeo {
  int64_t Bd;
  int Bq, Tq, Tqp, Td;
  int64_t ct_stride;  // bytes of ct per document: Bq * Tqp rounded up to 16
  uint32_t mq, mqp;   // ibx_magic(Tq), ibx_magic(Tqp)
};

// n / d for n < 2^16, d < 2^16, with m = ceil(2^32 / d) (d >= 2) or 0 (d = 1):
// the error of n * m / 2^32 against n / d is n * (m * d - 2^32) / (d * 2^32) < 1 / d.
__device__ __forceinline__ uint32_t ibx_div(uint32_t n, uint32_t m) {
  return m == 0u ? n : __umulhi(n, m);
}

// Workgroup (x, y) covers dwords y * kIbxCompactSpan .. + kIbxCompactSpan - 1 of
// document j's bytes; dword k holds tokens 4 * (k % (Tqp / 4)) .. + 3 of query
// k / (Tqp / 4).  delta_p = Delta[p] * inv_n[i] in fp32, as bwd_delta computes
// it.  Documents 512 m + 64 x' .. + 63 go to XCD x' (workgroup index x mod 8),
// so the 64 documents whose cotangents share a 128-byte line of Delta meet in
// one L2.  Each thread loads its kIbxCompactPer dwords' tape entries before it
// combines any.  vec4: the tape rows start 16-byte aligned (Tq a multiple of
// 4, aligned buffer).
constexpr int kIbxCompactPer = 4;
constexpr int kIbxCompactSpan = kIbxCompactPer * kBwdThreads;
constexpr int kIbxCompactGroup = 64;  // documents per XCD in a row of 8 * 64
template <class E>
__global__ void __launch_bounds__(kBwdThreads) bwd_ib_compact_kernel(const int32_t* args,
                                                                     const char* Delta,
                                                                     const char* inv_n,
                                                                     const uint8_t* qm, IbxGeo g,
                                                                     int vec4, uint32_t* ct,
                                                                     float* dT) {
  const int64_t n = blockIdx.x >> 3;
  const int64_t j = (n / kIbxCompactGroup) * (8 * kIbxCompactGroup) +
                    (int64_t)(blockIdx.x & 7) * kIbxCompactGroup + n % kIbxCompactGroup;
  if (j >= g.Bd) return;
  auto delta = [&](int64_t p, int i) {
    return E::ld(Delta + p * E::kSz) * (inv_n ? E::ld(inv_n + (int64_t)i * E::kSz) : 1.0f);
  };
  const int tq4 = g.Tqp >> 2;
  const int nk = (int)(g.ct_stride >> 2), nv = g.Bq * tq4;
  uint32_t* out = ct + j * nk;
  const int k0 = (int)blockIdx.y * kIbxCompactSpan + (int)threadIdx.x;
  int u[kIbxCompactPer][4], iq[kIbxCompactPer], tq[kIbxCompactPer];
  float dl[kIbxCompactPer];
#pragma unroll
  for (int q = 0; q < kIbxCompactPer; ++q) {
    const int k = k0 + q * kBwdThreads;
    const bool in = k < nv;
    const int i = in ? k / tq4 : 0, t0 = in ? (k - i * tq4) * 4 : g.Tq;
    iq[q] = i;
    tq[q] = t0;
    const int64_t p = j + g.Bd * i;
    dl[q] = in ? delta(p, i) : 0.0f;
    const int32_t* a = args + p * g.Tq;
    if (in && vec4) {
      const int4 v = *reinterpret_cast<const int4*>(a + t0);
      u[q][0] = v.x;
      u[q][1] = v.y;
      u[q][2] = v.z;
      u[q][3] = v.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) u[q][e] = t0 + e < g.Tq ? a[t0 + e] : 0;
    }
  }
#pragma unroll
  for (int q = 0; q < kIbxCompactPer; ++q) {
    const int k = k0 + q * kBwdThreads;
    uint32_t word = 0u;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = tq[q] + e;
      const bool ok = t < g.Tq && u[q][e] >= 1 && u[q][e] <= g.Td && dl[q] != 0.0f &&
                      (qm == nullptr || qm[(int64_t)iq[q] * g.Tq + t] != 0);
      word |= (ok ? (uint32_t)u[q][e] : 0u) << (8 * e);
    }
    if (k < nk) out[k] = word;
  }
  if (blockIdx.y == 0)
    for (int i = threadIdx.x; i < g.Bq; i += kBwdThreads) dT[j * g.Bq + i] = delta(j + g.Bd * i, i);
}

// dD rows of document j, feature half h.  Dynamic LDS: counters [waves / 2][256]
// (two 16-bit counters a word, waves 2v and 2v + 1: no count or cursor passes
// Bq * Tqp <= 32768), row starts [256], delta [Bq + 1] (the last 0), list
// [Bq * Tqp] (uint16 query rows).  kHC: 16-byte chunks per half row; kHC lanes
// per row, 64 / kHC rows per wave.
// Waves per SIMD asked of bwd_ib_dd: 8 (64 registers, and 4 workgroups per CU
// when the LDS allows) where that costs no spill, else the compiler's choice.
template <class E, int kHC>
struct IbxDdWaves {
  static constexpr int kMin = (std::is_same<E, EF16>::value && kHC <= 8) ? 8 : 1;
};

template <class E, int kHC>
__global__ void __launch_bounds__(kIbxDdThreads)
    __attribute__((amdgpu_waves_per_eu(IbxDdWaves<E, kHC>::kMin, 8))) bwd_ib_dd_kernel(const uint32_t* ct,
                                                                 const float* dT, IbxGeo g,
                                                                 int64_t rb, const char* Q,
                                                                 int64_t q_bytes, char* dD) {
  constexpr int kRG = 64 / kHC;
  constexpr int kCw = kIbxDdWaves / 2;        // counter sets (one per wave pair)
  constexpr int kB = kHC < 8 ? kHC : 8;       // query half-rows in flight per row group
  constexpr int kSw = 0x1F & ~(kHC - 1);      // ds_swizzle and-mask: the group's first lane
  extern __shared__ uint32_t ibx_smem[];
  __shared__ uint32_t wtot[4];
  uint32_t* cnt = ibx_smem;
  uint32_t* rs = cnt + 256 * kCw;
  float* dl = reinterpret_cast<float*>(rs + 256);
  uint16_t* list = reinterpret_cast<uint16_t*>(dl + g.Bq + 1);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int xcd = blockIdx.x & 7, h = xcd & 1;
  const int64_t j = (int64_t)(blockIdx.x >> 3) * 4 + (xcd >> 1);
  if (j >= g.Bd) return;
  const int nchunk = (int)(g.ct_stride >> 4);
  const uint4* kj = reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(ct) + j * g.ct_stride);
  uint4 key[kIbxKeep];
#pragma unroll
  for (int q = 0; q < kIbxKeep; ++q) {
    const int c = q * kIbxDdThreads + tid;
    key[q] = c < nchunk ? kj[c] : make_uint4(0u, 0u, 0u, 0u);
  }
  for (int x = tid; x < 256 * kCw; x += kIbxDdThreads) cnt[x] = 0u;
  const float* dtj = dT + j * g.Bq;
  for (int x = tid; x <= g.Bq; x += kIbxDdThreads) dl[x] = x < g.Bq ? dtj[x] : 0.0f;
  __syncthreads();
  uint32_t* cw = cnt + (w >> 1) * 256;
  const int csh = 16 * (w & 1);
  // fn(u, f) for every source of this thread: row u (1-based), key byte f of the document
  auto each = [&](auto fn) {
#pragma unroll
    for (int q = 0; q < kIbxKeep; ++q) {
      if (q * kIbxDdThreads >= nchunk) break;  // (uniform)
      const uint32_t kw[4] = {key[q].x, key[q].y, key[q].z, key[q].w};
      const uint32_t f0 = (uint32_t)(q * kIbxDdThreads + tid) * 16u;
#pragma unroll
      for (int d = 0; d < 4; ++d)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const uint32_t u = (kw[d] >> (8 * b)) & 255u;
          if (u != 0u) fn(u, f0 + (uint32_t)(d * 4 + b));
        }
    }
  };
  each([&](uint32_t u, uint32_t) { atomicAdd(&cw[u], 1u << csh); });
  __syncthreads();
  // Row r = u - 1 starts at rs[r]; wave v's sources of row r fill from
  // rs[r] + (those of waves < v), its counter becoming that cursor.
  uint32_t tot = 0u, x = 0u;
  uint32_t cv[kIbxDdWaves];
  if (tid < 256) {
#pragma unroll
    for (int v = 0; v < kIbxDdWaves; ++v)
      cv[v] = tid < g.Td ? (cnt[(v >> 1) * 256 + tid + 1] >> (16 * (v & 1))) & 0xFFFFu : 0u;
#pragma unroll
    for (int v = 0; v < kIbxDdWaves; ++v) tot += cv[v];
    x = tot;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t y = __shfl_up(x, o);
      if (lane >= o) x += y;
    }
    if (lane == 63) wtot[w] = x;
  }
  __syncthreads();
  if (tid < g.Td) {
    uint32_t run = x - tot;
    for (int v = 0; v < w; ++v) run += wtot[v];
    rs[tid] = run;
#pragma unroll
    for (int v = 0; v < kIbxDdWaves; v += 2) {
      const uint32_t lo = run, hi = run + cv[v];
      cnt[(v >> 1) * 256 + tid + 1] = lo | (hi << 16);
      run = hi + cv[v + 1];
    }
    if (tid == g.Td - 1) rs[g.Td] = run;
  }
  __syncthreads();
  each([&](uint32_t u, uint32_t f) {
    const uint32_t i = ibx_div(f, g.mqp);
    const uint32_t qr = i * (uint32_t)g.Tq + (f - i * (uint32_t)g.Tqp);
    const uint32_t old = atomicAdd(&cw[u], 1u << csh);
    list[(old >> csh) & 0xFFFFu] = (uint16_t)qr;
  });
  __syncthreads();
  // Row sums: lanes gq * kHC .. + kHC - 1 own row r, chunk c of the half row.
  // Per batch of kHC entries lane c reads entry k + c (past the row's end:
  // query row Bq * Tq, whose delta dl[Bq] is 0 and whose load falls outside Q
  // and returns 0) and the group takes each entry's row offset and delta from
  // its lane by ds_swizzle.
  const int gq = lane / kHC, c = lane - gq * kHC;
  const uint32_t cof = (uint32_t)(h * kHC + c) * 16u;
  const uint32_t sent = (uint32_t)(g.Bq * g.Tq);
  const rsrc_t rQ = make_rsrc_u(Q, (uint32_t)q_bytes);
  char* dj = dD + j * (int64_t)g.Td * rb + cof;
  for (int r0 = 0; r0 < g.Td; r0 += kIbxDdWaves * kRG) {
    const int r = r0 + w * kRG + gq;
    const bool rv = r < g.Td;
    const uint32_t a = rv ? rs[r] : 0u;
    const uint32_t n = rv ? rs[r + 1] - a : 0u;
    const uint32_t nmax = wave_max_u32(n);
    float acc[E::kV];
#pragma unroll
    for (int e = 0; e < E::kV; ++e) acc[e] = 0.0f;
    for (uint32_t k = 0; k < nmax; k += kHC) {
      const uint32_t idx = k + (uint32_t)c;
      const uint32_t qr = idx < n ? (uint32_t)list[a + idx] : sent;
      const int dlane = __float_as_int(dl[ibx_div(qr, g.mq)]);
      const int olane = (int)(qr * (uint32_t)rb);
      static_for<0, kHC / kB>([&](auto bc) {
        uint4 raw[kB];
        float d[kB];
        static_for<0, kB>([&](auto ec) {
          constexpr int e = decltype(ec)::value;
          constexpr int pat = kSw | ((decltype(bc)::value * kB + e) << 5);
          d[e] = __int_as_float(__builtin_amdgcn_ds_swizzle(dlane, pat));
          const uint32_t off = (uint32_t)__builtin_amdgcn_ds_swizzle(olane, pat) + cof;
          const u32x4 v = buf_load16(rQ, (int)off);
          raw[e] = make_uint4(v[0], v[1], v[2], v[3]);
        });
#pragma unroll
        for (int e = 0; e < kB; ++e) E::fma_chunk(raw[e], d[e], acc);
      });
    }
    if (rv) *reinterpret_cast<uint4*>(dj + (int64_t)r * rb) = E::pack(acc);
  }
}

// dQ partial of document quarter qd = XCD index >> 1, feature half h: work item
// (query i, token block tb) per wave; lane (gq, c) owns tokens tb * kTpi + 4 gq
// .. + 3, chunk c of the half row.  Each step stages kS documents' half rows:
// document e of the step as Td + 1 rows from LDS chunk e * (Td + 1) * kHC, row
// u holding its row u (1-based) and row 0 zeros, which a token with no source
// (entry 0) reads.
template <class E, int kHC, int kS>
__global__ void __launch_bounds__(kIbThreads) bwd_ib_dq_kernel(const uint32_t* ct, const float* dT,
                                                              const char* D, IbxGeo g, int ntb,
                                                              int64_t nitems, int64_t rb,
                                                              float* part, int64_t nq_rows,
                                                              int dim) {
  constexpr int kG = 64 / kHC;
  constexpr int kTpi = 4 * kG;
  constexpr int kPer = kIbxStage / kIbThreads;  // copies per thread per step
  constexpr int kOps = kPer + 2 * kS;           // loads a wave issues per step
  __shared__ uint4 dbuf0[kIbxStage], dbuf1[kIbxStage], dbuf2[kIbxStage];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int xcd = blockIdx.x & 7, h = xcd & 1, qd = xcd >> 1;
  const int64_t item = (int64_t)(blockIdx.x >> 3) * kIbItems + w;
  const bool live = item < nitems;  // (a dead wave still copies and meets the barriers)
  const int64_t i = live ? item / ntb : 0;
  const int tb = live ? (int)(item - i * ntb) : 0;
  const int gq = lane / kHC, c = lane - gq * kHC;
  const int t0 = tb * kTpi + 4 * gq;
  const bool tl = live && t0 < g.Tqp;
  const int64_t ps = (g.Bd + kIbxQuarters - 1) / kIbxQuarters;
  const int64_t ja = std::min<int64_t>(g.Bd, qd * ps);
  const int64_t len = std::min<int64_t>(g.Bd, ja + ps) - ja;
  const int64_t nsteps = (len + kS - 1) / kS;
  // Workgroups of one quarter start at different documents, so the quarter
  // is requested from HBM by many workgroups at once rather than in lockstep.
  const int64_t rot = len > 0 ? ((int64_t)(blockIdx.x >> 3) * 2 * kS) % len : 0;
  const int docch = (g.Td + 1) * kHC;
  int ce[kPer];
  uint32_t coff[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int x = (k * kIbItems + w) * 64 + lane;
    const int e = x / docch, rem = x - e * docch, u = rem / kHC;
    ce[k] = (e < kS && u >= 1) ? e : -1;  // (-1: the copy reads out of range and writes 0)
    coff[k] = (uint32_t)((u - 1) * rb + (h * kHC + rem % kHC) * 16);
  }
  const rsrc_t rD = make_rsrc_u(D, (uint32_t)(g.Bd * g.Td * rb));
  const rsrc_t rC = make_rsrc_u(ct, (uint32_t)(g.Bd * g.ct_stride));
  const rsrc_t rT = make_rsrc_u(dT, (uint32_t)(g.Bd * g.Bq * 4));
  float acc[4][E::kV];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int e = 0; e < E::kV; ++e) acc[q][e] = 0.0f;
  // step position s -> document (s >= len: the last one; its delta is not used)
  auto docj = [&](int64_t s) {
    int64_t x = rot + std::min<int64_t>(s, len - 1);
    if (x >= len) x -= len;
    return ja + x;
  };
  // Per-lane parts of the tape and delta offsets (a lane past its query's
  // tokens: out of range, the load returns 0); the document parts are uniform.
  const uint32_t ctl = tl ? (uint32_t)(i * g.Tqp + t0) : 0x80000000u;
  const uint32_t dtl = (uint32_t)(i * 4);
  auto fetch = [&](int64_t k, uint4* buf, uint32_t(&cv)[kS], float(&dv)[kS]) {
    uint32_t dbe[kS], cte[kS], dte[kS];
#pragma unroll
    for (int e = 0; e < kS; ++e) {
      const int64_t jj = docj(k * kS + e);
      dbe[e] = (uint32_t)(jj * g.Td * rb);
      cte[e] = (uint32_t)(jj * g.ct_stride);
      dte[e] = (uint32_t)(jj * g.Bq * 4);
    }
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      uint32_t b = dbe[0];
#pragma unroll
      for (int e = 1; e < kS; ++e)
        if (ce[q] == e) b = dbe[e];
      const uint32_t voff = ce[q] >= 0 ? b + coff[q] : 0x80000000u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rD, (lds_ptr_t)(buf + (q * kIbItems + w) * 64), 16,
                                               (int)voff, 0, 0, 0);
    }
#pragma unroll
    for (int e = 0; e < kS; ++e) {
      cv[e] = buf_load4(rC, (int)(cte[e] + ctl));
      dv[e] = __uint_as_float(buf_load4(rT, (int)(dte[e] + dtl)));
    }
  };
  // Entries are 0 or 1..Td (the compaction's output), entry 0 reading the zero
  // row; a non-finite delta (0 * it is not 0) leaves entry 0 out instead.  (The
  // branch on a zero delta also keeps each document's reads and multiply-adds
  // in a block of their own: without it the scheduler interleaves the steps
  // past the register budget.)
  auto gather = [&](const uint4* rd, const uint32_t(&cv)[kS], const float(&dv)[kS], int64_t k) {
    const uint32_t lb = lds_addr(rd) + (uint32_t)c * 16u;
#pragma unroll
    for (int e = 0; e < kS; ++e) {
      const float de = (live && k * kS + e < len) ? uniform_f(dv[e]) : 0.0f;
      if (de == 0.0f) continue;
      const bool fin = __builtin_isfinite(de);
      uint32_t addr[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        addr[q] = lb + (uint32_t)(e * docch) * 16u + ((cv[e] >> (8 * q)) & 255u) * (kHC * 16u);
      uint4 raw[4];
      lds_read4(raw, addr);
      // One path for every delta (an if / else here copies all 32 accumulators
      // at the join): the zero row times 0 for a non-finite delta, then that
      // delta on the tokens with a source.
      const float dm = fin ? de : 0.0f;
#pragma unroll
      for (int q = 0; q < 4; ++q) E::fma_chunk(raw[q], dm, acc[q]);
      if (!fin) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (((cv[e] >> (8 * q)) & 255u) != 0u) E::fma_chunk(raw[q], de, acc[q]);
      }
    }
  };
  uint32_t c0v[kS], c1v[kS], c2v[kS];
  float d0v[kS], d1v[kS], d2v[kS];
  if (len > 0) {
    fetch(0, dbuf0, c0v, d0v);
    fetch(std::min<int64_t>(1, nsteps - 1), dbuf1, c1v, d1v);
  }
  dma_wait_barrier<kOps>();  // step 0 ready
  // step k: gather from `rd`; fetch step k + 2 into `wr` (read at step k - 1).
  // Straight-line body (the last round pads with empty steps), so the
  // compiler's own load counting stays exact across the back edge.
  auto step = [&](int64_t k, const uint4* rd, uint4* wr, const uint32_t(&cc)[kS],
                  const float(&dc)[kS], uint32_t(&cn)[kS], float(&dn)[kS]) {
    fetch(std::min(k + 2, nsteps - 1), wr, cn, dn);
    gather(rd, cc, dc, k);
    dma_wait_barrier<kOps>();  // k + 1 ready; k + 2 may stay in flight
  };
  for (int64_t k = 0; k < nsteps; k += 3) {
    step(k, dbuf0, dbuf2, c0v, d0v, c2v, d2v);
    step(k + 1, dbuf1, dbuf0, c1v, d1v, c0v, d0v);
    step(k + 2, dbuf2, dbuf1, c2v, d2v, c1v, d1v);
  }
  dma_wait_barrier<0>();  // no copy may land after the workgroup's LDS is released
  if (!live) return;
  float* pq = part + (int64_t)qd * nq_rows * dim + (int64_t)(h * kHC + c) * E::kV;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int t = t0 + q;
    if (t >= g.Tq) continue;
    float* dst = pq + (i * g.Tq + t) * dim;
#pragma unroll
    for (int e = 0; e < E::kV; e += 4)
      *reinterpret_cast<float4*>(dst + e) = make_float4(acc[q][e], acc[q][e + 1], acc[q][e + 2], acc[q][e + 3]);
  }
}

// ---- generic path (any row size) -----------------------------------------------------------

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

// ---- per-layout document views (host) ------------------------------------------------------

// Candidates need the document order: make_docs runs the grouping into `gws`
// (docs_workspace bytes) and reports its status in *e.
DocsInBatch make_docs(const LayInBatch& l, const PullbackArgs& a, void*, hipStream_t, hipError_t*) {
  DocsInBatch d;
  d.ndocs = l.Bd;
  d.Bd = (uint32_t)l.Bd;
  d.Bq = (uint32_t)(a.npairs / l.Bd);
  d.rows = a.rows;
  d.Tq = l.Tq;
  d.qm = l.qm;
  return d;
}
DocsPaired make_docs(const LayPaired& l, const PullbackArgs& a, void*, hipStream_t, hipError_t*) {
  DocsPaired d;
  d.ndocs = a.npairs;
  d.rows = a.rows;
  d.Tq = l.Tq;
  d.qm = l.qm;
  return d;
}
DocsCand make_docs(const LayCand& l, const PullbackArgs& a, void* gws, hipStream_t st, hipError_t* e) {
  DocsCand d;
  d.ndocs = l.N;
  d.C = (uint32_t)l.C;
  d.rows = a.rows;
  d.Tq = l.Tq;
  d.qm = l.qm;
  *e = group_pairs_by_document(l.idx, l.idx64, a.npairs, l.N, gws, &d.order, &d.end, st);
  return d;
}
DocsPacked make_docs(const LayPacked& l, const PullbackArgs& a, void*, hipStream_t, hipError_t*) {
  DocsPacked d;
  d.ndocs = a.npairs;
  d.rows = a.rows;
  d.qm = l.qm;
  return d;
}
DocsVarlen make_docs(const LayVarlen& l, const PullbackArgs& a, void*, hipStream_t, hipError_t*) {
  DocsVarlen d;
  d.ndocs = a.npairs;
  d.rows = a.rows;
  d.cu_q = l.cu_q;
  d.nq = l.nq;
  return d;
}
template <class L> size_t docs_workspace(const L&, int64_t) { return 0; }
template <> size_t docs_workspace<LayCand>(const LayCand& l, int64_t npairs) {
  return al256(group_workspace_bytes(npairs, l.N));
}

// Document rows the staged in-batch dQ kernel copies per document (-1: the
// layout has no staged kernel).
template <class L> int64_t staged_rows(const L&) { return -1; }
template <> int64_t staged_rows<LayInBatch>(const LayInBatch& l) { return l.Td; }

template <class E, class L>
void launch_dq_staged(const L&, const PullbackArgs&, const RowGeo&, const float*, int, int, int64_t,
                      int64_t, float*, hipStream_t) {}
template <class E>
void launch_dq_staged(const LayInBatch& lay, const PullbackArgs& a, const RowGeo& geo,
                      const float* delta, int ntb, int nsplit, int64_t nitems, int64_t rb, float* part,
                      hipStream_t st) {
  const int64_t nblk = bcdiv(nitems, kIbItems) * nsplit;
  if constexpr (E::kSz != 2) return;  // (16-bit features only, see launch_vec)
  if (geo.cpl == 1)
    hipLaunchKernelGGL((bwd_dq_ib_kernel<E, 1>), dim3((unsigned)nblk), dim3(kIbThreads), 0, st, lay,
                       delta, a.args, a.rows, ntb, nsplit, nitems, geo, rb, a.dim, a.dQ, part, a.nq_rows);
  else
    hipLaunchKernelGGL((bwd_dq_ib_kernel<E, 2>), dim3((unsigned)nblk), dim3(kIbThreads), 0, st, lay,
                       delta, a.args, a.rows, ntb, nsplit, nitems, geo, rb, a.dim, a.dQ, part, a.nq_rows);
}

// The feature-half in-batch path (16-bit features, half rows of 4, 8 or 16
// chunks, Td <= 255 so a tape entry fits a byte, the document's sources
// within the dD kernel's LDS, D within 31-bit buffer offsets): returns false
// when the call does not fit it, else runs the whole pullback and sets *err.
template <class E, class L>
bool launch_ib_split(const L&, const PullbackArgs&, hipStream_t, hipError_t*) {
  return false;
}
uint32_t ibx_magic(int d) {
  return d <= 1 ? 0u : (uint32_t)(((uint64_t)1 << 32) / (uint64_t)d + (((uint64_t)1 << 32) % d != 0));
}
template <class E>
bool launch_ib_split(const LayInBatch& lay, const PullbackArgs& a, hipStream_t st,
                     hipError_t* err) {
  if constexpr (E::kSz != 2) {
    return false;
  } else {
    const int64_t rb = (int64_t)a.dim * 2;
    const int hc = (int)(rb / 32);
    if (rb % 32 != 0 || (hc != 4 && hc != 8 && hc != 16)) return false;
    const int64_t Bd = lay.Bd;
    if (Bd < 1 || a.npairs % Bd != 0) return false;
    const int64_t Bq = a.npairs / Bd;
    const int Tq = lay.Tq, Td = lay.Td, Tqp = (Tq + 3) & ~3;
    if (Td < 1 || Td > 255 || Tq < 1 || a.rows != Tq || Bq > kIbxMaxBq || Bq * Tqp > kIbxMaxSrc)
      return false;
    if (lay.Q != a.Qbase || lay.D != a.Dbase || lay.qbytes != Tq * rb || lay.dbytes != Td * rb ||
        a.nq_rows != Bq * Tq || a.nd_rows != Bd * Td)
      return false;
    const int64_t ct_stride = (Bq * Tqp + 15) & ~(int64_t)15;
    if (Bd * Td * rb >= ((int64_t)1 << 31) || Bd * ct_stride >= ((int64_t)1 << 31)) return false;
    const size_t dd_lds = (size_t)(kIbxDdWaves / 2 * 256 + 256) * 4 + (size_t)(Bq + 1) * 4 + (size_t)Bq * Tqp * 2;
    if (dd_lds > (size_t)kIbxDdLdsMax) return false;
    const int spare = kIbxStage / ((Td + 1) * hc);  // documents per dQ step
    if (spare < 1) return false;
    // (bf16 widening takes more registers: 4 documents a step would spill)
    const int ks = (spare >= 4 && E::kSz == 2 && std::is_same<E, EF16>::value) ? 4 : (spare >= 2 ? 2 : 1);

    IbxGeo g;
    g.Bd = Bd;
    g.Bq = (int)Bq;
    g.Tq = Tq;
    g.Tqp = Tqp;
    g.Td = Td;
    g.ct_stride = ct_stride;
    g.mq = ibx_magic(Tq);
    g.mqp = ibx_magic(Tqp);
    const size_t b_ct = al256((size_t)(Bd * ct_stride));
    const size_t b_dt = al256((size_t)(Bd * Bq) * 4);
    const size_t b_part = al256((size_t)(kIbxQuarters * a.nq_rows * a.dim) * 4);
    void* ws = nullptr;
    hipError_t e = workspace_alloc(&ws, b_ct + b_dt + b_part, st);
    if (e != hipSuccess) {
      *err = e;
      return true;
    }
    char* w = static_cast<char*>(ws);
    uint32_t* ct = reinterpret_cast<uint32_t*>(w);
    float* dT = reinterpret_cast<float*>(w + b_ct);
    float* part = reinterpret_cast<float*>(w + b_ct + b_dt);
    const int vec4 = (Tq % 4 == 0) && (reinterpret_cast<uintptr_t>(a.args) & 15u) == 0;
    const unsigned nsub = (unsigned)bcdiv(ct_stride / 4, kIbxCompactSpan);
    const unsigned cgrid = (unsigned)(bcdiv(Bd, 8 * kIbxCompactGroup) * 8 * kIbxCompactGroup);
    hipLaunchKernelGGL(bwd_ib_compact_kernel<E>, dim3(cgrid, nsub), dim3(kBwdThreads), 0, st, a.args,
                       static_cast<const char*>(a.Delta), static_cast<const char*>(a.inv_n), lay.qm,
                       g, vec4, ct, dT);
    const unsigned dd_grid = (unsigned)(8 * bcdiv(Bd, 4));
    const int64_t q_bytes = a.nq_rows * rb;
    const int tpi = 256 / hc;
    const int ntb = (int)bcdiv(Tq, tpi);
    const int64_t nitems = Bq * ntb;
    const unsigned dq_grid = (unsigned)(8 * bcdiv(nitems, kIbItems));
    auto dq = [&](auto hck) {
      constexpr int kHC = decltype(hck)::value;
      hipLaunchKernelGGL((bwd_ib_dd_kernel<E, kHC>), dim3(dd_grid), dim3(kIbxDdThreads), dd_lds, st, ct,
                         dT, g, rb, a.Qbase, q_bytes, a.dD);
      if (ks == 4)
        hipLaunchKernelGGL((bwd_ib_dq_kernel<E, kHC, 4>), dim3(dq_grid), dim3(kIbThreads), 0, st, ct, dT,
                           a.Dbase, g, ntb, nitems, rb, part, a.nq_rows, a.dim);
      else if (ks == 2)
        hipLaunchKernelGGL((bwd_ib_dq_kernel<E, kHC, 2>), dim3(dq_grid), dim3(kIbThreads), 0, st, ct, dT,
                           a.Dbase, g, ntb, nitems, rb, part, a.nq_rows, a.dim);
      else
        hipLaunchKernelGGL((bwd_ib_dq_kernel<E, kHC, 1>), dim3(dq_grid), dim3(kIbThreads), 0, st, ct, dT,
                           a.Dbase, g, ntb, nitems, rb, part, a.nq_rows, a.dim);
    };
    if (hc == 4) dq(std::integral_constant<int, 4>());
    else if (hc == 8) dq(std::integral_constant<int, 8>());
    else dq(std::integral_constant<int, 16>());
    const int64_t nchunks = a.nq_rows * rb / 16;
    const unsigned blocks =
        (unsigned)std::min<int64_t>(65536, std::max<int64_t>(1, bcdiv(nchunks, kBwdThreads)));
    hipLaunchKernelGGL(bwd_dq_reduce_kernel<E>, dim3(blocks), dim3(kBwdThreads), 0, st, part,
                       kIbxQuarters, nchunks, a.nq_rows * a.dim, a.dQ);
    e = hipGetLastError();
    const hipError_t ef = workspace_free(ws, st);
    *err = e != hipSuccess ? e : ef;
    return true;
  }
}

// Vector-path geometry for rows of rb bytes, or false.
bool vec_geometry(int64_t rb, int esz, RowGeo* g) {
  if (rb % 16 != 0) return false;
  const int64_t nch = rb / 16;
  if (nch < 4 || nch > 128) return false;
  int64_t pc = 1;
  while (pc < nch) pc <<= 1;
  const int lr = (int)std::min<int64_t>(64, pc);
  g->lg_lr = 0;
  while ((1 << g->lg_lr) < lr) ++g->lg_lr;
  g->cpl = (int)(pc / lr);
  g->nch = (int)nch;
  const int slots = 64 / (16 / esz);
  g->tpl = std::min(slots / g->cpl, lr);
  g->tpw = g->tpl * (64 / lr);
  return true;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <class L, class E>
hipError_t launch_vec(const L& lay, const PullbackArgs& a, const RowGeo& geo, const float* delta,
                      hipStream_t st) {
  const int64_t rb = (int64_t)a.dim * E::kSz;
  const int64_t ngroups = a.npairs / a.G;
  const int ntb = (int)bcdiv(a.rows, geo.tpw);
  const int64_t nitems = ngroups * ntb;
  // dQ pair splits: aim at ~4096 workgroups (the staged in-batch kernel: one
  // 16-wave workgroup per CU), >= 16 pairs per split, a multiple of 8 splits
  // (one share per XCD), partials within 512 MB.
  // (16-bit features only: fp32 accumulators plus fp32 rows exceed the 128 registers
  // a 16-wave workgroup leaves each lane)
  const bool staged = E::kSz == 2 && staged_rows(lay) >= 0 &&
                      staged_rows(lay) * geo.nch <= kIbStageChunks;
  int64_t nsplit = 1;
  const bool wave_split = a.G >= 4;
  if (staged) {
    const int64_t nwg = bcdiv(nitems, kIbItems);
    nsplit = std::min<int64_t>(a.G, std::max<int64_t>(1, bcdiv(256, nwg)));
    if (nsplit >= 8) nsplit = std::min<int64_t>(a.G, (nsplit + 7) & ~(int64_t)7);
  } else if (a.G >= 16 && nitems < 4096) {
    nsplit = std::min<int64_t>(4096 / nitems, a.G / 16);
    if (nsplit >= 8) nsplit &= ~(int64_t)7;
  }
  while (nsplit > 1 && nsplit * a.nq_rows * a.dim * 4 > ((int64_t)512 << 20)) nsplit /= 2;
  if (nsplit < 1) nsplit = 1;
  // dD: document lists
  const int64_t nsrc = a.npairs * a.rows;
  const size_t b_part = nsplit > 1 ? al256((size_t)(nsplit * a.nq_rows * a.dim) * 4) : 0;
  const size_t b_rows = al256((size_t)std::max<int64_t>(a.nd_rows, 1) * 4);
  const size_t b_list = al256((size_t)std::max<int64_t>(nsrc, 1) * 8);
  const size_t b_docs = docs_workspace(lay, a.npairs);
  void* ws = nullptr;
  hipError_t e = workspace_alloc(&ws, b_part + 2 * b_rows + b_list + b_docs, st);
  if (e != hipSuccess) return e;
  char* w = static_cast<char*>(ws);
  float* part = reinterpret_cast<float*>(w);
  uint32_t* rstart = reinterpret_cast<uint32_t*>(w + b_part);
  uint32_t* rcount = reinterpret_cast<uint32_t*>(w + b_part + b_rows);
  uint2* list = reinterpret_cast<uint2*>(w + b_part + 2 * b_rows);
  void* gws = w + b_part + 2 * b_rows + b_list;

  if (staged) {
    launch_dq_staged<E>(lay, a, geo, delta, ntb, (int)nsplit, nitems, rb, part, st);
  } else if (wave_split) {
    const int64_t nblk = nitems * nsplit;
    hipLaunchKernelGGL((bwd_dq_vec_kernel<L, E, true>), dim3((unsigned)nblk), dim3(kBwdThreads), 0, st,
                       lay, delta, a.args, a.G, a.rows, ntb, (int)nsplit, nitems, geo, rb, a.dim,
                       a.Qbase, a.dQ, part, a.nq_rows);
  } else {
    hipLaunchKernelGGL((bwd_dq_vec_kernel<L, E, false>), dim3((unsigned)bcdiv(nitems, 4)),
                       dim3(kBwdThreads), 0, st, lay, delta, a.args, a.G, a.rows, ntb, 1, nitems,
                       geo, rb, a.dim, a.Qbase, a.dQ, part, a.nq_rows);
  }
  if (nsplit > 1) {
    const int64_t nchunks = a.nq_rows * rb / 16;
    const unsigned blocks =
        (unsigned)std::min<int64_t>(65536, std::max<int64_t>(1, bcdiv(nchunks, kBwdThreads)));
    hipLaunchKernelGGL(bwd_dq_reduce_kernel<E>, dim3(blocks), dim3(kBwdThreads), 0, st, part,
                       (int)nsplit, nchunks, a.nq_rows * a.dim, a.dQ);
  }
  if (a.nd_rows > 0) {
    hipError_t eg = hipSuccess;
    const auto docs = make_docs(lay, a, gws, st, &eg);
    if (eg == hipSuccess) {
      hipLaunchKernelGGL(bwd_zero_kernel, dim3(grid_for(bcdiv(a.nd_rows, 64))), dim3(kBwdThreads), 0,
                         st, rcount, a.nd_rows);
      const unsigned dblocks = (unsigned)std::min<int64_t>(std::max<int64_t>(docs.ndocs, 1), 65536);
      hipLaunchKernelGGL((bwd_doc_csr_kernel<L, decltype(docs)>), dim3(dblocks), dim3(kDocThreads), 0,
                         st, lay, docs, delta, a.args, a.rows, a.Dbase, rb, rstart, rcount, list);
      const int64_t per_block = 4 * (int64_t)(64 >> geo.lg_lr);
      const unsigned rblocks = (unsigned)std::min<int64_t>(1048576, bcdiv(a.nd_rows, per_block));
      if (geo.cpl == 1)
        hipLaunchKernelGGL((bwd_dd_vec_kernel<E, 1>), dim3(rblocks), dim3(kBwdThreads), 0, st, rstart,
                           rcount, list, (uint32_t)nsrc, a.nd_rows, geo, rb, a.Qbase, a.nq_rows, a.dD);
      else
        hipLaunchKernelGGL((bwd_dd_vec_kernel<E, 2>), dim3(rblocks), dim3(kBwdThreads), 0, st, rstart,
                           rcount, list, (uint32_t)nsrc, a.nd_rows, geo, rb, a.Qbase, a.nq_rows, a.dD);
    }
    e = eg;
  }
  if (e == hipSuccess) e = hipGetLastError();
  const hipError_t ef = workspace_free(ws, st);
  return e != hipSuccess ? e : ef;
}

template <class L>
hipError_t launch_generic(const L& lay, const PullbackArgs& a, const float* delta, hipStream_t st) {
  const int esz = a.dtype == 0 ? 4 : 2;
  const int64_t rb = (int64_t)a.dim * esz;
  // workspace: end offsets (nd_rows + 1), sources (npairs * rows), scan sums
  const int64_t nsrc = a.npairs * a.rows;
  const size_t b_end = al256((size_t)(a.nd_rows + 1) * 4);
  const size_t b_col = al256((size_t)(nsrc > 0 ? nsrc : 1) * 4), b_sums = scan_workspace_bytes(a.nd_rows);
  void* ws = nullptr;
  hipError_t e = workspace_alloc(&ws, b_end + b_col + b_sums, st);
  if (e != hipSuccess) return e;
  char* w = static_cast<char*>(ws);
  uint32_t* cnt = reinterpret_cast<uint32_t*>(w);
  uint32_t* col = reinterpret_cast<uint32_t*>(w + b_end);
  uint32_t* sums = reinterpret_cast<uint32_t*>(w + b_end + b_col);
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
  if (!a.zero_dq && aligned16(a.dQ) && aligned16(a.dD) && aligned16(a.Qbase) && aligned16(a.Dbase)) {
    hipError_t eib = hipSuccess;
    const bool took = a.dtype == 1   ? launch_ib_split<EF16>(lay, a, st, &eib)
                      : a.dtype == 2 ? launch_ib_split<EBF16>(lay, a, st, &eib)
                                     : false;
    if (took) return eib;
  }
  void* ws = nullptr;
  hipError_t e = workspace_alloc(&ws, al256((size_t)a.npairs * 4), st);
  if (e != hipSuccess) return e;
  float* delta = static_cast<float*>(ws);
  const unsigned flat =
      (unsigned)std::min<int64_t>(65536, std::max<int64_t>(1, bcdiv(a.npairs, kBwdThreads)));
  const char* Dl = static_cast<const char*>(a.Delta);
  const char* Il = static_cast<const char*>(a.inv_n);
  if (a.dtype == 0)
    hipLaunchKernelGGL(bwd_delta_kernel<EF32>, dim3(flat), dim3(kBwdThreads), 0, st, Dl, Il, a.npairs, a.G, delta);
  else if (a.dtype == 1)
    hipLaunchKernelGGL(bwd_delta_kernel<EF16>, dim3(flat), dim3(kBwdThreads), 0, st, Dl, Il, a.npairs, a.G, delta);
  else
    hipLaunchKernelGGL(bwd_delta_kernel<EBF16>, dim3(flat), dim3(kBwdThreads), 0, st, Dl, Il, a.npairs, a.G, delta);
  if (a.zero_dq) clear(a.dQ, a.nq_rows);
  RowGeo geo;
  const bool vec = vec_geometry(rb, esz, &geo) && aligned16(a.dQ) && aligned16(a.dD) &&
                   aligned16(a.Qbase) && aligned16(a.Dbase);
  if (vec) {
    if (a.dtype == 0) e = launch_vec<L, EF32>(lay, a, geo, delta, st);
    else if (a.dtype == 1) e = launch_vec<L, EF16>(lay, a, geo, delta, st);
    else e = launch_vec<L, EBF16>(lay, a, geo, delta, st);
  } else {
    e = launch_generic(lay, a, delta, st);
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
