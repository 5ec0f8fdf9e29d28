// fms_misc.hip -- the small kernels on either side of the scans:
//   * per-token symmetric INT8 quantiser (quantize_int8_symmetric),
//   * raw int32 dot products through the int8 MFMA path (test-only check),
//   * query-length normalisation epilogues,
//   * an MFMA accumulator-layout probe (test-only).
#include <float.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fms_device.hpp"
#include "fms_misc.hpp"

namespace fms {

// quantize_int8_symmetric (src/quant.jl:21-49), one wave per token, in the
// feature type T (Float32, or Float16 via kHalf):
//   am    = max_k |x[k]|                                  (exact in either type)
//   raw   = T(max(am, T(1f-8)) / T(127))                   (quant.jl:44)
//   scale = max(raw, floatmin(T))                          (quant.jl:45)
//   code  = round(Int8, clamp(T(x / scale), -127, 127))    (quant.jl:46-47)
// Julia evaluates a Float16 `/` as the fp32 quotient rounded to Float16; an
// fp32 quotient rounded once more to 11 bits equals the correctly rounded
// Float16 quotient (24 >= 2*11 + 2 bits), so both steps below are exact
// restatements.  T(1f-8) is 0 in Float16 (below half the least subnormal).
// `/` is IEEE-correctly rounded (built without fast-math and with
// -fhip-fp32-correctly-rounded-divide-sqrt); (_Float16) conversions and
// rintf round half to even, which is Julia's RoundNearest.
template <bool kHalf>
__global__ void __launch_bounds__(256) quantize_int8_kernel(const void* __restrict__ Xv,
                                                            int8_t* __restrict__ codes,
                                                            void* __restrict__ scales_v, int dim,
                                                            int64_t ntok) {
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * (blockDim.x >> 6);
  auto elem = [&](int64_t tok, int k) -> float {
    if constexpr (kHalf)
      return (float)static_cast<const _Float16*>(Xv)[tok * dim + k];
    else
      return static_cast<const float*>(Xv)[tok * dim + k];
  };
  auto to_t = [](float v) -> float {  // round to T
    if constexpr (kHalf)
      return (float)(_Float16)v;
    else
      return v;
  };
  const float eps = to_t(1.0e-8f);
  const float tmin = kHalf ? 6.103515625e-05f : FLT_MIN;  // floatmin(T)
  for (int64_t tok = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); tok < ntok;
       tok += nwaves) {
    float am = 0.0f;
    for (int k = lane; k < dim; k += 64) am = fmaxf(am, fabsf(elem(tok, k)));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) am = fmaxf(am, __shfl_xor(am, o));
    const float raw = to_t(fmaxf(am, eps) / 127.0f);  // quant.jl:44
    const float sc = fmaxf(raw, tmin);                // quant.jl:45
    int8_t* c = codes + tok * dim;
    for (int k = lane; k < dim; k += 64) {
      float v = to_t(elem(tok, k) / sc);              // quant.jl:46
      v = v > 127.0f ? 127.0f : (v < -127.0f ? -127.0f : v);
      c[k] = (int8_t)__builtin_rintf(v);
    }
    if (lane == 0) {
      if constexpr (kHalf)
        static_cast<_Float16*>(scales_v)[tok] = (_Float16)sc;
      else
        static_cast<float*>(scales_v)[tok] = sc;
    }
  }
}

hipError_t quantize_int8(bool half, const void* X, int8_t* codes, void* scales, int dim,
                         int64_t ntok, hipStream_t stream) {
  int64_t blocks = (ntok + 3) / 4;
  if (blocks > 65536) blocks = 65536;
  if (half)
    hipLaunchKernelGGL(quantize_int8_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, X,
                       codes, scales, dim, ntok);
  else
    hipLaunchKernelGGL(quantize_int8_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream,
                       X, codes, scales, dim, ntok);
  return hipGetLastError();
}

// Raw int32 dots via v_mfma_i32_32x32x32_i8, one wave per 32x32 (t, u)
// tile; out is (Td, Tq) column-major: out[u + Td*t].
__global__ void __launch_bounds__(64) int8_dots_kernel(int32_t* __restrict__ out,
                                                       const int8_t* qc, const int8_t* dc,
                                                       int dim, int Tq, int Td, int vec) {
  const int lane = threadIdx.x & 63, r32 = lane & 31, h = lane >> 5;
  const int qt = blockIdx.x, ch = blockIdx.y;
  const rsrc_t rq = make_rsrc(qc, (uint32_t)Tq * (uint32_t)dim);
  const rsrc_t rd = make_rsrc(dc, (uint32_t)Td * (uint32_t)dim);
  const int nkb = (dim + OpI8::kKb - 1) / OpI8::kKb;
  const int t = qt * kTile + r32, row = ch * kTile + r32;
  OpI8::Acc acc = {};
  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * OpI8::kKb + h * OpI8::kEpl;
    OpI8::Frag a, b;
    if (vec) {
      a = (k0 < dim) ? OpI8::load(rd, row * dim + k0) : OpI8::zero();
      b = (k0 < dim) ? OpI8::load(rq, t * dim + k0) : OpI8::zero();
    } else {
      a = OpI8::load_guarded(rd, row * dim + k0, k0, dim);
      b = OpI8::load_guarded(rq, t * dim + k0, k0, dim);
    }
    acc = OpI8::mma(a, b, acc);
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int u = ch * kTile + acc_row(r, h);
    if (t < Tq && u < Td) out[(int64_t)u + (int64_t)Td * t] = acc[r];
  }
}

hipError_t int8_dots(int32_t* out, const int8_t* qc, const int8_t* dc, int dim, int Tq, int Td,
                     bool vec, hipStream_t stream) {
  const dim3 grid((unsigned)((Tq + kTile - 1) / kTile), (unsigned)((Td + kTile - 1) / kTile));
  hipLaunchKernelGGL(int8_dots_kernel, grid, dim3(64), 0, stream, out, qc, dc, dim, Tq, Td,
                     vec ? 1 : 0);
  return hipGetLastError();
}

// length_normalize (src/normalize.jl:4-46): scores(row, col) *= 1/max(n_col, 1)
// with n_col = count(qmask[:, col]); candidate entries whose idx is out of
// range are (re)set to neg instead of being scaled.
__global__ void length_normalize_kernel(float* scores, const uint8_t* qmask, int64_t Tq,
                                        int64_t nrows, int64_t ncols, const void* idx, int idx64,
                                        int64_t N, float neg) {
  const int64_t col = blockIdx.x;
  __shared__ float inv_s;
  if (threadIdx.x == 0) {
    int64_t n = 0;
    if (qmask) {
      for (int64_t t = 0; t < Tq; ++t) n += qmask[col * Tq + t] != 0;
    } else {
      n = Tq;
    }
    const float nf = (float)n;
    inv_s = 1.0f / (nf > 1.0f ? nf : 1.0f);
  }
  __syncthreads();
  const float inv = inv_s;
  for (int64_t r = threadIdx.x; r < nrows; r += blockDim.x) {
    const int64_t o = col * nrows + r;
    if (idx) {
      const int64_t j = idx64 ? static_cast<const int64_t*>(idx)[o]
                              : (int64_t) static_cast<const int32_t*>(idx)[o];
      if (!(j >= 1 && j <= N)) {
        scores[o] = neg;
        continue;
      }
    }
    scores[o] = scores[o] * inv;
  }
}

hipError_t length_normalize(float* scores, const uint8_t* qmask, int64_t Tq, int64_t nrows,
                            int64_t ncols, const void* idx, int idx64, int64_t N, float neg,
                            hipStream_t stream) {
  hipLaunchKernelGGL(length_normalize_kernel, dim3((unsigned)ncols), dim3(256), 0, stream, scores,
                     qmask, Tq, nrows, ncols, idx, idx64, N, neg);
  return hipGetLastError();
}

// varlen_inv_n_kernel! + broadcast multiply (src/kernels_packed.jl:277-282,
// src/packed.jl:339-354).
__global__ void varlen_normalize_kernel(float* scores, const int32_t* cu_q, int64_t N) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  int64_t tq = (int64_t)cu_q[n + 1] - (int64_t)cu_q[n];
  if (tq < 1) tq = 1;
  const float inv = 1.0f / (float)tq;
  scores[n] = scores[n] * inv;
}

hipError_t varlen_normalize(float* scores, const int32_t* cu_q, int64_t N, hipStream_t stream) {
  hipLaunchKernelGGL(varlen_normalize_kernel, dim3((unsigned)((N + 255) / 256)), dim3(256), 0,
                     stream, scores, cu_q, N);
  return hipGetLastError();
}

// Accumulator layout probe: one wave, one 32x32 MFMA per feature type.
// Pass 0 puts A[i][0] = i+1, B[0][j] = 1 (result = row+1); pass 1 puts
// A[i][0] = 1, B[0][j] = j+1 (result = column+1).  "k = 0" is element 0 of
// the lanes in half 0 for both operands.  out[(pass*64 + lane)*16 + r].
template <class Op>
__device__ void probe_one(float* out, int lane) {
  const int r32 = lane & 31, h = lane >> 5;
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const float av = pass == 0 ? (float)(r32 + 1) : 1.0f;
    const float bv = pass == 0 ? 1.0f : (float)(r32 + 1);
    typename Op::Frag a = Op::zero(), b = Op::zero();
    if (h == 0) {
      if constexpr (Op::kInt) {
        a[0] = (uint32_t)(int)av & 0xffu;
        b[0] = (uint32_t)(int)bv & 0xffu;
      } else if constexpr (Op::kEsz == 4) {
        a = __builtin_bit_cast(uint32_t, av);
        b = __builtin_bit_cast(uint32_t, bv);
      } else if constexpr (sizeof(typename Op::Frag) == 16) {
        // f16 / bf16: element 0 is the low half of word 0
        uint16_t ab, bb;
        if constexpr (__is_same(Op, OpF16)) {
          ab = __builtin_bit_cast(uint16_t, (_Float16)av);
          bb = __builtin_bit_cast(uint16_t, (_Float16)bv);
        } else {
          ab = (uint16_t)(__builtin_bit_cast(uint32_t, av) >> 16);  // exact small integers
          bb = (uint16_t)(__builtin_bit_cast(uint32_t, bv) >> 16);
        }
        a[0] = ab;
        b[0] = bb;
      }
    }
    typename Op::Acc acc = {};
    acc = Op::mma(a, b, acc);
#pragma unroll
    for (int r = 0; r < 16; ++r) out[(pass * 64 + lane) * 16 + r] = (float)acc[r];
  }
}

__global__ void mfma_layout_probe_kernel(float* out, int op) {
  const int lane = threadIdx.x & 63;
  switch (op) {
    case 0: probe_one<OpF32>(out, lane); break;
    case 1: probe_one<OpF16>(out, lane); break;
    case 2: probe_one<OpBF16>(out, lane); break;
    default: probe_one<OpI8>(out, lane); break;
  }
}

// Streaming read of `bytes` (a multiple of 16) with 16-byte loads: the
// measured HBM read ceiling reported beside the scans' roofline, and the
// known-size reference that calibrates the FETCH_SIZE counter.  Each thread
// folds what it read into one word so the loads cannot be removed.
__global__ void __launch_bounds__(256) read_bandwidth_kernel(const u32x4* __restrict__ p,
                                                             int64_t n16, uint32_t* out) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  uint32_t acc = 0u;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4 a = __builtin_nontemporal_load(p + i);
    const u32x4 b = __builtin_nontemporal_load(p + i + stride);
    const u32x4 c = __builtin_nontemporal_load(p + i + 2 * stride);
    const u32x4 d = __builtin_nontemporal_load(p + i + 3 * stride);
    acc ^= a[0] ^ a[1] ^ a[2] ^ a[3] ^ b[0] ^ b[1] ^ b[2] ^ b[3];
    acc ^= c[0] ^ c[1] ^ c[2] ^ c[3] ^ d[0] ^ d[1] ^ d[2] ^ d[3];
  }
  for (; i < n16; i += stride) {
    const u32x4 a = __builtin_nontemporal_load(p + i);
    acc ^= a[0] ^ a[1] ^ a[2] ^ a[3];
  }
  out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

hipError_t read_bandwidth(const void* p, int64_t bytes, uint32_t* out, int blocks,
                          hipStream_t stream) {
  hipLaunchKernelGGL(read_bandwidth_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const u32x4*>(p), bytes / 16, out);
  return hipGetLastError();
}

// One workgroup per listed document: its doc16 16-byte units, nontemporal
// (the document is read once), XOR-folded so the loads are kept.
__global__ void __launch_bounds__(256) gather_bandwidth_kernel(const u32x4* __restrict__ g,
                                                               int64_t gallery16, int64_t doc16,
                                                               const int32_t* __restrict__ docs,
                                                               uint32_t* out) {
  const int64_t b = blockIdx.x;
  const int64_t d0 = (int64_t)docs[b] * doc16;
  uint32_t acc = 0u;
  if (docs[b] >= 0 && d0 + doc16 <= gallery16) {
    for (int64_t i = threadIdx.x; i < doc16; i += 256) {
      const u32x4 a = __builtin_nontemporal_load(g + d0 + i);
      acc ^= a[0] ^ a[1] ^ a[2] ^ a[3];
    }
  }
  out[b * 256 + threadIdx.x] = acc;
}

hipError_t gather_bandwidth(const void* g, int64_t gallery_bytes, int64_t doc_bytes,
                            const int32_t* docs, int64_t ndocs, uint32_t* out, hipStream_t stream) {
  hipLaunchKernelGGL(gather_bandwidth_kernel, dim3((unsigned)ndocs), dim3(256), 0, stream,
                     static_cast<const u32x4*>(g), gallery_bytes / 16, doc_bytes / 16, docs, out);
  return hipGetLastError();
}

// Cross-lane helper probe (one wave): out[l] = lane_xor32(l), out[64 + l] =
// half_sum(l) (the sum of lanes 0-31 in every lane), out[128 + l] /
// out[192 + l] = the (token, max) merge_halves keeps when lane l holds
// (max = l % 7, token = l + 1).
__global__ void cross_lane_probe_kernel(float* out) {
  const int lane = threadIdx.x & 63, h = lane >> 5;
  out[lane] = (float)lane_xor32((uint32_t)lane, h);
  out[64 + lane] = half_sum((float)lane);
  float mx = (float)(lane % 7);
  int tok = lane + 1;
  merge_halves(mx, tok, h);
  out[128 + lane] = (float)tok;
  out[192 + lane] = mx;
}

hipError_t cross_lane_probe(float* out, hipStream_t stream) {
  hipLaunchKernelGGL(cross_lane_probe_kernel, dim3(1), dim3(64), 0, stream, out);
  return hipGetLastError();
}

hipError_t mfma_layout_probe(float* out, int op, hipStream_t stream) {
  hipLaunchKernelGGL(mfma_layout_probe_kernel, dim3(1), dim3(64), 0, stream, out, op);
  return hipGetLastError();
}

}  // namespace fms
