// fms_runs.hip -- instantiations and launcher of the document-batch candidate
// scan (fms_runs.hpp) for 16-bit and INT8 features.
#include "fms_runs.hpp"

#include <type_traits>

namespace fms {

namespace {

// Query tiles per batch: KQ tiles of NKB fragments stay in registers beside
// two chunk buffers of NKB fragments, within the 256 registers of two waves
// per SIMD.
template <class Op, int NKB>
constexpr int runs_kq() {
  return NKB * (Op::kKb == 32 ? 2 : 1) >= 16 ? 2 : 4;
}

// 16-bit features of d = 64 or 128 stream their chunks through LDS
// (scan_runs_lds: two 8 KB slots per wave at d = 128, 64 KB per workgroup).
template <class Op, int NKB>
constexpr bool runs_lds() {
  return !Op::kInt && (NKB == 4 || NKB == 8);
}

template <class Op, int NKB>
hipError_t launch_nkb(const RunArgs& A, hipStream_t stream) {
  constexpr int KQ = runs_kq<Op, NKB>();
  RunArgs a = A;
  a.ppw = run_ppw(A.npairs, KQ);
  const int64_t waves = (A.npairs + a.ppw - 1) / a.ppw;
  const dim3 grid((unsigned)((waves + kWaves - 1) / kWaves)), block(64 * kWaves);
  if constexpr (runs_lds<Op, NKB>()) {
    if (a.qfrag) {
      // the queries' tiles in fragment order first (same stream)
      const int64_t B = a.npairs / a.lay.C;
      const int64_t nunits = B * a.nqt * NKB * 64;
      if (nunits > 0)
        hipLaunchKernelGGL((query_frag_kernel<NKB>), dim3((unsigned)((nunits + 255) / 256)), dim3(256),
                           0, stream, a.lay.Q, a.lay.Tq, a.dim * Op::kEsz, a.nqt, nunits,
                           reinterpret_cast<u32x4*>(a.qfrag));
      hipLaunchKernelGGL((scan_runs_lds<Op, NKB, KQ, true>), grid, block, 0, stream, a);
    } else {
      hipLaunchKernelGGL((scan_runs_lds<Op, NKB, KQ, false>), grid, block, 0, stream, a);
    }
  } else {
    hipLaunchKernelGGL((scan_runs<Op, NKB, KQ>), grid, block, 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace

template <class Op>
hipError_t launch_runs(const RunArgs& A, hipStream_t stream) {
  constexpr int b = (Op::kKb == 16) ? 4 : 2;
  const int nkb = fast_nkb<Op>(A.nkb);
  if (nkb == b) return launch_nkb<Op, b>(A, stream);
  if (nkb == 2 * b) return launch_nkb<Op, 2 * b>(A, stream);
  if (nkb == 4 * b) return launch_nkb<Op, 4 * b>(A, stream);
  return hipErrorInvalidValue;
}

template hipError_t launch_runs<OpF16>(const RunArgs&, hipStream_t);
template hipError_t launch_runs<OpBF16>(const RunArgs&, hipStream_t);
template hipError_t launch_runs<OpI8>(const RunArgs&, hipStream_t);
template hipError_t launch_runs<OpI8H>(const RunArgs&, hipStream_t);

}  // namespace fms
