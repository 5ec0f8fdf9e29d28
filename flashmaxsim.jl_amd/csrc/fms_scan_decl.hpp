// fms_scan_decl.hpp -- declarations of the explicitly instantiated scan
// launchers (definitions in fms_scan.hpp, instantiated per feature type in
// fms_scan_<type>.hip so the four families compile in parallel).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fms_device.hpp"
#include "fms_layouts.hpp"

namespace fms {

inline int pairs_per_wave(int64_t npairs) {
  // Aim for ~32k waves (8 resident per SIMD over 1024 SIMDs, several rounds)
  // so that each wave keeps its query tile across a handful of pairs.
  int64_t ppw = npairs / 32768;
  if (ppw < 1) ppw = 1;
  if (ppw > 32) ppw = 32;
  return (int)ppw;
}

// Whether a scan of npairs pairs fits one launch: the grid's work-items
// (64 per wave of pairs_per_wave pairs) must stay below 2^32.
inline bool scan_grid_fits(int64_t npairs) {
  if (npairs < 0) return false;
  const int64_t ppw = pairs_per_wave(npairs);
  const int64_t waves = (npairs + ppw - 1) / ppw;
  const int64_t blocks = (waves + 3) / 4;  // kWaves waves of 64 lanes per block
  return blocks * 256 < ((int64_t)1 << 32);
}

template <class Op, class L>
hipError_t launch_scan(const L& lay, int dim, int rows, int64_t npairs, int32_t* args,
                       float* partial, float* scores, float neg, bool norm, bool vec,
                       hipStream_t stream);

}  // namespace fms
