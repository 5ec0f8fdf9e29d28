// fms_scan_decl.hpp -- declarations of the explicitly instantiated scan
// launchers (definitions in fms_scan.hpp, instantiated per feature type in
// fms_scan_<type>.hip so the four families compile in parallel).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fms_device.hpp"
#include "fms_layouts.hpp"

namespace fms {

template <class Op, class L>
hipError_t launch_scan(const L& lay, int dim, int rows, int64_t npairs, int32_t* args,
                       float* partial, float* scores, float neg, bool norm, bool vec,
                       hipStream_t stream);

}  // namespace fms
