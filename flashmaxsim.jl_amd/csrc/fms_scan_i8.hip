// Explicit instantiation of the INT8 scan launchers (pair/paired and the
// candidate layout; the reference has no INT8 in-batch / packed methods).
#include "fms_scan.hpp"

namespace fms {
template hipError_t launch_scan<OpI8, LayPaired>(const LayPaired&, int, int, int64_t, int32_t*,
                                                 float*, float*, float, bool, bool, hipStream_t);
template hipError_t launch_scan<OpI8, LayCand>(const LayCand&, int, int, int64_t, int32_t*,
                                               float*, float*, float, bool, bool, hipStream_t);
template hipError_t launch_scan<OpI8, LayCandSorted>(const LayCandSorted&, int, int, int64_t,
                                                     int32_t*, float*, float*, float, bool, bool,
                                                     hipStream_t);
}  // namespace fms
