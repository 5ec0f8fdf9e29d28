// Explicit instantiation of the INT8 scan launchers (pair/paired and the
// candidate layout; the reference has no INT8 in-batch / packed methods).
#include "fms_scan.hpp"

namespace fms {
#define FMS_INST(L)                                                                    \
  template hipError_t launch_scan<OpI8, L>(const L&, int, int, int64_t, int32_t*, float*, \
                                           float*, float, bool, bool, hipStream_t);
FMS_INST(LayPaired)
FMS_INST(LayCand)
FMS_INST(LayCandSorted)
#undef FMS_INST
// fp16 document scales (an Int8Index quantised from Float16 features)
#define FMS_INST(L)                                                                     \
  template hipError_t launch_scan<OpI8H, L>(const L&, int, int, int64_t, int32_t*, float*, \
                                            float*, float, bool, bool, hipStream_t);
FMS_INST(LayPaired)
FMS_INST(LayCand)
FMS_INST(LayCandSorted)
#undef FMS_INST
}  // namespace fms
