// Explicit instantiation of the BF16 scan launchers for every float layout.
#include "fms_scan.hpp"

namespace fms {
#define FMS_INST(L)                                                                    \
  template hipError_t launch_scan<OpBF16, L>(const L&, int, int, int64_t, int32_t*, float*, \
                                            float*, float, bool, bool, hipStream_t);
FMS_INST(LayPaired)
FMS_INST(LayCand)
FMS_INST(LayCandSorted)
FMS_INST(LayInBatch)
FMS_INST(LayPacked)
FMS_INST(LayVarlen)
#undef FMS_INST
}  // namespace fms
