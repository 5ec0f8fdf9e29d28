// Explicit instantiation of the F32 split-d scan for every layout it serves.
#include "fms_split.hpp"

namespace fms {
template hipError_t launch_split<OpF32, LayPaired>(const ScanArgs<LayPaired>&, dim3, dim3, hipStream_t);
template hipError_t launch_split<OpF32, LayCand>(const ScanArgs<LayCand>&, dim3, dim3, hipStream_t);
template hipError_t launch_split<OpF32, LayCandSorted>(const ScanArgs<LayCandSorted>&, dim3, dim3, hipStream_t);
template hipError_t launch_split<OpF32, LayInBatch>(const ScanArgs<LayInBatch>&, dim3, dim3, hipStream_t);
template hipError_t launch_split<OpF32, LayPacked>(const ScanArgs<LayPacked>&, dim3, dim3, hipStream_t);
template hipError_t launch_split<OpF32, LayVarlen>(const ScanArgs<LayVarlen>&, dim3, dim3, hipStream_t);
}  // namespace fms
