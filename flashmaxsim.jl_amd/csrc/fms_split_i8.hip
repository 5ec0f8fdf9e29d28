// Explicit instantiation of the I8 split-d scan for every layout it serves.
#include "fms_split.hpp"

namespace fms {
template hipError_t launch_split<OpI8, LayPaired>(const ScanArgs<LayPaired>&, dim3, dim3, hipStream_t);
template hipError_t launch_split<OpI8, LayCand>(const ScanArgs<LayCand>&, dim3, dim3, hipStream_t);
template hipError_t launch_split<OpI8, LayCandSorted>(const ScanArgs<LayCandSorted>&, dim3, dim3, hipStream_t);
template hipError_t launch_split<OpI8H, LayPaired>(const ScanArgs<LayPaired>&, dim3, dim3, hipStream_t);
template hipError_t launch_split<OpI8H, LayCand>(const ScanArgs<LayCand>&, dim3, dim3, hipStream_t);
template hipError_t launch_split<OpI8H, LayCandSorted>(const ScanArgs<LayCandSorted>&, dim3, dim3, hipStream_t);
}  // namespace fms
