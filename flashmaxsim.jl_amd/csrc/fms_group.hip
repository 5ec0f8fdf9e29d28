// fms_group.hip -- counting sort of candidate pairs by document, and the
// workspace pool it draws from.
//
// Two levels, with every atomic in LDS (a device-scope atomic on an MI355X
// is performed past the XCDs' L2s, at memory: one per pair cost ~33 us per
// pass at C*B = 256k):
//   1. buckets of D consecutive documents: each block histograms its tile of
//      pairs by bucket in LDS, the (bucket, block) counts are prefix-summed,
//      and each block scatters its pairs to their bucket's slots;
//   2. one block per bucket counts its pairs per document in LDS, writes the
//      documents' run ends and scatters the pairs into document order.
// The older one-level sort (one global atomic per pair and per pass) remains
// for galleries too large for the bucket tables.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <mutex>

#include "fms_group.hpp"

namespace fms {

namespace {

constexpr int kScanThreads = 1024;                  // one block = 16 waves
constexpr int kScanPer = 4;                         // counters per thread
constexpr int kScanTile = kScanThreads * kScanPer;  // counters per block
constexpr int kFlat = 256;                          // threads of the flat kernels

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

inline unsigned flat_blocks(int64_t n) {
  const int64_t b = cdiv(n, kFlat);
  return (unsigned)(b < 1 ? 1 : (b > 65536 ? 65536 : b));
}

__device__ __forceinline__ int64_t load_index(const void* idx, int idx64, int64_t p) {
  return idx64 ? static_cast<const int64_t*>(idx)[p] : (int64_t) static_cast<const int32_t*>(idx)[p];
}

// Exclusive scan of one value per thread over a kScanThreads block; *total
// receives the block sum.  Every thread of the block must call it.
__device__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* total) {
  __shared__ uint32_t wsum[kScanThreads / 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) wsum[w] = x;
  __syncthreads();
  if (w == 0) {
    uint32_t s = lane < kScanThreads / 64 ? wsum[lane] : 0u;
#pragma unroll
    for (int o = 1; o < kScanThreads / 64; o <<= 1) {
      const uint32_t y = __shfl_up(s, o);
      if (lane >= o) s += y;
    }
    if (lane < kScanThreads / 64) wsum[lane] = s;  // inclusive wave totals
  }
  __syncthreads();
  const uint32_t r = (w > 0 ? wsum[w - 1] : 0u) + x - v;
  *total = wsum[kScanThreads / 64 - 1];
  __syncthreads();  // wsum is reused by the next call
  return r;
}

}  // namespace

__global__ void __launch_bounds__(kFlat) group_zero_kernel(uint32_t* c, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kFlat;
  for (int64_t i = (int64_t)blockIdx.x * kFlat + threadIdx.x; i < n; i += stride) c[i] = 0u;
}

// counts[j-1] += 1 for every pair with 1 <= j <= N, counts[N] += 1 otherwise.
__global__ void __launch_bounds__(kFlat) group_hist_kernel(const void* idx, int idx64, int64_t P,
                                                           int64_t N, uint32_t* counts) {
  const int64_t stride = (int64_t)gridDim.x * kFlat;
  for (int64_t p = (int64_t)blockIdx.x * kFlat + threadIdx.x; p < P; p += stride) {
    const int64_t j = load_index(idx, idx64, p);
    atomicAdd(&counts[(j >= 1 && j <= N) ? j - 1 : N], 1u);
  }
}

// sums[b] = sum of counters of tile b.
__global__ void __launch_bounds__(kScanThreads) scan_tile_sums_kernel(const uint32_t* c, int64_t n,
                                                                      uint32_t* sums) {
  const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanPer;
  uint32_t s = 0u;
#pragma unroll
  for (int i = 0; i < kScanPer; ++i)
    if (base + i < n) s += c[base + i];
  uint32_t tot;
  block_exclusive_scan(s, &tot);
  if (threadIdx.x == 0) sums[blockIdx.x] = tot;
}

// Exclusive scan of the nb tile sums in place (one block, carried over
// 1024-entry slices).
__global__ void __launch_bounds__(kScanThreads) scan_sums_kernel(uint32_t* sums, int64_t nb) {
  uint32_t carry = 0u;
  for (int64_t b0 = 0; b0 < nb; b0 += kScanThreads) {
    const int64_t i = b0 + threadIdx.x;
    const uint32_t v = i < nb ? sums[i] : 0u;
    uint32_t tot;
    const uint32_t ex = block_exclusive_scan(v, &tot);
    if (i < nb) sums[i] = carry + ex;
    carry += tot;
  }
}

// Counters -> exclusive offsets, in place, for at most kScanThreads tiles:
// block b first sums the totals of tiles 0..b-1 itself (one per thread).
__global__ void __launch_bounds__(kScanThreads) scan_apply_self_kernel(uint32_t* c, int64_t n,
                                                                       const uint32_t* tile_sums) {
  uint32_t off;
  block_exclusive_scan(threadIdx.x < blockIdx.x ? tile_sums[threadIdx.x] : 0u, &off);
  const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanPer;
  uint32_t v[kScanPer];
  uint32_t s = 0u;
#pragma unroll
  for (int i = 0; i < kScanPer; ++i) {
    v[i] = base + i < n ? c[base + i] : 0u;
    s += v[i];
  }
  uint32_t tot;
  uint32_t ex = block_exclusive_scan(s, &tot) + off;
#pragma unroll
  for (int i = 0; i < kScanPer; ++i) {
    if (base + i < n) c[base + i] = ex;
    ex += v[i];
  }
}

// Counters -> exclusive offsets, in place.
__global__ void __launch_bounds__(kScanThreads) scan_apply_kernel(uint32_t* c, int64_t n,
                                                                  const uint32_t* sums) {
  const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanPer;
  uint32_t v[kScanPer];
  uint32_t s = 0u;
#pragma unroll
  for (int i = 0; i < kScanPer; ++i) {
    v[i] = base + i < n ? c[base + i] : 0u;
    s += v[i];
  }
  uint32_t tot;
  uint32_t ex = block_exclusive_scan(s, &tot) + sums[blockIdx.x];
#pragma unroll
  for (int i = 0; i < kScanPer; ++i) {
    if (base + i < n) c[base + i] = ex;
    ex += v[i];
  }
}

// ---- two-level sort ------------------------------------------------------------

constexpr int kBucketTile = 1024;       // pairs per block in the bucket passes
constexpr int kMaxBuckets = 4096;       // LDS counters of the bucket passes
constexpr int kMaxBucketDocs = 8192;    // LDS counters of the per-bucket sort
constexpr int64_t kMaxBucketCells = 1 << 22;  // (bucket, block) counts: 16 MB

struct BucketPlan {
  int64_t nb;   // buckets
  int64_t D;    // documents (keys) per bucket
  int64_t G;    // blocks of the bucket passes
};

inline bool bucket_plan(int64_t npairs, int64_t N, BucketPlan* bp) {
  const int64_t nkeys = N + 1;  // key N: out-of-range index
  int64_t nb = cdiv(nkeys, 128);
  if (nb > kMaxBuckets) nb = kMaxBuckets;
  const int64_t D = cdiv(nkeys, nb);
  if (npairs <= 0 || D > kMaxBucketDocs) return false;
  bp->nb = cdiv(nkeys, D);
  bp->D = D;
  bp->G = cdiv(npairs, kBucketTile);
  return bp->nb * bp->G <= kMaxBucketCells;
}

__device__ __forceinline__ int64_t pair_key(const void* idx, int idx64, int64_t p, int64_t N) {
  const int64_t j = load_index(idx, idx64, p);
  return (j >= 1 && j <= N) ? j - 1 : N;
}

// H[b * G + g] = pairs of block g's tile in bucket b.
__global__ void __launch_bounds__(kFlat) bucket_hist_kernel(const void* idx, int idx64, int64_t P,
                                                            int64_t N, int64_t D, int64_t nb,
                                                            int64_t G, uint32_t* H) {
  __shared__ uint32_t cnt[kMaxBuckets];
  for (int64_t b = threadIdx.x; b < nb; b += kFlat) cnt[b] = 0u;
  __syncthreads();
  const int64_t p0 = (int64_t)blockIdx.x * kBucketTile;
  const int64_t p1 = p0 + kBucketTile < P ? p0 + kBucketTile : P;
  for (int64_t p = p0 + threadIdx.x; p < p1; p += kFlat)
    atomicAdd(&cnt[pair_key(idx, idx64, p, N) / D], 1u);
  __syncthreads();
  for (int64_t b = threadIdx.x; b < nb; b += kFlat) H[b * G + blockIdx.x] = cnt[b];
}

// Pairs of block g's tile to their bucket's slots: T[pos] = (p, key), pos from
// the exclusive scan of H (bucket-major), so bucket b's pairs are contiguous.
__global__ void __launch_bounds__(kFlat) bucket_scatter_kernel(const void* idx, int idx64, int64_t P,
                                                               int64_t N, int64_t D, int64_t nb,
                                                               int64_t G, const uint32_t* Hs,
                                                               PairRef* T) {
  __shared__ uint32_t cur[kMaxBuckets];
  for (int64_t b = threadIdx.x; b < nb; b += kFlat) cur[b] = Hs[b * G + blockIdx.x];
  __syncthreads();
  const int64_t p0 = (int64_t)blockIdx.x * kBucketTile;
  const int64_t p1 = p0 + kBucketTile < P ? p0 + kBucketTile : P;
  for (int64_t p = p0 + threadIdx.x; p < p1; p += kFlat) {
    const int64_t key = pair_key(idx, idx64, p, N);
    const uint32_t pos = atomicAdd(&cur[key / D], 1u);
    PairRef r;
    r.p = (int32_t)p;
    r.j = (int32_t)key;
    T[pos] = r;
  }
}

// Block b sorts bucket b (keys b*D .. b*D+D-1) by key: counts per key in LDS,
// doc_end[key] = end of the key's run, then the scatter into `order`
// (key N, the out-of-range indices, becomes j = -1).
__global__ void __launch_bounds__(kScanThreads) bucket_sort_kernel(const PairRef* T, int64_t P,
                                                                   int64_t N, int64_t D, int64_t nb,
                                                                   int64_t G, const uint32_t* Hs,
                                                                   uint32_t* doc_end,
                                                                   PairRef* order) {
  __shared__ uint32_t cnt[kMaxBucketDocs];
  const int64_t b = blockIdx.x;
  const int64_t k0 = b * D, nk = (k0 + D <= N + 1 ? D : N + 1 - k0);
  const int64_t e0 = Hs[b * G], e1 = b + 1 < nb ? (int64_t)Hs[(b + 1) * G] : P;
  for (int64_t k = threadIdx.x; k < nk; k += kScanThreads) cnt[k] = 0u;
  __syncthreads();
  for (int64_t e = e0 + threadIdx.x; e < e1; e += kScanThreads) atomicAdd(&cnt[T[e].j - k0], 1u);
  __syncthreads();
  // exclusive scan of the nk counters, kPer consecutive ones per thread
  constexpr int kPer = kMaxBucketDocs / kScanThreads;
  uint32_t v[kPer];
  uint32_t s = 0u;
  const int64_t base = (int64_t)threadIdx.x * kPer;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    v[i] = base + i < nk ? cnt[base + i] : 0u;
    s += v[i];
  }
  uint32_t tot;
  uint32_t ex = block_exclusive_scan(s, &tot) + (uint32_t)e0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    if (base + i < nk) {
      cnt[base + i] = ex;                 // cursor: start of the key's run
      doc_end[k0 + base + i] = ex + v[i];  // end of the key's run
    }
    ex += v[i];
  }
  __syncthreads();
  for (int64_t e = e0 + threadIdx.x; e < e1; e += kScanThreads) {
    const PairRef t = T[e];
    const uint32_t pos = atomicAdd(&cnt[t.j - k0], 1u);
    PairRef r;
    r.p = t.p;
    r.j = t.j == N ? -1 : t.j;
    order[pos] = r;
  }
}

// ---- one-level sort (galleries beyond the bucket tables) -------------------------

// order[cursor[key]++] = (p, document of p).
__global__ void __launch_bounds__(kFlat) group_scatter_kernel(const void* idx, int idx64, int64_t P,
                                                              int64_t N, uint32_t* cursor,
                                                              PairRef* order) {
  const int64_t stride = (int64_t)gridDim.x * kFlat;
  for (int64_t p = (int64_t)blockIdx.x * kFlat + threadIdx.x; p < P; p += stride) {
    const int64_t j = load_index(idx, idx64, p);
    const bool valid = j >= 1 && j <= N;
    const uint32_t pos = atomicAdd(&cursor[valid ? j - 1 : N], 1u);
    PairRef r;
    r.p = (int32_t)p;
    r.j = valid ? (int32_t)(j - 1) : -1;
    order[pos] = r;
  }
}

size_t group_workspace_bytes(int64_t npairs, int64_t N) {
  const int64_t ncount = N + 1;
  size_t bytes = align256((size_t)npairs * sizeof(PairRef)) + align256((size_t)ncount * 4) +
                 align256((size_t)cdiv(ncount, kScanTile) * 4);
  BucketPlan bp;
  if (bucket_plan(npairs, N, &bp)) {
    const int64_t nh = bp.nb * bp.G;
    bytes += align256((size_t)npairs * sizeof(PairRef)) + align256((size_t)nh * 4) +
             align256((size_t)cdiv(nh, kScanTile) * 4);
  }
  return bytes;
}

hipError_t group_pairs_by_document(const void* idx, int idx64, int64_t npairs, int64_t N,
                                   void* workspace, const PairRef** order_out,
                                   hipStream_t stream) {
  const int64_t ncount = N + 1;
  const int64_t nb = cdiv(ncount, kScanTile);
  char* w = static_cast<char*>(workspace);
  PairRef* order = reinterpret_cast<PairRef*>(w);
  uint32_t* counts = reinterpret_cast<uint32_t*>(w + align256((size_t)npairs * sizeof(PairRef)));
  uint32_t* sums = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(counts) +
                                               align256((size_t)ncount * 4));
  BucketPlan bp;
  if (bucket_plan(npairs, N, &bp)) {
    // counts doubles as doc_end (the run ends the bucket sort writes)
    char* t = reinterpret_cast<char*>(sums) + align256((size_t)nb * 4);
    PairRef* T = reinterpret_cast<PairRef*>(t);
    uint32_t* H = reinterpret_cast<uint32_t*>(t + align256((size_t)npairs * sizeof(PairRef)));
    const int64_t nh = bp.nb * bp.G;
    uint32_t* Hsums = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(H) + align256((size_t)nh * 4));
    hipLaunchKernelGGL(bucket_hist_kernel, dim3((unsigned)bp.G), dim3(kFlat), 0, stream, idx, idx64,
                       npairs, N, bp.D, bp.nb, bp.G, H);
    hipError_t e = exclusive_scan_u32(H, nh, Hsums, stream);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(bucket_scatter_kernel, dim3((unsigned)bp.G), dim3(kFlat), 0, stream, idx,
                       idx64, npairs, N, bp.D, bp.nb, bp.G, H, T);
    hipLaunchKernelGGL(bucket_sort_kernel, dim3((unsigned)bp.nb), dim3(kScanThreads), 0, stream, T,
                       npairs, N, bp.D, bp.nb, bp.G, H, counts, order);
    *order_out = order;
    return hipGetLastError();
  }
  hipLaunchKernelGGL(group_zero_kernel, dim3(flat_blocks(ncount)), dim3(kFlat), 0, stream, counts,
                     ncount);
  hipLaunchKernelGGL(group_hist_kernel, dim3(flat_blocks(npairs)), dim3(kFlat), 0, stream, idx,
                     idx64, npairs, N, counts);
  const hipError_t e = exclusive_scan_u32(counts, ncount, sums, stream);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(group_scatter_kernel, dim3(flat_blocks(npairs)), dim3(kFlat), 0, stream, idx,
                     idx64, npairs, N, counts, order);
  *order_out = order;
  return hipGetLastError();
}

hipError_t group_pairs_by_document(const void* idx, int idx64, int64_t npairs, int64_t N,
                                   void* workspace, const PairRef** order_out,
                                   const uint32_t** doc_end, hipStream_t stream) {
  // after the scatter, counter j holds the end of document j's run of pairs
  *doc_end = reinterpret_cast<const uint32_t*>(static_cast<const char*>(workspace) +
                                               align256((size_t)npairs * sizeof(PairRef)));
  return group_pairs_by_document(idx, idx64, npairs, N, workspace, order_out, stream);
}

size_t scan_workspace_bytes(int64_t n) { return align256((size_t)cdiv(n > 0 ? n : 1, kScanTile) * 4); }

hipError_t exclusive_scan_u32(uint32_t* counts, int64_t n, uint32_t* sums, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int64_t nb = cdiv(n, kScanTile);
  hipLaunchKernelGGL(scan_tile_sums_kernel, dim3((unsigned)nb), dim3(kScanThreads), 0, stream,
                     counts, n, sums);
  if (nb <= kScanThreads) {
    // at most one tile total per thread: every apply block sums the totals
    // before it (one launch fewer; `sums` keeps the tile totals)
    hipLaunchKernelGGL(scan_apply_self_kernel, dim3((unsigned)nb), dim3(kScanThreads), 0, stream,
                       counts, n, sums);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(scan_sums_kernel, dim3(1), dim3(kScanThreads), 0, stream, sums, nb);
  hipLaunchKernelGGL(scan_apply_kernel, dim3((unsigned)nb), dim3(kScanThreads), 0, stream, counts,
                     n, sums);
  return hipGetLastError();
}

// ---- workspace pool -------------------------------------------------------------

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_pool_mutex;
hipMemPool_t g_pool[kMaxDevices] = {};

hipError_t device_pool(int dev, hipMemPool_t* pool) {
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_pool_mutex);
  if (!g_pool[dev]) {
    hipMemPoolProps props = {};
    props.allocType = hipMemAllocationTypePinned;
    props.handleTypes = hipMemHandleTypeNone;
    props.location.type = hipMemLocationTypeDevice;
    props.location.id = dev;
    hipMemPool_t p = nullptr;
    hipError_t e = hipMemPoolCreate(&p, &props);
    if (e != hipSuccess) return e;
    uint64_t keep = UINT64_MAX;  // never trim at synchronisation points
    e = hipMemPoolSetAttribute(p, hipMemPoolAttrReleaseThreshold, &keep);
    if (e != hipSuccess) return e;
    g_pool[dev] = p;
  }
  *pool = g_pool[dev];
  return hipSuccess;
}

}  // namespace

hipError_t stream_device(hipStream_t stream, int* dev) {
  if (stream == nullptr) return hipGetDevice(dev);
  hipDevice_t d;
  const hipError_t e = hipStreamGetDevice(stream, &d);
  *dev = (int)d;
  return e;
}

namespace {
std::atomic<uint64_t> g_workspace_allocs{0};
}  // namespace

uint64_t workspace_alloc_count() { return g_workspace_allocs.load(std::memory_order_relaxed); }

hipError_t workspace_alloc(void** ptr, size_t bytes, hipStream_t stream) {
  g_workspace_allocs.fetch_add(1, std::memory_order_relaxed);
  int dev = 0;
  hipError_t e = stream_device(stream, &dev);
  if (e != hipSuccess) return e;
  hipMemPool_t pool;
  e = device_pool(dev, &pool);
  if (e != hipSuccess) return e;
  return hipMallocFromPoolAsync(ptr, bytes, pool, stream);
}

hipError_t workspace_free(void* ptr, hipStream_t stream) { return hipFreeAsync(ptr, stream); }

}  // namespace fms
