// fms_api.hip -- the extern "C" boundary of libflashmaxsim_hip.so.
//
// Validates shapes / pointers on the host (the reference validates in Julia
// before every launch: DimensionMismatch in forward_layouts.jl:20-47,
// forward_pair.jl:14-21, quant.jl:62-94, packed.jl:138-151), picks the
// kernel and enqueues it on the caller's stream without synchronising.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "../../include/flashmaxsim_hip.h"
#include "fms_backward.hpp"
#include "fms_group.hpp"
#include "fms_inbatch.hpp"
#include "fms_inbatch_split.hpp"
#include "fms_misc.hpp"
#include "fms_topk.hpp"
#include "fms_scan_decl.hpp"
#include "fms_runs.hpp"

#define FMS_VERSION_STRING "flashmaxsim-hip 0.1.0 (gfx950)"

// Grouping workspace of fms_launch_candidates_scan_noalloc (see scratch_address).
static __device__ __align__(256) unsigned char scratch[FMS_NOALLOC_SCRATCH_BYTES];

namespace {

using namespace fms;

constexpr int64_t kMaxSeqBytes = (int64_t)1 << 31;  // one buffer resource per sequence
constexpr int64_t kMaxTokens = ((int64_t)1 << 31) - 1;

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

fms_status from_hip(hipError_t e) { return e == hipSuccess ? FMS_OK : FMS_EHIP; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int elem_bytes(int32_t dtype) {
  switch (dtype) {
    case FMS_F32: return 4;
    case FMS_F16: return 2;
    case FMS_BF16: return 2;
    default: return 0;
  }
}

// Elements per 16-byte fragment for a stored type (row alignment unit).
int frag_elems(int esz) { return esz == 4 ? 1 : 16 / esz; }

bool seq_ok(int64_t tokens, int64_t dim, int esz) {
  return tokens >= 0 && tokens <= kMaxTokens && dim >= 0 && tokens * dim * esz < kMaxSeqBytes;
}

// Rows are 16-byte multiples and every base is 16-byte aligned: the fast
// fragment loads apply.  fp32 loads 4 bytes per lane and is always "vec".
bool vec_ok(int esz, int64_t dim, std::initializer_list<const void*> ptrs) {
  if (esz == 4) return true;
  if (dim % frag_elems(esz) != 0) return false;
  for (const void* p : ptrs)
    if (p && !aligned16(p)) return false;
  return true;
}

// Launches the scan for a float feature type (dtype already validated).
template <class L>
hipError_t launch_float(int32_t dtype, const L& lay, int dim, int rows, int64_t npairs,
                        int32_t* args, float* partial, float* scores, float neg, bool norm,
                        bool vec, hipStream_t st) {
  switch (dtype) {
    case FMS_F16:
      return launch_scan<OpF16, L>(lay, dim, rows, npairs, args, partial, scores, neg, norm, vec,
                                   st);
    case FMS_BF16:
      return launch_scan<OpBF16, L>(lay, dim, rows, npairs, args, partial, scores, neg, norm,
                                    vec, st);
    default:
      return launch_scan<OpF32, L>(lay, dim, rows, npairs, args, partial, scores, neg, norm, vec,
                                   st);
  }
}

template <class L>
fms_status run_float(int32_t dtype, const L& lay, int dim, int rows, int64_t npairs,
                     int32_t* args, float* partial, float* scores, float neg, bool norm, bool vec,
                     hipStream_t st) {
  if (elem_bytes(dtype) == 0) return FMS_EUNSUPPORTED;
  if (!scan_grid_fits(npairs)) return FMS_EUNSUPPORTED;  // 32-bit work-item count
  return from_hip(
      launch_float(dtype, lay, dim, rows, npairs, args, partial, scores, neg, norm, vec, st));
}

// Candidate pair grouping (fms_candidates_grouping): 0 auto, 1 always, 2 never,
// 3 always with the query tiles read from Q (no fragment-ordered copy).  Per
// host thread: a caller that sets it changes no other thread's calls.
thread_local int t_grouping = 0;

// Smallest candidate batch worth the five extra launches of the document sort.
constexpr int64_t kGroupMinPairs = 16384;

// Whether a candidate scan of P pairs over N documents of dbytes each runs in
// document order.  Auto: P >= kGroupMinPairs; the O(N) counter passes of the
// sort (16 bytes per document) stay under 5% of the document bytes the
// ungrouped scan would read; and the document reads saved are worth giving
// up the query-tile reuse of output order (consecutive candidates of one
// query): at least 30% of the reads, estimated for indices drawn uniformly
// over 1..N, where P draws hit N*(1 - exp(-P/N)) distinct documents.
// Pair ids and document ids must fit 32 bits.
bool group_candidates(int64_t P, int64_t N, int64_t dbytes) {
  if (P < 1 || P >= INT32_MAX || N < 1 || N >= INT32_MAX) return false;
  const int mode = t_grouping;
  if (mode == 2) return false;
  if (mode == 1 || mode == 3) return true;
  if (P < kGroupMinPairs || (double)(N + 1) * 16.0 > 0.05 * (double)P * (double)dbytes)
    return false;
  const double distinct = -(double)N * expm1(-(double)P / (double)N);
  return distinct <= 0.7 * (double)P;
}

// The in-batch kernel for a call: 1 the register-resident MFMA kernel
// (16-bit, dim 32..128 in steps of 32), 2 the split-K kernel (fp32, other
// 16-bit dims whose rows are whole 16-byte units), 0 the per-pair scan.
int inbatch_path(int32_t dtype, int64_t dim, int64_t Tq, int64_t Td, int64_t Bq, int64_t Bd,
                 const void* Q, const void* D) {
  const int esz = elem_bytes(dtype);
  if ((dtype == FMS_F16 || dtype == FMS_BF16) && inbatch_mfma_supported(dim, Tq, Td, Q, D) &&
      Bq * ((Tq + 31) / 32) <= kMaxTokens && Bd <= kMaxTokens)
    return 1;
  if (esz != 0 && inbatch_split_supported(esz, dim, Tq, Td, Bq, Bd, Q, D) &&
      Tq * dim * esz < kMaxSeqBytes)
    return 2;
  return 0;
}

// Where a candidate call's document-grouping workspace comes from: the
// library's stream-ordered memory pool, or the file-scope device array of
// the no-allocation entry point.
enum class Workspace { kPool, kScratch };

// ---- scratch of the no-allocation entry point --------------------------------------
// fms_launch_candidates_scan_noalloc takes its grouping workspace from this
// array instead of the pool, so the call allocates nothing.  Every GPU the
// library runs on holds its own copy for the life of the process; host code
// uses the address hipGetSymbolAddress returns for the current device (the
// array's name on the host is only a stand-in).  Calls on one GPU share it,
// so calls that overlap on one GPU race.
constexpr size_t kNoallocScratchBytes = (size_t)FMS_NOALLOC_SCRATCH_BYTES;

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// The device address of `scratch` on the stream's device, looked up once per
// device with that device current.
hipError_t scratch_address(hipStream_t st, void** out) {
  int dev = 0;
  hipError_t e = stream_device(st, &dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxScratchDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    int cur = 0;
    e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    const hipError_t er = cur != dev ? hipSetDevice(cur) : hipSuccess;
    if (e != hipSuccess) return e;
    if (er != hipSuccess) return er;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}

// The document-batch scan (fms_runs.hpp) for a grouped candidate call:
// `runs.applies()` says whether it serves the call's type and dim (else
// scan_fast runs over LayCandSorted), `runs(order, doc_end)` launches it.
struct NoRuns {
  bool applies() const { return false; }
  size_t qfrag_bytes() const { return 0; }
  hipError_t operator()(const PairRef*, const uint32_t*, char*) const {
    return hipErrorInvalidValue;
  }
};

template <class Op>
struct RunsLauncher {
  const LayCand* lay;
  int dim, rows;
  int64_t npairs;
  int32_t* args;
  float* partial;
  float* scores;
  float neg;
  bool norm, vec;
  bool applies() const { return runs_supported<Op>(dim, vec); }
  // Workspace for the query tiles in fragment order (0: the scan loads them
  // from Q directly).
  size_t qfrag_bytes() const { return runs_qfrag_bytes<Op>(dim, rows, npairs / lay->C); }
  hipError_t operator()(const PairRef* order, const uint32_t* doc_end, char* qfrag) const {
    RunArgs A;
    A.lay = *lay;
    A.dim = dim;
    A.nkb = (dim + Op::kKb - 1) / Op::kKb;
    A.rows = rows;
    A.nqt = rows > 0 ? (rows + kTile - 1) / kTile : 1;
    A.ppw = 0;  // set by launch_runs
    A.npairs = npairs;
    A.args = args;
    A.partial = partial;
    A.scores = scores;
    A.neg = neg;
    A.norm = norm ? 1 : 0;
    A.order = order;
    A.doc_end = doc_end;
    A.qfrag = qfrag;
    return launch_runs<Op>(A, st);
  }
  hipStream_t st;
};

// Runs launch(layout) on the candidate layout, in document order when
// group_candidates says so (through `runs` when it serves the call, else
// scan_fast over LayCandSorted), otherwise in output order.  The grouping
// workspace comes from `ws`:
//   kPool: the library pool, released on the same stream; an allocation
//     failure falls back to output order (the results are identical);
//   kScratch: the no-allocation array.  A workspace larger than it scans in
//     output order under automatic grouping (the order is only a
//     performance choice; the results are identical) and is FMS_ESCRATCH
//     when grouping was forced (nothing is launched).  The grouping kernels
//     clear every counter they use, so the array's previous contents do not
//     matter.
template <class Runs, class Launch>
fms_status run_candidates(const LayCand& lay, int64_t npairs, hipStream_t st, Workspace ws,
                          const Runs& runs, Launch&& launch) {
  if (!scan_grid_fits(npairs)) return FMS_EUNSUPPORTED;  // 32-bit work-item count
  if (group_candidates(npairs, lay.N, lay.dbytes)) {
    const size_t need = (group_workspace_bytes(npairs, lay.N) + 255) / 256 * 256;
    // the document-batch scan's fragment-ordered query tiles follow the
    // grouping workspace (dropped when the no-allocation scratch cannot
    // hold both: the scan then loads the tiles from Q)
    size_t qneed = runs.applies() && t_grouping != 3 ? runs.qfrag_bytes() : 0;
    void* buf = nullptr;
    bool pooled = false;
    if (ws == Workspace::kScratch && need > kNoallocScratchBytes) {
      if (t_grouping != 0) return FMS_ESCRATCH;  // forced grouping cannot be honoured
      // automatic grouping: buf stays null and the call scans in output order
    } else if (ws == Workspace::kScratch) {
      if (qneed > kNoallocScratchBytes - need) qneed = 0;
      const hipError_t e = scratch_address(st, &buf);
      if (e != hipSuccess) return from_hip(e);
    } else if (workspace_alloc(&buf, need + qneed, st) == hipSuccess) {
      pooled = true;
    } else {
      (void)hipGetLastError();  // clear the failed allocation; scan in output order
      buf = nullptr;
    }
    if (buf) {
      LayCandSorted sl;
      sl.c = lay;
      const uint32_t* doc_end = nullptr;
      hipError_t e = group_pairs_by_document(lay.idx, lay.idx64, npairs, lay.N, buf, &sl.order,
                                             &doc_end, st);
      char* qfrag = qneed ? static_cast<char*>(buf) + need : nullptr;
      if (e == hipSuccess) e = runs.applies() ? runs(sl.order, doc_end, qfrag) : launch(sl);
      const hipError_t ef = pooled ? workspace_free(buf, st) : hipSuccess;
      return from_hip(e != hipSuccess ? e : ef);
    }
  }
  return from_hip(launch(lay));
}

// Byte width of an INT8 scale type (fp32 or fp16); 0 = not a scale type.
int scale_bytes(int32_t dtype) {
  return dtype == FMS_F32 ? 4 : (dtype == FMS_F16 ? 2 : 0);
}

// The INT8 scan for the document-scale width (fp32: OpI8, fp16: OpI8H).
template <class L>
hipError_t launch_int8(int ds_esz, const L& lay, int dim, int rows, int64_t npairs, int32_t* args,
                       float* partial, float* scores, float neg, bool norm, bool vec,
                       hipStream_t st) {
  if (ds_esz == 2)
    return launch_scan<OpI8H, L>(lay, dim, rows, npairs, args, partial, scores, neg, norm, vec, st);
  return launch_scan<OpI8, L>(lay, dim, rows, npairs, args, partial, scores, neg, norm, vec, st);
}

}  // namespace

// ---- backward helpers ----------------------------------------------------------

namespace {

// Sources are numbered p * rows + t in 32 bits; destination rows index in 32 bits.
bool pullback_ok(int64_t npairs, int64_t rows, int64_t nd_rows) {
  return npairs * rows < ((int64_t)1 << 31) && nd_rows < ((int64_t)1 << 31);
}

PullbackArgs pullback_args(int32_t dtype, void* dQ, void* dD, const void* Q, const void* D,
                           const int32_t* args, const void* Delta, const void* inv_n,
                           int64_t npairs, int64_t G, int64_t nq_rows, int64_t nd_rows,
                           int64_t rows, int64_t dim) {
  PullbackArgs a;
  a.dtype = dtype;
  a.dQ = static_cast<char*>(dQ);
  a.dD = static_cast<char*>(dD);
  a.Qbase = static_cast<const char*>(Q);
  a.Dbase = static_cast<const char*>(D);
  a.args = args;
  a.Delta = Delta;
  a.inv_n = inv_n;
  a.npairs = npairs;
  a.G = npairs > 0 ? G : 1;
  a.nq_rows = nq_rows;
  a.nd_rows = nd_rows;
  a.rows = (int)rows;
  a.dim = (int)dim;
  a.zero_dq = false;
  return a;
}

// The pointers an output of `rows` rows needs, and the inputs the pairs read.
bool pullback_ptrs(int64_t nq_rows, const void* Q, const void* dQ, int64_t nd_rows, const void* D,
                   const void* dD, int64_t npairs, const void* args, const void* Delta) {
  if (nq_rows > 0 && (!Q || !dQ)) return false;
  if (nd_rows > 0 && (!D || !dD)) return false;
  return npairs == 0 || (args && Delta);
}

}  // namespace

extern "C" {

const char* fms_status_string(fms_status s) {
  switch (s) {
    case FMS_OK: return "ok";
    case FMS_EINVAL: return "invalid argument (shape, NULL pointer or alignment)";
    case FMS_EUNSUPPORTED: return "unsupported dtype or size";
    case FMS_EHIP: return "HIP runtime error";
    case FMS_ESCRATCH:
      return "the call needs more workspace than the no-allocation entry point's scratch "
             "(FMS_NOALLOC_SCRATCH_BYTES)";
    default: return "unknown status";
  }
}

const char* fms_version(void) { return FMS_VERSION_STRING; }

int fms_arch_supported(void) {
  // Asked before every call by the Julia overrides, so the answer is cached per
  // device (0 = not yet asked, 1 = gfx950, 2 = other); racing first calls store
  // the same value.
  static std::atomic<int> known[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < 64) {
    const int k = known[dev].load(std::memory_order_relaxed);
    if (k != 0) return k == 1 ? 1 : 0;
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return 0;
  const int ok = strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
  if (dev >= 0 && dev < 64) known[dev].store(ok ? 1 : 2, std::memory_order_relaxed);
  return ok;
}

fms_status fms_launch_paired_scan(int32_t dtype, int32_t* args, float* partial, const void* Q,
                                  const void* D, const uint8_t* qmask, const uint8_t* dmask,
                                  int64_t dim, int64_t Tq, int64_t Td, int64_t B, float* scores,
                                  int32_t normalize, void* stream) {
  const int esz = elem_bytes(dtype);
  if (esz == 0) return FMS_EUNSUPPORTED;
  if (dim < 0 || Tq < 0 || Td < 0 || B < 0 || (normalize & ~1)) return FMS_EINVAL;
  if (!seq_ok(Tq, dim, esz) || !seq_ok(Td, dim, esz)) return FMS_EUNSUPPORTED;
  if (B == 0 || (Tq == 0 && !scores)) return FMS_OK;
  if ((Tq * dim > 0 && !Q) || (Td * dim > 0 && !D)) return FMS_EINVAL;
  LayPaired lay;
  lay.Q = static_cast<const char*>(Q);
  lay.D = static_cast<const char*>(D);
  lay.qm = qmask;
  lay.dm = dmask;
  lay.Qs = nullptr;
  lay.Ds = nullptr;
  lay.qbytes = Tq * dim * esz;
  lay.dbytes = Td * dim * esz;
  lay.Tq = (int)Tq;
  lay.Td = (int)Td;
  return run_float(dtype, lay, (int)dim, (int)Tq, B, args, partial, scores, 0.0f, normalize != 0,
                   vec_ok(esz, dim, {Q, D}), as_stream(stream));
}

fms_status fms_launch_pair_scan(int32_t dtype, int32_t* argmax_u, float* partial, const void* q,
                                const void* d, const uint8_t* qmask, const uint8_t* dmask,
                                int64_t dim, int64_t Tq, int64_t Td, float* score,
                                int32_t normalize, void* stream) {
  return fms_launch_paired_scan(dtype, argmax_u, partial, q, d, qmask, dmask, dim, Tq, Td, 1,
                                score, normalize, stream);
}

}  // extern "C"

namespace {

// fms_launch_candidates_scan and its no-allocation variant: the same checks,
// kernels and results; only the grouping workspace differs.
fms_status candidates_scan(Workspace ws, int32_t dtype, int32_t* args, float* partial,
                           const void* Q, const void* gallery, const void* idx,
                           int32_t idx_bytes, const uint8_t* qmask, const uint8_t* dmask,
                           int64_t dim, int64_t Tq, int64_t B, int64_t Td, int64_t N, int64_t C,
                           float* scores, float neg, int32_t normalize, void* stream) {
  const int esz = elem_bytes(dtype);
  if (esz == 0) return FMS_EUNSUPPORTED;
  if (dim < 0 || Tq < 0 || Td < 0 || B < 0 || N < 0 || C < 0 || (normalize & ~1))
    return FMS_EINVAL;
  if (idx_bytes != 4 && idx_bytes != 8) return FMS_EINVAL;
  if (!seq_ok(Tq, dim, esz) || !seq_ok(Td, dim, esz)) return FMS_EUNSUPPORTED;
  if (C == 0 || B == 0 || (Tq == 0 && !scores)) return FMS_OK;
  if (B > INT64_MAX / C) return FMS_EUNSUPPORTED;
  if (!idx || (Tq * dim > 0 && !Q) || (N * Td * dim > 0 && !gallery)) return FMS_EINVAL;
  LayCand lay;
  lay.Q = static_cast<const char*>(Q);
  lay.G = static_cast<const char*>(gallery);
  lay.idx = idx;
  lay.idx64 = idx_bytes == 8;
  lay.qm = qmask;
  lay.dm = dmask;
  lay.Qs = nullptr;
  lay.Gs = nullptr;
  lay.qbytes = Tq * dim * esz;
  lay.dbytes = Td * dim * esz;
  lay.N = N;
  lay.C = C;
  lay.Tq = (int)Tq;
  lay.Td = (int)Td;
  const bool vec = vec_ok(esz, dim, {Q, gallery});
  const hipStream_t st = as_stream(stream);
  auto launch = [&](const auto& L) -> hipError_t {
    return launch_float(dtype, L, (int)dim, (int)Tq, C * B, args, partial, scores, neg,
                        normalize != 0, vec, st);
  };
  if (dtype == FMS_F16 || dtype == FMS_BF16) {
    const bool bf = dtype == FMS_BF16;
    RunsLauncher<OpF16> r16{&lay, (int)dim, (int)Tq, C * B, args, partial, scores, neg,
                            normalize != 0, vec, st};
    RunsLauncher<OpBF16> rbf{&lay, (int)dim, (int)Tq, C * B, args, partial, scores, neg,
                             normalize != 0, vec, st};
    return bf ? run_candidates(lay, C * B, st, ws, rbf, launch)
              : run_candidates(lay, C * B, st, ws, r16, launch);
  }
  return run_candidates(lay, C * B, st, ws, NoRuns{}, launch);
}

}  // namespace

extern "C" {

fms_status fms_launch_candidates_scan(int32_t dtype, int32_t* args, float* partial,
                                      const void* Q, const void* gallery, const void* idx,
                                      int32_t idx_bytes, const uint8_t* qmask,
                                      const uint8_t* dmask, int64_t dim, int64_t Tq, int64_t B,
                                      int64_t Td, int64_t N, int64_t C, float* scores, float neg,
                                      int32_t normalize, void* stream) {
  return candidates_scan(Workspace::kPool, dtype, args, partial, Q, gallery, idx, idx_bytes,
                         qmask, dmask, dim, Tq, B, Td, N, C, scores, neg, normalize, stream);
}

fms_status fms_launch_candidates_scan_noalloc(int32_t dtype, int32_t* args, float* partial,
                                              const void* Q, const void* gallery,
                                              const void* idx, int32_t idx_bytes,
                                              const uint8_t* qmask, const uint8_t* dmask,
                                              int64_t dim, int64_t Tq, int64_t B, int64_t Td,
                                              int64_t N, int64_t C, float* scores, float neg,
                                              int32_t normalize, void* stream) {
  return candidates_scan(Workspace::kScratch, dtype, args, partial, Q, gallery, idx, idx_bytes,
                         qmask, dmask, dim, Tq, B, Td, N, C, scores, neg, normalize, stream);
}

fms_status fms_inbatch_device_scan(int32_t dtype, float* S, int32_t* args, const void* Q,
                                   const void* D, const uint8_t* qmask, const uint8_t* dmask,
                                   int64_t dim, int64_t Tq, int64_t Bq, int64_t Td, int64_t Bd,
                                   int32_t normalize, void* stream) {
  const int esz = elem_bytes(dtype);
  if (esz == 0) return FMS_EUNSUPPORTED;
  if (dim < 0 || Tq < 0 || Td < 0 || Bq < 0 || Bd < 0 || (normalize & ~1)) return FMS_EINVAL;
  if (!seq_ok(Tq, dim, esz) || !seq_ok(Td, dim, esz)) return FMS_EUNSUPPORTED;
  if (Bq == 0 || Bd == 0) return FMS_OK;
  if (!S || (Tq * dim > 0 && !Q) || (Td * dim > 0 && !D)) return FMS_EINVAL;
  const int path = inbatch_path(dtype, dim, Tq, Td, Bq, Bd, Q, D);
  if (path == 1) {
    InBatchArgs a;
    a.Q = static_cast<const char*>(Q);
    a.D = static_cast<const char*>(D);
    a.qm = qmask;
    a.dm = dmask;
    a.S = S;
    a.args = args;
    a.Bq = (int)Bq;
    a.Bd = (int)Bd;
    a.Tq = (int)Tq;
    a.Td = (int)Td;
    a.dim = (int)dim;
    a.norm = normalize;
    return from_hip(launch_inbatch_mfma(dtype == FMS_BF16, a, as_stream(stream)));
  }
  // fp32, and 16-bit dims the register-resident kernel does not take: the
  // split-K kernel (document slices staged through LDS, query fragments in
  // registers, a K slice at a time)
  if (path == 2) {
    InBatchSplitArgs a;
    a.Q = static_cast<const char*>(Q);
    a.D = static_cast<const char*>(D);
    a.qm = qmask;
    a.dm = dmask;
    a.S = S;
    a.args = args;
    a.Bq = (int)Bq;
    a.Bd = (int)Bd;
    a.Tq = (int)Tq;
    a.Td = (int)Td;
    a.rowbytes = (int)(dim * esz);
    a.norm = normalize;
    return from_hip(launch_inbatch_split(dtype, a, as_stream(stream)));
  }
  // other shapes (rows not a multiple of 16 bytes, unaligned bases): the
  // per-pair scan over p = j + Bd*i
  LayInBatch lay;
  lay.Q = static_cast<const char*>(Q);
  lay.D = static_cast<const char*>(D);
  lay.qm = qmask;
  lay.dm = dmask;
  lay.qbytes = Tq * dim * esz;
  lay.dbytes = Td * dim * esz;
  lay.Bd = Bd;
  lay.Tq = (int)Tq;
  lay.Td = (int)Td;
  return run_float(dtype, lay, (int)dim, (int)Tq, Bq * Bd, args, nullptr, S, 0.0f,
                   normalize != 0, vec_ok(esz, dim, {Q, D}), as_stream(stream));
}

fms_status fms_launch_packed_scan(int32_t dtype, int32_t* args, float* partial, const void* q,
                                  const void* tokens, const int32_t* cu, const uint8_t* qmask,
                                  int64_t dim, int64_t Tq, int64_t B, int64_t ntokens,
                                  float* scores, int32_t normalize, void* stream) {
  const int esz = elem_bytes(dtype);
  if (esz == 0) return FMS_EUNSUPPORTED;
  if (dim < 0 || Tq < 0 || B < 0 || ntokens < 0 || (normalize & ~1)) return FMS_EINVAL;
  // Each document gets its own buffer resource; one longer than 2^31 bytes
  // is truncated to that size on device (LayPacked::get).
  if (!seq_ok(Tq, dim, esz)) return FMS_EUNSUPPORTED;
  if (B == 0 || (Tq == 0 && !scores)) return FMS_OK;
  if (!cu || (Tq * dim > 0 && !q) || (ntokens * dim > 0 && !tokens)) return FMS_EINVAL;
  LayPacked lay;
  lay.q = static_cast<const char*>(q);
  lay.tok = static_cast<const char*>(tokens);
  lay.cu = cu;
  lay.qm = qmask;
  lay.ntok = ntokens;
  lay.rowbytes = dim * esz;
  lay.Tq = (int)Tq;
  return run_float(dtype, lay, (int)dim, (int)Tq, B, args, partial, scores, 0.0f, normalize != 0,
                   vec_ok(esz, dim, {q, tokens}), as_stream(stream));
}

fms_status fms_launch_packed_multi_scan(int32_t dtype, int32_t* args, float* scores,
                                        const void* Q, const void* tokens, const int32_t* cu,
                                        const uint8_t* qmask, int64_t dim, int64_t Tq, int64_t nq,
                                        int64_t B, int64_t ntokens, int64_t max_len,
                                        int32_t normalize, void* stream) {
  const int esz = elem_bytes(dtype);
  if (esz == 0) return FMS_EUNSUPPORTED;
  if (dim < 0 || Tq < 0 || nq < 0 || B < 0 || ntokens < 0 || max_len < 0 || (normalize & ~1))
    return FMS_EINVAL;
  if (!seq_ok(Tq, dim, esz) || nq > kMaxTokens || B > kMaxTokens) return FMS_EUNSUPPORTED;
  if (nq == 0 || B == 0) return FMS_OK;
  if (!scores || !cu || (Tq * dim > 0 && !Q) || (ntokens * dim > 0 && !tokens)) return FMS_EINVAL;
  const hipStream_t st = as_stream(stream);
  if ((dtype == FMS_F16 || dtype == FMS_BF16) && inbatch_mfma_supported(dim, Tq, max_len, Q, tokens) &&
      max_len >= 1 && ntokens <= kMaxTokens && nq * ((Tq + 31) / 32) <= kMaxTokens) {
    InBatchArgs a;
    a.Q = static_cast<const char*>(Q);
    a.D = static_cast<const char*>(tokens);
    a.qm = qmask;
    a.dm = nullptr;
    a.cu = cu;
    a.ntok = ntokens;
    a.S = scores;
    a.args = args;
    a.Bq = (int)nq;
    a.Bd = (int)B;
    a.Tq = (int)Tq;
    a.Td = (int)max_len;
    a.dim = (int)dim;
    a.norm = normalize;
    return from_hip(launch_inbatch_mfma(dtype == FMS_BF16, a, st));
  }
  // other shapes / fp32: one packed scan per query
  for (int64_t i = 0; i < nq; ++i) {
    const fms_status r = fms_launch_packed_scan(
        dtype, args ? args + i * B * Tq : nullptr, nullptr,
        static_cast<const char*>(Q) + i * Tq * dim * esz, tokens, cu,
        qmask ? qmask + i * Tq : nullptr, dim, Tq, B, ntokens, scores + i * B, normalize, stream);
    if (r != FMS_OK) return r;
  }
  return FMS_OK;
}

fms_status fms_launch_varlen_scan(int32_t dtype, int32_t* args, float* partial,
                                  const void* Qtokens, const void* Dtokens, const int32_t* cu_q,
                                  const int32_t* cu_d, int64_t dim, int64_t max_q, int64_t N,
                                  int64_t nq_tokens, int64_t nd_tokens, float* scores,
                                  int32_t normalize, void* stream) {
  const int esz = elem_bytes(dtype);
  if (esz == 0) return FMS_EUNSUPPORTED;
  if (dim < 0 || max_q < 0 || N < 0 || nq_tokens < 0 || nd_tokens < 0 || (normalize & ~1))
    return FMS_EINVAL;
  if (!seq_ok(max_q, dim, esz)) return FMS_EUNSUPPORTED;
  if (N == 0 || (max_q == 0 && !scores)) return FMS_OK;
  if (!cu_q || !cu_d || (nq_tokens * dim > 0 && !Qtokens) || (nd_tokens * dim > 0 && !Dtokens))
    return FMS_EINVAL;
  LayVarlen lay;
  lay.Qt = static_cast<const char*>(Qtokens);
  lay.Dt = static_cast<const char*>(Dtokens);
  lay.cu_q = cu_q;
  lay.cu_d = cu_d;
  lay.nq = nq_tokens;
  lay.nd = nd_tokens;
  lay.rowbytes = dim * esz;
  lay.max_q = (int)max_q;
  return run_float(dtype, lay, (int)dim, (int)max_q, N, args, partial, scores, 0.0f,
                   normalize != 0, vec_ok(esz, dim, {Qtokens, Dtokens}), as_stream(stream));
}

fms_status fms_int8_quantize(int32_t dtype, const void* X, int8_t* codes, void* scales,
                             int64_t dim, int64_t ntok, void* stream) {
  if (dtype != FMS_F32 && dtype != FMS_F16) return FMS_EUNSUPPORTED;
  if (dim < 0 || ntok < 0 || dim > kMaxTokens) return FMS_EINVAL;
  if (ntok == 0) return FMS_OK;
  if (!scales || (dim > 0 && (!X || !codes))) return FMS_EINVAL;
  return from_hip(quantize_int8(dtype == FMS_F16, X, codes, scales, (int)dim, ntok,
                                as_stream(stream)));
}

fms_status fms_launch_int8_paired_scan(int32_t* args, float* partial, const int8_t* Qc,
                                       const void* Qs, int32_t qs_dtype, const int8_t* Dc,
                                       const void* Ds, int32_t ds_dtype, const uint8_t* qmask,
                                       const uint8_t* dmask, int64_t dim, int64_t Tq, int64_t Td,
                                       int64_t B, float* scores, int32_t normalize,
                                       void* stream) {
  const int qs_esz = scale_bytes(qs_dtype), ds_esz = scale_bytes(ds_dtype);
  if (qs_esz == 0 || ds_esz == 0) return FMS_EUNSUPPORTED;
  if (dim < 0 || Tq < 0 || Td < 0 || B < 0 || (normalize & ~1)) return FMS_EINVAL;
  if (!seq_ok(Tq, dim, 4) || !seq_ok(Td, dim, 4)) return FMS_EUNSUPPORTED;
  if (B == 0 || (Tq == 0 && !scores)) return FMS_OK;
  if ((Tq > 0 && (!Qs || (dim > 0 && !Qc))) || (Td > 0 && (!Ds || (dim > 0 && !Dc))))
    return FMS_EINVAL;
  LayPaired lay;
  lay.Q = reinterpret_cast<const char*>(Qc);
  lay.D = reinterpret_cast<const char*>(Dc);
  lay.qm = qmask;
  lay.dm = dmask;
  lay.Qs = static_cast<const char*>(Qs);
  lay.Ds = static_cast<const char*>(Ds);
  lay.qbytes = Tq * dim;
  lay.dbytes = Td * dim;
  lay.Tq = (int)Tq;
  lay.Td = (int)Td;
  lay.qs_esz = qs_esz;
  lay.ds_esz = ds_esz;
  const bool vec = vec_ok(1, dim, {Qc, Dc});
  if (!scan_grid_fits(B)) return FMS_EUNSUPPORTED;
  return from_hip(launch_int8(ds_esz, lay, (int)dim, (int)Tq, B, args, partial, scores, 0.0f,
                              normalize != 0, vec, as_stream(stream)));
}

fms_status fms_launch_int8_pair_scan(int32_t* args, float* partial, const int8_t* qc,
                                     const void* qs, int32_t qs_dtype, const int8_t* dc,
                                     const void* ds, int32_t ds_dtype, const uint8_t* qmask,
                                     const uint8_t* dmask, int64_t dim, int64_t Tq, int64_t Td,
                                     float* score, int32_t normalize, void* stream) {
  return fms_launch_int8_paired_scan(args, partial, qc, qs, qs_dtype, dc, ds, ds_dtype, qmask,
                                     dmask, dim, Tq, Td, 1, score, normalize, stream);
}

fms_status fms_launch_int8_candidates_scan(int32_t* args, float* partial, const int8_t* Qc,
                                           const void* Qs, int32_t qs_dtype, const int8_t* Gc,
                                           const void* Gs, int32_t ds_dtype, const void* idx,
                                           int32_t idx_bytes, const uint8_t* qmask,
                                           const uint8_t* dmask, int64_t dim, int64_t Tq,
                                           int64_t B, int64_t Td, int64_t N, int64_t C,
                                           float* scores, float neg, int32_t normalize,
                                           void* stream) {
  const int qs_esz = scale_bytes(qs_dtype), ds_esz = scale_bytes(ds_dtype);
  if (qs_esz == 0 || ds_esz == 0) return FMS_EUNSUPPORTED;
  if (dim < 0 || Tq < 0 || Td < 0 || B < 0 || N < 0 || C < 0 || (normalize & ~1))
    return FMS_EINVAL;
  if (idx_bytes != 4 && idx_bytes != 8) return FMS_EINVAL;
  if (!seq_ok(Tq, dim, 4) || !seq_ok(Td, dim, 4)) return FMS_EUNSUPPORTED;
  if (C == 0 || B == 0 || (Tq == 0 && !scores)) return FMS_OK;
  if (!idx || (Tq > 0 && (!Qs || (dim > 0 && !Qc))) ||
      (N * Td > 0 && (!Gs || (dim > 0 && !Gc))))
    return FMS_EINVAL;
  LayCand lay;
  lay.Q = reinterpret_cast<const char*>(Qc);
  lay.G = reinterpret_cast<const char*>(Gc);
  lay.idx = idx;
  lay.idx64 = idx_bytes == 8;
  lay.qm = qmask;
  lay.dm = dmask;
  lay.Qs = static_cast<const char*>(Qs);
  lay.Gs = static_cast<const char*>(Gs);
  lay.qbytes = Tq * dim;
  lay.dbytes = Td * dim;
  lay.N = N;
  lay.C = C;
  lay.Tq = (int)Tq;
  lay.Td = (int)Td;
  lay.qs_esz = qs_esz;
  lay.ds_esz = ds_esz;
  const bool vec = vec_ok(1, dim, {Qc, Gc});
  const hipStream_t st = as_stream(stream);
  auto launch = [&](const auto& L) -> hipError_t {
    return launch_int8(ds_esz, L, (int)dim, (int)Tq, C * B, args, partial, scores, neg,
                       normalize != 0, vec, st);
  };
  RunsLauncher<OpI8> r32{&lay, (int)dim, (int)Tq, C * B, args, partial, scores, neg,
                         normalize != 0, vec, st};
  RunsLauncher<OpI8H> r16{&lay, (int)dim, (int)Tq, C * B, args, partial, scores, neg,
                          normalize != 0, vec, st};
  return ds_esz == 2 ? run_candidates(lay, C * B, st, Workspace::kPool, r16, launch)
                     : run_candidates(lay, C * B, st, Workspace::kPool, r32, launch);
}

int32_t fms_candidates_grouping(int32_t mode) {
  if (mode < 0 || mode > 3) return -1;
  const int32_t prev = t_grouping;
  t_grouping = mode;
  return prev;
}

uint64_t fms_debug_workspace_allocs(void) { return workspace_alloc_count(); }

int32_t fms_debug_inbatch_kernel(int32_t dtype, int64_t dim, int64_t Tq, int64_t Td, int64_t Bq,
                                 int64_t Bd, const void* Q, const void* D) {
  return inbatch_path(dtype, dim, Tq, Td, Bq, Bd, Q, D);
}

fms_status fms_int8_dots(int32_t* out, const int8_t* qc, const int8_t* dc, int64_t dim,
                         int64_t Tq, int64_t Td, void* stream) {
  if (dim < 0 || Tq < 0 || Td < 0) return FMS_EINVAL;
  if (!seq_ok(Tq, dim, 1) || !seq_ok(Td, dim, 1) || Tq * Td >= kMaxSeqBytes)
    return FMS_EUNSUPPORTED;
  if (Tq == 0 || Td == 0) return FMS_OK;
  if (!out || (dim > 0 && (!qc || !dc))) return FMS_EINVAL;
  return from_hip(int8_dots(out, qc, dc, (int)dim, (int)Tq, (int)Td, vec_ok(1, dim, {qc, dc}),
                            as_stream(stream)));
}

fms_status fms_length_normalize(float* scores, const uint8_t* qmask, int64_t Tq, int64_t nrows,
                                int64_t ncols, const void* idx, int32_t idx_bytes, int64_t N,
                                float neg, void* stream) {
  if (Tq < 0 || nrows < 0 || ncols < 0 || N < 0 || ncols > kMaxTokens) return FMS_EINVAL;
  if (idx && idx_bytes != 4 && idx_bytes != 8) return FMS_EINVAL;
  if (nrows == 0 || ncols == 0) return FMS_OK;
  if (!scores) return FMS_EINVAL;
  return from_hip(length_normalize(scores, qmask, Tq, nrows, ncols, idx, idx_bytes == 8, N, neg,
                                   as_stream(stream)));
}

fms_status fms_varlen_normalize(float* scores, const int32_t* cu_q, int64_t N, void* stream) {
  if (N < 0) return FMS_EINVAL;
  if (N == 0) return FMS_OK;
  if (!scores || !cu_q) return FMS_EINVAL;
  return from_hip(varlen_normalize(scores, cu_q, N, as_stream(stream)));
}

fms_status fms_topk(const float* scores, int64_t nrows, int64_t ncols, int64_t k, float* vals,
                    int32_t* idx, void* stream) {
  if (nrows < 0 || ncols < 0 || k < 0 || k > ncols) return FMS_EINVAL;
  // (one 1024-thread workgroup per row: the grid's work-items must fit 32 bits)
  if (ncols > INT32_MAX || nrows > kTopkMaxRows || k > kTopkMaxK) return FMS_EUNSUPPORTED;
  if (nrows == 0 || k == 0) return FMS_OK;
  if (!scores || !vals || !idx) return FMS_EINVAL;
  return from_hip(topk_rows(scores, nrows, ncols, (int)k, vals, idx, as_stream(stream)));
}

fms_status fms_debug_mfma_layout(float* out, int32_t dtype_or_int8, void* stream) {
  if (!out || dtype_or_int8 < 0 || dtype_or_int8 > 3) return FMS_EINVAL;
  return from_hip(mfma_layout_probe(out, dtype_or_int8, as_stream(stream)));
}

fms_status fms_debug_cross_lane(float* out, void* stream) {
  if (!out) return FMS_EINVAL;
  return from_hip(cross_lane_probe(out, as_stream(stream)));
}

fms_status fms_debug_read_bandwidth(const void* p, int64_t bytes, uint32_t* out, int32_t blocks,
                                    void* stream) {
  if (bytes < 0 || bytes % 16 != 0 || blocks <= 0 || !out || (bytes > 0 && !p) ||
      !aligned16(p))
    return FMS_EINVAL;
  return from_hip(read_bandwidth(p, bytes, out, blocks, as_stream(stream)));
}

fms_status fms_debug_gather_bandwidth(const void* g, int64_t gallery_bytes, int64_t doc_bytes,
                                      const int32_t* docs, int64_t ndocs, uint32_t* out,
                                      void* stream) {
  if (gallery_bytes < 0 || doc_bytes <= 0 || doc_bytes % 16 != 0 || ndocs < 0 || ndocs > 0x7fffffff ||
      (ndocs > 0 && (!docs || !out)) || (gallery_bytes > 0 && !g) || !aligned16(g))
    return FMS_EINVAL;
  if (ndocs == 0) return FMS_OK;
  return from_hip(gather_bandwidth(g, gallery_bytes, doc_bytes, docs, ndocs, out, as_stream(stream)));
}

// ---- backward on the argmax tape ----------------------------------------------

fms_status fms_paired_pullback(int32_t dtype, void* dQ, void* dD, const void* Q, const void* D,
                               const uint8_t* qmask, const int32_t* args, const void* Delta,
                               const void* inv_n, int64_t dim, int64_t Tq, int64_t Td, int64_t B,
                               void* stream) {
  const int esz = elem_bytes(dtype);
  if (esz == 0) return FMS_EUNSUPPORTED;
  if (dim < 0 || Tq < 0 || Td < 0 || B < 0) return FMS_EINVAL;
  if (!seq_ok(Tq, dim, esz) || !seq_ok(Td, dim, esz) || !pullback_ok(B, Tq, B * Td))
    return FMS_EUNSUPPORTED;
  if (dim == 0 || B == 0 || (Tq == 0 && Td == 0)) return FMS_OK;
  const int64_t npairs = (Tq > 0 && Td > 0) ? B : 0;
  if (!pullback_ptrs(B * Tq, Q, dQ, B * Td, D, dD, npairs, args, Delta)) return FMS_EINVAL;
  LayPaired lay;
  lay.Q = static_cast<const char*>(Q);
  lay.D = static_cast<const char*>(D);
  lay.qm = qmask;
  lay.dm = nullptr;
  lay.Qs = nullptr;
  lay.Ds = nullptr;
  lay.qbytes = Tq * dim * esz;
  lay.dbytes = Td * dim * esz;
  lay.Tq = (int)Tq;
  lay.Td = (int)Td;
  const PullbackArgs a =
      pullback_args(dtype, dQ, dD, Q, D, args, Delta, inv_n, npairs, 1, B * Tq, B * Td, Tq, dim);
  return from_hip(launch_pullback(lay, a, as_stream(stream)));
}

fms_status fms_pair_pullback(int32_t dtype, void* dq, void* dd, const void* q, const void* d,
                             const uint8_t* qmask, const int32_t* argmax_u, const void* delta,
                             int64_t dim, int64_t Tq, int64_t Td, void* stream) {
  return fms_paired_pullback(dtype, dq, dd, q, d, qmask, argmax_u, delta, nullptr, dim, Tq, Td, 1,
                             stream);
}

fms_status fms_inbatch_pullback(int32_t dtype, void* dQ, void* dD, const void* Q, const void* D,
                                const uint8_t* qmask, const int32_t* args, const void* Delta,
                                const void* inv_n, int64_t dim, int64_t Tq, int64_t Td,
                                int64_t Bq, int64_t Bd, void* stream) {
  const int esz = elem_bytes(dtype);
  if (esz == 0) return FMS_EUNSUPPORTED;
  if (dim < 0 || Tq < 0 || Td < 0 || Bq < 0 || Bd < 0) return FMS_EINVAL;
  if (!seq_ok(Tq, dim, esz) || !seq_ok(Td, dim, esz) || Bq > kMaxTokens || Bd > kMaxTokens ||
      !pullback_ok(Bq * Bd, Tq, Bd * Td))
    return FMS_EUNSUPPORTED;
  if (dim == 0 || (Bq * Tq == 0 && Bd * Td == 0)) return FMS_OK;
  const int64_t npairs = (Tq > 0 && Td > 0) ? Bq * Bd : 0;
  if (!pullback_ptrs(Bq * Tq, Q, dQ, Bd * Td, D, dD, npairs, args, Delta)) return FMS_EINVAL;
  LayInBatch lay;
  lay.Q = static_cast<const char*>(Q);
  lay.D = static_cast<const char*>(D);
  lay.qm = qmask;
  lay.dm = nullptr;
  lay.qbytes = Tq * dim * esz;
  lay.dbytes = Td * dim * esz;
  lay.Bd = Bd > 0 ? Bd : 1;
  lay.Tq = (int)Tq;
  lay.Td = (int)Td;
  const PullbackArgs a = pullback_args(dtype, dQ, dD, Q, D, args, Delta, inv_n, npairs, Bd, Bq * Tq,
                                       Bd * Td, Tq, dim);
  return from_hip(launch_pullback(lay, a, as_stream(stream)));
}

fms_status fms_candidates_pullback(int32_t dtype, void* dQ, void* dG, const void* Q,
                                   const void* gallery, const void* idx, int32_t idx_bytes,
                                   const uint8_t* qmask, const int32_t* args, const void* Delta,
                                   const void* inv_n, int64_t dim, int64_t Tq, int64_t B,
                                   int64_t Td, int64_t N, int64_t C, void* stream) {
  const int esz = elem_bytes(dtype);
  if (esz == 0) return FMS_EUNSUPPORTED;
  if (dim < 0 || Tq < 0 || Td < 0 || B < 0 || N < 0 || C < 0) return FMS_EINVAL;
  if (idx_bytes != 4 && idx_bytes != 8) return FMS_EINVAL;
  if (!seq_ok(Tq, dim, esz) || !seq_ok(Td, dim, esz) || !pullback_ok(C * B, Tq, N * Td))
    return FMS_EUNSUPPORTED;
  if (dim == 0 || (B * Tq == 0 && N * Td == 0)) return FMS_OK;
  const int64_t npairs = (Tq > 0 && Td > 0) ? C * B : 0;
  if (!pullback_ptrs(B * Tq, Q, dQ, N * Td, gallery, dG, npairs, args, Delta) || (npairs > 0 && !idx))
    return FMS_EINVAL;
  LayCand lay;
  lay.Q = static_cast<const char*>(Q);
  lay.G = static_cast<const char*>(gallery);
  lay.idx = idx;
  lay.idx64 = idx_bytes == 8;
  lay.qm = qmask;
  lay.dm = nullptr;
  lay.Qs = nullptr;
  lay.Gs = nullptr;
  lay.qbytes = Tq * dim * esz;
  lay.dbytes = Td * dim * esz;
  lay.N = N;
  lay.C = C > 0 ? C : 1;
  lay.Tq = (int)Tq;
  lay.Td = (int)Td;
  const PullbackArgs a = pullback_args(dtype, dQ, dG, Q, gallery, args, Delta, inv_n, npairs, C,
                                       B * Tq, N * Td, Tq, dim);
  return from_hip(launch_pullback(lay, a, as_stream(stream)));
}

fms_status fms_packed_pullback(int32_t dtype, void* dq, void* dP, const void* q,
                               const void* tokens, const int32_t* cu, const uint8_t* qmask,
                               const int32_t* args, const void* Delta, const void* inv_n,
                               int64_t dim, int64_t Tq, int64_t B, int64_t ntokens,
                               void* stream) {
  const int esz = elem_bytes(dtype);
  if (esz == 0) return FMS_EUNSUPPORTED;
  if (dim < 0 || Tq < 0 || B < 0 || ntokens < 0) return FMS_EINVAL;
  if (!seq_ok(Tq, dim, esz) || ntokens > kMaxTokens || !pullback_ok(B, Tq, ntokens))
    return FMS_EUNSUPPORTED;
  if (dim == 0 || (Tq == 0 && ntokens == 0)) return FMS_OK;
  const int64_t npairs = (Tq > 0 && ntokens > 0) ? B : 0;
  if (!pullback_ptrs(Tq, q, dq, ntokens, tokens, dP, npairs, args, Delta) || (npairs > 0 && !cu))
    return FMS_EINVAL;
  LayPacked lay;
  lay.q = static_cast<const char*>(q);
  lay.tok = static_cast<const char*>(tokens);
  lay.cu = cu;
  lay.qm = qmask;
  lay.ntok = ntokens;
  lay.rowbytes = dim * esz;
  lay.Tq = (int)Tq;
  const PullbackArgs a =
      pullback_args(dtype, dq, dP, q, tokens, args, Delta, inv_n, npairs, B, Tq, ntokens, Tq, dim);
  return from_hip(launch_pullback(lay, a, as_stream(stream)));
}

fms_status fms_varlen_pullback(int32_t dtype, void* dQ, void* dD, const void* Qtokens,
                               const void* Dtokens, const int32_t* cu_q, const int32_t* cu_d,
                               const int32_t* args, const void* Delta, const void* inv_n,
                               int64_t dim, int64_t max_q, int64_t N, int64_t nq_tokens,
                               int64_t nd_tokens, void* stream) {
  const int esz = elem_bytes(dtype);
  if (esz == 0) return FMS_EUNSUPPORTED;
  if (dim < 0 || max_q < 0 || N < 0 || nq_tokens < 0 || nd_tokens < 0) return FMS_EINVAL;
  if (!seq_ok(max_q, dim, esz) || nq_tokens > kMaxTokens || nd_tokens > kMaxTokens ||
      !pullback_ok(N, max_q, nd_tokens))
    return FMS_EUNSUPPORTED;
  if (dim == 0 || (nq_tokens == 0 && nd_tokens == 0)) return FMS_OK;
  const int64_t npairs = (max_q > 0 && nq_tokens > 0 && nd_tokens > 0) ? N : 0;
  if (!pullback_ptrs(nq_tokens, Qtokens, dQ, nd_tokens, Dtokens, dD, npairs, args, Delta) ||
      (npairs > 0 && (!cu_q || !cu_d)))
    return FMS_EINVAL;
  LayVarlen lay;
  lay.Qt = static_cast<const char*>(Qtokens);
  lay.Dt = static_cast<const char*>(Dtokens);
  lay.cu_q = cu_q;
  lay.cu_d = cu_d;
  lay.nq = nq_tokens;
  lay.nd = nd_tokens;
  lay.rowbytes = dim * esz;
  lay.max_q = (int)max_q;
  PullbackArgs a = pullback_args(dtype, dQ, dD, Qtokens, Dtokens, args, Delta, inv_n, npairs, 1,
                                 nq_tokens, nd_tokens, max_q, dim);
  a.zero_dq = true;  // query tokens outside every pair's range get no gather
  return from_hip(launch_pullback(lay, a, as_stream(stream)));
}

}  // extern "C"
