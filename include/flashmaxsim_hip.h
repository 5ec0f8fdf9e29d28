/*
 * flashmaxsim_hip.h -- C ABI of libflashmaxsim_hip.so, the MI355X (gfx950)
 * implementation of FlashMaxSim.jl's fused MaxSim forward.
 *
 * Each entry point replaces one method of the reference's device plugin
 * boundary (the `launch_*_scan!` / `inbatch_device_scan!` generic functions
 * that a weak-dependency extension specialises per backend; the CUDA
 * extension overrides them in ext/FlashMaxSimCUDAExt.jl:57-167).  A Julia
 * AMDGPU.jl extension binds them with `ccall`
 * (flashmaxsim.jl_amd/julia/ext/FlashMaxSimHIPExt.jl); the Python host
 * mirror in flashmaxsim.jl_amd/flashmaxsim binds them with ctypes.
 *
 * Conventions (all from the reference):
 *   - Column-major (Julia) layout.  A feature array of Julia size
 *     (dim, T, B) has element (k, t, b) at k + dim*(t + T*b).  Tokens are
 *     therefore contiguous `dim`-vectors.
 *   - Outputs first; the caller owns every buffer (zeros_like, ka.jl:28-30).
 *     The library keeps no pointer after the call returns.
 *   - Asynchronous: work is enqueued on `stream` (a hipStream_t; NULL = the
 *     legacy default stream).  No host synchronisation (ka.jl:3-5,10-15).
 *   - Argmax tapes are int32, 1-based, 0 = no valid document token.
 *     partial[t] is the per-query-token max (0 for a masked query token or
 *     an empty / fully masked document), exactly like the reference's
 *     `partial` buffer (kernels_forward.jl:55).
 *   - Masks are Bool bytes (0 = false, nonzero = true); NULL = all true
 *     (what true_mask allocates, colocation.jl:4-6).
 *   - Fused epilogue (an extension over the reference boundary, which leaves
 *     Sigma_t to a later `sum(partial; dims=1)`): when `scores` is non-NULL
 *     the kernel also writes scores[p] = Sigma_t partial[t,p] (fp32), and for
 *     the candidate layouts an invalid index writes `neg` there, fusing
 *     forward_layouts.jl:285-287.  `partial` and `args` may be NULL when not
 *     wanted.
 *   - `normalize` (0 or 1; extension) fuses the normalize=true epilogue into
 *     the same write: every valid pair's score is multiplied by the fp32
 *     1 / max(n, 1), n = its query's valid tokens (qmask count; the pair's
 *     query length for varlen) -- length_normalize / packed_finalize /
 *     varlen_finalize (normalize.jl:4-25, packed.jl:316-354); invalid
 *     candidates keep `neg` (normalize.jl:37-46).  Partials stay unscaled.
 *   - Zero-size inputs return FMS_OK without launching (ka.jl:12); an empty
 *     document (Td = 0 or cu[b+1] = cu[b]) still writes zeros.
 *   - Kernels never trap: an out-of-range candidate index yields tape 0 /
 *     partial 0 / score `neg`; a malformed device cu is clamped into the
 *     token range (the reference trusts device cu, packed.jl:65-67).
 *   - Scores accumulate in fp32 for every feature type (f16/bf16 products
 *     are exact in fp32; int8 dots accumulate exactly in int32).
 *
 * Reentrant: concurrent calls on different streams are independent.  The
 * only process-wide state is a per-device memory pool that the candidate
 * scans draw their stream-ordered workspace from (kept for the life of the
 * process) and the no-allocation entry point's per-device scratch array;
 * the grouping mode of fms_candidates_grouping is per host thread.
 */
#ifndef FLASHMAXSIM_HIP_H
#define FLASHMAXSIM_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t fms_status;
#define FMS_OK 0
#define FMS_EINVAL 1       /* bad shape, NULL required pointer, misaligned buffer */
#define FMS_EUNSUPPORTED 2 /* dtype / size the library does not implement */
#define FMS_EHIP 3         /* a HIP runtime call or kernel launch failed */
#define FMS_ESCRATCH 4     /* more workspace than fms_launch_candidates_scan_noalloc holds */

/* Feature element types.  BF16 has no reference counterpart on device (the
 * reference's dot_accum(BFloat16) = BFloat16); here it accumulates in fp32. */
#define FMS_F32 0
#define FMS_F16 1
#define FMS_BF16 2

/* Human-readable text for a status code (static storage). */
const char* fms_status_string(fms_status s);

/* 1 when the current HIP device is gfx950 (the only target built), else 0.
 * Plays the role of tensor_cores_active(backend, T) (src/ka.jl:71). */
int fms_arch_supported(void);

/* Library version string. */
const char* fms_version(void);

/*
 * Pair scan.  Replaces launch_pair_scan!(backend, argmax_u, partial, q, d,
 * qmask, dmask) (src/forward_pair.jl:118-132; CUDA override
 * ext/FlashMaxSimCUDAExt.jl:57-68).  q is (dim,Tq), d is (dim,Td);
 * argmax_u/partial are (Tq,).  score (nullable, length 1) receives Sigma_t,
 * replacing sum_length1 (src/ka.jl:49-53).
 */
fms_status fms_launch_pair_scan(int32_t dtype, int32_t* argmax_u, float* partial,
                                const void* q, const void* d,
                                const uint8_t* qmask, const uint8_t* dmask,
                                int64_t dim, int64_t Tq, int64_t Td,
                                float* score, int32_t normalize, void* stream);

/*
 * Paired-batch scan.  Replaces launch_paired_scan!(backend, args, partial, Q,
 * D, qmask, dmask) (src/forward_layouts.jl:126-143; CUDA override
 * ext/FlashMaxSimCUDAExt.jl:70-82).  Q (dim,Tq,B), D (dim,Td,B), qmask
 * (Tq,B), dmask (Td,B); args/partial (Tq,B); scores (B,) nullable.
 */
fms_status fms_launch_paired_scan(int32_t dtype, int32_t* args, float* partial,
                                  const void* Q, const void* D,
                                  const uint8_t* qmask, const uint8_t* dmask,
                                  int64_t dim, int64_t Tq, int64_t Td, int64_t B,
                                  float* scores, int32_t normalize, void* stream);

/*
 * Candidate scan.  Replaces launch_candidates_scan!(backend, args, partial,
 * Q, gallery, idx, qmask, dmask, N) (src/forward_layouts.jl:292-310; CUDA
 * override ext/FlashMaxSimCUDAExt.jl:112-124).  Q (dim,Tq,B), gallery
 * (dim,Td,N), idx (C,B) 1-based integers of idx_bytes = 4 or 8 bytes
 * (Int32 / Int64), qmask (Tq,B), dmask (Td,N); args/partial (Tq,C,B);
 * scores (C,B) nullable: Sigma_t for 1 <= idx <= N, else `neg`.
 */
fms_status fms_launch_candidates_scan(int32_t dtype, int32_t* args, float* partial,
                                      const void* Q, const void* gallery,
                                      const void* idx, int32_t idx_bytes,
                                      const uint8_t* qmask, const uint8_t* dmask,
                                      int64_t dim, int64_t Tq, int64_t B,
                                      int64_t Td, int64_t N, int64_t C,
                                      float* scores, float neg, int32_t normalize, void* stream);

/*
 * Document-order grouping of the candidate scans (float and INT8).  No
 * reference counterpart: a tuning switch of this library.  In document order
 * the pairs that share a gallery document are scored together and the
 * document is read from HBM once per group instead of once per pair; the
 * results are bit-identical to output order.  Grouping needs a workspace of
 * about 8*C*B + 4*N bytes, allocated stream-ordered from a library-owned
 * pool and released on the same stream.  mode: 0 = automatic (C*B >= 16384,
 * the sort's O(N) passes cheap next to the scan, and uniformly drawn
 * indices would repeat enough to save >= 30% of the document reads),
 * 1 = always, 2 = never, 3 = always and without the query-tile copy (the
 * 16-bit document-batch scan then reads the query tiles from Q, as it does
 * when the no-allocation scratch cannot hold that copy; a test switch).
 * The mode belongs to the calling host thread and applies to that thread's
 * later calls only.  Returns the thread's previous mode, or -1 for an
 * invalid mode.
 */
int32_t fms_candidates_grouping(int32_t mode);

/*
 * No reference counterpart: for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  fms_launch_candidates_scan with the same arguments and the
 * same kernels and results, except that the document-grouping workspace
 * comes from a static device array of FMS_NOALLOC_SCRATCH_BYTES per GPU
 * instead of the library pool.  The array is part of the library's code
 * object, so every GPU the library runs any kernel on holds it from then
 * until the process ends, whether or not this entry point is called (32 MiB
 * of 288 GB).  The call performs no hipMalloc / hipFree and calls no
 * allocating library routine.  A call whose grouping workspace would exceed
 * the array -- about 20 bytes per pair plus 4 per gallery document, some
 * 1.4M pairs over a 1M-document gallery -- scans in output order (identical
 * results, no workspace) when the thread's grouping mode is automatic, and
 * returns FMS_ESCRATCH and launches nothing when grouping was forced
 * (modes 1 and 3).  Every call on one GPU uses that GPU's single array: calls that
 * overlap on one GPU (concurrent streams) race and must be serialised by the
 * caller.  The array's previous contents never matter (the kernels clear what
 * they count).
 */
#define FMS_NOALLOC_SCRATCH_BYTES (32u << 20)
fms_status fms_launch_candidates_scan_noalloc(int32_t dtype, int32_t* args, float* partial,
                                              const void* Q, const void* gallery,
                                              const void* idx, int32_t idx_bytes,
                                              const uint8_t* qmask, const uint8_t* dmask,
                                              int64_t dim, int64_t Tq, int64_t B,
                                              int64_t Td, int64_t N, int64_t C,
                                              float* scores, float neg, int32_t normalize,
                                              void* stream);

/*
 * In-batch scan.  Replaces inbatch_device_scan!(backend, S, args, Q, D,
 * qmask, dmask) (src/forward_layouts.jl:202-225; CUDA override
 * ext/FlashMaxSimCUDAExt.jl:126-140).  Q (dim,Tq,Bq), D (dim,Td,Bd);
 * S (Bd,Bq) receives S[j,i] = MaxSim(Q_i, D_j) (overwritten, as the CUDA
 * override does with `S .= ...`); args (Tq,Bd,Bq) nullable.  Kernels: f16
 * and bf16 at dim 32, 64, 96 or 128 keep whole query tiles in registers;
 * other dims that are a multiple of 8 (16-bit) or of 4 (fp32) take the dim
 * a 128-byte slice at a time (both with 16-byte aligned Q and D); any other
 * shape scores each pair on its own.  Results agree to the float
 * tolerances either way (the same products, summed in another order).
 * With args NULL (S alone, as the reference's maxsim(..., InBatch()) keeps
 * it, src/dispatch.jl:121-125) the register-resident kernel keeps a running
 * maximum without the argmax: the same S, bit for bit.
 */
fms_status fms_inbatch_device_scan(int32_t dtype, float* S, int32_t* args,
                                   const void* Q, const void* D,
                                   const uint8_t* qmask, const uint8_t* dmask,
                                   int64_t dim, int64_t Tq, int64_t Bq,
                                   int64_t Td, int64_t Bd, int32_t normalize, void* stream);

/*
 * Packed scan: one query against B ragged documents.  Replaces
 * launch_packed_scan!(backend, args, partial, q, packed, cu, qmask)
 * (src/packed.jl:219-234; CUDA override ext/FlashMaxSimCUDAExt.jl:84-96).
 * q (dim,Tq), tokens (dim,ntokens), cu (B+1,) int32 1-based CSR (document b
 * is tokens[:, cu[b]:cu[b+1]-1]); qmask (Tq,) nullable; args/partial (Tq,B)
 * with document-local 1-based argmax; scores (B,) nullable.
 */
fms_status fms_launch_packed_scan(int32_t dtype, int32_t* args, float* partial,
                                  const void* q, const void* tokens, const int32_t* cu,
                                  const uint8_t* qmask,
                                  int64_t dim, int64_t Tq, int64_t B, int64_t ntokens,
                                  float* scores, int32_t normalize, void* stream);

/*
 * Per-row top-k of an fp32 score matrix (no reference counterpart: ranking is
 * the caller's job in the reference, README.md:132, e.g.
 * partialsortperm(scores[:, i], 1:k; rev = true)).  scores is (ncols, nrows)
 * column-major -- one column per query, as fms_launch_packed_multi_scan and
 * fms_inbatch_device_scan write them; vals (k, nrows) receives each column's
 * k largest scores in descending order, idx (k, nrows) their 1-based row
 * indices.  Order: Julia's isless reversed (NaN first, +0.0 before -0.0),
 * equal scores by smaller index -- a stable reverse sort.  1 <= k <= 1024 and
 * at most 2^22 - 1 columns of scores, else FMS_EUNSUPPORTED; k > ncols is
 * FMS_EINVAL (a BoundsError in partialsortperm).  One 1024-thread workgroup
 * per column; columns of 16,384 rows or more are first ranked in slices (a
 * workspace of 8 * k bytes per slice from the library pool) and the slices'
 * survivors ranked again.
 */
fms_status fms_topk(const float* scores, int64_t nrows, int64_t ncols, int64_t k, float* vals,
                    int32_t* idx, void* stream);

/*
 * Multi-query packed scan (no reference counterpart: the reference scores one
 * query per `maxsim(q, P::PackedSeq)` call, packed.jl:178-210).  Scores nq
 * queries against every document of one PackedSeq in a single pass, reading
 * each document once for a block of 32 queries instead of once per query.
 * Q (dim,Tq,nq), tokens (dim,ntokens), cu (B+1,) 1-based, qmask (Tq,nq)
 * nullable; scores (B,nq) receives S[b, i] = Sigma_t of query i against
 * document b (required); args (Tq,B,nq) nullable, tapes as in
 * fms_launch_packed_scan (NULL: the MFMA kernel keeps a running maximum
 * without the argmax, the same scores).  max_len >= every document's length (PackedSeq's
 * max_len).  f16/bf16 with dim = 128, Tq <= 32 and max_len <= 2048 run on
 * MFMA; other shapes make one packed scan per query.  Row i of the result
 * equals fms_launch_packed_scan of query i within the score tolerance (tapes
 * equal except at near-ties).  On the MFMA path a document longer than
 * max_len breaks that contract and is not scored: its scores are NaN and its
 * tapes 0 (never a score of a truncated document; the per-query path does
 * not read max_len).
 */
fms_status fms_launch_packed_multi_scan(int32_t dtype, int32_t* args, float* scores,
                                        const void* Q, const void* tokens, const int32_t* cu,
                                        const uint8_t* qmask, int64_t dim, int64_t Tq, int64_t nq,
                                        int64_t B, int64_t ntokens, int64_t max_len,
                                        int32_t normalize, void* stream);

/*
 * Varlen scan: N ragged (query, document) pairs.  Replaces
 * launch_varlen_scan!(backend, args, partial, Qp, Dp, cu_q, cu_d)
 * (src/packed.jl:298-314; CUDA override ext/FlashMaxSimCUDAExt.jl:98-110).
 * args/partial (max_q,N); rows t >= Tq_n are written 0.  scores (N,) nullable.
 */
fms_status fms_launch_varlen_scan(int32_t dtype, int32_t* args, float* partial,
                                  const void* Qtokens, const void* Dtokens,
                                  const int32_t* cu_q, const int32_t* cu_d,
                                  int64_t dim, int64_t max_q, int64_t N,
                                  int64_t nq_tokens, int64_t nd_tokens,
                                  float* scores, int32_t normalize, void* stream);

/*
 * Per-token symmetric INT8 quantisation, bit-exact with
 * quantize_int8_symmetric (src/quant.jl:42-49), computed in the feature type
 * T = dtype (FMS_F32 or FMS_F16): scale = max(max(absmax, T(1f-8)) / T(127),
 * floatmin(T)) with one correctly rounded division in T; code =
 * round-to-nearest-even(clamp(x / scale, -127, 127)) where x / scale is
 * itself rounded to T first.  X (dim,ntok) of T -> codes (dim,ntok) int8,
 * scales (ntok,) of T.  Replaces the reference's broadcast for device arrays.
 */
fms_status fms_int8_quantize(int32_t dtype, const void* X, int8_t* codes, void* scales,
                             int64_t dim, int64_t ntok, void* stream);

/*
 * INT8 pair scan.  Replaces launch_int8_pair_scan!(backend, args, partial,
 * qc, qs, dc, ds, qmask, dmask) (src/quant.jl:139-154; CUDA override
 * ext/FlashMaxSimCUDAExt.jl:142-153).  Dots accumulate exactly in int32;
 * s = (qs[t]*ds[u]) * Float32(acc) evaluated left to right in fp32
 * (src/quant.jl:113, src/kernels_int8.jl:17-25).  The scales keep the eltype
 * of the features they were quantised from: qs_dtype / ds_dtype is FMS_F32
 * or FMS_F16 (widened exactly to fp32; dot_accum(Float16) = Float32), so
 * partial is fp32 either way.
 */
fms_status fms_launch_int8_pair_scan(int32_t* args, float* partial,
                                     const int8_t* qc, const void* qs, int32_t qs_dtype,
                                     const int8_t* dc, const void* ds, int32_t ds_dtype,
                                     const uint8_t* qmask, const uint8_t* dmask,
                                     int64_t dim, int64_t Tq, int64_t Td,
                                     float* score, int32_t normalize, void* stream);

/*
 * INT8 paired scan.  Replaces launch_int8_paired_scan!(backend, args,
 * partial, Qc, Qs, Dc, Ds, qmask, dmask) (src/quant.jl:199-217; CUDA
 * override ext/FlashMaxSimCUDAExt.jl:155-167).  Scale types as for the pair
 * scan.
 */
fms_status fms_launch_int8_paired_scan(int32_t* args, float* partial,
                                       const int8_t* Qc, const void* Qs, int32_t qs_dtype,
                                       const int8_t* Dc, const void* Ds, int32_t ds_dtype,
                                       const uint8_t* qmask, const uint8_t* dmask,
                                       int64_t dim, int64_t Tq, int64_t Td, int64_t B,
                                       float* scores, int32_t normalize, void* stream);

/*
 * INT8 candidate scan.  No reference counterpart: Int8Index has only pair
 * and paired methods (src/dispatch.jl:247-296).  Composes the INT8 pair scan
 * per (c,b) with the candidate conventions of launch_candidates_scan!
 * (src/forward_layouts.jl:292-310): idx (C,B), invalid -> tape 0 / `neg`.
 */
fms_status fms_launch_int8_candidates_scan(int32_t* args, float* partial,
                                           const int8_t* Qc, const void* Qs, int32_t qs_dtype,
                                           const int8_t* Gc, const void* Gs, int32_t ds_dtype,
                                           const void* idx, int32_t idx_bytes,
                                           const uint8_t* qmask, const uint8_t* dmask,
                                           int64_t dim, int64_t Tq, int64_t B,
                                           int64_t Td, int64_t N, int64_t C,
                                           float* scores, float neg, int32_t normalize,
                                           void* stream);

/*
 * Test-only: raw int32 dots out (Td,Tq) with out[u + Td*t] = <qc_t, dc_u>,
 * computed by the same int8 MFMA path as the scans.  No reference
 * counterpart (the reference never exposes dots); used for the bit-exact
 * check of the int32 accumulation (quant.jl:109-112).
 */
fms_status fms_int8_dots(int32_t* out, const int8_t* qc, const int8_t* dc,
                         int64_t dim, int64_t Tq, int64_t Td, void* stream);

/*
 * Query-length normalisation epilogues (src/normalize.jl:4-46,
 * src/forward_pair.jl:153-173, src/packed.jl:316-354).  scores (nrows,ncols)
 * column-major, scaled in place by inv = 1/max(count, 1) (fp32, multiply):
 *   fms_length_normalize: count = count(qmask[:,col]) per column (qmask
 *     (Tq,ncols); NULL = Tq); if idx is non-NULL (candidate layout,
 *     idx (nrows,ncols)), entries with idx outside 1..N are set to `neg`.
 *   fms_varlen_normalize: count = cu_q[n+1]-cu_q[n] per entry (N entries).
 */
fms_status fms_length_normalize(float* scores, const uint8_t* qmask, int64_t Tq,
                                int64_t nrows, int64_t ncols,
                                const void* idx, int32_t idx_bytes, int64_t N, float neg,
                                void* stream);
fms_status fms_varlen_normalize(float* scores, const int32_t* cu_q, int64_t N, void* stream);

/*
 * Backward on the argmax tape (paper Eqs. 2-3).  For every pair p and query
 * token t with qmask[t] and a tape entry 1 <= u = args[t,p] <= Td(p):
 *     dQ[:, t of p's query]     += delta_p * D[:, u of p's document]
 *     dD[:, u of p's document]  += delta_p * Q[:, t of p's query]
 * with delta_p = Delta[p] * inv_n[query of p] (inv_n NULL = all ones).
 * Replaces the device method `*_apply_pullback!` of each layout, the
 * InvGrid strategy (gather for dQ, destination CSR for dD).  Differences
 * from the reference boundary:
 *   - dQ and dD are OUTPUTS, overwritten in full (rows no source reaches are
 *     written 0), so the caller need not zero them (the reference allocates
 *     them with zeros_like and accumulates into them).
 *   - Sums run in fp32 for every feature type and are rounded once into the
 *     feature type (the reference accumulates in T).
 *   - Delta and inv_n are in the feature type (Julia's Vector{T}).
 *   - dQ sums a query token's pairs in pair order (deterministic).  dD sums
 *     a destination row's sources in the order a device CSR fill gave them,
 *     so its last bits may differ between runs, as the reference's device
 *     CSR's do (src/invgrid.jl:10-14).
 * Workspace (about 4*npairs*Tq + 4*ndest + 4*npairs bytes) comes from the
 * library's stream-ordered pool.  Masked or out-of-range tape entries and
 * pairs with delta 0 contribute nothing (src/backward_pair.jl:21-29).
 */

/* pair_apply_pullback!(mode, backend, dq, dd, q, d, qmask, argmax_u, δ, dim,
 * Tq, Td) (src/backward_pair.jl:73-87).  q (dim,Tq), d (dim,Td), delta (1,). */
fms_status fms_pair_pullback(int32_t dtype, void* dq, void* dd, const void* q, const void* d,
                             const uint8_t* qmask, const int32_t* argmax_u, const void* delta,
                             int64_t dim, int64_t Tq, int64_t Td, void* stream);

/* paired_apply_pullback!(mode, backend, dQ, dD, Q, D, qmask, args, Δ, inv_n,
 * dim, Tq, B, Td) (src/backward_layouts.jl:45-60).  Q (dim,Tq,B), D
 * (dim,Td,B), args (Tq,B), Delta (B,), inv_n (B,) nullable. */
fms_status fms_paired_pullback(int32_t dtype, void* dQ, void* dD, const void* Q, const void* D,
                               const uint8_t* qmask, const int32_t* args, const void* Delta,
                               const void* inv_n, int64_t dim, int64_t Tq, int64_t Td, int64_t B,
                               void* stream);

/* inbatch_apply_pullback!(mode, backend, dQ, dD, Q, D, qmask, args, Δ, inv_n,
 * dim, Tq, Bq, Td, Bd) (src/backward_layouts.jl:113-127).  Q (dim,Tq,Bq), D
 * (dim,Td,Bd), args (Tq,Bd,Bq), Delta (Bd,Bq) (pair (j,i) = query i against
 * document j), inv_n (Bq,) nullable. */
fms_status fms_inbatch_pullback(int32_t dtype, void* dQ, void* dD, const void* Q, const void* D,
                                const uint8_t* qmask, const int32_t* args, const void* Delta,
                                const void* inv_n, int64_t dim, int64_t Tq, int64_t Td,
                                int64_t Bq, int64_t Bd, void* stream);

/* candidates_apply_pullback!(mode, backend, dQ, dG, Q, gallery, idx, qmask,
 * args, Δ, inv_n, dim, Tq, B, Td, C, N) (src/backward_layouts.jl:187-202).
 * Q (dim,Tq,B), gallery (dim,Td,N), idx (C,B) of idx_bytes = 4 or 8,
 * args (Tq,C,B), Delta (C,B), inv_n (B,) nullable; dG (dim,Td,N).  An index
 * outside 1..N contributes nothing; a document chosen several times sums. */
fms_status fms_candidates_pullback(int32_t dtype, void* dQ, void* dG, const void* Q,
                                   const void* gallery, const void* idx, int32_t idx_bytes,
                                   const uint8_t* qmask, const int32_t* args, const void* Delta,
                                   const void* inv_n, int64_t dim, int64_t Tq, int64_t B,
                                   int64_t Td, int64_t N, int64_t C, void* stream);

/* packed_apply_pullback!(mode, backend, Δ, q, P, qmask, args, inv_n)
 * (src/packed.jl:384-417).  q (dim,Tq), tokens (dim,ntokens) with device cu
 * (B+1,) 1-based, args (Tq,B), Delta (B,), inv_n (1,) nullable; dP
 * (dim,ntokens).  cu is clamped into the token range as in the forward. */
fms_status fms_packed_pullback(int32_t dtype, void* dq, void* dP, const void* q,
                               const void* tokens, const int32_t* cu, const uint8_t* qmask,
                               const int32_t* args, const void* Delta, const void* inv_n,
                               int64_t dim, int64_t Tq, int64_t B, int64_t ntokens,
                               void* stream);

/* varlen_apply_pullback!(mode, backend, Δ, Q, D, args, inv_n)
 * (src/packed.jl:449-485).  Query tokens (dim,nq_tokens) with cu_q (N+1,),
 * document tokens (dim,nd_tokens) with cu_d (N+1,), args (max_q,N) (rows
 * past a query's length unread), Delta (N,), inv_n (N,) nullable. */
fms_status fms_varlen_pullback(int32_t dtype, void* dQ, void* dD, const void* Qtokens,
                               const void* Dtokens, const int32_t* cu_q, const int32_t* cu_d,
                               const int32_t* args, const void* Delta, const void* inv_n,
                               int64_t dim, int64_t max_q, int64_t N, int64_t nq_tokens,
                               int64_t nd_tokens, void* stream);

/*
 * Test-only: MFMA accumulator layout probe (no reference counterpart).  Runs
 * one 32x32 MFMA of the given feature type (FMS_F32 / FMS_F16 / FMS_BF16, or
 * 3 = int8) twice -- A[i][0] = i+1, B[0][j] = 1, then A[i][0] = 1,
 * B[0][j] = j+1 -- and writes out[(pass*64 + lane)*16 + reg] (2048 floats),
 * so a test can confirm the (lane, register) -> (row, column) map the scans
 * rely on.
 */
fms_status fms_debug_mfma_layout(float* out, int32_t dtype_or_int8, void* stream);

/*
 * Test-only: cross-lane helper probe (no reference counterpart).  One wave
 * writes 256 floats: out[l] = the lane its l ^ 32 exchange reads, out[64+l]
 * = the sum of the lane ids 0..31 (in every lane), out[128+l] / out[192+l] =
 * the (token, max) kept by the half merge when lane l holds max l % 7 and
 * token l + 1 -- what the scans' tile close relies on.
 */
fms_status fms_debug_cross_lane(float* out, void* stream);

/*
 * Test-only: the number of workspace allocations the library has requested
 * from its stream-ordered pool in this process (no reference counterpart).
 * Lets a test show that fms_launch_candidates_scan_noalloc takes none.
 */
uint64_t fms_debug_workspace_allocs(void);

/*
 * Test-only: which kernel fms_inbatch_device_scan runs for these arguments
 * (no reference counterpart): 1 the register-resident MFMA kernel (16-bit
 * features, dim 32, 64, 96 or 128), 2 the split-K MFMA kernel (fp32, and
 * 16-bit dims whose rows are whole 16-byte units), 0 the per-pair scan.
 */
int32_t fms_debug_inbatch_kernel(int32_t dtype, int64_t dim, int64_t Tq, int64_t Td, int64_t Bq,
                                 int64_t Bd, const void* Q, const void* D);

/*
 * Test-only: streaming read of `bytes` (multiple of 16, 16-byte aligned)
 * with `blocks` workgroups of 256 threads; out receives blocks*256 words.
 * No reference counterpart: it measures the HBM read ceiling reported
 * beside the scans' roofline and calibrates the FETCH_SIZE counter.
 */
fms_status fms_debug_read_bandwidth(const void* p, int64_t bytes, uint32_t* out, int32_t blocks,
                                    void* stream);

/*
 * Test-only: gathered read of whole documents, the candidate scans' access
 * pattern.  One 256-thread workgroup per entry of docs[0..ndocs) reads the
 * doc_bytes (multiple of 16) at g + docs[i] * doc_bytes with 16-byte
 * nontemporal loads; entries whose document does not lie inside the
 * gallery's gallery_bytes are skipped.  out receives ndocs*256 words.  No
 * reference counterpart: it measures the read ceiling of a gathered-document
 * stream, reported beside the candidate scans' roofline.
 */
fms_status fms_debug_gather_bandwidth(const void* g, int64_t gallery_bytes, int64_t doc_bytes,
                                      const int32_t* docs, int64_t ndocs, uint32_t* out,
                                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLASHMAXSIM_HIP_H */
