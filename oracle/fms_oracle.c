/*
 * fms_oracle.c -- CPU restatement of FlashMaxSim.jl's forward semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity oracle and the timed
 * CPU baseline ("port" of the reference's CPU Array path).  It is never
 * linked into, loaded by, or called from the product library
 * (libflashmaxsim_hip.so) or its Python host mirror.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it.
 *
 * Every function cites the reference file:line it restates (paths are
 * relative to the FlashMaxSim.jl source tree).  Arrays follow the
 * reference's Julia column-major layout: feature element (k, t, b) of an
 * array shaped (dim, T, B) lives at  k + dim * (t + T * b)  (0-based).
 * Argmax tapes are int32, 1-based, 0 = "no valid document token".
 *
 * Arithmetic conventions (all from the reference):
 *   - Float16 / BFloat16 features are widened exactly to fp32; products and
 *     sums run in fp32 (dot_accum, src/kernels_forward.jl:16-21).  The
 *     reference itself accumulates BFloat16 in BFloat16 (dot_accum(T)=T);
 *     this oracle pins the fp32-accumulate mathematics instead.
 *   - The per-tile GEMM (src/forward_pair.jl:76, BLAS mul!) is restated as
 *     an in-order k loop, which is exactly the KA token kernels' order
 *     (src/kernels_forward.jl:45-48).  BLAS's blocked order is not pinned.
 *   - Running max per query token: first valid document token wins, then
 *     strictly greater replaces (src/forward_pair.jl:82-85).
 *   - Sigma_t in fp32, ascending t (src/forward_pair.jl:90-93).
 *
 * Build: see oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
#include <float.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { FMSO_F32 = 0, FMSO_F16 = 1, FMSO_BF16 = 2, FMSO_F64 = 3 };

/* reference: src/forward_pair.jl:12 (DOC_TILE = 64) */
#define FMSO_DOC_TILE 64

/* ---- exact widening of stored features ---------------------------------- */

/* IEEE binary16 -> binary32, exact (every half is representable). */
static float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: renormalise */
            int e = -1;
            do { man <<= 1; ++e; } while ((man & 0x400u) == 0);
            man &= 0x3ffu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static float bf16_to_float(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static int elem_size(int dtype) {
    switch (dtype) {
    case FMSO_F32: return 4;
    case FMSO_F16: return 2;
    case FMSO_BF16: return 2;
    case FMSO_F64: return 8;
    default: return 0;
    }
}

/* Widen n consecutive stored elements to fp32 (exact for f16/bf16/f32). */
static void widen_f32(int dtype, const void* src, int64_t n, float* dst) {
    int64_t i;
    switch (dtype) {
    case FMSO_F32: memcpy(dst, src, (size_t)n * 4); break;
    case FMSO_F16: {
        const uint16_t* s = (const uint16_t*)src;
        for (i = 0; i < n; ++i) dst[i] = half_to_float(s[i]);
        break;
    }
    case FMSO_BF16: {
        const uint16_t* s = (const uint16_t*)src;
        for (i = 0; i < n; ++i) dst[i] = bf16_to_float(s[i]);
        break;
    }
    default: break;
    }
}

static double load_f64(int dtype, const void* base, int64_t i) {
    switch (dtype) {
    case FMSO_F32: return (double)((const float*)base)[i];
    case FMSO_F16: return (double)half_to_float(((const uint16_t*)base)[i]);
    case FMSO_BF16: return (double)bf16_to_float(((const uint16_t*)base)[i]);
    case FMSO_F64: return ((const double*)base)[i];
    default: return 0.0;
    }
}

static const char* advance(const void* base, int64_t elems, int dtype) {
    return (const char*)base + elems * elem_size(dtype);
}

/* ---- pair core ----------------------------------------------------------- */

/*
 * Restates pair_forward_host! (src/forward_pair.jl:59-95) for fp32
 * accumulation.  q is (dim, Tq), d is (dim, Td), masks are Bool bytes
 * (NULL = all true, as true_mask, src/colocation.jl:4-6).  Writes argmax_u
 * (Tq) and mx (Tq); mx is the per-token partial (0 for a masked token or an
 * empty document, like partial[t] in src/kernels_forward.jl:55).  Returns
 * Sigma_t over qmask[t] && argmax_u[t] > 0, accumulated in ascending t.
 *
 * qf/tile are caller scratch: qf holds dim*Tq fp32, tile holds
 * dim*DOC_TILE + DOC_TILE*Tq fp32.
 */
static float pair_core(int dtype, const void* q, const void* d,
                       const uint8_t* qmask, const uint8_t* dmask,
                       int64_t dim, int64_t Tq, int64_t Td,
                       int32_t* argmax_u, float* mx, float* qf, float* tile) {
    int64_t t, u, uu, k;
    float* dT = tile;                         /* DOC_TILE x dim, token-fastest */
    float* St = tile + dim * FMSO_DOC_TILE;   /* DOC_TILE x Tq, fp32 */
    for (t = 0; t < Tq; ++t) { argmax_u[t] = 0; mx[t] = 0.0f; } /* :68-69 */
    widen_f32(dtype, q, dim * Tq, qf);                            /* :70 */
    for (u = 0; u < Td; u += FMSO_DOC_TILE) {                     /* :72-74 */
        int64_t w = (Td - u < FMSO_DOC_TILE) ? (Td - u) : FMSO_DOC_TILE;
        /* widen the tile (:75), stored transposed so the GEMM below
         * vectorises over document tokens */
        for (uu = 0; uu < w; ++uu) {
            const void* src = advance(d, (u + uu) * dim, dtype);
            if (dtype == FMSO_F32) {
                const float* s = (const float*)src;
                for (k = 0; k < dim; ++k) dT[k * FMSO_DOC_TILE + uu] = s[k];
            } else if (dtype == FMSO_F16) {
                const uint16_t* s = (const uint16_t*)src;
                for (k = 0; k < dim; ++k) dT[k * FMSO_DOC_TILE + uu] = half_to_float(s[k]);
            } else {
                const uint16_t* s = (const uint16_t*)src;
                for (k = 0; k < dim; ++k) dT[k * FMSO_DOC_TILE + uu] = bf16_to_float(s[k]);
            }
        }
        /* Stile = dA' * qA  (:76).  Each cell accumulates k = 1..dim in
         * order (the KA token kernel's order, kernels_forward.jl:45-48);
         * the loop nest only vectorises across document tokens. */
        for (t = 0; t < Tq; ++t) {
            const float* qt = qf + t * dim;
            float* st = St + FMSO_DOC_TILE * t;
            for (uu = 0; uu < w; ++uu) st[uu] = 0.0f;
            for (k = 0; k < dim; ++k) {
                const float qk = qt[k];
                const float* dk = dT + k * FMSO_DOC_TILE;
                for (uu = 0; uu < w; ++uu) st[uu] += dk[uu] * qk;
            }
        }
        for (t = 0; t < Tq; ++t) {                                 /* :77-87 */
            if (qmask && !qmask[t]) continue;
            for (uu = 0; uu < w; ++uu) {
                if (dmask && !dmask[u + uu]) continue;
                float s = St[uu + FMSO_DOC_TILE * t];
                if (argmax_u[t] == 0 || s > mx[t]) {
                    mx[t] = s;
                    argmax_u[t] = (int32_t)(u + uu + 1);
                }
            }
        }
    }
    float score = 0.0f;                                            /* :90-93 */
    for (t = 0; t < Tq; ++t) {
        if ((!qmask || qmask[t]) && argmax_u[t] > 0) score += mx[t];
        else mx[t] = 0.0f;
    }
    return score;
}

typedef struct { float* qf; float* tile; float* mx; int32_t* arg; } scratch_t;

static int scratch_alloc(scratch_t* s, int64_t dim, int64_t Tq) {
    int64_t tq = Tq > 0 ? Tq : 1;
    int64_t dm = dim > 0 ? dim : 1;
    s->qf = (float*)malloc(sizeof(float) * (size_t)(dm * tq));
    s->tile = (float*)malloc(sizeof(float) * (size_t)(dm * FMSO_DOC_TILE + FMSO_DOC_TILE * tq));
    s->mx = (float*)malloc(sizeof(float) * (size_t)tq);
    s->arg = (int32_t*)malloc(sizeof(int32_t) * (size_t)tq);
    return s->qf && s->tile && s->mx && s->arg;
}

static void scratch_free(scratch_t* s) {
    free(s->qf); free(s->tile); free(s->mx); free(s->arg);
}

static void set_threads(int nthreads) {
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
}

/* ---- public oracle entry points ------------------------------------------ */

int fmso_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* pair_forward_host (src/forward_pair.jl:45-51).  partial may be NULL. */
float fmso_pair_forward(int dtype, const void* q, const void* d,
                        const uint8_t* qmask, const uint8_t* dmask,
                        int64_t dim, int64_t Tq, int64_t Td,
                        int32_t* argmax_u, float* partial) {
    scratch_t s;
    if (!scratch_alloc(&s, dim, Tq)) return NAN;
    float score = pair_core(dtype, q, d, qmask, dmask, dim, Tq, Td, s.arg, s.mx, s.qf, s.tile);
    if (argmax_u) memcpy(argmax_u, s.arg, sizeof(int32_t) * (size_t)Tq);
    if (partial) memcpy(partial, s.mx, sizeof(float) * (size_t)Tq);
    scratch_free(&s);
    return score;
}

/*
 * paired_forward(::CPU) (src/forward_layouts.jl:86-103): scores (B,),
 * args (Tq,B), partial (Tq,B) (nullable).
 */
void fmso_paired_forward(int dtype, const void* Q, const void* D,
                         const uint8_t* qmask, const uint8_t* dmask,
                         int64_t dim, int64_t Tq, int64_t Td, int64_t B,
                         float* scores, int32_t* args, float* partial, int nthreads) {
    set_threads(nthreads);
    #pragma omp parallel
    {
        scratch_t s;
        int ok = scratch_alloc(&s, dim, Tq);
        int64_t b;
        #pragma omp for schedule(dynamic, 4)
        for (b = 0; b < B; ++b) {
            if (!ok) continue;
            float sc = pair_core(dtype, advance(Q, b * dim * Tq, dtype),
                                 advance(D, b * dim * Td, dtype),
                                 qmask ? qmask + b * Tq : NULL,
                                 dmask ? dmask + b * Td : NULL,
                                 dim, Tq, Td, s.arg, s.mx, s.qf, s.tile);
            scores[b] = sc;
            if (args) memcpy(args + b * Tq, s.arg, sizeof(int32_t) * (size_t)Tq);
            if (partial) memcpy(partial + b * Tq, s.mx, sizeof(float) * (size_t)Tq);
        }
        scratch_free(&s);
    }
}

/*
 * candidates_forward(::CPU) (src/forward_layouts.jl:239-261): S (C,B) starts
 * filled with neg, args (Tq,C,B) zeros; only 1 <= idx <= N is scored.
 * idxs are int64, 1-based, column-major (C,B).  pair_subset (nullable) limits
 * the work to the listed linear pair ids c + C*b (used for a bounded CPU
 * baseline sample); outputs of other pairs are left untouched.
 */
void fmso_candidates_forward(int dtype, const void* Q, const void* G, const int64_t* idxs,
                             const uint8_t* qmask, const uint8_t* dmask,
                             int64_t dim, int64_t Tq, int64_t B, int64_t Td, int64_t N,
                             int64_t C, float neg, float* S, int32_t* args, float* partial,
                             const int64_t* pair_subset, int64_t n_subset, int nthreads) {
    int64_t npairs = pair_subset ? n_subset : C * B;
    set_threads(nthreads);
    #pragma omp parallel
    {
        scratch_t s;
        int ok = scratch_alloc(&s, dim, Tq);
        int64_t i;
        #pragma omp for schedule(dynamic, 16)
        for (i = 0; i < npairs; ++i) {
            if (!ok) continue;
            int64_t p = pair_subset ? pair_subset[i] : i;
            int64_t b = p / C;
            int64_t j = idxs[p];
            if (!(1 <= j && j <= N)) {                      /* :253 */
                S[p] = neg;
                if (args) memset(args + p * Tq, 0, sizeof(int32_t) * (size_t)Tq);
                if (partial) memset(partial + p * Tq, 0, sizeof(float) * (size_t)Tq);
                continue;
            }
            float sc = pair_core(dtype, advance(Q, b * dim * Tq, dtype),
                                 advance(G, (j - 1) * dim * Td, dtype),
                                 qmask ? qmask + b * Tq : NULL,
                                 dmask ? dmask + (j - 1) * Td : NULL,
                                 dim, Tq, Td, s.arg, s.mx, s.qf, s.tile);
            S[p] = sc;
            if (args) memcpy(args + p * Tq, s.arg, sizeof(int32_t) * (size_t)Tq);
            if (partial) memcpy(partial + p * Tq, s.mx, sizeof(float) * (size_t)Tq);
        }
        scratch_free(&s);
    }
}

/*
 * inbatch_forward(::CPU) (src/forward_layouts.jl:155-179 with
 * inbatch_accumulate_host! :49-74): S (Bd,Bq), args (Tq,Bd,Bq).  The GEMM
 * chunking (INBATCH_TILE_BYTES) only changes memory traffic, not per-cell
 * arithmetic: each cell is the pair scan of (Q_i, D_j), with S[j,i]
 * accumulated over ascending t (the t-innermost loop of :56-72).
 */
void fmso_inbatch_forward(int dtype, const void* Q, const void* D,
                          const uint8_t* qmask, const uint8_t* dmask,
                          int64_t dim, int64_t Tq, int64_t Bq, int64_t Td, int64_t Bd,
                          float* S, int32_t* args, int nthreads) {
    set_threads(nthreads);
    #pragma omp parallel
    {
        scratch_t s;
        int ok = scratch_alloc(&s, dim, Tq);
        int64_t p;
        #pragma omp for schedule(dynamic, 8)
        for (p = 0; p < Bq * Bd; ++p) {
            if (!ok) continue;
            int64_t j = p % Bd, i = p / Bd;
            float sc = pair_core(dtype, advance(Q, i * dim * Tq, dtype),
                                 advance(D, j * dim * Td, dtype),
                                 qmask ? qmask + i * Tq : NULL,
                                 dmask ? dmask + j * Td : NULL,
                                 dim, Tq, Td, s.arg, s.mx, s.qf, s.tile);
            S[p] = sc;
            if (args) memcpy(args + p * Tq, s.arg, sizeof(int32_t) * (size_t)Tq);
        }
        scratch_free(&s);
    }
}

/* inbatch_doc_chunk (src/forward_layouts.jl:11-18), integer only. */
int64_t fmso_inbatch_doc_chunk(int64_t elsize, int64_t Td, int64_t Tq, int64_t Bq, int64_t Bd) {
    const int64_t tile_bytes = 64LL * 1024 * 1024;
    if (Bd <= 0) return 1;
    int64_t denom = elsize * (Td > 1 ? Td : 1) * (Tq > 1 ? Tq : 1) * (Bq > 1 ? Bq : 1);
    int64_t c = tile_bytes / denom;
    if (c < 1) c = 1;
    return Bd < c ? Bd : c;
}

/*
 * packed_forward_host (src/packed.jl:153-176): one query (dim,Tq) against
 * B ragged documents tokens[:, cu[b]:cu[b+1]-1] (cu 1-based int32, B+1).
 * No document mask; argmax is local to the document.
 */
void fmso_packed_forward(int dtype, const void* q, const void* tokens, const int32_t* cu,
                         const uint8_t* qmask, int64_t dim, int64_t Tq, int64_t B,
                         float* scores, int32_t* args, float* partial,
                         const int64_t* doc_subset, int64_t n_subset, int nthreads) {
    int64_t n = doc_subset ? n_subset : B;
    set_threads(nthreads);
    #pragma omp parallel
    {
        scratch_t s;
        int ok = scratch_alloc(&s, dim, Tq);
        int64_t i;
        #pragma omp for schedule(dynamic, 4)
        for (i = 0; i < n; ++i) {
            if (!ok) continue;
            int64_t b = doc_subset ? doc_subset[i] : i;
            int64_t a = (int64_t)cu[b] - 1;
            int64_t Td = (int64_t)cu[b + 1] - (int64_t)cu[b];
            if (Td < 0) Td = 0;                              /* :169 */
            float sc = pair_core(dtype, q, advance(tokens, a * dim, dtype), qmask, NULL,
                                 dim, Tq, Td, s.arg, s.mx, s.qf, s.tile);
            scores[b] = sc;
            if (args) memcpy(args + b * Tq, s.arg, sizeof(int32_t) * (size_t)Tq);
            if (partial) memcpy(partial + b * Tq, s.mx, sizeof(float) * (size_t)Tq);
        }
        scratch_free(&s);
    }
}

/*
 * varlen_forward_host (src/packed.jl:236-260): N pairs (Q_n, D_n) from two
 * CSR packings.  args/partial are (max_q, N); rows t >= Tq_n stay 0.
 */
void fmso_varlen_forward(int dtype, const void* Qt, const void* Dt,
                         const int32_t* cu_q, const int32_t* cu_d,
                         int64_t dim, int64_t N, int64_t max_q,
                         float* scores, int32_t* args, float* partial, int nthreads) {
    set_threads(nthreads);
    #pragma omp parallel
    {
        scratch_t s;
        int ok = scratch_alloc(&s, dim, max_q);
        int64_t nn;
        #pragma omp for schedule(dynamic, 4)
        for (nn = 0; nn < N; ++nn) {
            if (!ok) continue;
            int64_t qa = (int64_t)cu_q[nn] - 1, da = (int64_t)cu_d[nn] - 1;
            int64_t tq = (int64_t)cu_q[nn + 1] - (int64_t)cu_q[nn];
            int64_t td = (int64_t)cu_d[nn + 1] - (int64_t)cu_d[nn];
            if (td < 0) td = 0;
            if (tq < 0) tq = 0;
            float sc = pair_core(dtype, advance(Qt, qa * dim, dtype), advance(Dt, da * dim, dtype),
                                 NULL, NULL, dim, tq, td, s.arg, s.mx, s.qf, s.tile);
            scores[nn] = sc;
            if (args) {
                memset(args + nn * max_q, 0, sizeof(int32_t) * (size_t)max_q);
                memcpy(args + nn * max_q, s.arg, sizeof(int32_t) * (size_t)tq);
            }
            if (partial) {
                memset(partial + nn * max_q, 0, sizeof(float) * (size_t)max_q);
                memcpy(partial + nn * max_q, s.mx, sizeof(float) * (size_t)tq);
            }
        }
        scratch_free(&s);
    }
}

/* ---- INT8 -------------------------------------------------------------------- */

/*
 * quantize_int8_symmetric for Float32 (src/quant.jl:21-49): per token
 *   am    = max_k |x[k,t]|                     (token_absmax, :25-33)
 *   raw   = max(am, 1f-8) / 127f0              (IEEE fp32 division, :44)
 *   scale = max(raw, floatmin(Float32))        (:45)
 *   code  = round(Int8, clamp(x/scale, -127, 127))  RoundNearest = ties
 *           to even (:46-47); nearbyintf in the default rounding mode.
 */
void fmso_quantize_int8(const float* x, int64_t dim, int64_t ntok, int8_t* codes, float* scales) {
    int64_t t, k;
    for (t = 0; t < ntok; ++t) {
        const float* xt = x + t * dim;
        float am = 0.0f;
        for (k = 0; k < dim; ++k) {
            float a = fabsf(xt[k]);
            if (a > am) am = a;
        }
        float raw = (am > 1.0e-8f ? am : 1.0e-8f) / 127.0f;
        float sc = raw > FLT_MIN ? raw : FLT_MIN;
        scales[t] = sc;
        for (k = 0; k < dim; ++k) {
            float v = xt[k] / sc;
            if (v > 127.0f) v = 127.0f;
            else if (v < -127.0f) v = -127.0f;
            codes[t * dim + k] = (int8_t)nearbyintf(v);
        }
    }
}

/*
 * binary32 -> binary16, round to nearest, ties to even (IEEE 754), with
 * overflow to Inf and gradual underflow; NaN stays NaN.
 */
static uint16_t float_to_half_rne(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);          /* NaN */
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);         /* >= 65520: Inf */
    int e = (int)(ax >> 23) - 127;
    uint32_t mant = (ax & 0x7fffffu) | 0x800000u;                     /* 24-bit significand */
    uint32_t q, rem, half;
    int s;
    if (e >= -14) {                   /* normal half: keep 11 significant bits */
        s = 13;
        q = ((uint32_t)(e + 15) << 10) + ((mant >> s) & 0x3ffu);
    } else {                          /* subnormal half: units of 2^-24 */
        if (e < -25) return (uint16_t)sign;
        s = -e - 1;                   /* 14 .. 24 */
        q = mant >> s;
    }
    rem = mant & ((1u << s) - 1u);
    half = 1u << (s - 1);
    if (rem > half || (rem == half && (q & 1u))) q += 1u;             /* carries into the exponent */
    return (uint16_t)(sign | q);
}

/*
 * quantize_int8_symmetric for Float16 features (src/quant.jl:21-49): the
 * same steps with every operation in Float16 arithmetic, which Julia
 * evaluates as the fp32 operation rounded back to Float16:
 *   am    = max_k |x[k,t]|                              (exact)
 *   raw   = Float16(max(am, Float16(1f-8)) / 127)       (Float16(1f-8) == 0)
 *   scale = max(raw, floatmin(Float16))                 (2^-14)
 *   code  = round(Int8, clamp(Float16(x / scale), -127, 127))
 * x and scales are binary16 bit patterns.
 */
void fmso_quantize_int8_f16(const uint16_t* x, int64_t dim, int64_t ntok, int8_t* codes,
                            uint16_t* scales) {
    int64_t t, k;
    const float eps = half_to_float(float_to_half_rne(1.0e-8f));
    const float tmin = half_to_float(0x0400u);
    for (t = 0; t < ntok; ++t) {
        const uint16_t* xt = x + t * dim;
        float am = 0.0f;
        for (k = 0; k < dim; ++k) {
            float a = fabsf(half_to_float(xt[k]));
            if (a > am) am = a;
        }
        float raw = half_to_float(float_to_half_rne((am > eps ? am : eps) / 127.0f));
        float sc = raw > tmin ? raw : tmin;
        scales[t] = float_to_half_rne(sc);
        for (k = 0; k < dim; ++k) {
            float v = half_to_float(float_to_half_rne(half_to_float(xt[k]) / sc));
            if (v > 127.0f) v = 127.0f;
            else if (v < -127.0f) v = -127.0f;
            codes[t * dim + k] = (int8_t)nearbyintf(v);
        }
    }
}

/* Test hook: float_to_half_rne over n values (pinned against numpy's conversion). */
void fmso_f32_to_f16(const float* x, int64_t n, uint16_t* out) {
    int64_t i;
    for (i = 0; i < n; ++i) out[i] = float_to_half_rne(x[i]);
}

/* Raw int32 dot products out[u + Td*t] = sum_k qc[k,t]*dc[k,u] (quant.jl:109-112). */
void fmso_int8_dots(const int8_t* qc, const int8_t* dc, int64_t dim, int64_t Tq, int64_t Td,
                    int32_t* out) {
    int64_t t, u, k;
    for (t = 0; t < Tq; ++t)
        for (u = 0; u < Td; ++u) {
            int32_t acc = 0;
            for (k = 0; k < dim; ++k) acc += (int32_t)qc[t * dim + k] * (int32_t)dc[u * dim + k];
            out[u + Td * t] = acc;
        }
}

/*
 * int8_pair_forward_host (src/quant.jl:96-125): deferred dequant
 *   s = (qs[t] * ds[u]) * Float32(acc)   evaluated left to right (:113).
 */
static float int8_pair_core(const int8_t* qc, const float* qs, const int8_t* dc, const float* ds,
                            const uint8_t* qmask, const uint8_t* dmask,
                            int64_t dim, int64_t Tq, int64_t Td, int32_t* args, float* mx) {
    int64_t t, u, k;
    for (t = 0; t < Tq; ++t) { args[t] = 0; mx[t] = 0.0f; }
    for (t = 0; t < Tq; ++t) {
        if (qmask && !qmask[t]) continue;
        float qt = qs[t];
        for (u = 0; u < Td; ++u) {
            if (dmask && !dmask[u]) continue;
            int32_t acc = 0;
            for (k = 0; k < dim; ++k) acc += (int32_t)qc[t * dim + k] * (int32_t)dc[u * dim + k];
            float s = qt * ds[u] * (float)acc;
            if (args[t] == 0 || s > mx[t]) { mx[t] = s; args[t] = (int32_t)(u + 1); }
        }
    }
    float score = 0.0f;
    for (t = 0; t < Tq; ++t) {
        if ((!qmask || qmask[t]) && args[t] > 0) score += mx[t];
        else mx[t] = 0.0f;
    }
    return score;
}

/* int8_paired_forward_host (src/quant.jl:172-185). */
void fmso_int8_paired_forward(const int8_t* Qc, const float* Qs, const int8_t* Dc, const float* Ds,
                              const uint8_t* qmask, const uint8_t* dmask,
                              int64_t dim, int64_t Tq, int64_t Td, int64_t B,
                              float* scores, int32_t* args, float* partial, int nthreads) {
    set_threads(nthreads);
    #pragma omp parallel
    {
        int64_t tq = Tq > 0 ? Tq : 1;
        int32_t* a = (int32_t*)malloc(sizeof(int32_t) * (size_t)tq);
        float* m = (float*)malloc(sizeof(float) * (size_t)tq);
        int64_t b;
        #pragma omp for schedule(dynamic, 4)
        for (b = 0; b < B; ++b) {
            scores[b] = int8_pair_core(Qc + b * dim * Tq, Qs + b * Tq, Dc + b * dim * Td, Ds + b * Td,
                                       qmask ? qmask + b * Tq : NULL, dmask ? dmask + b * Td : NULL,
                                       dim, Tq, Td, a, m);
            if (args) memcpy(args + b * Tq, a, sizeof(int32_t) * (size_t)Tq);
            if (partial) memcpy(partial + b * Tq, m, sizeof(float) * (size_t)Tq);
        }
        free(a); free(m);
    }
}

/*
 * INT8 candidate layout: not a reference method (Int8Index has only pair /
 * paired methods, src/dispatch.jl:247-296).  It composes the INT8 pair scan
 * (src/quant.jl:96-125) per (c,b) with the candidate conventions of
 * src/forward_layouts.jl:239-261 (invalid idx -> neg, tape 0).
 */
void fmso_int8_candidates_forward(const int8_t* Qc, const float* Qs, const int8_t* Gc, const float* Gs,
                                  const int64_t* idxs, const uint8_t* qmask, const uint8_t* dmask,
                                  int64_t dim, int64_t Tq, int64_t B, int64_t Td, int64_t N, int64_t C,
                                  float neg, float* S, int32_t* args, float* partial,
                                  const int64_t* pair_subset, int64_t n_subset, int nthreads) {
    int64_t npairs = pair_subset ? n_subset : C * B;
    set_threads(nthreads);
    #pragma omp parallel
    {
        int64_t tq = Tq > 0 ? Tq : 1;
        int32_t* a = (int32_t*)malloc(sizeof(int32_t) * (size_t)tq);
        float* m = (float*)malloc(sizeof(float) * (size_t)tq);
        int64_t i;
        #pragma omp for schedule(dynamic, 16)
        for (i = 0; i < npairs; ++i) {
            int64_t p = pair_subset ? pair_subset[i] : i;
            int64_t b = p / C;
            int64_t j = idxs[p];
            if (!(1 <= j && j <= N)) {
                S[p] = neg;
                if (args) memset(args + p * Tq, 0, sizeof(int32_t) * (size_t)Tq);
                if (partial) memset(partial + p * Tq, 0, sizeof(float) * (size_t)Tq);
                continue;
            }
            S[p] = int8_pair_core(Qc + b * dim * Tq, Qs + b * Tq, Gc + (j - 1) * dim * Td,
                                  Gs + (j - 1) * Td, qmask ? qmask + b * Tq : NULL,
                                  dmask ? dmask + (j - 1) * Td : NULL, dim, Tq, Td, a, m);
            if (args) memcpy(args + p * Tq, a, sizeof(int32_t) * (size_t)Tq);
            if (partial) memcpy(partial + p * Tq, m, sizeof(float) * (size_t)Tq);
        }
        free(a); free(m);
    }
}

/* ---- finalize (src/normalize.jl, src/forward_pair.jl:153-173) ------------- */

/*
 * inv_token_counts (src/normalize.jl:4-10): inv[b] = 1 / max(count(qmask[:,b]), 1)
 * in fp32.  Scores are multiplied by inv (length_normalize, :23-25), never
 * divided; invalid candidates keep neg (length_normalize_candidates, :37-46).
 */
void fmso_inv_token_counts(const uint8_t* qmask, int64_t Tq, int64_t B, float* inv) {
    int64_t b, t;
    for (b = 0; b < B; ++b) {
        int64_t n = 0;
        for (t = 0; t < Tq; ++t) n += (qmask == NULL || qmask[b * Tq + t]) ? 1 : 0;
        float nf = (float)n;
        inv[b] = 1.0f / (nf > 1.0f ? nf : 1.0f);
    }
}

/* ---- fp64 dense oracle (src/dense.jl:26-56) -------------------------------- */

/*
 * maxsim_dense with accum = Float64: materialises S = d' * q in fp64, first
 * valid hit wins with strict >, Sigma over hit tokens, optional divide by
 * max(nq, 1).  args_out (Tq, nullable) receives the 1-based argmax.
 */
double fmso_dense_pair_f64(int dtype, const void* q, const void* d,
                           const uint8_t* qmask, const uint8_t* dmask,
                           int64_t dim, int64_t Tq, int64_t Td, int normalize, int32_t* args_out) {
    double score = 0.0;
    int64_t nq = 0, t, u, k;
    for (t = 0; t < Tq; ++t) {
        if (args_out) args_out[t] = 0;
        if (qmask && !qmask[t]) continue;
        double mx = 0.0;
        int64_t hit = 0;
        for (u = 0; u < Td; ++u) {
            if (dmask && !dmask[u]) continue;
            double s = 0.0;
            for (k = 0; k < dim; ++k)
                s += load_f64(dtype, d, u * dim + k) * load_f64(dtype, q, t * dim + k);
            if (!hit || s > mx) { mx = s; hit = u + 1; }
        }
        if (!hit) continue;
        if (args_out) args_out[t] = (int32_t)hit;
        score += mx;
        ++nq;
    }
    return normalize ? score / (double)(nq > 1 ? nq : 1) : score;
}

/* ---- backward on the argmax tape (src/backward_pair.jl, src/backward_layouts.jl,
 *      src/packed.jl:361-377, :424-442) ---------------------------------------- */

/*
 * The reference's CPU pullback for one pair (pair_pullback, backward_pair.jl:14-37,
 * with accumulate_doc! AtomicUnified, accumulate.jl:12-29): for every query token t
 * with qmask[t] and 1 <= u = argmax[t] <= Td,
 *     dq[:, t] += delta * d[:, u]      and      dd[:, u] += delta * q[:, t],
 * t ascending.  InvGrid (accumulate.jl:31-39, invgrid.jl:46-65) visits the same
 * sources of each destination in the same (ascending t) order.
 * The reference computes in the feature type T; this restatement pins the
 * mathematics: delta and both accumulations in fp64.  dq/dd are ADDED to.
 */
static void pair_pullback_f64(int dtype, double delta, const void* q, const void* d,
                              const uint8_t* qmask, const int32_t* args,
                              int64_t dim, int64_t Tq, int64_t Td, double* dq, double* dd) {
    int64_t t, k;
    if (delta == 0.0) return; /* backward_pair.jl:21 */
    for (t = 0; t < Tq; ++t) {
        if (qmask && !qmask[t]) continue;
        const int64_t u = (int64_t)args[t];
        if (u < 1 || u > Td) continue;
        for (k = 0; k < dim; ++k) {
            dq[t * dim + k] += delta * load_f64(dtype, d, (u - 1) * dim + k);
            dd[(u - 1) * dim + k] += delta * load_f64(dtype, q, t * dim + k);
        }
    }
}

/* paired_pullback CPU (backward_layouts.jl:13-26): pair b, delta = Delta[b] * inv_n[b].
 * dQ (B,Tq,dim) and dD (B,Td,dim) are overwritten.  inv_n NULL = all ones. */
void fmso_paired_backward(int dtype, const void* Q, const void* D, const uint8_t* qmask,
                          const int32_t* args, const double* Delta, const double* inv_n,
                          int64_t dim, int64_t Tq, int64_t Td, int64_t B,
                          double* dQ, double* dD) {
    int64_t b;
    memset(dQ, 0, sizeof(double) * (size_t)(B * Tq * dim));
    memset(dD, 0, sizeof(double) * (size_t)(B * Td * dim));
    for (b = 0; b < B; ++b)
        pair_pullback_f64(dtype, Delta[b] * (inv_n ? inv_n[b] : 1.0),
                          advance(Q, b * Tq * dim, dtype), advance(D, b * Td * dim, dtype),
                          qmask ? qmask + b * Tq : NULL, args + b * Tq, dim, Tq, Td,
                          dQ + b * Tq * dim, dD + b * Td * dim);
}

/* inbatch_pullback CPU (backward_layouts.jl:69-94): j outer, i inner; pair (i, j) has
 * delta = Delta[j, i] * inv_n[i] (Delta (Bd, Bq) column-major: j + Bd*i) and tape
 * args[t, j, i] at t + Tq*(j + Bd*i). */
void fmso_inbatch_backward(int dtype, const void* Q, const void* D, const uint8_t* qmask,
                           const int32_t* args, const double* Delta, const double* inv_n,
                           int64_t dim, int64_t Tq, int64_t Td, int64_t Bq, int64_t Bd,
                           double* dQ, double* dD) {
    int64_t i, j;
    memset(dQ, 0, sizeof(double) * (size_t)(Bq * Tq * dim));
    memset(dD, 0, sizeof(double) * (size_t)(Bd * Td * dim));
    for (j = 0; j < Bd; ++j)
        for (i = 0; i < Bq; ++i) {
            const int64_t p = j + Bd * i;
            pair_pullback_f64(dtype, Delta[p] * (inv_n ? inv_n[i] : 1.0),
                              advance(Q, i * Tq * dim, dtype), advance(D, j * Td * dim, dtype),
                              qmask ? qmask + i * Tq : NULL, args + p * Tq, dim, Tq, Td,
                              dQ + i * Tq * dim, dD + j * Td * dim);
        }
}

/* candidates_pullback CPU (backward_layouts.jl:137-165): b outer, c inner; pair
 * p = c + C*b scores Q_b against gallery doc idxs[p] (1-based; outside 1..N the
 * pair contributes nothing); delta = Delta[p] * inv_n[b]. */
void fmso_candidates_backward(int dtype, const void* Q, const void* G, const int64_t* idxs,
                              const uint8_t* qmask, const int32_t* args, const double* Delta,
                              const double* inv_n, int64_t dim, int64_t Tq, int64_t Td,
                              int64_t B, int64_t C, int64_t N, double* dQ, double* dG) {
    int64_t b, c;
    memset(dQ, 0, sizeof(double) * (size_t)(B * Tq * dim));
    memset(dG, 0, sizeof(double) * (size_t)(N * Td * dim));
    for (b = 0; b < B; ++b)
        for (c = 0; c < C; ++c) {
            const int64_t p = c + C * b, j = idxs[p];
            if (j < 1 || j > N) continue;
            pair_pullback_f64(dtype, Delta[p] * (inv_n ? inv_n[b] : 1.0),
                              advance(Q, b * Tq * dim, dtype), advance(G, (j - 1) * Td * dim, dtype),
                              qmask ? qmask + b * Tq : NULL, args + p * Tq, dim, Tq, Td,
                              dQ + b * Tq * dim, dG + (j - 1) * Td * dim);
        }
}

/* packed_pullback CPU (packed.jl:361-377): document b = tokens[cu[b]..cu[b+1]-1]
 * (1-based cu), delta = Delta[b] * inv_n (one value for the single query). */
void fmso_packed_backward(int dtype, const void* q, const void* tokens, const int32_t* cu,
                          const uint8_t* qmask, const int32_t* args, const double* Delta,
                          double inv_n, int64_t dim, int64_t Tq, int64_t B, int64_t ntok,
                          double* dq, double* dP) {
    int64_t b;
    memset(dq, 0, sizeof(double) * (size_t)(Tq * dim));
    memset(dP, 0, sizeof(double) * (size_t)(ntok * dim));
    for (b = 0; b < B; ++b) {
        const int64_t a = (int64_t)cu[b] - 1, z = (int64_t)cu[b + 1] - 1;
        pair_pullback_f64(dtype, Delta[b] * inv_n, q, advance(tokens, a * dim, dtype), qmask,
                          args + b * Tq, dim, Tq, z - a, dq, dP + a * dim);
    }
}

/* varlen_pullback CPU (packed.jl:424-442): pair n = (Q tokens cu_q[n]..cu_q[n+1]-1,
 * D tokens cu_d[n]..cu_d[n+1]-1), no masks, tape column n of args (max_q, N);
 * delta = Delta[n] * inv_n[n]. */
void fmso_varlen_backward(int dtype, const void* Qt, const void* Dt, const int32_t* cu_q,
                          const int32_t* cu_d, const int32_t* args, const double* Delta,
                          const double* inv_n, int64_t dim, int64_t max_q, int64_t N,
                          int64_t nq, int64_t nd, double* dQ, double* dD) {
    int64_t n;
    memset(dQ, 0, sizeof(double) * (size_t)(nq * dim));
    memset(dD, 0, sizeof(double) * (size_t)(nd * dim));
    for (n = 0; n < N; ++n) {
        const int64_t qa = (int64_t)cu_q[n] - 1, qz = (int64_t)cu_q[n + 1] - 1;
        const int64_t da = (int64_t)cu_d[n] - 1, dz = (int64_t)cu_d[n + 1] - 1;
        pair_pullback_f64(dtype, Delta[n] * (inv_n ? inv_n[n] : 1.0), advance(Qt, qa * dim, dtype),
                          advance(Dt, da * dim, dtype), NULL, args + n * max_q, dim, qz - qa,
                          dz - da, dQ + qa * dim, dD + da * dim);
    }
}

/* ---- per-row top-k (no reference counterpart) ------------------------------
 *
 * What a retrieval caller does with a score column in the reference
 * (README.md:132: ranking is the caller's job), i.e.
 * partialsortperm(scores[:, i], 1:k; rev = true) with a stable sort: the order
 * is Base.isless reversed, equal scores by smaller index.  isless on floats:
 * NaN is above everything (every NaN equal), -0.0 below +0.0, otherwise <.
 * Restated with a comparison sort (qsort on (value, index)), not with the
 * device kernel's radix keys.
 */
typedef struct { float v; int64_t i; } fmso_scored;

static int julia_isless_f32(float a, float b) {
    if (isnan(a)) return 0;
    if (isnan(b)) return 1;
    if (a < b) return 1;
    if (a > b) return 0;
    return signbit(a) && !signbit(b); /* -0.0 < +0.0 */
}

static int topk_cmp(const void* pa, const void* pb) {
    const fmso_scored* a = (const fmso_scored*)pa;
    const fmso_scored* b = (const fmso_scored*)pb;
    if (julia_isless_f32(b->v, a->v)) return -1; /* a ranks first */
    if (julia_isless_f32(a->v, b->v)) return 1;
    return a->i < b->i ? -1 : (a->i > b->i ? 1 : 0);
}

/* scores (nrows, ncols) row-major; vals/idx (nrows, k), idx 1-based. 0 <= k <= ncols. */
void fmso_topk(const float* scores, int64_t nrows, int64_t ncols, int64_t k, float* vals,
               int32_t* idx) {
    int64_t r, j;
    fmso_scored* buf = (fmso_scored*)malloc(sizeof(fmso_scored) * (size_t)(ncols > 0 ? ncols : 1));
    for (r = 0; r < nrows; ++r) {
        for (j = 0; j < ncols; ++j) { buf[j].v = scores[r * ncols + j]; buf[j].i = j; }
        qsort(buf, (size_t)ncols, sizeof(fmso_scored), topk_cmp);
        for (j = 0; j < k; ++j) {
            vals[r * k + j] = buf[j].v;
            idx[r * k + j] = (int32_t)(buf[j].i + 1);
        }
    }
    free(buf);
}
