/*
 * asan_check.c -- memory check of the CPU oracle (TEST INFRASTRUCTURE ONLY).
 *
 * Built with AddressSanitizer and UndefinedBehaviorSanitizer by `make -C
 * oracle asan` (oracle/_asan/fms_oracle_check) and run by
 * tests/test_oracle_asan.py.  Every fms_oracle.c entry point is called on
 * small inputs held in heap buffers of exactly the documented size, so a read
 * or write one element past any of them stops the run.  The inputs take the
 * edge cases the reference's own tests take: empty documents (cu runs of
 * length 0, Td = 0), fully masked query and document rows, tape entries that
 * name no token (0, past Td, negative), candidate indices outside 1..N,
 * k = ncols in the top-k.  A few cheap invariants (tapes within 1..Td or 0,
 * finite scores) are checked on the way; exact values are the other oracle
 * tests' business.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* fms_oracle.c's entry points (no header: the oracle is loaded by ctypes). */
float fmso_pair_forward(int, const void*, const void*, const uint8_t*, const uint8_t*, int64_t,
                        int64_t, int64_t, int32_t*, float*);
void fmso_paired_forward(int, const void*, const void*, const uint8_t*, const uint8_t*, int64_t,
                         int64_t, int64_t, int64_t, float*, int32_t*, float*, int);
void fmso_candidates_forward(int, const void*, const void*, const int64_t*, const uint8_t*,
                             const uint8_t*, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t,
                             float, float*, int32_t*, float*, const int64_t*, int64_t, int);
void fmso_inbatch_forward(int, const void*, const void*, const uint8_t*, const uint8_t*, int64_t,
                          int64_t, int64_t, int64_t, int64_t, float*, int32_t*, int);
int64_t fmso_inbatch_doc_chunk(int64_t, int64_t, int64_t, int64_t, int64_t);
void fmso_packed_forward(int, const void*, const void*, const int32_t*, const uint8_t*, int64_t,
                         int64_t, int64_t, float*, int32_t*, float*, const int64_t*, int64_t, int);
void fmso_varlen_forward(int, const void*, const void*, const int32_t*, const int32_t*, int64_t,
                         int64_t, int64_t, float*, int32_t*, float*, int);
void fmso_quantize_int8(const float*, int64_t, int64_t, int8_t*, float*);
void fmso_quantize_int8_f16(const uint16_t*, int64_t, int64_t, int8_t*, uint16_t*);
void fmso_f32_to_f16(const float*, int64_t, uint16_t*);
void fmso_int8_dots(const int8_t*, const int8_t*, int64_t, int64_t, int64_t, int32_t*);
void fmso_int8_paired_forward(const int8_t*, const float*, const int8_t*, const float*,
                              const uint8_t*, const uint8_t*, int64_t, int64_t, int64_t, int64_t,
                              float*, int32_t*, float*, int);
void fmso_int8_candidates_forward(const int8_t*, const float*, const int8_t*, const float*,
                                  const int64_t*, const uint8_t*, const uint8_t*, int64_t, int64_t,
                                  int64_t, int64_t, int64_t, int64_t, float, float*, int32_t*,
                                  float*, const int64_t*, int64_t, int);
void fmso_inv_token_counts(const uint8_t*, int64_t, int64_t, float*);
double fmso_dense_pair_f64(int, const void*, const void*, const uint8_t*, const uint8_t*, int64_t,
                           int64_t, int64_t, int, int32_t*);
void fmso_paired_backward(int, const void*, const void*, const uint8_t*, const int32_t*,
                          const double*, const double*, int64_t, int64_t, int64_t, int64_t, double*,
                          double*);
void fmso_inbatch_backward(int, const void*, const void*, const uint8_t*, const int32_t*,
                           const double*, const double*, int64_t, int64_t, int64_t, int64_t,
                           int64_t, double*, double*);
void fmso_candidates_backward(int, const void*, const void*, const int64_t*, const uint8_t*,
                              const int32_t*, const double*, const double*, int64_t, int64_t,
                              int64_t, int64_t, int64_t, int64_t, double*, double*);
void fmso_packed_backward(int, const void*, const void*, const int32_t*, const uint8_t*,
                          const int32_t*, const double*, double, int64_t, int64_t, int64_t, int64_t,
                          double*, double*);
void fmso_varlen_backward(int, const void*, const void*, const int32_t*, const int32_t*,
                          const int32_t*, const double*, const double*, int64_t, int64_t, int64_t,
                          int64_t, int64_t, double*, double*);
void fmso_topk(const float*, int64_t, int64_t, int64_t, float*, int32_t*);

static int g_fail = 0;
#define CHECK(c, what)                                  \
  do {                                                  \
    if (!(c)) {                                         \
      fprintf(stderr, "check failed: %s\n", (what));    \
      g_fail = 1;                                       \
    }                                                   \
  } while (0)

/* malloc of exactly n bytes (at least 1, so a zero-size array is still a
 * distinct allocation whose first byte is already out of bounds for writes
 * past it) */
static void* xm(size_t n) {
  void* p = malloc(n ? n : 1);
  if (!p) {
    fprintf(stderr, "out of memory\n");
    exit(2);
  }
  return p;
}

static uint32_t g_rng = 12345u;
static float frand(void) { /* uniform in [-1, 1) */
  g_rng = g_rng * 1664525u + 1013904223u;
  return (float)((g_rng >> 8) & 0xffffffu) / 8388608.0f - 1.0f;
}
static uint32_t urand(uint32_t n) {
  g_rng = g_rng * 1664525u + 1013904223u;
  return (g_rng >> 8) % n;
}

/* n feature elements of type dt (0 f32, 1 f16, 2 bf16) */
static void* feats(int dt, int64_t n) {
  float* f = xm((size_t)n * sizeof(float));
  for (int64_t i = 0; i < n; ++i) f[i] = frand();
  if (dt == 0) return f;
  uint16_t* h = xm((size_t)n * 2);
  if (dt == 1) {
    fmso_f32_to_f16(f, n, h);
  } else {
    for (int64_t i = 0; i < n; ++i) {
      uint32_t u;
      memcpy(&u, &f[i], 4);
      h[i] = (uint16_t)(u >> 16);
    }
  }
  free(f);
  return h;
}
static uint8_t* mask(int64_t n, int pct) {
  uint8_t* m = xm((size_t)n);
  for (int64_t i = 0; i < n; ++i) m[i] = (uint8_t)(urand(100) < (uint32_t)pct);
  return m;
}
static double* drand_vec(int64_t n) {
  double* d = xm((size_t)n * sizeof(double));
  for (int64_t i = 0; i < n; ++i) d[i] = frand();
  return d;
}
/* a tape of n entries within 0..Td, with junk entries (past Td, negative) */
static int32_t* tape(int64_t n, int64_t Td) {
  int32_t* a = xm((size_t)n * 4);
  for (int64_t i = 0; i < n; ++i) a[i] = (int32_t)urand((uint32_t)Td + 1);
  if (n >= 3) {
    a[0] = (int32_t)Td + 3;
    a[n / 2] = -2;
    a[n - 1] = 0;
  }
  return a;
}
static void tape_in_range(const int32_t* a, int64_t n, int64_t Td, const char* what) {
  for (int64_t i = 0; i < n; ++i) CHECK(a[i] >= 0 && a[i] <= Td, what);
}

static void forward_layouts(int dt) {
  const int64_t dim = 8, Tq = 5, Td = 7, B = 3;
  /* pair, with a fully masked query and an empty document */
  {
    void* q = feats(dt, dim * Tq);
    void* d = feats(dt, dim * Td);
    uint8_t* qm = mask(Tq, 70);
    uint8_t* dm = mask(Td, 60);
    int32_t* a = xm(Tq * 4);
    float* p = xm(Tq * 4);
    float s = fmso_pair_forward(dt, q, d, qm, dm, dim, Tq, Td, a, p);
    CHECK(isfinite(s), "pair score finite");
    tape_in_range(a, Tq, Td, "pair tape");
    memset(qm, 0, Tq);
    s = fmso_pair_forward(dt, q, d, qm, dm, dim, Tq, Td, a, p);
    CHECK(s == 0.0f, "fully masked query scores 0");
    s = fmso_pair_forward(dt, q, d, NULL, NULL, dim, Tq, 0, a, p);
    CHECK(s == 0.0f, "empty document scores 0");
    double s64 = fmso_dense_pair_f64(dt, q, d, NULL, dm, dim, Tq, Td, 1, a);
    CHECK(isfinite(s64), "dense f64 finite");
    free(q), free(d), free(qm), free(dm), free(a), free(p);
  }
  /* paired */
  {
    void* Q = feats(dt, dim * Tq * B);
    void* D = feats(dt, dim * Td * B);
    uint8_t* qm = mask(Tq * B, 80);
    uint8_t* dm = mask(Td * B, 50);
    float* s = xm(B * 4);
    int32_t* a = xm(B * Tq * 4);
    float* p = xm(B * Tq * 4);
    fmso_paired_forward(dt, Q, D, qm, dm, dim, Tq, Td, B, s, a, p, 2);
    tape_in_range(a, B * Tq, Td, "paired tape");
    free(Q), free(D), free(qm), free(dm), free(s), free(a), free(p);
  }
  /* candidates: indices outside 1..N, a pair subset */
  {
    const int64_t N = 5, C = 4;
    void* Q = feats(dt, dim * Tq * B);
    void* G = feats(dt, dim * Td * N);
    int64_t* idx = xm(B * C * 8);
    const int64_t pick[12] = {1, 5, 0, 3, N + 1, -3, 2, 2, 4, 1, 5, 3};
    memcpy(idx, pick, sizeof pick);
    uint8_t* qm = mask(Tq * B, 80);
    uint8_t* dm = mask(Td * N, 60);
    float* S = xm(B * C * 4);
    int32_t* a = xm(B * C * Tq * 4);
    float* p = xm(B * C * Tq * 4);
    fmso_candidates_forward(dt, Q, G, idx, qm, dm, dim, Tq, B, Td, N, C, -1.0e4f, S, a, p, NULL, 0, 2);
    tape_in_range(a, B * C * Tq, Td, "candidates tape");
    int64_t* sub = xm(3 * 8);
    sub[0] = 0, sub[1] = 5, sub[2] = B * C - 1;
    fmso_candidates_forward(dt, Q, G, idx, NULL, NULL, dim, Tq, B, Td, N, C, -1.0e4f, S, a, p, sub, 3, 1);
    int32_t* ta = tape(B * C * Tq, Td);
    double* De = drand_vec(B * C);
    double* iv = drand_vec(B);
    double* dQ = xm(B * Tq * dim * 8);
    double* dG = xm(N * Td * dim * 8);
    fmso_candidates_backward(dt, Q, G, idx, qm, ta, De, iv, dim, Tq, Td, B, C, N, dQ, dG);
    free(Q), free(G), free(idx), free(qm), free(dm), free(S), free(a), free(p), free(sub);
    free(ta), free(De), free(iv), free(dQ), free(dG);
  }
  /* in-batch: a fully masked document */
  {
    const int64_t Bq = 3, Bd = 4;
    void* Q = feats(dt, dim * Tq * Bq);
    void* D = feats(dt, dim * Td * Bd);
    uint8_t* qm = mask(Tq * Bq, 80);
    uint8_t* dm = mask(Td * Bd, 60);
    memset(dm + Td, 0, Td);
    float* S = xm(Bq * Bd * 4);
    int32_t* a = xm(Bq * Bd * Tq * 4);
    fmso_inbatch_forward(dt, Q, D, qm, dm, dim, Tq, Bq, Td, Bd, S, a, 2);
    tape_in_range(a, Bq * Bd * Tq, Td, "in-batch tape");
    CHECK(fmso_inbatch_doc_chunk(dt == 0 ? 4 : 2, Td, Tq, Bq, Bd) >= 1, "doc chunk >= 1");
    int32_t* ta = tape(Bq * Bd * Tq, Td);
    double* De = drand_vec(Bq * Bd);
    double* iv = drand_vec(Bq);
    double* dQ = xm(Bq * Tq * dim * 8);
    double* dD = xm(Bd * Td * dim * 8);
    fmso_inbatch_backward(dt, Q, D, qm, ta, De, iv, dim, Tq, Td, Bq, Bd, dQ, dD);
    int32_t* tp = tape(B * Tq, Td);
    double* Dp = drand_vec(B);
    fmso_paired_backward(dt, Q, D, qm, tp, Dp, iv, dim, Tq, Td, B, dQ, dD);
    free(Q), free(D), free(qm), free(dm), free(S), free(a), free(ta), free(De), free(iv);
    free(dQ), free(dD), free(tp), free(Dp);
  }
  /* packed: empty documents, a document subset */
  {
    const int32_t lens[4] = {3, 0, 5, 1};
    const int64_t nb = 4, ntok = 9;
    int32_t* cu = xm((nb + 1) * 4);
    cu[0] = 1;
    for (int b = 0; b < nb; ++b) cu[b + 1] = cu[b] + lens[b];
    void* q = feats(dt, dim * Tq);
    void* tok = feats(dt, dim * ntok);
    uint8_t* qm = mask(Tq, 80);
    float* s = xm(nb * 4);
    int32_t* a = xm(nb * Tq * 4);
    float* p = xm(nb * Tq * 4);
    fmso_packed_forward(dt, q, tok, cu, qm, dim, Tq, nb, s, a, p, NULL, 0, 2);
    CHECK(s[1] == 0.0f, "empty packed document scores 0");
    int64_t* sub = xm(2 * 8);
    sub[0] = 0, sub[1] = 2;
    fmso_packed_forward(dt, q, tok, cu, NULL, dim, Tq, nb, s, a, p, sub, 2, 1);
    int32_t* ta = tape(nb * Tq, 5);
    double* De = drand_vec(nb);
    double* dq = xm(Tq * dim * 8);
    double* dP = xm(ntok * dim * 8);
    fmso_packed_backward(dt, q, tok, cu, qm, ta, De, 0.25, dim, Tq, nb, ntok, dq, dP);
    free(cu), free(q), free(tok), free(qm), free(s), free(a), free(p), free(sub), free(ta);
    free(De), free(dq), free(dP);
  }
  /* varlen: an empty query and an empty document */
  {
    const int64_t N = 3, max_q = 3, nq = 5, nd = 6;
    int32_t cq[4] = {1, 3, 3, 6}, cd[4] = {1, 5, 7, 7};
    int32_t* cu_q = xm(4 * 4);
    int32_t* cu_d = xm(4 * 4);
    memcpy(cu_q, cq, sizeof cq);
    memcpy(cu_d, cd, sizeof cd);
    void* Qt = feats(dt, dim * nq);
    void* Dt = feats(dt, dim * nd);
    float* s = xm(N * 4);
    int32_t* a = xm(N * max_q * 4);
    float* p = xm(N * max_q * 4);
    fmso_varlen_forward(dt, Qt, Dt, cu_q, cu_d, dim, N, max_q, s, a, p, 2);
    CHECK(s[1] == 0.0f && s[2] == 0.0f, "empty query / document score 0");
    int32_t* ta = tape(N * max_q, 4);
    double* De = drand_vec(N);
    double* iv = drand_vec(N);
    double* dQ = xm(nq * dim * 8);
    double* dD = xm(nd * dim * 8);
    fmso_varlen_backward(dt, Qt, Dt, cu_q, cu_d, ta, De, iv, dim, max_q, N, nq, nd, dQ, dD);
    free(cu_q), free(cu_d), free(Qt), free(Dt), free(s), free(a), free(p), free(ta), free(De);
    free(iv), free(dQ), free(dD);
  }
}

static void int8_paths(void) {
  const int64_t dim = 16, Tq = 4, Td = 6, B = 2, N = 3, C = 3;
  float* xq = feats(0, dim * Tq * B);
  float* xd = feats(0, dim * Td * N);
  for (int64_t k = 0; k < dim; ++k) xd[k] = 0.0f; /* an all-zero token: scale floor */
  int8_t* Qc = xm(dim * Tq * B);
  int8_t* Dc = xm(dim * Td * N);
  float* Qs = xm(Tq * B * 4);
  float* Ds = xm(Td * N * 4);
  fmso_quantize_int8(xq, dim, Tq * B, Qc, Qs);
  fmso_quantize_int8(xd, dim, Td * N, Dc, Ds);
  uint16_t* h = xm(dim * Tq * B * 2);
  fmso_f32_to_f16(xq, dim * Tq * B, h);
  int8_t* hc = xm(dim * Tq * B);
  uint16_t* hs = xm(Tq * B * 2);
  fmso_quantize_int8_f16(h, dim, Tq * B, hc, hs);
  int32_t* dots = xm(Tq * Td * 4);
  fmso_int8_dots(Qc, Dc, dim, Tq, Td, dots);
  uint8_t* qm = mask(Tq * B, 80);
  uint8_t* dm = mask(Td * N, 60);
  float* s = xm(B * 4);
  int32_t* a = xm(B * Tq * 4);
  float* p = xm(B * Tq * 4);
  fmso_int8_paired_forward(Qc, Qs, Dc, Ds, qm, dm, dim, Tq, Td, B, s, a, p, 2);
  tape_in_range(a, B * Tq, Td, "int8 paired tape");
  int64_t* idx = xm(B * C * 8);
  const int64_t pick[6] = {1, 0, 3, N + 2, 2, -1};
  memcpy(idx, pick, sizeof pick);
  float* S = xm(B * C * 4);
  int32_t* ac = xm(B * C * Tq * 4);
  float* pc = xm(B * C * Tq * 4);
  fmso_int8_candidates_forward(Qc, Qs, Dc, Ds, idx, qm, dm, dim, Tq, B, Td, N, C, -1.0e4f, S, ac, pc,
                               NULL, 0, 2);
  tape_in_range(ac, B * C * Tq, Td, "int8 candidates tape");
  float* inv = xm(B * 4);
  fmso_inv_token_counts(qm, Tq, B, inv);
  for (int64_t b = 0; b < B; ++b) CHECK(inv[b] > 0.0f && inv[b] <= 1.0f, "inverse token count");
  free(xq), free(xd), free(Qc), free(Dc), free(Qs), free(Ds), free(h), free(hc), free(hs);
  free(dots), free(qm), free(dm), free(s), free(a), free(p), free(idx), free(S), free(ac), free(pc);
  free(inv);
}

static void topk(void) {
  const int64_t nrows = 3, ncols = 10;
  float* sc = feats(0, nrows * ncols);
  for (int64_t k = 1; k <= ncols; k += 3) {
    float* v = xm(nrows * k * 4);
    int32_t* ix = xm(nrows * k * 4);
    fmso_topk(sc, nrows, ncols, k, v, ix);
    for (int64_t i = 0; i < nrows * k; ++i) CHECK(ix[i] >= 1 && ix[i] <= ncols, "top-k index");
    free(v), free(ix);
  }
  free(sc);
}

int main(void) {
  for (int dt = 0; dt < 3; ++dt) forward_layouts(dt);
  int8_paths();
  topk();
  if (g_fail) return 1;
  printf("oracle asan check ok\n");
  return 0;
}
