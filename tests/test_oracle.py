"""Pins the CPU oracle (oracle/fms_oracle.c) before it is trusted as the checker.

The reference (Julia) cannot run here and its tests hold no stored vectors,
so each oracle function is pinned by
  * the closed-form / known-answer cases of the reference's own tests,
  * an independent numpy implementation that MATERIALISES the similarity
    matrix in fp64 and takes np.argmax (first occurrence) -- a different
    algorithm from the oracle's tiled fp32 running max,
  * exact integer arithmetic (numpy int64 matmul) for the INT8 dots, and the
    same fixed dequant order for INT8 scores,
  * layout invariants (identity candidates == paired, packed single doc ==
    pair, permuted idxs permute outputs),
  * the committed golden fixtures in tests/golden/ (numpy fp64 vectors).
A planted mistake (dropped mask, off-by-one tape, lost sign, transposed
operand, wrong tie-break) fails at least one of these.
"""
import os

import numpy as np
import pytest

import oracle
from helpers import tokens

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---- independent numpy implementation (fp64, materialising) ---------------------------

def np_pair(q, d, qm=None, dm=None):
    """Returns (score, tape, partial) like the reference's pair scan, in fp64."""
    q = q.astype(np.float64)
    d = d.astype(np.float64)
    Tq, Td = q.shape[0], d.shape[0]
    S = d @ q.T  # (Td, Tq)
    valid_u = np.ones(Td, bool) if dm is None else dm.astype(bool)
    valid_t = np.ones(Tq, bool) if qm is None else qm.astype(bool)
    tape = np.zeros(Tq, np.int32)
    part = np.zeros(Tq, np.float64)
    if valid_u.any():
        Sm = np.where(valid_u[:, None], S, -np.inf)
        am = np.argmax(Sm, axis=0)
        tape = np.where(valid_t, am + 1, 0).astype(np.int32)
        part = np.where(valid_t, Sm[am, np.arange(Tq)], 0.0)
    return part.sum(), tape, part, S


def widen(a, bf16):
    return oracle.bf16_bits_to_f32(a) if bf16 else a.astype(np.float32)


def feature(x, kind):
    if kind == "f32":
        return x.astype(np.float32), False
    if kind == "f16":
        return x.astype(np.float16), False
    return oracle.f32_to_bf16_bits(x), True


def check_tape(got, want, S, valid_u, rtol=1e-5):
    """Equal except at fp64-vs-fp32 near ties (both picks must be valid and tied)."""
    for t in np.nonzero(got != want)[0]:
        g, w = got[t], want[t]
        assert g > 0 and w > 0 and valid_u[g - 1] and valid_u[w - 1]
        assert abs(S[g - 1, t] - S[w - 1, t]) <= rtol * max(1.0, abs(S[w - 1, t]))


# ---- known answers from the reference's tests -----------------------------------------------

def test_all_negative_dots():
    """test_regressions.jl:136-147: q=ones(4,3), d=-ones(4,5) => -12, every tape entry 1."""
    s, a, p = oracle.pair_forward(np.ones((3, 4), np.float32), -np.ones((5, 4), np.float32))
    assert s == np.float32(-12.0)
    assert (a == 1).all() and (p == -4.0).all()


def test_empty_document_scores_zero():
    """test_regressions.jl:65-86: all-false dmask => score 0 (not neg), tape 0."""
    rng = np.random.default_rng(11)
    q, d = tokens(rng, (5, 8)), tokens(rng, (6, 8))
    s, a, p = oracle.pair_forward(q, d, None, np.zeros(6, np.uint8))
    assert s == 0.0 and (a == 0).all() and (p == 0).all()
    s, a, p = oracle.packed_forward(q, d[:0], np.array([1, 1], np.int32))
    assert s[0] == 0.0 and (a == 0).all()


def test_invalid_candidate_gets_neg():
    """test_forward.jl:41-49 / test_ka_cpu.jl:50-57: idx 0 => neg, tape 0."""
    rng = np.random.default_rng(3)
    Q, G = tokens(rng, (4, 8, 16)), tokens(rng, (12, 10, 16))
    idxs = np.array([[1, 5, 0], [2, 6, 1], [3, 7, 2], [4, 8, 3]], np.int64)  # Julia [1 2 3 4; 5 6 7 8; 0 1 2 3]
    S, a, _ = oracle.candidates_forward(Q, G, idxs)
    assert S[0, 2] == np.float32(-1.0e4)
    assert (a[0, 2] == 0).all()
    s11, _, _ = oracle.pair_forward(Q[0], G[0])
    assert S[0, 0] == s11
    for neg in (0.0, 10.0, -1.0e4):  # adversarial neg: never a similarity clamp
        S2, _, _ = oracle.candidates_forward(Q, G, idxs, neg=neg)
        assert S2[0, 2] == np.float32(neg) and S2[1, 1] == S[1, 1]


def test_inbatch_doc_chunk_known_answers():
    """test_regressions.jl:149-154."""
    assert oracle.inbatch_doc_chunk(4, 128, 32, 32, 10_000) == 128
    assert oracle.inbatch_doc_chunk(8, 128, 32, 32, 10_000) == 64
    assert oracle.inbatch_doc_chunk(4, 128, 32, 32, 0) == 1


def test_inv_token_counts():
    qm = np.array([[1, 1, 0, 1], [0, 0, 0, 0], [1, 1, 1, 1]], np.uint8)
    inv = oracle.inv_token_counts(qm)
    assert inv.tolist() == [np.float32(1) / np.float32(3), 1.0, 0.25]


# ---- oracle vs independent numpy (all layouts, all feature types) ------------------------------

@pytest.mark.parametrize("kind", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("shape", [(40, 33, 65, 3), (16, 12, 130, 2), (128, 32, 180, 2), (8, 6, 7, 3)])
def test_paired_vs_numpy(kind, shape):
    dim, Tq, Td, B = shape
    rng = np.random.default_rng(list(shape) + [len(kind)])
    Q, bf = feature(tokens(rng, (B, Tq, dim)), kind)
    D, _ = feature(tokens(rng, (B, Td, dim)), kind)
    qm = (rng.random((B, Tq)) < 0.8).astype(np.uint8)
    dm = (rng.random((B, Td)) < 0.7).astype(np.uint8)
    dm[-1] = 0
    s, a, p = oracle.paired_forward(Q, D, qm, dm, bf16=bf)
    for b in range(B):
        ref, tape, part, S = np_pair(widen(Q[b], bf), widen(D[b], bf), qm[b], dm[b])
        assert abs(s[b] - ref) <= 1e-5 * max(1, abs(ref))
        np.testing.assert_allclose(p[b], part, rtol=1e-5, atol=1e-6)
        check_tape(a[b], tape, S, dm[b].astype(bool))


def test_candidates_inbatch_packed_varlen_vs_numpy():
    rng = np.random.default_rng(2024)
    dim, Tq, Td, N, C, B = 24, 9, 37, 7, 4, 3
    Q = tokens(rng, (B, Tq, dim))
    G = tokens(rng, (N, Td, dim))
    qm = (rng.random((B, Tq)) < 0.8).astype(np.uint8)
    dmG = np.array([[(u + 1) % 4 != 0 for u in range(Td)] for _ in range(N)], np.uint8)
    idxs = rng.integers(0, N + 2, size=(B, C))
    S, a, _ = oracle.candidates_forward(Q, G, idxs, qm, dmG, neg=-7.0)
    for b in range(B):
        for c in range(C):
            j = idxs[b, c]
            if not (1 <= j <= N):
                assert S[b, c] == np.float32(-7.0) and (a[b, c] == 0).all()
                continue
            ref, tape, _, Sm = np_pair(Q[b], G[j - 1], qm[b], dmG[j - 1])
            assert abs(S[b, c] - ref) <= 1e-5 * max(1, abs(ref))
            check_tape(a[b, c], tape, Sm, dmG[j - 1].astype(bool))
    # in-batch: S[i, j] = MaxSim(Q_i, D_j) (Julia S[j,i])
    D = G[:5]
    dm = dmG[:5]
    Sib, aib = oracle.inbatch_forward(Q, D, qm, dm)
    for i in range(B):
        for j in range(5):
            ref, tape, _, Sm = np_pair(Q[i], D[j], qm[i], dm[j])
            assert abs(Sib[i, j] - ref) <= 1e-5 * max(1, abs(ref))
            check_tape(aib[i, j], tape, Sm, dm[j].astype(bool))
    # packed: document-local tape, no dmask
    lens = [5, 0, 3, 9]
    tok = tokens(rng, (sum(lens), dim))
    cu = np.concatenate([[1], 1 + np.cumsum(lens)]).astype(np.int32)
    sp, ap, _ = oracle.packed_forward(Q[0], tok, cu, qm[0])
    for b, n in enumerate(lens):
        ref, tape, _, Sm = np_pair(Q[0], tok[cu[b] - 1: cu[b + 1] - 1], qm[0])
        assert abs(sp[b] - ref) <= 1e-5 * max(1, abs(ref))
        check_tape(ap[b], tape, Sm, np.ones(n, bool))
    # varlen: rows beyond Tq_n stay 0
    qlens, dlens = [4, 2, 0], [5, 0, 3]
    Qt, Dt = tokens(rng, (sum(qlens), dim)), tokens(rng, (sum(dlens), dim))
    cq = np.concatenate([[1], 1 + np.cumsum(qlens)]).astype(np.int32)
    cd = np.concatenate([[1], 1 + np.cumsum(dlens)]).astype(np.int32)
    sv, av, _ = oracle.varlen_forward(Qt, Dt, cq, cd)
    assert av.shape == (3, 4)
    for n in range(3):
        ref, tape, _, Sm = np_pair(Qt[cq[n] - 1: cq[n + 1] - 1], Dt[cd[n] - 1: cd[n + 1] - 1])
        assert abs(sv[n] - ref) <= 1e-5 * max(1, abs(ref))
        assert (av[n, qlens[n]:] == 0).all()
        check_tape(av[n, :qlens[n]], tape, Sm, np.ones(dlens[n], bool))


def test_dense_f64_matches_numpy():
    rng = np.random.default_rng(9)
    q, d = tokens(rng, (12, 16)), tokens(rng, (20, 16))
    qm = np.array([(t + 1) % 2 == 1 for t in range(12)], np.uint8)
    dm = np.array([(u + 1) % 3 != 0 for u in range(20)], np.uint8)
    s, a = oracle.dense_pair_f64(q, d, qm, dm)
    ref, tape, _, _ = np_pair(q, d, qm, dm)
    assert abs(s - ref) < 1e-12 and (a == tape).all()
    sn, _ = oracle.dense_pair_f64(q, d, qm, dm, normalize=True)
    assert abs(sn - ref / qm.sum()) < 1e-12
    s32, _, _ = oracle.pair_forward(q, d, qm, dm)
    assert abs(s32 - s) < 1e-5


# ---- invariants ----------------------------------------------------------------------------

def test_layout_invariants():
    rng = np.random.default_rng(77)
    dim, Tq, Td, B = 32, 10, 45, 4
    Q = tokens(rng, (B, Tq, dim)).astype(np.float16)
    D = tokens(rng, (B, Td, dim)).astype(np.float16)
    s, a, p = oracle.paired_forward(Q, D)
    # paired == candidates with identity indices (C = 1)
    S, ac, _ = oracle.candidates_forward(Q, D, np.arange(1, B + 1).reshape(B, 1))
    assert np.array_equal(S[:, 0], s) and np.array_equal(ac[:, 0], a)
    # permuting candidate columns permutes outputs
    idx = rng.integers(1, B + 1, size=(B, 6))
    perm = rng.permutation(6)
    S1, a1, _ = oracle.candidates_forward(Q, D, idx)
    S2, a2, _ = oracle.candidates_forward(Q, D, idx[:, perm])
    assert np.array_equal(S1[:, perm], S2) and np.array_equal(a1[:, perm], a2)
    # packed with one document == pair
    sp, ap, _ = oracle.packed_forward(Q[1], D[1], np.array([1, Td + 1], np.int32))
    assert sp[0] == s[1] and np.array_equal(ap[0], a[1])
    # splitting the embedding into halves: dots add up (closed form of split-d)
    ref, _, _, S_full = np_pair(Q[0], D[0])
    _, _, _, S_lo = np_pair(Q[0][:, :16], D[0][:, :16])
    _, _, _, S_hi = np_pair(Q[0][:, 16:], D[0][:, 16:])
    np.testing.assert_allclose(S_lo + S_hi, S_full, atol=1e-12)


def test_bounded_subset_matches_full():
    rng = np.random.default_rng(8)
    Q, G = tokens(rng, (3, 8, 16)), tokens(rng, (9, 12, 16))
    idx = rng.integers(1, 10, size=(3, 5))
    S, a, p = oracle.candidates_forward(Q, G, idx)
    sub = np.array([0, 7, 14], np.int64)
    S2, a2, _ = oracle.candidates_forward(Q, G, idx, subset=sub)
    assert np.array_equal(S2.reshape(-1)[sub], S.reshape(-1)[sub])
    assert np.array_equal(a2.reshape(-1, 8)[sub], a.reshape(-1, 8)[sub])


# ---- INT8 ---------------------------------------------------------------------------------

def np_quantize(x):
    am = np.abs(x).max(-1)
    raw = np.maximum(am, np.float32(1e-8)) / np.float32(127)
    sc = np.maximum(raw, np.finfo(np.float32).tiny).astype(np.float32)
    v = np.clip(x / sc[..., None], np.float32(-127), np.float32(127))
    return np.rint(v).astype(np.int8), sc


def test_quantize_closed_forms():
    x = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5],
                  [0.0] * 8,
                  [1e-12] * 8], np.float32)
    c, s = oracle.quantize_int8(x)
    assert s[0] == np.float32(1.0)
    assert c[0].tolist() == [127, 0, 2, 2, 0, -2, -2, 4]  # round half to even
    assert s[1] == np.float32(1e-8) / np.float32(127) and (c[1] == 0).all()
    assert s[2] == s[1]


def test_quantize_vs_numpy():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((500, 48)).astype(np.float32) * rng.uniform(1e-6, 1e6, (500, 1)).astype(np.float32)
    c, s = oracle.quantize_int8(x)
    c2, s2 = np_quantize(x)
    assert np.array_equal(s.view(np.uint32), s2.view(np.uint32))
    assert np.array_equal(c, c2)
    assert np.abs(c).max() == 127


def test_f32_to_f16_matches_numpy():
    """The oracle's binary32 -> binary16 RNE against numpy's conversion: random bit
    patterns over the whole fp32 range, exact ties between neighbouring halves
    (normal and subnormal), the overflow threshold, Inf and NaN."""
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 2 ** 32, size=200_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    h = np.arange(0, 0x7c00, dtype=np.uint16).view(np.float16).astype(np.float32)
    ties = ((h[:-1].astype(np.float64) + h[1:].astype(np.float64)) / 2).astype(np.float32)
    special = np.array([65504.0, 65519.99, 65520.0, 1e6, np.inf, -np.inf, 2.0 ** -25,
                        2.0 ** -25 * 1.0000001, 2.0 ** -26, -0.0, 0.0], np.float32)
    for arr in (x, ties, -ties, special):
        got = oracle.f32_to_f16(arr)
        with np.errstate(over="ignore"):
            want = arr.astype(np.float16)
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan].view(np.uint16), want[~nan].view(np.uint16))


def np_quantize_f16(x):
    """quantize_int8_symmetric in numpy float16 arithmetic (numpy rounds every float16
    operation's fp32 result to float16, as Julia does)."""
    x = x.astype(np.float16)
    am = np.abs(x).max(-1)
    raw = np.maximum(am, np.float16(1e-8)) / np.float16(127)
    sc = np.maximum(raw, np.finfo(np.float16).tiny)
    v = np.clip(x / sc[..., None], np.float16(-127), np.float16(127))
    return np.rint(v).astype(np.int8), sc


def test_quantize_f16_closed_forms():
    x = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5],
                  [0.0] * 8,
                  [1e-7] * 8], np.float16)
    c, s = oracle.quantize_int8(x)
    assert s.dtype == np.float16
    assert s[0] == np.float16(1.0)
    assert c[0].tolist() == [127, 0, 2, 2, 0, -2, -2, 4]  # round half to even
    # Float16(1f-8) == 0, so an all-zero token's scale is floatmin(Float16) = 2^-14
    assert s[1] == np.float16(2.0 ** -14) and (c[1] == 0).all()
    # a tiny token: absmax/127 underflows below floatmin -> floored at 2^-14
    assert s[2] == np.float16(2.0 ** -14)


def test_quantize_f16_vs_numpy_and_rounds_the_quotient():
    """Random Float16 tokens: codes and scales bit-exact with numpy float16 arithmetic.
    At least one code differs from what an fp32 quotient would give, so the
    rounding of x / scale to Float16 before round(Int8, .) is pinned too."""
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((2000, 64)) * rng.uniform(1e-3, 1e3, (2000, 1))).astype(np.float16)
    c, s = oracle.quantize_int8(x)
    c2, s2 = np_quantize_f16(x)
    assert np.array_equal(s.view(np.uint16), s2.view(np.uint16))
    assert np.array_equal(c, c2)
    v32 = np.clip(x.astype(np.float32) / s.astype(np.float32)[:, None], -127, 127)
    assert (np.rint(v32).astype(np.int8) != c).any()


def test_int8_dots_and_scan_exact():
    rng = np.random.default_rng(42)
    dim, Tq, Td, B = 40, 7, 11, 3
    Qc, Qs = oracle.quantize_int8(tokens(rng, (B, Tq, dim)))
    Dc, Ds = oracle.quantize_int8(tokens(rng, (B, Td, dim)))
    qm = (rng.random((B, Tq)) < 0.8).astype(np.uint8)
    dm = (rng.random((B, Td)) < 0.8).astype(np.uint8)
    s, a, p = oracle.int8_paired_forward(Qc, Qs, Dc, Ds, qm, dm)
    for b in range(B):
        dots = oracle.int8_dots(Qc[b], Dc[b])
        assert np.array_equal(dots.astype(np.int64), Qc[b].astype(np.int64) @ Dc[b].astype(np.int64).T)
        cell = (Qs[b][:, None] * Ds[b][None, :]).astype(np.float32) * dots.astype(np.float32)
        cell = np.where(dm[b][None, :].astype(bool), cell, -np.inf)
        am = np.argmax(cell, axis=1)
        for t in range(Tq):
            if not qm[b, t] or not dm[b].any():
                assert a[b, t] == 0 and p[b, t] == 0
                continue
            assert a[b, t] == am[t] + 1
            assert p[b, t].view(np.uint32) == np.float32(cell[t, am[t]]).view(np.uint32)
    # candidates compose the same cells; invalid -> neg
    idx = np.array([[1, 0], [2, 3], [3, 1]], np.int64)
    S, ac, pc = oracle.int8_candidates_forward(Qc, Qs, Dc, Ds, idx, qm, dm, neg=-3.0)
    assert S[0, 1] == np.float32(-3.0)
    assert np.array_equal(pc[1, 0], p[1]) and np.array_equal(ac[2, 0], a[2])


# ---- committed fixtures ------------------------------------------------------------------------

def test_golden_fixtures():
    path = os.path.join(GOLDEN, "pair_fixtures.npz")
    z = np.load(path, allow_pickle=False)
    n = int(z["n_cases"])
    assert n >= 4
    for i in range(n):
        q, d = z[f"q{i}"], z[f"d{i}"]
        qm, dm = z[f"qm{i}"], z[f"dm{i}"]
        s, a, p = oracle.pair_forward(q, d, qm, dm)
        want = float(z[f"score{i}"])
        assert abs(float(s) - want) <= 1e-5 * max(1.0, abs(want)), i
        assert np.array_equal(a, z[f"tape{i}"]), i


# ---- property tests of the reference (generator independent) -----------------------

def test_sister_documents_separate_in_fp32():
    """test_edge_cases.jl:26-84: a ranking gap below one Float16 score ulp survives
    Float16 features because scores stay fp32 (pair, paired, candidates, in-batch,
    packed layouts of the oracle)."""
    import sisters
    q, d, sis = sisters.sister_pair()
    gap64 = sisters.maxsim_dense(q, d) - sisters.maxsim_dense(q, sis)
    assert 1e-4 < gap64 < 0.02
    q16, d16, s16 = (x.astype(np.float16) for x in (q, d, sis))
    sa, sb = oracle.pair_forward(q16, d16)[0], oracle.pair_forward(q16, s16)[0]
    assert sa.dtype == np.float32 and sa > sb
    assert abs(float(sa) - float(sb)) < sisters.f16_ulp(float(sa))
    D = np.stack([d16, s16])
    Q2 = np.stack([q16, q16])
    assert np.diff(oracle.paired_forward(Q2, D)[0])[0] < 0
    Sc = oracle.candidates_forward(q16[None], D, np.array([[1, 2]]))[0]
    assert Sc[0, 0] > Sc[0, 1]
    Sib = oracle.inbatch_forward(q16[None], D)[0]
    assert Sib[0, 0] > Sib[0, 1]
    cu = np.array([1, 41, 81], np.int32)
    sp = oracle.packed_forward(q16, np.concatenate([d16, s16]), cu)[0]
    assert sp[0] > sp[1]


def test_sister_ladder_order_matches_f64():
    """test_edge_cases.jl:86-107: five sisters keep the fp64 order in fp32 scores,
    though rounding the scores to Float16 would merge them."""
    import sisters
    q, docs = sisters.sister_ladder()
    s64 = np.array([sisters.maxsim_dense(q, d) for d in docs])
    q16 = q.astype(np.float16)
    s16 = np.array([oracle.pair_forward(q16, d.astype(np.float16))[0] for d in docs])
    assert (np.diff(s16) < 0).all()
    assert (np.argsort(-s16) == np.argsort(-s64)).all()
    assert len(np.unique(s16)) == len(s16)
    assert len(np.unique(s16.astype(np.float16))) < len(s16)
    assert (np.abs(np.diff(s64)) < sisters.F16_ULP_AT_32).all()


def test_int8_ranking_vs_fp32():
    """test_int8.jl:46-59: INT8 scores rank a 64-document gallery like fp32
    (Spearman >= 0.95, top-20 overlap >= 0.7); the helpers themselves are
    pinned on permutations."""
    import sisters
    assert abs(sisters.spearman([1, 2, 3, 4], [10, 20, 30, 40]) - 1.0) < 1e-12
    assert abs(sisters.spearman([1, 2, 3, 4], [4, 3, 2, 1]) + 1.0) < 1e-12
    # 1 - 6 sum(d^2) / (n (n^2 - 1)) for distinct ranks: d = (1, -1, 0, 0) -> 0.8
    assert abs(sisters.spearman([1, 2, 3, 4], [2, 1, 3, 4]) - 0.8) < 1e-12
    assert sisters.topk_overlap([5, 4, 3, 2, 1], [5, 4, 0, 0, 9], 2) == 0.5
    rng = np.random.default_rng(41)
    dim, Tq, Td, N = 32, 12, 20, 64
    q = tokens(rng, (Tq, dim))
    G = tokens(rng, (N, Td, dim))
    s_fp = oracle.paired_forward(np.broadcast_to(q, (N, Tq, dim)).copy(), G)[0]
    qc, qs = oracle.quantize_int8(q)
    gc, gs = oracle.quantize_int8(G)
    s_i8 = oracle.int8_paired_forward(np.broadcast_to(qc, (N, Tq, dim)).copy(),
                                      np.broadcast_to(qs, (N, Tq)).copy(), gc, gs)[0]
    assert sisters.spearman(s_fp, s_i8) >= 0.95
    assert sisters.topk_overlap(s_fp, s_i8, 20) >= 0.7
