"""GPU parity with Inf / NaN features: the reference's running max starts empty
(`arg == 0 || s > mx`, kernels_forward.jl:49-52), so the first valid document
token is always taken whatever its score -- a NaN there sticks (nothing compares
greater than NaN), all -Inf scores keep the first token with -Inf, and a NaN
anywhere later is skipped.  Every kernel family (fast, split-d, generic, the
in-batch MFMA kernel and its fallback, candidates in both orders, packed single
and multi-query) is compared with the oracle, which applies that rule literally.
Scores must agree in class (NaN, +Inf, -Inf) and, where finite, within the
feature type's tolerance; tapes must be identical in every cell."""
import numpy as np
import pytest
import torch

import oracle
from helpers import FEATURE_TOL, as_feature, tokens

from flashmaxsim import boundary

pytestmark = pytest.mark.gpu

NAN, INF = np.float32(np.nan), np.float32(np.inf)
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def assert_class_equal(got, want, rtol, what):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, what
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), f"{what}: NaN at {np.argwhere(gn != wn)[:5].tolist()}"
    inf = np.isinf(want)
    assert np.array_equal(np.isinf(got), inf), f"{what}: Inf pattern differs"
    assert np.array_equal(got[inf], want[inf]), f"{what}: Inf signs differ"
    fin = np.isfinite(want)
    err = np.abs(got[fin] - want[fin])
    assert np.all(err <= rtol * np.maximum(1.0, np.abs(want[fin]))), (what, err.max(initial=0))


def nonfinite_pairs(rng, B, Tq, Td, dim):
    """(Q, D, qmask, dmask) fp32 with one non-finite pattern per pair (see the cases)."""
    assert B >= 8 and Tq >= 8 and Td >= 8
    Q = tokens(rng, (B, Tq, dim))
    D = tokens(rng, (B, Td, dim))
    qm = np.ones((B, Tq), np.uint8)
    dm = np.ones((B, Td), np.uint8)
    D[0, 0, 3] = NAN                       # first valid row NaN: (NaN, 1) for every token
    dm[1, :5] = 0
    D[1, 5, 7] = NAN                       # first valid row (6) NaN after masked rows
    D[2, 3, 0] = NAN                       # a NaN row that is not first: skipped
    Q[3, 2, 5] = NAN                       # a NaN query token: all its scores NaN
    Q[3, 7, 0] = NAN
    qm[3, 7] = 0                           # ... but masked: partial 0, tape 0
    Q[4, 1, 0] = INF                       # token 1: first row -Inf, then +Inf, then NaN
    D[4, 0, 0], D[4, 1, 0], D[4, 2, 0] = -0.5, 0.3, 0.0
    Q[5, 4, 0] = INF                       # token 4: every score -Inf
    D[5, :, 0] = -np.abs(D[5, :, 0]) - 0.1
    Q[6, 0, 0] = -INF                      # token 0: first score NaN (-Inf * 0), then +-Inf
    D[6, 0, 0] = 0.0
    D[6, 1:, 0] = np.where(np.abs(D[6, 1:, 0]) < 0.05, 0.2, D[6, 1:, 0])
    return Q, D, qm, dm                    # pair 7 (and beyond): finite


def _dev(x, device):
    return x.to(device) if isinstance(x, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(x)).to(device)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("dim", [128, 40, 1024])
def test_paired_nonfinite(device, dtype, dim):
    rng = np.random.default_rng(dim)
    B, Tq, Td = 9, 33 if dim == 40 else 12, 70
    Q, D, qm, dm = nonfinite_pairs(rng, B, Tq, Td, dim)
    Qt, Qo, bf = as_feature(Q, dtype)
    Dt, Do, _ = as_feature(D, dtype)
    s_o, a_o, p_o = oracle.paired_forward(Qo, Do, qm, dm, bf16=bf)
    args = torch.zeros(B, Tq, dtype=torch.int32, device=device)
    part = torch.zeros(B, Tq, dtype=torch.float32, device=device)
    S = torch.zeros(B, dtype=torch.float32, device=device)
    boundary.launch_paired_scan(args, part, _dev(Qt, device), _dev(Dt, device),
                                _dev(qm.astype(bool), device), _dev(dm.astype(bool), device), S)
    torch.cuda.synchronize()
    tol = FEATURE_TOL[dtype]
    assert np.array_equal(args.cpu().numpy(), a_o)
    assert_class_equal(part.cpu().numpy(), p_o, tol, "partial")
    assert_class_equal(S.cpu().numpy(), s_o, tol * Tq, "scores")
    # the constructed cases really exercise the rule
    assert np.isnan(s_o[0]) and a_o[0].tolist() == [1] * Tq
    assert (a_o[1] == 6).all() and np.isnan(s_o[1])
    assert np.isfinite(s_o[2]) and np.isnan(s_o[3]) and a_o[3, 7] == 0 and p_o[3, 7] == 0
    assert a_o[4, 1] == 2 and p_o[4, 1] == np.inf
    assert a_o[5, 4] == 1 and p_o[5, 4] == -np.inf and s_o[5] == -np.inf
    assert a_o[6, 0] == 1 and np.isnan(p_o[6, 0])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("order", ["always", "never"])
def test_candidates_nonfinite(device, dtype, order):
    rng = np.random.default_rng(3)
    Bq, Tq, Td, dim = 9, 12, 50, 128
    Q, G, qm, gm = nonfinite_pairs(rng, Bq, Tq, Td, dim)
    N, C = Bq, 6
    idx = rng.integers(1, N + 1, size=(Bq, C)).astype(np.int64)
    idx[:, 0] = np.arange(1, Bq + 1)         # every pattern reaches its own query
    idx[2, 1] = 0                            # invalid -> neg
    Qt, Qo, bf = as_feature(Q, dtype)
    Gt, Go, _ = as_feature(G, dtype)
    S_o, a_o, p_o = oracle.candidates_forward(Qo, Go, idx, qm, gm, -7.0, bf16=bf)
    args = torch.zeros(Bq, C, Tq, dtype=torch.int32, device=device)
    part = torch.zeros(Bq, C, Tq, dtype=torch.float32, device=device)
    S = torch.zeros(Bq, C, dtype=torch.float32, device=device)
    prev = boundary.candidates_grouping(order)
    try:
        boundary.launch_candidates_scan(args, part, _dev(Qt, device), _dev(Gt, device),
                                        _dev(idx, device), _dev(qm.astype(bool), device),
                                        _dev(gm.astype(bool), device), N, S, -7.0)
        torch.cuda.synchronize()
    finally:
        boundary.candidates_grouping(prev)
    tol = FEATURE_TOL[dtype]
    assert np.array_equal(args.cpu().numpy(), a_o)
    assert_class_equal(part.cpu().numpy(), p_o, tol, "partial")
    assert_class_equal(S.cpu().numpy(), S_o, tol * Tq, "scores")
    assert S_o[2, 1] == np.float32(-7.0)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("dim", [128, 256], ids=lambda d: f"d{d}")
def test_inbatch_nonfinite(device, dtype, dim):
    """dim 128: f16 / bf16 take the register-resident MFMA kernel (Tq <= 32), fp32
    the split-K kernel; dim 256: all three take the split-K kernel.  Query tokens
    and documents with non-finite first rows sit in several query groups."""
    rng = np.random.default_rng(17)
    Bq, Bd, Tq, Td = 40, 37, 24, 70
    Q = tokens(rng, (Bq, Tq, dim))
    D = tokens(rng, (Bd, Td, dim))
    qm = np.ones((Bq, Tq), np.uint8)
    dm = np.ones((Bd, Td), np.uint8)
    qm[5, 20:] = 0
    dm[3, :9] = 0
    D[3, 9, 11] = NAN                        # first valid row of document 3 is NaN
    D[7, 0, 0] = INF                         # first row of document 7 is +Inf at k = 0
    D[7, 1:, 0] = np.where(np.abs(D[7, 1:, 0]) < 0.05, 0.2, D[7, 1:, 0])
    D[12, 40, 2] = NAN                       # a NaN row in the middle: skipped
    dm[20, :] = 0                            # an empty document
    Q[1, 3, 0] = NAN                         # query 1 token 3 NaN (block 0)
    Q[33, 0, 0] = -INF                       # query 33 token 0 -Inf (block 1)
    Q[5, 22, 1] = NAN                        # a masked NaN token
    Qt, Qo, bf = as_feature(Q, dtype)
    Dt, Do, _ = as_feature(D, dtype)
    S_o, a_o = oracle.inbatch_forward(Qo, Do, qm, dm, bf16=bf)  # S (Bq, Bd), args (Bq, Bd, Tq)
    S = torch.zeros(Bq, Bd, dtype=torch.float32, device=device)
    args = torch.zeros(Bq, Bd, Tq, dtype=torch.int32, device=device)
    boundary.inbatch_device_scan(S, args, _dev(Qt, device), _dev(Dt, device),
                                 _dev(qm.astype(bool), device), _dev(dm.astype(bool), device))
    torch.cuda.synchronize()
    tol = FEATURE_TOL[dtype]
    assert np.array_equal(args.cpu().numpy(), a_o)
    assert_class_equal(S.cpu().numpy(), S_o, tol * Tq, "S")
    assert np.isnan(S_o[:, 3]).all() and (a_o[:, 3, :20] == 10).all()
    live = np.arange(Bd) != 20
    assert np.isnan(S_o[1, live]).all() and not np.isfinite(S_o[33, live]).any()
    assert np.isfinite(S_o[0, 12]) and S_o[0, 20] == 0.0 and S_o[1, 20] == 0.0


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_packed_nonfinite(device, dtype):
    """Single-query packed scan and the multi-query MFMA scan (every row valid, the
    first token of a document is its first row)."""
    rng = np.random.default_rng(23)
    lens = [40, 0, 33, 70, 1, 64]
    dim, Tq, nq = 128, 20, 5
    ntok = sum(lens)
    tok = tokens(rng, (ntok, dim))
    cu = np.concatenate([[1], 1 + np.cumsum(lens)]).astype(np.int32)
    tok[cu[0] - 1, 4] = NAN                   # document 0's first row NaN
    tok[cu[3] - 1 + 10, 4] = NAN              # document 3: a later NaN row, skipped
    Qm = tokens(rng, (nq, Tq, dim))
    Qm[2, 6, 0] = NAN                         # query 2 token 6 NaN
    Tt, To, bf = as_feature(tok, dtype)
    Qt, Qo, _ = as_feature(Qm, dtype)
    S_multi = torch.zeros(nq, len(lens), dtype=torch.float32, device=device)
    a_multi = torch.zeros(nq, len(lens), Tq, dtype=torch.int32, device=device)
    boundary.launch_packed_multi_scan(a_multi, S_multi, _dev(Qt, device), _dev(Tt, device),
                                      _dev(cu, device), None, max(lens))
    torch.cuda.synchronize()
    tol = FEATURE_TOL[dtype]
    for i in range(nq):
        s_o, a_o, p_o = oracle.packed_forward(Qo[i], To, cu, None, bf16=bf)
        s1 = torch.zeros(len(lens), dtype=torch.float32, device=device)
        a1 = torch.zeros(len(lens), Tq, dtype=torch.int32, device=device)
        boundary.launch_packed_scan(a1, None, _dev(Qt[i], device), _dev(Tt, device),
                                    _dev(cu, device), None, s1)
        torch.cuda.synchronize()
        for what, S_got, a_got in (("single", s1, a1), ("multi", S_multi[i], a_multi[i])):
            assert np.array_equal(a_got.cpu().numpy(), a_o), (what, i)
            assert_class_equal(S_got.cpu().numpy(), s_o, tol * Tq, f"{what} query {i}")
        assert np.isnan(s_o[0]) and np.isfinite(s_o[3]) == (i != 2)


def test_packed_multi_rejects_documents_longer_than_max_len(device):
    """A max_len below a document's length breaks the PackedSeq contract: that
    document's scores are NaN and its tapes 0 (never a truncated document's score);
    the other documents are unaffected."""
    rng = np.random.default_rng(29)
    lens = [10, 50, 20]
    dim, Tq, nq = 128, 16, 3
    tok = tokens(rng, (sum(lens), dim))
    cu = np.concatenate([[1], 1 + np.cumsum(lens)]).astype(np.int32)
    Qm = tokens(rng, (nq, Tq, dim))
    Tt, To, _ = as_feature(tok, torch.float16)
    Qt, Qo, _ = as_feature(Qm, torch.float16)
    S = torch.zeros(nq, 3, dtype=torch.float32, device=device)
    a = torch.full((nq, 3, Tq), 7, dtype=torch.int32, device=device)
    boundary.launch_packed_multi_scan(a, S, _dev(Qt, device), _dev(Tt, device), _dev(cu, device),
                                      None, 32)
    torch.cuda.synchronize()
    S, a = S.cpu().numpy(), a.cpu().numpy()
    assert np.isnan(S[:, 1]).all() and (a[:, 1] == 0).all()
    for i in range(nq):
        s_o, a_o, _ = oracle.packed_forward(Qo[i], To, cu, None)
        assert np.allclose(S[i, [0, 2]], s_o[[0, 2]], rtol=2e-3, atol=2e-3)
        assert np.array_equal(a[i, [0, 2]], a_o[[0, 2]])
