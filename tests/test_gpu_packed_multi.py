"""GPU: the multi-query packed scan (an extension with no reference method).

Row i of ``packed_multi_forward(Q, P)`` must equal the single-query packed scan
of query i (the reference's ``maxsim(q, P)`` path) and the CPU oracle on the
same inputs: fp16/bf16 scores within 2e-3 relative, fp32 within 1e-5; tapes
equal except at near-ties within that tolerance.  Shapes: a query count that
is not a multiple of the kernel's 32-query block, Lq = 24 with a random
qmask, documents of length 0, 1, 31, 32, 33 and ColPali-like 700..1100, at
dims 128, 96, 64 and 32 (the MFMA kernel's 8, 6, 4 and 2 k-blocks), Lq = 40 and
70 (query tiles of 32); dim 48 takes the per-query fallback.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import FEATURE_TOL, as_feature, assert_scores, assert_tape, tokens, widened

import flashmaxsim as fm

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16, torch.float32]
DT_ID = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}


def _case(rng, dtype, dim, nq, Tq, lens, device):
    Qt, Qo, bf = as_feature(tokens(rng, (nq, Tq, dim)), dtype)
    tt, to, _ = as_feature(np.concatenate([tokens(rng, (n, dim)) for n in lens], 0), dtype)
    cu = np.concatenate([[1], 1 + np.cumsum(lens)]).astype(np.int32)
    qm = rng.random((nq, Tq)) < 0.9
    P = fm.PackedSeq(tt, torch.from_numpy(cu)).to(device)
    return Qt.to(device), Qo, bf, P, to, cu, qm


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("case", ["edges", "colpali", "edges_d64", "edges_d96", "colpali_d32",
                                  "edges_t40", "colpali_t70"])
def test_packed_multi_matches_single_and_oracle(device, dtype, case):
    rng = np.random.default_rng({"edges": 61, "colpali": 62, "edges_d64": 64, "edges_d96": 65,
                                 "colpali_d32": 66, "edges_t40": 67, "colpali_t70": 68}[case])
    dim = {"edges_d64": 64, "edges_d96": 96, "colpali_d32": 32}.get(case, 128)
    Tq_over = {"edges_t40": 40, "colpali_t70": 70}.get(case)
    case = case.split("_")[0]
    if case == "edges":
        nq, Tq, lens = 40, 24, [5, 0, 1, 31, 32, 33, 64, 65, 0, 200, 17]
    else:
        nq, Tq, lens = 33, 24, list(rng.integers(700, 1101, size=9))
    Tq = Tq_over or Tq
    Q, Qo, bf, P, to, cu, qm = _case(rng, dtype, dim, nq, Tq, lens, device)
    qmt = torch.from_numpy(qm).to(device)
    S, args = fm.packed_multi_forward(Q, P, qmt)
    torch.cuda.synchronize()
    tol = FEATURE_TOL[dtype]
    tf = widened(to, bf)
    for i in range(nq):
        s1, a1 = fm.packed_forward(Q[i], P, qmt[i])
        s_o, a_o, _ = oracle.packed_forward(Qo[i], to, cu, qm[i].astype(np.uint8), bf16=bf)
        assert_scores(S[i].cpu(), s_o, tol, what=f"query {i} vs oracle")
        assert_scores(S[i].cpu(), s1.cpu(), tol, what=f"query {i} vs single-query scan")
        qf = widened(Qo[i], bf)
        sims = lambda idx: tf[cu[idx[0]] - 1: cu[idx[0] + 1] - 1] @ qf[idx[1]]
        assert_tape(args[i].cpu().numpy(), a_o, sims, tol, what=f"query {i} tape")
    for b, n in enumerate(lens):
        if n == 0:
            assert (S[:, b].cpu() == 0).all() and (args[:, b].cpu() == 0).all()


def test_packed_multi_fallback_shape_and_api(device):
    """dim 48 (no MFMA path) makes one packed scan per query: bit-identical rows."""
    rng = np.random.default_rng(63)
    Q, Qo, bf, P, to, cu, qm = _case(rng, torch.float16, 48, 5, 7, [3, 0, 9, 40], device)
    S, args = fm.packed_multi_forward(Q, P)
    for i in range(5):
        s1, a1 = fm.packed_forward(Q[i], P)
        assert torch.equal(S[i], s1) and torch.equal(args[i], a1)
    # maxsim dispatch: a 3-D query against a PackedSeq, normalised per query
    qmt = torch.from_numpy(qm).to(device)
    Sn = fm.maxsim(Q, P, qmt, normalize=True)
    Sr, _ = fm.packed_multi_forward(Q, P, qmt)
    cnt = qmt.sum(1).clamp(min=1).float()
    assert torch.allclose(Sn, Sr / cnt[:, None], rtol=1e-6, atol=0)
    # empty batches
    S0, a0 = fm.packed_multi_forward(Q[:0], P)
    assert S0.shape == (0, 4) and a0.shape == (0, 4, 7)


def test_packed_multi_autograd_matches_per_query(device):
    rng = np.random.default_rng(64)
    Q, Qo, bf, P, to, cu, qm = _case(rng, torch.float32, 32, 3, 5, [4, 7, 0, 2], device)
    Qg = Q.clone().requires_grad_(True)
    tok = P.tokens.clone().requires_grad_(True)
    Pg = fm.PackedSeq(tok, P.cu, P.max_len)
    W = torch.randn(3, 4, device=device, generator=torch.Generator(device).manual_seed(5))
    (fm.maxsim(Qg, Pg) * W).sum().backward()
    dQ = torch.zeros_like(Q)
    dP = torch.zeros_like(P.tokens)
    for i in range(3):
        q = Q[i].clone().requires_grad_(True)
        t = P.tokens.clone().requires_grad_(True)
        (fm.maxsim(q, fm.PackedSeq(t, P.cu, P.max_len)) * W[i]).sum().backward()
        dQ[i] = q.grad
        dP += t.grad
    assert torch.allclose(Qg.grad, dQ, rtol=1e-5, atol=1e-6)
    assert torch.allclose(tok.grad, dP, rtol=1e-5, atol=1e-6)
