"""GPU: the reverse rules (src/rrule.jl) and the torch autograd binding of ``maxsim``.

Semantics are checked against a dense fp64 reference differentiated by torch
autograd on the CPU (src/dense.jl semantics: masked document tokens excluded
from the max, an empty max contributes 0, masked query tokens excluded from
the sum, ``normalize`` divides by max(count, 1)); the max picks the argmax
token, so its gradient is the reference's sparse pullback.  Features are
fp32 and random, so the dense argmax and the device tape agree; tolerance
1e-4 relative to the gradient's largest entry (the sums' own precision is
tested to 1e-5 in test_gpu_backward.py -- this file checks which terms are
summed and how they are scaled: a wrong mask, normalisation or cotangent
layout is an O(1) error).
"""
import numpy as np
import pytest
import torch

from helpers import tokens

import flashmaxsim as fm
from flashmaxsim import backward as bw

pytestmark = pytest.mark.gpu


def dense_scores(Q, D, qm, dm, normalize):
    """Q (B,Tq,dim) D (B,Td,dim) fp64 CPU; qm (B,Tq) dm (B,Td) bool -> (B,)."""
    sims = Q @ D.transpose(1, 2).contiguous()
    sims = sims.masked_fill(~dm[:, None, :], float("-inf"))
    mx = sims.max(-1).values
    mx = torch.where(torch.isinf(mx), torch.zeros_like(mx), mx) * qm
    s = mx.sum(-1)
    if normalize:
        s = s / qm.sum(-1).clamp(min=1)
    return s


def close(got, want, what):
    g = got.detach().double().cpu()
    w = want.detach().double().cpu()
    scale = float(w.abs().max()) or 1.0
    err = float((g - w).abs().max())
    assert err <= 1e-4 * scale, (what, err, scale)


def _feat(rng, shape, device):
    return torch.from_numpy(tokens(rng, shape)).to(device)


@pytest.mark.parametrize("normalize", [False, True])
def test_autograd_paired_matches_dense(device, normalize):
    rng = np.random.default_rng(1)
    B, Tq, Td, dim = 6, 9, 23, 64
    Q = _feat(rng, (B, Tq, dim), device).requires_grad_(True)
    D = _feat(rng, (B, Td, dim), device).requires_grad_(True)
    qm = torch.from_numpy(rng.random((B, Tq)) < 0.8).to(device)
    dm = torch.from_numpy(rng.random((B, Td)) < 0.7).to(device)
    dm[-1] = False  # an empty document: score 0, no gradient
    w = torch.randn(B, device=device, generator=torch.Generator(device).manual_seed(0))
    s = fm.maxsim(Q, D, qm, dm, normalize=normalize)
    (s * w).sum().backward()
    Qr = Q.detach().double().cpu().requires_grad_(True)
    Dr = D.detach().double().cpu().requires_grad_(True)
    sr = dense_scores(Qr, Dr, qm.cpu(), dm.cpu(), normalize)
    (sr * w.double().cpu()).sum().backward()
    close(s, sr, "scores")
    close(Q.grad, Qr.grad, "dQ")
    close(D.grad, Dr.grad, "dD")
    assert float(D.grad[-1].abs().max()) == 0.0


def test_autograd_inbatch_and_candidates_match_dense(device):
    rng = np.random.default_rng(2)
    Bq, Bd, Tq, Td, dim = 5, 7, 8, 19, 32
    Q = _feat(rng, (Bq, Tq, dim), device).requires_grad_(True)
    D = _feat(rng, (Bd, Td, dim), device).requires_grad_(True)
    qm = torch.from_numpy(rng.random((Bq, Tq)) < 0.85).to(device)
    W = torch.randn(Bq, Bd, device=device, generator=torch.Generator(device).manual_seed(1))
    S = fm.maxsim(Q, D, qm, None, fm.InBatch(), normalize=True)  # (Bq, Bd)
    (S * W).sum().backward()
    Qr = Q.detach().double().cpu().requires_grad_(True)
    Dr = D.detach().double().cpu().requires_grad_(True)
    ii, jj = np.meshgrid(np.arange(Bq), np.arange(Bd), indexing="ij")
    Sr = dense_scores(Qr[ii.ravel()], Dr[jj.ravel()], qm.cpu()[ii.ravel()],
                      torch.ones(Bq * Bd, Td, dtype=torch.bool), True).reshape(Bq, Bd)
    (Sr * W.double().cpu()).sum().backward()
    close(S, Sr, "in-batch scores")
    close(Q.grad, Qr.grad, "in-batch dQ")
    close(D.grad, Dr.grad, "in-batch dD")

    # candidates: invalid indices score `neg` and carry no gradient
    N, C = 6, 4
    Q2 = _feat(rng, (Bq, Tq, dim), device).requires_grad_(True)
    G = _feat(rng, (N, Td, dim), device).requires_grad_(True)
    idx = torch.from_numpy(rng.integers(1, N + 1, size=(Bq, C))).to(device)
    idx[0, 1] = 0
    idx[2, 3] = N + 5
    Wc = torch.randn(Bq, C, device=device, generator=torch.Generator(device).manual_seed(2))
    Sc = fm.maxsim(Q2, G, idx, normalize=False)
    (Sc * Wc).sum().backward()
    Q2r = Q2.detach().double().cpu().requires_grad_(True)
    Gr = G.detach().double().cpu().requires_grad_(True)
    ic = idx.cpu().numpy()
    valid = (ic >= 1) & (ic <= N)
    bb, cc = np.nonzero(valid)
    sv = dense_scores(Q2r[bb], Gr[ic[bb, cc] - 1], torch.ones(len(bb), Tq, dtype=torch.bool),
                      torch.ones(len(bb), Td, dtype=torch.bool), False)
    (sv * Wc.double().cpu()[bb, cc]).sum().backward()
    assert float(Sc.detach()[0, 1]) == -1.0e4 and float(Sc.detach()[2, 3]) == -1.0e4
    close(Q2.grad, Q2r.grad, "candidates dQ")
    close(G.grad, Gr.grad, "candidates dG")


def test_rrule_packed_and_varlen_match_pullbacks(device):
    rng = np.random.default_rng(3)
    dim, Tq = 32, 6
    lens = [4, 0, 9, 1]
    q = _feat(rng, (Tq, dim), device)
    P = fm.PackedSeq(torch.from_numpy(np.concatenate([tokens(rng, (n, dim)) for n in lens])),
                     torch.from_numpy(np.concatenate([[1], 1 + np.cumsum(lens)]).astype(np.int32))
                     ).to(device)
    qm = torch.tensor([1, 1, 0, 1, 1, 1], dtype=torch.bool, device=device)
    cfg = fm.MaxSim(torch.float32, normalize=True)
    y, pb = fm.rrule(cfg, q, P, qm)
    Dl = torch.randn(len(lens), device=device, generator=torch.Generator(device).manual_seed(3))
    dq, dP, dm_ = pb(Dl)
    assert dm_ is None
    _, tape = fm.packed_forward(q, P, qm)
    eq, eP = bw.packed_pullback(Dl, q, P, qm, tape, 1.0 / 5)
    torch.cuda.synchronize()
    assert torch.equal(dq, eq)
    close(dP, eP, "packed dP")
    # varlen, normalised: inv_n[n] = 1 / max(Tq_n, 1)
    Qp = fm.PackedSeq(torch.from_numpy(tokens(rng, (7, dim))),
                      torch.tensor([1, 3, 3, 8], dtype=torch.int32)).to(device)
    Dp = fm.PackedSeq(torch.from_numpy(tokens(rng, (9, dim))),
                      torch.tensor([1, 5, 7, 10], dtype=torch.int32)).to(device)
    y2, pb2 = fm.rrule(cfg, Qp, Dp)
    d2 = torch.randn(3, device=device, generator=torch.Generator(device).manual_seed(4))
    gQ, gD = pb2(d2)
    _, t2 = fm.varlen_forward(Qp, Dp)
    inv = torch.tensor([1 / 2, 1.0, 1 / 5], device=device)
    eQ, eD = bw.varlen_pullback(d2, Qp, Dp, t2, inv)
    close(gQ, eQ, "varlen dQ")
    close(gD, eD, "varlen dD")
    assert torch.allclose(y2, fm.varlen_forward(Qp, Dp)[0] * inv)


def test_autograd_packed_tokens_gradient(device):
    """A PackedSeq argument's gradient lands on its token array."""
    rng = np.random.default_rng(4)
    dim, Tq, lens = 16, 5, [3, 6]
    q = _feat(rng, (Tq, dim), device).requires_grad_(True)
    tok = torch.from_numpy(np.concatenate([tokens(rng, (n, dim)) for n in lens])).to(device)
    tok.requires_grad_(True)
    P = fm.PackedSeq(tok, torch.tensor([1, 4, 10], dtype=torch.int32, device=device), max_len=6)
    s = fm.maxsim(q, P)
    s.sum().backward()
    _, tape = fm.packed_forward(q.detach(), fm.PackedSeq(tok.detach(), P.cu, max_len=6))
    eq, eP = bw.packed_pullback(torch.ones(2, device=device), q.detach(),
                                fm.PackedSeq(tok.detach(), P.cu, max_len=6), None, tape)
    close(q.grad, eq, "dq")
    close(tok.grad, eP, "dP")


def test_rrule_cotangent_rules_and_int8(device):
    rng = np.random.default_rng(5)
    Q = _feat(rng, (3, 4, 16), device)
    D = _feat(rng, (3, 5, 16), device)
    cfg = fm.MaxSim(torch.float32)
    y, pb = fm.rrule(cfg, Q, D)
    z = pb(None)  # ZeroTangent
    assert all(float(t.abs().max()) == 0.0 for t in z[:2])
    with pytest.raises(fm.DimensionMismatch):
        pb(torch.ones(4, device=device))
    with pytest.raises(fm.ArgumentError):
        pb(1.0)  # scalar cotangent for a 3-element score
    q1, d1 = Q[0], D[0]
    y1, pb1 = fm.rrule(cfg, q1, d1)
    g1 = pb1(2.0)  # a scalar cotangent is fine for the length-1 pair score
    e1 = bw.pair_pullback(2.0, q1, d1, None, fm.pair_forward(q1, d1)[1])
    assert torch.equal(g1[0], e1[0])
    # INT8 is forward-only
    idx8 = fm.quantize_int8_symmetric(D)
    y8, pb8 = fm.rrule(cfg, Q, idx8)
    assert pb8(None) == (None, None)
    with pytest.raises(fm.ArgumentError):
        pb8(torch.ones_like(y8))
