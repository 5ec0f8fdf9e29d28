"""Pins the backward half of the CPU oracle (oracle/fms_oracle.c, *_backward) before
it is trusted as the checker of the HIP pullback kernels.

The reference's pullbacks (src/backward_pair.jl, src/backward_layouts.jl,
src/packed.jl:361-377, :424-442) scatter the cotangent along the forward's argmax
tape: dQ[:, t] += delta * D[:, u] and dD[:, u] += delta * Q[:, t] for every valid
(t, u = args[t]).  Each oracle function is pinned by
  * an independent numpy implementation (np.add.at scatters, written here),
  * finite differences of the fp64 dense forward score (src/dense.jl semantics:
    the score is piecewise linear in Q and D, so a small step along a random
    direction changes it by exactly <grad, step> while no argmax moves),
  * linearity in the cotangent and the delta == 0 / masked-token / empty-tape
    known answers (backward_pair.jl:21-29),
  * layout invariants (diagonal in-batch == paired, identity candidates ==
    paired, single-document packed == pair, equal-length varlen == paired).
"""
import numpy as np
import pytest

import oracle
from helpers import tokens


def np_pair_backward(q, d, qm, tape, delta):
    """dq (Tq,dim), dd (Td,dim) for one pair, fp64, by np.add.at."""
    q = q.astype(np.float64)
    d = d.astype(np.float64)
    dq = np.zeros_like(q)
    dd = np.zeros_like(d)
    Td = d.shape[0]
    valid = (tape >= 1) & (tape <= Td)
    if qm is not None:
        valid &= qm.astype(bool)
    t = np.nonzero(valid)[0]
    u = tape[t] - 1
    dq[t] = delta * d[u]
    np.add.at(dd, u, delta * q[t])
    return dq, dd


def rand_case(rng, B, Tq, Td, dim, dtype=np.float32):
    Q = tokens(rng, (B, Tq, dim)).astype(dtype)
    D = tokens(rng, (B, Td, dim)).astype(dtype)
    qm = rng.random((B, Tq)) < 0.85
    dm = rng.random((B, Td)) < 0.8
    return Q, D, qm, dm


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_paired_backward_matches_numpy(dtype):
    rng = np.random.default_rng(1)
    B, Tq, Td, dim = 5, 9, 13, 24
    Q, D, qm, dm = rand_case(rng, B, Tq, Td, dim, dtype)
    _, args, _ = oracle.paired_forward(Q, D, qm, dm)
    Delta = rng.standard_normal(B)
    inv = 1.0 / np.maximum(qm.sum(1), 1)
    dQ, dD = oracle.paired_backward(Q, D, args, Delta, inv, qm)
    for b in range(B):
        eq, ed = np_pair_backward(Q[b], D[b], qm[b], args[b], Delta[b] * inv[b])
        np.testing.assert_allclose(dQ[b], eq, rtol=1e-12, atol=1e-14)
        np.testing.assert_allclose(dD[b], ed, rtol=1e-12, atol=1e-14)
    # masked query tokens and empty tape entries give zero rows of dQ
    assert (dQ[~qm] == 0).all()
    assert (dQ[args == 0] == 0).all()


def test_backward_is_the_gradient_of_the_dense_score():
    """Finite differences of the fp64 dense forward (src/dense.jl:26-56)."""
    rng = np.random.default_rng(2)
    Tq, Td, dim = 7, 11, 16
    q = tokens(rng, (Tq, dim)).astype(np.float64)
    d = tokens(rng, (Td, dim)).astype(np.float64)
    qm = np.array([1, 1, 0, 1, 1, 1, 0], bool)
    s0, args = oracle.dense_pair_f64(q, d, qm)
    dQ, dD = oracle.paired_backward(q[None], d[None], args[None], np.array([1.0]), None, qm[None])
    eps = 1e-7
    for _ in range(4):
        eq = rng.standard_normal(q.shape)
        ed = rng.standard_normal(d.shape)
        s1, a1 = oracle.dense_pair_f64(q + eps * eq, d + eps * ed, qm)
        assert (a1 == args).all()  # the step moves no argmax
        fd = (s1 - s0) / eps
        an = (dQ[0] * eq).sum() + (dD[0] * ed).sum()
        assert abs(fd - an) <= 1e-6 * max(1.0, abs(an)), (fd, an)


def test_backward_linear_in_cotangent_and_zero_delta():
    rng = np.random.default_rng(3)
    B, Tq, Td, dim = 4, 6, 9, 8
    Q, D, qm, dm = rand_case(rng, B, Tq, Td, dim)
    _, args, _ = oracle.paired_forward(Q, D, qm, dm)
    d1, d2 = rng.standard_normal(B), rng.standard_normal(B)
    a = oracle.paired_backward(Q, D, args, d1, None, qm)
    b = oracle.paired_backward(Q, D, args, d2, None, qm)
    c = oracle.paired_backward(Q, D, args, 2.0 * d1 + d2, None, qm)
    for x, y, z in zip(a, b, c):
        np.testing.assert_allclose(z, 2.0 * x + y, rtol=1e-12, atol=1e-13)
    z = oracle.paired_backward(Q, D, args, np.zeros(B), None, qm)
    assert all((v == 0).all() for v in z)  # backward_pair.jl:21


def test_inbatch_backward_matches_numpy_and_paired():
    rng = np.random.default_rng(4)
    Bq, Bd, Tq, Td, dim = 4, 5, 6, 10, 12
    Q = tokens(rng, (Bq, Tq, dim))
    D = tokens(rng, (Bd, Td, dim))
    qm = rng.random((Bq, Tq)) < 0.8
    dm = rng.random((Bd, Td)) < 0.8
    _, args = oracle.inbatch_forward(Q, D, qm, dm)  # args (Bq, Bd, Tq)
    Delta = rng.standard_normal((Bq, Bd))
    inv = 1.0 / np.maximum(qm.sum(1), 1)
    dQ, dD = oracle.inbatch_backward(Q, D, args, Delta, inv, qm)
    eQ = np.zeros_like(dQ)
    eD = np.zeros_like(dD)
    for i in range(Bq):
        for j in range(Bd):
            a, b = np_pair_backward(Q[i], D[j], qm[i], args[i, j], Delta[i, j] * inv[i])
            eQ[i] += a
            eD[j] += b
    np.testing.assert_allclose(dQ, eQ, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(dD, eD, rtol=1e-12, atol=1e-13)
    # only the diagonal cotangent: the paired pullback of pairs (i, i)
    B = 4
    Dd = D[:B]
    _, pa, _ = oracle.paired_forward(Q, Dd, qm, dm[:B])
    diag = np.zeros((Bq, B))
    dv = rng.standard_normal(B)
    diag[np.arange(B), np.arange(B)] = dv
    _, a_ib = oracle.inbatch_forward(Q, Dd, qm, dm[:B])
    assert (a_ib[np.arange(B), np.arange(B)] == pa).all()
    iQ, iD = oracle.inbatch_backward(Q, Dd, a_ib, diag, None, qm)
    pQ, pD = oracle.paired_backward(Q, Dd, pa, dv, None, qm)
    np.testing.assert_allclose(iQ, pQ, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(iD, pD, rtol=1e-12, atol=1e-13)


def test_candidates_backward_matches_numpy_and_paired():
    rng = np.random.default_rng(5)
    B, C, N, Tq, Td, dim = 3, 5, 6, 7, 9, 10
    Q = tokens(rng, (B, Tq, dim))
    G = tokens(rng, (N, Td, dim))
    qm = rng.random((B, Tq)) < 0.85
    dm = rng.random((N, Td)) < 0.8
    idxs = rng.integers(1, N + 1, size=(B, C))
    idxs[0, 1] = 0
    idxs[2, 3] = N + 4  # out of range: no contribution
    idxs[1, :2] = 3     # a repeated document within one query
    _, args, _ = oracle.candidates_forward(Q, G, idxs, qm, dm)
    Delta = rng.standard_normal((B, C))
    inv = 1.0 / np.maximum(qm.sum(1), 1)
    dQ, dG = oracle.candidates_backward(Q, G, idxs, args, Delta, inv, qm)
    eQ = np.zeros_like(dQ)
    eG = np.zeros_like(dG)
    for b in range(B):
        for c in range(C):
            j = idxs[b, c]
            if not 1 <= j <= N:
                continue
            a, g = np_pair_backward(Q[b], G[j - 1], qm[b], args[b, c], Delta[b, c] * inv[b])
            eQ[b] += a
            eG[j - 1] += g
    np.testing.assert_allclose(dQ, eQ, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(dG, eG, rtol=1e-12, atol=1e-13)
    # identity candidates (C = 1, idx b+1) == paired
    ident = np.arange(1, B + 1)[:, None]
    _, a1, _ = oracle.candidates_forward(Q, G[:B], ident, qm, dm[:B])
    d1 = rng.standard_normal((B, 1))
    cQ, cG = oracle.candidates_backward(Q, G[:B], ident, a1, d1, None, qm)
    pQ, pD = oracle.paired_backward(Q, G[:B], a1[:, 0], d1[:, 0], None, qm)
    np.testing.assert_allclose(cQ, pQ, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(cG, pD, rtol=1e-12, atol=1e-13)


def test_packed_and_varlen_backward_match_numpy_and_pair():
    rng = np.random.default_rng(6)
    Tq, dim = 6, 12
    lens = [5, 0, 9, 1, 12]
    q = tokens(rng, (Tq, dim))
    docs = [tokens(rng, (n, dim)) for n in lens]
    tok = np.concatenate(docs, 0)
    cu = np.concatenate([[1], 1 + np.cumsum(lens)]).astype(np.int32)
    qm = np.array([1, 1, 0, 1, 1, 1], bool)
    _, args, _ = oracle.packed_forward(q, tok, cu, qm)  # (B, Tq)
    Delta = rng.standard_normal(len(lens))
    dq, dP = oracle.packed_backward(q, tok, cu, args, Delta, 0.25, qm)
    eq = np.zeros_like(dq)
    eP = np.zeros_like(dP)
    for b, n in enumerate(lens):
        a = cu[b] - 1
        x, y = np_pair_backward(q, tok[a:a + n], qm, args[b], Delta[b] * 0.25)
        eq += x
        eP[a:a + n] += y
    np.testing.assert_allclose(dq, eq, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(dP, eP, rtol=1e-12, atol=1e-13)
    # varlen with equal lengths == paired
    B, Lq, Ld = 3, 4, 6
    Q = tokens(rng, (B, Lq, dim))
    D = tokens(rng, (B, Ld, dim))
    _, pa, _ = oracle.paired_forward(Q, D)
    cu_q = (1 + Lq * np.arange(B + 1)).astype(np.int32)
    cu_d = (1 + Ld * np.arange(B + 1)).astype(np.int32)
    _, va = oracle.varlen_forward(Q.reshape(B * Lq, dim), D.reshape(B * Ld, dim), cu_q, cu_d)[:2]
    assert (va == pa).all()
    dv = rng.standard_normal(B)
    iv = rng.random(B)
    vQ, vD = oracle.varlen_backward(Q.reshape(B * Lq, dim), D.reshape(B * Ld, dim), cu_q, cu_d,
                                    va, dv, iv)
    pQ, pD = oracle.paired_backward(Q, D, pa, dv, iv)
    np.testing.assert_allclose(vQ, pQ.reshape(B * Lq, dim), rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(vD, pD.reshape(B * Ld, dim), rtol=1e-12, atol=1e-13)
