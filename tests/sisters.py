"""Near-duplicate ("sister") documents whose MaxSim gap is smaller than one
Float16 ulp of the score (test_edge_cases.jl:26-107).

A document whose first Tq tokens are exact copies of the query scores about
Tq; its sister perturbs token 1 towards an orthogonal direction by a mix
weight alpha and re-normalises, which lowers the score by a few 1e-3 -- less
than eps(Float16(32)) = 0.03125.  Scores must come back in fp32 to keep the
two apart.  Everything here is float64 numpy; callers round to fp16.
"""
from __future__ import annotations

import numpy as np


def l2rows(x):
    """Token rows scaled to unit length (test_edge_cases.jl:3 uses floatmin as the floor)."""
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + np.finfo(x.dtype).tiny)


def sister_token(dtok, noise, alpha):
    """test_edge_cases.jl:6-12: mix in the part of `noise` orthogonal to `dtok`."""
    n = noise - dtok * np.dot(noise, dtok)
    n = n / np.sqrt(np.dot(n, n))
    v = (1.0 - alpha) * dtok + alpha * n
    return v / np.sqrt(np.dot(v, v))


def maxsim_dense(q, d):
    """Float64 MaxSim of (Tq, dim) against (Td, dim), all tokens valid."""
    return float((q @ d.T).max(axis=1).sum())


def sister_pair(seed=2026, dim=128, Tq=32, Td=40, alpha=0.08):
    """(q, d, sister) float64 with d[:Tq] = q (test_edge_cases.jl:26-37)."""
    rng = np.random.default_rng(seed)
    q = l2rows(rng.standard_normal((Tq, dim)))
    d = l2rows(rng.standard_normal((Td, dim)))
    d[:Tq] = q
    sis = d.copy()
    sis[0] = sister_token(d[0], rng.standard_normal(dim), alpha)
    return q, d, sis


def sister_ladder(seed=2027, dim=128, Tq=32, Td=32, alphas=(0.0, 0.04, 0.08, 0.12, 0.16)):
    """(q, [docs]) float64: one base document and sisters of rising alpha
    (test_edge_cases.jl:87-99); their exact scores fall with alpha."""
    rng = np.random.default_rng(seed)
    q = l2rows(rng.standard_normal((Tq, dim)))
    d0 = l2rows(rng.standard_normal((Td, dim)))
    d0[:Tq] = q
    docs = []
    for a in alphas:
        d = d0.copy()
        if a > 0:
            d[0] = sister_token(d0[0], rng.standard_normal(dim), a)
        docs.append(d)
    return q, docs


F16_ULP_AT_32 = float(np.spacing(np.float16(32)))  # eps(Float16(32)) = 0.03125


def f16_ulp(x: float) -> float:
    return float(np.spacing(np.float16(x)))


def spearman(a, b) -> float:
    """test_int8.jl:1-14: Pearson correlation of the ranks (ties broken by position)."""
    def ranks(x):
        x = np.asarray(x, np.float64).ravel()
        r = np.empty(x.size)
        r[np.argsort(x, kind="stable")] = np.arange(1, x.size + 1)
        return r
    ra, rb = ranks(a), ranks(b)
    ra -= ra.mean()
    rb -= rb.mean()
    na, nb = np.sqrt((ra * ra).sum()), np.sqrt((rb * rb).sum())
    if na == 0 or nb == 0:
        return 1.0
    return float((ra * rb).sum() / (na * nb))


def topk_overlap(a, b, k) -> float:
    """test_int8.jl:16-20: shared fraction of the two top-k sets."""
    pa = np.argsort(-np.asarray(a, np.float64).ravel(), kind="stable")[:k]
    pb = np.argsort(-np.asarray(b, np.float64).ravel(), kind="stable")[:k]
    return len(set(pa.tolist()) & set(pb.tolist())) / k
