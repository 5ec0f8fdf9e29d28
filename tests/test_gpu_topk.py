"""GPU: per-row top-k (fms_topk; no reference counterpart -- the caller's
stable partialsortperm(rev = true), README.md:132) against the CPU oracle.

Bit-exact: the same values (NaN where the oracle has a NaN; the kernel writes
one canonical NaN) and the same 1-based indices, at row widths that are not
multiples of the 1024-entry tile, k from 1 to the 1024 maximum and k = ncols,
heavy ties (three levels, all equal), NaN / +-Inf / signed zeros -- in rows
short enough for one workgroup and long enough for the two-stage split, where
ties cross slice boundaries -- and the score matrices the multi-query packed
and in-batch scans write.
"""
import numpy as np
import pytest
import torch

import oracle

import flashmaxsim as fm

pytestmark = pytest.mark.gpu


def _check(got, S, k):
    gv, gi = (t.cpu().numpy() for t in got)
    ev, ei = oracle.topk(S, k)
    gv, gi = gv.reshape(ev.shape), gi.reshape(ei.shape)
    assert np.array_equal(gi, ei)
    nan = np.isnan(ev)
    assert np.array_equal(np.isnan(gv), nan)
    assert np.array_equal(gv[~nan].view(np.uint32), ev[~nan].view(np.uint32))


@pytest.mark.parametrize("nrows,ncols,k", [
    (1, 1, 1), (3, 5, 5), (7, 1000, 1), (2, 1025, 64), (64, 20000, 100), (5, 3000, 1024),
    (1, 100_000, 10), (513, 512, 16), (2, 700, 700),
])
def test_topk_random_rows(device, nrows, ncols, k):
    rng = np.random.default_rng(nrows * 7 + ncols + k)
    S = rng.standard_normal((nrows, ncols)).astype(np.float32)
    print(f"topk random nrows={nrows} ncols={ncols} k={k}", flush=True)
    _check(fm.topk(torch.from_numpy(S).to(device), k), S, k)


@pytest.mark.parametrize("ncols", [4099, 40000])  # one stage; two stages (ties across slices)
@pytest.mark.parametrize("kind", ["three_levels", "all_equal", "special"])
def test_topk_ties_and_special_values(device, kind, ncols):
    rng = np.random.default_rng(5)
    nrows, k = 4, 300
    if kind == "three_levels":
        S = rng.integers(0, 3, size=(nrows, ncols)).astype(np.float32)
    elif kind == "all_equal":
        S = np.full((nrows, ncols), -1.0e4, np.float32)  # e.g. a row of invalid candidates
    else:
        S = rng.standard_normal((nrows, ncols)).astype(np.float32)
        picks = rng.integers(0, ncols, size=(nrows, 60))
        vals = np.array([np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0], np.float32)
        for r in range(nrows):
            S[r, picks[r]] = vals[rng.integers(0, len(vals), 60)]
    print(f"topk {kind} ncols={ncols}", flush=True)
    _check(fm.topk(torch.from_numpy(S).to(device), k), S, k)


def test_topk_vector_and_validation(device):
    rng = np.random.default_rng(6)
    s = rng.standard_normal(333).astype(np.float32)
    v, i = fm.topk(torch.from_numpy(s).to(device), 20)
    assert v.shape == (20,) and i.shape == (20,)
    _check((v, i), s[None, :], 20)
    v0, i0 = fm.topk(torch.from_numpy(s).to(device), 0)
    assert v0.shape == (0,)
    with pytest.raises(fm.ArgumentError):
        fm.topk(torch.from_numpy(s).to(device), 334)
    with pytest.raises(fm.UnsupportedError):
        fm.topk(torch.zeros(2, 2000, device=device), 1025)


def test_topk_of_multi_query_packed_scores(device):
    """Retrieval: the multi-query packed scan's (nq, B) scores, then the best 10
    documents per query."""
    rng = np.random.default_rng(7)
    dim, nq, Tq = 128, 40, 24
    lens = rng.integers(0, 90, size=300)
    tok = torch.from_numpy(rng.standard_normal((int(lens.sum()), dim)).astype(np.float32))
    cu = torch.from_numpy(np.concatenate([[1], 1 + np.cumsum(lens)]).astype(np.int32))
    P = fm.PackedSeq(tok.to(torch.bfloat16), cu).to(device)
    Q = torch.from_numpy(rng.standard_normal((nq, Tq, dim)).astype(np.float32)).to(
        device, torch.bfloat16)
    S, _ = fm.packed_multi_forward(Q, P)
    got = fm.topk(S, 10)
    _check(got, S.cpu().numpy(), 10)
