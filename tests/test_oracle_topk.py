"""CPU: pinning the oracle's per-row top-k (oracle.topk).

Top-k has no counterpart in the reference (ranking is the caller's job,
README.md:132), so there are no golden vectors; the oracle is pinned by
independent routes:
  - numpy's stable argsort of the negated scores (a library sort) on data
    without NaN or signed zeros, with heavy ties -- equal scores must come out
    by smaller index, the stable reverse sort Julia's partialsortperm gives;
  - brute force on tiny rows: the top-k set is the k largest and every
    returned entry outranks every entry left out;
  - Julia's isless on the cases a plain `<` leaves open, written out by hand
    from its documented rules (NaN above +Inf, -0.0 below +0.0).
"""
import numpy as np
import pytest

import oracle


def _numpy_topk(S, k):
    order = np.argsort(-S, axis=1, kind="stable")[:, :k]
    return np.take_along_axis(S, order, 1), (order + 1).astype(np.int32)


@pytest.mark.parametrize("nrows,ncols,k,levels", [
    (3, 50, 10, 5), (4, 1000, 100, 7), (2, 257, 257, 3), (5, 64, 1, 2), (1, 3000, 1024, 40),
])
def test_oracle_topk_matches_stable_numpy_sort(nrows, ncols, k, levels):
    rng = np.random.default_rng(ncols + k)
    S = (rng.integers(1, levels + 1, size=(nrows, ncols)) * 0.25 - 1.1).astype(np.float32)
    S[:, ::7] = rng.standard_normal((nrows, len(range(0, ncols, 7)))).astype(np.float32)
    v, i = oracle.topk(S, k)
    ev, ei = _numpy_topk(S, k)
    assert np.array_equal(v, ev)
    assert np.array_equal(i, ei)


def test_oracle_topk_brute_force_tiny():
    rng = np.random.default_rng(11)
    for _ in range(200):
        n = int(rng.integers(1, 9))
        k = int(rng.integers(0, n + 1))
        s = rng.integers(-2, 3, size=n).astype(np.float32)
        v, i = oracle.topk(s[None, :], k)
        picked = set((i[0] - 1).tolist())
        assert len(picked) == k
        for a in picked:  # every pick outranks (score, then smaller index) every other entry
            for b in set(range(n)) - picked:
                assert s[a] > s[b] or (s[a] == s[b] and a < b)
        assert list(v[0]) == [s[j - 1] for j in i[0]]
        assert all(v[0][t] >= v[0][t + 1] for t in range(k - 1))


def test_oracle_topk_julia_isless_special_values():
    nan, inf = float("nan"), float("inf")
    s = np.array([[1.0, -0.0, nan, 0.0, -inf, inf, -nan, 1.0]], np.float32)
    v, i = oracle.topk(s, 8)
    # isless: NaNs equal and above +Inf (ties by index), -0.0 below +0.0
    assert list(i[0]) == [3, 7, 6, 1, 8, 4, 2, 5]
    assert np.isnan(v[0][:2]).all() and v[0][2] == inf and v[0][7] == -inf
    assert not np.signbit(v[0][5]) and np.signbit(v[0][6])


def test_oracle_topk_k_zero():
    v, i = oracle.topk(np.ones((2, 5), np.float32), 0)
    assert v.shape == (2, 0) and i.shape == (2, 0)
