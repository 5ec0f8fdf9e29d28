"""Shared input generation and comparison helpers for the parity tests.

Inputs are seeded numpy draws (PCG64), L2-normalised per token like the
reference's tests (``x ./= sqrt.(sum(abs2, x; dims=1) .+ eps)``,
test_math_oracle.jl:71-74 / test_cuda.jl:10-11), then rounded to the feature
type.  The same bytes go to the oracle (numpy) and to the device (torch).
"""
from __future__ import annotations

import numpy as np
import torch

import oracle

FEATURE_TOL = {  # relative score tolerance per feature type
    torch.float32: 1e-5,
    torch.float16: 2e-3,
    torch.bfloat16: 2e-3,
}


def tokens(rng, shape, normalize=True):
    x = rng.standard_normal(shape, dtype=np.float32)
    if normalize:
        x /= np.sqrt((x * x).sum(-1, keepdims=True) + np.finfo(np.float32).eps)
    return x.astype(np.float32)


def as_feature(x: np.ndarray, dtype):
    """Round fp32 numpy features to `dtype`; return (torch CPU tensor, oracle array, bf16 flag)."""
    t = torch.from_numpy(np.ascontiguousarray(x)).to(dtype)
    if dtype == torch.bfloat16:
        return t, t.view(torch.int16).numpy().view(np.uint16).copy(), True
    return t, t.numpy().copy(), False


def widened(arr: np.ndarray, bf16: bool) -> np.ndarray:
    """fp64 copy of stored features (exact)."""
    if bf16:
        return oracle.bf16_bits_to_f32(arr).astype(np.float64)
    return arr.astype(np.float64)


def assert_scores(got, want, rtol, atol=None, what="scores"):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    if atol is None:
        atol = rtol
    bad = np.abs(got - want) > atol + rtol * np.abs(want)
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} differ; first at {tuple(i)}: "
                             f"got {got[tuple(i)]!r} want {want[tuple(i)]!r}")


def assert_tape(got, want, pair_sims, rtol, what="argmax tape"):
    """Tapes must match except at near-ties.

    got/want: int arrays (..., Tq) of 1-based document tokens.  pair_sims(idx)
    returns the fp64 similarity row s[u] (0-based u) of the query token at the
    multi-index ``idx`` (all but the last axis identify the pair, the last
    the query token) -- used only for mismatching cells: there the two chosen
    tokens must be valid and their similarities equal within tolerance.
    """
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    mism = np.argwhere(got != want)
    for idx in mism:
        idx = tuple(int(v) for v in idx)
        g, w = int(got[idx]), int(want[idx])
        assert g > 0 and w > 0, f"{what}: at {idx} got {g} want {w} (one side empty)"
        s = pair_sims(idx)
        sg, sw = s[g - 1], s[w - 1]
        assert abs(sg - sw) <= rtol * max(1.0, abs(sw)), (
            f"{what}: at {idx} got token {g} (s={sg}) want {w} (s={sw}) -- not a near-tie")
    return len(mism)


def to_dev(t, device):
    return None if t is None else t.to(device)


def mask_np(m):
    return None if m is None else m.numpy().astype(np.uint8)
