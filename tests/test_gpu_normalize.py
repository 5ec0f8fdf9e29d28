"""GPU: the normalize=true epilogue fused into every scan's score write.

The reference normalises after the scan (normalize.jl:4-46, packed.jl:316-354):
scores .* inv_n with inv_n = 1 / max(count(qmask[:, b]), 1) in Float32, the
varlen pair's query length instead of a mask count, and `neg` kept for
invalid candidates.  One fp32 multiply of the same two fp32 values, so the
fused result must be BIT-identical to the unnormalised scan's scores times
the fp32 inverse computed on the host side of the test, and to the library's
standalone normalize kernel.  Covered: each kernel family that writes scores
(fast 16-bit d=128, split-d d=1024, generic fp32, in-batch MFMA, multi-query
packed MFMA, INT8), output and document order for candidates, Tq above one
64-token pass of the count, all-masked queries (count 0 -> inverse 1).
"""
import numpy as np
import pytest
import torch

from helpers import tokens

import flashmaxsim as fm
from flashmaxsim import boundary
from flashmaxsim import forward as F

pytestmark = pytest.mark.gpu


def _inv(qm, B, Tq, device):
    if qm is None:
        return torch.full((B,), 1.0 / max(Tq, 1), dtype=torch.float32, device=device)
    return 1.0 / qm.reshape(B, Tq).sum(1).to(torch.float32).clamp(min=1.0)


def _qmask(rng, B, Tq, device):
    qm = torch.from_numpy(rng.random((B, Tq)) < 0.7).to(device)
    qm[0] = False  # a query with no valid token: inverse 1
    return qm


@pytest.mark.parametrize("dtype,dim,Tq", [
    (torch.float16, 128, 32),    # fast kernel
    (torch.bfloat16, 1024, 20),  # split-d kernel
    (torch.float32, 96, 100),    # generic kernel, Tq > 64
])
def test_paired_and_candidates_fused_normalize(device, dtype, dim, Tq):
    rng = np.random.default_rng(dim + Tq)
    B, Td, N, C = 6, 45, 9, 7
    print(f"normalize paired/candidates dtype={dtype} dim={dim} Tq={Tq}", flush=True)
    Q = torch.from_numpy(tokens(rng, (B, Tq, dim))).to(device, dtype)
    D = torch.from_numpy(tokens(rng, (B, Td, dim))).to(device, dtype)
    G = torch.from_numpy(tokens(rng, (N, Td, dim))).to(device, dtype)
    qm = _qmask(rng, B, Tq, device)
    inv = _inv(qm, B, Tq, device)
    s, tape = F.paired_forward(Q, D, qm, None)
    sn, tape_n = F.paired_forward(Q, D, qm, None, normalize=True)
    assert torch.equal(sn, s * inv)
    assert torch.equal(tape, tape_n)
    # the standalone kernel gives the same bits
    assert torch.equal(sn, F.length_normalize(s, qm, Tq))
    idx = torch.from_numpy(rng.integers(0, N + 2, size=(B, C))).to(device)  # 0, N+1 invalid
    for mode in ("never", "always"):
        prev = boundary.candidates_grouping(mode)
        try:
            S, _ = F.candidates_forward(Q, G, idx, qm, None)
            Sn, _ = F.candidates_forward(Q, G, idx, qm, None, normalize=True)
        finally:
            boundary.candidates_grouping(prev)
        valid = (idx >= 1) & (idx <= N)
        assert torch.equal(Sn, torch.where(valid, S * inv[:, None], S))
        assert bool((Sn[~valid] == -1.0e4).all())
        assert torch.equal(Sn, F.length_normalize_candidates(S, qm, Tq, idx, N, -1.0e4))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("Tq", [24, 70], ids=lambda t: f"Tq{t}")
def test_inbatch_and_packed_multi_fused_normalize(device, dtype, Tq):
    """Tq = 70: three query tiles per query, normalised over all 70 tokens."""
    rng = np.random.default_rng(3 + Tq)
    Bq, Bd, Td, dim = 37, 50, 70, 128
    print(f"normalize in-batch / multi-query dtype={dtype}", flush=True)
    Q = torch.from_numpy(tokens(rng, (Bq, Tq, dim))).to(device, dtype)
    D = torch.from_numpy(tokens(rng, (Bd, Td, dim))).to(device, dtype)
    qm = _qmask(rng, Bq, Tq, device)
    dm = torch.from_numpy(rng.random((Bd, Td)) < 0.8).to(device)
    inv = _inv(qm, Bq, Tq, device)
    S, _ = F.inbatch_forward(Q, D, qm, dm)
    Sn, _ = F.inbatch_forward(Q, D, qm, dm, normalize=True)
    assert torch.equal(Sn, S * inv[:, None])
    lens = rng.integers(0, 90, size=40)
    tok = torch.from_numpy(tokens(rng, (int(lens.sum()), dim))).to(dtype)
    P = fm.PackedSeq(tok, np.concatenate([[1], 1 + np.cumsum(lens)]).astype(np.int32)).to(device)
    M, _ = F.packed_multi_forward(Q, P, qm)
    Mn, _ = F.packed_multi_forward(Q, P, qm, normalize=True)
    assert torch.equal(Mn, M * inv[:, None])
    # single-query packed and varlen through the per-pair scans
    s1, _ = F.packed_forward(Q[3], P, qm[3])
    s1n, _ = F.packed_forward(Q[3], P, qm[3], normalize=True)
    assert torch.equal(s1n, s1 * inv[3])
    Qp, Dp = fm.pack_pairs([Q[1][:5], Q[2][:0], Q[4]], [D[0], D[1], D[2][:3]])
    v, _ = F.varlen_forward(Qp, Dp)
    vn, _ = F.varlen_forward(Qp, Dp, normalize=True)
    assert torch.equal(vn, v * torch.tensor([1 / 5, 1.0, 1 / Tq], dtype=torch.float32,
                                            device=device))


def test_int8_fused_normalize(device):
    rng = np.random.default_rng(8)
    B, Tq, Td, dim, N, C = 4, 12, 33, 64, 6, 5
    print("normalize int8", flush=True)
    Q = torch.from_numpy(tokens(rng, (B, Tq, dim))).to(device)
    D = fm.quantize_int8_symmetric(torch.from_numpy(tokens(rng, (B, Td, dim))).to(device))
    G = fm.quantize_int8_symmetric(torch.from_numpy(tokens(rng, (N, Td, dim))).to(device))
    qm = _qmask(rng, B, Tq, device)
    inv = _inv(qm, B, Tq, device)
    s, _ = F.int8_paired_forward(Q, D, qm, None)
    sn, _ = F.int8_paired_forward(Q, D, qm, None, normalize=True)
    assert torch.equal(sn, s * inv)
    idx = torch.from_numpy(rng.integers(0, N + 1, size=(B, C))).to(device)
    S, _ = F.int8_candidates_forward(Q, G, idx, qm, None)
    Sn, _ = F.int8_candidates_forward(Q, G, idx, qm, None, normalize=True)
    valid = (idx >= 1) & (idx <= N)
    assert torch.equal(Sn, torch.where(valid, S * inv[:, None], S))
    assert torch.equal(fm.maxsim(Q, G, idx, qm, normalize=True), Sn)
