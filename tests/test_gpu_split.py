"""GPU parity of the split-d scan (scan_split): dims whose query tile does not fit
in registers (16-bit features at multiples of 128 other than 64/128/256, int8 at
multiples of 256 other than 256, fp32 at multiples of 32).  Each batch of 8 k-blocks
is multiplied while the next is loaded, across chunk and pair boundaries; even and
odd k-blocks accumulate separately.  Compared with the CPU oracle at the north-star
tolerances (INT8 dots and per-token partials bit-exact), and grouped vs output-order
candidate scans bit for bit.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import FEATURE_TOL, as_feature, assert_scores, assert_tape, mask_np, tokens, widened

import flashmaxsim as fm
from flashmaxsim import boundary

pytestmark = pytest.mark.gpu

DT_ID = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}
SPLIT_CASES = [(torch.float16, 1024), (torch.bfloat16, 384), (torch.float32, 512),
               (torch.float32, 96)]


@pytest.fixture
def grouping():
    prev = boundary.candidates_grouping("auto")
    yield boundary.candidates_grouping
    boundary.candidates_grouping(prev)


@pytest.mark.parametrize("dtype,dim", SPLIT_CASES, ids=lambda x: DT_ID.get(x, str(x)))
def test_split_paired_parity(device, dtype, dim):
    Tq, Td, B = 33, 70, 3   # two query tiles, a ragged last chunk
    rng = np.random.default_rng([dim, 7])
    Qt, Qo, bf = as_feature(tokens(rng, (B, Tq, dim)), dtype)
    Dt, Do, _ = as_feature(tokens(rng, (B, Td, dim)), dtype)
    qm = torch.from_numpy(rng.random((B, Tq)) < 0.85)
    dm = torch.from_numpy(rng.random((B, Td)) < 0.75)
    dm[1, :] = False  # a fully masked document scores 0
    S_o, a_o, p_o = oracle.paired_forward(Qo, Do, mask_np(qm), mask_np(dm), bf16=bf)
    scores, args = fm.paired_forward(Qt.to(device), Dt.to(device), qm.to(device), dm.to(device))
    torch.cuda.synchronize()
    tol = FEATURE_TOL[dtype]
    assert_scores(scores.cpu(), S_o, tol)
    assert scores.cpu()[1] == 0
    Qf, Df = widened(Qo, bf), widened(Do, bf)
    assert_tape(args.cpu().numpy(), a_o, lambda p: Df[p[0]] @ Qf[p[0]][p[1]], tol)


@pytest.mark.parametrize("dtype,dim", SPLIT_CASES[:3], ids=lambda x: DT_ID.get(x, str(x)))
def test_split_candidates_grouped_and_output_order(device, grouping, dtype, dim):
    Tq, Td, N, C, B = 24, 40, 5, 9, 4
    rng = np.random.default_rng([dim, 8])
    Qt, Qo, bf = as_feature(tokens(rng, (B, Tq, dim)), dtype)
    Gt, Go, _ = as_feature(tokens(rng, (N, Td, dim)), dtype)
    idx = rng.integers(1, N + 1, size=(B, C)).astype(np.int64)
    idx[0, 0] = 0
    idx[3, 8] = N + 1
    dm = torch.from_numpy(rng.random((N, Td)) < 0.8)
    S_o, a_o, p_o = oracle.candidates_forward(Qo, Go, idx, None, mask_np(dm), -1.0e4, bf16=bf)
    outs = []
    for mode in ("always", "never"):
        grouping(mode)
        S, args = fm.candidates_forward(Qt.to(device), Gt.to(device),
                                        torch.from_numpy(idx).to(device), None, dm.to(device))
        torch.cuda.synchronize()
        outs.append((S.cpu(), args.cpu()))
    assert torch.equal(outs[0][0].view(torch.int32), outs[1][0].view(torch.int32))
    assert torch.equal(outs[0][1], outs[1][1])
    tol = FEATURE_TOL[dtype]
    assert_scores(outs[0][0], S_o, tol)
    Qf, Gf = widened(Qo, bf), widened(Go, bf)
    assert_tape(outs[0][1].numpy(), a_o, lambda p: Gf[idx[p[0], p[1]] - 1] @ Qf[p[0]][p[2]], tol)


@pytest.mark.parametrize("dim", [512, 1024])
def test_split_int8_exact(device, dim):
    Tq, Td, B = 40, 37, 3
    rng = np.random.default_rng(dim)
    Qc, Qs = oracle.quantize_int8(tokens(rng, (B, Tq, dim)))
    Dc, Ds = oracle.quantize_int8(tokens(rng, (B, Td, dim)))
    dm = (rng.random((B, Td)) < 0.8).astype(np.uint8)
    S_o, a_o, p_o = oracle.int8_paired_forward(Qc, Qs, Dc, Ds, None, dm)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    args = torch.zeros(B, Tq, dtype=torch.int32, device=device)
    part = torch.zeros(B, Tq, dtype=torch.float32, device=device)
    S = torch.zeros(B, dtype=torch.float32, device=device)
    boundary.launch_int8_paired_scan(args, part, dev(Qc), dev(Qs), dev(Dc), dev(Ds), None,
                                     dev(dm), S)
    torch.cuda.synchronize()
    assert np.array_equal(args.cpu().numpy(), a_o)
    assert np.array_equal(part.cpu().numpy().view(np.uint32), p_o.view(np.uint32))
    np.testing.assert_allclose(S.cpu().numpy(), S_o, rtol=1e-6, atol=1e-6)


def test_split_varlen_parity(device):
    dtype, dim = torch.bfloat16, 1024
    rng = np.random.default_rng(34)
    qlens, dlens = [4, 33, 0, 7], [70, 3, 5, 0]
    Qt, Qo, bf = as_feature(np.concatenate([tokens(rng, (n, dim)) for n in qlens], 0), dtype)
    Dt, Do, _ = as_feature(np.concatenate([tokens(rng, (n, dim)) for n in dlens], 0), dtype)
    cu_q = np.concatenate([[1], 1 + np.cumsum(qlens)]).astype(np.int32)
    cu_d = np.concatenate([[1], 1 + np.cumsum(dlens)]).astype(np.int32)
    s_o, a_o, _ = oracle.varlen_forward(Qo, Do, cu_q, cu_d, max(qlens), bf16=bf)
    Qp = fm.PackedSeq(Qt, torch.from_numpy(cu_q)).to(device)
    Dp = fm.PackedSeq(Dt, torch.from_numpy(cu_d)).to(device)
    scores, args = fm.varlen_forward(Qp, Dp)
    torch.cuda.synchronize()
    tol = FEATURE_TOL[dtype]
    assert_scores(scores.cpu(), s_o, tol)
    Qf, Df = widened(Qo, bf), widened(Do, bf)
    assert_tape(args.cpu().numpy(), a_o,
                lambda p: Df[cu_d[p[0]] - 1: cu_d[p[0] + 1] - 1] @ Qf[cu_q[p[0]] - 1 + p[1]], tol)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("dim,Tq", [(1024, 24), (512, 64), (1024, 40), (384, 7)],
                         ids=lambda x: str(x))
def test_split_packed_query_staging(device, dtype, dim, Tq):
    """Packed calls score one query against every document; the split kernel
    stages that query in LDS when it fits (1024x24, 512x64: two query tiles,
    384x7) and reads it from global memory otherwise (1024x40)."""
    rng = np.random.default_rng(dim + Tq)
    lens = [40, 0, 97, 3, 33, 64, 1]
    docs = [tokens(rng, (n, dim)) for n in lens]
    Qt, Qo, bf = as_feature(tokens(rng, (Tq, dim)), dtype)
    Tt, To, _ = as_feature(np.concatenate(docs, 0), dtype)
    cu = np.concatenate([[1], 1 + np.cumsum(lens)]).astype(np.int32)
    qm = torch.from_numpy(rng.random(Tq) < 0.9)
    s_o, a_o, _ = oracle.packed_forward(Qo, To, cu, mask_np(qm), bf16=bf)
    P = fm.PackedSeq(Tt, torch.from_numpy(cu)).to(device)
    scores, args = fm.packed_forward(Qt.to(device), P, qm.to(device))
    torch.cuda.synchronize()
    tol = FEATURE_TOL[dtype]
    assert_scores(scores.cpu(), s_o, tol)
    Qf, Tf = widened(Qo, bf), widened(To, bf)
    assert_tape(args.cpu().numpy(), a_o,
                lambda p: Tf[cu[p[0]] - 1: cu[p[0] + 1] - 1] @ Qf[p[1]], tol)
