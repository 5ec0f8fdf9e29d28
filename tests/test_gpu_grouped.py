"""GPU parity of the candidate scans in document order.

fms_launch_candidates_scan / fms_launch_int8_candidates_scan may score the
pairs grouped by gallery document (a counting sort on idx, then a scan in
that order).  Every pair is computed by the same arithmetic in either order,
so grouped results must equal the output-order results BIT FOR BIT, and both
must match the CPU oracle to the feature type's tolerance.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import FEATURE_TOL, as_feature, assert_scores, assert_tape, mask_np, tokens, widened

from flashmaxsim import boundary

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16, torch.float32]
DT_ID = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}


@pytest.fixture
def grouping():
    prev = boundary.candidates_grouping("auto")
    yield boundary.candidates_grouping
    boundary.candidates_grouping(prev)


def _run_float(device, Qt, Gt, idx_t, qm, dm, N, neg):
    B, C = idx_t.shape
    Tq = Qt.shape[1]
    args = torch.full((B, C, Tq), -7, dtype=torch.int32, device=device)
    part = torch.full((B, C, Tq), -7.0, dtype=torch.float32, device=device)
    S = torch.full((B, C), -7.0, dtype=torch.float32, device=device)
    boundary.launch_candidates_scan(args, part, Qt, Gt, idx_t, qm, dm, N, S, neg)
    torch.cuda.synchronize()
    return S.cpu(), args.cpu(), part.cpu()


def _bitwise_equal(a, b):
    for x, y in zip(a, b):
        assert torch.equal(x.view(torch.int32) if x.dtype == torch.float32 else x,
                           y.view(torch.int32) if y.dtype == torch.float32 else y)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("shape", [(128, 32, 180, 7, 33, 9), (40, 33, 65, 5, 9, 6),
                                   (128, 24, 100, 3, 40, 8), (8, 6, 7, 1, 17, 5),
                                   (64, 40, 70, 6, 25, 9), (128, 70, 33, 5, 20, 3),
                                   (64, 32, 1, 4, 11, 2)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64], ids=["i32", "i64"])
def test_grouped_matches_output_order_and_oracle(device, grouping, dtype, shape, idx_dtype):
    """Document order (with and, for 16-bit d = 64 / 128, without the query tiles
    copied in fragment order) against output order and the oracle.  Shapes cover
    the LDS-streamed batch scan at d = 64 and 128, Tq of 24, 32, 40 and 70 (one to
    three query tiles), ragged and one-token documents, and the generic dims."""
    dim, Tq, Td, N, C, B = shape
    rng = np.random.default_rng([dim, Tq, Td, N, C, B])
    Qt, Qo, bf = as_feature(tokens(rng, (B, Tq, dim)), dtype)
    Gt, Go, _ = as_feature(tokens(rng, (N, Td, dim)), dtype)
    idx = rng.integers(1, N + 1, size=(B, C)).astype(np.int64)  # N small: many repeats
    idx[0, 0] = 0
    idx[B - 1, C - 1] = N + 1
    idx[B // 2, C // 2] = -3
    qm = torch.from_numpy(rng.random((B, Tq)) < 0.85)
    dm = torch.from_numpy(rng.random((N, Td)) < 0.8)
    dm[N - 1, :] = False  # a fully masked document scores 0
    neg = -1.0e4
    dev_in = (Qt.to(device), Gt.to(device), torch.from_numpy(idx).to(idx_dtype).to(device),
              qm.to(device), dm.to(device))
    grouping("never")
    ref = _run_float(device, *dev_in, N, neg)
    grouping("always")
    got = _run_float(device, *dev_in, N, neg)
    _bitwise_equal(got, ref)
    grouping("always_direct_queries")
    _bitwise_equal(_run_float(device, *dev_in, N, neg), ref)

    S_o, a_o, p_o = oracle.candidates_forward(Qo, Go, idx, mask_np(qm), mask_np(dm), neg, bf16=bf)
    tol = FEATURE_TOL[dtype]
    assert_scores(got[0], S_o, tol)
    assert_scores(got[2], p_o, tol, what="partial")
    assert (got[0].numpy()[(idx < 1) | (idx > N)] == np.float32(neg)).all()
    Qf, Gf = widened(Qo, bf), widened(Go, bf)
    assert_tape(got[1].numpy(), a_o,
                lambda p: Gf[idx[p[0], p[1]] - 1] @ Qf[p[0]][p[2]], tol)


def test_auto_grouping_at_scale(device, grouping):
    """C*B = 32768 >= the automatic threshold: the default mode groups; results equal the
    output-order scan bit for bit and a sample matches the oracle."""
    dim, Tq, Td, N, C, B = 128, 32, 48, 3000, 512, 64
    rng = np.random.default_rng(77)
    Qt, Qo, _ = as_feature(tokens(rng, (B, Tq, dim)), torch.float16)
    Gt, Go, _ = as_feature(tokens(rng, (N, Td, dim)), torch.float16)
    idx = rng.integers(1, N + 1, size=(B, C)).astype(np.int64)
    idx[rng.random((B, C)) < 0.01] = 0
    dev_in = (Qt.to(device), Gt.to(device), torch.from_numpy(idx).to(device), None, None)
    grouping("auto")
    got = _run_float(device, *dev_in, N, -1.0e4)
    grouping("never")
    ref = _run_float(device, *dev_in, N, -1.0e4)
    _bitwise_equal(got, ref)
    sub = np.sort(rng.choice(B * C, size=300, replace=False))
    S_o, a_o, _ = oracle.candidates_forward(Qo, Go, idx, None, None, -1.0e4, subset=sub)
    assert_scores(got[0].numpy().reshape(-1)[sub], S_o.reshape(-1)[sub], FEATURE_TOL[torch.float16])


@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64], ids=["i32", "i64"])
def test_grouped_int8_bit_exact(device, grouping, idx_dtype):
    dim, Tq, Td, N, C, B = 128, 32, 180, 9, 21, 7
    rng = np.random.default_rng(91)
    Qc, Qs = oracle.quantize_int8(tokens(rng, (B, Tq, dim)))
    Gc, Gs = oracle.quantize_int8(tokens(rng, (N, Td, dim)))
    idx = rng.integers(1, N + 1, size=(B, C)).astype(np.int64)
    idx[2, 5] = 0
    idx[6, 20] = N + 2
    dm = np.arange(Td)[None, :] < rng.integers(0, Td + 1, size=(N, 1))
    S_o, a_o, p_o = oracle.int8_candidates_forward(Qc, Qs, Gc, Gs, idx, None, dm.astype(np.uint8))
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    outs = []
    for mode in ("always", "never"):
        grouping(mode)
        args = torch.zeros(B, C, Tq, dtype=torch.int32, device=device)
        part = torch.zeros(B, C, Tq, dtype=torch.float32, device=device)
        S = torch.zeros(B, C, dtype=torch.float32, device=device)
        boundary.launch_int8_candidates_scan(args, part, dev(Qc), dev(Qs), dev(Gc), dev(Gs),
                                             dev(idx).to(idx_dtype), None, dev(dm), N, S, -1.0e4)
        torch.cuda.synchronize()
        outs.append((S.cpu(), args.cpu(), part.cpu()))
    _bitwise_equal(outs[0], outs[1])
    S, args, part = outs[0]
    assert np.array_equal(args.numpy(), a_o)
    assert np.array_equal(part.numpy().view(np.uint32), p_o.view(np.uint32))
    np.testing.assert_allclose(S.numpy(), S_o, rtol=1e-6, atol=1e-6)


def test_one_level_sort_and_three_launch_scan(device, grouping):
    """A gallery too large for the two-level bucket sort: 4,200,000 one-token
    documents (d = 32, 269 MB) and 1,126,400 pairs give 4,096 buckets x 1,100
    pair tiles, past the bucket table, so the pairs take the one-level sort, and
    4,200,001 document counters are 1,026 prefix-scan tiles, past the 1,024 that
    the two-launch scan handles.  Forced document order must equal output order
    bit for bit, and a sample of queries must match the oracle."""
    rng = np.random.default_rng(4200)
    N, Td, dim, Tq, B, C = 4_200_000, 1, 32, 4, 1100, 1024
    gen = torch.Generator(device=device)
    gen.manual_seed(4200)
    Q = torch.randn(B, Tq, dim, generator=gen, device=device).to(torch.float16)
    G = torch.randn(N, Td, dim, generator=gen, device=device).to(torch.float16)
    idx = torch.randint(1, N + 1, (B, C), generator=gen, device=device, dtype=torch.int64)
    idx.view(-1)[::101] = 0
    qm = torch.ones(B, Tq, dtype=torch.bool, device=device)
    dm = torch.ones(N, Td, dtype=torch.bool, device=device)
    grouping("always")
    grouped = _run_float(device, Q, G, idx, qm, dm, N, -2.0)
    grouping("never")
    direct = _run_float(device, Q, G, idx, qm, dm, N, -2.0)
    _bitwise_equal(grouped, direct)
    rows = rng.choice(B, size=32, replace=False)
    rows_t = torch.from_numpy(rows).to(device)
    sub = idx[rows_t].cpu().numpy()
    used = np.unique(sub[sub > 0])
    remap = np.zeros(N + 1, np.int64)
    remap[used] = np.arange(1, len(used) + 1)
    Go = G[torch.from_numpy(used - 1).to(device)].cpu().numpy()
    S_o, a_o, _ = oracle.candidates_forward(Q[rows_t].cpu().numpy(), Go, remap[sub],
                                            np.ones((32, Tq), np.uint8),
                                            np.ones((len(used), Td), np.uint8), -2.0)
    S_g = grouped[0].numpy()[rows]
    a_g = grouped[1].numpy()[rows]
    assert np.allclose(S_g, S_o, rtol=2e-3, atol=2e-3)
    assert np.array_equal(a_g, a_o)
