"""GPU parity: every HIP scan layout vs the CPU oracle on the same seeded inputs.

Bars (north star): fp32 scores within 1e-5 relative, fp16/bf16 within 2e-3;
argmax tapes equal except at near-ties within that tolerance; INT8 int32
dots and per-token partials bit-exact.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import (FEATURE_TOL, as_feature, assert_scores, assert_tape, mask_np, to_dev,
                     tokens, widened)

import flashmaxsim as fm
from flashmaxsim import _lib, boundary

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16, torch.float32]
DT_ID = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}


def _acc_row(r, h):
    return 8 * (r >> 2) + 4 * h + (r & 3)


@pytest.mark.parametrize("op", [0, 1, 2, 3], ids=["f32", "f16", "bf16", "i8"])
def test_mfma_accumulator_layout(device, op):
    out = torch.zeros(2048, dtype=torch.float32, device=device)
    _lib.check(_lib.lib().fms_debug_mfma_layout(out.data_ptr(), op,
                                                torch.cuda.current_stream().cuda_stream),
               "probe")
    o = out.cpu().numpy().reshape(2, 64, 16)
    for lane in range(64):
        for r in range(16):
            assert o[0, lane, r] == _acc_row(r, lane // 32) + 1, (lane, r, o[0, lane, r])
            assert o[1, lane, r] == (lane % 32) + 1, (lane, r, o[1, lane, r])


def test_cross_lane_helpers(device):
    """The lane exchanges the tile close relies on (v_permlane32/16_swap, DPP): xor-32
    partner, the sum over lanes 0-31 broadcast to every lane, and the half merge's tie
    rule (larger max wins, equal maxima keep the lower token)."""
    out = torch.zeros(256, dtype=torch.float32, device=device)
    _lib.check(_lib.lib().fms_debug_cross_lane(out.data_ptr(),
                                               torch.cuda.current_stream().cuda_stream), "probe")
    o = out.cpu().numpy()
    for lane in range(64):
        assert o[lane] == lane ^ 32, (lane, o[lane])
        assert o[64 + lane] == 496.0, (lane, o[64 + lane])
        mine, other = (lane % 7, lane + 1), ((lane ^ 32) % 7, (lane ^ 32) + 1)
        want = other if (other[0] > mine[0] or (other[0] == mine[0] and other[1] < mine[1])) else mine
        assert (o[128 + lane], o[192 + lane]) == (want[1], want[0]), (lane, o[128 + lane], o[192 + lane])


def test_gather_bandwidth_probe(device):
    """fms_debug_gather_bandwidth (the gathered-document read ceiling bench.py reports):
    workgroup i XOR-folds the 16-byte units of document docs[i], each thread over units
    tid, tid+256, ...; a document outside the gallery is skipped (its words stay 0)."""
    rng = np.random.default_rng(7)
    N, doc_bytes = 37, 1040
    g = rng.integers(0, 2**32, size=N * doc_bytes // 4, dtype=np.uint64).astype(np.uint32)
    docs = np.array([3, 0, 36, 3, 37, 12], np.int32)  # 37: past the end
    out = torch.full((len(docs) * 256,), -1, dtype=torch.int32, device=device)
    gt = torch.from_numpy(g.view(np.int32)).to(device)
    dt = torch.from_numpy(docs).to(device)
    _lib.check(_lib.lib().fms_debug_gather_bandwidth(gt.data_ptr(), N * doc_bytes, doc_bytes,
                                                     dt.data_ptr(), len(docs), out.data_ptr(),
                                                     torch.cuda.current_stream().cuda_stream),
               "gather probe")
    got = out.cpu().numpy().view(np.uint32).reshape(len(docs), 256)
    units = g.reshape(N, doc_bytes // 16, 4)
    for i, d in enumerate(docs):
        for t in range(256):
            want = 0
            if d < N:
                for u in range(t, doc_bytes // 16, 256):
                    want ^= int(np.bitwise_xor.reduce(units[d, u]))
            assert got[i, t] == want, (i, t)


def _masks(rng, B, Tq, Td, kind):
    if kind == "none":
        return None, None
    if kind == "pattern":  # test_ka_cpu.jl:19-21 patterns
        qm = np.array([[(t + 1) % 2 == 1 for t in range(Tq)] for _ in range(B)])
        dm = np.array([[(u + 1) % 3 != 0 for u in range(Td)] for _ in range(B)])
    else:  # random, with one fully masked document row
        qm = rng.random((B, Tq)) < 0.8
        dm = rng.random((B, Td)) < 0.7
        dm[-1, :] = False
    return torch.from_numpy(qm), torch.from_numpy(dm)


def _pair_sims_fn(qf, df, pair_of):
    """qf (P?, Tq, dim) f64, df(...) -> callable(idx) -> s[u] for (pair, t)."""
    def sims(idx):
        *pidx, t = idx
        q, d = pair_of(tuple(pidx))
        return d @ q[t]
    return sims


PAIRED_SHAPES = [
    (128, 32, 180, 8),   # fast kernel, C2-like tokens
    (40, 33, 65, 2),     # tile-straddling dim/Tq/Td (test_cuda.jl:102-117)
    (768, 8, 17, 2),     # split-d (test_cuda.jl:174-187)
    (256, 32, 64, 3),    # fast kernel, second register bucket
    (16, 12, 130, 3),    # host DOC_TILE straddle (test_regressions.jl:88-98)
    (8, 3, 5, 2),
    (12, 5, 9, 2),       # row not a 16-byte multiple for 16-bit types
]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("shape", PAIRED_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("masks", ["none", "pattern", "random"])
def test_paired_parity(device, dtype, shape, masks):
    dim, Tq, Td, B = shape
    rng = np.random.default_rng([dim, Tq, Td, B, ["none", "pattern", "random"].index(masks)])
    Qt, Qo, bf = as_feature(tokens(rng, (B, Tq, dim)), dtype)
    Dt, Do, _ = as_feature(tokens(rng, (B, Td, dim)), dtype)
    qm, dm = _masks(rng, B, Tq, Td, masks)
    s_o, a_o, p_o = oracle.paired_forward(Qo, Do, mask_np(qm), mask_np(dm), bf16=bf)
    args = torch.zeros(B, Tq, dtype=torch.int32, device=device)
    part = torch.zeros(B, Tq, dtype=torch.float32, device=device)
    scores = torch.zeros(B, dtype=torch.float32, device=device)
    boundary.launch_paired_scan(args, part, Qt.to(device), Dt.to(device), to_dev(qm, device),
                                to_dev(dm, device), scores)
    torch.cuda.synchronize()
    tol = FEATURE_TOL[dtype]
    assert_scores(scores.cpu(), s_o, tol, what="scores")
    assert_scores(part.cpu(), p_o, tol, what="partial")
    Qf, Df = widened(Qo, bf), widened(Do, bf)
    assert_tape(args.cpu().numpy(), a_o, _pair_sims_fn(Qf, Df, lambda p: (Qf[p[0]], Df[p[0]])), tol)
    # the driver path (fused scores, no partial) agrees with the boundary path
    s2, a2 = fm.paired_forward(Qt.to(device), Dt.to(device), to_dev(qm, device), to_dev(dm, device))
    torch.cuda.synchronize()
    assert torch.equal(s2.cpu(), scores.cpu()) and torch.equal(a2.cpu(), args.cpu())


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("shape", [(128, 32, 180), (40, 33, 65), (8, 6, 7), (128, 24, 100)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64], ids=["i32", "i64"])
def test_candidates_parity(device, dtype, shape, idx_dtype):
    dim, Tq, Td = shape
    N, C, B = 23, 9, 5
    rng = np.random.default_rng(dim * 1000 + Tq * 10 + Td)
    Qt, Qo, bf = as_feature(tokens(rng, (B, Tq, dim)), dtype)
    Gt, Go, _ = as_feature(tokens(rng, (N, Td, dim)), dtype)
    idx = rng.integers(1, N + 1, size=(B, C)).astype(np.int64)
    idx[0, 2] = 0
    idx[3, 0] = N + 1
    idx[4, 8] = -5
    qm = torch.from_numpy(rng.random((B, Tq)) < 0.9)
    dm = torch.from_numpy(np.array([[(u + 1) % 4 != 0 for u in range(Td)] for _ in range(N)]))
    neg = -1.0e4
    S_o, a_o, p_o = oracle.candidates_forward(Qo, Go, idx, mask_np(qm), mask_np(dm), neg, bf16=bf)
    idx_t = torch.from_numpy(idx).to(idx_dtype).to(device)
    args = torch.zeros(B, C, Tq, dtype=torch.int32, device=device)
    part = torch.zeros(B, C, Tq, dtype=torch.float32, device=device)
    S = torch.zeros(B, C, dtype=torch.float32, device=device)
    boundary.launch_candidates_scan(args, part, Qt.to(device), Gt.to(device), idx_t,
                                    qm.to(device), dm.to(device), N, S, neg)
    torch.cuda.synchronize()
    tol = FEATURE_TOL[dtype]
    assert_scores(S.cpu(), S_o, tol, what="scores")
    assert (S.cpu().numpy()[idx < 1] == np.float32(neg)).all()
    assert (S.cpu().numpy()[idx > N] == np.float32(neg)).all()
    assert_scores(part.cpu(), p_o, tol, what="partial")
    Qf, Gf = widened(Qo, bf), widened(Go, bf)
    assert_tape(args.cpu().numpy(), a_o,
                _pair_sims_fn(Qf, Gf, lambda p: (Qf[p[0]], Gf[idx[p[0], p[1]] - 1])), tol)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("shape", [(128, 32, 180, 6, 5), (40, 33, 65, 3, 4), (16, 8, 10, 4, 4),
                                   # dim 128: the MFMA-tiled in-batch kernel
                                   (128, 32, 180, 40, 37), (128, 1, 1, 3, 2), (128, 24, 65, 17, 9),
                                   (128, 32, 33, 20, 3), (128, 8, 40, 512, 1024),
                                   # long documents: a block's chunk stream holds the
                                   # full 512-entry list (padded past it)
                                   (128, 32, 1000, 20, 40), (128, 16, 2048, 17, 9),
                                   # dim 32, 64, 96: the same kernel with 2, 4, 6 k-blocks
                                   (64, 32, 180, 40, 37), (96, 24, 65, 17, 9), (32, 16, 100, 33, 20),
                                   (64, 8, 40, 300, 600), (96, 32, 1000, 20, 40),
                                   # Tq > 32: query tiles of 32 (2, 3, 4 per query; a last
                                   # tile of 8, 32 and 4 tokens)
                                   (128, 40, 65, 33, 9), (128, 64, 100, 20, 17), (64, 100, 50, 10, 12),
                                   (96, 300, 33, 5, 7)],
                         ids=lambda s: "x".join(map(str, s)))
def test_inbatch_parity(device, dtype, shape):
    dim, Tq, Td, Bq, Bd = shape
    rng = np.random.default_rng(sum(shape))
    Qt, Qo, bf = as_feature(tokens(rng, (Bq, Tq, dim)), dtype)
    Dt, Do, _ = as_feature(tokens(rng, (Bd, Td, dim)), dtype)
    lens = rng.integers(min(Td, 3), Td + 1, size=Bd)
    lens[0] = 0  # an empty document contributes 0 (test_regressions.jl:65-86)
    dm = torch.from_numpy(np.arange(Td)[None, :] < lens[:, None])
    qm = torch.from_numpy(rng.random((Bq, Tq)) < 0.9)
    S_o, a_o = oracle.inbatch_forward(Qo, Do, mask_np(qm), mask_np(dm), bf16=bf)
    S, args = fm.inbatch_forward(Qt.to(device), Dt.to(device), qm.to(device), dm.to(device))
    torch.cuda.synchronize()
    tol = FEATURE_TOL[dtype]
    assert_scores(S.cpu(), S_o, tol, what="S")
    assert (S.cpu().numpy()[:, 0] == 0).all()
    Qf, Df = widened(Qo, bf), widened(Do, bf)
    assert_tape(args.cpu().numpy(), a_o, _pair_sims_fn(Qf, Df, lambda p: (Qf[p[0]], Df[p[1]])), tol)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("shape", [(32, 180, 24, 21), (17, 65, 40, 33), (32, 32, 16, 16),
                                   (8, 300, 20, 17), (5, 7, 18, 6),
                                   # Tq = 24: four queries packed into three tiles
                                   (24, 180, 24, 21), (24, 33, 9, 5), (24, 700, 37, 5),
                                   # Tq > 32: query tiles
                                   (40, 65, 33, 9), (96, 180, 12, 11)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("dim", [128, 64], ids=lambda d: f"d{d}")
def test_inbatch_masks_and_ties(device, dtype, shape, dim):
    """Non-prefix document masks, leading masked tokens, fully masked and
    single-token documents, and exact duplicate tokens (exact ties must keep
    the first occurrence, forward_pair.jl:82-85) on the MFMA-tiled kernel,
    which substitutes masked rows by copies of the first valid token."""
    Tq, Td, Bq, Bd = shape
    rng = np.random.default_rng(Tq * 1000 + Td + dim)
    q32 = tokens(rng, (Bq, Tq, dim))
    d32 = tokens(rng, (Bd, Td, dim))
    dm = rng.random((Bd, Td)) < 0.7
    for j in range(Bd):  # later rows copy earlier ones: exact ties
        for _ in range(3):
            a, b = np.sort(rng.choice(Td, 2, replace=False)) if Td > 1 else (0, 0)
            d32[j, b] = d32[j, a]
    dm[0, : min(Td - 1, 40)] = False          # leading masked tokens
    dm[1, :] = False                           # no valid token
    dm[2, :] = False
    dm[2, Td - 1] = True                       # only the last token
    if Td > 3:                                 # first valid token also at a later valid row
        first = int(np.argmax(dm[3])) if dm[3].any() else 0
        dm[3, first] = True
        d32[3, Td - 1] = d32[3, first]
        dm[3, Td - 1] = True
    Qt, Qo, bf = as_feature(q32, dtype)
    Dt, Do, _ = as_feature(d32, dtype)
    qm = torch.from_numpy(rng.random((Bq, Tq)) < 0.9)
    dmt = torch.from_numpy(dm)
    S_o, a_o = oracle.inbatch_forward(Qo, Do, mask_np(qm), mask_np(dmt), bf16=bf)
    S, args = fm.inbatch_forward(Qt.to(device), Dt.to(device), qm.to(device), dmt.to(device))
    torch.cuda.synchronize()
    tol = FEATURE_TOL[dtype]
    assert_scores(S.cpu(), S_o, tol, what="S")
    assert (S.cpu().numpy()[:, 1] == 0).all()
    got = args.cpu().numpy()
    assert (got[:, 1] == 0).all()
    # every recorded token is a valid document token
    ii, jj, tt = np.nonzero(got)
    assert dm[jj, got[ii, jj, tt] - 1].all()
    # mismatches only at near-ties between tokens that are not exact copies
    Qf, Df = widened(Qo, bf), widened(Do, bf)
    assert_tape(got, a_o, _pair_sims_fn(Qf, Df, lambda p: (Qf[p[0]], Df[p[1]])), tol)
    for i, j, t in np.argwhere(got != a_o):
        g, w = got[i, j, t] - 1, a_o[i, j, t] - 1
        assert not np.array_equal(Do[j, g], Do[j, w]), (i, j, t, g, w)


def _unit_stream_case(rng, case):
    """(Tq, Td, Bq, Bd, dim, dmask) for test_inbatch_unit_stream."""
    if case == "short":
        # documents of 0..40 rows (prefix masks), a third of them within one
        # 16-row unit: split entries whose second document also closes there
        Tq, Td, Bq, Bd, dim = 32, 40, 20, 96, 64
        lens = rng.integers(0, Td + 1, Bd)
        lens[::3] = rng.integers(1, 17, len(lens[::3]))
        dm = np.arange(Td)[None, :] < lens[:, None]
    elif case == "holes":
        # valid rows in scattered runs: fully masked units inside a document
        # (streamed, substituted), leading masked units (skipped), last valid
        # row anywhere
        Tq, Td, Bq, Bd, dim = 40, 100, 17, 45, 64
        dm = np.zeros((Bd, Td), bool)
        for j in range(Bd):
            for _ in range(rng.integers(0, 4)):
                a = int(rng.integers(0, Td))
                dm[j, a:a + int(rng.integers(1, 12))] = True
        dm[0, 37] = True
        dm[1, :] = False
        dm[2, [0, 99]] = True
    else:  # "full_blocks": 40 documents per block (the per-block maximum)
        Tq, Td, Bq, Bd, dim = 32, 48, 512, 640, 32
        lens = rng.integers(1, Td + 1, Bd)
        dm = np.arange(Td)[None, :] < lens[:, None]
        dm &= rng.random((Bd, Td)) < 0.9
        dm[:, 0] |= ~dm.any(1)
    return Tq, Td, Bq, Bd, dim, dm


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("case", ["short", "holes", "full_blocks"])
def test_inbatch_unit_stream(device, dtype, case):
    """The in-batch kernel streams documents in 16-row units, two per chunk, so one
    chunk can hold a document's last unit and the next document's first (folded as
    two halves with a close between).  Short documents (split and close in one
    chunk), masked runs inside documents, leading masked units, and blocks at the
    40-document maximum, with exact duplicate tokens: scores and tapes against the
    oracle (forward_layouts.jl:155-179), every recorded token a valid one."""
    rng = np.random.default_rng({"short": 161, "holes": 162, "full_blocks": 163}[case])
    Tq, Td, Bq, Bd, dim, dm = _unit_stream_case(rng, case)
    q32 = tokens(rng, (Bq, Tq, dim))
    d32 = tokens(rng, (Bd, Td, dim))
    for j in range(0, Bd, 2):  # later rows copy earlier ones: exact ties
        a, b = np.sort(rng.choice(Td, 2, replace=False))
        d32[j, b] = d32[j, a]
    Qt, Qo, bf = as_feature(q32, dtype)
    Dt, Do, _ = as_feature(d32, dtype)
    dmt = torch.from_numpy(dm)
    S_o, a_o = oracle.inbatch_forward(Qo, Do, None, mask_np(dmt), bf16=bf)
    S, args = fm.inbatch_forward(Qt.to(device), Dt.to(device), None, dmt.to(device))
    torch.cuda.synchronize()
    tol = FEATURE_TOL[dtype]
    assert_scores(S.cpu(), S_o, tol, what="S")
    got = args.cpu().numpy()
    empty = ~dm.any(1)
    assert (got[:, empty] == 0).all() and (S.cpu().numpy()[:, empty] == 0).all()
    ii, jj, tt = np.nonzero(got)
    assert dm[jj, got[ii, jj, tt] - 1].all()
    Qf, Df = widened(Qo, bf), widened(Do, bf)
    assert_tape(got, a_o, _pair_sims_fn(Qf, Df, lambda p: (Qf[p[0]], Df[p[1]])), tol)
    for i, j, t in np.argwhere(got != a_o):
        g, w = got[i, j, t] - 1, a_o[i, j, t] - 1
        assert not np.array_equal(Do[j, g], Do[j, w]), (i, j, t, g, w)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("shape", [(32, 180, 24, 21), (17, 65, 40, 33), (8, 300, 20, 17)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("dim", [128, 96], ids=lambda d: f"d{d}")
def test_inbatch_negative_maxima(device, dtype, shape, dim):
    """Every dot product negative (queries in the positive orthant, documents
    in the negative one), with exact duplicate tokens: every chunk maximum is
    below zero, which the MFMA-tiled kernel folds on its exact path; exact
    ties must still keep the first occurrence (forward_pair.jl:82-85) and
    the all-negative maxima stay negative (test_regressions.jl:136-147)."""
    Tq, Td, Bq, Bd = shape
    rng = np.random.default_rng(Tq * 7 + Td + dim)
    q32 = np.abs(tokens(rng, (Bq, Tq, dim)))
    d32 = -np.abs(tokens(rng, (Bd, Td, dim)))
    q32 /= np.linalg.norm(q32, axis=-1, keepdims=True)
    d32 /= np.linalg.norm(d32, axis=-1, keepdims=True)
    for j in range(Bd):  # later rows copy earlier ones: exact ties
        for _ in range(4):
            a, b = np.sort(rng.choice(Td, 2, replace=False))
            d32[j, b] = d32[j, a]
    dm = rng.random((Bd, Td)) < 0.8
    dm[:, 0] = True
    Qt, Qo, bf = as_feature(q32.astype(np.float32), dtype)
    Dt, Do, _ = as_feature(d32.astype(np.float32), dtype)
    qm = torch.ones(Bq, Tq, dtype=torch.bool)
    dmt = torch.from_numpy(dm)
    S_o, a_o = oracle.inbatch_forward(Qo, Do, mask_np(qm), mask_np(dmt), bf16=bf)
    S, args = fm.inbatch_forward(Qt.to(device), Dt.to(device), qm.to(device), dmt.to(device))
    torch.cuda.synchronize()
    tol = FEATURE_TOL[dtype]
    assert (S_o < 0).all()
    assert_scores(S.cpu(), S_o, tol, what="S")
    got = args.cpu().numpy()
    Qf, Df = widened(Qo, bf), widened(Do, bf)
    assert_tape(got, a_o, _pair_sims_fn(Qf, Df, lambda p: (Qf[p[0]], Df[p[1]])), tol)
    for i, j, t in np.argwhere(got != a_o):
        g, w = got[i, j, t] - 1, a_o[i, j, t] - 1
        assert not np.array_equal(Do[j, g], Do[j, w]), (i, j, t, g, w)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("case", ["small", "colpali", "splitd"])
def test_packed_parity(device, dtype, case):
    rng = np.random.default_rng({"small": 31, "colpali": 4, "splitd": 44}[case])
    if case == "small":
        dim, Tq, lens = 16, 7, [5, 0, 3, 9, 1, 33, 64, 65]
    elif case == "colpali":
        dim, Tq, lens = 128, 24, list(rng.integers(700, 1101, size=12))
        lens[3] = 0
    else:
        dim, Tq, lens = 1024, 24, [40, 0, 97, 3]
    docs = [tokens(rng, (n, dim)) for n in lens]
    q32 = tokens(rng, (Tq, dim))
    qt, qo, bf = as_feature(q32, dtype)
    tok_t, tok_o, _ = as_feature(np.concatenate(docs, 0), dtype)
    cu = np.concatenate([[1], 1 + np.cumsum(lens)]).astype(np.int32)
    qm = torch.from_numpy(rng.random(Tq) < 0.9)
    s_o, a_o, p_o = oracle.packed_forward(qo, tok_o, cu, mask_np(qm), bf16=bf)
    P = fm.PackedSeq(tok_t, torch.from_numpy(cu)).to(device)
    scores, args = fm.packed_forward(qt.to(device), P, qm.to(device))
    torch.cuda.synchronize()
    tol = FEATURE_TOL[dtype]
    assert_scores(scores.cpu(), s_o, tol)
    assert scores.cpu()[lens.index(0)] == 0
    qf, tf = widened(qo, bf), widened(tok_o, bf)
    assert_tape(args.cpu().numpy(), a_o,
                _pair_sims_fn(qf, tf, lambda p: (qf, tf[cu[p[0]] - 1: cu[p[0] + 1] - 1])), tol)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: DT_ID[d])
def test_varlen_parity(device, dtype):
    rng = np.random.default_rng(32)
    dim = 12 if dtype == torch.float32 else 64
    qlens = [4, 2, 35, 1, 0, 7]
    dlens = [5, 3, 70, 0, 4, 33]
    qs = [tokens(rng, (n, dim)) for n in qlens]
    ds = [tokens(rng, (n, dim)) for n in dlens]
    Qt, Qo, bf = as_feature(np.concatenate(qs, 0), dtype)
    Dt, Do, _ = as_feature(np.concatenate(ds, 0), dtype)
    cu_q = np.concatenate([[1], 1 + np.cumsum(qlens)]).astype(np.int32)
    cu_d = np.concatenate([[1], 1 + np.cumsum(dlens)]).astype(np.int32)
    max_q = max(qlens)
    s_o, a_o, p_o = oracle.varlen_forward(Qo, Do, cu_q, cu_d, max_q, bf16=bf)
    Qp = fm.PackedSeq(Qt, torch.from_numpy(cu_q)).to(device)
    Dp = fm.PackedSeq(Dt, torch.from_numpy(cu_d)).to(device)
    scores, args = fm.varlen_forward(Qp, Dp)
    torch.cuda.synchronize()
    tol = FEATURE_TOL[dtype]
    assert_scores(scores.cpu(), s_o, tol)
    Qf, Df = widened(Qo, bf), widened(Do, bf)
    assert_tape(args.cpu().numpy(), a_o,
                _pair_sims_fn(Qf, Df, lambda p: (Qf[cu_q[p[0]] - 1: cu_q[p[0] + 1] - 1],
                                                 Df[cu_d[p[0]] - 1: cu_d[p[0] + 1] - 1])), tol)


# ---- known answers from the reference's own tests, on the device ----------------------

def test_all_negative_dots_keep_true_max(device):
    """test_regressions.jl:136-147: q = ones(4,3), d = -ones(4,5) => -12, tape > 0."""
    for dtype in DTYPES:
        q = torch.ones(3, 4, dtype=dtype, device=device)
        d = -torch.ones(5, 4, dtype=dtype, device=device)
        s, a = fm.pair_forward(q, d)
        assert s.item() == -12.0
        assert (a.cpu() == 1).all()


def test_empty_doc_scores_zero_not_neg(device):
    """test_regressions.jl:65-86: a fully masked document contributes 0."""
    rng = np.random.default_rng(11)
    q = torch.from_numpy(tokens(rng, (5, 8))).to(device)
    d = torch.from_numpy(tokens(rng, (6, 8))).to(device)
    dm = torch.zeros(6, dtype=torch.bool, device=device)
    assert fm.maxsim(q, d, None, dm).item() == 0.0
    assert fm.maxsim(q, d, None, dm, normalize=True).item() == 0.0


def test_candidate_neg_and_normalize(device):
    """test_forward.jl:41-49 / test_regressions.jl:25-41: invalid idx => neg, kept by normalize."""
    rng = np.random.default_rng(7)
    Q = torch.from_numpy(tokens(rng, (2, 4, 8))).to(device)
    G = torch.from_numpy(tokens(rng, (4, 5, 8))).to(device)
    idxs = torch.tensor([[1, 0], [2, 1]], dtype=torch.int32, device=device)  # Julia [1 2; 0 1]
    S = fm.maxsim(Q, G, idxs)
    assert S[0, 1].item() == -1.0e4
    Sn = fm.maxsim(Q, G, idxs, normalize=True)
    assert Sn[0, 1].item() == -1.0e4
    assert abs(Sn[0, 0].item() - S[0, 0].item() / 4) < 1e-5


def test_normalize_layouts(device):
    rng = np.random.default_rng(5)
    Q = torch.from_numpy(tokens(rng, (3, 6, 16))).to(device)
    D = torch.from_numpy(tokens(rng, (3, 9, 16))).to(device)
    qm = torch.tensor([[1, 1, 0, 1, 0, 1], [0] * 6, [1] * 6], dtype=torch.bool, device=device)
    s = fm.maxsim(Q, D, qm, None)
    sn = fm.maxsim(Q, D, qm, None, normalize=True)
    inv = 1.0 / torch.clamp(qm.sum(1).float(), min=1.0)
    assert torch.equal(sn, s * inv)
    S = fm.maxsim(Q, D, qm, None, fm.InBatch())
    Sn = fm.maxsim(Q, D, qm, None, fm.InBatch(), normalize=True)
    assert torch.equal(Sn, S * inv[:, None])
    P = fm.pack_docs([D[0], D[1][:4], D[2][:0]])
    sp = fm.maxsim(Q[0], P)
    spn = fm.maxsim(Q[0], P, normalize=True)
    assert torch.equal(spn, sp * (1.0 / 6.0))
    Qp, Dp = fm.pack_pairs([Q[0], Q[1][:2]], [D[0], D[1]])
    sv = fm.maxsim(Qp, Dp)
    svn = fm.maxsim(Qp, Dp, normalize=True)
    assert torch.equal(svn, sv * torch.tensor([1 / 6, 1 / 2], device=device, dtype=torch.float32))


def test_float16_returns_float32_scores(device):
    """test_edge_cases.jl:14-24 and the CUDA WMMA checks (test_cuda.jl:154-172)."""
    rng = np.random.default_rng(20)
    q = torch.from_numpy(tokens(rng, (17, 32))).to(device)
    d = torch.from_numpy(tokens(rng, (23, 32))).to(device)
    s16 = fm.maxsim(q.half(), d.half())
    assert s16.dtype == torch.float32 and s16.numel() == 1
    s32 = fm.maxsim(q, d)
    assert abs(s16.item() - s32.item()) <= 1e-3 * (1 + abs(s32.item()))


def test_host_arrays_are_refused(device):
    """test_cuda.jl:22,90: host masks / host idxs with device features throw ArgumentError."""
    q = torch.randn(4, 8, device=device)
    d = torch.randn(5, 8, device=device)
    with pytest.raises(fm.ArgumentError):
        fm.maxsim(q, d, torch.ones(4, dtype=torch.bool), torch.ones(5, dtype=torch.bool))
    Q = torch.randn(2, 4, 8, device=device)
    G = torch.randn(3, 5, 8, device=device)
    with pytest.raises(fm.ArgumentError):
        fm.maxsim(Q, G, torch.ones(2, 2, dtype=torch.int32))
