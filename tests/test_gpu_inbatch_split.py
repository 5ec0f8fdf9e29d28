"""GPU parity of the split-K in-batch kernel (csrc/fms_inbatch_split.hip): fp32
features, and 16-bit feature dims whose query tiles do not fit in registers
(past 128) or are not whole 32-feature blocks.  The reference scores the same
layout with D'Q chunks and an argmax-accumulate (src/forward_layouts.jl:202-225)
and tests split-d at d = 768 (test/test_forward.jl:93-108).  Every case first
checks that the call takes the split-K kernel, then compares scores and tapes
with the oracle (tapes equal except at near-ties within the score tolerance)."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from helpers import FEATURE_TOL, as_feature, assert_scores, assert_tape, mask_np, tokens, widened

import flashmaxsim as fm
from flashmaxsim import _lib

pytestmark = pytest.mark.gpu

DT_ID = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}
CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def _kernel(Q, D):
    Bq, Tq, dim = Q.shape
    Bd, Td = D.shape[0], D.shape[1]
    return _lib.lib().fms_debug_inbatch_kernel(CODE[Q.dtype], dim, Tq, Td, Bq, Bd,
                                               ctypes.c_void_p(Q.data_ptr()),
                                               ctypes.c_void_p(D.data_ptr()))


def _tape_check(got, a_o, Qf, Df, tol):
    """assert_tape over (Bq, Bd, Tq) tapes: mismatches only at near-ties (the
    similarity row of query token t of pair (i, j) is D_j @ Q_i[t])."""
    def sims(idx):
        i, j, t = idx
        return Df[j] @ Qf[i][t]
    assert_tape(got, a_o, sims, tol)


def _run(device, dtype, dim, Tq, Td, Bq, Bd, seed, ties=False, normalize=False):
    rng = np.random.default_rng(seed)
    q32 = tokens(rng, (Bq, Tq, dim))
    d32 = tokens(rng, (Bd, Td, dim))
    dm = rng.random((Bd, Td)) < 0.8
    if Td > 1:
        dm[0, :] = False                       # no valid token: score 0, tape 0
        dm[min(1, Bd - 1), : Td // 2] = False  # leading masked tokens
    if ties:
        for j in range(Bd):  # later rows copy earlier ones: exact ties keep the first
            for _ in range(3):
                if Td > 1:
                    a, b = np.sort(rng.choice(Td, 2, replace=False))
                    d32[j, b] = d32[j, a]
    Qt, Qo, bf = as_feature(q32, dtype)
    Dt, Do, _ = as_feature(d32, dtype)
    qm = torch.from_numpy(rng.random((Bq, Tq)) < 0.9)
    dmt = torch.from_numpy(dm)
    Qd, Dd = Qt.to(device), Dt.to(device)
    assert _kernel(Qd, Dd) == 2, "the split-K in-batch kernel serves this call"
    S, args = fm.inbatch_forward(Qd, Dd, qm.to(device), dmt.to(device), normalize=normalize)
    torch.cuda.synchronize()
    S_o, a_o = oracle.inbatch_forward(Qo, Do, mask_np(qm), mask_np(dmt), bf16=bf)
    if normalize:  # 1 / max(valid query tokens, 1) in fp32 (normalize.jl:4-10)
        n = qm.numpy().sum(axis=1).astype(np.float32)
        S_o = (S_o * (np.float32(1.0) / np.maximum(n, np.float32(1.0)))[:, None]).astype(np.float32)
    tol = FEATURE_TOL[dtype]
    assert_scores(S.cpu(), S_o, tol, what="S")
    if Td > 1:
        assert (S.cpu().numpy()[:, 0] == 0).all()
    got = args.cpu().numpy()
    ii, jj, tt = np.nonzero(got)
    assert dm[jj, got[ii, jj, tt] - 1].all(), "every recorded token is a valid one"
    Qf, Df = widened(Qo, bf), widened(Do, bf)
    _tape_check(got, a_o, Qf, Df, tol)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32],
                         ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("shape", [(32, 180, 24, 21), (7, 65, 9, 6), (70, 33, 5, 7),
                                   (32, 400, 11, 5), (24, 1, 8, 9)],
                         ids=lambda s: "x".join(map(str, s)))
def test_split_d768(device, dtype, shape):
    """d = 768 (test_forward.jl:93-108's split-d dim) in three float types: query
    tiles of 7, 24, 32 and 70 tokens (three tiles), documents of 1 to 400 tokens
    (three chunk groups), masked documents and exact duplicate tokens."""
    Tq, Td, Bq, Bd = shape
    _run(device, dtype, 768, Tq, Td, Bq, Bd, seed=Tq * 1000 + Td, ties=True)


@pytest.mark.parametrize("dtype,dim", [(torch.float16, 40), (torch.float16, 160),
                                       (torch.bfloat16, 192), (torch.float16, 256),
                                       (torch.bfloat16, 1024), (torch.float32, 4),
                                       (torch.float32, 36), (torch.float32, 128),
                                       (torch.float32, 100), (torch.float32, 256)],
                         ids=lambda v: DT_ID.get(v, str(v)) if isinstance(v, torch.dtype) else f"d{v}")
def test_split_dims(device, dtype, dim):
    """Dims whose rows end inside a 128-byte K slice (the last slice's units past the
    row read zeros) and dims of one to sixteen slices."""
    _run(device, dtype, dim, 32, 100, 13, 11, seed=dim * 7 + CODE[dtype], ties=True)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("shape", [(8, 40, 300, 64, 256), (40, 400, 75, 40, 72)],
                         ids=lambda s: "x".join(map(str, s)))
def test_split_many_items_per_block(device, dtype, shape):
    """A block walks many (document, query group) items in turn, its loads
    running ahead across item and chunk-group boundaries: 300 queries of 8
    tokens (the last group's rows past query 299 hold no query) x 64
    documents is some 2,400 items for 256 blocks; 75 queries of 40 tokens (two
    tiles each, 150 rows) x 40 documents of 400 tokens (three chunk groups)
    at d = 72.  Every item must start from a clean running max, whatever the
    block's previous item was."""
    Tq, Td, Bq, Bd, dim = shape
    _run(device, dtype, dim, Tq, Td, Bq, Bd, seed=Tq * 7 + Bq, ties=True)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=lambda d: DT_ID[d])
def test_split_normalize(device, dtype):
    """The normalize epilogue (1 / max(valid query tokens, 1), normalize.jl:4-10) for
    one tile per query and for queries of several tiles (summed after the scan)."""
    _run(device, dtype, 384, 32, 90, 9, 10, seed=5, normalize=True)
    _run(device, dtype, 384, 50, 90, 9, 10, seed=6, normalize=True)


def test_split_no_tape_and_negative_maxima(device):
    """args = None writes scores only; all-negative dots keep the first valid token
    (test_regressions.jl:136-147: q = ones, d = -ones gives -Tq per pair)."""
    dim, Tq, Td, Bq, Bd = 768, 3, 5, 2, 3
    Q = torch.ones(Bq, Tq, dim, dtype=torch.float32, device=device)
    D = -torch.ones(Bd, Td, dim, dtype=torch.float32, device=device)
    assert _kernel(Q, D) == 2
    S, args = fm.inbatch_forward(Q, D)
    torch.cuda.synchronize()
    assert torch.equal(S.cpu(), torch.full((Bq, Bd), -3.0 * dim))
    assert (args.cpu() == 1).all()
    S2 = torch.zeros(Bq, Bd, dtype=torch.float32, device=device)
    from flashmaxsim import boundary
    boundary.inbatch_device_scan(S2, None, Q, D, None, None)
    torch.cuda.synchronize()
    assert torch.equal(S2.cpu(), S.cpu())


def test_split_c3_shape_d768_sampled(device):
    """The C3 configuration at d = 768 (512 queries x 512 documents, lengths
    U[64, 180], fp16): the full launch, with 6 queries x all 512 documents checked
    against the oracle."""
    dim, Tq, Td, Bq, Bd = 768, 32, 180, 512, 512
    gen = torch.Generator(device=device)
    gen.manual_seed(33)
    Q = torch.randn(Bq, Tq, dim, generator=gen, device=device)
    Q = (Q / Q.norm(dim=-1, keepdim=True)).to(torch.float16)
    D = torch.randn(Bd, Td, dim, generator=gen, device=device)
    D = (D / D.norm(dim=-1, keepdim=True)).to(torch.float16)
    lens = torch.randint(64, Td + 1, (Bd,), generator=gen, device=device)
    dmask = torch.arange(Td, device=device)[None, :] < lens[:, None]
    assert _kernel(Q, D) == 2
    S, args = fm.inbatch_forward(Q, D, None, dmask)
    torch.cuda.synchronize()
    rows = np.array([0, 1, 99, 256, 400, 511])
    Qo = Q[torch.from_numpy(rows).to(device)].cpu().numpy()
    S_o, a_o = oracle.inbatch_forward(Qo, D.cpu().numpy(), None, mask_np(dmask.cpu()))
    tol = FEATURE_TOL[torch.float16]
    assert_scores(S.cpu()[rows], S_o, tol, what="S")
    Qf, Df = widened(Qo, False), widened(D.cpu().numpy(), False)
    _tape_check(args.cpu().numpy()[rows], a_o, Qf, Df, tol)


@pytest.mark.parametrize("Tq", [20, 45], ids=lambda t: f"Tq{t}")
def test_split_empty_documents(device, Tq):
    """Documents with no tokens (Td = 0): every pair scores 0 and the tape is
    all zeros, with one tile per query and with two (summed after the scan),
    normalised or not (test_regressions.jl:65-86: an empty document gives 0).
    The host API answers Td = 0 itself; the boundary call here reaches the
    kernel, with the outputs filled beforehand so that every write shows."""
    from flashmaxsim import boundary
    dim, Bq, Bd = 256, 3, 5
    Q = torch.randn(Bq, Tq, dim, device=device).to(torch.float16)
    D = torch.empty(Bd, 0, dim, dtype=torch.float16, device=device)
    assert _kernel(Q, D) == 2
    for normalize in (False, True):
        S = torch.full((Bq, Bd), 7.0, device=device)
        args = torch.full((Bq, Bd, Tq), 5, dtype=torch.int32, device=device)
        boundary.inbatch_device_scan(S, args, Q, D, None, None, normalize)
        torch.cuda.synchronize()
        assert torch.equal(S.cpu(), torch.zeros(Bq, Bd))
        assert (args.cpu() == 0).all()

