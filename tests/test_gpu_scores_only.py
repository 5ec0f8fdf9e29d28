"""GPU: scores without the argmax tape (args null), and every maxsim verb without one.

The reference's ``maxsim(Q, D, qmask, dmask, InBatch())`` keeps S and drops the
tape (``S, _ = inbatch_forward(...)``, dispatch.jl:124).  Called with args null,
the in-batch and multi-query packed MFMA kernels keep a running maximum alone
(no argmax).  Their S must be bit-identical to the tape kernels' S on the same
inputs -- the same maxima summed in the same order -- and within the feature
type's tolerance of the oracle.  The cases cover every stream the kernel has:
16-row units with split entries (short documents), masked runs inside
documents, exact duplicate tokens, all-negative maxima, empty documents, query
tiles past 32 tokens, four queries in three tiles (Tq = 24), 2 to 8 k-blocks,
the fused normalisation, the NaN first-token rule, and the split-K kernel
(dim 256, fp32), which takes a null args as well.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import FEATURE_TOL, as_feature, assert_scores, mask_np, tokens

import flashmaxsim as fm
from flashmaxsim import boundary

pytestmark = pytest.mark.gpu

DT_ID = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}


def _inbatch_inputs(rng, dim, Tq, Td, Bq, Bd, kind):
    q32 = tokens(rng, (Bq, Tq, dim))
    d32 = tokens(rng, (Bd, Td, dim))
    if kind == "negative":  # every dot product below zero
        q32, d32 = np.abs(q32), -np.abs(d32)
    for j in range(0, Bd, 2):  # later rows copy earlier ones: exact ties
        a, b = np.sort(rng.choice(Td, 2, replace=False)) if Td > 1 else (0, 0)
        d32[j, b] = d32[j, a]
    if kind == "holes":
        dm = np.zeros((Bd, Td), bool)
        for j in range(Bd):
            for _ in range(rng.integers(0, 4)):
                a = int(rng.integers(0, Td))
                dm[j, a:a + int(rng.integers(1, 12))] = True
    elif kind == "short":  # a third of the documents within one 16-row unit
        lens = rng.integers(0, Td + 1, Bd)
        lens[::3] = rng.integers(1, 17, len(lens[::3]))
        dm = np.arange(Td)[None, :] < lens[:, None]
    else:
        lens = rng.integers(min(Td, 3), Td + 1, Bd)
        dm = np.arange(Td)[None, :] < lens[:, None]
    dm[0, :] = False  # an empty document scores 0
    qm = rng.random((Bq, Tq)) < 0.9
    return q32, d32, qm, dm


INBATCH = [
    # (dim, Tq, Td, Bq, Bd, mask kind)
    (128, 32, 180, 40, 96, "prefix"),      # the C3 shape, smaller batch
    (128, 32, 100, 17, 45, "holes"),
    (64, 32, 40, 20, 96, "short"),         # split entries: a close inside a chunk
    (32, 16, 48, 64, 640, "prefix"),       # 40 documents per block
    (96, 24, 65, 17, 9, "prefix"),         # Tq = 24: four queries in three tiles
    (128, 40, 65, 33, 9, "holes"),         # query tiles of 32 and 8
    (128, 8, 300, 20, 17, "negative"),
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("shape", INBATCH, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("normalize", [False, True], ids=["raw", "norm"])
def test_inbatch_scores_only_match_tape_path(device, dtype, shape, normalize):
    dim, Tq, Td, Bq, Bd, kind = shape
    rng = np.random.default_rng(dim + 7 * Tq + Td + Bq + Bd)
    q32, d32, qm, dm = _inbatch_inputs(rng, dim, Tq, Td, Bq, Bd, kind)
    Qt, Qo, bf = as_feature(q32, dtype)
    Dt, Do, _ = as_feature(d32, dtype)
    Q, D = Qt.to(device), Dt.to(device)
    qmt, dmt = torch.from_numpy(qm).to(device), torch.from_numpy(dm).to(device)
    S_t, args = fm.inbatch_forward(Q, D, qmt, dmt, normalize=normalize)
    S_s, none = fm.inbatch_forward(Q, D, qmt, dmt, normalize=normalize, tape=False)
    torch.cuda.synchronize()
    assert none is None
    assert torch.equal(S_s, S_t), (S_s - S_t).abs().max().item()
    S_o, _ = oracle.inbatch_forward(Qo, Do, mask_np(torch.from_numpy(qm)),
                                    mask_np(torch.from_numpy(dm)), bf16=bf)
    if normalize:
        S_o = S_o / np.maximum(qm.sum(1), 1)[:, None]
    assert_scores(S_s.cpu(), S_o, FEATURE_TOL[dtype], what="S (no tape) vs oracle")
    assert (S_s.cpu().numpy()[:, 0] == 0).all()
    if kind == "negative":
        assert (S_o[:, 1:] < 0).all()
    # the public verb takes this path (it drops the tape, as the reference's does)
    S_m = fm.maxsim(Q, D, qmt, dmt, fm.InBatch(), normalize=normalize)
    assert torch.equal(S_m, S_t)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=lambda d: DT_ID[d])
def test_inbatch_split_k_takes_null_args(device, dtype):
    """dim 256 (and fp32 at any dim) runs the split-K kernel: a null args gives the
    same S."""
    rng = np.random.default_rng(256)
    q32, d32, qm, dm = _inbatch_inputs(rng, 256, 32, 70, 20, 30, "holes")
    Qt, _, _ = as_feature(q32, dtype)
    Dt, _, _ = as_feature(d32, dtype)
    Q, D = Qt.to(device), Dt.to(device)
    qmt, dmt = torch.from_numpy(qm).to(device), torch.from_numpy(dm).to(device)
    S_t, _ = fm.inbatch_forward(Q, D, qmt, dmt)
    S_s, _ = fm.inbatch_forward(Q, D, qmt, dmt, tape=False)
    torch.cuda.synchronize()
    assert torch.equal(S_s, S_t)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("dim,Tq", [(128, 24), (64, 24), (128, 40), (96, 16)],
                         ids=lambda v: str(v))
def test_packed_multi_scores_only_match_tape_path(device, dtype, dim, Tq):
    rng = np.random.default_rng(dim * 3 + Tq)
    lens = [5, 0, 1, 31, 32, 33, 64, 65, 0, 200, 17] + list(rng.integers(700, 1101, size=4))
    nq = 40
    Qt, Qo, bf = as_feature(tokens(rng, (nq, Tq, dim)), dtype)
    tt, to, _ = as_feature(np.concatenate([tokens(rng, (n, dim)) for n in lens], 0), dtype)
    cu = np.concatenate([[1], 1 + np.cumsum(lens)]).astype(np.int32)
    qm = rng.random((nq, Tq)) < 0.9
    P = fm.PackedSeq(tt, torch.from_numpy(cu)).to(device)
    Q, qmt = Qt.to(device), torch.from_numpy(qm).to(device)
    S_t, _ = fm.packed_multi_forward(Q, P, qmt)
    S_s, none = fm.packed_multi_forward(Q, P, qmt, tape=False)
    torch.cuda.synchronize()
    assert none is None
    assert torch.equal(S_s, S_t), (S_s - S_t).abs().max().item()
    for i in (0, 17, nq - 1):
        s_o, _, _ = oracle.packed_forward(Qo[i], to, cu, qm[i].astype(np.uint8), bf16=bf)
        assert_scores(S_s[i].cpu(), s_o, FEATURE_TOL[dtype], what=f"query {i} vs oracle")
    assert torch.equal(fm.maxsim(Q, P, qmt), S_t)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=lambda d: DT_ID[d])
def test_inbatch_scores_only_nonfinite(device, dtype):
    """The NaN first-token rule (kernels_forward.jl:49-52) without a tape: a NaN at a
    document's first valid row, or in a valid query token, makes the score NaN; a
    NaN row later is skipped; -Inf and +Inf classes as the tape path gives them."""
    rng = np.random.default_rng(17)
    Bq, Bd, Tq, Td, dim = 40, 37, 24, 70, 128
    Q = tokens(rng, (Bq, Tq, dim))
    D = tokens(rng, (Bd, Td, dim))
    qm = np.ones((Bq, Tq), bool)
    dm = np.ones((Bd, Td), bool)
    qm[5, 20:] = False
    dm[3, :9] = False
    D[3, 9, 11] = np.nan                     # first valid row of document 3
    D[7, 0, 0] = np.inf                      # first row of document 7
    D[7, 1:, 0] = np.where(np.abs(D[7, 1:, 0]) < 0.05, 0.2, D[7, 1:, 0])
    D[12, 40, 2] = np.nan                    # a NaN row in the middle: skipped
    dm[20, :] = False                        # an empty document
    Q[1, 3, 0] = np.nan
    Q[33, 0, 0] = -np.inf
    Q[5, 22, 1] = np.nan                     # a masked NaN token
    Qt, Qo, bf = as_feature(Q, dtype)
    Dt, Do, _ = as_feature(D, dtype)
    Qd, Dd = Qt.to(device), Dt.to(device)
    qmt, dmt = torch.from_numpy(qm).to(device), torch.from_numpy(dm).to(device)
    S_t = torch.zeros(Bq, Bd, dtype=torch.float32, device=device)
    S_s = torch.zeros(Bq, Bd, dtype=torch.float32, device=device)
    args = torch.zeros(Bq, Bd, Tq, dtype=torch.int32, device=device)
    boundary.inbatch_device_scan(S_t, args, Qd, Dd, qmt, dmt)
    boundary.inbatch_device_scan(S_s, None, Qd, Dd, qmt, dmt)
    torch.cuda.synchronize()
    st, ss = S_t.cpu().numpy(), S_s.cpu().numpy()
    assert np.array_equal(st, ss, equal_nan=True)
    S_o, _ = oracle.inbatch_forward(Qo, Do, qm.astype(np.uint8), dm.astype(np.uint8), bf16=bf)
    assert np.array_equal(np.isnan(ss), np.isnan(S_o))
    assert np.isnan(ss[:, 3]).all() and np.isfinite(ss[0, 12]) and ss[0, 20] == 0.0


# ---- every maxsim verb: S without a tape ----------------------------------------------

def _mask(rng, n, T, p, device):
    m = rng.random((n, T)) < p
    m[:, 0] = True
    return torch.from_numpy(m).to(device)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32],
                         ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("layout", ["pair", "paired", "candidates_grouped", "candidates_ordered",
                                    "packed", "varlen"])
@pytest.mark.parametrize("normalize", [False, True], ids=["raw", "norm"])
def test_maxsim_makes_no_tape(device, dtype, layout, normalize):
    """The reference's maxsim drops the tape for every layout (src/dispatch.jl:44, 83,
    164, 201, 229): maxsim here makes none (tape=False, null args), and its scores are
    bit-identical to the drivers' with the tape."""
    rng = np.random.default_rng(sum(map(ord, layout + DT_ID[dtype])) + int(normalize))
    dim, Tq, Td = 128, 32, 96
    dev = lambda x: as_feature(x, dtype)[0].to(device)  # noqa: E731
    if layout == "pair":
        q, d = dev(tokens(rng, (Tq, dim))), dev(tokens(rng, (Td, dim)))
        qm, dm = _mask(rng, 1, Tq, 0.9, device)[0], _mask(rng, 1, Td, 0.8, device)[0]
        want, _ = fm.pair_forward(q, d, qm, dm, normalize=normalize)
        got, none = fm.pair_forward(q, d, qm, dm, normalize=normalize, tape=False)
        verb = fm.maxsim(q, d, qm, dm, normalize=normalize)
    elif layout == "paired":
        B = 37
        Q, D = dev(tokens(rng, (B, Tq, dim))), dev(tokens(rng, (B, Td, dim)))
        qm, dm = _mask(rng, B, Tq, 0.9, device), _mask(rng, B, Td, 0.8, device)
        want, _ = fm.paired_forward(Q, D, qm, dm, normalize=normalize)
        got, none = fm.paired_forward(Q, D, qm, dm, normalize=normalize, tape=False)
        verb = fm.maxsim(Q, D, qm, dm, normalize=normalize)
    elif layout.startswith("candidates"):
        B, C, N = 24, 40, 300
        Q, G = dev(tokens(rng, (B, Tq, dim))), dev(tokens(rng, (N, Td, dim)))
        idx = torch.from_numpy(rng.integers(0, N + 2, size=(B, C))).to(device)
        qm, dm = _mask(rng, B, Tq, 0.9, device), _mask(rng, N, Td, 0.8, device)
        prev = boundary.candidates_grouping("always" if layout.endswith("grouped") else "never")
        try:
            want, _ = fm.candidates_forward(Q, G, idx, qm, dm, -7.0, normalize=normalize)
            got, none = fm.candidates_forward(Q, G, idx, qm, dm, -7.0, normalize=normalize,
                                              tape=False)
            verb = fm.maxsim(Q, G, idx, qm, dm, neg=-7.0, normalize=normalize)
        finally:
            boundary.candidates_grouping(prev)
    elif layout == "packed":
        lens = [5, 0, 33, 64, 200, 1]
        q = dev(tokens(rng, (Tq, dim)))
        tt = as_feature(np.concatenate([tokens(rng, (n, dim)) for n in lens], 0), dtype)[0]
        cu = torch.from_numpy(np.concatenate([[1], 1 + np.cumsum(lens)]).astype(np.int32))
        P = fm.PackedSeq(tt, cu).to(device)
        qm = _mask(rng, 1, Tq, 0.9, device)[0]
        want, _ = fm.packed_forward(q, P, qm, normalize=normalize)
        got, none = fm.packed_forward(q, P, qm, normalize=normalize, tape=False)
        verb = fm.maxsim(q, P, qm, normalize=normalize)
    else:  # varlen
        ql, dl = [7, 32, 1, 40], [50, 3, 90, 0]
        qt = as_feature(np.concatenate([tokens(rng, (n, dim)) for n in ql], 0), dtype)[0]
        dt = as_feature(np.concatenate([tokens(rng, (n, dim)) for n in dl], 0), dtype)[0]
        cq = torch.from_numpy(np.concatenate([[1], 1 + np.cumsum(ql)]).astype(np.int32))
        cd = torch.from_numpy(np.concatenate([[1], 1 + np.cumsum(dl)]).astype(np.int32))
        Qp, Dp = fm.PackedSeq(qt, cq).to(device), fm.PackedSeq(dt, cd).to(device)
        want, _ = fm.varlen_forward(Qp, Dp, normalize=normalize)
        got, none = fm.varlen_forward(Qp, Dp, normalize=normalize, tape=False)
        verb = fm.maxsim(Qp, Dp, normalize=normalize)
    torch.cuda.synchronize()
    assert none is None
    assert torch.equal(got, want) and torch.equal(verb, want)


@pytest.mark.parametrize("layout", ["pair", "paired", "candidates"])
def test_int8_maxsim_makes_no_tape(device, layout):
    """The INT8 verbs (src/dispatch.jl:261, 287; candidates: no reference method) without
    the tape: scores bit-identical to the drivers' with it."""
    rng = np.random.default_rng({"pair": 81, "paired": 82, "candidates": 83}[layout])
    dim, Tq, Td = 128, 32, 96
    if layout == "pair":
        q = torch.from_numpy(tokens(rng, (Tq, dim))).to(device)
        d = fm.quantize_int8_symmetric(torch.from_numpy(tokens(rng, (Td, dim))).to(device))
        want, _ = fm.int8_pair_forward(q, d)
        got, none = fm.int8_pair_forward(q, d, tape=False)
        verb = fm.maxsim(q, d)
    elif layout == "paired":
        B = 21
        Q = torch.from_numpy(tokens(rng, (B, Tq, dim))).to(device)
        D = fm.quantize_int8_symmetric(torch.from_numpy(tokens(rng, (B, Td, dim))).to(device))
        want, _ = fm.int8_paired_forward(Q, D)
        got, none = fm.int8_paired_forward(Q, D, tape=False)
        verb = fm.maxsim(Q, D)
    else:
        B, C, N = 16, 30, 200
        Q = torch.from_numpy(tokens(rng, (B, Tq, dim))).to(device)
        G = fm.quantize_int8_symmetric(torch.from_numpy(tokens(rng, (N, Td, dim))).to(device))
        idx = torch.from_numpy(rng.integers(0, N + 2, size=(B, C))).to(device)
        want, _ = fm.int8_candidates_forward(Q, G, idx, neg=-3.0)
        got, none = fm.int8_candidates_forward(Q, G, idx, neg=-3.0, tape=False)
        verb = fm.maxsim(Q, G, idx, neg=-3.0)
    torch.cuda.synchronize()
    assert none is None
    assert torch.equal(got, want) and torch.equal(verb, want)
