"""GPU parity of the pullbacks on the argmax tape: every layout vs the fp64 CPU oracle.

The device pullback is fed the oracle's forward tape (so a forward near-tie
cannot move a gradient row) and cotangents rounded to the feature type; the
oracle gets the same tape and the same rounded values.  Tolerance, per
element: the rounding of the result into the feature type (2^-8 relative for
bf16, 2^-11 for fp16, none for fp32) plus 1e-5 of the absolute sum of the
element's terms (fp32 accumulation; the absolute sum is the oracle run on
|Q|, |D|, |Delta|, |inv_n|), plus one fp16 subnormal step (2^-24) for fp16
results below the normal range.  For fp32 features that is 1e-5 relative
whenever the terms do not cancel.  Outputs are pre-filled with NaN: the
library must overwrite every element.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import as_feature, mask_np, tokens

import flashmaxsim as fm
from flashmaxsim import boundary
from flashmaxsim import backward as bw

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16, torch.float32]
DT_ID = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}
ROUND = {torch.float32: 0.0, torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}
FLOOR = {torch.float32: 1e-38, torch.float16: 2.0 ** -24, torch.bfloat16: 1e-38}


def _abs(a, bf):
    return (a & np.uint16(0x7FFF)) if bf else np.abs(a)


def _vals(rng, shape, dtype, device, positive=False):
    """A feature-type device array and the fp64 values it holds."""
    x = rng.standard_normal(shape).astype(np.float32)
    if positive:
        x = np.abs(x) + 0.05
    t = torch.from_numpy(x).to(dtype)
    return t.to(device), t.float().numpy().astype(np.float64)


def _nan_like(shape, dtype, device):
    return torch.full(shape, float("nan"), dtype=dtype, device=device)


def assert_grad(got, want, mag, dtype, what):
    g = got.float().cpu().numpy().astype(np.float64)
    assert g.shape == want.shape, (what, g.shape, want.shape)
    tol = ROUND[dtype] * np.abs(want) + 1e-5 * mag + FLOOR[dtype]
    bad = ~(np.abs(g - want) <= tol)
    if bad.any():
        i = tuple(np.argwhere(bad)[0])
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} differ; first at {i}: "
                             f"got {g[i]!r} want {want[i]!r} (mag {mag[i]!r})")


def _junk(rng, args, Td):
    """Tape entries the pullback must skip: 0, past Td, negative."""
    a = args.copy()
    flat = a.reshape(-1)
    n = flat.size
    if n >= 3:
        k = rng.choice(n, size=max(1, n // 50) * 3, replace=True)
        flat[k[0::3]] = 0
        flat[k[1::3]] = Td + 3
        flat[k[2::3]] = -2
    return a


# ---- paired / pair --------------------------------------------------------------------------

PAIRED = [(128, 32, 180, 6), (40, 33, 65, 3), (768, 8, 17, 2), (12, 5, 9, 4), (256, 32, 300, 5)]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("shape", PAIRED, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("masks", [False, True], ids=["nomask", "mask"])
def test_paired_pullback_parity(device, dtype, shape, masks):
    dim, Tq, Td, B = shape
    rng = np.random.default_rng([dim, Tq, Td, B, int(masks)])
    Qt, Qo, bf = as_feature(tokens(rng, (B, Tq, dim)), dtype)
    Dt, Do, _ = as_feature(tokens(rng, (B, Td, dim)), dtype)
    qm = rng.random((B, Tq)) < 0.8 if masks else None
    dm = rng.random((B, Td)) < 0.7 if masks else None
    _, args, _ = oracle.paired_forward(Qo, Do, qm, dm, bf16=bf)
    args = _junk(rng, args, Td)
    Dl_t, Dl = _vals(rng, (B,), dtype, device)
    Dl_t[0] = 0.0  # a zero cotangent adds nothing (backward_pair.jl:21)
    Dl[0] = 0.0
    iv_t, iv = _vals(rng, (B,), dtype, device, positive=True)
    want = oracle.paired_backward(Qo, Do, args, Dl, iv, qm, bf16=bf)
    mag = oracle.paired_backward(_abs(Qo, bf), _abs(Do, bf), args, np.abs(Dl), iv, qm, bf16=bf)
    Q, D = Qt.to(device), Dt.to(device)
    dQ, dD = _nan_like(Q.shape, dtype, device), _nan_like(D.shape, dtype, device)
    qmt = None if qm is None else torch.from_numpy(qm).to(device)
    boundary.paired_apply_pullback(dQ, dD, Q, D, qmt, torch.from_numpy(args).to(device), Dl_t, iv_t)
    torch.cuda.synchronize()
    assert_grad(dQ, want[0], mag[0], dtype, "dQ")
    assert_grad(dD, want[1], mag[1], dtype, "dD")
    # the driver (inv_n = None means ones) agrees with the oracle too
    gQ, gD = bw.paired_pullback(Dl_t, Q, D, qmt, torch.from_numpy(args).to(device))
    w1 = oracle.paired_backward(Qo, Do, args, Dl, None, qm, bf16=bf)
    m1 = oracle.paired_backward(_abs(Qo, bf), _abs(Do, bf), args, np.abs(Dl), None, qm, bf16=bf)
    torch.cuda.synchronize()
    assert_grad(gQ, w1[0], m1[0], dtype, "dQ (driver)")
    assert_grad(gD, w1[1], m1[1], dtype, "dD (driver)")


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: DT_ID[d])
def test_pair_pullback_scalar_and_zero(device, dtype):
    rng = np.random.default_rng(11)
    dim, Tq, Td = 64, 9, 23
    qt, qo, bf = as_feature(tokens(rng, (Tq, dim)), dtype)
    dt, do, _ = as_feature(tokens(rng, (Td, dim)), dtype)
    qm = np.array([1, 1, 0, 1, 1, 1, 1, 0, 1], bool)
    _, tape = oracle.pair_forward(qo, do, qm.astype(np.uint8), bf16=bf)[:2]
    delta = float(torch.tensor(0.75).to(dtype))
    q, d = qt.to(device), dt.to(device)
    qmt = torch.from_numpy(qm).to(device)
    tt = torch.from_numpy(np.ascontiguousarray(tape, dtype=np.int32)).to(device)
    dq, dd = bw.pair_pullback(delta, q, d, qmt, tt)
    want = oracle.paired_backward(qo[None], do[None], tape[None], np.array([delta]), None,
                                  qm[None], bf16=bf)
    mag = oracle.paired_backward(_abs(qo, bf)[None], _abs(do, bf)[None], tape[None],
                                 np.array([delta]), None, qm[None], bf16=bf)
    torch.cuda.synchronize()
    assert_grad(dq, want[0][0], mag[0][0], dtype, "dq")
    assert_grad(dd, want[1][0], mag[1][0], dtype, "dd")
    assert (dq.float().cpu()[torch.from_numpy(~qm)] == 0).all()
    z = bw.pair_pullback(torch.zeros(1, dtype=dtype, device=device), q, d, qmt, tt)
    torch.cuda.synchronize()
    assert all((g.float().cpu() == 0).all() for g in z)
    with pytest.raises(fm.DimensionMismatch):
        bw.pair_pullback(torch.ones(2, dtype=dtype, device=device), q, d, qmt, tt)


# ---- in-batch -------------------------------------------------------------------------------

INBATCH = [(128, 32, 64, 8, 12), (40, 7, 13, 5, 3), (96, 16, 300, 17, 9), (1024, 4, 20, 3, 4)]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("shape", INBATCH, ids=lambda s: "x".join(map(str, s)))
def test_inbatch_pullback_parity(device, dtype, shape):
    dim, Tq, Td, Bq, Bd = shape
    rng = np.random.default_rng([dim, Tq, Td, Bq, Bd])
    Qt, Qo, bf = as_feature(tokens(rng, (Bq, Tq, dim)), dtype)
    Dt, Do, _ = as_feature(tokens(rng, (Bd, Td, dim)), dtype)
    qm = rng.random((Bq, Tq)) < 0.85
    dm = rng.random((Bd, Td)) < 0.75
    _, args = oracle.inbatch_forward(Qo, Do, qm, dm, bf16=bf)
    args = _junk(rng, args, Td)
    Dl_t, Dl = _vals(rng, (Bq, Bd), dtype, device)
    iv_t, iv = _vals(rng, (Bq,), dtype, device, positive=True)
    want = oracle.inbatch_backward(Qo, Do, args, Dl, iv, qm, bf16=bf)
    mag = oracle.inbatch_backward(_abs(Qo, bf), _abs(Do, bf), args, np.abs(Dl), iv, qm, bf16=bf)
    Q, D = Qt.to(device), Dt.to(device)
    qmt = torch.from_numpy(qm).to(device)
    dQ, dD = _nan_like(Q.shape, dtype, device), _nan_like(D.shape, dtype, device)
    at = torch.from_numpy(args).to(device)
    boundary.inbatch_apply_pullback(dQ, dD, Q, D, qmt, at, Dl_t, iv_t)
    torch.cuda.synchronize()
    assert_grad(dQ, want[0], mag[0], dtype, "dQ")
    assert_grad(dD, want[1], mag[1], dtype, "dD")
    # dQ is a gather in pair order: bit-identical on a second run
    gQ, _ = bw.inbatch_pullback(Dl_t, Q, D, qmt, at, iv_t)
    torch.cuda.synchronize()
    assert torch.equal(gQ.cpu(), dQ.cpu())


# (dim, Tq, Td, Bq, Bd) for the in-batch feature-half path (16-bit features, Td <= 255):
# half rows of 4, 8 and 16 chunks (dim 64, 128, 256); 4, 2 and 1 documents per dQ
# step; Tq not a multiple of 4 (the byte tape from single-entry loads); Tq over one
# token block (32 tokens at dim 128, 16 at dim 256); Td = 255, the largest entry a
# byte holds; ragged and empty document quarters (Bd = 13, 3, 2); the C3 shape.
HALF = [(128, 32, 180, 24, 13), (64, 7, 255, 9, 6), (256, 16, 90, 10, 5),
        (256, 20, 180, 6, 3), (128, 40, 33, 12, 2), (128, 32, 180, 512, 512)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("shape", HALF, ids=lambda s: "x".join(map(str, s)))
def test_inbatch_pullback_feature_halves(device, dtype, shape):
    """A random tape (with junk entries), a query mask and some zero cotangents."""
    dim, Tq, Td, Bq, Bd = shape
    rng = np.random.default_rng([11, dim, Tq, Td, Bq, Bd])
    Qt, Qo, bf = as_feature(tokens(rng, (Bq, Tq, dim)), dtype)
    Dt, Do, _ = as_feature(tokens(rng, (Bd, Td, dim)), dtype)
    qm = rng.random((Bq, Tq)) < 0.85
    args = _junk(rng, rng.integers(0, Td + 1, size=(Bq, Bd, Tq)).astype(np.int32), Td)
    Dl_t, Dl = _vals(rng, (Bq, Bd), dtype, device)
    zero = rng.random((Bq, Bd)) < 0.05
    Dl[zero] = 0.0
    Dl_t[torch.from_numpy(zero).to(device)] = 0.0
    iv_t, iv = _vals(rng, (Bq,), dtype, device, positive=True)
    want = oracle.inbatch_backward(Qo, Do, args, Dl, iv, qm, bf16=bf)
    mag = oracle.inbatch_backward(_abs(Qo, bf), _abs(Do, bf), args, np.abs(Dl), iv, qm, bf16=bf)
    Q, D = Qt.to(device), Dt.to(device)
    qmt = torch.from_numpy(qm).to(device)
    dQ, dD = _nan_like(Q.shape, dtype, device), _nan_like(D.shape, dtype, device)
    at = torch.from_numpy(args).to(device)
    boundary.inbatch_apply_pullback(dQ, dD, Q, D, qmt, at, Dl_t, iv_t)
    torch.cuda.synchronize()
    assert_grad(dQ, want[0], mag[0], dtype, "dQ")
    assert_grad(dD, want[1], mag[1], dtype, "dD")
    gQ, _ = bw.inbatch_pullback(Dl_t, Q, D, qmt, at, iv_t)
    torch.cuda.synchronize()
    assert torch.equal(gQ.cpu(), dQ.cpu())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("shape", [(128, 32, 64, 8, 12), (128, 40, 33, 12, 2)],
                         ids=lambda s: "x".join(map(str, s)))
def test_inbatch_pullback_nonfinite_cotangent(device, dtype, shape):
    """NaN and +-inf cotangents reach exactly the rows their sources reach (a token
    with no source stays finite, src/backward_pair.jl:21-29); the rest within tolerance."""
    dim, Tq, Td, Bq, Bd = shape
    rng = np.random.default_rng([13, dim, Tq, Td, Bq, Bd])
    Qt, Qo, bf = as_feature(tokens(rng, (Bq, Tq, dim)), dtype)
    Dt, Do, _ = as_feature(tokens(rng, (Bd, Td, dim)), dtype)
    qm = rng.random((Bq, Tq)) < 0.85
    args = rng.integers(0, Td + 1, size=(Bq, Bd, Tq)).astype(np.int32)
    args[1, 0, :Tq // 2] = 0  # a pair whose tokens partly have no source
    Dl_t, Dl = _vals(rng, (Bq, Bd), dtype, device)
    for (i, j), v in zip([(1, 0), (3, Bd - 1), (Bq - 1, 1)], [np.nan, np.inf, -np.inf]):
        Dl[i, j] = v
        Dl_t[i, j] = float(v)
    iv_t, iv = _vals(rng, (Bq,), dtype, device, positive=True)
    want = oracle.inbatch_backward(Qo, Do, args, Dl, iv, qm, bf16=bf)
    fin = np.where(np.isfinite(Dl), np.abs(Dl), 0.0)
    mag = oracle.inbatch_backward(_abs(Qo, bf), _abs(Do, bf), args, fin, iv, qm, bf16=bf)
    Q, D = Qt.to(device), Dt.to(device)
    qmt = torch.from_numpy(qm).to(device)
    dQ, dD = _nan_like(Q.shape, dtype, device), _nan_like(D.shape, dtype, device)
    boundary.inbatch_apply_pullback(dQ, dD, Q, D, qmt, torch.from_numpy(args).to(device), Dl_t, iv_t)
    torch.cuda.synchronize()
    for got, w, m, what in ((dQ, want[0], mag[0], "dQ"), (dD, want[1], mag[1], "dD")):
        g = got.float().cpu().numpy().astype(np.float64)
        for cls in (np.isnan, np.isposinf, np.isneginf):
            assert np.array_equal(cls(g), cls(w)), (what, cls.__name__, int(cls(g).sum()), int(cls(w).sum()))
        ok = np.isfinite(w)
        assert ok.sum() > 0 and (~ok).sum() > 0
        err = np.abs(g[ok] - w[ok])
        tol = ROUND[dtype] * np.abs(w[ok]) + 1e-5 * m[ok] + FLOOR[dtype]
        assert (err <= tol).all(), (what, float((err - tol).max()))


# ---- candidates -----------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("shape", [(128, 32, 180), (40, 33, 65), (8, 6, 7)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64], ids=["i32", "i64"])
def test_candidates_pullback_parity(device, dtype, shape, idx_dtype):
    dim, Tq, Td = shape
    N, C, B = 23, 9, 5
    rng = np.random.default_rng(dim * 1000 + Tq * 10 + Td)
    Qt, Qo, bf = as_feature(tokens(rng, (B, Tq, dim)), dtype)
    Gt, Go, _ = as_feature(tokens(rng, (N, Td, dim)), dtype)
    idx = rng.integers(1, N + 1, size=(B, C)).astype(np.int64)
    idx[0, 2] = 0
    idx[3, 0] = N + 1
    idx[4, 8] = -5
    idx[1, :3] = 7  # one document three times for one query, and for others too
    idx[2, 5] = 7
    qm = rng.random((B, Tq)) < 0.9
    dm = np.array([[(u + 1) % 4 != 0 for u in range(Td)] for _ in range(N)])
    _, args, _ = oracle.candidates_forward(Qo, Go, idx, qm, dm, -1.0e4, bf16=bf)
    args = _junk(rng, args, Td)
    Dl_t, Dl = _vals(rng, (B, C), dtype, device)
    iv_t, iv = _vals(rng, (B,), dtype, device, positive=True)
    want = oracle.candidates_backward(Qo, Go, idx, args, Dl, iv, qm, bf16=bf)
    mag = oracle.candidates_backward(_abs(Qo, bf), _abs(Go, bf), idx, args, np.abs(Dl), iv, qm,
                                     bf16=bf)
    Q, G = Qt.to(device), Gt.to(device)
    idx_t = torch.from_numpy(idx).to(idx_dtype).to(device)
    dQ, dG = _nan_like(Q.shape, dtype, device), _nan_like(G.shape, dtype, device)
    boundary.candidates_apply_pullback(dQ, dG, Q, G, idx_t, torch.from_numpy(qm).to(device),
                                       torch.from_numpy(args).to(device), Dl_t, iv_t)
    torch.cuda.synchronize()
    assert_grad(dQ, want[0], mag[0], dtype, "dQ")
    assert_grad(dG, want[1], mag[1], dtype, "dG")
    # gallery documents no valid index names get exact zeros
    unused = sorted(set(range(1, N + 1)) - set(idx[(idx >= 1) & (idx <= N)].tolist()))
    for j in unused:
        assert (dG[j - 1].float().cpu() == 0).all()


# ---- packed / varlen ------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("case", ["small", "colpali", "splitd"])
def test_packed_pullback_parity(device, dtype, case):
    rng = np.random.default_rng({"small": 31, "colpali": 4, "splitd": 44}[case])
    if case == "small":
        dim, Tq, lens = 16, 7, [5, 0, 3, 9, 1, 33, 64, 65]
    elif case == "colpali":
        dim, Tq, lens = 128, 24, list(rng.integers(700, 1101, size=12))
        lens[3] = 0
    else:
        dim, Tq, lens = 1024, 24, [40, 0, 97, 3]
    q32 = tokens(rng, (Tq, dim))
    qt, qo, bf = as_feature(q32, dtype)
    tok_t, tok_o, _ = as_feature(np.concatenate([tokens(rng, (n, dim)) for n in lens], 0), dtype)
    cu = np.concatenate([[1], 1 + np.cumsum(lens)]).astype(np.int32)
    qm = rng.random(Tq) < 0.9
    _, args, _ = oracle.packed_forward(qo, tok_o, cu, qm.astype(np.uint8), bf16=bf)
    args = _junk(rng, args, 1)  # (Td differs per document; 0 and -2 are always skipped)
    B = len(lens)
    Dl_t, Dl = _vals(rng, (B,), dtype, device)
    inv = float(torch.tensor(1.0 / max(qm.sum(), 1)).to(dtype))
    want = oracle.packed_backward(qo, tok_o, cu, args, Dl, inv, qm, bf16=bf)
    mag = oracle.packed_backward(_abs(qo, bf), _abs(tok_o, bf), cu, args, np.abs(Dl), inv, qm,
                                 bf16=bf)
    P = fm.PackedSeq(tok_t, torch.from_numpy(cu)).to(device)
    q = qt.to(device)
    dq, dP = bw.packed_pullback(Dl_t, q, P, torch.from_numpy(qm).to(device),
                                torch.from_numpy(args).to(device), inv)
    torch.cuda.synchronize()
    assert_grad(dq, want[0], mag[0], dtype, "dq")
    assert_grad(dP, want[1], mag[1], dtype, "dP")


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: DT_ID[d])
def test_varlen_pullback_parity(device, dtype):
    rng = np.random.default_rng(32)
    dim = 12 if dtype == torch.float32 else 64
    qlens = [4, 2, 35, 1, 0, 7]
    dlens = [5, 3, 70, 0, 4, 33]
    Qt, Qo, bf = as_feature(np.concatenate([tokens(rng, (n, dim)) for n in qlens], 0), dtype)
    Dt, Do, _ = as_feature(np.concatenate([tokens(rng, (n, dim)) for n in dlens], 0), dtype)
    cu_q = np.concatenate([[1], 1 + np.cumsum(qlens)]).astype(np.int32)
    cu_d = np.concatenate([[1], 1 + np.cumsum(dlens)]).astype(np.int32)
    max_q = max(qlens)
    _, args, _ = oracle.varlen_forward(Qo, Do, cu_q, cu_d, max_q, bf16=bf)
    args = _junk(rng, args, max(dlens))
    N = len(qlens)
    Dl_t, Dl = _vals(rng, (N,), dtype, device)
    iv_t, iv = _vals(rng, (N,), dtype, device, positive=True)
    want = oracle.varlen_backward(Qo, Do, cu_q, cu_d, args, Dl, iv, bf16=bf)
    mag = oracle.varlen_backward(_abs(Qo, bf), _abs(Do, bf), cu_q, cu_d, args, np.abs(Dl), iv,
                                 bf16=bf)
    Qp = fm.PackedSeq(Qt, torch.from_numpy(cu_q)).to(device)
    Dp = fm.PackedSeq(Dt, torch.from_numpy(cu_d)).to(device)
    dQ, dD = bw.varlen_pullback(Dl_t, Qp, Dp, torch.from_numpy(args).to(device), iv_t)
    torch.cuda.synchronize()
    assert_grad(dQ, want[0], mag[0], dtype, "dQ")
    assert_grad(dD, want[1], mag[1], dtype, "dD")


# ---- end to end and size-independent properties --------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_inbatch_forward_then_pullback(device, dtype):
    """The device forward's own tape drives the pullback; the oracle pulls back on the
    same tape (a near-tie the forward broke differently is the forward's choice)."""
    rng = np.random.default_rng(77)
    dim, Tq, Td, Bq, Bd = 128, 32, 300, 16, 16
    Qt, Qo, bf = as_feature(tokens(rng, (Bq, Tq, dim)), dtype)
    Dt, Do, _ = as_feature(tokens(rng, (Bd, Td, dim)), dtype)
    Q, D = Qt.to(device), Dt.to(device)
    S, args = fm.inbatch_forward(Q, D)
    Dl_t, Dl = _vals(rng, (Bq, Bd), dtype, device)
    dQ, dD = bw.inbatch_pullback(Dl_t, Q, D, None, args)
    a = args.cpu().numpy()
    want = oracle.inbatch_backward(Qo, Do, a, Dl, None, None, bf16=bf)
    mag = oracle.inbatch_backward(_abs(Qo, bf), _abs(Do, bf), a, np.abs(Dl), None, None, bf16=bf)
    torch.cuda.synchronize()
    assert_grad(dQ, want[0], mag[0], dtype, "dQ")
    assert_grad(dD, want[1], mag[1], dtype, "dD")


def test_pullback_linear_in_cotangent_at_size(device):
    """At the in-batch benchmark's per-query shape (dim 128, Tq 32, Td 300) with 128
    queries and documents: pb(2*D1 + D2) == 2*pb(D1) + pb(D2) in fp32 features."""
    rng = np.random.default_rng(5)
    dim, Tq, Td, B = 128, 32, 300, 128
    Q = torch.from_numpy(tokens(rng, (B, Tq, dim))).to(device)
    D = torch.from_numpy(tokens(rng, (B, Td, dim))).to(device)
    _, args = fm.inbatch_forward(Q, D)
    d1 = torch.randn(B, B, device=device, generator=torch.Generator(device).manual_seed(1))
    d2 = torch.randn(B, B, device=device, generator=torch.Generator(device).manual_seed(2))
    a = bw.inbatch_pullback(d1, Q, D, None, args)
    b = bw.inbatch_pullback(d2, Q, D, None, args)
    c = bw.inbatch_pullback(2 * d1 + d2, Q, D, None, args)
    ma = bw.inbatch_pullback(d1.abs(), Q.abs(), D.abs(), None, args)
    mb = bw.inbatch_pullback(d2.abs(), Q.abs(), D.abs(), None, args)
    for x, y, z, u, v in zip(a, b, c, ma, mb):
        err = (z - (2 * x + y)).abs()
        assert (err <= 1e-5 * (2 * u + v) + 1e-30).all(), float(err.max())


def test_pullback_empty_and_degenerate(device):
    dt = torch.float16
    Q = torch.randn(3, 4, 8, device=device).to(dt)
    D = torch.randn(5, 6, 8, device=device).to(dt)
    # Bq = 0: dD exists and is zero
    dQ0, dD0 = bw.inbatch_pullback(torch.zeros(0, 5, device=device), Q[:0], D, None,
                                   torch.zeros(0, 5, 4, dtype=torch.int32, device=device))
    torch.cuda.synchronize()
    assert dQ0.shape == (0, 4, 8) and (dD0.float().cpu() == 0).all()
    # Td = 0: no source at all, dQ zero
    dQ1, dD1 = bw.inbatch_pullback(torch.ones(3, 5, device=device), Q, D[:, :0], None,
                                   torch.zeros(3, 5, 4, dtype=torch.int32, device=device))
    torch.cuda.synchronize()
    assert (dQ1.float().cpu() == 0).all() and dD1.shape == (5, 0, 8)
    # an all-zero tape: both gradients zero
    dQ2, dD2 = bw.inbatch_pullback(torch.ones(3, 5, device=device), Q, D, None,
                                   torch.zeros(3, 5, 4, dtype=torch.int32, device=device))
    torch.cuda.synchronize()
    assert (dQ2.float().cpu() == 0).all() and (dD2.float().cpu() == 0).all()
    # B = 0 candidates over a non-empty gallery: dG zero
    G = torch.randn(7, 6, 8, device=device).to(dt)
    dQ3, dG3 = bw.candidates_pullback(torch.zeros(0, 2, device=device), Q[:0], G,
                                      torch.zeros(0, 2, dtype=torch.int64, device=device), None,
                                      torch.zeros(0, 2, 4, dtype=torch.int32, device=device))
    torch.cuda.synchronize()
    assert (dG3.float().cpu() == 0).all()
    # shape errors raise before any launch
    with pytest.raises(fm.DimensionMismatch):
        bw.paired_pullback(torch.ones(2, device=device), Q, D[:3], None,
                           torch.zeros(3, 4, dtype=torch.int32, device=device))
    with pytest.raises(fm.DimensionMismatch):
        bw.paired_pullback(torch.ones(3, device=device), Q, D[:3], None,
                           torch.zeros(3, 5, dtype=torch.int32, device=device))
