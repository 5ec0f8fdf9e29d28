"""GPU parity for the INT8 path: quantiser and int32 dots bit-exact, and per
query-token partials / tapes exactly equal to the oracle (the dequantised
cell score (qs*ds)*Float32(acc) is evaluated in the same order on both
sides, so every cell is bit-identical)."""
import numpy as np
import pytest
import torch

import oracle
from helpers import mask_np, tokens

import flashmaxsim as fm
from flashmaxsim import boundary

pytestmark = pytest.mark.gpu


def _edge_tokens():
    """Hand-made tokens that hit the quantiser's corner cases (quant.jl:21-49)."""
    rows = [
        np.zeros(16, np.float32),                                     # absmax 0 -> eps floor
        np.full(16, 1e-12, np.float32),                               # below eps
        np.array([127.0, 63.5, -63.5, 0.5, -0.5, 1.5, -2.5, 2.5] * 2, np.float32) / 127.0,
        np.array([1.0, -1.0] * 8, np.float32),
        np.array([3.0e38, -3.0e38] + [1.0] * 14, np.float32),
        np.array([1e-38, 2e-38] * 8, np.float32),                     # subnormal-range scale
    ]
    return np.stack(rows)


@pytest.mark.parametrize("dim", [16, 128, 40, 7])
def test_quantize_bit_exact(device, dim):
    rng = np.random.default_rng(dim)
    x = rng.standard_normal((300, dim)).astype(np.float32) * rng.uniform(1e-3, 1e3, (300, 1)).astype(np.float32)
    if dim == 16:
        x = np.concatenate([x, _edge_tokens()], 0)
    c_o, s_o = oracle.quantize_int8(x)
    idx = fm.quantize_int8_symmetric(torch.from_numpy(x).to(device))
    torch.cuda.synchronize()
    assert np.array_equal(idx.scales.cpu().numpy().view(np.uint32), s_o.view(np.uint32))
    assert np.array_equal(idx.codes.cpu().numpy(), c_o)


@pytest.mark.parametrize("shape", [(128, 32, 180), (16, 8, 11), (40, 33, 65), (1024, 5, 40), (7, 3, 4)])
def test_int8_dots_bit_exact(device, shape):
    dim, Tq, Td = shape
    rng = np.random.default_rng(Tq * Td)
    qc = rng.integers(-127, 128, size=(Tq, dim)).astype(np.int8)
    dc = rng.integers(-127, 128, size=(Td, dim)).astype(np.int8)
    want = oracle.int8_dots(qc, dc)
    out = torch.zeros(Tq, Td, dtype=torch.int32, device=device)
    boundary.int8_dots(out, torch.from_numpy(qc).to(device), torch.from_numpy(dc).to(device))
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), want)
    # numpy int64 matmul as an independent check of the oracle itself
    assert np.array_equal(want.astype(np.int64), qc.astype(np.int64) @ dc.astype(np.int64).T)


@pytest.mark.parametrize("shape", [(128, 32, 180, 4), (16, 8, 11, 3), (40, 33, 65, 2)])
def test_int8_paired_exact(device, shape):
    dim, Tq, Td, B = shape
    rng = np.random.default_rng(dim + Tq)
    Q = tokens(rng, (B, Tq, dim))
    D = tokens(rng, (B, Td, dim))
    Dc, Ds = oracle.quantize_int8(D)
    Qc, Qs = oracle.quantize_int8(Q)
    qm = rng.random((B, Tq)) < 0.9
    dm = rng.random((B, Td)) < 0.8
    s_o, a_o, p_o = oracle.int8_paired_forward(Qc, Qs, Dc, Ds, qm.astype(np.uint8), dm.astype(np.uint8))
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    args = torch.zeros(B, Tq, dtype=torch.int32, device=device)
    part = torch.zeros(B, Tq, dtype=torch.float32, device=device)
    scores = torch.zeros(B, dtype=torch.float32, device=device)
    boundary.launch_int8_paired_scan(args, part, dev(Qc), dev(Qs), dev(Dc), dev(Ds), dev(qm), dev(dm), scores)
    torch.cuda.synchronize()
    assert np.array_equal(args.cpu().numpy(), a_o)
    assert np.array_equal(part.cpu().numpy().view(np.uint32), p_o.view(np.uint32))
    np.testing.assert_allclose(scores.cpu().numpy(), s_o, rtol=1e-6, atol=1e-6)
    # public API: on-device query quantisation + scan == the same numbers
    D8 = fm.Int8Index(dev(Dc), dev(Ds))
    s_api = fm.maxsim(dev(Q), D8, dev(qm), dev(dm))
    torch.cuda.synchronize()
    np.testing.assert_allclose(s_api.cpu().numpy(), s_o, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64])
def test_int8_candidates_exact(device, idx_dtype):
    dim, Tq, Td, N, C, B = 128, 32, 180, 40, 11, 6
    rng = np.random.default_rng(55)
    Q = tokens(rng, (B, Tq, dim))
    G = tokens(rng, (N, Td, dim))
    Gc, Gs = oracle.quantize_int8(G)
    Qc, Qs = oracle.quantize_int8(Q)
    idx = rng.integers(1, N + 1, size=(B, C)).astype(np.int64)
    idx[1, 3] = 0
    idx[5, 10] = N + 7
    dm = np.arange(Td)[None, :] < rng.integers(1, Td + 1, size=(N, 1))
    S_o, a_o, p_o = oracle.int8_candidates_forward(Qc, Qs, Gc, Gs, idx, None, dm.astype(np.uint8))
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    args = torch.zeros(B, C, Tq, dtype=torch.int32, device=device)
    part = torch.zeros(B, C, Tq, dtype=torch.float32, device=device)
    S = torch.zeros(B, C, dtype=torch.float32, device=device)
    boundary.launch_int8_candidates_scan(args, part, dev(Qc), dev(Qs), dev(Gc), dev(Gs),
                                         dev(idx).to(idx_dtype), None, dev(dm), N, S, -1.0e4)
    torch.cuda.synchronize()
    assert np.array_equal(args.cpu().numpy(), a_o)
    assert np.array_equal(part.cpu().numpy().view(np.uint32), p_o.view(np.uint32))
    np.testing.assert_allclose(S.cpu().numpy(), S_o, rtol=1e-6, atol=1e-6)
    assert S.cpu()[1, 3].item() == -1.0e4 and S.cpu()[5, 10].item() == -1.0e4


def test_int8_matches_dequantised_fp(device):
    """test_int8.jl:22-44: INT8 score == fp MaxSim of dequantised inputs (rtol 1e-5)."""
    rng = np.random.default_rng(40)
    q = torch.from_numpy(tokens(rng, (8, 16), normalize=False)).to(device)
    d = torch.from_numpy(tokens(rng, (11, 16), normalize=False)).to(device)
    d_idx = fm.quantize_int8_symmetric(d)
    q_idx = fm.quantize_int8_symmetric(q)
    s8 = fm.maxsim(q, d_idx)
    s_hat = fm.maxsim(fm.dequant_int8(q_idx), fm.dequant_int8(d_idx))
    assert abs(s8.item() - s_hat.item()) <= 1e-5 * (1 + abs(s_hat.item()))
    assert abs(fm.maxsim(q, d_idx, normalize=True).item() - s_hat.item() / 8) <= 1e-5 * (1 + abs(s_hat.item()))


def test_int8_index_at_rest_scans_identically(device, tmp_path):
    """A gallery quantised on the device, saved (save_int8_index) and loaded
    back onto the device, scores bit-identically to the in-memory index."""
    rng = np.random.default_rng(21)
    B, Tq, Td, dim = 3, 8, 21, 64
    Q = torch.from_numpy(tokens(rng, (B, Tq, dim))).to(device)
    D = torch.from_numpy(tokens(rng, (B, Td, dim))).to(device)
    idx8 = fm.quantize_int8_symmetric(D)
    path = str(tmp_path / "g.safetensors")
    fm.save_int8_index(idx8, path)
    back = fm.load_int8_index(path, device)
    assert back.codes.device.type == "cuda"
    s0 = fm.maxsim(Q, idx8)
    s1 = fm.maxsim(Q, back)
    assert torch.equal(s0, s1)


# ---- Float16 features: scales in Float16 (quant.jl:42-49 computes in T) ------------------

def _edge_tokens_f16():
    """Float16 corner cases: zero and tiny tokens (scale floored at floatmin(Float16)),
    the largest finite half, ties of x / scale at .5, subnormal inputs."""
    rows = [
        np.zeros(16, np.float32),
        np.full(16, 1e-7, np.float32),
        np.array([127.0, 63.5, -63.5, 0.5, -0.5, 1.5, -2.5, 2.5] * 2, np.float32),
        np.array([65504.0, -65504.0] + [1.0] * 14, np.float32),
        np.array([3e-6, -6e-8] * 8, np.float32),
        np.array([100.0, 3.0, 7.0, 11.0, -13.0, 0.1, 50.0, 99.0] * 2, np.float32),
    ]
    return np.stack(rows).astype(np.float16)


@pytest.mark.parametrize("dim", [16, 128, 40])
def test_quantize_f16_bit_exact(device, dim):
    rng = np.random.default_rng(100 + dim)
    x = (rng.standard_normal((400, dim)) * rng.uniform(1e-3, 1e3, (400, 1))).astype(np.float16)
    if dim == 16:
        x = np.concatenate([x, _edge_tokens_f16()], 0)
    c_o, s_o = oracle.quantize_int8(x)
    idx = fm.quantize_int8_symmetric(torch.from_numpy(x).to(device))
    torch.cuda.synchronize()
    assert idx.scales.dtype == torch.float16
    assert np.array_equal(idx.scales.cpu().numpy().view(np.uint16), s_o.view(np.uint16))
    assert np.array_equal(idx.codes.cpu().numpy(), c_o)


@pytest.mark.parametrize("dim", [128, 1024, 40])
@pytest.mark.parametrize("qs_type,ds_type", [(np.float16, np.float16), (np.float32, np.float16),
                                             (np.float16, np.float32)])
def test_int8_f16_scales_exact(device, dim, qs_type, ds_type):
    """Paired and candidate scans with Float16 scales on either side (the fast, split-d
    and generic kernels): tapes and partials bit-identical to the oracle, which widens
    the scales to fp32 and evaluates (qs * ds) * Float32(acc) (kernels_int8.jl:17-25)."""
    rng = np.random.default_rng(dim + 7)
    B, Tq, Td, N, C = 5, 20, 45, 6, 4
    Qf = tokens(rng, (B, Tq, dim))
    Df = tokens(rng, (B, Td, dim))
    Gf = tokens(rng, (N, Td, dim))
    Qc, Qs = oracle.quantize_int8(Qf.astype(qs_type))
    Dc, Ds = oracle.quantize_int8(Df.astype(ds_type))
    Gc, Gs = oracle.quantize_int8(Gf.astype(ds_type))
    assert Qs.dtype == qs_type and Ds.dtype == ds_type
    qm = rng.random((B, Tq)) < 0.9
    dm = rng.random((B, Td)) < 0.85
    gm = rng.random((N, Td)) < 0.85
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    # paired
    s_o, a_o, p_o = oracle.int8_paired_forward(Qc, Qs, Dc, Ds, qm.astype(np.uint8), dm.astype(np.uint8))
    args = torch.zeros(B, Tq, dtype=torch.int32, device=device)
    part = torch.zeros(B, Tq, dtype=torch.float32, device=device)
    scores = torch.zeros(B, dtype=torch.float32, device=device)
    boundary.launch_int8_paired_scan(args, part, dev(Qc), dev(Qs), dev(Dc), dev(Ds), dev(qm),
                                     dev(dm), scores)
    torch.cuda.synchronize()
    assert np.array_equal(args.cpu().numpy(), a_o)
    assert np.array_equal(part.cpu().numpy().view(np.uint32), p_o.view(np.uint32))
    np.testing.assert_allclose(scores.cpu().numpy(), s_o, rtol=1e-6, atol=1e-6)
    # candidates (output order and document order)
    idx = rng.integers(0, N + 1, size=(B, C)).astype(np.int64)
    S_o, ac_o, pc_o = oracle.int8_candidates_forward(Qc, Qs, Gc, Gs, idx, qm.astype(np.uint8),
                                                     gm.astype(np.uint8), neg=-5.0)
    for order in ("never", "always"):
        prev = boundary.candidates_grouping(order)
        try:
            ac = torch.zeros(B, C, Tq, dtype=torch.int32, device=device)
            pc = torch.zeros(B, C, Tq, dtype=torch.float32, device=device)
            S = torch.zeros(B, C, dtype=torch.float32, device=device)
            boundary.launch_int8_candidates_scan(ac, pc, dev(Qc), dev(Qs), dev(Gc), dev(Gs),
                                                 dev(idx), dev(qm), dev(gm), N, S, -5.0)
            torch.cuda.synchronize()
        finally:
            boundary.candidates_grouping(prev)
        assert np.array_equal(ac.cpu().numpy(), ac_o), order
        assert np.array_equal(pc.cpu().numpy().view(np.uint32), pc_o.view(np.uint32)), order
        np.testing.assert_allclose(S.cpu().numpy(), S_o, rtol=1e-6, atol=1e-6)


def test_maxsim_float16_features_on_int8_index(device):
    """maxsim(Q::Float16, D::Int8Index) end to end: Q quantised on the device in Float16,
    the index quantised from Float16 features (Float16 scales); the same numbers as the
    oracle quantising and scanning the same bytes."""
    rng = np.random.default_rng(71)
    B, Tq, Td, dim = 6, 32, 90, 128
    Q16 = tokens(rng, (B, Tq, dim)).astype(np.float16)
    D16 = tokens(rng, (B, Td, dim)).astype(np.float16)
    D8 = fm.quantize_int8_symmetric(torch.from_numpy(D16).to(device))
    got = fm.maxsim(torch.from_numpy(Q16).to(device), D8)
    torch.cuda.synchronize()
    Qc, Qs = oracle.quantize_int8(Q16)
    Dc, Ds = oracle.quantize_int8(D16)
    s_o, _, _ = oracle.int8_paired_forward(Qc, Qs, Dc, Ds)
    assert got.dtype == torch.float32
    np.testing.assert_allclose(got.cpu().numpy(), s_o, rtol=1e-6, atol=1e-6)
