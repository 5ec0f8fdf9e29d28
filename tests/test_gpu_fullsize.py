"""GPU parity at the benchmark configurations' full sizes, plus the reference's
generator-independent property tests.

* C2: all 256,000 candidate pairs over the 100,000-document fp16 gallery
  against the full oracle (the grouped document-batch scan).
* C3: the in-batch launch at its exact shape (512 x 512, Tq 32, Td 180,
  document lengths U[64, 180]) against the full oracle.
* C4: one Lq = 24 bf16 query against all 20,000 packed documents (lengths
  U[700, 1100]), 64 documents at d = 1024 (the split-d kernel), and the
  multi-query packed scan of 64 queries with two rows checked in full.
* C5: the 10^6-document INT8 gallery generated and quantised on the device;
  256 sampled pairs' tapes and per-token partials bit-exact.
* Sister documents (test_edge_cases.jl:26-107) through pair, paired,
  candidates, in-batch, packed and varlen; INT8 ranking vs fp32
  (test_int8.jl:46-59).

Large inputs are drawn on the device (torch Philox, seeded) and copied to the
host once; the oracle sees the same bytes.  Bars: fp16/bf16 scores within
2e-3 relative, tapes equal except at near-ties, INT8 partials and tapes
bit-exact.
"""
import numpy as np
import pytest
import torch

import oracle
import sisters
from helpers import FEATURE_TOL, as_feature, assert_scores, assert_tape, mask_np, tokens, widened

import flashmaxsim as fm
from flashmaxsim import boundary
from flashmaxsim import forward as F

pytestmark = pytest.mark.gpu


def dev_tokens(shape, gen, dtype, device, chunk_rows=1 << 20):
    """randn token rows, L2-normalised in fp32 on the device, stored as dtype."""
    out = torch.empty(shape, dtype=dtype, device=device)
    flat = out.view(-1, shape[-1])
    eps = torch.finfo(torch.float32).eps
    for a in range(0, flat.shape[0], chunk_rows):
        b = min(flat.shape[0], a + chunk_rows)
        x = torch.randn(b - a, shape[-1], generator=gen, device=device, dtype=torch.float32)
        x /= torch.sqrt((x * x).sum(-1, keepdim=True) + eps)
        flat[a:b] = x.to(dtype)
    return out


def host_bits(t):
    """Host numpy copy as the oracle takes it (bf16 as uint16 bits)."""
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def test_c2_candidates_all_pairs(device):
    dim, Lq, Ld, C, B, N = 128, 32, 180, 1000, 256, 100_000
    gen = torch.Generator(device=device)
    gen.manual_seed(12)
    G = dev_tokens((N, Ld, dim), gen, torch.float16, device)
    Q = dev_tokens((B, Lq, dim), gen, torch.float16, device)
    idx = torch.randint(1, N + 1, (B, C), generator=gen, device=device, dtype=torch.int64)
    flat = torch.randperm(C * B, generator=gen, device=device)[:(C * B) // 100]
    idx.view(-1)[flat] = 0
    S, args = F.candidates_forward(Q, G, idx, None, None, -1.0e4)
    torch.cuda.synchronize()
    Gh, Qh, idx_h = G.cpu().numpy(), Q.cpu().numpy(), idx.cpu().numpy()
    del G
    S_o, a_o, _ = oracle.candidates_forward(Qh, Gh, idx_h, None, None, -1.0e4)
    assert_scores(S.cpu(), S_o, FEATURE_TOL[torch.float16], what="S")
    assert (S.cpu().numpy()[idx_h == 0] == np.float32(-1.0e4)).all()

    def sims(i):
        b, c, t = i
        return Gh[idx_h[b, c] - 1].astype(np.float64) @ Qh[b, t].astype(np.float64)
    n = assert_tape(args.cpu().numpy(), a_o, sims, FEATURE_TOL[torch.float16])
    print(f"c2: {C * B} pairs, {n} near-tie tape cells")


def test_c3_inbatch_exact_shape(device):
    dim, Tq, Td, Bq, Bd = 128, 32, 180, 512, 512
    rng = np.random.default_rng(3)
    Qt, Qo, _ = as_feature(tokens(rng, (Bq, Tq, dim)), torch.float16)
    Dt, Do, _ = as_feature(tokens(rng, (Bd, Td, dim)), torch.float16)
    lens = rng.integers(64, Td + 1, size=Bd)
    dm = torch.from_numpy(np.arange(Td)[None, :] < lens[:, None])
    S, args = F.inbatch_forward(Qt.to(device), Dt.to(device), None, dm.to(device))
    Sn = fm.maxsim(Qt.to(device), Dt.to(device), None, dm.to(device), fm.InBatch(),
                   normalize=True)
    torch.cuda.synchronize()
    S_o, a_o = oracle.inbatch_forward(Qo, Do, None, mask_np(dm))
    tol = FEATURE_TOL[torch.float16]
    assert_scores(S.cpu(), S_o, tol, what="S")
    assert_scores(Sn.cpu(), S_o / Tq, tol, what="S normalised")
    Qf, Df = widened(Qo, False), widened(Do, False)
    n = assert_tape(args.cpu().numpy(), a_o, lambda i: Df[i[1]] @ Qf[i[0], i[2]], tol)
    assert (args.cpu().numpy() <= lens[None, :, None]).all()
    print(f"c3: {Bq * Bd} pairs, {n} near-tie tape cells")


def _packed_store(device, nd, dim, seed):
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    lens = torch.randint(700, 1101, (nd,), generator=gen, device=device)
    cu = torch.ones(nd + 1, dtype=torch.int32, device=device)
    cu[1:] += torch.cumsum(lens, 0).to(torch.int32)
    ntok = int(lens.sum().item())
    tok = dev_tokens((ntok, dim), gen, torch.bfloat16, device)
    return gen, cu, tok, int(lens.max().item())


def _packed_sims(tok_h, cu_h, q):
    qf = widened(q, True)

    def sims(i):
        b, t = i
        d = widened(tok_h[cu_h[b] - 1:cu_h[b + 1] - 1], True)
        return d @ qf[t]
    return sims


def test_c4_packed_full_store(device):
    """One query against all 20,000 documents (single-query scan), and the
    multi-query scan of 64 queries with rows 0 and 41 checked in full."""
    dim, Lq, nd, nq = 128, 24, 20_000, 64
    gen, cu, tok, max_len = _packed_store(device, nd, dim, 4)
    Qs = dev_tokens((nq, Lq, dim), gen, torch.bfloat16, device)
    P = fm.PackedSeq(tok, cu, max_len)
    s1, a1 = F.packed_forward(Qs[0], P)
    Sm, am = F.packed_multi_forward(Qs, P)
    torch.cuda.synchronize()
    tok_h, cu_h = host_bits(tok), cu.cpu().numpy()
    del P, tok
    tol = FEATURE_TOL[torch.bfloat16]
    for i, (s, a) in [(0, (s1, a1)), (0, (Sm[0], am[0])), (41, (Sm[41], am[41]))]:
        q = host_bits(Qs[i])
        s_o, a_o, _ = oracle.packed_forward(q, tok_h, cu_h, None, bf16=True)
        assert_scores(s.cpu(), s_o, tol, what=f"packed scores q{i}")
        n = assert_tape(a.cpu().numpy(), a_o, _packed_sims(tok_h, cu_h, q), tol)
        print(f"c4 q{i}: {nd} documents, {n} near-tie tape cells")


def test_c4_packed_d1024(device):
    dim, Lq, nd = 1024, 24, 64
    gen, cu, tok, max_len = _packed_store(device, nd, dim, 41)
    q = dev_tokens((Lq, dim), gen, torch.bfloat16, device)
    s, a = F.packed_forward(q, fm.PackedSeq(tok, cu, max_len))
    torch.cuda.synchronize()
    tok_h, cu_h, qh = host_bits(tok), cu.cpu().numpy(), host_bits(q)
    s_o, a_o, _ = oracle.packed_forward(qh, tok_h, cu_h, None, bf16=True)
    tol = FEATURE_TOL[torch.bfloat16]
    assert_scores(s.cpu(), s_o, tol, what="packed d1024 scores")
    assert_tape(a.cpu().numpy(), a_o, _packed_sims(tok_h, cu_h, qh), tol)


def test_c5_int8_gallery_1e6(device):
    dim, Lq, Ld, C, B, N = 128, 32, 180, 1000, 256, 1_000_000
    gen = torch.Generator(device=device)
    gen.manual_seed(5)
    Gc = torch.empty(N, Ld, dim, dtype=torch.int8, device=device)
    Gs = torch.empty(N, Ld, dtype=torch.float32, device=device)
    for a in range(0, N, 20_000):
        b = min(N, a + 20_000)
        x = dev_tokens((b - a, Ld, dim), gen, torch.float32, device)
        boundary.int8_quantize(x, Gc[a:b], Gs[a:b])
        del x
    Qf = dev_tokens((B, Lq, dim), gen, torch.float32, device)
    idx = torch.randint(1, N + 1, (B, C), generator=gen, device=device, dtype=torch.int64)
    Qc = torch.empty(B, Lq, dim, dtype=torch.int8, device=device)
    Qs = torch.empty(B, Lq, dtype=torch.float32, device=device)
    boundary.int8_quantize(Qf, Qc, Qs)
    args = torch.zeros(B, C, Lq, dtype=torch.int32, device=device)
    part = torch.zeros(B, C, Lq, dtype=torch.float32, device=device)
    S = torch.zeros(B, C, dtype=torch.float32, device=device)
    boundary.launch_int8_candidates_scan(args, part, Qc, Qs, Gc, Gs, idx, None, None, N, S,
                                         -1.0e4)
    torch.cuda.synchronize()
    # the device quantiser is the oracle's, bit for bit, on the queries
    qc_o, qs_o = oracle.quantize_int8(Qf.cpu().numpy())
    assert np.array_equal(Qc.cpu().numpy(), qc_o)
    assert np.array_equal(Qs.cpu().numpy().view(np.uint32), qs_o.view(np.uint32))
    # 256 sampled pairs, as a compact candidates problem over their queries/documents
    rng = np.random.default_rng(0)
    pairs = np.sort(rng.choice(B * C, 256, replace=False))
    idx_h = idx.cpu().numpy()
    b, c = pairs // C, pairs % C
    j = idx_h[b, c]
    ub, bi = np.unique(b, return_inverse=True)
    uj, ji = np.unique(j, return_inverse=True)
    idx_c = np.zeros((len(ub), C), np.int64)
    idx_c[bi, c] = ji + 1
    keep = bi * C + c
    uj_t = torch.from_numpy(uj - 1).to(device)
    S_o, a_o, p_o = oracle.int8_candidates_forward(qc_o[ub], qs_o[ub], Gc[uj_t].cpu().numpy(),
                                                   Gs[uj_t].cpu().numpy(), idx_c, None, None,
                                                   -1.0e4, subset=keep)
    pt = torch.from_numpy(pairs).to(device)
    a_g = args.view(B * C, Lq)[pt].cpu().numpy()
    p_g = part.view(B * C, Lq)[pt].cpu().numpy()
    s_g = S.view(-1)[pt].cpu().numpy()
    assert np.array_equal(a_g, a_o.reshape(-1, Lq)[keep])
    assert np.array_equal(p_g.view(np.uint32), p_o.reshape(-1, Lq)[keep].view(np.uint32))
    np.testing.assert_allclose(s_g, S_o.reshape(-1)[keep], rtol=1e-6, atol=1e-6)


# ---- sister documents (test_edge_cases.jl:26-107) -------------------------------------

def _f16(device, *xs):
    return [torch.from_numpy(x.astype(np.float16)).to(device) for x in xs]


def test_sister_documents_every_layout(device):
    q, d, sis = sisters.sister_pair()
    gap64 = sisters.maxsim_dense(q, d) - sisters.maxsim_dense(q, sis)
    assert 1e-4 < gap64 < 0.02
    q16, d16, s16 = _f16(device, q, d, sis)
    sa, sb = fm.maxsim(q16, d16), fm.maxsim(q16, s16)
    assert sa.dtype == torch.float32 and sb.dtype == torch.float32
    sa, sb = sa.item(), sb.item()
    assert sa > sb and abs(sa - sb) < sisters.f16_ulp(sa)
    D = torch.stack([d16, s16])
    Q1 = q16[None]
    paired = fm.maxsim(torch.cat([Q1, Q1]), D)
    assert paired.dtype == torch.float32 and paired[0] > paired[1]
    Sc = fm.maxsim(Q1, D, torch.tensor([[1, 2]], dtype=torch.int32, device=device))
    assert Sc.dtype == torch.float32 and Sc[0, 0] > Sc[0, 1] and Sc[0, 0] != Sc[0, 1]
    Sib = fm.maxsim(Q1, D, fm.InBatch())
    assert Sib.dtype == torch.float32 and Sib[0, 0] > Sib[0, 1]
    sp = fm.maxsim(q16, fm.pack_docs([d16, s16]))
    assert sp.dtype == torch.float32 and sp[0] > sp[1]
    Qp, Dp = fm.pack_pairs([q16, q16], [d16, s16])
    sv = fm.maxsim(Qp, Dp)
    assert sv.dtype == torch.float32 and sv[0] > sv[1]
    # every layout returns the same two scores to within the fp16 bar
    for s in (paired, Sc[0], Sib[0], sp, sv):
        assert np.allclose(s.cpu().numpy(), [sa, sb], rtol=2e-3, atol=0)
        assert (s[0] - s[1]).item() > 0


def test_sister_ladder_every_layout(device):
    q, docs = sisters.sister_ladder()
    s64 = np.array([sisters.maxsim_dense(q, d) for d in docs])
    assert (np.abs(np.diff(s64)) < sisters.F16_ULP_AT_32).all()
    order64 = np.argsort(-s64)
    q16, = _f16(device, q)
    D = torch.stack(_f16(device, *docs))
    n = len(docs)
    layouts = {
        "pair": torch.stack([fm.maxsim(q16, D[i]) for i in range(n)]),
        "paired": fm.maxsim(q16[None].expand(n, -1, -1).contiguous(), D),
        "candidates": fm.maxsim(q16[None], D, torch.arange(1, n + 1, device=device)[None]),
        "inbatch": fm.maxsim(q16[None], D, fm.InBatch()),
        "packed": fm.maxsim(q16, fm.pack_docs(list(D))),
    }
    for name, s in layouts.items():
        s = s.reshape(-1).cpu().numpy()
        assert s.dtype == np.float32, name
        assert (np.diff(s) < 0).all(), (name, s)
        assert (np.argsort(-s) == order64).all(), name
        assert len(np.unique(s)) == n, name
        assert len(np.unique(s.astype(np.float16))) < n, name


# ---- INT8 ranking vs fp32 (test_int8.jl:46-59) -----------------------------------------

@pytest.mark.parametrize("shape", [(32, 12, 20, 64), (128, 32, 180, 1000)],
                         ids=["ref_32x12x20x64", "c5_128x32x180x1000"])
def test_int8_ranking_vs_fp32(device, shape):
    dim, Tq, Td, N = shape
    rng = np.random.default_rng(41)
    q = torch.from_numpy(tokens(rng, (Tq, dim))).to(device)
    G = torch.from_numpy(tokens(rng, (N, Td, dim))).to(device)
    idx = torch.arange(1, N + 1, device=device)[None]
    s_fp = fm.maxsim(q[None], G, idx)[0].cpu().numpy()
    s_i8 = fm.maxsim(q[None], fm.quantize_int8_symmetric(G), idx)[0].cpu().numpy()
    if N <= 64:  # the reference's per-document calls
        one = [fm.maxsim(q, fm.quantize_int8_symmetric(G[j])).item() for j in range(N)]
        np.testing.assert_allclose(np.float32(one), s_i8, rtol=1e-6, atol=1e-6)
    assert sisters.spearman(s_fp, s_i8) >= 0.95
    assert sisters.topk_overlap(s_fp, s_i8, 20) >= 0.7
