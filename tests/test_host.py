"""CPU checks of the host mirror: PackedSeq / pack_docs CSR logic, MaxSim
config semantics, argument validation, and that no CPU scoring path exists
(host tensors are refused, as the MI355X library is the only scorer)."""
import numpy as np
import pytest
import torch

import flashmaxsim as fm
from flashmaxsim import forward as F


def test_pack_docs_cu_and_max_len():
    """test_packed.jl:1-27."""
    dim = 8
    docs = [torch.randn(5, dim), torch.randn(0, dim), torch.randn(3, dim)]
    P = fm.pack_docs(docs)
    assert P.cu.tolist() == [1, 6, 6, 9]
    assert P.max_len == 5 and fm.nseq(P) == 3
    assert tuple(P.tokens.shape) == (8, dim)
    assert torch.equal(P.tokens[0:5], docs[0]) and torch.equal(P.tokens[5:8], docs[2])
    assert fm.PackedSeq(P.tokens, P.cu).max_len == 5
    with pytest.raises(fm.ArgumentError):
        fm.PackedSeq(P.tokens, torch.tensor([1, 6, 6, 7], dtype=torch.int32))  # does not cover
    with pytest.raises(fm.ArgumentError):
        fm.PackedSeq(P.tokens, torch.tensor([2, 6, 6, 9], dtype=torch.int32))  # does not start at 1
    with pytest.raises(fm.ArgumentError):
        fm.PackedSeq(P.tokens, torch.tensor([1, 6, 4, 9], dtype=torch.int32))  # decreasing
    with pytest.raises(fm.ArgumentError):
        fm.pack_docs([])
    with pytest.raises(fm.DimensionMismatch):
        fm.pack_docs([torch.randn(2, 4), torch.randn(2, 5)])


def test_pack_pairs():
    qs = [torch.randn(4, 8), torch.randn(2, 8)]
    ds = [torch.randn(5, 8), torch.randn(3, 8)]
    Qp, Dp = fm.pack_pairs(qs, ds)
    assert Qp.cu.tolist() == [1, 5, 7] and Dp.cu.tolist() == [1, 6, 9]
    assert Qp.max_len == 4 and Dp.max_len == 5
    with pytest.raises(fm.DimensionMismatch):
        fm.pack_pairs(qs, ds[:1])


def test_maxsim_config_semantics():
    cfg = fm.MaxSim(torch.float16)
    assert cfg.neg == -1.0e4 and not cfg.normalize
    assert fm.MaxSim(torch.bfloat16).neg == -9984.0  # BFloat16(-1f4) rounds to -9984
    assert fm.MaxSim(torch.float32, neg=0, normalize=True).normalize
    assert isinstance(fm.MaxSim(backward=fm.InvGrid).backward, fm.InvGrid)
    assert fm.score_eltype(torch.float16) == torch.float32
    assert fm.score_eltype(torch.bfloat16) == torch.float32
    assert "MaxSim" in repr(cfg)


def test_host_tensors_have_no_cpu_path():
    q, d = torch.randn(3, 8), torch.randn(5, 8)
    with pytest.raises(fm.ArgumentError):
        fm.maxsim(q, d)
    with pytest.raises(fm.ArgumentError):
        fm.maxsim(q.unsqueeze(0), d.unsqueeze(0), fm.InBatch())
    with pytest.raises(fm.ArgumentError):
        fm.maxsim(q, fm.pack_docs([d]))


def test_shape_checks_match_reference():
    """test_forward.jl:77-91 (DimensionMismatch cases), checked before any launch."""
    Q, D = torch.randn(2, 3, 4), torch.randn(2, 5, 4)
    with pytest.raises(fm.DimensionMismatch):
        F.require_paired_shapes(Q, D, torch.ones(2, 3, dtype=torch.bool), torch.ones(3, 5, dtype=torch.bool))
    with pytest.raises(fm.DimensionMismatch):
        F.require_paired_shapes(Q, D, torch.ones(2, 2, dtype=torch.bool), None)
    with pytest.raises(fm.DimensionMismatch):
        F.require_paired_shapes(Q, torch.randn(2, 5, 5), None, None)
    with pytest.raises(fm.DimensionMismatch):
        F.require_paired_shapes(Q, torch.randn(3, 5, 4), None, None)
    with pytest.raises(fm.DimensionMismatch):
        F.require_inbatch_shapes(Q, D, torch.ones(2, 3, dtype=torch.bool), torch.ones(2, 4, dtype=torch.bool))
    G = torch.randn(4, 5, 4)
    idxs = torch.tensor([[1, 3, 0], [2, 4, 1]])
    with pytest.raises(fm.DimensionMismatch):
        F.require_candidates_shapes(Q, G, idxs, torch.ones(3, 3, dtype=torch.bool), None)
    with pytest.raises(fm.DimensionMismatch):
        F.require_candidates_shapes(Q, G, torch.tensor([[1, 0], [2, 1], [3, 2]]), None, None)
    with pytest.raises(fm.DimensionMismatch):
        F.require_candidates_shapes(Q, torch.randn(4, 5, 5), idxs, None, None)
    with pytest.raises(fm.DimensionMismatch):
        F.require_pair_shapes(torch.randn(3, 4), torch.randn(5, 4), torch.ones(2, dtype=torch.bool), None)


def test_unsupported_feature_type():
    from flashmaxsim import boundary
    with pytest.raises(fm.UnsupportedError):
        boundary.dtype_code(torch.randn(2, 2, dtype=torch.float64))
    assert boundary.dtype_code(torch.randn(2, 2).half()) == 1


def test_int8index_shape_checks():
    from flashmaxsim.quant import require_int8_index
    require_int8_index(fm.Int8Index(torch.zeros(5, 8, dtype=torch.int8), torch.zeros(5)))
    with pytest.raises(fm.DimensionMismatch):
        require_int8_index(fm.Int8Index(torch.zeros(5, 8, dtype=torch.int8), torch.zeros(4)))
    with pytest.raises(fm.DimensionMismatch):
        require_int8_index(fm.Int8Index(torch.zeros(2, 5, 8, dtype=torch.int8), torch.zeros(3, 5)))
    deq = fm.dequant_int8(fm.Int8Index(torch.tensor([[1, -2]], dtype=torch.int8), torch.tensor([0.5])))
    assert deq.tolist() == [[0.5, -1.0]]


def test_rrule_refuses_host_arrays_and_bad_config():
    """rrule mirrors the forward's colocation rule: host tensors never take a CPU path."""
    import flashmaxsim as fm
    Q = torch.zeros(2, 3, 8)
    with pytest.raises(fm.ArgumentError):
        fm.rrule(fm.MaxSim(torch.float32), Q, Q)
    with pytest.raises(fm.ArgumentError):
        fm.rrule("not a config", Q, Q)


def test_cu_seqlens_interop():
    """0-based cu_seqlens <-> 1-based cu (packed.jl:5-6: `cu = cu_seqlens .+ 1`)."""
    dim = 4
    tok = torch.randn(9, dim)
    P = fm.PackedSeq.from_cu_seqlens(tok, [0, 5, 5, 9])
    assert P.cu.dtype == torch.int32 and P.cu.tolist() == [1, 6, 6, 10]
    assert P.max_len == 5 and P.nseq() == 3
    assert P.cu_seqlens().tolist() == [0, 5, 5, 9]
    P64 = fm.PackedSeq.from_cu_seqlens(tok, torch.tensor([0, 2, 9], dtype=torch.int64))
    assert P64.cu.tolist() == [1, 3, 10] and P64.max_len == 7
    # the same validation as a 1-based cu (packed.jl:47-57)
    with pytest.raises(fm.ArgumentError):
        fm.PackedSeq.from_cu_seqlens(tok, [1, 5, 9])  # does not start at 0
    with pytest.raises(fm.ArgumentError):
        fm.PackedSeq.from_cu_seqlens(tok, [0, 5, 8])  # does not cover the tokens
    with pytest.raises(fm.ArgumentError):
        fm.PackedSeq.from_cu_seqlens(tok, [0, 6, 5, 9])  # decreasing
    with pytest.raises(fm.ArgumentError):
        fm.PackedSeq.from_cu_seqlens(tok, torch.tensor([0.0, 9.0]))  # not integers


def test_int8_index_at_rest_round_trip(tmp_path):
    """save_int8_index / load_int8_index keep the codes and scales bytes."""
    g = torch.Generator().manual_seed(0)
    codes = torch.randint(-127, 128, (6, 11, 32), generator=g, dtype=torch.int8)
    scales = torch.rand(6, 11, generator=g) * 0.01
    idx = fm.Int8Index(codes, scales)
    path = str(tmp_path / "gallery.safetensors")
    fm.save_int8_index(idx, path)
    back = fm.load_int8_index(path)
    assert torch.equal(back.codes, codes) and torch.equal(back.scales, scales)
    assert back.codes.dtype == torch.int8 and back.scales.dtype == torch.float32
    # the file's tensors are the in-memory layout, byte for byte
    from safetensors import safe_open
    with safe_open(path, framework="pt") as f:
        assert f.metadata()["format"] == "flashmaxsim-int8-index-v1"
        assert f.get_tensor("codes").numpy().tobytes() == codes.numpy().tobytes()
    with pytest.raises(fm.DimensionMismatch):
        fm.save_int8_index(fm.Int8Index(codes, scales[:, :10]), str(tmp_path / "bad.safetensors"))
    from safetensors.torch import save_file
    save_file({"codes": codes, "scales": scales}, str(tmp_path / "plain.safetensors"))
    with pytest.raises(fm.ArgumentError):
        fm.load_int8_index(str(tmp_path / "plain.safetensors"))
