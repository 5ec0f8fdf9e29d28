"""Layout drivers: allocate outputs, call the boundary, finalize.

Each ``*_forward`` mirrors the reference's device driver ``*_forward_ka``
(outputs allocated with zeros_like, one scan launch, scores kept on device)
and returns ``(scores, argmax_tape)``.  Σ_t, the candidate ``neg`` fill and,
with ``normalize=True``, the length normalisation are fused into the scan
kernel's score write (the reference runs ``sum(partial; dims=1)``,
``ifelse.(valid, S, neg)`` and ``scores .* inv_n`` as separate device
kernels; normalize.jl, packed.jl:316-354).  The tape is the same either way.

Shapes follow the package convention (Julia ``(a, b, c)`` is torch
``(c, b, a)``): a paired tape Julia ``(Tq, B)`` is ``(B, Tq)``, a candidate
score matrix ``(C, B)`` is ``(B, C)``, an in-batch ``S (Bd, Bq)`` is
``(Bq, Bd)``.
"""
from __future__ import annotations

import torch

from . import boundary
from .errors import ArgumentError, DimensionMismatch
from .packed import PackedSeq
from .quant import Int8Index, quantize_int8_symmetric, require_int8_index

SCORE_DTYPE = torch.float32


def _zeros(like: torch.Tensor, dtype, *shape):
    return torch.zeros(shape, dtype=dtype, device=like.device)


# ---- shape checks (DimensionMismatch, as in the reference) ---------------------------

def require_pair_shapes(q, d, qmask, dmask):
    """forward_pair.jl:14-21."""
    if q.dim() != 2 or d.dim() != 2:
        raise DimensionMismatch("pair features must be (T, dim)")
    Tq, dim = q.shape
    Td = d.shape[0]
    if d.shape[1] != dim:
        raise DimensionMismatch("feature dim")
    if qmask is not None and qmask.numel() != Tq:
        raise DimensionMismatch("qmask")
    if dmask is not None and dmask.numel() != Td:
        raise DimensionMismatch("dmask")
    return dim, Tq, Td


def require_paired_shapes(Q, D, qmask, dmask):
    """forward_layouts.jl:20-28."""
    B, Tq, dim = Q.shape
    Td = D.shape[1]
    if D.shape[2] != dim:
        raise DimensionMismatch("feature dim")
    if D.shape[0] != B:
        raise DimensionMismatch("batch")
    if qmask is not None and tuple(qmask.shape) != (B, Tq):
        raise DimensionMismatch("qmask")
    if dmask is not None and tuple(dmask.shape) != (B, Td):
        raise DimensionMismatch("dmask")
    return dim, Tq, Td, B


def require_inbatch_shapes(Q, D, qmask, dmask):
    """forward_layouts.jl:30-37."""
    Bq, Tq, dim = Q.shape
    Bd, Td = D.shape[0], D.shape[1]
    if D.shape[2] != dim:
        raise DimensionMismatch("feature dim")
    if qmask is not None and tuple(qmask.shape) != (Bq, Tq):
        raise DimensionMismatch("qmask")
    if dmask is not None and tuple(dmask.shape) != (Bd, Td):
        raise DimensionMismatch("dmask")
    return dim, Tq, Bq, Td, Bd


def require_candidates_shapes(Q, gallery, idxs, qmask, dmask):
    """forward_layouts.jl:39-47."""
    B, Tq, dim = Q.shape
    N, Td = gallery.shape[0], gallery.shape[1]
    if gallery.shape[2] != dim:
        raise DimensionMismatch("feature dim")
    if idxs.dim() != 2 or idxs.shape[0] != B:
        raise DimensionMismatch("idxs")
    if qmask is not None and tuple(qmask.shape) != (B, Tq):
        raise DimensionMismatch("qmask")
    if dmask is not None and tuple(dmask.shape) != (N, Td):
        raise DimensionMismatch("dmask")
    return dim, Tq, B, Td, N


def indices_on(prototype: torch.Tensor, idxs: torch.Tensor) -> torch.Tensor:
    """indices_on (ka.jl:41-46): refuse a host->device copy of idxs in the hot path."""
    if idxs.device != prototype.device:
        from .errors import ArgumentError
        raise ArgumentError(
            "FlashMaxSim requires idxs on the same KernelAbstractions backend as features "
            "(e.g. idxs.to('cuda')); refusing a host→device copy in the hot path")
    return idxs


# ---- forward drivers ---------------------------------------------------------------------

def pair_forward(q, d, qmask=None, dmask=None, neg=None, normalize=False, tape=True):
    """pair_forward_ka (forward_pair.jl:104-116): (score (1,), argmax_u (Tq,)).
    tape=False: (score, None), no tape made (every driver below takes the same
    keyword; ``maxsim`` passes it, as the reference's drops the tape,
    dispatch.jl:44-287)."""
    boundary.require_device(q, d, qmask, dmask)
    _, Tq, _ = require_pair_shapes(q, d, qmask, dmask)
    argmax_u = _zeros(q, torch.int32, Tq) if tape else None
    partial = _zeros(q, SCORE_DTYPE, Tq) if tape else None
    score = _zeros(q, SCORE_DTYPE, 1)
    boundary.launch_pair_scan(argmax_u, partial, q, d, qmask, dmask, score, normalize)
    return score, argmax_u


def paired_forward(Q, D, qmask=None, dmask=None, neg=None, normalize=False, tape=True):
    """paired_forward_ka (forward_layouts.jl:112-124): (scores (B,), args (B,Tq))."""
    boundary.require_device(Q, D, qmask, dmask)
    _, Tq, _, B = require_paired_shapes(Q, D, qmask, dmask)
    args = _zeros(Q, torch.int32, B, Tq) if tape else None
    scores = _zeros(Q, SCORE_DTYPE, B)
    boundary.launch_paired_scan(args, None, Q, D, qmask, dmask, scores, normalize)
    return scores, args


def inbatch_forward(Q, D, qmask=None, dmask=None, neg=None, normalize=False, tape=True):
    """inbatch_forward_ka (forward_layouts.jl:188-200): (S (Bq,Bd), args (Bq,Bd,Tq)).

    tape=False returns (S, None) and makes no tape: the reference's ``maxsim``
    discards it (``S, _ = inbatch_forward(...)``, dispatch.jl:124), and without
    it the kernel keeps a running maximum alone (the same S)."""
    boundary.require_device(Q, D, qmask, dmask)
    _, Tq, Bq, Td, Bd = require_inbatch_shapes(Q, D, qmask, dmask)
    S = _zeros(Q, SCORE_DTYPE, Bq, Bd)
    args = _zeros(Q, torch.int32, Bq, Bd, Tq) if tape else None
    if Bd == 0 or Bq == 0 or Tq == 0 or Td == 0:
        return S, args
    boundary.inbatch_device_scan(S, args, Q, D, qmask, dmask, normalize)
    return S, args


def candidates_forward(Q, gallery, idxs, qmask=None, dmask=None, neg=-1.0e4, normalize=False,
                       tape=True):
    """candidates_forward_ka (forward_layouts.jl:272-290): (S (B,C), args (B,C,Tq))."""
    boundary.require_device(Q, gallery, qmask, dmask)
    _, Tq, B, _, N = require_candidates_shapes(Q, gallery, idxs, qmask, dmask)
    idx = indices_on(Q, idxs)
    C = idx.shape[1]
    args = _zeros(Q, torch.int32, B, C, Tq) if tape else None
    S = _zeros(Q, SCORE_DTYPE, B, C)
    boundary.launch_candidates_scan(args, None, Q, gallery, idx, qmask, dmask, N, S, neg,
                                    normalize)
    return S, args


def packed_forward(q, P: PackedSeq, qmask=None, neg=None, normalize=False, tape=True):
    """packed_forward_ka (packed.jl:191-202): (scores (B,), args (B,Tq))."""
    boundary.require_device(q, P.tokens, P.cu, qmask)
    Tq = q.shape[0]
    if P.tokens.shape[1] != q.shape[1]:
        raise DimensionMismatch("feature dim")
    if qmask is not None and qmask.numel() != Tq:
        raise DimensionMismatch("qmask")
    B = P.nseq()
    args = _zeros(q, torch.int32, B, Tq) if tape else None
    scores = _zeros(q, SCORE_DTYPE, B)
    boundary.launch_packed_scan(args, None, q, P.tokens, P.cu, qmask, scores, normalize)
    return scores, args


def packed_multi_forward(Q, P: PackedSeq, qmask=None, neg=None, normalize=False, tape=True):
    """nq queries against one PackedSeq in one pass: (S (nq,B), args (nq,B,Tq)).

    No reference counterpart (the reference's packed_forward takes one query,
    packed.jl:191-202); row i equals packed_forward(Q[i], P, qmask[i]) within
    the score tolerance.  Each document is read once per block of 32 queries
    (the in-batch MFMA kernel over CSR documents).  tape=False returns
    (S, None): no tape, the kernel keeps a running maximum alone (the same S)."""
    boundary.require_device(Q, P.tokens, P.cu, qmask)
    if Q.dim() != 3:
        raise DimensionMismatch("multi-query packed scan takes Q (nq, Tq, dim)")
    nq, Tq, dim = Q.shape
    if P.tokens.shape[1] != dim:
        raise DimensionMismatch("feature dim")
    if qmask is not None and tuple(qmask.shape) != (nq, Tq):
        raise DimensionMismatch("qmask")
    B = P.nseq()
    S = _zeros(Q, SCORE_DTYPE, nq, B)
    args = _zeros(Q, torch.int32, nq, B, Tq) if tape else None
    if nq == 0 or B == 0:
        return S, args
    boundary.launch_packed_multi_scan(args, S, Q, P.tokens, P.cu, qmask, P.max_len, normalize)
    return S, args


def topk(scores: torch.Tensor, k: int):
    """The k best scores of every row: (vals, idx), each (..., k), idx 1-based.

    No reference counterpart: it is what a retrieval caller does with the
    score matrix (``partialsortperm(S[:, i], 1:k; rev = true)`` per query in
    the reference's column-major terms, README.md:132).  ``scores`` is fp32
    of shape (ncols,) or (nrows, ncols) -- one row per query, as
    ``packed_multi_forward`` and ``inbatch_forward`` return them.  Rows are
    ranked descending by Julia's isless (NaN first, +0.0 before -0.0), equal
    scores by smaller index.  1 <= k <= 1024 and k <= ncols.
    """
    boundary.require_device(scores)
    if scores.dtype != SCORE_DTYPE:
        raise ArgumentError("topk takes fp32 scores")
    if scores.dim() not in (1, 2):
        raise DimensionMismatch("topk takes a score vector or a (rows, columns) matrix")
    S2 = scores.reshape(1, -1) if scores.dim() == 1 else scores
    S2 = S2.contiguous()
    nrows, ncols = S2.shape
    if k < 0 or k > ncols:
        raise ArgumentError(f"topk: k = {k} outside 0..{ncols}")
    vals = torch.empty(nrows, k, dtype=SCORE_DTYPE, device=S2.device)
    idx = torch.empty(nrows, k, dtype=torch.int32, device=S2.device)
    if nrows and k:
        boundary.topk_rows(vals, idx, S2, k)
    if scores.dim() == 1:
        return vals[0], idx[0]
    return vals, idx


def varlen_forward(Qp: PackedSeq, Dp: PackedSeq, neg=None, normalize=False, tape=True):
    """varlen_forward_ka (packed.jl:274-284): (scores (N,), args (N,max_q))."""
    boundary.require_device(Qp.tokens, Dp.tokens, Qp.cu, Dp.cu)
    N = Qp.nseq()
    if N != Dp.nseq():
        raise DimensionMismatch("varlen pair count")
    if Qp.tokens.shape[1] != Dp.tokens.shape[1]:
        raise DimensionMismatch("feature dim")
    max_q = Qp.max_len
    args = _zeros(Qp.tokens, torch.int32, N, max_q) if tape else None
    scores = _zeros(Qp.tokens, SCORE_DTYPE, N)
    boundary.launch_varlen_scan(args, None, Qp.tokens, Dp.tokens, Qp.cu, Dp.cu, scores, normalize,
                                max_q=max_q)
    return scores, args


def int8_pair_forward(q, d: Int8Index, qmask=None, dmask=None, normalize=False, tape=True):
    """int8_pair_forward (quant.jl:156-170): quantise q on device, then the INT8 scan."""
    qq = quantize_int8_symmetric(q)
    require_int8_index(d)
    boundary.require_device(q, qq.codes, qq.scales, d.codes, d.scales, qmask, dmask)
    Tq, dim = qq.codes.shape
    Td = d.codes.shape[0]
    if d.codes.shape[1] != dim:
        raise DimensionMismatch("feature dim")
    if d.scales.numel() != Td:
        raise DimensionMismatch("document scales")
    if qmask is not None and qmask.numel() != Tq:
        raise DimensionMismatch("qmask")
    if dmask is not None and dmask.numel() != Td:
        raise DimensionMismatch("dmask")
    args = _zeros(q, torch.int32, Tq) if tape else None
    score = _zeros(q, SCORE_DTYPE, 1)
    boundary.launch_int8_pair_scan(args, None, qq.codes, qq.scales, d.codes, d.scales, qmask,
                                   dmask, score, normalize)
    return score, args


def int8_paired_forward(Q, D: Int8Index, qmask=None, dmask=None, normalize=False, tape=True):
    """int8_paired_forward (quant.jl:219-226)."""
    QQ = quantize_int8_symmetric(Q)
    require_int8_index(D)
    boundary.require_device(Q, QQ.codes, QQ.scales, D.codes, D.scales, qmask, dmask)
    B, Tq, dim = QQ.codes.shape
    Td = D.codes.shape[1]
    if D.codes.shape[2] != dim:
        raise DimensionMismatch("feature dim")
    if D.codes.shape[0] != B:
        raise DimensionMismatch("batch")
    if tuple(D.scales.shape) != (B, Td):
        raise DimensionMismatch("document scales")
    if qmask is not None and tuple(qmask.shape) != (B, Tq):
        raise DimensionMismatch("qmask")
    if dmask is not None and tuple(dmask.shape) != (B, Td):
        raise DimensionMismatch("dmask")
    args = _zeros(Q, torch.int32, B, Tq) if tape else None
    scores = _zeros(Q, SCORE_DTYPE, B)
    boundary.launch_int8_paired_scan(args, None, QQ.codes, QQ.scales, D.codes, D.scales, qmask,
                                     dmask, scores, normalize)
    return scores, args


def int8_candidates_forward(Q, G: Int8Index, idxs, qmask=None, dmask=None, neg=-1.0e4,
                            normalize=False, tape=True):
    """INT8 candidate layout (no reference method): quantised Q_b vs gallery[idxs[c,b]]."""
    QQ = quantize_int8_symmetric(Q)
    boundary.require_device(Q, QQ.codes, QQ.scales, G.codes, G.scales, qmask, dmask)
    B, Tq, dim = QQ.codes.shape
    N, Td = G.codes.shape[0], G.codes.shape[1]
    if G.codes.shape[2] != dim:
        raise DimensionMismatch("feature dim")
    if tuple(G.scales.shape) != (N, Td):
        raise DimensionMismatch("document scales")
    if idxs.dim() != 2 or idxs.shape[0] != B:
        raise DimensionMismatch("idxs")
    if qmask is not None and tuple(qmask.shape) != (B, Tq):
        raise DimensionMismatch("qmask")
    if dmask is not None and tuple(dmask.shape) != (N, Td):
        raise DimensionMismatch("dmask")
    idx = indices_on(Q, idxs)
    C = idx.shape[1]
    args = _zeros(Q, torch.int32, B, C, Tq) if tape else None
    S = _zeros(Q, SCORE_DTYPE, B, C)
    boundary.launch_int8_candidates_scan(args, None, QQ.codes, QQ.scales, G.codes, G.scales, idx,
                                         qmask, dmask, N, S, neg, normalize)
    return S, args


# ---- finalize (normalize.jl, forward_pair.jl:153-173, packed.jl:316-354) ------------------

def length_normalize(scores, qmask, Tq):
    """scores (ncols,) or (ncols, nrows) with one query per column; returns a new tensor."""
    out = scores.clone()
    ncols = out.shape[0] if out.dim() >= 1 else 1
    nrows = out.numel() // max(ncols, 1)
    boundary.length_normalize_(out, qmask, Tq, nrows, ncols)
    return out


def length_normalize_candidates(S, qmask, Tq, idxs, N, neg):
    """length_normalize_candidates (normalize.jl:28-46): invalid idx keep neg."""
    out = S.clone()
    B, C = out.shape
    boundary.length_normalize_(out, qmask, Tq, C, B, idxs, N, neg)
    return out


def packed_finalize(scores, qmask, Tq, normalize: bool):
    """packed_finalize (packed.jl:333-337): one query count scales every document."""
    if not normalize:
        return scores
    out = scores.clone()
    boundary.length_normalize_(out, qmask, Tq, out.numel(), 1)
    return out


def varlen_finalize(scores, Qp: PackedSeq, normalize: bool):
    """varlen_finalize (packed.jl:351-354): scores[n] *= 1/max(Tq_n, 1)."""
    if not normalize:
        return scores
    out = scores.clone()
    boundary.varlen_normalize_(out, Qp.cu)
    return out
