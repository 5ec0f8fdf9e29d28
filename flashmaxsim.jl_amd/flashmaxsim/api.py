"""Public API: one verb ``maxsim`` dispatching on argument types (src/dispatch.jl),
the callable config ``MaxSim`` (src/types.jl:26-50) and the ``InBatch`` marker.

Argument forms (Julia shapes in brackets; torch shapes are reversed):

    maxsim(q, d[, qmask, dmask])                 pair          -> (1,) device score
    maxsim(Q, D[, qmask, dmask])                 paired        -> (B,)
    maxsim(Q, D[, qmask, dmask], InBatch())      in-batch      -> (Bq, Bd)  [Julia (Bd, Bq)]
    maxsim(Q, gallery, idxs[, qmask, dmask])     candidates    -> (B, C)    [Julia (C, B)]
    maxsim(q, P::PackedSeq[, qmask])             packed        -> (B,)
    maxsim(Q, P::PackedSeq[, qmask])             packed, nq queries in one pass (extension)
                                                               -> (nq, B)   [Julia (B, nq)]
    maxsim(Qp::PackedSeq, Dp::PackedSeq)         varlen        -> (N,)
    maxsim(q, d::Int8Index[, qmask, dmask])      INT8 pair     -> (1,)
    maxsim(Q, D::Int8Index[, qmask, dmask])      INT8 paired   -> (B,)
    maxsim(Q, G::Int8Index, idxs[, ...])         INT8 candidates (extension) -> (B, C)

Keywords ``neg`` (fill for invalid candidate indices only, default
T(-1f4)), ``normalize`` (divide by the number of valid query tokens) and
``backward`` (∇D strategy marker; the HIP pullback computes the same sums for
either).  When a feature tensor requires grad, the call is recorded for torch
autograd and back-propagates through the sparse pullbacks (``rrule``).
Scores are Float32 for every feature type (score_eltype).
"""
from __future__ import annotations

import torch

from . import forward as F
from .errors import ArgumentError
from .packed import PackedSeq
from .quant import Int8Index


class InBatch:
    """Marker: ``S[j,i] = MaxSim(Q[i], D[j])`` (types.jl:57-58)."""

    def __repr__(self):
        return "InBatch()"


class AtomicUnified:
    """∇D strategy marker (types.jl:10-11).  The reference scatters dD with atomics; the
    HIP pullback computes the same sums through a destination-sorted source list."""


class InvGrid:
    """∇D strategy marker (types.jl:13-14): gather for dQ, destination CSR for dD."""


def score_eltype(dtype):
    """score_eltype (kernels_forward.jl:16-21); the MI355X path accumulates in fp32 for
    every feature type (the reference keeps BFloat16 accumulation in BFloat16)."""
    if dtype == torch.float64:
        return torch.float64
    return torch.float32


dot_accum = score_eltype


def _cast_neg(neg, dtype) -> float:
    """MaxSim{T} stores T(neg) (types.jl:35-38); scores report it as Float32."""
    if dtype in (torch.float16, torch.bfloat16, torch.float32, torch.float64):
        return float(torch.tensor(float(neg), dtype=dtype).to(torch.float32))
    return float(torch.tensor(float(neg), dtype=torch.float32))


class MaxSim:
    """Callable MaxSim scorer ``MaxSim(T; neg, normalize, backward)`` (types.jl:16-50)."""

    def __init__(self, dtype=torch.float32, *, neg=-1.0e4, normalize: bool = False,
                 backward=AtomicUnified):
        self.dtype = dtype
        self.neg = _cast_neg(neg, dtype)
        self.normalize = bool(normalize)
        self.backward = backward() if isinstance(backward, type) else backward

    def __repr__(self):
        return (f"MaxSim{{{self.dtype}}}(neg={self.neg}, normalize={self.normalize}, "
                f"backward={type(self.backward).__name__}())")

    def __call__(self, *args):
        return maxsim(self, *args)


def _is_mask(x) -> bool:
    return isinstance(x, torch.Tensor) and x.dtype in (torch.bool, torch.uint8)


def _is_index(x) -> bool:
    return isinstance(x, torch.Tensor) and x.dtype in (torch.int32, torch.int64) and x.dim() == 2


def _feature_dtype(x):
    if isinstance(x, PackedSeq):
        return x.tokens.dtype
    return x.dtype


def maxsim(*args, neg=None, normalize=None, backward=None):
    """One verb, layout by argument types (dispatch.jl:31-296)."""
    cfg = None
    if args and isinstance(args[0], MaxSim):
        cfg, args = args[0], args[1:]
    if len(args) < 2:
        raise ArgumentError("maxsim needs at least a query and a document argument")
    a, b, rest = args[0], args[1], list(args[2:])
    inbatch = bool(rest) and isinstance(rest[-1], InBatch)
    if inbatch:
        rest = rest[:-1]
    T = _feature_dtype(a)
    if cfg is None:
        cfg = MaxSim(T, neg=-1.0e4 if neg is None else neg,
                     normalize=bool(normalize), backward=backward or AtomicUnified)
    else:
        if neg is not None or normalize is not None:
            raise ArgumentError("pass either a MaxSim config or keywords, not both")
        if not isinstance(b, Int8Index) and cfg.dtype != T and not isinstance(a, PackedSeq):
            raise ArgumentError("MaxSim feature eltype must match the callable's parameter")

    # ---- differentiable call: record the tape and the pullback (rrule.jl) ----
    from .rrule import maxsim_autograd, needs_grad
    if needs_grad(args):
        return maxsim_autograd(cfg, args)

    # ---- varlen pairs ----
    if isinstance(a, PackedSeq):
        if not isinstance(b, PackedSeq) or rest:
            raise ArgumentError("varlen maxsim takes two PackedSeq")
        scores, _ = F.varlen_forward(a, b, cfg.neg, cfg.normalize, tape=False)
        return scores

    # ---- packed ----
    if isinstance(b, PackedSeq):
        qmask = rest[0] if rest else None
        if a.dim() == 3:  # several queries in one pass (extension): (nq, B) scores
            S, _ = F.packed_multi_forward(a, b, qmask, cfg.neg, cfg.normalize, tape=False)
            return S
        scores, _ = F.packed_forward(a, b, qmask, cfg.neg, cfg.normalize, tape=False)
        return scores

    # ---- INT8 index ----
    if isinstance(b, Int8Index):
        if rest and _is_index(rest[0]):
            idxs, masks = rest[0], rest[1:]
            qmask, dmask = (masks + [None, None])[:2]
            S, _ = F.int8_candidates_forward(a, b, idxs, qmask, dmask, cfg.neg, cfg.normalize,
                                             tape=False)
            return S
        qmask, dmask = (rest + [None, None])[:2]
        if a.dim() == 2:
            score, _ = F.int8_pair_forward(a, b, qmask, dmask, cfg.normalize, tape=False)
            return score
        scores, _ = F.int8_paired_forward(a, b, qmask, dmask, cfg.normalize, tape=False)
        return scores

    # ---- dense features ----
    if rest and _is_index(rest[0]) and not inbatch:
        idxs, masks = rest[0], rest[1:]
        qmask, dmask = (masks + [None, None])[:2]
        S, _ = F.candidates_forward(a, b, idxs, qmask, dmask, cfg.neg, cfg.normalize, tape=False)
        return S
    qmask, dmask = (rest + [None, None])[:2]
    if inbatch:
        S, _ = F.inbatch_forward(a, b, qmask, dmask, cfg.neg, cfg.normalize, tape=False)
        return S
    if a.dim() == 2:
        score, _ = F.pair_forward(a, b, qmask, dmask, cfg.neg, cfg.normalize, tape=False)
        return score
    scores, _ = F.paired_forward(a, b, qmask, dmask, cfg.neg, cfg.normalize, tape=False)
    return scores
