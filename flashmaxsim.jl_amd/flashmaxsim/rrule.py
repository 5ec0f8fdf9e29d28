"""Reverse rules of ``maxsim`` on the argmax tape (src/rrule.jl) and their torch
autograd binding.

``rrule(cfg, *args)`` mirrors ``ChainRulesCore.rrule(maxsim, cfg, args...)``
(rrule.jl:38-143): it runs the forward once (scores and argmax tape, no dense
similarity matrix), applies the ``normalize`` finalisation, and returns
``(y, pullback)``.  ``pullback(Δ)`` returns one tangent per positional
argument after the config (``None`` where the reference returns
``NoTangent()``); feature tangents are device arrays of the feature eltype,
computed by the HIP pullback kernels through ``flashmaxsim.backward``.  The
tangent of a ``PackedSeq`` argument is its token-gradient array (the
reference's ``Tangent{PackedSeq}(tokens = dP)``, packed.jl:134-136).

Cotangents follow as_array_cotangent / as_scalar_cotangent (rrule.jl:8-36):
an array of the score's shape, a real number for a one-element score, or
``None`` (a zero tangent).  The cotangent is converted to the feature eltype,
and so is inv_n (convert_scores, ka.jl:65-68).  INT8 layouts are forward-only:
a nonzero cotangent raises ArgumentError (rrule.jl:145-168).

When a feature tensor ``requires_grad`` and grad mode is on, ``maxsim`` runs
through ``MaxSimFunction`` (a ``torch.autograd.Function``), so a loss built on
the scores back-propagates into the same pullbacks.
"""
from __future__ import annotations

import torch

from . import backward as BW
from . import forward as F
from .errors import ArgumentError, DimensionMismatch
from .packed import PackedSeq
from .quant import Int8Index


def _inv_counts(qmask, B: int, Tq: int, device) -> torch.Tensor:
    """inv_token_counts (normalize.jl:4-10): fp32 (B,) = 1 / max(count(qmask[:, b]), 1)."""
    if qmask is None:
        return torch.full((B,), 1.0 / max(Tq, 1), dtype=torch.float32, device=device)
    c = qmask.reshape(B, Tq).to(torch.float32).sum(1).clamp(min=1.0)
    return 1.0 / c


def _varlen_inv(Q: PackedSeq) -> torch.Tensor:
    """varlen_inv_n_kernel! (kernels_packed.jl:277-282): 1 / max(Tq_n, 1) per pair."""
    cu = Q.cu
    n = (cu[1:] - cu[:-1]).clamp(min=1).to(torch.float32)
    return 1.0 / n


def _cotangent(delta, y: torch.Tensor) -> torch.Tensor:
    """as_array_cotangent (rrule.jl:8-27): fp32 device array of y's shape."""
    if delta is None:
        return torch.zeros_like(y, dtype=torch.float32)
    if isinstance(delta, torch.Tensor):
        if tuple(delta.shape) != tuple(y.shape):
            if delta.numel() == 1 and y.numel() == 1:
                return delta.reshape(y.shape).to(device=y.device, dtype=torch.float32)
            raise DimensionMismatch(
                f"MaxSim cotangent axes {tuple(delta.shape)} do not match score axes "
                f"{tuple(y.shape)}")
        return delta.to(device=y.device, dtype=torch.float32)
    if isinstance(delta, (int, float)):
        if y.numel() != 1:
            raise ArgumentError(f"scalar MaxSim cotangent for a {y.numel()}-element score array")
        return torch.full(y.shape, float(delta), dtype=torch.float32, device=y.device)
    raise ArgumentError(f"unsupported MaxSim cotangent type {type(delta).__name__}")


def _pad(tangents, nargs):
    out = list(tangents) + [None] * nargs
    return tuple(out[:nargs])


def rrule(cfg, *args):
    """(y, pullback) for ``maxsim(cfg, *args)``; same argument forms as ``maxsim``."""
    from .api import InBatch, MaxSim, _is_index  # (api imports this module lazily)
    if not isinstance(cfg, MaxSim):
        raise ArgumentError("rrule(maxsim, cfg, args...) needs a MaxSim config")
    if len(args) < 2:
        raise ArgumentError("maxsim needs at least a query and a document argument")
    nargs = len(args)
    a, b, rest = args[0], args[1], list(args[2:])
    inbatch = bool(rest) and isinstance(rest[-1], InBatch)
    if inbatch:
        rest = rest[:-1]
    norm = cfg.normalize
    mode = cfg.backward

    # ---- varlen pairs (rrule.jl:132-143) ----
    if isinstance(a, PackedSeq):
        if not isinstance(b, PackedSeq) or rest:
            raise ArgumentError("varlen maxsim takes two PackedSeq")
        scores, tape = F.varlen_forward(a, b, cfg.neg)
        inv = _varlen_inv(a) if norm else None
        y = scores * inv if norm else scores
        T = a.tokens.dtype

        def pullback(delta):
            dh = _cotangent(delta, y).to(T)
            dQ, dD = BW.varlen_pullback(dh, a, b, tape, None if inv is None else inv.to(T), mode)
            return _pad((dQ, dD), nargs)
        return y, pullback

    # ---- several queries against one PackedSeq (extension): per-query pullbacks ----
    if isinstance(b, PackedSeq) and a.dim() == 3:
        qmask = rest[0] if rest else None
        S, tape = F.packed_multi_forward(a, b, qmask, cfg.neg)
        nq, Tq = a.shape[0], a.shape[1]
        inv = _inv_counts(qmask, nq, Tq, a.device) if norm else None
        y = S * inv[:, None] if norm else S
        T = a.dtype

        def pullback(delta):
            dh = _cotangent(delta, y).to(T)
            dQ = torch.empty_like(a)
            dP = None
            for i in range(nq):
                qi = None if qmask is None else qmask[i].contiguous()
                iv = None if inv is None else inv[i:i + 1].to(T)
                dq, dp = BW.packed_pullback(dh[i].contiguous(), a[i], b, qi, tape[i].contiguous(),
                                            iv, mode)
                dQ[i] = dq
                dP = dp if dP is None else dP + dp
            return _pad((dQ, dP), nargs)
        return y, pullback

    # ---- packed (rrule.jl:119-130) ----
    if isinstance(b, PackedSeq):
        qmask = rest[0] if rest else None
        scores, tape = F.packed_forward(a, b, qmask, cfg.neg)
        inv = _inv_counts(qmask, 1, a.shape[0], a.device) if norm else None
        y = scores * inv if norm else scores
        T = a.dtype

        def pullback(delta):
            dh = _cotangent(delta, y).to(T)
            dq, dP = BW.packed_pullback(dh, a, b, qmask, tape, None if inv is None else inv.to(T),
                                        mode)
            return _pad((dq, dP), nargs)
        return y, pullback

    # ---- INT8: forward-only (rrule.jl:145-168) ----
    if isinstance(b, Int8Index):
        from .api import maxsim
        y = maxsim(cfg, *args)

        def pullback(delta):
            if delta is None or (isinstance(delta, torch.Tensor) and not bool(delta.any())) \
                    or (isinstance(delta, (int, float)) and delta == 0):
                return _pad((), nargs)
            raise ArgumentError("INT8 MaxSim is forward-only (no ChainRules pullback)")
        return y, pullback

    T = a.dtype
    # ---- candidates (rrule.jl:101-117) ----
    if rest and _is_index(rest[0]) and not inbatch:
        idxs, masks = rest[0], rest[1:]
        qmask, dmask = (masks + [None, None])[:2]
        S, tape = F.candidates_forward(a, b, idxs, qmask, dmask, cfg.neg)
        B, Tq = a.shape[0], a.shape[1]
        inv = _inv_counts(qmask, B, Tq, a.device) if norm else None
        y = F.length_normalize_candidates(S, qmask, Tq, idxs, b.shape[0], cfg.neg) if norm else S

        def pullback(delta):
            dh = _cotangent(delta, y).to(T)
            dQ, dG = BW.candidates_pullback(dh, a, b, idxs, qmask, tape,
                                            None if inv is None else inv.to(T), mode)
            return _pad((dQ, dG), nargs)
        return y, pullback

    qmask, dmask = (rest + [None, None])[:2]
    # ---- in-batch (rrule.jl:84-99) ----
    if inbatch:
        S, tape = F.inbatch_forward(a, b, qmask, dmask, cfg.neg)
        Bq, Tq = a.shape[0], a.shape[1]
        inv = _inv_counts(qmask, Bq, Tq, a.device) if norm else None
        y = S * inv[:, None] if norm else S

        def pullback(delta):
            dh = _cotangent(delta, y).to(T)
            dQ, dD = BW.inbatch_pullback(dh, a, b, qmask, tape,
                                         None if inv is None else inv.to(T), mode)
            return _pad((dQ, dD), nargs)
        return y, pullback

    # ---- pair (rrule.jl:38-66) ----
    if a.dim() == 2:
        score, tape = F.pair_forward(a, b, qmask, dmask, cfg.neg)
        inv = _inv_counts(qmask, 1, a.shape[0], a.device) if norm else None
        y = score * inv if norm else score

        def pullback(delta):
            d32 = _cotangent(delta, y)
            dl = (d32 * inv if norm else d32).to(T)  # δ = convert_scores(T, Δ * inv_n)
            dq, dd = BW.pair_pullback(dl, a, b, qmask, tape, mode)
            return _pad((dq, dd), nargs)
        return y, pullback

    # ---- paired (rrule.jl:68-82) ----
    scores, tape = F.paired_forward(a, b, qmask, dmask, cfg.neg)
    B, Tq = a.shape[0], a.shape[1]
    inv = _inv_counts(qmask, B, Tq, a.device) if norm else None
    y = scores * inv if norm else scores

    def pullback(delta):
        dh = _cotangent(delta, y).to(T)
        dQ, dD = BW.paired_pullback(dh, a, b, qmask, tape, None if inv is None else inv.to(T),
                                    mode)
        return _pad((dQ, dD), nargs)
    return y, pullback


def _diff_inputs(args):
    """The tensors gradients flow to: features and PackedSeq tokens, in argument order."""
    out = []
    for i, x in enumerate(args[:2]):
        if isinstance(x, PackedSeq):
            out.append((i, x.tokens))
        elif isinstance(x, torch.Tensor) and x.is_floating_point():
            out.append((i, x))
    return out


class MaxSimFunction(torch.autograd.Function):
    """torch autograd node around ``rrule``: forward = the fused scan, backward = the
    HIP pullback of the tape the forward recorded."""

    @staticmethod
    def forward(ctx, cfg, args, *tensors):
        y, pb = rrule(cfg, *args)
        ctx.pb = pb
        ctx.slots = [i for i, _ in _diff_inputs(args)]
        return y

    @staticmethod
    def backward(ctx, gy):
        tangents = ctx.pb(gy)
        return (None, None) + tuple(tangents[i] for i in ctx.slots)


def needs_grad(args) -> bool:
    return torch.is_grad_enabled() and any(t.requires_grad for _, t in _diff_inputs(args))


def maxsim_autograd(cfg, args):
    """``maxsim(cfg, *args)`` recorded on the autograd tape."""
    return MaxSimFunction.apply(cfg, tuple(args), *[t for _, t in _diff_inputs(args)])
