"""Sparse pullbacks on the argmax tape: the device drivers ``*_pullback``.

Each function mirrors the reference's device driver of the same name
(``*_pullback_ka`` / ``*_pullback_invgrid``): check shapes, allocate the
gradients, launch one pullback through the C ABI, return the gradients on
the device.  For every pair p and query token t with qmask and a tape entry
1 <= u <= Td(p):

    dQ[t of p's query]    += delta_p * D[u of p's document]
    dD[u of p's document] += delta_p * Q[t of p's query]

with delta_p = Delta[p] * inv_n[query of p] (paper Eqs. 2-3).  ``mode``
(AtomicUnified / InvGrid) is accepted for API parity; the HIP library runs
the InvGrid form (gather for dQ, destination CSR for dD) for both, so dQ is
deterministic and dD is summed in fp32 per destination row.  Sums run in
fp32 and are rounded once into the feature eltype.

Shapes follow the package convention (Julia ``(a, b, c)`` is torch
``(c, b, a)``).  Cotangents and inv_n are converted to the feature eltype
(convert_scores, ka.jl:65-68) on the device.

| here                | reference                                              |
|---------------------|--------------------------------------------------------|
| pair_pullback       | pair_pullback / pair_pullback_ka (backward_pair.jl:39-71) |
| paired_pullback     | paired_pullback_ka      (backward_layouts.jl:33-43)    |
| inbatch_pullback    | inbatch_pullback_ka     (backward_layouts.jl:101-111)  |
| candidates_pullback | candidates_pullback_ka  (backward_layouts.jl:173-185)  |
| packed_pullback     | packed_pullback_invgrid (packed.jl:403-417)            |
| varlen_pullback     | varlen_pullback_invgrid (packed.jl:470-485)            |
"""
from __future__ import annotations

import torch

from . import boundary
from .errors import DimensionMismatch
from .forward import (indices_on, require_candidates_shapes, require_inbatch_shapes,
                      require_paired_shapes, require_pair_shapes)
from .packed import PackedSeq


def _cotangent(x, proto: torch.Tensor, shape, what: str) -> torch.Tensor:
    """A device array of the feature eltype with `shape` (scalars fill, ka.jl:65-68)."""
    if x is None:
        raise DimensionMismatch(f"{what}: missing")
    if not isinstance(x, torch.Tensor):
        return torch.full(shape, float(x), dtype=proto.dtype, device=proto.device)
    if tuple(x.shape) != tuple(shape):
        raise DimensionMismatch(f"{what} shape {tuple(x.shape)}, expected {tuple(shape)}")
    return x.to(device=proto.device, dtype=proto.dtype).contiguous()


def _inv_n(inv_n, proto, n, what="inv_n"):
    return None if inv_n is None else _cotangent(inv_n, proto, (n,), what)


def pair_pullback(delta, q, d, qmask=None, argmax_u=None, mode=None):
    """(dq (Tq,dim), dd (Td,dim)) for one pair; delta a scalar or a (1,) array
    (backward_pair.jl:39-71, which also requires length(δ) == 1)."""
    boundary.require_device(q, d, qmask, argmax_u)
    _, Tq, Td = require_pair_shapes(q, d, qmask, None)
    if argmax_u is None or argmax_u.numel() != Tq:
        raise DimensionMismatch("argmax_u vs query tokens")
    if isinstance(delta, torch.Tensor) and delta.numel() != 1:
        raise DimensionMismatch("pair δ must be length 1")
    dv = _cotangent(delta.reshape(1) if isinstance(delta, torch.Tensor) else delta, q, (1,), "δ")
    dq = torch.empty_like(q)
    dd = torch.empty_like(d)
    boundary.pair_apply_pullback(dq, dd, q, d, qmask, argmax_u.contiguous(), dv)
    return dq, dd


def paired_pullback(Delta, Q, D, qmask=None, args=None, inv_n=None, mode=None):
    """(dQ (B,Tq,dim), dD (B,Td,dim)); Delta (B,), args (B,Tq), inv_n (B,) or None."""
    boundary.require_device(Q, D, qmask, args)
    _, Tq, _, B = require_paired_shapes(Q, D, qmask, None)
    if args is None or tuple(args.shape) != (B, Tq):
        raise DimensionMismatch("args")
    Dv = _cotangent(Delta, Q, (B,), "Δ")
    dQ = torch.empty_like(Q)
    dD = torch.empty_like(D)
    boundary.paired_apply_pullback(dQ, dD, Q, D, qmask, args, Dv, _inv_n(inv_n, Q, B))
    return dQ, dD


def inbatch_pullback(Delta, Q, D, qmask=None, args=None, inv_n=None, mode=None):
    """(dQ (Bq,Tq,dim), dD (Bd,Td,dim)); Delta (Bq,Bd) [Julia (Bd,Bq)], args (Bq,Bd,Tq)."""
    boundary.require_device(Q, D, qmask, args)
    _, Tq, Bq, _, Bd = require_inbatch_shapes(Q, D, qmask, None)
    if args is None or tuple(args.shape) != (Bq, Bd, Tq):
        raise DimensionMismatch("args")
    Dv = _cotangent(Delta, Q, (Bq, Bd), "Δ")
    dQ = torch.empty_like(Q)
    dD = torch.empty_like(D)
    boundary.inbatch_apply_pullback(dQ, dD, Q, D, qmask, args, Dv, _inv_n(inv_n, Q, Bq))
    return dQ, dD


def candidates_pullback(Delta, Q, gallery, idxs, qmask=None, args=None, inv_n=None, mode=None):
    """(dQ (B,Tq,dim), dG (N,Td,dim)); Delta (B,C) [Julia (C,B)], args (B,C,Tq)."""
    boundary.require_device(Q, gallery, qmask, args)
    _, Tq, B, _, _ = require_candidates_shapes(Q, gallery, idxs, qmask, None)
    idx = indices_on(Q, idxs)
    C = idx.shape[1]
    if args is None or tuple(args.shape) != (B, C, Tq):
        raise DimensionMismatch("args")
    Dv = _cotangent(Delta, Q, (B, C), "Δ")
    dQ = torch.empty_like(Q)
    dG = torch.empty_like(gallery)
    boundary.candidates_apply_pullback(dQ, dG, Q, gallery, idx, qmask, args, Dv,
                                       _inv_n(inv_n, Q, B))
    return dQ, dG


def packed_pullback(Delta, q, P: PackedSeq, qmask=None, args=None, inv_n=None, mode=None):
    """(dq (Tq,dim), dP (ntokens,dim)); Delta (B,), args (B,Tq), inv_n (1,) or None."""
    boundary.require_device(q, P.tokens, P.cu, qmask, args)
    Tq = q.shape[0]
    if P.tokens.shape[1] != q.shape[1]:
        raise DimensionMismatch("feature dim")
    if qmask is not None and qmask.numel() != Tq:
        raise DimensionMismatch("qmask")
    B = P.nseq()
    if args is None or tuple(args.shape) != (B, Tq):
        raise DimensionMismatch("args")
    Dv = _cotangent(Delta, q, (B,), "Δ")
    dq = torch.empty_like(q)
    dP = torch.empty_like(P.tokens)
    iv = None if inv_n is None else _cotangent(
        inv_n.reshape(1) if isinstance(inv_n, torch.Tensor) else inv_n, q, (1,), "inv_n")
    boundary.packed_apply_pullback(dq, dP, q, P.tokens, P.cu, qmask, args, Dv, iv)
    return dq, dP


def varlen_pullback(Delta, Q: PackedSeq, D: PackedSeq, args=None, inv_n=None, mode=None):
    """(dQ tokens (nq,dim), dD tokens (nd,dim)); Delta (N,), args (N,max_q), inv_n (N,)."""
    boundary.require_device(Q.tokens, D.tokens, Q.cu, D.cu, args)
    N = Q.nseq()
    if N != D.nseq():
        raise DimensionMismatch("varlen pair count")
    if Q.tokens.shape[1] != D.tokens.shape[1]:
        raise DimensionMismatch("feature dim")
    if args is None or tuple(args.shape) != (N, Q.max_len):
        raise DimensionMismatch("args")
    Dv = _cotangent(Delta, Q.tokens, (N,), "Δ")
    dQ = torch.empty_like(Q.tokens)
    dD = torch.empty_like(D.tokens)
    boundary.varlen_apply_pullback(dQ, dD, Q.tokens, D.tokens, Q.cu, D.cu, args, Dv,
                                   _inv_n(inv_n, Q.tokens, N))
    return dQ, dD
