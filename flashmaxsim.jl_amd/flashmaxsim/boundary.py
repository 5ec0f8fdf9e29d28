"""The device plugin boundary: one function per reference ``launch_*_scan!``.

Each function takes device tensors (outputs first, mutated in place, as in
the reference) and enqueues the HIP kernel on the current torch stream.  No
host synchronisation.  Tensors use the reversed-shape convention of the
package (Julia ``(dim, T, B)`` == torch ``(B, T, dim)``).

| here                      | reference                                         |
|---------------------------|---------------------------------------------------|
| launch_pair_scan          | launch_pair_scan!        (forward_pair.jl:118-132)   |
| launch_paired_scan        | launch_paired_scan!      (forward_layouts.jl:126-143)|
| launch_candidates_scan    | launch_candidates_scan!  (forward_layouts.jl:292-310)|
| inbatch_device_scan       | inbatch_device_scan!     (forward_layouts.jl:202-225)|
| launch_packed_scan        | launch_packed_scan!      (packed.jl:219-234)         |
| launch_varlen_scan        | launch_varlen_scan!      (packed.jl:298-314)         |
| launch_int8_pair_scan     | launch_int8_pair_scan!   (quant.jl:139-154)          |
| launch_int8_paired_scan   | launch_int8_paired_scan! (quant.jl:199-217)          |
| launch_int8_candidates_scan | (no reference method; candidate conventions)    |
| launch_packed_multi_scan  | (no reference method; nq packed scans in one pass) |
| topk_rows                 | (no reference method; the caller's partialsortperm) |
| tensor_cores_active       | tensor_cores_active      (ka.jl:71)                  |
| pair_apply_pullback       | pair_apply_pullback!     (backward_pair.jl:73-87)    |
| paired_apply_pullback     | paired_apply_pullback!   (backward_layouts.jl:45-60) |
| inbatch_apply_pullback    | inbatch_apply_pullback!  (backward_layouts.jl:113-127)|
| candidates_apply_pullback | candidates_apply_pullback! (backward_layouts.jl:187-202)|
| packed_apply_pullback     | packed_apply_pullback!   (packed.jl:384-417)         |
| varlen_apply_pullback     | varlen_apply_pullback!   (packed.jl:449-485)         |

The pullbacks overwrite their gradient outputs in full (the reference
accumulates into zeros_like buffers); all of them run the InvGrid form
(gather for dQ, destination CSR for dD) whatever strategy marker the caller
holds, since both strategies compute the same sums.
"""
from __future__ import annotations

import torch

from . import _lib
from .errors import ArgumentError, UnsupportedError

_DTYPES = {torch.float32: _lib.FMS_F32, torch.float16: _lib.FMS_F16, torch.bfloat16: _lib.FMS_BF16}


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise UnsupportedError(
            f"feature eltype {t.dtype} has no MI355X scan (float32 / float16 / bfloat16)") from None


def tensor_cores_active(dtype) -> bool:
    """Whether the MFMA scans serve ``dtype`` on the current device (ka.jl:71)."""
    ok = dtype in _DTYPES or dtype == torch.int8
    return ok and torch.cuda.is_available() and _lib.arch_supported()


def ptr(t):
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device):
    return torch.cuda.current_stream(device).cuda_stream


def require_device(*ts):
    """Every tensor must live on one HIP device (require_colocated, colocation.jl:27-35)."""
    dev = None
    for t in ts:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise ArgumentError(f"expected a torch.Tensor, got {type(t).__name__}")
        if t.device.type != "cuda":
            raise ArgumentError(
                "FlashMaxSim requires colocated arrays (same KernelAbstractions backend) for "
                "features and masks; the MI355X path needs every array on the HIP device")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ArgumentError("FlashMaxSim requires colocated arrays (same device)")
        if not t.is_contiguous():
            raise ArgumentError("FlashMaxSim device arrays must be dense (contiguous)")
    return dev


def _mask(m):
    if m is None:
        return None
    if m.dtype not in (torch.bool, torch.uint8):
        raise ArgumentError("masks must be Bool (torch.bool / uint8) arrays")
    return m


def _idx_bytes(idx: torch.Tensor) -> int:
    if idx.dtype == torch.int64:
        return 8
    if idx.dtype == torch.int32:
        return 4
    raise ArgumentError("candidate indices must be Int32 or Int64")


def _norm(normalize) -> int:
    """The scans' fused normalize=true epilogue flag (0 or 1)."""
    return 1 if normalize else 0


def launch_pair_scan(argmax_u, partial, q, d, qmask, dmask, score=None, normalize=False):
    dev = require_device(argmax_u, partial, q, d, qmask, dmask, score)
    Tq, dim = q.shape
    Td = d.shape[0]
    st = _lib.lib().fms_launch_pair_scan(
        dtype_code(q), ptr(argmax_u), ptr(partial), ptr(q), ptr(d), ptr(_mask(qmask)),
        ptr(_mask(dmask)), dim, Tq, Td, ptr(score), _norm(normalize), stream_handle(dev))
    _lib.check(st, "launch_pair_scan")


def launch_paired_scan(args, partial, Q, D, qmask, dmask, scores=None, normalize=False):
    dev = require_device(args, partial, Q, D, qmask, dmask, scores)
    B, Tq, dim = Q.shape
    Td = D.shape[1]
    st = _lib.lib().fms_launch_paired_scan(
        dtype_code(Q), ptr(args), ptr(partial), ptr(Q), ptr(D), ptr(_mask(qmask)),
        ptr(_mask(dmask)), dim, Tq, Td, B, ptr(scores), _norm(normalize), stream_handle(dev))
    _lib.check(st, "launch_paired_scan")


def launch_candidates_scan(args, partial, Q, gallery, idx, qmask, dmask, N, scores=None,
                           neg=-1.0e4, normalize=False):
    dev = require_device(args, partial, Q, gallery, idx, qmask, dmask, scores)
    B, Tq, dim = Q.shape
    Td = gallery.shape[1]
    C = idx.shape[1]
    st = _lib.lib().fms_launch_candidates_scan(
        dtype_code(Q), ptr(args), ptr(partial), ptr(Q), ptr(gallery), ptr(idx), _idx_bytes(idx),
        ptr(_mask(qmask)), ptr(_mask(dmask)), dim, Tq, B, Td, N, C, ptr(scores), float(neg),
        _norm(normalize), stream_handle(dev))
    _lib.check(st, "launch_candidates_scan")


GROUPING_MODES = {"auto": 0, "always": 1, "never": 2}


def candidates_grouping(mode: str) -> str:
    """Set how candidate scans order their pairs ("auto", "always", "never"); returns
    the previous mode.  In document order the pairs that share a gallery document are
    scored together, so the document leaves HBM once per group; results are
    bit-identical either way.  Process-wide (fms_candidates_grouping)."""
    if mode not in GROUPING_MODES:
        raise ArgumentError(f"grouping mode must be one of {sorted(GROUPING_MODES)}")
    prev = _lib.lib().fms_candidates_grouping(GROUPING_MODES[mode])
    return {v: k for k, v in GROUPING_MODES.items()}[prev]


def inbatch_device_scan(S, args, Q, D, qmask, dmask, normalize=False):
    dev = require_device(S, args, Q, D, qmask, dmask)
    Bq, Tq, dim = Q.shape
    Bd, Td = D.shape[0], D.shape[1]
    st = _lib.lib().fms_inbatch_device_scan(
        dtype_code(Q), ptr(S), ptr(args), ptr(Q), ptr(D), ptr(_mask(qmask)), ptr(_mask(dmask)),
        dim, Tq, Bq, Td, Bd, _norm(normalize), stream_handle(dev))
    _lib.check(st, "inbatch_device_scan")


def launch_packed_scan(args, partial, q, tokens, cu, qmask, scores=None, normalize=False):
    dev = require_device(args, partial, q, tokens, cu, qmask, scores)
    Tq, dim = q.shape
    B = cu.shape[0] - 1
    if cu.dtype != torch.int32:
        raise ArgumentError("PackedSeq cu must be Int32 on device")
    st = _lib.lib().fms_launch_packed_scan(
        dtype_code(q), ptr(args), ptr(partial), ptr(q), ptr(tokens), ptr(cu), ptr(_mask(qmask)),
        dim, Tq, B, tokens.shape[0], ptr(scores), _norm(normalize), stream_handle(dev))
    _lib.check(st, "launch_packed_scan")


def launch_packed_multi_scan(args, scores, Q, tokens, cu, qmask, max_len, normalize=False):
    """nq queries Q (nq, Tq, dim) against one PackedSeq in one pass (no reference
    method: the reference scores one query per call).  scores (nq, B) [Julia (B, nq)],
    args (nq, B, Tq) nullable."""
    dev = require_device(args, scores, Q, tokens, cu, qmask)
    nq, Tq, dim = Q.shape
    B = cu.shape[0] - 1
    if cu.dtype != torch.int32:
        raise ArgumentError("PackedSeq cu must be Int32 on device")
    st = _lib.lib().fms_launch_packed_multi_scan(
        dtype_code(Q), ptr(args), ptr(scores), ptr(Q), ptr(tokens), ptr(cu), ptr(_mask(qmask)),
        dim, Tq, nq, B, tokens.shape[0], int(max_len), _norm(normalize), stream_handle(dev))
    _lib.check(st, "launch_packed_multi_scan")


def topk_rows(vals, idx, scores, k):
    """k best entries of every row of scores (nrows, ncols) fp32 [Julia (ncols, nrows),
    one column per query]: vals (nrows, k) descending, idx (nrows, k) 1-based int32.
    No reference method (ranking is the caller's partialsortperm)."""
    dev = require_device(vals, idx, scores)
    nrows, ncols = scores.shape
    st = _lib.lib().fms_topk(ptr(scores), nrows, ncols, int(k), ptr(vals), ptr(idx),
                             stream_handle(dev))
    _lib.check(st, "topk")


def launch_varlen_scan(args, partial, Qp, Dp, cu_q, cu_d, scores=None, normalize=False):
    dev = require_device(args, partial, Qp, Dp, cu_q, cu_d, scores)
    N, max_q = args.shape
    dim = Qp.shape[1]
    if cu_q.dtype != torch.int32 or cu_d.dtype != torch.int32:
        raise ArgumentError("PackedSeq cu must be Int32 on device")
    st = _lib.lib().fms_launch_varlen_scan(
        dtype_code(Qp), ptr(args), ptr(partial), ptr(Qp), ptr(Dp), ptr(cu_q), ptr(cu_d), dim,
        max_q, N, Qp.shape[0], Dp.shape[0], ptr(scores), _norm(normalize), stream_handle(dev))
    _lib.check(st, "launch_varlen_scan")


def _int8(t, what):
    if t is not None and t.dtype != torch.int8:
        raise ArgumentError(f"{what} must be Int8 codes")
    return t


def _f32(t, what):
    if t is not None and t.dtype != torch.float32:
        raise UnsupportedError(f"{what} must be Float32 scales")
    return t


def launch_int8_pair_scan(args, partial, qc, qs, dc, ds, qmask, dmask, score=None,
                          normalize=False):
    dev = require_device(args, partial, qc, qs, dc, ds, qmask, dmask, score)
    Tq, dim = qc.shape
    Td = dc.shape[0]
    st = _lib.lib().fms_launch_int8_pair_scan(
        ptr(args), ptr(partial), ptr(_int8(qc, "qc")), ptr(_f32(qs, "qs")), ptr(_int8(dc, "dc")),
        ptr(_f32(ds, "ds")), ptr(_mask(qmask)), ptr(_mask(dmask)), dim, Tq, Td, ptr(score),
        _norm(normalize), stream_handle(dev))
    _lib.check(st, "launch_int8_pair_scan")


def launch_int8_paired_scan(args, partial, Qc, Qs, Dc, Ds, qmask, dmask, scores=None,
                            normalize=False):
    dev = require_device(args, partial, Qc, Qs, Dc, Ds, qmask, dmask, scores)
    B, Tq, dim = Qc.shape
    Td = Dc.shape[1]
    st = _lib.lib().fms_launch_int8_paired_scan(
        ptr(args), ptr(partial), ptr(_int8(Qc, "Qc")), ptr(_f32(Qs, "Qs")), ptr(_int8(Dc, "Dc")),
        ptr(_f32(Ds, "Ds")), ptr(_mask(qmask)), ptr(_mask(dmask)), dim, Tq, Td, B, ptr(scores),
        _norm(normalize), stream_handle(dev))
    _lib.check(st, "launch_int8_paired_scan")


def launch_int8_candidates_scan(args, partial, Qc, Qs, Gc, Gs, idx, qmask, dmask, N,
                                scores=None, neg=-1.0e4, normalize=False):
    dev = require_device(args, partial, Qc, Qs, Gc, Gs, idx, qmask, dmask, scores)
    B, Tq, dim = Qc.shape
    Td = Gc.shape[1]
    C = idx.shape[1]
    st = _lib.lib().fms_launch_int8_candidates_scan(
        ptr(args), ptr(partial), ptr(_int8(Qc, "Qc")), ptr(_f32(Qs, "Qs")), ptr(_int8(Gc, "Gc")),
        ptr(_f32(Gs, "Gs")), ptr(idx), _idx_bytes(idx), ptr(_mask(qmask)), ptr(_mask(dmask)), dim,
        Tq, B, Td, N, C, ptr(scores), float(neg), _norm(normalize), stream_handle(dev))
    _lib.check(st, "launch_int8_candidates_scan")


def int8_quantize(X, codes, scales):
    dev = require_device(X, codes, scales)
    if X.dtype != torch.float32:
        raise UnsupportedError("quantize_int8_symmetric on device takes Float32 features")
    dim = X.shape[-1] if X.dim() > 0 else 0
    ntok = scales.numel()
    st = _lib.lib().fms_int8_quantize(ptr(X), ptr(codes), ptr(scales), dim, ntok,
                                      stream_handle(dev))
    _lib.check(st, "int8_quantize")


def int8_dots(out, qc, dc):
    """Test-only raw int32 dots: out (Tq, Td) with out[t, u] = <qc_t, dc_u>."""
    dev = require_device(out, qc, dc)
    Tq, dim = qc.shape
    Td = dc.shape[0]
    st = _lib.lib().fms_int8_dots(ptr(out), ptr(qc), ptr(dc), dim, Tq, Td, stream_handle(dev))
    _lib.check(st, "int8_dots")


def length_normalize_(scores, qmask, Tq, nrows, ncols, idx=None, N=0, neg=0.0):
    """In place on the Julia-(nrows, ncols) score matrix (torch (ncols, nrows)):
    column c is multiplied by 1/max(count(qmask[:, c]), 1); invalid idx -> neg."""
    dev = require_device(scores, qmask, idx)
    if scores.numel() != nrows * ncols:
        raise ArgumentError("length_normalize: score shape")
    st = _lib.lib().fms_length_normalize(
        ptr(scores), ptr(_mask(qmask)), Tq, nrows, ncols, ptr(idx),
        0 if idx is None else _idx_bytes(idx), N, float(neg), stream_handle(dev))
    _lib.check(st, "length_normalize")


def varlen_normalize_(scores, cu_q):
    dev = require_device(scores, cu_q)
    st = _lib.lib().fms_varlen_normalize(ptr(scores), ptr(cu_q), scores.numel(),
                                         stream_handle(dev))
    _lib.check(st, "varlen_normalize")


# ---- backward on the argmax tape -------------------------------------------------

def _tape(args):
    if args.dtype != torch.int32:
        raise ArgumentError("argmax tapes are Int32 on device")
    return args


def _like(t, proto, what):
    """Cotangents, inv_n and gradient buffers carry the feature eltype (Vector{T})."""
    if t is not None and t.dtype != proto.dtype:
        raise ArgumentError(f"{what} must have the feature eltype {proto.dtype}, got {t.dtype}")
    return t


def pair_apply_pullback(dq, dd, q, d, qmask, argmax_u, delta):
    """dq (Tq,dim), dd (Td,dim) <- pullback of one pair; delta is a (1,) device array."""
    dev = require_device(dq, dd, q, d, qmask, argmax_u, delta)
    Tq, dim = q.shape
    Td = d.shape[0]
    for t, w in ((dq, "dq"), (dd, "dd"), (d, "d"), (delta, "delta")):
        _like(t, q, w)
    st = _lib.lib().fms_pair_pullback(
        dtype_code(q), ptr(dq), ptr(dd), ptr(q), ptr(d), ptr(_mask(qmask)), ptr(_tape(argmax_u)),
        ptr(delta), dim, Tq, Td, stream_handle(dev))
    _lib.check(st, "pair_apply_pullback")


def paired_apply_pullback(dQ, dD, Q, D, qmask, args, Delta, inv_n):
    dev = require_device(dQ, dD, Q, D, qmask, args, Delta, inv_n)
    B, Tq, dim = Q.shape
    Td = D.shape[1]
    for t, w in ((dQ, "dQ"), (dD, "dD"), (D, "D"), (Delta, "Delta"), (inv_n, "inv_n")):
        _like(t, Q, w)
    st = _lib.lib().fms_paired_pullback(
        dtype_code(Q), ptr(dQ), ptr(dD), ptr(Q), ptr(D), ptr(_mask(qmask)), ptr(_tape(args)),
        ptr(Delta), ptr(inv_n), dim, Tq, Td, B, stream_handle(dev))
    _lib.check(st, "paired_apply_pullback")


def inbatch_apply_pullback(dQ, dD, Q, D, qmask, args, Delta, inv_n):
    """Delta is the torch (Bq, Bd) cotangent (Julia (Bd, Bq)); args (Bq, Bd, Tq)."""
    dev = require_device(dQ, dD, Q, D, qmask, args, Delta, inv_n)
    Bq, Tq, dim = Q.shape
    Bd, Td = D.shape[0], D.shape[1]
    for t, w in ((dQ, "dQ"), (dD, "dD"), (D, "D"), (Delta, "Delta"), (inv_n, "inv_n")):
        _like(t, Q, w)
    st = _lib.lib().fms_inbatch_pullback(
        dtype_code(Q), ptr(dQ), ptr(dD), ptr(Q), ptr(D), ptr(_mask(qmask)), ptr(_tape(args)),
        ptr(Delta), ptr(inv_n), dim, Tq, Td, Bq, Bd, stream_handle(dev))
    _lib.check(st, "inbatch_apply_pullback")


def candidates_apply_pullback(dQ, dG, Q, gallery, idx, qmask, args, Delta, inv_n):
    """Delta (B, C) (Julia (C, B)); args (B, C, Tq); dG like gallery (N, Td, dim)."""
    dev = require_device(dQ, dG, Q, gallery, idx, qmask, args, Delta, inv_n)
    B, Tq, dim = Q.shape
    N, Td = gallery.shape[0], gallery.shape[1]
    C = idx.shape[1]
    for t, w in ((dQ, "dQ"), (dG, "dG"), (gallery, "gallery"), (Delta, "Delta"), (inv_n, "inv_n")):
        _like(t, Q, w)
    st = _lib.lib().fms_candidates_pullback(
        dtype_code(Q), ptr(dQ), ptr(dG), ptr(Q), ptr(gallery), ptr(idx), _idx_bytes(idx),
        ptr(_mask(qmask)), ptr(_tape(args)), ptr(Delta), ptr(inv_n), dim, Tq, B, Td, N, C,
        stream_handle(dev))
    _lib.check(st, "candidates_apply_pullback")


def packed_apply_pullback(dq, dP, q, tokens, cu, qmask, args, Delta, inv_n):
    dev = require_device(dq, dP, q, tokens, cu, qmask, args, Delta, inv_n)
    Tq, dim = q.shape
    B = cu.shape[0] - 1
    if cu.dtype != torch.int32:
        raise ArgumentError("PackedSeq cu must be Int32 on device")
    for t, w in ((dq, "dq"), (dP, "dP"), (tokens, "tokens"), (Delta, "Delta"), (inv_n, "inv_n")):
        _like(t, q, w)
    st = _lib.lib().fms_packed_pullback(
        dtype_code(q), ptr(dq), ptr(dP), ptr(q), ptr(tokens), ptr(cu), ptr(_mask(qmask)),
        ptr(_tape(args)), ptr(Delta), ptr(inv_n), dim, Tq, B, tokens.shape[0],
        stream_handle(dev))
    _lib.check(st, "packed_apply_pullback")


def varlen_apply_pullback(dQ, dD, Qp, Dp, cu_q, cu_d, args, Delta, inv_n):
    """args (N, max_q) (Julia (max_q, N))."""
    dev = require_device(dQ, dD, Qp, Dp, cu_q, cu_d, args, Delta, inv_n)
    N, max_q = args.shape
    dim = Qp.shape[1]
    if cu_q.dtype != torch.int32 or cu_d.dtype != torch.int32:
        raise ArgumentError("PackedSeq cu must be Int32 on device")
    for t, w in ((dQ, "dQ"), (dD, "dD"), (Dp, "D tokens"), (Delta, "Delta"), (inv_n, "inv_n")):
        _like(t, Qp, w)
    st = _lib.lib().fms_varlen_pullback(
        dtype_code(Qp), ptr(dQ), ptr(dD), ptr(Qp), ptr(Dp), ptr(cu_q), ptr(cu_d),
        ptr(_tape(args)), ptr(Delta), ptr(inv_n), dim, max_q, N, Qp.shape[0], Dp.shape[0],
        stream_handle(dev))
    _lib.check(st, "varlen_apply_pullback")
