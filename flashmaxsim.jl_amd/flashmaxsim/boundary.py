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
from .errors import ArgumentError, DimensionMismatch, UnsupportedError

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


# ---- argument checks ---------------------------------------------------------------
# The library writes fp32 partials / scores and int32 tapes and reads features of the
# declared type and dim; a buffer of another type or size would be read or written
# out of bounds on the device.  So every tensor is checked here, before the call:
# wrong element types raise ArgumentError, wrong sizes DimensionMismatch (the
# reference's pre-launch checks, forward_layouts.jl:20-47, forward_pair.jl:14-21,
# packed.jl:138-151, quant.jl:62-94).

def _buf(t, what, dtype, numel):
    """An optional output / index buffer: exact dtype and element count."""
    if t is None:
        return None
    if t.dtype != dtype:
        raise ArgumentError(f"{what} must be {dtype}, got {t.dtype}")
    if t.numel() != numel:
        raise DimensionMismatch(f"{what}: {t.numel()} elements, expected {numel}")
    return t


def _maskn(m, what, numel):
    m = _mask(m)
    if m is not None and m.numel() != numel:
        raise DimensionMismatch(f"{what}: {m.numel()} elements, expected {numel}")
    return m


def _feat(t, what, ndim, proto=None):
    """A feature array of `ndim` dimensions; with `proto`, the same eltype and dim."""
    if t.dim() != ndim:
        raise DimensionMismatch(f"{what} must have {ndim} dimensions, got {t.dim()}")
    if proto is not None:
        if t.dtype != proto.dtype:
            raise ArgumentError(f"{what} must have the feature eltype {proto.dtype}, got {t.dtype}")
        if t.shape[-1] != proto.shape[-1]:
            raise DimensionMismatch(f"feature dim: {what} has {t.shape[-1]}, expected {proto.shape[-1]}")
    return t


def _cu(cu, what, n):
    if cu.dtype != torch.int32:
        raise ArgumentError("PackedSeq cu must be Int32 on device")
    if cu.dim() != 1 or cu.numel() != n:
        raise DimensionMismatch(f"{what}: {cu.numel()} entries, expected {n}")
    return cu


def launch_pair_scan(argmax_u, partial, q, d, qmask, dmask, score=None, normalize=False):
    _feat(q, "q", 2)
    _feat(d, "d", 2, q)
    Tq, dim = q.shape
    Td = d.shape[0]
    _buf(argmax_u, "argmax_u", torch.int32, Tq)
    _buf(partial, "partial", torch.float32, Tq)
    _buf(score, "score", torch.float32, 1)
    dev = require_device(argmax_u, partial, q, d, qmask, dmask, score)
    st = _lib.lib().fms_launch_pair_scan(
        dtype_code(q), ptr(argmax_u), ptr(partial), ptr(q), ptr(d), ptr(_maskn(qmask, "qmask", Tq)),
        ptr(_maskn(dmask, "dmask", Td)), dim, Tq, Td, ptr(score), _norm(normalize),
        stream_handle(dev))
    _lib.check(st, "launch_pair_scan")


def launch_paired_scan(args, partial, Q, D, qmask, dmask, scores=None, normalize=False):
    _feat(Q, "Q", 3)
    _feat(D, "D", 3, Q)
    B, Tq, dim = Q.shape
    Td = D.shape[1]
    if D.shape[0] != B:
        raise DimensionMismatch("batch")
    _buf(args, "args", torch.int32, B * Tq)
    _buf(partial, "partial", torch.float32, B * Tq)
    _buf(scores, "scores", torch.float32, B)
    dev = require_device(args, partial, Q, D, qmask, dmask, scores)
    st = _lib.lib().fms_launch_paired_scan(
        dtype_code(Q), ptr(args), ptr(partial), ptr(Q), ptr(D), ptr(_maskn(qmask, "qmask", B * Tq)),
        ptr(_maskn(dmask, "dmask", B * Td)), dim, Tq, Td, B, ptr(scores), _norm(normalize),
        stream_handle(dev))
    _lib.check(st, "launch_paired_scan")


def launch_candidates_scan(args, partial, Q, gallery, idx, qmask, dmask, N, scores=None,
                           neg=-1.0e4, normalize=False, noalloc=False):
    """launch_candidates_scan! (forward_layouts.jl:292-310).  noalloc=True calls
    fms_launch_candidates_scan_noalloc: the same scan with its grouping workspace in
    the library's static device scratch instead of the memory pool (no device
    allocation).  A call that needs more than that scratch scans in output order
    under automatic grouping and raises UnsupportedError under forced grouping."""
    _feat(Q, "Q", 3)
    _feat(gallery, "gallery", 3, Q)
    B, Tq, dim = Q.shape
    Td = gallery.shape[1]
    if N != gallery.shape[0]:
        raise DimensionMismatch(f"N = {N} but the gallery holds {gallery.shape[0]} documents")
    if idx.dim() != 2 or idx.shape[0] != B:
        raise DimensionMismatch("idxs")
    C = idx.shape[1]
    _buf(args, "args", torch.int32, B * C * Tq)
    _buf(partial, "partial", torch.float32, B * C * Tq)
    _buf(scores, "scores", torch.float32, B * C)
    dev = require_device(args, partial, Q, gallery, idx, qmask, dmask, scores)
    fn = (_lib.lib().fms_launch_candidates_scan_noalloc if noalloc
          else _lib.lib().fms_launch_candidates_scan)
    st = fn(
        dtype_code(Q), ptr(args), ptr(partial), ptr(Q), ptr(gallery), ptr(idx), _idx_bytes(idx),
        ptr(_maskn(qmask, "qmask", B * Tq)), ptr(_maskn(dmask, "dmask", N * Td)), dim, Tq, B, Td, N,
        C, ptr(scores), float(neg), _norm(normalize), stream_handle(dev))
    _lib.check(st, "launch_candidates_scan")


GROUPING_MODES = {"auto": 0, "always": 1, "never": 2, "always_direct_queries": 3}


def candidates_grouping(mode: str) -> str:
    """Set how candidate scans order their pairs ("auto", "always", "never", or
    "always_direct_queries": in document order without the query-tile copy the 16-bit
    document-batch scan otherwise makes, a test switch); returns the previous mode.
    In document order the pairs that share a gallery document are scored together,
    so the document leaves HBM once per group; results are bit-identical either
    way.  Per host thread (fms_candidates_grouping): it changes this thread's later
    calls only."""
    if mode not in GROUPING_MODES:
        raise ArgumentError(f"grouping mode must be one of {sorted(GROUPING_MODES)}")
    prev = _lib.lib().fms_candidates_grouping(GROUPING_MODES[mode])
    return {v: k for k, v in GROUPING_MODES.items()}[prev]


def inbatch_device_scan(S, args, Q, D, qmask, dmask, normalize=False):
    _feat(Q, "Q", 3)
    _feat(D, "D", 3, Q)
    Bq, Tq, dim = Q.shape
    Bd, Td = D.shape[0], D.shape[1]
    if S is None:
        raise ArgumentError("inbatch_device_scan needs the score matrix S")
    _buf(S, "S", torch.float32, Bq * Bd)
    _buf(args, "args", torch.int32, Bq * Bd * Tq)
    dev = require_device(S, args, Q, D, qmask, dmask)
    st = _lib.lib().fms_inbatch_device_scan(
        dtype_code(Q), ptr(S), ptr(args), ptr(Q), ptr(D), ptr(_maskn(qmask, "qmask", Bq * Tq)),
        ptr(_maskn(dmask, "dmask", Bd * Td)), dim, Tq, Bq, Td, Bd, _norm(normalize),
        stream_handle(dev))
    _lib.check(st, "inbatch_device_scan")


def launch_packed_scan(args, partial, q, tokens, cu, qmask, scores=None, normalize=False):
    _feat(q, "q", 2)
    _feat(tokens, "tokens", 2, q)
    Tq, dim = q.shape
    B = cu.shape[0] - 1
    _cu(cu, "cu", B + 1)
    _buf(args, "args", torch.int32, B * Tq)
    _buf(partial, "partial", torch.float32, B * Tq)
    _buf(scores, "scores", torch.float32, B)
    dev = require_device(args, partial, q, tokens, cu, qmask, scores)
    st = _lib.lib().fms_launch_packed_scan(
        dtype_code(q), ptr(args), ptr(partial), ptr(q), ptr(tokens), ptr(cu),
        ptr(_maskn(qmask, "qmask", Tq)), dim, Tq, B, tokens.shape[0], ptr(scores),
        _norm(normalize), stream_handle(dev))
    _lib.check(st, "launch_packed_scan")


def launch_packed_multi_scan(args, scores, Q, tokens, cu, qmask, max_len, normalize=False):
    """nq queries Q (nq, Tq, dim) against one PackedSeq in one pass (no reference
    method: the reference scores one query per call).  scores (nq, B) [Julia (B, nq)],
    args (nq, B, Tq) nullable.  Every document must be at most max_len tokens (the
    PackedSeq's max_len); the library checks that on the device and flags a
    violation through a NaN score row (see fms_launch_packed_multi_scan)."""
    _feat(Q, "Q", 3)
    _feat(tokens, "tokens", 2, Q)
    nq, Tq, dim = Q.shape
    B = cu.shape[0] - 1
    _cu(cu, "cu", B + 1)
    if scores is None:
        raise ArgumentError("launch_packed_multi_scan needs the score matrix")
    _buf(scores, "scores", torch.float32, nq * B)
    _buf(args, "args", torch.int32, nq * B * Tq)
    dev = require_device(args, scores, Q, tokens, cu, qmask)
    st = _lib.lib().fms_launch_packed_multi_scan(
        dtype_code(Q), ptr(args), ptr(scores), ptr(Q), ptr(tokens), ptr(cu),
        ptr(_maskn(qmask, "qmask", nq * Tq)), dim, Tq, nq, B, tokens.shape[0], int(max_len),
        _norm(normalize), stream_handle(dev))
    _lib.check(st, "launch_packed_multi_scan")


def topk_rows(vals, idx, scores, k):
    """k best entries of every row of scores (nrows, ncols) fp32 [Julia (ncols, nrows),
    one column per query]: vals (nrows, k) descending, idx (nrows, k) 1-based int32.
    No reference method (ranking is the caller's partialsortperm)."""
    if scores.dim() != 2:
        raise DimensionMismatch("top-k scores must be a matrix")
    nrows, ncols = scores.shape
    _buf(scores, "scores", torch.float32, nrows * ncols)
    if 0 <= k <= ncols:
        _buf(vals, "vals", torch.float32, nrows * k)
        _buf(idx, "idx", torch.int32, nrows * k)
    dev = require_device(vals, idx, scores)
    st = _lib.lib().fms_topk(ptr(scores), nrows, ncols, int(k), ptr(vals), ptr(idx),
                             stream_handle(dev))
    _lib.check(st, "topk")


def launch_varlen_scan(args, partial, Qp, Dp, cu_q, cu_d, scores=None, normalize=False,
                       max_q=None):
    """The shapes come from args (N, max_q), as in the reference method; without a
    tape (args None) max_q is given and N is the pair count of cu_q."""
    if args is None:
        if max_q is None or scores is None:
            raise ArgumentError("launch_varlen_scan without args needs max_q and scores")
        N = cu_q.numel() - 1
    elif args.dim() != 2:
        raise DimensionMismatch("varlen args must be (N, max_q)")
    else:
        N, max_q = args.shape
    _feat(Qp, "Q tokens", 2)
    _feat(Dp, "D tokens", 2, Qp)
    dim = Qp.shape[1]
    _cu(cu_q, "cu_q", N + 1)
    _cu(cu_d, "cu_d", N + 1)
    _buf(args, "args", torch.int32, N * max_q)
    _buf(partial, "partial", torch.float32, N * max_q)
    _buf(scores, "scores", torch.float32, N)
    dev = require_device(args, partial, Qp, Dp, cu_q, cu_d, scores)
    st = _lib.lib().fms_launch_varlen_scan(
        dtype_code(Qp), ptr(args), ptr(partial), ptr(Qp), ptr(Dp), ptr(cu_q), ptr(cu_d), dim,
        max_q, N, Qp.shape[0], Dp.shape[0], ptr(scores), _norm(normalize), stream_handle(dev))
    _lib.check(st, "launch_varlen_scan")


_SCALE_CODES = {torch.float32: _lib.FMS_F32, torch.float16: _lib.FMS_F16}


def _int8(t, what):
    if t is not None and t.dtype != torch.int8:
        raise ArgumentError(f"{what} must be Int8 codes")
    return t


def _scales(t, what, numel):
    """INT8 scales: Float32 or Float16 (an Int8Index keeps its features' eltype)."""
    if t.dtype not in _SCALE_CODES:
        raise UnsupportedError(f"{what} must be Float32 or Float16 scales, got {t.dtype}")
    if t.numel() != numel:
        raise DimensionMismatch(f"{what}: {t.numel()} scales, expected {numel}")
    return _SCALE_CODES[t.dtype]


def launch_int8_pair_scan(args, partial, qc, qs, dc, ds, qmask, dmask, score=None,
                          normalize=False):
    _feat(_int8(qc, "qc"), "qc", 2)
    _feat(_int8(dc, "dc"), "dc", 2, qc)
    Tq, dim = qc.shape
    Td = dc.shape[0]
    qsc, dsc = _scales(qs, "qs", Tq), _scales(ds, "ds", Td)
    _buf(args, "args", torch.int32, Tq)
    _buf(partial, "partial", torch.float32, Tq)
    _buf(score, "score", torch.float32, 1)
    dev = require_device(args, partial, qc, qs, dc, ds, qmask, dmask, score)
    st = _lib.lib().fms_launch_int8_pair_scan(
        ptr(args), ptr(partial), ptr(qc), ptr(qs), qsc, ptr(dc), ptr(ds), dsc,
        ptr(_maskn(qmask, "qmask", Tq)), ptr(_maskn(dmask, "dmask", Td)), dim, Tq, Td, ptr(score),
        _norm(normalize), stream_handle(dev))
    _lib.check(st, "launch_int8_pair_scan")


def launch_int8_paired_scan(args, partial, Qc, Qs, Dc, Ds, qmask, dmask, scores=None,
                            normalize=False):
    _feat(_int8(Qc, "Qc"), "Qc", 3)
    _feat(_int8(Dc, "Dc"), "Dc", 3, Qc)
    B, Tq, dim = Qc.shape
    Td = Dc.shape[1]
    if Dc.shape[0] != B:
        raise DimensionMismatch("batch")
    qsc, dsc = _scales(Qs, "Qs", B * Tq), _scales(Ds, "Ds", B * Td)
    _buf(args, "args", torch.int32, B * Tq)
    _buf(partial, "partial", torch.float32, B * Tq)
    _buf(scores, "scores", torch.float32, B)
    dev = require_device(args, partial, Qc, Qs, Dc, Ds, qmask, dmask, scores)
    st = _lib.lib().fms_launch_int8_paired_scan(
        ptr(args), ptr(partial), ptr(Qc), ptr(Qs), qsc, ptr(Dc), ptr(Ds), dsc,
        ptr(_maskn(qmask, "qmask", B * Tq)), ptr(_maskn(dmask, "dmask", B * Td)), dim, Tq, Td, B,
        ptr(scores), _norm(normalize), stream_handle(dev))
    _lib.check(st, "launch_int8_paired_scan")


def launch_int8_candidates_scan(args, partial, Qc, Qs, Gc, Gs, idx, qmask, dmask, N,
                                scores=None, neg=-1.0e4, normalize=False):
    _feat(_int8(Qc, "Qc"), "Qc", 3)
    _feat(_int8(Gc, "Gc"), "Gc", 3, Qc)
    B, Tq, dim = Qc.shape
    Td = Gc.shape[1]
    if N != Gc.shape[0]:
        raise DimensionMismatch(f"N = {N} but the gallery holds {Gc.shape[0]} documents")
    if idx.dim() != 2 or idx.shape[0] != B:
        raise DimensionMismatch("idxs")
    C = idx.shape[1]
    qsc, dsc = _scales(Qs, "Qs", B * Tq), _scales(Gs, "Gs", N * Td)
    _buf(args, "args", torch.int32, B * C * Tq)
    _buf(partial, "partial", torch.float32, B * C * Tq)
    _buf(scores, "scores", torch.float32, B * C)
    dev = require_device(args, partial, Qc, Qs, Gc, Gs, idx, qmask, dmask, scores)
    st = _lib.lib().fms_launch_int8_candidates_scan(
        ptr(args), ptr(partial), ptr(Qc), ptr(Qs), qsc, ptr(Gc), ptr(Gs), dsc, ptr(idx),
        _idx_bytes(idx), ptr(_maskn(qmask, "qmask", B * Tq)), ptr(_maskn(dmask, "dmask", N * Td)),
        dim, Tq, B, Td, N, C, ptr(scores), float(neg), _norm(normalize), stream_handle(dev))
    _lib.check(st, "launch_int8_candidates_scan")


def int8_quantize(X, codes, scales):
    """quantize_int8_symmetric (quant.jl:42-49) of Float32 or Float16 features X
    (..., dim): codes int8 of X's shape, scales (...) of X's eltype."""
    if X.dtype not in _SCALE_CODES:
        raise UnsupportedError("quantize_int8_symmetric on device takes Float32 or Float16 features")
    if X.dim() < 1:
        raise DimensionMismatch("features need a feature dimension")
    dim = X.shape[-1]
    ntok = X.numel() // dim if dim > 0 else scales.numel()
    _buf(_int8(codes, "codes"), "codes", torch.int8, X.numel())
    _buf(scales, "scales", X.dtype, ntok)
    dev = require_device(X, codes, scales)
    st = _lib.lib().fms_int8_quantize(_SCALE_CODES[X.dtype], ptr(X), ptr(codes), ptr(scales), dim,
                                      ntok, stream_handle(dev))
    _lib.check(st, "int8_quantize")


def int8_dots(out, qc, dc):
    """Test-only raw int32 dots: out (Tq, Td) with out[t, u] = <qc_t, dc_u>."""
    _feat(_int8(qc, "qc"), "qc", 2)
    _feat(_int8(dc, "dc"), "dc", 2, qc)
    Tq, dim = qc.shape
    Td = dc.shape[0]
    _buf(out, "out", torch.int32, Tq * Td)
    dev = require_device(out, qc, dc)
    st = _lib.lib().fms_int8_dots(ptr(out), ptr(qc), ptr(dc), dim, Tq, Td, stream_handle(dev))
    _lib.check(st, "int8_dots")


def length_normalize_(scores, qmask, Tq, nrows, ncols, idx=None, N=0, neg=0.0):
    """In place on the Julia-(nrows, ncols) score matrix (torch (ncols, nrows)):
    column c is multiplied by 1/max(count(qmask[:, c]), 1); invalid idx -> neg."""
    _buf(scores, "scores", torch.float32, nrows * ncols)
    _maskn(qmask, "qmask", Tq * ncols)
    if idx is not None and idx.numel() != nrows * ncols:
        raise DimensionMismatch("length_normalize: idx shape")
    dev = require_device(scores, qmask, idx)
    st = _lib.lib().fms_length_normalize(
        ptr(scores), ptr(_mask(qmask)), Tq, nrows, ncols, ptr(idx),
        0 if idx is None else _idx_bytes(idx), N, float(neg), stream_handle(dev))
    _lib.check(st, "length_normalize")


def varlen_normalize_(scores, cu_q):
    _buf(scores, "scores", torch.float32, scores.numel())
    _cu(cu_q, "cu_q", scores.numel() + 1)
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
