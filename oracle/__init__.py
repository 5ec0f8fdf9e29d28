"""CPU parity oracle for the fused MaxSim forward -- TEST INFRASTRUCTURE ONLY.

ctypes wrapper over ``oracle/libfms_oracle.so`` (built from
``oracle/fms_oracle.c`` by ``oracle/Makefile``), a C restatement of
FlashMaxSim.jl's CPU semantics.  Only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg may import this package, and only as
the checker or the timed CPU baseline -- never as the product path.

Array convention: numpy arrays in *reversed-shape C order*, which is
byte-for-byte the reference's Julia column-major layout.  A Julia
``Q::Array{T,3}`` of size ``(dim, Tq, B)`` is the numpy array
``Q.shape == (B, Tq, dim)``; a mask ``(Tq, B)`` is ``(B, Tq)``; an index
matrix ``(C, B)`` is ``(B, C)``; a tape ``(Tq, C, B)`` is ``(B, C, Tq)``.
Feature dtypes: ``float32``, ``float16``, and bfloat16 carried as ``uint16``
bit patterns (pass ``bf16=True``).

Function-level parity pins (each is exercised in ``tests/test_oracle.py``):

* pair/paired/candidates/in-batch/packed/varlen scans -- closed forms from
  the reference's tests (all-negative dots => -Tq*dim, empty doc => 0,
  invalid idx => neg), an fp64 dense brute force (``dense_pair_f64``), an
  independent numpy materialising implementation, and layout invariants.
* quantize_int8 -- closed-form cases (ties-to-even, clamp, eps and floatmin
  floors) and numpy's round-half-even on random data; for Float16 features,
  numpy's own float16 arithmetic (an independent binary16 implementation).
* int8 dots / int8 scans -- exact integer arithmetic vs numpy int32 matmul,
  fixed dequant order ``(qs*ds)*float(acc)``.
* backward (``*_backward``) -- an independent numpy scatter (``np.add.at``)
  on the same tapes, finite differences of the forward score, linearity in
  the cotangent, and the layout invariants the forward has.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libfms_oracle.so")

F32, F16, BF16, F64 = 0, 1, 2, 3

_lib = None


def build() -> str:
    """Compile the oracle (gcc; CPU only)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f = ctypes.c_float


def _declare(L):
    L.fmso_max_threads.restype = _int
    L.fmso_pair_forward.restype = _f
    L.fmso_pair_forward.argtypes = [_int, _p, _p, _p, _p, _i64, _i64, _i64, _p, _p]
    L.fmso_paired_forward.restype = None
    L.fmso_paired_forward.argtypes = [_int, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p, _p, _p, _int]
    L.fmso_candidates_forward.restype = None
    L.fmso_candidates_forward.argtypes = [_int, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                          _i64, _f, _p, _p, _p, _p, _i64, _int]
    L.fmso_inbatch_forward.restype = None
    L.fmso_inbatch_forward.argtypes = [_int, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _int]
    L.fmso_inbatch_doc_chunk.restype = _i64
    L.fmso_inbatch_doc_chunk.argtypes = [_i64] * 5
    L.fmso_packed_forward.restype = None
    L.fmso_packed_forward.argtypes = [_int, _p, _p, _p, _p, _i64, _i64, _i64, _p, _p, _p, _p, _i64, _int]
    L.fmso_varlen_forward.restype = None
    L.fmso_varlen_forward.argtypes = [_int, _p, _p, _p, _p, _i64, _i64, _i64, _p, _p, _p, _int]
    L.fmso_quantize_int8.restype = None
    L.fmso_quantize_int8.argtypes = [_p, _i64, _i64, _p, _p]
    L.fmso_quantize_int8_f16.restype = None
    L.fmso_quantize_int8_f16.argtypes = [_p, _i64, _i64, _p, _p]
    L.fmso_f32_to_f16.restype = None
    L.fmso_f32_to_f16.argtypes = [_p, _i64, _p]
    L.fmso_int8_dots.restype = None
    L.fmso_int8_dots.argtypes = [_p, _p, _i64, _i64, _i64, _p]
    L.fmso_int8_paired_forward.restype = None
    L.fmso_int8_paired_forward.argtypes = [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p, _p, _p, _int]
    L.fmso_int8_candidates_forward.restype = None
    L.fmso_int8_candidates_forward.argtypes = [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                               _i64, _f, _p, _p, _p, _p, _i64, _int]
    L.fmso_inv_token_counts.restype = None
    L.fmso_inv_token_counts.argtypes = [_p, _i64, _i64, _p]
    L.fmso_dense_pair_f64.restype = ctypes.c_double
    L.fmso_dense_pair_f64.argtypes = [_int, _p, _p, _p, _p, _i64, _i64, _i64, _int, _p]
    L.fmso_paired_backward.restype = None
    L.fmso_paired_backward.argtypes = [_int, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p, _p]
    L.fmso_inbatch_backward.restype = None
    L.fmso_inbatch_backward.argtypes = [_int, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                        _p, _p]
    L.fmso_candidates_backward.restype = None
    L.fmso_candidates_backward.argtypes = [_int, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64,
                                           _i64, _i64, _p, _p]
    L.fmso_packed_backward.restype = None
    L.fmso_packed_backward.argtypes = [_int, _p, _p, _p, _p, _p, _p, ctypes.c_double, _i64, _i64,
                                       _i64, _i64, _p, _p]
    L.fmso_varlen_backward.restype = None
    L.fmso_varlen_backward.argtypes = [_int, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64,
                                       _i64, _p, _p]
    L.fmso_topk.restype = None
    L.fmso_topk.argtypes = [_p, _i64, _i64, _i64, _p, _p]


def max_threads() -> int:
    return int(lib().fmso_max_threads())


# ---- helpers -------------------------------------------------------------------

def _ptr(a):
    return None if a is None else a.ctypes.data


def _dtype_code(a: np.ndarray, bf16: bool) -> int:
    if bf16:
        if a.dtype != np.uint16:
            raise TypeError("bfloat16 features are carried as uint16 bit patterns")
        return BF16
    if a.dtype == np.float32:
        return F32
    if a.dtype == np.float16:
        return F16
    if a.dtype == np.float64:
        return F64
    raise TypeError(f"unsupported feature dtype {a.dtype}")


def _c(a, dtype=None):
    if a is None:
        return None
    a = np.ascontiguousarray(a if dtype is None else a.astype(dtype, copy=False))
    return a


def _mask(m):
    return None if m is None else np.ascontiguousarray(m, dtype=np.uint8)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round fp32 to bfloat16 (round-to-nearest-even), returned as uint16 bits."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def widen(x: np.ndarray, bf16: bool = False) -> np.ndarray:
    """Exact fp32 (or fp64) view of stored features."""
    if bf16:
        return bf16_bits_to_f32(x)
    return x.astype(np.float64 if x.dtype == np.float64 else np.float32)


# ---- layouts ---------------------------------------------------------------------

def pair_forward(q, d, qmask=None, dmask=None, bf16=False):
    """pair_forward_host (src/forward_pair.jl:45-95). q (Tq,dim), d (Td,dim)."""
    q, d = _c(q), _c(d)
    code = _dtype_code(q, bf16)
    Tq, dim = q.shape
    Td = d.shape[0]
    args = np.zeros(Tq, np.int32)
    part = np.zeros(Tq, np.float32)
    qm, dm = _mask(qmask), _mask(dmask)
    s = lib().fmso_pair_forward(code, _ptr(q), _ptr(d), _ptr(qm), _ptr(dm), dim, Tq, Td,
                                _ptr(args), _ptr(part))
    return np.float32(s), args, part


def paired_forward(Q, D, qmask=None, dmask=None, bf16=False, nthreads=0):
    """paired_forward(::CPU) (src/forward_layouts.jl:86-103). Q (B,Tq,dim), D (B,Td,dim)."""
    Q, D = _c(Q), _c(D)
    code = _dtype_code(Q, bf16)
    B, Tq, dim = Q.shape
    Td = D.shape[1]
    scores = np.zeros(B, np.float32)
    args = np.zeros((B, Tq), np.int32)
    part = np.zeros((B, Tq), np.float32)
    qm, dm = _mask(qmask), _mask(dmask)
    lib().fmso_paired_forward(code, _ptr(Q), _ptr(D), _ptr(qm), _ptr(dm), dim, Tq, Td, B,
                              _ptr(scores), _ptr(args), _ptr(part), nthreads)
    return scores, args, part


def candidates_forward(Q, G, idxs, qmask=None, dmask=None, neg=-1.0e4, bf16=False,
                       subset=None, nthreads=0):
    """candidates_forward(::CPU) (src/forward_layouts.jl:239-261).

    Q (B,Tq,dim), G (N,Td,dim), idxs (B,C) 1-based.  ``subset`` (optional)
    lists linear pair ids ``c + C*b`` to compute; other outputs stay
    neg / zero.  Returns S (B,C), args (B,C,Tq), partial (B,C,Tq).
    """
    Q, G = _c(Q), _c(G)
    code = _dtype_code(Q, bf16)
    B, Tq, dim = Q.shape
    N, Td = G.shape[0], G.shape[1]
    idx = _c(idxs, np.int64)
    C = idx.shape[1]
    S = np.full((B, C), np.float32(neg), np.float32)
    args = np.zeros((B, C, Tq), np.int32)
    part = np.zeros((B, C, Tq), np.float32)
    sub = None if subset is None else _c(subset, np.int64)
    qm, dm = _mask(qmask), _mask(dmask)
    lib().fmso_candidates_forward(code, _ptr(Q), _ptr(G), _ptr(idx), _ptr(qm), _ptr(dm), dim, Tq, B,
                                  Td, N, C, float(np.float32(neg)), _ptr(S), _ptr(args), _ptr(part),
                                  _ptr(sub), 0 if sub is None else sub.size, nthreads)
    return S, args, part


def inbatch_forward(Q, D, qmask=None, dmask=None, bf16=False, nthreads=0):
    """inbatch_forward(::CPU) (src/forward_layouts.jl:155-179). Returns S (Bq,Bd), args (Bq,Bd,Tq)."""
    Q, D = _c(Q), _c(D)
    code = _dtype_code(Q, bf16)
    Bq, Tq, dim = Q.shape
    Bd, Td = D.shape[0], D.shape[1]
    S = np.zeros((Bq, Bd), np.float32)
    args = np.zeros((Bq, Bd, Tq), np.int32)
    qm, dm = _mask(qmask), _mask(dmask)
    lib().fmso_inbatch_forward(code, _ptr(Q), _ptr(D), _ptr(qm), _ptr(dm), dim, Tq, Bq, Td, Bd,
                               _ptr(S), _ptr(args), nthreads)
    return S, args


def inbatch_doc_chunk(elsize, Td, Tq, Bq, Bd):
    return int(lib().fmso_inbatch_doc_chunk(elsize, Td, Tq, Bq, Bd))


def packed_forward(q, tokens, cu, qmask=None, bf16=False, subset=None, nthreads=0):
    """packed_forward_host (src/packed.jl:153-176). q (Tq,dim), tokens (ntok,dim), cu (B+1,) 1-based."""
    q, tokens = _c(q), _c(tokens)
    code = _dtype_code(q, bf16)
    Tq, dim = q.shape
    cu = _c(cu, np.int32)
    B = cu.size - 1
    scores = np.zeros(B, np.float32)
    args = np.zeros((B, Tq), np.int32)
    part = np.zeros((B, Tq), np.float32)
    sub = None if subset is None else _c(subset, np.int64)
    qm = _mask(qmask)
    lib().fmso_packed_forward(code, _ptr(q), _ptr(tokens), _ptr(cu), _ptr(qm), dim, Tq, B,
                              _ptr(scores), _ptr(args), _ptr(part), _ptr(sub),
                              0 if sub is None else sub.size, nthreads)
    return scores, args, part


def varlen_forward(Qt, Dt, cu_q, cu_d, max_q=None, bf16=False, nthreads=0):
    """varlen_forward_host (src/packed.jl:236-260). Returns scores (N,), args/partial (N,max_q)."""
    Qt, Dt = _c(Qt), _c(Dt)
    code = _dtype_code(Qt, bf16)
    dim = Qt.shape[1]
    cu_q, cu_d = _c(cu_q, np.int32), _c(cu_d, np.int32)
    N = cu_q.size - 1
    if max_q is None:
        max_q = int(np.max(np.diff(cu_q))) if N > 0 else 0
    scores = np.zeros(N, np.float32)
    args = np.zeros((N, max_q), np.int32)
    part = np.zeros((N, max_q), np.float32)
    lib().fmso_varlen_forward(code, _ptr(Qt), _ptr(Dt), _ptr(cu_q), _ptr(cu_d), dim, N, max_q,
                              _ptr(scores), _ptr(args), _ptr(part), nthreads)
    return scores, args, part


def quantize_int8(x):
    """quantize_int8_symmetric (src/quant.jl:42-49) for Float32 or Float16 features
    x (..., dim); the scales keep x's dtype (computed in that type)."""
    half = np.asarray(x).dtype == np.float16
    x = _c(x, np.float16 if half else np.float32)
    dim = x.shape[-1]
    ntok = x.size // max(dim, 1) if dim > 0 else int(np.prod(x.shape[:-1]))
    codes = np.zeros(x.shape, np.int8)
    scales = np.zeros(x.shape[:-1], np.float16 if half else np.float32)
    if half:
        lib().fmso_quantize_int8_f16(_ptr(x), dim, ntok, _ptr(codes), _ptr(scales))
    else:
        lib().fmso_quantize_int8(_ptr(x), dim, ntok, _ptr(codes), _ptr(scales))
    return codes, scales


def f32_to_f16(x):
    """The oracle's binary32 -> binary16 rounding (RNE), as float16 values."""
    x = _c(x, np.float32)
    out = np.zeros(x.shape, np.uint16)
    lib().fmso_f32_to_f16(_ptr(x), x.size, _ptr(out))
    return out.view(np.float16)


def int8_dots(qc, dc):
    """Raw int32 dots (quant.jl:109-112): returns (Tq, Td) with out[t,u] = <qc_t, dc_u>."""
    qc, dc = _c(qc, np.int8), _c(dc, np.int8)
    Tq, dim = qc.shape
    Td = dc.shape[0]
    out = np.zeros((Tq, Td), np.int32)
    lib().fmso_int8_dots(_ptr(qc), _ptr(dc), dim, Tq, Td, _ptr(out))
    return out


def int8_paired_forward(Qc, Qs, Dc, Ds, qmask=None, dmask=None, nthreads=0):
    """int8_paired_forward_host (src/quant.jl:172-185)."""
    Qc, Dc = _c(Qc, np.int8), _c(Dc, np.int8)
    Qs, Ds = _c(Qs, np.float32), _c(Ds, np.float32)
    B, Tq, dim = Qc.shape
    Td = Dc.shape[1]
    scores = np.zeros(B, np.float32)
    args = np.zeros((B, Tq), np.int32)
    part = np.zeros((B, Tq), np.float32)
    qm, dm = _mask(qmask), _mask(dmask)
    lib().fmso_int8_paired_forward(_ptr(Qc), _ptr(Qs), _ptr(Dc), _ptr(Ds), _ptr(qm), _ptr(dm),
                                   dim, Tq, Td, B, _ptr(scores), _ptr(args), _ptr(part), nthreads)
    return scores, args, part


def int8_candidates_forward(Qc, Qs, Gc, Gs, idxs, qmask=None, dmask=None, neg=-1.0e4,
                            subset=None, nthreads=0):
    """INT8 pair scan composed with the candidate conventions (no reference method)."""
    Qc, Gc = _c(Qc, np.int8), _c(Gc, np.int8)
    Qs, Gs = _c(Qs, np.float32), _c(Gs, np.float32)
    B, Tq, dim = Qc.shape
    N, Td = Gc.shape[0], Gc.shape[1]
    idx = _c(idxs, np.int64)
    C = idx.shape[1]
    S = np.full((B, C), np.float32(neg), np.float32)
    args = np.zeros((B, C, Tq), np.int32)
    part = np.zeros((B, C, Tq), np.float32)
    sub = None if subset is None else _c(subset, np.int64)
    qm, dm = _mask(qmask), _mask(dmask)
    lib().fmso_int8_candidates_forward(_ptr(Qc), _ptr(Qs), _ptr(Gc), _ptr(Gs), _ptr(idx), _ptr(qm),
                                       _ptr(dm), dim, Tq, B, Td, N, C, float(np.float32(neg)),
                                       _ptr(S), _ptr(args), _ptr(part), _ptr(sub),
                                       0 if sub is None else sub.size, nthreads)
    return S, args, part


def inv_token_counts(qmask, Tq=None, B=None):
    """src/normalize.jl:4-10 with normalize=true. qmask (B,Tq)."""
    qm = _mask(qmask)
    B, Tq = qm.shape
    inv = np.zeros(B, np.float32)
    lib().fmso_inv_token_counts(_ptr(qm), Tq, B, _ptr(inv))
    return inv


def dense_pair_f64(q, d, qmask=None, dmask=None, normalize=False, bf16=False):
    """maxsim_dense with accum=Float64 (src/dense.jl:26-56). Returns (score, first-hit args)."""
    q, d = _c(q), _c(d)
    code = _dtype_code(q, bf16)
    Tq, dim = q.shape
    Td = d.shape[0]
    args = np.zeros(Tq, np.int32)
    qm, dm = _mask(qmask), _mask(dmask)
    s = lib().fmso_dense_pair_f64(code, _ptr(q), _ptr(d), _ptr(qm), _ptr(dm), dim, Tq, Td,
                                  int(bool(normalize)), _ptr(args))
    return float(s), args


# ---- backward on the argmax tape ---------------------------------------------------

def _f64(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float64)


def paired_backward(Q, D, args, Delta, inv_n=None, qmask=None, bf16=False):
    """paired_pullback (src/backward_layouts.jl:13-26), fp64.  Q (B,Tq,dim), D (B,Td,dim),
    args (B,Tq) 1-based tape, Delta (B,), inv_n (B,) or None.  Returns (dQ, dD) fp64."""
    Q, D = _c(Q), _c(D)
    code = _dtype_code(Q, bf16)
    B, Tq, dim = Q.shape
    Td = D.shape[1]
    args = _c(args, np.int32)
    dQ = np.zeros((B, Tq, dim), np.float64)
    dD = np.zeros((B, Td, dim), np.float64)
    qm, De, iv = _mask(qmask), _f64(Delta), _f64(inv_n)
    lib().fmso_paired_backward(code, _ptr(Q), _ptr(D), _ptr(qm), _ptr(args), _ptr(De), _ptr(iv),
                               dim, Tq, Td, B, _ptr(dQ), _ptr(dD))
    return dQ, dD


def inbatch_backward(Q, D, args, Delta, inv_n=None, qmask=None, bf16=False):
    """inbatch_pullback (src/backward_layouts.jl:68-94), fp64.  Q (Bq,Tq,dim), D (Bd,Td,dim),
    args (Bq,Bd,Tq), Delta (Bq,Bd) [Julia (Bd,Bq)], inv_n (Bq,)."""
    Q, D = _c(Q), _c(D)
    code = _dtype_code(Q, bf16)
    Bq, Tq, dim = Q.shape
    Bd, Td = D.shape[0], D.shape[1]
    args = _c(args, np.int32)
    dQ = np.zeros((Bq, Tq, dim), np.float64)
    dD = np.zeros((Bd, Td, dim), np.float64)
    qm, De, iv = _mask(qmask), _f64(Delta), _f64(inv_n)
    lib().fmso_inbatch_backward(code, _ptr(Q), _ptr(D), _ptr(qm), _ptr(args), _ptr(De), _ptr(iv),
                                dim, Tq, Td, Bq, Bd, _ptr(dQ), _ptr(dD))
    return dQ, dD


def candidates_backward(Q, G, idxs, args, Delta, inv_n=None, qmask=None, bf16=False):
    """candidates_pullback (src/backward_layouts.jl:136-165), fp64.  Q (B,Tq,dim),
    G (N,Td,dim), idxs (B,C) 1-based, args (B,C,Tq), Delta (B,C), inv_n (B,)."""
    Q, G = _c(Q), _c(G)
    code = _dtype_code(Q, bf16)
    B, Tq, dim = Q.shape
    N, Td = G.shape[0], G.shape[1]
    C = idxs.shape[1]
    idxs = _c(idxs, np.int64)
    args = _c(args, np.int32)
    dQ = np.zeros((B, Tq, dim), np.float64)
    dG = np.zeros((N, Td, dim), np.float64)
    qm, De, iv = _mask(qmask), _f64(Delta), _f64(inv_n)
    lib().fmso_candidates_backward(code, _ptr(Q), _ptr(G), _ptr(idxs), _ptr(qm), _ptr(args),
                                   _ptr(De), _ptr(iv), dim, Tq, Td, B, C, N, _ptr(dQ), _ptr(dG))
    return dQ, dG


def packed_backward(q, tokens, cu, args, Delta, inv_n=1.0, qmask=None, bf16=False):
    """packed_pullback (src/packed.jl:361-377), fp64.  q (Tq,dim), tokens (ntok,dim),
    cu (B+1,) 1-based, args (B,Tq), Delta (B,), inv_n scalar."""
    q, tokens = _c(q), _c(tokens)
    code = _dtype_code(q, bf16)
    Tq, dim = q.shape
    ntok = tokens.shape[0]
    cu = _c(cu, np.int32)
    B = cu.shape[0] - 1
    args = _c(args, np.int32)
    dq = np.zeros((Tq, dim), np.float64)
    dP = np.zeros((ntok, dim), np.float64)
    qm, De = _mask(qmask), _f64(Delta)
    lib().fmso_packed_backward(code, _ptr(q), _ptr(tokens), _ptr(cu), _ptr(qm), _ptr(args),
                               _ptr(De), float(inv_n), dim, Tq, B, ntok, _ptr(dq), _ptr(dP))
    return dq, dP


def varlen_backward(Qt, Dt, cu_q, cu_d, args, Delta, inv_n=None, bf16=False):
    """varlen_pullback (src/packed.jl:424-442), fp64.  Qt (nq,dim), Dt (nd,dim),
    cu_q/cu_d (N+1,) 1-based, args (N,max_q), Delta (N,), inv_n (N,)."""
    Qt, Dt = _c(Qt), _c(Dt)
    code = _dtype_code(Qt, bf16)
    nq, dim = Qt.shape
    nd = Dt.shape[0]
    cu_q, cu_d = _c(cu_q, np.int32), _c(cu_d, np.int32)
    N = cu_q.shape[0] - 1
    args = _c(args, np.int32)
    max_q = args.shape[1]
    dQ = np.zeros((nq, dim), np.float64)
    dD = np.zeros((nd, dim), np.float64)
    De, iv = _f64(Delta), _f64(inv_n)
    lib().fmso_varlen_backward(code, _ptr(Qt), _ptr(Dt), _ptr(cu_q), _ptr(cu_d), _ptr(args),
                               _ptr(De), _ptr(iv), dim, max_q, N, nq, nd, _ptr(dQ), _ptr(dD))
    return dQ, dD


def topk(scores, k):
    """Per-row top-k (no reference counterpart; the caller's stable
    partialsortperm(rev = true) in the reference, README.md:132).  scores
    (nrows, ncols) fp32 -> (vals (nrows, k) fp32, idx (nrows, k) int32 1-based)."""
    S = _c(scores, np.float32)
    if S.ndim == 1:
        S = S.reshape(1, -1)
    nrows, ncols = S.shape
    vals = np.zeros((nrows, k), np.float32)
    idx = np.zeros((nrows, k), np.int32)
    lib().fmso_topk(_ptr(S), nrows, ncols, k, _ptr(vals), _ptr(idx))
    return vals, idx
