"""flashmaxsim -- host mirror of FlashMaxSim.jl's forward and pullback API over the MI355X library.

Every score is computed by libflashmaxsim_hip.so (hand-written gfx950 HIP
kernels) through its C ABI; this package only validates arguments, allocates
outputs on the device and enqueues the kernels on the current torch stream.
There is no CPU path: host tensors raise ``ArgumentError``.

Array convention: a Julia array of size ``(a, b, c)`` (column-major) is the
torch tensor of shape ``(c, b, a)`` (row-major) -- the same bytes.  So
``Q::(dim, Tq, B)`` is ``Q.shape == (B, Tq, dim)``, masks ``(Tq, B)`` are
``(B, Tq)``, candidate indices ``(C, B)`` are ``(B, C)`` (1-based), and tapes
``(Tq, C, B)`` are ``(B, C, Tq)``.
"""
from .api import AtomicUnified, InBatch, InvGrid, MaxSim, dot_accum, maxsim, score_eltype
from .backward import (candidates_pullback, inbatch_pullback, packed_pullback, pair_pullback,
                       paired_pullback, varlen_pullback)
from .boundary import (inbatch_device_scan, launch_candidates_scan, launch_int8_candidates_scan,
                       launch_int8_pair_scan, launch_int8_paired_scan, launch_packed_scan,
                       launch_pair_scan, launch_paired_scan, launch_varlen_scan,
                       tensor_cores_active)
from .errors import ArgumentError, DimensionMismatch, HIPError, UnsupportedError
from .forward import (candidates_forward, inbatch_forward, int8_candidates_forward,
                      int8_pair_forward, int8_paired_forward, packed_forward,
                      packed_multi_forward, paired_forward, pair_forward, topk, varlen_forward)
from .packed import PackedSeq, nseq, pack_docs, pack_pairs
from .quant import (Int8Index, dequant_int8, load_int8_index, quantize_int8_symmetric,
                    save_int8_index)
from .rrule import MaxSimFunction, rrule

__all__ = [
    "maxsim", "MaxSim", "InBatch", "AtomicUnified", "InvGrid", "score_eltype", "dot_accum",
    "PackedSeq", "nseq", "pack_docs", "pack_pairs",
    "Int8Index", "quantize_int8_symmetric", "dequant_int8", "save_int8_index", "load_int8_index",
    "pair_forward", "paired_forward", "inbatch_forward", "candidates_forward",
    "packed_forward", "packed_multi_forward", "varlen_forward", "int8_pair_forward", "int8_paired_forward",
    "int8_candidates_forward", "topk",
    "pair_pullback", "paired_pullback", "inbatch_pullback", "candidates_pullback",
    "packed_pullback", "varlen_pullback", "rrule", "MaxSimFunction",
    "launch_pair_scan", "launch_paired_scan", "launch_candidates_scan", "inbatch_device_scan",
    "launch_packed_scan", "launch_varlen_scan", "launch_int8_pair_scan",
    "launch_int8_paired_scan", "launch_int8_candidates_scan", "tensor_cores_active",
    "ArgumentError", "DimensionMismatch", "HIPError", "UnsupportedError",
]
