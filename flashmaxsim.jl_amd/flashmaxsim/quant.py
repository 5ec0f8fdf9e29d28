"""Per-token symmetric INT8 index (src/quant.jl:1-60).

``Int8Index.codes`` has the feature shape ((T, dim) or (B, T, dim)) as Int8;
``scales`` is (T,) or (B, T) Float32.  Quantisation runs on the device
(``fms_int8_quantize``) and is bit-exact with quantize_int8_symmetric.
"""
from __future__ import annotations

import torch

from . import boundary
from .errors import DimensionMismatch, UnsupportedError


class Int8Index:
    """INT8 token embeddings plus per-token absmax scales (quant.jl:11-14)."""

    def __init__(self, codes: torch.Tensor, scales: torch.Tensor):
        self.codes = codes
        self.scales = scales

    def to(self, device) -> "Int8Index":
        return Int8Index(self.codes.to(device), self.scales.to(device))

    def __repr__(self):
        return (f"Int8Index(codes={tuple(self.codes.shape)}, scales={tuple(self.scales.shape)}, "
                f"eltype={self.scales.dtype})")


def quantize_int8_symmetric(x: torch.Tensor) -> Int8Index:
    """quantize_int8_symmetric (quant.jl:42-49) for Float32 device features."""
    if x.dtype != torch.float32:
        raise UnsupportedError("quantize_int8_symmetric on device takes Float32 features")
    x = x.contiguous()
    codes = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    scales = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    boundary.int8_quantize(x, codes, scales)
    return Int8Index(codes, scales)


def dequant_int8(idx: Int8Index) -> torch.Tensor:
    """dequant_int8 (quant.jl:55-57): T.(codes) .* scales (fp32, elementwise)."""
    return idx.codes.to(idx.scales.dtype) * idx.scales.unsqueeze(-1)


def require_int8_index(d: Int8Index) -> None:
    """require_int8_index (quant.jl:62-71)."""
    if d.codes.dim() == 2:
        if d.codes.shape[0] != d.scales.numel():
            raise DimensionMismatch("Int8Index token count")
    else:
        if d.codes.shape[1] != d.scales.shape[-1]:
            raise DimensionMismatch("Int8Index token count")
        if d.codes.shape[0] != d.scales.shape[0]:
            raise DimensionMismatch("Int8Index batch")
