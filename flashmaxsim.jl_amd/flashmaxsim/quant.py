"""Per-token symmetric INT8 index (src/quant.jl:1-60).

``Int8Index.codes`` has the feature shape ((T, dim) or (B, T, dim)) as Int8;
``scales`` is (T,) or (B, T) in the features' eltype, Float32 or Float16
(quant.jl:42-49 computes them in T).  Quantisation runs on the device
(``fms_int8_quantize``) and is bit-exact with quantize_int8_symmetric.

At rest (``save_int8_index`` / ``load_int8_index``) an index is one
safetensors file with two tensors, ``codes`` and ``scales``, in exactly the
in-memory layout above -- Julia's column-major ``codes (dim, Td, N)`` and
``scales (Td, N)`` byte for byte (quant.jl:11-14) -- plus the format name in
the metadata.  Byte layout: a little-endian uint64 header length n, n bytes of
JSON naming each tensor's dtype ("I8", "F32" / "F16"), shape (row-major, i.e.
Julia's reversed) and data_offsets [begin, end) after the header, then the
tensor bytes.  The Julia extension reads the same file with
``FlashMaxSimHIPExt.load_int8_index`` (plain ``read!``, no JSON package).
Loading reads the bytes without executing anything from the file and moves
them to the requested device.
"""
from __future__ import annotations

import torch

from . import boundary
from .errors import ArgumentError, DimensionMismatch, UnsupportedError

INT8_INDEX_FORMAT = "flashmaxsim-int8-index-v1"


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
    """quantize_int8_symmetric (quant.jl:42-49) for Float32 or Float16 device
    features, computed in the features' type; the scales keep that type."""
    if x.dtype not in (torch.float32, torch.float16):
        raise UnsupportedError("quantize_int8_symmetric on device takes Float32 or Float16 features")
    x = x.contiguous()
    codes = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    scales = torch.empty(x.shape[:-1], dtype=x.dtype, device=x.device)
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


def save_int8_index(idx: Int8Index, path: str) -> None:
    """Write an Int8Index to ``path`` as safetensors (codes int8, scales fp32 / fp16)."""
    from safetensors.torch import save_file
    require_int8_index(idx)
    if idx.codes.dtype != torch.int8 or idx.scales.dtype not in (torch.float32, torch.float16):
        raise ArgumentError("Int8Index at rest holds Int8 codes and Float32 or Float16 scales")
    save_file({"codes": idx.codes.detach().contiguous().cpu(),
               "scales": idx.scales.detach().contiguous().cpu()}, path,
              metadata={"format": INT8_INDEX_FORMAT,
                        "layout": "codes (N, Td, dim) row-major = Julia (dim, Td, N); "
                                  "scales (N, Td) = Julia (Td, N)"})


def load_int8_index(path: str, device="cpu") -> Int8Index:
    """Read an Int8Index written by ``save_int8_index`` onto ``device``."""
    from safetensors import safe_open
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        if meta.get("format") != INT8_INDEX_FORMAT:
            raise ArgumentError(f"{path}: not a {INT8_INDEX_FORMAT} file")
        codes, scales = f.get_tensor("codes"), f.get_tensor("scales")
    if codes.dtype != torch.int8 or scales.dtype not in (torch.float32, torch.float16):
        raise ArgumentError(f"{path}: codes must be Int8 and scales Float32 or Float16")
    idx = Int8Index(codes, scales)
    require_int8_index(idx)
    return idx.to(device)
