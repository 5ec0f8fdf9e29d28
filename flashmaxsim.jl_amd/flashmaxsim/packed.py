"""Ragged sequences with 1-based cu_seqlens (src/packed.jl:1-127).

``PackedSeq.tokens`` is ``(ntokens, dim)`` (Julia ``(dim, ntokens)``);
``cu`` is an Int32 vector of length B+1, 1-based: sequence b (0-based here)
owns ``tokens[cu[b]-1 : cu[b+1]-1]``.  Python 0-based cu_seqlens convert
with ``PackedSeq(tokens, cu + 1)`` (packed.jl:5-6).
"""
from __future__ import annotations

from typing import Sequence

import numpy as np
import torch

from .errors import ArgumentError, DimensionMismatch


def _backend(t: torch.Tensor):
    return t.device.type


def _packed_max_len(cu) -> int:
    """packed_max_len (packed.jl:31-45)."""
    n = cu.numel() - 1
    if n <= 0:
        return 0
    return int((cu[1:].to(torch.int64) - cu[:-1].to(torch.int64)).max().item())


def require_host_csr(tokens: torch.Tensor, cu: torch.Tensor) -> None:
    """require_host_csr (packed.jl:47-57)."""
    c = cu.to(torch.int64)
    if c.numel() < 1:
        raise ArgumentError("PackedSeq cu must have length B+1")
    if int(c[0]) != 1:
        raise ArgumentError("PackedSeq cu must start at 1")
    if int(c[-1]) - 1 != tokens.shape[0]:
        raise ArgumentError("PackedSeq cu does not cover tokens")
    if c.numel() > 1 and bool((c[1:] < c[:-1]).any()):
        raise ArgumentError("PackedSeq cu must be nondecreasing")


class PackedSeq:
    """Ragged token matrix plus 1-based CSR (packed.jl:9-21, 59-75).

    A host (CPU) ``cu`` is validated; a device ``cu`` is trusted, as in the
    reference (the device kernels clamp it into range instead of faulting).
    """

    def __init__(self, tokens: torch.Tensor, cu, max_len: int | None = None):
        if not isinstance(cu, torch.Tensor):
            cu = torch.as_tensor(np.asarray(cu), dtype=torch.int32)
        if _backend(tokens) != _backend(cu):
            raise ArgumentError(
                "PackedSeq requires tokens and cu on the same KernelAbstractions backend")
        if cu.numel() < 1:
            raise ArgumentError("PackedSeq cu must have length B+1")
        if max_len is None:
            if cu.device.type == "cpu":
                require_host_csr(tokens, cu)
            max_len = _packed_max_len(cu)
        if max_len < 0:
            raise ArgumentError("PackedSeq max_len must be ≥ 0")
        self.tokens = tokens
        self.cu = cu
        self.max_len = int(max_len)

    @classmethod
    def from_cu_seqlens(cls, tokens: torch.Tensor, cu_seqlens,
                        max_len: int | None = None) -> "PackedSeq":
        """From a 0-based ``cu_seqlens`` (length B+1, starting at 0, the
        flash-attention varlen convention): ``cu = cu_seqlens + 1`` as Int32 on
        the same device (packed.jl:5-6).  A host ``cu_seqlens`` is validated
        like a host ``cu``; a device one is converted on the device without a
        host round trip (pass ``max_len`` to avoid the one read it costs)."""
        if not isinstance(cu_seqlens, torch.Tensor):
            cu_seqlens = torch.as_tensor(np.asarray(cu_seqlens))
        if cu_seqlens.dim() != 1 or cu_seqlens.numel() < 1:
            raise ArgumentError("cu_seqlens must be a vector of length B+1")
        if cu_seqlens.is_floating_point() or cu_seqlens.dtype == torch.bool:
            raise ArgumentError("cu_seqlens must hold integers")
        if cu_seqlens.device.type == "cpu" and cu_seqlens.numel() and int(cu_seqlens[-1]) >= 2**31 - 1:
            raise ArgumentError("cu_seqlens exceeds the Int32 range of cu")
        return cls(tokens, (cu_seqlens.to(torch.int64) + 1).to(torch.int32), max_len)

    def cu_seqlens(self) -> torch.Tensor:
        """The 0-based Int32 ``cu_seqlens`` of this sequence set (``cu - 1``)."""
        return self.cu - 1

    def nseq(self) -> int:
        return self.cu.numel() - 1

    def to(self, device) -> "PackedSeq":
        """Adapt.adapt_structure (packed.jl:77-78)."""
        return PackedSeq(self.tokens.to(device), self.cu.to(device=device, dtype=torch.int32),
                         self.max_len)

    def __repr__(self):
        return (f"PackedSeq{{{self.tokens.dtype}}}(dim={self.tokens.shape[1]}, "
                f"tokens={self.tokens.shape[0]}, nseq={self.nseq()}, max_len={self.max_len})")


def nseq(p: PackedSeq) -> int:
    return p.nseq()


def pack_docs(docs: Sequence[torch.Tensor]) -> PackedSeq:
    """pack_docs (packed.jl:85-116): concatenate (Ld_i, dim) documents."""
    B = len(docs)
    if B == 0:
        raise ArgumentError("pack_docs: empty document list")
    proto = docs[0]
    dim = proto.shape[1]
    lens = []
    for d in docs:
        if d.shape[1] != dim:
            raise DimensionMismatch("pack_docs: feature dim")
        if d.device != proto.device:
            raise ArgumentError("pack_docs: documents must share a KernelAbstractions backend")
        lens.append(int(d.shape[0]))
    cu_h = np.empty(B + 1, dtype=np.int32)
    cu_h[0] = 1
    cu_h[1:] = 1 + np.cumsum(np.asarray(lens, dtype=np.int64)).astype(np.int32)
    tokens = torch.cat([d.reshape(-1, dim) for d in docs], dim=0) if B else proto[:0]
    cu = torch.from_numpy(cu_h).to(proto.device)
    return PackedSeq(tokens, cu, max(lens) if lens else 0)


def pack_pairs(qs: Sequence[torch.Tensor], ds: Sequence[torch.Tensor]):
    """pack_pairs (packed.jl:123-127)."""
    if len(qs) != len(ds):
        raise DimensionMismatch("pack_pairs: pair count")
    return pack_docs(qs), pack_docs(ds)
