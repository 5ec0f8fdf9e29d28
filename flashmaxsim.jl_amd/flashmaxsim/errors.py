"""Exception types mirroring the Julia exceptions the reference throws."""


class DimensionMismatch(ValueError):
    """Julia ``DimensionMismatch`` (shape checks, e.g. forward_layouts.jl:20-47)."""


class ArgumentError(ValueError):
    """Julia ``ArgumentError`` (colocation, idxs placement, CSR validity)."""


class UnsupportedError(ArgumentError):
    """A feature type or size the MI355X library does not implement."""


class HIPError(RuntimeError):
    """A HIP runtime call or kernel launch failed inside the library."""
