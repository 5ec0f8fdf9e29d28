"""ctypes binding of libflashmaxsim_hip.so (the C ABI in include/flashmaxsim_hip.h).

The library must be built (``make -C flashmaxsim.jl_amd``, or
``__graft_entry__.build()``); there is no fallback of any kind: a missing
library or a non-gfx950 device raises.  ``torch`` is imported first so that
the library binds to the HIP runtime PyTorch already loaded (same SONAME),
which keeps torch's streams and allocations valid inside the library.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

from .errors import ArgumentError, DimensionMismatch, HIPError, UnsupportedError

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# The in-tree build, and only it: every run loads the library built from this tree.
LIB_PATH = os.path.join(_PKG_DIR, "lib", "libflashmaxsim_hip.so")

FMS_OK, FMS_EINVAL, FMS_EUNSUPPORTED, FMS_EHIP, FMS_ESCRATCH = 0, 1, 2, 3, 4
FMS_F32, FMS_F16, FMS_BF16 = 0, 1, 2

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f = ctypes.c_float

# name -> argtypes (restype fms_status = int32 unless listed in _RESTYPES)
SIGNATURES = {
    "fms_status_string": [_i32],
    "fms_arch_supported": [],
    "fms_version": [],
    "fms_launch_pair_scan": [_i32, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _i32, _p],
    "fms_launch_paired_scan": [_i32, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p, _i32, _p],
    "fms_launch_candidates_scan": [_i32, _p, _p, _p, _p, _p, _i32, _p, _p, _i64, _i64, _i64,
                                   _i64, _i64, _i64, _p, _f, _i32, _p],
    "fms_launch_candidates_scan_noalloc": [_i32, _p, _p, _p, _p, _p, _i32, _p, _p, _i64, _i64,
                                           _i64, _i64, _i64, _i64, _p, _f, _i32, _p],
    "fms_inbatch_device_scan": [_i32, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _p],
    "fms_launch_packed_scan": [_i32, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p, _i32, _p],
    "fms_launch_varlen_scan": [_i32, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _i32, _p],
    "fms_int8_quantize": [_i32, _p, _p, _p, _i64, _i64, _p],
    "fms_launch_int8_pair_scan": [_p, _p, _p, _p, _i32, _p, _p, _i32, _p, _p, _i64, _i64, _i64, _p,
                                  _i32, _p],
    "fms_launch_int8_paired_scan": [_p, _p, _p, _p, _i32, _p, _p, _i32, _p, _p, _i64, _i64, _i64,
                                    _i64, _p, _i32, _p],
    "fms_launch_int8_candidates_scan": [_p, _p, _p, _p, _i32, _p, _p, _i32, _p, _i32, _p, _p, _i64,
                                        _i64, _i64, _i64, _i64, _i64, _p, _f, _i32, _p],
    "fms_int8_dots": [_p, _p, _p, _i64, _i64, _i64, _p],
    "fms_length_normalize": [_p, _p, _i64, _i64, _i64, _p, _i32, _i64, _f, _p],
    "fms_varlen_normalize": [_p, _p, _i64, _p],
    "fms_debug_mfma_layout": [_p, _i32, _p],
    "fms_debug_read_bandwidth": [_p, _i64, _p, _i32, _p],
    "fms_debug_gather_bandwidth": [_p, _i64, _i64, _p, _i64, _p, _p],
    "fms_candidates_grouping": [_i32],
    "fms_debug_workspace_allocs": [],
    "fms_debug_inbatch_kernel": [_i32, _i64, _i64, _i64, _i64, _i64, _p, _p],
    "fms_debug_cross_lane": [_p, _p],
    "fms_topk": [_p, _i64, _i64, _i64, _p, _p, _p],
    "fms_launch_packed_multi_scan": [_i32, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                     _i64, _i32, _p],
    "fms_pair_pullback": [_i32, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p],
    "fms_paired_pullback": [_i32, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p],
    "fms_inbatch_pullback": [_i32, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                             _p],
    "fms_candidates_pullback": [_i32, _p, _p, _p, _p, _p, _i32, _p, _p, _p, _p, _i64, _i64, _i64,
                                _i64, _i64, _i64, _p],
    "fms_packed_pullback": [_i32, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p],
    "fms_varlen_pullback": [_i32, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                            _p],
}
_RESTYPES = {
    "fms_status_string": ctypes.c_char_p,
    "fms_arch_supported": ctypes.c_int,
    "fms_version": ctypes.c_char_p,
    "fms_debug_workspace_allocs": ctypes.c_uint64,
}

_lib = None


def lib() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libflashmaxsim_hip.so not found at {LIB_PATH}; build it with "
                "`make -C flashmaxsim.jl_amd` (or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, ctypes.c_int32)
        _lib = L
    return _lib


def check(status: int, what: str) -> None:
    """Map a C-ABI status to the reference's exception types."""
    if status == FMS_OK:
        return
    msg = f"{what}: {lib().fms_status_string(status).decode()}"
    if status == FMS_EINVAL:
        raise DimensionMismatch(msg)
    if status in (FMS_EUNSUPPORTED, FMS_ESCRATCH):
        raise UnsupportedError(msg)
    if status == FMS_EHIP:
        raise HIPError(msg)
    raise ArgumentError(msg)


def arch_supported() -> bool:
    return bool(lib().fms_arch_supported())


def version() -> str:
    return lib().fms_version().decode()
