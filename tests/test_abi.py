"""CPU checks of the C ABI: the library loads, exports every function the
public header declares, and its host-side validation returns the documented
status codes without touching a GPU (every call here returns before any HIP
call is made)."""
import os
import re

import pytest

from flashmaxsim import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flashmaxsim_hip.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fms_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = header_functions()
    for required in ["fms_launch_pair_scan", "fms_launch_paired_scan",
                     "fms_launch_candidates_scan", "fms_inbatch_device_scan",
                     "fms_launch_packed_scan", "fms_launch_varlen_scan",
                     "fms_launch_int8_pair_scan", "fms_launch_int8_paired_scan",
                     "fms_int8_quantize", "fms_arch_supported"]:
        assert required in names


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    for name in header_functions():
        assert hasattr(L, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_status_strings_and_version():
    L = _lib.lib()
    assert L.fms_status_string(0) == b"ok"
    assert b"invalid" in L.fms_status_string(1)
    assert b"unsupported" in L.fms_status_string(2)
    assert b"HIP" in L.fms_status_string(3)
    assert _lib.version().startswith("flashmaxsim-hip")


EINVAL, EUNSUP, OK = _lib.FMS_EINVAL, _lib.FMS_EUNSUPPORTED, _lib.FMS_OK


@pytest.mark.parametrize("call,expect", [
    # unsupported feature type
    (lambda L: L.fms_launch_paired_scan(9, None, None, None, None, None, None, 8, 4, 5, 2, None, 0, None), EUNSUP),
    # negative extents
    (lambda L: L.fms_launch_paired_scan(1, None, None, None, None, None, None, -1, 4, 5, 2, None, 0, None), EINVAL),
    # zero batch: nothing to do (ka.jl:12)
    (lambda L: L.fms_launch_paired_scan(1, None, None, None, None, None, None, 8, 4, 5, 0, None, 0, None), OK),
    # work but NULL features
    (lambda L: L.fms_launch_paired_scan(1, None, None, None, None, None, None, 8, 4, 5, 2, None, 0, None), EINVAL),
    # normalize must be 0 or 1
    (lambda L: L.fms_launch_paired_scan(1, None, None, None, None, None, None, 8, 4, 5, 2, None, 2, None), EINVAL),
    (lambda L: L.fms_inbatch_device_scan(1, None, None, None, None, None, None, 8, 4, 2, 5, 3, -1, None), EINVAL),
    # bad index width
    (lambda L: L.fms_launch_candidates_scan(1, None, None, 1, 1, 1, 3, None, None, 8, 4, 2, 5, 7, 3, None, 0.0, 0, None), EINVAL),
    # zero candidates
    (lambda L: L.fms_launch_candidates_scan(1, None, None, None, None, None, 8, None, None, 8, 4, 2, 5, 7, 0, None, 0.0, 0, None), OK),
    # NULL idx with work
    (lambda L: L.fms_launch_candidates_scan(1, None, None, 1, 1, None, 8, None, None, 8, 4, 2, 5, 7, 3, None, 0.0, 0, None), EINVAL),
    # a single sequence too large for one buffer resource
    (lambda L: L.fms_launch_paired_scan(0, None, None, 1, 1, None, None, 1 << 20, 1 << 10, 5, 2, None, 0, None), EUNSUP),
    (lambda L: L.fms_inbatch_device_scan(1, None, None, 1, 1, None, None, 8, 4, 2, 5, 3, 0, None), EINVAL),
    (lambda L: L.fms_launch_packed_scan(1, None, None, 1, 1, None, None, 8, 4, 3, 10, None, 0, None), EINVAL),
    (lambda L: L.fms_launch_varlen_scan(2, None, None, 1, 1, None, 1, 8, 4, 3, 10, 10, None, 0, None), EINVAL),
    (lambda L: L.fms_int8_quantize(0, None, None, None, 8, 4, None), EINVAL),
    (lambda L: L.fms_int8_quantize(1, None, None, None, 8, 4, None), EINVAL),
    (lambda L: L.fms_int8_quantize(0, None, None, None, 8, 0, None), OK),
    # INT8 quantisation and scales take Float32 or Float16 only
    (lambda L: L.fms_int8_quantize(2, 1, 1, 1, 8, 4, None), EUNSUP),
    (lambda L: L.fms_launch_int8_paired_scan(None, None, 1, None, 0, 1, 1, 0, None, None, 8, 4, 5, 2, None, 0, None), EINVAL),
    (lambda L: L.fms_launch_int8_paired_scan(None, None, 1, 1, 2, 1, 1, 0, None, None, 8, 4, 5, 2, None, 0, None), EUNSUP),
    (lambda L: L.fms_launch_int8_paired_scan(None, None, 1, 1, 0, 1, 1, 9, None, None, 8, 4, 5, 2, None, 0, None), EUNSUP),
    (lambda L: L.fms_launch_int8_pair_scan(None, None, 1, 1, 1, 1, 1, 2, None, None, 8, 4, 5, None, 0, None), EUNSUP),
    (lambda L: L.fms_launch_int8_candidates_scan(None, None, 1, 1, 0, 1, 1, 0, 1, 2, None, None, 8, 4, 2, 5, 7, 3, None, 0.0, 0, None), EINVAL),
    (lambda L: L.fms_launch_int8_candidates_scan(None, None, 1, 1, 0, 1, 1, 2, 1, 8, None, None, 8, 4, 2, 5, 7, 3, None, 0.0, 0, None), EUNSUP),
    # a scan whose grid would exceed 2^32 work-items (returns before any HIP call)
    (lambda L: L.fms_launch_paired_scan(1, None, None, 1, 1, None, None, 8, 1, 1, 1 << 31, None, 0, None), EUNSUP),
    (lambda L: L.fms_launch_candidates_scan(1, None, None, 1, 1, 1, 8, None, None, 8, 1, 1 << 16, 1, 7, 1 << 16, None, 0.0, 0, None), EUNSUP),
    (lambda L: L.fms_launch_varlen_scan(1, None, None, 1, 1, 1, 1, 8, 1, 1 << 31, 10, 10, None, 0, None), EUNSUP),
    (lambda L: L.fms_launch_int8_paired_scan(None, None, 1, 1, 0, 1, 1, 0, None, None, 8, 1, 1, 1 << 31, None, 0, None), EUNSUP),
    (lambda L: L.fms_int8_dots(None, 1, 1, 8, 4, 5, None), EINVAL),
    (lambda L: L.fms_length_normalize(None, None, 4, 3, 2, None, 0, 0, 0.0, None), EINVAL),
    (lambda L: L.fms_length_normalize(None, None, 4, 0, 2, None, 0, 0, 0.0, None), OK),
    (lambda L: L.fms_varlen_normalize(None, None, 3, None), EINVAL),
    (lambda L: L.fms_debug_mfma_layout(None, 1, None), EINVAL),
    # pullbacks: bad dtype, NULL buffers, empty batches, bad index width, negative sizes
    (lambda L: L.fms_paired_pullback(9, None, None, None, None, None, None, None, None, 8, 4, 5, 2, None), EUNSUP),
    (lambda L: L.fms_paired_pullback(1, None, None, None, None, None, None, None, None, 8, 4, 5, 2, None), EINVAL),
    (lambda L: L.fms_paired_pullback(1, None, None, None, None, None, None, None, None, 8, 4, 5, 0, None), OK),
    (lambda L: L.fms_pair_pullback(1, None, None, 1, 1, None, None, None, 8, 4, 5, None), EINVAL),
    (lambda L: L.fms_inbatch_pullback(2, None, None, None, None, None, None, None, None, 8, 4, 5, 0, 0, None), OK),
    (lambda L: L.fms_inbatch_pullback(2, 1, 1, 1, 1, None, None, None, None, 8, 4, 5, 3, 2, None), EINVAL),
    (lambda L: L.fms_candidates_pullback(1, 1, 1, 1, 1, 1, 3, None, 1, 1, None, 8, 4, 2, 5, 7, 3, None), EINVAL),
    (lambda L: L.fms_candidates_pullback(1, 1, 1, 1, 1, None, 8, None, 1, 1, None, 8, 4, 2, 5, 7, 3, None), EINVAL),
    (lambda L: L.fms_packed_pullback(0, None, None, None, None, None, None, None, None, None, -1, 4, 3, 10, None), EINVAL),
    (lambda L: L.fms_varlen_pullback(0, 1, 1, 1, 1, None, None, 1, 1, None, 8, 4, 3, 10, 10, None), EINVAL),
    (lambda L: L.fms_varlen_pullback(0, None, None, None, None, None, None, None, None, None, 8, 4, 3, 0, 0, None), OK),
    # top-k: k beyond the row, k beyond the LDS sort, empty, NULL buffers
    (lambda L: L.fms_topk(None, 2, 5, 6, None, None, None), EINVAL),
    (lambda L: L.fms_topk(None, 2, 5000, 1025, None, None, None), EUNSUP),
    (lambda L: L.fms_topk(None, 1 << 22, 5, 3, None, None, None), EUNSUP),
    (lambda L: L.fms_topk(None, 0, 5, 3, None, None, None), OK),
    (lambda L: L.fms_topk(None, 2, 5, 0, None, None, None), OK),
    (lambda L: L.fms_topk(None, 2, 5, 3, None, None, None), EINVAL),
    (lambda L: L.fms_topk(None, -1, 5, 3, None, None, None), EINVAL),
])
def test_validation_status_codes(call, expect):
    assert call(_lib.lib()) == expect


def test_status_maps_to_reference_exceptions():
    import flashmaxsim as fm
    with pytest.raises(fm.DimensionMismatch):
        _lib.check(EINVAL, "x")
    with pytest.raises(fm.UnsupportedError):
        _lib.check(EUNSUP, "x")
    with pytest.raises(fm.HIPError):
        _lib.check(_lib.FMS_EHIP, "x")
    _lib.check(OK, "x")


def test_candidates_grouping_mode_switch():
    """fms_candidates_grouping is host-only state: returns the previous mode, rejects others."""
    L = _lib.lib()
    prev = L.fms_candidates_grouping(1)
    try:
        assert L.fms_candidates_grouping(2) == 1
        assert L.fms_candidates_grouping(0) == 2
        assert L.fms_candidates_grouping(3) == 0
        assert L.fms_candidates_grouping(4) == -1
        assert L.fms_candidates_grouping(-1) == -1
        assert L.fms_candidates_grouping(0) == 3
    finally:
        L.fms_candidates_grouping(prev)


def test_noalloc_rejects_workspace_beyond_its_scratch():
    """fms_launch_candidates_scan_noalloc refuses (FMS_ESCRATCH, before any HIP call) a
    grouped call whose workspace exceeds FMS_NOALLOC_SCRATCH_BYTES: 5M pairs need 40 MB
    of order entries."""
    L = _lib.lib()
    prev = L.fms_candidates_grouping(1)
    try:
        st = L.fms_launch_candidates_scan_noalloc(1, None, None, 1, 1, 1, 8, None, None, 8, 1, 5,
                                                  1, 1, 1_000_000, None, 0.0, 0, None)
        assert st == _lib.FMS_ESCRATCH
        assert b"scratch" in L.fms_status_string(st)
        # the same validation as fms_launch_candidates_scan otherwise
        assert L.fms_launch_candidates_scan_noalloc(9, None, None, 1, 1, 1, 8, None, None, 8, 1,
                                                    5, 1, 1, 3, None, 0.0, 0, None) == EUNSUP
        assert L.fms_launch_candidates_scan_noalloc(1, None, None, 1, 1, None, 8, None, None, 8,
                                                    1, 5, 1, 1, 3, None, 0.0, 0, None) == EINVAL
    finally:
        L.fms_candidates_grouping(prev)
    import flashmaxsim as fm
    with pytest.raises(fm.UnsupportedError):
        _lib.check(_lib.FMS_ESCRATCH, "x")
