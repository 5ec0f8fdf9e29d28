"""fms_launch_candidates_scan_noalloc against fms_launch_candidates_scan: the same
scores and tapes, bit for bit, on two calls in a row (the second smaller), with
the document grouping running in the static scratch (an automatically grouped
call and a forced one), and again in output order; both compared with the
oracle as well."""
import numpy as np
import pytest
import torch

import oracle
from helpers import as_feature, tokens

from flashmaxsim import boundary

pytestmark = pytest.mark.gpu


def _problem(rng, B, C, N, Td, Tq, dim, dtype):
    Q = tokens(rng, (B, Tq, dim))
    G = tokens(rng, (N, Td, dim))
    idx = rng.integers(1, N + 1, size=(B, C)).astype(np.int64)
    idx.reshape(-1)[rng.choice(B * C, size=max(1, B * C // 100), replace=False)] = 0
    qm = rng.random((B, Tq)) < 0.95
    gm = rng.random((N, Td)) < 0.9
    Qt, Qo, bf = as_feature(Q, dtype)
    Gt, Go, _ = as_feature(G, dtype)
    return Qt, Qo, Gt, Go, idx, qm, gm, bf


def _scan(device, noalloc, Qt, Gt, idx, qm, gm, N):
    B, Tq = Qt.shape[0], Qt.shape[1]
    C = idx.shape[1]
    args = torch.full((B, C, Tq), -5, dtype=torch.int32, device=device)
    S = torch.full((B, C), 123.0, dtype=torch.float32, device=device)
    boundary.launch_candidates_scan(args, None, Qt.to(device), Gt.to(device),
                                    torch.from_numpy(idx).to(device),
                                    torch.from_numpy(qm).to(device),
                                    torch.from_numpy(gm).to(device), N, S, -3.0,
                                    noalloc=noalloc)
    torch.cuda.synchronize()
    return S.cpu().numpy(), args.cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_noalloc_matches_pool_on_two_calls(device, dtype):
    rng = np.random.default_rng(404)
    # call 1 groups by document automatically (20,000 pairs over 5,000 documents);
    # call 2 is smaller and groups only because grouping is forced
    calls = [(40, 500, 5000, 60, 32, 128, "auto"), (8, 100, 300, 45, 20, 128, "always")]
    for B, C, N, Td, Tq, dim, mode in calls:
        Qt, Qo, Gt, Go, idx, qm, gm, bf = _problem(rng, B, C, N, Td, Tq, dim, dtype)
        prev = boundary.candidates_grouping(mode)
        try:
            S0, a0 = _scan(device, False, Qt, Gt, idx, qm, gm, N)
            S1, a1 = _scan(device, True, Qt, Gt, idx, qm, gm, N)
        finally:
            boundary.candidates_grouping(prev)
        assert np.array_equal(S1.view(np.uint32), S0.view(np.uint32)), (B, C, mode)
        assert np.array_equal(a1, a0), (B, C, mode)
        S_o, a_o, _ = oracle.candidates_forward(Qo, Go, idx, qm.astype(np.uint8),
                                                gm.astype(np.uint8), -3.0, bf16=bf)
        assert np.allclose(S1, S_o, rtol=2e-3, atol=2e-3)
        assert (a1 == a_o).mean() > 0.999


def test_noalloc_output_order_and_scratch_reuse(device):
    """Output order needs no workspace; and a grouped call after a larger one
    reuses the scratch that still holds the larger call's counters and order."""
    rng = np.random.default_rng(405)
    big = _problem(rng, 64, 400, 2000, 40, 16, 128, torch.float16)
    small = _problem(rng, 4, 37, 50, 33, 9, 128, torch.float16)
    prev = boundary.candidates_grouping("always")
    try:
        for Qt, Qo, Gt, Go, idx, qm, gm, bf in (big, small):
            N = Gt.shape[0]
            S0, a0 = _scan(device, False, Qt, Gt, idx, qm, gm, N)
            S1, a1 = _scan(device, True, Qt, Gt, idx, qm, gm, N)
            assert np.array_equal(S1.view(np.uint32), S0.view(np.uint32))
            assert np.array_equal(a1, a0)
        boundary.candidates_grouping("never")
        Qt, Qo, Gt, Go, idx, qm, gm, bf = small
        S0, a0 = _scan(device, False, Qt, Gt, idx, qm, gm, Gt.shape[0])
        S1, a1 = _scan(device, True, Qt, Gt, idx, qm, gm, Gt.shape[0])
        assert np.array_equal(S1.view(np.uint32), S0.view(np.uint32))
        assert np.array_equal(a1, a0)
    finally:
        boundary.candidates_grouping(prev)


def test_noalloc_takes_no_pool_workspace(device):
    """The property the entry point exists for: grouped calls through it request no
    workspace from the library pool (fms_debug_workspace_allocs stays put), while
    the same grouped call through fms_launch_candidates_scan requests one."""
    from flashmaxsim import _lib
    L = _lib.lib()
    rng = np.random.default_rng(406)
    Qt, Qo, Gt, Go, idx, qm, gm, bf = _problem(rng, 16, 300, 800, 40, 32, 128, torch.float16)
    N = Gt.shape[0]
    prev = boundary.candidates_grouping("always")
    try:
        _scan(device, True, Qt, Gt, idx, qm, gm, N)   # first call on the device: set-up
        n0 = L.fms_debug_workspace_allocs()
        S1, a1 = _scan(device, True, Qt, Gt, idx, qm, gm, N)
        S2, a2 = _scan(device, True, Qt, Gt, idx, qm, gm, N)
        assert L.fms_debug_workspace_allocs() == n0
        S0, a0 = _scan(device, False, Qt, Gt, idx, qm, gm, N)
        assert L.fms_debug_workspace_allocs() == n0 + 1
    finally:
        boundary.candidates_grouping(prev)
    for S, a in ((S1, a1), (S2, a2)):
        assert np.array_equal(S.view(np.uint32), S0.view(np.uint32))
        assert np.array_equal(a, a0)


def test_noalloc_auto_falls_back_to_output_order_beyond_its_scratch(device):
    """Under automatic grouping a call whose grouping workspace exceeds the scratch
    (2,000,000 pairs over 100,000 documents: about 40 MB of order entries against
    32 MiB) scans in output order instead of failing: the same scores and tapes as
    the pooled call (which groups), and a sample checked against the oracle.
    Forced grouping still refuses it."""
    from flashmaxsim import errors
    rng = np.random.default_rng(407)
    B, C, N, Td, Tq, dim = 2000, 1000, 100_000, 8, 8, 64
    gen = torch.Generator(device=device)
    gen.manual_seed(407)
    Q = torch.randn(B, Tq, dim, generator=gen, device=device).to(torch.float16)
    G = torch.randn(N, Td, dim, generator=gen, device=device).to(torch.float16)
    idx = torch.randint(1, N + 1, (B, C), generator=gen, device=device, dtype=torch.int64)
    idx.view(-1)[::97] = 0
    qm = torch.ones(B, Tq, dtype=torch.bool, device=device)
    gm = torch.ones(N, Td, dtype=torch.bool, device=device)

    def run(noalloc):
        args = torch.full((B, C, Tq), -5, dtype=torch.int32, device=device)
        S = torch.full((B, C), 123.0, dtype=torch.float32, device=device)
        boundary.launch_candidates_scan(args, None, Q, G, idx, qm, gm, N, S, -3.0,
                                        noalloc=noalloc)
        torch.cuda.synchronize()
        return S, args

    prev = boundary.candidates_grouping("auto")
    try:
        S0, a0 = run(False)
        S1, a1 = run(True)
        assert torch.equal(S1.view(torch.int32), S0.view(torch.int32))
        assert torch.equal(a1, a0)
        boundary.candidates_grouping("always")
        with pytest.raises(errors.UnsupportedError):
            run(True)
    finally:
        boundary.candidates_grouping(prev)
    # 64 sampled queries x all their candidates against the oracle
    rows = rng.choice(B, size=64, replace=False)
    rows_t = torch.from_numpy(rows).to(device)
    sub_idx = idx[rows_t].cpu().numpy()
    used = np.unique(sub_idx[sub_idx > 0])
    remap = np.zeros(N + 1, np.int64)
    remap[used] = np.arange(1, len(used) + 1)
    Go = G[torch.from_numpy(used - 1).to(device)].cpu().numpy()
    S_o, a_o, _ = oracle.candidates_forward(Q[rows_t].cpu().numpy(), Go, remap[sub_idx],
                                            np.ones((64, Tq), np.uint8),
                                            np.ones((len(used), Td), np.uint8), -3.0)
    S_g = S1[rows_t].cpu().numpy()
    a_g = a1[rows_t].cpu().numpy()
    assert np.allclose(S_g, S_o, rtol=2e-3, atol=2e-3)
    assert (a_g == a_o).mean() > 0.999
