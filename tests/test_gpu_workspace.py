"""GPU: calls queued on two streams with no synchronisation between them.

Each call takes its workspace on its own stream (stream-ordered from the
library's pool) and frees it there after its kernels.  Calls of growing and
shrinking sizes, in-batch and candidate layouts, are queued on two streams at
once, three times over, and every result must be bit-identical to the same
call made alone on a synchronised stream.
"""
import numpy as np
import pytest
import torch

from helpers import tokens

import flashmaxsim as fm
from flashmaxsim import _lib

pytestmark = pytest.mark.gpu


def _inbatch_case(rng, Bq, Bd, Td, dim=128):
    Q = torch.from_numpy(tokens(rng, (Bq, 32, dim))).half()
    D = torch.from_numpy(tokens(rng, (Bd, Td, dim))).half()
    dm = np.zeros((Bd, Td), bool)
    for j, n in enumerate(rng.integers(1, Td + 1, Bd)):
        dm[j, :n] = True
    return Q, D, torch.ones(Bq, 32, dtype=torch.bool), torch.from_numpy(dm)


def _candidates_case(rng, B, C, N, Ld=96, dim=128):
    Q = torch.from_numpy(tokens(rng, (B, 32, dim))).half()
    G = torch.from_numpy(tokens(rng, (N, Ld, dim))).half()
    idx = torch.from_numpy(rng.integers(0, N, (B, C)).astype(np.int64))
    return Q, G, idx


def test_queued_calls_on_two_streams_match_lone_calls(device):
    rng = np.random.default_rng(20261202)
    cases = []
    for i in range(14):  # sizes grow and shrink: buffers are replaced and reused
        if i % 3 == 2:
            Q, G, idx = _candidates_case(rng, 16, 64 * (1 + i), 3000)
            cases.append(("candidates", [t.to(device) for t in (Q, G, idx)]))
        else:
            Bd = 32 * (1 + (i * 5) % 9)
            cases.append(("inbatch", [t.to(device) for t in _inbatch_case(rng, 64, Bd, 96)]))

    def call(kind, t):
        if kind == "inbatch":
            return fm.forward.inbatch_forward(*t, tape=True)
        return fm.forward.candidates_forward(*t, tape=True)

    lone = []
    for kind, t in cases:
        S, A = call(kind, t)
        torch.cuda.synchronize(device)
        lone.append((S.cpu(), A.cpu()))

    n0 = _lib.lib().fms_debug_workspace_allocs()
    streams = [torch.cuda.Stream(device=device), torch.cuda.Stream(device=device)]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream(device))
    queued = []
    for rep in range(3):
        for i, (kind, t) in enumerate(cases):
            s = streams[(i + rep) % 2]
            with torch.cuda.stream(s):
                for x in t:
                    x.record_stream(s)
                S, A = call(kind, t)
            queued.append((i, S, A))
    torch.cuda.synchronize(device)
    assert _lib.lib().fms_debug_workspace_allocs() > n0
    for i, S, A in queued:
        print("case", i, cases[i][0], flush=True)
        assert torch.equal(S.cpu(), lone[i][0]), i
        assert torch.equal(A.cpu(), lone[i][1]), i
