"""GPU: the benchmark's CPU-runnable configuration at its exact shape -- paired-batch MaxSim in Float32,
Q (128, 32, 64) and D (128, 180, 64) in Julia terms (torch (64, 32, 128) and
(64, 180, 128)), randn token columns L2-normalised, all-true masks; outputs the
64 scores and the 32 x 64 Int32 argmax tape.  This is the reference's own
CPU-runnable case; here it runs on the device and is checked against the CPU
oracle: scores within 1e-5 relative (fp32), tapes equal except at near-ties,
with normalize false and true (1/32 per pair).
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import assert_scores, assert_tape, tokens

import flashmaxsim as fm

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("normalize", [False, True])
def test_config0_paired_f32(device, normalize):
    rng = np.random.default_rng(0)
    B, Tq, Td, dim = 64, 32, 180, 128
    Q = tokens(rng, (B, Tq, dim))
    D = tokens(rng, (B, Td, dim))
    qm = torch.ones(B, Tq, dtype=torch.bool, device=device)
    dm = torch.ones(B, Td, dtype=torch.bool, device=device)
    s_o, a_o, _ = oracle.paired_forward(Q, D, None, None)
    want = s_o / Tq if normalize else s_o
    cfg = fm.MaxSim(torch.float32, normalize=normalize)
    got = cfg(torch.from_numpy(Q).to(device), torch.from_numpy(D).to(device), qm, dm)
    assert got.shape == (B,) and got.dtype == torch.float32
    assert_scores(got.cpu(), want.astype(np.float32) if normalize else want, 1e-5,
                  what="config0 scores")
    _, tape = fm.paired_forward(torch.from_numpy(Q).to(device), torch.from_numpy(D).to(device),
                                qm, dm)
    assert tape.shape == (B, Tq) and tape.dtype == torch.int32

    def sims(idx):
        b, t = idx
        return D[b].astype(np.float64) @ Q[b, t].astype(np.float64)
    assert_tape(tape.cpu().numpy(), a_o, sims, 1e-5)
