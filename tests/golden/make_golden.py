"""Writes tests/golden/pair_fixtures.npz: small pair-scan fixtures.

The reference's tests hold no stored numeric vectors (every input is drawn
from Julia's RNG), so these fixtures are computed here, independently of the
C oracle, by materialising the similarity matrix in numpy fp64 and taking
the first maximum (np.argmax) over valid document tokens -- the definition
MaxSim(q, d) = sum_t max_u <q_t, d_u> with first-valid-wins ties
(src/dense.jl:26-56).  The closed-form cases come from the reference's
tests (test_regressions.jl:65-86, 136-147).

Run:  python tests/golden/make_golden.py
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def dense(q, d, qm, dm):
    S = d.astype(np.float64) @ q.astype(np.float64).T  # (Td, Tq)
    Sm = np.where(dm.astype(bool)[:, None], S, -np.inf)
    tape = np.zeros(q.shape[0], np.int32)
    score = 0.0
    if dm.any():
        am = np.argmax(Sm, axis=0)
        for t in range(q.shape[0]):
            if qm[t]:
                tape[t] = am[t] + 1
                score += Sm[am[t], t]
    return score, tape


def main():
    rng = np.random.default_rng(20261201)
    cases = []
    # closed forms: all-negative dots (-12) and an empty document (0)
    cases.append((np.ones((3, 4), np.float32), -np.ones((5, 4), np.float32),
                  np.ones(3, np.uint8), np.ones(5, np.uint8)))
    cases.append((rng.standard_normal((5, 8)).astype(np.float32),
                  rng.standard_normal((6, 8)).astype(np.float32),
                  np.ones(5, np.uint8), np.zeros(6, np.uint8)))
    # masked random cases at reference test shapes
    for (Tq, Td, dim) in [(6, 8, 16), (12, 130, 16), (33, 65, 40), (8, 17, 768)]:
        q = rng.standard_normal((Tq, dim)).astype(np.float32)
        d = rng.standard_normal((Td, dim)).astype(np.float32)
        qm = (rng.random(Tq) < 0.8).astype(np.uint8)
        dm = (rng.random(Td) < 0.7).astype(np.uint8)
        cases.append((q, d, qm, dm))
    out = {"n_cases": np.int64(len(cases))}
    for i, (q, d, qm, dm) in enumerate(cases):
        s, tape = dense(q, d, qm, dm)
        out.update({f"q{i}": q, f"d{i}": d, f"qm{i}": qm, f"dm{i}": dm,
                    f"score{i}": np.float64(s), f"tape{i}": tape})
    np.savez_compressed(os.path.join(HERE, "pair_fixtures.npz"), **out)
    print(f"wrote {len(cases)} cases")


if __name__ == "__main__":
    main()
