"""Writes tests/golden/closed_form_rows.npz: small sampler fixtures computed
by the float64 closed form (tests/closed_form.py, the restatement of
tests/test_decode.py:100-109 of SeungheonOh/drama3-mlx plus the race of
src/sampling.c:45-47), independent of the C oracle and of the kernels.

The reference itself commits no vectors for this path (its pinning tests
compute expectations at run time on Apple hardware), so these fixtures fix the
expected behaviour of a set of rows once: regressions in the oracle or the
kernels show up as a changed id, candidate list or probability.

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import closed_form as CF  # noqa: E402

V, K_MAX = 257, 40


def rows():
    rng = np.random.default_rng(20241201)
    out = []
    for r in range(96):
        kind = r % 6
        x = (rng.standard_normal(V) * rng.choice([0.3, 1.0, 2.5, 4.0])).astype(np.float32)
        if kind == 1:  # a few peaks
            x[rng.integers(0, V, 4)] += np.float32(6.0)
        if kind == 2:  # integer logits: ties across the k-th place
            x = np.round(x).astype(np.float32)
        if kind == 3:  # masked entries
            x[rng.integers(0, V, 30)] = -np.inf
        if kind == 4:  # a flat row
            x = (rng.standard_normal(V) * 0.05).astype(np.float32)
        T = np.float32(rng.choice([0.5, 0.7, 1.0, 1.3]))
        top_p = np.float32(rng.choice([0.5, 0.7, 0.9, 0.95, 1.0]))
        k = int(rng.choice([1, 5, 30, K_MAX]))
        u = rng.random(k).astype(np.float32)
        out.append((x, u, T, top_p, k))
    return out


def main():
    rs = rows()
    n = len(rs)
    logits = np.stack([r[0] for r in rs])
    u = np.zeros((n, K_MAX), np.float32)
    k = np.array([r[4] for r in rs], np.int32)
    T = np.array([r[2] for r in rs], np.float32)
    top_p = np.array([r[3] for r in rs], np.float32)
    ids = np.zeros(n, np.int32)
    cand = np.full((n, K_MAX), -1, np.int32)
    probs = np.zeros((n, K_MAX), np.float64)
    min_gap = np.zeros(n)
    race_gap = np.zeros(n)
    lse_scale = np.zeros(n)
    for i, (x, uu, t, p, kk) in enumerate(rs):
        u[i, :kk] = uu
        c = CF.row(x, uu, t, p, kk)
        ids[i] = c["id"]
        cand[i, :kk] = c["cand"]
        probs[i, :kk] = c["probs"]
        min_gap[i], race_gap[i], lse_scale[i] = c["min_gap"], c["race_gap"], c["lse_scale"]
    np.savez_compressed(os.path.join(HERE, "closed_form_rows.npz"), logits=logits, u=u, k=k,
                        temperature=T, top_p=top_p, ids=ids, cand=cand, probs=probs,
                        min_gap=min_gap, race_gap=race_gap, lse_scale=lse_scale)
    print(f"wrote {n} rows")


if __name__ == "__main__":
    main()
