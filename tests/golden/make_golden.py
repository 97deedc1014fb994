"""Writes sampler fixtures computed by the float64 closed form
(tests/closed_form.py, the restatement of tests/test_decode.py:100-109 of
SeungheonOh/drama3-mlx plus the race of src/sampling.c:45-47), independent of
the C oracle and of the kernels:
  closed_form_rows.npz     96 rows of V = 257, k <= 40 (the one-wave kernel);
  closed_form_nucleus.npz  rows with k > 64 up to k = V (top-k disabled, the
                           reference's op graph, src/sampling.c:22-49): the
                           nucleus and generic kernels;
  closed_form_wide.npz     rows wider than one wave's registers (V 10000 to
                           151936, k <= 64; bf16 logits, also read widened to
                           fp32): the fused, wide and generic kernels, and rows
                           past the reference kernel's V <= 65536;
  closed_form_sorted.npz   k beyond 16384 on rows of 16500 and 20000 (k up to
                           V; bf16 values): the sorting kernel.

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


def bf16_bits(x):
    """fp32 -> bf16 bits, round to nearest even (finite values; -inf kept)"""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    return b.astype(np.uint16)


def widen(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def nucleus_rows():
    """k > 64 (up to k = V): near-flat rows where the nucleus holds most of the
    row, peaked rows, ties and masked entries."""
    rng = np.random.default_rng(20261202)
    out = []
    for V, k in [(300, 300), (300, 200), (300, 65), (1000, 1000), (1000, 500), (1000, 65), (4097, 4097),
                 (4097, 700), (300, 300), (1000, 1000), (4097, 4097), (4097, 100)]:
        kind = len(out) % 4
        x = (rng.standard_normal(V) * rng.choice([0.3, 1.0])).astype(np.float32)
        if kind == 1:
            x[rng.integers(0, V, 6)] += np.float32(4.0)
        if kind == 2:
            x = (np.round(x * 4) / 4).astype(np.float32)
        if kind == 3:
            x[rng.integers(0, V, V // 5)] = -np.inf
        T = np.float32(rng.choice([0.7, 1.0, 1.3]))
        top_p = np.float32(rng.choice([0.5, 0.9, 0.95, 1.0]))
        u = rng.random(k).astype(np.float32)
        out.append((x, u, T, top_p, k))
    return out


def wide_rows():
    """Rows past one wave's registers, k <= 64: the logits are bf16 values (so
    the same row is exact in either dtype)."""
    rng = np.random.default_rng(20261203)
    out = []
    for V, k in [(10000, 30), (10000, 64), (10000, 1), (20000, 30), (40000, 30), (70000, 30),
                 (151936, 30)]:
        kind = len(out) % 4
        x = (rng.standard_normal(V) * rng.choice([2.5, 3.0])).astype(np.float32)
        if kind == 0:
            x[rng.integers(0, V, 20)] += np.float32(6.0)
        if kind == 1:
            x = np.round(x).astype(np.float32)
        if kind == 2:
            a = int(rng.integers(0, V // 2))
            x[a:a + V // 3] = -np.inf
        T = np.float32(rng.choice([0.7, 1.0]))
        top_p = np.float32(rng.choice([0.7, 0.9, 1.0]))
        u = rng.random(k).astype(np.float32)
        out.append((bf16_bits(x), u, T, top_p, k))
    return out


def sorted_rows():
    """k beyond 16384 on rows past the nucleus kernel's 8192 (top-k disabled
    on a wide row): the sorting kernel.  bf16 values, as wide_rows."""
    rng = np.random.default_rng(20261204)
    out = []
    for V, k, kind in [(16500, 16500, 0), (20000, 16400, 1)]:
        x = (rng.standard_normal(V) * 1.5).astype(np.float32)
        if kind == 0:
            x[rng.integers(0, V, 12)] += np.float32(5.0)
        else:  # ties, and a masked stretch
            x = (np.round(x * 2) / 2).astype(np.float32)
            x[3000:5000] = -np.inf
        T = np.float32(1.0 if kind == 0 else 0.7)
        top_p = np.float32(0.9 if kind == 0 else 0.95)
        u = rng.random(k).astype(np.float32)
        out.append((bf16_bits(x), u, T, top_p, k))
    return out


def write(name, rs, ragged=False):
    """rows (x, u, T, top_p, k) and their closed-form answers; ragged rows
    (different V) are stored flat with offsets"""
    n = len(rs)
    kmax = max(r[4] for r in rs)
    u = np.zeros((n, kmax), np.float32)
    k = np.array([r[4] for r in rs], np.int32)
    T = np.array([r[2] for r in rs], np.float32)
    top_p = np.array([r[3] for r in rs], np.float32)
    ids = np.zeros(n, np.int32)
    cand = np.full((n, kmax), -1, np.int32)
    probs = np.zeros((n, kmax), np.float64)
    min_gap = np.zeros(n)
    race_gap = np.zeros(n)
    lse_scale = np.zeros(n)
    for i, (x, uu, t, p, kk) in enumerate(rs):
        u[i, :kk] = uu
        c = CF.row(widen(x) if x.dtype == np.uint16 else x, uu, t, p, kk)
        ids[i] = c["id"]
        cand[i, :kk] = c["cand"]
        probs[i, :kk] = c["probs"]
        min_gap[i], race_gap[i], lse_scale[i] = c["min_gap"], c["race_gap"], c["lse_scale"]
    if ragged:
        arrays = dict(logits_flat=np.concatenate([r[0] for r in rs]),
                      vocab=np.array([r[0].shape[0] for r in rs], np.int64))
    else:
        arrays = dict(logits=np.stack([r[0] for r in rs]))
    arrays.update(u=u, k=k, temperature=T, top_p=top_p, ids=ids, cand=cand, probs=probs,
                  min_gap=min_gap, race_gap=race_gap, lse_scale=lse_scale)
    np.savez_compressed(os.path.join(HERE, name), **arrays)
    print(f"wrote {n} rows to {name}")


def main():
    write("closed_form_rows.npz", rows())
    write("closed_form_nucleus.npz", nucleus_rows(), ragged=True)
    write("closed_form_wide.npz", wide_rows(), ragged=True)
    write("closed_form_sorted.npz", sorted_rows(), ragged=True)


if __name__ == "__main__":
    main()
