"""Synthetic inputs for the five sampler configurations of BASELINE.json.

Seeded numpy generators (identical on every host) produce the logits; the
uniforms u[r, :] are the per-row Philox streams of d3s_math.h (seed, stream=r),
so the same rows can be rebuilt anywhere without shipping data.

C1 backbone head, one row at a time: fp32 [1, 4097], N(0, 2.5), 5 indices +8,
   T 0.7 / top_p 0.7 / top_k 30, 10 000 seeded rows (row r: stream r, seed 42).
C2 tower codebooks: bf16 [9, 4096], N(0, 2.0) plus a Zipf(s=1.1) bump over a
   random permutation of the indices, 0.7 / 0.7 / 30.
C3 batched backbone head: fp32 [256, 4097], N(0, 2.5) plus 1-8 peaks of +4..+10
   per row; rows [0, N/2) use 0.7 / 0.7 / 30, rows [N/2, N) use 1.0 / 0.9 / 30.
C4 full text vocabulary: bf16 [64, 151936], N(0, 3.0) plus 20 peaks of +6,
   1.0 / 0.9 / 30.
C5 top-p only: fp32 [4096, 4097], N(0, 0.3), top-k "disabled" (k = V: the
   reference clamps top_k to V, src/sampling.c:207), top_p 0.95, T 1.0; index 0
   (eos) banned (-inf) on a seeded 50% of rows.
"""
import numpy as np

CONFIGS = {
    "C1": dict(rows=1, V=4097, dtype="f32", k=30),
    "C2": dict(rows=9, V=4096, dtype="bf16", k=30),
    "C3": dict(rows=256, V=4097, dtype="f32", k=30),
    "C4": dict(rows=64, V=151936, dtype="bf16", k=30),
    "C5": dict(rows=4096, V=4097, dtype="f32", k=4097),
}

ZIPF_SCALE = 8.0  # height of the Zipf bump's first term in C2 (BASELINE.json gives none)


def f32_to_bf16_bits(x):
    """fp32 -> bf16 bits, round to nearest even (finite inputs)."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    return b.astype(np.uint16)


def bf16_bits_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def _logits(name, rows, V, rng):
    if name == "C1":
        x = rng.standard_normal((rows, V), np.float32) * np.float32(2.5)
        for r in range(rows):
            x[r, rng.choice(V, 5, replace=False)] += np.float32(8.0)
    elif name == "C2":
        x = rng.standard_normal((rows, V), np.float32) * np.float32(2.0)
        ranks = np.arange(1, V + 1, dtype=np.float64)
        bump = (ZIPF_SCALE * ranks ** -1.1).astype(np.float32)
        for r in range(rows):
            x[r, rng.permutation(V)] += bump
    elif name == "C3":
        x = rng.standard_normal((rows, V), np.float32) * np.float32(2.5)
        for r in range(rows):
            n = int(rng.integers(1, 9))
            x[r, rng.choice(V, n, replace=False)] += rng.uniform(4.0, 10.0, n).astype(np.float32)
    elif name == "C4":
        x = rng.standard_normal((rows, V), np.float32) * np.float32(3.0)
        for r in range(rows):
            x[r, rng.choice(V, 20, replace=False)] += np.float32(6.0)
    elif name == "C5":
        x = rng.standard_normal((rows, V), np.float32) * np.float32(0.3)
    else:
        raise KeyError(name)
    return x


def make(name, rows=None, seed=42, stream0=0, uniforms=True):
    """Build config `name` with `rows` rows (default: the config's own).
    Returns dict(logits: float32 or uint16-bits [rows, V], dtype, V, k,
    u: float32 [rows, k] or None, temperature, top_p (scalar or float32 [rows]),
    banned: int32 [rows] or None)."""
    cfg = CONFIGS[name]
    rows = cfg["rows"] if rows is None else rows
    V, k = cfg["V"], cfg["k"]
    rng = np.random.default_rng([seed, stream0, list(CONFIGS).index(name)])
    x = _logits(name, rows, V, rng)
    temperature, top_p, banned = 0.7, 0.7, None
    if name == "C3":
        half = rows // 2
        temperature = np.where(np.arange(rows) < half, 0.7, 1.0).astype(np.float32)
        top_p = np.where(np.arange(rows) < half, 0.7, 0.9).astype(np.float32)
    elif name == "C4":
        temperature, top_p = 1.0, 0.9
    elif name == "C5":
        temperature, top_p = 1.0, 0.95
        banned = np.where(rng.random(rows) < 0.5, 0, -1).astype(np.int32)
    logits = f32_to_bf16_bits(x) if cfg["dtype"] == "bf16" else x
    u = None
    if uniforms:
        u = uniform_rows(seed, stream0, rows, k)
    return dict(name=name, logits=logits, dtype=cfg["dtype"], V=V, k=k, u=u,
                temperature=temperature, top_p=top_p, banned=banned)


def uniform_rows(seed, stream0, rows, k):
    """u[r, j] = Philox uniform j of stream (stream0 + r) under seed, computed
    with numpy from the definition in d3s_math.h (d3s_uniform)."""
    j = np.arange(k, dtype=np.uint64)
    q = j >> np.uint64(2)
    out = np.empty((rows, k), np.float32)
    for r in range(rows):
        s = np.uint64(stream0 + r)
        c = [(q & np.uint64(0xFFFFFFFF)).astype(np.uint32), (q >> np.uint64(32)).astype(np.uint32),
             np.full(k, np.uint32(s & np.uint64(0xFFFFFFFF))), np.full(k, np.uint32(s >> np.uint64(32)))]
        words = philox4x32_10(c, np.uint32(seed & 0xFFFFFFFF), np.uint32((seed >> 32) & 0xFFFFFFFF))
        w = np.choose((j & np.uint64(3)).astype(np.int64), words)
        out[r] = (w >> np.uint32(8)).astype(np.float32) * np.float32(2.0 ** -24)
    return out


def philox4x32_10(c, k0, k1):
    """Vectorised Philox4x32-10 (Salmon et al., SC'11) over uint32 arrays."""
    c0, c1, c2, c3 = [np.asarray(v, np.uint32).astype(np.uint64) for v in c]
    k0, k1 = np.uint64(k0), np.uint64(k1)
    M = np.uint64(0xFFFFFFFF)
    for _ in range(10):
        p0 = np.uint64(0xD2511F53) * c0
        p1 = np.uint64(0xCD9E8D57) * c2
        hi0, lo0 = p0 >> np.uint64(32), p0 & M
        hi1, lo1 = p1 >> np.uint64(32), p1 & M
        c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
        k0 = (k0 + np.uint64(0x9E3779B9)) & M
        k1 = (k1 + np.uint64(0xBB67AE85)) & M
    return [v.astype(np.uint32) for v in (c0, c1, c2, c3)]
