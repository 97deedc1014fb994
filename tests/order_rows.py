"""Rows whose top-p cut depends on the order of the cumulative sum.

The reference computes the cumulative c_r = sum_{j<=r} exp(x_j - lse) in two
ways (src/sampling.c:197): its kernel adds the fp32 terms left to right
(:126-127); its op graph takes MLX's cumsum (:39), which the oracle models as
the exact fixed-point prefix sum rounded once.  The two differ in the last bits
on most rows.  Placing top_p at the smaller of the two values at a rank where
they differ makes the two orders cut at different ranks, so a sampler that
takes the wrong order for a call gets other probabilities (and often another
id).  Test helper; it uses the oracle's elementwise exp and fixed-point image,
the same arithmetic the oracle's own sum uses."""
import numpy as np


def u64_to_f32(v):
    """round to nearest even of a non-negative integer, in fp32"""
    v = int(v)
    if v < (1 << 24):
        return np.float32(v)
    sh = v.bit_length() - 24
    q, rem = v >> sh, v & ((1 << sh) - 1)
    half = 1 << (sh - 1)
    if rem > half or (rem == half and q & 1):
        q += 1
    return np.float32(q * 2.0 ** sh)


def cumulatives(oracle, xr, lse, k):
    """The first k cumulative values of row x (fp32, already divided by T) in
    both orders: (kernel order: fp32 left to right, op graph order: exact
    prefix rounded once)."""
    V = xr.shape[0]
    order = np.lexsort((np.arange(V), -xr))[:k]
    e = oracle.expf((xr[order] - np.float32(lse)).astype(np.float32))
    seq, c = [], np.float32(0)
    for t in e:
        c = np.float32(c + t)
        seq.append(c)
    fx = oracle.fix40(e)
    ex, P = [], 0
    for t in fx:
        P += int(t)
        ex.append(np.float32(u64_to_f32(P) * np.float32(2.0 ** -40)))
    return np.array(seq, np.float32), np.array(ex, np.float32)


def split_top_p(oracle, logits_f32, T, k, banned=None):
    """Per row, a top_p at which the two orders cut at different ranks (NaN
    where no rank in [1, k) tells them apart).  logits_f32: [N, V] fp32 (bf16
    rows widened)."""
    N = logits_f32.shape[0]
    out = np.full(N, np.nan, np.float32)
    for r in range(N):
        xr = logits_f32[r].copy()
        if banned is not None and banned[r] >= 0:
            xr[banned[r]] = -np.inf
        t = np.float32(T[r] if np.ndim(T) else T)
        x = (xr / t).astype(np.float32)
        u = np.full((1, k), 0.5, np.float32)
        lse = oracle.sample(logits_f32[r:r + 1], u, t, 2.0,
                            banned=None if banned is None else banned[r:r + 1])["lse"][0]
        seq, ex = cumulatives(oracle, x, lse, k)
        for j in range(1, k):
            if seq[j] != ex[j] and seq[j - 1] < min(seq[j], ex[j]) and ex[j - 1] < min(seq[j], ex[j]):
                out[r] = min(seq[j], ex[j])
                break
    return out
