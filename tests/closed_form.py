"""Float64 closed form of the sampler, independent of the oracle's C code.

Restates the reference's own check, tests/test_decode.py:100-109 of
SeungheonOh/drama3-mlx (stable sort of logits/T, full-row softmax, keep =
not(cumsum > top_p or rank >= k) with rank 0 always kept, renormalise), and adds
the exponential race of src/sampling.c:45-47 (argmax of p / -log(1 - u), first
maximum) so that it predicts the sampled id too.  Everything after the fp32
division x = logit / T (src/sampling.c:25) is float64.
"""
import numpy as np


def clamp_temperature(t):
    t = np.float32(t)
    return np.float32(1e-5) if t < np.float32(1e-5) else t  # src/sampling.c:16,195


def row(logits, u, temperature, top_p, k):
    """logits: float32 [V]; u: float32 [k].  Returns dict with the ranked ids
    (top k), the float64 post-filter probabilities by rank, the float64 id of
    the race, min |c_r - top_p| over r in [1, k) and the relative gap between
    the two best race scores."""
    x = np.asarray(logits, np.float32) / clamp_temperature(temperature)
    V = x.size
    order = np.argsort(-x, kind="stable")
    values = x[order].astype(np.float64)
    p = np.exp(values - values.max())
    p /= p.sum()
    c = np.cumsum(p)
    keep = ~((c > top_p) | (np.arange(V) >= k))
    keep[0] = True
    probs = np.where(keep, p, 0.0)
    probs /= probs.sum()
    u64 = np.asarray(u, np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        noise = -np.log1p(-u64)
        score = probs[:k] / noise
    valid = np.where(np.isfinite(score) & (noise > 0), score, -1.0)
    choice = int(np.argmax(valid)) if valid.max() > -1.0 else 0
    srt = np.sort(valid)[::-1]
    race_gap = (srt[0] - srt[1]) / srt[0] if k > 1 and srt[0] > 0 and srt[1] >= 0 else np.inf
    min_gap = np.min(np.abs(c[1:k] - top_p)) if k > 1 else np.inf
    log_s = float(np.log(np.exp(values - values.max()).sum()))
    return dict(cand=order[:k].astype(np.int32), probs=probs[:k], id=int(order[choice]),
                lse=float(values.max()) + log_s, lse_scale=max(abs(float(values.max())), log_s),
                min_gap=float(min_gap), race_gap=float(race_gap), kept=int(keep[:k].sum()))


def lse_tolerance(lse_scale):
    """fp32 lse = m + log(S): the rounding of m + log(S) and of log(S), measured
    in ulps of the larger of |m| and log(S) (they can cancel)."""
    return 3.0 * float(np.spacing(np.float32(lse_scale)))


def fp32_tolerance(lse_scale, k):
    """How far an fp32 evaluation of c_r may sit from the float64 one: the fp32
    rounding of lse (c_r moves by c_r * |d lse| <= lse_tolerance), the exp rounding
    (one ulp of each term, at most 2^-24 in total) and the additions (k <= 64:
    sequential fp32, at most 2^-24 each; k > 64: one rounding of an exact sum).
    Rows with min_gap below this are boundary rows for a float64-vs-fp32 check."""
    adds = k if k <= 64 else 1
    return 1e-6 + lse_tolerance(lse_scale) + (adds + 4) * 2.0 ** -24
