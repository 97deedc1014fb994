"""The deterministic arithmetic of d3s_math.h (CPU build), pinned against
double-precision libm, exact integer arithmetic and published known answers."""
import numpy as np
import pytest


def ulps(got, ref):
    ref32 = ref.astype(np.float32)
    return np.abs(got.astype(np.float64) - ref) / np.spacing(np.abs(ref32)).astype(np.float64)


def test_expf_faithful(oracle):
    rng = np.random.default_rng(0)
    x = np.concatenate([np.linspace(-87.3, 88.72, 1_000_001, dtype=np.float32),
                        (-np.abs(rng.standard_normal(500_000)) * 20).astype(np.float32),
                        rng.uniform(-1e-3, 1e-3, 100_000).astype(np.float32)])
    got = oracle.expf(x)
    ref = np.exp(x.astype(np.float64))
    assert ulps(got, ref).max() < 1.0  # faithfully rounded


def test_expf_subnormal_and_special(oracle):
    x = np.linspace(-103.97, -87.4, 200_001, dtype=np.float32)
    got = oracle.expf(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    assert (np.abs(got - ref) / 2.0 ** -149).max() < 1.0  # within one subnormal step
    sp = np.array([0.0, -0.0, np.inf, -np.inf, 89.0, -104.5, -1000.0, 88.72283935546875],
                  np.float32)
    out = oracle.expf(sp)
    assert out[0] == 1.0 and out[1] == 1.0
    assert out[2] == np.inf and out[3] == 0.0 and out[4] == np.inf
    assert out[5] == 0.0 and out[6] == 0.0 and out[7] == np.inf  # e^88.7228394 > FLT_MAX
    assert np.isnan(oracle.expf(np.array([np.nan], np.float32)))[0]


def test_logf_faithful(oracle):
    rng = np.random.default_rng(1)
    y = np.concatenate([np.exp(rng.uniform(np.log(1e-37), np.log(3e38), 1_000_000)),
                        rng.uniform(0.5, 2.0, 500_000)]).astype(np.float32)
    y = y[(y > 0) & (y != 1)]
    assert ulps(oracle.logf(y), np.log(y.astype(np.float64))).max() < 1.0


def test_logf_of_one_minus_u_grid(oracle):
    """The race's noise -log(1 - u) over every u the Philox draw can produce
    (multiples of 2^-24): 1 - u is exact in fp32 there."""
    u = (np.arange(1 << 24, dtype=np.float64) * 2.0 ** -24).astype(np.float32)
    y = np.float32(1) - u
    assert np.array_equal(y.astype(np.float64), 1.0 - u.astype(np.float64))
    got = oracle.logf(y)
    ref = np.log(y.astype(np.float64))
    nz = y != 1
    assert got[~nz][0] == 0.0
    assert ulps(got[nz], ref[nz]).max() < 1.0


def test_logf_special(oracle):
    sp = np.array([1.0, 0.0, -0.0, -1.0, np.inf, 1e-45, 2.0, 0.5], np.float32)
    out = oracle.logf(sp)
    assert out[0] == 0.0 and out[1] == -np.inf and out[2] == -np.inf
    assert np.isnan(out[3]) and out[4] == np.inf
    assert out[5] == np.float32(np.log(2.0 ** -149))  # least subnormal input
    assert out[6] == np.float32(np.log(2.0)) and out[7] == np.float32(np.log(0.5))


def test_fix40_is_floor_of_scaled_value(oracle):
    rng = np.random.default_rng(2)
    e = np.concatenate([rng.random(200_000), np.exp(-rng.uniform(0, 120, 200_000)),
                        [0.0, 1.0, 0.5, 2.0 ** -40, 2.0 ** -41, 1e-45]]).astype(np.float32)
    got = oracle.fix40(e)
    # exact reference: floor(e * 2^40) with e an exact binary fraction
    from fractions import Fraction
    for i in rng.choice(e.size, 2000, replace=False).tolist() + list(range(e.size - 6, e.size)):
        assert int(got[i]) == int(Fraction(float(e[i])) * 2 ** 40), e[i]
    assert int(oracle.fix40(np.array([np.nan, -1.0, 3.0], np.float32))[0]) == 0
    assert int(oracle.fix40(np.array([3.0], np.float32))[0]) == 1 << 40


def test_fused_fix40_exp_equals_two_steps(oracle):
    """fix40(expf(z)) formed from exp's polynomial value (the kernels' row sums)
    against the two-step form, on every 61st float of [-110, 0] and the ends."""
    b = np.arange(0x80000000, 0xC2DC0000, 61, dtype=np.uint64).astype(np.uint32)
    z = np.concatenate([b.view(np.float32), np.array([0.0, -0.0, -np.inf, -104.0, -103.97], np.float32)])
    assert np.array_equal(oracle.fix40_exp(z), oracle.fix40(oracle.expf(z)))


def test_nonpositive_expf_and_unit_fix40_equal_the_general_forms(oracle):
    """The kernels' shortcuts for arguments they know the range of: expf up
    to 88 (every 61st float of [-110, 0], a grid of [0, 88], -inf) and fix40 on [0, 1]
    (every 101st float, the ends), bit for bit against the general forms."""
    b = np.arange(0x80000000, 0xC2DC0000, 61, dtype=np.uint64).astype(np.uint32)
    a = np.concatenate([b.view(np.float32), np.linspace(0, 88, 100_001, dtype=np.float32),
                        np.float32([0.0, -0.0, -np.inf, -104.0, -103.97, -87.3, -88.0, 88.0, 1e-30])])
    assert np.array_equal(oracle.expf_nonpos(a).view(np.uint32), oracle.expf(a).view(np.uint32))
    b = np.arange(0, 0x3F800001, 101, dtype=np.uint64).astype(np.uint32)
    e = np.concatenate([b.view(np.float32), np.float32([0.0, -0.0, 1.0, 0.5, 2.0 ** -40, 2.0 ** -41, 1e-45,
                                                       np.nextafter(np.float32(1), np.float32(0))])])
    assert np.array_equal(oracle.fix40_unit(e), oracle.fix40(e))


def test_fixsum_threshold_is_the_least_sum_above(oracle):
    """The cut's integer test: s = threshold(c) is the least fixed-point sum with
    fixsum_to_f32(s) > c.  Conversions here are exact (s < 2^53 in float64, then
    one rounding to float32)."""
    b = np.arange(0, 0x45800000, 389, dtype=np.uint64).astype(np.uint32)  # [0, 2^12)
    c = np.concatenate([b.view(np.float32), np.float32([0.95, 0.7, 0.9, 1.0, 2.0 ** -16, 2.0 ** -17])])
    s = oracle.fixsum_gt_threshold(c)
    f = lambda v: v.astype(np.float64).astype(np.float32) * np.float32(2.0 ** -40)
    assert np.all(f(s) > c)
    pos = s > 0
    assert np.all(f(s[pos] - np.uint64(1)) <= c[pos])
    top = np.uint64(2 ** 64 - 1)
    sp = oracle.fixsum_gt_threshold(np.float32([-1.0, -0.0, np.nan, np.inf, 2.0 ** 23, -np.inf]))
    assert sp.tolist() == [0, 1, int(top), int(top), int(top), 0]


def test_u64_to_f32_round_to_nearest_even(oracle):
    rng = np.random.default_rng(3)
    vals = [0, 1, 2 ** 24, 2 ** 24 + 1, 2 ** 24 + 3, 2 ** 25 + 2, 2 ** 25 + 6, 2 ** 63 + 2 ** 39,
            2 ** 64 - 1] + [int(v) for v in rng.integers(0, 2 ** 63, 3000, dtype=np.int64)] + \
        [int(v) >> int(s) for v, s in zip(rng.integers(0, 2 ** 63, 3000, dtype=np.int64),
                                           rng.integers(0, 62, 3000))]
    from fractions import Fraction
    for v in vals:
        # the correctly rounded fp32 of v is the nearest of the fp32 values around
        # it (ties to the even significand), decided in exact rational arithmetic
        near = np.float32(float(v))
        cands = [near, np.nextafter(near, np.float32(np.inf)), np.nextafter(near, np.float32(0))]
        best = min(cands, key=lambda c: (abs(Fraction(float(c)) - v),
                                          int(np.float32(c).view(np.uint32)) & 1))
        assert oracle.u64_to_f32(v) == float(best), v


@pytest.mark.parametrize("b", [0.7, 1.0, 0.3, 1e-5, 1e4, 1.9999999, 1.0000001, 0.99999994, 3.9999998,
                               1.4142135, 0.123456, 7.0, 1e-3])
def test_fma_division_is_correctly_rounded(oracle, b):
    """d3s_div_rn (Markstein's correction step) equals the IEEE division for
    every significand in [1, 2) and for random operands over its whole range,
    including the ones it hands to the division (tiny, huge, zero, inf, NaN)."""
    b = np.float32(b)
    a = (np.arange(1 << 23, dtype=np.uint32) | np.uint32(0x3F800000)).view(np.float32)
    got = oracle.div_rn(a, b)
    assert np.array_equal(got.view(np.uint32), (a / b).view(np.uint32))
    rng = np.random.default_rng(int(b.view(np.uint32)))
    bits = rng.integers(0, 2 ** 32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    a = bits.view(np.float32)
    a = np.concatenate([a[np.isfinite(a)], np.float32([0.0, -0.0, 1e-45, -3e-39, np.inf, -np.inf])])
    got = oracle.div_rn(a, b)
    ref = a / b
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert np.isnan(oracle.div_rn(np.float32([np.nan]), b))[0]


@pytest.mark.parametrize("ctr,key,expected", [
    # Random123 kat_vectors, philox4x32 with 10 rounds
    ([0, 0, 0, 0], [0, 0], [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]),
    ([0xffffffff] * 4, [0xffffffff] * 2, [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]),
    ([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0],
     [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]),
])
def test_philox_known_answers(oracle, ctr, key, expected):
    assert oracle.philox(ctr, key).tolist() == expected


def test_uniform_stream_matches_numpy_restatement(oracle):
    import d3s_workloads as W
    a = oracle.uniform(42, 7, 5, 33)
    b = W.uniform_rows(42, 7, 5, 33)
    assert np.array_equal(a, b)
    u = oracle.uniform(1, 0, 200, 1000).ravel()
    assert u.min() >= 0.0 and u.max() < 1.0
    assert np.all((u * 2 ** 24) == np.floor(u * 2 ** 24))  # 24-bit grid
    # uniformity: chi-square over 64 bins, generous bound (p ~ 1e-6)
    h = np.bincount((u * 64).astype(int), minlength=64)
    chi2 = ((h - u.size / 64) ** 2 / (u.size / 64)).sum()
    assert chi2 < 130
