"""The committed closed-form fixtures (tests/golden/*.npz, made by
tests/golden/make_golden.py from the float64 restatement of
tests/test_decode.py:100-109) against the C oracle and, on a GPU, against the
HIP library: ranked candidates equal, ids equal except boundary rows (counted),
post-filter probabilities within 1e-5 relative where the kept set agrees.

closed_form_rows.npz reaches the one-wave kernel (V = 257, k <= 40);
closed_form_nucleus.npz the nucleus and generic kernels (k > 64 up to k = V);
closed_form_wide.npz the fused, wide and generic kernels (V 10000 to 151936,
bf16 values read as bf16 and widened to fp32); closed_form_sorted.npz the
sorting kernels (k beyond 16384 on rows of 16500 and 20000)."""
import os

import numpy as np
import pytest

import closed_form as CF

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = ["closed_form_rows.npz", "closed_form_nucleus.npz", "closed_form_wide.npz", "closed_form_sorted.npz"]
RTOL = 1e-5


def load(name):
    z = np.load(os.path.join(GOLDEN, name))  # plain arrays: no pickle
    return {n: z[n] for n in z.files}


def row_logits(g, i, widen):
    """row i as [1, V]: fp32, or bf16 bits (widened to fp32 when asked)"""
    if "logits" in g:
        x = g["logits"][i:i + 1]
    else:
        off = int(np.sum(g["vocab"][:i]))
        x = g["logits_flat"][off:off + int(g["vocab"][i])][None, :]
    if x.dtype == np.uint16 and widen:
        x = (x.astype(np.uint32) << 16).view(np.float32)
    return np.ascontiguousarray(x)


def check(sample_row, label, name, widen=False):
    g = load(name)
    boundary = mismatched = 0
    for i in range(len(g["ids"])):
        k = int(g["k"][i])
        got = sample_row(row_logits(g, i, widen), g["u"][i:i + 1, :k], g["temperature"][i], g["top_p"][i])
        edge = (g["min_gap"][i] < CF.fp32_tolerance(g["lse_scale"][i], k) or g["race_gap"][i] < 1e-6)
        boundary += int(edge)
        assert np.array_equal(got["cand"][0], g["cand"][i, :k]), (label, name, i)
        if got["ids"][0] != g["ids"][i]:
            mismatched += 1
            assert edge, (label, name, i, got["ids"][0], g["ids"][i])
        kept_same = np.array_equal(got["probs"][0] > 0, g["probs"][i, :k] > 0)
        if kept_same:
            np.testing.assert_allclose(got["probs"][0], g["probs"][i, :k], rtol=RTOL, atol=1e-30,
                                       err_msg=f"{label} {name} row {i}")
        else:
            assert edge, (label, name, i)
    print(f"[golden] {label} {name}: {len(g['ids'])} rows, boundary {boundary}, id mismatches {mismatched}")


@pytest.mark.parametrize("name", FIXTURES)
def test_fixture_is_the_closed_form(name):
    """the fixture file still says what the closed form computes"""
    g = load(name)
    step = 7 if len(g["ids"]) > 20 else 1
    for i in range(0, len(g["ids"]), step):
        k = int(g["k"][i])
        c = CF.row(row_logits(g, i, True)[0], g["u"][i, :k], g["temperature"][i], g["top_p"][i], k)
        assert c["id"] == g["ids"][i] and np.array_equal(c["cand"], g["cand"][i, :k])
        assert np.array_equal(c["probs"], g["probs"][i, :k])


@pytest.mark.parametrize("name,widen", [(FIXTURES[0], False), (FIXTURES[1], False), (FIXTURES[2], False),
                                        (FIXTURES[2], True), (FIXTURES[3], False)])
def test_oracle_matches_golden_rows(oracle, name, widen):
    check(lambda x, u, T, p: oracle.sample(x, u, T, p), "oracle", name, widen)


@pytest.mark.gpu
@pytest.mark.parametrize("flags", [0, 1])
@pytest.mark.parametrize("name,widen", [(FIXTURES[0], False), (FIXTURES[1], False), (FIXTURES[2], False),
                                        (FIXTURES[2], True), (FIXTURES[3], False), (FIXTURES[3], True)])
def test_gpu_matches_golden_rows(name, widen, flags):
    """every route's kernels (flags 1: the generic kernel) against the fixtures"""
    import d3s
    import hiprt
    d3s.lib()
    if hiprt.device_count() < 1:
        pytest.skip("no GPU")
    check(lambda x, u, T, p: d3s.sample(x, u, T, p, flags=flags), f"gpu flags={flags}", name, widen)
