"""k beyond the generic kernel's LDS sort on rows longer than the nucleus
kernel takes: the reference's op graph with top-k disabled on a wide row
(src/sampling.c:33-35, a full argsort), here the sorting kernels (k_bk_*: a
radix sort over the row's segments, then the tail).

Ids, candidates (the index of every rank) and probabilities must equal the
oracle's bit for bit; the oracle is pinned by the closed form and brute force
(tests/test_oracle.py)."""
import sys

import numpy as np
import pytest

import d3s_workloads as W
import parity_report

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    import d3s
    import hiprt
    d3s.lib()
    if hiprt.device_count() < 1:
        pytest.skip("no GPU")
    return d3s


def banner(msg):
    print(f"[bigk] {msg}", flush=True)
    sys.stdout.flush()


def check(gpu, oracle, logits, u, T, top_p, banned=None, label="", noalloc=False):
    banner(f"{label} shape={logits.shape} k={u.shape[1]}")
    exp = oracle.sample(logits, u, T, top_p, banned=banned, n_threads=8)
    got = gpu.sample(logits, u, T, top_p, banned=banned, noalloc=noalloc)
    assert got["rc"] == 0, got["rc"]
    bad = np.nonzero(got["ids"] != exp["ids"])[0]
    edge = int(np.sum((exp["flags"] & (oracle.TOPP_EDGE | oracle.RACE_EDGE)) != 0))
    parity_report.record(label, len(exp["ids"]), len(bad), edge)
    assert len(bad) == 0, (bad[:10], got["ids"][bad[:10]], exp["ids"][bad[:10]])
    assert np.array_equal(got["cand"], exp["cand"])
    both_nan = np.isnan(got["probs"]) & np.isnan(exp["probs"])
    assert np.array_equal(np.isnan(got["probs"]), np.isnan(exp["probs"]))
    assert np.array_equal(got["probs"][~both_nan], exp["probs"][~both_nan])
    if not noalloc:
        ids_only = gpu.sample(logits, u, T, top_p, banned=banned, want_probs=False)
        assert np.array_equal(ids_only["ids"], exp["ids"])
    return got, exp


@pytest.mark.parametrize("V,k,dtype", [(20000, 16385, "f32"), (20000, 20000, "f32"), (17000, 17000, "bf16"),
                                       (40000, 30000, "bf16")])
def test_large_k_equals_the_oracle(gpu, oracle, V, k, dtype):
    rng = np.random.default_rng([V, k])
    x = (rng.standard_normal((3, V)) * np.array([[0.3], [1.0], [3.0]])).astype(np.float32)
    logits = W.f32_to_bf16_bits(x) if dtype == "bf16" else x
    u = oracle.uniform(7, V, 3, k)
    T = np.array([1.0, 0.7, 1.3], np.float32)
    P = np.array([0.95, 0.9, 0.5], np.float32)
    check(gpu, oracle, logits, u, T, P, label=f"bigk V={V} k={k} {dtype}")


def test_c4_shape_with_top_k_disabled(gpu, oracle):
    """BASELINE.json's C4 rows (bf16 [64, 151936], T 1.0, top_p 0.9) with top-k
    disabled: k = V, every rank's candidate and probability."""
    w = W.make("C4", rows=64, seed=42, uniforms=False)
    V = w["logits"].shape[1]
    u = oracle.uniform(42, 1, 64, V)
    check(gpu, oracle, w["logits"], u, w["temperature"], w["top_p"], label="config C4, k = V")


def test_large_k_edge_rows(gpu, oracle):
    """A refused row (NaN), an all -inf row, all-equal logits (ties keep the
    lowest indices), a banned index, masked stretches."""
    V, k = 18000, 17000
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((5, V)) * 2.0).astype(np.float32)
    x[0, 123] = np.nan
    x[1, :] = -np.inf
    x[2, :] = 0.25
    x[4, 100:9000] = -np.inf
    u = oracle.uniform(5, 0, 5, k)
    banned = np.array([-1, -1, 7, int(np.argmax(x[3])), -1], np.int32)
    got, _ = check(gpu, oracle, x, u, 1.0, 0.9, banned=banned, label="bigk edge rows")
    assert got["ids"][0] == -1 and got["ids"][1] == 0


def test_large_k_bf16_at_unit_temperature(gpu, oracle):
    """bf16 logits at a scalar T of 1 (x = L: every x has zero low 16 bits), the
    rows whose first two radix passes are skipped and not launched: ordinary
    rows, a row of one value (no pass runs at all), a masked stretch, a banned
    index, both signs, ties."""
    V, k = 20000, 20000
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((5, V)) * 2.0).astype(np.float32)
    x[1, :] = -0.75
    x[2, 5000:15000] = -np.inf
    x[3] = np.round(x[3] * 2) / 2  # a few values, many ties of each sign
    logits = W.f32_to_bf16_bits(x)
    u = oracle.uniform(6, 0, 5, k)
    banned = np.array([-1, -1, 3, -1, 17], np.int32)
    for T, P in ((1.0, 0.9), (1.0, 1.0)):
        check(gpu, oracle, logits, u, T, P, banned=banned, label=f"bigk bf16 T={T} top_p={P}")
    check(gpu, oracle, logits, u, 1.0, 0.9, banned=banned, label="bigk bf16 T=1 no-alloc", noalloc=True)
    # the same values as fp32 logits: every pass launched, the rows find the
    # first two to skip on the device
    check(gpu, oracle, W.bf16_bits_to_f32(logits), u, 1.0, 0.9, banned=banned, label="bigk fp32 of bf16 values, T=1")


def test_large_k_no_positive_kept_score(gpu, oracle):
    """k = V with uniforms that leave no kept rank a positive score (u = 0:
    score -inf; u = 1: score 0; u NaN or above 1: NaN): the dropped ranks race
    too, across the race's segments."""
    V = k = 20000
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((5, V)) * 3.0).astype(np.float32)
    u = oracle.uniform(7, 0, 5, k)
    u[0, :3000] = 0.0     # kept ranks -inf: the first dropped rank past 3000 with a finite noise wins
    u[1, :3000] = 1.0     # kept scores 0: rank 0 wins the tie with the dropped ranks' 0
    u[2, :] = np.nan      # every score -1: rank 0
    u[3, :3000] = 1.5     # kept scores NaN: a dropped rank wins
    u[4, 0] = 0.0         # rank 0 alone scores -inf: another kept rank wins
    got, exp = check(gpu, oracle, x, u, 1.0, 0.3, label="bigk no positive kept score")
    won = lambda r: int(np.nonzero(exp["cand"][r] == exp["ids"][r])[0][0])
    assert exp["probs"][0, won(0)] == 0.0 and exp["probs"][3, won(3)] == 0.0  # a dropped rank won
    assert won(1) == 0 and won(2) == 0


def test_large_k_without_allocation(gpu, oracle):
    """d3s_sample_noalloc sorts one row at a time in its fixed scratch (after
    the segmented kernel's counters, which stay zero)."""
    w = W.make("C4", rows=3, seed=9, uniforms=False)
    V = w["logits"].shape[1]
    u = oracle.uniform(9, 2, 3, V)
    check(gpu, oracle, w["logits"], u, 1.0, 0.9, label="bigk no-alloc", noalloc=True)
    # the segmented kernel still finds its counters zero afterwards
    w2 = W.make("C4", rows=4, seed=10, uniforms=False)
    u2 = oracle.uniform(10, 0, 4, w2["k"])
    got = gpu.sample(w2["logits"], u2, w2["temperature"], w2["top_p"], noalloc=True)
    assert np.array_equal(got["ids"], oracle.sample(w2["logits"], u2, w2["temperature"], w2["top_p"],
                                                    n_threads=8)["ids"])
