"""A head's gemv and its sample (d3s_linear_sample_bf16), in one launch
(D3S_FLAG_ONE_LAUNCH) and in the default two: the
backbone head (src/backbone.c:1213-1215) and the tower's codebook heads
(src/tower.c:228-232,:264,:440-443), m_linear's single-row gemv
(src/mlxu.c:454-496) followed by sample_with_noise on its logits.

Every call is checked against the oracle's two steps on the same inputs:
oracle.linear_bf16 (pinned by the order vectors of test_linear.py), then
oracle.sample on those bf16 logits.  Logits, ids, candidates and
probabilities must be identical, and the same as the two-launch path
(d3s_linear_bf16 then d3s_sample)."""
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
    print(f"[head] {msg}", flush=True)
    sys.stdout.flush()


def bf16(a):
    return W.f32_to_bf16_bits(np.asarray(a, np.float32))


def head_inputs(seed, N, K, V, scale=0.06, peaks=0):
    rng = np.random.default_rng([seed, N, K, V])
    x = bf16(rng.standard_normal((N, K)))
    w = rng.standard_normal((V, K)) * scale
    for _ in range(peaks):  # rows aligned with x give large logits
        r = int(rng.integers(V))
        w[r] += 4.0 * scale * np.sign(W.bf16_bits_to_f32(x[0]))
    return x, bf16(w)


def compare_head(gpu, oracle, x, w, u, T, top_p, flags=0, label="", keep_logits=True):
    op_graph = bool(flags & gpu.FLAG_OP_GRAPH)
    banner(f"{label} x={x.shape} w={w.shape} k={u.shape[1]} flags={flags}")
    logits = oracle.linear_bf16(x, w)
    exp = oracle.sample(logits, u, T, top_p, n_threads=8, op_graph=op_graph)
    got = gpu.linear_sample_bf16(x, w, u, T, top_p, flags=flags | gpu.FLAG_ONE_LAUNCH, keep_logits=keep_logits)
    assert got["rc"] == 0, got["rc"]
    if keep_logits:
        assert np.array_equal(got["y"], logits)
    bad = np.nonzero(got["ids"] != exp["ids"])[0]
    edge = int(np.sum((exp["flags"] & (oracle.TOPP_EDGE | oracle.RACE_EDGE)) != 0))
    banner(f"  rows={len(exp['ids'])} mismatched={len(bad)} boundary={edge} counters={got['counters'].tolist()}")
    parity_report.record(label, len(exp["ids"]), len(bad), edge)
    assert len(bad) == 0, (bad[:10], got["ids"][bad[:10]], exp["ids"][bad[:10]])
    assert np.array_equal(got["cand"], exp["cand"])
    both_nan = np.isnan(got["probs"]) & np.isnan(exp["probs"])
    assert np.array_equal(np.isnan(got["probs"]), np.isnan(exp["probs"]))
    assert np.array_equal(got["probs"][~both_nan], exp["probs"][~both_nan])
    # the default two-launch form, and d3s_sample on the oracle's logits, give the same bits
    two = gpu.linear_sample_bf16(x, w, u, T, top_p, flags=flags, keep_logits=keep_logits)
    assert two["rc"] == 0, two["rc"]
    for key in ("ids", "cand") + (("y",) if keep_logits else ()):
        assert np.array_equal(two[key], got[key]), key
    assert np.array_equal(two["probs"].view(np.uint32), got["probs"].view(np.uint32))
    assert np.array_equal(gpu.sample(logits, u, T, top_p, flags=flags)["ids"], got["ids"])
    return got, exp


@pytest.mark.parametrize("N,K,V,k", [(1, 2048, 4097, 30), (1, 2048, 4096, 30), (1, 2048, 4097, 64),
                                     (1, 2048, 4097, 1), (3, 2048, 4097, 30), (1, 128, 1, 1),
                                     (2, 384, 7, 5), (1, 256, 17, 16), (1, 1024, 8192, 30),
                                     (1, 256, 8193, 30), (1, 512, 3000, 100), (2, 256, 300, 300)])
def test_head_equals_the_oracle(gpu, oracle, N, K, V, k):
    """The fused launch (k <= 64, V <= 8192) and the two-launch route (wider
    rows, k > 64, k = V) on the head's shapes and their edges."""
    x, w = head_inputs(1, N, K, V, peaks=3)
    u = oracle.uniform(5, V, N, k)
    T = np.linspace(0.5, 1.2, N).astype(np.float32) if N > 1 else 0.7
    P = np.linspace(0.6, 0.95, N).astype(np.float32) if N > 1 else 0.7
    compare_head(gpu, oracle, x, w, u, T, P, label=f"head N={N} K={K} V={V} k={k}")


def test_head_many_draws(gpu, oracle):
    """Backbone-head draws with the CLI's parameters and the retry's, over many
    hidden rows and seeds (each call one row, as the reference's decode step)."""
    K, V, k = 2048, 4097, 30
    rng = np.random.default_rng(77)
    w = bf16(rng.standard_normal((V, K)) * 0.06)
    mism = 0
    for i in range(40):
        x = bf16(rng.standard_normal((1, K)))
        T, P = (0.7, 0.7) if i % 2 == 0 else (1.0, 0.95)
        u = oracle.uniform(77, i, 1, k)
        logits = oracle.linear_bf16(x, w)
        exp = oracle.sample(logits, u, T, P)
        got = gpu.linear_sample_bf16(x, w, u, T, P, flags=gpu.FLAG_ONE_LAUNCH, keep_logits=(i % 3 == 0))
        assert got["rc"] == 0
        mism += int(got["ids"][0] != exp["ids"][0])
        assert np.array_equal(got["probs"], exp["probs"]), i
        assert np.array_equal(got["cand"], exp["cand"]), i
    parity_report.record("head: 40 backbone draws", 40, mism, 0)
    assert mism == 0


@pytest.mark.parametrize("flag", ["EXACT_LSE", "EXACT_SELECT", "OP_GRAPH", "GENERIC"])
def test_head_flags(gpu, oracle, flag):
    """Each flag takes its path (the exact lse, the generic procedure from the
    merger's LDS row, the op graph's order, the two-launch route) with the same
    result bits."""
    x, w = head_inputs(3, 1, 2048, 4097, peaks=2)
    u = oracle.uniform(3, 1, 1, 30)
    got, _ = compare_head(gpu, oracle, x, w, u, 0.8, 0.8, flags=getattr(gpu, "FLAG_" + flag),
                          label=f"head flag {flag}")
    if flag == "EXACT_LSE":
        assert got["counters"][gpu.COUNTER_EXACT_LSE] == 1
    if flag == "EXACT_SELECT":
        assert got["counters"][gpu.COUNTER_EXACT_SELECT] == 1


def test_head_without_logits_output(gpu, oracle):
    x, w = head_inputs(4, 2, 1024, 4096)
    u = oracle.uniform(4, 0, 2, 30)
    compare_head(gpu, oracle, x, w, u, 0.7, 0.7, label="head, y = NULL", keep_logits=False)
    x, w = head_inputs(4, 1, 256, 9000)  # the two-launch route with its logits in the workspace
    u = oracle.uniform(4, 1, 1, 30)
    compare_head(gpu, oracle, x, w, u, 0.7, 0.7, label="head V=9000, y = NULL", keep_logits=False)


def test_head_edge_rows(gpu, oracle):
    """Non-finite and degenerate logits out of the gemv: a NaN logit (refused,
    id -1), every logit -inf (id 0), all logits equal (every element a
    candidate: the generic procedure), logits too large for the fast sum at a
    small temperature, and a cut placed on a cumulative boundary."""
    K, V, k = 256, 4097, 30
    x = bf16(np.ones((1, K)))
    rng = np.random.default_rng(8)
    base = rng.standard_normal((V, K)) * 0.05
    # a NaN weight: logit 100 is NaN
    w = base.copy()
    w[100, 3] = np.nan
    got, _ = compare_head(gpu, oracle, x, bf16(w), oracle.uniform(8, 0, 1, k), 0.7, 0.7, label="head NaN")
    assert got["ids"][0] == -1
    # every logit -inf
    w = base.copy()
    w[:, 0] = -np.inf
    got, _ = compare_head(gpu, oracle, x, bf16(w), oracle.uniform(8, 1, 1, k), 0.7, 0.7, label="head -inf")
    assert got["ids"][0] == 0
    # all equal: ties keep the lowest indices
    w = np.zeros((V, K))
    w[:, 0] = 1.0
    compare_head(gpu, oracle, x, bf16(w), oracle.uniform(8, 2, 1, k), 0.7, 0.9, label="head all equal")
    # large logits at the smallest temperature
    w = base * 4000.0
    compare_head(gpu, oracle, x, bf16(w), oracle.uniform(8, 3, 1, k), 0.0, 0.7, label="head huge / T")
    # top_p just at a fast cumulative value: the merger's margin test must take
    # the exact lse and still match
    w = base
    logits = oracle.linear_bf16(x, bf16(w))
    u = oracle.uniform(8, 4, 1, k)
    L = np.sort(W.bf16_bits_to_f32(logits[0]).astype(np.float64))[::-1]
    e = np.exp(L - L.max())
    cum = np.cumsum(e[:k]) / e.sum()
    for r in (3, 10, 20):
        top_p = np.float32(cum[r])
        for tp in (top_p, np.nextafter(top_p, np.float32(0)), np.nextafter(top_p, np.float32(2))):
            compare_head(gpu, oracle, x, bf16(w), u, 1.0, float(tp), label=f"head cut at rank {r}")


def test_head_back_to_back_calls(gpu, oracle):
    """Calls queued on one stream without a synchronisation between them (each
    launch's last arrival resets the row counters the next one counts on), and
    the sampler's other kernels on the same stream in between."""
    import hiprt
    K, V, k, n = 1024, 4097, 30, 6
    rng = np.random.default_rng(12)
    w = bf16(rng.standard_normal((V, K)) * 0.06)
    xs = [bf16(rng.standard_normal((1, K))) for _ in range(n)]
    us = [oracle.uniform(12, i, 1, k) for i in range(n)]
    s = hiprt.Stream()
    bw = hiprt.to_device(w)
    bx = [hiprt.to_device(x) for x in xs]
    bu = [hiprt.to_device(u) for u in us]
    ids = hiprt.DeviceBuffer(4 * n)
    wide = W.make("C4", rows=2, seed=3, uniforms=False)
    uw = oracle.uniform(3, 0, 2, wide["k"])
    bwl, buw, bwid = hiprt.to_device(wide["logits"]), hiprt.to_device(uw), hiprt.DeviceBuffer(8)
    L = gpu.lib()
    for i in range(n):
        assert L.d3s_linear_sample_bf16(bx[i].ptr, bw.ptr, 1, K, V, None, bu[i].ptr, k, None, None, 0.7, 0.7,
                                        ids.ptr + 4 * i, None, None, None, gpu.FLAG_ONE_LAUNCH, s.ptr) == 0
        if i == 2:  # the segmented kernel between them (it shares the counters)
            assert gpu.sample_raw(bwl.ptr, gpu.DTYPE_BF16, 2, wide["logits"].shape[1], wide["logits"].shape[1],
                                  buw.ptr, wide["k"], 1.0, 0.9, None, bwid.ptr, stream=s.ptr) == 0
    s.synchronize()
    got = ids.download((n,), np.int32)
    for i in range(n):
        assert got[i] == oracle.sample(oracle.linear_bf16(xs[i], w), us[i], 0.7, 0.7)["ids"][0], i
    exp_w = oracle.sample(wide["logits"], uw, 1.0, 0.9, n_threads=8)["ids"]
    assert np.array_equal(bwid.download((2,), np.int32), exp_w)
    for b in [bw, ids, bwl, buw, bwid] + bx + bu:
        b.free()
    s.destroy()
