"""GPU parity: the HIP sampler through the C-ABI against the CPU oracle on the
same logits and the same uniforms.

Ids and candidate lists must be identical on every row and probabilities
bit-identical (the north-star bar is ids equal except boundary rows and
probabilities within 1e-5 relative; both kernels compute the oracle's exact
definition, so the test asks for equality and reports the boundary rows, i.e.
rows where an fp32 implementation with another summation order could differ)."""
import sys

import numpy as np
import pytest

import d3s_workloads as W
import parity_report

pytestmark = pytest.mark.gpu

RTOL = 1e-5  # the north-star tolerance for post-filter probabilities


@pytest.fixture(scope="module")
def gpu():
    import d3s
    import hiprt
    d3s.lib()
    if hiprt.device_count() < 1:
        pytest.skip("no GPU")
    return d3s


def banner(msg):
    print(f"[gpu-parity] {msg}", flush=True)
    sys.stdout.flush()


def compare(oracle, gpu, logits, u, T, top_p, banned=None, flags=0, label="", row_stride=None,
            vocab=None, op_graph=False):
    """GPU against the oracle; op_graph: every row in the op graph's order on
    both sides (D3S_FLAG_OP_GRAPH, the reference's D3_NO_FUSED_SAMPLER)."""
    if op_graph:
        flags |= gpu.FLAG_OP_GRAPH
    banner(f"{label} shape={logits.shape} k={u.shape[1]} flags={flags}")
    exp = oracle.sample(logits, u, T, top_p, banned=banned, n_threads=8, row_stride=row_stride,
                        vocab=vocab, op_graph=op_graph)
    got = gpu.sample(logits, u, T, top_p, banned=banned, flags=flags, row_stride=row_stride,
                     vocab=vocab)
    assert got["rc"] == 0, got["rc"]
    bad = np.nonzero(got["ids"] != exp["ids"])[0]
    edge = int(np.sum((exp["flags"] & (oracle.TOPP_EDGE | oracle.RACE_EDGE)) != 0))
    banner(f"  rows={len(exp['ids'])} mismatched={len(bad)} boundary={edge} "
           f"counters={got['counters'].tolist()}")
    parity_report.record(label, len(exp["ids"]), len(bad), edge)
    assert len(bad) == 0, (bad[:10], got["ids"][bad[:10]], exp["ids"][bad[:10]])
    assert np.array_equal(got["cand"], exp["cand"])
    both_nan = np.isnan(got["probs"]) & np.isnan(exp["probs"])
    assert np.array_equal(got["probs"][~both_nan], exp["probs"][~both_nan])
    np.testing.assert_allclose(got["probs"][~both_nan], exp["probs"][~both_nan], rtol=RTOL)
    # the same call asking for ids only (the nucleus kernel then skips the
    # ranking it needs only for probabilities and candidates)
    ids_only = gpu.sample(logits, u, T, top_p, banned=banned, flags=flags, row_stride=row_stride,
                          vocab=vocab, want_probs=False)
    assert ids_only["rc"] == 0, ids_only["rc"]
    bad = np.nonzero(ids_only["ids"] != exp["ids"])[0]
    assert len(bad) == 0, ("ids only", bad[:10], ids_only["ids"][bad[:10]], exp["ids"][bad[:10]])
    return got, exp


def test_device_math_is_bit_exact(gpu, oracle):
    rng = np.random.default_rng(0)
    x = np.concatenate([np.linspace(-110, 95, 400_001, dtype=np.float32),
                        (rng.standard_normal(200_000) * 30).astype(np.float32),
                        np.exp(rng.uniform(-100, 88, 200_000)).astype(np.float32),
                        rng.random(100_000).astype(np.float32),
                        np.array([0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 1.0], np.float32)])
    for divisor in (0.7, 1.0, 1e-5, 3.3, 0.123456):
        e, l, d, f = gpu.math_selftest(x, divisor)
        assert np.array_equal(e.view(np.uint32), oracle.expf(x).view(np.uint32))
        assert np.array_equal(l.view(np.uint32), oracle.logf(x).view(np.uint32))
        ref = x / np.float32(divisor)
        assert np.array_equal(np.isnan(d), np.isnan(ref))
        assert np.array_equal(d[~np.isnan(d)].view(np.uint32), ref[~np.isnan(ref)].view(np.uint32))
        assert np.array_equal(f, oracle.fix40(x))


EPS_EXP2 = 2.0 ** -21  # the bound the wave kernel's top-p margin assumes for v_exp_f32


def test_hardware_exp2_error_bound(gpu):
    """The wave kernel's fast row sum uses the hardware 2^x; its margin test
    assumes a relative error below 2^-21 wherever the result is normal.  Dense
    grid over [-126, 1], every float in [-1, 0] near the grid, random points."""
    rng = np.random.default_rng(21)
    t = np.concatenate([np.linspace(-126, 1, 1 << 22, dtype=np.float32),
                        rng.uniform(-126, 1, 1 << 22).astype(np.float32),
                        (np.arange(-(1 << 20), 0, dtype=np.int64) + 0x3f800000).astype(np.uint32)
                        .view(np.float32) * np.float32(-1),
                        np.array([0.0, -0.0, 1.0, -1.0, -126.0, 0.5, -0.5], np.float32)])
    got = gpu.exp2_selftest(t).astype(np.float64)
    ref = np.exp2(t.astype(np.float64))
    ok = ref >= 2.0 ** -126
    rel = np.abs(got[ok] - ref[ok]) / ref[ok]
    banner(f"v_exp_f32: max relative error {rel.max():.3e} over {ok.sum()} inputs")
    assert rel.max() < EPS_EXP2
    assert gpu.exp2_selftest(np.array([-np.inf], np.float32))[0] == 0.0


def test_hardware_log2_error_bound(gpu):
    """The wave kernel's fast log-sum-exp takes the hardware log2 of its row sum
    (at least about 1, at most V); its margin assumes an error below one ulp of
    the result, bounded as 2^-23 |log2 x| + 2^-24, over dense and random samples
    of [2^-1, 2^24] and every float in [1 - 2^-8, 1 + 2^-8]."""
    rng = np.random.default_rng(22)
    one = np.float32(1.0).view(np.uint32)
    near1 = np.arange(one - (1 << 16), one + (1 << 15), dtype=np.uint32).view(np.float32)
    x = np.concatenate([np.exp2(np.linspace(-1, 24, 1 << 22)).astype(np.float32),
                        np.exp2(rng.uniform(-1, 24, 1 << 22)).astype(np.float32), near1,
                        np.array([0.5, 1.0, 2.0, 4097.0, 2.0 ** 24], np.float32)])
    got = gpu.log2_selftest(x).astype(np.float64)
    ref = np.log2(x.astype(np.float64))
    err = np.abs(got - ref)
    bound = 2.0 ** -23 * np.abs(ref) + 2.0 ** -24
    banner(f"v_log_f32: max absolute error {err.max():.3e}, max error / bound {(err / bound).max():.3f} "
           f"over {x.size} inputs")
    assert np.all(err < bound)


def test_uniform_fill_matches_host(gpu, oracle):
    u = gpu.uniform_fill(100_003, 42, 7)
    assert np.array_equal(u, oracle.uniform(42, 7, 1, 100_003)[0])


@pytest.mark.parametrize("name,rows", [("C1", 10000), ("C2", 9), ("C3", 256), ("C4", 64),
                                       ("C5", 4096)])
def test_parity_on_configs(gpu, oracle, name, rows):
    """BASELINE.json's five configurations at their full shapes (C1: its
    10 000 seeded rows in one launch, which takes k_wave; the kernel that
    serves C1's own calls is tested by test_c1_rows_on_the_latency_kernel)."""
    w = W.make(name, rows=rows, seed=42, uniforms=False)
    u = oracle.uniform(42, 0, rows, w["k"])
    compare(oracle, gpu, w["logits"], u, w["temperature"], w["top_p"], w["banned"],
            label=f"config {name}" + (" (k_wave, one launch of 10 000 rows)" if name == "C1" else ""))


def test_single_row_launches(gpu, oracle):
    """C1 as the CLI runs it: one row per call (the few-row instantiation)."""
    w = W.make("C1", rows=24, seed=3, uniforms=False)
    u = oracle.uniform(42, 100, 24, 30)
    exp = oracle.sample(w["logits"], u, 0.7, 0.7)
    for r in range(24):
        got = gpu.sample(w["logits"][r:r + 1], u[r:r + 1], 0.7, 0.7)
        assert got["ids"][0] == exp["ids"][r]
        assert np.array_equal(got["probs"][0], exp["probs"][r])


def test_c1_rows_on_the_latency_kernel(gpu, oracle):
    """BASELINE.json's 10 000 seeded C1 rows through the kernel that serves C1
    (k_wave_row: launches of at most 1024 rows, one row per 4-wave workgroup):
    the 10 000 rows as launches of 1024 rows and fewer, then 500 of them one
    row per launch, as the CLI samples them (device-resident rows, one
    d3s_sample call per row).  Ids, candidates and probabilities bit-equal to
    the oracle; rows and boundary rows recorded for the parity summary."""
    import hiprt
    N, K = 10000, 30
    w = W.make("C1", rows=N, seed=42, uniforms=False)
    x = w["logits"]
    u = oracle.uniform(42, 0, N, K)
    exp = oracle.sample(x, u, 0.7, 0.7, n_threads=8)
    edge = (exp["flags"] & (oracle.TOPP_EDGE | oracle.RACE_EDGE)) != 0
    bad = 0
    for r0 in range(0, N, 1024):
        r1 = min(r0 + 1024, N)
        banner(f"C1 k_wave_row launch rows {r0}..{r1 - 1}")
        got = gpu.sample(x[r0:r1], u[r0:r1], 0.7, 0.7)
        assert got["rc"] == 0, got["rc"]
        bad += int(np.sum(got["ids"] != exp["ids"][r0:r1]))
        assert np.array_equal(got["ids"], exp["ids"][r0:r1]), r0
        assert np.array_equal(got["cand"], exp["cand"][r0:r1]), r0
        assert np.array_equal(got["probs"], exp["probs"][r0:r1]), r0
    parity_report.record("config C1 (k_wave_row, launches of <= 1024 rows)", N, bad, int(edge.sum()))

    n1 = 500
    rows = np.arange(0, N, N // n1)[:n1]
    V = x.shape[1]
    bl, bu = hiprt.to_device(x), hiprt.to_device(u)
    ids, probs, cand = (hiprt.DeviceBuffer(4 * n1), hiprt.DeviceBuffer(4 * n1 * K),
                        hiprt.DeviceBuffer(4 * n1 * K))
    banner(f"C1 k_wave_row: {n1} one-row launches")
    for i, r in enumerate(rows):
        rc = gpu.sample_raw(bl.ptr + int(r) * V * 4, gpu.DTYPE_F32, 1, V, V, bu.ptr + int(r) * K * 4, K, 0.7, 0.7,
                            None, ids.ptr + 4 * i, probs.ptr + 4 * K * i, cand.ptr + 4 * K * i)
        assert rc == 0, (r, rc)
    hiprt.synchronize()
    got_ids = ids.download((n1,), np.int32)
    bad1 = int(np.sum(got_ids != exp["ids"][rows]))
    parity_report.record("config C1 (k_wave_row, one row per launch)", n1, bad1, int(edge[rows].sum()))
    assert np.array_equal(got_ids, exp["ids"][rows])
    assert np.array_equal(cand.download((n1, K), np.int32), exp["cand"][rows])
    assert np.array_equal(probs.download((n1, K), np.float32), exp["probs"][rows])
    for b in (bl, bu, ids, probs, cand):
        b.free()


@pytest.mark.parametrize("flags", [1, 2, 4, 6, 5])
@pytest.mark.parametrize("name", ["C2", "C3"])
def test_every_path_gives_the_same_bits(gpu, oracle, name, flags):
    w = W.make(name, rows=64 if name == "C3" else 9, seed=5, uniforms=False)
    u = oracle.uniform(5, 0, w["logits"].shape[0], w["k"])
    compare(oracle, gpu, w["logits"], u, w["temperature"], w["top_p"], flags=flags,
            label=f"{name} flags")


@pytest.mark.parametrize("V,k", [(4097, 30), (1024, 30), (4097, 5)])
def test_ties_fused_equals_generic(gpu, oracle, V, k):
    """tests/test_decode.py:73-86 restated: integer-valued logits tie across the
    k-th place; every path keeps the same (lowest-id) candidates."""
    rng = np.random.default_rng(1)
    logits = np.round(rng.standard_normal((8, V)) * 2).astype(np.float32)
    for seed in range(0, 40, 8):
        u = oracle.uniform(seed, 0, 8, k)
        a, _ = compare(oracle, gpu, logits, u, 1.0, 2.0, label=f"ties seed {seed}")
        b, _ = compare(oracle, gpu, logits, u, 1.0, 2.0, flags=gpu.FLAG_GENERIC, label="ties generic")
        assert np.array_equal(a["ids"], b["ids"])


def test_top_p_on_a_cumulative_boundary(gpu, oracle):
    """top_p placed one ulp either side of a row's own cumulative value c_j: the
    cut then depends on the last bit of every term, and the kernel's exact,
    order-independent row sum still reproduces it."""
    w = W.make("C3", rows=64, seed=9, uniforms=False)
    u = oracle.uniform(9, 0, 64, 30)
    x = w["logits"]
    T = np.float32(0.9)
    top_p = np.empty(64, np.float32)
    for r in range(64):
        o = oracle.sample(x[r:r + 1], u[r:r + 1], T, 2.0)
        lse = o["lse"][0]
        xs = np.sort(x[r] / T)[::-1][:30]
        c = np.float32(0)
        cs = []
        for v in xs:
            c = np.float32(c + oracle.expf(np.array([v - lse], np.float32))[0])
            cs.append(c)
        j = 1 + r % 5
        top_p[r] = np.nextafter(cs[j], np.float32(0 if r % 2 else 2))
    got, _ = compare(oracle, gpu, x, u, T, top_p, label="top_p on a boundary")
    # every row is within the wave kernel's margin: each takes the exact row sum
    assert got["counters"][gpu.COUNTER_EXACT_LSE] == 64
    compare(oracle, gpu, x, u, T, top_p, flags=gpu.FLAG_GENERIC, label="top_p on a boundary, generic")


@pytest.mark.parametrize("bf16", [False, True])
def test_many_rows_per_row_parameters(gpu, oracle, bf16):
    """1501 rows (past 1024 rows the wave kernel packs four rows per
    workgroup: the last one is ragged), a different temperature and top_p on
    every row."""
    rng = np.random.default_rng(14)
    x = (rng.standard_normal((1501, 4097)) * 2.5).astype(np.float32)
    x[np.arange(1501), rng.integers(0, 4097, 1501)] += 8.0
    T = rng.uniform(0.2, 1.5, 1501).astype(np.float32)
    top_p = rng.uniform(0.3, 1.0, 1501).astype(np.float32)
    u = oracle.uniform(14, 0, 1501, 30)
    if bf16:
        x = W.f32_to_bf16_bits(x)
    got, _ = compare(oracle, gpu, x, u, T, top_p, label="1501 rows")
    # the fast row sum settles almost every row
    assert got["counters"][gpu.COUNTER_EXACT_LSE] < 50


def test_edge_rows(gpu, oracle):
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((12, 300)) * 2).astype(np.float32)
    x[0, 5] = np.nan
    x[1, 7] = np.inf
    x[2, :] = -np.inf
    x[3, ::2] = -np.inf
    x[4, :] = 3.0
    x[5, :] = np.round(x[5])
    x[6, 10] = 1e30
    x[7, :] = 0.0
    x[7, 3] = -0.0
    u = rng.random((12, 20)).astype(np.float32)
    u[8, :] = 0.0
    u[9, 0] = 0.0
    got, _ = compare(oracle, gpu, x, u, 0.8, 0.9, label="edge rows")
    assert got["ids"][0] == -1 and got["ids"][1] == -1 and got["ids"][2] == 0
    assert got["counters"][gpu.COUNTER_REFUSED] == 2 and got["counters"][gpu.COUNTER_ALL_MASKED] == 1
    compare(oracle, gpu, x, u, 0.8, 0.9, flags=gpu.FLAG_GENERIC, label="edge rows generic")


def test_finite_logit_overflowing_after_temperature(gpu, oracle):
    """x = L / T overflowing to +inf refuses the row (id -1), as the oracle's
    rule on x; the same logits at T = 1 are sampled; on the one-wave and the
    generic kernel."""
    rng = np.random.default_rng(13)
    x = (rng.standard_normal((6, 4097)) * 2).astype(np.float32)
    x[:, 11] = 3e38
    x[3:, 20] = -np.inf
    T = np.array([0.7, 1e-5, 0.5, 1.0, 1.0, 0.99999], np.float32)
    u = rng.random((6, 30)).astype(np.float32)
    for flags in (0, gpu.FLAG_GENERIC):
        got, _ = compare(oracle, gpu, x, u, T, 0.9, flags=flags, label=f"overflow after T flags={flags}")
        assert np.all(got["ids"][:3] == -1) and np.all(got["ids"][3:5] == 11)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("op_graph", [False, True])
def test_exact_row_sum_edges(gpu, oracle, bf16, op_graph):
    """Every row takes the exact row sum (D3S_FLAG_EXACT_LSE) with tiny, zero
    and subnormal logits beside ordinary ones, logits below -2^100, rows whose
    max x lies below 2^-15 (all tiny, or tiny after a large T), and
    temperatures past 2^21 and at the 1e-5 floor: the one-row kernel's
    exact-sum helper waves take x = L / T by the product and two fmas only
    where that cannot change a term."""
    rng = np.random.default_rng(17)
    N, V = 10, 4097
    x = (rng.standard_normal((N, V)) * 2.5).astype(np.float32)
    tiny = np.array([1e-30, -1e-30, 1e-40, -1e-44, 0.0, -0.0, 3e-19, -2e-25, 7e-21], np.float32)
    x[0, :900] = np.resize(tiny, 900)
    x[1, ::3] = -1e35
    x[2, 100:140] = -3e38
    x[3] = np.resize(tiny, V)
    x[3, 7] = 1e-6
    x[4] = (rng.standard_normal(V) * 4e-5).astype(np.float32)
    x[5, :500] = np.resize(tiny, 500)
    x[6, :500] = np.resize(tiny, 500)
    x[7, ::5] = -2e32
    x[8] = np.resize(tiny, V) * np.float32(1e20)
    T = np.array([0.7, 1.0, 0.9, 1.0, 1.0, 4194304.0, 1e-5, 3e6, 0.7, 1.3], np.float32)
    u = oracle.uniform(17, 0, N, 30)
    if bf16:
        x = W.f32_to_bf16_bits(x)
    got, _ = compare(oracle, gpu, x, u, T, 0.9, flags=gpu.FLAG_EXACT_LSE, op_graph=op_graph,
                     label=f"exact row sum edges bf16={bf16} op_graph={op_graph}")
    assert got["counters"][gpu.COUNTER_EXACT_LSE] == N


@pytest.mark.parametrize("bf16,V", [(False, 200), (False, 1500), (False, 3000), (False, 4097),
                                    (False, 6000), (True, 1000), (True, 3000), (True, 5000),
                                    (True, 8000)])
def test_exact_row_sum_shares_every_width(gpu, oracle, bf16, V):
    """Every row width the one-row kernel is built for (fp32 4, 8, 16, 17, 24
    and bf16 4, 8, 10, 16 chunks a lane), every row taking the exact row sum
    (D3S_FLAG_EXACT_LSE): the helper waves' three shares of it must add to
    the oracle's sum at each width's split of the lanes' elements.  Rows
    with T past 2^21 take the shares' re-read with the exact quotient; every
    row has a banned index."""
    rng = np.random.default_rng(300 + V)
    N = 12
    x = (rng.standard_normal((N, V)) * 2.5).astype(np.float32)
    x[np.arange(N), rng.integers(0, V, N)] += 7.0
    T = rng.uniform(0.5, 1.5, N).astype(np.float32)
    T[3] = 3e6
    T[7] = 4194304.0
    top_p = rng.uniform(0.5, 0.99, N).astype(np.float32)
    ban = rng.integers(0, V, N).astype(np.int32)
    u = oracle.uniform(300 + V, 0, N, 30)
    if bf16:
        x = W.f32_to_bf16_bits(x)
    got, _ = compare(oracle, gpu, x, u, T, top_p, banned=ban, flags=gpu.FLAG_EXACT_LSE,
                     label=f"exact row sum shares V={V} bf16={bf16}")
    assert got["counters"][gpu.COUNTER_EXACT_LSE] == N


@pytest.mark.parametrize("T,top_p", [(0.0, 0.7), (np.inf, 0.9), (np.nan, 0.9), (1e-5, 0.5),
                                     (1e4, 0.8), (0.7, np.nan), (0.7, -1.0), (0.7, 1.0)])
def test_parameter_edges(gpu, oracle, T, top_p):
    rng = np.random.default_rng(12)
    x = (rng.standard_normal((16, 500)) * 3).astype(np.float32)
    u = rng.random((16, 30)).astype(np.float32)
    compare(oracle, gpu, x, u, T, top_p, label=f"T={T} top_p={top_p}")


@pytest.mark.parametrize("V,k", [(1, 1), (2, 1), (2, 2), (63, 63), (64, 64), (65, 64), (65, 65),
                                 (100, 80), (5117, 30), (5118, 30), (8189, 64), (8190, 64),
                                 (16381, 30), (16382, 30), (40000, 64), (40000, 300)])
def test_shapes(gpu, oracle, V, k):
    rng = np.random.default_rng([V, k])
    N = 70
    x = (rng.standard_normal((N, V)) * 2.5).astype(np.float32)
    u = oracle.uniform(1, 0, N, k)
    compare(oracle, gpu, x, u, 0.7, 0.8, label=f"V={V}")
    xb = W.f32_to_bf16_bits(x)
    compare(oracle, gpu, xb, u, 0.7, 0.8, label=f"V={V} bf16")


WIDE_MAX = {False: 77821, True: 155641}  # k_wide: 16 waves x 19 chunk rows, any start offset


@pytest.mark.parametrize("bf16", [False, True])
def test_wide_rows_at_and_past_the_limit(gpu, oracle, bf16):
    """Rows held by a whole workgroup's registers, at the widest such row and
    one past it (the generic kernel's); per-row T and top_p."""
    rng = np.random.default_rng(31 + bf16)
    for V in (WIDE_MAX[bf16], WIDE_MAX[bf16] + 1, 33000):
        N = 6
        x = (rng.standard_normal((N, V)) * 3).astype(np.float32)
        x[np.arange(N), rng.integers(0, V, N)] += 7.0
        T = rng.uniform(0.5, 1.5, N).astype(np.float32)
        top_p = rng.uniform(0.5, 1.0, N).astype(np.float32)
        u = oracle.uniform(31, 0, N, 30)
        if bf16:
            x = W.f32_to_bf16_bits(x)
        compare(oracle, gpu, x, u, T, top_p, label=f"wide V={V} bf16={bf16}")


@pytest.mark.parametrize("flags", [0, 1, 2, 4])
def test_wide_paths_give_the_same_bits(gpu, oracle, flags):
    """C4 rows through the wide kernel's fast path and each forced exact path
    (the generic row procedure), and through the generic kernel."""
    w = W.make("C4", rows=12, seed=8, uniforms=False)
    u = oracle.uniform(8, 0, 12, 30)
    got, _ = compare(oracle, gpu, w["logits"], u, w["temperature"], w["top_p"], flags=flags,
                     label=f"C4 flags={flags}")
    if flags == 2:
        assert got["counters"][gpu.COUNTER_EXACT_LSE] == 12
    if flags == 4:
        assert got["counters"][gpu.COUNTER_EXACT_SELECT] == 12


def test_wide_unaligned_banned_and_edge_rows(gpu, oracle):
    rng = np.random.default_rng(33)
    V, stride, N = 100000, 100003, 14
    x = (rng.standard_normal((N, stride)) * 3).astype(np.float32)
    x[0, 5] = np.nan                 # refused
    x[1, 99999] = np.inf             # refused (last element)
    x[2, :] = -np.inf                # all masked: id 0
    x[3, ::2] = -np.inf              # half masked
    x[4, :] = 1.5                    # every element ties: too many candidates, exact select
    x[5, 40000:40010] = 1e30         # logits too large for the fast row sum
    x[6, :] = np.round(x[6])         # heavy ties across the k-th place
    x[7, 0] = 40.0                   # the maximum at the row start
    x[8, V - 1] = 40.0               # the maximum at the row end
    ban = np.full(N, -1, np.int32)
    ban[7], ban[8], ban[9] = 0, V - 1, int(np.argmax(x[9, :V]))
    u = oracle.uniform(33, 0, N, 30)
    for bf16 in (False, True):
        xs = W.f32_to_bf16_bits(x) if bf16 else x
        got, _ = compare(oracle, gpu, xs, u, 0.8, 0.9, banned=ban, row_stride=stride, vocab=V,
                         label=f"wide edge rows bf16={bf16}")
        assert got["ids"][0] == -1 and got["ids"][1] == -1 and got["ids"][2] == 0
    for T in (np.inf, 0.0, 1e-5):
        compare(oracle, gpu, x[6:12], u[6:12], T, 0.9, row_stride=stride, vocab=V,
                label=f"wide rows T={T}")


@pytest.mark.parametrize("bf16,V", [(True, 200003), (False, 100000), (True, 151936)])
def test_wide_rows_with_structure_across_the_row(gpu, oracle, bf16, V):
    """Wide rows (the one-workgroup kernel's, and past it the generic
    kernel's) with structure spread over the row: the top k at the bounds of
    32 KB stretches, a refusal near the end, masked halves, ties everywhere,
    the banned index, the top k inside one stretch, a wide value range and
    fewer finite elements than k; against the oracle and the generic kernel."""
    rng = np.random.default_rng([V, 7])
    N = 12
    seg = 8192  # a 32 KB (bf16: 16 KB) stretch
    nseg = -(-V // seg)
    x = (rng.standard_normal((N, V)) * 2.5).astype(np.float32)
    bounds = np.arange(1, nseg) * seg
    x[1, np.clip(np.concatenate([bounds - 1, bounds, bounds + 1]), 0, V - 1)] += 9.0  # top k at stretch bounds
    x[2, V - 3] = np.nan                   # refused, in the last segment
    x[3, : V // 2] = -np.inf               # half the row masked
    x[5] = np.round(x[5])                  # ties across the row
    x[6, seg + 10: seg + 60] += 20.0       # the top k inside one stretch
    x[7] *= 40.0                           # most of the row far below its max
    x[8, :] = -np.inf
    x[8, [3, V // 2, V - 1]] = 0.5         # three finite elements: fewer than k
    ban = np.full(N, -1, np.int32)
    ban[4] = int(np.argmax(x[4]))
    ban[9] = int(bounds[0])
    x[9, bounds[0]] = 30.0                 # the banned index would be the max
    T = rng.uniform(0.5, 1.5, N).astype(np.float32)
    top_p = rng.uniform(0.5, 1.0, N).astype(np.float32)
    u = oracle.uniform(41, 0, N, 30)
    xs = W.f32_to_bf16_bits(x) if bf16 else x
    got, _ = compare(oracle, gpu, xs, u, T, top_p, banned=ban, label=f"wide structured V={V} bf16={bf16}")
    assert got["ids"][2] == -1
    gen, _ = compare(oracle, gpu, xs, u, T, top_p, banned=ban, flags=gpu.FLAG_GENERIC,
                     label="wide structured rows, generic kernel")
    assert np.array_equal(got["ids"], gen["ids"])
    for T1 in (np.inf, 1e-5):
        compare(oracle, gpu, xs[:6], u[:6], T1, 0.9, label=f"wide structured rows T={T1}")


@pytest.mark.parametrize("bf16", [False, True])
def test_wide_kernel_on_many_rows(gpu, oracle, bf16):
    """A launch of many rows too wide for one wave (one workgroup each)."""
    rng = np.random.default_rng(44 + bf16)
    N, V = 130, 70000
    x = (rng.standard_normal((N, V)) * 3).astype(np.float32)
    x[np.arange(N), rng.integers(0, V, N)] += 7.0
    u = oracle.uniform(44, 0, N, 30)
    xs = W.f32_to_bf16_bits(x) if bf16 else x
    compare(oracle, gpu, xs, u, 0.8, 0.9, label=f"wide kernel, {N} rows bf16={bf16}")


def split_shape(V, bf16, N, cus=256):
    """(chunks per lane, segments per row) the segmented kernel picks for N rows
    of V (0 segments: it does not take them): 8 chunks per lane, or 10 when
    that launch fills whole rounds of the CUs more evenly and fits in one
    round (three bf16 workgroups per CU); segments of 4 waves x 64 lanes."""
    EPC = 8 if bf16 else 4
    nchunks = (EPC - 1 + V + EPC - 1) // EPC
    best, fill_best = (8, 0), -1.0
    for cpt in (8, 10):
        nseg = -(-nchunks // (256 * cpt))
        blocks = N * nseg
        if not (2 <= nseg <= 16 and blocks <= 4096):
            continue
        if cpt == 10 and blocks > cus * (3 if bf16 else 4):
            continue
        fill = blocks / (-(-blocks // cus) * cus)
        if fill > fill_best + 1e-9:
            best, fill_best = (cpt, nseg), fill
    return best


def split_bounds(V, bf16, row, N):
    """Positions where the segmented kernel's segments of row `row` begin (rows
    contiguous from a 16-byte aligned base): the row's 16-byte chunks from the
    aligned address at or below its start, in nseg equal parts (split_shape).
    Empty when the row is not cut."""
    EPC, ES = (8, 2) if bf16 else (4, 4)
    off = (row * V * ES) % 16 // ES
    nseg = split_shape(V, bf16, N)[1]
    if nseg == 0:
        return np.array([], np.int64)
    segc = -(-((off + V + EPC - 1) // EPC) // nseg)
    return np.array([s * segc * EPC - off for s in range(1, nseg)], np.int64)


@pytest.mark.parametrize("V,bf16,N", [(8190, False, 20), (16381, False, 12), (16382, True, 9),
                                      (131069, False, 4), (262137, True, 3), (262138, True, 2),
                                      (327674, True, 2), (40000, True, 40), (151936, True, 6),
                                      (151936, True, 64)])
def test_segmented_rows(gpu, oracle, V, bf16, N):
    """Rows cut into equal segments of at most 2048 or 2560 chunks (2 to 16 per
    row, and one past the most: the generic kernel), with structure across
    segments: the top k at segment bounds, a NaN in the last segment, a
    segment all -inf, the banned index at a bound, fewer finite elements than
    k, per-row T and top_p; against the oracle and the generic kernel."""
    rng = np.random.default_rng([V, 91])
    x = (rng.standard_normal((N, V)) * 2.5).astype(np.float32)
    seg = 8192 * (2 if bf16 else 1)  # nominal bounds for rows that are not cut

    def bounds(r):
        b = split_bounds(V, bf16, r, N)
        return b if len(b) else np.arange(seg, V, seg)

    if N > 1 and len(bounds(1)):
        b1 = bounds(1)
        x[1, np.clip(np.concatenate([b1 - 1, b1]), 0, V - 1)] += 9.0
    if N > 2:
        x[2, V - 2] = np.nan
    if N > 3:
        b3 = bounds(3)
        x[3, : (b3[0] if len(b3) else V)] = -np.inf
    if N > 4:
        x[4, :] = -np.inf
        x[4, [0, V // 2, V - 1]] = 1.0
    ban = np.full(N, -1, np.int32)
    if len(bounds(0)):
        b0 = int(bounds(0)[0])
        ban[0] = b0
        x[0, b0] = 40.0
    T = rng.uniform(0.5, 1.5, N).astype(np.float32)
    top_p = rng.uniform(0.5, 1.0, N).astype(np.float32)
    u = oracle.uniform(91, 0, N, 30)
    xs = W.f32_to_bf16_bits(x) if bf16 else x
    got, _ = compare(oracle, gpu, xs, u, T, top_p, banned=ban, label=f"segmented V={V} bf16={bf16}")
    if N > 2:
        assert got["ids"][2] == -1
    compare(oracle, gpu, xs, u, T, top_p, banned=ban, flags=gpu.FLAG_GENERIC,
            label=f"segmented V={V}, generic kernel")


@pytest.mark.parametrize("V,bf16", [(300, False), (4097, False), (4097, True), (20000, False), (100000, True)])
def test_top_k_reaching_minus_inf_x(gpu, oracle, V, bf16):
    """T at its 1e-5 clamp: 10 logits near 0 give finite x, 25 logits of -1e35
    overflow to x = -inf, every other logit is -inf (masked), among them the
    lowest indices.  The top 30 end in 20 ties at x = -inf, ranked by index,
    where the masked logits come first: the candidates a threshold on the
    logits files (the -1e35 ones) are not those ties.  Every route against the
    oracle."""
    rng = np.random.default_rng([V, 57])
    N = 6
    x = np.full((N, V), -np.inf, np.float32)
    for r in range(N):
        pos = rng.choice(np.arange(V // 3, V), 35, replace=False)
        x[r, pos[:10]] = rng.standard_normal(10).astype(np.float32)
        x[r, pos[10:]] = -1e35 if not bf16 else -9.9e34
    u = oracle.uniform(57, 0, N, 30)
    xs = W.f32_to_bf16_bits(x) if bf16 else x
    for top_p in (2.0, 0.9):
        got, exp = compare(oracle, gpu, xs, u, 0.0, top_p, label=f"-inf ties V={V} bf16={bf16}")
        assert np.all(np.isneginf(np.float32(x[0, exp["cand"][0, 10:]])))  # masked logits rank there
        compare(oracle, gpu, xs, u, 0.0, top_p, flags=gpu.FLAG_GENERIC, label=f"-inf ties V={V} generic")


def test_segmented_launches_of_changing_row_counts(gpu, oracle):
    """The segmented kernel's workspace (records and arrival counters) carried
    from launch to launch on one stream while the row count changes: 1, 64, 8,
    64, 3, 300 rows of C4's width; every launch equal to the oracle."""
    w = W.make("C4", rows=300, seed=47, uniforms=False)
    u = oracle.uniform(47, 0, 300, 30)
    exp = oracle.sample(w["logits"], u, 1.0, 0.9, n_threads=8)
    for n in (1, 64, 8, 64, 3, 300):
        got = gpu.sample(w["logits"][:n], u[:n], 1.0, 0.9, want_probs=False)
        banner(f"segmented launch of {n} rows")
        assert got["rc"] == 0
        assert np.array_equal(got["ids"], exp["ids"][:n]), n


def test_wide_kernel_past_the_segment_limit(gpu, oracle):
    """A launch of more segments than the segmented kernel takes at once (600
    rows of 9 segments): one workgroup per row (the wide kernel)."""
    rng = np.random.default_rng(46)
    N, V = 600, 70000
    x = (rng.standard_normal((N, V)) * 3).astype(np.float32)
    x[np.arange(N), rng.integers(0, V, N)] += 7.0
    u = oracle.uniform(46, 0, N, 30)
    T = rng.uniform(0.6, 1.2, N).astype(np.float32)
    compare(oracle, gpu, x, u, T, 0.9, label=f"wide kernel, {N} rows")


def test_wide_top_p_on_a_cumulative_boundary(gpu, oracle):
    """top_p one ulp either side of a row's own cumulative value: every row is
    within the fast sum's margin and takes the exact fallback."""
    w = W.make("C4", rows=8, seed=9, uniforms=False)
    u = oracle.uniform(9, 0, 8, 30)
    x = w["logits"]
    xf = (x.astype(np.uint32) << 16).view(np.float32)
    top_p = np.empty(8, np.float32)
    for r in range(8):
        o = oracle.sample(x[r:r + 1], u[r:r + 1], 1.0, 2.0)
        lse = o["lse"][0]
        xs = np.sort(xf[r])[::-1][:30]
        c = np.float32(0)
        cs = []
        for v in xs:
            c = np.float32(c + oracle.expf(np.array([v - lse], np.float32))[0])
            cs.append(c)
        j = 1 + r % 5
        top_p[r] = np.nextafter(cs[j], np.float32(0 if r % 2 else 2))
    got, _ = compare(oracle, gpu, x, u, 1.0, top_p, label="wide top_p on a boundary")
    assert got["counters"][gpu.COUNTER_EXACT_LSE] == 8


@pytest.mark.parametrize("V,k", [(4097, 4097), (4097, 700), (1000, 65), (4608, 4608), (4609, 2000),
                                 (5120, 5120), (5121, 700), (8192, 8192), (8193, 300), (300, 200)])
def test_ranked_nucleus_rows(gpu, oracle, V, k):
    """k > 64 (the op graph's semantics: every rank exact, prefix sums exact):
    near-flat rows, per-row T and top_p, and the same bits as the generic
    kernel."""
    rng = np.random.default_rng([V, k, 3])
    N = 24
    x = (rng.standard_normal((N, V)) * 0.3).astype(np.float32)
    T = rng.uniform(0.5, 1.5, N).astype(np.float32)
    top_p = rng.uniform(0.5, 1.0, N).astype(np.float32)
    u = oracle.uniform(5, 0, N, k)
    for bf16 in (False, True):
        xs = W.f32_to_bf16_bits(x) if bf16 else x
        a, _ = compare(oracle, gpu, xs, u, T, top_p, label=f"nucleus V={V} k={k} bf16={bf16}")
        b, _ = compare(oracle, gpu, xs, u, T, top_p, flags=gpu.FLAG_GENERIC, label="nucleus generic")
        assert np.array_equal(a["ids"], b["ids"])


def test_ranked_nucleus_edge_rows(gpu, oracle):
    rng = np.random.default_rng(34)
    V, N = 4097, 12
    x = (rng.standard_normal((N, V)) * 0.3).astype(np.float32)
    x[0, 17] = np.nan                # refused
    x[1, 4096] = np.inf              # refused
    x[2, :] = -np.inf                # all masked
    x[3, :] = 0.25                   # one bucket: every rank by index
    x[4, :] = np.round(x[4] * 4)     # a few values, many ties each
    x[5, ::3] = -np.inf              # a third masked
    x[6, 100] = 30.0                 # one logit holds the nucleus
    x[7, :2048] = -1e30              # a huge range of x
    ban = np.where(np.arange(N) % 2 == 0, 0, -1).astype(np.int32)
    ban[9] = 4096
    u = oracle.uniform(34, 0, N, V)
    u[10, :5] = 0.0                  # u = 0: noise 0, score infinite or NaN
    got, _ = compare(oracle, gpu, x, u, 1.0, 0.95, banned=ban, label="nucleus edge rows")
    assert got["ids"][0] == -1 and got["ids"][1] == -1 and got["ids"][2] == 0
    for T in (np.inf, 0.0, 3.0):
        compare(oracle, gpu, x[3:], u[3:], T, 0.9, label=f"nucleus rows T={T}")


def test_ranked_nucleus_exact_retry_on_every_row(gpu, oracle):
    """k = V, ids only, D3S_FLAG_EXACT_LSE: every row of the nucleus kernel's
    ids path goes straight to its exact retry (exact group sums of
    fix40(expf(x - lse)) give the group holding the cut), which otherwise only
    the rows whose first try cannot settle take; C5 rows, ties, masked
    stretches, a banned index, per-row T and top_p, the 1024-thread form."""
    w = W.make("C5", rows=512, seed=23, uniforms=False)
    u = oracle.uniform(23, 0, 512, 4097)
    compare(oracle, gpu, w["logits"], u, w["temperature"], w["top_p"], w["banned"], flags=gpu.FLAG_EXACT_LSE,
            label="nucleus exact retry, C5 rows")
    rng = np.random.default_rng(24)
    for V in (4097, 5000):
        N = 16
        x = (rng.standard_normal((N, V)) * 0.3).astype(np.float32)
        x[1] = np.round(x[1] * 4)        # a few values, many ties each
        x[2, ::3] = -np.inf              # a third masked
        x[3, 7] = 20.0                   # one logit holds the nucleus
        T = rng.uniform(0.5, 1.5, N).astype(np.float32)
        top_p = rng.uniform(0.5, 1.0, N).astype(np.float32)
        ban = np.where(np.arange(N) % 3 == 0, 5, -1).astype(np.int32)
        u = oracle.uniform(24, V, N, V)
        compare(oracle, gpu, x, u, T, top_p, ban, flags=gpu.FLAG_EXACT_LSE, label=f"nucleus exact retry V={V}")


def test_ranked_nucleus_no_positive_kept_score(gpu, oracle):
    """k = V with uniforms that leave no kept rank a positive score (u = 0:
    noise -0, score -inf; u = 1: noise +inf, score 0; u NaN or above 1): the
    dropped ranks (p = 0, score 0 or NaN) race too, and the first maximum may
    be a dropped rank."""
    rng = np.random.default_rng(35)
    V, N = 4097, 8
    x = (rng.standard_normal((N, V)) * 3.0).astype(np.float32)
    u = oracle.uniform(35, 0, N, V)
    u[0, :3000] = 0.0          # kept ranks -inf: a dropped rank wins
    u[1, :3000] = 1.0          # kept scores 0: rank 0 wins the tie
    u[2, :] = np.nan           # every score -1: rank 0
    u[3, :3000] = 1.5          # kept scores NaN: a dropped rank wins
    u[4, :3000] = 1e-30        # 1 - u rounds to 1: noise -0
    u[5, 0] = 0.0              # rank 0 alone scores -inf (p / -0): another kept rank wins
    got, exp = compare(oracle, gpu, x, u, 1.0, 0.3, label="nucleus no positive kept score")
    won = lambda r: int(np.nonzero(exp["cand"][r] == exp["ids"][r])[0][0])
    for r in (0, 3, 4):
        assert exp["probs"][r, won(r)] == 0.0  # a dropped rank won
    assert won(1) == 0 and won(2) == 0


def _u64_to_f32(v):
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


def test_ranked_nucleus_top_p_on_a_prefix(gpu, oracle):
    """k = V: top_p one ulp either side of a row's own exact prefix sum
    (fixed point of d3s_expf(x_r - lse) over ranks, rounded once): the cut
    depends on the last bit of that sum."""
    w = W.make("C5", rows=16, seed=12, uniforms=False)
    x, N, V = w["logits"], 16, 4097
    u = oracle.uniform(12, 0, N, V)
    top_p = np.empty(N, np.float32)
    for r in range(N):
        xr = x[r].copy()
        if w["banned"][r] >= 0:
            xr[w["banned"][r]] = -np.inf
        lse = oracle.sample(x[r:r + 1], u[r:r + 1], 1.0, 2.0, banned=w["banned"][r:r + 1])["lse"][0]
        order = np.lexsort((np.arange(V), -xr))
        terms = oracle.fix40(oracle.expf((xr[order] - lse).astype(np.float32)))
        j = 500 + 211 * r
        P = int(np.sum(terms[:j + 1].astype(object)))
        f = np.float32(_u64_to_f32(P) * np.float32(2.0 ** -40))
        top_p[r] = np.nextafter(f, np.float32(0 if r % 2 else 2))
    compare(oracle, gpu, x, u, 1.0, top_p, banned=w["banned"], label="nucleus top_p on a prefix")


def test_strided_and_unaligned_rows(gpu, oracle):
    rng = np.random.default_rng(13)
    for stride, V in [(4099, 4097), (4097, 4000), (301, 300), (8195, 8190)]:
        x = (rng.standard_normal((40, stride)) * 2).astype(np.float32)
        u = oracle.uniform(2, 0, 40, 30)
        compare(oracle, gpu, x, u, 0.7, 0.7, row_stride=stride, vocab=V, label=f"stride {stride}")
        xb = W.f32_to_bf16_bits(x)
        compare(oracle, gpu, xb, u, 0.7, 0.7, row_stride=stride, vocab=V, label=f"stride {stride} bf16")


def test_banned_rows(gpu, oracle):
    w = W.make("C5", rows=64, seed=4, uniforms=False)
    u = oracle.uniform(4, 0, 64, 4097)
    compare(oracle, gpu, w["logits"], u, 1.0, 0.95, banned=w["banned"], label="C5 banned")
    w3 = W.make("C3", rows=64, seed=4, uniforms=False)
    u3 = oracle.uniform(4, 0, 64, 30)
    ban = np.where(np.arange(64) % 3 == 0, np.argmax(w3["logits"], axis=1), -1).astype(np.int32)
    compare(oracle, gpu, w3["logits"], u3, 0.7, 0.7, banned=ban, label="C3 banned argmax")


# every route's register forms start and end at these lengths (and some
# between): one wave, a workgroup, the nucleus kernel's three forms, generic
ROUTE_EDGES = [1, 2, 17, 63, 64, 65, 300, 1000, 2047, 3841, 4096, 4097, 4352, 4353, 4608, 4609, 5120,
               5121, 6141, 6142, 8185, 8186, 8192, 8193, 16381, 16382, 32761, 32762, 40000]


@pytest.mark.parametrize("case", range(200))
def test_random_configurations_across_routes(gpu, oracle, case):
    """Seeded random configurations: a length at or near a route's edge, k up
    to 64 or above, either dtype, one to six rows (one case in ten a batch of
    200 to 1501), per-row T and top_p (including T = 0 and top_p >= 1), a
    padded row stride, banned indices, ties, masked stretches, all -inf rows,
    peaks; every id, candidate and probability equal to the oracle's."""
    rng = np.random.default_rng([7919, case])
    V = int(rng.choice(ROUTE_EDGES))
    bf16 = bool(rng.integers(0, 2))
    if V > 64 and rng.random() < 0.4:
        k = int(rng.integers(65, min(V, 2000) + 1))
    else:
        k = int(rng.integers(1, min(V, 64) + 1))
    N = int(rng.integers(1, 7)) if rng.random() < 0.9 else int(rng.choice([200, 1100, 1501]))
    stride = V + int(rng.integers(0, 8))
    sigma = float(rng.choice([0.3, 2.5, 6.0]))
    x = (rng.standard_normal((N, stride)) * sigma).astype(np.float32)
    for r in range(N):
        kind = rng.integers(0, 6)
        if kind == 0:
            x[r, rng.integers(0, V, 5)] += 8.0                  # peaks
        elif kind == 1:
            x[r] = np.round(x[r] * 2) / 2                        # many ties
        elif kind == 2:
            a = int(rng.integers(0, V))
            x[r, a:a + V // 3] = -np.inf                         # a masked stretch
        elif kind == 3 and N > 1:
            x[r, :V] = -np.inf                                   # all masked
    T = rng.choice(np.float32([0.0, 0.3, 0.7, 1.0, 2.5]), N).astype(np.float32)
    top_p = rng.choice(np.float32([0.1, 0.7, 0.95, 1.0, 1.5]), N).astype(np.float32)
    ban = np.where(rng.random(N) < 0.5, rng.integers(0, V, N), -1).astype(np.int32)
    u = oracle.uniform(int(rng.integers(0, 1 << 30)), 0, N, k)
    xs = W.f32_to_bf16_bits(x) if bf16 else x
    compare(oracle, gpu, xs, u, T, top_p, banned=ban, row_stride=stride, vocab=V,
            label=f"random case {case}: V={V} k={k} N={N} stride={stride} bf16={bf16} sigma={sigma}")


def test_calls_on_several_streams_at_once(gpu, oracle):
    """d3s_sample is reentrant across streams: four streams each take another
    route (a 512-row batch for the wave kernel, wide bf16 rows, k = V rows
    for the nucleus kernel, one row), their launches issued in turn three
    times with no wait between the streams, each writing its own ids; after
    one device-wide wait every stream's ids equal the oracle's."""
    import hiprt
    rng = np.random.default_rng(77)
    cases = [(4097, 30, 512, False), (151936, 30, 8, True), (4097, 4097, 64, False), (4097, 30, 1, False)]
    streams, runs = [], []
    try:
        for V, k, N, bf16 in cases:
            x = (rng.standard_normal((N, V)) * 2.5).astype(np.float32)
            xs = W.f32_to_bf16_bits(x) if bf16 else x
            u = oracle.uniform(77, V, N, k)
            runs.append((xs, u, N, V, k, bf16, hiprt.to_device(xs), hiprt.to_device(u), hiprt.DeviceBuffer(4 * N)))
            streams.append(hiprt.Stream())
        hiprt.synchronize()
        banner("four routes on four streams, three rounds")
        for _ in range(3):
            for s, (xs, u, N, V, k, bf16, bl, bu, bi) in zip(streams, runs):
                dt = gpu.DTYPE_BF16 if bf16 else gpu.DTYPE_F32
                assert gpu.sample_raw(bl.ptr, dt, N, V, V, bu.ptr, k, 0.8, 0.9, None, bi.ptr, stream=s.ptr) == 0
        hiprt.synchronize()
        for xs, u, N, V, k, bf16, bl, bu, bi in runs:
            exp = oracle.sample(xs, u, 0.8, 0.9, n_threads=8)
            assert np.array_equal(bi.download((N,), np.int32), exp["ids"]), (V, k, N, bf16)
    finally:
        for s in streams:
            s.destroy()


def test_shim_entry_points(gpu, oracle):
    """d3_sample (src/testapi.c:155-166): m_seed, device draws, sample."""
    w = W.make("C3", rows=32, seed=6, uniforms=False)
    x = w["logits"]
    ids = gpu.d3_sample(x, 0.7, 30, 0.7, 1234)
    u = oracle.uniform(1234, 0, 1, 32 * 30).reshape(32, 30)  # draw 0, flat index r*k+j
    assert np.array_equal(ids, oracle.sample(x, u, 0.7, 0.7)["ids"])
    ids2 = gpu.d3_sample_with_noise(x, u, 0.7, 0.7)
    assert np.array_equal(ids, ids2)
    # top_k above V clamps to V (src/sampling.c:207)
    small = x[:, :20].copy()
    ids3 = gpu.d3_sample(small, 1.0, 50, 0.9, 7)
    u3 = oracle.uniform(7, 0, 1, 32 * 20).reshape(32, 20)
    assert np.array_equal(ids3, oracle.sample(small, u3, 1.0, 0.9)["ids"])


@pytest.mark.parametrize("temperature,top_k,top_p",
                         [(0.7, 30, 0.7), (1.0, 30, 0.9), (1.0, 5, 1.0), (0.3, 30, 0.95)])
def test_distribution(gpu, temperature, top_k, top_p):
    """tests/test_decode.py:89-114 restated on the GPU: 4000 draws against the
    float64 closed form, within 4 sigma + 1e-3."""
    import closed_form as CF
    rng = np.random.default_rng(0)
    logits = (rng.standard_normal((1, 4097)) * 3).astype(np.float32)
    n = 4000
    u = W.uniform_rows(0, 0, n, top_k)
    ours = gpu.sample(np.repeat(logits, n, axis=0), u, temperature, top_p, want_probs=False)["ids"]
    cf = CF.row(logits[0], u[0], temperature, top_p, top_k)
    expected = dict(zip(cf["cand"][:cf["kept"]], cf["probs"][:cf["kept"]]))
    for token, prob in expected.items():
        freq = np.mean(ours == token)
        assert abs(freq - prob) < 4 * np.sqrt(prob * (1 - prob) / n) + 1e-3, (token, freq, prob)
    assert set(np.unique(ours)) <= set(expected)
