"""d3s_sample_noalloc (the entry point that allocates nothing: its scratch is
one fixed block of static device memory per GPU) against d3s_sample, through
the C-ABI, on two calls in a row, the second with a smaller input: rows the
segmented kernel spreads over several CUs and the nucleus kernel's ids-only
rows (the calls that use the scratch), then one-wave rows (no scratch); every
id, probability and candidate equal."""
import numpy as np
import pytest

import d3s_workloads as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    import d3s
    import hiprt
    d3s.lib()
    if hiprt.device_count() < 1:
        pytest.skip("no GPU")
    return d3s


def run(gpu, fn, x, u, T, top_p, k, banned=None, want_probs=True):
    """one call of fn (d3s_sample or d3s_sample_noalloc) on device copies"""
    import hiprt
    N, V = x.shape
    dt = gpu.DTYPE_BF16 if x.dtype == np.uint16 else gpu.DTYPE_F32
    bl, bu = hiprt.to_device(x), hiprt.to_device(u)
    bb = hiprt.to_device(banned) if banned is not None else None
    ids = hiprt.DeviceBuffer(4 * N)
    probs = hiprt.DeviceBuffer(4 * N * k) if want_probs else None
    cand = hiprt.DeviceBuffer(4 * N * k) if want_probs else None
    cnt = hiprt.DeviceBuffer(16).zero()
    rc = fn(bl.ptr, dt, N, V, V, bu.ptr, k, None, None, T, top_p, bb.ptr if bb else None, ids.ptr,
            probs.ptr if probs else None, cand.ptr if cand else None, cnt.ptr, 0, None)
    assert rc == 0, rc
    hiprt.synchronize()
    out = (ids.download((N,), np.int32),)
    if want_probs:
        out += (probs.download((N, k), np.float32), cand.download((N, k), np.int32))
    for b in (bl, bu, bb, ids, probs, cand, cnt):
        if b is not None:
            b.free()
    return out


@pytest.mark.parametrize("case", ["C4", "wide fp32"])
def test_no_alloc_equals_sample_twice(gpu, oracle, case):
    L = gpu.lib()
    if case == "C4":
        big = W.make("C4", rows=64, seed=71, uniforms=False)["logits"]
        T, top_p = 1.0, 0.9
    else:
        rng = np.random.default_rng(72)
        big = (rng.standard_normal((24, 100000)) * 3).astype(np.float32)
        T, top_p = 0.8, 0.9
    small = big[:5].copy()
    for x in (big, small):  # two calls in a row, the second smaller
        u = oracle.uniform(71, x.shape[0], x.shape[0], 30)
        a = run(gpu, L.d3s_sample, x, u, T, top_p, 30)
        b = run(gpu, L.d3s_sample_noalloc, x, u, T, top_p, 30)
        print(f"[no-alloc] {case} rows={x.shape[0]} V={x.shape[1]}", flush=True)
        for p, q in zip(a, b):
            assert np.array_equal(p, q)
        assert np.array_equal(b[0], oracle.sample(x, u, T, top_p, n_threads=8)["ids"])


def test_no_alloc_nucleus_ids_only(gpu, oracle):
    """k = V, ids only: the nucleus kernel's ids path files the rows it cannot
    settle in the scratch (rows of one value, heavy ties) for its second
    kernel; two calls, the second smaller."""
    L = gpu.lib()
    w = W.make("C5", rows=256, seed=73, uniforms=False)
    big, ban = w["logits"].copy(), w["banned"]
    big[3, :] = 0.5                      # one value: the full path
    big[7, :] = np.round(big[7] * 2)     # a few values, heavy ties
    big[11, :] = np.round(big[11] * 8)
    for n in (256, 13):  # two calls in a row, the second smaller
        x, b_ = big[:n], ban[:n]
        u = oracle.uniform(73, n, n, x.shape[1])
        a = run(gpu, L.d3s_sample, x, u, 1.0, 0.95, x.shape[1], banned=b_, want_probs=False)
        b = run(gpu, L.d3s_sample_noalloc, x, u, 1.0, 0.95, x.shape[1], banned=b_, want_probs=False)
        print(f"[no-alloc] nucleus ids only rows={n}", flush=True)
        assert np.array_equal(a[0], b[0])
        assert np.array_equal(b[0], oracle.sample(x, u, 1.0, 0.95, banned=b_, n_threads=8)["ids"])


def test_no_alloc_sorting_scratch_limit(gpu, oracle):
    """k > 16384 on a wide row sorts one row at a time in the scratch: a row
    of 239 296 elements (the longest whose keys, count tables, records and
    tile sums fit after the counters) is sampled; one element more is refused
    with D3S_ERR_SCRATCH before anything is launched."""
    rng = np.random.default_rng(74)
    for V, rc in ((239296, 0), (239297, -6)):
        x = (rng.standard_normal((1, V)) * 2.0).astype(np.float32)
        u = oracle.uniform(74, V, 1, V)
        got = gpu.sample(x, u, 1.0, 0.9, want_probs=False, noalloc=True)
        print(f"[no-alloc] sorting V={V} rc={got['rc']}", flush=True)
        assert got["rc"] == rc
        if rc == 0:
            assert got["ids"][0] == oracle.sample(x, u, 1.0, 0.9, n_threads=8)["ids"][0]


def test_no_alloc_one_wave_rows(gpu, oracle):
    """rows that use no scratch at all: the same route and bits as d3s_sample"""
    L = gpu.lib()
    w = W.make("C3", rows=256, seed=73, uniforms=False)
    for n in (256, 7):
        x = np.ascontiguousarray(w["logits"][:n])
        u = oracle.uniform(73, n, n, 30)
        a = run(gpu, L.d3s_sample, x, u, 0.7, 0.7, 30)
        b = run(gpu, L.d3s_sample_noalloc, x, u, 0.7, 0.7, 30)
        for p, q in zip(a, b):
            assert np.array_equal(p, q)


def test_no_alloc_argument_checks(gpu):
    """the same argument checks as d3s_sample (nothing launched)"""
    L = gpu.lib()
    p = 16
    assert L.d3s_sample_noalloc(p, 5, 4, 100, 100, p, 10, None, None, 1.0, 0.9, None, p, None, None, None, 0,
                                None) == -4
    assert L.d3s_sample_noalloc(p, 0, 4, 100, 100, p, 0, None, None, 1.0, 0.9, None, p, None, None, None, 0,
                                None) == -1
    assert L.d3s_sample_noalloc(p, 0, 0, 100, 100, p, 10, None, None, 1.0, 0.9, None, p, None, None, None, 0,
                                None) == 0
