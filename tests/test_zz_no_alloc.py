"""d3s_sample_noalloc (the entry point that allocates nothing: its scratch is
one fixed block of static device memory per GPU) against d3s_sample, through
the C-ABI, on two calls in a row, the second with a smaller input: rows the
segmented kernel spreads over several CUs (the calls that use the scratch),
then one-wave rows (no scratch); every id, probability and candidate equal."""
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


def run(gpu, fn, x, u, T, top_p, k):
    """one call of fn (d3s_sample or d3s_sample_noalloc) on device copies"""
    import hiprt
    N, V = x.shape
    dt = gpu.DTYPE_BF16 if x.dtype == np.uint16 else gpu.DTYPE_F32
    bl, bu = hiprt.to_device(x), hiprt.to_device(u)
    ids, probs, cand = hiprt.DeviceBuffer(4 * N), hiprt.DeviceBuffer(4 * N * k), hiprt.DeviceBuffer(4 * N * k)
    cnt = hiprt.DeviceBuffer(16).zero()
    rc = fn(bl.ptr, dt, N, V, V, bu.ptr, k, None, None, T, top_p, None, ids.ptr, probs.ptr, cand.ptr,
            cnt.ptr, 0, None)
    assert rc == 0, rc
    hiprt.synchronize()
    out = (ids.download((N,), np.int32), probs.download((N, k), np.float32), cand.download((N, k), np.int32))
    for b in (bl, bu, ids, probs, cand, cnt):
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
