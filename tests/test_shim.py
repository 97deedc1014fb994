"""The drop-in shim (include/d3s_model_sampling.h) through its own names, as
drama3-mlx's callers would bind them: m_seed, sample_noise, sample_with_noise
and sample_top_k_top_p (src/sampling.c:179-209, src/mlxu.c:769-774) on device
arrays in the call arena, against the oracle on the same draws.  Each draw
after m_seed(s) is the next Philox stream (s, draw): draw 0 first."""
import ctypes

import numpy as np
import pytest

import d3s_workloads as W

pytestmark = pytest.mark.gpu

F32, BF16, I32 = 0, 1, 2


@pytest.fixture(scope="module")
def shim():
    import d3s
    import hiprt
    L = d3s.lib()
    if hiprt.device_count() < 1:
        pytest.skip("no GPU")
    vp, i32, f32, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    for name, args, res in [
        ("m_seed", [ctypes.c_uint64], None),
        ("sample_noise", [i32, i32, i32], vp),
        ("sample_with_noise", [vp, vp, f32, f32], vp),
        ("sample_top_k_top_p", [vp, f32, i32, f32], vp),
        ("d3s_array_from_host", [vp, i32, i32, i32], vp),
        ("d3s_array_rows", [vp], i32),
        ("d3s_array_cols", [vp], i32),
        ("d3s_array_dtype", [vp], i32),
        ("d3s_array_ndim", [vp], i32),
        ("d3s_array_dim", [vp, i32], i32),
        ("d3s_array_copy_to_host", [vp, vp], None),
        ("d3s_arena_mark", [], sz),
        ("d3s_arena_release", [sz], None),
    ]:
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    return L


def to_host(L, arr, dtype):
    out = np.empty((L.d3s_array_rows(arr), L.d3s_array_cols(arr)), dtype)
    L.d3s_array_copy_to_host(arr, out.ctypes.data)
    return out


def test_reference_names_on_device_arrays(shim, oracle):
    L = shim
    mark = L.d3s_arena_mark()
    try:
        w = W.make("C3", rows=16, seed=13, uniforms=False)
        x = np.ascontiguousarray(w["logits"])
        lx = L.d3s_array_from_host(x.ctypes.data, F32, 16, 4097)
        L.m_seed(99)
        ids = L.sample_top_k_top_p(lx, 0.7, 30, 0.7)  # draw 0
        assert L.d3s_array_dtype(ids) == I32
        # ids are 1-D [N], as the reference's (src/sampling.c:48,161)
        assert L.d3s_array_ndim(ids) == 1
        assert L.d3s_array_dim(ids, 0) == 16 and L.d3s_array_dim(ids, -1) == 16
        assert L.d3s_array_ndim(lx) == 2 and L.d3s_array_dim(lx, -1) == 4097
        got = to_host(L, ids, np.int32).reshape(-1)  # [rows, 1]
        u0 = oracle.uniform(99, 0, 1, 16 * 30).reshape(16, 30)
        assert np.array_equal(got, oracle.sample(x, u0, 0.7, 0.7)["ids"])
        # sample_noise: the next draw, [rows, k]; then the sample on those draws
        un = L.sample_noise(16, 4097, 30)  # draw 1
        u1 = to_host(L, un, np.float32)
        assert u1.shape == (16, 30)
        assert np.array_equal(u1, oracle.uniform(99, 1, 1, 16 * 30).reshape(16, 30))
        ids1 = L.sample_with_noise(lx, un, 1.0, 0.9)
        got1 = to_host(L, ids1, np.int32).reshape(-1)
        assert np.array_equal(got1, oracle.sample(x, u1, 1.0, 0.9)["ids"])
        # bf16 logits, and top_k above V (clamped to V, src/sampling.c:186,207)
        xb = np.ascontiguousarray(W.f32_to_bf16_bits(x[:, :40]))
        lb = L.d3s_array_from_host(xb.ctypes.data, BF16, 16, 40)
        ub = L.sample_noise(16, 40, 100)  # draw 2, k = 40
        u2 = to_host(L, ub, np.float32)
        assert u2.shape == (16, 40)
        got2 = to_host(L, L.sample_with_noise(lb, ub, 0.8, 0.95), np.int32).reshape(-1)
        assert np.array_equal(got2, oracle.sample(xb, u2, 0.8, 0.95)["ids"])
        # m_seed again restarts the draws
        L.m_seed(99)
        again = to_host(L, L.sample_top_k_top_p(lx, 0.7, 30, 0.7), np.int32).reshape(-1)
        assert np.array_equal(again, got)
    finally:
        L.d3s_arena_release(mark)
