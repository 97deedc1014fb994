"""The backbone head's logits (src/backbone.c:1213-1215: m_linear of one
hidden row, the reference's gemv, src/mlxu.c:365-400,:492-495) and their
sampling fused into the same launch.

The oracle is pinned by hand-derived vectors whose answer depends on the
gemv's order (within a lane, across blocks, and in the lane tree: a sum of
2^24, 1 and -2^24 is 0 or 1 depending on which pair meets first), by float64
within the bf16 rounding, and by exact integer dot products.  Whether the
reference's Metal compiler fuses its multiply-adds is not pinned (fast-math
contraction); the oracle fuses them, and a bf16 product's exactness in fp32
makes the choice immaterial unless a product overflows or goes subnormal (a
hand-derived row shows the split)."""
import numpy as np
import pytest

import d3s_workloads as W


def bf16(a):
    return W.f32_to_bf16_bits(np.asarray(a, np.float32))


def f32(b):
    return (np.asarray(b, np.uint32) << 16).view(np.float32)


def _one_row(K, placements):
    """x = 1 everywhere, w[0] = the given values at the given element indices."""
    x = bf16(np.ones((1, K)))
    w = np.zeros((1, K), np.float32)
    for i, v in placements:
        w[0, i] = v
    return x, bf16(w)


BIG = 2.0 ** 24


@pytest.mark.parametrize("placements,expected", [
    # one lane (0), one block: elements 0, 1, 2 added in that order: (2^24 + 1) - 2^24 = 0
    ([(0, BIG), (1, 1.0), (2, -BIG)], 0.0),
    # the same lane across blocks 0, 1, 2 (elements 0, 128, 256): 0
    ([(0, BIG), (128, 1.0), (256, -BIG)], 0.0),
    # the tree meets lanes 0 and 16 first (elements 0, 64), then lane 8 (element 32): 1
    ([(0, BIG), (32, 1.0), (64, -BIG)], 1.0),
    # lanes 0 and 1 meet at the last step of the tree (elements 0, 4, 8 -> lanes 0, 1, 2):
    # 16: none; 8: none; 4: none; 2: lane0 + lane2 = 0; 1: 0 + lane1 = 1
    ([(0, BIG), (4, 1.0), (8, -BIG)], 1.0),
])
def test_gemv_order_known_answers(oracle, placements, expected):
    x, w = _one_row(384, placements)
    y = oracle.linear_bf16(x, w)
    assert f32(y)[0, 0] == np.float32(expected)


# Lane 0, block 0: element 0 adds -1.5 * 2^127, element 1 adds 1.5 * 2^127 * 2
# (a product of 1.5 * 2^128, above FLT_MAX).  Fused, the exact running sum
# 1.5 * 2^127 is finite; a multiply then an add gives +inf first.
FMA_SPLIT = ([(0, -1.5 * 2.0 ** 127), (1, 1.5 * 2.0 ** 127)], 1, 2.0)


def _fma_split_row():
    placements, xi, xv = FMA_SPLIT
    x, w = _one_row(128, placements)
    xf = f32(x).copy()
    xf[0, xi] = xv
    return bf16(xf), w


def test_gemv_fused_multiply_add_known_answer(oracle):
    """A bf16 x bf16 product has at most 16 significant bits, so it is exact in
    fp32 whenever it lies in fp32's normal range, and then a fused multiply-add
    RN(w x + acc) equals RN(RN(w x) + acc): the reference's unpinned contraction
    (Metal fast math on `result += in[t] * v[t]`, src/mlxu.c:393) cannot change
    such sums.  The two differ only when a product overflows or falls below
    2^-133 (its 16 bits then reach under 2^-149).  This row separates them: the
    oracle fuses, so the sum is 1.5 * 2^127 (exact in bf16), not +inf."""
    x, w = _fma_split_row()
    y = f32(oracle.linear_bf16(x, w))[0, 0]
    assert y == np.float32(1.5 * 2.0 ** 127)


def _mul_then_add(x, w):
    """the gemv order with a separate fp32 multiply and add (numpy float32)"""
    xf, wf = f32(x)[0], f32(w)
    V, K = wf.shape
    acc = np.zeros((V, 32), np.float32)
    for c in range(K // 128):
        for t in range(4):
            cols = c * 128 + 4 * np.arange(32) + t
            acc = acc + (wf[:, cols] * xf[cols]).astype(np.float32)
    for sn in (16, 8, 4, 2, 1):
        acc[:, :sn] = acc[:, :sn] + acc[:, sn:2 * sn]
    return bf16(acc[:, 0])[None, :]


def test_gemv_normal_range_products_do_not_depend_on_fusing(oracle):
    """On data whose products stay in fp32's normal range (as a head's do) the
    oracle's fused sums equal a multiply-then-add restatement of the same order
    bit for bit, as the exactness of bf16 products implies."""
    rng = np.random.default_rng(5)
    x = bf16(rng.standard_normal((1, 512)))
    w = bf16(rng.standard_normal((300, 512)) * 0.05)
    assert np.array_equal(oracle.linear_bf16(x, w), _mul_then_add(x, w))
    xs, ws = _fma_split_row()
    assert f32(_mul_then_add(xs, ws))[0, 0] == np.inf  # the split row does tell them apart


def test_gemv_exact_integers(oracle):
    rng = np.random.default_rng(3)
    K, V = 512, 300
    xi = rng.integers(-3, 4, (2, K))
    wi = rng.integers(-3, 4, (V, K))
    y = f32(oracle.linear_bf16(bf16(xi), bf16(wi)))
    exact = (xi @ wi.T).astype(np.float32)  # |.| <= 4608: every partial sum is exact in fp32
    assert np.array_equal(y, f32(bf16(exact)))


def test_gemv_against_float64(oracle):
    rng = np.random.default_rng(4)
    x = bf16(rng.standard_normal((1, 2048)))
    w = bf16(rng.standard_normal((4097, 2048)) * 0.02)
    y = f32(oracle.linear_bf16(x, w)).astype(np.float64)
    ref = f32(x).astype(np.float64) @ f32(w).astype(np.float64).T
    acc = np.abs(f32(x)).astype(np.float64) @ np.abs(f32(w)).astype(np.float64).T
    # bf16 rounding (half an ulp: 2^-9 relative) and fp32 accumulation (K = 2048 terms)
    assert np.all(np.abs(y - ref) <= 2.0 ** -8 * np.abs(ref) + 2048 * 2.0 ** -23 * acc)


def test_bf16_rounding_is_nearest_even(oracle):
    """Sums of two exact bf16 values that fall on, or just past, a tie between
    two bf16 neighbours (spacing 2^-7 at 1)."""
    pairs = [((1.0, 2 ** -8), 1.0),                       # tie: to even (1.0)
             ((1.0, 3 * 2 ** -8), 1.0 + 2 ** -6),         # tie: to even (1 + 2^-6)
             ((1.0 + 2 ** -7, 2 ** -8), 1.0 + 2 ** -6),   # tie from an odd neighbour: up
             ((1.0, 2 ** -8 + 2 ** -15), 1.0 + 2 ** -7),  # past the tie: up
             ((-1.0, -(2 ** -8)), -1.0),                  # negative tie: to even
             ((2.0 ** 127, 2.0 ** 127), np.inf)]          # overflow
    x = bf16(np.ones((1, 128)))
    w = np.zeros((len(pairs), 128), np.float32)
    for r, ((a, b), _) in enumerate(pairs):
        w[r, 0], w[r, 1] = a, b  # lane 0, added in that order
    wb = bf16(w)
    assert np.array_equal(f32(wb)[:, :2], w[:, :2])  # the inputs are exact in bf16
    y = f32(oracle.linear_bf16(x, wb))[0]
    assert y.tolist() == [np.float32(e) for _, e in pairs]


@pytest.fixture(scope="module")
def gpu():
    import d3s
    import hiprt
    d3s.lib()
    if hiprt.device_count() < 1:
        pytest.skip("no GPU")
    return d3s


@pytest.mark.gpu
@pytest.mark.parametrize("N,K,V", [(1, 2048, 4097), (3, 2048, 4097), (1, 128, 1), (2, 384, 7),
                                   (1, 1024, 9000), (1, 2048, 4096)])
def test_gemv_equals_the_oracle(gpu, oracle, N, K, V):
    rng = np.random.default_rng([N, K, V])
    x = bf16(rng.standard_normal((N, K)))
    w = bf16(rng.standard_normal((V, K)) * 0.05)
    rc, y = gpu.linear_bf16(x, w)
    assert rc == 0
    assert np.array_equal(y, oracle.linear_bf16(x, w))
    x2, w2 = _one_row(384, [(0, BIG), (32, 1.0), (64, -BIG)])
    assert np.array_equal(gpu.linear_bf16(x2, w2)[1], oracle.linear_bf16(x2, w2))
    x3, w3 = _fma_split_row()  # fused multiply-add: finite, where multiply-then-add overflows
    assert np.array_equal(gpu.linear_bf16(x3, w3)[1], oracle.linear_bf16(x3, w3))


@pytest.mark.gpu
def test_head_gemv_and_sample_replayed_as_a_graph(gpu, oracle):
    """The head's two launches (d3s_linear_bf16, then d3s_sample on its logits)
    captured in one HIP graph and replayed; between replays the hidden row and
    the uniforms change (eager uploads), and every replay's ids and logits
    must equal the oracle's."""
    import ctypes
    import hiprt
    H = hiprt.hip()
    K, V, k = 2048, 4097, 30
    rng = np.random.default_rng(9)
    w = bf16(rng.standard_normal((V, K)) * 0.06)
    bw, bx = hiprt.to_device(w), hiprt.DeviceBuffer(2 * K)
    by, bu, bids = hiprt.DeviceBuffer(2 * V), hiprt.DeviceBuffer(4 * k), hiprt.DeviceBuffer(4)
    s = hiprt.Stream()
    graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
    hiprt.check(H.hipStreamBeginCapture(s.ptr, 0), "begin capture")
    assert gpu.lib().d3s_linear_bf16(bx.ptr, bw.ptr, 1, K, V, by.ptr, s.ptr) == 0
    assert gpu.sample_raw(by.ptr, gpu.DTYPE_BF16, 1, V, V, bu.ptr, k, 0.7, 0.7, None, bids.ptr,
                          stream=s.ptr) == 0
    hiprt.check(H.hipStreamEndCapture(s.ptr, ctypes.byref(graph)), "end capture")
    hiprt.check(H.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0), "instantiate")
    try:
        for rep in range(6):
            x = bf16(rng.standard_normal((1, K)))
            u = oracle.uniform(9, rep, 1, k)
            bx.upload(x)
            bu.upload(u)
            hiprt.synchronize()
            hiprt.check(H.hipGraphLaunch(exe, s.ptr), "graph launch")
            s.synchronize()
            logits = oracle.linear_bf16(x, w)
            assert np.array_equal(by.download((1, V), np.uint16), logits), rep
            assert bids.download((1,), np.int32)[0] == oracle.sample(logits, u, 0.7, 0.7)["ids"][0], rep
    finally:
        H.hipGraphExecDestroy(exe)
        H.hipGraphDestroy(graph)
        s.destroy()
