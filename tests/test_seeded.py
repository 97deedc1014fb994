"""d3s_sample_seeded: the uniform draw and the sample in one launch.  Its
results must be the oracle's on the uniforms d3s_uniform_fill would write
(u[r, j] = draw r k + j of (seed, draw), the oracle's own Philox), and the
same bits as the two-launch pair, on every row width of the one-wave
kernel's one-row-a-workgroup form, which draws them (launches of up to 1024
rows)."""
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


def flat_uniforms(oracle, seed, draw, n, k):
    return oracle.uniform(seed, draw, 1, n * k).reshape(n, k)


def check(oracle, gpu, x, k, T, top_p, seed, draw, banned=None, flags=0, label="", vocab=None):
    """vocab: rows of that many elements read at x's row stride (the oracle
    gets the rows alone)"""
    print(f"[seeded] {label} shape={x.shape} k={k} flags={flags}", flush=True)
    u = flat_uniforms(oracle, seed, draw, x.shape[0], k)
    sub = dict(row_stride=x.shape[1], vocab=vocab) if vocab else {}
    got = gpu.sample(x, k, T, top_p, banned=banned, flags=flags, seed_draw=(seed, draw), **sub)
    assert got["rc"] == 0, got["rc"]
    exp = oracle.sample(np.ascontiguousarray(x[:, :vocab]) if vocab else x, u, T, top_p, banned=banned,
                        n_threads=8, op_graph=bool(flags & gpu.FLAG_OP_GRAPH))
    pair = gpu.sample(x, u, T, top_p, banned=banned, flags=flags, **sub)
    assert pair["rc"] == 0
    bad = np.nonzero(got["ids"] != exp["ids"])[0]
    parity_report.record(f"seeded {label}", len(exp["ids"]), len(bad), 0)
    assert len(bad) == 0, (bad[:10], got["ids"][bad[:10]], exp["ids"][bad[:10]])
    assert np.array_equal(got["cand"], exp["cand"])
    nan = np.isnan(got["probs"]) & np.isnan(exp["probs"])
    assert np.array_equal(got["probs"][~nan], exp["probs"][~nan])
    for key in ("ids", "cand", "counters"):
        assert np.array_equal(got[key], pair[key]), key
    assert np.array_equal(got["probs"].view(np.uint32), pair["probs"].view(np.uint32))
    return got


@pytest.mark.parametrize("name", ["C1", "C2", "C3"])
def test_seeded_configs(gpu, oracle, name):
    w = W.make(name, rows=300 if name == "C1" else None, seed=21, uniforms=False)
    check(oracle, gpu, w["logits"], w["k"], w["temperature"], w["top_p"], 42, 5, banned=w["banned"],
          label=name)


@pytest.mark.parametrize("bf16,V,k", [(False, 200, 64), (False, 1500, 1), (False, 3000, 30), (False, 6000, 17),
                                      (True, 1000, 30), (True, 5000, 64), (True, 8000, 30)])
def test_seeded_widths(gpu, oracle, bf16, V, k):
    rng = np.random.default_rng(500 + V + k)
    x = (rng.standard_normal((40, V)) * 2.5).astype(np.float32)
    x[np.arange(40), rng.integers(0, V, 40)] += 6.0
    T = rng.uniform(0.5, 1.5, 40).astype(np.float32)
    top_p = rng.uniform(0.5, 0.99, 40).astype(np.float32)
    ban = rng.integers(0, V, 40).astype(np.int32)
    if bf16:
        x = W.f32_to_bf16_bits(x)
    check(oracle, gpu, x, k, T, top_p, 7, 1234567890123, banned=ban, label=f"V={V} k={k} bf16={bf16}")


@pytest.mark.parametrize("bf16", [False, True])
def test_seeded_high_words_and_row_stride(gpu, oracle, bf16):
    """Seeds and draws with their high 32 bits set (the kernel takes both as
    leading arguments, the draw split into two words), on rows read at a
    stride wider than the row."""
    rng = np.random.default_rng(91 + bf16)
    V, stride = 3001, 3072
    x = (rng.standard_normal((24, stride)) * 2.5).astype(np.float32)
    if bf16:
        x = W.f32_to_bf16_bits(x)
    for seed, draw in ((0xFEDCBA9876543210, 0x8000000000000007), (0x100000000, 0xFFFFFFFF)):
        check(oracle, gpu, x, 30, 0.9, 0.85, seed, draw, vocab=V,
              label=f"seed={seed:#x} draw={draw:#x} V={V} stride={stride} bf16={bf16}")


def test_seeded_largest_launch_and_flags(gpu, oracle):
    """1024 rows (the largest launch that draws its own uniforms), then the
    op graph's order and the forced exact row sum."""
    rng = np.random.default_rng(77)
    x = (rng.standard_normal((1024, 1000)) * 2.5).astype(np.float32)
    check(oracle, gpu, x, 30, 0.8, 0.9, 3, 9, label="1024 rows")
    y = x[:64]
    check(oracle, gpu, y, 30, 0.8, 0.9, 3, 10, flags=gpu.FLAG_OP_GRAPH, label="op graph")
    got = check(oracle, gpu, y, 30, 0.8, 0.9, 3, 11, flags=gpu.FLAG_EXACT_LSE, label="exact lse")
    assert got["counters"][gpu.COUNTER_EXACT_LSE] == 64


def test_seeded_refuses_other_routes(gpu, oracle):
    """k above 64, rows wider than one wave's registers, the generic flag and
    launches of more than 1024 rows: D3S_ERR_UNSUPPORTED, nothing launched."""
    rng = np.random.default_rng(78)
    x = (rng.standard_normal((4, 9000)) * 2.5).astype(np.float32)
    many = (rng.standard_normal((1025, 300)) * 2.5).astype(np.float32)
    for k, flags, xx in ((65, 0, x[:, :4000]), (30, 0, x), (30, 1, x[:, :4000]), (30, 0, many)):
        got = gpu.sample(np.ascontiguousarray(xx), k, 1.0, 0.9, flags=flags, seed_draw=(1, 2))
        assert got["rc"] == gpu.ERR_UNSUPPORTED
