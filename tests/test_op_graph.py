"""GPU: the two orders of the reference's cumulative sum and where each applies.

sample_with_noise (src/sampling.c:194-203) runs its kernel, whose cumulative
and kept sum are left-to-right fp32 sums (:123-131), iff k <= 64, k < V,
V <= 65536 and D3_NO_FUSED_SAMPLER is unset (:197, getenv at every call);
every other call takes the op graph (:22-49), which the oracle models with
exact prefix sums.  Rows with top_p placed where the two orders cut at
different ranks (tests/order_rows.py) make a wrong choice visible in the
probabilities; every comparison is bit for bit against the oracle."""
import os
import subprocess
import sys

import numpy as np
import pytest

import d3s_workloads as W
import order_rows
from test_gpu_parity import banner, compare

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def gpu():
    import d3s
    import hiprt
    d3s.lib()
    if hiprt.device_count() < 1:
        pytest.skip("no GPU")
    return d3s


def rows_with_split(oracle, N, V, k, T, seed, bf16=False, sigma=2.5):
    """N rows of N(0, sigma) with peaks; top_p on a split between the orders
    on the rows that have one, random in [0.5, 1) on the others."""
    rng = np.random.default_rng([seed, V, k])
    x = (rng.standard_normal((N, V)) * sigma).astype(np.float32)
    x[np.arange(N), rng.integers(0, V, N)] += 6.0
    xs = W.f32_to_bf16_bits(x) if bf16 else x
    xf = W.bf16_bits_to_f32(xs) if bf16 else x
    top_p = order_rows.split_top_p(oracle, xf, T, k)
    n_split = int(np.sum(~np.isnan(top_p)))
    top_p = np.where(np.isnan(top_p), rng.uniform(0.5, 1.0, N), top_p).astype(np.float32)
    return xs, top_p, n_split


def kernel_routed(V, k):
    """the reference runs its kernel for this call (src/sampling.c:197)"""
    return k <= 64 and k < V and V <= 1024 * 64


def orders_differ(oracle, xs, u, T, top_p):
    """the rows' answers differ between the kernel's order (the oracle's
    default for a kernel-routed call) and the op graph's"""
    a = oracle.sample(xs, u, T, top_p, op_graph=False)
    b = oracle.sample(xs, u, T, top_p, op_graph=True)
    return not np.array_equal(a["probs"], b["probs"])


@pytest.mark.parametrize("V,k,bf16,N", [
    (4097, 30, False, 48),      # the one-wave kernel
    (8185, 64, True, 16),       # the one-wave kernel's widest bf16 rows
    (10000, 30, False, 16),     # the fused kernel's range: the op graph's order runs on the wide kernel
    (70000, 30, False, 8),      # the wide kernel, past the reference kernel's 65536
    (151936, 30, True, 8),      # C4's shape
    (4097, 4097, False, 16),    # the nucleus kernel (k = V: always the op graph)
    (200000, 30, True, 4),      # the generic kernel
])
def test_op_graph_order_on_every_route(gpu, oracle, V, k, bf16, N):
    """D3S_FLAG_OP_GRAPH on each kernel's rows, and through the generic
    kernel: the same bits as the oracle's op-graph order, including rows whose
    cut falls between the two orders (they take the exact lse)."""
    T = 0.9
    xs, top_p, n_split = rows_with_split(oracle, N, V, min(k, 64), T, seed=1)
    u = oracle.uniform(3, 0, N, k)
    banner(f"op graph V={V} k={k}: {n_split} of {N} rows split the orders")
    got, _ = compare(oracle, gpu, xs, u, T, top_p, op_graph=True, label=f"op graph V={V} k={k}")
    compare(oracle, gpu, xs, u, T, top_p, op_graph=True, flags=gpu.FLAG_GENERIC,
            label=f"op graph V={V} k={k}, generic kernel")
    if kernel_routed(V, k) and n_split:
        assert orders_differ(oracle, xs, u, T, top_p)


@pytest.mark.parametrize("V,k,bf16", [
    (65536, 30, False), (65537, 30, False),   # V <= 1024 * 64 (src/sampling.c:197)
    (65536, 64, True), (65537, 64, True),
    (1000, 64, False), (1000, 65, False),     # k <= 64
    (64, 64, False), (64, 63, False),         # k < V
    (20, 20, True), (2, 2, False),
])
def test_default_order_follows_the_reference_routing(gpu, oracle, V, k, bf16):
    """Without the switch, each call takes the order the reference's routing
    gives it, at both sides of each of its three conditions."""
    N = 12
    xs, top_p, n_split = rows_with_split(oracle, N, V, min(k, 64), 1.0, seed=2, bf16=bf16)
    u = oracle.uniform(4, 0, N, k)
    banner(f"routing V={V} k={k}: {n_split} of {N} rows split the orders")
    compare(oracle, gpu, xs, u, 1.0, top_p, label=f"routing V={V} k={k} bf16={bf16}")
    compare(oracle, gpu, xs, u, 1.0, top_p, flags=gpu.FLAG_GENERIC, label=f"routing V={V} k={k} generic")
    if kernel_routed(V, k) and n_split:
        assert orders_differ(oracle, xs, u, 1.0, top_p)


def test_environment_switch_read_at_every_call(gpu, oracle, monkeypatch):
    """tests/test_decode.py:73-86 restated: D3_NO_FUSED_SAMPLER set or unset
    between calls of one process (set with any value, the empty string too,
    as getenv tests it).  Tied rows give the same ids either way; rows whose
    cut falls between the orders follow the switch."""
    import d3s
    rng = np.random.default_rng(1)
    ties = np.round(rng.standard_normal((8, 4097)) * 2).astype(np.float32)
    xs, top_p, n_split = rows_with_split(oracle, 16, 4097, 30, 1.0, seed=3)
    assert n_split >= 8
    u = oracle.uniform(8, 0, 16, 30)
    fused_exp = oracle.sample(xs, u, 1.0, top_p, op_graph=False)
    ops_exp = oracle.sample(xs, u, 1.0, top_p, op_graph=True)
    assert not np.array_equal(fused_exp["probs"], ops_exp["probs"])
    for seed in range(0, 40, 8):
        ut = oracle.uniform(seed, 0, 8, 30)
        monkeypatch.delenv("D3_NO_FUSED_SAMPLER", raising=False)
        fused = d3s.sample(ties, ut, 1.0, 2.0)
        again = d3s.sample(ties, ut, 1.0, 2.0)
        monkeypatch.setenv("D3_NO_FUSED_SAMPLER", "1")
        ops = d3s.sample(ties, ut, 1.0, 2.0)
        assert fused["ids"].tolist() == again["ids"].tolist() == ops["ids"].tolist(), seed
    for value in (None, "1", "", None):
        if value is None:
            monkeypatch.delenv("D3_NO_FUSED_SAMPLER", raising=False)
        else:
            monkeypatch.setenv("D3_NO_FUSED_SAMPLER", value)
        got = d3s.sample(xs, u, 1.0, top_p)
        exp = fused_exp if value is None else ops_exp
        banner(f"D3_NO_FUSED_SAMPLER={value!r}")
        assert np.array_equal(got["ids"], exp["ids"]) and np.array_equal(got["probs"], exp["probs"])
        assert np.array_equal(got["cand"], exp["cand"])


CHILD = """
import sys
import numpy as np
sys.path[:0] = [{pkg!r}, {oracle!r}, {tests!r}]
import d3s
import d3s_workloads as W
data = np.load({inp!r})
out = {{}}
for name in ("c3", "c4", "split"):
    g = d3s.sample(data[name], data[name + "_u"], float(data[name + "_T"]), data[name + "_p"])
    assert g["rc"] == 0, g["rc"]
    for f in ("ids", "probs", "cand"):
        out[name + "_" + f] = g[f]
np.savez({out!r}, **out)
print("child ok", flush=True)
"""


def test_environment_switch_in_a_fresh_process(gpu, oracle, tmp_path):
    """tests/test_fused.py:32-40's pattern: a child process started with
    D3_NO_FUSED_SAMPLER=1 samples C3 and C4 rows and rows that split the
    orders; every row equals the oracle's op-graph order."""
    w3 = W.make("C3", rows=64, seed=21, uniforms=False)
    w4 = W.make("C4", rows=8, seed=21, uniforms=False)
    xs, top_p, n_split = rows_with_split(oracle, 16, 4097, 30, 1.0, seed=4)
    data = {"c3": w3["logits"], "c3_u": oracle.uniform(21, 0, 64, 30), "c3_T": np.float32(0.7),
            "c3_p": w3["top_p"],
            "c4": w4["logits"], "c4_u": oracle.uniform(21, 64, 8, 30), "c4_T": np.float32(1.0),
            "c4_p": np.float32(w4["top_p"]),
            "split": xs, "split_u": oracle.uniform(22, 0, 16, 30), "split_T": np.float32(1.0),
            "split_p": top_p}
    inp, out = tmp_path / "in.npz", tmp_path / "out.npz"
    np.savez(inp, **data)
    env = dict(os.environ, D3_NO_FUSED_SAMPLER="1")
    script = CHILD.format(pkg=os.path.join(ROOT, "drama3-mlx_amd"), oracle=os.path.join(ROOT, "oracle"),
                          tests=os.path.join(ROOT, "tests"), inp=str(inp), out=str(out))
    banner("child process with D3_NO_FUSED_SAMPLER=1")
    r = subprocess.run([sys.executable, "-c", script], env=env, cwd=ROOT, timeout=300,
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    got = np.load(out)
    for name in ("c3", "c4", "split"):
        exp = oracle.sample(data[name], data[name + "_u"], float(data[name + "_T"]), data[name + "_p"],
                            op_graph=True)
        assert np.array_equal(got[name + "_ids"], exp["ids"]), name
        assert np.array_equal(got[name + "_cand"], exp["cand"]), name
        both_nan = np.isnan(got[name + "_probs"]) & np.isnan(exp["probs"])
        assert np.array_equal(got[name + "_probs"][~both_nan], exp["probs"][~both_nan]), name
    assert orders_differ(oracle, xs, data["split_u"], 1.0, top_p)
