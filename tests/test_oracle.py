"""The CPU oracle against what pins it without running the reference: the
reference's own float64 closed form (tests/test_decode.py:100-109), brute force,
special cases that reduce to textbook routines, invariants, and the reference's
distribution test restated (tests/test_decode.py:89-114)."""
import numpy as np
import pytest

import closed_form as CF
import d3s_workloads as W


def check_rows(oracle, logits, u, T, top_p, k, banned=None):
    """Oracle vs closed form, row by row.  Returns (n_rows, n_boundary)."""
    out = oracle.sample(logits, u, T, top_p, banned=banned)
    N = logits.shape[0]
    L = W.bf16_bits_to_f32(logits) if logits.dtype == np.uint16 else logits
    n_edge = 0
    for r in range(N):
        row = L[r].copy()
        if banned is not None and banned[r] >= 0:
            row[banned[r]] = -np.inf
        t = T[r] if np.ndim(T) else T
        p = top_p[r] if np.ndim(top_p) else top_p
        cf = CF.row(row, u[r], t, p, k)
        edge = cf["min_gap"] < CF.fp32_tolerance(cf["lse_scale"], k) or cf["race_gap"] < 1e-6
        n_edge += edge
        if edge:
            continue
        kept = cf["kept"]
        assert np.array_equal(out["cand"][r][:kept], cf["cand"][:kept]), r
        assert np.all(out["probs"][r][kept:] == 0), r
        np.testing.assert_allclose(out["probs"][r], cf["probs"], rtol=1e-5, atol=1e-37)
        assert out["ids"][r] == cf["id"], r
        assert abs(out["lse"][r] - cf["lse"]) <= CF.lse_tolerance(cf["lse_scale"]), r
    return N, n_edge


@pytest.mark.parametrize("V,k,T,top_p,dtype", [
    (4097, 30, 0.7, 0.7, "f32"), (4097, 30, 1.0, 0.9, "f32"), (4096, 30, 0.7, 0.7, "bf16"),
    (1024, 5, 1.0, 1.0, "f32"), (4097, 30, 0.3, 0.95, "f32"), (257, 64, 1.3, 0.8, "f32"),
    (300, 1, 0.7, 0.7, "bf16"), (50, 50, 1.0, 0.9, "f32"), (4097, 4097, 1.0, 0.95, "f32"),
    (700, 200, 0.9, 0.99, "bf16"), (2, 2, 1.0, 0.5, "f32"),
])
def test_oracle_matches_closed_form(oracle, V, k, T, top_p, dtype):
    rng = np.random.default_rng([V, k, int(T * 100)])
    N = 24 if V > 1000 else 64
    x = (rng.standard_normal((N, V)) * 2.5).astype(np.float32)
    x[np.arange(N), rng.integers(0, V, N)] += 8
    logits = W.f32_to_bf16_bits(x) if dtype == "bf16" else x
    u = W.uniform_rows(5, V, N, k)
    n, n_edge = check_rows(oracle, logits, u, T, top_p, k)
    assert n_edge <= n // 3


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C4", "C5"])
def test_oracle_matches_closed_form_on_configs(oracle, name):
    rows = {"C1": 64, "C2": 9, "C3": 64, "C4": 8, "C5": 8}[name]
    w = W.make(name, rows=rows, seed=11)
    n, n_edge = check_rows(oracle, w["logits"], w["u"], w["temperature"], w["top_p"], w["k"],
                           w["banned"])
    assert n_edge <= max(1, n // 3)


@pytest.mark.parametrize("V,k", [(65536, 30), (65537, 30), (1000, 64), (1000, 65), (64, 64),
                                 (64, 63), (4097, 30)])
def test_oracle_order_follows_the_reference_routing(oracle, V, k):
    """The cumulative's order: the reference kernel's left-to-right fp32 sum iff
    k <= 64, k < V and V <= 65536 (src/sampling.c:197), else the op graph's,
    modelled as the exact prefix sum rounded once; op_graph=True forces the
    latter (D3_NO_FUSED_SAMPLER).  Checked on rows whose top_p lies where the
    two orders cut at different ranks, against both orders' cumulatives built
    here from the elementwise exp and fixed-point image: the number of kept
    ranks must be the cut of the order the routing names."""
    import order_rows
    rng = np.random.default_rng([V, k, 17])
    N = 8
    x = (rng.standard_normal((N, V)) * 2.5).astype(np.float32)
    x[np.arange(N), rng.integers(0, V, N)] += 6.0
    kk = min(k, V)
    top_p = order_rows.split_top_p(oracle, x, 1.0, kk)
    split = ~np.isnan(top_p)
    assert split.sum() >= 3
    top_p = np.where(split, top_p, 0.9).astype(np.float32)
    u = W.uniform_rows(17, 0, N, kk)
    default = oracle.sample(x, u, 1.0, top_p)
    forced = oracle.sample(x, u, 1.0, top_p, op_graph=True)
    kernel = k <= 64 and k < V and V <= 65536
    for r in np.nonzero(split)[0]:
        seq, ex = order_rows.cumulatives(oracle, x[r], default["lse"][r], kk)
        cut = lambda c: next((j for j in range(1, kk) if c[j] > top_p[r]), kk)
        assert cut(seq) != cut(ex)
        assert np.count_nonzero(default["probs"][r]) == (cut(seq) if kernel else cut(ex)), r
        assert np.count_nonzero(forced["probs"][r]) == cut(ex), r


def test_brute_force_tiny_rows(oracle):
    """Every row of V <= 6 with values on a small grid (many ties), every k."""
    rng = np.random.default_rng(4)
    for V in range(1, 7):
        for k in range(1, V + 1):
            x = rng.integers(-2, 3, (40, V)).astype(np.float32)
            u = rng.random((40, k)).astype(np.float32)
            check_rows(oracle, x, u, 1.0, 0.6, k)


def test_ties_take_the_lowest_ids(oracle):
    """Restates tests/test_decode.py:73-86: integer-valued logits tie across the
    k-th place; the kept candidates are the lowest ids, as a stable sort's."""
    rng = np.random.default_rng(1)
    for V, k in [(4097, 30), (1024, 30), (4097, 5)]:
        logits = np.round(rng.standard_normal((8, V)) * 2).astype(np.float32)
        u = W.uniform_rows(3, 0, 8, k)
        out = oracle.sample(logits, u, 1.0, 2.0)
        for r in range(8):
            order = np.argsort(-logits[r], kind="stable")[:k]
            assert np.array_equal(out["cand"][r], order)
        again = oracle.sample(logits, u, 1.0, 2.0)
        assert np.array_equal(out["ids"], again["ids"])


def test_top_k_1_is_argmax(oracle):
    rng = np.random.default_rng(5)
    x = np.round(rng.standard_normal((50, 999)) * 3).astype(np.float32)
    out = oracle.sample(x, rng.random((50, 1)).astype(np.float32), 0.7, 0.7)
    assert np.array_equal(out["ids"], np.argmax(x, axis=1))  # first maximum
    assert np.all(out["probs"] == 1.0)


def test_top_p_at_least_one_is_pure_top_k_softmax(oracle):
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((20, 500)) * 2).astype(np.float32)
    k = 17
    out = oracle.sample(x, rng.random((20, k)).astype(np.float32), 1.0, 1.5)
    for r in range(20):
        v = np.sort(x[r])[::-1][:k].astype(np.float64)
        p = np.exp(v - v[0])
        np.testing.assert_allclose(out["probs"][r], p / p.sum(), rtol=1e-5)


def test_all_equal_row_keeps_lowest_ids(oracle):
    x = np.full((3, 100), 1.5, np.float32)
    out = oracle.sample(x, np.full((3, 10), 0.5, np.float32), 1.0, 2.0)
    assert np.all(out["cand"] == np.arange(10))
    np.testing.assert_allclose(out["probs"], 0.1, rtol=1e-6)
    assert np.all(out["ids"] == 0)  # equal scores: the first rank wins


def test_zero_uniform_gives_minus_inf_score(oracle):
    """u = 0 makes noise -0 and the score -inf (src/sampling.c:135-137): such a
    rank never wins while another has a positive score."""
    x = np.array([[5.0, 4.0, 3.0, -50.0]], np.float32)
    u = np.array([[0.0, 0.5, 0.5, 0.5]], np.float32)
    out = oracle.sample(x, u, 1.0, 2.0)
    assert out["ids"][0] == 1
    u = np.zeros((1, 4), np.float32)
    out = oracle.sample(x, u, 1.0, 2.0)
    assert out["ids"][0] == 0  # every score NaN or -inf: the initial choice 0


def test_temperature_clamp_and_k_clamp(oracle):
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((10, 300))).astype(np.float32)
    u = rng.random((10, 30)).astype(np.float32)
    a = oracle.sample(x, u, 0.0, 0.7)
    b = oracle.sample(x, u, 1e-5, 0.7)
    c = oracle.sample(x, u, -3.0, 0.7)
    assert np.array_equal(a["ids"], b["ids"]) and np.array_equal(a["ids"], c["ids"])
    assert np.array_equal(a["ids"], np.argmax(x, axis=1))  # T -> 1e-5 concentrates on the max


def test_non_finite_rows_are_refused(oracle):
    x = np.zeros((4, 64), np.float32)
    x[0, 3] = np.nan
    x[1, 5] = np.inf
    x[2, :] = -np.inf
    x[3, 7] = 2.0
    out = oracle.sample(x, np.full((4, 8), 0.5, np.float32), 1.0, 0.9)
    assert out["ids"][0] == -1 and out["ids"][1] == -1
    assert out["flags"][0] & oracle.BAD and out["flags"][1] & oracle.BAD
    assert out["ids"][2] == 0 and out["flags"][2] & oracle.ALL_MASKED
    assert np.array_equal(out["cand"][2], np.arange(8))
    assert out["ids"][3] == 7


def test_finite_logit_overflowing_after_temperature_is_refused(oracle):
    """The refusal rule is on x = L / T, not on L (a deliberate deviation: the
    reference's generation loop dies on any non-finite logit, -inf included,
    src/generate.c:91,123, and never on finite ones): a finite logit whose x
    overflows to +inf refuses the row; the same row at T = 1 does not; -inf
    logits are masked, not refused."""
    x = np.zeros((3, 64), np.float32)
    x[:, 9] = 3e38
    x[2, 4] = -np.inf
    u = np.full((3, 8), 0.5, np.float32)
    T = np.array([0.7, 1.0, 1.0], np.float32)
    out = oracle.sample(x, u, T, 0.9)
    assert out["ids"][0] == -1 and out["flags"][0] & oracle.BAD
    assert out["ids"][1] == 9 and out["ids"][2] == 9
    assert not (out["flags"][1] & oracle.BAD) and not (out["flags"][2] & oracle.BAD)


def test_banned_index_and_minus_inf_entries(oracle):
    rng = np.random.default_rng(8)
    x = (rng.standard_normal((16, 200)) * 0.3).astype(np.float32)
    x[:, 0] = 10.0
    banned = np.where(np.arange(16) % 2 == 0, 0, -1).astype(np.int32)
    u = rng.random((16, 200)).astype(np.float32)
    out = oracle.sample(x, u, 1.0, 0.95, banned=banned)
    assert np.all(out["ids"][banned == 0] != 0)
    assert np.all(out["cand"][banned == 0][:, -1] == 0)  # -inf ranks last
    assert np.all(out["ids"][banned == -1] == 0)  # p(0) ~ 1 otherwise


def test_lse_is_order_independent(oracle):
    """The exact fixed-point row sum: permuting the row never changes lse."""
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((1, 5000)) * 4).astype(np.float32)
    u = rng.random((1, 1)).astype(np.float32)
    base = oracle.sample(x, u, 0.8, 0.9)["lse"][0]
    for _ in range(5):
        y = x[:, rng.permutation(5000)]
        assert oracle.sample(y, u, 0.8, 0.9)["lse"][0] == base


def test_per_row_parameters(oracle):
    w = W.make("C3", rows=16, seed=3)
    out = oracle.sample(w["logits"], w["u"], w["temperature"], w["top_p"])
    for r in (0, 15):
        one = oracle.sample(w["logits"][r:r + 1], w["u"][r:r + 1], float(w["temperature"][r]),
                            float(w["top_p"][r]))
        assert one["ids"][0] == out["ids"][r]
        assert np.array_equal(one["probs"][0], out["probs"][r])


def test_row_stride(oracle):
    rng = np.random.default_rng(10)
    x = (rng.standard_normal((6, 130)) * 2).astype(np.float32)
    u = rng.random((6, 9)).astype(np.float32)
    a = oracle.sample(x[:, :100].copy(), u, 0.9, 0.8)
    b = oracle.sample(x, u, 0.9, 0.8, row_stride=130, vocab=100)
    assert np.array_equal(a["ids"], b["ids"]) and np.array_equal(a["probs"], b["probs"])


@pytest.mark.parametrize("temperature,top_k,top_p",
                         [(0.7, 30, 0.7), (1.0, 30, 0.9), (1.0, 5, 1.0), (0.3, 30, 0.95)])
def test_distribution(oracle, temperature, top_k, top_p):
    """Restates tests/test_decode.py:89-114 with this build's uniforms: 4000
    draws, frequencies within 4 sigma + 1e-3 of the closed-form probabilities."""
    rng = np.random.default_rng(0)
    logits = (rng.standard_normal((1, 4097)) * 3).astype(np.float32)
    n = 4000
    u = W.uniform_rows(0, 0, n, top_k)
    out = oracle.sample(np.repeat(logits, n, axis=0), u, temperature, top_p)
    ours = out["ids"]
    cf = CF.row(logits[0], u[0], temperature, top_p, top_k)
    expected = dict(zip(cf["cand"][:cf["kept"]], cf["probs"][:cf["kept"]]))
    for token, prob in expected.items():
        freq = np.mean(ours == token)
        assert abs(freq - prob) < 4 * np.sqrt(prob * (1 - prob) / n) + 1e-3, (token, freq, prob)
    assert set(np.unique(ours)) <= set(expected)
