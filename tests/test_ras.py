"""Repetition-aware sampling of the main token (src/tower.c:13-16,:405-433):
the oracle's selection against known answers, the C-ABI's argument checks, and
(on the GPU) the fused two-draw kernel against the oracle's two draws.

The token map's ids are illustrative (the model's config files are not in the
reference's sources); the band has the backbone head's shape: candidate index
0 is eos and 1..4096 are the semantic codes (lm_head_audio [1 + code_vocab,
hidden], src/model.h:71)."""
import numpy as np
import pytest

import d3s_workloads as W

EOS, START, CODES = 151645, 151669, 4096
END = START + CODES - 1
MAP = dict(eos_id=EOS, semantic_start=START, semantic_end=END, code_vocab=CODES)


@pytest.fixture(scope="module")
def gpu():
    import d3s
    import hiprt
    d3s.lib()
    if hiprt.device_count() < 1:
        pytest.skip("no GPU")
    return d3s


def test_selection_known_answers(oracle):
    """Each case follows from src/tower.c:405-409 and :425-433 by hand."""
    first = np.array([0, 5, 5, 5, -1, 4096, 1, 3], np.int32)
    retry = np.array([7, 9, 9, 0, 3, 2, 2, 8], np.int32)
    hist = np.full((8, 3), -7, np.int32)
    hist[0] = EOS                   # eos repeated: a stop is never redrawn
    hist[1, 2] = START + 4          # token(5) seen: the retry's token
    hist[3, 0] = START + 4          # seen, and the retry is eos
    hist[4, :] = START - 2          # token(-1) = START - 2 is not semantic
    hist[5, 1] = END                # the last code, seen
    hist[6, 0] = START              # the first code, seen
    main, code0 = oracle.ras_select(first, retry, hist, EOS, START, END, CODES)
    # row 4: the first draw was refused (non-finite logits): -1 for both outputs
    assert main.tolist() == [EOS, START + 8, START + 4, EOS, -1, START + 1, START + 1, START + 2]
    assert code0.tolist() == [0, 8, 4, 0, -1, 1, 1, 2]  # eos lies below the band: clipped to 0
    # no history: the first draw always stands
    main0, _ = oracle.ras_select(first, retry, np.zeros((8, 0), np.int32), EOS, START, END, CODES)
    ok = first >= 0
    assert np.array_equal(main0[ok], np.where(first == 0, EOS, first + START - 1)[ok])
    # a refused retry refuses the row too, repeated or not
    m2, c2 = oracle.ras_select(np.array([5, 5], np.int32), np.array([-1, -1], np.int32),
                               np.array([[START + 4], [7]], np.int32), EOS, START, END, CODES)
    assert m2.tolist() == [-1, -1] and c2.tolist() == [-1, -1]


def test_ras_argument_validation_without_device():
    import d3s
    p = 16  # never dereferenced: every call below fails validation or launches nothing
    P = d3s.ras_params(temperature=0.7, top_p=0.7, top_k=30, **MAP)
    base = dict(logits=p, dtype=1, n_rows=1, vocab=4097, row_stride=4097, u=p, u_retry=p,
                history=None, history_len=0, params=P, main_tok=p)
    assert d3s.sample_ras_raw(**{**base, "params": None}) == -1
    assert d3s.sample_ras_raw(**{**base, "dtype": 3}) == -4
    assert d3s.sample_ras_raw(**{**base, "history_len": 65, "history": p}) == -1
    assert d3s.sample_ras_raw(**{**base, "history_len": 4}) == -1  # history missing
    assert d3s.sample_ras_raw(**{**base, "main_tok": None}) == -1
    assert d3s.sample_ras_raw(**{**base, "row_stride": 4096}) == -1
    bad_k = d3s.ras_params(temperature=0.7, top_p=0.7, top_k=0, **MAP)
    assert d3s.sample_ras_raw(**{**base, "params": bad_k}) == -1
    assert d3s.sample_ras_raw(**{**base, "n_rows": 0}) == 0


def _case(oracle, name, rows, seed, top_k=30, temperature=0.7, top_p=0.7, H=16, repeat_every=2):
    """Rows of config `name`, both draws' uniforms, and a history that holds
    the first draw's token on every `repeat_every`-th row."""
    w = W.make(name, rows=rows, seed=seed, uniforms=False)
    x = w["logits"]
    V = x.shape[1]
    k, k2 = min(top_k, V), min(30, V)
    u = oracle.uniform(seed, 0, rows, k)
    u2 = oracle.uniform(seed, 1, rows, k2)
    first = oracle.sample(x, u, temperature, top_p, n_threads=8)["ids"]
    tok = np.where(first == 0, EOS, first + START - 1)
    rng = np.random.default_rng(seed)
    hist = rng.integers(START, END + 1, (rows, H)).astype(np.int32)
    rep = np.arange(rows) % repeat_every == 0
    if H:
        hist[rep, rng.integers(0, H, rep.sum())] = tok[rep]
    params = dict(temperature=temperature, top_p=top_p, top_k=top_k, **MAP)
    return x, u, u2, hist, params


def _check(oracle, gpu, x, u, u2, hist, params, indices=True):
    exp = oracle.ras(x, u, u2, params, hist, n_threads=8)
    got = gpu.sample_ras(x, u, u2, params, hist, indices=indices)
    assert got["rc"] == 0, got["rc"]
    for name in ("first", "retry", "main", "code0") if indices else ("main", "code0"):
        bad = np.nonzero(got[name] != exp[name])[0]
        assert len(bad) == 0, (name, bad[:8], got[name][bad[:8]], exp[name][bad[:8]])
    return got, exp


@pytest.mark.gpu
@pytest.mark.parametrize("name,rows", [("C1", 1), ("C1", 300), ("C1", 2000), ("C2", 9), ("C3", 256)])
def test_ras_fused_equals_two_draws(gpu, oracle, name, rows):
    x, u, u2, hist, params = _case(oracle, name, rows, seed=21 + rows)
    got, exp = _check(oracle, gpu, x, u, u2, hist, params)
    # the case exercises both outcomes
    if rows >= 256:
        assert np.any(exp["main"] != np.where(exp["first"] == 0, EOS, exp["first"] + START - 1))
        assert np.any(exp["main"] == np.where(exp["first"] == 0, EOS, exp["first"] + START - 1))


@pytest.mark.gpu
def test_ras_bf16_head_and_parameters(gpu, oracle):
    """The tower's backbone head: bf16 [1, 4097] rows (src/tower.c:420-433), with
    several first-draw parameters, no history and the longest history."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((64, 4097)) * 2.5).astype(np.float32)
    x[np.arange(64), rng.integers(0, 4097, 64)] += 6.0
    xb = W.f32_to_bf16_bits(x)
    for top_k, T, top_p, H in [(30, 0.7, 0.7, 16), (5, 1.3, 0.9, 0), (64, 0.3, 1.0, 64), (1, 0.7, 0.7, 16)]:
        k = top_k
        u = oracle.uniform(7, 0, 64, k)
        u2 = oracle.uniform(7, 1, 64, 30)
        first = oracle.sample(xb, u, T, top_p)["ids"]
        hist = np.full((64, H), START, np.int32)
        if H:
            hist[::2, -1] = np.where(first[::2] == 0, EOS, first[::2] + START - 1)
        _check(oracle, gpu, xb, u, u2, hist, dict(temperature=T, top_p=top_p, top_k=top_k, **MAP))


@pytest.mark.gpu
@pytest.mark.parametrize("indices", [True, False])
def test_ras_rows_beyond_the_wave_kernel(gpu, oracle, indices):
    """What the fused launch does not hold runs as two routed draws and a pick
    (the reference draws both for any top_k >= 1 and any head width,
    src/tower.c:425-433, src/main.c:165): top_k 100 for either draw, fp32 rows
    of 20000 and bf16 rows of 151936.  Without the index outputs the first
    draw's indices pass through main_tok and the retry's through the library's
    workspace."""
    rng = np.random.default_rng(23)
    cases = []
    x = (rng.standard_normal((64, 4097)) * 2.5).astype(np.float32)
    x[np.arange(64), rng.integers(0, 4097, 64)] += 6.0
    cases.append((x, 100, 30))
    cases.append((x, 30, 100))
    w = (rng.standard_normal((8, 20000)) * 2.5).astype(np.float32)
    w[np.arange(8), rng.integers(0, 20000, 8)] += 8.0
    cases.append((w, 30, 30))
    c4 = W.make("C4", rows=4, seed=23, uniforms=False)["logits"]
    cases.append((c4, 30, 30))
    for xs, top_k, retry_top_k in cases:
        N, V = xs.shape
        k, k2 = min(top_k, V), min(retry_top_k, V)
        u = oracle.uniform(23, 0, N, k)
        u2 = oracle.uniform(23, 1, N, k2)
        first = oracle.sample(xs, u, 0.7, 0.7, n_threads=8)["ids"]
        hist = rng.integers(START, END + 1, (N, 16)).astype(np.int32)
        hist[::2, 3] = np.where(first[::2] == 0, EOS, first[::2] + START - 1)
        params = dict(temperature=0.7, top_p=0.7, top_k=top_k, retry_top_k=retry_top_k, **MAP)
        print(f"[ras] fallback V={V} top_k={top_k} retry_top_k={retry_top_k} indices={indices}", flush=True)
        _check(oracle, gpu, xs, u, u2, hist, params, indices=indices)


@pytest.mark.gpu
def test_ras_refused_rows_signal(gpu, oracle):
    """A row whose logits hold a NaN or +inf, or whose finite logits overflow
    at the first draw's temperature only: main_tok = code0 = -1 (the caller's
    check, where the reference's generation loop dies, src/generate.c:92,130),
    on the fused launch and on the fallback; the other rows as the oracle's."""
    rng = np.random.default_rng(29)
    x = (rng.standard_normal((8, 4097)) * 2.5).astype(np.float32)
    x[1, 100] = np.nan
    x[3, 4096] = np.inf
    x[5, 7] = 3e38  # x = 3e38 / 0.7 overflows; the retry's T = 1.0 does not
    u = oracle.uniform(29, 0, 8, 30)
    u2 = oracle.uniform(29, 1, 8, 30)
    hist = np.full((8, 16), START, np.int32)
    for top_k in (30, 100):
        uk = oracle.uniform(29, 0, 8, top_k)
        params = dict(temperature=0.7, top_p=0.7, top_k=top_k, **MAP)
        got, exp = _check(oracle, gpu, x, uk if top_k > 30 else u, u2, hist, params)
        for r in (1, 3, 5):
            assert got["main"][r] == -1 and got["code0"][r] == -1, (top_k, r)
        assert np.all(got["main"][[0, 2, 4, 6, 7]] >= 0)
        assert got["retry"][5] >= 0  # the retry alone was not refused
        assert got["counters"][gpu.COUNTER_REFUSED] == 5  # rows 1 and 3 twice, row 5 once


@pytest.mark.gpu
def test_frame_assembled_in_place(gpu, oracle):
    """A decode step's frame [main, code0, code_1 .. code_9] (src/tower.c:420-451)
    written in place on the device: d3s_sample_ras into frame[0..1], then each
    codebook head's d3s_sample into frame[2 + j]."""
    import hiprt
    rng = np.random.default_rng(17)
    head = W.f32_to_bf16_bits((rng.standard_normal((1, 4097)) * 2.5).astype(np.float32))
    books = [W.make("C2", rows=9, seed=17, uniforms=False)["logits"][j:j + 1] for j in range(9)]
    u0, u1 = oracle.uniform(17, 0, 1, 30), oracle.uniform(17, 1, 1, 30)
    uj = [oracle.uniform(17, 2 + j, 1, 30) for j in range(9)]
    first = oracle.sample(head, u0, 0.7, 0.7)["ids"]
    hist = np.array([[first[0] + START - 1 if first[0] else EOS] * 4 + [START] * 12], np.int32)
    params = dict(temperature=0.7, top_p=0.7, top_k=30, **MAP)
    exp = oracle.ras(head, u0, u1, params, hist)
    expected = [exp["main"][0], exp["code0"][0]] + [oracle.sample(books[j], uj[j], 0.7, 0.7)["ids"][0]
                                                    for j in range(9)]
    frame = hiprt.DeviceBuffer(4 * 11)
    dh, d0, d1, dhist = (hiprt.to_device(head), hiprt.to_device(u0), hiprt.to_device(u1),
                         hiprt.to_device(hist))
    rc = gpu.sample_ras_raw(dh.ptr, gpu.DTYPE_BF16, 1, 4097, 4097, d0.ptr, d1.ptr, dhist.ptr, 16,
                            gpu.ras_params(**params), frame.ptr, frame.ptr + 4)
    assert rc == 0
    keep = []
    for j in range(9):
        db, du = hiprt.to_device(books[j]), hiprt.to_device(uj[j])
        keep += [db, du]
        assert gpu.sample_raw(db.ptr, gpu.DTYPE_BF16, 1, 4096, 4096, du.ptr, 30, 0.7, 0.7, None,
                              frame.ptr + 4 * (2 + j)) == 0
    hiprt.synchronize()
    assert frame.download((11,), np.int32).tolist() == [int(v) for v in expected]


@pytest.mark.gpu
def test_fallback_workspace_leaves_the_segment_counters(gpu, oracle):
    """The fallback's retry indices live in the stream's workspace; a later
    launch of the segmented kernel on the same stream (whose arrival counters
    open that workspace) still samples every row right."""
    rng = np.random.default_rng(31)
    x = (rng.standard_normal((64, 4097)) * 2.5).astype(np.float32)
    u = oracle.uniform(31, 0, 64, 100)
    u2 = oracle.uniform(31, 1, 64, 30)
    hist = np.full((64, 16), START, np.int32)
    _check(oracle, gpu, x, u, u2, hist, dict(temperature=0.7, top_p=0.7, top_k=100, **MAP), indices=False)
    w = W.make("C4", rows=8, seed=31, uniforms=False)
    uc = oracle.uniform(31, 2, 8, 30)
    got = gpu.sample(w["logits"], uc, 1.0, 0.9, want_probs=False)
    assert np.array_equal(got["ids"], oracle.sample(w["logits"], uc, 1.0, 0.9, n_threads=8)["ids"])
