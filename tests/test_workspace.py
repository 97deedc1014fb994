"""The caller's workspace: d3s_sample_ws, d3s_sample_ras_ws and
d3s_linear_sample_bf16_ws take their device state from memory the caller
sized with the *_workspace_bytes queries, allocated once and cleared once with
d3s_workspace_init, and never allocate (the raw core's contract: workspace
preallocated per context, as the reference sets its kernel up once,
src/sampling.c:142-157).

CPU: the size queries and the refusals (a workspace too small, rows beyond
D3S_MAX_VOCAB) return before anything reaches the device.
GPU: one HIP graph holding a C4 call (the segmented kernel), a C5 ids-only
call (the nucleus kernel's two launches) and a k = V row of 20 000 (the
sorting kernels) on one workspace, with no memset, copy or allocation node,
replayed five times with new uniforms and the program's eager work between
replays, every replay's ids equal to the oracle's; every *_ws entry point
against its counterpart that takes the library's per-stream block (the same
bits); and the release of a stream's block."""
import ctypes

import numpy as np
import pytest

import d3s_workloads as W

EOS, START, CODES = 151645, 151669, 4096
MAP = dict(eos_id=EOS, semantic_start=START, semantic_end=START + CODES - 1, code_vocab=CODES)


@pytest.fixture(scope="module")
def lib():
    import d3s
    return d3s


@pytest.fixture(scope="module")
def gpu():
    import d3s
    import hiprt
    d3s.lib()
    if hiprt.device_count() < 1:
        pytest.skip("no GPU")
    return d3s


def banner(msg):
    print(f"[workspace] {msg}", flush=True)


# ---------------------------------------------------------------- CPU

def test_size_queries(lib):
    """0 where the route keeps nothing on the device (one-wave rows, the
    nucleus kernel's full path needs none, the fused draw), more where it
    does; the same status codes as the calls for bad arguments."""
    L = lib.lib()
    f32, bf16 = lib.DTYPE_F32, lib.DTYPE_BF16
    assert lib.workspace_bytes(f32, 256, 4097, 30) == 0          # C3: one wave per row
    assert lib.workspace_bytes(f32, 1, 4097, 30) == 0            # C1
    c4 = lib.workspace_bytes(bf16, 64, 151936, 30)               # C4: segment records and counters
    assert c4 >= 256 * 1024 + 64 * 2 * 66 * 8 and c4 % 256 == 0
    c5 = lib.workspace_bytes(f32, 4096, 4097, 4097)              # C5 ids: counters and filed rows
    assert c5 >= 256 * 1024 + 4096 * 4
    big = lib.workspace_bytes(f32, 1, 20000, 20000)              # sorting: keys after the counters
    assert big >= 256 * 1024 + 2 * 20000 * 8
    assert lib.workspace_bytes(f32, 0, 4097, 30) == 0
    assert lib.workspace_bytes(f32, 64, 151936, 30, lib.FLAG_GENERIC) == 0  # the streaming kernel
    assert lib.workspace_bytes(7, 1, 10, 3) == -4
    assert lib.workspace_bytes(f32, 1, 10, 11) == -1
    assert lib.workspace_bytes(f32, 1, 10, 3, 64) == -1
    assert lib.workspace_bytes(f32, 1, lib.MAX_VOCAB + 1, 3) == -2
    assert lib.workspace_bytes(f32, 1, lib.MAX_VOCAB, 3) == 0
    P = lib.ras_params(temperature=0.7, top_p=0.7, top_k=30, **MAP)
    assert L.d3s_sample_ras_workspace_bytes(bf16, 1, 4097, ctypes.byref(P), 0) == 0  # one launch
    P100 = lib.ras_params(temperature=0.7, top_p=0.7, top_k=100, **MAP)
    assert L.d3s_sample_ras_workspace_bytes(f32, 64, 4097, ctypes.byref(P100), 1) == 0
    idx = L.d3s_sample_ras_workspace_bytes(f32, 64, 4097, ctypes.byref(P100), 0)
    assert idx >= 256 * 1024 + 64 * 4  # the retry's indices, past the counters
    assert L.d3s_sample_ras_workspace_bytes(f32, 4, 151936, ctypes.byref(P), 1) > 256 * 1024  # segmented
    assert L.d3s_sample_ras_workspace_bytes(f32, 1, 10, None, 1) == -1
    assert L.d3s_linear_sample_workspace_bytes(1, 2048, 4097, 30, 0, 1) == 0
    y_ws = L.d3s_linear_sample_workspace_bytes(1, 2048, 4097, 30, 0, 0)
    assert y_ws >= 256 * 1024 + 4097 * 2
    one = L.d3s_linear_sample_workspace_bytes(1, 2048, 4097, 30, lib.FLAG_ONE_LAUNCH, 1)
    assert one > 0
    assert L.d3s_linear_sample_workspace_bytes(1, 100, 4097, 30, 0, 1) == -1  # K % 128


def test_refusals_before_the_device(lib):
    """A workspace smaller than the call needs: D3S_ERR_WORKSPACE; one
    misaligned: D3S_ERR_ARG; a row wider than D3S_MAX_VOCAB:
    D3S_ERR_UNSUPPORTED (its exact row sum could wrap).  Nothing is launched
    (the pointers are never dereferenced)."""
    p = 1 << 20
    f32, bf16 = lib.DTYPE_F32, lib.DTYPE_BF16
    need = lib.workspace_bytes(bf16, 64, 151936, 30)
    base = dict(logits=p, dtype=bf16, n_rows=64, vocab=151936, row_stride=151936, u=p, k=30,
                temperature=1.0, top_p=0.9, banned=None, ids=p)
    assert lib.sample_raw(**base, workspace=(p, need - 256)) == lib.ERR_WORKSPACE
    assert lib.sample_raw(**base, workspace=(None, 0)) == lib.ERR_WORKSPACE
    assert lib.sample_raw(**base, workspace=(p + 64, need)) == lib.ERR_ARG
    assert lib.sample_raw(**base, workspace=(p, -1)) == lib.ERR_ARG
    wide = dict(base, dtype=f32, vocab=lib.MAX_VOCAB + 1, row_stride=lib.MAX_VOCAB + 1, n_rows=1)
    assert lib.sample_raw(**wide) == lib.ERR_UNSUPPORTED
    assert lib.sample_raw(**wide, noalloc=True) == lib.ERR_UNSUPPORTED
    assert lib.sample_raw(**wide, workspace=(p, 1 << 30)) == lib.ERR_UNSUPPORTED
    L = lib.lib()
    assert L.d3s_workspace_init(p + 4, 256, None) == lib.ERR_ARG
    assert L.d3s_workspace_init(p, 6, None) == lib.ERR_ARG
    assert L.d3s_workspace_init(None, 0, None) == 0
    P = lib.ras_params(temperature=0.7, top_p=0.7, top_k=100, **MAP)
    need = L.d3s_sample_ras_workspace_bytes(f32, 64, 4097, ctypes.byref(P), 0)
    assert L.d3s_sample_ras_ws(p, f32, 64, 4097, 4097, p, p, None, 0, ctypes.byref(P), p, None, None, None,
                               None, p, need - 256, None) == lib.ERR_WORKSPACE
    need = L.d3s_linear_sample_workspace_bytes(1, 2048, 4097, 30, 0, 0)
    assert L.d3s_linear_sample_bf16_ws(p, p, 1, 2048, 4097, None, p, 30, None, None, 0.7, 0.7, p, None, None,
                                       None, 0, p, need - 256, None) == lib.ERR_WORKSPACE


def test_flat_row_at_the_vocab_limit(oracle):
    """The widest row taken, all logits equal: the exact row sum holds
    (2^24 - 1) * 2^40 without wrapping, so lse = x + log V as float64 gives it,
    the top 30 are indices 0..29 (ties by index) with probability 1/30; one
    element more is refused (its sum would be 2^64, which wraps to 0)."""
    V = (1 << 24) - 1
    x = np.full((1, V), 1.25, np.float32)
    u = oracle.uniform(3, 0, 1, 30)
    r = oracle.sample(x, u, 1.0, 0.9, n_threads=8)
    assert abs(float(r["lse"][0]) - (1.25 + np.log(V))) <= 4 * np.spacing(np.float32(1.25 + np.log(V)))
    assert r["cand"][0].tolist() == list(range(30))
    assert np.allclose(r["probs"][0], 1 / 30, rtol=1e-6)
    with pytest.raises(ValueError):
        oracle.sample(np.zeros((1, V + 1), np.float32), u, 1.0, 0.9)


# ---------------------------------------------------------------- GPU

def _device_call(hiprt, x, k, T, top_p, banned=None):
    d = dict(x=x, N=x.shape[0], V=x.shape[1], k=k, T=T, top_p=top_p, banned=banned,
             dt=0 if x.dtype == np.float32 else 1)
    d["bx"] = hiprt.to_device(x)
    d["bu"] = hiprt.DeviceBuffer(4 * d["N"] * k)
    d["ids"] = hiprt.DeviceBuffer(4 * d["N"])
    d["ban"] = hiprt.to_device(banned) if banned is not None else None
    return d


def _enqueue(gpu, c, ws, stream, ids=None):
    return gpu.sample_raw(c["bx"].ptr, c["dt"], c["N"], c["V"], c["V"], c["bu"].ptr, c["k"], c["T"], c["top_p"],
                          c["ban"].ptr if c["ban"] else None, (ids or c["ids"]).ptr, stream=stream.ptr,
                          workspace=ws.arg())


@pytest.mark.gpu
def test_graph_of_three_routes_on_one_workspace(gpu, oracle):
    """C4 (k_split), C5 ids only (k_topp_ids + k_topp_redo) and one k = V row
    of 20 000 (the sorting kernels) captured into one HIP graph with a
    preallocated workspace: kernel nodes only (no memset, copy or allocation),
    replayed five times, each time with new uniforms (uploaded eagerly) and an
    eager C4 call on the same workspace between replays; every replay's ids
    equal the oracle's."""
    import hiprt
    H = hiprt.hip()
    c4 = W.make("C4", seed=81, uniforms=False)
    c5 = W.make("C5", seed=82, uniforms=False)
    rng = np.random.default_rng(83)
    big = (rng.standard_normal((1, 20000)) * 2.0).astype(np.float32)
    calls = [_device_call(hiprt, c4["logits"], 30, 1.0, 0.9),
             _device_call(hiprt, c5["logits"], 4097, 1.0, 0.95, c5["banned"]),
             _device_call(hiprt, big, 20000, 1.0, 0.9)]
    need = max(gpu.workspace_bytes(c["dt"], c["N"], c["V"], c["k"]) for c in calls)
    banner(f"graph: workspace {need} B")
    s = hiprt.Stream()
    ws = gpu.Workspace(need, s)
    eager_ids = hiprt.DeviceBuffer(4 * 64)
    s.synchronize()
    graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
    hiprt.check(H.hipStreamBeginCapture(s.ptr, 0), "begin capture")
    rcs = [_enqueue(gpu, c, ws, s) for c in calls]
    hiprt.check(H.hipStreamEndCapture(s.ptr, ctypes.byref(graph)), "end capture")
    try:
        assert rcs == [0, 0, 0], rcs
        types = hiprt.graph_node_types(graph)
        banner(f"graph nodes: {len(types)} ({sorted(set(types))})")
        assert types and all(t == "kernel" for t in types), types
        assert len(types) >= 1 + 2 + 6
        hiprt.check(H.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0), "instantiate")
        for rep in range(5):
            us = []
            for i, c in enumerate(calls):
                u = oracle.uniform(90 + rep, 100 * i, c["N"], c["k"])
                c["bu"].upload(u)
                us.append(u)
            # the program's own eager work between replays, on the same workspace
            assert _enqueue(gpu, calls[0], ws, s, ids=eager_ids) == 0
            s.synchronize()
            hiprt.check(H.hipGraphLaunch(exe, s.ptr), "graph launch")
            s.synchronize()
            for c, u in zip(calls, us):
                exp = oracle.sample(c["x"], u, c["T"], c["top_p"], banned=c["banned"], n_threads=8,
                                    detail=False)["ids"]
                got = c["ids"].download((c["N"],), np.int32)
                bad = np.nonzero(got != exp)[0]
                banner(f"replay {rep}: [{c['N']}, {c['V']}] k={c['k']} mismatched={len(bad)}")
                assert len(bad) == 0, (rep, c["V"], bad[:8], got[bad[:8]], exp[bad[:8]])
            assert np.array_equal(eager_ids.download((64,), np.int32), calls[0]["ids"].download((64,), np.int32))
    finally:
        if exe.value:
            H.hipGraphExecDestroy(exe)
        H.hipGraphDestroy(graph)
        s.destroy()
        ws.free()


ROUTES = [("C3 one wave", "C3"), ("C4 segmented", "C4"), ("C5 nucleus", "C5"),
          ("wide fp32 segmented", "wide"), ("k = V sorting", "bigk"), ("k 100 nucleus", "k100")]


def _route_case(oracle, name):
    rng = np.random.default_rng(91)
    if name in ("C3", "C4", "C5"):
        w = W.make(name, rows={"C3": 256, "C4": 64, "C5": 512}[name], seed=91, uniforms=False)
        return w["logits"], w["k"], w["temperature"], w["top_p"], w["banned"]
    if name == "wide":
        return (rng.standard_normal((24, 100000)) * 3).astype(np.float32), 30, 0.8, 0.9, None
    if name == "bigk":
        return (rng.standard_normal((3, 17000)) * 2).astype(np.float32), 17000, 1.0, 0.9, None
    return (rng.standard_normal((32, 4097)) * 2).astype(np.float32), 100, 1.0, 0.9, None


@pytest.mark.gpu
@pytest.mark.parametrize("label,name", ROUTES)
@pytest.mark.parametrize("want_probs", [False, True])
def test_ws_equals_the_stream_block(gpu, oracle, label, name, want_probs):
    """d3s_sample_ws on a caller's workspace against d3s_sample on the
    library's block: every id (and probability and candidate) equal, and the
    oracle's ids."""
    x, k, T, top_p, banned = _route_case(oracle, name)
    N, V = x.shape
    u = oracle.uniform(92, 0, N, k)
    need = gpu.workspace_bytes(0 if x.dtype == np.float32 else 1, N, V, k)
    ws = gpu.Workspace(need)
    banner(f"{label}: [{N}, {V}] k={k} workspace {need} B probs={want_probs}")
    a = gpu.sample(x, u, T, top_p, banned=banned, want_probs=want_probs)
    b = gpu.sample(x, u, T, top_p, banned=banned, want_probs=want_probs, workspace=ws)
    ws.free()
    assert a["rc"] == 0 and b["rc"] == 0, (a["rc"], b["rc"])
    for key in ("ids", "cand", "counters") if want_probs else ("ids", "counters"):
        assert np.array_equal(a[key], b[key]), key
    if want_probs:
        assert np.array_equal(a["probs"].view(np.uint32), b["probs"].view(np.uint32))
    exp = oracle.sample(x, u, T, top_p, banned=banned, n_threads=8, detail=False)["ids"]
    assert np.array_equal(b["ids"], exp)


@pytest.mark.gpu
@pytest.mark.parametrize("top_k,V,outs", [(30, 4097, "none"), (100, 4097, "none"), (100, 4097, "code0"),
                                          (30, 20000, "none"), (30, 151936, "retry")])
def test_ras_ws_equals_the_stream_block(gpu, oracle, top_k, V, outs):
    """d3s_sample_ras_ws against d3s_sample_ras: the fused launch (no
    workspace), and the two routed draws with the retry's indices in the
    workspace, in code0 (which the pick then overwrites) or in retry_idx."""
    import hiprt
    rng = np.random.default_rng(93)
    N = 16
    x = (rng.standard_normal((N, V)) * 2.5).astype(np.float32)
    x[np.arange(N), rng.integers(0, V, N)] += 7.0
    k, k2 = min(top_k, V), 30
    u, u2 = oracle.uniform(93, 0, N, k), oracle.uniform(93, 1, N, k2)
    first = oracle.sample(x, u, 0.7, 0.7, n_threads=8)["ids"]
    hist = np.full((N, 16), START, np.int32)
    hist[::2, 5] = np.where(first[::2] == 0, EOS, first[::2] + START - 1)
    params = dict(temperature=0.7, top_p=0.7, top_k=top_k, **MAP)
    exp = oracle.ras(x, u, u2, params, hist, n_threads=8)
    P = gpu.ras_params(**params)
    L = gpu.lib()
    need = L.d3s_sample_ras_workspace_bytes(0, N, V, ctypes.byref(P), 1 if outs != "none" else 0)
    banner(f"ras top_k={top_k} V={V} outputs={outs} workspace {need} B")
    ws = gpu.Workspace(need)
    b = dict(x=hiprt.to_device(x), u=hiprt.to_device(u), u2=hiprt.to_device(u2), h=hiprt.to_device(hist),
             main=hiprt.DeviceBuffer(4 * N), code0=hiprt.DeviceBuffer(4 * N), retry=hiprt.DeviceBuffer(4 * N))
    code0 = b["code0"].ptr if outs in ("code0", "retry") else None
    retry = b["retry"].ptr if outs == "retry" else None
    rc = L.d3s_sample_ras_ws(b["x"].ptr, 0, N, V, V, b["u"].ptr, b["u2"].ptr, b["h"].ptr, 16, ctypes.byref(P),
                             b["main"].ptr, code0, None, retry, None, ws.buf.ptr, ws.nbytes, None)
    assert rc == 0, rc
    hiprt.synchronize()
    assert np.array_equal(b["main"].download((N,), np.int32), exp["main"])
    if code0:
        assert np.array_equal(b["code0"].download((N,), np.int32), exp["code0"])
    if retry:
        assert np.array_equal(b["retry"].download((N,), np.int32), exp["retry"])
    lazy = gpu.sample_ras(x, u, u2, params, hist, indices=False)
    assert lazy["rc"] == 0 and np.array_equal(lazy["main"], exp["main"])
    for buf in b.values():
        buf.free()
    ws.free()


@pytest.mark.gpu
@pytest.mark.parametrize("flags,keep", [(0, True), (0, False), (16, True), (16, False)])
def test_linear_sample_ws_equals_the_stream_block(gpu, oracle, flags, keep):
    """d3s_linear_sample_bf16_ws against the oracle's gemv and sample: two
    launches (no workspace unless the logits go to it) and one launch (the
    fused head's records in the workspace)."""
    import hiprt
    rng = np.random.default_rng(94)
    N, K, V, k = 1, 2048, 4097, 30
    x = W.f32_to_bf16_bits(rng.standard_normal((N, K)).astype(np.float32))
    w = W.f32_to_bf16_bits((rng.standard_normal((V, K)) * 0.06).astype(np.float32))
    u = oracle.uniform(94, 0, N, k)
    exp = oracle.sample(oracle.linear_bf16(x, w), u, 0.7, 0.7)["ids"]
    L = gpu.lib()
    need = L.d3s_linear_sample_workspace_bytes(N, K, V, k, flags, 1 if keep else 0)
    banner(f"linear+sample flags={flags} keep_logits={keep} workspace {need} B")
    ws = gpu.Workspace(need)
    bx, bw, bu, ids = hiprt.to_device(x), hiprt.to_device(w), hiprt.to_device(u), hiprt.DeviceBuffer(4 * N)
    by = hiprt.DeviceBuffer(2 * N * V) if keep else None
    for rep in range(2):  # twice: the workspace is left ready for the next call
        rc = L.d3s_linear_sample_bf16_ws(bx.ptr, bw.ptr, N, K, V, by.ptr if by else None, bu.ptr, k, None, None,
                                         0.7, 0.7, ids.ptr, None, None, None, flags, ws.buf.ptr, ws.nbytes, None)
        assert rc == 0, rc
        hiprt.synchronize()
        assert np.array_equal(ids.download((N,), np.int32), exp), rep
    for buf in (bx, bw, bu, ids, by):
        if buf is not None:
            buf.free()
    ws.free()


@pytest.mark.gpu
def test_stream_block_release(gpu, oracle):
    """d3s_sample on a new stream takes the library's block for it (C4 needs
    one); d3s_stream_workspace_release frees it; the next call allocates a new
    block and samples the same ids."""
    import hiprt
    w = W.make("C4", rows=16, seed=95, uniforms=False)
    u = oracle.uniform(95, 0, 16, 30)
    exp = oracle.sample(w["logits"], u, 1.0, 0.9, n_threads=8, detail=False)["ids"]
    s = hiprt.Stream()
    for rep in range(2):
        got = gpu.sample(w["logits"], u, 1.0, 0.9, want_probs=False, stream=s)
        assert got["rc"] == 0 and np.array_equal(got["ids"], exp), rep
        assert gpu.lib().d3s_stream_workspace_release(s.ptr) == 0
    assert gpu.lib().d3s_stream_workspace_release(s.ptr) == 0  # nothing left: still fine
    s.destroy()


@pytest.mark.gpu
def test_stream_block_shared_by_threads(gpu, oracle):
    """Two host threads on one stream, one with calls the segmented kernel takes
    (a 1 MiB block), the other with calls the sorting kernels take (k = V =
    20 000, a block of several MiB): the stream's block grows while the other
    thread may be enqueueing on the old one, which is kept, not freed. Every
    call's ids equal the oracle's."""
    import threading
    import hiprt
    rng = np.random.default_rng(96)
    c4 = W.make("C4", rows=16, seed=96, uniforms=False)["logits"]
    big = (rng.standard_normal((8, 20000)) * 2.0).astype(np.float32)
    cases = [(c4, 30, 1, 1.0, 0.9), (big, 20000, 0, 1.0, 0.9)]
    s = hiprt.Stream()
    errors = []

    def worker(x, k, dt, T, top_p, reps):
        try:
            N, V = x.shape
            u = oracle.uniform(97, 0, N, k)
            exp = oracle.sample(x, u, T, top_p, n_threads=4, detail=False)["ids"]
            bx, bu, ids = hiprt.to_device(x), hiprt.to_device(u), hiprt.DeviceBuffer(4 * N)
            for rep in range(reps):
                rc = gpu.sample_raw(bx.ptr, dt, N, V, V, bu.ptr, k, T, top_p, None, ids.ptr, stream=s.ptr)
                if rc != 0:
                    errors.append(("rc", V, rep, rc))
                    return
                s.synchronize()
                got = ids.download((N,), np.int32)
                if not np.array_equal(got, exp):
                    errors.append(("ids", V, rep))
            for b in (bx, bu, ids):
                b.free()
        except Exception as e:  # reported below
            errors.append(("exception", repr(e)))

    threads = [threading.Thread(target=worker, args=c + (10,)) for c in cases]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert gpu.lib().d3s_stream_workspace_release(s.ptr) == 0
    s.destroy()
    banner(f"two threads on one stream: errors {errors}")
    assert not errors, errors
