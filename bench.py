"""Benchmark of the MI355X token sampler on BASELINE.json's configurations.

Headline (`value`): sampled rows/s on C3, the batched backbone head
(fp32 [256, 4097], per-row T/top_p, k = 30) in steady state: multi-batch
launches, `--batches-per-launch` batches of 256 rows per d3s_sample call
(default 512: 131 072 rows), taken in turn by `--headline-streams` streams
(default 3), so that one launch's last waves overlap the next one's first.
A step is one such launch: 40 ms of untimed launches and `--warmup` more,
back to back (sustained load runs slower for its first ~30 ms), then
`--steps` timed ones (ms_per_step is per launch).  The launches cycle over
a pool of `--pool-batches` batches in device memory (default 512 batches,
2.2 GB, over eight times the 256 MB Infinity Cache, so every launch reads HBM;
16 distinct generated contents, every batch with its own uniforms).  Beside it: one batch
per launch on one stream and on `--streams` streams.

roofline.achieved = algorithmic bytes per launch (16 524 B per row) divided by
the kernel's mean launch duration: the same launches back to back on one
stream, timed with HIP events on that stream (what a kernel trace reports);
roofline.whole_job is the headline's rate in the same units.
cpu_baseline = the C oracle (the port of the
reference semantics; the reference's own CPU path needs mlx-c, absent here)
on a bounded sample of the same workload, all host cores.
Also reported: p50 / p90 of single-row C1 launches ([1, 4097] fp32), from
Python and from a C caller (drama3-mlx_amd/d3s_latency); launch times of C2,
C4 and C5 at their own shapes, the fused repetition-aware draw against its two
separate launches, the backbone head's gemv and its sample as two launches and
as one HIP graph, one decode frame's sampler launches and the reference's
"samplers (11)" micro-benchmark (`other_configs`).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "drama3-mlx_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "sampled rows/sec at B=256×4097 (% HBM roofline); p50 µs per single-row sample"
HBM_PEAK_GBS = 8000.0
ROWS, V, K = 256, 4097, 30
K_SAMPLE = K
BYTES_PER_ROW = V * 4 + K * 4 + 4 + 12  # logits, uniforms, id, (T, top_p, k)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Pool:
    """n_batches C3 batches (fp32 [256, 4097] each) in one contiguous device
    buffer, cycling over n_distinct generated batches, each batch with its own
    device uniforms (draw b) and the per-row T / top_p of C3."""

    def __init__(self, n_batches, n_distinct):
        import d3s
        import d3s_workloads as W
        import hiprt
        self.n = n_batches
        distinct = [W.make("C3", rows=ROWS, seed=1000 + i, uniforms=False) for i in range(n_distinct)]
        self.logits = hiprt.DeviceBuffer(n_batches * ROWS * V * 4)
        for b in range(n_batches):
            self.logits.upload(distinct[b % n_distinct]["logits"], offset=b * ROWS * V * 4)
        self.u = hiprt.DeviceBuffer(n_batches * ROWS * K * 4)
        for b in range(n_batches):
            assert d3s.lib().d3s_uniform_fill(self.u.ptr + b * ROWS * K * 4, ROWS * K, 42, b, None) == 0
        self.T = hiprt.to_device(np.tile(distinct[0]["temperature"], n_batches))
        self.top_p = hiprt.to_device(np.tile(distinct[0]["top_p"], n_batches))
        hiprt.synchronize()

    def launch(self, b, g, ids, stream):
        """one d3s_sample call over batches b .. b+g-1 (g * 256 rows)"""
        import d3s
        r0 = b * ROWS
        return d3s.sample_raw(self.logits.ptr + r0 * V * 4, d3s.DTYPE_F32, g * ROWS, V, V,
                              self.u.ptr + r0 * K * 4, K, ("ptr", self.T.ptr + r0 * 4),
                              ("ptr", self.top_p.ptr + r0 * 4), None, ids.ptr, stream=stream)


def time_launches(pool, launches, warmup, g, n_streams, settle=0):
    """`settle` then `warmup` untimed launches, enqueued back to back, then
    `launches` timed launches of g batches each, round robin over n_streams
    streams, between a start event on the first stream (the others wait on
    it) and a stop event after every stream's last launch; returns (device ms
    between the events, host wall s, launches timed)."""
    import hiprt
    streams = [hiprt.Stream() for _ in range(n_streams)]
    ids = [hiprt.DeviceBuffer(4 * ROWS * g) for _ in range(n_streams)]
    windows = pool.n // g
    for i in range(settle):
        s = i % n_streams
        assert pool.launch((i % windows) * g, g, ids[s], streams[s].ptr) == 0
    for i in range(warmup):
        s = i % n_streams
        assert pool.launch((i % windows) * g, g, ids[s], streams[s].ptr) == 0
    hiprt.synchronize()
    start, stop = hiprt.Event(), hiprt.Event()
    joins = [hiprt.Event() for _ in streams[1:]]
    t0 = time.perf_counter()
    start.record(streams[0])
    for st in streams[1:]:
        st.wait(start)
    for i in range(launches):
        s = i % n_streams
        assert pool.launch(((warmup + i) % windows) * g, g, ids[s], streams[s].ptr) == 0
    for st, ev in zip(streams[1:], joins):
        ev.record(st)
        streams[0].wait(ev)
    stop.record(streams[0])
    stop.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_ms(stop)
    hiprt.synchronize()
    for ev in [start, stop] + joins:
        ev.destroy()
    for st in streams:
        st.destroy()
    return ms, wall, launches


PREWARM_S = 0.3
# Sustained load that starts after more than a few ms of idle runs slower for
# its first ~30 ms: per-launch events on one stream, headline launches back
# to back, read 330 us, then rise to 400-460 us from the sixth launch on and
# fall back to ~330 us over the next ~100 launches; 5 warm-up + 20 timed
# launches after 10-200 ms idle read 383-405 us per launch, after 120
# back-to-back launches 313-316 us.  Every timed phase therefore follows
# SETTLE_S of the same launches, enqueued back to back with its warm-up.
SETTLE_S = 0.04


def settle_launches(t_launch):
    """launches of t_launch seconds each that fill SETTLE_S"""
    return int(SETTLE_S / max(t_launch, 5e-6)) + 1


def prewarm(pool, g):
    """Headline launches back to back until PREWARM_S seconds have passed
    (the GPU's clocks ramp up over the first milliseconds of work)."""
    import hiprt
    ids = hiprt.DeviceBuffer(4 * ROWS * g)
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < PREWARM_S:
        for _ in range(8):
            assert pool.launch((n % (pool.n // g)) * g, g, ids, None) == 0
            n += 1
        hiprt.synchronize()
    return n


def traffic_probe(pool, g, n):
    """For rocprofv3 --pmc runs: one 256 MiB device-to-device copy (the
    calibration dispatch of known traffic: 256 MiB read, 256 MiB written),
    then n launches of g C3 batches on one stream."""
    import hiprt
    nbytes = 256 << 20
    src, dst = hiprt.DeviceBuffer(nbytes), hiprt.DeviceBuffer(nbytes)
    hiprt.synchronize()
    hiprt.check(hiprt.hip().hipMemcpyAsync(dst.ptr, src.ptr, nbytes, hiprt.D2D, None), "copy")
    hiprt.synchronize()
    ids = hiprt.DeviceBuffer(4 * ROWS * g)
    for i in range(n):
        assert pool.launch((i % (pool.n // g)) * g, g, ids, None) == 0
    hiprt.synchronize()
    log(f"traffic probe: 1 copy of {nbytes} B, {n} launches of {g} C3 batches")


def calibration_copy():
    """One 256 MiB device-to-device copy: the dispatch of known traffic (256 MiB
    read, 256 MiB written) that scales the FETCH_SIZE / WRITE_SIZE counters."""
    import hiprt
    nbytes = 256 << 20
    src, dst = hiprt.DeviceBuffer(nbytes), hiprt.DeviceBuffer(nbytes)
    hiprt.synchronize()
    hiprt.check(hiprt.hip().hipMemcpyAsync(dst.ptr, src.ptr, nbytes, hiprt.D2D, None), "copy")
    hiprt.synchronize()
    src.free()
    dst.free()
    return nbytes


def head_probe(one_launch, n=20):
    """The backbone head's gemv and its sample (bf16 [1, 2048] x [4097, 2048],
    k 30): n calls of d3s_linear_sample_bf16, two launches (k_linear, then
    k_wave_row) or one (k_head), each followed by a synchronisation, the
    weights rotating over 8 copies."""
    import d3s
    import d3s_workloads as W
    import hiprt
    K, Vh, copies = 2048, 4097, 8
    rng = np.random.default_rng(11)
    x = W.f32_to_bf16_bits(rng.standard_normal((1, K)).astype(np.float32))
    w = W.f32_to_bf16_bits((rng.standard_normal((Vh, K)) * 0.06).astype(np.float32))
    bx = hiprt.to_device(x)
    bw = hiprt.DeviceBuffer(copies * w.nbytes)
    for c in range(copies):
        bw.upload(w, offset=c * w.nbytes)
    y, u, ids = hiprt.DeviceBuffer(2 * Vh), hiprt.DeviceBuffer(4 * K_SAMPLE), hiprt.DeviceBuffer(16)
    assert d3s.lib().d3s_uniform_fill(u.ptr, K_SAMPLE, 11, 0, None) == 0
    hiprt.synchronize()
    flags = d3s.FLAG_ONE_LAUNCH if one_launch else 0
    for i in range(n):
        assert d3s.lib().d3s_linear_sample_bf16(bx.ptr, bw.ptr + (i % copies) * w.nbytes, 1, K, Vh, y.ptr, u.ptr,
                                                K_SAMPLE, None, None, 0.7, 0.7, ids.ptr, None, None, None, flags,
                                                None) == 0
        hiprt.synchronize()


def samplers_probe(n=50):
    """The reference's samplers(11) loop (tools/bench.c:287-328): eleven
    samples on fp32 [1, 4097] uniform(0, 1) logits, T 1.0, top_k 30, top_p 0.9,
    n times as eleven d3s_sample_seeded launches and then as eleven pairs of
    d3s_uniform_fill and d3s_sample (the same uniforms), each group followed by
    a synchronisation."""
    import d3s
    import hiprt
    Vs, k = 4097, 30
    rng = np.random.default_rng(31)
    lg = hiprt.to_device(rng.random((1, Vs)).astype(np.float32))
    u = hiprt.DeviceBuffer(4 * 11 * k)
    ids = hiprt.DeviceBuffer(4 * 11)
    for i in range(n):
        for j in range(11):
            assert d3s.sample_seeded_raw(lg.ptr, d3s.DTYPE_F32, 1, Vs, Vs, 42, 11 * i + j, k, 1.0, 0.9, None,
                                         ids.ptr + 4 * j) == 0
        hiprt.synchronize()
        for j in range(11):
            assert d3s.lib().d3s_uniform_fill(u.ptr + j * k * 4, k, 42, 11 * i + j, None) == 0
            assert d3s.sample_raw(lg.ptr, d3s.DTYPE_F32, 1, Vs, Vs, u.ptr + j * k * 4, k, 1.0, 0.9, None,
                                  ids.ptr + 4 * j) == 0
        hiprt.synchronize()


def counter_probe(name, pool, g_head):
    """For rocprofv3 --pmc runs: the calibration copy, then launches of one
    workload only, each followed by a synchronisation, so every other dispatch
    in the profile is that workload's.  c1: 200 single C1 rows; c1rows /
    c1long: 20 launches of 1024 C1 rows (one row per workgroup, k_wave_row) /
    1025 (four rows per workgroup, k_wave); c2: 50 C2
    launches (nine rows); c3one: 50 one-batch C3 launches; c3: 20 headline
    launches (g_head batches each); c4 / c5: 20 launches of C4 / C5 (ids only);
    head / head1: 20 backbone-head gemv + sample calls, two launches / one;
    samplers: the samplers(11) loop 50 times, seeded and as pairs."""
    import d3s
    import d3s_workloads as W
    import hiprt
    calibration_copy()
    if name in ("head", "head1"):
        head_probe(name == "head1")
        log(f"counter probe {name}: done")
        return
    if name == "samplers":
        samplers_probe()
        log(f"counter probe {name}: done")
        return
    if name in ("c3", "c3one"):
        g = g_head if name == "c3" else 1
        ids = hiprt.DeviceBuffer(4 * ROWS * g)
        for i in range(20 if name == "c3" else 50):
            assert pool.launch((i % (pool.n // g)) * g, g, ids, None) == 0
            hiprt.synchronize()
        log(f"counter probe {name}: done")
        return
    cfg = {"c1": "C1", "c1rows": "C1", "c1long": "C1", "c2": "C2", "c4": "C4", "c5": "C5"}[name]
    w = W.make(cfg, rows={"c1": 256, "c1rows": 1024, "c1long": 1025}.get(name), seed=5, uniforms=False)
    x = w["logits"]
    N, Vc = x.shape
    k = w["k"]
    dt = d3s.DTYPE_F32 if x.dtype == np.float32 else d3s.DTYPE_BF16
    lg = hiprt.to_device(x)
    u = hiprt.DeviceBuffer(4 * N * k)
    assert d3s.lib().d3s_uniform_fill(u.ptr, N * k, 42, 0, None) == 0
    ban = hiprt.to_device(w["banned"]) if w["banned"] is not None else None
    ids = hiprt.DeviceBuffer(4 * N)
    T, P = w["temperature"], w["top_p"]
    T = float(T) if np.ndim(T) == 0 else float(T[0])
    P = float(P) if np.ndim(P) == 0 else float(P[0])
    for i in range({"c1": 200, "c2": 50}.get(name, 20)):
        if name == "c1":
            r = i % N
            rc = d3s.sample_raw(lg.ptr + r * Vc * x.itemsize, dt, 1, Vc, Vc, u.ptr + r * k * 4, k, T, P,
                                None, ids.ptr)
        else:
            rc = d3s.sample_raw(lg.ptr, dt, N, Vc, Vc, u.ptr, k, T, P, ban.ptr if ban else None, ids.ptr)
        assert rc == 0
        hiprt.synchronize()
    log(f"counter probe {name}: done")


def launch_floor(n):
    """Events around a near-empty launch (the uniform fill of 64 values): the
    part of any event-timed launch that is dispatch, not work."""
    import d3s
    import hiprt
    buf = hiprt.DeviceBuffer(256)
    s = hiprt.Stream()
    a, b = hiprt.Event(), hiprt.Event()
    d = []
    for i in range(n + 20):
        a.record(s)
        assert d3s.lib().d3s_uniform_fill(buf.ptr, 64, 1, i, s.ptr) == 0
        b.record(s)
        b.synchronize()
        if i >= 20:
            d.append(a.elapsed_ms(b) * 1e3)
    s.destroy()
    return float(np.median(d))


def single_row_latency(n):
    """C1: one [1, 4097] fp32 row per call.  GPU time (events around the
    launch) and host time (call to completion) per row, p50 / p90."""
    import d3s
    import d3s_workloads as W
    import hiprt
    w = W.make("C1", rows=256, seed=42, uniforms=False)
    lg = hiprt.to_device(w["logits"])
    u = hiprt.DeviceBuffer(4 * 256 * K)
    assert d3s.lib().d3s_uniform_fill(u.ptr, 256 * K, 42, 0, None) == 0
    ids = hiprt.DeviceBuffer(4)
    s = hiprt.Stream()
    a, b = hiprt.Event(), hiprt.Event()
    gpu_us, host_us = [], []
    for i in range(n + 50):
        r = i % 256
        t0 = time.perf_counter()
        a.record(s)
        rc = d3s.sample_raw(lg.ptr + r * V * 4, d3s.DTYPE_F32, 1, V, V, u.ptr + r * K * 4, K, 0.7,
                            0.7, None, ids.ptr, stream=s.ptr)
        b.record(s)
        b.synchronize()
        t1 = time.perf_counter()
        assert rc == 0
        if i >= 50:
            gpu_us.append(a.elapsed_ms(b) * 1e3)
            host_us.append((t1 - t0) * 1e6)
    s.destroy()
    g, h = np.array(gpu_us), np.array(host_us)
    return dict(p50_us=float(np.median(g)), p90_us=float(np.percentile(g, 90)),
                host_p50_us=float(np.median(h)), host_p90_us=float(np.percentile(h, 90)), rows=n)


def other_configs(reps):
    """Launch times of C2, C4 and C5 at their own shapes (BASELINE.json's
    configs; C3 and C1 are the headline).  Events on one stream around
    back-to-back launches after SETTLE_S of the same launches.  C4 and C5
    rotate over copies of the inputs totalling over 600 MB (more than twice
    the 256 MB Infinity Cache), so the reads come from HBM.  C2 (75 KB a launch) is a latency figure: the nine
    codebook rows as nine one-row launches (as the tower samples them) and as
    one nine-row launch, p50 over `reps` repetitions."""
    import d3s
    import d3s_workloads as W
    import hiprt
    out = {}
    s = hiprt.Stream()
    a, b = hiprt.Event(), hiprt.Event()
    for name in ("C2", "C4", "C5"):
        w = W.make(name, seed=5, uniforms=False)
        x = w["logits"]
        N, Vc = x.shape
        k = w["k"]
        es = x.itemsize
        dt = d3s.DTYPE_F32 if x.dtype == np.float32 else d3s.DTYPE_BF16
        b_row = Vc * es + k * 4 + 4 + 12 + (4 if w["banned"] is not None else 0)
        per_launch = N * b_row
        copies = 1 if name == "C2" else -(-600_000_000 // per_launch)
        lg = hiprt.DeviceBuffer(copies * x.nbytes)
        for c in range(copies):
            lg.upload(x, offset=c * x.nbytes)
        u = hiprt.DeviceBuffer(copies * N * k * 4)
        for c in range(copies):
            assert d3s.lib().d3s_uniform_fill(u.ptr + c * N * k * 4, N * k, 42, c, None) == 0
        ban = hiprt.to_device(w["banned"]) if w["banned"] is not None else None
        ids = hiprt.DeviceBuffer(4 * N)
        T, P = float(w["temperature"]), float(w["top_p"])

        def launch(c, r0=0, n=N):
            return d3s.sample_raw(lg.ptr + c * x.nbytes + r0 * Vc * es, dt, n, Vc, Vc,
                                  u.ptr + (c * N + r0) * k * 4, k, T, P,
                                  ban.ptr + 4 * r0 if ban is not None else None, ids.ptr, stream=s.ptr)
        hiprt.synchronize()
        if name == "C2":
            fused, rows = [], []
            for i in range(reps + 20):
                a.record(s)
                assert launch(0) == 0
                b.record(s)
                b.synchronize()
                t_f = a.elapsed_ms(b) * 1e3
                a.record(s)
                for r in range(N):
                    assert launch(0, r, 1) == 0
                b.record(s)
                b.synchronize()
                if i >= 20:
                    fused.append(t_f)
                    rows.append(a.elapsed_ms(b) * 1e3)
            out[name] = {"shape": [N, Vc], "dtype": "bf16", "k": k,
                         "one_launch_p50_us": float(np.median(fused)),
                         "nine_launches_p50_us": float(np.median(rows))}
            log(f"C2: one 9-row launch p50 {out[name]['one_launch_p50_us']:.2f} us, "
                f"9 one-row launches p50 {out[name]['nine_launches_p50_us']:.2f} us")
            continue
        # a first estimate of the launch time, then SETTLE_S of the same
        # launches back to back (as before every headline phase), then the
        # timed launches
        a.record(s)
        for c in range(copies):
            assert launch(c) == 0
        b.record(s)
        b.synchronize()
        t_est = a.elapsed_ms(b) * 1e-3 / copies
        for i in range(settle_launches(t_est)):
            assert launch(i % copies) == 0
        hiprt.synchronize()
        n = max(2 * copies, 100)
        a.record(s)
        for i in range(n):
            assert launch(i % copies) == 0
        b.record(s)
        b.synchronize()
        us = a.elapsed_ms(b) * 1e3 / n
        gbs = per_launch / (us * 1e-6) / 1e9
        out[name] = {"shape": [N, Vc], "dtype": "bf16" if es == 2 else "f32", "k": k,
                     "us_per_launch": us, "rows_per_s": N / (us * 1e-6),
                     "bytes_per_launch": per_launch, "achieved_GBs": gbs,
                     "frac": gbs / HBM_PEAK_GBS}
        log(f"{name}: {us:.1f} us per launch of {N} rows, {gbs:.0f} GB/s "
            f"({100 * gbs / HBM_PEAK_GBS:.1f} % of HBM peak)")
        del lg, u
    # C4's rows with top-k disabled (k = V, the op graph's full argsort,
    # src/sampling.c:33-35): the sorting kernel
    w = W.make("C4", seed=5, uniforms=False)
    x = w["logits"]
    N, Vc = x.shape
    lg, u, ids = hiprt.to_device(x), hiprt.DeviceBuffer(N * Vc * 4), hiprt.DeviceBuffer(4 * N)
    assert d3s.lib().d3s_uniform_fill(u.ptr, N * Vc, 42, 0, None) == 0
    hiprt.synchronize()
    a.record(s)
    for _ in range(2):
        assert d3s.sample_raw(lg.ptr, d3s.DTYPE_BF16, N, Vc, Vc, u.ptr, Vc, 1.0, 0.9, None, ids.ptr,
                              stream=s.ptr) == 0
    b.record(s)
    b.synchronize()
    for _ in range(settle_launches(a.elapsed_ms(b) * 1e-3 / 2)):
        assert d3s.sample_raw(lg.ptr, d3s.DTYPE_BF16, N, Vc, Vc, u.ptr, Vc, 1.0, 0.9, None, ids.ptr,
                              stream=s.ptr) == 0
    hiprt.synchronize()
    n = 40
    a.record(s)
    for _ in range(n):
        assert d3s.sample_raw(lg.ptr, d3s.DTYPE_BF16, N, Vc, Vc, u.ptr, Vc, 1.0, 0.9, None, ids.ptr,
                              stream=s.ptr) == 0
    b.record(s)
    b.synchronize()
    us = a.elapsed_ms(b) * 1e3 / n
    per_launch = N * (Vc * 2 + Vc * 4 + 4 + 12)
    out["C4_k_eq_V"] = {"shape": [N, Vc], "dtype": "bf16", "k": Vc, "us_per_launch": us,
                        "rows_per_s": N / (us * 1e-6), "bytes_per_launch": per_launch,
                        "achieved_GBs": per_launch / (us * 1e-6) / 1e9}
    log(f"C4 with top-k disabled (k = V = {Vc}): {us:.1f} us per launch of {N} rows")
    for buf in (lg, u, ids):
        buf.free()
    s.destroy()
    return out


def ras_latency(reps):
    """The main token's repetition-aware draw (src/tower.c:420-433) on the
    backbone head's shape, bf16 [1, 4097]: one d3s_sample_ras launch (both
    draws, the row read once from HBM) against the two d3s_sample launches it
    replaces.  p50 of events around each, over `reps` rows."""
    import d3s
    import d3s_workloads as W
    import hiprt
    w = W.make("C1", rows=64, seed=9, uniforms=False)
    xb = W.f32_to_bf16_bits(w["logits"])
    lg = hiprt.to_device(xb)
    u = hiprt.DeviceBuffer(4 * 64 * K)
    u2 = hiprt.DeviceBuffer(4 * 64 * K)
    assert d3s.lib().d3s_uniform_fill(u.ptr, 64 * K, 9, 0, None) == 0
    assert d3s.lib().d3s_uniform_fill(u2.ptr, 64 * K, 9, 1, None) == 0
    hist = hiprt.to_device(np.full(16, 151669, np.int32))
    out = hiprt.DeviceBuffer(16)
    P = d3s.ras_params(temperature=0.7, top_p=0.7, top_k=K, eos_id=151645, semantic_start=151669,
                       semantic_end=151669 + 4095, code_vocab=4096)
    s = hiprt.Stream()
    a, b = hiprt.Event(), hiprt.Event()
    fused, two = [], []
    for i in range(reps + 20):
        r = i % 64
        row, ur, u2r = lg.ptr + r * V * 2, u.ptr + r * K * 4, u2.ptr + r * K * 4
        a.record(s)
        assert d3s.sample_ras_raw(row, d3s.DTYPE_BF16, 1, V, V, ur, u2r, hist.ptr, 16, P, out.ptr,
                                  stream=s.ptr) == 0
        b.record(s)
        b.synchronize()
        tf = a.elapsed_ms(b) * 1e3
        a.record(s)
        assert d3s.sample_raw(row, d3s.DTYPE_BF16, 1, V, V, ur, K, 0.7, 0.7, None, out.ptr, stream=s.ptr) == 0
        assert d3s.sample_raw(row, d3s.DTYPE_BF16, 1, V, V, u2r, K, 1.0, 0.95, None, out.ptr + 4,
                              stream=s.ptr) == 0
        b.record(s)
        b.synchronize()
        if i >= 20:
            fused.append(tf)
            two.append(a.elapsed_ms(b) * 1e3)
    s.destroy()
    res = {"shape": [1, V], "dtype": "bf16", "k": K, "retry": [1.0, 0.95, 30],
           "fused_p50_us": float(np.median(fused)), "two_launches_p50_us": float(np.median(two)),
           "hbm_bytes_fused": V * 2 + 2 * K * 4 + 16 * 4 + 8,
           "hbm_bytes_two_launches": 2 * (V * 2 + K * 4 + 4)}
    log(f"RAS main token, bf16 [1, {V}]: one fused launch p50 {res['fused_p50_us']:.2f} us, "
        f"two launches p50 {res['two_launches_p50_us']:.2f} us")
    return res


def head_latency(reps):
    """The backbone head (src/backbone.c:1213-1215) and its sample: bf16 hidden
    [1, 2048] x lm_head [4097, 2048]^T, then one draw.  p50 of events around
    one d3s_linear_sample_bf16 launch with D3S_FLAG_ONE_LAUNCH (gemv and sample
    fused), around the two launches d3s_linear_bf16 + d3s_sample (the entry
    point's default), and around one replay of a HIP graph holding those two
    (one weight copy, as a graph fixes its pointers).  Each of the first two,
    and the gemv alone, also rotating over 32 weight copies (537 MB, over twice
    the Infinity Cache) so each call reads them from HBM."""
    import ctypes
    import d3s
    import d3s_workloads as W
    import hiprt
    H = hiprt.hip()
    K, Vh, copies = 2048, 4097, 32
    rng = np.random.default_rng(11)
    x = W.f32_to_bf16_bits(rng.standard_normal((1, K)).astype(np.float32))
    w = W.f32_to_bf16_bits((rng.standard_normal((Vh, K)) * 0.06).astype(np.float32))
    bx = hiprt.to_device(x)
    bw = hiprt.DeviceBuffer(copies * w.nbytes)
    for c in range(copies):
        bw.upload(w, offset=c * w.nbytes)
    y = hiprt.DeviceBuffer(2 * Vh)
    u = hiprt.DeviceBuffer(4 * K_SAMPLE)
    assert d3s.lib().d3s_uniform_fill(u.ptr, K_SAMPLE, 11, 0, None) == 0
    ids = hiprt.DeviceBuffer(16)
    hiprt.synchronize()
    s = hiprt.Stream()
    L = d3s.lib()

    def both(wp):
        assert L.d3s_linear_bf16(bx.ptr, wp, 1, K, Vh, y.ptr, s.ptr) == 0
        assert d3s.sample_raw(y.ptr, d3s.DTYPE_BF16, 1, Vh, Vh, u.ptr, K_SAMPLE, 0.7, 0.7, None, ids.ptr,
                              stream=s.ptr) == 0
    def fused(wp):
        assert L.d3s_linear_sample_bf16(bx.ptr, wp, 1, K, Vh, y.ptr, u.ptr, K_SAMPLE, None, None, 0.7, 0.7,
                                        ids.ptr, None, None, None, d3s.FLAG_ONE_LAUNCH, s.ptr) == 0
    graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
    hiprt.check(H.hipStreamBeginCapture(s.ptr, 0), "begin capture")
    both(bw.ptr)
    hiprt.check(H.hipStreamEndCapture(s.ptr, ctypes.byref(graph)), "end capture")
    hiprt.check(H.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0), "instantiate")
    a, b = hiprt.Event(), hiprt.Event()
    two, two_hbm, replay, gemv, one, one_hbm = [], [], [], [], [], []
    for i in range(reps + 20):
        a.record(s)
        both(bw.ptr)
        b.record(s)
        b.synchronize()
        t2 = a.elapsed_ms(b) * 1e3
        a.record(s)
        both(bw.ptr + ((i + 7) % copies) * w.nbytes)
        b.record(s)
        b.synchronize()
        t2h = a.elapsed_ms(b) * 1e3
        a.record(s)
        fused(bw.ptr)
        b.record(s)
        b.synchronize()
        t1 = a.elapsed_ms(b) * 1e3
        a.record(s)
        fused(bw.ptr + (i % copies) * w.nbytes)
        b.record(s)
        b.synchronize()
        t1h = a.elapsed_ms(b) * 1e3
        a.record(s)
        hiprt.check(H.hipGraphLaunch(exe, s.ptr), "graph launch")
        b.record(s)
        b.synchronize()
        tg = a.elapsed_ms(b) * 1e3
        a.record(s)
        assert L.d3s_linear_bf16(bx.ptr, bw.ptr + (i % copies) * w.nbytes, 1, K, Vh, y.ptr, s.ptr) == 0
        b.record(s)
        b.synchronize()
        if i >= 20:
            two.append(t2)
            two_hbm.append(t2h)
            one.append(t1)
            one_hbm.append(t1h)
            replay.append(tg)
            gemv.append(a.elapsed_ms(b) * 1e3)
    H.hipGraphExecDestroy(exe)
    H.hipGraphDestroy(graph)
    s.destroy()
    g = float(np.median(gemv))
    res = {"shape": [[1, K], [Vh, K]], "dtype": "bf16", "k": K_SAMPLE,
           "fused_p50_us": float(np.median(one)), "fused_hbm_p50_us": float(np.median(one_hbm)),
           "two_launches_p50_us": float(np.median(two)), "two_launches_hbm_p50_us": float(np.median(two_hbm)),
           "graph_replay_p50_us": float(np.median(replay)),
           "gemv_p50_us": g, "gemv_weight_GBs": w.nbytes / (g * 1e-6) / 1e9}
    log(f"head gemv + sample, [1, {K}] x [{Vh}, {K}] bf16: one fused launch p50 {res['fused_p50_us']:.2f} us "
        f"({res['fused_hbm_p50_us']:.2f} us with the weights from HBM), "
        f"two launches p50 {res['two_launches_p50_us']:.2f} us ({res['two_launches_hbm_p50_us']:.2f} us from HBM), "
        f"one graph replay p50 {res['graph_replay_p50_us']:.2f} us; gemv alone (HBM) {g:.2f} us "
        f"({res['gemv_weight_GBs']:.0f} GB/s of weights)")
    return res


def frame_latency(reps):
    """The sampler work of one decode frame (src/tower.c:420-446), on one
    stream: the main token's repetition-aware draw on the backbone head's bf16
    [1, 4097] row (one d3s_sample_ras launch holding both draws), then the nine
    codebook heads' bf16 [1, 4096] draws, one launch each (each head's logits
    follow from the code before it, so the tower cannot batch them).  Beside
    it, the reference's own sampler micro-benchmark (tools/bench.c:287-328,
    "samplers (11)"): eleven sample_top_k_top_p calls on fp32 [1, 4097]
    uniform(0, 1) logits with T 1.0, top_k 30, top_p 0.9 (bench.c:313), here
    eleven d3s_sample_seeded calls (sample_top_k_top_p's draw and kernel in
    one launch, as the shim runs it), and beside them eleven pairs of
    d3s_uniform_fill and d3s_sample.  p50 / p90 of events around each frame
    over `reps` frames, and the host wall time per frame."""
    import d3s
    import d3s_workloads as W
    import hiprt
    L = d3s.lib()
    rng = np.random.default_rng(31)
    head = W.f32_to_bf16_bits((rng.standard_normal((64, V)) * 2.5).astype(np.float32))
    books = W.make("C2", rows=9 * 8, seed=31, uniforms=False)["logits"]
    dh, db = hiprt.to_device(head), hiprt.to_device(books)
    u = hiprt.DeviceBuffer(4 * 64 * 11 * K)
    assert L.d3s_uniform_fill(u.ptr, 64 * 11 * K, 31, 0, None) == 0
    hist = hiprt.to_device(np.full(16, 151669, np.int32))
    frame = hiprt.DeviceBuffer(4 * 11)
    P = d3s.ras_params(temperature=0.7, top_p=0.7, top_k=K, eos_id=151645, semantic_start=151669,
                       semantic_end=151669 + 4095, code_vocab=4096)
    lg = hiprt.to_device(rng.random((1, V)).astype(np.float32))
    u11 = hiprt.DeviceBuffer(4 * 11 * K)
    ids11 = hiprt.DeviceBuffer(4 * 11)
    s = hiprt.Stream()
    a, b = hiprt.Event(), hiprt.Event()

    def one_frame(i):
        r = i % 64
        ub = u.ptr + r * 11 * K * 4
        assert d3s.sample_ras_raw(dh.ptr + r * V * 2, d3s.DTYPE_BF16, 1, V, V, ub, ub + K * 4, hist.ptr, 16, P,
                                  frame.ptr, frame.ptr + 4, stream=s.ptr) == 0
        for j in range(9):
            row = db.ptr + ((r % 8) * 9 + j) * 4096 * 2
            assert d3s.sample_raw(row, d3s.DTYPE_BF16, 1, 4096, 4096, ub + (2 + j) * K * 4, K, 0.7, 0.7, None,
                                  frame.ptr + 4 * (2 + j), stream=s.ptr) == 0

    def samplers11(i):
        for j in range(11):
            assert d3s.sample_seeded_raw(lg.ptr, d3s.DTYPE_F32, 1, V, V, 42, 11 * i + j, K, 1.0, 0.9, None,
                                         ids11.ptr + 4 * j, stream=s.ptr) == 0

    def samplers11_pairs(i):
        for j in range(11):
            assert L.d3s_uniform_fill(u11.ptr + j * K * 4, K, 42, 11 * i + j, s.ptr) == 0
            assert d3s.sample_raw(lg.ptr, d3s.DTYPE_F32, 1, V, V, u11.ptr + j * K * 4, K, 1.0, 0.9, None,
                                  ids11.ptr + 4 * j, stream=s.ptr) == 0

    out = {}
    for name, fn in (("frame", one_frame), ("samplers_11", samplers11), ("samplers_11_pairs", samplers11_pairs)):
        ev, wall = [], []
        for i in range(reps + 20):
            t0 = time.perf_counter()
            a.record(s)
            fn(i)
            b.record(s)
            b.synchronize()
            t1 = time.perf_counter()
            if i >= 20:
                ev.append(a.elapsed_ms(b) * 1e3)
                wall.append((t1 - t0) * 1e6)
        out[name] = {"p50_us": float(np.median(ev)), "p90_us": float(np.percentile(ev, 90)),
                     "host_p50_us": float(np.median(wall)), "frames": reps}
    out["frame"]["launches"] = 10
    out["frame"]["what"] = ("d3s_sample_ras on bf16 [1,4097] (both draws) + 9 d3s_sample on bf16 [1,4096], "
                            "one stream (src/tower.c:420-446)")
    out["samplers_11"]["launches"] = 11
    out["samplers_11"]["what"] = ("11 x d3s_sample_seeded (the uniform draw and the sample in one launch) on fp32 "
                                  "[1,4097] uniform(0,1) logits, T 1.0, top_k 30, top_p 0.9 (tools/bench.c:313)")
    out["samplers_11_pairs"]["launches"] = 22
    out["samplers_11_pairs"]["what"] = ("the same as 11 x (d3s_uniform_fill + d3s_sample)")
    s.destroy()
    log(f"frame (RAS + 9 codebooks, 10 launches): p50 {out['frame']['p50_us']:.2f} us; "
        f"samplers (11) as tools/bench.c: p50 {out['samplers_11']['p50_us']:.2f} us in 11 launches, "
        f"{out['samplers_11_pairs']['p50_us']:.2f} us as 22")
    return out


def c_caller_latency(calls):
    """C1 one-row calls timed by drama3-mlx_amd/d3s_latency, a C program
    linked to the library (what a C caller such as tower.c sees, without
    Python's call overhead): host call-to-synchronize p50, call-to-done p50
    when the caller polls the stream, and event p50; then the same under
    spin-wait scheduling (hipDeviceScheduleSpin, set by the child before any
    other HIP call).  Run in child processes before this process touches the
    GPU."""
    import subprocess
    import tempfile
    import d3s_workloads as W
    exe = os.path.join(ROOT, "drama3-mlx_amd", "d3s_latency")
    if not os.path.exists(exe):
        return None
    w = W.make("C1", rows=256, seed=42, uniforms=True)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "c1.bin")
        with open(path, "wb") as f:
            f.write(np.ascontiguousarray(w["logits"], np.float32).tobytes())
            f.write(np.ascontiguousarray(w["u"], np.float32).tobytes())
        runs = {}
        for mode in ("default", "spin"):
            extra = ["spin"] if mode == "spin" else []
            r = subprocess.run([exe, path, "256", str(V), str(K), str(calls), "0.7", "0.7"] + extra,
                               capture_output=True, text=True, timeout=300)
            if r.returncode != 0:
                log(f"d3s_latency ({mode}) failed: {r.stderr.strip()[-300:]}")
                return None
            runs[mode] = json.loads(r.stdout.strip().splitlines()[-1])
    res = runs["default"]
    res["spin_wait"] = {key: runs["spin"][key] for key in ("host_p50_us", "host_p90_us", "host_poll_p50_us",
                                                           "host_poll_p90_us")}
    log(f"C caller, C1 one row: host p50 {res['host_p50_us']:.2f} us (blocking synchronize), "
        f"{res['host_poll_p50_us']:.2f} us (polling the stream), {res['spin_wait']['host_p50_us']:.2f} us "
        f"(synchronize under spin-wait scheduling); event p50 {res['event_p50_us']:.2f} us")
    return res


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(seconds):
    """The oracle (ids only: no probabilities or float64 boundary shadow) on
    all host cores over a bounded sample of C3 rows, and its per-row time on
    one thread for C1 rows (a 2000-row call, so the per-call cost is spread)."""
    import tempfile
    import d3s_oracle
    import d3s_workloads as W
    tmp = tempfile.mkdtemp()
    native = d3s_oracle.build_native(tmp)
    if native:
        d3s_oracle.use_library(native)
        flags = "-O3 -march=native, built on this host"
    else:
        flags = "-O2 -march=x86-64-v3 (no C compiler on this host)"
    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    w = W.make("C3", rows=ROWS, seed=7, uniforms=False)
    u = d3s_oracle.uniform(42, 0, ROWS, K)
    run = lambda: d3s_oracle.sample(w["logits"], u, w["temperature"], w["top_p"], n_threads=threads,
                                    detail=False)
    # calibrate, then run about `seconds` of work
    t0 = time.perf_counter()
    run()
    per_batch = time.perf_counter() - t0
    n = max(1, int(seconds / max(per_batch, 1e-6)))
    t0 = time.perf_counter()
    for _ in range(n):
        run()
    dt = time.perf_counter() - t0
    c1 = W.make("C1", rows=2000, seed=7, uniforms=False)
    u1 = d3s_oracle.uniform(42, 1, 2000, K)
    t0 = time.perf_counter()
    d3s_oracle.sample(c1["logits"], u1, 0.7, 0.7, n_threads=1, detail=False)
    c1_us = (time.perf_counter() - t0) / 2000 * 1e6
    return dict(value=n * ROWS / dt, unit="rows/s", cores=int(threads), kind="port",
                sample=f"{n} batches x {ROWS} rows of C3 (fp32 [256,4097], k=30), C oracle "
                       f"({flags}, OpenMP over rows, ids only) on {threads} threads, {dt:.1f} s",
                cpu_model=cpu_model(), c1_row_us_1_thread=c1_us,
                configs=cpu_configs(threads))


def cpu_configs(threads, min_seconds=0.5):
    """The oracle on every configuration at its own shape: rows/s on one
    thread and on `threads` (C2: the nine rows; C4 and C5: their full row
    counts), each timed over repeated calls for at least `min_seconds`."""
    import d3s_oracle
    import d3s_workloads as W
    out = {}
    for name in ("C2", "C3", "C4", "C5"):
        w = W.make(name, seed=9, uniforms=False)
        x = w["logits"]
        N = x.shape[0]
        u = d3s_oracle.uniform(42, 2, N, w["k"])
        rates = {}
        for nt in (1, threads):
            rows_timed, t0 = 0, time.perf_counter()
            while True:
                d3s_oracle.sample(x, u, w["temperature"], w["top_p"], banned=w["banned"], n_threads=nt,
                                  detail=False)
                rows_timed += N
                dt = time.perf_counter() - t0
                if dt >= min_seconds:
                    break
            rates[nt] = rows_timed / dt
        out[name] = {"rows": N, "vocab": int(x.shape[1]), "k": int(w["k"]),
                     "rows_per_s_1_thread": rates[1], f"rows_per_s_{threads}_threads": rates[threads],
                     "us_per_row_1_thread": 1e6 / rates[1]}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40,
                    help="timed launches, each of --batches-per-launch C3 batches")
    ap.add_argument("--warmup", type=int, default=8, help="untimed launches before (clocks settle)")
    ap.add_argument("--batches-per-launch", type=int, default=512,
                    help="C3 batches one d3s_sample call carries in the headline figure")
    ap.add_argument("--headline-streams", type=int, default=3,
                    help="streams the headline's launches take in turn (launches overlap)")
    ap.add_argument("--streams", type=int, default=4,
                    help="streams for the one-batch-per-launch figure beside the headline")
    ap.add_argument("--pool-batches", type=int, default=512)
    ap.add_argument("--single-rows", type=int, default=10000)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-other", action="store_true", help="skip the C2 / C4 / C5 figures")
    ap.add_argument("--counter-probe", choices=["c1", "c1rows", "c1long", "c2", "c3one", "c3", "c4", "c5", "head",
                                                "head1", "samplers"], default=None,
                    help="only run one workload's launches (for --pmc runs)")
    ap.add_argument("--traffic-probe", type=int, default=0, metavar="N",
                    help="only run the copy calibration and N headline launches (for --pmc runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build targets one GPU; --gpus {args.gpus} is not supported "
              "(rows are independent: N GPUs would each run this kernel on N/G rows)",
              file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        sys.exit("bench.py: --steps must be at least 1 and --warmup at least 0")
    # the C caller's figure first, in a child process, before this one starts HIP
    c_lat = c_caller_latency(10000) if args.single_rows else None
    import hiprt
    if hiprt.device_count() < 1:
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    import d3s
    d3s.lib()
    G = args.batches_per_launch
    if args.pool_batches % G:
        sys.exit("bench.py: --pool-batches must be a multiple of --batches-per-launch")

    if args.counter_probe and args.counter_probe not in ("c3", "c3one"):
        counter_probe(args.counter_probe, None, G)  # (needs no C3 pool)
        return
    log("building the C3 batch pool")
    pool = Pool(args.pool_batches, 16)
    pool_mb = args.pool_batches * ROWS * BYTES_PER_ROW / 1e6
    log(f"pool: {args.pool_batches} batches, {pool_mb:.0f} MB")
    if args.traffic_probe:
        traffic_probe(pool, G, args.traffic_probe)
        return
    if args.counter_probe:
        counter_probe(args.counter_probe, pool, G)
        return
    # clocks settle: headline launches for at least PREWARM_S seconds before
    # anything is timed (a fresh box runs its first ~10 ms of launches about
    # 15 % slower); then each timed phase: SETTLE_S of untimed launches and
    # --warmup more, back to back, a synchronisation, --steps timed launches
    prewarm_launches = prewarm(pool, G)
    n_settle = settle_launches(PREWARM_S / prewarm_launches)
    log(f"pre-warm: {prewarm_launches} launches over {PREWARM_S} s; {n_settle} settle launches per phase")
    # the dominant kernel alone: G batches per launch, back to back on one
    # stream, HIP events on that stream (the roofline's launch duration)
    bytes_per_launch = G * ROWS * BYTES_PER_ROW
    ms_k, _, lk = time_launches(pool, args.steps, args.warmup, G, 1, n_settle)
    kmean = ms_k * 1e3 / lk
    achieved = bytes_per_launch / (kmean * 1e-6) / 1e9
    log(f"one stream: {lk} timed launches of {G} batches after {args.warmup} untimed, {kmean:.2f} us per "
        f"launch -> {achieved:.0f} GB/s")
    # headline: the same launches taken in turn by S streams, so that one
    # launch's last waves overlap the next launch's first
    S = args.headline_streams
    ms, wall, launches = time_launches(pool, args.steps, args.warmup, G, S, n_settle)
    batches = launches * G
    value = batches * ROWS / (ms * 1e-3)
    job_gbs = value * BYTES_PER_ROW / 1e9
    log(f"steady state: {launches} timed launches of {G} batches ({batches} batches) over {S} streams in "
        f"{ms:.2f} ms: {value:.3e} rows/s -> {job_gbs:.0f} GB/s (host wall {wall:.3f} s)")
    # one batch (256 rows) per launch, one stream and several
    n1 = 5000
    n1_settle = settle_launches(1e-5)
    ms1, _, l1 = time_launches(pool, n1, 100, 1, 1, n1_settle)
    single = l1 * ROWS / (ms1 * 1e-3)
    log(f"one batch per launch, one stream: {single:.3e} rows/s ({ms1 * 1e3 / l1:.2f} us/launch)")
    msS, _, lS = time_launches(pool, n1, 100, 1, args.streams, n1_settle)
    multi = lS * ROWS / (msS * 1e-3)
    log(f"one batch per launch, {args.streams} streams: {multi:.3e} rows/s")
    floor_us = launch_floor(500)
    log(f"empty-launch floor (events): {floor_us:.2f} us")
    lat = None
    if args.single_rows:
        lat = single_row_latency(args.single_rows)
        log(f"C1 single row: p50 {lat['p50_us']:.2f} us (GPU), host p50 {lat['host_p50_us']:.2f} us")
    others = None
    if not args.no_other:
        others = other_configs(200)
        others["RAS"] = ras_latency(500)
        others["head"] = head_latency(300)
        others.update(frame_latency(300))
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic_k_wave_C3.json")
    if os.path.exists(tpath):
        t = json.load(open(tpath))
        if t.get("batches_per_launch") == G:
            traffic = t.get("hbm_bytes_per_launch")
    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        cpu = cpu_baseline(args.cpu_seconds)
        log(f"cpu: {cpu['value']:.3e} rows/s on {cpu['cores']} threads; C1 row on one thread "
            f"{cpu['c1_row_us_1_thread']:.1f} us")
    out = {
        "metric": METRIC,
        "value": value,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": launches,
        "warmup": args.warmup,
        "ms_per_step": ms / launches,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "C3 batched backbone head: fp32 logits [256,4097], N(0,2.5) + 1-8 "
                               "peaks, rows 0-127 T 0.7/top_p 0.7, rows 128-255 T 1.0/top_p 0.9, "
                               "top_k 30, per-row Philox uniforms",
                   "global_batch": ROWS, "vocab": V, "k": K, "pool_MB": round(pool_mb),
                   "step": f"one d3s_sample launch of {G} batches of 256 rows ({G * ROWS} rows)",
                   "steady_state": f"multi-batch launches: {G} batches per d3s_sample call, "
                                   f"taken in turn by {S} streams",
                   "batches_per_launch": G, "streams": S,
                   "prewarm": f"{prewarm_launches} untimed launches over {PREWARM_S} s before the "
                              f"first phase (clocks settle)",
                   "settle": f"{n_settle} untimed launches ({SETTLE_S * 1e3:.0f} ms) back to back with "
                             f"the --warmup launches before each timed phase: sustained load runs "
                             f"slower for its first ~30 ms"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "kernel_us_mean": kmean, "bytes_per_launch": bytes_per_launch,
                     "kernel": "k_wave<17, fp32> (one wave per row)",
                     "launches": "one stream, back to back (the kernel's own duration)",
                     "whole_job": {"GBs": job_gbs, "frac": job_gbs / HBM_PEAK_GBS, "streams": S}},
        "cpu_baseline": cpu,
        "one_batch_per_launch": {"rows_per_s": single, "us_per_launch": ms1 * 1e3 / l1,
                                 "rows_per_s_streams": multi, "streams": args.streams},
        "p50_us_single_row": lat["p50_us"] if lat else None,
        "event_floor_us": floor_us,
        "single_row": lat,
        "single_row_c_caller": c_lat,
        "other_configs": others,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
