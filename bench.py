"""Benchmark of the MI355X token sampler on BASELINE.json's configurations.

Headline (`value`): sampled rows/s on C3, the batched backbone head
(fp32 [256, 4097], per-row T/top_p, k = 30), one d3s_sample launch per batch
of 256 rows, batches rotating over a pool larger than 512 MB so every launch
reads HBM rather than the 256 MB Infinity Cache.  `--streams S` spreads the
batches over S HIP streams (independent batches in flight, as a server would
have); the single-stream rate is reported beside it.

roofline.achieved = algorithmic bytes per launch (16 524 B per row)
divided by the kernel's mean duration, timed with HIP events around each
launch on its own stream.  cpu_baseline = the C oracle (the port of the
reference semantics; the reference's own CPU path needs mlx-c, absent here)
on a bounded sample of the same workload, all host cores.
Also reported: p50 / p90 of single-row C1 launches ([1, 4097] fp32).
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
BYTES_PER_ROW = V * 4 + K * 4 + 4 + 12  # logits, uniforms, id, (T, top_p, k)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_pool(n_batches, n_distinct):
    """n_batches device batches of C3 (fp32 [256, 4097]) cycling over
    n_distinct generated batches, each with its own device uniforms."""
    import d3s
    import d3s_workloads as W
    import hiprt
    batches = []
    distinct = [W.make("C3", rows=ROWS, seed=1000 + i, uniforms=False) for i in range(n_distinct)]
    for b in range(n_batches):
        w = distinct[b % n_distinct]
        lg = hiprt.to_device(w["logits"])
        u = hiprt.DeviceBuffer(4 * ROWS * K)
        assert d3s.lib().d3s_uniform_fill(u.ptr, ROWS * K, 42, b, None) == 0
        batches.append((lg, u))
    params = (hiprt.to_device(distinct[0]["temperature"]), hiprt.to_device(distinct[0]["top_p"]))
    hiprt.synchronize()
    return batches, params


def launch(batch, params, ids, stream):
    import d3s
    lg, u = batch
    return d3s.sample_raw(lg.ptr, d3s.DTYPE_F32, ROWS, V, V, u.ptr, K, ("ptr", params[0].ptr),
                          ("ptr", params[1].ptr), None, ids.ptr, stream=stream)


def time_throughput(batches, params, steps, warmup, n_streams):
    import hiprt
    streams = [hiprt.Stream() for _ in range(n_streams)]
    ids = [hiprt.DeviceBuffer(4 * ROWS) for _ in range(n_streams)]
    nb = len(batches)
    for i in range(warmup):
        s = i % n_streams
        assert launch(batches[i % nb], params, ids[s], streams[s].ptr) == 0
    hiprt.synchronize()
    start, stop = hiprt.Event(), hiprt.Event()
    t0 = time.perf_counter()
    start.record(streams[0])
    # every stream waits for `start` implicitly through the device sync above;
    # the end is the last stream's event after all streams are joined
    for i in range(steps):
        s = i % n_streams
        assert launch(batches[i % nb], params, ids[s], streams[s].ptr) == 0
    for st in streams[1:]:
        st.synchronize()
    stop.record(streams[0])
    stop.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_ms(stop)
    hiprt.synchronize()
    for st in streams:
        st.destroy()
    return ms, wall


def time_kernel(batches, params, n):
    """Mean duration of one launch: n launches back to back on one stream,
    bracketed by HIP events recorded on that stream.  This is what a kernel
    trace reports as the kernel's duration plus the dispatch gap between two
    launches, so it is an upper bound of the traced mean."""
    import hiprt
    s = hiprt.Stream()
    ids = hiprt.DeviceBuffer(4 * ROWS)
    nb = len(batches)
    for i in range(50):
        assert launch(batches[i % nb], params, ids, s.ptr) == 0
    a, b = hiprt.Event(), hiprt.Event()
    a.record(s)
    for i in range(n):
        assert launch(batches[i % nb], params, ids, s.ptr) == 0
    b.record(s)
    b.synchronize()
    mean = a.elapsed_ms(b) * 1e3 / n
    a.destroy()
    b.destroy()
    s.destroy()
    return float(mean)


def traffic_probe(batches, params, n):
    """For rocprofv3 --pmc runs: one 256 MiB device-to-device copy (the
    calibration dispatch of known traffic: 256 MiB read, 256 MiB written),
    then n C3 launches on one stream."""
    import hiprt
    nbytes = 256 << 20
    src, dst = hiprt.DeviceBuffer(nbytes), hiprt.DeviceBuffer(nbytes)
    hiprt.synchronize()
    hiprt.check(hiprt.hip().hipMemcpyAsync(dst.ptr, src.ptr, nbytes, hiprt.D2D, None), "copy")
    hiprt.synchronize()
    ids = hiprt.DeviceBuffer(4 * ROWS)
    for i in range(n):
        assert launch(batches[i % len(batches)], params, ids, None) == 0
    hiprt.synchronize()
    log(f"traffic probe: 1 copy of {nbytes} B, {n} C3 launches")

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


def cpu_baseline(seconds):
    """The oracle on all host cores over a bounded sample of C3 rows."""
    import d3s_oracle
    import d3s_workloads as W
    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    w = W.make("C3", rows=ROWS, seed=7, uniforms=False)
    u = d3s_oracle.uniform(42, 0, ROWS, K)
    # calibrate, then run about `seconds` of work
    t0 = time.perf_counter()
    d3s_oracle.sample(w["logits"], u, w["temperature"], w["top_p"], n_threads=threads)
    per_batch = time.perf_counter() - t0
    n = max(1, int(seconds / max(per_batch, 1e-6)))
    t0 = time.perf_counter()
    for _ in range(n):
        d3s_oracle.sample(w["logits"], u, w["temperature"], w["top_p"], n_threads=threads)
    dt = time.perf_counter() - t0
    return dict(value=n * ROWS / dt, unit="rows/s", cores=int(threads), kind="port",
                sample=f"{n} batches x {ROWS} rows of C3 (fp32 [256,4097], k=30), C oracle "
                       f"(-O2, OpenMP over rows) on {threads} threads, {dt:.1f} s")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20000)
    ap.add_argument("--warmup", type=int, default=500)
    ap.add_argument("--streams", type=int, default=4)
    ap.add_argument("--pool-batches", type=int, default=128)
    ap.add_argument("--single-rows", type=int, default=10000)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--traffic-probe", type=int, default=0, metavar="N",
                    help="only run the copy calibration and N C3 launches (for --pmc runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build targets one GPU; --gpus {args.gpus} is not supported "
              "(rows are independent: N GPUs would each run this kernel on N/G rows)",
              file=sys.stderr)
        sys.exit(2)
    import hiprt
    if hiprt.device_count() < 1:
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    import d3s
    d3s.lib()

    log("building the C3 batch pool")
    batches, params = build_pool(args.pool_batches, 16)
    pool_mb = args.pool_batches * ROWS * BYTES_PER_ROW / 1e6
    log(f"pool: {args.pool_batches} batches, {pool_mb:.0f} MB")
    if args.traffic_probe:
        traffic_probe(batches, params, args.traffic_probe)
        return
    ms, wall = time_throughput(batches, params, args.steps, args.warmup, args.streams)
    value = args.steps * ROWS / (ms * 1e-3)
    log(f"throughput: {args.steps} launches on {args.streams} streams in {ms:.2f} ms "
        f"({value:.3e} rows/s, host wall {wall:.3f} s)")
    ms1, _ = time_throughput(batches, params, min(args.steps, 5000), 100, 1)
    single_stream = min(args.steps, 5000) * ROWS / (ms1 * 1e-3)
    log(f"single stream: {single_stream:.3e} rows/s ({ms1 / min(args.steps, 5000) * 1e3:.2f} us/launch)")
    kmean = time_kernel(batches, params, 2000)
    bytes_per_launch = ROWS * BYTES_PER_ROW
    achieved = bytes_per_launch / (kmean * 1e-6) / 1e9
    log(f"kernel: {kmean:.2f} us per launch back to back on one stream -> {achieved:.0f} GB/s")
    floor_us = launch_floor(500)
    log(f"empty-launch floor (events): {floor_us:.2f} us")
    lat = None
    if args.single_rows:
        lat = single_row_latency(args.single_rows)
        log(f"C1 single row: p50 {lat['p50_us']:.2f} us (GPU), host p50 {lat['host_p50_us']:.2f} us")
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic_C3.json")
    if os.path.exists(tpath):
        traffic = json.load(open(tpath)).get("hbm_bytes_per_launch")
    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        cpu = cpu_baseline(args.cpu_seconds)
        log(f"cpu: {cpu['value']:.3e} rows/s on {cpu['cores']} threads")
    out = {
        "metric": METRIC,
        "value": value,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "C3 batched backbone head: fp32 logits [256,4097], N(0,2.5) + 1-8 "
                               "peaks, rows 0-127 T 0.7/top_p 0.7, rows 128-255 T 1.0/top_p 0.9, "
                               "top_k 30, per-row Philox uniforms",
                   "global_batch": ROWS, "vocab": V, "k": K, "streams": args.streams,
                   "pool_MB": round(pool_mb), "step": "one d3s_sample launch over one batch"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "kernel_us_mean": kmean,
                     "bytes_per_launch": bytes_per_launch},
        "cpu_baseline": cpu,
        "single_stream_rows_per_s": single_stream,
        "p50_us_single_row": lat["p50_us"] if lat else None,
        "event_floor_us": floor_us,
        "single_row": lat,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
