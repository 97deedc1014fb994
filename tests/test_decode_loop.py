"""A 64-frame decode loop on one stream against the oracle's loop, frame by
frame: the sampler calls of tower_decode_step (src/tower.c:411-451) with the
main token's history fed back on the device, as generate() does
(src/generate.c:64-100: the last RAS_WINDOW_FRAMES = 16 main tokens,
src/generate.h:11).

Per frame: d3s_sample_ras on the backbone head's bf16 logits [1, 4097] (the
first draw with the caller's T / top_p / top_k, the retry with RAS_TEMPERATURE,
RAS_TOP_P, RAS_TOP_K = 1.0, 0.95, 30, src/tower.c:13-16) into frame[0..1], then
the nine codebook heads' d3s_sample on bf16 [1, 4096] into frame[2..10].  The
caller then shifts frame[0] into the 16-entry history with two device copies on
the same stream; nothing returns to the host until the 64 frames are done.
Logits are synthetic (the model's weights are not in the reference's tree):
the head's favour a few semantic codes, so the first draw often repeats a
recent main token and the retry replaces it.  Uniforms come from
d3s_uniform_fill, draw f * 11 + i for the i-th sampler of frame f, in the
order tower_decode_step draws them (src/tower.c:415-424).

The reference pins whole generations the same way, fused against
D3_NO_FUSED_SAMPLER over 64 frames (tests/test_fused.py:13-48); here each
mode runs against the oracle in the same order: the kernel's order in this
process, the op graph's in a child started with D3_NO_FUSED_SAMPLER=1."""
import os
import subprocess
import sys

import numpy as np
import pytest

import d3s_workloads as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EOS, START, CODES = 151645, 151669, 4096
MAP = dict(eos_id=EOS, semantic_start=START, semantic_end=START + CODES - 1, code_vocab=CODES)
FRAMES, BOOKS, K = 64, 9, 30
T, TOP_P = 0.8, 0.9  # tests/test_fused.py:27: temperature 0.8, top_k 30, top_p 0.9
SEED = 11


def loop_inputs(seed=SEED):
    """The head's and the codebooks' logits of every frame and the prompt's
    last 16 main tokens."""
    rng = np.random.default_rng(seed)
    favourites = 1 + rng.choice(CODES, 6, replace=False)  # candidate indices of six codes
    head = rng.standard_normal((FRAMES, 1 + CODES)) * 2.5
    head[:, favourites] += 8.0 + rng.random((FRAMES, 6))
    head[:, 0] -= 4.0  # eos rarely drawn
    books = rng.standard_normal((FRAMES, BOOKS, CODES)) * 2.0
    books += 3.0 * (rng.random((FRAMES, BOOKS, CODES)) < 0.002)
    hist0 = (START + rng.integers(0, CODES, 16)).astype(np.int32)
    hist0[-1] = START + favourites[0] - 1
    return dict(head=W.f32_to_bf16_bits(head.astype(np.float32)),
                books=W.f32_to_bf16_bits(books.astype(np.float32)), hist0=hist0)


def gpu_decode_loop(data):
    """The 64 frames on one stream; returns int32 [64, 11]."""
    import d3s
    import hiprt
    H = hiprt.hip()
    L = d3s.lib()
    s = hiprt.Stream()
    head, books = data["head"], data["books"]
    dh, db = hiprt.to_device(head), hiprt.to_device(books)
    du = hiprt.DeviceBuffer(4 * FRAMES * 11 * K)
    for f in range(FRAMES):
        for i in range(11):
            assert L.d3s_uniform_fill(du.ptr + 4 * K * (11 * f + i), K, SEED, 11 * f + i, s.ptr) == 0
    hist = [hiprt.to_device(data["hist0"]), hiprt.DeviceBuffer(4 * 16)]
    frames = hiprt.DeviceBuffer(4 * FRAMES * 11)
    P = d3s.ras_params(temperature=T, top_p=TOP_P, top_k=K, **MAP)
    cur = 0
    for f in range(FRAMES):
        fr = frames.ptr + 4 * 11 * f
        uf = du.ptr + 4 * K * 11 * f
        rc = d3s.sample_ras_raw(dh.ptr + 2 * (1 + CODES) * f, d3s.DTYPE_BF16, 1, 1 + CODES, 1 + CODES, uf,
                                uf + 4 * K, hist[cur].ptr, 16, P, fr, fr + 4, stream=s.ptr)
        assert rc == 0, (f, rc)
        for j in range(BOOKS):
            rc = d3s.sample_raw(db.ptr + 2 * CODES * (BOOKS * f + j), d3s.DTYPE_BF16, 1, CODES, CODES,
                                uf + 4 * K * (2 + j), K, T, TOP_P, None, fr + 4 * (2 + j), stream=s.ptr)
            assert rc == 0, (f, j, rc)
        # the caller's history on the device: the last 15 entries, then this frame's main token
        nxt = 1 - cur
        hiprt.check(H.hipMemcpyAsync(hist[nxt].ptr, hist[cur].ptr + 4, 4 * 15, hiprt.D2D, s.ptr), "shift")
        hiprt.check(H.hipMemcpyAsync(hist[nxt].ptr + 4 * 15, fr, 4, hiprt.D2D, s.ptr), "append")
        cur = nxt
    s.synchronize()
    out = frames.download((FRAMES, 11), np.int32)
    for b in (dh, db, du, frames, *hist):
        b.free()
    s.destroy()
    return out


def oracle_decode_loop(oracle, data, op_graph):
    """The same loop on the oracle; returns (frames int32 [64, 11], per frame
    whether the first draw repeated a recent main token)."""
    hist = list(data["hist0"])
    frames, repeated = [], []
    for f in range(FRAMES):
        u = [oracle.uniform(SEED, 11 * f + i, 1, K) for i in range(11)]
        x = data["head"][f:f + 1]
        first = oracle.sample(x, u[0], T, TOP_P, op_graph=op_graph)["ids"]
        retry = oracle.sample(x, u[1], 1.0, 0.95, op_graph=op_graph)["ids"]
        main, code0 = oracle.ras_select(first, retry, np.array([hist], np.int32), **MAP)
        tok = EOS if first[0] == 0 else START + int(first[0]) - 1
        repeated.append(tok in hist and tok != EOS)
        codes = [int(oracle.sample(data["books"][f, j:j + 1], u[2 + j], T, TOP_P, op_graph=op_graph)["ids"][0])
                 for j in range(BOOKS)]
        frames.append([int(main[0]), int(code0[0])] + codes)
        hist = hist[1:] + [int(main[0])]
    return np.array(frames, np.int32), np.array(repeated)


def _check(got, exp, repeated, label):
    bad = np.nonzero(np.any(got != exp, axis=1))[0]
    print(f"[decode-loop] {label}: {FRAMES} frames, {len(bad)} differ, {int(repeated.sum())} took the retry",
          flush=True)
    assert len(bad) == 0, (label, bad[:4], got[bad[:4]], exp[bad[:4]])
    assert 0 < repeated.sum() < FRAMES  # both outcomes of the repeat test occur


@pytest.mark.gpu
def test_decode_loop_kernel_order(oracle):
    import hiprt
    if hiprt.device_count() < 1:
        pytest.skip("no GPU")
    os.environ.pop("D3_NO_FUSED_SAMPLER", None)
    data = loop_inputs()
    exp, repeated = oracle_decode_loop(oracle, data, op_graph=False)
    _check(gpu_decode_loop(data), exp, repeated, "kernel order")


CHILD = """
import sys
import numpy as np
sys.path[:0] = [{pkg!r}, {oracle!r}, {tests!r}]
import test_decode_loop as T
np.save({out!r}, T.gpu_decode_loop(T.loop_inputs()))
print("child ok", flush=True)
"""


@pytest.mark.gpu
def test_decode_loop_op_graph_order_in_a_fresh_process(oracle, tmp_path):
    """The loop in a child process started with D3_NO_FUSED_SAMPLER=1 (the
    switch src/sampling.c:197 reads): every frame as the oracle's op-graph
    order gives it.  The two modes' frames are also compared with each other,
    as tests/test_fused.py:43-48 does; they may differ only where a cut falls
    between the two summation orders."""
    import hiprt
    if hiprt.device_count() < 1:
        pytest.skip("no GPU")
    data = loop_inputs()
    out = tmp_path / "frames.npy"
    script = CHILD.format(pkg=os.path.join(ROOT, "drama3-mlx_amd"), oracle=os.path.join(ROOT, "oracle"),
                          tests=os.path.join(ROOT, "tests"), out=str(out))
    env = dict(os.environ, D3_NO_FUSED_SAMPLER="1")
    print("[decode-loop] child process with D3_NO_FUSED_SAMPLER=1", flush=True)
    r = subprocess.run([sys.executable, "-c", script], env=env, cwd=ROOT, timeout=300, capture_output=True,
                       text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    got = np.load(out)
    exp, repeated = oracle_decode_loop(oracle, data, op_graph=True)
    _check(got, exp, repeated, "op graph order (D3_NO_FUSED_SAMPLER=1)")
    kern, _ = oracle_decode_loop(oracle, data, op_graph=False)
    diff = int(np.sum(np.any(kern != exp, axis=1)))
    print(f"[decode-loop] frames where the two orders differ: {diff}", flush=True)


def test_oracle_loop_takes_both_outcomes(oracle):
    """CPU: the oracle's loop on these inputs repeats a recent token on some
    frames and not on others, in either order, and every code lies in its
    codebook (the loop the GPU test runs is not degenerate)."""
    data = loop_inputs()
    for op_graph in (False, True):
        frames, repeated = oracle_decode_loop(oracle, data, op_graph)
        assert 0 < repeated.sum() < FRAMES
        assert np.all((frames[:, 2:] >= 0) & (frames[:, 2:] < CODES))
        assert np.all((frames[:, 1] >= 0) & (frames[:, 1] < CODES))
