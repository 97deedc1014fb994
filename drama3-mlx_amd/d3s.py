"""ctypes binding of libd3sampler.so, the MI355X token sampler.

The host-side counterpart of the reference's ctypes layer for this path
(tests/d3.py:211-217 binds d3_sample of src/testapi.c:155-166).  It loads the
in-tree library and fails loudly when it is missing: there is no CPU fallback.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libd3sampler.so")

DTYPE_F32 = 0
DTYPE_BF16 = 1
FLAG_GENERIC = 1
FLAG_EXACT_LSE = 2
FLAG_EXACT_SELECT = 4
FLAG_OP_GRAPH = 8
FLAG_ONE_LAUNCH = 16
COUNTER_REFUSED, COUNTER_ALL_MASKED, COUNTER_EXACT_SELECT, COUNTER_EXACT_LSE = range(4)
NUM_COUNTERS = 4
OK = 0
ERR_ARG = -1
ERR_UNSUPPORTED = -2
ERR_SCRATCH = -6
ERR_WORKSPACE = -7
SCRATCH_BYTES = 4 << 20
MAX_VOCAB = (1 << 24) - 1

_lib = None


class RasParams(ctypes.Structure):
    """d3s_ras_params (include/d3s_sampler.h)"""
    _fields_ = [("temperature", ctypes.c_float), ("top_p", ctypes.c_float), ("top_k", ctypes.c_int),
                ("retry_temperature", ctypes.c_float), ("retry_top_p", ctypes.c_float),
                ("retry_top_k", ctypes.c_int), ("eos_id", ctypes.c_int32),
                ("semantic_start", ctypes.c_int32), ("semantic_end", ctypes.c_int32),
                ("code_vocab", ctypes.c_int32)]


def ras_params(**kw):
    """RasParams from keyword fields; the retry defaults to the reference's
    RAS_TEMPERATURE / RAS_TOP_P / RAS_TOP_K (src/tower.c:13-16)."""
    d = dict(retry_temperature=1.0, retry_top_p=0.95, retry_top_k=30)
    d.update(kw)
    return RasParams(**d)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C drama3-mlx_amd` "
                               "(or __graft_entry__.build()); there is no fallback")
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, i32, f32, u32 = (ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float,
                                  ctypes.c_uint)
        L.d3s_sample.argtypes = [vp, i32, i64, i64, i64, vp, i32, vp, vp, f32, f32, vp, vp, vp, vp,
                                 vp, u32, vp]
        L.d3s_sample.restype = i32
        L.d3s_sample_noalloc.argtypes = [vp, i32, i64, i64, i64, vp, i32, vp, vp, f32, f32, vp, vp, vp, vp,
                                         vp, u32, vp]
        L.d3s_sample_noalloc.restype = i32
        L.d3s_sample_ws.argtypes = [vp, i32, i64, i64, i64, vp, i32, vp, vp, f32, f32, vp, vp, vp, vp,
                                    vp, u32, vp, i64, vp]
        L.d3s_sample_ws.restype = i32
        L.d3s_sample_seeded.argtypes = [vp, i32, i64, i64, i64, ctypes.c_uint64, ctypes.c_uint64, i32, vp, vp,
                                        f32, f32, vp, vp, vp, vp, vp, u32, vp]
        L.d3s_sample_seeded.restype = i32
        L.d3s_sample_workspace_bytes.argtypes = [i32, i64, i64, i32, u32]
        L.d3s_sample_workspace_bytes.restype = i64
        L.d3s_workspace_init.argtypes = [vp, i64, vp]
        L.d3s_workspace_init.restype = i32
        L.d3s_stream_workspace_release.argtypes = [vp]
        L.d3s_stream_workspace_release.restype = i32
        L.d3s_sample_ras_ws.argtypes = [vp, i32, i64, i64, i64, vp, vp, vp, i32,
                                        ctypes.POINTER(RasParams), vp, vp, vp, vp, vp, vp, i64, vp]
        L.d3s_sample_ras_ws.restype = i32
        L.d3s_sample_ras_workspace_bytes.argtypes = [i32, i64, i64, ctypes.POINTER(RasParams), i32]
        L.d3s_sample_ras_workspace_bytes.restype = i64
        L.d3s_linear_sample_bf16_ws.argtypes = [vp, vp, i64, i64, i64, vp, vp, i32, vp, vp, f32, f32, vp, vp,
                                                vp, vp, u32, vp, i64, vp]
        L.d3s_linear_sample_bf16_ws.restype = i32
        L.d3s_linear_sample_workspace_bytes.argtypes = [i64, i64, i64, i32, u32, i32]
        L.d3s_linear_sample_workspace_bytes.restype = i64
        L.d3s_sample_ras.argtypes = [vp, i32, i64, i64, i64, vp, vp, vp, i32,
                                     ctypes.POINTER(RasParams), vp, vp, vp, vp, vp, vp]
        L.d3s_sample_ras.restype = i32
        L.d3s_linear_bf16.argtypes = [vp, vp, i64, i64, i64, vp, vp]
        L.d3s_linear_bf16.restype = i32
        L.d3s_linear_sample_bf16.argtypes = [vp, vp, i64, i64, i64, vp, vp, i32, vp, vp, f32, f32, vp, vp,
                                             vp, vp, u32, vp]
        L.d3s_linear_sample_bf16.restype = i32
        L.d3s_uniform_fill.argtypes = [vp, i64, ctypes.c_uint64, ctypes.c_uint64, vp]
        L.d3s_uniform_fill.restype = i32
        L.d3s_max_k.argtypes = []
        L.d3s_max_k.restype = i32
        L.d3s_fused_max_vocab.argtypes = [i32]
        L.d3s_fused_max_vocab.restype = i32
        L.d3s_math_selftest.argtypes = [vp, vp, vp, vp, vp, i64, f32, vp]
        L.d3s_math_selftest.restype = i32
        L.d3s_exp2_selftest.argtypes = [vp, vp, i64, vp]
        L.d3s_exp2_selftest.restype = i32
        L.d3s_log2_selftest.argtypes = [vp, vp, i64, vp]
        L.d3s_log2_selftest.restype = i32
        L.d3s_version.argtypes = []
        L.d3s_version.restype = ctypes.c_char_p
        L.d3_sample.argtypes = [vp, i32, i32, f32, i32, f32, ctypes.c_ulonglong, vp]
        L.d3_sample.restype = None
        L.d3_sample_with_noise.argtypes = [vp, vp, i32, i32, i32, f32, f32, vp]
        L.d3_sample_with_noise.restype = None
        _lib = L
    return _lib


def sample_raw(logits, dtype, n_rows, vocab, row_stride, u, k, temperature, top_p, banned, ids,
               probs=None, cand=None, counters=None, flags=0, stream=None, noalloc=False, workspace=None):
    """d3s_sample (or d3s_sample_noalloc, or d3s_sample_ws with workspace =
    (address, bytes)) on device pointers (ints).  temperature / top_p: a
    float (scalar) or a device pointer wrapped as ("ptr", address)."""
    t_ptr, t_s = (temperature[1], 0.0) if isinstance(temperature, tuple) else (None, float(temperature))
    p_ptr, p_s = (top_p[1], 0.0) if isinstance(top_p, tuple) else (None, float(top_p))
    if workspace is not None:
        return lib().d3s_sample_ws(logits, dtype, n_rows, vocab, row_stride, u, k, t_ptr, p_ptr, t_s, p_s,
                                   banned, ids, probs, cand, counters, flags, workspace[0], workspace[1], stream)
    fn = lib().d3s_sample_noalloc if noalloc else lib().d3s_sample
    return fn(logits, dtype, n_rows, vocab, row_stride, u, k, t_ptr, p_ptr, t_s, p_s,
              banned, ids, probs, cand, counters, flags, stream)


def sample_seeded_raw(logits, dtype, n_rows, vocab, row_stride, seed, draw, k, temperature, top_p, banned, ids,
                      probs=None, cand=None, counters=None, flags=0, stream=None):
    """d3s_sample_seeded on device pointers (ints): the uniforms drawn in the
    kernel from (seed, draw), as d3s_uniform_fill would write them.
    temperature / top_p as in sample_raw."""
    t_ptr, t_s = (temperature[1], 0.0) if isinstance(temperature, tuple) else (None, float(temperature))
    p_ptr, p_s = (top_p[1], 0.0) if isinstance(top_p, tuple) else (None, float(top_p))
    return lib().d3s_sample_seeded(logits, dtype, n_rows, vocab, row_stride, seed, draw, k, t_ptr, p_ptr, t_s,
                                   p_s, banned, ids, probs, cand, counters, flags, stream)


def workspace_bytes(dtype, n_rows, vocab, k, flags=0):
    """d3s_sample_workspace_bytes: the workspace d3s_sample_ws needs (or a
    negative status)."""
    return lib().d3s_sample_workspace_bytes(dtype, n_rows, vocab, k, flags)


class Workspace:
    """A caller-owned workspace for the *_ws entry points: device memory of
    `nbytes`, cleared once by d3s_workspace_init on `stream`."""

    def __init__(self, nbytes, stream=None):
        import hiprt
        self.nbytes = max(int(nbytes), 256)
        self.buf = hiprt.DeviceBuffer(self.nbytes)
        rc = lib().d3s_workspace_init(self.buf.ptr, self.nbytes, stream.ptr if stream else None)
        if rc != OK:
            raise RuntimeError(f"d3s_workspace_init: {rc}")

    def arg(self):
        return (self.buf.ptr, self.nbytes)

    def free(self):
        self.buf.free()


def sample(logits, u, temperature, top_p, banned=None, flags=0, want_probs=True, row_stride=None,
           vocab=None, stream=None, noalloc=False, workspace=None, seed_draw=None):
    """Host arrays in, host arrays out (copies through device memory).
    logits: float32 or uint16 (bf16 bits) [N, row_stride]; u: float32 [N, k];
    temperature / top_p: scalars or float32 [N].  seed_draw = (seed, draw):
    d3s_sample_seeded instead, u then an int, k.  Returns dict(ids, probs,
    cand, counters, rc)."""
    import hiprt
    logits = np.ascontiguousarray(logits)
    dtype = DTYPE_F32 if logits.dtype == np.float32 else DTYPE_BF16
    if logits.dtype not in (np.float32, np.uint16):
        raise TypeError("logits must be float32 or uint16 (bf16 bits)")
    N = logits.shape[0]
    stride = logits.shape[1] if row_stride is None else row_stride
    V = stride if vocab is None else vocab
    bufs = dict(logits=hiprt.to_device(logits), ids=hiprt.DeviceBuffer(4 * N),
                counters=hiprt.DeviceBuffer(4 * NUM_COUNTERS).zero())
    if seed_draw is None:
        u = np.ascontiguousarray(u, np.float32)
        k = u.shape[1]
        bufs["u"] = hiprt.to_device(u)
    else:
        k = int(u)
    if want_probs:
        bufs["probs"] = hiprt.DeviceBuffer(4 * N * k)
        bufs["cand"] = hiprt.DeviceBuffer(4 * N * k)
    T = float(temperature) if not np.ndim(temperature) else None
    if np.ndim(temperature):
        bufs["Tbuf"] = hiprt.to_device(np.asarray(temperature, np.float32))
        T = ("ptr", bufs["Tbuf"].ptr)
    P = float(top_p) if not np.ndim(top_p) else None
    if np.ndim(top_p):
        bufs["Pbuf"] = hiprt.to_device(np.asarray(top_p, np.float32))
        P = ("ptr", bufs["Pbuf"].ptr)
    ban = None
    if banned is not None:
        bufs["ban"] = hiprt.to_device(np.asarray(banned, np.int32))
        ban = bufs["ban"].ptr
    if seed_draw is not None:
        rc = sample_seeded_raw(bufs["logits"].ptr, dtype, N, V, stride, seed_draw[0], seed_draw[1], k, T, P,
                               ban, bufs["ids"].ptr, bufs["probs"].ptr if want_probs else None,
                               bufs["cand"].ptr if want_probs else None, bufs["counters"].ptr, flags,
                               stream.ptr if stream else None)
    else:
        rc = sample_raw(bufs["logits"].ptr, dtype, N, V, stride, bufs["u"].ptr, k, T, P, ban,
                        bufs["ids"].ptr, bufs["probs"].ptr if want_probs else None,
                        bufs["cand"].ptr if want_probs else None, bufs["counters"].ptr, flags,
                        stream.ptr if stream else None, noalloc=noalloc,
                        workspace=workspace.arg() if isinstance(workspace, Workspace) else workspace)
    out = dict(rc=rc)
    if rc != OK:
        return out
    hiprt.synchronize()
    out["ids"] = bufs["ids"].download((N,), np.int32)
    out["counters"] = bufs["counters"].download((NUM_COUNTERS,), np.uint32)
    if want_probs:
        out["probs"] = bufs["probs"].download((N, k), np.float32)
        out["cand"] = bufs["cand"].download((N, k), np.int32)
    for b in bufs.values():
        if isinstance(b, hiprt.DeviceBuffer):
            b.free()
    return out


def uniform_fill(n, seed, draw):
    import hiprt
    buf = hiprt.DeviceBuffer(4 * n)
    rc = lib().d3s_uniform_fill(buf.ptr, n, seed, draw, None)
    if rc != OK:
        raise RuntimeError(f"d3s_uniform_fill: {rc}")
    hiprt.synchronize()
    return buf.download((n,), np.float32)


def math_selftest(x, divisor):
    import hiprt
    x = np.ascontiguousarray(x, np.float32)
    n = x.size
    bi = hiprt.to_device(x)
    be, bl, bd, bf = (hiprt.DeviceBuffer(4 * n), hiprt.DeviceBuffer(4 * n), hiprt.DeviceBuffer(4 * n),
                      hiprt.DeviceBuffer(8 * n))
    rc = lib().d3s_math_selftest(bi.ptr, be.ptr, bl.ptr, bd.ptr, bf.ptr, n, divisor, None)
    if rc != OK:
        raise RuntimeError(f"d3s_math_selftest: {rc}")
    hiprt.synchronize()
    return (be.download((n,), np.float32), bl.download((n,), np.float32),
            bd.download((n,), np.float32), bf.download((n,), np.uint64))


def exp2_selftest(x):
    """The hardware 2^x (v_exp_f32) behind the wave kernel's fast row sum."""
    import hiprt
    x = np.ascontiguousarray(x, np.float32)
    bi, bo = hiprt.to_device(x), hiprt.DeviceBuffer(4 * x.size)
    rc = lib().d3s_exp2_selftest(bi.ptr, bo.ptr, x.size, None)
    if rc != OK:
        raise RuntimeError(f"d3s_exp2_selftest: {rc}")
    hiprt.synchronize()
    return bo.download((x.size,), np.float32)


def log2_selftest(x):
    """The hardware log2 x (v_log_f32) behind the wave kernel's fast row sum's log."""
    import hiprt
    x = np.ascontiguousarray(x, np.float32)
    bi, bo = hiprt.to_device(x), hiprt.DeviceBuffer(4 * x.size)
    rc = lib().d3s_log2_selftest(bi.ptr, bo.ptr, x.size, None)
    if rc != OK:
        raise RuntimeError(f"d3s_log2_selftest: {rc}")
    hiprt.synchronize()
    return bo.download((x.size,), np.float32)


def d3_sample(logits, temperature, top_k, top_p, seed):
    """The reference's test export (src/testapi.c:155-166): host fp32 logits,
    a seed, host ids."""
    logits = np.ascontiguousarray(logits, np.float32)
    out = np.zeros(len(logits), np.int32)
    lib().d3_sample(logits.ctypes.data, logits.shape[0], logits.shape[1], temperature, top_k, top_p,
                    seed, out.ctypes.data)
    return out


def d3_sample_with_noise(logits, u, temperature, top_p):
    logits = np.ascontiguousarray(logits, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.zeros(len(logits), np.int32)
    lib().d3_sample_with_noise(logits.ctypes.data, u.ctypes.data, logits.shape[0], logits.shape[1],
                               u.shape[1], temperature, top_p, out.ctypes.data)
    return out


def sample_ras_raw(logits, dtype, n_rows, vocab, row_stride, u, u_retry, history, history_len,
                   params, main_tok, code0=None, first_idx=None, retry_idx=None, counters=None,
                   stream=None):
    """d3s_sample_ras on device pointers (ints); params: RasParams."""
    return lib().d3s_sample_ras(logits, dtype, n_rows, vocab, row_stride, u, u_retry, history,
                                history_len, ctypes.byref(params) if params is not None else None,
                                main_tok, code0, first_idx, retry_idx, counters, stream)


def sample_ras(logits, u, u_retry, params, history=None, indices=True):
    """Host arrays in and out: logits float32 or uint16 (bf16 bits) [N, V];
    u [N, k], u_retry [N, k2]; history int32 [N, H] or None; params: dict of
    d3s_ras_params' fields; indices: ask for the two draws' indices too.
    Returns dict(rc, main, code0, first, retry, counters) (first / retry
    only with indices)."""
    import hiprt
    logits = np.ascontiguousarray(logits)
    dtype = DTYPE_F32 if logits.dtype == np.float32 else DTYPE_BF16
    N, V = logits.shape
    P = ras_params(**params)
    bufs = dict(logits=hiprt.to_device(logits), u=hiprt.to_device(np.ascontiguousarray(u, np.float32)),
                u2=hiprt.to_device(np.ascontiguousarray(u_retry, np.float32)),
                main=hiprt.DeviceBuffer(4 * N), code0=hiprt.DeviceBuffer(4 * N),
                first=hiprt.DeviceBuffer(4 * N), retry=hiprt.DeviceBuffer(4 * N),
                counters=hiprt.DeviceBuffer(4 * NUM_COUNTERS).zero())
    H = 0
    hist = None
    if history is not None and np.size(history):
        history = np.ascontiguousarray(history, np.int32).reshape(N, -1)
        H = history.shape[1]
        bufs["hist"] = hiprt.to_device(history)
        hist = bufs["hist"].ptr
    rc = sample_ras_raw(bufs["logits"].ptr, dtype, N, V, V, bufs["u"].ptr, bufs["u2"].ptr, hist, H, P,
                        bufs["main"].ptr, bufs["code0"].ptr, bufs["first"].ptr if indices else None,
                        bufs["retry"].ptr if indices else None, bufs["counters"].ptr)
    out = dict(rc=rc)
    if rc == OK:
        hiprt.synchronize()
        for name in ("main", "code0", "first", "retry") if indices else ("main", "code0"):
            out[name] = bufs[name].download((N,), np.int32)
        out["counters"] = bufs["counters"].download((NUM_COUNTERS,), np.uint32)
    for b in bufs.values():
        b.free()
    return out


def linear_bf16(x, w):
    """Host helper: x uint16 [N, K], w uint16 [V, K] (bf16 bits) -> uint16 [N, V]."""
    import hiprt
    x = np.ascontiguousarray(x, np.uint16)
    w = np.ascontiguousarray(w, np.uint16)
    N, K = x.shape
    V = w.shape[0]
    bx, bw, by = hiprt.to_device(x), hiprt.to_device(w), hiprt.DeviceBuffer(2 * N * V)
    rc = lib().d3s_linear_bf16(bx.ptr, bw.ptr, N, K, V, by.ptr, None)
    out = None
    if rc == OK:
        hiprt.synchronize()
        out = by.download((N, V), np.uint16)
    for b in (bx, bw, by):
        b.free()
    return rc, out



def linear_sample_bf16(x, w, u, temperature, top_p, flags=0, want_probs=True, keep_logits=True, stream=None):
    """Host helper for d3s_linear_sample_bf16: x uint16 [N, K], w uint16 [V, K]
    (bf16 bits), u float32 [N, k]; temperature / top_p scalars or float32 [N].
    Returns dict(rc, ids, probs, cand, counters, y) (y: the logits, uint16
    [N, V], when keep_logits)."""
    import hiprt
    x = np.ascontiguousarray(x, np.uint16)
    w = np.ascontiguousarray(w, np.uint16)
    u = np.ascontiguousarray(u, np.float32)
    N, K = x.shape
    V = w.shape[0]
    k = u.shape[1]
    bufs = dict(x=hiprt.to_device(x), w=hiprt.to_device(w), u=hiprt.to_device(u), ids=hiprt.DeviceBuffer(4 * N),
                counters=hiprt.DeviceBuffer(4 * NUM_COUNTERS).zero())
    if keep_logits:
        bufs["y"] = hiprt.DeviceBuffer(2 * N * V)
    if want_probs:
        bufs["probs"] = hiprt.DeviceBuffer(4 * N * k)
        bufs["cand"] = hiprt.DeviceBuffer(4 * N * k)
    t_ptr, t_s, p_ptr, p_s = None, 0.0, None, 0.0
    if np.ndim(temperature):
        bufs["T"] = hiprt.to_device(np.asarray(temperature, np.float32))
        t_ptr = bufs["T"].ptr
    else:
        t_s = float(temperature)
    if np.ndim(top_p):
        bufs["P"] = hiprt.to_device(np.asarray(top_p, np.float32))
        p_ptr = bufs["P"].ptr
    else:
        p_s = float(top_p)
    g = lambda name: bufs[name].ptr if name in bufs else None
    rc = lib().d3s_linear_sample_bf16(g("x"), g("w"), N, K, V, g("y"), g("u"), k, t_ptr, p_ptr, t_s, p_s,
                                      g("ids"), g("probs"), g("cand"), g("counters"), flags,
                                      stream.ptr if stream else None)
    out = dict(rc=rc)
    if rc == OK:
        hiprt.synchronize()
        out["ids"] = bufs["ids"].download((N,), np.int32)
        out["counters"] = bufs["counters"].download((NUM_COUNTERS,), np.uint32)
        if keep_logits:
            out["y"] = bufs["y"].download((N, V), np.uint16)
        if want_probs:
            out["probs"] = bufs["probs"].download((N, k), np.float32)
            out["cand"] = bufs["cand"].download((N, k), np.int32)
    for b in bufs.values():
        b.free()
    return out
