"""ctypes binding of the CPU oracle (oracle/libd3s_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline.  The
product path (drama3-mlx_amd/) never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libd3s_oracle.so")

DTYPE_F32 = 0
DTYPE_BF16 = 1
BAD = 1
TOPP_EDGE = 2
RACE_EDGE = 4
ALL_MASKED = 8

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def build_native(out_dir):
    """Compile the oracle for the host it runs on (-O3 -march=native, the same
    flags otherwise) into out_dir; returns the library's path, or None when no
    C compiler is at hand.  The shipped build (oracle/Makefile) targets
    x86-64-v3 so that one binary runs on every host; this one is for timing
    the CPU baseline where it runs."""
    path = os.path.join(out_dir, "libd3s_oracle_native.so")
    cmd = ["gcc", "-O3", "-march=native", "-std=c11", "-fPIC", "-ffp-contract=off", "-fno-fast-math",
           "-fopenmp", "-shared", "-o", path, os.path.join(HERE, "d3s_oracle.c"), "-lm"]
    try:
        subprocess.run(cmd, check=True, capture_output=True)
    except (OSError, subprocess.CalledProcessError):
        return None
    return path


def use_library(path):
    """Load the oracle from `path` instead of oracle/libd3s_oracle.so (the
    native build of build_native) for the calls that follow."""
    global _lib
    _lib = None
    return lib(path)


def lib(path=None):
    global _lib
    if _lib is None:
        if path is None:
            path = LIB_PATH
            if not os.path.exists(LIB_PATH):
                build()
        L = ctypes.CDLL(path)
        vp, i64, f32, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int
        L.d3s_oracle_sample.argtypes = [vp, i32, i64, i64, i64, vp, i32, vp, vp, f32, f32, vp, vp,
                                        vp, vp, vp, vp, vp, i32, i32]
        L.d3s_oracle_sample.restype = i32
        for name in ("d3s_oracle_expf", "d3s_oracle_logf", "d3s_oracle_fix40", "d3s_oracle_fix40_exp",
                     "d3s_oracle_fixsum_gt_threshold", "d3s_oracle_fix40_unit", "d3s_oracle_expf_nonpos"):
            getattr(L, name).argtypes = [vp, vp, i64]
            getattr(L, name).restype = None
        L.d3s_oracle_div_rn.argtypes = [vp, f32, vp, i64]
        L.d3s_oracle_div_rn.restype = None
        L.d3s_oracle_u64_to_f32.argtypes = [ctypes.c_uint64]
        L.d3s_oracle_u64_to_f32.restype = f32
        L.d3s_oracle_philox.argtypes = [vp, vp, vp]
        L.d3s_oracle_philox.restype = None
        L.d3s_oracle_ras_select.argtypes = [vp, vp, i64, vp, i32, i32, i32, i32, i32, vp, vp]
        L.d3s_oracle_ras_select.restype = None
        L.d3s_oracle_linear_bf16.argtypes = [vp, vp, i64, i64, i64, vp]
        L.d3s_oracle_linear_bf16.restype = None
        L.d3s_oracle_uniform.argtypes = [ctypes.c_uint64, ctypes.c_uint64, i64, i64, vp]
        L.d3s_oracle_uniform.restype = None
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def sample(logits, u, temperature, top_p, banned=None, n_threads=1, row_stride=None, vocab=None,
           detail=True, op_graph=False):
    """Oracle sampling.  logits: float32 [N, >=V] or uint16 (bf16 bits) [N, >=V];
    u: float32 [N, k]; temperature / top_p: scalars or float32 [N] arrays.
    op_graph: every row in the op graph's order (the reference with
    D3_NO_FUSED_SAMPLER set); otherwise the order follows the reference's
    routing (src/sampling.c:197).
    Returns dict(ids, probs, cand, lse, flags, gaps); with detail=False only
    ids (no probabilities, candidates, lse or float64 boundary shadow)."""
    logits = np.ascontiguousarray(logits)
    if logits.dtype == np.float32:
        dtype = DTYPE_F32
    elif logits.dtype == np.uint16:
        dtype = DTYPE_BF16
    else:
        raise TypeError("logits must be float32 or uint16 (bf16 bits)")
    N = logits.shape[0]
    stride = logits.shape[1] if row_stride is None else row_stride
    V = stride if vocab is None else vocab
    u = np.ascontiguousarray(u, np.float32)
    k = u.shape[1]
    t_arr = t_s = None
    if np.ndim(temperature):
        t_arr = np.ascontiguousarray(temperature, np.float32)
        t_s = 0.0
    else:
        t_s = float(temperature)
    p_arr = p_s = None
    if np.ndim(top_p):
        p_arr = np.ascontiguousarray(top_p, np.float32)
        p_s = 0.0
    else:
        p_s = float(top_p)
    ban = None if banned is None else np.ascontiguousarray(banned, np.int32)
    ids = np.empty(N, np.int32)
    probs = np.empty((N, k), np.float32) if detail else None
    cand = np.empty((N, k), np.int32) if detail else None
    lse = np.empty(N, np.float32) if detail else None
    flags = np.empty(N, np.uint8) if detail else None
    gaps = np.empty((N, 2), np.float64) if detail else None
    rc = lib().d3s_oracle_sample(_p(logits), dtype, N, V, stride, _p(u), k, _p(t_arr), _p(p_arr), t_s,
                                 p_s, _p(ban), _p(ids), _p(probs), _p(cand), _p(lse), _p(flags),
                                 _p(gaps), 1 if op_graph else 0, n_threads)
    if rc != 0:
        raise ValueError("oracle rejected the arguments")
    return dict(ids=ids, probs=probs, cand=cand, lse=lse, flags=flags, gaps=gaps)


def expf(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().d3s_oracle_expf(_p(x), _p(out), x.size)
    return out


def logf(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().d3s_oracle_logf(_p(x), _p(out), x.size)
    return out


def fix40(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint64)
    lib().d3s_oracle_fix40(_p(x), _p(out), x.size)
    return out


def fix40_unit(e):
    e = np.ascontiguousarray(e, np.float32)
    out = np.empty(e.shape, np.uint64)
    lib().d3s_oracle_fix40_unit(_p(e), _p(out), e.size)
    return out


def expf_nonpos(a):
    a = np.ascontiguousarray(a, np.float32)
    out = np.empty(a.shape, np.float32)
    lib().d3s_oracle_expf_nonpos(_p(a), _p(out), a.size)
    return out


def fix40_exp(z):
    z = np.ascontiguousarray(z, np.float32)
    out = np.empty(z.shape, np.uint64)
    lib().d3s_oracle_fix40_exp(_p(z), _p(out), z.size)
    return out


def fixsum_gt_threshold(c):
    c = np.ascontiguousarray(c, np.float32)
    out = np.empty(c.shape, np.uint64)
    lib().d3s_oracle_fixsum_gt_threshold(_p(c), _p(out), c.size)
    return out


def div_rn(a, b):
    a = np.ascontiguousarray(a, np.float32)
    out = np.empty_like(a)
    lib().d3s_oracle_div_rn(_p(a), float(b), _p(out), a.size)
    return out


def u64_to_f32(v):
    return lib().d3s_oracle_u64_to_f32(int(v))


def philox(ctr, key):
    c = np.ascontiguousarray(ctr, np.uint32)
    k = np.ascontiguousarray(key, np.uint32)
    out = np.empty(4, np.uint32)
    lib().d3s_oracle_philox(_p(c), _p(k), _p(out))
    return out


def uniform(seed, stream0, rows, k):
    """u[r, j] = uniform draw j of stream (stream0 + r) under seed."""
    u = np.empty((rows, k), np.float32)
    lib().d3s_oracle_uniform(seed, stream0, rows, k, _p(u))
    return u


def ras_select(first, retry, history, eos_id, semantic_start, semantic_end, code_vocab):
    """The RAS selection (src/tower.c:405-409,:425-433) over the two draws'
    indices [N]; history int32 [N, H] (H may be 0).  Returns (main_tok, code0)."""
    first = np.ascontiguousarray(first, np.int32)
    retry = np.ascontiguousarray(retry, np.int32)
    N = first.shape[0]
    history = np.ascontiguousarray(history, np.int32).reshape(N, -1)
    main, code0 = np.empty(N, np.int32), np.empty(N, np.int32)
    lib().d3s_oracle_ras_select(_p(first), _p(retry), N, _p(history) if history.size else None,
                                history.shape[1], eos_id, semantic_start, semantic_end, code_vocab,
                                _p(main), _p(code0))
    return main, code0


def ras(logits, u, u_retry, params, history, n_threads=1):
    """Both RAS draws of every row and the selection: the oracle of
    d3s_sample_ras.  params: dict of d3s_ras_params' fields (the retry's
    default to RAS_TEMPERATURE / RAS_TOP_P / RAS_TOP_K); the draws' k are
    u's and u_retry's widths."""
    p = dict(retry_temperature=1.0, retry_top_p=0.95, retry_top_k=30)  # src/tower.c:13-16
    p.update(params)
    first = sample(logits, u, p["temperature"], p["top_p"], n_threads=n_threads)["ids"]
    retry = sample(logits, u_retry, p["retry_temperature"], p["retry_top_p"], n_threads=n_threads)["ids"]
    main, code0 = ras_select(first, retry, history, p["eos_id"], p["semantic_start"],
                             p["semantic_end"], p["code_vocab"])
    return dict(first=first, retry=retry, main=main, code0=code0)


def linear_bf16(x, w):
    """The reference's single-row gemv (bf16 bits in and out): x uint16 [N, K],
    w uint16 [V, K] -> uint16 [N, V]."""
    x = np.ascontiguousarray(x, np.uint16)
    w = np.ascontiguousarray(w, np.uint16)
    N, K = x.shape
    V = w.shape[0]
    assert w.shape[1] == K and K % 128 == 0
    y = np.empty((N, V), np.uint16)
    lib().d3s_oracle_linear_bf16(_p(x), _p(w), N, K, V, _p(y))
    return y
