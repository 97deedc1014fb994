"""The C-ABI library: it loads, exports every function include/*.h declares,
and rejects bad arguments before touching the device (no GPU needed)."""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in sorted(os.listdir(os.path.join(ROOT, "include")))
           if h.endswith(".h")]


def declared_functions(path):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"#.*", "", text)
    names = set()
    for m in re.finditer(r"([A-Za-z_][A-Za-z0-9_]*)\s*\(([^()]*)\)\s*;", text):
        name = m.group(1)
        if name not in {"if", "while", "for", "return", "sizeof"}:
            names.add(name)
    return names


def exported_symbols(path):
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True,
                         check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


@pytest.fixture(scope="module")
def lib():
    import d3s
    return d3s.lib()


def test_headers_declare_the_reference_names():
    names = set().union(*(declared_functions(h) for h in HEADERS))
    for ref_name in ("sample_top_k_top_p", "sample_noise", "sample_with_noise", "m_seed",
                     "d3_sample", "d3s_sample"):
        assert ref_name in names


def test_library_exports_every_declared_function(lib):
    import d3s
    exported = exported_symbols(d3s.LIB_PATH)
    for h in HEADERS:
        missing = declared_functions(h) - exported
        assert not missing, (os.path.basename(h), missing)


def test_host_queries(lib):
    assert lib.d3s_version().startswith(b"d3sampler")
    assert lib.d3s_max_k() == (1 << 24) - 1  # any k up to the vocab limit, D3S_MAX_VOCAB
    assert lib.d3s_fused_max_vocab(0) >= 4097 and lib.d3s_fused_max_vocab(1) >= 4096
    assert lib.d3s_fused_max_vocab(7) == -4


def test_argument_validation_without_device(lib):
    import d3s
    p = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation
    base = dict(logits=p.value, dtype=0, n_rows=4, vocab=100, row_stride=100, u=p.value, k=10,
                temperature=1.0, top_p=0.9, banned=None, ids=p.value)
    assert d3s.sample_raw(**{**base, "dtype": 5}) == -4
    assert d3s.sample_raw(**{**base, "k": 0}) == -1
    assert d3s.sample_raw(**{**base, "k": 101}) == -1
    assert d3s.sample_raw(**{**base, "row_stride": 99}) == -1
    assert d3s.sample_raw(**{**base, "vocab": 0, "row_stride": 0}) == -1
    assert d3s.sample_raw(**{**base, "n_rows": -1}) == -1
    assert d3s.sample_raw(**{**base, "ids": None}) == -1
    assert d3s.sample_raw(**{**base, "flags": 64}) == -1
    assert d3s.sample_raw(**{**base, "flags": 16}) == -1  # 1, 2, 4, 8 are flags; 16 is not
    assert d3s.sample_raw(**{**base, "flags": 2 | 64}) == -1
    huge = dict(base, vocab=1 << 24, row_stride=1 << 24)
    assert d3s.sample_raw(**huge) == -2  # beyond D3S_MAX_VOCAB (any k up to V is taken)
    assert d3s.sample_raw(**dict(base, vocab=(1 << 26) + 1, row_stride=(1 << 26) + 1)) == -2
    assert d3s.sample_raw(**{**base, "n_rows": 0}) == 0  # nothing to do, nothing launched


def test_seeded_validation_without_device(lib):
    """d3s_sample_seeded: d3s_sample's checks, and the routes whose kernels
    read u from memory refused before anything is launched."""
    import d3s
    p = ctypes.c_void_p(16)  # never dereferenced: every call below returns before a launch
    base = dict(logits=p.value, dtype=0, n_rows=4, vocab=100, row_stride=100, seed=1, draw=2, k=10,
                temperature=1.0, top_p=0.9, banned=None, ids=p.value)
    assert d3s.sample_seeded_raw(**{**base, "dtype": 5}) == -4
    assert d3s.sample_seeded_raw(**{**base, "k": 0}) == -1
    assert d3s.sample_seeded_raw(**{**base, "k": 101}) == -1
    assert d3s.sample_seeded_raw(**{**base, "ids": None}) == -1
    assert d3s.sample_seeded_raw(**{**base, "flags": 64}) == -1
    assert d3s.sample_seeded_raw(**{**base, "n_rows": 0}) == 0
    assert d3s.sample_seeded_raw(**{**base, "flags": 1}) == -2  # D3S_FLAG_GENERIC
    assert d3s.sample_seeded_raw(**{**base, "k": 65}) == -2
    # rows longer than one wave's registers: 6141 fp32 / 8185 bf16 at a row start off 16 bytes
    assert d3s.sample_seeded_raw(**{**base, "vocab": 6142, "row_stride": 6142}) == -2
    assert d3s.sample_seeded_raw(**{**base, "dtype": 1, "vocab": 8186, "row_stride": 8186}) == -2
    assert d3s.sample_seeded_raw(**{**base, "n_rows": 1025}) == -2  # more rows than one a workgroup


def test_product_fails_loudly_without_the_library(monkeypatch, tmp_path):
    """No CPU fallback: with the built library absent, the first call into the
    product raises instead of computing anything."""
    import d3s
    monkeypatch.setattr(d3s, "LIB_PATH", str(tmp_path / "libd3sampler.so"))
    monkeypatch.setattr(d3s, "_lib", None)
    with pytest.raises(RuntimeError, match="no fallback"):
        d3s.lib()
    with pytest.raises(RuntimeError, match="no fallback"):
        d3s.sample(np.zeros((1, 8), np.float32), np.zeros((1, 2), np.float32), 1.0, 0.9)
