"""CPU checks of the C-ABI library and the host mirror (no GPU compute).

librq.so must load, export every symbol include/rq.h declares, and answer
host-side questions (geometry, argument checks, missing device) without a GPU.
The product package must not route through the oracle.
"""
import ctypes
import os
import re

import numpy as np
import pytest

from rllm_amd import _lib
from rllm_amd.dtype import DType
from rllm_amd.errors import BackendError, RllmError, ShapeError, UnsupportedError

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_declared_symbol():
    declared = _lib.declared_symbols()
    assert len(declared) >= 15
    L = _lib.lib()
    missing = [s for s in declared if not hasattr(L, s)]
    assert not missing, f"declared in include/rq.h but not exported: {missing}"
    # and nothing the bindings use is undeclared
    assert set(_lib._SIGNATURES) <= set(declared)


def test_exported_symbols_are_only_the_abi():
    import subprocess

    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True).stdout
    funcs = sorted(l.split()[-1] for l in out.splitlines() if " T " in l)
    assert funcs == _lib.declared_symbols()


def test_row_bytes_matches_geometry(orc):
    L = _lib.lib()
    for t in DType:
        for cols in (256, 512, 4096, 14336):
            assert L.rq_row_bytes(int(t), cols) == t.row_bytes(cols) == orc.row_bytes(int(t), cols)
    assert L.rq_row_bytes(12, 100) == -1
    assert L.rq_row_bytes(0, 256) == -1  # F32 is not served by this library
    assert L.rq_row_bytes(8, 32) == 34


def test_dtype_mirror():
    assert DType.from_ggml(12) is DType.Q4_K
    assert DType.from_ggml(13) is None
    assert [t.block_size for t in DType] == [32, 32, 256, 256]
    assert str(DType.Q6_K) == "Q6_K"
    with pytest.raises(ValueError):
        DType.Q4_K.row_bytes(300)


def test_null_arguments_are_rejected():
    L = _lib.lib()
    h = ctypes.c_void_p()
    assert L.rq_upload(None, 12, 1, 256, None, 0, ctypes.byref(h)) == _lib.RQ_ERR_INVALID
    assert "null" in _lib.last_error()
    assert L.rq_matmul(None, None, 0, 1, None, None, 0) == _lib.RQ_ERR_INVALID
    assert L.rq_set_stream(None, None) == _lib.RQ_ERR_INVALID
    assert L.rq_open(0, None) == _lib.RQ_ERR_INVALID
    assert L.rq_close(None) == _lib.RQ_OK
    assert L.rq_weight_free(None) == _lib.RQ_OK


def test_open_without_device_is_a_backend_error():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    ctx = ctypes.c_void_p()
    st = _lib.lib().rq_open(0, ctypes.byref(ctx))
    assert st == _lib.RQ_ERR_BACKEND
    assert re.match(r"\w+: \w+ \(\d+\)", _lib.last_error()), _lib.last_error()
    with pytest.raises(BackendError):
        _lib.check(st)


def test_status_mapping():
    for code, exc in ((_lib.RQ_ERR_SHAPE, ShapeError), (_lib.RQ_ERR_UNSUPPORTED, UnsupportedError),
                      (_lib.RQ_ERR_BACKEND, BackendError), (_lib.RQ_ERR_INVALID, RllmError)):
        with pytest.raises(exc):
            _lib.check(code)
    _lib.check(_lib.RQ_OK)


def test_host_tensor_as_2d():
    from rllm_amd.backend import HostTensor

    t = HostTensor("w", DType.Q4_K, (2, 3, 512), np.zeros(6 * 288, np.uint8))
    assert t.as_2d() == (6, 512)
    assert t.numel() == 6 * 512


def test_product_never_uses_the_oracle():
    """The shipped path has no CPU fallback: nothing under rllm_amd/ or
    include/ refers to the oracle."""
    for base in ("rllm_amd", "include"):
        for dirpath, _, files in os.walk(os.path.join(ROOT, base)):
            for f in files:
                if f.endswith((".py", ".cpp", ".h", ".hip")):
                    text = open(os.path.join(dirpath, f)).read()
                    for pat in (r"^\s*(from|import)\s+oracle", r"liborq", r"\borq_"):
                        assert not re.search(pat, text, flags=re.M), (os.path.join(dirpath, f), pat)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "librq.so"))
    with pytest.raises(RllmError, match="not built"):
        _lib.lib()


def test_timeline_library_exports_the_abi_and_its_reader():
    """librq_tl.so (the -DRQ_TIMELINE build bench.py --timeline loads)
    exports include/rq.h's symbols plus include/rq_timeline.h's, nothing
    else."""
    import subprocess

    from rllm_amd import build as rq_build

    if not os.path.exists(rq_build.TIMELINE_LIB):
        pytest.skip("librq_tl.so not built")
    out = subprocess.run(["nm", "-D", "--defined-only", rq_build.TIMELINE_LIB], capture_output=True, text=True,
                         check=True).stdout
    funcs = sorted(l.split()[-1] for l in out.splitlines() if " T " in l)
    want = sorted(_lib.declared_symbols() + _lib.declared_symbols(os.path.join(ROOT, "include", "rq_timeline.h")))
    assert funcs == want
