"""The C ABI library loads and exports every entry point the header declares.

CPU only: argument validation happens before anything touches the GPU, so the
error paths (negative return codes + helm_last_error) are exercised here too —
the counterpart of the reference's TORCH_CHECK errors (fp16_gemv.cpp:110-126).
"""
import ctypes
import pathlib
import re

import pytest

from helm_amd import _native

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "helm_mi355x.h"


def header_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(helm_[a-z0-9_]+)\s*\(", text)))


def test_library_loads():
    assert _native.is_available(), _native.load_error()
    assert _native.load_error() is None
    assert "gfx950" in _native.version()


def test_every_declared_symbol_is_exported():
    lib = ctypes.CDLL(str(_native.LIB_PATH))
    declared = header_functions()
    assert len(declared) >= 12
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, f"declared in helm_mi355x.h but not exported: {missing}"


def test_binding_matches_header():
    assert sorted(_native.exported_symbols()) == header_functions()


def _last_error():
    return _native.lib().helm_last_error().decode()


def test_gemv_rejects_null_pointer():
    rc = _native.lib().helm_int8_gemv(None, 16, None, 16, None, None, None, 16, 1, 16, 16, None)
    assert rc == -1
    assert "null pointer" in _last_error()


def test_gemv_rejects_large_m():
    fake = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    rc = _native.lib().helm_int8_gemv(fake, 16, fake, 16, fake, None, fake, 16, 17, 16, 16, None)
    assert rc == -2
    assert "M <= 16" in _last_error()


def test_gemv_rejects_unaligned_k():
    fake = ctypes.c_void_p(16)
    rc = _native.lib().helm_int8_gemv(fake, 24, fake, 24, fake, None, fake, 16, 1, 16, 24, None)
    assert rc == -2
    assert "multiple of 16" in _last_error()


def test_check_raises_runtime_error():
    _native.lib().helm_int8_gemv(None, 16, None, 16, None, None, None, 16, 1, 16, 16, None)
    with pytest.raises(RuntimeError, match="null pointer"):
        _native.check(-1)


def test_attention_rejects_bad_head_dim():
    fake = ctypes.c_void_p(16)
    rc = _native.lib().helm_paged_decode_attn(fake, 96, 96, fake, fake, 96, 96, fake, 4, fake, 8,
                                              fake, fake, 0, 4, 1, 8, 8, 96, 16, 4, 4, 0.1, None)
    assert rc == -2
    assert "head_dim" in _last_error()


def test_attention_rejects_split_overflow():
    fake = ctypes.c_void_p(16)
    rc = _native.lib().helm_paged_decode_attn(fake, 128, 128, fake, fake, 2048, 2048, fake, 4, fake,
                                              8, fake, fake, 3, 4, 1, 8, 8, 128, 16, 4, 2, 0.1, None)
    assert rc == -1
    assert "total_splits" in _last_error()


def test_gemm_rejects_k_not_multiple_of_64():
    fake = ctypes.c_void_p(16)
    rc = _native.lib().helm_int8_gemm(fake, 96, fake, 96, fake, None, fake, 16, 32, 16, 96, None)
    assert rc == -2


def test_workspace_size():
    assert _native.workspace_floats(1, 32, 128, 64) == 32 * 64 * 130
    assert _native.workspace_floats(0, 32, 128, 64) == 0


def test_ops_refuse_cpu_tensors():
    import torch
    from helm_amd.kernels import int8_linear
    x = torch.zeros(1, 16, dtype=torch.float16)
    q = torch.zeros(16, 16, dtype=torch.int8)
    s = torch.ones(16, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="GPU"):
        int8_linear(x, q, s)
