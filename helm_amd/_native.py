"""ctypes binding of libhelm_mi355x.so (the C ABI declared in include/helm_mi355x.h).

The library is loaded once, lazily.  A missing or unloadable library is an error
that names the cause: there is no CPU or pure-PyTorch fallback for any op.  A
non-zero return code becomes ``RuntimeError(helm_last_error())``, the way the
reference's TORCH_CHECKs surface (helm/kernels/fp16_gemv.cpp:110-126).
"""
from __future__ import annotations

import ctypes
import os
import pathlib
from typing import Optional

import torch

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libhelm_mi355x.so"

_lib: Optional[ctypes.CDLL] = None
_load_error: Optional[str] = None

_i32, _i64, _f32, _vp, _sz = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t

# name -> argtypes (every entry point returns int except where noted)
_SIGNATURES = {
    "helm_int8_gemv": [_vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _vp],
    "helm_fp16_gemv": [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _i32, _i32, _i32, _vp],
    "helm_int8_gemv_fused": [_vp, _i64, _vp, _f32, _vp, _i64, _vp, _vp, _vp, _vp, _i64,
                             _i32, _i32, _i32, _vp],
    "helm_int8_gemv_ws": [_vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _vp,
                          _i64, _vp],
    "helm_int8_gemv_swiglu": [_vp, _i64, _vp, _f32, _vp, _vp, _vp, _vp, _i64, _vp, _i64,
                              _i32, _i32, _i32, _vp],
    "helm_int8_gemm": [_vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _vp],
    "helm_paged_decode_attn": [_vp, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _i32, _i32,
                               _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _vp],
    "helm_decode_attn_fused": [_vp, _i64, _vp, _vp, _f32, _vp, _vp, _vp, _vp, _vp, _vp, _i64,
                               _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32,
                               _vp],
    "helm_decode_attn_fused_cs": [_vp, _i64, _vp, _vp, _f32, _vp, _vp, _i64, _vp, _vp, _vp, _vp,
                                  _i64, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                  _f32, _vp],
    "helm_prefill_attn": [_vp, _i64, _i64, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _f32,
                          _vp, _i64, _i64, _vp],
    "helm_prefill_attn_mask": [_vp, _i64, _i64, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32,
                               _f32, _vp, _i64, _i64, _vp, _vp, _i64, _i64, _vp],
    "helm_paged_attn_reduce": [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp],
    "helm_paged_decode_attn_noalloc": [_vp, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _i32, _i32,
                                       _i32, _i32, _i32, _i32, _i32, _f32, _vp],
    "helm_kv_append": [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp],
    "helm_stage_pages_h2d": [_vp, _vp, _vp, _i32, _i64, _sz, _vp, _vp],
    "helm_gather_pages_h2d": [_vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _vp],
    "helm_qk_norm_rope_cs": [_vp, _vp, _vp, _f32, _vp, _vp, _i64, _vp, _vp, _i32, _i32, _i32, _i32,
                             _vp],
    "helm_qk_norm_rope_append": [_vp, _vp, _vp, _f32, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32,
                                 _i32, _i32, _i32, _vp],
    "helm_rmsnorm": [_vp, _vp, _f32, _vp, _i32, _i32, _vp],
    "helm_silu_mul": [_vp, _vp, _vp, _i64, _vp],
    "helm_fp16_gemv_rmsnorm": [_vp, _i64, _vp, _f32, _vp, _i64, _vp, _i64, _i32, _i32, _i32, _vp],
    "helm_argmax_f16": [_vp, _i64, _i32, _i32, _vp, _vp],
    "helm_argmax_f16_ws": [_vp, _i64, _i32, _i32, _vp, _vp, _i64, _vp],
}
_OTHER = {
    "helm_last_error": ([], ctypes.c_char_p),
    "helm_version": ([], ctypes.c_char_p),
    "helm_paged_attn_workspace_floats": ([_i32, _i32, _i32, _i32], _i64),
    "helm_paged_attn_max_split_pages": ([], _i32),
    "helm_paged_attn_noalloc_max_floats": ([], _i64),
    "helm_argmax_workspace_bytes": ([_i32], _i64),
    "helm_int8_gemv_workspace_bytes": ([_i32, _i32, _i32], _i64),
}


def _load() -> None:
    global _lib, _load_error
    if _lib is not None or _load_error is not None:
        return
    path = os.environ.get("HELM_MI355X_LIB", str(LIB_PATH))
    try:
        lib = ctypes.CDLL(path)
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int
        for name, (argtypes, restype) in _OTHER.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = restype
        _lib = lib
    except (OSError, AttributeError) as e:
        _load_error = f"cannot load {path}: {e} (build it with `python -m helm_amd.build`)"


def is_available() -> bool:
    """True when libhelm_mi355x.so is loaded (mirrors helm/kernels/__init__.py:91-94)."""
    _load()
    return _lib is not None


def load_error() -> Optional[str]:
    """Why the library could not be loaded, or None (mirrors helm/kernels/__init__.py:97-100)."""
    _load()
    return _load_error


def lib() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError when it is missing."""
    _load()
    if _lib is None:
        raise RuntimeError(f"helm_amd native library unavailable: {_load_error}")
    return _lib


def exported_symbols() -> list:
    """Names of every C entry point this binding expects the library to export."""
    return sorted(list(_SIGNATURES) + list(_OTHER))


def check(rc: int) -> None:
    if rc != 0:
        msg = lib().helm_last_error().decode(errors="replace")
        raise RuntimeError(msg or f"helm_amd native call failed with code {rc}")


_bound: dict = {}


def call(name: str, *args) -> None:
    """Call entry point `name` and raise RuntimeError on a non-zero return."""
    f = _bound.get(name)
    if f is None:
        f = _bound[name] = getattr(lib(), name)
    check(f(*args))


def version() -> str:
    return lib().helm_version().decode()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_ptr(device: Optional[torch.device] = None) -> int:
    """hipStream_t of torch's current stream on `device` (as an int for ctypes).
    Read through torch's raw accessor where it has one (a few us less per call
    than building the Stream object, which the Python decode loops pay per kernel)."""
    if _raw_stream is not None:
        idx = device.index if device is not None and device.index is not None \
            else torch.cuda.current_device()
        return _raw_stream(idx)
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def require_cuda(*tensors: Optional[torch.Tensor], what: str = "helm_amd") -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(f"{what}: tensors must be on the GPU (got {t.device}); "
                               "this library has no CPU path")


def workspace_floats(B: int, Hq: int, D: int, total_splits: int) -> int:
    return int(lib().helm_paged_attn_workspace_floats(B, Hq, D, total_splits))
