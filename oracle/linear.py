"""Oracle for the INT8 weight-only linear — TEST INFRASTRUCTURE ONLY.

The reference has no INT8 code; its linear is the fp16 GEMV of
helm/kernels/fp16_gemv.cpp:45-157 (fp32 accumulate, bias in fp32, one rounding
to fp16).  The INT8 arithmetic is the target path's definition: symmetric,
per-output-channel, 127 levels, dequant fused into the product.

Pinning (tests/test_oracle_linear.py):
  * int8_linear_exact: fp64 brute force; special case scale == 1 with an
    fp16-exact integer weight equals torch.nn.functional.linear in fp32;
    linearity in x; doubling every scale doubles y exactly.
  * gemv_ref.c (fp16_gemv / int8_gemv): agrees with int8_linear_exact to fp32
    accumulation error, and with torch's fp32 linear; its fp16 GEMV keeps the
    reference's summation order (4 x 8-lane accumulators, fp16_gemv.cpp:53-85).
  * quantize_per_channel: |W - q*s| <= s/2 per element, max |q| == 127 on
    every non-zero row, zero rows map to (q=0, s=0).
"""
from __future__ import annotations

import ctypes
import pathlib
import subprocess
from typing import Optional, Tuple

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB = HERE / "_build" / "liboracle_cpu.so"
_lib = None


def build() -> pathlib.Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def _load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = ctypes.CDLL(str(LIB))
        vp, i64 = ctypes.c_void_p, ctypes.c_int64
        lib.oracle_fp16_gemv.argtypes = [vp, vp, vp, vp, i64, i64, i64]
        lib.oracle_int8_gemv.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64]
        lib.oracle_int8_gemv_f32.argtypes = [vp, vp, vp, vp, i64, i64, i64]
        for f in (lib.oracle_fp16_gemv, lib.oracle_int8_gemv, lib.oracle_int8_gemv_f32):
            f.restype = None
        _lib = lib
    return _lib


def quantize_per_channel(w: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """(q int8 [N,K], scale fp16 [N]): scale = fp16(max|W_n|/127),
    q = clamp(round_half_even(W / scale), -127, 127), 0 where scale == 0."""
    w = np.asarray(w, dtype=np.float32)
    scale = (np.abs(w).max(axis=1) / np.float32(127.0)).astype(np.float16)
    s32 = scale.astype(np.float32)
    safe = np.where(s32 > 0, s32, np.float32(1.0))
    q = np.clip(np.rint(w / safe[:, None]), -127, 127)
    q[s32 == 0] = 0
    return q.astype(np.int8), scale


def int8_linear_exact(x: np.ndarray, q: np.ndarray, scale: np.ndarray,
                      bias: Optional[np.ndarray] = None) -> np.ndarray:
    """fp64 closed form y[m,n] = scale[n] * sum_k q[n,k] x[m,k] + bias[n] (unrounded)."""
    y = np.asarray(x, np.float64) @ np.asarray(q, np.float64).T
    y *= np.asarray(scale, np.float64)[None, :]
    if bias is not None:
        y += np.asarray(bias, np.float64)[None, :]
    return y


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def fp16_gemv(x: np.ndarray, w: np.ndarray, bias: Optional[np.ndarray] = None) -> np.ndarray:
    """The reference's fp16 GEMV (fp16_gemv.cpp:45-157), one GEMV per token row."""
    lib = _load()
    x = _c(np.atleast_2d(x), np.float16)
    w = _c(w, np.float16)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), np.float16)
    b = _c(bias, np.float16) if bias is not None else None
    lib.oracle_fp16_gemv(x.ctypes.data, w.ctypes.data, None if b is None else b.ctypes.data,
                         y.ctypes.data, M, N, K)
    return y


def int8_gemv(x: np.ndarray, q: np.ndarray, scale: np.ndarray,
              bias: Optional[np.ndarray] = None) -> np.ndarray:
    """INT8 weight-only GEMV with the reference GEMV's loop structure, fp16 out."""
    lib = _load()
    x = _c(np.atleast_2d(x), np.float16)
    q = _c(q, np.int8)
    s = _c(scale, np.float16)
    M, K = x.shape
    N = q.shape[0]
    y = np.empty((M, N), np.float16)
    b = _c(bias, np.float16) if bias is not None else None
    lib.oracle_int8_gemv(x.ctypes.data, q.ctypes.data, s.ctypes.data,
                         None if b is None else b.ctypes.data, y.ctypes.data, M, N, K)
    return y


def int8_gemv_f32(x: np.ndarray, q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    lib = _load()
    x = _c(np.atleast_2d(x), np.float16)
    q = _c(q, np.int8)
    s = _c(scale, np.float16)
    M, K = x.shape
    N = q.shape[0]
    y = np.empty((M, N), np.float32)
    lib.oracle_int8_gemv_f32(x.ctypes.data, q.ctypes.data, s.ctypes.data, y.ctypes.data, M, N, K)
    return y


def fp16_round(a: np.ndarray) -> np.ndarray:
    return np.asarray(a).astype(np.float16).astype(np.float64)


def gemv_tolerance_ok(y_gpu: np.ndarray, y_exact: np.ndarray, rel: float = 1e-2) -> Tuple[bool, float]:
    """The GEMV/GEMM bar: |y - exact| <= rel * max(1, |exact|) elementwise, where
    exact is the fp64 (fp32-accumulation-free) result before fp16 rounding.
    Returns (ok, worst normalised error)."""
    y = np.asarray(y_gpu, np.float64)
    e = np.abs(y - y_exact) / np.maximum(1.0, np.abs(y_exact))
    worst = float(e.max()) if e.size else 0.0
    return worst <= rel, worst
