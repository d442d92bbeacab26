"""helm_amd.kernels — INT8 weight-only linear on MI355X (gfx950).

Mirrors the reference's linear operator binding (helm/kernels/__init__.py):

=====================================  =============================================
reference (helm/kernels/__init__.py)   here
=====================================  =============================================
fp16_linear(input, weight, bias)       fp16_linear (GPU fp16 GEMV, :55-88)
  :55-88                               int8_linear(input, qweight, scale, bias)
_AVXLinear(linear) :107-130            Int8Linear(linear) / Int8Linear.from_linear
patch_cpu_linears(module, verbose)     patch_linears(module, verbose, exclude) (INT8);
  :133-157                             patch_cpu_linears / patch_fp16_linears (fp16
                                       weights kept, FP16Linear = _AVXLinear)
HELM_DISABLE_AVX (env) :80             HELM_DISABLE_GEMV (env): fp16_linear decode calls
                                       take the fp32 F.linear branch (ablation)
is_available() :91-94                  is_available()
load_error() :97-100                   load_error()
=====================================  =============================================

Dispatch follows the reference's shape rule (fp16_linear :72-88): a call whose
leading dims multiply to <= 16 tokens is a decode GEMV (helm_int8_gemv_ws /
helm_fp16_gemv), a larger one a prefill GEMM (helm_int8_gemm on MFMA).  Unlike the
reference there is no fallback: a missing library or a CPU tensor raises
RuntimeError.
"""
from __future__ import annotations

import functools
import os
from typing import Iterable, Optional, Tuple

import torch
import torch.nn as nn

from .. import _native
from .._native import is_available, load_error

__all__ = [
    "int8_linear", "fp16_linear", "quantize_per_channel", "dequantize",
    "Int8Linear", "patch_linears", "FP16Linear", "patch_fp16_linears", "patch_cpu_linears",
    "is_available", "load_error", "GEMV_MAX_TOKENS",
]

GEMV_MAX_TOKENS = 16


def quantize_per_channel(weight: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Symmetric per-output-channel INT8 quantisation of a [N, K] weight.

    scale[n] = fp16(max_k |W[n, k]| / 127)
    q[n, k]  = clamp(round_half_even(W[n, k] / scale[n]), -127, 127)   (0 if scale[n] == 0)

    The division uses the fp16-rounded scale, so ``q * scale`` is the weight the
    kernels actually apply.
    """
    if weight.dim() != 2:
        raise ValueError(f"quantize_per_channel: expected a 2-D weight, got {tuple(weight.shape)}")
    w = weight.detach().float()
    amax = w.abs().amax(dim=1)
    scale = (amax / 127.0).to(torch.float16)
    s32 = scale.float()
    safe = torch.where(s32 > 0, s32, torch.ones_like(s32))
    q = torch.round(w / safe[:, None]).clamp_(-127, 127)
    q[s32 == 0] = 0
    return q.to(torch.int8).contiguous(), scale.contiguous()


def dequantize(qweight: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """fp32 [N, K] weight represented by (qweight, scale)."""
    return qweight.float() * scale.float()[:, None]


def _flatten(x: torch.Tensor, K: int, what: str) -> torch.Tensor:
    if x.shape[-1] != K:
        raise RuntimeError(f"{what}: input last dim ({x.shape[-1]}) != weight K ({K})")
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 != 0 or x2.data_ptr() % 16 != 0:
        x2 = x2.contiguous()
    return x2


def int8_linear(input: torch.Tensor, qweight: torch.Tensor, scale: torch.Tensor,
                bias: Optional[torch.Tensor] = None,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = fp16(scale * (input @ qweight.T) + bias) on the GPU, fp32 accumulate.

    input [..., K] fp16, qweight [N, K] int8 (row-major), scale [N] fp16, bias [N]
    fp16 or None.  Decode (<= 16 tokens) runs the GEMV, prefill the MFMA GEMM.
    """
    _native.require_cuda(input, qweight, scale, bias, what="int8_linear")
    if input.dtype != torch.float16:
        raise RuntimeError(f"int8_linear: input must be fp16 (got {input.dtype})")
    if qweight.dtype != torch.int8 or qweight.dim() != 2 or not qweight.is_contiguous():
        raise RuntimeError("int8_linear: qweight must be a contiguous 2-D int8 tensor")
    N, K = qweight.shape
    if scale.dtype != torch.float16 or scale.numel() != N:
        raise RuntimeError("int8_linear: scale must be fp16 [N]")
    if bias is not None and (bias.dtype != torch.float16 or bias.numel() != N):
        raise RuntimeError("int8_linear: bias must be fp16 [N]")
    x2 = _flatten(input, K, "int8_linear")
    M = x2.shape[0]
    lead = input.shape[:-1]
    if out is None:
        out = torch.empty(*lead, N, dtype=torch.float16, device=input.device)
    y2 = out.view(-1, N)
    if M == 0:
        return out
    stream = _native.stream_ptr(input.device)
    if M <= GEMV_MAX_TOKENS:
        ws_bytes = gemv_workspace_bytes(M, N, K)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=input.device) if ws_bytes else None
        _native.call("helm_int8_gemv_ws", x2.data_ptr(), x2.stride(0), qweight.data_ptr(),
                     qweight.stride(0), scale.data_ptr(), _native.ptr(bias), None, y2.data_ptr(),
                     y2.stride(0), M, N, K, _native.ptr(ws), ws_bytes, stream)
        return out
    _native.call("helm_int8_gemm", x2.data_ptr(), x2.stride(0), qweight.data_ptr(), qweight.stride(0),
                 scale.data_ptr(), _native.ptr(bias), y2.data_ptr(), y2.stride(0), M, N, K, stream)
    return out


@functools.lru_cache(maxsize=None)
def gemv_workspace_bytes(M: int, N: int, K: int) -> int:
    """Workspace helm_int8_gemv_ws uses at this shape (0: none): the split-K
    form's fp32 partial sums for 8-16 tokens over long K."""
    return int(_native.lib().helm_int8_gemv_workspace_bytes(int(M), int(N), int(K)))


def fp16_linear(input: torch.Tensor, weight: torch.Tensor,
                bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """GPU counterpart of the reference's fp16_linear (helm/kernels/__init__.py:55-88).

    Decode (<= 16 tokens): helm_fp16_gemv, fp32 accumulate, bias added in fp32,
    one rounding to fp16 (fp16_gemv.cpp:139-151).  Prefill: the arithmetic of
    the reference's prefill branch (F.linear in fp32, :84-86) without its fp32
    copies: the fp16 product accumulated and returned in fp32 (torch.mm with
    out_dtype), the bias added in fp32, one rounding to fp16.  HELM_DISABLE_GEMV
    runs the reference's branch as written (F.linear on fp32 copies) for every
    call, as its HELM_DISABLE_AVX does (:80-86).
    """
    _native.require_cuda(input, weight, bias, what="fp16_linear")
    if input.dtype != torch.float16 or weight.dtype != torch.float16 or weight.dim() != 2:
        raise RuntimeError("fp16_linear: input and weight must be fp16, weight 2-D")
    N, K = weight.shape
    x2 = _flatten(input, K, "fp16_linear")
    M = x2.shape[0]
    if os.environ.get("HELM_DISABLE_GEMV"):
        b32 = bias.float() if bias is not None else None
        return torch.nn.functional.linear(input.float(), weight.float(), b32).half()
    if M > GEMV_MAX_TOKENS:
        try:
            y = torch.mm(x2, weight.t(), out_dtype=torch.float32)
        except RuntimeError:   # a torch without fp32-output fp16 products: the fp32 copies
            b32 = bias.float() if bias is not None else None
            return torch.nn.functional.linear(input.float(), weight.float(), b32).half()
        if bias is not None:
            y += bias.float()
        return y.half().view(*input.shape[:-1], N)
    w = weight if weight.is_contiguous() else weight.contiguous()
    out = torch.empty(*input.shape[:-1], N, dtype=torch.float16, device=input.device)
    if M == 0:
        return out
    _native.call("helm_fp16_gemv", x2.data_ptr(), x2.stride(0), w.data_ptr(), w.stride(0),
                 _native.ptr(bias), out.data_ptr(), N, M, N, K, _native.stream_ptr(input.device))
    return out


class Int8Linear(nn.Module):
    """INT8 weight-only replacement for nn.Linear (counterpart of _AVXLinear,
    helm/kernels/__init__.py:107-130).

    Buffers: ``qweight`` int8 [out, in], ``scale`` fp16 [out], optional ``bias``
    fp16 [out].  ``weight`` returns the dequantised fp16 weight (computed on
    access) so code that reads ``.weight.shape``/``.dtype`` keeps working.
    """

    def __init__(self, in_features: int, out_features: int, bias: bool = False,
                 device=None):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.register_buffer("qweight", torch.zeros(out_features, in_features, dtype=torch.int8,
                                                    device=device))
        self.register_buffer("scale", torch.zeros(out_features, dtype=torch.float16, device=device))
        self.register_buffer("bias", torch.zeros(out_features, dtype=torch.float16,
                                                 device=device) if bias else None)

    @classmethod
    def from_quantized(cls, qweight: torch.Tensor, scale: torch.Tensor,
                       bias: Optional[torch.Tensor] = None) -> "Int8Linear":
        mod = cls(qweight.shape[1], qweight.shape[0], bias=False, device="meta")
        mod.qweight = qweight
        mod.scale = scale
        mod.bias = bias
        return mod

    @classmethod
    def from_linear(cls, linear: nn.Linear) -> "Int8Linear":
        q, s = quantize_per_channel(linear.weight)
        b = linear.bias.detach().to(torch.float16) if linear.bias is not None else None
        return cls.from_quantized(q.to(linear.weight.device), s.to(linear.weight.device),
                                  None if b is None else b.to(linear.weight.device))

    @property
    def weight(self) -> torch.Tensor:
        return dequantize(self.qweight, self.scale).to(torch.float16)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return int8_linear(x, self.qweight, self.scale, self.bias)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, int8=True")


def patch_linears(module: nn.Module, verbose: bool = False,
                  exclude: Iterable[str] = ()) -> int:
    """Replace every nn.Linear under `module` with an Int8Linear (quantising its
    weight); returns the number replaced.  Counterpart of patch_cpu_linears
    (helm/kernels/__init__.py:133-157): walks children recursively and swaps leaf
    nn.Linear modules in place, graph structure unchanged.  Children whose
    attribute name is in `exclude` (e.g. "lm_head") are left as they are.

    Unlike the reference, which returns 0 when its extension failed to build,
    quantisation does not need the native library, so the count is returned
    either way; forward() is what requires the GPU library.
    """
    exclude = set(exclude)
    count = 0
    for name, child in list(module.named_children()):
        if name in exclude:
            continue
        if isinstance(child, nn.Linear):
            setattr(module, name, Int8Linear.from_linear(child))
            count += 1
        else:
            count += patch_linears(child, verbose=verbose, exclude=exclude)
    if verbose and count:
        print(f"[helm_amd.kernels] patched {count} nn.Linear -> Int8Linear under "
              f"{module.__class__.__name__}")
    return count


class FP16Linear(nn.Module):
    """fp16-weight wrapper of an nn.Linear (counterpart of _AVXLinear,
    helm/kernels/__init__.py:107-130): keeps the linear's ``weight`` and ``bias``
    by reference (no copy); fp16 input with fp16 GPU weights goes through
    fp16_linear (the fp16 GEMV for <= 16 tokens), anything else through F.linear,
    as the reference routes its non-CPU cases."""

    def __init__(self, linear: nn.Linear):
        super().__init__()
        self.weight = linear.weight
        self.bias = linear.bias

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.weight.dtype == torch.float16 and self.weight.is_cuda and x.dtype == torch.float16:
            return fp16_linear(x, self.weight, self.bias)
        return torch.nn.functional.linear(x, self.weight, self.bias)

    def extra_repr(self) -> str:
        return (f"in_features={self.weight.shape[1]}, out_features={self.weight.shape[0]}, "
                f"bias={self.bias is not None}, fp16_gemv=True")


def patch_fp16_linears(module: nn.Module, verbose: bool = False) -> int:
    """Replace every nn.Linear under `module` whose weight is fp16 on a GPU with
    FP16Linear; returns the number replaced (helm/kernels/__init__.py:133-157 with
    the GEMV's device: the reference patches fp16 CPU linears because its GEMV
    runs on the CPU).  Leaf modules only, graph structure unchanged; returns 0
    without touching the module when the native library is not available."""
    if not is_available():
        if verbose:
            print(f"[helm_amd.kernels] native library unavailable ({load_error()}); skipping patch")
        return 0
    count = 0
    for name, child in list(module.named_children()):
        if isinstance(child, nn.Linear):
            if child.weight.dtype == torch.float16 and child.weight.is_cuda:
                setattr(module, name, FP16Linear(child))
                count += 1
        else:
            count += patch_fp16_linears(child, verbose=verbose)
    return count


# the reference's name for the same operation
patch_cpu_linears = patch_fp16_linears
