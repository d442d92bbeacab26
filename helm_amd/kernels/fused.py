"""Fused decode-step ops around the INT8 GEMV (functional layer over the C ABI).

These merge the torch ops that the reference runs inside the HF decoder layer
around its attention patch (helm/runtime/kv_offload.py:241-271 and transformers'
Qwen3DecoderLayer / Qwen3MLP): RMSNorm into the following projection, the
residual add into the projection epilogue, SiLU(gate) * up into the gate/up
projection, and q/k-norm + RoPE + the paged KV write into one kernel.
"""
from __future__ import annotations

from typing import Optional

import torch

from .. import _native
from . import gemv_workspace_bytes


def _check_fp16(*ts):
    for t in ts:
        if t is not None and t.dtype != torch.float16:
            raise RuntimeError(f"expected fp16 tensor, got {t.dtype}")


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float,
            out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """fp16(w * fp16(x * rsqrt(mean(x^2) + eps))) over the last dim (Qwen3RMSNorm)."""
    _native.require_cuda(x, weight, what="rmsnorm")
    _check_fp16(x, weight)
    K = x.shape[-1]
    x2 = x.reshape(-1, K).contiguous()
    if out is None:
        out = torch.empty_like(x2)
    _native.call("helm_rmsnorm", x2.data_ptr(), weight.data_ptr(), float(eps), out.data_ptr(),
                 x2.shape[0], K, _native.stream_ptr(x.device))
    return out.view(x.shape)


def qk_norm_rope_cs(qkv: torch.Tensor, q_norm_w: Optional[torch.Tensor],
                    k_norm_w: Optional[torch.Tensor], eps: float, cos: torch.Tensor,
                    sin: torch.Tensor, n_heads: int, n_kv_heads: int, head_dim: int):
    """(q [B, Hq, D], k [B, Hkv, D]) of the fused projection output qkv
    [B, (Hq + 2 Hkv) * D]: per-head RMSNorm (when the norm weights are given),
    then RoPE with the model's fp16 cos / sin rows [B, D] (helm_qk_norm_rope_cs)."""
    _native.require_cuda(qkv, q_norm_w, k_norm_w, cos, sin, what="qk_norm_rope_cs")
    _check_fp16(qkv, q_norm_w, k_norm_w, cos, sin)
    B = qkv.shape[0]
    if qkv.shape[-1] != (n_heads + 2 * n_kv_heads) * head_dim or not qkv.is_contiguous():
        raise RuntimeError("qk_norm_rope_cs: qkv must be contiguous [B, (Hq + 2 Hkv) * D]")
    if cos.shape[0] != B or cos.shape[-1] != head_dim or cos.stride(-1) != 1 or sin.stride() != cos.stride():
        raise RuntimeError("qk_norm_rope_cs: cos / sin must be [B, D] rows with unit stride")
    q = torch.empty(B, n_heads, head_dim, dtype=torch.float16, device=qkv.device)
    k = torch.empty(B, n_kv_heads, head_dim, dtype=torch.float16, device=qkv.device)
    _native.call("helm_qk_norm_rope_cs", qkv.data_ptr(), _native.ptr(q_norm_w), _native.ptr(k_norm_w),
                 float(eps), cos.data_ptr(), sin.data_ptr(), cos.stride(0), q.data_ptr(), k.data_ptr(),
                 B, n_heads, n_kv_heads, head_dim, _native.stream_ptr(qkv.device))
    return q, k


def int8_gemv_fused(x: torch.Tensor, qweight: torch.Tensor, scale: torch.Tensor,
                    norm_weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
                    bias: Optional[torch.Tensor] = None,
                    residual: Optional[torch.Tensor] = None,
                    out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = [residual +] linear_int8(rmsnorm(x) if norm_weight else x), M <= 16 tokens."""
    _native.require_cuda(x, qweight, scale, norm_weight, bias, residual, what="int8_gemv_fused")
    _check_fp16(x, scale, norm_weight, bias, residual)
    N, K = qweight.shape
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    if out is None:
        out = torch.empty(M, N, dtype=torch.float16, device=x.device)
    y2 = out.view(M, N)
    res = None
    if residual is not None:
        r2 = residual.reshape(M, N)
        if r2.data_ptr() == y2.data_ptr() or (r2.stride(1) == 1 and r2.stride(0) == y2.stride(0)):
            res = r2.data_ptr()          # read in place (row stride ldy, may alias y)
        else:
            y2.copy_(r2)
            res = y2.data_ptr()
    if norm_weight is None:
        # no norm prologue: the workspace form (split K for long K at 5-16 tokens)
        ws_bytes = gemv_workspace_bytes(M, N, K)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
        _native.call("helm_int8_gemv_ws", x2.data_ptr(), x2.stride(0), qweight.data_ptr(),
                     qweight.stride(0), scale.data_ptr(), _native.ptr(bias), res, y2.data_ptr(),
                     y2.stride(0), M, N, K, _native.ptr(ws), ws_bytes, _native.stream_ptr(x.device))
        return out
    _native.call("helm_int8_gemv_fused", x2.data_ptr(), x2.stride(0), _native.ptr(norm_weight),
                 float(eps), qweight.data_ptr(), qweight.stride(0), scale.data_ptr(),
                 _native.ptr(bias), res, y2.data_ptr(), y2.stride(0), M, N, K,
                 _native.stream_ptr(x.device))
    return out


def int8_gemv_swiglu(x: torch.Tensor, q_gate: torch.Tensor, s_gate: torch.Tensor,
                     q_up: torch.Tensor, s_up: torch.Tensor,
                     norm_weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
                     out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """fp16(silu(gate(xn)) * up(xn)), xn = rmsnorm(x) if norm_weight else x."""
    _native.require_cuda(x, q_gate, s_gate, q_up, s_up, norm_weight, what="int8_gemv_swiglu")
    _check_fp16(x, s_gate, s_up, norm_weight)
    N, K = q_gate.shape
    if tuple(q_up.shape) != (N, K) or q_up.stride(0) != q_gate.stride(0):
        raise RuntimeError("int8_gemv_swiglu: gate and up weights must have the same shape/stride")
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    if out is None:
        out = torch.empty(M, N, dtype=torch.float16, device=x.device)
    _native.call("helm_int8_gemv_swiglu", x2.data_ptr(), x2.stride(0), _native.ptr(norm_weight),
                 float(eps), q_gate.data_ptr(), s_gate.data_ptr(), q_up.data_ptr(),
                 s_up.data_ptr(), q_gate.stride(0), out.data_ptr(), out.stride(0), M, N, K,
                 _native.stream_ptr(x.device))
    return out


def rope_inv_freq(head_dim: int, theta: float, device=None) -> torch.Tensor:
    """inv_freq[i] = 1 / theta^(2i / head_dim) in fp32, computed as transformers'
    Qwen3RotaryEmbedding.compute_default_rope_parameters does."""
    return (1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).to(
        device=device, dtype=torch.float) / head_dim))).float()


def qk_norm_rope_append(qkv: torch.Tensor, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor,
                        eps: float, positions: torch.Tensor, inv_freq: torch.Tensor,
                        q_out: torch.Tensor, pool, slots: torch.Tensor, offsets: torch.Tensor,
                        num_q_heads: int, num_kv_heads: int, head_dim: int,
                        page_size: int) -> torch.Tensor:
    """q/k RMSNorm + RoPE of the fused qkv [B, (Hq+2Hkv)*D]; writes k, v into the
    page slots of `pool` (an attention.PoolView) and the rotated q into q_out
    [B, Hq, D]."""
    _native.require_cuda(qkv, q_norm_w, k_norm_w, positions, inv_freq, q_out, pool.k, pool.v,
                         slots, offsets, what="qk_norm_rope_append")
    B = qkv.shape[0]
    _native.call("helm_qk_norm_rope_append", qkv.data_ptr(), q_norm_w.data_ptr(),
                 k_norm_w.data_ptr(), float(eps), positions.data_ptr(), inv_freq.data_ptr(),
                 q_out.data_ptr(), pool.c_ref(), slots.data_ptr(), offsets.data_ptr(), B,
                 num_q_heads, num_kv_heads, head_dim, page_size, _native.stream_ptr(qkv.device))
    return q_out


def fp16_gemv_rmsnorm(x: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                      weight: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = fp16(weight . rmsnorm(x)) for <= 16 tokens (final norm + lm_head)."""
    _native.require_cuda(x, norm_weight, weight, what="fp16_gemv_rmsnorm")
    _check_fp16(x, norm_weight, weight)
    N, K = weight.shape
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    if out is None:
        out = torch.empty(M, N, dtype=torch.float16, device=x.device)
    _native.call("helm_fp16_gemv_rmsnorm", x2.data_ptr(), x2.stride(0), norm_weight.data_ptr(),
                 float(eps), weight.data_ptr(), weight.stride(0), out.data_ptr(), out.stride(0),
                 M, N, K, _native.stream_ptr(x.device))
    return out


def silu_mul(gate: torch.Tensor, up: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """fp16(fp16(silu(gate)) * up) elementwise (the fused SwiGLU epilogue's rounding)."""
    _native.require_cuda(gate, up, what="silu_mul")
    _check_fp16(gate)
    _check_fp16(up)
    if gate.shape != up.shape or not gate.is_contiguous() or not up.is_contiguous():
        raise RuntimeError("silu_mul: gate and up must be contiguous tensors of one shape")
    if out is None:
        out = torch.empty_like(gate)
    _native.call("helm_silu_mul", gate.data_ptr(), up.data_ptr(), out.data_ptr(), gate.numel(),
                 _native.stream_ptr(gate.device))
    return out


def argmax_workspace(M: int, device) -> torch.Tensor:
    """Workspace of helm_argmax_f16_ws for M rows (reusable across calls on one stream)."""
    n = int(_native.lib().helm_argmax_workspace_bytes(int(M)))
    return torch.empty(max(1, n // 4), dtype=torch.int32, device=device)


def argmax(x: torch.Tensor, out: Optional[torch.Tensor] = None,
           workspace: Optional[torch.Tensor] = None, single_workgroup: bool = False) -> torch.Tensor:
    """Index of the first maximum of each row of fp16 x [M, N] (torch.argmax(x, -1)):
    64 workgroups per row and a merge kernel (`workspace` from argmax_workspace,
    allocated here when not given), or with single_workgroup one workgroup per
    row and no workspace."""
    _native.require_cuda(x, what="argmax")
    _check_fp16(x)
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    M, N = x2.shape
    if out is None:
        out = torch.empty(M, dtype=torch.int64, device=x.device)
    stream = _native.stream_ptr(x.device)
    if single_workgroup:
        _native.call("helm_argmax_f16", x2.data_ptr(), x2.stride(0), M, N, out.data_ptr(), stream)
        return out
    if workspace is None:
        workspace = argmax_workspace(M, x.device)
    _native.require_cuda(workspace, what="argmax")
    _native.call("helm_argmax_f16_ws", x2.data_ptr(), x2.stride(0), M, N, out.data_ptr(),
                 workspace.data_ptr(), workspace.numel() * workspace.element_size(), stream)
    return out
