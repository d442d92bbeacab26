"""Oracle for paged decode attention — TEST INFRASTRUCTURE ONLY.

Restates perform_streaming_attention (helm/runtime/kv_cache.py:318-442) in numpy:

  * page filter (:350-351): active GPU pages are used>0, state 'GPU', device
    cuda; active CPU pages are used>0, state 'CPU', device not cuda; DEAD and
    empty pages drop out; nothing left -> zeros like the query (:353-354);
  * GQA (:356-363): kv head of query head h is h // (Hq // Hkv) (repeat_interleave);
  * all-GPU (:367-371) and all-CPU with a CPU query (:376-380): one softmax over
    the concatenated pages, computed here in fp32 and cast to the query dtype;
  * causal prefill (kv_offload.py:253-265, SDPA with the causal mask built by
    pipeline_runtime.py:25-29): query i at position q_start + i sees keys
    0 .. q_start + i (`causal_prefill_reference`);
  * the prefill SDPA under any other mask (`masked_prefill_reference`);
  * otherwise (:387-442): the fp32 online softmax, GPU block first, then the CPU
    pages in list order, alpha = nan_to_num(exp(m - m'), 0), out / max(l, 1e-12).

Pinning (tests/test_oracle_attention.py): the reference's own unit tests
(tests/unit/runtime/test_streaming_attention.py:47-241 — single/multi page,
empty pages, custom/default scale, dtype, GQA, large logits) are restated
against this module; `eager` is the fp64 closed form softmax(q K^T s) V, checked
against torch.nn.functional.scaled_dot_product_attention (a library routine) and
brute-force loops; the online-softmax path must agree with `eager` for any page
split (page order and split boundaries change only rounding).  The causal
prefill form is checked against torch SDPA with is_causal=True (q_start = 0)
and against `eager` row by row on the visible keys (any q_start); the masked
form against torch SDPA with boolean and additive masks, brute-force loops, and
the causal form when handed the causal mask.
"""
from __future__ import annotations

import math
from typing import List, Optional, Sequence

import numpy as np


def _np(t) -> np.ndarray:
    if hasattr(t, "detach"):
        t = t.detach().cpu()
        if str(t.dtype) == "torch.bfloat16":
            t = t.float()
        return t.numpy()
    return np.asarray(t)


def _dev_type(d) -> str:
    return d if isinstance(d, str) else getattr(d, "type", str(d))


def expand_kv(k: np.ndarray, num_q_heads: int) -> np.ndarray:
    """[B, Hkv, S, D] -> [B, Hq, S, D] by repeat_interleave over heads (kv_cache.py:356-363)."""
    hkv = k.shape[1]
    if hkv == num_q_heads:
        return k
    return np.repeat(k, num_q_heads // hkv, axis=1)


def eager(q, k, v, scale: Optional[float] = None) -> np.ndarray:
    """fp64 closed form: softmax(q K^T * scale) V, GQA-expanded.  q [B,Hq,Sq,D],
    k/v [B,Hkv,S,D]; returns fp64 [B,Hq,Sq,D]."""
    q = _np(q).astype(np.float64)
    k = expand_kv(_np(k).astype(np.float64), q.shape[1])
    v = expand_kv(_np(v).astype(np.float64), q.shape[1])
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    s = np.einsum("bhqd,bhkd->bhqk", q, k) * scale
    s -= s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("bhqk,bhkd->bhqd", p, v)


def _softmax_fp32(q32: np.ndarray, K: np.ndarray, V: np.ndarray, scale: float) -> np.ndarray:
    s = (q32 @ np.swapaxes(K, -1, -2)) * np.float32(scale)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(axis=-1, keepdims=True)
    return (p @ V).astype(np.float32)


def online_softmax(q32: np.ndarray, blocks: Sequence[tuple], scale: float) -> np.ndarray:
    """The fp32 online-softmax loop of kv_cache.py:387-441 over (K, V) blocks in
    the given order (K/V already GQA-expanded, fp32).  Returns fp32 out."""
    bsz, hq, qlen, d = q32.shape
    out = np.zeros((bsz, hq, qlen, d), np.float32)
    m = np.full((bsz, hq, qlen, 1), -np.inf, np.float32)
    l = np.zeros((bsz, hq, qlen, 1), np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        for K, V in blocks:
            scores = (q32 @ np.swapaxes(K, -1, -2)) * np.float32(scale)
            bmax = scores.max(axis=-1, keepdims=True)
            m_new = np.maximum(m, bmax)
            alpha = np.nan_to_num(np.exp(m - m_new), nan=0.0).astype(np.float32)
            p = np.exp(scores - m_new).astype(np.float32)
            out = out * alpha + p @ V
            l = l * alpha + p.sum(axis=-1, keepdims=True)
            m = m_new
    return out / np.maximum(l, np.float32(1e-12))


def streaming_attention(query, pages: List, scale: Optional[float] = None,
                        query_device: str = "cpu") -> np.ndarray:
    """Restatement of perform_streaming_attention.  `query` [B,Hq,Sq,D] (array or
    tensor); pages expose k_tensor, v_tensor ([1,Hkv,cap,D]), used_tokens, state,
    device.  `query_device` is the device type the reference's query would be on
    ('cuda' selects the online-softmax path whenever a CPU page is present).
    Returns an array in the query's dtype."""
    q = _np(query)
    dtype = q.dtype
    hq = q.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    gpu = [p for p in pages if p.used_tokens > 0 and p.state == "GPU" and _dev_type(p.device) == "cuda"]
    cpu = [p for p in pages if p.used_tokens > 0 and p.state == "CPU" and _dev_type(p.device) != "cuda"]
    if not gpu and not cpu:
        return np.zeros_like(q)

    def kv(p):
        u = p.used_tokens
        k = _np(p.k_tensor)[:, :, :u, :].astype(np.float32)
        v = _np(p.v_tensor)[:, :, :u, :].astype(np.float32)
        return expand_kv(k, hq), expand_kv(v, hq)

    q32 = q.astype(np.float32)
    if not cpu or (not gpu and query_device != "cuda"):
        sel = gpu if not cpu else cpu
        ks, vs = zip(*(kv(p) for p in sel))
        return _softmax_fp32(q32, np.concatenate(ks, axis=2), np.concatenate(vs, axis=2),
                             scale).astype(dtype)
    blocks = []
    if gpu:
        ks, vs = zip(*(kv(p) for p in gpu))
        blocks.append((np.concatenate(ks, axis=2), np.concatenate(vs, axis=2)))
    blocks.extend(kv(p) for p in cpu)
    return online_softmax(q32, blocks, scale).astype(dtype)


def paged_decode_reference(q, k_pool, v_pool, page_table, seq_lens, page_size: int,
                           scale: float) -> np.ndarray:
    """fp64 decode attention over a paged pool laid out [slots, Hkv, P, D]:
    item b attends to its first seq_lens[b] tokens, page i of item b being slot
    page_table[b, i].  q [B, Hq, D]; returns fp64 [B, Hq, D] (zeros for an empty
    item).  This is the closed form the split-K GPU kernel must reproduce."""
    q = _np(q).astype(np.float64)
    kp = _np(k_pool)
    vp = _np(v_pool)
    pt = _np(page_table)
    sl = _np(seq_lens)
    B, hq, d = q.shape
    out = np.zeros((B, hq, d))
    for b in range(B):
        n = int(sl[b])
        if n == 0:
            continue
        npg = (n + page_size - 1) // page_size
        slots = pt[b, :npg]
        k = kp[slots].transpose(1, 0, 2, 3).reshape(kp.shape[1], npg * page_size, d)[:, :n]
        v = vp[slots].transpose(1, 0, 2, 3).reshape(vp.shape[1], npg * page_size, d)[:, :n]
        out[b] = eager(q[b][None, :, None, :], k[None], v[None], scale)[0, :, 0, :]
    return out


def all_cpu_decode_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float) -> np.ndarray:
    """The reference's all-CPU path (kv_cache.py:376-380) on already concatenated
    pages: K/V [1, Hkv, T, D] fp16 -> fp32, GQA expand, fp32 softmax(q K^T s) V,
    cast back to the query dtype.  q [1, Hq, 1, D]."""
    hq = q.shape[1]
    K = expand_kv(k.astype(np.float32), hq)
    V = expand_kv(v.astype(np.float32), hq)
    return _softmax_fp32(q.astype(np.float32), K, V, scale).astype(q.dtype)


def causal_prefill_reference(q, k, v, q_start: int, scale: float) -> np.ndarray:
    """fp64 causal attention of T queries at positions q_start .. q_start+T-1 over
    N = q_start + T keys (kv_offload.py:253-265 with the causal mask of
    pipeline_runtime.py:25-29).  q [T, Hq, D]; k, v [N, Hkv, D]; GQA h -> h // G.
    Returns [T, Hq, D] float64."""
    q = _np(q).astype(np.float64)
    k = _np(k).astype(np.float64)
    v = _np(v).astype(np.float64)
    T, Hq, D = q.shape
    N, Hkv, _ = k.shape
    g = Hq // Hkv
    kh = np.repeat(k.transpose(1, 0, 2), g, axis=0)        # [Hq, N, D]
    vh = np.repeat(v.transpose(1, 0, 2), g, axis=0)
    s = np.einsum("thd,hnd->htn", q, kh) * scale           # [Hq, T, N]
    visible = np.arange(N)[None, :] <= (q_start + np.arange(T))[:, None]
    s = np.where(visible[None], s, -np.inf)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return np.einsum("htn,hnd->thd", p, vh)


def masked_prefill_reference(q, k, v, mask, scale: float) -> np.ndarray:
    """fp64 prefill attention under an arbitrary mask, as the reference's prefill
    SDPA applies the attention_mask it is handed (kv_offload.py:253-265):
    softmax(q K^T scale + mask) V over all N keys.  q [T, Hq, D]; k, v [N, Hkv, D];
    mask [Hm, T, N] (Hm 1 or Hq) boolean (True = attend, False = -inf) or additive.
    A row whose keys are all at -inf gives zeros (torch's SDPA since 2.5).
    Returns [T, Hq, D] float64."""
    q = _np(q).astype(np.float64)
    k = _np(k).astype(np.float64)
    v = _np(v).astype(np.float64)
    m = _np(mask)
    add = np.where(m, 0.0, -np.inf) if m.dtype == np.bool_ else m.astype(np.float64)
    T, Hq, D = q.shape
    N, Hkv, _ = k.shape
    g = Hq // Hkv
    kh = np.repeat(k.transpose(1, 0, 2), g, axis=0)        # [Hq, N, D]
    vh = np.repeat(v.transpose(1, 0, 2), g, axis=0)
    s = np.einsum("thd,hnd->htn", q, kh) * scale + add      # [Hq, T, N]
    mx = s.max(-1, keepdims=True)
    dead = np.isneginf(mx)
    p = np.exp(s - np.where(dead, 0.0, mx))
    l = p.sum(-1, keepdims=True)
    p = np.where(dead, 0.0, p / np.where(dead, 1.0, l))
    return np.einsum("htn,hnd->thd", p, vh)
