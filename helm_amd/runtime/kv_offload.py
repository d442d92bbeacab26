"""KV offload integration: class-level patched attention forward over the paged
cache (mirror of helm/runtime/kv_offload.py).

KVOffloadManager(model, config, batch_size) builds one KVAllocator shared by one
KVCacheManager per batch item (watermark split per item, :356-360), patches the
model family's attention class at class level (:403-433), and routes decode
through _decode_batched's three paths (:82-167):

  1. contiguous: in-place write into a preallocated buffer of cap tokens per item
     and layer (K [B, Hkv, cap, D], V in the pools' page-block layout), attention
     over it read as pages (:106-126);
  2. paged, every page GPU-resident: all_gpu is computed BEFORE the append and
     passed as skip_residency (:133-137 — the watermark is not enforced while
     everything is on the GPU), then one batched kernel over the device page
     table (:141-160);
  3. mixed residency: per-item perform_streaming_attention (:163-167).

Every attention runs on the split-K paged kernel; the new token's K/V is written
into its page slot by helm_kv_append.
"""
from __future__ import annotations

import contextlib
import math
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch
import torch.nn.functional as F

from ..kernels import Int8Linear, int8_linear
from ..kernels import attention as ka
from ..kernels.fused import int8_gemv_fused, int8_gemv_swiglu, qk_norm_rope_cs, rmsnorm
from .kv_allocator import KVAllocator
from .kv_cache import ContiguousKV, KVCacheManager, perform_streaming_attention
from .page_table import DevicePageTable, PinnedRing


def _hooked(*mods) -> bool:
    """True when a fused path would skip a hook: any of `mods` has forward or
    forward-pre hooks, an accelerate `_hf_hook`, or global module hooks are set.
    The fused forwards call such modules' kernels directly instead of through
    __call__, so with a hook present they run the original forward instead."""
    from torch.nn.modules import module as _m
    if _m._global_forward_hooks or _m._global_forward_pre_hooks:
        return True
    for m in mods:
        if m is None:
            continue
        if m._forward_hooks or m._forward_pre_hooks or getattr(m, "_hf_hook", None) is not None:
            return True
    return False


@dataclass
class KVOffloadConfig:
    num_layers: int
    num_kv_heads: int
    head_dim: int
    page_size: int = 64
    dtype: torch.dtype = torch.float16
    # GPU KV bytes (evictable pages) kept before the oldest pages move to host
    # memory; default ~512 tokens per layer (kv_offload.py:47-52).
    gpu_watermark_bytes: Optional[int] = None
    # contiguous buffer capacity in tokens (0 disables Path 1)
    cont_capacity: int = 32768
    # Off (the reference's behaviour): only <Arch>Attention.forward is patched.
    # On: the family's MLP, RMSNorm and decoder-layer classes are patched too, so
    # a decode step fuses the norms into the GEMV prologues, the residual adds
    # into their epilogues and gate / up / SiLU into one launch (same roundings).
    fuse_decoder_layers: bool = False

    def __post_init__(self):
        if self.gpu_watermark_bytes is None:
            elem = torch.tensor([], dtype=self.dtype).element_size()
            per_token_bytes = 2 * self.num_kv_heads * self.head_dim * elem
            self.gpu_watermark_bytes = 512 * per_token_bytes * self.num_layers

    @staticmethod
    def from_model(model, page_size: int = 64, gpu_watermark_bytes: Optional[int] = None,
                   cont_capacity: Optional[int] = None,
                   fuse_decoder_layers: bool = False) -> "KVOffloadConfig":
        cfg = model.config
        num_layers = cfg.num_hidden_layers
        num_kv_heads = getattr(cfg, "num_key_value_heads", cfg.num_attention_heads)
        head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        dtype = next(model.parameters()).dtype
        if cont_capacity is None:
            cont_capacity = getattr(cfg, "max_position_embeddings", 32768)
        return KVOffloadConfig(num_layers=num_layers, num_kv_heads=num_kv_heads,
                               head_dim=head_dim, page_size=page_size, dtype=dtype,
                               gpu_watermark_bytes=gpu_watermark_bytes,
                               cont_capacity=cont_capacity,
                               fuse_decoder_layers=fuse_decoder_layers)


class _DecodeIO:
    """Per-manager device scratch of the decode path (slots, offsets, seq lens)."""

    def __init__(self, batch: int, num_layers: int, device: torch.device, ring: PinnedRing):
        self.ring = ring
        # slots, offsets and seq lens as the rows of one buffer, so a decode layer
        # stages all three with one host-to-device copy (put_meta)
        self.meta = torch.empty(3, batch, dtype=torch.int32, device=device)
        self.slots, self.offsets, self.seq_lens = self.meta[0], self.meta[1], self.meta[2]
        # a planned step's values for every layer [L, 3, B], uploaded once per step
        self.plan_meta = torch.zeros(num_layers, 3, batch, dtype=torch.int32, device=device)
        self.workspace = ka.AttnWorkspace(device)
        # split-K partials of planned steps (only planned steps grow it, and only
        # when their key changes)
        self.plan_workspace = ka.AttnWorkspace(device)

    def put(self, arr, dst):
        self.ring.upload(np.asarray(arr, np.int32), dst)

    def put_meta(self, n: int, slots, offsets, seq_lens) -> None:
        """The first n entries of slots, offsets and seq_lens in one upload."""
        arr = np.zeros((3, self.meta.shape[1]), np.int32)
        arr[0, :n], arr[1, :n], arr[2, :n] = slots, offsets, seq_lens
        self.ring.upload(arr, self.meta)


PLAN_BUCKET_PAGES = 64   # a planned step's page-table width is a multiple of this


@dataclass(frozen=True)
class DecodePlan:
    """A decode step whose host bookkeeping ran for every layer before the
    forward (KVOffloadManager.plan_decode_step): the path every layer takes
    (1 contiguous buffers, 2 paged with every page on the GPU), the batch, the
    page-table width the kernels read (the live pages rounded up to
    PLAN_BUCKET_PAGES) and the split count.  Everything a layer's launches read
    sits in device buffers whose addresses `key` pins, so the step's forward can
    be captured once and replayed while the key holds."""
    path: int
    bsz: int
    pages: int
    splits: int
    key: tuple


def _bucket(n_pages: int, cap: int) -> int:
    return max(1, min(cap, -(-max(1, n_pages) // PLAN_BUCKET_PAGES) * PLAN_BUCKET_PAGES))


def plan_paged_slots(kvcms, num_layers: int, device, meta: np.ndarray) -> Optional[int]:
    """Paged bookkeeping of a whole decode step ahead of the forward: when every
    page of every layer and item is GPU-resident and no layer holds a partial
    page before its tail, reserve the new token's slot layer by layer, item by
    item (reserve_decode_slot with skip_residency, which is what
    _decode_batched does per layer when all_gpu holds, kv_offload.py:132-137 —
    and with no eviction no layer's all_gpu can change during the step), and
    write slot, index in page and new length to meta[layer, 0:3, item].
    Returns the longest page list after the step, or None (nothing reserved)
    when the step is not of that kind."""
    for li in range(num_layers):
        for m in kvcms:
            if not m.all_gpu_resident(li) or m.layer_is_ragged(li):
                return None
    longest = 1
    for li in range(num_layers):
        for i, m in enumerate(kvcms):
            page, idx = m.reserve_decode_slot(li, device, skip_residency=True)
            if page.state != "GPU":
                raise RuntimeError("decode tail page is not GPU-resident")
            meta[li, 0, i] = page.slot
            meta[li, 1, i] = idx
            meta[li, 2, i] = m.layers[li].total_tokens
            longest = max(longest, len(m.layers[li].pages))
    return longest


def _decode_planned(mgr: "KVOffloadManager", plan: DecodePlan, q, k, v, layer_idx: int,
                    scale: float):
    """A layer of a planned step: the slots, offsets and lengths come from the
    plan's device buffer; no host bookkeeping and no upload, so the launches are
    the same on every step the plan's key covers."""
    bsz, n_q_heads, _, head_dim = q.shape
    if bsz != plan.bsz:
        raise RuntimeError(f"planned decode step for batch {plan.bsz} got batch {bsz}")
    io = mgr._io(q.device)
    meta = io.plan_meta[layer_idx]
    slots, offs, lens = meta[0, :bsz], meta[1, :bsz], meta[2, :bsz]
    cfg = mgr.config
    P = cfg.page_size
    pool, table = mgr._plan_pool_table(plan, layer_idx, q.device)
    ka.kv_append(k.to(cfg.dtype), v.to(cfg.dtype), pool, slots, offs, P)
    part_o, part_ml = io.plan_workspace.get(bsz, n_q_heads, head_dim, plan.splits)
    qh = q.reshape(bsz, n_q_heads, head_dim).to(torch.float16)
    ka.paged_decode_attention_partial(qh, pool, table, lens, P, scale, part_o, part_ml, plan.splits)
    out = torch.empty(bsz, n_q_heads, head_dim, dtype=torch.float16, device=q.device)
    ka.paged_attn_reduce(part_o, part_ml, out, plan.splits)
    return out.view(bsz, n_q_heads, 1, head_dim).to(q.dtype)


def _decode_planned_fused(mgr: "KVOffloadManager", plan: DecodePlan, qkv, q_norm_w, k_norm_w,
                          eps: float, cos, sin, layer_idx: int, scale: float, n_heads: int,
                          n_kv_heads: int, head_dim: int):
    """A layer of a planned step from the raw q|k|v projection [B, (Hq + 2 Hkv) D]:
    q / k norms, RoPE with the layer's own cos / sin rows, the new token's K/V
    write and the split-K partials in one launch (helm_decode_attn_fused_cs),
    then the merge; returns [B, Hq, 1, D].  The same roundings as
    helm_qk_norm_rope_cs + kv_append + the partial kernel of _decode_planned."""
    bsz = qkv.shape[0]
    if bsz != plan.bsz:
        raise RuntimeError(f"planned decode step for batch {plan.bsz} got batch {bsz}")
    io = mgr._io(qkv.device)
    meta = io.plan_meta[layer_idx]
    pool, table = mgr._plan_pool_table(plan, layer_idx, qkv.device)
    part_o, part_ml = io.plan_workspace.get(bsz, n_heads, head_dim, plan.splits)
    ka.decode_attention_fused_cs(qkv, q_norm_w, k_norm_w, eps, cos, sin, pool, meta[0, :bsz],
                                 meta[1, :bsz], table, meta[2, :bsz], mgr.config.page_size, scale,
                                 part_o, part_ml, plan.splits, n_heads, n_kv_heads, head_dim)
    out = torch.empty(bsz, n_heads, head_dim, dtype=torch.float16, device=qkv.device)
    ka.paged_attn_reduce(part_o, part_ml, out, plan.splits)
    return out.view(bsz, n_heads, 1, head_dim)


def _decode_batched(mgr: "KVOffloadManager", q, k, v, layer_idx: int, scale: float):
    """Decode step shared by the attention patches; returns [bsz, Hq, 1, D]."""
    if mgr._plan is not None:
        return _decode_planned(mgr, mgr._plan, q, k, v, layer_idx, scale)
    kvcms = mgr.kvcms
    bsz, n_q_heads, _, head_dim = q.shape
    device = q.device
    io = mgr._io(device)

    # ── Path 1: contiguous in-place buffers ─────────────────────────────────
    if kvcms[0].use_contiguous:
        pos = kvcms[0].cont_seq_len
        if pos < kvcms[0].cont_capacity:
            shared = mgr._shared_contiguous(bsz)
            staged = shared is not None
            if staged:   # the append's slots / offsets (the token's page of each item's
                # buffer read as pages) and the attention's lengths
                per_item = shared.capacity // mgr.config.page_size
                io.put_meta(bsz, np.arange(bsz) * per_item + pos // mgr.config.page_size,
                            np.full(bsz, pos % mgr.config.page_size), np.full(bsz, pos + 1))
            mgr._write_contiguous(layer_idx, k, v, pos, io, staged)
            if layer_idx == kvcms[0].cont_num_layers - 1:
                for kvcm in kvcms:
                    kvcm.advance_contiguous()
            out = mgr._contiguous_attention(layer_idx, q, pos + 1, scale, io, staged)
            return out.view(bsz, n_q_heads, 1, head_dim)
        for kvcm in kvcms:
            kvcm.migrate_contiguous_to_pages()

    # ── Paths 2 & 3: paged ──────────────────────────────────────────────────
    all_gpu = all(kvcms[i].all_gpu_resident(layer_idx) for i in range(bsz))
    slots, offs = [], []
    for i in range(bsz):
        page, idx = kvcms[i].reserve_decode_slot(layer_idx, device, skip_residency=all_gpu)
        if page.state != "GPU":
            raise RuntimeError("decode tail page is not GPU-resident")
        slots.append(page.slot)
        offs.append(idx)
    pool = ka.PoolView.of_pool(*mgr._device_pool(device))
    # Path 2 reads token t of an item at page t // P; a layer whose pages include a
    # partial one before the tail (decode tokens migrated out of the contiguous
    # buffer after a prompt that did not fill its last page) takes Path 3, which
    # attends every run of pages with its own length
    path2 = all_gpu and not any(kvcms[i].layer_is_ragged(layer_idx) for i in range(bsz))
    if path2:   # slots, offsets and the lengths Path 2 reads, in one upload
        io.put_meta(bsz, slots, offs, [kvcm.layers[layer_idx].total_tokens for kvcm in kvcms])
    else:
        io.put(slots, io.slots)
        io.put(offs, io.offsets)
    ka.kv_append(k.to(mgr.config.dtype), v.to(mgr.config.dtype), pool, io.slots, io.offsets,
                 mgr.config.page_size)

    if path2:
        pt = mgr.page_table
        pt.flush()
        max_pages = max(len(kvcm.layers[layer_idx].pages) for kvcm in kvcms)
        rows = pt.rows(layer_idx)
        splits = ka.choose_num_splits(bsz, pool.num_kv_heads, max_pages, mgr.config.page_size)
        part_o, part_ml = io.workspace.get(bsz, n_q_heads, head_dim, splits)
        qh = q.reshape(bsz, n_q_heads, head_dim).to(torch.float16)
        # [B, max_pages] view with row stride = table capacity
        ka.paged_decode_attention_partial(qh, pool, rows[:, :max(1, max_pages)], io.seq_lens,
                                          mgr.config.page_size, scale, part_o, part_ml, splits)
        out = torch.empty(bsz, n_q_heads, head_dim, dtype=torch.float16, device=device)
        ka.paged_attn_reduce(part_o, part_ml, out, splits)
        return out.view(bsz, n_q_heads, 1, head_dim).to(q.dtype)

    # ── Path 3: mixed residency — per-item streaming attention ──────────────
    outs = [perform_streaming_attention(q[i:i + 1], kvcms[i].iterate_layer_pages(layer_idx),
                                        scale=scale, allocator=mgr.allocator)
            for i in range(bsz)]
    return torch.cat(outs, dim=0)


def _is_causal_mask(mask, q_len: int) -> bool:
    """True when `mask` is absent or is the plain causal mask over q_len keys (the
    one pipeline_runtime.py:25-29 builds: large negative strictly above the
    diagonal, zero elsewhere, for every batch row)."""
    if mask is None:
        return True
    if mask.dim() != 4 or mask.shape[-2] != q_len or mask.shape[-1] < q_len:
        return False
    m = mask[:, :, :, :q_len]
    if m.dtype == torch.bool:     # True = attend
        above = ~m
    else:
        above = m < -1e3
        if bool(((m != 0) & ~above).any()):
            return False
    tri = torch.ones(q_len, q_len, dtype=torch.bool, device=m.device).triu(1)
    return bool((above == tri).all())


def _item_masks(mask, bsz: int, n_heads: int, q_len: int):
    """Per-item [Hm, q_len, q_len] views of a 4-D attention mask [1 or bsz, 1 or
    n_heads, q_len, >= q_len] over the prompt's own keys (the first q_len, as the
    SDPA call is given them), or None for any other shape."""
    if mask is None or mask.dim() != 4 or mask.shape[-2] != q_len or mask.shape[-1] < q_len:
        return None
    if mask.shape[0] not in (1, bsz) or mask.shape[1] not in (1, n_heads):
        return None
    return [mask[i if mask.shape[0] > 1 else 0, :, :, :q_len] for i in range(bsz)]


def _decode_fast(attn_self, x) -> bool:
    """The decode projections can run as one fused INT8 GEMV: fp16 on the GPU, not
    training, q / k / v all Int8Linear over the same inputs, biases all or none,
    and (Qwen3) q / k norms that are fp16 RMSNorm modules."""
    if x.dtype != torch.float16 or not x.is_cuda or attn_self.training:
        return False
    mods = (attn_self.q_proj, attn_self.k_proj, attn_self.v_proj)
    if not all(isinstance(m, Int8Linear) and m.qweight.is_cuda for m in mods):
        return False
    if len({m.in_features for m in mods}) != 1 or len({m.bias is None for m in mods}) != 1:
        return False
    if _hooked(*mods, getattr(attn_self, "q_norm", None), getattr(attn_self, "k_norm", None)):
        return False
    for name in ("q_norm", "k_norm"):
        nm = getattr(attn_self, name, None)
        if nm is not None and (getattr(nm, "weight", None) is None or nm.weight.dtype != torch.float16
                               or not hasattr(nm, "variance_epsilon")):
            return False
    return True


def _fused_qkv(attn_self):
    """(qweight, scale, bias) of q|k|v stacked, built on first use: the three
    Int8Linear modules' buffers become views of the stacked ones, so the weights
    are held once and a module read or swapped later is seen (a module whose
    buffer no longer views the stack rebuilds it)."""
    mods = (attn_self.q_proj, attn_self.k_proj, attn_self.v_proj)
    cached = getattr(attn_self, "_helm_qkv", None)
    if cached is not None:
        qw, sc, bias = cached
        rows = 0
        ok = True
        for m in mods:
            n = m.out_features
            ok = (ok and m.qweight.data_ptr() == qw[rows:].data_ptr() and m.qweight.shape[0] == n
                  and m.scale.data_ptr() == sc[rows:].data_ptr()
                  and (bias is None) == (m.bias is None)
                  and (bias is None or m.bias.data_ptr() == bias[rows:].data_ptr()))
            rows += n
        if ok:
            return cached
    qw = torch.cat([m.qweight for m in mods]).contiguous()
    sc = torch.cat([m.scale for m in mods]).contiguous()
    bias = None if mods[0].bias is None else torch.cat([m.bias for m in mods]).contiguous()
    rows = 0
    for m in mods:
        n = m.out_features
        m.qweight, m.scale = qw[rows:rows + n], sc[rows:rows + n]
        if bias is not None:
            m.bias = bias[rows:rows + n]
        rows += n
    attn_self._helm_qkv = (qw, sc, bias)
    return attn_self._helm_qkv


_ROPE_MODULES = {
    "qwen3": "transformers.models.qwen3.modeling_qwen3",
    "qwen2": "transformers.models.qwen2.modeling_qwen2",
    "llama": "transformers.models.llama.modeling_llama",
}


def _make_attention_forward(mgr: "KVOffloadManager", arch: str):
    """Patched <Arch>Attention.forward (helm/runtime/kv_offload.py:174-323): q/k/v
    projections (RMS-normed q/k for Qwen3), RoPE, then prefill -> page writes +
    causal attention, decode -> _decode_batched over the paged cache, o_proj.
    The three families differ only in the q/k norms (Qwen3) and where
    apply_rotary_pos_emb is imported from."""
    import importlib
    rope_mod = importlib.import_module(_ROPE_MODULES[arch])
    apply_rotary_pos_emb = rope_mod.apply_rotary_pos_emb
    qk_norm = arch == "qwen3"

    def forward(attn_self, hidden_states, position_embeddings, attention_mask=None,
                past_key_values=None, cache_position=None, **kwargs):
        # set by the patched decoder layer: the layer's residual, added to o_proj's
        # output here (in the GEMV's epilogue where o_proj is an Int8Linear)
        residual = kwargs.pop("_helm_residual", None)
        # also set by the patched decoder layer: hidden_states is then the layer's
        # input and this its input norm, applied here (inside the q|k|v GEMV on the
        # decode path)
        in_norm = kwargs.pop("_helm_input_norm", None)
        bsz, q_len, _ = hidden_states.shape
        hidden_shape = (bsz, q_len, -1, attn_self.head_dim)
        cos, sin = position_embeddings
        fused = _fused_qkv(attn_self) if q_len == 1 and _decode_fast(attn_self, hidden_states) else None
        fast = fused is not None and cos.dtype == torch.float16 and cos.shape[-2] == 1
        if in_norm is not None and not (fast and in_norm.weight.dtype == torch.float16
                                        and in_norm.weight.is_cuda and not _hooked(in_norm)):
            hidden_states, in_norm = in_norm(hidden_states), None
        out = None
        if fast:
            # decode: [input norm +] q|k|v in one INT8 GEMV over the modules' shared
            # weight rows, then the q / k norms and RoPE (the model's own cos / sin)
            # in one kernel -- and in a planned step the K/V write and the
            # attention partials in that same kernel
            if in_norm is None:
                qkv = int8_linear(hidden_states, *fused).view(bsz, -1)
            else:
                qkv = int8_gemv_fused(hidden_states, fused[0], fused[1], norm_weight=in_norm.weight,
                                      eps=in_norm.variance_epsilon, bias=fused[2]).view(bsz, -1)
            nq, nk = attn_self.q_proj.out_features, attn_self.k_proj.out_features
            D = attn_self.head_dim
            cos_r = cos.reshape(cos.shape[0], -1).expand(bsz, D)
            sin_r = sin.reshape(sin.shape[0], -1).expand(bsz, D)
            qn = attn_self.q_norm.weight if qk_norm else None
            kn = attn_self.k_norm.weight if qk_norm else None
            eps = attn_self.q_norm.variance_epsilon if qk_norm else 0.0
            if mgr._plan is not None and mgr.config.dtype == torch.float16:
                out = _decode_planned_fused(mgr, mgr._plan, qkv, qn, kn, eps, cos_r, sin_r,
                                            attn_self.layer_idx, 1.0 / math.sqrt(D), nq // D,
                                            nk // D, D)
            else:
                q, k = qk_norm_rope_cs(qkv, qn, kn, eps, cos_r, sin_r, nq // D, nk // D, D)
                q, k = q.unsqueeze(2), k.unsqueeze(2)
                v = qkv[:, nq + nk:].view(bsz, 1, -1, D).transpose(1, 2)
        else:
            q = attn_self.q_proj(hidden_states).view(hidden_shape)
            k = attn_self.k_proj(hidden_states).view(hidden_shape)
            if qk_norm:
                q, k = attn_self.q_norm(q), attn_self.k_norm(k)
            v = attn_self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
            q, k = q.transpose(1, 2), k.transpose(1, 2)
            q, k = apply_rotary_pos_emb(q, k, cos, sin)
        scale = 1.0 / math.sqrt(attn_self.head_dim)
        kvcms = mgr.kvcms
        if out is not None:
            pass
        elif q_len > 1:
            for i in range(bsz):
                kvcms[i].append_prefill(attn_self.layer_idx, k[i:i + 1], v[i:i + 1])
                if kvcms[i].use_contiguous:
                    kvcms[i].prefill_contiguous(attn_self.layer_idx, k[i:i + 1], v[i:i + 1])
            on_kernels = q.dtype == torch.float16 and q.is_cuda and not attn_self.training
            causal = on_kernels and _is_causal_mask(attention_mask, q_len)
            masks = (None if causal or not on_kernels
                     else _item_masks(attention_mask, bsz, q.shape[1], q_len))
            if causal or masks is not None:
                # prefill on the matrix cores, one item at a time, over the prompt
                # K/V where the appends above just wrote them (the item's contiguous
                # buffer, or its pages when all are in the device pool), else over a
                # dense page-layout copy: the plain causal mask by helm_prefill_attn,
                # any other 4-D mask (padding ...) added to the scores by
                # helm_prefill_attn_mask
                out = torch.empty_like(q)
                for i in range(bsz):
                    src = mgr._prefill_kv_source(i, attn_self.layer_idx, q_len, q.device)
                    if src is None:
                        pool, pt = ka.dense_prefill_kv(k[i].transpose(0, 1), v[i].transpose(0, 1), 16)
                        P = 16
                    else:
                        pool, pt, P = src
                    o = ka.prefill_attention(q[i].transpose(0, 1), pool, pt, P, 0, scale,
                                             mask=None if causal else masks[i])
                    out[i].copy_(o.transpose(0, 1))
            else:
                # bf16 / fp32 models, training, masks of other shapes: torch SDPA, the
                # reference's call
                groups = q.shape[1] // k.shape[1]
                k_exp = k.repeat_interleave(groups, dim=1)
                v_exp = v.repeat_interleave(groups, dim=1)
                mask = attention_mask
                if mask is not None and mask.dim() == 4 and mask.dtype != torch.bool:
                    mask = mask[:, :, :, : k_exp.shape[2]].to(q.dtype)
                out = F.scaled_dot_product_attention(
                    q.contiguous(), k_exp.contiguous(), v_exp.contiguous(), attn_mask=mask,
                    is_causal=mask is None,
                    dropout_p=attn_self.attention_dropout if attn_self.training else 0.0, scale=scale)
        else:
            out = _decode_batched(mgr, q, k, v, attn_self.layer_idx, scale)
        out = out.transpose(1, 2).contiguous().reshape(bsz, q_len, -1)
        if residual is None:
            return attn_self.o_proj(out), None
        o = attn_self.o_proj
        if (type(o) is Int8Linear and out.dtype == torch.float16 and bsz * q_len <= 16
                and o.qweight.is_cuda and not _hooked(o)):
            y = int8_gemv_fused(out, o.qweight, o.scale, bias=o.bias, residual=residual)
            return y.view(residual.shape), None
        return residual + o(out), None

    return forward


def _make_qwen3_forward(mgr: "KVOffloadManager"):
    """Patched Qwen3Attention.forward (helm/runtime/kv_offload.py:225-273)."""
    return _make_attention_forward(mgr, "qwen3")


def _make_qwen2_forward(mgr: "KVOffloadManager"):
    """Patched Qwen2Attention.forward (helm/runtime/kv_offload.py:174-222)."""
    return _make_attention_forward(mgr, "qwen2")


def _make_llama_forward(mgr: "KVOffloadManager"):
    """Patched LlamaAttention.forward (helm/runtime/kv_offload.py:276-323)."""
    return _make_attention_forward(mgr, "llama")


def _make_mlp_forward(orig, silu_types):
    """Decoder MLP forward (transformers' Qwen3MLP / Qwen2MLP / LlamaMLP:
    down(act(gate(x)) * up(x))) with gate, up and the SiLU product in one launch
    (helm_int8_gemv_swiglu) for 1-16 fp16 tokens on the GPU when both
    projections are Int8Linear without bias and the activation is SiLU: the same
    int8 products, fp16 roundings of gate and up, fp32 SiLU rounded to fp16 and
    product rounded to fp16 as the three separate calls.  Anything else (prefill,
    training, other modules) runs the original forward."""
    def forward(self, x):
        g, u = self.gate_proj, self.up_proj
        if (x.is_cuda and x.dtype == torch.float16 and not self.training
                and type(g) is Int8Linear and type(u) is Int8Linear
                and g.qweight.is_cuda and u.qweight.is_cuda
                and g.bias is None and u.bias is None and isinstance(self.act_fn, silu_types)
                and 0 < x.numel() <= 16 * x.shape[-1]
                and g.qweight.shape == u.qweight.shape
                and g.qweight.stride(0) == u.qweight.stride(0)
                and not _hooked(g, u, self.act_fn)):
            h = int8_gemv_swiglu(x, g.qweight, g.scale, u.qweight, u.scale)
            return self.down_proj(h.view(*x.shape[:-1], h.shape[-1]))
        return orig(self, x)
    return forward


def _make_decoder_forward(orig, silu_types):
    """Decoder layer forward (transformers' Qwen3DecoderLayer / Qwen2DecoderLayer /
    LlamaDecoderLayer: h = x + attn(norm1(x)); out = h + mlp(norm2(h))) for 1-16
    fp16 tokens on the GPU outside autograd, with INT8 MLP projections (gate / up
    without bias) and a SiLU activation: the patched attention takes x, norm1 and
    the residual, runs norm1 in the q|k|v GEMV's prologue at decode and the first
    residual add in o_proj's GEMV epilogue; norm2 runs in the gate / up SwiGLU
    GEMV's prologue and the second residual add in the down GEMV's epilogue -
    four launches fewer per layer, the same roundings (the norms' fp32 sums of
    squares in another order).  Anything else runs the original forward."""
    def forward(self, hidden_states, attention_mask=None, position_ids=None,
                past_key_values=None, use_cache=False, position_embeddings=None, **kwargs):
        mlp, post = self.mlp, self.post_attention_layernorm
        g, u, d = mlp.gate_proj, mlp.up_proj, mlp.down_proj
        if not (hidden_states.is_cuda and hidden_states.dtype == torch.float16
                and not self.training and not torch.is_grad_enabled()
                and 0 < hidden_states.numel() <= 16 * hidden_states.shape[-1]
                and type(g) is Int8Linear and type(u) is Int8Linear and type(d) is Int8Linear
                and g.qweight.is_cuda and u.qweight.is_cuda and d.qweight.is_cuda
                and g.bias is None and u.bias is None and isinstance(mlp.act_fn, silu_types)
                and g.qweight.shape == u.qweight.shape
                and g.qweight.stride(0) == u.qweight.stride(0)
                and post.weight.dtype == torch.float16 and post.weight.is_cuda
                and not _hooked(mlp, post, g, u, d, mlp.act_fn)):
            return orig(self, hidden_states, attention_mask=attention_mask,
                        position_ids=position_ids, past_key_values=past_key_values,
                        use_cache=use_cache, position_embeddings=position_embeddings, **kwargs)
        h, _ = self.self_attn(hidden_states=hidden_states, attention_mask=attention_mask,
                              position_ids=position_ids, past_key_values=past_key_values,
                              use_cache=use_cache, position_embeddings=position_embeddings,
                              _helm_input_norm=self.input_layernorm,
                              _helm_residual=hidden_states, **kwargs)
        act = int8_gemv_swiglu(h, g.qweight, g.scale, u.qweight, u.scale,
                               norm_weight=post.weight, eps=post.variance_epsilon)
        return int8_gemv_fused(act, d.qweight, d.scale, bias=d.bias, residual=h).view(h.shape)
    return forward


def _make_rmsnorm_forward(orig):
    """Decoder RMSNorm forward (transformers' Qwen3RMSNorm / Qwen2RMSNorm /
    LlamaRMSNorm: fp16(w * fp16(x * rsqrt(mean(x^2) + eps))), mean in fp32) as one
    helm_rmsnorm launch for fp16 inputs and weights on the GPU when no gradient
    is needed: the same roundings, the fp32 sum of squares in another order.
    Anything else runs the original forward."""
    def forward(self, hidden_states):
        w = self.weight
        if (hidden_states.is_cuda and hidden_states.dtype == torch.float16
                and w.dtype == torch.float16 and w.is_cuda and hidden_states.numel() > 0
                and hidden_states.shape[-1] == w.shape[0]
                and not (torch.is_grad_enabled() and (hidden_states.requires_grad or w.requires_grad))):
            return rmsnorm(hidden_states, w, self.variance_epsilon)
        return orig(self, hidden_states)
    return forward


class KVOffloadManager:
    """Installs the paged-KV attention patch and manages the cache lifecycle.

    Usage mirrors the reference:
        mgr = KVOffloadManager(model, KVOffloadConfig.from_model(model), batch_size=B)
        runtime = PipelineRuntime(model, kv_offload_mgr=mgr)
        runtime.generate(input_ids, max_new_tokens=32)
    """

    def __init__(self, model, config: KVOffloadConfig, batch_size: int = 1,
                 gpu_capacity_pages: Optional[int] = None):
        self.config = config
        self.batch_size = batch_size
        pages_per_seq = max(1, (config.cont_capacity or 4096) // config.page_size + 1)
        self.allocator = KVAllocator(
            num_layers=config.num_layers, num_kv_heads=config.num_kv_heads,
            head_dim=config.head_dim, page_size=config.page_size, dtype=config.dtype,
            gpu_capacity_pages=gpu_capacity_pages or min(1 << 16, config.num_layers * batch_size * 64),
            async_eviction=True)
        watermark_per_item = max(config.gpu_watermark_bytes // batch_size, 1)
        self.kvcms = [KVCacheManager(self.allocator, gpu_high_watermark_bytes=watermark_per_item)
                      for _ in range(batch_size)]
        self.device = next(model.parameters()).device
        self.num_q_heads = model.config.num_attention_heads
        self.ring = PinnedRing() if self.device.type == "cuda" else None
        self.page_table = None
        if self.device.type == "cuda":
            self.page_table = DevicePageTable(config.num_layers, batch_size,
                                              min(pages_per_seq, 4096), self.device, self.ring)
            for i, kvcm in enumerate(self.kvcms):
                kvcm.page_table = self.page_table
                kvcm.item = i
        self._io_state: Optional[_DecodeIO] = None
        self._plan: Optional[DecodePlan] = None   # set while a planned step's forward runs
        self._cont_table = None   # page table of the batched contiguous buffers
        self._patched: dict = {}
        self._apply_patches(model)

        if config.cont_capacity > 0 and self.device.type == "cuda":
            self._build_contiguous(config.cont_capacity)

    # ── contiguous storage shared by all items ──────────────────────────────
    def _build_contiguous(self, capacity: int) -> None:
        """One set of [B, Hkv, cap, D] buffers per layer for all items (row b is item
        b's ContiguousKV); the capacity is halved on allocation failure down to
        1024 (kv_cache.py:213-234).  When nothing fits, every item runs paged, as
        the reference drops Path 1 for all items when any of them failed
        (kv_offload.py:380-382) — with one allocation for the batch, the items
        cannot disagree."""
        cfg = self.config
        rows = ContiguousKV.allocate(self.batch_size, cfg.num_layers, cfg.num_kv_heads,
                                     cfg.head_dim, capacity, self.device, cfg.dtype,
                                     page_size=cfg.page_size)
        for b, kvcm in enumerate(self.kvcms):
            if rows:
                kvcm.build_contiguous(cfg.num_layers, cfg.num_kv_heads, cfg.head_dim,
                                      rows[b].capacity, self.device, cfg.dtype, storage=rows[b])
            else:
                kvcm.drop_contiguous()
        self._cont_table = None

    def _shared_contiguous(self, bsz: int):
        """The batch's shared ContiguousKV storage (row b = item b), or None when the
        items' buffers were built separately."""
        first = self.kvcms[0].contiguous_storage
        if first is None:
            return None
        for b in range(bsz):
            c = self.kvcms[b].contiguous_storage
            if c is None or c.k_layers is not first.k_layers or c.row != b:
                return None
        return first

    def _write_contiguous(self, layer_idx: int, k, v, pos: int, io: "_DecodeIO",
                          staged: bool = False) -> None:
        """Every item's decode K/V [B, Hkv, 1, D] at position `pos`: one
        helm_kv_append over the batch's buffers read as pages (page i of item b =
        slot b * cap/P + i).  `staged`: io already holds those slots and the
        offsets pos % P."""
        bsz = k.shape[0]
        shared = self._shared_contiguous(bsz)
        if shared is None:
            for i in range(bsz):
                self.kvcms[i].write_decode_contiguous(layer_idx, k[i:i + 1], v[i:i + 1])
            return
        P = self.config.page_size
        view = ka.PoolView.of_blocked_sequences(shared.k_layers[layer_idx],
                                                shared.v_blocks[layer_idx], P)
        if not staged:
            io.put(np.arange(bsz) * (shared.capacity // P) + pos // P, io.slots[:bsz])
            io.put(np.full(bsz, pos % P), io.offsets[:bsz])
        ka.kv_append(k.to(self.config.dtype), v.to(self.config.dtype), view, io.slots[:bsz],
                     io.offsets[:bsz], P)

    def _contiguous_attention(self, layer_idx: int, q, n: int, scale: float, io: "_DecodeIO",
                              staged: bool = False):
        """Decode attention of the B items over the first n tokens of their
        contiguous buffers, read as pages (page i of item b = slot b*cap/P + i).
        `staged`: io already holds the lengths n."""
        cfg = self.config
        P = cfg.page_size
        bsz, hq, _, d = q.shape
        n_pages = (n + P - 1) // P
        if not staged:
            io.put(np.full(bsz, n), io.seq_lens[:bsz])
        splits = ka.choose_num_splits(bsz, cfg.num_kv_heads, n_pages, P)
        part_o, part_ml = io.workspace.get(bsz, hq, d, splits)
        qh = q.reshape(bsz, hq, d).to(torch.float16)
        shared = self._shared_contiguous(bsz)
        if shared is not None:
            K, Vb = shared.k_layers[layer_idx][:bsz], shared.v_blocks[layer_idx][:, :bsz]
            table = self._contiguous_table(bsz, K.shape[2] // P, q.device)
            ka.paged_decode_attention_partial(qh, ka.PoolView.of_blocked_sequences(K, Vb, P),
                                              table[:, :n_pages], io.seq_lens[:bsz], P,
                                              scale, part_o, part_ml, splits)
        else:
            # items whose buffers were built one by one: each item's row read in
            # place by its own launch into its rows of the shared partials (no copy)
            table = torch.arange(n_pages, dtype=torch.int32, device=q.device)[None]
            per_o, per_ml = hq * splits * d, hq * splits * 2
            for i in range(bsz):
                c = self.kvcms[i].contiguous_storage
                ka.paged_decode_attention_partial(
                    qh[i:i + 1], ka.PoolView.of_blocked_sequences(c.k(layer_idx), c.v_block(layer_idx), P),
                    table, io.seq_lens[i:i + 1], P, scale, part_o[i * per_o:], part_ml[i * per_ml:],
                    splits)
        out = torch.empty(bsz, hq, d, dtype=torch.float16, device=q.device)
        ka.paged_attn_reduce(part_o, part_ml, out, splits)
        return out.to(q.dtype)

    def _plan_pool_table(self, plan: DecodePlan, layer_idx: int, device):
        """The pool view and page table [bsz, plan.pages] a planned step's layer reads."""
        if plan.path == 1:
            shared = self._shared_contiguous(plan.bsz)
            pool = ka.PoolView.of_blocked_sequences(shared.k_layers[layer_idx][:plan.bsz],
                                                    shared.v_blocks[layer_idx][:, :plan.bsz],
                                                    self.config.page_size)
            table = self._contiguous_table(plan.bsz, shared.capacity // self.config.page_size,
                                           device)
        else:
            pool = ka.PoolView.of_pool(*self._device_pool(device))
            table = self.page_table.rows(layer_idx)
        return pool, table[:plan.bsz, :plan.pages]

    def _prefill_kv_source(self, item: int, layer_idx: int, n_tokens: int, device):
        """(pool view, page table, page size) of item's prompt K/V of `layer_idx` as
        the prefill appends left them, for the prefill attention to read in place:
        the item's contiguous buffer (Path 1), or its pages when every one is in the
        device pool; None when neither holds the prompt whole (pages evicted to the
        host) or the page size is one the prefill kernel does not take."""
        cfg = self.config
        P = cfg.page_size
        if P not in (16, 32, 64) or cfg.dtype != torch.float16 or device.type != "cuda":
            return None
        n_pages = -(-n_tokens // P)
        kvcm = self.kvcms[item]
        c = kvcm.contiguous_storage
        if kvcm.use_contiguous and c is not None and c.prompt_len == n_tokens:
            ident = self._ident_pages(n_pages, device)
            return ka.PoolView.of_blocked_sequences(c.k(layer_idx), c.v_block(layer_idx), P), ident, P
        layer = kvcm.layers.get(layer_idx)
        if (self.page_table is None or layer is None or len(layer.pages) != n_pages
                or layer.total_tokens != n_tokens or not kvcm.all_gpu_resident(layer_idx)):
            return None
        self.page_table.flush()
        row = self.page_table.rows(layer_idx)[item, :n_pages]
        return ka.PoolView.of_pool(*self._device_pool(device)), row, P

    def _ident_pages(self, n: int, device) -> torch.Tensor:
        """int32 0 .. n-1 on `device` (the page table of a buffer read as pages)."""
        t = getattr(self, "_ident", None)
        if t is None or t.numel() < n or t.device != device:
            t = self._ident = torch.arange(max(n, 1024), dtype=torch.int32, device=device)
        return t[:n]

    def _contiguous_table(self, bsz: int, per_item: int, device) -> torch.Tensor:
        """Page table of the batched contiguous buffers: page i of item b is slot
        b * per_item + i (built once per batch size and capacity)."""
        if self._cont_table is None or self._cont_table.shape != (bsz, per_item):
            self._cont_table = (torch.arange(bsz, dtype=torch.int32, device=device)[:, None] * per_item
                                + torch.arange(per_item, dtype=torch.int32, device=device)[None, :])
        return self._cont_table

    def _device_pool(self, device):
        p = self.allocator.pool(device)
        return p.k, p.v

    def _io(self, device) -> _DecodeIO:
        if self._io_state is None:
            self._io_state = _DecodeIO(self.batch_size, self.config.num_layers, device, self.ring)
        return self._io_state

    # ── planned decode steps (bookkeeping before the forward) ───────────────
    def plan_decode_step(self, bsz: int) -> Optional[DecodePlan]:
        """Run the host bookkeeping of one decode step for every layer now, before
        the forward, and upload the slots, offsets and lengths the layers read
        (one copy), as _decode_batched would per layer (kv_offload.py:106-160).
        Only for steps on which no layer can evict: every item on the contiguous
        path with room left (Path 1), or every page of every layer and item on
        the GPU with no partial page before a tail (Path 2, skip_residency for
        every layer as the reference's all_gpu rule gives).  The layers then
        reserve in the same order (layer by layer, item by item), so the page
        ids and slots are the reference's.  Returns None, with nothing done,
        for every other step (the forward then does its own bookkeeping)."""
        if self.device.type != "cuda" or bsz < 1 or bsz > self.batch_size or not self._patched:
            return None
        kvcms = self.kvcms[:bsz]
        cfg = self.config
        L, P = cfg.num_layers, cfg.page_size
        io = self._io(self.device)
        meta = np.zeros((L, 3, self.batch_size), np.int32)
        if kvcms[0].use_contiguous:
            shared = self._shared_contiguous(bsz)
            pos = kvcms[0].cont_seq_len
            if (shared is None or pos >= shared.capacity
                    or any(not m.use_contiguous or m.cont_seq_len != pos for m in kvcms)):
                return None
            per_item = shared.capacity // P
            # the token's page / offset in the buffers read as pages (page i of
            # item b = slot b * per_item + i)
            meta[:, 0, :bsz] = np.arange(bsz) * per_item + pos // P
            meta[:, 1, :bsz] = pos % P
            meta[:, 2, :bsz] = pos + 1
            for kvcm in kvcms:     # the eager path counts the token after its last layer
                kvcm.advance_contiguous()
            pages = _bucket(-(-(pos + 1) // P), per_item)
            table = self._contiguous_table(bsz, per_item, self.device)
            key = (1, bsz, pages, shared.k_layers[0].data_ptr(), shared.capacity, table.data_ptr())
            path = 1
        else:
            longest = plan_paged_slots(kvcms, L, self.device, meta)
            if longest is None:
                return None
            pt = self.page_table
            pt.flush()
            pages = _bucket(longest, pt.cap)
            pool = self.allocator.pool(self.device)
            key = (2, bsz, pages, pool.k.data_ptr(), pool.v.data_ptr(), pt.dev.data_ptr(), pt.cap)
            path = 2
        self.ring.upload(meta, io.plan_meta)
        splits = ka.choose_num_splits(bsz, cfg.num_kv_heads, pages, P)
        part_o, _ = io.plan_workspace.get(bsz, self.num_q_heads, cfg.head_dim, splits)
        key += (splits, part_o.data_ptr(), io.plan_meta.data_ptr())
        return DecodePlan(path=path, bsz=bsz, pages=pages, splits=splits, key=key)

    @contextlib.contextmanager
    def planned(self, plan: Optional[DecodePlan]):
        """Run a forward under `plan`: every decode layer reads the planned slots."""
        prev, self._plan = self._plan, plan
        try:
            yield
        finally:
            self._plan = prev

    # ── public API (kv_offload.py:386-399) ──────────────────────────────────
    def reset(self):
        """Clear all paged caches and re-arm the contiguous path."""
        if self.device.type == "cuda":
            torch.cuda.current_stream(self.device).synchronize()
        for kvcm in self.kvcms:
            kvcm.clear()
            kvcm.reset_contiguous()

    def restore(self):
        for arch, (cls, orig) in self._patched.items():
            cls.forward = orig
        self._patched.clear()

    def report(self) -> dict:
        return self.allocator.report_usage()

    # ── patch dispatch (kv_offload.py:403-433) ──────────────────────────────
    def _apply_patches(self, model):
        """By lower-cased model class name: qwen3, then qwen2, then llama / mistral
        (a Mistral model gets the Llama patch, as in the reference, which replaces
        LlamaAttention.forward), else NotImplementedError."""
        name = model.__class__.__name__.lower()
        if "qwen3" in name:
            self._patch("qwen3")
        elif "qwen2" in name:
            self._patch("qwen2")
        elif "llama" in name or "mistral" in name:
            self._patch("llama")
        else:
            raise NotImplementedError(
                f"KVOffloadManager: no attention patch for {model.__class__.__name__}")

    def _patch(self, arch: str):
        """Replace <Arch>Attention.forward (kv_offload.py:416-433).  With
        config.fuse_decoder_layers the family's MLP, RMSNorm and decoder-layer
        classes are replaced too (restored together by restore())."""
        if arch == "qwen2":
            import transformers.models.qwen2.modeling_qwen2 as m
            cls, new_fwd, mlp, norm = m.Qwen2Attention, _make_qwen2_forward(self), m.Qwen2MLP, m.Qwen2RMSNorm
            layer = m.Qwen2DecoderLayer
        elif arch == "qwen3":
            import transformers.models.qwen3.modeling_qwen3 as m
            cls, new_fwd, mlp, norm = m.Qwen3Attention, _make_qwen3_forward(self), m.Qwen3MLP, m.Qwen3RMSNorm
            layer = m.Qwen3DecoderLayer
        elif arch == "llama":
            import transformers.models.llama.modeling_llama as m
            cls, new_fwd, mlp, norm = m.LlamaAttention, _make_llama_forward(self), m.LlamaMLP, m.LlamaRMSNorm
            layer = m.LlamaDecoderLayer
        else:
            raise ValueError(arch)
        self._patched[arch] = (cls, cls.forward)
        cls.forward = new_fwd
        if not self.config.fuse_decoder_layers:
            return
        # the MLP's gate / up / SiLU product as one launch at decode (same results)
        from transformers.activations import SiLUActivation
        self._patched[arch + "_mlp"] = (mlp, mlp.forward)
        mlp.forward = _make_mlp_forward(mlp.forward, (torch.nn.SiLU, SiLUActivation))
        # the decoder's RMSNorms as one launch each (same roundings)
        self._patched[arch + "_norm"] = (norm, norm.forward)
        norm.forward = _make_rmsnorm_forward(norm.forward)
        # the decoder layer: residual adds in the o / down GEMV epilogues, the
        # post-attention norm in the gate / up GEMV's prologue
        self._patched[arch + "_layer"] = (layer, layer.forward)
        layer.forward = _make_decoder_forward(layer.forward, (torch.nn.SiLU, SiLUActivation))
