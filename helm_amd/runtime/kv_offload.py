"""KV offload integration: class-level patched attention forward over the paged
cache (mirror of helm/runtime/kv_offload.py).

KVOffloadManager(model, config, batch_size) builds one KVAllocator shared by one
KVCacheManager per batch item (watermark split per item, :356-360), patches the
model family's attention class at class level (:403-433), and routes decode
through _decode_batched's three paths (:82-167):

  1. contiguous: in-place write into a preallocated [B, Hkv, cap, D] buffer per
     layer, attention over it (:106-126);
  2. paged, every page GPU-resident: all_gpu is computed BEFORE the append and
     passed as skip_residency (:133-137 — the watermark is not enforced while
     everything is on the GPU), then one batched kernel over the device page
     table (:141-160);
  3. mixed residency: per-item perform_streaming_attention (:163-167).

Every attention runs on the split-K paged kernel; the new token's K/V is written
into its page slot by helm_kv_append.
"""
from __future__ import annotations

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

    def __post_init__(self):
        if self.gpu_watermark_bytes is None:
            elem = torch.tensor([], dtype=self.dtype).element_size()
            per_token_bytes = 2 * self.num_kv_heads * self.head_dim * elem
            self.gpu_watermark_bytes = 512 * per_token_bytes * self.num_layers

    @staticmethod
    def from_model(model, page_size: int = 64, gpu_watermark_bytes: Optional[int] = None,
                   cont_capacity: Optional[int] = None) -> "KVOffloadConfig":
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
                               cont_capacity=cont_capacity)


class _DecodeIO:
    """Per-manager device scratch of the decode path (slots, offsets, seq lens)."""

    def __init__(self, batch: int, device: torch.device, ring: PinnedRing):
        self.ring = ring
        # slots, offsets and seq lens as the rows of one buffer, so a decode layer
        # stages all three with one host-to-device copy (put_meta)
        self.meta = torch.empty(3, batch, dtype=torch.int32, device=device)
        self.slots, self.offsets, self.seq_lens = self.meta[0], self.meta[1], self.meta[2]
        self.workspace = ka.AttnWorkspace(device)

    def put(self, arr, dst):
        self.ring.upload(np.asarray(arr, np.int32), dst)

    def put_meta(self, n: int, slots, offsets, seq_lens) -> None:
        """The first n entries of slots, offsets and seq_lens in one upload."""
        arr = np.zeros((3, self.meta.shape[1]), np.int32)
        arr[0, :n], arr[1, :n], arr[2, :n] = slots, offsets, seq_lens
        self.ring.upload(arr, self.meta)


def _decode_batched(mgr: "KVOffloadManager", q, k, v, layer_idx: int, scale: float):
    """Decode step shared by the attention patches; returns [bsz, Hq, 1, D]."""
    kvcms = mgr.kvcms
    bsz, n_q_heads, _, head_dim = q.shape
    device = q.device
    io = mgr._io(device)

    # ── Path 1: contiguous in-place buffers ─────────────────────────────────
    if kvcms[0].use_contiguous:
        pos = kvcms[0].cont_seq_len
        if pos < kvcms[0].cont_capacity:
            staged = mgr._shared_contiguous(bsz) is not None
            if staged:   # the append's slots / offsets and the attention's lengths
                io.put_meta(bsz, np.arange(bsz), np.full(bsz, pos), np.full(bsz, pos + 1))
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


def _pack_sequences(K: torch.Tensor, V: torch.Tensor):
    """Copies of [n, Hkv, cap, D] K/V views in the layout of ka.alloc_sequences."""
    n, hkv, cap, d = K.shape
    kb, vb = ka.alloc_sequences(n, hkv, cap, d, K.dtype, K.device, zero=False)
    kb.copy_(K)
    vb.copy_(V)
    return kb, vb


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
    if not all(isinstance(m, Int8Linear) for m in mods):
        return False
    if len({m.in_features for m in mods}) != 1 or len({m.bias is None for m in mods}) != 1:
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
            ok = ok and m.qweight.data_ptr() == qw[rows:].data_ptr() and m.qweight.shape[0] == n
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
                                        and in_norm.weight.is_cuda):
            hidden_states, in_norm = in_norm(hidden_states), None
        if fast:
            # decode: [input norm +] q|k|v in one INT8 GEMV over the modules' shared
            # weight rows, then the q / k norms and RoPE (the model's own cos / sin)
            # in one kernel
            if in_norm is None:
                qkv = int8_linear(hidden_states, *fused).view(bsz, -1)
            else:
                qkv = int8_gemv_fused(hidden_states, fused[0], fused[1], norm_weight=in_norm.weight,
                                      eps=in_norm.variance_epsilon, bias=fused[2]).view(bsz, -1)
            nq, nk = attn_self.q_proj.out_features, attn_self.k_proj.out_features
            D = attn_self.head_dim
            q, k = qk_norm_rope_cs(
                qkv, attn_self.q_norm.weight if qk_norm else None,
                attn_self.k_norm.weight if qk_norm else None,
                attn_self.q_norm.variance_epsilon if qk_norm else 0.0,
                cos.reshape(cos.shape[0], -1).expand(bsz, D), sin.reshape(sin.shape[0], -1).expand(bsz, D),
                nq // D, nk // D, D)
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
        if q_len > 1:
            for i in range(bsz):
                kvcms[i].append_prefill(attn_self.layer_idx, k[i:i + 1], v[i:i + 1])
                if kvcms[i].use_contiguous:
                    kvcms[i].prefill_contiguous(attn_self.layer_idx, k[i:i + 1], v[i:i + 1])
            on_kernels = q.dtype == torch.float16 and q.is_cuda and not attn_self.training
            causal = on_kernels and _is_causal_mask(attention_mask, q_len)
            masks = (None if causal or not on_kernels
                     else _item_masks(attention_mask, bsz, q.shape[1], q_len))
            if causal or masks is not None:
                # prefill on the matrix cores, one item at a time over a dense
                # page-layout copy of its prompt K/V: the plain causal mask by
                # helm_prefill_attn, any other 4-D mask (padding ...) added to the
                # scores by helm_prefill_attn_mask
                out = torch.empty_like(q)
                for i in range(bsz):
                    pool, pt = ka.dense_prefill_kv(k[i].transpose(0, 1), v[i].transpose(0, 1), 16)
                    o = ka.prefill_attention(q[i].transpose(0, 1), pool, pt, 16, 0, scale,
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
        if type(o) is Int8Linear and out.dtype == torch.float16 and bsz * q_len <= 16:
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
                and g.bias is None and u.bias is None and isinstance(self.act_fn, silu_types)
                and 0 < x.numel() <= 16 * x.shape[-1]
                and g.qweight.shape == u.qweight.shape
                and g.qweight.stride(0) == u.qweight.stride(0)):
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
                and g.bias is None and u.bias is None and isinstance(mlp.act_fn, silu_types)
                and g.qweight.shape == u.qweight.shape
                and g.qweight.stride(0) == u.qweight.stride(0)
                and post.weight.dtype == torch.float16 and post.weight.is_cuda):
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
        self.ring = PinnedRing() if self.device.type == "cuda" else None
        self.page_table = None
        if self.device.type == "cuda":
            self.page_table = DevicePageTable(config.num_layers, batch_size,
                                              min(pages_per_seq, 4096), self.device, self.ring)
            for i, kvcm in enumerate(self.kvcms):
                kvcm.page_table = self.page_table
                kvcm.item = i
        self._io_state: Optional[_DecodeIO] = None
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
                                     multiple=cfg.page_size)
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
        helm_kv_append over the batch's buffers (one slot per sequence, page = the
        whole capacity).  `staged`: io already holds slots 0..B-1 and offsets pos."""
        bsz = k.shape[0]
        shared = self._shared_contiguous(bsz)
        if shared is None:
            for i in range(bsz):
                self.kvcms[i].write_decode_contiguous(layer_idx, k[i:i + 1], v[i:i + 1])
            return
        view = ka.PoolView.of_whole_sequences(shared.k_layers[layer_idx], shared.v_layers[layer_idx])
        if not staged:
            io.put(np.arange(bsz), io.slots[:bsz])
            io.put(np.full(bsz, pos), io.offsets[:bsz])
        ka.kv_append(k.to(self.config.dtype), v.to(self.config.dtype), view, io.slots[:bsz],
                     io.offsets[:bsz], shared.capacity)

    def _contiguous_attention(self, layer_idx: int, q, n: int, scale: float, io: "_DecodeIO",
                              staged: bool = False):
        """Decode attention of the B items over the first n tokens of their
        contiguous buffers, read as pages (page i of item b = slot b*cap/P + i).
        `staged`: io already holds the lengths n."""
        cfg = self.config
        P = cfg.page_size
        bsz, hq, _, d = q.shape
        shared = self._shared_contiguous(bsz)
        if shared is not None:
            K, V = shared.k_layers[layer_idx][:bsz], shared.v_layers[layer_idx][:bsz]
        else:
            K = torch.cat([self.kvcms[i].contiguous_storage.k(layer_idx) for i in range(bsz)])
            V = torch.cat([self.kvcms[i].contiguous_storage.v(layer_idx) for i in range(bsz)])
            K, V = _pack_sequences(K, V)
        cap = K.shape[2]
        per_item = cap // P
        if self._cont_table is None or self._cont_table.shape != (bsz, per_item):
            self._cont_table = (torch.arange(bsz, dtype=torch.int32, device=q.device)[:, None] * per_item
                                + torch.arange(per_item, dtype=torch.int32, device=q.device)[None, :])
        n_pages = (n + P - 1) // P
        if not staged:
            io.put(np.full(bsz, n), io.seq_lens[:bsz])
        splits = ka.choose_num_splits(bsz, cfg.num_kv_heads, n_pages, P)
        part_o, part_ml = io.workspace.get(bsz, hq, d, splits)
        qh = q.reshape(bsz, hq, d).to(torch.float16)
        ka.paged_decode_attention_partial(qh, ka.PoolView.of_sequences(K, V, P),
                                          self._cont_table[:, :n_pages], io.seq_lens[:bsz], P,
                                          scale, part_o, part_ml, splits)
        out = torch.empty(bsz, hq, d, dtype=torch.float16, device=q.device)
        ka.paged_attn_reduce(part_o, part_ml, out, splits)
        return out.to(q.dtype)

    def _device_pool(self, device):
        p = self.allocator.pool(device)
        return p.k, p.v

    def _io(self, device) -> _DecodeIO:
        if self._io_state is None:
            self._io_state = _DecodeIO(self.batch_size, device, self.ring)
        return self._io_state

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
