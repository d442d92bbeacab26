"""Native decode engine for Qwen3-shaped INT8 models on MI355X.

The reference's decode step is the HF decoder layer with its attention forward
patched (helm/runtime/kv_offload.py:225-273) driven by PipelineRuntime
(pipeline_runtime.py:88-176).  The engine computes the same step from the same
page tables, but with the glue around the hot path fused into the kernels and
the whole step replayed as one HIP graph:

  per layer   helm_int8_gemv_fused   input RMSNorm + packed q|k|v projection
              helm_decode_attn_fused  q/k RMSNorm, RoPE, K/V into the page slot,
                                     split-K attention partials
              helm_paged_attn_reduce
              helm_int8_gemv_fused   o projection + residual add
              helm_int8_gemv_swiglu  post-attn RMSNorm + gate/up + SiLU(gate)*up
              helm_int8_gemv_fused   down projection + residual add
  then        helm_rmsnorm, helm_fp16_gemv (fp16 lm_head), argmax on the device.

Host work per step is the KVCacheManager bookkeeping for every layer
(reserve_decode_slot: page allocation, token counts, residency policy with the
reference's all_gpu/skip_residency rule), one packed upload of the step's
position / slot / offset values and the page-table rows that changed.  The
graph is used while every page is GPU-resident; otherwise the step runs eagerly:
each layer's host-resident pages (a prefix of its pages) are staged one layer
ahead by the gather kernel on a copy stream and attended next to the
device-resident suffix (see _eager_mixed_step).
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Dict, List, Optional

import numpy as np
import torch

from .. import _native
from ..kernels import attention as ka
from ..kernels import fused, int8_linear, quantize_per_channel
from .kv_allocator import KVAllocator
from .kv_cache import KVCacheManager, perform_streaming_attention
from .page_table import DevicePageTable, PinnedRing


@dataclass(frozen=True)
class Qwen3Shape:
    hidden: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn: int
    n_layers: int
    vocab: int
    eps: float = 1e-6
    rope_theta: float = 1e6

    @property
    def qkv_out(self) -> int:
        return (self.n_heads + 2 * self.n_kv_heads) * self.head_dim

    def linear_bytes(self) -> int:
        """INT8 weight bytes of all decoder-layer linears."""
        H, F = self.hidden, self.ffn
        per = self.qkv_out * H + self.n_heads * self.head_dim * H + 2 * F * H + H * F
        return per * self.n_layers


QWEN3_8B = Qwen3Shape(hidden=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=12288,
                      n_layers=36, vocab=151936)
QWEN3_32B = Qwen3Shape(hidden=5120, n_heads=64, n_kv_heads=8, head_dim=128, ffn=25600,
                       n_layers=64, vocab=151936)
QWEN3_PLUMBING = Qwen3Shape(hidden=1024, n_heads=16, n_kv_heads=8, head_dim=64, ffn=3072,
                            n_layers=2, vocab=32000)


class Int8Qwen3Weights:
    """Weights laid out for the decode kernels: packed q|k|v rows per layer,
    separate gate / up / down / o, fp16 norms, fp16 embedding and lm_head."""

    def __init__(self, shape: Qwen3Shape):
        self.shape = shape
        self.layers: List[Dict[str, torch.Tensor]] = []
        self.embed: Optional[torch.Tensor] = None
        self.norm: Optional[torch.Tensor] = None
        self.lm_head: Optional[torch.Tensor] = None

    @staticmethod
    def _quant(w: torch.Tensor):
        return quantize_per_channel(w)

    @classmethod
    def random(cls, shape: Qwen3Shape, device, seed: int = 0, std: float = 0.02,
               norm_jitter: float = 0.0) -> "Int8Qwen3Weights":
        """Random-init weights N(0, std), each linear INT8 per-channel quantised;
        norms are 1 (+ optional jitter).  Generated on `device`."""
        self = cls(shape)
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        H, D = shape.hidden, shape.head_dim

        def normal(*size):
            return (torch.randn(*size, generator=g, device=device, dtype=torch.float32) * std).half()

        def norm_w(n):
            w = torch.ones(n, device=device, dtype=torch.float32)
            if norm_jitter:
                w += torch.randn(n, generator=g, device=device) * norm_jitter
            return w.half()

        for _ in range(shape.n_layers):
            lay = {}
            lay["qkv_q"], lay["qkv_s"] = cls._quant(normal(shape.qkv_out, H))
            lay["o_q"], lay["o_s"] = cls._quant(normal(H, shape.n_heads * D))
            lay["gate_q"], lay["gate_s"] = cls._quant(normal(shape.ffn, H))
            lay["up_q"], lay["up_s"] = cls._quant(normal(shape.ffn, H))
            lay["down_q"], lay["down_s"] = cls._quant(normal(H, shape.ffn))
            lay["in_ln"] = norm_w(H)
            lay["post_ln"] = norm_w(H)
            lay["q_norm"] = norm_w(D)
            lay["k_norm"] = norm_w(D)
            self.layers.append(lay)
        self.embed = normal(shape.vocab, H)
        self.norm = norm_w(H)
        self.lm_head = normal(shape.vocab, H)
        return self

    @classmethod
    def from_hf(cls, model) -> "Int8Qwen3Weights":
        """Take the weights of a transformers Qwen3ForCausalLM whose linears were
        replaced by Int8Linear (helm_amd.kernels.patch_linears); q/k/v are packed
        into one buffer and the modules are re-pointed at views of it, so the
        patched-forward path and the engine share storage."""
        cfg = model.config
        D = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        shape = Qwen3Shape(cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads, D,
                           cfg.intermediate_size, cfg.num_hidden_layers, cfg.vocab_size,
                           cfg.rms_norm_eps, float(cfg.rope_parameters["rope_theta"])
                           if hasattr(cfg, "rope_parameters") and cfg.rope_parameters
                           else float(getattr(cfg, "rope_theta", 1e6)))
        self = cls(shape)
        for layer in model.model.layers:
            at, mlp = layer.self_attn, layer.mlp
            q = torch.cat([at.q_proj.qweight, at.k_proj.qweight, at.v_proj.qweight], 0).contiguous()
            s = torch.cat([at.q_proj.scale, at.k_proj.scale, at.v_proj.scale], 0).contiguous()
            nq, nk = at.q_proj.qweight.shape[0], at.k_proj.qweight.shape[0]
            at.q_proj.qweight, at.q_proj.scale = q[:nq], s[:nq]
            at.k_proj.qweight, at.k_proj.scale = q[nq:nq + nk], s[nq:nq + nk]
            at.v_proj.qweight, at.v_proj.scale = q[nq + nk:], s[nq + nk:]
            self.layers.append({
                "qkv_q": q, "qkv_s": s,
                "o_q": at.o_proj.qweight, "o_s": at.o_proj.scale,
                "gate_q": mlp.gate_proj.qweight, "gate_s": mlp.gate_proj.scale,
                "up_q": mlp.up_proj.qweight, "up_s": mlp.up_proj.scale,
                "down_q": mlp.down_proj.qweight, "down_s": mlp.down_proj.scale,
                "in_ln": layer.input_layernorm.weight.detach(),
                "post_ln": layer.post_attention_layernorm.weight.detach(),
                "q_norm": at.q_norm.weight.detach(), "k_norm": at.k_norm.weight.detach(),
            })
        self.embed = model.model.embed_tokens.weight.detach()
        self.norm = model.model.norm.weight.detach()
        self.lm_head = model.lm_head.weight.detach()
        return self


def prefill_layers(w: Int8Qwen3Weights, kvcm: KVCacheManager, allocator: KVAllocator,
                   pool_view, P: int, scale: float, inv_freq: torch.Tensor,
                   tokens: torch.Tensor) -> torch.Tensor:
    """The decoder layers over a new sequence's prompt `tokens` [S] (int64, on the
    device), its K/V left in `kvcm`'s pages; returns the last layer's hidden states
    [S, H].  pool_view() returns the kernels' view of the device pool (it may
    have grown when pages were reserved).

    Per layer: helm_rmsnorm, the INT8 q|k|v GEMM, helm_qk_norm_rope_append over
    the S tokens (q/k RMSNorm + RoPE, the prompt's K/V written into pages),
    causal helm_prefill_attn over those pages, and the o / gate / up / down
    GEMMs.  When no page of this prompt can be evicted (the watermark cannot be
    crossed) the K/V go straight into the layer's pool pages and the attention
    reads them there; otherwise they go to a dense page-layout buffer first and
    append_prefill moves them into pages in the reference's write-then-enforce
    order (an evicted page holds its tokens)."""
    sh = w.shape
    S = tokens.shape[0]
    D = sh.head_dim
    dev = tokens.device
    nq = sh.n_heads * D
    h = w.embed.index_select(0, tokens)
    positions = torch.arange(S, dtype=torch.int32, device=dev)
    q = torch.empty(S, sh.n_heads, D, dtype=torch.float16, device=dev)
    n_pages = (S + P - 1) // P
    page_bytes = allocator.page_bytes()
    for li, lay in enumerate(w.layers):
        x = fused.rmsnorm(h, lay["in_ln"], sh.eps)
        qkv = int8_linear(x, lay["qkv_q"], lay["qkv_s"])
        direct = (kvcm.gpu_evictable_bytes() + n_pages * page_bytes
                  <= kvcm.gpu_high_watermark_bytes)
        if direct:
            kvcm.reserve_prefill(li, S, dev)
            pool = pool_view()
            pages = kvcm.layers[li].pages[-n_pages:]
            pt = torch.tensor([p.slot for p in pages], dtype=torch.int32).to(dev)
        else:
            pool, pt = ka.dense_prefill_pool(S, sh.n_kv_heads, D, P, dev)
        slots = pt.repeat_interleave(P)[:S]
        offsets = positions.remainder(P)
        fused.qk_norm_rope_append(qkv, lay["q_norm"], lay["k_norm"], sh.eps, positions,
                                  inv_freq, q, pool, slots, offsets, sh.n_heads,
                                  sh.n_kv_heads, D, P)
        if not direct:
            kvcm.append_prefill(li, pool.k[:, :, :S], pool.v[:, :, :S])
        a = ka.prefill_attention(q, pool, pt, P, 0, scale).view(S, nq)
        h = h + int8_linear(a, lay["o_q"], lay["o_s"])
        x = fused.rmsnorm(h, lay["post_ln"], sh.eps)
        gt = int8_linear(x, lay["gate_q"], lay["gate_s"])
        up = int8_linear(x, lay["up_q"], lay["up_s"])
        # fp16(fp16(silu(gate)) * up) in one kernel (torch's two ops round the same)
        h = h + int8_linear(fused.silu_mul(gt, up), lay["down_q"], lay["down_s"])
    pool_view()
    return h


class DecodeEngine:
    """Prefill + greedy decode of one sequence over a paged KV cache."""

    def __init__(self, weights: Int8Qwen3Weights, max_context: int, page_size: int = 16,
                 gpu_watermark_bytes: Optional[int] = None, device=None,
                 use_graph: bool = True, fused_attention: bool = True,
                 int8_lm_head: bool = False):
        self.w = weights
        # int8_lm_head: the lm_head quantised like the layers' linears (per-channel
        # symmetric INT8) and run by the INT8 GEMV with the final RMSNorm fused;
        # default: the fp16 lm_head
        self.lm_q = self.lm_s = None
        if int8_lm_head:
            self.lm_q, self.lm_s = quantize_per_channel(weights.lm_head)
        sh = weights.shape
        self.shape = sh
        self.device = torch.device(device or weights.embed.device)
        self.P = page_size
        self.max_context = max_context
        self.max_pages = (max_context + page_size - 1) // page_size
        # pool sized for every page of every layer, so slots never move mid-run
        gpu_pages = sh.n_layers * (self.max_pages + 1) + 8
        self.allocator = KVAllocator(sh.n_layers, sh.n_kv_heads, sh.head_dim, page_size,
                                     torch.float16, gpu_capacity_pages=gpu_pages,
                                     async_eviction=True, scatter_slots=True)
        wm = gpu_watermark_bytes if gpu_watermark_bytes is not None else 1 << 62
        self.kvcm = KVCacheManager(self.allocator, gpu_high_watermark_bytes=wm)
        self.ring = PinnedRing()
        self.pt = DevicePageTable(sh.n_layers, 1, self.max_pages + 1, self.device, self.ring)
        self.kvcm.page_table = self.pt
        self.kvcm.item = 0
        self.use_graph = use_graph
        # one launch for q/k norm + RoPE + KV write + attention partials
        # (helm_decode_attn_fused) instead of two
        self.fused_attention = fused_attention
        self.scale = 1.0 / math.sqrt(sh.head_dim)
        self.inv_freq = fused.rope_inv_freq(sh.head_dim, sh.rope_theta, self.device)
        self._pool_gen = -1
        self._refresh_pool()
        # static device buffers of the decode step
        dev = self.device
        self.tok = torch.zeros(1, dtype=torch.long, device=dev)
        self.h = torch.zeros(1, sh.hidden, dtype=torch.float16, device=dev)
        self.qkv = torch.empty(1, sh.qkv_out, dtype=torch.float16, device=dev)
        self.q = torch.empty(1, sh.n_heads, sh.head_dim, dtype=torch.float16, device=dev)
        self.attn = torch.empty(1, sh.n_heads, sh.head_dim, dtype=torch.float16, device=dev)
        self.act = torch.empty(1, sh.ffn, dtype=torch.float16, device=dev)
        self.xn = torch.empty(1, sh.hidden, dtype=torch.float16, device=dev)
        self.logits = torch.empty(1, sh.vocab, dtype=torch.float16, device=dev)
        self.argmax_ws = fused.argmax_workspace(1, dev)
        # packed step parameters: [pos, seq_len, slots[L], offsets[L]]
        self.params = torch.zeros(2 + 2 * sh.n_layers, dtype=torch.int32, device=dev)
        # the split count follows the page-table width a graph is captured for
        # (_graph_pages); the workspace holds the most any width here needs
        self.splits = self._splits_for(self.max_pages)
        most = max(self._splits_for(n) for n in range(64, self.max_pages + 64, 64))
        self.ws = ka.AttnWorkspace(dev)
        self.part_o, self.part_ml = self.ws.get(1, sh.n_heads, sh.head_dim, max(most, self.splits))
        self.graph = None
        self.graph_pages = 0
        self.seq = 0          # tokens in the cache
        self.all_gpu = True

    def _refresh_pool(self) -> None:
        """(Re)build the kernels' view of the device page pool after it moved."""
        pool = self.allocator.pool(self.device)
        if pool.generation != self._pool_gen:
            self.pool = ka.PoolView.of_pool(pool.k, pool.v)
            self.pool_c = self.pool.c_struct()
            self._pool_gen = pool.generation
            self.graph = None

    def _pool_view(self) -> ka.PoolView:
        self._refresh_pool()
        return self.pool

    # ── prefill (MFMA GEMMs, kernel glue) ───────────────────────────────────
    @torch.no_grad()
    def prefill(self, tokens: torch.Tensor) -> torch.Tensor:
        """tokens [S] int64 on the device; returns the last position's logits [V]
        and leaves the KV of all S tokens in the page tables (prefill_layers).
        The final RMSNorm + lm_head of the last position is the decode head's
        GEMV."""
        if self.seq != 0:
            raise RuntimeError("DecodeEngine.prefill starts a sequence; continuing one is not "
                               "supported (the KV of earlier tokens would not be attended)")
        S = tokens.shape[0]
        h = prefill_layers(self.w, self.kvcm, self.allocator, self._pool_view, self.P,
                           self.scale, self.inv_freq, tokens)
        self._refresh_pool()
        self.seq += S
        self.h.copy_(h[-1:])
        self._head_kernels(torch.cuda.current_stream(self.device).cuda_stream, argmax=False)
        self.all_gpu = all(self.kvcm.all_gpu_resident(li) for li in range(self.shape.n_layers))
        return self.logits[0].clone()

    def fill_synthetic_context(self, n_tokens: int, seed: int = 0) -> None:
        """Give every layer `n_tokens` of random N(0,1) fp16 KV (no forward pass):
        the decode cost at a context length does not depend on the KV values.
        The pages are reserved exactly as prefill would place them, then the whole
        device pool is filled with random values in one pass."""
        sh = self.shape
        for li in range(sh.n_layers):
            self.kvcm.reserve_prefill(li, n_tokens, self.device)
        self.allocator.synchronize()       # eviction copies land before the pools are refilled
        g = torch.Generator(device=self.device)
        g.manual_seed(seed)
        pool = self.allocator.pool(self.device)
        pool.k.normal_(generator=g)
        pool.v_store.normal_(generator=g)
        # pages the watermark moved to the host get random values too (copied from
        # the device pool in chunks)
        host = self.allocator._pools.get(("cpu", None))
        if host is not None and host.next_slot > 0 and pool.capacity > 0:
            for i in range(0, host.next_slot, pool.capacity):
                n = min(pool.capacity, host.next_slot - i)
                host.k[i:i + n].copy_(pool.k[:n])
                host.v_store[i:i + n].copy_(pool.v_store[:n])
            torch.cuda.synchronize(self.device)
        self.seq += n_tokens
        self.all_gpu = all(self.kvcm.all_gpu_resident(li) for li in range(sh.n_layers))

    # ── one decode step ─────────────────────────────────────────────────────
    def _reserve(self) -> None:
        """Bookkeeping for the new token in every layer (kv_offload.py:133-137)."""
        sh = self.shape
        L = sh.n_layers
        vals = np.empty(2 + 2 * L, np.int32)
        vals[0] = self.seq
        vals[1] = self.seq + 1
        all_gpu = True
        for li in range(L):
            layer_all_gpu = self.kvcm.all_gpu_resident(li)
            page, idx = self.kvcm.reserve_decode_slot(li, self.device, skip_residency=layer_all_gpu)
            vals[2 + li] = page.slot
            vals[2 + L + li] = idx
            all_gpu = all_gpu and self.kvcm.all_gpu_resident(li)
        self.all_gpu = all_gpu
        self.pt.flush()
        self.ring.upload(vals, self.params)
        self.seq += 1

    def _layer_kernels(self, li: int, n_pages: int, stream: int) -> None:
        sh, lay = self.shape, self.w.layers[li]
        L = sh.n_layers
        H, D = sh.hidden, sh.head_dim
        p = self.params
        c = _native.call
        c("helm_int8_gemv_fused", self.h.data_ptr(), H, lay["in_ln"].data_ptr(), sh.eps,
          lay["qkv_q"].data_ptr(), H, lay["qkv_s"].data_ptr(), None, None,
          self.qkv.data_ptr(), sh.qkv_out, 1, sh.qkv_out, H, stream)
        pool = ctypes.byref(self.pool_c)
        rows = self.pt.rows(li)
        if self.fused_attention:
            c("helm_decode_attn_fused", self.qkv.data_ptr(), sh.qkv_out, lay["q_norm"].data_ptr(),
              lay["k_norm"].data_ptr(), sh.eps, p.data_ptr(), self.inv_freq.data_ptr(),
              p[2 + li:].data_ptr(), p[2 + L + li:].data_ptr(), pool, rows.data_ptr(),
              rows.stride(0), p[1:].data_ptr(), self.part_o.data_ptr(), self.part_ml.data_ptr(),
              1, sh.n_heads, sh.n_kv_heads, D, self.P, n_pages, self.splits, self.scale, stream)
        else:
            c("helm_qk_norm_rope_append", self.qkv.data_ptr(), lay["q_norm"].data_ptr(),
              lay["k_norm"].data_ptr(), sh.eps, p.data_ptr(), self.inv_freq.data_ptr(),
              self.q.data_ptr(), pool, p[2 + li:].data_ptr(), p[2 + L + li:].data_ptr(), 1,
              sh.n_heads, sh.n_kv_heads, D, self.P, stream)
            c("helm_paged_decode_attn", self.q.data_ptr(), sh.n_heads * D, D, pool,
              rows.data_ptr(), rows.stride(0), p[1:].data_ptr(), self.part_o.data_ptr(),
              self.part_ml.data_ptr(), 0, self.splits, 1, sh.n_heads, sh.n_kv_heads, D, self.P,
              n_pages, self.splits, self.scale, stream)
        c("helm_paged_attn_reduce", self.part_o.data_ptr(), self.part_ml.data_ptr(),
          self.attn.data_ptr(), 1, sh.n_heads, D, self.splits, stream)
        c("helm_int8_gemv_fused", self.attn.data_ptr(), sh.n_heads * D, None, 0.0,
          lay["o_q"].data_ptr(), sh.n_heads * D, lay["o_s"].data_ptr(), None,
          self.h.data_ptr(), self.h.data_ptr(), H, 1, H, sh.n_heads * D, stream)
        c("helm_int8_gemv_swiglu", self.h.data_ptr(), H, lay["post_ln"].data_ptr(), sh.eps,
          lay["gate_q"].data_ptr(), lay["gate_s"].data_ptr(), lay["up_q"].data_ptr(),
          lay["up_s"].data_ptr(), H, self.act.data_ptr(), sh.ffn, 1, sh.ffn, H, stream)
        c("helm_int8_gemv_fused", self.act.data_ptr(), sh.ffn, None, 0.0,
          lay["down_q"].data_ptr(), sh.ffn, lay["down_s"].data_ptr(), None,
          self.h.data_ptr(), self.h.data_ptr(), H, 1, H, sh.ffn, stream)

    def _head_kernels(self, stream: int, argmax: bool = True) -> None:
        sh = self.shape
        # final RMSNorm fused into the lm_head GEMV (fp16, or INT8), then the greedy token
        if self.lm_q is not None:
            _native.call("helm_int8_gemv_fused", self.h.data_ptr(), sh.hidden, self.w.norm.data_ptr(),
                         sh.eps, self.lm_q.data_ptr(), sh.hidden, self.lm_s.data_ptr(), None, None,
                         self.logits.data_ptr(), sh.vocab, 1, sh.vocab, sh.hidden, stream)
        else:
            _native.call("helm_fp16_gemv_rmsnorm", self.h.data_ptr(), sh.hidden,
                         self.w.norm.data_ptr(), sh.eps, self.w.lm_head.data_ptr(), sh.hidden,
                         self.logits.data_ptr(), sh.vocab, 1, sh.vocab, sh.hidden, stream)
        if argmax:
            _native.call("helm_argmax_f16_ws", self.logits.data_ptr(), sh.vocab, 1, sh.vocab,
                         self.tok.data_ptr(), self.argmax_ws.data_ptr(),
                         self.argmax_ws.numel() * self.argmax_ws.element_size(), stream)

    def _step_kernels(self, n_pages: int) -> None:
        stream = torch.cuda.current_stream(self.device).cuda_stream
        torch.index_select(self.w.embed, 0, self.tok, out=self.h)
        for li in range(self.shape.n_layers):
            self._layer_kernels(li, n_pages, stream)
        self._head_kernels(stream)

    def _splits_for(self, n_pages: int) -> int:
        return ka.choose_num_splits(1, self.shape.n_kv_heads, min(n_pages, self.max_pages), self.P)

    def _graph_pages(self) -> int:
        """Page count the graph is captured for (max_pages argument): covers the
        current context, rounded up to 64 pages so one capture serves 1024 tokens."""
        need = (self.seq + self.P - 1) // self.P
        return min(self.max_pages, ((need + 63) // 64) * 64)

    def _capture(self, n_pages: int) -> None:
        self.graph = None
        self.splits = self._splits_for(n_pages)
        torch.cuda.synchronize(self.device)
        saved_tok = self.tok.clone()
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):   # warm the code paths outside the capture
            # the warm-up runs the real step once (same inputs, so its KV write is
            # the one the replay repeats); the input token is restored afterwards
            self._step_kernels(n_pages)
        torch.cuda.current_stream(self.device).wait_stream(s)
        torch.cuda.synchronize(self.device)
        self.tok.copy_(saved_tok)
        # Two identical executable graphs, replayed alternately: a launch of a graph
        # waits for that graph's previous launch, so with one graph the host could
        # not prepare step t+1 while step t runs.  Stream order still serialises
        # the two.
        graphs = []
        for _ in range(2):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._step_kernels(n_pages)
            graphs.append(g)
        self.graphs = graphs
        self.graph = graphs[0]
        self.graph_pages = n_pages

    @torch.no_grad()
    def decode_step(self) -> torch.Tensor:
        """Consume self.tok (the previous token), append its KV, write the next
        greedy token into self.tok and return it (device tensor [1])."""
        if self.seq + 1 > self.max_context:
            raise RuntimeError(f"DecodeEngine: context {self.seq + 1} exceeds max_context {self.max_context}")
        self._reserve()
        self._refresh_pool()   # page allocation may have grown the pool
        if self.all_gpu and self.use_graph:
            n_pages = self._graph_pages()
            if self.graph is None or n_pages != self.graph_pages:
                # the step's uploads were issued on this stream; capture re-runs the
                # step body once outside the graph, so re-upload after it
                self._capture(n_pages)
            self.graphs[self.seq & 1].replay()
        elif self.all_gpu:
            # same max_pages (and split count) as the graph would use, so the split-K
            # partitioning (and therefore every rounding) is identical to a replay
            n_pages = self._graph_pages()
            self.splits = self._splits_for(n_pages)
            self._step_kernels(n_pages)
        else:
            self._eager_mixed_step()
        return self.tok

    def _offload_state(self) -> dict:
        """Device staging for host-resident pages: two buffers of max_pages pages
        (layers alternate between them), per-layer host-slot rows, the
        per-layer (device-suffix, host-prefix) lengths, a copy stream and the
        events that order the two streams."""
        st = getattr(self, "_off", None)
        if st is None:
            sh, dev = self.shape, self.device
            cap = self.max_pages + 1
            shape = (sh.n_kv_heads, self.P, sh.head_dim)
            k = torch.empty((2 * cap, *shape), dtype=torch.float16, device=dev)
            v = ka.alloc_v((2 * cap, *shape), dtype=torch.float16, device=dev)
            st = self._off = dict(
                cap=cap, k=k, v=v, view=ka.PoolView.of_pool(k, v),
                copy=torch.cuda.Stream(device=dev),   # default priority
                slots=torch.full((sh.n_layers, cap), -1, dtype=torch.int32, device=dev),
                slots_np=np.full((sh.n_layers, cap), -1, np.int32), n_host=[0] * sh.n_layers,
                stage_pt=torch.arange(2 * cap, dtype=torch.int32, device=dev).view(2, cap),
                lens=torch.zeros(2 * sh.n_layers, dtype=torch.int32, device=dev),
                gathered=[torch.cuda.Event(), torch.cuda.Event()],
                free=[torch.cuda.Event(), torch.cuda.Event()], used=[False, False])
        return st

    def _eager_mixed_step(self) -> None:
        """Step with host-resident pages.  Oldest-first eviction keeps each layer's
        host pages a prefix of its page list (in token order), so a layer's
        attention is two segments: the device suffix read in place, and the host
        prefix staged by the gather kernel (pinned host memory read directly over
        the host link) into one of two device buffers.  The staging runs on its own
        stream one layer ahead (layer l + 2 is staged into the buffer layer l has
        just read), so the host link stays busy while the layers compute; one
        reduce merges both segments' partials (kv_cache.py:318-442 order-free)."""
        sh = self.shape
        L, H, D, P = sh.n_layers, sh.hidden, sh.head_dim, self.P
        st = self._offload_state()
        cap = st["cap"]
        compute = torch.cuda.current_stream(self.device)
        stream = compute.cuda_stream
        copy = st["copy"]
        # host prefixes only grow (evictions append the layer's next-oldest page)
        changed = False
        for li in range(L):
            hp = self.kvcm._host_pages.get(li, ())
            n0 = st["n_host"][li]
            if len(hp) != n0:
                if len(hp) < n0:
                    n0 = 0
                st["slots_np"][li, n0:len(hp)] = [pg.slot for pg in hp[n0:]]
                st["n_host"][li] = len(hp)
                changed = True
        if changed:
            self.ring.upload(st["slots_np"], st["slots"])
        n_pages = (self.seq + P - 1) // P
        lens = np.empty(2 * L, np.int32)
        for li in range(L):
            lens[li] = self.seq - st["n_host"][li] * P       # device suffix tokens (incl. the new one)
            lens[L + li] = st["n_host"][li] * P              # host prefix: whole pages
        self.ring.upload(lens, st["lens"])
        host_pool = self.allocator.pool(torch.device("cpu"))
        # the gathers read host pages that evictions of this step may still be writing
        copy.wait_stream(self.allocator._evict_stream(self.device))
        copy.wait_stream(compute)   # slot rows and lengths were uploaded on the compute stream

        def gather(li: int) -> None:
            b = li % 2
            n = st["n_host"][li]
            if n == 0:
                return
            if st["used"][b]:
                copy.wait_event(st["free"][b])
            with torch.cuda.stream(copy):
                ka.gather_pages_h2d(host_pool.k, host_pool.v, st["k"], st["v"],
                                    st["slots"][li, :n], b * cap, copy)
                st["gathered"][b].record(copy)

        gather(0)
        if L > 1:
            gather(1)
        torch.index_select(self.w.embed, 0, self.tok, out=self.h)
        p = self.params
        pool = ctypes.byref(self.pool_c)
        stage_c = st["view"].c_struct()
        stage = ctypes.byref(stage_c)
        q = self.q
        for li, lay in enumerate(self.w.layers):
            _native.call("helm_int8_gemv_fused", self.h.data_ptr(), H, lay["in_ln"].data_ptr(),
                         sh.eps, lay["qkv_q"].data_ptr(), H, lay["qkv_s"].data_ptr(), None, None,
                         self.qkv.data_ptr(), sh.qkv_out, 1, sh.qkv_out, H, stream)
            _native.call("helm_qk_norm_rope_append", self.qkv.data_ptr(), lay["q_norm"].data_ptr(),
                         lay["k_norm"].data_ptr(), sh.eps, p.data_ptr(), self.inv_freq.data_ptr(),
                         q.data_ptr(), pool, p[2 + li:].data_ptr(), p[2 + L + li:].data_ptr(), 1,
                         sh.n_heads, sh.n_kv_heads, D, P, stream)
            nh = st["n_host"][li]
            nd = n_pages - nh
            s_dev = ka.choose_num_splits(1, sh.n_kv_heads, nd, P)
            s_host = ka.choose_num_splits(1, sh.n_kv_heads, nh, P) if nh else 0
            total = s_dev + s_host
            part_o, part_ml = self.ws.get(1, sh.n_heads, D, total)
            rows = self.pt.rows(li)
            _native.call("helm_paged_decode_attn", q.data_ptr(), sh.n_heads * D, D, pool,
                         rows[:, nh:].data_ptr(), rows.stride(0), st["lens"][li:].data_ptr(),
                         part_o.data_ptr(), part_ml.data_ptr(), 0, total, 1, sh.n_heads,
                         sh.n_kv_heads, D, P, nd, s_dev, self.scale, stream)
            if nh:
                b = li % 2
                compute.wait_event(st["gathered"][b])
                _native.call("helm_paged_decode_attn", q.data_ptr(), sh.n_heads * D, D,
                             stage, st["stage_pt"][b].data_ptr(), cap,
                             st["lens"][L + li:].data_ptr(), part_o.data_ptr(), part_ml.data_ptr(),
                             s_dev, total, 1, sh.n_heads, sh.n_kv_heads, D, P, nh, s_host,
                             self.scale, stream)
                st["free"][b].record(compute)
                st["used"][b] = True
                if li + 2 < L:
                    gather(li + 2)
            _native.call("helm_paged_attn_reduce", part_o.data_ptr(), part_ml.data_ptr(),
                         self.attn.data_ptr(), 1, sh.n_heads, D, total, stream)
            _native.call("helm_int8_gemv_fused", self.attn.data_ptr(), sh.n_heads * D, None, 0.0,
                         lay["o_q"].data_ptr(), sh.n_heads * D, lay["o_s"].data_ptr(), None,
                         self.h.data_ptr(), self.h.data_ptr(), H, 1, H, sh.n_heads * D, stream)
            _native.call("helm_int8_gemv_swiglu", self.h.data_ptr(), H, lay["post_ln"].data_ptr(),
                         sh.eps, lay["gate_q"].data_ptr(), lay["gate_s"].data_ptr(),
                         lay["up_q"].data_ptr(), lay["up_s"].data_ptr(), H, self.act.data_ptr(),
                         sh.ffn, 1, sh.ffn, H, stream)
            _native.call("helm_int8_gemv_fused", self.act.data_ptr(), sh.ffn, None, 0.0,
                         lay["down_q"].data_ptr(), sh.ffn, lay["down_s"].data_ptr(), None,
                         self.h.data_ptr(), self.h.data_ptr(), H, 1, H, sh.ffn, stream)
        self._head_kernels(stream)

    @torch.no_grad()
    def generate(self, prompt: torch.Tensor, max_new_tokens: int) -> torch.Tensor:
        """Greedy decode (pipeline_runtime.py:140-176): the first new token is the
        argmax of the prefill logits; each decode step feeds the previous token."""
        logits = self.prefill(prompt)
        self.tok.copy_(torch.argmax(logits, dim=-1, keepdim=True))
        out = [self.tok.clone()]
        for _ in range(max_new_tokens - 1):
            out.append(self.decode_step().clone())
        return torch.cat(out)

    def step_logits(self) -> torch.Tensor:
        return self.logits[0]
