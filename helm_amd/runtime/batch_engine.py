"""Greedy decode of a batch of sequences over one paged KV pool, replayed as HIP
graphs: the batched counterpart of DecodeEngine for the all-on-GPU case.

The reference decodes a batch through `_decode_batched` (helm/runtime/
kv_offload.py:82-167): B KVCacheManagers share one KVAllocator
(kv_offload.py:344-360), every item's new K/V are appended to its own pages
(:133-137) and, with every page on the GPU, one batched attention runs over the
items (Path 2, :141-160).  Here the same bookkeeping (one KVCacheManager per
item on a shared allocator, one page-table row per (layer, item)) drives one
step of fused kernels for all B items:

  embedding rows of the B previous tokens
  per layer  RMSNorm + q|k|v          helm_int8_gemv_fused, the norm in the GEMV's
                                      prologue (1-2 items; 3-4 items at hidden
                                      4096 on the matrix cores), else
                                      helm_rmsnorm + the matrix-core GEMV
             q/k norm + RoPE + KV write + split-K attention over each item's pages
                                      helm_decode_attn_fused, helm_paged_attn_reduce
             o + residual              helm_int8_gemv_fused
             RMSNorm + gate/up + SwiGLU helm_int8_gemv_swiglu, one launch (1-2
                                      items; 3-16 items at hidden 4096), else
                                      helm_rmsnorm, two GEMVs and helm_silu_mul
             down + residual           helm_int8_gemv_ws (8-16 items: k split over
                                      workgroups, partial sums in a workspace)
  head       final RMSNorm + fp16 lm_head (helm_fp16_gemv_rmsnorm), greedy tokens
                                      (helm_argmax_f16_ws)

Items may hold different context lengths (ragged page-table rows, per-item
sequence lengths).  Host-resident pages (a watermark) are not handled here:
the batch-1 DecodeEngine and the drop-in path cover offloading.
"""
from __future__ import annotations

import ctypes
import math
from typing import List, Optional

import numpy as np
import torch

from .. import _native
from .. import kernels as hk
from ..kernels import attention as ka
from ..kernels import fused
from .decode_engine import Int8Qwen3Weights, prefill_layers
from .kv_allocator import KVAllocator
from .kv_cache import KVCacheManager
from .page_table import DevicePageTable, PinnedRing

# hidden size whose RMSNorms run inside the matrix-core GEMVs at 3-16 items
# (helm_int8_gemv_fused / helm_int8_gemv_swiglu with a norm weight take K = 4096
# there).  Every workgroup normalises its own x copy, which pays for the
# gate / up + SwiGLU launch at every item count (4096 -> 2 x 12288: 8 items 20.2
# against 21.4 us with a separate RMSNorm) but for q|k|v only up to 4 items (8.8
# against 10.3 us; 16 items 18.3 against 14.2 us).
FUSED_NORM_HIDDEN = 4096
FUSED_NORM_QKV_MAX_ITEMS = 4

MAX_BATCH = 16   # the decode GEMVs take at most 16 tokens


class BatchDecodeEngine:
    """Prefill + greedy decode of `batch` sequences (all KV on the GPU)."""

    def __init__(self, weights: Int8Qwen3Weights, batch: int, max_context: int,
                 page_size: int = 16, device=None, use_graph: bool = True):
        if not 1 <= batch <= MAX_BATCH:
            raise ValueError(f"BatchDecodeEngine: batch must be 1..{MAX_BATCH}, got {batch}")
        self.w = weights
        sh = weights.shape
        self.shape = sh
        self.B = batch
        self.device = torch.device(device or weights.embed.device)
        self.P = page_size
        self.max_context = max_context
        self.max_pages = (max_context + page_size - 1) // page_size
        gpu_pages = batch * sh.n_layers * (self.max_pages + 1) + 8
        self.allocator = KVAllocator(sh.n_layers, sh.n_kv_heads, sh.head_dim, page_size,
                                     torch.float16, gpu_capacity_pages=gpu_pages,
                                     scatter_slots=True)
        self.ring = PinnedRing()
        self.pt = DevicePageTable(sh.n_layers, batch, self.max_pages + 1, self.device, self.ring)
        # one manager per item on the shared allocator (kv_offload.py:344-360); the
        # watermark never moves a page here
        self.kvcms: List[KVCacheManager] = []
        for i in range(batch):
            m = KVCacheManager(self.allocator, gpu_high_watermark_bytes=1 << 62)
            m.page_table = self.pt
            m.item = i
            self.kvcms.append(m)
        self.use_graph = use_graph
        self.scale = 1.0 / math.sqrt(sh.head_dim)
        self.inv_freq = fused.rope_inv_freq(sh.head_dim, sh.rope_theta, self.device)
        self._pool_gen = -1
        self._refresh_pool()
        dev, B = self.device, batch
        self.tok = torch.zeros(B, dtype=torch.long, device=dev)
        self.h = torch.zeros(B, sh.hidden, dtype=torch.float16, device=dev)
        self.xn = torch.empty(B, sh.hidden, dtype=torch.float16, device=dev)
        self.qkv = torch.empty(B, sh.qkv_out, dtype=torch.float16, device=dev)
        self.attn = torch.empty(B, sh.n_heads, sh.head_dim, dtype=torch.float16, device=dev)
        self.gate = torch.empty(B, sh.ffn, dtype=torch.float16, device=dev)
        self.up = torch.empty(B, sh.ffn, dtype=torch.float16, device=dev)
        self.act = torch.empty(B, sh.ffn, dtype=torch.float16, device=dev)
        self.logits = torch.empty(B, sh.vocab, dtype=torch.float16, device=dev)
        self.argmax_ws = fused.argmax_workspace(B, dev)
        self.gemv_ws_bytes = hk.gemv_workspace_bytes(B, sh.hidden, sh.ffn)
        self.gemv_ws = torch.empty(max(self.gemv_ws_bytes, 16), dtype=torch.uint8, device=dev)
        # step parameters: positions[B], seq_lens[B], slots[L][B], offsets[L][B]
        self.params = torch.zeros(2 * B + 2 * sh.n_layers * B, dtype=torch.int32, device=dev)
        most = max(self._splits_for(n) for n in range(64, self.max_pages + 64, 64))
        self.splits = self._splits_for(self.max_pages)
        self.ws = ka.AttnWorkspace(dev)
        self.part_o, self.part_ml = self.ws.get(B, sh.n_heads, sh.head_dim, max(most, self.splits))
        self.graphs = None
        self.graph_pages = 0
        self.seq = [0] * B      # tokens in each item's cache
        self.steps = 0

    def _refresh_pool(self) -> None:
        pool = self.allocator.pool(self.device)
        if pool.generation != self._pool_gen:
            self.pool = ka.PoolView.of_pool(pool.k, pool.v)
            self.pool_c = self.pool.c_struct()
            self._pool_gen = pool.generation
            self.graphs = None

    def _pool_view(self) -> ka.PoolView:
        self._refresh_pool()
        return self.pool

    # ── filling the caches ──────────────────────────────────────────────────
    @torch.no_grad()
    def prefill(self, item: int, tokens: torch.Tensor) -> torch.Tensor:
        """Prompt `tokens` [S] (int64, on the device) of `item`, whose cache must be
        empty; returns the last position's logits [V] and sets the item's next
        input token to their greedy token."""
        if self.seq[item] != 0:
            raise RuntimeError("BatchDecodeEngine.prefill starts a sequence")
        if tokens.shape[0] > self.max_context:
            raise RuntimeError("BatchDecodeEngine.prefill: prompt longer than max_context")
        h = prefill_layers(self.w, self.kvcms[item], self.allocator, self._pool_view, self.P,
                           self.scale, self.inv_freq, tokens)
        self.seq[item] = tokens.shape[0]
        sh = self.shape
        logits = fused.fp16_gemv_rmsnorm(h[-1:], self.w.norm, sh.eps, self.w.lm_head)[0]
        self.tok[item] = torch.argmax(logits)
        return logits

    def fill_synthetic_context(self, n_tokens, seed: int = 0) -> None:
        """Give each item n_tokens (an int, or one per item) of random N(0,1) KV in
        every layer, placed as prefill would place them (no forward pass)."""
        sh = self.shape
        counts = [n_tokens] * self.B if isinstance(n_tokens, int) else list(n_tokens)
        for i, n in enumerate(counts):
            for li in range(sh.n_layers):
                self.kvcms[i].reserve_prefill(li, n, self.device)
            self.seq[i] += n
        self._refresh_pool()
        g = torch.Generator(device=self.device)
        g.manual_seed(seed)
        pool = self.allocator.pool(self.device)
        pool.k.normal_(generator=g)
        pool.v_store.normal_(generator=g)

    # ── one decode step ─────────────────────────────────────────────────────
    def _reserve(self) -> None:
        """Each item's new token in every layer (kv_offload.py:133-137)."""
        B, L = self.B, self.shape.n_layers
        vals = np.empty(2 * B + 2 * L * B, np.int32)
        vals[:B] = self.seq
        vals[B:2 * B] = [s + 1 for s in self.seq]
        for i, m in enumerate(self.kvcms):
            for li in range(L):
                page, idx = m.reserve_decode_slot(li, self.device, skip_residency=True)
                vals[2 * B + li * B + i] = page.slot
                vals[2 * B + L * B + li * B + i] = idx
        self.pt.flush()
        self.ring.upload(vals, self.params)
        self.seq = [s + 1 for s in self.seq]

    def _splits_for(self, n_pages: int) -> int:
        return ka.choose_num_splits(self.B, self.shape.n_kv_heads, min(n_pages, self.max_pages),
                                    self.P)

    def _graph_pages(self) -> int:
        need = (max(self.seq) + self.P - 1) // self.P
        return min(self.max_pages, ((need + 63) // 64) * 64)

    def _layer_kernels(self, li: int, n_pages: int, stream: int) -> None:
        sh, lay, B = self.shape, self.w.layers[li], self.B
        L, H, D, F = sh.n_layers, sh.hidden, sh.head_dim, sh.ffn
        nq = sh.n_heads * D
        p = self.params
        c = _native.call
        if B <= 2 or (B <= FUSED_NORM_QKV_MAX_ITEMS and H == FUSED_NORM_HIDDEN):
            # RMSNorm in the GEMV's prologue
            c("helm_int8_gemv_fused", self.h.data_ptr(), H, lay["in_ln"].data_ptr(), sh.eps,
              lay["qkv_q"].data_ptr(), H, lay["qkv_s"].data_ptr(), None, None,
              self.qkv.data_ptr(), sh.qkv_out, B, sh.qkv_out, H, stream)
        else:
            c("helm_rmsnorm", self.h.data_ptr(), lay["in_ln"].data_ptr(), sh.eps,
              self.xn.data_ptr(), B, H, stream)
            c("helm_int8_gemv_fused", self.xn.data_ptr(), H, None, 0.0, lay["qkv_q"].data_ptr(),
              H, lay["qkv_s"].data_ptr(), None, None, self.qkv.data_ptr(), sh.qkv_out, B,
              sh.qkv_out, H, stream)
        rows = self.pt.rows(li)
        c("helm_decode_attn_fused", self.qkv.data_ptr(), sh.qkv_out, lay["q_norm"].data_ptr(),
          lay["k_norm"].data_ptr(), sh.eps, p.data_ptr(), self.inv_freq.data_ptr(),
          p[2 * B + li * B:].data_ptr(), p[2 * B + L * B + li * B:].data_ptr(),
          ctypes.byref(self.pool_c), rows.data_ptr(), rows.stride(0), p[B:].data_ptr(),
          self.part_o.data_ptr(), self.part_ml.data_ptr(), B, sh.n_heads, sh.n_kv_heads, D,
          self.P, n_pages, self.splits, self.scale, stream)
        c("helm_paged_attn_reduce", self.part_o.data_ptr(), self.part_ml.data_ptr(),
          self.attn.data_ptr(), B, sh.n_heads, D, self.splits, stream)
        c("helm_int8_gemv_fused", self.attn.data_ptr(), nq, None, 0.0, lay["o_q"].data_ptr(), nq,
          lay["o_s"].data_ptr(), None, self.h.data_ptr(), self.h.data_ptr(), H, B, H, nq, stream)
        if B <= 2 or H == FUSED_NORM_HIDDEN:
            # RMSNorm, gate, up and SwiGLU in one launch (the streaming kernel at 1-2
            # items, the matrix cores at 3-16)
            c("helm_int8_gemv_swiglu", self.h.data_ptr(), H, lay["post_ln"].data_ptr(), sh.eps,
              lay["gate_q"].data_ptr(), lay["gate_s"].data_ptr(), lay["up_q"].data_ptr(),
              lay["up_s"].data_ptr(), H, self.act.data_ptr(), F, B, F, H, stream)
        else:
            c("helm_rmsnorm", self.h.data_ptr(), lay["post_ln"].data_ptr(), sh.eps,
              self.xn.data_ptr(), B, H, stream)
            for q, s, out in ((lay["gate_q"], lay["gate_s"], self.gate),
                              (lay["up_q"], lay["up_s"], self.up)):
                c("helm_int8_gemv_fused", self.xn.data_ptr(), H, None, 0.0, q.data_ptr(), H,
                  s.data_ptr(), None, None, out.data_ptr(), F, B, F, H, stream)
            # fp16(fp16(silu(gate)) * up): the SwiGLU of the fused epilogue
            c("helm_silu_mul", self.gate.data_ptr(), self.up.data_ptr(), self.act.data_ptr(),
              B * F, stream)
        c("helm_int8_gemv_ws", self.act.data_ptr(), F, lay["down_q"].data_ptr(), F,
          lay["down_s"].data_ptr(), None, self.h.data_ptr(), self.h.data_ptr(), H, B, H, F,
          self.gemv_ws.data_ptr(), self.gemv_ws_bytes, stream)

    def _step_kernels(self, n_pages: int) -> None:
        sh = self.shape
        stream = torch.cuda.current_stream(self.device).cuda_stream
        torch.index_select(self.w.embed, 0, self.tok, out=self.h)
        for li in range(sh.n_layers):
            self._layer_kernels(li, n_pages, stream)
        _native.call("helm_fp16_gemv_rmsnorm", self.h.data_ptr(), sh.hidden, self.w.norm.data_ptr(),
                     sh.eps, self.w.lm_head.data_ptr(), sh.hidden, self.logits.data_ptr(),
                     sh.vocab, self.B, sh.vocab, sh.hidden, stream)
        _native.call("helm_argmax_f16_ws", self.logits.data_ptr(), sh.vocab, self.B, sh.vocab,
                     self.tok.data_ptr(), self.argmax_ws.data_ptr(),
                     self.argmax_ws.numel() * self.argmax_ws.element_size(), stream)

    def _capture(self, n_pages: int) -> None:
        self.graphs = None
        self.splits = self._splits_for(n_pages)
        torch.cuda.synchronize(self.device)
        saved_tok = self.tok.clone()
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):   # the real step once, outside the capture
            self._step_kernels(n_pages)
        torch.cuda.current_stream(self.device).wait_stream(s)
        torch.cuda.synchronize(self.device)
        self.tok.copy_(saved_tok)
        # two identical graphs replayed alternately (a graph launch waits for that
        # graph's previous launch)
        graphs = []
        for _ in range(2):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._step_kernels(n_pages)
            graphs.append(g)
        self.graphs = graphs
        self.graph_pages = n_pages

    @torch.no_grad()
    def decode_step(self) -> torch.Tensor:
        """Consume self.tok [B] (each item's previous token), append their KV,
        write the next greedy tokens into self.tok and return it."""
        if max(self.seq) + 1 > self.max_context:
            raise RuntimeError(f"BatchDecodeEngine: context {max(self.seq) + 1} exceeds "
                               f"max_context {self.max_context}")
        self._reserve()
        self._refresh_pool()
        n_pages = self._graph_pages()
        if self.use_graph:
            if self.graphs is None or n_pages != self.graph_pages:
                self._capture(n_pages)
            self.graphs[self.steps & 1].replay()
        else:
            # the split count the graph would use, so every rounding matches a replay
            self.splits = self._splits_for(n_pages)
            self._step_kernels(n_pages)
        self.steps += 1
        return self.tok

    def step_logits(self) -> torch.Tensor:
        """Logits [B, V] of the last decode step."""
        return self.logits
