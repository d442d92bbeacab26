"""Paged KV cache manager + streaming decode attention (mirror of helm/runtime/kv_cache.py).

KVCacheManager keeps the reference's API and decisions (kv_cache.py:30-311):
append_prefill / append_decode / evict_pages / _enforce_residency_policy /
all_gpu_resident / clear / contiguous path / report_bytes_per_tier.  What changes
is the cost: the reference rescans every page of every layer on each append
(:161-172) and sorts all candidates on each eviction (:126-137).  Here

  * the evictable set (GPU, cuda, full, not the layer's tail) is maintained
    incrementally: a page joins it when it stops being its layer's tail, leaves
    it when evicted; its byte total is a counter;
  * eviction pops a heap keyed (start_token, layer insertion rank) — exactly the
    order of the reference's stable sort by start_token over layers in dict
    order — so the same pages are evicted in the same order;
  * every page remembers its index in its layer's list, so the in-place
    replacement (:151-153) needs no list.index scan;
  * all_gpu_resident checks only the layer's non-GPU pages.

perform_streaming_attention (:318-442) runs on the GPU kernels: device-resident
pool pages are attended in place through their slot page table, host-resident
pages are staged to the device in chunks on a side copy stream (double-buffered,
one event per chunk) while the previous chunk is attended, and every launch
writes its own split range of one fp32 partial buffer that a final reduce merges.
"""
from __future__ import annotations

import collections.abc
import heapq
import math
from collections import Counter
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import torch

import numpy as np

from ..kernels import attention as ka
from .kv_allocator import KVAllocator, KVPage  # noqa: F401  (KVPage re-exported)
from .page_table import PinnedRing


@dataclass(eq=False)
class LayerKVCache:
    """The pages of one layer of one sequence in token order, the page that takes
    the next decode token (`tail_page`) and the token count: the reference's
    per-layer record (kv_cache.py:19-28).  `ragged` is this build's addition: it
    turns True once a page that is not full stops being the tail (a second
    prefill, or the decode tokens migrated out of the contiguous buffer, appended
    after a partial page), after which token t is no longer at page t // P."""
    layer_id: int
    pages: List[KVPage] = field(default_factory=list)
    tail_page: Optional[KVPage] = None
    total_tokens: int = 0
    ragged: bool = False

    def append_page(self, page: KVPage) -> None:
        prev = self.tail_page
        if prev is not None and prev.used_tokens < prev.capacity_tokens:
            self.ragged = True
        self.pages.append(page)
        self.tail_page = page


class KVCacheManager:
    """Owns all layer KV state of one sequence: append, residency, attention inputs."""

    def __init__(self, allocator: KVAllocator, gpu_high_watermark_bytes: int = 0.25 * 1024 * 1024):
        self.allocator = allocator
        self.layers: Dict[int, LayerKVCache] = {}
        self.gpu_high_watermark_bytes = gpu_high_watermark_bytes
        # Path 1 storage (ContiguousKV) and whether decode uses it
        self._cont: Optional[ContiguousKV] = None
        self.use_contiguous: bool = False
        # incremental residency state
        self._page_bytes = allocator.page_bytes()
        self._heap: list = []              # (start_token, layer_rank, page_id)
        self._evictable: Dict[int, tuple] = {}   # page_id -> (layer, page)
        self._evictable_bytes = 0
        self._rank: Dict[int, int] = {}
        self._next_rank = 0
        self._index: Dict[int, int] = {}   # page_id -> position in its layer's list
        self._host_pages: Dict[int, List[KVPage]] = {}  # layer -> non-GPU pages, list order
        self.page_table = None             # optional device page-table mirror
        self.item = 0                      # row of this sequence in that mirror
        self._prefill_src = None           # (K, V) of the append_prefill in progress
        self._prefill_pending: list = []   # its GPU pages not written yet: (page, start, n)

    # ── layer bookkeeping ───────────────────────────────────────────────────
    def initialize_layer_caches(self, num_layers: int):
        for i in range(num_layers):
            self._new_layer(i)

    def _new_layer(self, layer_id: int) -> LayerKVCache:
        layer = LayerKVCache(layer_id=layer_id)
        self.layers[layer_id] = layer
        self._rank[layer_id] = self._next_rank
        self._next_rank += 1
        self._host_pages[layer_id] = []
        return layer

    def _layer(self, layer_id: int) -> LayerKVCache:
        layer = self.layers.get(layer_id)
        if layer is None:
            layer = self._new_layer(layer_id)
        return layer

    def _attach(self, layer: LayerKVCache, page: KVPage) -> None:
        """layer.append_page plus the incremental bookkeeping."""
        prev = layer.tail_page
        self._index[page.page_id] = len(layer.pages)
        layer.append_page(page)
        if page.state != "GPU":
            self._host_pages.setdefault(layer.layer_id, []).append(page)
        if prev is not None:
            self._maybe_evictable(layer, prev)
        if self.page_table is not None:
            self.page_table.set(layer.layer_id, self.item, len(layer.pages) - 1, page)

    def _maybe_evictable(self, layer: LayerKVCache, page: KVPage) -> None:
        if (page.state == "GPU" and page.device.type == "cuda" and page is not layer.tail_page
                and page.used_tokens == page.capacity_tokens
                and page.page_id not in self._evictable):
            self._evictable[page.page_id] = (layer, page)
            self._evictable_bytes += self._page_bytes
            heapq.heappush(self._heap, (page.start_token, self._rank[layer.layer_id], page.page_id))

    # ── append paths (kv_cache.py:55-113) ───────────────────────────────────
    def append_prefill(self, layer_id: int, K_prefill: torch.Tensor, V_prefill: torch.Tensor,
                       device: Optional[torch.device] = None):
        """Append prefill KV ([1, Hkv, S, D]) in page-sized chunks, enforcing the
        watermark after every page.  Pages go to K_prefill's device unless
        `device` names the tier explicitly."""
        device = K_prefill.device if device is None else torch.device(device)

        def copy(page, start_idx, chunk_len):
            page.k_tensor[:, :, :chunk_len, :].copy_(K_prefill[:, :, start_idx:start_idx + chunk_len, :])
            page.v_tensor[:, :, :chunk_len, :].copy_(V_prefill[:, :, start_idx:start_idx + chunk_len, :])
        if device.type != "cuda" or not K_prefill.is_cuda:
            self._append_pages(layer_id, K_prefill.size(2), device, copy)
            return
        # GPU pages: the writes are queued and issued as one helm_kv_append per
        # run of pages, before any eviction could move a queued page (evict_pages
        # flushes first) and at the end, so every page holds its tokens before it
        # can be copied anywhere, as with the reference's write-then-enforce order.
        self._prefill_src = (K_prefill, V_prefill)
        self._prefill_pending = []

        def queue(page, start_idx, chunk_len):
            if page.state == "GPU" and page.device.type == "cuda":
                self._prefill_pending.append((page, start_idx, chunk_len))
            else:
                copy(page, start_idx, chunk_len)
        try:
            self._append_pages(layer_id, K_prefill.size(2), device, queue)
        finally:
            self._flush_prefill_writes()
            self._prefill_src = None

    def _flush_prefill_writes(self) -> None:
        """Write the queued prompt pages: full pages (consecutive token chunks) in
        one helm_kv_append over [pages, Hkv, P, D], a partial last page in a
        second call with its own token count."""
        pending, self._prefill_pending = self._prefill_pending, []
        if not pending:
            return
        K, V = self._prefill_src
        P = self.allocator.page_size
        dev = pending[0][0].k_tensor.device
        pool = self.allocator.pool(dev)
        view = ka.PoolView.of_pool(pool.k, pool.v)
        full = [e for e in pending if e[2] == P]
        part = [e for e in pending if e[2] != P]
        if full:
            s0, n = full[0][1], len(full)
            assert all(e[1] == s0 + i * P for i, e in enumerate(full)), "prefill pages out of order"
            hkv, d = K.size(1), K.size(3)
            kn = K[0, :, s0:s0 + n * P].reshape(hkv, n, P, d).transpose(0, 1).contiguous()
            vn = V[0, :, s0:s0 + n * P].reshape(hkv, n, P, d).transpose(0, 1).contiguous()
            slots = torch.tensor([e[0].slot for e in full], dtype=torch.int32).to(dev)
            ka.kv_append(kn, vn, view, slots, torch.zeros_like(slots), P)
        for page, start, n in part:
            slots = torch.tensor([page.slot], dtype=torch.int32).to(dev)
            ka.kv_append(K[:, :, start:start + n], V[:, :, start:start + n], view, slots,
                         torch.zeros_like(slots), P)

    def reserve_prefill(self, layer_id: int, n_tokens: int, device: torch.device) -> None:
        """Bookkeeping half of append_prefill: the same pages, page order and
        residency decisions for `n_tokens` tokens, without writing any KV (the
        caller fills the pages)."""
        self._append_pages(layer_id, n_tokens, torch.device(device), None)

    def _append_pages(self, layer_id: int, seq_len: int, device: torch.device, copy) -> None:
        layer = self._layer(layer_id)
        page_size = self.allocator.page_size
        for start_idx in range(0, seq_len, page_size):
            chunk_len = min(page_size, seq_len - start_idx)
            page = self.allocator.allocate(device)
            page.layer_id = layer_id
            page.start_token = layer.total_tokens
            page.used_tokens = chunk_len
            if copy is not None:
                copy(page, start_idx, chunk_len)
            self._attach(layer, page)
            layer.total_tokens += chunk_len
            self._enforce_residency_policy()

    def reserve_decode_slot(self, layer_id: int, device: torch.device,
                            skip_residency: bool = False):
        """Bookkeeping half of append_decode: make room for one token on the
        layer's tail page (allocating a page if the tail is full), count it, and
        enforce the watermark unless skipped.  Returns (page, index in page) —
        the page is the tail as it was BEFORE residency ran, which never evicts
        a tail.  The caller writes the token's K/V there."""
        layer = self._layer(layer_id)
        if layer.tail_page is None or layer.tail_page.used_tokens == layer.tail_page.capacity_tokens:
            page = self.allocator.allocate(device)
            page.layer_id = layer_id
            page.start_token = layer.total_tokens
            page.used_tokens = 0
            self._attach(layer, page)
        page = layer.tail_page
        idx = page.used_tokens
        page.used_tokens += 1
        layer.total_tokens += 1
        if not skip_residency:
            self._enforce_residency_policy()
        return page, idx

    def append_decode(self, layer_id: int, K_new: torch.Tensor, V_new: torch.Tensor,
                      skip_residency: bool = False, device: Optional[torch.device] = None):
        """Append a single token KV pair ([1, Hkv, 1, D]) for the given layer."""
        layer = self._layer(layer_id)
        if layer.tail_page is None or layer.tail_page.used_tokens == layer.tail_page.capacity_tokens:
            page = self.allocator.allocate(K_new.device if device is None else torch.device(device))
            page.layer_id = layer_id
            page.start_token = layer.total_tokens
            page.used_tokens = 0
            self._attach(layer, page)
        page = layer.tail_page
        idx = page.used_tokens
        page.k_tensor[:, :, idx:idx + 1, :].copy_(K_new)
        page.v_tensor[:, :, idx:idx + 1, :].copy_(V_new)
        page.used_tokens += 1
        layer.total_tokens += 1
        if not skip_residency:
            self._enforce_residency_policy()

    def iterate_layer_pages(self, layer_id: int):
        if layer_id not in self.layers:
            return []
        return list(self.layers[layer_id].pages)

    # ── residency (kv_cache.py:121-172) ─────────────────────────────────────
    def _pop_evictable(self):
        while self._heap:
            _, _, pid = heapq.heappop(self._heap)
            entry = self._evictable.pop(pid, None)
            if entry is None:
                continue
            layer, page = entry
            self._evictable_bytes -= self._page_bytes
            if (self.layers.get(layer.layer_id) is layer and page.state == "GPU"
                    and page.device.type == "cuda" and page is not layer.tail_page
                    and page.used_tokens == page.capacity_tokens):
                return layer, page
        return None

    def evict_pages(self, bytes_to_evict: int):
        """Global oldest-page-first eviction to the CPU (pinned host pool)."""
        if bytes_to_evict <= 0:
            return
        self._flush_prefill_writes()       # queued prompt pages hold their tokens first
        evicted_bytes = 0
        cpu = torch.device("cpu")
        while evicted_bytes < bytes_to_evict:
            entry = self._pop_evictable()
            if entry is None:
                break
            layer, page = entry
            where = (page.layer_id, page.start_token, page.used_tokens)
            new_page = self.allocator.move_page(page, cpu)
            if (new_page.layer_id, new_page.start_token, new_page.used_tokens) != where:
                raise RuntimeError(f"evict_pages: page {page.page_id} moved to the host as "
                                   f"(layer, start, used) = {(new_page.layer_id, new_page.start_token, new_page.used_tokens)}, "
                                   f"expected {where}")
            idx = self._index.pop(page.page_id)
            layer.pages[idx] = new_page
            self._index[new_page.page_id] = idx
            self._insert_host_page(layer.layer_id, new_page)
            if layer.tail_page is page:
                layer.tail_page = new_page
            if self.page_table is not None:
                self.page_table.set(layer.layer_id, self.item, idx, new_page)
            evicted_bytes += new_page.k_tensor.numel() * new_page.k_tensor.element_size() * 2

    def _insert_host_page(self, layer_id: int, page: KVPage) -> None:
        lst = self._host_pages.setdefault(layer_id, [])
        pos = self._index[page.page_id]
        if not lst or self._index[lst[-1].page_id] < pos:
            lst.append(page)
        else:  # keep list order (evictions normally arrive oldest first)
            i = len(lst)
            while i > 0 and self._index[lst[i - 1].page_id] > pos:
                i -= 1
            lst.insert(i, page)

    def _enforce_residency_policy(self):
        # the watermark applies to evictable pages only (full, GPU, not a tail)
        if self._evictable_bytes > self.gpu_high_watermark_bytes:
            self.evict_pages(self._evictable_bytes - self.gpu_high_watermark_bytes)

    def gpu_evictable_bytes(self) -> int:
        return self._evictable_bytes

    # ── queries ─────────────────────────────────────────────────────────────
    def seq_len(self):
        if 0 in self.layers:
            return self.layers[0].total_tokens
        return 0

    def num_layers(self):
        return len(self.layers)

    def layers_keys(self):
        return sorted(self.layers.keys())

    def all_gpu_resident(self, layer_id: int) -> bool:
        """True if every used page of the layer is GPU-resident (kv_cache.py:195-202)."""
        if layer_id not in self.layers:
            return True
        for page in self._host_pages.get(layer_id, ()):
            if page.used_tokens > 0 and page.state != "GPU":
                return False
        return True

    def host_pages(self, layer_id: int) -> List[KVPage]:
        """The layer's non-GPU pages in list (token) order."""
        return list(self._host_pages.get(layer_id, ()))

    def page_index(self, page: KVPage) -> int:
        return self._index[page.page_id]

    def clear(self):
        for layer in self.layers.values():
            for page in layer.pages:
                if page.state != "DEAD":
                    self.allocator.free(page)
            layer.pages.clear()
            layer.tail_page = None
            layer.total_tokens = 0
        self.layers.clear()
        self._heap.clear()
        self._evictable.clear()
        self._evictable_bytes = 0
        self._rank.clear()
        self._index.clear()
        self._host_pages.clear()
        if self.page_table is not None:
            self.page_table.clear_item(self.item)

    def layer_is_ragged(self, layer_id: int) -> bool:
        """True when a page before the layer's tail is not full (LayerKVCache.ragged)."""
        layer = self.layers.get(layer_id)
        return layer is not None and layer.ragged

    def report_bytes_per_tier(self) -> dict:
        """K+V bytes of the pages held per tier (kv_cache.py:294-311): a page counts
        its tensors' full size whatever its fill; DEAD placeholders count nothing."""
        per_state = Counter()
        for layer in self.layers.values():
            for page in layer.pages:
                per_state[page.state] += 2 * page.k_tensor.numel() * page.k_tensor.element_size()
        return {"gpu_active_bytes": per_state["GPU"], "cpu_active_bytes": per_state["CPU"]}

    # ── contiguous storage, the reference's Path 1 (kv_cache.py:206-289) ────
    # One ContiguousKV per sequence (None when the path is off); the attributes
    # and methods below keep the reference's names and meaning on top of it.
    @property
    def cont_K(self) -> dict:
        c = self._cont
        return {} if c is None else {i: c.k(i) for i in range(c.num_layers)}

    @property
    def cont_V(self):
        """Layer -> V [1, Hkv, capacity, D]; each lookup copies that layer's V out of
        its page blocks (the buffers store V as the pools do)."""
        c = self._cont
        return {} if c is None else _LayerV(c)

    @property
    def cont_capacity(self) -> int:
        return 0 if self._cont is None else self._cont.capacity

    @property
    def cont_num_layers(self) -> int:
        return 0 if self._cont is None else self._cont.num_layers

    @property
    def cont_seq_len(self) -> int:
        """Tokens every layer's buffer holds (the decode token in flight excluded)."""
        return 0 if self._cont is None else self._cont.committed

    @property
    def cont_prefill_len(self) -> int:
        return 0 if self._cont is None else self._cont.prompt_len

    @property
    def contiguous_storage(self) -> Optional["ContiguousKV"]:
        return self._cont

    def build_contiguous(self, num_layers: int, num_kv_heads: int, head_dim: int,
                         capacity: int, device: torch.device, dtype: torch.dtype,
                         storage: Optional["ContiguousKV"] = None) -> bool:
        """Give this sequence contiguous K/V buffers of `capacity` tokens per layer
        (halved on allocation failure down to 1024, as kv_cache.py:213-234);
        False, with the path off, when even that fails.  `storage` hands in a
        row of buffers a caller allocated for several sequences at once."""
        if storage is None:
            storage = ContiguousKV.allocate(1, num_layers, num_kv_heads, head_dim, capacity,
                                            device, dtype, page_size=self.allocator.page_size)
            storage = storage[0] if storage else None
        self._cont = storage
        self.use_contiguous = storage is not None
        return self.use_contiguous

    def prefill_contiguous(self, layer_id: int, K: torch.Tensor, V: torch.Tensor):
        """Prompt K/V [1, Hkv, n, D] into positions 0..n-1 (layer 0 sets the counts)."""
        self._cont.write(layer_id, 0, K, V)
        if layer_id == 0:
            self._cont.prompt_len = self._cont.committed = K.shape[2]

    def write_decode_contiguous(self, layer_id: int, K_new: torch.Tensor, V_new: torch.Tensor):
        """The decode token's K/V [1, Hkv, 1, D] at the first free position."""
        self._cont.write(layer_id, self._cont.committed, K_new, V_new)

    def get_kv_contiguous(self, layer_id: int):
        """The layer's tokens including the decode token in flight: K a view, V a
        copy out of its page blocks."""
        n = self._cont.committed + 1
        return self._cont.k(layer_id)[:, :, :n], self._cont.v_tokens(layer_id, 0, n)

    def advance_contiguous(self):
        """Count the decode token in flight once the last layer has written it."""
        self._cont.committed += 1

    def migrate_contiguous_to_pages(self):
        """Leave Path 1: the decode tokens written since the prompt go to pages of
        every layer (the prompt's pages were written at prefill), then the buffers
        are released.  The new pages follow the prompt's last page even when that
        one is partial, as the reference appends them with append_prefill."""
        c = self._cont
        if c is None:
            return
        lo, hi = c.prompt_len, c.committed
        for layer_id in range(c.num_layers if hi > lo else 0):
            self.append_prefill(layer_id, c.k(layer_id)[:, :, lo:hi], c.v_tokens(layer_id, lo, hi),
                                device=c.device)
        self.drop_contiguous()

    def drop_contiguous(self):
        self._cont = None
        self.use_contiguous = False

    def reset_contiguous(self):
        """Re-arm Path 1 for the next request when buffers are still held."""
        if self._cont is not None:
            self._cont.prompt_len = self._cont.committed = 0
            self.use_contiguous = True


class _LayerV(collections.abc.Mapping):
    """cont_V of one sequence: layer -> its V [1, Hkv, capacity, D], copied out of
    the page blocks when looked up."""

    def __init__(self, cont: "ContiguousKV"):
        self._c = cont

    def __getitem__(self, layer: int) -> torch.Tensor:
        if not isinstance(layer, int) or not 0 <= layer < self._c.num_layers:
            raise KeyError(layer)
        return self._c.v(layer)

    def __iter__(self):
        return iter(range(self._c.num_layers))

    def __len__(self) -> int:
        return self._c.num_layers


class ContiguousKV:
    """Path 1 storage of one sequence: row `row` of per-layer K/V buffers of
    `capacity` tokens shared by a batch of sequences (ka.alloc_blocked_sequences:
    K token rows, V in P-token page blocks), which the decode kernels read as
    pages through PoolView.of_blocked_sequences.  `prompt_len` counts the prompt
    tokens, `committed` every token all layers hold."""

    def __init__(self, k_layers: List[torch.Tensor], v_blocks: List[torch.Tensor], row: int,
                 page_size: int, device: Optional[torch.device] = None):
        self.k_layers, self.v_blocks, self.row = k_layers, v_blocks, row
        self.page_size = page_size
        self.num_layers = len(k_layers)
        self.capacity = k_layers[0].shape[2]
        # the tier the decode tokens' pages go to when they migrate (the device
        # the buffers were asked for)
        self.device = torch.device(device) if device is not None else k_layers[0].device
        self.prompt_len = 0
        self.committed = 0

    @staticmethod
    def allocate(n_seqs: int, num_layers: int, num_kv_heads: int, head_dim: int, capacity: int,
                 device, dtype, floor: int = 1024, page_size: int = 16) -> List["ContiguousKV"]:
        """Buffers for `n_seqs` sequences, zero-filled, one allocation per layer and
        K/V.  The capacity (rounded down to a multiple of the page size) is halved
        after an allocation failure while it stays >= `floor`; [] when nothing
        fits."""
        device = torch.device(device)
        P = page_size
        cap = (int(capacity) // P) * P
        while cap >= floor:
            try:
                bufs = [ka.alloc_blocked_sequences(n_seqs, num_kv_heads, cap, head_dim, P, dtype,
                                                   device, zero=True) for _ in range(num_layers)]
            except (torch.cuda.OutOfMemoryError, RuntimeError):
                bufs = None
                if device.type == "cuda" and torch.cuda.is_available():
                    torch.cuda.empty_cache()
            if bufs is not None:
                k_layers = [b[0] for b in bufs]
                v_blocks = [b[1] for b in bufs]
                return [ContiguousKV(k_layers, v_blocks, r, P, device) for r in range(n_seqs)]
            cap = ((cap // 2) // P) * P
        return []

    def k(self, layer: int) -> torch.Tensor:
        """K of this sequence, a view [1, Hkv, capacity, D]."""
        return self.k_layers[layer][self.row:self.row + 1]

    def v_block(self, layer: int) -> torch.Tensor:
        """V of this sequence in page blocks, a view [Hkv, 1, capacity / P, D, P]."""
        return self.v_blocks[layer][:, self.row:self.row + 1]

    def v_tokens(self, layer: int, lo: int, hi: int) -> torch.Tensor:
        """V of positions lo .. hi-1 as a new tensor [1, Hkv, hi - lo, D]."""
        P = self.page_size
        p0, p1 = lo // P, -(-hi // P)
        vb = self.v_blocks[layer][:, self.row, p0:p1]            # [Hkv, pages, D, P]
        hkv, pages, d, _ = vb.shape
        tok = vb.transpose(-1, -2).reshape(hkv, pages * P, d)    # [Hkv, tokens, D]
        return tok[:, lo - p0 * P:hi - p0 * P].unsqueeze(0).contiguous()

    def v(self, layer: int) -> torch.Tensor:
        """V of this sequence as a new tensor [1, Hkv, capacity, D] (V is stored
        in page blocks, so this is a copy, not a view)."""
        return self.v_tokens(layer, 0, self.capacity)

    def write(self, layer: int, start: int, K: torch.Tensor, V: torch.Tensor) -> None:
        """K/V [1, Hkv, n, D] into positions start .. start+n-1 of `layer`: whole
        pages in one copy, a partial first or last page on its own."""
        n = K.shape[2]
        if start + n > self.capacity:
            raise RuntimeError(f"contiguous KV: tokens {start}..{start + n - 1} exceed the "
                               f"capacity of {self.capacity}")
        self.k(layer)[:, :, start:start + n].copy_(K)
        P = self.page_size
        vb = self.v_blocks[layer][:, self.row]                   # [Hkv, pages, D, P]
        hkv, d = vb.shape[0], vb.shape[2]
        t = 0
        while t < n:
            pos = start + t
            pg, off = pos // P, pos % P
            if off == 0 and n - t >= P:
                m = (n - t) // P
                vb[:, pg:pg + m].copy_(V[0, :, t:t + m * P].reshape(hkv, m, P, d).transpose(-1, -2))
                t += m * P
            else:
                m = min(P - off, n - t)
                vb[:, pg, :, off:off + m].copy_(V[0, :, t:t + m].transpose(-1, -2))
                t += m


# ─────────────────────────────────────────────────────────────────────────────
# Streaming decode attention on the GPU
# ─────────────────────────────────────────────────────────────────────────────

class _StreamState:
    """Per-device reusable resources of perform_streaming_attention."""

    def __init__(self, device: torch.device):
        self.device = device
        self.copy_stream = torch.cuda.Stream(device=device)   # default priority
        self.workspace = ka.AttnWorkspace(device)
        self.staging = None   # (k, v) device staging pools [2 * chunk, Hkv, P, D]
        self.buf_free = [torch.cuda.Event(), torch.cuda.Event()]
        # marks a staging half's pages landed; re-recorded by the half's next
        # gather only after every wait on its previous record has been enqueued
        self.buf_ready = [torch.cuda.Event(), torch.cuda.Event()]
        self.buf_used = [False, False]
        self.ring = PinnedRing(1 << 20)   # snapshot uploads of page tables / lengths
        self.stage_rows = None   # device int32 0 .. 2 * chunk - 1: the staging page tables

    def upload_i32(self, values) -> torch.Tensor:
        """Device int32 copy of `values`, uploaded asynchronously from a pinned
        snapshot (never from a temporary pageable buffer)."""
        arr = np.ascontiguousarray(np.asarray(values, dtype=np.int32))
        out = torch.empty(arr.shape, dtype=torch.int32, device=self.device)
        self.ring.upload(arr, out)
        return out

    def staging_pools(self, chunk: int, shape, dtype):
        need = (2 * chunk, *shape)
        if self.staging is None or tuple(self.staging[0].shape) != need or self.staging[0].dtype != dtype:
            # same layout as the host pool (K token rows, V token-contiguous per dim)
            self.staging = (torch.empty(need, dtype=dtype, device=self.device),
                            ka.alloc_v(need, dtype=dtype, device=self.device))
        if self.stage_rows is None or self.stage_rows.numel() != 2 * chunk:
            self.stage_rows = torch.arange(2 * chunk, dtype=torch.int32, device=self.device)
        return self.staging


_STATE: Dict[int, _StreamState] = {}
STAGE_CHUNK_PAGES = 256  # pages per staged chunk (8 MiB of K+V at Hkv=8, P=16, D=128)


def _state(device: torch.device) -> _StreamState:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    st = _STATE.get(idx)
    if st is None:
        st = _STATE[idx] = _StreamState(torch.device("cuda", idx))
    return st


def _split_count(n_pages: int, n_heads: int, page_size: int) -> int:
    return ka.choose_num_splits(1, n_heads, max(1, n_pages), page_size)


def _wait_ready(stream, page: KVPage) -> None:
    """Order `stream` after the eviction copy into host page `page`; once that copy
    is known complete the event is dropped, so later steps skip it."""
    ev = page.ready
    if ev is not None:
        if ev.query():
            page.ready = None
        else:
            stream.wait_event(ev)


class PageWalk:
    """What perform_streaming_attention does with each page of its list, from one
    pass over it (helm/runtime/kv_cache.py:350-351 for the page filter: pages
    with no used tokens, and pages on the other tier than their state says, are
    skipped):
      first_active   the first page attended (None: nothing to attend)
      run_lens       page counts of the runs of in-place device-pool pages (a run
                     ends at a partial page: token t of a run is at its page t // P)
      run_meta       int32: each run's slots, then its token count
      chunk_slots    int32 host-pool slots of each chunk of full host pages to stage
      chunk_waits    each chunk's pages whose eviction copy may still be in flight
      gpu_rest, cpu_rest  the other attended pages, for the dense repack
    A chunk closes when it holds `chunk_pages` pages, or, while fewer than two
    chunks are closed (a staging half still free), when its run of host pages
    ends, so its transfer can start before the rest of the list is attended."""
    __slots__ = ("first_active", "run_lens", "run_meta", "chunk_slots", "chunk_waits",
                 "gpu_rest", "cpu_rest")

    def __init__(self, first_active, run_lens, run_meta, chunk_slots, chunk_waits, gpu_rest,
                 cpu_rest):
        self.first_active = first_active
        self.run_lens = run_lens
        self.run_meta = run_meta
        self.chunk_slots = chunk_slots
        self.chunk_waits = chunk_waits
        self.gpu_rest = gpu_rest
        self.cpu_rest = cpu_rest


def walk_pages_py(pages, gbound, gviews, hbound, hviews, chunk_pages: int,
                  page_size: int) -> PageWalk:
    """PageWalk of `pages` in Python.  gbound / hbound map a device / host pool
    slot to the page bound to it, gviews / hviews the slot to the (k, v) views
    that page holds; a page is read in place (device) or staged by slot (host)
    only while it is the slot's bound page and still holds those views."""
    runs_meta, run_lens = [], []
    run_slots = []
    chunks, chunk, waits, chunk_waits = [], [], [], []
    gpu_rest, cpu_rest = [], []
    first_active = None
    is_cuda = {}

    def close_chunk():
        nonlocal chunk, waits
        chunks.append(chunk)
        chunk_waits.append(waits)
        chunk, waits = [], []

    for p in pages:
        u = p.used_tokens
        if u <= 0:
            continue
        state = p.state
        if state == "GPU" or state == "CPU":
            dev = p.device
            cu = is_cuda.get(id(dev))
            if cu is None:
                cu = is_cuda[id(dev)] = (dev.type == "cuda")
            if cu != (state == "GPU"):
                continue
        else:
            continue
        if first_active is None:
            first_active = p
        sl = p.slot
        if state == "GPU":
            if chunk and len(chunks) < 2:
                close_chunk()
            if gbound.get(sl) is p:
                kv = gviews.get(sl)
                if kv is not None and kv[0] is p.k_tensor and kv[1] is p.v_tensor:
                    run_slots.append(sl)
                    if u != p.capacity_tokens:
                        runs_meta.extend(run_slots)
                        runs_meta.append((len(run_slots) - 1) * page_size + u)
                        run_lens.append(len(run_slots))
                        run_slots = []
                    continue
            gpu_rest.append(p)
        else:
            if u == p.capacity_tokens and hbound.get(sl) is p:
                kv = hviews.get(sl)
                if kv is not None and kv[0] is p.k_tensor and kv[1] is p.v_tensor:
                    chunk.append(sl)
                    if p.ready is not None:
                        waits.append(p)
                    if len(chunk) == chunk_pages:
                        close_chunk()
                    continue
            if chunk and len(chunks) < 2:
                close_chunk()
            cpu_rest.append(p)
    if run_slots:
        # every page of an open run is full
        runs_meta.extend(run_slots)
        runs_meta.append(len(run_slots) * page_size)
        run_lens.append(len(run_slots))
    if chunk:
        close_chunk()
    return PageWalk(first_active, run_lens, np.asarray(runs_meta, dtype=np.int32),
                    [np.asarray(c, dtype=np.int32) for c in chunks], chunk_waits, gpu_rest,
                    cpu_rest)


try:   # the same walk in C (helm_amd/csrc/page_walk.c), built by helm_amd.build
    from .. import _page_walk
except ImportError:   # pragma: no cover - exercised when the module is not built
    _page_walk = None


def walk_pages(pages, gbound, gviews, hbound, hviews, chunk_pages: int, page_size: int) -> PageWalk:
    """PageWalk of `pages`: the C walk when it is built (about 30x faster than the
    Python one, whose result it equals), else walk_pages_py."""
    if _page_walk is not None:
        fa, rl, rm, cs, cw, gr, cr = _page_walk.classify(pages, gbound, gviews, hbound, hviews,
                                                         chunk_pages, page_size)
        return PageWalk(fa, rl, np.frombuffer(rm, dtype=np.int32),
                        [np.frombuffer(c, dtype=np.int32) for c in cs], cw, gr, cr)
    return walk_pages_py(pages, gbound, gviews, hbound, hviews, chunk_pages, page_size)


def perform_streaming_attention(query: torch.Tensor, pages: List[KVPage], scale: float = None,
                                allocator: Optional[KVAllocator] = None) -> torch.Tensor:
    """Decode attention of `query` [B, Hq, Sq, D] (on the GPU) over `pages` in token
    order, as helm/runtime/kv_cache.py:318-442 defines it: empty and DEAD pages are
    skipped, no active page -> zeros, GQA by repeat_interleave mapping, fp32
    online softmax; output in the query's dtype.

    Pages that are slots of `allocator`'s device pool are read in place; every
    other page (host-resident, or free-standing tensors) is staged to the device
    in chunks on a side stream while the previous chunk is attended.  The page
    list is walked once (walk_pages: in C, tens of ns per page) and the first
    two chunks of host pages are queued on the copy stream right after it.  The
    kernels' page tables and lengths go up in one upload."""
    if query.device.type != "cuda":
        raise RuntimeError("perform_streaming_attention: the query must be on the GPU "
                           "(this build has no CPU-stage attention)")
    device = query.device
    B, Hq, Sq, D = query.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    items = B * Sq
    st = _state(device)
    # pool pages share the allocator's page size; free-standing pages may be any size
    P = allocator.page_size if allocator is not None else 16
    pool = allocator.pool(device) if allocator is not None else None
    host_pool = allocator.pool(torch.device("cpu")) if allocator is not None else None
    in_place_ok = pool is not None and B == 1 and P % 16 == 0
    stage_ok = host_pool is not None and B == 1 and P % 16 == 0
    compute = torch.cuda.current_stream(device)

    def gather(c: int):
        """Queue chunk c's host pages into staging half c % 2 on the copy stream;
        returns the event that marks them landed."""
        buf = c % 2
        if st.buf_used[buf]:
            st.copy_stream.wait_event(st.buf_free[buf])   # previous reader of this half done
        ready = st.buf_ready[buf]
        for pg in walk.chunk_waits[c]:    # eviction copies into these host pages
            _wait_ready(st.copy_stream, pg)
        # one kernel reads the chunk's pages out of pinned host memory (any host
        # slot order) into consecutive staging slots, in token order
        with torch.cuda.stream(st.copy_stream):
            slots_dev = st.upload_i32(walk.chunk_slots[c])
            ka.gather_pages_h2d(host_pool.k, host_pool.v, sk, sv, slots_dev, buf * STAGE_CHUNK_PAGES,
                                st.copy_stream)
            ready.record(st.copy_stream)
        return ready

    # One pass over the page list (PageWalk: runs of in-place pool pages, chunks
    # of full host-pool pages to stage, and the rest for a dense repack, device
    # pages first, then host pages, each in list order); the first two chunks'
    # transfers are queued right after it.
    walk = walk_pages(pages, pool.bound if in_place_ok else {}, pool.views if in_place_ok else {},
                      host_pool.bound if stage_ok else {}, host_pool.views if stage_ok else {},
                      STAGE_CHUNK_PAGES, P)
    first_active = walk.first_active
    if first_active is None:
        return torch.zeros_like(query)
    n_chunks = len(walk.chunk_slots)
    sk = sv = None
    ready_evs = []
    if n_chunks:
        sk, sv = st.staging_pools(STAGE_CHUNK_PAGES, tuple(host_pool.k.shape[1:]), host_pool.dtype)
        for c in range(min(2, n_chunks)):
            ready_evs.append(gather(c))

    q = query.to(torch.float16).permute(0, 2, 1, 3).reshape(B * Sq, Hq, D).contiguous()
    Hkv = first_active.k_tensor.shape[1]
    generic = walk.gpu_rest + walk.cpu_rest

    seg_splits = [_split_count(n, Hkv, P) for n in walk.run_lens]
    chunk_splits = [_split_count(len(c), Hkv, P) for c in walk.chunk_slots]
    seg_splits.extend(chunk_splits)
    generic_tokens = sum(p.used_tokens for p in generic)
    if generic:
        seg_splits.append(_split_count((generic_tokens + 15) // 16, Hkv, 16))
    total = sum(seg_splits)
    part_o, part_ml = st.workspace.get(items, Hq, D, total)
    off = 0

    # one upload of the kernels' metadata: each run's slot row and token count,
    # then each chunk's token count (a chunk's page table is a range of staging
    # slots, kept on the device)
    meta_host = walk.run_meta
    if n_chunks:
        meta_host = np.concatenate([meta_host, np.array([len(c) * P for c in walk.chunk_slots],
                                                        dtype=np.int32)])
    meta = st.upload_i32(meta_host) if len(meta_host) else None
    mo = 0

    def launch(pool_view, page_table, seq_lens, n_split):
        nonlocal off
        page_table = page_table[None]
        if items > 1:
            page_table, seq_lens = page_table.expand(items, -1), seq_lens.expand(items)
        ka.paged_decode_attention_partial(q, pool_view, page_table, seq_lens, P, scale,
                                          part_o, part_ml, n_split, off, total)
        off += n_split

    for n, n_split in zip(walk.run_lens, seg_splits):
        launch(ka.PoolView.of_pool(pool.k, pool.v), meta[mo:mo + n], meta[mo + n:mo + n + 1], n_split)
        mo += n + 1

    for c in range(n_chunks):
        buf = c % 2
        first = buf * STAGE_CHUNK_PAGES
        ready = ready_evs[c] if c < len(ready_evs) else gather(c)
        compute.wait_event(ready)
        launch(ka.PoolView.of_pool(sk, sv), st.stage_rows[first:first + len(walk.chunk_slots[c])],
               meta[mo:mo + 1], chunk_splits[c])
        mo += 1
        st.buf_free[buf].record(compute)
        st.buf_used[buf] = True

    if generic:
        # dense repack of the remaining pages (any batch / fill pattern) into one
        # 16-token-paged buffer per batch row; query row (b, s) reads batch row b
        T = generic_tokens
        Tp = ((T + 15) // 16) * 16
        kb, vb = ka.alloc_sequences(B, Hkv, Tp, D, torch.float16, device, zero=True)
        t0 = 0
        for p in generic:
            if p.ready is not None:
                torch.cuda.current_stream(device).wait_event(p.ready)
            u = p.used_tokens
            kb[:, :, t0:t0 + u].copy_(p.k_tensor[:, :, :u].to(device, non_blocking=False))
            vb[:, :, t0:t0 + u].copy_(p.v_tensor[:, :, :u].to(device, non_blocking=False))
            t0 += u
        pages_per_item = Tp // 16
        view = ka.PoolView.of_sequences(kb, vb, 16)
        rows = torch.arange(B, dtype=torch.int32).repeat_interleave(Sq)
        pt = (rows[:, None] * pages_per_item
              + torch.arange(pages_per_item, dtype=torch.int32)[None, :]).to(device)
        sl = torch.full((items,), T, dtype=torch.int32, device=device)
        ka.paged_decode_attention_partial(q, view, pt, sl, 16, scale, part_o, part_ml,
                                          seg_splits[-1], off, total)
        off += seg_splits[-1]

    out = torch.empty(items, Hq, D, dtype=torch.float16, device=device)
    ka.paged_attn_reduce(part_o, part_ml, out, total)
    return out.view(B, Sq, Hq, D).permute(0, 2, 1, 3).to(query.dtype)
