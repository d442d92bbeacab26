"""Oracle for the KV page pool, page tables and eviction — TEST INFRASTRUCTURE ONLY.

A plain-Python restatement of the reference's bookkeeping, with pages holding
numpy arrays instead of torch tensors and devices as the strings 'cuda'/'cpu':

  KVAllocator      helm/runtime/kv_allocator.py:6-163
    _create_page :22-48   monotonic page_id, per-device page counters
    reserve_batch :50-57  append new pages to the device's free pool
    allocate :59-78       empty pool -> reserve 8 (GPU) / 16 (CPU); pop() from
                          the END (LIFO); state GPU/CPU; metadata reset
    free :80-93           state FREE, metadata reset, append to the pool
    move_page :95-144     same device -> same page; else allocate on the target,
                          copy [:, :, :used], copy metadata; GPU->CPU turns the old
                          page into a 0-element DEAD placeholder (gpu_total -= 1),
                          otherwise the old page is freed
    report_usage :146-163
  KVPage / LayerKVCache   helm/runtime/kv_cache.py:7-28
  KVCacheManager          helm/runtime/kv_cache.py:30-311 (paged part)
    append_prefill :55-85   one page per P-token chunk, start_token =
                            total_tokens, residency enforced after EVERY page
    append_decode :87-113   new page only if the tail is full; enforce unless
                            skip_residency
    evict_pages :121-159    candidates: state GPU, device cuda, not the layer's
                            tail, full; stable sort by start_token over all
                            layers (ties: layer insertion order, then page order);
                            evict until evicted bytes >= target
    _enforce_residency_policy :161-172  gpu_bytes over full non-tail GPU pages;
                            evict (gpu_bytes - watermark) only if strictly above
    all_gpu_resident :195-202, clear :183-193, seq_len :174-178,
    report_bytes_per_tier :294-311
  contiguous path           helm/runtime/kv_cache.py:206-289 (buffers of
                            `capacity` tokens per layer, halved after a failed
                            allocation while >= 1024; decode tokens written in
                            place and committed after the last layer; on overflow
                            the decode tokens are appended to pages as a prefill)
  decode_step_kv            helm/runtime/kv_offload.py:106-138 (the KV side of one
                            decode call: Path 1, migration, paged append)
  decode_batched_pages      helm/runtime/kv_offload.py:132-138 (all_gpu computed
                            BEFORE the append, then append_decode(skip_residency
                            = all_gpu) per item)

Pinning (tests/test_oracle_kv_pages.py): the reference's own unit tests
(tests/unit/runtime/test_kv_allocator.py, test_kv_cache.py, test_batch_kv_offload.py,
including the CUDA-only eviction tests test_kv_cache.py:260-295, runnable here
because devices are plain strings) are restated against this module, plus
invariants: eviction takes the globally oldest full non-tail GPU pages, tails
are never evicted, page ids are unique and monotonic, pool accounting balances.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np


def _is_cuda(device: str) -> bool:
    return device == "cuda"


@dataclass(eq=False)
class KVPage:
    page_id: int
    layer_id: int
    start_token: int
    used_tokens: int
    capacity_tokens: int
    k: np.ndarray
    v: np.ndarray
    device: str
    state: str  # FREE / GPU / CPU / DEAD


class KVAllocator:
    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, page_size: int = 64,
                 elem_bytes: int = 2, dtype=np.float16):
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.page_size = page_size
        self.elem_bytes = elem_bytes
        self.dtype = dtype
        self.gpu_free_pool: List[KVPage] = []
        self.cpu_free_pool: List[KVPage] = []
        self.gpu_total_pages = 0
        self.cpu_total_pages = 0
        self._next_page_id = 0

    def page_bytes(self) -> int:
        return 2 * self.num_kv_heads * self.page_size * self.head_dim * self.elem_bytes

    def _create_page(self, device: str) -> KVPage:
        shape = (1, self.num_kv_heads, self.page_size, self.head_dim)
        page = KVPage(self._next_page_id, -1, 0, 0, self.page_size,
                      np.zeros(shape, self.dtype), np.zeros(shape, self.dtype), device, "FREE")
        self._next_page_id += 1
        if _is_cuda(device):
            self.gpu_total_pages += 1
        else:
            self.cpu_total_pages += 1
        return page

    def reserve_batch(self, batch_size: int, device: str) -> None:
        for _ in range(batch_size):
            page = self._create_page(device)
            (self.gpu_free_pool if _is_cuda(device) else self.cpu_free_pool).append(page)

    def allocate(self, device: str) -> KVPage:
        if _is_cuda(device):
            if not self.gpu_free_pool:
                self.reserve_batch(8, device)
            page = self.gpu_free_pool.pop()
            page.state = "GPU"
        else:
            if not self.cpu_free_pool:
                self.reserve_batch(16, device)
            page = self.cpu_free_pool.pop()
            page.state = "CPU"
        page.layer_id = -1
        page.start_token = 0
        page.used_tokens = 0
        page.device = device
        return page

    def free(self, page: KVPage) -> None:
        page.state = "FREE"
        page.layer_id = -1
        page.start_token = 0
        page.used_tokens = 0
        (self.gpu_free_pool if _is_cuda(page.device) else self.cpu_free_pool).append(page)

    def move_page(self, page: KVPage, target: str) -> KVPage:
        if page.device == target:
            return page
        new = self.allocate(target)
        used = page.used_tokens
        if used > 0:
            new.k[:, :, :used, :] = page.k[:, :, :used, :]
            new.v[:, :, :used, :] = page.v[:, :, :used, :]
        new.layer_id = page.layer_id
        new.start_token = page.start_token
        new.used_tokens = used
        new.device = target
        if _is_cuda(page.device) and not _is_cuda(target):
            page.k = np.zeros(0, self.dtype)
            page.v = np.zeros(0, self.dtype)
            page.state = "DEAD"
            self.gpu_total_pages -= 1
        else:
            self.free(page)
        return new

    def report_usage(self) -> dict:
        bpp = self.page_bytes()
        gu = self.gpu_total_pages - len(self.gpu_free_pool)
        cu = self.cpu_total_pages - len(self.cpu_free_pool)
        return {
            "gpu_pool_size": self.gpu_total_pages, "cpu_pool_size": self.cpu_total_pages,
            "active_gpu_pages": gu, "active_cpu_pages": cu,
            "gpu_free_pages": len(self.gpu_free_pool), "cpu_free_pages": len(self.cpu_free_pool),
            "gpu_reserved_bytes": self.gpu_total_pages * bpp,
            "cpu_reserved_bytes": self.cpu_total_pages * bpp,
            "gpu_used_bytes": gu * bpp, "cpu_used_bytes": cu * bpp,
        }


@dataclass(eq=False)
class LayerKVCache:
    layer_id: int
    pages: List[KVPage] = field(default_factory=list)
    tail_page: Optional[KVPage] = None
    total_tokens: int = 0

    def append_page(self, page: KVPage) -> None:
        self.pages.append(page)
        self.tail_page = page


class OutOfMemory(Exception):
    """Raised by a test's allocation hook to stand for a failed device allocation."""


class KVCacheManager:
    def __init__(self, allocator: KVAllocator, gpu_high_watermark_bytes: int = 256 * 1024):
        self.allocator = allocator
        self.layers: Dict[int, LayerKVCache] = {}
        self.gpu_high_watermark_bytes = gpu_high_watermark_bytes
        # contiguous path state (kv_cache.py:43-51)
        self.cont_K: Dict[int, np.ndarray] = {}
        self.cont_V: Dict[int, np.ndarray] = {}
        self.cont_device = "cuda"
        self.cont_capacity = 0
        self.cont_num_layers = 0
        self.cont_seq_len = 0
        self.cont_prefill_len = 0
        self.use_contiguous = False

    def initialize_layer_caches(self, num_layers: int) -> None:
        for i in range(num_layers):
            self.layers[i] = LayerKVCache(i)

    def _layer(self, layer_id: int) -> LayerKVCache:
        if layer_id not in self.layers:
            self.layers[layer_id] = LayerKVCache(layer_id)
        return self.layers[layer_id]

    def append_prefill(self, layer_id: int, k: np.ndarray, v: np.ndarray, device: str) -> None:
        layer = self._layer(layer_id)
        seq = k.shape[2]
        P = self.allocator.page_size
        for s in range(0, seq, P):
            n = min(P, seq - s)
            page = self.allocator.allocate(device)
            page.layer_id = layer_id
            page.start_token = layer.total_tokens
            page.used_tokens = n
            page.k[:, :, :n, :] = k[:, :, s:s + n, :]
            page.v[:, :, :n, :] = v[:, :, s:s + n, :]
            layer.append_page(page)
            layer.total_tokens += n
            self._enforce_residency_policy()

    def append_decode(self, layer_id: int, k: np.ndarray, v: np.ndarray, device: str,
                      skip_residency: bool = False) -> None:
        layer = self._layer(layer_id)
        if layer.tail_page is None or layer.tail_page.used_tokens == layer.tail_page.capacity_tokens:
            page = self.allocator.allocate(device)
            page.layer_id = layer_id
            page.start_token = layer.total_tokens
            page.used_tokens = 0
            layer.append_page(page)
        page = layer.tail_page
        i = page.used_tokens
        page.k[:, :, i:i + 1, :] = k
        page.v[:, :, i:i + 1, :] = v
        page.used_tokens += 1
        layer.total_tokens += 1
        if not skip_residency:
            self._enforce_residency_policy()

    def iterate_layer_pages(self, layer_id: int) -> List[KVPage]:
        return list(self.layers[layer_id].pages) if layer_id in self.layers else []

    def evict_pages(self, bytes_to_evict: int) -> List[int]:
        """Returns the page_ids evicted, in eviction order."""
        if bytes_to_evict <= 0:
            return []
        cands = []
        for layer in self.layers.values():
            for page in layer.pages:
                if page.state == "GPU" and _is_cuda(page.device):
                    if page is not layer.tail_page and page.used_tokens == page.capacity_tokens:
                        cands.append((layer, page))
        cands.sort(key=lambda t: t[1].start_token)   # stable
        evicted, done = 0, []
        for layer, page in cands:
            if evicted >= bytes_to_evict:
                break
            new = self.allocator.move_page(page, "cpu")
            idx = layer.pages.index(page)
            layer.pages[idx] = new
            if layer.tail_page is page:
                layer.tail_page = new
            done.append(page.page_id)
            evicted += self.allocator.page_bytes()
        return done

    def gpu_evictable_bytes(self) -> int:
        b = 0
        for layer in self.layers.values():
            for page in layer.pages:
                if page.state == "GPU" and _is_cuda(page.device):
                    if page is not layer.tail_page and page.used_tokens == page.capacity_tokens:
                        b += self.allocator.page_bytes()
        return b

    def _enforce_residency_policy(self) -> None:
        gb = self.gpu_evictable_bytes()
        if gb > self.gpu_high_watermark_bytes:
            self.evict_pages(gb - self.gpu_high_watermark_bytes)

    def seq_len(self) -> int:
        return self.layers[0].total_tokens if 0 in self.layers else 0

    def num_layers(self) -> int:
        return len(self.layers)

    def clear(self) -> None:
        for layer in self.layers.values():
            for page in layer.pages:
                if page.state != "DEAD":
                    self.allocator.free(page)
            layer.pages.clear()
            layer.tail_page = None
            layer.total_tokens = 0
        self.layers.clear()

    def all_gpu_resident(self, layer_id: int) -> bool:
        if layer_id not in self.layers:
            return True
        return all(not (p.used_tokens > 0 and p.state != "GPU") for p in self.layers[layer_id].pages)

    def report_bytes_per_tier(self) -> dict:
        g = c = 0
        for layer in self.layers.values():
            for page in layer.pages:
                if page.state == "DEAD":
                    continue
                if page.state == "GPU":
                    g += self.allocator.page_bytes()
                elif page.state == "CPU":
                    c += self.allocator.page_bytes()
        return {"gpu_active_bytes": g, "cpu_active_bytes": c}

    # ── contiguous path (kv_cache.py:206-289) ──
    def build_contiguous(self, num_layers, num_kv_heads, head_dim, capacity, device="cuda",
                         alloc=None):
        # :206-234: try `capacity`, halve after a failed allocation while >= 1024
        alloc = alloc or (lambda shape: np.zeros(shape, self.allocator.dtype))
        cap = capacity
        while cap >= 1024:
            try:
                self.cont_K, self.cont_V = {}, {}
                for lid in range(num_layers):
                    self.cont_K[lid] = alloc((1, num_kv_heads, cap, head_dim))
                    self.cont_V[lid] = alloc((1, num_kv_heads, cap, head_dim))
                self.cont_capacity, self.cont_num_layers = cap, num_layers
                self.cont_device = device
                self.use_contiguous = True
                return True
            except OutOfMemory:
                self.cont_K, self.cont_V = {}, {}
                cap //= 2
        self.use_contiguous = False
        return False

    def prefill_contiguous(self, layer_id, k, v):          # :236-243
        n = k.shape[2]
        self.cont_K[layer_id][:, :, :n] = k
        self.cont_V[layer_id][:, :, :n] = v
        if layer_id == 0:
            self.cont_prefill_len = self.cont_seq_len = n

    def write_decode_contiguous(self, layer_id, k, v):     # :245-249
        i = self.cont_seq_len
        self.cont_K[layer_id][:, :, i:i + 1] = k
        self.cont_V[layer_id][:, :, i:i + 1] = v

    def get_kv_contiguous(self, layer_id):                 # :251-254
        n = self.cont_seq_len + 1
        return self.cont_K[layer_id][:, :, :n], self.cont_V[layer_id][:, :, :n]

    def advance_contiguous(self):                          # :256-258
        self.cont_seq_len += 1

    def migrate_contiguous_to_pages(self):                 # :260-276
        if not self.cont_K:
            return
        a, b = self.cont_prefill_len, self.cont_seq_len
        if b > a:
            for lid in range(self.cont_num_layers):
                self.append_prefill(lid, self.cont_K[lid][:, :, a:b].copy(),
                                    self.cont_V[lid][:, :, a:b].copy(), self.cont_device)
        self.drop_contiguous()

    def drop_contiguous(self):                             # :278-282
        self.cont_K, self.cont_V = {}, {}
        self.use_contiguous = False

    def reset_contiguous(self):                            # :284-289
        if self.cont_K:
            self.use_contiguous = True
            self.cont_seq_len = self.cont_prefill_len = 0


def decode_step_kv(kvcms: List[KVCacheManager], layer_idx: int, k_list, v_list,
                   device: str) -> str:
    """The KV side of one _decode_batched call (kv_offload.py:106-138), attention
    left out: Path 1 writes into the contiguous buffers (and commits the token
    after the last layer); on overflow every item migrates and the paged append
    follows.  Returns the path taken: "contiguous", "paged_gpu" or "streaming"
    (Path 2 is taken when every item's layer was GPU-resident before the append
    and all items have the same token count, :141-160)."""
    if kvcms[0].use_contiguous:
        if kvcms[0].cont_seq_len < kvcms[0].cont_capacity:
            for i, kvcm in enumerate(kvcms):
                kvcm.write_decode_contiguous(layer_idx, k_list[i], v_list[i])
            if layer_idx == kvcms[0].cont_num_layers - 1:
                for kvcm in kvcms:
                    kvcm.advance_contiguous()
            return "contiguous"
        for kvcm in kvcms:
            kvcm.migrate_contiguous_to_pages()
    all_gpu = all(kvcm.all_gpu_resident(layer_idx) for kvcm in kvcms)
    for i, kvcm in enumerate(kvcms):
        kvcm.append_decode(layer_idx, k_list[i], v_list[i], device, skip_residency=all_gpu)
    lens = {sum(p.used_tokens for p in kvcm.iterate_layer_pages(layer_idx)) for kvcm in kvcms}
    return "paged_gpu" if all_gpu and len(lens) == 1 else "streaming"


def layer_tokens(kvcm: KVCacheManager, layer_idx: int):
    """(K, V) [1, Hkv, T, D] of a layer: its pages' used tokens concatenated in list
    order, as Path 2 / perform_streaming_attention read them (kv_offload.py:145-146)."""
    pages = [p for p in kvcm.iterate_layer_pages(layer_idx) if p.used_tokens > 0]
    return (np.concatenate([p.k[:, :, :p.used_tokens] for p in pages], axis=2),
            np.concatenate([p.v[:, :, :p.used_tokens] for p in pages], axis=2))


def decode_batched_pages(kvcms: List[KVCacheManager], layer_idx: int, k_list, v_list,
                         device: str) -> List[List[KVPage]]:
    """Paged part of _decode_batched (kv_offload.py:132-138): all_gpu over every
    item BEFORE the append, append_decode(skip_residency=all_gpu) per item, then
    each item's page list."""
    all_gpu = all(kvcm.all_gpu_resident(layer_idx) for kvcm in kvcms)
    pages = []
    for i, kvcm in enumerate(kvcms):
        kvcm.append_decode(layer_idx, k_list[i], v_list[i], device, skip_residency=all_gpu)
        pages.append(kvcm.iterate_layer_pages(layer_idx))
    return pages


def snapshot(kvcm: KVCacheManager) -> list:
    """Bit-exact view of the page tables: per layer (in dict order) the list of
    (page_id, state, device, start_token, used_tokens) plus tail and total."""
    out = []
    for lid, layer in kvcm.layers.items():
        out.append((lid, [(p.page_id, p.state, p.device, p.start_token, p.used_tokens)
                          for p in layer.pages],
                    None if layer.tail_page is None else layer.tail_page.page_id,
                    layer.total_tokens))
    return out
