"""Device page tables for the paged attention kernel, kept in step with the
KVCacheManagers' page lists.

The reference has no device page table: every decode step it concatenates the
pages of a layer with torch.cat (helm/runtime/kv_offload.py:141-160,
kv_cache.py:367-371).  Here each (layer, sequence) has an int32 row of slot
indices on the device that the kernel indexes directly; a row entry is the
page's device slot, or -1 for a host-resident page.  The host edits a numpy
mirror and `flush()` uploads only the dirty index ranges.

Uploads go through PinnedRing: the bytes are snapshotted into a pinned staging
region and copied with non_blocking H2D on the current stream; the ring is
reused from its start only after every copy of the previous lap completed — so
the host can keep editing its mirror while earlier copies are still queued
behind kernels.
"""
from __future__ import annotations

from collections import deque
from typing import Dict, Tuple

import numpy as np
import torch


class PinnedRing:
    """Ring of pinned host memory for asynchronous small H2D uploads."""

    ALIGN = 256

    def __init__(self, nbytes: int = 1 << 22):
        self.cap = nbytes
        self.buf = torch.empty(nbytes, dtype=torch.uint8, pin_memory=torch.cuda.is_available())
        self.np = self.buf.numpy()
        self.pos = 0
        self.pending: deque = deque()   # (start, end, event) in allocation order

    def _reserve(self, n: int) -> int:
        n = (n + self.ALIGN - 1) // self.ALIGN * self.ALIGN
        if n > self.cap:
            raise RuntimeError(f"PinnedRing: upload of {n} bytes exceeds ring size {self.cap}")
        if self.pos + n <= self.cap:
            start = self.pos
        else:
            # A new lap rewrites bytes of earlier laps: every copy still queued from
            # them is waited for (one host wait per `cap` bytes of uploads).  Within
            # a lap regions are handed out at increasing positions, so no region of
            # the lap itself is ever overwritten.
            start = 0
            while self.pending:
                self.pending.popleft()[2].synchronize()
        # completed copies leave the queue from the front (one query per upload)
        while self.pending and self.pending[0][2].query():
            self.pending.popleft()
        self.pos = start + n
        return start

    def upload(self, src: np.ndarray, dst: torch.Tensor) -> None:
        """dst (a contiguous device tensor) <- src (same number of bytes), async."""
        src = np.ascontiguousarray(src)
        n = src.nbytes
        start = self._reserve(n)
        self.np[start:start + n] = src.view(np.uint8).reshape(-1)
        stage = self.buf[start:start + n].view(dst.dtype).view(dst.shape)
        dst.copy_(stage, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self.pending.append((start, start + ((n + self.ALIGN - 1) // self.ALIGN) * self.ALIGN, ev))

    def sync(self) -> None:
        while self.pending:
            self.pending.popleft()[2].synchronize()


class DevicePageTable:
    """int32 [num_layers, batch, capacity] page-slot table on the device (+ mirror)."""

    def __init__(self, num_layers: int, batch: int, capacity_pages: int, device: torch.device,
                 ring: PinnedRing = None):
        self.L, self.B = num_layers, batch
        self.cap = max(1, capacity_pages)
        self.device = torch.device(device)
        self.host = np.full((self.L, self.B, self.cap), -1, np.int32)
        self.dev = torch.full((self.L, self.B, self.cap), -1, dtype=torch.int32, device=self.device)
        self.ring = ring or PinnedRing()
        self.dirty: Dict[Tuple[int, int], list] = {}
        self.generation = 0   # bumps when `dev` is reallocated

    def _grow(self, need: int) -> None:
        cap = self.cap
        while cap < need:
            cap *= 2
        host = np.full((self.L, self.B, cap), -1, np.int32)
        host[:, :, : self.cap] = self.host
        dev = torch.full((self.L, self.B, cap), -1, dtype=torch.int32, device=self.device)
        dev[:, :, : self.cap].copy_(self.dev)
        self.host, self.dev, self.cap = host, dev, cap
        self.generation += 1

    def set(self, layer: int, item: int, idx: int, page) -> None:
        if layer >= self.L:
            raise IndexError(f"DevicePageTable: layer {layer} >= {self.L}")
        if idx >= self.cap:
            self._grow(idx + 1)
        self.host[layer, item, idx] = page.slot if (page.state == "GPU" and page.slot >= 0) else -1
        r = self.dirty.get((layer, item))
        if r is None:
            self.dirty[(layer, item)] = [idx, idx + 1]
        else:
            r[0] = min(r[0], idx)
            r[1] = max(r[1], idx + 1)

    def clear_item(self, item: int) -> None:
        self.host[:, item, :] = -1
        for layer in range(self.L):
            self.dirty[(layer, item)] = [0, self.cap]

    def flush(self) -> None:
        """Upload every dirty range on the current stream."""
        for (layer, item), (lo, hi) in self.dirty.items():
            self.ring.upload(self.host[layer, item, lo:hi], self.dev[layer, item, lo:hi])
        self.dirty.clear()

    def rows(self, layer: int) -> torch.Tensor:
        """Device table of `layer`: [batch, capacity] int32 (row stride = capacity)."""
        return self.dev[layer]
