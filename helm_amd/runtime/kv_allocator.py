"""KV page pool (mirror of helm/runtime/kv_allocator.py) backed by slot pools.

Logical behaviour is the reference's, line for line in effect:
  * ``_create_page`` hands out monotonically increasing ``page_id``s and counts
    pages per device tier (kv_allocator.py:22-48);
  * ``allocate`` reserves 8 (GPU) / 16 (CPU) new pages when the tier's free pool
    is empty and pops from the END of the pool (LIFO) (:59-78);
  * ``free`` resets metadata and appends to the pool (:80-93);
  * ``move_page`` copies ``[:, :, :used]`` synchronously (or, with
    ``async_eviction``, a GPU->CPU move copies on a side stream, see below); a GPU->CPU move turns
    the old page into a 0-element ``DEAD`` placeholder and decrements
    ``gpu_total_pages``, any other move frees the old page (:95-144);
  * ``report_usage`` (:146-163).

Physical storage is MI355X-first: instead of two small tensors per page, every
GPU page is a slot of one device pool (so the paged attention kernel addresses
any page as ``pool + slot * slot_stride``), and every CPU page a slot of one
pinned host pool of the same layout (so a page moves by one DMA per K/V).  K is
stored ``[slots, Hkv, P, D]``; V token-contiguous per dim, ``[slots, Hkv, D, P]``
(the attention kernel feeds 8 consecutive tokens of one dim to the matrix cores
with one 16-byte load), and exposed as its transposed view.  A page's
``k_tensor``/``v_tensor`` are the slot views ``k[slot:slot+1]``,
``v[slot:slot+1]`` — the reference's ``(1, Hkv, P, D)`` page tensors (V with
transposed strides).  A DEAD page returns its device slot to the pool.  Pools grow by doubling (views are rebound; all GPU
work is waited for first, since in-flight eviction copies and kernels may still
use the old storage); callers that capture device pointers (graph replay) size
them up front with ``gpu_capacity_pages``.

Asynchronous eviction (``async_eviction=True``): a GPU->CPU move issues its
copy on a side stream, ordered after the work already queued on the current
stream, and returns at once.  The page bookkeeping is the same as the
synchronous move; the bytes are guarded instead: the host page carries the
copy's event in ``ready`` (every reader of host pages waits for it on its own
stream), and the freed device slot joins the free list only when that event has
completed.  Host code that reads host page tensors directly calls
``synchronize()`` first.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional

import math

import torch


@dataclass
class KVPage:
    """Page record (helm/runtime/kv_cache.py:7-17) plus its physical slot."""
    page_id: int
    layer_id: int
    start_token: int
    used_tokens: int
    capacity_tokens: int
    k_tensor: torch.Tensor
    v_tensor: torch.Tensor
    device: torch.device
    state: str  # 'FREE', 'GPU', 'CPU', 'DEAD'
    slot: int = field(default=-1, compare=False)
    # set on a host page whose eviction copy is still in flight (asynchronous
    # eviction): readers wait for it on their stream before touching the bytes
    ready: Optional[object] = field(default=None, compare=False, repr=False)


def _is_cuda(device: torch.device) -> bool:
    return torch.device(device).type == "cuda"


class PagePool:
    """Slot storage of one tier: ``k`` ``[capacity, Hkv, P, D]`` and ``v`` (a
    ``[capacity, Hkv, P, D]`` view of ``[capacity, Hkv, D, P]`` storage)."""

    def __init__(self, num_kv_heads: int, page_size: int, head_dim: int, dtype: torch.dtype,
                 device: torch.device, capacity: int, pinned: bool, scatter: bool = False):
        self.shape = (num_kv_heads, page_size, head_dim)
        self.dtype = dtype
        self.device = torch.device(device)
        self.pinned = pinned
        self.capacity = 0
        self.k = self._alloc(0)
        self.v = self._alloc(0, transposed=True)
        self.free_slots: List[int] = []
        self.pending: List[tuple] = []       # (slot, event): released once the event completes
        self.next_slot = 0
        self.bound: Dict[int, KVPage] = {}   # slot -> page holding views of it
        self.views: Dict[int, tuple] = {}    # slot -> the (k, v) views handed to it
        self.generation = 0                  # bumps when the storage moves
        # called before the storage moves: work still in flight on any stream
        # (eviction copies into a host pool, kernels reading either pool) must
        # finish before the old buffers are copied and released
        self.before_resize = None
        self._resize(max(1, capacity))
        # Scattered slot order (fixed-capacity pools only): the n-th new slot is
        # n * mul mod capacity with gcd(mul, capacity) = 1, a bijection that spreads
        # consecutive pages of a layer over the pool instead of one contiguous run
        # (contiguous runs read in lockstep by the attention splits concentrate on
        # the same HBM channels; measured ~1 us slower per 16K-context layer).
        self.scatter = bool(scatter)
        self._mul = 1
        if self.scatter:
            m = max(1, int(self.capacity * 0.6180339887)) | 1
            while math.gcd(m, self.capacity) != 1:
                m += 2
            self._mul = m

    def _alloc(self, n: int, transposed: bool = False) -> torch.Tensor:
        hkv, p, d = self.shape
        shape = (n, hkv, d, p) if transposed else (n, hkv, p, d)
        if self.device.type == "cpu" and self.pinned:
            t = torch.empty(shape, dtype=self.dtype, pin_memory=True)
        elif self.device.type == "cuda" and not torch.cuda.is_available():
            # No GPU in this process: the GPU tier's bytes live in host memory so the
            # page bookkeeping (ids, states, eviction order) can be exercised; every
            # kernel entry point rejects these CPU tensors.
            t = torch.empty(shape, dtype=self.dtype)
        else:
            t = torch.empty(shape, dtype=self.dtype, device=self.device)
        return t.transpose(2, 3) if transposed else t

    @property
    def v_store(self) -> torch.Tensor:
        """V storage ``[capacity, Hkv, D, P]``."""
        return self.v.transpose(2, 3)

    def _resize(self, capacity: int) -> None:
        if self.capacity and self.before_resize is not None:
            self.before_resize()
        k, v = self._alloc(capacity), self._alloc(capacity, transposed=True)
        if self.capacity:
            k[: self.capacity].copy_(self.k)
            v.transpose(2, 3)[: self.capacity].copy_(self.v_store)
        self.k, self.v, self.capacity = k, v, capacity
        self.generation += 1
        for slot, page in self.bound.items():
            self._bind(page, slot)

    def _reap(self, wait: bool = False) -> None:
        """Return slots whose pending copies finished (the oldest one waited for
        when `wait`) to the free list, in release order."""
        while self.pending:
            slot, ev = self.pending[0]
            if not ev.query():
                if not wait:
                    break
                ev.synchronize()
                wait = False
            self.pending.pop(0)
            self.free_slots.append(slot)

    def acquire(self, page: KVPage) -> int:
        if self.pending:
            self._reap(wait=not self.free_slots and self.next_slot >= self.capacity)
        if self.free_slots:
            slot = self.free_slots.pop()
        else:
            if self.next_slot >= self.capacity:
                if self.scatter:
                    raise RuntimeError(f"page pool on {self.device} is full ({self.capacity} slots; "
                                       "a scattered pool has a fixed capacity)")
                self._resize(self.capacity * 2)
            slot = (self.next_slot * self._mul) % self.capacity if self.scatter else self.next_slot
            self.next_slot += 1
        self.bound[slot] = page
        self._bind(page, slot)
        return slot

    def _bind(self, page: KVPage, slot: int) -> None:
        page.slot = slot
        page.k_tensor = self.k[slot:slot + 1]
        page.v_tensor = self.v[slot:slot + 1]
        self.views[slot] = (page.k_tensor, page.v_tensor)

    def owns(self, page: KVPage) -> bool:
        """True when `page`'s tensors are still this pool's slot views (identity of
        the view objects handed out at binding; no tensor calls, so a per-page
        check over long page lists stays cheap)."""
        s = page.slot
        if self.bound.get(s) is not page:
            return False
        kv = self.views.get(s)
        return kv is not None and kv[0] is page.k_tensor and kv[1] is page.v_tensor

    def release(self, page: KVPage, after=None) -> None:
        """Return the page's slot; with `after` (an event) only once it completed."""
        self.bound.pop(page.slot, None)
        self.views.pop(page.slot, None)
        if after is None:
            self.free_slots.append(page.slot)
        else:
            self.pending.append((page.slot, after))
        page.slot = -1

    def synchronize(self) -> None:
        for _, ev in self.pending:
            ev.synchronize()
        self._reap()

    @property
    def slots_in_use(self) -> int:
        return self.next_slot - len(self.free_slots) - len(self.pending)


class KVAllocator:
    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, page_size: int = 64,
                 dtype: torch.dtype = torch.bfloat16, gpu_capacity_pages: Optional[int] = None,
                 cpu_capacity_pages: Optional[int] = None, pin_host: bool = True,
                 async_eviction: bool = False, scatter_slots: bool = False):
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.page_size = page_size
        self.dtype = dtype

        self.gpu_free_pool: List[KVPage] = []
        self.cpu_free_pool: List[KVPage] = []
        self.gpu_total_pages = 0
        self.cpu_total_pages = 0
        self._next_page_id = 0

        self._gpu_capacity = gpu_capacity_pages or 1024
        self._cpu_capacity = cpu_capacity_pages or 1024
        self._pin_host = pin_host
        self._pools: Dict[tuple, PagePool] = {}
        # GPU -> host moves copy on a side stream instead of blocking the host
        self.async_eviction = bool(async_eviction) and torch.cuda.is_available()
        self._evict_streams: Dict[int, "torch.cuda.Stream"] = {}
        # device pool: fixed capacity, slots handed out in a scattered order
        self._scatter_slots = bool(scatter_slots)
        self._devices: Dict[tuple, torch.device] = {}

    # ── physical pools ──────────────────────────────────────────────────────
    def pool(self, device: torch.device) -> PagePool:
        """The slot pool of `device` (created on first use)."""
        device = torch.device(device)
        if device.type == "cuda" and device.index is None:
            device = torch.device("cuda", torch.cuda.current_device() if torch.cuda.is_available() else 0)
        key = (device.type, device.index)
        p = self._pools.get(key)
        if p is None:
            cuda = device.type == "cuda"
            pinned = (not cuda) and self._pin_host and torch.cuda.is_available()
            p = PagePool(self.num_kv_heads, self.page_size, self.head_dim, self.dtype, device,
                         self._gpu_capacity if cuda else self._cpu_capacity, pinned,
                         scatter=cuda and self._scatter_slots)
            p.before_resize = self._quiesce
            self._pools[key] = p
        return p

    def page_bytes(self) -> int:
        """Bytes of one page's K+V tensors (the unit of the watermark accounting)."""
        return 2 * self.num_kv_heads * self.page_size * self.head_dim * \
            torch.tensor([], dtype=self.dtype).element_size()

    def _intern(self, device) -> torch.device:
        """One torch.device object per distinct device value, so that pages share
        their device object (equal to what the caller asked for) and per-page
        residency checks can key on it."""
        device = torch.device(device)
        key = (device.type, device.index)
        d = self._devices.get(key)
        if d is None:
            d = self._devices[key] = device
        return d

    # ── reference API ───────────────────────────────────────────────────────
    def _create_page(self, device: torch.device) -> KVPage:
        device = self._intern(device)
        page = KVPage(page_id=self._next_page_id, layer_id=-1, start_token=0, used_tokens=0,
                      capacity_tokens=self.page_size, k_tensor=None, v_tensor=None,
                      device=device, state="FREE")
        self.pool(device).acquire(page)
        self._next_page_id += 1
        if device.type == "cuda":
            self.gpu_total_pages += 1
        else:
            self.cpu_total_pages += 1
        return page

    def reserve_batch(self, batch_size: int, device: torch.device) -> None:
        """Allocate a batch of free pages on the specified device."""
        for _ in range(batch_size):
            page = self._create_page(device)
            if _is_cuda(device):
                self.gpu_free_pool.append(page)
            else:
                self.cpu_free_pool.append(page)

    def allocate(self, device: torch.device) -> KVPage:
        """Get a free page from the pool, allocating if necessary."""
        device = self._intern(device)
        if device.type == "cuda":
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
        page.ready = None
        return page

    def free(self, page: KVPage) -> None:
        """Recycle a page back to the free pool (tensors are not cleared)."""
        page.state = "FREE"
        page.layer_id = -1
        page.start_token = 0
        page.used_tokens = 0
        if page.device.type == "cuda":
            self.gpu_free_pool.append(page)
        else:
            self.cpu_free_pool.append(page)

    def move_page(self, page: KVPage, target_device: torch.device) -> KVPage:
        """Move a page between CPU and GPU: allocate on the target, copy the valid
        tokens synchronously, recycle (or kill) the old page, return the new one."""
        target_device = torch.device(target_device)
        if page.device == target_device:
            return page
        new_page = self.allocate(target_device)
        used = page.used_tokens
        done = None
        src_pool, dst_pool = self.pool(page.device), self.pool(target_device)
        if page.ready is not None:   # a host page whose eviction copy may still run
            torch.cuda.current_stream().wait_event(page.ready)
        if (used > 0 and self.async_eviction and page.device.type == "cuda"
                and target_device.type != "cuda" and src_pool.owns(page) and dst_pool.owns(new_page)):
            # asynchronous eviction: the copy runs on a side stream after the work
            # already queued on the current stream; the device slot is recycled
            # only once the copy completed, and readers of the host page wait for
            # `new_page.ready`
            st = self._evict_stream(page.device)
            st.wait_stream(torch.cuda.current_stream(page.device))
            with torch.cuda.stream(st):
                dst_pool.k[new_page.slot].copy_(src_pool.k[page.slot], non_blocking=True)
                dst_pool.v_store[new_page.slot].copy_(src_pool.v_store[page.slot], non_blocking=True)
            done = torch.cuda.Event()
            done.record(st)
            new_page.ready = done
        elif used > 0:
            # synchronous: the old slot may be reused by the very next allocation
            if src_pool.owns(page) and dst_pool.owns(new_page):
                # whole slots (same layout on both tiers): one contiguous copy per K/V
                dst_pool.k[new_page.slot].copy_(src_pool.k[page.slot])
                dst_pool.v_store[new_page.slot].copy_(src_pool.v_store[page.slot])
            else:
                new_page.k_tensor[:, :, :used, :].copy_(page.k_tensor[:, :, :used, :])
                new_page.v_tensor[:, :, :used, :].copy_(page.v_tensor[:, :, :used, :])
        new_page.layer_id = page.layer_id
        new_page.start_token = page.start_token
        new_page.used_tokens = used
        new_page.device = self._intern(target_device)
        if page.device.type == "cuda" and target_device.type != "cuda":
            # GPU -> CPU eviction: the device slot goes back to the pool; the page
            # object stays as a 0-element placeholder so stale references fail loudly.
            self.pool(page.device).release(page, after=done)
            page.k_tensor = torch.empty(0, dtype=self.dtype)
            page.v_tensor = torch.empty(0, dtype=self.dtype)
            page.state = "DEAD"
            self.gpu_total_pages -= 1
        else:
            self.free(page)
        return new_page

    def _evict_stream(self, device: torch.device):
        idx = device.index if device.index is not None else torch.cuda.current_device()
        st = self._evict_streams.get(idx)
        if st is None:
            st = self._evict_streams[idx] = torch.cuda.Stream(device=idx)   # default priority
        return st

    def _quiesce(self) -> None:
        """Before a pool's storage moves: wait for all GPU work that may still read
        or write either tier's buffers (eviction copies on the side streams write
        into the host pool and read the device pool; attention and staging
        kernels read both), so the old storage is complete when it is copied and
        unused when it is released.  Pools grow by doubling, so this runs a
        logarithmic number of times."""
        if not torch.cuda.is_available():
            return
        for key in self._pools:
            if key[0] == "cuda":
                torch.cuda.synchronize(torch.device("cuda", key[1]))
        for st in self._evict_streams.values():
            st.synchronize()

    def synchronize(self) -> None:
        """Wait for every in-flight eviction copy (before reading host pages on the
        host) and recycle the device slots they held."""
        for p in self._pools.values():
            p.synchronize()

    def report_usage(self) -> dict:
        bytes_per_page = self.page_bytes()
        gpu_used_pages = self.gpu_total_pages - len(self.gpu_free_pool)
        cpu_used_pages = self.cpu_total_pages - len(self.cpu_free_pool)
        return {
            "gpu_pool_size": self.gpu_total_pages,
            "cpu_pool_size": self.cpu_total_pages,
            "active_gpu_pages": gpu_used_pages,
            "active_cpu_pages": cpu_used_pages,
            "gpu_free_pages": len(self.gpu_free_pool),
            "cpu_free_pages": len(self.cpu_free_pool),
            "gpu_reserved_bytes": self.gpu_total_pages * bytes_per_page,
            "cpu_reserved_bytes": self.cpu_total_pages * bytes_per_page,
            "gpu_used_bytes": gpu_used_pages * bytes_per_page,
            "cpu_used_bytes": cpu_used_pages * bytes_per_page,
        }
