"""Pins the KV-page oracle (oracle/kv_pages.py) to the reference's own unit tests.

Restates tests/unit/runtime/test_kv_allocator.py, test_kv_cache.py and
test_batch_kv_offload.py of the reference against the oracle, including the
CUDA-only eviction tests (test_kv_cache.py:260-295), which run here because the
oracle's devices are plain strings; plus invariants of the eviction order.
"""
import numpy as np
import pytest

from oracle import kv_pages as ok

CPU, GPU = "cpu", "cuda"


def alloc(**kw):
    d = dict(num_layers=2, num_kv_heads=2, head_dim=8, page_size=4, elem_bytes=4, dtype=np.float32)
    d.update(kw)
    return ok.KVAllocator(**d)


def kv(n, h=2, d=8, seed=0):
    g = np.random.default_rng(seed)
    return (g.standard_normal((1, h, n, d)).astype(np.float32),
            g.standard_normal((1, h, n, d)).astype(np.float32))


# ── test_kv_allocator.py ─────────────────────────────────────────────────────
def test_allocate_cpu_state():                       # :28-32
    p = alloc().allocate(CPU)
    assert p.state == "CPU" and p.device == CPU


def test_allocate_resets_metadata():                 # :35-45
    a = alloc()
    p = a.allocate(CPU)
    p.layer_id, p.start_token, p.used_tokens = 99, 500, 3
    a.free(p)
    p2 = a.allocate(CPU)
    assert (p2.layer_id, p2.start_token, p2.used_tokens) == (-1, 0, 0)


def test_allocate_triggers_batch_reserve():          # :48-53
    a = alloc()
    a.allocate(CPU)
    assert a.cpu_total_pages == 16
    a.allocate(GPU)
    assert a.gpu_total_pages == 8


def test_page_ids_unique_and_lifo():                 # :69-74, :95-100
    a = alloc()
    p0, p1 = a.allocate(CPU), a.allocate(CPU)
    assert (p0.page_id, p1.page_id) == (15, 14)      # pop() from the end of 0..15
    a.free(p1)
    assert a.allocate(CPU) is p1


def test_reserve_batch_accumulates():                # :107-118
    a = alloc()
    a.reserve_batch(3, CPU)
    a.reserve_batch(4, CPU)
    assert a.cpu_total_pages == 7 and len(a.cpu_free_pool) == 7


def test_move_page_same_device_returns_same():       # :125-141
    a = alloc()
    p = a.allocate(CPU)
    p.used_tokens = 2
    p.k[:, :, :2] = 42.0
    assert a.move_page(p, CPU) is p


def test_move_page_cpu_to_gpu_copies_data():         # :183-200
    a = alloc()
    p = a.allocate(CPU)
    p.layer_id, p.start_token, p.used_tokens = 2, 8, 3
    p.k[:, :, :3] = 7.0
    p.v[:, :, :3] = 8.0
    cpu_free = len(a.cpu_free_pool)
    n = a.move_page(p, GPU)
    assert (n.device, n.layer_id, n.start_token, n.used_tokens) == (GPU, 2, 8, 3)
    assert (n.k[:, :, :3] == 7.0).all() and (n.v[:, :, :3] == 8.0).all()
    assert len(a.cpu_free_pool) == cpu_free + 1      # :203-209 old page freed


def test_move_gpu_to_cpu_kills_old_page():           # kv_allocator.py:135-140
    a = alloc()
    p = a.allocate(GPU)
    p.used_tokens = 4
    total = a.gpu_total_pages
    n = a.move_page(p, CPU)
    assert p.state == "DEAD" and p.k.size == 0 and a.gpu_total_pages == total - 1
    assert n.state == "CPU"


def test_report_usage_keys_and_counts():             # :148-168
    a = alloc()
    a.allocate(CPU)
    r = a.report_usage()
    assert r["active_cpu_pages"] == 1 and r["cpu_used_bytes"] <= r["cpu_reserved_bytes"]
    assert set(r) == {"gpu_pool_size", "cpu_pool_size", "active_gpu_pages", "active_cpu_pages",
                      "gpu_free_pages", "cpu_free_pages", "gpu_reserved_bytes",
                      "cpu_reserved_bytes", "gpu_used_bytes", "cpu_used_bytes"}


# ── test_kv_cache.py ─────────────────────────────────────────────────────────
@pytest.fixture()
def cache():
    a = ok.KVAllocator(4, 2, 8, 4, 4, np.float32)
    m = ok.KVCacheManager(a, gpu_high_watermark_bytes=0)
    m.initialize_layer_caches(4)
    return m


def test_prefill_page_counts(cache):                 # :85-103
    cache.append_prefill(0, *kv(3), CPU)
    assert len(cache.layers[0].pages) == 1 and cache.layers[0].total_tokens == 3
    cache.append_prefill(1, *kv(9), CPU)
    assert len(cache.layers[1].pages) == 3 and cache.layers[1].total_tokens == 9


def test_prefill_start_tokens_and_data(cache):       # :106-118
    k, v = kv(8)
    cache.append_prefill(0, k, v, CPU)
    assert [p.start_token for p in cache.layers[0].pages] == [0, 4]
    assert np.array_equal(cache.layers[0].pages[1].k[:, :, :4], k[:, :, 4:8])


def test_decode_paths(cache):                        # :133-168
    cache.append_prefill(0, *kv(2), CPU)
    cache.append_decode(0, *kv(1), CPU)
    assert len(cache.layers[0].pages) == 1 and cache.layers[0].tail_page.used_tokens == 3
    cache.append_prefill(1, *kv(4), CPU)
    cache.append_decode(1, *kv(1), CPU)
    assert len(cache.layers[1].pages) == 2 and cache.layers[1].tail_page.used_tokens == 1
    for _ in range(6):
        cache.append_decode(2, *kv(1), CPU)
    assert len(cache.layers[2].pages) == 2 and cache.layers[2].total_tokens == 6


def test_iterate_and_seq_len(cache):                 # :175-195
    cache.append_prefill(0, *kv(5), CPU)
    assert len(cache.iterate_layer_pages(0)) == 2 and cache.iterate_layer_pages(99) == []
    assert cache.seq_len() == 5
    del cache.layers[0]
    assert cache.seq_len() == 0


def test_clear_returns_pages(cache):                 # :221-235
    cache.append_prefill(0, *kv(4), CPU)
    before = len(cache.allocator.cpu_free_pool)
    cache.clear()
    assert cache.num_layers() == 0 and len(cache.allocator.cpu_free_pool) > before


def test_evict_gpu_pages_to_cpu():                   # :260-275 (CUDA-only in the reference)
    a = ok.KVAllocator(2, 2, 8, 4, 4, np.float32)
    m = ok.KVCacheManager(a, gpu_high_watermark_bytes=0)
    m.initialize_layer_caches(2)
    m.append_prefill(0, *kv(8), GPU)
    m.evict_pages(999999)
    for p in m.layers[0].pages[:-1]:
        assert p.state in ("CPU", "FREE")


def test_tail_page_protected():                      # :278-295
    a = ok.KVAllocator(2, 2, 8, 4, 4, np.float32)
    m = ok.KVCacheManager(a, gpu_high_watermark_bytes=0)
    m.initialize_layer_caches(2)
    m.append_prefill(0, *kv(4), GPU)
    tail = m.layers[0].tail_page
    m.evict_pages(999999)
    assert m.layers[0].tail_page is tail and tail.state == "GPU"


# ── test_batch_kv_offload.py ─────────────────────────────────────────────────
def test_batch_independence_and_reset():             # :53-160
    a = ok.KVAllocator(4, 2, 16, 8, 4, np.float32)
    ms = [ok.KVCacheManager(a, 0) for _ in range(3)]
    ms[0].append_prefill(0, *kv(4, d=16), CPU)
    assert 0 in ms[0].layers and 0 not in ms[1].layers
    ms[1].append_prefill(0, *kv(8, d=16), CPU)
    ms[1].append_decode(0, *kv(1, d=16), CPU)
    assert (ms[0].layers[0].total_tokens, ms[1].layers[0].total_tokens) == (4, 9)
    for m in ms:
        m.clear()
    assert a.report_usage()["active_cpu_pages"] == 0


# ── invariants of the watermark policy ───────────────────────────────────────
def test_watermark_evicts_globally_oldest_first():
    """Eviction picks the full non-tail GPU pages with the smallest start_token
    across ALL layers; ties go to the earlier-inserted layer (stable sort)."""
    a = ok.KVAllocator(3, 1, 4, 4, 4, np.float32)
    pb = a.page_bytes()
    m = ok.KVCacheManager(a, gpu_high_watermark_bytes=10 ** 9)
    for layer in (2, 0, 1):                          # insertion order 2, 0, 1
        m.append_prefill(layer, *kv(16, h=1, d=4), GPU)
    evicted = m.evict_pages(4 * pb)
    # pages with start 0 in layers 2, 0, 1 (insertion order), then start 4 of layer 2
    starts = {p.page_id: (l, p.start_token) for l, L in m.layers.items() for p in L.pages}
    assert len(evicted) == 4
    gone = [(lid, st) for lid, L in m.layers.items() for p in L.pages if p.state == "CPU"
            for st in [p.start_token]]
    assert sorted(gone) == sorted([(2, 0), (0, 0), (1, 0), (2, 4)])
    assert starts  # page table still consistent


def test_skip_residency_quirk():
    """While every page is GPU-resident the decode append does not enforce the
    watermark (kv_offload.py:133-137), so GPU KV grows past it."""
    a = ok.KVAllocator(1, 1, 4, 4, 4, np.float32)
    m = ok.KVCacheManager(a, gpu_high_watermark_bytes=a.page_bytes())
    for _ in range(20):
        ok.decode_batched_pages([m], 0, [kv(1, h=1, d=4)[0]], [kv(1, h=1, d=4)[1]], GPU)
    assert all(p.state == "GPU" for p in m.layers[0].pages)
    assert m.gpu_evictable_bytes() > m.gpu_high_watermark_bytes


# ── planted mistakes: the checks above and below must catch each one ───────────
# Each variant plants one plausible slip in the oracle's residency rule
# (kv_cache.py:121-172).  `_pinning_failures` runs hand-worked scenarios whose
# expected page states are derived in the comments (not by running the oracle)
# and returns the scenarios a manager class gets wrong: none for the oracle, at
# least one for every planted mistake that can change an observable result.

def _states(m, lid=0):
    return [p.state for p in m.layers[lid].pages]


def _pinning_failures(cls):
    failed = []
    # page bytes: K+V of 1 head x 4 tokens x 4 dims fp32 = 128
    # S1: W = 2 pages, one layer, 16 tokens = pages p0..p3 (p3 the tail).  After
    # p2 the full non-tail pages p0, p1 hold exactly W (strictly above is needed:
    # no eviction); after p3 p0..p2 hold 3 pages, one over W: p0 alone goes.
    a = ok.KVAllocator(1, 1, 4, 4, 4, np.float32)
    m = cls(a, gpu_high_watermark_bytes=2 * a.page_bytes())
    m.append_prefill(0, *kv(16, h=1, d=4), GPU)
    if _states(m) != ["CPU", "GPU", "GPU", "GPU"]:
        failed.append("S1")
    # S2: W = 1 page.  6 tokens (p0 full, p1 = 2 tokens, the tail), then 8 more
    # (p2, p3 full).  p1 stops being the tail while partial, so it never counts
    # and is never evicted; after p3 the candidates are p0 and p2 (one over W):
    # p0 goes.
    a = ok.KVAllocator(1, 1, 4, 4, 4, np.float32)
    m = cls(a, gpu_high_watermark_bytes=a.page_bytes())
    m.append_prefill(0, *kv(6, h=1, d=4), GPU)
    m.append_prefill(0, *kv(8, h=1, d=4), GPU)
    if _states(m) != ["CPU", "GPU", "GPU", "GPU"]:
        failed.append("S2")
    # S3: layers inserted in the order 2, 0, 1 with 4 full pages each (page ids
    # 0-3, 4-7, 8-11); evicting 4 pages takes start 0 of layers 2, 0, 1 (ties in
    # insertion order), then start 4 of layer 2 — not the smallest page ids.
    a = ok.KVAllocator(3, 1, 4, 4, 4, np.float32)
    m = cls(a, gpu_high_watermark_bytes=10 ** 9)
    for layer in (2, 0, 1):
        m.append_prefill(layer, *kv(16, h=1, d=4), GPU)
    m.evict_pages(4 * a.page_bytes())
    gone = sorted((lid, p.start_token) for lid, L in m.layers.items() for p in L.pages
                  if p.state == "CPU")
    if gone != [(0, 0), (1, 0), (2, 0), (2, 4)]:
        failed.append("S3")
    # S4: decode appends with the watermark enforced (skip_residency False): W = 1
    # page, 3 pages of decode tokens one at a time.  When token 9 opens p2, p1
    # stops being the tail: p0, p1 are 2 pages, one over W, p0 goes.
    a = ok.KVAllocator(1, 1, 4, 4, 4, np.float32)
    m = cls(a, gpu_high_watermark_bytes=a.page_bytes())
    for t in range(12):
        m.append_decode(0, *kv(1, h=1, d=4, seed=t), GPU)
    if _states(m) != ["CPU", "GPU", "GPU"]:
        failed.append("S4")
    # S5: W = 0, two layers.  Layer 0 takes 8 tokens (a0, a1): when a1 arrives a0
    # goes.  A decode append with skip_residency (the all-GPU quirk of
    # kv_offload.py:133-137) opens a2, leaving a1 evictable but still on the GPU.
    # Layer 1 takes 7 tokens (b0 full, b1 = 3 tokens): enforcing after every page,
    # b0's arrival evicts a1 (the only candidate then) and b1's arrival evicts b0;
    # enforcing once at the end of the prefill would evict b0 (start 0) before a1
    # (start 4).  The order shows in the host pages' ids: GPU pages take ids 7, 6,
    # 5, 4, 3 (the first reserve of 8, popped from the end) and the host copies
    # 23, 22, 21 (the first host reserve of 16, ids 8..23) in eviction order.
    a = ok.KVAllocator(2, 1, 4, 4, 4, np.float32)
    m = cls(a, gpu_high_watermark_bytes=0)
    m.append_prefill(0, *kv(8, h=1, d=4), GPU)
    m.append_decode(0, *kv(1, h=1, d=4), GPU, skip_residency=True)
    m.append_prefill(1, *kv(7, h=1, d=4), GPU)
    got = {lid: [(p.page_id, p.state) for p in L.pages] for lid, L in m.layers.items()}
    if got != {0: [(23, "CPU"), (22, "CPU"), (5, "GPU")], 1: [(21, "CPU"), (3, "GPU")]}:
        failed.append("S5")
    return failed


class _EvictOneTooMany(ok.KVCacheManager):
    """The eviction loop stops only once the evicted bytes EXCEED the target."""

    def evict_pages(self, bytes_to_evict):
        if bytes_to_evict <= 0:
            return []
        cands = [(L, p) for L in self.layers.values() for p in L.pages
                 if p.state == "GPU" and p is not L.tail_page and p.used_tokens == p.capacity_tokens]
        cands.sort(key=lambda t: t[1].start_token)
        done = 0
        for L, p in cands:
            if done > bytes_to_evict:
                break
            L.pages[L.pages.index(p)] = self.allocator.move_page(p, "cpu")
            done += self.allocator.page_bytes()
        return []


class _TailCounted(ok.KVCacheManager):
    """The tail page counts toward the watermark."""

    def gpu_evictable_bytes(self):
        return super().gpu_evictable_bytes() + sum(
            self.allocator.page_bytes() for L in self.layers.values()
            if L.tail_page is not None and L.tail_page.state == "GPU"
            and L.tail_page.used_tokens == L.tail_page.capacity_tokens)


class _PartialCountedByTokens(ok.KVCacheManager):
    """Non-tail partial pages count their used tokens' bytes toward the watermark."""

    def gpu_evictable_bytes(self):
        extra = 0
        for L in self.layers.values():
            for p in L.pages:
                if p.state == "GPU" and p is not L.tail_page and p.used_tokens < p.capacity_tokens:
                    extra += self.allocator.page_bytes() * p.used_tokens // p.capacity_tokens
        return super().gpu_evictable_bytes() + extra


class _SortedByPageId(ok.KVCacheManager):
    """Oldest = smallest page id instead of smallest start_token."""

    def evict_pages(self, bytes_to_evict):
        if bytes_to_evict <= 0:
            return []
        cands = [(L, p) for L in self.layers.values() for p in L.pages
                 if p.state == "GPU" and p is not L.tail_page and p.used_tokens == p.capacity_tokens]
        cands.sort(key=lambda t: t[1].page_id)
        done = 0
        for L, p in cands:
            if done >= bytes_to_evict:
                break
            L.pages[L.pages.index(p)] = self.allocator.move_page(p, "cpu")
            done += self.allocator.page_bytes()
        return []


class _NoPrefillEnforcement(ok.KVCacheManager):
    """The watermark is enforced by decode appends only."""

    def append_prefill(self, layer_id, k, v, device):
        enforce = self._enforce_residency_policy
        self._enforce_residency_policy = lambda: None
        try:
            super().append_prefill(layer_id, k, v, device)
        finally:
            self._enforce_residency_policy = enforce


class _OncePerPrefill(ok.KVCacheManager):
    """The watermark is enforced once at the end of each append_prefill instead of
    after every page."""

    def append_prefill(self, layer_id, k, v, device):
        enforce = self._enforce_residency_policy
        self._enforce_residency_policy = lambda: None
        try:
            super().append_prefill(layer_id, k, v, device)
        finally:
            self._enforce_residency_policy = enforce
        enforce()


def test_pinning_scenarios_hold_for_the_oracle():
    assert _pinning_failures(ok.KVCacheManager) == []


@pytest.mark.parametrize("variant", [_EvictOneTooMany, _TailCounted, _PartialCountedByTokens,
                                     _SortedByPageId, _NoPrefillEnforcement, _OncePerPrefill])
def test_pinning_scenarios_catch_planted_mistake(variant):
    assert _pinning_failures(variant), f"{variant.__name__} passed every pinning scenario"


# Two slips that cannot change any observable result of the reference's rule,
# shown by running each against the oracle over random operation streams:
#   * `>=` instead of `>` at the watermark: at equality it asks evict_pages for 0
#     bytes, which returns at once (kv_cache.py:123-124);
#   * counting evicted bytes by used tokens instead of whole pages: only full
#     pages are evicted (:134), so the two counts agree.

class _GeWatermark(ok.KVCacheManager):
    def _enforce_residency_policy(self):
        gb = self.gpu_evictable_bytes()
        if gb >= self.gpu_high_watermark_bytes:
            self.evict_pages(gb - self.gpu_high_watermark_bytes)


class _UsedTokenBytes(ok.KVCacheManager):
    def evict_pages(self, bytes_to_evict):
        if bytes_to_evict <= 0:
            return []
        cands = [(L, p) for L in self.layers.values() for p in L.pages
                 if p.state == "GPU" and p is not L.tail_page and p.used_tokens == p.capacity_tokens]
        cands.sort(key=lambda t: t[1].start_token)
        done, per_token = 0, self.allocator.page_bytes() // self.allocator.page_size
        for L, p in cands:
            if done >= bytes_to_evict:
                break
            new = self.allocator.move_page(p, "cpu")
            L.pages[L.pages.index(p)] = new
            done += new.used_tokens * per_token
        return []


@pytest.mark.parametrize("variant", [_GeWatermark, _UsedTokenBytes])
def test_equivalent_slips_agree_with_the_oracle_on_random_streams(variant):
    for seed in range(40):
        g = np.random.default_rng(seed)
        n_layers, P = int(g.integers(1, 4)), 4
        mk = lambda: ok.KVAllocator(n_layers, 1, 4, P, 4, np.float32)   # noqa: E731
        a1, a2 = mk(), mk()
        wm = int(g.integers(0, 6)) * a1.page_bytes()
        ms = (ok.KVCacheManager(a1, wm), variant(a2, wm))
        for _ in range(40):
            op = g.choice(["prefill", "decode", "decode", "clear"], p=[0.3, 0.3, 0.35, 0.05])
            lid = int(g.integers(0, n_layers))
            n = int(g.integers(1, 14))
            skip = bool(g.integers(0, 2))
            for m in ms:
                if op == "prefill":
                    m.append_prefill(lid, *kv(n, h=1, d=4), GPU)
                elif op == "decode":
                    m.append_decode(lid, *kv(1, h=1, d=4), GPU, skip_residency=skip)
                else:
                    m.clear()
            assert ok.snapshot(ms[0]) == ok.snapshot(ms[1]), (variant.__name__, seed)
            assert a1.report_usage() == a2.report_usage()


# ── contiguous path (kv_cache.py:206-289) ─────────────────────────────────────
def _run_contiguous(cls, prompt, decode, P=4, cap=1024):
    """Prefill `prompt` tokens (pages + contiguous buffer), decode `decode` tokens
    through decode_step_kv (two layers); returns the manager and the tokens
    written per layer."""
    a = ok.KVAllocator(2, 1, 4, P, 4, np.float32)
    m = cls(a, gpu_high_watermark_bytes=10 ** 9)
    assert m.build_contiguous(2, 1, 4, cap, GPU)
    written = {}
    for lid in range(2):
        k, v = kv(prompt, h=1, d=4, seed=lid)
        m.append_prefill(lid, k, v, GPU)
        m.prefill_contiguous(lid, k, v)
        written[lid] = [k]
    for t in range(decode):
        for lid in range(2):
            k, v = kv(1, h=1, d=4, seed=1000 + 2 * t + lid)
            ok.decode_step_kv([m], lid, [k], [v], GPU)
            written[lid].append(k)
    return m, {lid: np.concatenate(ks, axis=2) for lid, ks in written.items()}


def _contiguous_failures(cls):
    failed = []
    # 1021 prompt tokens in pages of 4 (255 full + one of 1), 9 decode tokens: 3
    # fit the buffer, the 4th overflows it: the 3 buffered tokens migrate as a
    # prefill (a new page of 3 after the 1-token page, now the tail), and paged
    # decode fills it (4) and continues: pages ... 4, 1, 4, 4, 1.
    m, written = _run_contiguous(cls, 1021, 9)
    for lid in range(2):
        k, _ = ok.layer_tokens(m, lid)
        if k.shape != written[lid].shape or not np.array_equal(k, written[lid]):
            failed.append(f"tokens L{lid}")
        used = [p.used_tokens for p in m.layers[lid].pages]
        if used != [4] * 255 + [1, 4, 4, 1]:
            failed.append(f"pages L{lid}")
    if m.use_contiguous or m.cont_K:
        failed.append("buffers kept")
    return failed


class _MigrateSkipsOne(ok.KVCacheManager):
    """Migration starts one token after the prompt."""

    def migrate_contiguous_to_pages(self):
        self.cont_prefill_len += 1
        super().migrate_contiguous_to_pages()


class _MigrateDropsInFlight(ok.KVCacheManager):
    """Commits the decode token before the last layer has written it."""

    def advance_contiguous(self):
        pass

    def write_decode_contiguous(self, layer_id, k, v):
        super().write_decode_contiguous(layer_id, k, v)
        if layer_id == 0:
            self.cont_seq_len += 1


def test_contiguous_oracle_keeps_every_token_in_order():
    assert _contiguous_failures(ok.KVCacheManager) == []


@pytest.mark.parametrize("variant", [_MigrateSkipsOne, _MigrateDropsInFlight])
def test_contiguous_checks_catch_planted_mistake(variant):
    assert _contiguous_failures(variant)


def test_contiguous_capacity_halving_closed_form():
    """Capacities tried: c, c/2, ... while >= 1024; the first that fits is kept."""
    for cap, limit, want in [(32768, 10 ** 9, 32768), (32768, 5000, 4096), (3000, 1500, 1500),
                             (32768, 1000, 0), (1000, 10 ** 9, 0)]:
        tried = []

        def alloc(shape):
            tried.append(shape[2])
            if shape[2] > limit:
                raise ok.OutOfMemory()
            return np.zeros(shape, np.float32)
        m = ok.KVCacheManager(ok.KVAllocator(1, 1, 4, 4, 4, np.float32), 0)
        built = m.build_contiguous(1, 1, 4, cap, GPU, alloc=alloc)
        assert built == (want > 0) and m.cont_capacity == (want if want else 0)
        expect = []
        c = cap
        while c >= 1024:
            expect.append(c)
            if c <= limit:
                break
            c //= 2
        assert sorted(set(tried), reverse=True) == expect
