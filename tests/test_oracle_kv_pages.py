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
