"""GPU tests of the runtime: page pools, eviction data integrity, and
perform_streaming_attention over device-resident (in place) and host-resident
(staged, double-buffered) pages.  Attention bar: 2e-3 max abs vs the fp64 form."""
import math

import numpy as np
import pytest
import torch

from helm_amd.runtime import KVAllocator, KVCacheManager, perform_streaming_attention
from helm_amd.runtime import kv_cache as kc
from oracle import attention as oa
from oracle import kv_pages as okp

pytestmark = pytest.mark.gpu
GPU, CPU = torch.device("cuda"), torch.device("cpu")
ATOL = 2e-3


def test_allocator_cuda_cases():
    """Reference CUDA-only tests test_kv_allocator.py:175-220 on the product."""
    a = KVAllocator(2, 2, 8, 4, torch.float16)
    p = a.allocate(GPU)
    assert p.state == "GPU" and p.device.type == "cuda" and p.k_tensor.is_cuda
    c = a.allocate(CPU)
    c.layer_id, c.start_token, c.used_tokens = 2, 8, 3
    c.k_tensor[:, :, :3] = 7.0
    c.v_tensor[:, :, :3] = 8.0
    free_before = len(a.cpu_free_pool)
    n = a.move_page(c, GPU)
    assert n.device.type == "cuda" and (n.layer_id, n.start_token, n.used_tokens) == (2, 8, 3)
    assert torch.all(n.k_tensor[:, :, :3].cpu() == 7.0) and torch.all(n.v_tensor[:, :, :3].cpu() == 8.0)
    assert len(a.cpu_free_pool) == free_before + 1
    e = a.allocate(CPU)
    e.used_tokens = 0
    assert a.move_page(e, GPU).used_tokens == 0


def test_eviction_moves_data_and_frees_slots():
    a = KVAllocator(2, 2, 8, 4, torch.float16)
    m = KVCacheManager(a, gpu_high_watermark_bytes=0)
    m.initialize_layer_caches(2)
    k = torch.randn(1, 2, 16, 8, dtype=torch.float16, device=GPU)
    v = torch.randn(1, 2, 16, 8, dtype=torch.float16, device=GPU)
    m.append_prefill(0, k, v)
    pages = m.layers[0].pages
    assert [p.state for p in pages] == ["CPU", "CPU", "CPU", "GPU"]   # tail protected
    for i, p in enumerate(pages):
        assert torch.equal(p.k_tensor[:, :, :4].cpu(), k[:, :, 4 * i:4 * i + 4].cpu())
        assert torch.equal(p.v_tensor[:, :, :4].cpu(), v[:, :, 4 * i:4 * i + 4].cpu())
    pool = a.pool(GPU)
    assert len(pool.free_slots) == 3          # DEAD pages returned their device slots


@pytest.mark.parametrize("seed", range(4))
def test_batched_prefill_writes_match_oracle_under_evictions(seed):
    """append_prefill with device K/V queues its GPU pages and writes them with one
    helm_kv_append per run (flushed before any eviction): page tables, states and
    every page's tokens equal the oracle's page-by-page copy, with watermarks that
    evict in the middle of a prompt."""
    g = np.random.default_rng(seed)
    H, D, P = 2, 8, 4
    pa = KVAllocator(3, H, D, P, torch.float16, gpu_capacity_pages=4)
    oa_ = okp.KVAllocator(3, H, D, P, 2, np.float16)
    pb = oa_.page_bytes()
    for wm in (0, 3 * pb, 7 * pb + pb // 2, 10 ** 9):
        pm = KVCacheManager(pa, gpu_high_watermark_bytes=wm)
        om = okp.KVCacheManager(oa_, gpu_high_watermark_bytes=wm)
        pm.initialize_layer_caches(3)
        om.initialize_layer_caches(3)
        for _ in range(8):
            layer = int(g.integers(3))
            n = int(g.integers(1, 23))
            k = g.standard_normal((1, H, n, D)).astype(np.float16)
            v = g.standard_normal((1, H, n, D)).astype(np.float16)
            pm.append_prefill(layer, torch.from_numpy(k).to(GPU), torch.from_numpy(v).to(GPU))
            om.append_prefill(layer, k, v, "cuda")
        torch.cuda.synchronize()
        snap = [(lid, [(p.page_id, p.state, p.device.type, p.start_token, p.used_tokens)
                       for p in L.pages],
                 None if L.tail_page is None else L.tail_page.page_id, L.total_tokens)
                for lid, L in pm.layers.items()]
        assert snap == okp.snapshot(om)
        for lid, L in om.layers.items():
            for pp, op in zip(pm.layers[lid].pages, L.pages):
                u = op.used_tokens
                np.testing.assert_array_equal(pp.k_tensor[:, :, :u].cpu().numpy(), op.k[:, :, :u])
                np.testing.assert_array_equal(pp.v_tensor[:, :, :u].cpu().numpy(), op.v[:, :, :u])
        pm.initialize_layer_caches(0)
        om.initialize_layer_caches(0)


def test_gather_pages_h2d_reads_scattered_host_pages():
    """helm_gather_pages_h2d: pages at scattered pinned host slots land bit-exact in
    consecutive staging slots from dev_first_slot on; slots outside the host pool
    leave their staging page untouched; pageable host memory is refused."""
    from helm_amd.kernels import attention as ka
    g = torch.Generator().manual_seed(5)
    cap, Hkv, P, D = 300, 8, 16, 128
    hk = torch.randn(cap, Hkv, P, D, generator=g).half().pin_memory()
    hv = torch.randn(cap, Hkv, D, P, generator=g).half().pin_memory()
    dk = torch.full((64, Hkv, P, D), float("nan"), dtype=torch.float16, device=GPU)
    dv = torch.full((64, Hkv, D, P), float("nan"), dtype=torch.float16, device=GPU)
    slots = [299, 3, 150, -1, 7, 8, 9, 300, 0, 42]
    st = torch.cuda.Stream()
    sd = torch.tensor(slots, dtype=torch.int32, device=GPU)
    ka.gather_pages_h2d(hk, hv, dk, dv, sd, 20, st)
    st.synchronize()
    for i, s in enumerate(slots):
        if 0 <= s < cap:
            assert torch.equal(dk[20 + i].cpu(), hk[s]) and torch.equal(dv[20 + i].cpu(), hv[s])
        else:
            assert torch.isnan(dk[20 + i]).all() and torch.isnan(dv[20 + i]).all()
    assert torch.isnan(dk[:20]).all() and torch.isnan(dk[30:]).all()
    with pytest.raises(RuntimeError, match="pinned"):
        ka.gather_pages_h2d(hk.clone(), hv, dk, dv, sd, 0, st)


def make_pages(a, n_gpu_full, n_cpu_full, tail, Hkv, D, seed):
    """A layer's page list: full pages (a mix moved to the host) then a partial tail."""
    g = torch.Generator().manual_seed(seed)
    P = a.page_size
    m = KVCacheManager(a, gpu_high_watermark_bytes=10 ** 12)
    T = (n_gpu_full + n_cpu_full) * P + tail
    k = torch.randn(1, Hkv, T, D, generator=g).half()
    v = torch.randn(1, Hkv, T, D, generator=g).half()
    m.append_prefill(0, k.to(GPU), v.to(GPU))
    m.evict_pages(n_cpu_full * a.page_bytes())        # oldest pages go to the host
    return m, k, v


@pytest.mark.parametrize("n_gpu,n_cpu,tail", [(10, 0, 5), (0, 10, 3), (37, 150, 16), (3, 200, 1),
                                              (5, 600, 7), (2, 1100, 9)])
def test_streaming_attention_mixed_residency(n_gpu, n_cpu, tail):
    Hq, Hkv, D, P = 32, 8, 128, 16
    a = KVAllocator(1, Hkv, D, P, torch.float16)
    m, k, v = make_pages(a, n_gpu, n_cpu, tail, Hkv, D, seed=n_gpu + n_cpu)
    states = [p.state for p in m.layers[0].pages]
    assert states.count("CPU") == n_cpu
    q = torch.randn(1, Hq, 1, D, dtype=torch.float16, device=GPU)
    out = perform_streaming_attention(q, m.iterate_layer_pages(0), allocator=a)
    ref = oa.eager(q.cpu().numpy(), k.numpy(), v.numpy())
    assert out.dtype == torch.float16 and out.shape == (1, Hq, 1, D)
    assert np.abs(out.cpu().numpy().astype(np.float64) - ref).max() <= ATOL
    # host pages were staged in chunks of STAGE_CHUNK_PAGES, the two staging halves
    # in turn; more than two chunks reuse them
    n_chunks = -(-n_cpu // kc.STAGE_CHUNK_PAGES)
    assert all(kc._state(GPU).buf_used[:min(n_chunks, 2)])


def test_streaming_attention_interleaved_host_runs():
    """Host and device runs alternate along the list (pages of three sequences of
    one allocator, attended as one): a host run that ends early closes its chunk
    and is staged while the walk goes on; later runs share the chunks that
    remain."""
    Hq, Hkv, D, P = 32, 8, 128, 16
    a = KVAllocator(1, Hkv, D, P, torch.float16)
    parts = [make_pages(a, n_gpu, n_cpu, tail, Hkv, D, seed=11 + i)
             for i, (n_gpu, n_cpu, tail) in enumerate([(4, 100, 16), (3, 300, 5), (0, 40, 2)])]
    pages = [pg for m, _, _ in parts for pg in m.iterate_layer_pages(0)]
    k = torch.cat([kk for _, kk, _ in parts], dim=2)
    v = torch.cat([vv for _, _, vv in parts], dim=2)
    q = torch.randn(1, Hq, 1, D, dtype=torch.float16, device=GPU)
    out = perform_streaming_attention(q, pages, allocator=a)
    ref = oa.eager(q.cpu().numpy(), k.numpy(), v.numpy())
    assert np.abs(out.cpu().numpy().astype(np.float64) - ref).max() <= ATOL
    # the same pages again, reusing both staging halves
    out2 = perform_streaming_attention(q, pages, allocator=a)
    assert torch.equal(out, out2)


def test_streaming_attention_free_standing_pages():
    """Pages that are not pool slots (reference tests build them by hand) are
    repacked; batch>1 queries and GQA follow test_streaming_attention.py."""
    from helm_amd.runtime import KVPage
    Hq, Hkv, D = 4, 2, 64
    q = torch.randn(2, Hq, 1, D, dtype=torch.float16, device=GPU)
    ks = [torch.randn(2, Hkv, n, D, dtype=torch.float16) for n in (3, 5, 2)]
    vs = [torch.randn(2, Hkv, n, D, dtype=torch.float16) for n in (3, 5, 2)]
    pages = []
    for i, (kk, vv) in enumerate(zip(ks, vs)):
        dev = GPU if i == 1 else CPU
        pages.append(KVPage(i, 0, 0, kk.shape[2], kk.shape[2], kk.to(dev), vv.to(dev), dev,
                            "GPU" if i == 1 else "CPU"))
    empty = KVPage(9, 0, 0, 0, 4, torch.zeros(2, Hkv, 4, D).half(), torch.zeros(2, Hkv, 4, D).half(),
                   CPU, "CPU")
    out = perform_streaming_attention(q, [empty] + pages)
    # reference order: GPU pages first, then CPU pages (softmax is order-free)
    kk = torch.cat([ks[1], ks[0], ks[2]], 2).numpy()
    vv = torch.cat([vs[1], vs[0], vs[2]], 2).numpy()
    ref = oa.eager(q.cpu().numpy(), kk, vv)
    assert np.abs(out.cpu().numpy().astype(np.float64) - ref).max() <= ATOL
    assert torch.all(perform_streaming_attention(q, []) == 0)
    assert torch.all(perform_streaming_attention(q, [empty]) == 0)


def test_async_eviction_keeps_data_and_recycles_slots_after_copy():
    """With asynchronous eviction the host thread does not wait for the D2H copies:
    attention issued right after the evictions still sees every byte (readers wait
    on the pages' copy events), the host copies equal the originals once
    synchronised, and the device slots return to the pool only after the copies."""
    Hq, Hkv, D, P = 32, 8, 128, 16
    a = KVAllocator(1, Hkv, D, P, torch.float16, async_eviction=True)
    m = KVCacheManager(a, gpu_high_watermark_bytes=10 ** 12)
    T = 300 * P + 5
    g = torch.Generator().manual_seed(5)
    k = torch.randn(1, Hkv, T, D, generator=g).half()
    v = torch.randn(1, Hkv, T, D, generator=g).half()
    m.append_prefill(0, k.to(GPU), v.to(GPU))
    m.evict_pages(250 * a.page_bytes())
    pages = m.iterate_layer_pages(0)
    assert sum(p.state == "CPU" for p in pages) == 250
    assert any(p.ready is not None for p in pages)
    q = torch.randn(1, Hq, 1, D, dtype=torch.float16, device=GPU)
    out = perform_streaming_attention(q, pages, allocator=a)       # no synchronisation before
    ref = oa.eager(q.cpu().numpy(), k.numpy(), v.numpy())
    assert np.abs(out.cpu().numpy().astype(np.float64) - ref).max() <= ATOL
    a.synchronize()
    pool = a.pool(GPU)
    assert not pool.pending and len(pool.free_slots) >= 250
    for i, p in enumerate(pages[:250]):
        assert torch.equal(p.k_tensor[:, :, :P], k[:, :, i * P:(i + 1) * P])
        assert torch.equal(p.v_tensor[:, :, :P], v[:, :, i * P:(i + 1) * P])


def test_streaming_attention_rejects_cpu_query():
    with pytest.raises(RuntimeError, match="GPU"):
        perform_streaming_attention(torch.zeros(1, 2, 1, 8), [])


def test_pinned_ring_uploads_across_wraps_behind_busy_gpu():
    """Uploads of mixed sizes through a small pinned ring while the GPU is kept
    busy, so copies queue behind the work and the host wraps the ring several
    times: every destination receives its own bytes."""
    from helm_amd.runtime.page_table import PinnedRing
    ring = PinnedRing(1 << 15)
    rng = np.random.default_rng(3)
    a = torch.randn(4096, 4096, device=GPU, dtype=torch.float16)
    outs = []
    for i in range(300):
        if i % 40 == 0:
            for _ in range(4):
                a = (a @ a).clamp_(-1, 1)        # keep the stream busy
        n = int(rng.choice([16, 64, 700, 2500]))
        src = rng.integers(-2 ** 31, 2 ** 31 - 1, n, dtype=np.int64).astype(np.int32)
        dst = torch.empty(n, dtype=torch.int32, device=GPU)
        ring.upload(src, dst)
        outs.append((src, dst))
    torch.cuda.synchronize()
    assert sum(s.nbytes for s, _ in outs) > 4 * ring.cap
    for src, dst in outs:
        np.testing.assert_array_equal(dst.cpu().numpy(), src)


def test_stage_pages_h2d_equals_gather_kernel():
    """helm_stage_pages_h2d (hipMemcpyAsync per run of consecutive host slots, on a
    copy stream) and helm_gather_pages_h2d (one kernel reading the pinned pool)
    stage the same host pages to the same device slots, bit for bit."""
    from helm_amd.kernels import attention as ka
    g = torch.Generator().manual_seed(21)
    cap, Hkv, P, D = 200, 8, 16, 128
    hk = torch.randn(cap, Hkv, P, D, generator=g).half().pin_memory()
    hv = torch.randn(cap, Hkv, D, P, generator=g).half().pin_memory()
    slots = [5, 6, 7, 8, 150, 3, 4, 199, 0, 1, 2, 77]     # runs and singles
    st = torch.cuda.Stream()
    dk1 = torch.zeros(32, Hkv, P, D, dtype=torch.float16, device=GPU)
    dv1 = torch.zeros(32, Hkv, D, P, dtype=torch.float16, device=GPU)
    done = torch.cuda.Event()
    ka.stage_pages_h2d(hk, dk1, slots, 9, st, done)
    ka.stage_pages_h2d(hv, dv1, slots, 9, st)
    dk2 = torch.zeros_like(dk1)
    dv2 = torch.zeros_like(dv1)
    ka.gather_pages_h2d(hk, hv, dk2, dv2, torch.tensor(slots, dtype=torch.int32, device=GPU), 9, st)
    torch.cuda.current_stream().wait_event(done)
    st.synchronize()
    assert torch.equal(dk1, dk2) and torch.equal(dv1, dv2)
    for i, s in enumerate(slots):
        assert torch.equal(dk1[9 + i].cpu(), hk[s])
    assert not dk1[:9].any() and not dk1[9 + len(slots):].any()


def test_stream_pointer_follows_torch_current_stream():
    """The hipStream_t the kernels are launched on is torch's current stream:
    the default one, a side stream inside `torch.cuda.stream`, and the capturing
    stream of a graph."""
    from helm_amd import _native
    dev = torch.device("cuda")
    assert _native.stream_ptr(dev) == torch.cuda.current_stream(dev).cuda_stream
    assert _native.stream_ptr() == torch.cuda.current_stream().cuda_stream
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        assert _native.stream_ptr(dev) == side.cuda_stream
    assert _native.stream_ptr(dev) == torch.cuda.current_stream(dev).cuda_stream
    seen = []
    g = torch.cuda.CUDAGraph()
    x = torch.zeros(4, device=dev)
    with torch.cuda.graph(g):
        seen.append((_native.stream_ptr(dev), torch.cuda.current_stream(dev).cuda_stream))
        x.add_(1)
    g.replay()
    torch.cuda.synchronize()
    assert seen[0][0] == seen[0][1]
