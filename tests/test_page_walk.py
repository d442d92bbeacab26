"""The page walk of perform_streaming_attention: the C module (helm_amd._page_walk)
against the Python walk (walk_pages_py) on random page lists, and both against
hand-worked lists.  CPU only: pages carry tensors and devices, nothing is launched.

The walk decides what the kernels read (helm/runtime/kv_cache.py:350-351 for the
page filter: pages with used tokens, on the tier their state names), so every
field of its result must be the same object or the same int32 array.
"""
import numpy as np
import pytest
import torch

from helm_amd.runtime import kv_cache as kc
from helm_amd.runtime.kv_allocator import KVPage

P = 16
CUDA, CPU = torch.device("cuda"), torch.device("cpu")


def c_walk():
    if kc._page_walk is None:
        pytest.fail("helm_amd._page_walk is not built (python -m helm_amd.build)")
    return kc._page_walk


def as_tuple(w: kc.PageWalk):
    ids = lambda seq: [id(p) for p in seq]  # noqa: E731
    return (id(w.first_active), list(w.run_lens), np.asarray(w.run_meta).tolist(),
            [np.asarray(c).tolist() for c in w.chunk_slots], [ids(ws) for ws in w.chunk_waits],
            ids(w.gpu_rest), ids(w.cpu_rest))


def c_result(pages, gb, gv, hb, hv, chunk_pages):
    fa, rl, rm, cs, cw, gr, cr = c_walk().classify(pages, gb, gv, hb, hv, chunk_pages, P)
    return kc.PageWalk(fa, rl, np.frombuffer(rm, dtype=np.int32),
                       [np.frombuffer(c, dtype=np.int32) for c in cs], cw, gr, cr)


def random_pages(rng, n):
    """Pages of every kind the walk tells apart: device / host pool pages (bound to
    their slot with their views, or stale), free-standing pages, pages on the other
    tier than their state, empty, FREE / DEAD, partial, with an eviction in flight."""
    pages, gb, gv, hb, hv = [], {}, {}, {}, {}
    for i in range(n):
        state = rng.choice(["GPU", "CPU", "GPU", "CPU", "DEAD", "FREE"])
        wrong_tier = rng.random() < 0.05
        on_gpu = (state == "GPU") != wrong_tier
        dev = CUDA if on_gpu else CPU
        k, v = torch.zeros(1), torch.zeros(1)
        used = int(rng.choice([0, P, P, P, P, int(rng.integers(1, P))]))
        slot = int(rng.integers(0, 4 * n))
        p = KVPage(i, 0, i * P, used, P, k, v, dev, state, slot=slot)
        if rng.random() < 0.3:
            p.ready = object()
        kind = rng.random()
        bound, views = (gb, gv) if state == "GPU" else (hb, hv)
        if kind < 0.75:                    # a pool page holding its slot's views
            bound[slot] = p
            views[slot] = (k, v)
        elif kind < 0.85:                  # bound, but the slot's views were handed on
            bound[slot] = p
            views[slot] = (torch.zeros(1), v)
        elif kind < 0.9:                   # bound with no views recorded
            bound[slot] = p
        pages.append(p)                    # else free-standing
    return pages, gb, gv, hb, hv


@pytest.mark.parametrize("seed", range(40))
@pytest.mark.parametrize("chunk_pages", [1, 3, 256])
def test_c_walk_equals_python_walk(seed, chunk_pages):
    rng = np.random.default_rng(seed)
    pages, gb, gv, hb, hv = random_pages(rng, int(rng.integers(0, 300)))
    py = kc.walk_pages_py(pages, gb, gv, hb, hv, chunk_pages, P)
    assert as_tuple(c_result(pages, gb, gv, hb, hv, chunk_pages)) == as_tuple(py)
    # and through the dispatching entry point
    assert as_tuple(kc.walk_pages(pages, gb, gv, hb, hv, chunk_pages, P)) == as_tuple(py)


def test_oldest_half_on_host_at_4k():
    """4K tokens, the oldest 128 pages on the host (the watermark case): one chunk of
    the 128 host slots, closed at the first device page, and one run of the 128
    device pages ending at the partial last page."""
    pages, gb, gv, hb, hv = [], {}, {}, {}, {}
    for i in range(256):
        host = i < 128
        k, v = torch.zeros(1), torch.zeros(1)
        used = 5 if i == 255 else P
        p = KVPage(i, 0, i * P, used, P, k, v, CPU if host else CUDA, "CPU" if host else "GPU",
                   slot=1000 + i)
        (hb if host else gb)[p.slot] = p
        (hv if host else gv)[p.slot] = (k, v)
        pages.append(p)
    for w in (kc.walk_pages_py(pages, gb, gv, hb, hv, 256, P), c_result(pages, gb, gv, hb, hv, 256)):
        assert w.first_active is pages[0]
        assert w.run_lens == [128]
        assert np.asarray(w.run_meta).tolist() == list(range(1128, 1256)) + [127 * P + 5]
        assert [np.asarray(c).tolist() for c in w.chunk_slots] == [list(range(1000, 1128))]
        assert w.chunk_waits == [[]] and w.gpu_rest == [] and w.cpu_rest == []


def test_hand_worked_chunk_and_run_boundaries():
    """Host pages H, device pages D (pool pages with their views), chunk size 2:
      H0 H1 H2 D3 H4 D5(partial) X6(free-standing host page) H7 H8 D9
    chunks: [H0 H1] (full), [H2] (closed at D3: a half still free), then [H4] is
    closed at D5 only while fewer than two chunks are closed, which is no longer
    so: it stays open, X6 goes to the repack list, and H7 makes it full -> [H4 H7];
    H8 stays open to the end -> [H8].  Runs: D3 D5 end at the partial D5
    (1 * P + 7 tokens); D9 is an open run of one full page."""
    pages, gb, gv, hb, hv = [], {}, {}, {}, {}
    kinds = ["H", "H", "H", "D", "H", "D", "X", "H", "H", "D"]
    for i, kind in enumerate(kinds):
        k, v = torch.zeros(1), torch.zeros(1)
        used = 7 if i == 5 else P
        dev, state = (CUDA, "GPU") if kind == "D" else (CPU, "CPU")
        p = KVPage(i, 0, i * P, used, P, k, v, dev, state, slot=100 + i)
        if i == 4:
            p.ready = object()
        if kind == "H":
            hb[p.slot], hv[p.slot] = p, (k, v)
        elif kind == "D":
            gb[p.slot], gv[p.slot] = p, (k, v)
        pages.append(p)
    for w in (kc.walk_pages_py(pages, gb, gv, hb, hv, 2, P), c_result(pages, gb, gv, hb, hv, 2)):
        assert [np.asarray(c).tolist() for c in w.chunk_slots] == [[100, 101], [102], [104, 107], [108]]
        assert [[q.page_id for q in ws] for ws in w.chunk_waits] == [[], [], [4], []]
        assert w.run_lens == [2, 1]
        assert np.asarray(w.run_meta).tolist() == [103, 105, P + 7, 109, P]
        assert [q.page_id for q in w.cpu_rest] == [6] and w.gpu_rest == []
        assert w.first_active is pages[0]


def test_nothing_to_attend():
    p = KVPage(0, 0, 0, 0, P, torch.zeros(1), torch.zeros(1), CUDA, "GPU", slot=0)
    d = KVPage(1, 0, P, P, P, torch.zeros(1), torch.zeros(1), CUDA, "DEAD", slot=1)
    for w in (kc.walk_pages_py([p, d], {}, {}, {}, {}, 256, P), c_result([p, d], {}, {}, {}, {}, 256)):
        assert w.first_active is None and w.run_lens == [] and w.chunk_slots == []


def test_c_walk_rejects_bad_arguments():
    with pytest.raises(ValueError):
        c_walk().classify([], {}, {}, {}, {}, 0, P)
    with pytest.raises(TypeError):
        c_walk().classify([], [], {}, {}, {}, 1, P)
    with pytest.raises(AttributeError):
        c_walk().classify([object()], {}, {}, {}, {}, 1, P)


def test_c_walk_leaks_no_references():
    """Walks whose results are dropped leave every page's and device's reference
    count where it was."""
    import sys
    rng = np.random.default_rng(7)
    pages, gb, gv, hb, hv = random_pages(rng, 200)
    before = [sys.getrefcount(p) for p in pages] + [sys.getrefcount(CUDA), sys.getrefcount(CPU)]
    for _ in range(50):
        c_walk().classify(pages, gb, gv, hb, hv, 3, P)
    after = [sys.getrefcount(p) for p in pages] + [sys.getrefcount(CUDA), sys.getrefcount(CPU)]
    assert before == after
