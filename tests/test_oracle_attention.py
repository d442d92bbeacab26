"""Pins the attention oracle (oracle/attention.py).

Restates the reference's tests/unit/runtime/test_streaming_attention.py:47-241
(atol 1e-4, fp32 CPU tensors) against oracle.streaming_attention, checks the
fp64 closed form against torch's scaled_dot_product_attention (a library
routine) and a brute-force loop, exercises the online-softmax path (a CUDA query
with CPU pages, :387-442) and the paged reference against the eager form.
"""
import math
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import attention as oa


def page(k, v, page_id=0, start=0, state="CPU", device="cpu"):
    return SimpleNamespace(page_id=page_id, layer_id=0, start_token=start, used_tokens=k.shape[2],
                           capacity_tokens=k.shape[2], k_tensor=k.copy(), v_tensor=v.copy(),
                           device=device, state=state)


def eager32(q, k, v, scale=None):
    """The reference test's _eager (test_streaming_attention.py:34-40)."""
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    w = torch.softmax(torch.from_numpy(q).float() @ torch.from_numpy(k).float().transpose(-2, -1) * scale, -1)
    return (w @ torch.from_numpy(v).float()).numpy().astype(q.dtype)


def rnd(*shape, seed=0):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def test_single_page():                                     # :47-55
    q, k, v = rnd(1, 2, 1, 8), rnd(1, 2, 4, 8, seed=1), rnd(1, 2, 4, 8, seed=2)
    r = oa.streaming_attention(q, [page(k, v)])
    assert r.shape == (1, 2, 1, 8)
    assert np.allclose(r, eager32(q, k, v), atol=1e-4)


def test_two_and_three_pages():                             # :58-88
    q = rnd(1, 2, 1, 8)
    k1, v1, k2, v2 = rnd(1, 2, 4, 8, seed=1), rnd(1, 2, 4, 8, seed=2), rnd(1, 2, 3, 8, seed=3), rnd(1, 2, 3, 8, seed=4)
    r = oa.streaming_attention(q, [page(k1, v1, 0, 0), page(k2, v2, 1, 4)])
    assert np.allclose(r, eager32(q, np.concatenate([k1, k2], 2), np.concatenate([v1, v2], 2)), atol=1e-4)
    q = rnd(1, 1, 1, 16, seed=5)
    ks = [rnd(1, 1, n, 16, seed=10 + n) for n in (3, 5, 2)]
    vs = [rnd(1, 1, n, 16, seed=20 + n) for n in (3, 5, 2)]
    r = oa.streaming_attention(q, [page(k, v, i) for i, (k, v) in enumerate(zip(ks, vs))])
    assert np.allclose(r, eager32(q, np.concatenate(ks, 2), np.concatenate(vs, 2)), atol=1e-4)


def test_no_pages_and_empty_pages():                        # :95-127
    q = rnd(1, 2, 1, 8)
    assert (oa.streaming_attention(q, []) == 0).all()
    k, v = rnd(1, 2, 4, 8, seed=1), rnd(1, 2, 4, 8, seed=2)
    empty = page(k, v)
    empty.used_tokens = 0
    assert np.allclose(oa.streaming_attention(q, [empty]), 0, atol=1e-6)
    real = page(k, v, 1)
    z = page(np.zeros_like(k), np.zeros_like(v))
    z.used_tokens = 0
    assert np.allclose(oa.streaming_attention(q, [z, real]), oa.streaming_attention(q, [real]), atol=1e-5)


def test_scales():                                          # :134-154
    q, k, v = rnd(1, 1, 1, 4), rnd(1, 1, 3, 4, seed=1), rnd(1, 1, 3, 4, seed=2)
    assert np.allclose(oa.streaming_attention(q, [page(k, v)], scale=0.25), eager32(q, k, v, 0.25), atol=1e-4)
    q, k, v = rnd(1, 1, 1, 16), rnd(1, 1, 4, 16, seed=1), rnd(1, 1, 4, 16, seed=2)
    assert np.allclose(oa.streaming_attention(q, [page(k, v)]),
                       oa.streaming_attention(q, [page(k, v)], scale=1 / 4.0), atol=1e-5)


def test_dtype_and_shape():                                 # :161-185
    for dt in (np.float32, np.float16):
        q, k, v = (rnd(1, 2, 1, 8).astype(dt), rnd(1, 2, 4, 8, seed=1).astype(dt),
                   rnd(1, 2, 4, 8, seed=2).astype(dt))
        assert oa.streaming_attention(q, [page(k, v)]).dtype == dt
    q, k, v = rnd(2, 4, 1, 16), rnd(2, 4, 6, 16, seed=1), rnd(2, 4, 6, 16, seed=2)
    assert oa.streaming_attention(q, [page(k, v)]).shape == (2, 4, 1, 16)


def test_gqa():                                             # :192-227
    q, k, v = rnd(1, 4, 1, 8), rnd(1, 2, 6, 8, seed=1), rnd(1, 2, 6, 8, seed=2)
    r = oa.streaming_attention(q, [page(k, v)])
    exp = eager32(q, np.repeat(k, 2, 1), np.repeat(v, 2, 1))
    assert r.shape == (1, 4, 1, 8) and np.allclose(r, exp, atol=1e-4)
    ks = [rnd(1, 2, n, 8, seed=30 + n) for n in (4, 3)]
    vs = [rnd(1, 2, n, 8, seed=40 + n) for n in (4, 3)]
    r = oa.streaming_attention(q, [page(a, b, i) for i, (a, b) in enumerate(zip(ks, vs))])
    exp = eager32(q, np.repeat(np.concatenate(ks, 2), 2, 1), np.repeat(np.concatenate(vs, 2), 2, 1))
    assert np.allclose(r, exp, atol=1e-4)


def test_large_logits_no_nan():                             # :234-242
    q = np.ones((1, 1, 1, 64), np.float32) * 100
    k = np.ones((1, 1, 8, 64), np.float32) * 100
    r = oa.streaming_attention(q, [page(k, rnd(1, 1, 8, 64))])
    assert np.isfinite(r).all()


def test_online_softmax_path_matches_eager():
    """CUDA query with GPU + CPU pages takes the online-softmax loop (:387-442)."""
    q = rnd(1, 8, 1, 16)
    pages, ks, vs = [], [], []
    for i in range(6):
        k, v = rnd(1, 2, 5, 16, seed=50 + i), rnd(1, 2, 5, 16, seed=60 + i)
        st, dev = ("GPU", "cuda") if i % 2 == 0 else ("CPU", "cpu")
        pages.append(page(k, v, i, 5 * i, st, dev))
        ks.append(k)
        vs.append(v)
    r = oa.streaming_attention(q, pages, query_device="cuda")
    # GPU block first, then CPU pages: softmax is order-free up to rounding
    exp = oa.eager(q, np.concatenate(ks, 2), np.concatenate(vs, 2))
    assert np.allclose(r, exp, atol=1e-5)


def test_eager_closed_form_vs_torch_sdpa_and_loops():
    g = np.random.default_rng(3)
    q, k, v = g.standard_normal((2, 8, 1, 32)), g.standard_normal((2, 2, 37, 32)), g.standard_normal((2, 2, 37, 32))
    e = oa.eager(q, k, v, 0.2)
    t = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q), torch.from_numpy(np.repeat(k, 4, 1)), torch.from_numpy(np.repeat(v, 4, 1)),
        scale=0.2).numpy()
    assert np.allclose(e, t, atol=1e-12)
    b, h = 1, 5                                             # brute force, GQA h -> h // 4
    s = np.array([np.dot(q[b, h, 0], k[b, h // 4, j]) * 0.2 for j in range(37)])
    p = np.exp(s - s.max())
    p /= p.sum()
    assert np.allclose(e[b, h, 0], (p[:, None] * v[b, h // 4]).sum(0), atol=1e-12)


def test_paged_reference_equals_eager_on_permuted_pool():
    g = np.random.default_rng(4)
    P, D = 16, 8
    kp, vp = g.standard_normal((10, 2, P, D)), g.standard_normal((10, 2, P, D))
    pt = np.array([[7, 2, 9, 0]], np.int32)
    q = g.standard_normal((1, 4, D))
    n = 3 * P + 5
    r = oa.paged_decode_reference(q, kp, vp, pt, np.array([n]), P, 0.3)
    k = np.concatenate([kp[s] for s in pt[0]], 1)[None, :, :n]
    v = np.concatenate([vp[s] for s in pt[0]], 1)[None, :, :n]
    assert np.allclose(r, oa.eager(q[:, :, None], k, v, 0.3)[:, :, 0], atol=1e-12)
    # a dropped term (one page missing) must be detected
    bad = oa.paged_decode_reference(q, kp, vp, pt, np.array([2 * P]), P, 0.3)
    assert not np.allclose(bad, r, atol=1e-3)


def test_causal_prefill_reference_vs_sdpa_and_rows():
    """q_start = 0: torch SDPA with is_causal (a library routine); q_start > 0:
    each query row equals the non-causal closed form over its visible keys."""
    import torch
    g = np.random.default_rng(8)
    T, Hq, Hkv, D = 9, 6, 2, 16
    q = g.standard_normal((T, Hq, D))
    k = g.standard_normal((T, Hkv, D))
    v = g.standard_normal((T, Hkv, D))
    out = oa.causal_prefill_reference(q, k, v, 0, 0.3)
    qt = torch.from_numpy(q).permute(1, 0, 2)[None]
    kt = torch.from_numpy(k).permute(1, 0, 2).repeat_interleave(Hq // Hkv, 0)[None]
    vt = torch.from_numpy(v).permute(1, 0, 2).repeat_interleave(Hq // Hkv, 0)[None]
    ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, is_causal=True, scale=0.3)
    np.testing.assert_allclose(out, ref[0].permute(1, 0, 2).numpy(), atol=1e-12)
    # with 5 earlier keys
    k2 = g.standard_normal((5 + T, Hkv, D))
    v2 = g.standard_normal((5 + T, Hkv, D))
    out2 = oa.causal_prefill_reference(q, k2, v2, 5, 0.3)
    for i in range(T):
        n = 5 + i + 1
        row = oa.eager(q[i].reshape(1, Hq, 1, D), k2[None, :n].transpose(0, 2, 1, 3),
                       v2[None, :n].transpose(0, 2, 1, 3), 0.3)
        np.testing.assert_allclose(out2[i], row[0, :, 0, :], atol=1e-12)
    # a slip (mask off by one) is caught
    bad = oa.causal_prefill_reference(q, k2, v2, 6, 0.3)
    assert np.abs(bad - out2).max() > 1e-3


def test_masked_prefill_reference_vs_sdpa_loops_and_causal():
    """masked_prefill_reference: torch SDPA with a boolean and an additive mask (a
    library routine, per-head masks, a fully masked row -> zeros), brute-force
    loops on a tiny case, and the causal form when handed the causal mask."""
    import torch
    g = np.random.default_rng(9)
    T, N, Hq, Hkv, D = 7, 11, 4, 2, 8
    q = g.standard_normal((T, Hq, D))
    k = g.standard_normal((N, Hkv, D))
    v = g.standard_normal((N, Hkv, D))
    qt = torch.from_numpy(q).permute(1, 0, 2)[None]
    kt = torch.from_numpy(k).permute(1, 0, 2).repeat_interleave(Hq // Hkv, 0)[None]
    vt = torch.from_numpy(v).permute(1, 0, 2).repeat_interleave(Hq // Hkv, 0)[None]
    boolm = g.random((Hq, T, N)) < 0.7
    boolm[:, :, 0] = True
    boolm[1, 3, :] = False                        # one row with no key at all
    add = np.where(g.random((1, T, N)) < 0.3, -65504.0, g.standard_normal((1, T, N)))
    for m in (boolm, add):
        out = oa.masked_prefill_reference(q, k, v, m, 0.4)
        ref = torch.nn.functional.scaled_dot_product_attention(
            qt, kt, vt, attn_mask=torch.from_numpy(m)[None], scale=0.4)
        np.testing.assert_allclose(out, ref[0].permute(1, 0, 2).numpy(), atol=1e-12)
    assert np.all(oa.masked_prefill_reference(q, k, v, boolm, 0.4)[3, 1] == 0)
    # brute force: explicit loops over heads, queries and keys
    out = oa.masked_prefill_reference(q, k, v, add, 0.4)
    for h in range(Hq):
        for t in range(T):
            w = [math.exp(0.4 * float(q[t, h] @ k[j, h // 2]) + add[0, t, j]) for j in range(N)]
            row = sum(w[j] * v[j, h // 2] for j in range(N)) / sum(w)
            np.testing.assert_allclose(out[t, h], row, atol=1e-9)
    # the causal mask reproduces the causal form; a transposed mask does not
    causal = np.tril(np.ones((T, T), bool))[None]
    kc, vc = k[:T], v[:T]
    np.testing.assert_allclose(oa.masked_prefill_reference(q, kc, vc, causal, 0.4),
                               oa.causal_prefill_reference(q, kc, vc, 0, 0.4), atol=1e-12)
    bad = oa.masked_prefill_reference(q, kc, vc, causal.transpose(0, 2, 1), 0.4)
    assert np.abs(bad - oa.causal_prefill_reference(q, kc, vc, 0, 0.4)).max() > 1e-3
