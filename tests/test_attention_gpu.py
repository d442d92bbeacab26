"""GPU parity of the paged GQA decode attention (split-K partials + reduce).

Bar: max |out - exact| <= 2e-3 (the task's attention tolerance), exact being
the fp64 closed form softmax(q K^T s) V over each item's pages in token order
(oracle.attention.paged_decode_reference, itself pinned against torch SDPA and
the reference's unit tests on the CPU).
"""
import math

import numpy as np
import pytest
import torch

from helm_amd.kernels import attention as ka
from oracle import attention as oa

pytestmark = pytest.mark.gpu
ATOL = 2e-3


def make_case(B, Hq, Hkv, D, P, seq_lens, seed, extra_slots=7):
    g = np.random.default_rng(seed)
    pages = [(n + P - 1) // P for n in seq_lens]
    max_pages = max(1, max(pages))
    n_slots = sum(pages) + extra_slots
    k_pool = g.standard_normal((n_slots, Hkv, P, D)).astype(np.float16)
    v_pool = g.standard_normal((n_slots, Hkv, P, D)).astype(np.float16)
    perm = g.permutation(n_slots).astype(np.int32)   # pages scattered over the pool
    pt = np.full((B, max_pages), -1, np.int32)
    c = 0
    for b, npg in enumerate(pages):
        pt[b, :npg] = perm[c:c + npg]
        c += npg
    q = g.standard_normal((B, Hq, D)).astype(np.float16)
    return q, k_pool, v_pool, pt, np.asarray(seq_lens, np.int32)


def device_pool(k_pool, v_pool):
    """Device pool of logical [slots, Hkv, P, D] numpy K/V; V stored token-contiguous."""
    dev = torch.device("cuda")
    k = torch.from_numpy(np.ascontiguousarray(k_pool)).to(dev)
    v = torch.from_numpy(np.ascontiguousarray(v_pool.transpose(0, 1, 3, 2))).to(dev).transpose(2, 3)
    return ka.PoolView.of_pool(k, v)


def run_gpu(q, k_pool, v_pool, pt, sl, P, scale, num_splits=None):
    dev = torch.device("cuda")
    qd = torch.from_numpy(q).to(dev)
    pool = device_pool(k_pool, v_pool)
    out = ka.paged_decode_attention(qd, pool, torch.from_numpy(pt).to(dev),
                                    torch.from_numpy(sl).to(dev), P, scale, num_splits=num_splits)
    return out.cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("Hq,Hkv,D,P", [(32, 8, 128, 16), (16, 8, 64, 16), (40, 8, 128, 16),
                                        (8, 8, 128, 32), (4, 1, 64, 64), (64, 8, 128, 16)])
@pytest.mark.parametrize("num_splits", [None, 1, 3])
def test_matches_exact_small(Hq, Hkv, D, P, num_splits):
    seq = [1, P - 1, P, P + 1, 5 * P + 3, 0, 37]
    B = len(seq)
    q, kp, vp, pt, sl = make_case(B, Hq, Hkv, D, P, seq, seed=Hq * 31 + D + P)
    scale = 1.0 / math.sqrt(D)
    out = run_gpu(q, kp, vp, pt, sl, P, scale, num_splits)
    ref = oa.paged_decode_reference(q, kp, vp, pt, sl, P, scale)
    assert np.abs(out - ref).max() <= ATOL
    assert (out[5] == 0).all()     # empty item -> zeros (kv_cache.py:353-354)


@pytest.mark.parametrize("ctx", [4096, 16384, 32768])
@pytest.mark.parametrize("B", [1, 8])
def test_qwen3_8b_decode_shapes(ctx, B):
    """32 q / 8 kv heads, D=128, P=16, fp16 N(0,1) Q/K/V, scale 1/sqrt(128)."""
    Hq, Hkv, D, P = 32, 8, 128, 16
    q, kp, vp, pt, sl = make_case(B, Hq, Hkv, D, P, [ctx] * B, seed=ctx + B)
    scale = 1.0 / math.sqrt(D)
    out = run_gpu(q, kp, vp, pt, sl, P, scale)
    items = range(B) if ctx <= 16384 else [0, B - 1]
    for b in items:   # fp64 reference per item
        ref = oa.paged_decode_reference(q[b:b + 1], kp, vp, pt[b:b + 1], sl[b:b + 1], P, scale)
        assert np.abs(out[b] - ref[0]).max() <= ATOL


def test_large_logits_stay_finite():
    """Reference test_large_logits_no_nan (test_streaming_attention.py:234-242) at decode shape."""
    Hq, Hkv, D, P = 8, 2, 64, 16
    B = 1
    q = np.full((B, Hq, D), 100.0, np.float16)
    kp = np.full((4, Hkv, P, D), 100.0, np.float16)
    vp = np.random.default_rng(0).standard_normal((4, Hkv, P, D)).astype(np.float16)
    pt = np.array([[2, 0, 3]], np.int32)
    sl = np.array([40], np.int32)
    out = run_gpu(q, kp, vp, pt, sl, P, 1.0 / math.sqrt(D))
    assert np.isfinite(out).all()
    ref = oa.paged_decode_reference(q, kp, vp, pt, sl, P, 1.0 / math.sqrt(D))
    assert np.abs(out - ref).max() <= ATOL


@pytest.mark.parametrize("P,width,num_splits", [(16, 401, 32), (16, 401, 7), (16, 333, 64),
                                                 (64, 101, 32), (32, 129, 9)])
def test_round_robin_splits_over_wide_tables(P, width, num_splits):
    """A page table much wider than the live lengths (as the decode engines round it
    for graph capture), odd widths (the last 32-token step of the table runs past
    it at P = 16) and split counts that do not divide the steps: the splits take the
    table's steps round robin, and the result is the one exact attention."""
    Hq, Hkv, D = 32, 8, 128
    seq = [min(width * P, 5000), 37, 1, 0, 700, width * P]
    B = len(seq)
    q, kp, vp, pt, sl = make_case(B, Hq, Hkv, D, P, seq, seed=P * 7 + width + num_splits)
    wide = np.full((B, width), -1, np.int32)
    wide[:, :pt.shape[1]] = pt
    # columns past an item's pages hold valid slots that must not be read as tokens
    g = np.random.default_rng(width)
    for b, n in enumerate(seq):
        used = (n + P - 1) // P
        wide[b, used:] = g.integers(0, kp.shape[0], width - used)
    scale = 1.0 / math.sqrt(D)
    out = run_gpu(q, kp, vp, wide, sl, P, scale, num_splits)
    ref = oa.paged_decode_reference(q, kp, vp, pt, sl, P, scale)
    assert np.abs(out - ref).max() <= ATOL
    assert (out[3] == 0).all()


def test_invalid_slots_are_skipped():
    """Page-table entries outside the pool contribute nothing (never dereferenced)."""
    Hq, Hkv, D, P = 8, 2, 128, 16
    q, kp, vp, pt, sl = make_case(1, Hq, Hkv, D, P, [64], seed=9)
    n_slots = kp.shape[0]
    bad = pt.copy()
    bad[0, 1] = -1
    bad[0, 2] = n_slots + 1000
    out = run_gpu(q, kp, vp, bad, sl, P, 0.1)
    # reference: only pages 0 and 3 (tokens 0-15 and 48-63)
    keep = [0, 3]
    k = np.concatenate([kp[pt[0, i]] for i in keep], axis=1)[None]
    v = np.concatenate([vp[pt[0, i]] for i in keep], axis=1)[None]
    ref = oa.eager(q[:, :, None, :], k, v, 0.1)[:, :, 0, :]
    assert np.abs(out - ref).max() <= ATOL


def test_split_ranges_compose():
    """Two launches writing disjoint split ranges + one reduce == one launch."""
    Hq, Hkv, D, P = 32, 8, 128, 16
    q, kp, vp, pt, sl = make_case(2, Hq, Hkv, D, P, [300, 513], seed=12)
    dev = torch.device("cuda")
    qd = torch.from_numpy(q).to(dev)
    pool = device_pool(kp, vp)
    ptd = torch.from_numpy(pt).to(dev)
    # first launch: first 10 pages of every item; second: the rest (as a shifted table)
    first = torch.from_numpy(np.minimum(sl, 10 * P).astype(np.int32)).to(dev)
    rest_pt = torch.from_numpy(np.ascontiguousarray(pt[:, 10:])).to(dev)
    rest_sl = torch.from_numpy(np.maximum(sl - 10 * P, 0).astype(np.int32)).to(dev)
    total = 5 + 4
    ws = ka.AttnWorkspace(dev)
    po, pml = ws.get(2, Hq, D, total)
    ka.paged_decode_attention_partial(qd, pool, ptd, first, P, 0.088, po, pml, 5, 0, total)
    ka.paged_decode_attention_partial(qd, pool, rest_pt, rest_sl, P, 0.088, po, pml, 4, 5, total)
    out = torch.empty(2, Hq, D, dtype=torch.float16, device=dev)
    ka.paged_attn_reduce(po, pml, out, total)
    ref = oa.paged_decode_reference(q, kp, vp, pt, sl, P, 0.088)
    assert np.abs(out.cpu().numpy().astype(np.float64) - ref).max() <= ATOL


def test_contiguous_buffer_view():
    """A contiguous [1, Hkv, cap, D] buffer (the reference's Path 1 storage) is read
    through an identity page table."""
    Hq, Hkv, D, P, cap, n = 16, 8, 64, 16, 256, 200
    g = np.random.default_rng(3)
    kb = g.standard_normal((1, Hkv, cap, D)).astype(np.float16)
    vb = g.standard_normal((1, Hkv, cap, D)).astype(np.float16)
    q = g.standard_normal((1, Hq, D)).astype(np.float16)
    dev = torch.device("cuda")
    kd, vd = ka.alloc_sequences(1, Hkv, cap, D, torch.float16, dev)
    kd.copy_(torch.from_numpy(kb))
    vd.copy_(torch.from_numpy(vb))
    pool = ka.PoolView.of_sequences(kd, vd, P)
    pt = torch.arange(cap // P, dtype=torch.int32, device=dev)[None]
    out = ka.paged_decode_attention(torch.from_numpy(q).to(dev), pool, pt,
                                    torch.tensor([n], dtype=torch.int32, device=dev), P, 0.125)
    ref = oa.eager(q[:, :, None, :], kb[:, :, :n], vb[:, :, :n], 0.125)[:, :, 0, :]
    assert np.abs(out.cpu().numpy().astype(np.float64) - ref).max() <= ATOL


def test_kv_append_writes_slots():
    Hkv, D, P = 8, 128, 16
    dev = torch.device("cuda")
    kp = torch.zeros(10, Hkv, P, D, dtype=torch.float16, device=dev)
    vp = ka.alloc_v((10, Hkv, P, D), device=dev, zero=True)
    pool = ka.PoolView.of_pool(kp, vp)
    kn = torch.randn(3, Hkv, 2, D, dtype=torch.float16, device=dev)
    vn = torch.randn(3, Hkv, 2, D, dtype=torch.float16, device=dev)
    slots = torch.tensor([4, 0, 9], dtype=torch.int32, device=dev)
    offs = torch.tensor([0, 14, 7], dtype=torch.int32, device=dev)
    ka.kv_append(kn, vn, pool, slots, offs, P)
    for b, (s, o) in enumerate(zip([4, 0, 9], [0, 14, 7])):
        assert torch.equal(kp[s, :, o:o + 2], kn[b])
        assert torch.equal(vp[s, :, o:o + 2], vn[b])
    assert int((kp != 0).sum()) == kn.numel()   # nothing else written


def test_unwritten_slots_holding_nan_are_ignored():
    """Tokens past seq_len in the last page are unwritten memory (possibly NaN/Inf
    bit patterns in a fresh pool); they must not reach the output."""
    Hq, Hkv, D, P = 32, 8, 128, 16
    for n in (5, 16 * 3 + 1, 16 * 4 - 1):
        q, kp, vp, pt, sl = make_case(1, Hq, Hkv, D, P, [n], seed=n)
        last = pt[0, (n - 1) // P]
        kbad, vbad = kp.copy(), vp.copy()
        kbad[last, :, n % P or P:] = np.inf
        vbad[last, :, n % P or P:] = np.nan
        out = run_gpu(q, kbad, vbad, pt, sl, P, 1.0 / math.sqrt(D))
        ref = oa.paged_decode_reference(q, kp, vp, pt, sl, P, 1.0 / math.sqrt(D))
        assert np.isfinite(out).all()
        assert np.abs(out - ref).max() <= ATOL


def _fused_case(B, Hq, Hkv, D, P, seq_lens, seed):
    """Pool with the cached tokens of every item plus a free slot position for the
    new token (the last token of seq_lens[b]); raw fused projection output qkv."""
    from helm_amd.kernels import fused
    g = np.random.default_rng(seed)
    q, kp, vp, pt, sl = make_case(B, Hq, Hkv, D, P, seq_lens, seed)
    qkv = (g.standard_normal((B, (Hq + 2 * Hkv) * D)) * 2).astype(np.float16)
    qn = (1 + 0.1 * g.standard_normal(D)).astype(np.float16)
    kn = (1 + 0.1 * g.standard_normal(D)).astype(np.float16)
    pos = (sl - 1).astype(np.int32) + 7          # RoPE position need not equal the index
    slots = np.array([pt[b, (n - 1) // P] for b, n in enumerate(sl)], np.int32)
    offs = ((sl - 1) % P).astype(np.int32)
    dev = torch.device("cuda")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    inv = fused.rope_inv_freq(D, 1e6, dev)
    return dict(qkv=t(qkv), qn=t(qn), kn=t(kn), pos=t(pos), slots=t(slots), offs=t(offs),
                pt=t(pt), sl=t(sl), inv=inv, kp=kp, vp=vp)


@pytest.mark.parametrize("Hq,Hkv,D,P,seq", [(32, 8, 128, 16, [1000, 37]), (16, 8, 64, 16, [5, 300]),
                                            (40, 8, 128, 32, [4097]), (64, 8, 128, 16, [1, 2000]),
                                            (4, 1, 64, 64, [129])])
@pytest.mark.parametrize("num_splits", [None, 1])
def test_fused_decode_attention_equals_three_kernels(Hq, Hkv, D, P, seq, num_splits):
    """helm_decode_attn_fused (norm + RoPE + KV write + attention partials) + reduce
    against helm_qk_norm_rope_append + helm_paged_decode_attn + reduce."""
    import ctypes
    from helm_amd import _native
    from helm_amd.kernels import fused
    B = len(seq)
    c = _fused_case(B, Hq, Hkv, D, P, seq, seed=D + P + len(seq))
    dev = torch.device("cuda")
    scale = 1.0 / math.sqrt(D)
    # three-kernel path
    pool3 = device_pool(c["kp"], c["vp"])
    q3 = torch.empty(B, Hq, D, dtype=torch.float16, device=dev)
    fused.qk_norm_rope_append(c["qkv"], c["qn"], c["kn"], 1e-6, c["pos"], c["inv"], q3, pool3,
                              c["slots"], c["offs"], Hq, Hkv, D, P)
    out3 = ka.paged_decode_attention(q3, pool3, c["pt"], c["sl"], P, scale, num_splits=num_splits)
    # fused
    poolf = device_pool(c["kp"], c["vp"])
    S = num_splits or ka.choose_num_splits(B, Hkv, c["pt"].shape[1], P)
    ws = ka.AttnWorkspace(dev)
    po, pml = ws.get(B, Hq, D, S)
    outf = torch.empty(B, Hq, D, dtype=torch.float16, device=dev)
    for rep in range(2):   # a repeat writes the same K/V again and gives the same output
        _native.call("helm_decode_attn_fused", c["qkv"].data_ptr(), c["qkv"].stride(0),
                     c["qn"].data_ptr(), c["kn"].data_ptr(), 1e-6, c["pos"].data_ptr(),
                     c["inv"].data_ptr(), c["slots"].data_ptr(), c["offs"].data_ptr(),
                     poolf.c_ref(), c["pt"].data_ptr(), c["pt"].stride(0), c["sl"].data_ptr(),
                     po.data_ptr(), pml.data_ptr(), B, Hq, Hkv, D, P, c["pt"].shape[1], S, scale,
                     _native.stream_ptr(dev))
        ka.paged_attn_reduce(po, pml, outf, S)
        torch.cuda.synchronize()
        # the new token's K/V land in the pool exactly as the three-kernel path writes them
        assert torch.equal(poolf.k, pool3.k) and torch.equal(poolf.v, pool3.v)
        err = (outf.float() - out3.float()).abs().max().item()
        assert err <= ATOL, f"fused vs three-kernel max err {err}"
    # and both against the fp64 closed form over the updated pool
    ref = oa.paged_decode_reference(q3.cpu().numpy(), pool3.k.cpu().numpy(),
                                    pool3.v.cpu().numpy(), c["pt"].cpu().numpy(),
                                    c["sl"].cpu().numpy(), P, scale)
    assert np.abs(outf.cpu().numpy().astype(np.float64) - ref).max() <= ATOL


@pytest.mark.parametrize("Hq,Hkv,D,P,seq", [(32, 8, 128, 16, [1000, 37]), (16, 8, 64, 16, [5, 300]),
                                            (40, 8, 128, 32, [4097]), (64, 8, 128, 16, [1, 2000]),
                                            (4, 1, 64, 64, [129])])
@pytest.mark.parametrize("norms", [True, False], ids=["qk_norm", "no_norm"])
def test_fused_cs_attention_equals_norm_rope_append_attention(Hq, Hkv, D, P, seq, norms):
    """helm_decode_attn_fused_cs (the drop-in decode's one launch: optional q / k
    norm, RoPE from the model's own fp16 cos / sin rows, K/V write, partials) +
    reduce against helm_qk_norm_rope_cs + helm_kv_append + helm_paged_decode_attn
    + reduce: the same pool bytes (the same roundings of q, k in the same order),
    the outputs within the bar (the new token is folded into the last split's
    state instead of being read back from the pool, so the fp32 sums run in
    another order); and against the fp64 closed form over the updated pool.
    The cos / sin rows are not a pure RoPE table (the second half differs from
    the first), so a kernel that read only half a row would fail."""
    from helm_amd.kernels import fused
    B = len(seq)
    c = _fused_case(B, Hq, Hkv, D, P, seq, seed=3 * D + P + len(seq))
    dev = torch.device("cuda")
    g = np.random.default_rng(D + B)
    cos = torch.from_numpy(g.uniform(-1, 1, (B, D)).astype(np.float16)).to(dev)
    sin = torch.from_numpy(g.uniform(-1, 1, (B, D)).astype(np.float16)).to(dev)
    qn, kn = (c["qn"], c["kn"]) if norms else (None, None)
    scale = 1.0 / math.sqrt(D)
    S = ka.choose_num_splits(B, Hkv, c["pt"].shape[1], P)
    ws = ka.AttnWorkspace(dev)
    po, pml = ws.get(B, Hq, D, S)
    # three-kernel path
    pool3 = device_pool(c["kp"], c["vp"])
    q3, k3 = fused.qk_norm_rope_cs(c["qkv"], qn, kn, 1e-6, cos, sin, Hq, Hkv, D)
    v3 = c["qkv"][:, (Hq + Hkv) * D:].view(B, Hkv, 1, D)
    ka.kv_append(k3.view(B, Hkv, 1, D), v3, pool3, c["slots"], c["offs"], P)
    ka.paged_decode_attention_partial(q3, pool3, c["pt"], c["sl"], P, scale, po, pml, S)
    out3 = torch.empty(B, Hq, D, dtype=torch.float16, device=dev)
    ka.paged_attn_reduce(po, pml, out3, S)
    # one launch
    poolf = device_pool(c["kp"], c["vp"])
    outf = torch.empty(B, Hq, D, dtype=torch.float16, device=dev)
    for rep in range(2):   # a repeat writes the same K/V again and gives the same output
        ka.decode_attention_fused_cs(c["qkv"], qn, kn, 1e-6, cos, sin, poolf, c["slots"], c["offs"],
                                     c["pt"], c["sl"], P, scale, po, pml, S, Hq, Hkv, D)
        ka.paged_attn_reduce(po, pml, outf, S)
        torch.cuda.synchronize()
        assert torch.equal(poolf.k, pool3.k) and torch.equal(poolf.v, pool3.v)
        err = (outf.float() - out3.float()).abs().max().item()
        assert err <= ATOL, f"fused (cos / sin rows) vs three-kernel max err {err}"
    ref = oa.paged_decode_reference(q3.cpu().numpy(), pool3.k.cpu().numpy(),
                                    pool3.v.cpu().numpy(), c["pt"].cpu().numpy(),
                                    c["sl"].cpu().numpy(), P, scale)
    assert np.abs(outf.cpu().numpy().astype(np.float64) - ref).max() <= ATOL


@pytest.mark.parametrize("Hq,Hkv,D,P,T,q_start", [(32, 8, 128, 16, 300, 0), (40, 8, 128, 16, 257, 0),
                                                  (16, 8, 64, 32, 100, 0), (4, 1, 64, 64, 70, 0),
                                                  (32, 8, 128, 16, 77, 45), (8, 2, 128, 16, 1, 0),
                                                  (8, 8, 64, 16, 33, 16), (16, 1, 128, 32, 200, 10)])
def test_prefill_attention_matches_causal_reference(Hq, Hkv, D, P, T, q_start):
    """helm_prefill_attn: query i (position q_start + i) over keys 0..q_start+i of
    scattered pages, against the fp64 causal form (bar 2e-3)."""
    g = np.random.default_rng(T + q_start + D)
    N = q_start + T
    n_pages = (N + P - 1) // P
    n_slots = n_pages + 5
    k_all = g.standard_normal((N, Hkv, D)).astype(np.float16)
    v_all = g.standard_normal((N, Hkv, D)).astype(np.float16)
    kp = g.standard_normal((n_slots, Hkv, P, D)).astype(np.float16)   # garbage elsewhere
    vp = np.full((n_slots, Hkv, P, D), np.nan, np.float16)            # unwritten slots hold NaN
    pt = g.permutation(n_slots)[:n_pages].astype(np.int32)
    for t in range(N):
        kp[pt[t // P], :, t % P] = k_all[t]
        vp[pt[t // P], :, t % P] = v_all[t]
    q = g.standard_normal((T, Hq, D)).astype(np.float16)
    scale = 1.0 / math.sqrt(D)
    dev = torch.device("cuda")
    out = ka.prefill_attention(torch.from_numpy(q).to(dev), device_pool(kp, vp),
                               torch.from_numpy(pt).to(dev), P, q_start, scale)
    ref = oa.causal_prefill_reference(q, k_all, v_all, q_start, scale)
    got = out.cpu().numpy().astype(np.float64)
    assert np.isfinite(got).all()
    assert np.abs(got - ref).max() <= ATOL


def _mask_case(kind, Hq, T, N, g):
    """Masks of the shapes a drop-in prefill receives: [Hm, T, N]."""
    causal = np.arange(N)[None, :] <= np.arange(T)[:, None] + (N - T)
    if kind == "left_pad":          # HF padding mask: causal and not a pad key; pad rows see nothing
        keep = causal & (np.arange(N)[None, :] >= 37)
        return keep[None]
    if kind == "hf_min":            # additive, large negative (fp16 min) above the diagonal and on
        noise = np.where(g.random((T, N)) < 0.5, g.standard_normal((T, N)), 0.0)
        add = np.where(causal, noise, -65504.0)  # and on every key of rows 0..4
        add[:5] = -65504.0
        return add.astype(np.float16)[None]
    if kind == "per_head":          # one boolean mask per query head, non-causal
        m = g.random((Hq, T, N)) < 0.6
        m[:, :, 3] = True
        return m
    if kind == "full":              # bidirectional
        return np.ones((1, T, N), bool)
    raise ValueError(kind)


@pytest.mark.parametrize("Hq,Hkv,D,P,T,N,kind", [(32, 8, 128, 16, 300, 300, "left_pad"),
                                                 (40, 8, 128, 16, 257, 257, "hf_min"),
                                                 (16, 8, 64, 32, 100, 130, "per_head"),
                                                 (4, 1, 64, 64, 70, 70, "full"),
                                                 (8, 2, 128, 16, 1, 45, "per_head"),
                                                 (32, 8, 128, 16, 129, 2049, "hf_min"),
                                                 (40, 8, 128, 16, 700, 700, "left_pad")])
@pytest.mark.parametrize("key_ranges", [True, False])
def test_prefill_attention_mask_matches_reference(Hq, Hkv, D, P, T, N, kind, key_ranges):
    """helm_prefill_attn_mask: T queries over N keys of scattered pages with an
    additive / boolean mask (per head or broadcast), against the fp64 masked
    form (bar 2e-3); fully masked rows give zeros.  With the per-row key ranges
    (steps no row of a workgroup sees are skipped) and without."""
    g = np.random.default_rng(T + N + D)
    n_pages = (N + P - 1) // P
    n_slots = n_pages + 5
    k_all = g.standard_normal((N, Hkv, D)).astype(np.float16)
    v_all = g.standard_normal((N, Hkv, D)).astype(np.float16)
    kp = g.standard_normal((n_slots, Hkv, P, D)).astype(np.float16)
    vp = np.full((n_slots, Hkv, P, D), np.nan, np.float16)            # unwritten slots hold NaN
    pt = g.permutation(n_slots)[:n_pages].astype(np.int32)
    for t in range(N):
        kp[pt[t // P], :, t % P] = k_all[t]
        vp[pt[t // P], :, t % P] = v_all[t]
    q = g.standard_normal((T, Hq, D)).astype(np.float16)
    mask = _mask_case(kind, Hq, T, N, g)
    scale = 1.0 / math.sqrt(D)
    dev = torch.device("cuda")
    print(f"[prefill mask] {kind} Hq={Hq} D={D} P={P} T={T} N={N} ranges={key_ranges}", flush=True)
    out = ka.prefill_attention(torch.from_numpy(q).to(dev), device_pool(kp, vp),
                               torch.from_numpy(pt).to(dev), P, 0, scale,
                               mask=torch.from_numpy(mask).to(dev), key_ranges=key_ranges)
    ref = oa.masked_prefill_reference(q, k_all, v_all, mask, scale)
    got = out.cpu().numpy().astype(np.float64)
    assert np.isfinite(got).all()
    assert np.abs(got - ref).max() <= ATOL
    if kind == "left_pad":
        assert np.all(got[:37] == 0)


def test_prefill_attention_mask_rejects_bad_shapes():
    dev = torch.device("cuda")
    kp = np.zeros((4, 2, 16, 64), np.float16)
    pool = device_pool(kp, kp)
    pt = torch.arange(4, dtype=torch.int32, device=dev)
    q = torch.zeros(10, 4, 64, dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match="mask must be"):
        ka.prefill_attention(q, pool, pt, 16, mask=torch.ones(2, 10, 10, dtype=torch.bool, device=dev))
    with pytest.raises(RuntimeError, match="q_start must be 0"):
        ka.prefill_attention(q, pool, pt, 16, q_start=3,
                             mask=torch.ones(1, 10, 13, dtype=torch.bool, device=dev))
    with pytest.raises(RuntimeError, match="does not cover"):
        ka.prefill_attention(q, pool, pt, 16, mask=torch.ones(1, 10, 65, dtype=torch.bool, device=dev))


def test_dense_prefill_kv_view_matches_reference():
    """The engine's prefill path: prompt K/V copied into page layout, identity table."""
    g = np.random.default_rng(4)
    S, Hq, Hkv, D = 130, 32, 8, 128
    q = g.standard_normal((S, Hq, D)).astype(np.float16)
    k = g.standard_normal((S, Hkv, D)).astype(np.float16)
    v = g.standard_normal((S, Hkv, D)).astype(np.float16)
    dev = torch.device("cuda")
    pool, pt = ka.dense_prefill_kv(torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev), 16)
    out = ka.prefill_attention(torch.from_numpy(q).to(dev), pool, pt, 16, 0, 0.088)
    ref = oa.causal_prefill_reference(q, k, v, 0, 0.088)
    assert np.abs(out.cpu().numpy().astype(np.float64) - ref).max() <= ATOL


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("S", [1, 4, 8, 9, 16, 17, 32, 33, 64, 65, 100])
def test_split_reduce_merges_to_full_softmax(D, S):
    """helm_paged_attn_reduce over S split partials of one sequence equals the
    fp64 softmax attention over the whole sequence (covers every block width of
    the register form and the chunked form past it).  Each split's partial is
    built here from its own token segment, in the kernel's format: o normalised,
    (max of scale*log2(e)*s, sum of exp2(. - max)); empty segments carry
    (-inf, 0) and o = 0, as the partial kernel writes them."""
    B, Hq = 2, 4
    g = np.random.default_rng(1000 * D + S)
    lens = g.integers(0, 24, size=S)
    lens[g.integers(0, S)] += 1                       # at least one token
    if S > 2:
        lens[g.choice(S, size=max(1, S // 4), replace=False)] = 0   # empty splits
        lens[int(np.argmax(lens))] += 1
    T = int(lens.sum())
    q = g.standard_normal((B, Hq, 1, D))
    k = g.standard_normal((B, Hq, T, D))
    v = g.standard_normal((B, Hq, T, D))
    scale = 1.0 / math.sqrt(D)
    c = scale * math.log2(math.e)
    part_o = np.zeros((B, Hq, S, D), np.float32)
    part_ml = np.zeros((B, Hq, S, 2), np.float32)
    part_ml[..., 0] = -np.inf
    t0 = 0
    for s_i, n in enumerate(lens):
        if n:
            sc = np.einsum("bhd,bhtd->bht", q[:, :, 0], k[:, :, t0:t0 + n]) * c
            m = sc.max(-1, keepdims=True)
            p = np.exp2(sc - m)
            part_o[:, :, s_i] = np.einsum("bht,bhtd->bhd", p, v[:, :, t0:t0 + n]) / p.sum(-1, keepdims=True)
            part_ml[:, :, s_i, 0] = m[..., 0]
            part_ml[:, :, s_i, 1] = p.sum(-1)
        t0 += n
    ref = oa.eager(q, k, v, scale)[:, :, 0]
    dev = torch.device("cuda")
    out = torch.empty((B, Hq, D), dtype=torch.float16, device=dev)
    ka.paged_attn_reduce(torch.from_numpy(part_o).to(dev).view(-1), torch.from_numpy(part_ml).to(dev).view(-1),
                         out, S)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    err = float(np.abs(got - ref).max())
    assert err <= ATOL, f"D={D} S={S}: max err {err}"


def test_qk_norm_rope_append_matches_closed_form():
    """helm_qk_norm_rope_append against the closed form of Qwen3's q/k RMSNorm
    (x * rsqrt(mean(x^2) + eps) * w over head_dim) and rotate-half RoPE at the
    angle fp32(inv_freq * position) (transformers computes the angles in fp32),
    in fp64, and against the same ops run by torch in fp16 on the GPU
    (transformers' Qwen3RMSNorm and apply_rotary_pos_emb arithmetic): q_out and
    the K/V written into the pages.  Positions up to 16383 (large angles)."""
    from helm_amd.kernels import fused
    B, Hq, Hkv, D, P, eps, theta = 4, 32, 8, 128, 16, 1e-6, 1e6
    g = np.random.default_rng(99)
    qkv = (g.standard_normal((B, (Hq + 2 * Hkv) * D)) * 3).astype(np.float16)
    qn = (1 + 0.2 * g.standard_normal(D)).astype(np.float16)
    kn = (1 + 0.2 * g.standard_normal(D)).astype(np.float16)
    pos = np.array([0, 7, 4096, 16383], np.int32)
    n_slots = 6
    slots = np.array([5, 0, 3, 1], np.int32)
    offs = np.array([0, 15, 7, 3], np.int32)
    dev = torch.device("cuda")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    kp = np.zeros((n_slots, Hkv, P, D), np.float16)
    pool = device_pool(kp, kp)
    inv = fused.rope_inv_freq(D, theta, dev)
    q_out = torch.empty(B, Hq, D, dtype=torch.float16, device=dev)
    fused.qk_norm_rope_append(t(qkv), t(qn), t(kn), eps, t(pos), inv, q_out, pool, t(slots),
                              t(offs), Hq, Hkv, D, P)
    torch.cuda.synchronize()
    k_pool, v_pool = pool.k.cpu().numpy(), pool.v.cpu().numpy()
    got_q = q_out.cpu().numpy().astype(np.float64)
    got_k = np.stack([k_pool[slots[b], :, offs[b]] for b in range(B)]).astype(np.float64)
    got_v = np.stack([v_pool[slots[b], :, offs[b]] for b in range(B)])
    x = qkv.astype(np.float64)
    q_in = x[:, :Hq * D].reshape(B, Hq, D)
    k_in = x[:, Hq * D:(Hq + Hkv) * D].reshape(B, Hkv, D)
    v_in = qkv[:, (Hq + Hkv) * D:].reshape(B, Hkv, D)
    # angles as fp32 products (the reference's fp32 frequency computation)
    ang = (inv.cpu().numpy()[None, :] * pos.astype(np.float32)[:, None]).astype(np.float32)
    emb = np.concatenate([ang, ang], -1).astype(np.float64)[:, None, :]
    cos, sin = np.cos(emb), np.sin(emb)

    def closed(xh, w):
        xn = xh / np.sqrt((xh * xh).mean(-1, keepdims=True) + eps) * w.astype(np.float64)
        rot = np.concatenate([-xn[..., D // 2:], xn[..., :D // 2]], -1)
        return xn * cos + rot * sin, np.abs(xn * cos) + np.abs(rot * sin)
    (ref_q, terms_q), (ref_k, terms_k) = closed(q_in, qn), closed(k_in, kn)

    # torch fp16 ops as transformers runs them on an fp16 model
    def torch16(xh, w):
        xt = torch.from_numpy(xh.astype(np.float16)).to(dev)
        x32 = xt.float()
        xn = torch.from_numpy(w).to(dev) * (x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + eps)).half()
        c = torch.from_numpy(np.cos(emb.astype(np.float32))).to(dev).half()
        s = torch.from_numpy(np.sin(emb.astype(np.float32))).to(dev).half()
        rot = torch.cat([-xn[..., D // 2:], xn[..., :D // 2]], -1)
        return (xn * c + rot * s).cpu().numpy().astype(np.float64)
    t_q, t_k = torch16(q_in, qn), torch16(k_in, kn)
    for got, ref, terms, tt, what in ((got_q, ref_q, terms_q, t_q, "q"),
                                      (got_k, ref_k, terms_k, t_k, "k")):
        # fp16 arithmetic of the reference: two roundings in the norm, cos/sin,
        # two products and their sum: a few units in the last place of the terms
        bound = 4 * 2.0 ** -11 * (terms + 1.0)
        assert (np.abs(got - ref) <= bound).all(), f"{what}: {np.abs(got - ref).max()}"
        # against torch's fp16 ops: the fp32 sums of squares (reduction order) and
        # the fp32 cos / sin may land a normalised value or a factor on the other
        # neighbouring fp16 value, i.e. one unit in the last place of each product
        # term, plus one of the sum
        mag = np.maximum(np.maximum(np.abs(tt), np.abs(got)), 2.0 ** -14)
        ulp = 2.0 ** (np.floor(np.log2(mag)) - 10)
        tb = 2.0 ** -10 * terms + ulp
        bad = np.abs(got - tt) > tb
        assert not bad.any(), (f"{what} vs torch fp16 at {np.argwhere(bad)[:4].tolist()}: "
                               f"kernel {got[bad][:4]}, torch {tt[bad][:4]}, fp64 {ref[bad][:4]}")
    np.testing.assert_array_equal(got_v, v_in)    # v is written unchanged


@pytest.mark.parametrize("norm,shared_rows,rope_scaling", [(True, False, None), (False, False, None),
                                                            (True, True, None),
                                                            (True, False, {"rope_type": "yarn", "factor": 4.0,
                                                                           "original_max_position_embeddings": 10240})])
def test_qk_norm_rope_cs_matches_transformers_ops(norm, shared_rows, rope_scaling):
    """helm_qk_norm_rope_cs against the ops it replaces in the drop-in decode:
    transformers' Qwen3RMSNorm on q and k (when the model has q / k norms), then
    apply_rotary_pos_emb with the cos / sin of the model's rotary embedding (any
    RoPE scaling it configures), all in fp16 on the GPU.  Equal to within one fp16
    ulp per element (the RMS sum's order differs), almost all bit-equal."""
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import (Qwen3RMSNorm, Qwen3RotaryEmbedding,
                                                          apply_rotary_pos_emb)
    from helm_amd.kernels import fused
    B, Hq, Hkv, D, eps = 4, 32, 8, 128, 1e-6
    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(7)
    qkv = (torch.randn(B, (Hq + 2 * Hkv) * D, generator=g) * 3).half().to(dev)
    cfg = Qwen3Config(hidden_size=Hq * D, num_attention_heads=Hq, num_key_value_heads=Hkv,
                      head_dim=D, rope_theta=1e6, max_position_embeddings=40960,
                      rope_scaling=rope_scaling)
    rot = Qwen3RotaryEmbedding(cfg).to(dev)
    pos = torch.tensor([[16383]] if shared_rows else [[0], [7], [4096], [16383]], device=dev)
    cos, sin = rot(qkv.view(B, 1, -1)[:pos.shape[0]], pos)     # [B or 1, 1, D] fp16
    q_in = qkv[:, :Hq * D].view(B, 1, Hq, D)
    k_in = qkv[:, Hq * D:(Hq + Hkv) * D].view(B, 1, Hkv, D)
    qn = kn = None
    if norm:
        qn_mod, kn_mod = Qwen3RMSNorm(D, eps).to(dev).half(), Qwen3RMSNorm(D, eps).to(dev).half()
        with torch.no_grad():
            qn_mod.weight.copy_(1 + 0.2 * torch.randn(D, generator=g))
            kn_mod.weight.copy_(1 + 0.2 * torch.randn(D, generator=g))
            q_in, k_in = qn_mod(q_in), kn_mod(k_in)
        qn, kn = qn_mod.weight.detach(), kn_mod.weight.detach()
    ref_q, ref_k = apply_rotary_pos_emb(q_in.transpose(1, 2), k_in.transpose(1, 2), cos, sin)
    c2, s2 = cos.reshape(cos.shape[0], D).expand(B, D), sin.reshape(sin.shape[0], D).expand(B, D)
    q, k = fused.qk_norm_rope_cs(qkv, qn, kn, eps, c2, s2, Hq, Hkv, D)
    torch.cuda.synchronize()
    cf, sf = c2.float().cpu().numpy()[:, None, :], s2.float().cpu().numpy()[:, None, :]
    for got, ref, xn in ((q, ref_q[:, :, 0], q_in[:, 0]), (k, ref_k[:, :, 0], k_in[:, 0])):
        g64 = got.float().cpu().numpy().astype(np.float64)
        r64 = ref.float().cpu().numpy().astype(np.float64)
        if not norm:   # same values, same fp16 operations: bit-equal
            np.testing.assert_array_equal(g64, r64)
            continue
        # the fp32 sum of squares in another order can put a normalised value on the
        # neighbouring fp16 value: one unit in the last place of each product term,
        # plus one of the sum
        x = xn.float().cpu().numpy().astype(np.float64)
        rot = np.concatenate([-x[..., D // 2:], x[..., :D // 2]], -1)
        terms = np.abs(x * cf) + np.abs(rot * sf)
        mag = np.maximum(np.maximum(np.abs(g64), np.abs(r64)), 2.0 ** -14)
        bound = 2.0 ** -10 * terms + 2.0 ** (np.floor(np.log2(mag)) - 10)
        assert (np.abs(g64 - r64) <= bound).all(), float(np.abs(g64 - r64).max())
        assert (g64 == r64).mean() > 0.99
