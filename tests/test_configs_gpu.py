"""GPU parity at the benchmark configurations' full sizes.

  * Qwen3-14B causal prefill attention: T = 2048 prompt tokens, 40 q / 8 kv heads,
    D = 128, pages of 16 scattered over a pool, against the fp64 causal form on
    sampled query rows (the last 32 and 32 spread over the prompt); bar 2e-3.
  * Qwen3-8B paged decode attention with the oldest 50% of pages on the host:
    perform_streaming_attention at 16K and 32K context, and one batch-8 decode
    step at 16K through KVOffloadManager's dispatch (kv_offload.py:82-167), each
    item against the fp64 form over its own tokens; bar 2e-3.
  * Qwen3-32B shape end to end (64 layers, hidden 5120, 64/8 heads, FFN 25600,
    vocab 151936, ~32 GB of INT8 linears): graph replay bit-identical to eager
    execution at 16K context; the step with every page resident and with the
    oldest 50% of pages on the host at 16K and 32K, both against a plain-torch
    fp32 step of the full model over the same KV, and the offloaded step's last
    layer attention against fp64; a real 1024-token prefill and the same tokens
    decoded one at a time, both against the torch fp32 forward; and a 2-layer
    model of this shape teacher-forced against the fp32 oracle.
"""
import math

import numpy as np
import pytest
import torch

from helm_amd.kernels import attention as ka
from helm_amd.runtime import KVAllocator, KVCacheManager, perform_streaming_attention
from oracle import attention as oa

pytestmark = pytest.mark.gpu
ATOL = 2e-3
GPU = torch.device("cuda")


def _pool(kp, vp):
    k = torch.from_numpy(np.ascontiguousarray(kp)).to(GPU)
    v = torch.from_numpy(np.ascontiguousarray(vp.transpose(0, 1, 3, 2))).to(GPU).transpose(2, 3)
    return ka.PoolView.of_pool(k, v)


def test_prefill_attention_qwen3_14b_t2048():
    T, Hq, Hkv, D, P = 2048, 40, 8, 128, 16
    g = np.random.default_rng(2048)
    n_pages = T // P
    n_slots = n_pages + 37
    k_all = g.standard_normal((T, Hkv, D)).astype(np.float16)
    v_all = g.standard_normal((T, Hkv, D)).astype(np.float16)
    kp = g.standard_normal((n_slots, Hkv, P, D)).astype(np.float16)
    vp = g.standard_normal((n_slots, Hkv, P, D)).astype(np.float16)
    pt = g.permutation(n_slots)[:n_pages].astype(np.int32)
    kp[pt] = k_all.reshape(n_pages, P, Hkv, D).transpose(0, 2, 1, 3)
    vp[pt] = v_all.reshape(n_pages, P, Hkv, D).transpose(0, 2, 1, 3)
    q = g.standard_normal((T, Hq, D)).astype(np.float16)
    scale = 1.0 / math.sqrt(D)
    out = ka.prefill_attention(torch.from_numpy(q).to(GPU), _pool(kp, vp),
                               torch.from_numpy(pt).to(GPU), P, 0, scale)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    # the last 32 queries (the longest rows) as one block
    last = T - 32
    ref = oa.causal_prefill_reference(q[last:], k_all, v_all, last, scale)
    assert np.abs(got[last:] - ref).max() <= ATOL
    # 32 rows spread over the prompt, one at a time (q_start = the row)
    for i in sorted(g.choice(last, size=32, replace=False)):
        ref = oa.causal_prefill_reference(q[i:i + 1], k_all[:i + 1], v_all[:i + 1], i, scale)
        err = float(np.abs(got[i:i + 1] - ref).max())
        assert err <= ATOL, f"row {i}: {err}"


@pytest.mark.parametrize("ctx", [16384, 32768])
def test_streaming_attention_half_on_host_qwen3_8b(ctx):
    """perform_streaming_attention over ctx tokens (the last page partial: ctx - 5
    tokens) whose oldest 50% of pages the watermark moved to pinned host memory;
    pool slots scattered (seeded permutation of a fixed pool)."""
    Hq, Hkv, D, P = 32, 8, 128, 16
    T = ctx - 5
    n_pages = -(-T // P)
    a = KVAllocator(1, Hkv, D, P, torch.float16, gpu_capacity_pages=n_pages + 64,
                    cpu_capacity_pages=n_pages, scatter_slots=True)
    m = KVCacheManager(a, gpu_high_watermark_bytes=(n_pages // 2) * a.page_bytes())
    g = torch.Generator().manual_seed(ctx)
    k = torch.randn(1, Hkv, T, D, generator=g).half()
    v = torch.randn(1, Hkv, T, D, generator=g).half()
    print(f"[configs] streaming attention ctx={ctx}", flush=True)
    m.append_prefill(0, k.to(GPU), v.to(GPU))
    pages = m.iterate_layer_pages(0)
    n_host = sum(p.state == "CPU" for p in pages)
    assert abs(n_host - n_pages // 2) <= 1
    assert all(p.state == "CPU" for p in pages[:n_host])        # the oldest ones
    q = torch.randn(1, Hq, 1, D, generator=g).half().to(GPU)
    out = perform_streaming_attention(q, pages, allocator=a)
    ref = oa.eager(q.cpu().numpy(), k.numpy(), v.numpy(), 1.0 / math.sqrt(D))
    assert np.abs(out.float().cpu().numpy() - ref).max() <= ATOL


@pytest.mark.parametrize("B,ctx", [(1, 4096), (8, 4096), (8, 16384), (8, 32768)])
def test_decode_half_on_host_through_offload_manager(B, ctx):
    """One decode step of B sequences of ctx tokens through _decode_batched: the
    manager's watermark (split per item, kv_offload.py:356-360) keeps about half
    of each item's pages on the host, so the step takes the per-item streaming
    path (Path 3); every item against the fp64 form over its ctx tokens."""
    import transformers as tf
    from helm_amd.runtime import KVOffloadConfig, KVOffloadManager
    from helm_amd.runtime.kv_offload import _decode_batched
    Hq, Hkv, D, P = 32, 8, 128, 16
    cfg = tf.Qwen3Config(vocab_size=64, hidden_size=64, intermediate_size=128, num_hidden_layers=1,
                         num_attention_heads=4, num_key_value_heads=2, head_dim=16)
    model = tf.Qwen3ForCausalLM(cfg).to(GPU).half()         # only to be patched
    page_bytes = 2 * Hkv * P * D * 2
    kvcfg = KVOffloadConfig(num_layers=1, num_kv_heads=Hkv, head_dim=D, page_size=P,
                            gpu_watermark_bytes=B * (ctx // P // 2) * page_bytes, cont_capacity=0)
    mgr = KVOffloadManager(model, kvcfg, batch_size=B, gpu_capacity_pages=B * (ctx // P + 2))
    try:
        g = torch.Generator().manual_seed(8)
        ks, vs = [], []
        for i in range(B):
            k = torch.randn(1, Hkv, ctx - 1, D, generator=g).half()
            v = torch.randn(1, Hkv, ctx - 1, D, generator=g).half()
            mgr.kvcms[i].append_prefill(0, k.to(GPU), v.to(GPU))
            ks.append(k)
            vs.append(v)
        q = torch.randn(B, Hq, 1, D, generator=g).half()
        kn = torch.randn(B, Hkv, 1, D, generator=g).half()
        vn = torch.randn(B, Hkv, 1, D, generator=g).half()
        print(f"[configs] batch-{B} {ctx}-token decode step, half on the host", flush=True)
        out = _decode_batched(mgr, q.to(GPU), kn.to(GPU), vn.to(GPU), 0, 1.0 / math.sqrt(D))
        torch.cuda.synchronize()
        for i in range(B):
            pages = mgr.kvcms[i].iterate_layer_pages(0)
            n_host = sum(p.state == "CPU" for p in pages)
            assert 0.45 * len(pages) <= n_host <= 0.55 * len(pages)
            assert mgr.kvcms[i].layers[0].total_tokens == ctx
            kk = torch.cat([ks[i], kn[i:i + 1]], 2).numpy()
            vv = torch.cat([vs[i], vn[i:i + 1]], 2).numpy()
            ref = oa.eager(q[i:i + 1].numpy(), kk, vv, 1.0 / math.sqrt(D))
            err = float(np.abs(out[i:i + 1].float().cpu().numpy() - ref).max())
            assert err <= ATOL, f"item {i}: {err}"
    finally:
        mgr.restore()


# ── Qwen3-32B shape ──────────────────────────────────────────────────────────
@pytest.fixture(scope="module")
def w32():
    from helm_amd.runtime.decode_engine import QWEN3_32B, Int8Qwen3Weights
    print("[configs] building 32B-shape INT8 weights", flush=True)
    w = Int8Qwen3Weights.random(QWEN3_32B, GPU, seed=0)
    torch.cuda.synchronize()
    yield w
    del w
    torch.cuda.empty_cache()


def _engine(w, ctx, watermark=None, use_graph=True):
    from helm_amd.runtime.decode_engine import DecodeEngine
    return DecodeEngine(w, max_context=ctx + 8, page_size=16, gpu_watermark_bytes=watermark,
                        use_graph=use_graph)


def test_32b_graph_replay_equals_eager_at_16k(w32):
    ctx = 16384
    engines = []
    for use_graph in (True, False):
        e = _engine(w32, ctx, use_graph=use_graph)
        e.fill_synthetic_context(ctx - 1, seed=3)
        engines.append(e)
    print("[configs] 32B graph vs eager at 16K", flush=True)
    for tok in (17, 4242):
        outs = []
        for e in engines:
            e.tok.fill_(tok)
            e.decode_step()
            outs.append((e.step_logits().clone(), int(e.tok)))
        torch.cuda.synchronize()
        assert engines[0].graph is not None and engines[1].graph is None
        assert torch.equal(outs[0][0], outs[1][0]) and outs[0][1] == outs[1][1]
    del engines
    torch.cuda.empty_cache()


def _copy_kv_by_token(src, dst):
    """dst's pages get the K/V that src's pages hold for the same tokens (page i of
    layer l in both); src keeps every page on the device, dst may have host pages."""
    sp = src.allocator.pool(src.device)
    dp = dst.allocator.pool(dst.device)
    hp = dst.allocator.pool(torch.device("cpu"))
    dev_s, dev_d, host_s, host_d = [], [], [], []
    for li in range(src.shape.n_layers):
        for ps, pd in zip(src.kvcm.layers[li].pages, dst.kvcm.layers[li].pages):
            assert ps.state == "GPU" and (ps.start_token, ps.used_tokens) == (pd.start_token, pd.used_tokens)
            if pd.state == "GPU":
                dev_s.append(ps.slot)
                dev_d.append(pd.slot)
            else:
                host_s.append(ps.slot)
                host_d.append(pd.slot)
    dst.allocator.synchronize()
    for s, d in ((dev_s, dev_d),):
        si = torch.tensor(s, device=GPU)
        di = torch.tensor(d, device=GPU)
        dp.k.index_copy_(0, di, sp.k.index_select(0, si))
        dp.v_store.index_copy_(0, di, sp.v_store.index_select(0, si))
    for c in range(0, len(host_s), 4096):
        si = torch.tensor(host_s[c:c + 4096], device=GPU)
        di = torch.tensor(host_d[c:c + 4096])
        hp.k[di] = sp.k.index_select(0, si).cpu()
        hp.v_store[di] = sp.v_store.index_select(0, si).cpu()
    torch.cuda.synchronize()
    return len(host_s)


def _torch_forward(w, tokens, start, past, dtype):
    """The engine's model in plain torch on the GPU, the reference for the
    full-depth Qwen3-32B-shape checks (the numpy oracle cannot hold this model):
    `tokens` [S] at positions start .. start + S - 1 after the cached tokens that
    past(layer) returns as (K, V) [Hkv, T, D] (None: no cache).  Weights are the
    dequantised INT8 weights q * s.  dtype float32: no intermediate rounding
    (scores and softmax in fp32).  dtype float16: the roundings of transformers'
    fp16 model (norms in fp32 cast back, products with fp32 accumulation rounded
    to fp16, fp16 RoPE, SDPA).  Returns fp32 logits [S, V]."""
    import torch.nn.functional as F
    sh = w.shape
    D, Hq, Hkv = sh.head_dim, sh.n_heads, sh.n_kv_heads
    S = tokens.shape[0]
    dev = GPU
    pos = torch.arange(start, start + S, device=dev, dtype=torch.float32)
    inv = 1.0 / (sh.rope_theta ** (torch.arange(0, D, 2, device=dev, dtype=torch.float32) / D))
    ang = pos[:, None] * inv[None]
    emb = torch.cat([ang, ang], -1)
    cos, sin = emb.cos().to(dtype), emb.sin().to(dtype)

    def rms(x, wt):
        xf = x.float()
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + sh.eps)
        return wt.to(dtype) * y.to(dtype)

    def lin(x, q, sc):
        wd = (q.float() * sc.float()[:, None]).to(dtype)
        return x @ wd.t().contiguous()

    def rope(x):   # x [S, H, D]
        h = D // 2
        rot = torch.cat([-x[..., h:], x[..., :h]], -1)
        return x * cos[:, None, :] + rot * sin[:, None, :]

    h = w.embed[tokens.to(dev)].to(dtype)
    for li, lay in enumerate(w.layers):
        x = rms(h, lay["in_ln"])
        qkv = lin(x, lay["qkv_q"], lay["qkv_s"])
        q = qkv[:, :Hq * D].reshape(S, Hq, D)
        k = qkv[:, Hq * D:(Hq + Hkv) * D].reshape(S, Hkv, D)
        v = qkv[:, (Hq + Hkv) * D:].reshape(S, Hkv, D)
        q, k = rope(rms(q, lay["q_norm"])), rope(rms(k, lay["k_norm"]))
        K, V = k.transpose(0, 1), v.transpose(0, 1)          # [Hkv, S, D]
        T0 = 0
        if past is not None:
            pk, pv = past(li)
            T0 = pk.shape[1]
            K, V = torch.cat([pk.to(dtype), K], 1), torch.cat([pv.to(dtype), V], 1)
        g = Hq // Hkv
        K = K.repeat_interleave(g, 0).contiguous()
        V = V.repeat_interleave(g, 0).contiguous()
        qh = q.transpose(0, 1).contiguous()                   # [Hq, S, D]
        allowed = (torch.arange(T0 + S, device=dev)[None, :]
                   <= T0 + torch.arange(S, device=dev)[:, None])   # causal over the new tokens
        # scores and softmax as SDPA's math form computes them in `dtype` (fp16:
        # products rounded to fp16, softmax in fp32 rounded back); every product
        # takes contiguous operands
        sc = (qh @ K.transpose(1, 2).contiguous()) * (1.0 / math.sqrt(D))
        sc = sc.float().masked_fill(~allowed[None], float("-inf"))
        a = torch.softmax(sc, -1).to(dtype) @ V
        a = a.transpose(0, 1).reshape(S, Hq * D)
        h = h + lin(a, lay["o_q"], lay["o_s"])
        x = rms(h, lay["post_ln"])
        gt = lin(x, lay["gate_q"], lay["gate_s"])
        up = lin(x, lay["up_q"], lay["up_s"])
        h = h + lin(F.silu(gt) * up, lay["down_q"], lay["down_s"])
    xf = rms(h, w.norm)
    return (xf @ w.lm_head.to(dtype).t().contiguous()).float()


def _engine_layer_kv(e, li, n_tokens):
    """(K, V) [Hkv, n_tokens, D] of layer li in token order from engine e's pages
    (device pool or pinned host pool)."""
    pages = e.kvcm.layers[li].pages
    dp = e.allocator.pool(e.device)
    ks, vs = [], []
    run, run_dev = [], None
    def flush():
        if not run:
            return
        pool = dp if run_dev else e.allocator.pool(torch.device("cpu"))
        idx = torch.tensor(run, device=pool.k.device)
        ks.append(pool.k.index_select(0, idx).to(GPU))
        vs.append(pool.v.index_select(0, idx).to(GPU))
    for pg in pages:
        on_dev = pg.state == "GPU"
        if run and on_dev != run_dev:
            flush()
            run = []
        run_dev = on_dev
        run.append(pg.slot)
    flush()
    K = torch.cat(ks)   # [n_pages, Hkv, P, D]
    V = torch.cat(vs)
    n, hkv, P, D = K.shape
    K = K.permute(1, 0, 2, 3).reshape(hkv, n * P, D)[:, :n_tokens]
    V = V.permute(1, 0, 2, 3).reshape(hkv, n * P, D)[:, :n_tokens]
    return K.float(), V.float()


def _fp16_bar(ref32, ref16):
    """The end-to-end bar of this suite: max(2e-2, 1.5 x the error of the same
    model in transformers' fp16 roundings), on the logits."""
    return max(2e-2, 1.5 * float((ref16 - ref32).abs().max()))


@pytest.mark.parametrize("ctx", [16384, 32768])
def test_32b_half_on_host_step_against_torch_reference(w32, ctx):
    """One decode step of the 64-layer Qwen3-32B shape at ctx tokens with every
    page in HBM (graph replay) and with the oldest 50% of pages on the host (the
    eager step: device suffix in place, host prefix staged by the gather kernel,
    one reduce over both), both against the plain-torch fp32 step over the same
    cached K/V, within the suite's end-to-end bar (max(2e-2, 1.5 x the fp16
    torch step's error)).  The offloaded step's last layer is also checked
    directly: its attention output against the fp64 form over that layer's
    cached tokens plus the new one, bar 2e-3."""
    from helm_amd.runtime.decode_engine import QWEN3_32B as sh
    kv_bytes = (ctx - 1) * 2 * sh.n_kv_heads * sh.head_dim * 2 * sh.n_layers
    res = _engine(w32, ctx)
    res.fill_synthetic_context(ctx - 1, seed=5)
    off = _engine(w32, ctx, watermark=kv_bytes // 2)
    off.fill_synthetic_context(ctx - 1, seed=6)
    n_host = _copy_kv_by_token(res, off)
    total = sum(len(res.kvcm.layers[li].pages) for li in range(sh.n_layers))
    assert 0.45 * total <= n_host <= 0.55 * total
    tok = torch.tensor([777])
    print(f"[configs] 32B torch reference step at {ctx}", flush=True)
    with torch.no_grad():
        past = lambda li: _engine_layer_kv(res, li, ctx - 1)  # noqa: E731
        ref32 = _torch_forward(w32, tok, ctx - 1, past, torch.float32)[0]
        ref16 = _torch_forward(w32, tok, ctx - 1, past, torch.float16)[0]
    bar = _fp16_bar(ref32, ref16)
    for e in (res, off):
        e.tok.fill_(int(tok))
        e.decode_step()
    torch.cuda.synchronize()
    assert res.graph is not None and not off.all_gpu
    errs = [float((e.step_logits().float() - ref32).abs().max()) for e in (res, off)]
    print(f"[configs] 32B step at {ctx}: {n_host} of {total} pages on the host; logits error "
          f"resident {errs[0]:.3e}, offloaded {errs[1]:.3e}, bar {bar:.3e}", flush=True)
    assert max(errs) <= bar, (errs, bar)
    top2 = torch.topk(ref32, 2).values
    if float(top2[0] - top2[1]) > 2 * bar:
        assert int(res.tok) == int(off.tok) == int(ref32.argmax())
    # the offloaded step's last layer: q and attention output against fp64 (its
    # pages read once the step's eviction copies have landed)
    off.allocator.synchronize()
    torch.cuda.synchronize()
    L = sh.n_layers - 1
    K, V = _engine_layer_kv(off, L, ctx)     # the new token's K/V written by the step
    q = off.q[0].float().cpu().numpy()[None, :, None, :].astype(np.float64)
    ref = oa.eager(q, K.cpu().numpy()[None].astype(np.float64), V.cpu().numpy()[None].astype(np.float64),
                   1.0 / math.sqrt(sh.head_dim))[0, :, 0, :]
    err = float(np.abs(off.attn[0].float().cpu().numpy() - ref).max())
    assert err <= ATOL, f"ctx {ctx}: last layer attention of the offloaded step {err}"
    del res, off
    torch.cuda.empty_cache()


def test_8b_headline_step_graph_equals_eager_and_torch_reference():
    """The headline configuration (bench.py's default workload): the 36-layer
    Qwen3-8B shape, INT8 weights, 16K cached tokens, page 16.  Graph-replayed
    and eager steps give the same bits over two steps, and the first step's
    logits land within the suite's end-to-end bar (max(2e-2, 1.5 x the fp16 torch
    step's error)) of the plain-torch fp32 step over the same cached K/V."""
    from helm_amd.runtime.decode_engine import QWEN3_8B as sh, Int8Qwen3Weights
    ctx = 16384
    print("[configs] building 8B-shape INT8 weights", flush=True)
    w8 = Int8Qwen3Weights.random(sh, GPU, seed=3, norm_jitter=0.1)
    engines = []
    for use_graph in (True, False):
        e = _engine(w8, ctx, use_graph=use_graph)
        e.fill_synthetic_context(ctx - 1, seed=4)
        engines.append(e)
    tok = torch.tensor([777])
    print("[configs] 8B torch reference step at 16K", flush=True)
    with torch.no_grad():
        past = lambda li: _engine_layer_kv(engines[0], li, ctx - 1)  # noqa: E731
        ref32 = _torch_forward(w8, tok, ctx - 1, past, torch.float32)[0]
        ref16 = _torch_forward(w8, tok, ctx - 1, past, torch.float16)[0]
    bar = _fp16_bar(ref32, ref16)
    for step, t in enumerate((777, 4242)):
        outs = []
        for e in engines:
            e.tok.fill_(t)
            e.decode_step()
            outs.append((e.step_logits().clone(), int(e.tok)))
        torch.cuda.synchronize()
        assert engines[0].graph is not None and engines[1].graph is None
        assert torch.equal(outs[0][0], outs[1][0]) and outs[0][1] == outs[1][1]
        if step == 0:
            err = float((outs[0][0].float() - ref32).abs().max())
            print(f"[configs] 8B step at 16K: logits error {err:.3e}, bar {bar:.3e}", flush=True)
            assert err <= bar
            top2 = torch.topk(ref32, 2).values
            if float(top2[0] - top2[1]) > 2 * bar:
                assert outs[0][1] == int(ref32.argmax())
    del engines, w8
    torch.cuda.empty_cache()


def test_8b_batch8_step_graph_equals_eager_and_torch_reference():
    """The batched-decode benchmark configuration (bench.py --workload batch8b):
    8 sequences of 16K cached tokens through the 36-layer Qwen3-8B shape.
    Graph-replayed and eager steps give the same bits, and every item's logits
    land within the end-to-end bar of its own plain-torch fp32 step."""
    from types import SimpleNamespace
    from helm_amd.runtime.batch_engine import BatchDecodeEngine
    from helm_amd.runtime.decode_engine import QWEN3_8B as sh, Int8Qwen3Weights
    B, ctx = 8, 16384
    print("[configs] building 8B-shape INT8 weights (batch 8)", flush=True)
    w8 = Int8Qwen3Weights.random(sh, GPU, seed=5, norm_jitter=0.1)
    engines = []
    for use_graph in (True, False):
        e = BatchDecodeEngine(w8, B, max_context=ctx + 8, use_graph=use_graph)
        e.fill_synthetic_context(ctx - 1, seed=6)
        engines.append(e)
    toks = torch.tensor([777 + 1013 * i for i in range(B)])
    refs = []
    with torch.no_grad():
        for i in range(B):
            view = SimpleNamespace(kvcm=engines[0].kvcms[i], allocator=engines[0].allocator,
                                   device=engines[0].device)
            past = lambda li, v=view: _engine_layer_kv(v, li, ctx - 1)  # noqa: E731
            r32 = _torch_forward(w8, toks[i:i + 1], ctx - 1, past, torch.float32)[0]
            r16 = _torch_forward(w8, toks[i:i + 1], ctx - 1, past, torch.float16)[0]
            refs.append((r32, _fp16_bar(r32, r16)))
    print("[configs] 8B batch-8 torch reference steps done", flush=True)
    outs = []
    for e in engines:
        e.tok.copy_(toks.to(e.tok.device, e.tok.dtype))
        e.decode_step()
        outs.append((e.step_logits().clone(), e.tok.clone()))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    errs = [float((outs[0][0][i].float() - r32).abs().max()) for i, (r32, _) in enumerate(refs)]
    print(f"[configs] 8B batch-8 step at 16K: logits errors {max(errs):.3e} max, "
          f"bars {min(b for _, b in refs):.3e} min", flush=True)
    for i, (r32, bar) in enumerate(refs):
        assert errs[i] <= bar, (i, errs[i], bar)
    del engines, w8
    torch.cuda.empty_cache()


def test_8b_dropin_step_against_torch_reference():
    """The drop-in configuration (bench.py --workload dropin8b) at full depth:
    transformers Qwen3ForCausalLM of the 36-layer 8B shape with patch_linears /
    patch_cpu_linears, KVOffloadManager (contiguous buffer with the decoder
    layers fused, and every page in HBM) and PipelineRuntime's prefill of a
    2048-token prompt, then three decode steps (the later ones replayed from HIP
    graphs); the last step's logits land within the end-to-end bar of the plain
    torch fp32 forward of the whole sequence on the same INT8 weights."""
    from transformers import Qwen3Config, Qwen3ForCausalLM
    from helm_amd.kernels import patch_cpu_linears, patch_linears
    from helm_amd.runtime import KVOffloadConfig, KVOffloadManager, PipelineRuntime
    from helm_amd.runtime.decode_engine import QWEN3_8B as sh, Int8Qwen3Weights
    cfg = Qwen3Config(vocab_size=sh.vocab, hidden_size=sh.hidden, intermediate_size=sh.ffn,
                      num_hidden_layers=sh.n_layers, num_attention_heads=sh.n_heads,
                      num_key_value_heads=sh.n_kv_heads, head_dim=sh.head_dim,
                      rms_norm_eps=sh.eps, rope_theta=sh.rope_theta,
                      max_position_embeddings=40960, tie_word_embeddings=False,
                      attention_bias=False)
    cfg._attn_implementation = "sdpa"
    print("[configs] building the 8B-shape transformers model", flush=True)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float16)
    try:
        with torch.device(GPU), torch.no_grad():
            model = Qwen3ForCausalLM(cfg).eval()
            gen = torch.Generator(device=GPU).manual_seed(8)
            for p in model.parameters():
                if p.dim() == 2:
                    p.normal_(0.0, 0.02, generator=gen)
                else:
                    p.fill_(1.0)
                    p.add_(torch.randn(p.shape, device=GPU, generator=gen).half() * 0.1)
    finally:
        torch.set_default_dtype(prev)
    patch_linears(model, exclude=("lm_head",))
    patch_cpu_linears(model)
    w = Int8Qwen3Weights.from_hf(model)
    g = torch.Generator().manual_seed(9)
    T = 2048
    prompt = torch.randint(0, sh.vocab, (1, T), generator=g).to(GPU)
    forced = [777, 4242, 31337]
    seq = torch.cat([prompt[0].cpu(), torch.tensor(forced)])
    with torch.no_grad():
        ref32 = _torch_forward(w, seq, 0, None, torch.float32)[-1]
        ref16 = _torch_forward(w, seq, 0, None, torch.float16)[-1]
    bar = _fp16_bar(ref32, ref16)
    for fused, kw in ((True, {}), (False, {"cont_capacity": 0})):
        kcfg = KVOffloadConfig.from_model(model, page_size=16, gpu_watermark_bytes=10 ** 15,
                                          fuse_decoder_layers=fused, **kw)
        mgr = KVOffloadManager(model, kcfg, batch_size=1)
        try:
            rt = PipelineRuntime(model, kv_offload_mgr=mgr)
            mgr.reset()
            with torch.no_grad():
                rt.prefill(prompt)
                for i, t in enumerate(forced):
                    logits = rt.decode_step(torch.tensor([[t]], device=GPU), T + i)
            torch.cuda.synchronize()
            err = float((logits[0, -1].float() - ref32).abs().max())
            print(f"[configs] 8B drop-in ({'contiguous, fused layers' if fused else 'paged'}): "
                  f"logits error {err:.3e}, bar {bar:.3e}", flush=True)
            assert err <= bar
        finally:
            mgr.restore()
            del mgr
            torch.cuda.empty_cache()
    del model, w
    torch.cuda.empty_cache()


def test_8b_half_on_host_step_against_torch_reference():
    """The offload configuration (bench.py --workload offload8b): the 36-layer
    Qwen3-8B shape at 16K tokens with the oldest 50% of pages in pinned host
    memory (the eager mixed-residency step) and with every page in HBM (graph
    replay), over the same cached K/V, both within the end-to-end bar of the
    plain-torch fp32 step."""
    from helm_amd.runtime.decode_engine import QWEN3_8B as sh, Int8Qwen3Weights
    ctx = 16384
    w8 = Int8Qwen3Weights.random(sh, GPU, seed=12, norm_jitter=0.1)
    kv_bytes = (ctx - 1) * 2 * sh.n_kv_heads * sh.head_dim * 2 * sh.n_layers
    res = _engine(w8, ctx)
    res.fill_synthetic_context(ctx - 1, seed=13)
    off = _engine(w8, ctx, watermark=kv_bytes // 2)
    off.fill_synthetic_context(ctx - 1, seed=14)
    n_host = _copy_kv_by_token(res, off)
    total = sum(len(res.kvcm.layers[li].pages) for li in range(sh.n_layers))
    assert 0.45 * total <= n_host <= 0.55 * total
    tok = torch.tensor([4242])
    with torch.no_grad():
        past = lambda li: _engine_layer_kv(res, li, ctx - 1)  # noqa: E731
        ref32 = _torch_forward(w8, tok, ctx - 1, past, torch.float32)[0]
        ref16 = _torch_forward(w8, tok, ctx - 1, past, torch.float16)[0]
    bar = _fp16_bar(ref32, ref16)
    for e in (res, off):
        e.tok.fill_(int(tok))
        e.decode_step()
    torch.cuda.synchronize()
    assert res.graph is not None and not off.all_gpu
    errs = [float((e.step_logits().float() - ref32).abs().max()) for e in (res, off)]
    print(f"[configs] 8B step at 16K: {n_host} of {total} pages on the host; logits error "
          f"resident {errs[0]:.3e}, offloaded {errs[1]:.3e}, bar {bar:.3e}", flush=True)
    assert max(errs) <= bar, (errs, bar)
    del res, off, w8
    torch.cuda.empty_cache()


def test_32b_prefill_matches_token_by_token_decode(w32):
    """A real 1024-token random prompt through the 64-layer Qwen3-32B shape:
    the prefill's last-position logits (INT8 GEMMs, the prompt's K/V written into
    pages, causal prefill attention over them) and the logits of feeding the
    same 1024 tokens one decode step at a time (GEMVs, paged decode attention)
    on a second engine, each against the plain-torch fp32 forward of the prompt
    within the suite's bar B = max(2e-2, 1.5 x the fp16 torch forward's error),
    so the two engine paths agree within 2B (triangle inequality); the greedy
    token is the reference's wherever its top-2 margin exceeds 2B."""
    from helm_amd.runtime.decode_engine import QWEN3_32B as sh
    S = 1024
    g = torch.Generator().manual_seed(1024)
    prompt = torch.randint(0, sh.vocab, (S,), generator=g)
    a = _engine(w32, S + 8)
    print("[configs] 32B 1024-token prefill", flush=True)
    la = a.prefill(prompt.to(GPU)).float()
    del a
    b = _engine(w32, S + 8)
    b.prefill(prompt[:1].to(GPU))
    print("[configs] 32B the same tokens one decode step at a time", flush=True)
    for t in range(1, S):
        b.tok.fill_(int(prompt[t]))
        b.decode_step()
    lb = b.step_logits().float()
    torch.cuda.synchronize()
    assert b.graph is not None
    del b
    torch.cuda.empty_cache()
    with torch.no_grad():
        ref32 = _torch_forward(w32, prompt, 0, None, torch.float32)[-1]
        ref16 = _torch_forward(w32, prompt, 0, None, torch.float16)[-1]
    bar = _fp16_bar(ref32, ref16)
    ea, eb = float((la - ref32).abs().max()), float((lb - ref32).abs().max())
    d = float((la - lb).abs().max())
    print(f"[configs] 32B prefill vs torch fp32 {ea:.3e}, token by token {eb:.3e}, between "
          f"them {d:.3e}, bar {bar:.3e}", flush=True)
    assert ea <= bar and eb <= bar and d <= 2 * bar
    top2 = torch.topk(ref32, 2).values
    if float(top2[0] - top2[1]) > 2 * bar:
        assert int(la.argmax()) == int(lb.argmax()) == int(ref32.argmax())


def test_32b_shape_two_layers_teacher_forced_against_oracle():
    """Two decoder layers of the Qwen3-32B shape (full vocab), prefill of 40 random
    tokens and 8 teacher-forced decode steps on the engine, against the fp32
    oracle; bar max(2e-2, 1.5 x the fp16 torch model's error)."""
    from helm_amd.runtime.decode_engine import QWEN3_32B, DecodeEngine, Int8Qwen3Weights, Qwen3Shape
    from oracle.qwen3 import Qwen3Oracle, hf_model_from_weights
    sh = Qwen3Shape(hidden=QWEN3_32B.hidden, n_heads=QWEN3_32B.n_heads,
                    n_kv_heads=QWEN3_32B.n_kv_heads, head_dim=QWEN3_32B.head_dim,
                    ffn=QWEN3_32B.ffn, n_layers=2, vocab=QWEN3_32B.vocab)
    w = Int8Qwen3Weights.random(sh, GPU, seed=9, norm_jitter=0.1)
    g = torch.Generator().manual_seed(3)
    S, N = 40, 8
    prompt = torch.randint(0, sh.vocab, (S,), generator=g)
    forced = torch.randint(0, sh.vocab, (N,), generator=g)
    eng = DecodeEngine(w, max_context=S + N + 8, page_size=16)
    logits = [eng.prefill(prompt.to(GPU)).float().cpu()]
    for i in range(N - 1):
        eng.tok.fill_(int(forced[i]))
        eng.decode_step()
        logits.append(eng.step_logits().float().cpu())
    logits = torch.stack(logits).numpy()
    print("[configs] 32B-shape 2-layer oracle", flush=True)
    wc = Int8Qwen3Weights(sh)
    wc.layers = [{k: v.cpu() for k, v in lay.items()} for lay in w.layers]
    wc.embed, wc.norm, wc.lm_head = w.embed.cpu(), w.norm.cpu(), w.lm_head.cpu()
    seq = np.concatenate([prompt.numpy(), forced[:-1].numpy()])
    ref = Qwen3Oracle(wc).forward(seq)[S - 1:]
    m = hf_model_from_weights(wc, dtype=torch.float16).to(GPU)
    m.config._attn_implementation = "sdpa"
    with torch.no_grad():
        ref16 = m(torch.from_numpy(seq)[None].to(GPU)).logits[0, S - 1:].float().cpu().numpy()
    del m
    tol = max(2e-2, 1.5 * float(np.abs(ref16 - ref).max()))
    err = float(np.abs(logits - ref).max())
    assert err <= tol, f"teacher-forced logits max err {err} > {tol}"
