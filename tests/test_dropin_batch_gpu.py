"""The HF drop-in path (transformers Qwen3ForCausalLM + patch_linears +
KVOffloadManager + PipelineRuntime) at batch > 1 and through the contiguous
path's overflow, on the plumbing configuration (2 layers, hidden 1024, 16/8
heads, D 64, FFN 3072, vocab 32000, INT8 weights N(0,0.02), page 16).

Every item of a batch is teacher-forced on its own random tokens and its logits
are compared with the fp32 oracle run on that item alone (bar: max(2e-2, 1.5 x
the fp16 torch model's error), as the batch-1 tests).  The branches covered
(reference kv_offload.py:82-167, :344-382, kv_cache.py:206-289):
  * batched Path 1 (one contiguous buffer row per item),
  * batched Path 2 (every page on the GPU, one kernel over the page table),
  * per-item Path 3 (the watermark, split per item, puts pages on the host),
  * the contiguous buffer overflowing mid-decode: the decode tokens migrate to
    pages after a partial prompt page, and decode continues over that ragged
    page list, with the page tables bit-identical to the oracle's restatement.
"""
import numpy as np
import pytest
import torch

from helm_amd.kernels import patch_linears
from helm_amd.runtime import KVOffloadConfig, KVOffloadManager, PipelineRuntime
from helm_amd.runtime.decode_engine import QWEN3_PLUMBING, Int8Qwen3Weights
from oracle import kv_pages as okp
from oracle.qwen3 import Qwen3Oracle, hf_model_from_weights

pytestmark = pytest.mark.gpu
LOGIT_ATOL = 2e-2
PAGE = 16


@pytest.fixture(scope="module")
def weights():
    return Int8Qwen3Weights.random(QWEN3_PLUMBING, torch.device("cuda"), seed=0, norm_jitter=0.1)


def _cpu_weights(weights):
    w = Int8Qwen3Weights(QWEN3_PLUMBING)
    w.layers = [{k: v.cpu() for k, v in lay.items()} for lay in weights.layers]
    w.embed, w.norm, w.lm_head = weights.embed.cpu(), weights.norm.cpu(), weights.lm_head.cpu()
    return w


@pytest.fixture(scope="module")
def model(weights):
    m = hf_model_from_weights(_cpu_weights(weights), dtype=torch.float16).cuda()
    m.config._attn_implementation = "sdpa"
    assert patch_linears(m, exclude=("lm_head",)) == 14
    return m


@pytest.fixture(scope="module")
def oracle(weights):
    return Qwen3Oracle(weights)


def _tokens(seed, n):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, QWEN3_PLUMBING.vocab, (n,), generator=g)


def _oracle_logits(oracle, prompt, forced):
    seq = np.concatenate([prompt.numpy(), forced[:-1].numpy()])
    return oracle.forward(seq)[len(prompt) - 1:]


def _bar(weights, prompt, forced, ref):
    """max(2e-2, 1.5 x the error of plain fp16 torch (unpatched) against the oracle)."""
    m = hf_model_from_weights(_cpu_weights(weights), dtype=torch.float16).cuda()
    m.config._attn_implementation = "sdpa"
    seq = torch.cat([prompt, forced[:-1]])[None].cuda()
    with torch.no_grad():
        ref16 = m(seq).logits[0, len(prompt) - 1:].float().cpu().numpy()
    del m
    return max(LOGIT_ATOL, 1.5 * float(np.abs(ref16 - ref).max()))


def _run_dropin(model, prompts, forced, cont, watermark=None, fused=False, page_size=PAGE):
    """Teacher-forced drop-in run of a batch: prompts [B, S], forced [B, N];
    returns (logits [B, N, V], manager) — the manager restored, its caches kept.
    `fused`: the manager also patches the MLP, RMSNorm and decoder-layer classes."""
    B, S = prompts.shape
    N = forced.shape[1]
    cfg = KVOffloadConfig.from_model(model, page_size=page_size, cont_capacity=cont,
                                     gpu_watermark_bytes=watermark, fuse_decoder_layers=fused)
    mgr = KVOffloadManager(model, cfg, batch_size=B)
    try:
        rt = PipelineRuntime(model, kv_offload_mgr=mgr)
        mgr.reset()
        logits = [rt.prefill(prompts.cuda())[:, -1].float().cpu()]
        for i in range(N - 1):
            logits.append(rt.decode_step(forced[:, i:i + 1].cuda(), S + i)[:, -1].float().cpu())
        torch.cuda.synchronize()
    finally:
        mgr.restore()
    return torch.stack(logits, 1).numpy(), mgr


@pytest.fixture(scope="module")
def batch4(oracle, weights):
    B, S, N = 4, 512, 32
    prompts = torch.stack([_tokens(1 + b, S) for b in range(B)])
    forced = torch.stack([_tokens(100 + b, N) for b in range(B)])
    refs = [_oracle_logits(oracle, prompts[b], forced[b]) for b in range(B)]
    tol = _bar(weights, prompts[0], forced[0], refs[0])
    return prompts, forced, refs, tol


def _check_items(logits, refs, tol, what):
    for b, ref in enumerate(refs):
        err = float(np.abs(logits[b] - ref).max())
        assert err <= tol, f"{what}: item {b} teacher-forced logits max err {err} > {tol}"


@pytest.mark.parametrize("fused", [False, True], ids=["attention_patch", "fused_layers"])
@pytest.mark.parametrize("path", ["contiguous", "paged_gpu", "mixed"])
def test_batch4_items_match_oracle(model, batch4, path, fused):
    prompts, forced, refs, tol = batch4
    print(f"[dropin] batch 4 path={path} fused={fused}", flush=True)
    page_bytes = 2 * 8 * PAGE * 64 * 2
    if path == "contiguous":
        logits, mgr = _run_dropin(model, prompts, forced, cont=4096, fused=fused)
        assert all(m.use_contiguous for m in mgr.kvcms)
        assert mgr.kvcms[0].cont_seq_len == prompts.shape[1] + forced.shape[1] - 1
    elif path == "paged_gpu":
        logits, mgr = _run_dropin(model, prompts, forced, cont=0, watermark=10 ** 12, fused=fused)
        assert all(p.state == "GPU" for m in mgr.kvcms for L in m.layers.values() for p in L.pages)
    else:
        # 8 pages of watermark in total: 2 per item (kv_offload.py:356-360)
        logits, mgr = _run_dropin(model, prompts, forced, cont=0, watermark=8 * page_bytes,
                                  fused=fused)
        for m in mgr.kvcms:
            assert m.gpu_high_watermark_bytes == 2 * page_bytes
            assert sum(p.state == "CPU" for p in m.layers[0].pages) > 20
    _check_items(logits, refs, tol, path)


def test_contiguous_buffers_built_per_item_are_read_in_place(model, batch4):
    """Items whose contiguous buffers were built one by one (not rows of one
    batched allocation): decode reads each item's buffer in place, one launch
    per item into the shared partials, and every item still matches the
    oracle."""
    prompts, forced, refs, tol = batch4
    B, S = prompts.shape
    N = forced.shape[1]
    cfg = KVOffloadConfig.from_model(model, page_size=PAGE, cont_capacity=2048)
    mgr = KVOffloadManager(model, cfg, batch_size=B)
    try:
        for m in mgr.kvcms:
            assert m.build_contiguous(cfg.num_layers, cfg.num_kv_heads, cfg.head_dim, 2048,
                                      torch.device("cuda"), cfg.dtype)
        assert mgr._shared_contiguous(B) is None
        rt = PipelineRuntime(model, kv_offload_mgr=mgr)
        mgr.reset()
        logits = [rt.prefill(prompts.cuda())[:, -1].float().cpu()]
        for i in range(N - 1):
            logits.append(rt.decode_step(forced[:, i:i + 1].cuda(), S + i)[:, -1].float().cpu())
        assert rt._graphs is None          # not planned: the per-layer path ran
        assert all(m.use_contiguous and m.cont_seq_len == S + N - 1 for m in mgr.kvcms)
    finally:
        mgr.restore()
    _check_items(torch.stack(logits, 1).numpy(), refs, tol, "per-item contiguous buffers")


def test_batch_items_equal_their_batch1_runs(model, batch4):
    """Each item of a paged batch-4 run against the same item run alone: within
    the oracle bar (the batch changes only the GEMV's token count and the split
    structure, i.e. rounding)."""
    prompts, forced, refs, tol = batch4
    logits4, _ = _run_dropin(model, prompts, forced, cont=0, watermark=10 ** 12)
    for b in (0, 3):
        logits1, _ = _run_dropin(model, prompts[b:b + 1], forced[b:b + 1], cont=0,
                                 watermark=10 ** 12)
        assert np.abs(logits1[0] - logits4[b]).max() <= tol


def _oracle_page_trace(B, S, N, L, cont, watermark):
    """Page tables of the oracle restatement driven like the drop-in run: each
    item's contiguous buffer, every layer prefilled item by item (pages and
    buffer), then N-1 decode steps of every layer (kv_offload.py:106-138).  The
    K/V values do not matter for the page tables: zeros."""
    oa = okp.KVAllocator(L, 8, 64, PAGE, 2, np.float16)
    oms = [okp.KVCacheManager(oa, max(watermark // B, 1)) for _ in range(B)]
    for m in oms:
        assert m.build_contiguous(L, 8, 64, cont, "cuda")
    kz = np.zeros((1, 8, S, 64), np.float16)
    for lid in range(L):
        for m in oms:
            m.append_prefill(lid, kz, kz, "cuda")
            m.prefill_contiguous(lid, kz, kz)
    one = np.zeros((1, 8, 1, 64), np.float16)
    paths = [okp.decode_step_kv(oms, lid, [one] * B, [one] * B, "cuda")
             for _ in range(N - 1) for lid in range(L)]
    return oms, oa, paths


@pytest.mark.parametrize("B,watermark", [(1, 10 ** 12), (2, None)])
def test_contiguous_overflow_migrates_and_continues(model, oracle, weights, B, watermark):
    """cont_capacity 1024 with a 1000-token prompt (1000 % 16 = 8, so the prompt's
    last page holds 8 tokens) and 40 decode tokens: 24 decode tokens fit the
    buffer, the 25th migrates them to pages after the partial prompt page and
    decode continues paged over that ragged list.  Every page on the GPU (batch
    1: Path 3's in-place page runs) or the default watermark (512 tokens per
    layer, split over 2 items: prompt pages evicted during prefill and while the
    migrated tokens are appended).  Logits within the oracle bar at every step;
    page tables bit-identical to the oracle's restatement of the same calls."""
    S, N, cont = 1000, 40, 1024
    prompts = torch.stack([_tokens(7 + b, S) for b in range(B)])
    forced = torch.stack([_tokens(70 + b, N) for b in range(B)])
    print(f"[dropin] overflow B={B} watermark={watermark}", flush=True)
    logits, mgr = _run_dropin(model, prompts, forced, cont=cont, watermark=watermark)
    refs = [_oracle_logits(oracle, prompts[b], forced[b]) for b in range(B)]
    tol = _bar(weights, prompts[0], forced[0], refs[0])
    _check_items(logits, refs, tol, f"overflow B={B}")
    assert not any(m.use_contiguous for m in mgr.kvcms)
    wm = mgr.config.gpu_watermark_bytes
    oms, oa, paths = _oracle_page_trace(B, S, N, 2, cont, wm)
    assert paths.count("contiguous") == 2 * (cont - S)
    for pm, om in zip(mgr.kvcms, oms):
        for lid in range(2):
            got = [(p.page_id, p.state, p.start_token, p.used_tokens) for p in pm.layers[lid].pages]
            want = [(p.page_id, p.state, p.start_token, p.used_tokens) for p in om.layers[lid].pages]
            assert got == want
            assert pm.layer_is_ragged(lid)
    if watermark is None:
        assert any(p.state == "CPU" for m in mgr.kvcms for p in m.layers[0].pages)
    assert mgr.allocator.report_usage() == oa.report_usage()


def test_async_eviction_while_both_pools_grow():
    """Asynchronous eviction with pools that start tiny (8 device slots, 4 host
    slots) so both double many times while eviction copies are in flight: the
    attention issued right after, and every host page once synchronised, hold
    exactly the source K/V."""
    import math
    from helm_amd.runtime import KVAllocator, KVCacheManager, perform_streaming_attention
    from oracle import attention as oa
    Hq, Hkv, D, P = 32, 8, 128, 16
    a = KVAllocator(2, Hkv, D, P, torch.float16, gpu_capacity_pages=8, cpu_capacity_pages=4,
                    async_eviction=True)
    m = KVCacheManager(a, gpu_high_watermark_bytes=3 * a.page_bytes())
    g = torch.Generator().manual_seed(11)
    T = 150 * P + 9
    kv = [(torch.randn(1, Hkv, T, D, generator=g).half(), torch.randn(1, Hkv, T, D, generator=g).half())
          for _ in range(2)]
    for lid, (k, v) in enumerate(kv):
        m.append_prefill(lid, k.cuda(), v.cuda())
    n_host = [sum(p.state == "CPU" for p in m.layers[lid].pages) for lid in range(2)]
    assert sum(n_host) > 250
    assert a.pool(torch.device("cpu")).capacity >= 256 and a.pool(torch.device("cuda")).capacity > 8
    q = torch.randn(1, Hq, 1, D, dtype=torch.float16, device="cuda")
    for lid, (k, v) in enumerate(kv):
        out = perform_streaming_attention(q, m.iterate_layer_pages(lid), allocator=a)
        ref = oa.eager(q.cpu().numpy(), k.numpy(), v.numpy(), 1 / math.sqrt(D))
        assert np.abs(out.cpu().numpy().astype(np.float64) - ref).max() <= 2e-3
    a.synchronize()
    for lid, (k, v) in enumerate(kv):
        for i, p in enumerate(m.layers[lid].pages):
            u = p.used_tokens
            assert torch.equal(p.k_tensor[:, :, :u].cpu(), k[:, :, i * P:i * P + u])
            assert torch.equal(p.v_tensor[:, :, :u].cpu(), v[:, :, i * P:i * P + u])


def test_left_padded_prefill_matches_unpadded_items(model, monkeypatch):
    """A left-padded batch (HF turns the 2-D attention_mask into a 4-D padding
    mask) through the patched forward: its prefill attention runs on
    helm_prefill_attn_mask (the reference hands that mask to SDPA,
    kv_offload.py:253-265), and each item's logits at its real tokens equal the
    item's unpadded batch-1 run (bar LOGIT_ATOL: only rounding differs)."""
    from helm_amd.kernels import attention as ka
    S, pad = 200, 37
    a, b = _tokens(7, S), _tokens(8, S - pad)
    ids = torch.stack([a, torch.cat([torch.zeros(pad, dtype=torch.long), b])])
    am = torch.ones(2, S, dtype=torch.long)
    am[1, :pad] = 0
    pos = (am.cumsum(-1) - 1).clamp(min=0)
    masked = []
    orig = ka.prefill_attention

    def spy(*args, mask=None, **kw):
        masked.append(mask is not None)
        return orig(*args, mask=mask, **kw)

    monkeypatch.setattr(ka, "prefill_attention", spy)

    def run(ids, am=None, pos=None):
        cfg = KVOffloadConfig.from_model(model, page_size=PAGE, cont_capacity=0,
                                         gpu_watermark_bytes=10 ** 12)
        mgr = KVOffloadManager(model, cfg, batch_size=ids.shape[0])
        try:
            mgr.reset()
            with torch.no_grad():
                out = model(input_ids=ids.cuda(), use_cache=False,
                            attention_mask=None if am is None else am.cuda(),
                            position_ids=None if pos is None else pos.cuda())
            torch.cuda.synchronize()
        finally:
            mgr.restore()
        return out.logits.float().cpu().numpy()

    print("[dropin] left-padded batch 2 prefill", flush=True)
    padded = run(ids, am, pos)
    assert masked and all(masked), "the padding mask did not reach helm_prefill_attn_mask"
    masked.clear()
    single_a = run(a[None])[0]
    single_b = run(b[None])[0]
    assert masked and not any(masked)      # unpadded prompts take the causal kernel
    err_a = float(np.abs(padded[0] - single_a).max())
    err_b = float(np.abs(padded[1, pad:] - single_b).max())
    assert err_a <= LOGIT_ATOL and err_b <= LOGIT_ATOL, (err_a, err_b)


@pytest.mark.parametrize("shape", [(1, 1), (2, 1), (4, 1), (1, 16), (3, 5), (1, 20)])
def test_patched_mlp_matches_the_unfused_module(shape):
    """The decode MLP patch (gate, up and the SiLU product in one launch) against
    transformers' own Qwen3MLP.forward over the same Int8Linear leaves, 8B shape
    (hidden 4096, FFN 12288): bit-equal at 1-2 tokens (the same GEMV rows, the
    same roundings); from 3 tokens the one-launch form sums K in another order
    (fp32), so within a few fp16 ulps of the output scale; past 16 tokens the
    original forward runs (bit-equal)."""
    import transformers.models.qwen3.modeling_qwen3 as m
    from transformers import Qwen3Config
    cfg = Qwen3Config(hidden_size=4096, intermediate_size=12288, hidden_act="silu")
    torch.manual_seed(0)
    mlp = m.Qwen3MLP(cfg)
    with torch.no_grad():
        for p in mlp.parameters():
            p.normal_(0.0, 0.02)
    mlp = mlp.half().cuda().eval()
    patch_linears(mlp)
    x = torch.randn(*shape, 4096, dtype=torch.float16, device="cuda")
    orig = m.Qwen3MLP.forward
    with torch.no_grad():
        ref = orig(mlp, x)
        tiny = m.Qwen3ForCausalLM(Qwen3Config(vocab_size=64, hidden_size=64, intermediate_size=128,
                                              num_hidden_layers=1, num_attention_heads=4,
                                              num_key_value_heads=2, max_position_embeddings=64))
        mgr = KVOffloadManager(tiny, KVOffloadConfig.from_model(tiny, page_size=4, cont_capacity=0,
                                                                fuse_decoder_layers=True))
        try:
            assert m.Qwen3MLP.forward is not orig
            got = mlp(x)
        finally:
            mgr.restore()
    assert m.Qwen3MLP.forward is orig
    assert got.shape == ref.shape and got.dtype == torch.float16
    tokens = shape[0] * shape[1]
    if tokens <= 2 or tokens > 16:
        assert torch.equal(got, ref)
    else:
        scale = float(ref.abs().max())
        assert float((got.float() - ref.float()).abs().max()) <= 4 * 2.0 ** -11 * scale


@pytest.mark.parametrize("shape", [(1, 1, 4096), (2, 7, 4096), (1, 2048, 4096), (3, 1, 8, 128),
                                   (1, 5, 5120)])
def test_patched_rmsnorm_matches_the_module(shape):
    """The decoder RMSNorm patch (one helm_rmsnorm launch) against transformers'
    own Qwen3RMSNorm.forward, fp16 on the GPU: the same roundings (fp16 of
    x * rstd, then fp16 of w times it), the fp32 sum of squares in another order,
    so an output may move by an ulp of x * rstd and of the product; a tensor that
    needs a gradient keeps the original forward (bit-equal)."""
    import transformers.models.qwen3.modeling_qwen3 as m
    from transformers import Qwen3Config
    torch.manual_seed(1)
    norm = m.Qwen3RMSNorm(shape[-1], eps=1e-6)
    with torch.no_grad():
        norm.weight.normal_(1.0, 0.3)
    norm = norm.half().cuda()
    x = (torch.randn(*shape, device="cuda") * 3).half()
    orig = m.Qwen3RMSNorm.forward
    tiny = m.Qwen3ForCausalLM(Qwen3Config(vocab_size=64, hidden_size=64, intermediate_size=128,
                                          num_hidden_layers=1, num_attention_heads=4,
                                          num_key_value_heads=2, max_position_embeddings=64))
    with torch.no_grad():
        ref = orig(norm, x)
    mgr = KVOffloadManager(tiny, KVOffloadConfig.from_model(tiny, page_size=4, cont_capacity=0,
                                                            fuse_decoder_layers=True))
    try:
        with torch.no_grad():
            got = norm(x)
        with torch.enable_grad():
            kept = norm(x)              # the weight needs a gradient: original forward
    finally:
        mgr.restore()
    assert m.Qwen3RMSNorm.forward is orig
    assert got.shape == ref.shape and got.dtype == torch.float16
    assert torch.equal(kept.detach(), ref) and kept.requires_grad
    # |w * t| moves by at most an ulp of t scaled by |w| plus the product's own ulp
    # (doubled: t below is the fp32 value, whose binade may sit one below the fp16's)
    w = norm.weight.float()
    t = (x.float() / (x.float().pow(2).mean(-1, keepdim=True) + 1e-6).sqrt()).abs()
    ulp = lambda v: torch.exp2(torch.floor(torch.log2(v.clamp_min(2.0 ** -14)))) * 2.0 ** -10
    bound = 2 * (ulp(t) * w.abs() + ulp(ref.float().abs()))
    assert bool(((got.float() - ref.float()).abs() <= bound).all())
    assert float((got != ref).float().mean()) < 0.05   # most outputs bit-equal


def _decoder_patch_spread(model, B, S, N, vocab):
    """Teacher-forced logits of a drop-in run with the decoder-layer patch and of
    the same run with transformers' own Qwen3DecoderLayer.forward (attention,
    MLP and norm patches on in both); returns the largest difference."""
    import transformers.models.qwen3.modeling_qwen3 as m
    g = torch.Generator().manual_seed(300 + B)
    prompts = torch.randint(0, vocab, (B, S), generator=g)
    forced = torch.randint(0, vocab, (B, N), generator=g)
    orig_layer = m.Qwen3DecoderLayer.forward
    outs = []
    for fused in (True, False):
        cfg = KVOffloadConfig.from_model(model, page_size=PAGE, cont_capacity=0,
                                         fuse_decoder_layers=True)
        mgr = KVOffloadManager(model, cfg, batch_size=B)
        try:
            assert m.Qwen3DecoderLayer.forward is not mgr._patched["qwen3_layer"][1]
            if not fused:
                m.Qwen3DecoderLayer.forward = mgr._patched["qwen3_layer"][1]
            rt = PipelineRuntime(model, kv_offload_mgr=mgr)
            mgr.reset()
            logits = [rt.prefill(prompts.cuda())[:, -1].float().cpu()]
            for i in range(N - 1):
                logits.append(rt.decode_step(forced[:, i:i + 1].cuda(), S + i)[:, -1].float().cpu())
        finally:
            mgr.restore()
        outs.append(torch.stack(logits, 1))
    assert m.Qwen3DecoderLayer.forward is orig_layer
    return float((outs[0] - outs[1]).abs().max())


@pytest.mark.parametrize("batch", [1, 4])
def test_patched_decoder_layer_matches_the_module_forward(model, batch):
    """The decoder-layer patch (residual adds in the o / down GEMV epilogues, the
    post-attention norm inside the gate / up GEMV) against the same drop-in run
    with transformers' own Qwen3DecoderLayer.forward: teacher-forced logits
    within the spread of a norm's fp32 summation order (bar 1e-2 on logits of
    magnitude ~1)."""
    diff = _decoder_patch_spread(model, batch, 40, 12, QWEN3_PLUMBING.vocab)
    assert diff <= 1e-2, f"decoder patch moves logits by {diff}"


def test_patched_decoder_layer_at_hidden_4096_batch_8():
    """The same comparison at the 8B layer shape (hidden 4096, 32 / 8 heads,
    FFN 12288; 2 layers, vocab 2048, N(0, 0.02) weights, norm weights
    1 + N(0, 0.1)) with 8 sequences, so every decode-step GEMV with the norm
    prologue takes the matrix-core small-M forms; same 1e-2 bar on logits of
    magnitude ~1."""
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(vocab_size=2048, hidden_size=4096, intermediate_size=12288,
                      num_hidden_layers=2, num_attention_heads=32, num_key_value_heads=8,
                      head_dim=128, rms_norm_eps=1e-6, rope_theta=1e6,
                      max_position_embeddings=4096, tie_word_embeddings=False,
                      attention_bias=False)
    cfg._attn_implementation = "sdpa"
    gen = torch.Generator(device="cuda").manual_seed(7)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float16)
    try:
        with torch.device("cuda"), torch.no_grad():
            m4k = Qwen3ForCausalLM(cfg).eval()
            for prm in m4k.parameters():
                if prm.dim() == 2:
                    prm.normal_(0.0, 0.02, generator=gen)
                else:
                    prm.normal_(1.0, 0.1, generator=gen)
    finally:
        torch.set_default_dtype(prev)
    assert patch_linears(m4k, exclude=("lm_head",)) == 14
    try:
        diff = _decoder_patch_spread(m4k, 8, 24, 6, 2048)
    finally:
        del m4k
        torch.cuda.empty_cache()
    assert diff <= 1e-2, f"decoder patch moves logits by {diff}"


@pytest.mark.parametrize("fused", [False, True], ids=["attention_patch", "fused_layers"])
@pytest.mark.parametrize("B,cont", [(1, 0), (1, 4096), (4, 0), (4, 4096)])
def test_graph_replay_equals_eager_planned_steps(model, B, cont, fused):
    """PipelineRuntime replays planned decode steps (bookkeeping for every layer
    before the forward) from HIP graphs.  Against the same planned steps run
    eagerly (decode_graphs=False): bit-identical logits over 48 steps whose
    context crosses a 64-page bucket (1024 tokens, a re-capture) and several
    page boundaries, and identical page tables; the graphs were used."""
    S, N = 1000, 48
    prompts = torch.stack([_tokens(500 + b, S) for b in range(B)]).cuda()
    forced = torch.stack([_tokens(600 + b, N) for b in range(B)]).cuda()
    runs, tables, keys = [], [], []
    for graphs in (True, False):
        cfg = KVOffloadConfig.from_model(model, page_size=PAGE, cont_capacity=cont,
                                         gpu_watermark_bytes=10 ** 12, fuse_decoder_layers=fused)
        mgr = KVOffloadManager(model, cfg, batch_size=B)
        try:
            rt = PipelineRuntime(model, kv_offload_mgr=mgr, decode_graphs=graphs)
            mgr.reset()
            rt.prefill(prompts)
            out, seen = [], set()
            for i in range(N):
                out.append(rt.decode_step(forced[:, i:i + 1], S + i)[:, -1].float().cpu())
                if rt._graphs is not None:
                    seen.add(rt._graphs.key)
            torch.cuda.synchronize()
            assert rt.decode_graphs == graphs
            keys.append(seen)
            tables.append([[(lid, [(p.page_id, p.state, p.slot, p.start_token, p.used_tokens)
                                   for p in L.pages], L.total_tokens) for lid, L in m.layers.items()]
                           for m in mgr.kvcms])
            if cont:
                assert all(m.cont_seq_len == S + N for m in mgr.kvcms)
        finally:
            mgr.restore()
        runs.append(torch.stack(out, 1))
    assert len(keys[0]) >= 2, "expected a re-capture at the 1024-token bucket"
    assert not keys[1]
    assert tables[0] == tables[1]
    assert torch.equal(runs[0], runs[1]), float((runs[0] - runs[1]).abs().max())


def test_hooked_modules_take_the_original_forwards(model):
    """A forward hook on a module the fused paths would call past (an MLP
    projection, the post-attention norm, a q / k / v projection) makes those
    paths run the module itself: the hooks fire on every decode step, and the
    logits equal the unhooked run within the decoder-patch bar."""
    B, S, N = 1, 40, 6
    prompts = torch.stack([_tokens(700, S)]).cuda()
    forced = torch.stack([_tokens(701, N)]).cuda()
    layer = model.model.layers[0]
    targets = [layer.mlp.gate_proj, layer.post_attention_layernorm, layer.self_attn.k_proj,
               layer.input_layernorm, layer.self_attn.o_proj]
    outs = []
    for hooked in (False, True):
        calls = {id(t): 0 for t in targets}
        handles = []
        if hooked:
            for t in targets:
                def hook(mod, args, out, key=id(t)):
                    calls[key] += 1
                handles.append(t.register_forward_hook(hook))
        cfg = KVOffloadConfig.from_model(model, page_size=PAGE, cont_capacity=0,
                                         fuse_decoder_layers=True)
        mgr = KVOffloadManager(model, cfg, batch_size=B)
        try:
            rt = PipelineRuntime(model, kv_offload_mgr=mgr, decode_graphs=False)
            mgr.reset()
            logits = [rt.prefill(prompts)[:, -1].float().cpu()]
            for i in range(N - 1):
                logits.append(rt.decode_step(forced[:, i:i + 1], S + i)[:, -1].float().cpu())
        finally:
            mgr.restore()
            for h in handles:
                h.remove()
        outs.append(torch.stack(logits, 1))
        if hooked:
            assert all(c == N for c in calls.values()), calls   # prefill + N - 1 decode steps
    assert float((outs[0] - outs[1]).abs().max()) <= 1e-2


@pytest.mark.parametrize("cont,watermark,in_place", [(0, 10 ** 12, True), (4096, None, True),
                                                     (0, 4 * 2 * 8 * PAGE * 64 * 2, False)],
                         ids=["pages_in_hbm", "contiguous", "pages_on_host"])
def test_prefill_attention_reads_the_appended_kv_in_place(model, monkeypatch, cont, watermark,
                                                          in_place):
    """The drop-in prefill attends each item's prompt K/V where the appends just
    wrote it (the contiguous buffer, or the device pool's pages) rather than a
    dense page-layout copy: the same tokens in the same 16-token pages, so the
    logits equal, bit for bit, those of a run forced onto the copy.  With pages
    evicted to the host during the prefill the copy is what runs."""
    B, S = 2, 500                      # a partial last page
    prompts = torch.stack([_tokens(40 + b, S) for b in range(B)])
    forced = torch.stack([_tokens(140 + b, 3) for b in range(B)])
    real = KVOffloadManager._prefill_kv_source
    used = []

    def spy(self, *args):
        r = real(self, *args)
        used.append(r is not None)
        return r
    monkeypatch.setattr(KVOffloadManager, "_prefill_kv_source", spy)
    logits, _ = _run_dropin(model, prompts, forced, cont=cont, watermark=watermark)
    assert len(used) == B * QWEN3_PLUMBING.n_layers
    if in_place:
        assert all(used)
    else:
        assert not all(used)
    monkeypatch.setattr(KVOffloadManager, "_prefill_kv_source", lambda self, *args: None)
    dense, _ = _run_dropin(model, prompts, forced, cont=cont, watermark=watermark)
    assert np.array_equal(logits, dense)


@pytest.mark.parametrize("page", [16, 32, 64])
@pytest.mark.parametrize("fused", [False, True], ids=["attention_patch", "fused_layers"])
def test_contiguous_and_paged_paths_give_the_same_bits(model, page, fused):
    """Path 1 (contiguous buffers: K token rows, V in page blocks, read as pages of
    P tokens) and Path 2 (the device pool's pages) hand the kernels the same tokens
    in the same P-token pages, so prefill and every decode step give the same
    logits, bit for bit, at each page size the kernels take.  (A planned step's
    table width, and with it the split count, is the context rounded up to 64
    pages, capped by the buffer's pages in Path 1: 4096 tokens keep that cap out
    of the way at every page size.)"""
    B, S, N = 2, 300, 6
    prompts = torch.stack([_tokens(60 + b, S) for b in range(B)])
    forced = torch.stack([_tokens(160 + b, N) for b in range(B)])
    cont, m1 = _run_dropin(model, prompts, forced, cont=4096, fused=fused, page_size=page)
    assert all(m.use_contiguous for m in m1.kvcms)
    paged, m2 = _run_dropin(model, prompts, forced, cont=0, watermark=10 ** 12, fused=fused,
                            page_size=page)
    assert not any(m.use_contiguous for m in m2.kvcms)
    assert np.array_equal(cont, paged)
