"""The batched decode engine (BatchDecodeEngine) on the plumbing configuration
(2 layers, hidden 1024, 16/8 heads, D 64, FFN 3072, vocab 32000, INT8 weights
N(0,0.02), page 16): each item of a batch, with prompts of different lengths,
teacher-forced against the fp32 oracle run on that item alone (the reference's
batched decode keeps items independent, kv_offload.py:82-167), at batch sizes
that take the fused-norm GEMVs (1, 2) and the matrix-core GEMVs (3-16); graph
replay equal to eager execution.

Bar: max(2e-2, 1.5 x the fp16 torch model's error) on the teacher-forced
logits, as the batch-1 engine tests."""
import dataclasses

import numpy as np
import pytest
import torch

from helm_amd.runtime.batch_engine import BatchDecodeEngine
from helm_amd.runtime.decode_engine import QWEN3_PLUMBING, Int8Qwen3Weights
from oracle.qwen3 import Qwen3Oracle, hf_model_from_weights

pytestmark = pytest.mark.gpu
LOGIT_ATOL = 2e-2
NEW = 10
PROMPTS = [300, 77, 512, 129, 200, 33, 450, 64]   # ragged lengths (partial last pages)


@pytest.fixture(scope="module")
def weights():
    return Int8Qwen3Weights.random(QWEN3_PLUMBING, torch.device("cuda"), seed=0, norm_jitter=0.1)


@pytest.fixture(scope="module")
def oracle(weights):
    return Qwen3Oracle(weights)


def _cpu_weights(weights, shape=QWEN3_PLUMBING):
    w = Int8Qwen3Weights(shape)
    w.layers = [{k: v.cpu() for k, v in lay.items()} for lay in weights.layers]
    w.embed, w.norm, w.lm_head = weights.embed.cpu(), weights.norm.cpu(), weights.lm_head.cpu()
    return w


def _tokens(seed, n):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, QWEN3_PLUMBING.vocab, (n,), generator=g)


@pytest.fixture(scope="module")
def items(oracle):
    """Per item: prompt, forced tokens, the oracle's teacher-forced logits."""
    out = []
    for i, n in enumerate(PROMPTS):
        prompt, forced = _tokens(10 + i, n), _tokens(50 + i, NEW)
        seq = np.concatenate([prompt.numpy(), forced[:-1].numpy()])
        out.append((prompt, forced, oracle.forward(seq)[n - 1:]))
    return out


@pytest.fixture(scope="module")
def tol(weights, items):
    """max(2e-2, 1.5 x the error of plain fp16 torch against the oracle) on item 0."""
    prompt, forced, ref = items[0]
    m = hf_model_from_weights(_cpu_weights(weights), dtype=torch.float16).cuda()
    m.config._attn_implementation = "sdpa"
    seq = torch.cat([prompt, forced[:-1]])[None].cuda()
    with torch.no_grad():
        ref16 = m(seq).logits[0, len(prompt) - 1:].float().cpu().numpy()
    del m
    return max(LOGIT_ATOL, 1.5 * float(np.abs(ref16 - ref).max()))


def run_batch(weights, items, B, use_graph=True):
    """Teacher-forced batch run: logits [B, NEW, V] (the prefill's last position,
    then one decode step per forced token)."""
    its = items[:B]
    eng = BatchDecodeEngine(weights, B, max_context=max(len(p) for p, _, _ in its) + NEW + 16,
                            use_graph=use_graph)
    logits = [[eng.prefill(i, p.cuda()).float().cpu()] for i, (p, _, _) in enumerate(its)]
    forced = torch.stack([f for _, f, _ in its]).cuda()
    eng.tok.copy_(forced[:, 0])
    for s in range(NEW - 1):
        eng.decode_step()
        lg = eng.step_logits().float().cpu()
        for i in range(B):
            logits[i].append(lg[i])
        eng.tok.copy_(forced[:, s + 1])
    return np.stack([torch.stack(x).numpy() for x in logits]), eng


@pytest.mark.parametrize("B", [1, 2, 3, 8])
def test_batch_items_match_oracle(weights, items, tol, B):
    print(f"[batch engine] B={B}", flush=True)
    logits, eng = run_batch(weights, items, B)
    assert eng.seq == [PROMPTS[i] + NEW - 1 for i in range(B)]
    for i in range(B):
        err = float(np.abs(logits[i] - items[i][2]).max())
        assert err <= tol, f"B={B} item {i}: teacher-forced logits max err {err} > {tol}"


def test_batch_graph_equals_eager(weights, items):
    print("[batch engine] graph vs eager, B=4", flush=True)
    g, _ = run_batch(weights, items, 4, use_graph=True)
    e, _ = run_batch(weights, items, 4, use_graph=False)
    assert np.array_equal(g, e)


def test_batch_greedy_tokens_follow_logits(weights, items):
    """Free-running greedy decode: every step's token is the argmax of that
    step's logits, for every item."""
    B = 5
    eng = BatchDecodeEngine(weights, B, max_context=600)
    for i in range(B):
        eng.prefill(i, items[i][0].cuda())
    for _ in range(6):
        tok = eng.decode_step().clone()
        assert torch.equal(tok, torch.argmax(eng.step_logits().float(), dim=-1))


def test_batch_split_k_down_projection():
    """Batch 8 with FFN 6144: the down projection (6144 -> 1024) takes the split-K
    small-M form (partial sums in the engine's workspace, one reduce kernel);
    every item teacher-forced against the oracle, graph replay as the other
    tests."""
    shape = dataclasses.replace(QWEN3_PLUMBING, ffn=6144)
    w = Int8Qwen3Weights.random(shape, torch.device("cuda"), seed=3, norm_jitter=0.1)
    orc = Qwen3Oracle(w)
    prompts = [100, 37, 64, 129, 80, 33, 50, 65]
    its = []
    for i, n in enumerate(prompts):
        prompt, forced = _tokens(70 + i, n), _tokens(90 + i, NEW)
        seq = np.concatenate([prompt.numpy(), forced[:-1].numpy()])
        its.append((prompt, forced, orc.forward(seq)[n - 1:]))
    logits, eng = run_batch(w, its, 8)
    assert eng.gemv_ws_bytes > 0, "the down projection should take the split form at batch 8"
    assert eng.seq == [n + NEW - 1 for n in prompts]
    m = hf_model_from_weights(_cpu_weights(w, shape), dtype=torch.float16).cuda()
    m.config._attn_implementation = "sdpa"
    prompt, forced, ref = its[0]
    with torch.no_grad():
        ref16 = m(torch.cat([prompt, forced[:-1]])[None].cuda()).logits[0, len(prompt) - 1:]
    tol = max(LOGIT_ATOL, 1.5 * float(np.abs(ref16.float().cpu().numpy() - ref).max()))
    del m
    for i in range(8):
        err = float(np.abs(logits[i] - its[i][2]).max())
        assert err <= tol, f"item {i}: teacher-forced logits max err {err} > {tol}"


@pytest.fixture(scope="module")
def wide_model():
    """Hidden 4096 (32 / 8 heads, D 128, FFN 6144, 2 layers, vocab 32000): the
    weights, 16 items (prompt, forced tokens, oracle logits) and the logit bar
    (as `tol`, from item 0)."""
    from helm_amd.runtime.batch_engine import FUSED_NORM_HIDDEN
    shape = dataclasses.replace(QWEN3_PLUMBING, hidden=FUSED_NORM_HIDDEN, n_heads=32,
                                n_kv_heads=8, head_dim=128, ffn=6144)
    w = Int8Qwen3Weights.random(shape, torch.device("cuda"), seed=5, norm_jitter=0.1)
    orc = Qwen3Oracle(w)
    prompts = [64, 33, 100, 17, 80, 50, 29, 96, 41, 70, 23, 88, 55, 19, 66, 37]
    its = []
    for i, n in enumerate(prompts):
        prompt, forced = _tokens(110 + i, n), _tokens(130 + i, NEW)
        seq = np.concatenate([prompt.numpy(), forced[:-1].numpy()])
        its.append((prompt, forced, orc.forward(seq)[n - 1:]))
    m = hf_model_from_weights(_cpu_weights(w, shape), dtype=torch.float16).cuda()
    m.config._attn_implementation = "sdpa"
    prompt, forced, ref = its[0]
    with torch.no_grad():
        ref16 = m(torch.cat([prompt, forced[:-1]])[None].cuda()).logits[0, len(prompt) - 1:]
    tol = max(LOGIT_ATOL, 1.5 * float(np.abs(ref16.float().cpu().numpy() - ref).max()))
    del m
    return w, its, tol


@pytest.mark.parametrize("B", [4, 8, 16])
def test_batch_hidden_4096_matrix_core_forms(wide_model, B):
    """Batches of 4, 8 and 16 at hidden 4096: every layer takes the matrix-core
    forms of the Qwen3-8B step at that item count: RMSNorm + q|k|v (fused up to 4
    items, else the RMSNorm kernel and four waves sharing x at 8 / eight at 16),
    RMSNorm + gate / up + SwiGLU in one launch, the down projection (split K from
    8 items) and the fp16 lm_head; each item teacher-forced against the oracle."""
    w, its, tol = wide_model
    logits, eng = run_batch(w, its, B)
    assert (eng.gemv_ws_bytes > 0) == (B >= 8)
    for i in range(B):
        err = float(np.abs(logits[i] - its[i][2]).max())
        assert err <= tol, f"B={B} item {i}: teacher-forced logits max err {err} > {tol}"
