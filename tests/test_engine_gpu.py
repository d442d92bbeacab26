"""End-to-end decode on the GPU: the fused graph engine and the HF drop-in path
(KVOffloadManager + PipelineRuntime) against the fp32 oracle, on the plumbing
configuration (2 layers, hidden 1024, 16/8 heads, D 64, FFN 3072, vocab 32000,
INT8 weights N(0,0.02), 512-token prompt, 64 greedy tokens, page 16).

Bar: teacher-forced logits within max(2e-2, 1.5 x floor) of the oracle's fp32
logits, where floor is the error of the same model run in fp16 by plain torch
on the GPU (transformers Qwen3ForCausalLM with the dequantised weights — the
reference's own numerics: activations rounded to fp16 at every op boundary);
greedy tokens equal to the oracle's wherever the oracle's top-2 margin exceeds
twice the bar.  Graph replay and eager execution of the engine are bit-identical.
"""
import numpy as np
import pytest
import torch

from helm_amd.runtime.decode_engine import QWEN3_PLUMBING, DecodeEngine, Int8Qwen3Weights
from oracle.qwen3 import Qwen3Oracle

pytestmark = pytest.mark.gpu
LOGIT_ATOL = 2e-2
PROMPT, NEW = 512, 64


@pytest.fixture(scope="module")
def weights():
    return Int8Qwen3Weights.random(QWEN3_PLUMBING, torch.device("cuda"), seed=0, norm_jitter=0.1)


@pytest.fixture(scope="module")
def prompt():
    g = torch.Generator().manual_seed(1)
    return torch.randint(0, QWEN3_PLUMBING.vocab, (PROMPT,), generator=g)


def run_engine(weights, prompt, use_graph=True, watermark=None, forced=None, fused=True,
               int8_head=False):
    """Greedy run; with `forced` tokens the engine is teacher-forced (each decode
    step consumes forced[i] instead of its own previous argmax)."""
    eng = DecodeEngine(weights, max_context=PROMPT + NEW + 16, page_size=16,
                       gpu_watermark_bytes=watermark, use_graph=use_graph, fused_attention=fused,
                       int8_lm_head=int8_head)
    logits = [eng.prefill(prompt.cuda()).float().cpu()]
    toks = [int(torch.argmax(logits[0]))]
    eng.tok.fill_(toks[0] if forced is None else int(forced[0]))
    for i in range(NEW - 1):
        eng.decode_step()
        logits.append(eng.step_logits().float().cpu())
        toks.append(int(eng.tok))
        if forced is not None:
            eng.tok.fill_(int(forced[i + 1]))
    return np.array(toks), torch.stack(logits).numpy(), eng


@pytest.fixture(scope="module")
def engine_run(weights, prompt):
    return run_engine(weights, prompt)


@pytest.fixture(scope="module")
def oracle_logits(weights, prompt, engine_run):
    toks = engine_run[0]
    seq = np.concatenate([prompt.numpy(), toks[:-1]])
    return Qwen3Oracle(weights).forward(seq)[PROMPT - 1:]


def cpu_weights(weights):
    w = Int8Qwen3Weights(QWEN3_PLUMBING)
    w.layers = [{k: v.cpu() for k, v in lay.items()} for lay in weights.layers]
    w.embed, w.norm, w.lm_head = weights.embed.cpu(), weights.norm.cpu(), weights.lm_head.cpu()
    return w


@pytest.fixture(scope="module")
def tol(weights, prompt, engine_run, oracle_logits):
    """max(2e-2, 1.5 x the fp16 torch model's error against the oracle)."""
    from oracle.qwen3 import hf_model_from_weights
    model = hf_model_from_weights(cpu_weights(weights), dtype=torch.float16).cuda()
    model.config._attn_implementation = "sdpa"
    seq = torch.from_numpy(np.concatenate([prompt.numpy(), engine_run[0][:-1]]))[None].cuda()
    with torch.no_grad():
        ref16 = model(seq).logits[0, PROMPT - 1:].float().cpu().numpy()
    floor = float(np.abs(ref16 - oracle_logits).max())
    del model
    return max(LOGIT_ATOL, 1.5 * floor)


def check_against_oracle(toks, logits, ref, tol):
    assert logits.shape == ref.shape
    err = np.abs(logits - ref).max()
    assert err <= tol, f"teacher-forced logits max err {err} > {tol}"
    top2 = np.sort(ref, -1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 2 * tol
    assert (toks[clear] == ref.argmax(-1)[clear]).all()
    assert clear.sum() >= NEW // 4


def test_engine_matches_oracle(engine_run, oracle_logits, tol):
    toks, logits, eng = engine_run
    check_against_oracle(toks, logits, oracle_logits, tol)
    assert eng.graph is not None      # the decode steps ran as graph replays
    assert eng.seq == PROMPT + NEW - 1


def test_graph_equals_eager(weights, prompt, engine_run):
    toks_e, logits_e, _ = run_engine(weights, prompt, use_graph=False)
    assert np.array_equal(toks_e, engine_run[0])
    assert np.array_equal(logits_e, engine_run[1])


def test_three_kernel_attention_path_matches(weights, prompt, engine_run, oracle_logits, tol):
    """The unfused step (q/k norm + RoPE kernel, attention, split reduce) agrees with
    the fused one, teacher-forced on the same tokens."""
    toks, logits, eng = run_engine(weights, prompt, forced=engine_run[0], fused=False)
    assert np.abs(logits - oracle_logits).max() <= tol
    assert np.abs(logits - engine_run[1]).max() <= 5e-3


def test_engine_with_host_offload(weights, prompt, engine_run, oracle_logits, tol):
    """A small watermark pushes the oldest pages to pinned host memory during
    prefill; decode then streams them back each step (eager mixed path).
    Teacher-forced on the resident run's tokens so the logits are comparable."""
    page_bytes = 2 * 8 * 16 * 64 * 2
    toks, logits, eng = run_engine(weights, prompt, watermark=8 * page_bytes, forced=engine_run[0])
    n_host = sum(1 for li in range(2) for p in eng.kvcm.layers[li].pages if p.state == "CPU")
    assert n_host > 40
    assert not eng.all_gpu and eng.graph is None
    assert np.abs(logits - oracle_logits).max() <= tol
    assert np.abs(logits - engine_run[1]).max() <= 5e-3


def first_unclear(ref, tol):
    top2 = np.sort(ref, -1)[:, -2:]
    bad = np.nonzero((top2[:, 1] - top2[:, 0]) <= 2 * tol)[0]
    return int(bad[0]) if bad.size else len(ref)


def test_hf_dropin_path_matches(weights, prompt, engine_run, oracle_logits, tol):
    """transformers Qwen3ForCausalLM + patch_linears + KVOffloadManager (class-level
    patched attention) + PipelineRuntime: teacher-forced logits within the bar
    of the oracle, and greedy generate() equal to the oracle's tokens up to the
    first step whose top-2 margin is within tolerance.  Run with the paged path
    (cont_capacity 0) and the contiguous path (4096)."""
    from helm_amd.kernels import patch_linears
    from helm_amd.runtime import KVOffloadConfig, KVOffloadManager, PipelineRuntime
    from oracle.qwen3 import hf_model_from_weights

    model = hf_model_from_weights(cpu_weights(weights), dtype=torch.float16).cuda()
    model.config._attn_implementation = "sdpa"
    assert patch_linears(model, exclude=("lm_head",)) == 14
    forced = engine_run[0]
    n_ok = first_unclear(oracle_logits, tol)
    for cont, fused in ((0, False), (4096, False), (0, True), (4096, True)):
        cfg = KVOffloadConfig.from_model(model, page_size=16, cont_capacity=cont,
                                         fuse_decoder_layers=fused)
        mgr = KVOffloadManager(model, cfg, batch_size=1)
        try:
            rt = PipelineRuntime(model, kv_offload_mgr=mgr)
            out = rt.generate(prompt[None].cuda(), max_new_tokens=NEW)[0].cpu().numpy()
            assert mgr.kvcms[0].use_contiguous == (cont > 0)
            mgr.reset()
            logits = [rt.prefill(prompt[None].cuda())[0, -1].float().cpu()]
            for i in range(NEW - 1):
                tok = torch.tensor([[int(forced[i])]], device="cuda")
                logits.append(rt.decode_step(tok, PROMPT + i)[0, -1].float().cpu())
        finally:
            mgr.restore()
        logits = torch.stack(logits).numpy()
        err = np.abs(logits - oracle_logits).max()
        assert err <= tol, f"cont={cont} fused={fused}: teacher-forced logits max err {err} > {tol}"
        assert (out[:n_ok] == oracle_logits.argmax(-1)[:n_ok]).all(), f"cont={cont} fused={fused}"


def test_engine_int8_lm_head(weights, prompt):
    """INT8 lm_head (per-channel quantised, final RMSNorm fused into the INT8 GEMV):
    teacher-forced logits equal, within the bar, those of the fp16-head engine
    whose lm_head holds the dequantised weights (the same matrix up to the fp16
    rounding of q * s); greedy tokens equal where the margin is clear."""
    import copy
    from helm_amd.kernels import dequantize, quantize_per_channel
    q, s = quantize_per_channel(weights.lm_head)
    wq = copy.copy(weights)
    wq.lm_head = dequantize(q, s).to(torch.float16)
    toks, logits, eng = run_engine(weights, prompt, int8_head=True)
    assert eng.lm_q is not None
    _, ref, _ = run_engine(wq, prompt, forced=toks)
    assert np.abs(logits - ref).max() <= LOGIT_ATOL
    top2 = np.sort(ref, -1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 2 * LOGIT_ATOL
    assert (toks[clear] == ref.argmax(-1)[clear]).all() and clear.sum() >= NEW // 4
