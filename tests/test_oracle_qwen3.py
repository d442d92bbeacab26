"""Pins the end-to-end oracle (oracle/qwen3.py) to transformers' Qwen3ForCausalLM
(a library implementation, fp32 on the CPU) on the plumbing configuration:
hidden 1024, 16 q / 8 kv heads, head_dim 64, FFN 3072, eps 1e-6, theta 1e6,
vocab 32000, 2 layers, weights N(0, 0.02) INT8 per channel (dequantised)."""
import numpy as np
import pytest
import torch

from helm_amd.runtime.decode_engine import QWEN3_PLUMBING, Int8Qwen3Weights
from oracle.qwen3 import Qwen3Oracle, hf_model_from_weights


@pytest.fixture(scope="module")
def setup():
    w = Int8Qwen3Weights.random(QWEN3_PLUMBING, "cpu", seed=0, norm_jitter=0.1)
    return w, Qwen3Oracle(w), hf_model_from_weights(w)


def test_prefill_logits_match_transformers(setup):
    _, orc, hf = setup
    toks = np.random.default_rng(1).integers(0, 32000, 48)
    lo = orc.forward(toks)
    with torch.no_grad():
        lh = hf(torch.from_numpy(toks)[None]).logits[0].numpy()
    assert np.abs(lo - lh).max() < 1e-4


def test_greedy_matches_transformers_generate(setup):
    _, orc, hf = setup
    prompt = np.random.default_rng(2).integers(0, 32000, 16)
    ours = orc.greedy(prompt, 6)
    with torch.no_grad():
        out = hf.generate(torch.from_numpy(prompt)[None], max_new_tokens=6, do_sample=False,
                          pad_token_id=0)
    assert ours.tolist() == out[0, 16:].tolist()


def test_dropped_term_is_detected(setup):
    """A plausible slip (RoPE sign flipped) changes the logits well beyond the bar."""
    w, orc, _ = setup
    toks = np.random.default_rng(3).integers(0, 32000, 24)
    good = orc.forward(toks)
    bad = Qwen3Oracle(w)
    bad.inv_freq = -bad.inv_freq
    assert np.abs(bad.forward(toks) - good).max() > 1e-2
