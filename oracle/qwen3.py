"""Oracle for the end-to-end decode step — TEST INFRASTRUCTURE ONLY.

fp32 numpy restatement of the Qwen3 decoder the reference patches and drives:
  * the patched attention forward (helm/runtime/kv_offload.py:241-271):
    q = q_norm(q_proj(x)), k = k_norm(k_proj(x)), v = v_proj(x), RoPE
    (rotate_half convention, angle = inv_freq * position), scale 1/sqrt(D),
    GQA attention over all cached tokens (causal in prefill), o_proj;
  * the decoder layer around it (transformers Qwen3DecoderLayer): RMSNorm
    x * rsqrt(mean(x^2) + eps) * w, residual adds, SwiGLU MLP
    down(silu(gate(x)) * up(x));
  * the greedy loop (helm/runtime/pipeline_runtime.py:140-176): first token =
    argmax of the prefill logits, then one token per step at position
    prompt_len + step.

Weights are the dequantised INT8 weights (q * scale), so the oracle computes the
model the INT8 kernels implement, in fp32 without intermediate fp16 rounding.

Pinning (tests/test_oracle_qwen3.py): logits equal those of transformers'
Qwen3ForCausalLM (a library implementation, fp32 on the CPU) loaded with the
same weights, for prefill and for teacher-forced decode positions.
"""
from __future__ import annotations

from typing import Dict, List

import numpy as np


def _f32(t) -> np.ndarray:
    if hasattr(t, "detach"):
        return t.detach().float().cpu().numpy()
    return np.asarray(t, np.float32)


class Qwen3Oracle:
    def __init__(self, weights):
        """`weights`: helm_amd.runtime.decode_engine.Int8Qwen3Weights (any device)."""
        sh = weights.shape
        self.sh = sh
        D = sh.head_dim
        self.layers: List[Dict[str, np.ndarray]] = []
        for lay in weights.layers:
            deq = lambda q, s: _f32(q) * _f32(s)[:, None]  # noqa: E731
            qkv = deq(lay["qkv_q"], lay["qkv_s"])
            nq, nk = sh.n_heads * D, sh.n_kv_heads * D
            self.layers.append({
                "q": qkv[:nq], "k": qkv[nq:nq + nk], "v": qkv[nq + nk:],
                "o": deq(lay["o_q"], lay["o_s"]), "gate": deq(lay["gate_q"], lay["gate_s"]),
                "up": deq(lay["up_q"], lay["up_s"]), "down": deq(lay["down_q"], lay["down_s"]),
                "in_ln": _f32(lay["in_ln"]), "post_ln": _f32(lay["post_ln"]),
                "q_norm": _f32(lay["q_norm"]), "k_norm": _f32(lay["k_norm"]),
            })
        self.embed = _f32(weights.embed)
        self.norm = _f32(weights.norm)
        self.lm_head = _f32(weights.lm_head)
        self.inv_freq = (1.0 / (sh.rope_theta ** (np.arange(0, D, 2, dtype=np.float32) / D))).astype(np.float32)

    def _rms(self, x, w):
        return x / np.sqrt((x * x).mean(-1, keepdims=True) + self.sh.eps) * w

    def _rope(self, x, pos):
        # x [heads, S, D]; pos [S]
        ang = pos[:, None].astype(np.float32) * self.inv_freq[None, :]
        emb = np.concatenate([ang, ang], -1)
        cos, sin = np.cos(emb), np.sin(emb)
        h = x.shape[-1] // 2
        rot = np.concatenate([-x[..., h:], x[..., :h]], -1)
        return x * cos + rot * sin

    def forward(self, tokens: np.ndarray) -> np.ndarray:
        """Causal forward over the whole token sequence; returns fp32 logits [S, V]."""
        sh = self.sh
        D = sh.head_dim
        S = len(tokens)
        pos = np.arange(S)
        h = self.embed[np.asarray(tokens)]
        mask = np.triu(np.full((S, S), -np.inf, np.float32), 1)
        g = sh.n_heads // sh.n_kv_heads
        for L in self.layers:
            x = self._rms(h, L["in_ln"])
            q = (x @ L["q"].T).reshape(S, sh.n_heads, D)
            k = (x @ L["k"].T).reshape(S, sh.n_kv_heads, D)
            v = (x @ L["v"].T).reshape(S, sh.n_kv_heads, D)
            q = self._rope(self._rms(q, L["q_norm"]).transpose(1, 0, 2), pos)
            k = self._rope(self._rms(k, L["k_norm"]).transpose(1, 0, 2), pos)
            v = v.transpose(1, 0, 2)
            k = np.repeat(k, g, axis=0)
            v = np.repeat(v, g, axis=0)
            s = q @ k.transpose(0, 2, 1) / np.sqrt(D) + mask
            s = s - s.max(-1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(-1, keepdims=True)
            a = (p @ v).transpose(1, 0, 2).reshape(S, -1)
            h = h + a @ L["o"].T
            x = self._rms(h, L["post_ln"])
            gt = x @ L["gate"].T
            up = x @ L["up"].T
            h = h + (gt / (1 + np.exp(-gt)) * up) @ L["down"].T
        return self._rms(h, self.norm) @ self.lm_head.T

    def greedy(self, prompt: np.ndarray, max_new_tokens: int) -> np.ndarray:
        seq = list(np.asarray(prompt))
        out = []
        for _ in range(max_new_tokens):
            t = int(np.argmax(self.forward(np.asarray(seq))[-1]))
            out.append(t)
            seq.append(t)
        return np.asarray(out)


def hf_model_from_weights(weights, dtype=None):
    """transformers Qwen3ForCausalLM (CPU) carrying the same dequantised weights."""
    import torch
    from transformers import Qwen3Config, Qwen3ForCausalLM

    sh = weights.shape
    cfg = Qwen3Config(vocab_size=sh.vocab, hidden_size=sh.hidden, intermediate_size=sh.ffn,
                      num_hidden_layers=sh.n_layers, num_attention_heads=sh.n_heads,
                      num_key_value_heads=sh.n_kv_heads, head_dim=sh.head_dim,
                      rms_norm_eps=sh.eps, rope_theta=sh.rope_theta,
                      max_position_embeddings=40960, tie_word_embeddings=False,
                      attention_bias=False)
    cfg._attn_implementation = "eager"
    model = Qwen3ForCausalLM(cfg).eval()
    orc = Qwen3Oracle(weights)
    with torch.no_grad():
        for hl, L in zip(model.model.layers, orc.layers):
            at, mlp = hl.self_attn, hl.mlp
            for mod, key in ((at.q_proj, "q"), (at.k_proj, "k"), (at.v_proj, "v"), (at.o_proj, "o"),
                             (mlp.gate_proj, "gate"), (mlp.up_proj, "up"), (mlp.down_proj, "down")):
                mod.weight.copy_(torch.from_numpy(L[key]))
            hl.input_layernorm.weight.copy_(torch.from_numpy(L["in_ln"]))
            hl.post_attention_layernorm.weight.copy_(torch.from_numpy(L["post_ln"]))
            at.q_norm.weight.copy_(torch.from_numpy(L["q_norm"]))
            at.k_norm.weight.copy_(torch.from_numpy(L["k_norm"]))
        model.model.embed_tokens.weight.copy_(torch.from_numpy(orc.embed))
        model.model.norm.weight.copy_(torch.from_numpy(orc.norm))
        model.lm_head.weight.copy_(torch.from_numpy(orc.lm_head))
    if dtype is not None:
        model = model.to(dtype)
    return model
