"""Greedy generation loop (mirror of helm/runtime/pipeline_runtime.py).

The reference runs the model as FX stage modules through StageRuntimeExecutor
(a CPU/GPU layer split that is out of scope here); this runtime calls the model
directly on one GPU and keeps the loop's semantics (pipeline_runtime.py:43-176):
prefill with a full causal mask, then one token per step with
position_ids = [[seq_len + step]], next token = argmax(logits[:, -1, :]), and
the KV offload manager reset before every generate().
"""
from __future__ import annotations

import time

import torch


class PipelineRuntime:
    """`PipelineRuntime(model, tokenizer=None, dtype=torch.float16,
    kv_offload_mgr=None)` runs a transformers model directly.  The reference's
    signature `PipelineRuntime(prefill_executor, decode_executor, tokenizer,
    dtype, kv_offload_mgr, decode_wrapper)` (pipeline_runtime.py:23-37) is
    accepted too: with a decode executor every forward goes through
    `decode_executor.run({"input_ids", "attention_mask", "position_ids",
    "cache_position"})` with the reference's masks (a triu causal mask for
    prefill, zeros [1, 1, 1, T] for a decode step) and its output's "logits"."""

    def __init__(self, model, decode_executor=None, tokenizer=None, dtype=torch.float16,
                 kv_offload_mgr=None, decode_wrapper=None):
        if decode_executor is not None and not hasattr(decode_executor, "run"):
            # PipelineRuntime(model, tokenizer, ...) called positionally
            tokenizer, decode_executor = decode_executor, None
        self.model = model
        self.prefill_executor = model if decode_executor is not None else None
        self.decode_executor = decode_executor
        self.tokenizer = tokenizer
        self.dtype = dtype
        self.kv_offload_mgr = kv_offload_mgr
        self.decode_wrapper = decode_wrapper
        self.last_timing = {}

    def _build_causal_mask(self, seq_len, device):
        """Full causal mask for prefill: (1, 1, S, S) (pipeline_runtime.py:43-48)."""
        min_val = torch.finfo(self.dtype).min
        mask = torch.full((seq_len, seq_len), min_val, device=device, dtype=self.dtype)
        return torch.triu(mask, diagonal=1)[None, None, :, :]

    def _build_decode_mask(self, total_len, device):
        """Decode mask: (1, 1, 1, total_len), every earlier position visible
        (pipeline_runtime.py:50-52)."""
        return torch.zeros((1, 1, 1, total_len), device=device, dtype=self.dtype)

    def _forward(self, input_ids, position_ids, attention_mask, cache_position=None):
        if self.decode_executor is not None:
            out = self.decode_executor.run({"input_ids": input_ids, "attention_mask": attention_mask,
                                            "position_ids": position_ids,
                                            "cache_position": cache_position})
            return out["logits"] if isinstance(out, dict) else out
        out = self.model(input_ids=input_ids, position_ids=position_ids,
                         attention_mask=attention_mask, use_cache=False)
        return out.logits if hasattr(out, "logits") else out

    @torch.no_grad()
    def prefill(self, input_ids):
        seq_len = input_ids.shape[1]
        dev = input_ids.device
        position_ids = torch.arange(seq_len, dtype=torch.long, device=dev).unsqueeze(0)
        position_ids = position_ids.expand(input_ids.shape[0], -1)
        if self.decode_executor is not None:
            return self._forward(input_ids, position_ids, self._build_causal_mask(seq_len, dev),
                                 torch.arange(seq_len, device=dev))
        return self._forward(input_ids, position_ids, None)

    @torch.no_grad()
    def decode_step(self, input_ids, step_position):
        dev = input_ids.device
        position_ids = torch.full((input_ids.shape[0], 1), step_position, dtype=torch.long,
                                  device=dev)
        if self.decode_executor is not None:
            return self._forward(input_ids, position_ids,
                                 self._build_decode_mask(step_position + 1, dev),
                                 torch.tensor([step_position], device=dev))
        return self._forward(input_ids, position_ids, None)

    @torch.no_grad()
    def generate(self, input_ids, max_new_tokens=8):
        """Prefill, then greedy decode; returns [B, max_new_tokens] token ids.
        self.last_timing holds ttft_s / decode_s / decode_tok_per_s measured like
        the reference's harness (experiments/paper_bench.py:755-790)."""
        if self.kv_offload_mgr is not None:
            self.kv_offload_mgr.reset()
        seq_len = input_ids.shape[1]
        dev = input_ids.device
        sync = torch.cuda.synchronize if dev.type == "cuda" else (lambda: None)
        sync()
        t0 = time.perf_counter()
        logits = self.prefill(input_ids)
        sync()
        t1 = time.perf_counter()
        generated = []
        for step in range(max_new_tokens):
            next_token = torch.argmax(logits[:, -1, :], dim=-1, keepdim=True)
            generated.append(next_token)
            logits = self.decode_step(next_token, seq_len + step)
        sync()
        t2 = time.perf_counter()
        out = torch.cat(generated, dim=1)
        decode_s = t2 - t1
        self.last_timing = {"ttft_s": t1 - t0, "decode_s": decode_s,
                            "decode_tok_per_s": out.numel() / decode_s if decode_s > 0 else 0.0}
        if self.tokenizer:
            print(self.tokenizer.batch_decode(out, skip_special_tokens=True)[0])
        return out
