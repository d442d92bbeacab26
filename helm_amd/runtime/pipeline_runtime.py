"""Greedy generation loop (mirror of helm/runtime/pipeline_runtime.py).

The reference runs the model as FX stage modules through StageRuntimeExecutor
(a CPU/GPU layer split that is out of scope here); this runtime calls the model
directly on one GPU and keeps the loop's semantics (pipeline_runtime.py:43-176):
prefill with a full causal mask, then one token per step with
position_ids = [[seq_len + step]], next token = argmax(logits[:, -1, :]), and
the KV offload manager reset before every generate().

With a KV offload manager on the GPU, a decode step on which no layer can
evict (the contiguous buffers have room, or every page is on the GPU) runs its
page bookkeeping for all layers before the forward
(KVOffloadManager.plan_decode_step) and replays the forward as a HIP graph,
captured once per page-table bucket (64 pages); other steps run eagerly with
the reference's per-layer bookkeeping.
"""
from __future__ import annotations

import time
import warnings
from dataclasses import dataclass

import torch


@dataclass
class _StepGraphs:
    """Two captures of one planned decode step's forward (replayed alternately, so
    the host can queue step t + 1 while step t runs) over static input ids and
    position ids; `outs` are the captured logits."""
    key: tuple
    ids: torch.Tensor
    pos: torch.Tensor
    graphs: list
    outs: list


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
                 kv_offload_mgr=None, decode_wrapper=None, decode_graphs: bool = True):
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
        # replay planned decode steps from HIP graphs (decode_graphs=False: run
        # them eagerly, same kernels and splits)
        self.decode_graphs = decode_graphs
        self._graphs = None
        self._flip = 0
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
        mgr = self.kv_offload_mgr
        if self.decode_executor is None and mgr is not None and dev.type == "cuda":
            plan = mgr.plan_decode_step(input_ids.shape[0])
            if plan is not None:
                return self._planned_step(plan, input_ids, step_position)
        position_ids = torch.full((input_ids.shape[0], 1), step_position, dtype=torch.long,
                                  device=dev)
        if self.decode_executor is not None:
            return self._forward(input_ids, position_ids,
                                 self._build_decode_mask(step_position + 1, dev),
                                 torch.tensor([step_position], device=dev))
        return self._forward(input_ids, position_ids, None)

    def _planned_step(self, plan, input_ids, step_position):
        """A decode step whose bookkeeping the manager has done: replay the graph
        captured for the plan's key (capturing it first when the key changed), or
        run the forward eagerly under the plan.  Returns a fresh logits tensor."""
        mgr = self.kv_offload_mgr
        bsz = input_ids.shape[0]
        g = self._graphs if self.decode_graphs else None
        if self.decode_graphs and (g is None or g.key != plan.key):
            self._graphs = None
            g = self._capture(plan, input_ids, step_position)
        if g is None:
            position_ids = torch.full((bsz, 1), step_position, dtype=torch.long,
                                      device=input_ids.device)
            with mgr.planned(plan):
                return self._forward(input_ids, position_ids, self._step_mask(bsz, input_ids.device))
        g.ids.copy_(input_ids)
        g.pos.fill_(step_position)
        i = self._flip
        self._flip ^= 1
        g.graphs[i].replay()
        return g.outs[i].clone()

    def _capture(self, plan, input_ids, step_position):
        """Warm the planned forward up once on a side stream (it runs the real step;
        the replay rewrites the same KV), then capture it twice.  A forward that
        cannot be captured (a host synchronisation inside a module, say) turns the
        graphs off for this runtime and returns None."""
        mgr = self.kv_offload_mgr
        dev = input_ids.device
        ids = input_ids.clone()
        pos = torch.full((ids.shape[0], 1), step_position, dtype=torch.long, device=dev)
        cur = torch.cuda.current_stream(dev)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(cur)
        mask = self._step_mask(ids.shape[0], dev)
        with torch.cuda.stream(side), mgr.planned(plan):
            self._forward(ids, pos, mask)
        cur.wait_stream(side)
        torch.cuda.synchronize(dev)
        graphs, outs = [], []
        try:
            for _ in range(2):
                graph = torch.cuda.CUDAGraph()
                with mgr.planned(plan), torch.cuda.graph(graph):
                    outs.append(self._forward(ids, pos, mask))
                graphs.append(graph)
        except Exception as exc:   # noqa: BLE001 — any capture failure means: run eagerly
            torch.cuda.synchronize(dev)
            self.decode_graphs = False
            warnings.warn(f"PipelineRuntime: decode step not capturable ({exc}); running eagerly")
            return None
        self._graphs = _StepGraphs(plan.key, ids, pos, graphs, outs)
        self._flip = 0
        return self._graphs

    def _step_mask(self, bsz, device):
        """The attention mask of a planned decode step: 4-D zeros [bsz, 1, 1, 1]
        (every cached position visible, as the reference's decode mask of zeros
        says; the patched attention reads the lengths from the page tables).  A
        4-D mask reaches the layers as it is, so transformers builds no mask of
        its own inside the step (one static tensor per batch size)."""
        m = getattr(self, "_masks", {}).get((bsz, device))
        if m is None:
            m = torch.zeros(bsz, 1, 1, 1, dtype=self.dtype, device=device)
            self._masks = {**getattr(self, "_masks", {}), (bsz, device): m}
        return m

    def _reset_decode_cache(self):
        """Fresh DynamicCache for the decode executor's wrapper
        (pipeline_runtime.py:117-138): the wrapper handed in as decode_wrapper,
        else the first object carrying `past_key_values` and `_kv_hooks` among
        the default arguments of a forward pre-hook in the executor's stages.
        Without an executor (the model is called directly with use_cache=False)
        there is no cache to reset."""
        if self.decode_wrapper is None and getattr(self.decode_executor, "stages", None) is None:
            return
        from transformers.cache_utils import DynamicCache
        if self.decode_wrapper is not None:
            self.decode_wrapper.past_key_values = DynamicCache()
            return
        for stage in self.decode_executor.stages:
            for _, module in stage.module.named_modules():
                for hook in module._forward_pre_hooks.values():
                    for obj in getattr(hook, "__defaults__", None) or ():
                        if hasattr(obj, "past_key_values") and hasattr(obj, "_kv_hooks"):
                            obj.past_key_values = DynamicCache()
                            return

    @torch.no_grad()
    def generate(self, input_ids, max_new_tokens=8):
        """Prefill, then greedy decode; returns [B, max_new_tokens] token ids.
        self.last_timing holds ttft_s / decode_s / decode_tok_per_s measured like
        the reference's harness (experiments/paper_bench.py:755-790)."""
        if self.kv_offload_mgr is not None:
            self.kv_offload_mgr.reset()
        self._reset_decode_cache()
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
            if self.kv_offload_mgr is not None:
                # the paged cache owns the KV: the executor's DynamicCache starts empty
                self._reset_decode_cache()
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
