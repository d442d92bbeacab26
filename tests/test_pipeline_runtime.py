"""PipelineRuntime's loop on the CPU (pipeline_runtime.py:43-176): the
reference's executor-style construction, the masks and positions each step
passes, greedy next-token choice, and the manager reset before generate()."""
import torch

from helm_amd.runtime import PipelineRuntime

V = 11


class RecordingExecutor:
    """Stands in for a decode executor: logits put all mass on (last id + 1) % V."""

    def __init__(self):
        self.calls = []

    def run(self, inputs):
        self.calls.append(inputs)
        ids = inputs["input_ids"]
        logits = torch.full((ids.shape[0], ids.shape[1], V), -1.0)
        logits.scatter_(2, ((ids + 1) % V)[..., None], 1.0)
        return {"logits": logits}


class CountingManager:
    def __init__(self):
        self.resets = 0

    def reset(self):
        self.resets += 1


def test_executor_signature_masks_positions_and_greedy_loop():
    ex, mgr = RecordingExecutor(), CountingManager()
    rt = PipelineRuntime(None, ex, None, torch.float32, kv_offload_mgr=mgr)
    out = rt.generate(torch.tensor([[3, 4, 5]]), max_new_tokens=4)
    assert out.tolist() == [[6, 7, 8, 9]]
    assert mgr.resets == 1
    pre = ex.calls[0]
    m = pre["attention_mask"]
    assert m.shape == (1, 1, 3, 3) and m[0, 0, 0, 1] == torch.finfo(torch.float32).min
    assert m[0, 0, 2, 0] == 0 and m[0, 0, 1, 1] == 0
    assert pre["position_ids"].tolist() == [[0, 1, 2]] and pre["cache_position"].tolist() == [0, 1, 2]
    for step, call in enumerate(ex.calls[1:]):
        assert call["position_ids"].tolist() == [[3 + step]]
        assert call["cache_position"].tolist() == [3 + step]
        assert call["attention_mask"].shape == (1, 1, 1, 4 + step)
        assert not call["attention_mask"].any()
    assert rt.last_timing["decode_tok_per_s"] > 0


def test_model_signature_positional_tokenizer():
    class Tok:
        def batch_decode(self, ids, skip_special_tokens=True):
            return ["x"]

    class Model(torch.nn.Module):
        def forward(self, input_ids, position_ids, attention_mask, use_cache):
            assert attention_mask is None and not use_cache
            logits = torch.zeros(input_ids.shape[0], input_ids.shape[1], V)
            logits[..., 2] = 1.0
            return logits

    rt = PipelineRuntime(Model(), Tok())
    assert rt.decode_executor is None and isinstance(rt.tokenizer, Tok)
    assert rt.generate(torch.tensor([[1, 2]]), max_new_tokens=3).tolist() == [[2, 2, 2]]


class Wrapper:
    """The decode wrapper the reference's tracer builds: holds the executor's cache."""

    def __init__(self):
        self.past_key_values = "stale"
        self._kv_hooks = []


def test_decode_cache_reset_through_the_wrapper_before_generate_and_every_offloaded_step():
    """pipeline_runtime.py:117-138, :151, :166-167: generate() gives the decode
    wrapper a fresh DynamicCache before the prefill, and before every decode step
    when a KV offload manager owns the KV."""
    from transformers.cache_utils import DynamicCache
    seen = []

    class Ex(RecordingExecutor):
        def run(self, inputs):
            seen.append(type(wrap.past_key_values).__name__)
            wrap.past_key_values = "filled"      # a forward fills the cache
            return super().run(inputs)

    wrap = Wrapper()
    ex = Ex()
    rt = PipelineRuntime(None, ex, None, torch.float32, kv_offload_mgr=CountingManager(),
                         decode_wrapper=wrap)
    rt.generate(torch.tensor([[1, 2]]), max_new_tokens=3)
    assert seen == ["DynamicCache"] * 4            # prefill + 3 decode steps, each on a fresh cache
    # without an offload manager only the reset before generate() happens
    seen.clear()
    rt = PipelineRuntime(None, ex, None, torch.float32, decode_wrapper=wrap)
    rt.generate(torch.tensor([[1, 2]]), max_new_tokens=3)
    assert seen == ["DynamicCache", "str", "str", "str"]
    assert isinstance(DynamicCache(), DynamicCache)


def test_decode_cache_reset_finds_the_wrapper_in_a_stage_hook():
    """Without decode_wrapper the wrapper is found among the default arguments of a
    forward pre-hook of a stage module (pipeline_runtime.py:130-138)."""
    from transformers.cache_utils import DynamicCache
    wrap = Wrapper()
    mod = torch.nn.Sequential(torch.nn.Linear(2, 2), torch.nn.Linear(2, 2))

    def hook(module, args, w=wrap):
        return None

    mod[1].register_forward_pre_hook(hook)

    class Stage:
        module = mod

    class Ex(RecordingExecutor):
        stages = [Stage()]

    rt = PipelineRuntime(None, Ex(), None, torch.float32)
    rt._reset_decode_cache()
    assert isinstance(wrap.past_key_values, DynamicCache)
    # the model-direct runtime has no executor cache: nothing to reset, no error
    PipelineRuntime(torch.nn.Identity())._reset_decode_cache()
