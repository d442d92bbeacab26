"""helm_amd — MI355X-native (gfx950) decode hot path of the HELM runtime.

INT8 weight-only linear (decode GEMV / MFMA prefill GEMM) and paged GQA decode
attention, behind HELM's Python API surface:

* ``helm_amd.kernels``  — int8_linear / Int8Linear / patch_linears (the module
  interface of helm/kernels/__init__.py) plus the attention and fused ops;
* ``helm_amd.runtime``  — KVAllocator, KVCacheManager, perform_streaming_attention,
  KVOffloadManager (class-level patched Qwen3 attention forward) and
  PipelineRuntime (greedy loop), mirroring helm/runtime/*.

All compute runs in libhelm_mi355x.so (hand-written HIP for gfx950) through a C
ABI (include/helm_mi355x.h); there is no CPU fallback.
"""
from ._native import is_available, load_error

__version__ = "0.1.0"
__all__ = ["is_available", "load_error", "__version__"]
