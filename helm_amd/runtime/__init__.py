"""helm_amd.runtime — paged KV cache, offload manager and greedy loop
(mirrors of helm/runtime/{kv_allocator,kv_cache,kv_offload,pipeline_runtime}.py)."""
from .kv_allocator import KVAllocator, KVPage, PagePool
from .kv_cache import KVCacheManager, LayerKVCache, perform_streaming_attention
from .kv_offload import KVOffloadConfig, KVOffloadManager
from .page_table import DevicePageTable, PinnedRing
from .pipeline_runtime import PipelineRuntime

__all__ = ["KVAllocator", "KVPage", "PagePool", "KVCacheManager", "LayerKVCache",
           "perform_streaming_attention", "KVOffloadConfig", "KVOffloadManager",
           "DevicePageTable", "PinnedRing", "PipelineRuntime"]
