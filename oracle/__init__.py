"""oracle — TEST INFRASTRUCTURE ONLY.

CPU restatements of the reference's decode hot path (Shashwatpandey4/HELM), used
to check the HIP implementation in `helm_amd` and as the timed CPU baseline.
Nothing in `helm_amd` imports, calls or links anything here; only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` do, and only
as the reference results are compared against (or timed), never as a product
path.  Each function cites the reference file:line it follows.

Modules
-------
linear      INT8 per-channel quantiser and linear: fp64 closed form, and a C
            restatement of the reference's AVX2/F16C GEMV (gemv_ref.c, built by
            the Makefile into oracle/_build/liboracle_cpu.so)
attention   perform_streaming_attention (helm/runtime/kv_cache.py:318-442):
            eager fp64 closed form and the fp32 online-softmax page loop
kv_pages    KVAllocator / KVCacheManager bookkeeping (helm/runtime/kv_allocator.py,
            helm/runtime/kv_cache.py:30-311) and the _decode_batched page path
            (helm/runtime/kv_offload.py:82-167)
qwen3       fp32 Qwen3 decoder step and greedy loop (kv_offload.py:225-273,
            pipeline_runtime.py:140-176) for the end-to-end check

How each part is pinned (checked against something other than itself) is
stated in its module docstring.
"""
