"""Decode throughput of a Qwen3-8B-shaped INT8 model at 16K context on one MI355X.

One step = one greedy decode token at batch 1: 36 layers of INT8 linears
(fused norm+q|k|v, o, gate/up+SwiGLU, down), q/k-norm + RoPE + KV page write,
split-K paged GQA attention over the whole context, fp16 lm_head, argmax.
Weights are random-init N(0, 0.02) quantised per channel; the context is
synthetic N(0, 1) KV in the paged pool (the step's cost does not depend on the
values).  The step is replayed as a HIP graph; page-table bookkeeping for every
layer runs on the host inside the timed region.

Prints ONE JSON line (metric, value, roofline of the dominant kernel — the one
with the largest share of the step's GPU time — per-kernel timings, and the CPU
baseline timed on the host cores).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode tok/s Qwen3-8B-shape INT8 bs1 @16K ctx; GEMV+paged-attn HBM GB/s"
# HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE (scaled by a
# copy kernel of known size); the summary and its commands are in this file
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_decode_kernels_qwen3_8b_16k.md")
HBM_PEAK_GBPS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--ctx", type=int, default=16384)
    ap.add_argument("--int8-lm-head", action="store_true",
                    help="decode8b with the lm_head INT8-quantised too (not the headline: "
                         "the headline keeps the fp16 lm_head)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-layers", type=int, default=2, help="layers in the CPU baseline sample")
    ap.add_argument("--probe", default=None,
                    help="only launch this step kernel --probe-iters times (hardware-counter runs)")
    ap.add_argument("--probe-iters", type=int, default=36)
    ap.add_argument("--workload", choices=["decode8b", "offload8b", "e2e32b", "batch8b", "dropin8b"],
                    default="decode8b",
                    help="decode8b: the headline (every KV page in HBM); offload8b: the same "
                         "step with the oldest 50%% of KV pages behind the watermark in pinned "
                         "host memory; e2e32b: Qwen3-32B-shape model, real 1024-token prefill "
                         "+ greedy decode, then 16K/32K contexts with and without offload; "
                         "batch8b: the 8B shape decoding --batch sequences of --ctx tokens at "
                         "once (BatchDecodeEngine); dropin8b: the same model through the "
                         "reference's API (transformers + patch_linears + KVOffloadManager + "
                         "PipelineRuntime)")
    ap.add_argument("--batch", type=int, default=8, help="sequences of the batch8b workload")
    ap.add_argument("--dropin-config", default="all",
                    choices=["all", "paged", "paged-fused", "contiguous", "contiguous-fused"],
                    help="dropin8b: run one KV path / API surface only (no engine line; for "
                         "kernel traces of one configuration)")
    ap.add_argument("--sweep", choices=["gemv", "attention", "prefill"], default=None,
                    help="kernel sweeps over the GEMV / paged-attention / prefill benchmark "
                         "shapes (one JSON line per case) instead of the decode benchmark")
    return ap.parse_args()


def time_graph(fn, reps: int, iters_per_graph: int):
    """Capture fn() `iters_per_graph` times in one graph, replay `reps` times;
    returns the average duration of one fn() in microseconds (HIP events on the
    replay stream, back-to-back launches)."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn(0)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(iters_per_graph):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * iters_per_graph)


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed counter summary, or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return json.loads(line.split(":", 1)[1]).get(kernel)
    except OSError:
        pass
    return None


def step_kernels(engine):
    """The decode step's kernels as launch closures over the 36 layers' own weights:
    name -> (fn(i) launching it for layer i % 36, algorithmic HBM bytes per launch,
    launches per step)."""
    import torch
    from helm_amd import _native
    sh = engine.shape
    H, F, D = sh.hidden, sh.ffn, sh.head_dim
    L = sh.n_layers
    W = engine.w.layers
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    n_pages = engine._graph_pages()
    p = engine.params
    pool = ctypes.byref(engine.pool_c)
    partials = sh.n_heads * engine.splits * (D + 2) * 4
    ks = {}

    def swiglu(i):
        lay = W[i % L]
        _native.call("helm_int8_gemv_swiglu", engine.h.data_ptr(), H, lay["post_ln"].data_ptr(),
                     sh.eps, lay["gate_q"].data_ptr(), lay["gate_s"].data_ptr(),
                     lay["up_q"].data_ptr(), lay["up_s"].data_ptr(), H, engine.act.data_ptr(), F,
                     1, F, H, st())
    ks["gate_up_swiglu_gemv"] = (swiglu, 2 * F * H + 2 * 2 * F + 2 * H + 2 * H + 2 * F, L)

    def down(i):
        lay = W[i % L]
        _native.call("helm_int8_gemv_fused", engine.act.data_ptr(), F, None, 0.0,
                     lay["down_q"].data_ptr(), F, lay["down_s"].data_ptr(), None,
                     engine.xn.data_ptr(), engine.xn.data_ptr(), H, 1, H, F, st())
    ks["down_gemv"] = (down, F * H + 2 * H + 2 * F + 2 * 2 * H, L)

    def qkv(i):
        lay = W[i % L]
        _native.call("helm_int8_gemv_fused", engine.h.data_ptr(), H, lay["in_ln"].data_ptr(),
                     sh.eps, lay["qkv_q"].data_ptr(), H, lay["qkv_s"].data_ptr(), None, None,
                     engine.qkv.data_ptr(), sh.qkv_out, 1, sh.qkv_out, H, st())
    ks["qkv_gemv"] = (qkv, sh.qkv_out * H + 2 * sh.qkv_out + 4 * H + 2 * sh.qkv_out, L)

    def o_proj(i):
        lay = W[i % L]
        _native.call("helm_int8_gemv_fused", engine.attn.data_ptr(), sh.n_heads * D, None, 0.0,
                     lay["o_q"].data_ptr(), sh.n_heads * D, lay["o_s"].data_ptr(), None,
                     engine.xn.data_ptr(), engine.xn.data_ptr(), H, 1, H, sh.n_heads * D, st())
    ks["o_gemv"] = (o_proj, H * sh.n_heads * D + 2 * H + 2 * sh.n_heads * D + 2 * 2 * H, L)

    def attn(i):
        li = i % L
        lay = W[li]
        rows = engine.pt.rows(li)
        _native.call("helm_decode_attn_fused", engine.qkv.data_ptr(), sh.qkv_out,
                     lay["q_norm"].data_ptr(), lay["k_norm"].data_ptr(), sh.eps, p.data_ptr(),
                     engine.inv_freq.data_ptr(), p[2 + li:].data_ptr(), p[2 + L + li:].data_ptr(),
                     pool, rows.data_ptr(), rows.stride(0), p[1:].data_ptr(),
                     engine.part_o.data_ptr(), engine.part_ml.data_ptr(), 1, sh.n_heads,
                     sh.n_kv_heads, D, engine.P, n_pages, engine.splits, engine.scale, st())
    ctx = engine.seq
    ks["decode_attn_fused"] = (attn, (ctx - 1) * 2 * sh.n_kv_heads * D * 2 + sh.qkv_out * 2
                               + 2 * sh.n_kv_heads * D * 2 + partials, L)

    def reduce(i):
        _native.call("helm_paged_attn_reduce", engine.part_o.data_ptr(), engine.part_ml.data_ptr(),
                     engine.attn.data_ptr(), 1, sh.n_heads, D, engine.splits, st())
    ks["attn_reduce"] = (reduce, partials + sh.n_heads * D * 2, L)

    if engine.lm_q is not None:
        def lm_head(i):
            _native.call("helm_int8_gemv_fused", engine.h.data_ptr(), H, engine.w.norm.data_ptr(),
                         sh.eps, engine.lm_q.data_ptr(), H, engine.lm_s.data_ptr(), None, None,
                         engine.logits.data_ptr(), sh.vocab, 1, sh.vocab, H, st())
        ks["lm_head_gemv"] = (lm_head, sh.vocab * H + 2 * sh.vocab + 4 * H + 2 * sh.vocab, 1)
    else:
        def lm_head(i):
            _native.call("helm_fp16_gemv", engine.xn.data_ptr(), H, engine.w.lm_head.data_ptr(), H,
                         None, engine.logits.data_ptr(), sh.vocab, 1, sh.vocab, H, st())
        ks["lm_head_gemv"] = (lm_head, 2 * sh.vocab * H + 2 * H + 2 * sh.vocab, 1)
    return ks


def kernel_rooflines(engine):
    """Average duration and achieved HBM GB/s of the step's kernels, each timed
    with HIP events over graph replays of back-to-back launches over the 36
    layers' own weights in order (no cache reuse across launches)."""
    out = {}
    for name, (fn, nbytes, per_step) in step_kernels(engine).items():
        us = time_graph(fn, 5, 2) if per_step == 1 else time_graph(fn, 20, engine.shape.n_layers)
        out[name] = {"us": round(us, 3), "bytes": nbytes, "gbps": round(nbytes / us / 1e3, 1),
                     "launches_per_step": per_step}
    return out


def probe(engine, name: str, iters: int) -> None:
    """Launch one step kernel `iters` times (eagerly, layers in order), then an
    elementwise copy of 256 MiB (read 256 MiB, write 256 MiB) as the calibration
    kernel of known traffic; for hardware-counter runs (rocprofv3 --pmc)."""
    import torch
    fn = step_kernels(engine)[name][0]
    for i in range(iters):
        fn(i)
    src = torch.randn(128 << 20, device="cuda").half()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)     # 256 MiB in, 256 MiB out
    torch.cuda.synchronize()
    print(json.dumps({"probe": name, "iters": iters, "calibration_bytes": src.numel() * 2}),
          flush=True)


def cpu_baseline(ctx: int, n_layers_sample: int):
    """The reference's CPU decode path on the host cores, over a bounded sample:
    `n_layers_sample` decoder layers at the 8B shape plus 1/8 of the lm_head,
    scaled to one 36-layer token.  Every linear runs the reference's own
    helm_fp16_linear (fp16_gemv.cpp compiled from its source by
    oracle/build_ref.py into oracle/_ref/) on fp16 weights, which is how the
    reference stores and multiplies them (it has no INT8 path), and the
    attention is the all-CPU fp32 path of perform_streaming_attention
    (kv_cache.py:376-380) as the oracle restates it: kind "reference".  Where
    that module is not built, the oracle's C restatement of the same GEMV runs
    the INT8 weights instead: kind "port"."""
    import numpy as np
    import torch
    from oracle import attention as oa
    from oracle import build_ref
    from oracle import linear as ol
    from helm_amd.runtime.decode_engine import QWEN3_8B as sh

    # threads: the cores in the affinity mask, capped at 16 (the host CPU share
    # that goes with one GPU on a shared node); both counts are reported
    available = len(os.sched_getaffinity(0))
    cores = min(16, available)
    os.environ.setdefault("OMP_NUM_THREADS", str(cores))
    ref = build_ref.load()
    g = np.random.default_rng(0)
    H, F, D = sh.hidden, sh.ffn, sh.head_dim

    if ref is not None:
        def weight(n, k):
            return torch.from_numpy((g.standard_normal((n, k), dtype=np.float32) * 0.02)
                                    .astype(np.float16))

        def linear(x, w):
            return ref.helm_fp16_linear(torch.from_numpy(x), w, None).numpy()
    else:
        def weight(n, k):   # q * s then has std ~0.02, as the benchmark's N(0, 0.02) weights
            return (g.integers(-127, 128, size=(n, k), dtype=np.int8),
                    g.uniform(2e-4, 3.5e-4, n).astype(np.float16))

        def linear(x, w):
            return ol.int8_gemv(x, *w)

    layers = [dict(qkv=weight(sh.qkv_out, H), o=weight(H, H), gate=weight(F, H), up=weight(F, H),
                   down=weight(H, F)) for _ in range(n_layers_sample)]
    kv = [(g.standard_normal((1, sh.n_kv_heads, ctx, D)).astype(np.float16),
           g.standard_normal((1, sh.n_kv_heads, ctx, D)).astype(np.float16))
          for _ in range(n_layers_sample)]
    lm_rows = sh.vocab // 8
    lm = (g.standard_normal((lm_rows, H)) * 0.02).astype(np.float16)
    lm_w = torch.from_numpy(lm)
    x = g.standard_normal((1, H)).astype(np.float16)
    scale = 1.0 / math.sqrt(D)

    def rms(v):
        v32 = v.astype(np.float32)
        return (v32 / np.sqrt((v32 ** 2).mean(-1, keepdims=True) + 1e-6)).astype(np.float16)

    def layer_step(lay, kvl, h):
        xn = rms(h)
        qkv = linear(xn, lay["qkv"])
        q = qkv[:, : sh.n_heads * D].reshape(1, sh.n_heads, 1, D)
        a = oa.all_cpu_decode_attention(q, kvl[0], kvl[1], scale).reshape(1, -1)
        h = (h.astype(np.float32) + linear(a, lay["o"]).astype(np.float32)).astype(np.float16)
        xn = rms(h)
        gt = linear(xn, lay["gate"]).astype(np.float32)
        up = linear(xn, lay["up"]).astype(np.float32)
        act = (gt / (1 + np.exp(-gt)) * up).astype(np.float16)
        return (h.astype(np.float32) + linear(act, lay["down"]).astype(np.float32)).astype(np.float16)

    def lm_head(v):
        if ref is not None:
            return ref.helm_fp16_linear(torch.from_numpy(v), lm_w, None).numpy()
        return ol.fp16_gemv(v, lm)

    linear(x, layers[0]["o"])  # load the library, warm the pages
    # repetitions until about 10 s of timed CPU work (at least 3, at most 20)
    t_layers, t_lm, spent = [], [], 0.0
    while len(t_layers) < 3 or (spent < 10.0 and len(t_layers) < 20):
        t0 = time.perf_counter()
        h = x
        for lay, kvl in zip(layers, kv):
            h = layer_step(lay, kvl, h)
        t1 = time.perf_counter()
        lm_head(rms(x))
        t2 = time.perf_counter()
        t_layers.append((t1 - t0) / n_layers_sample)
        t_lm.append((t2 - t1) * 8)
        spent += t2 - t0
    reps = len(t_layers)
    per_token = float(np.median(t_layers)) * sh.n_layers + float(np.median(t_lm))
    what = ("every linear on the reference's own helm_fp16_linear (fp16_gemv.cpp built from "
            "source, fp16 weights as the reference holds them)" if ref is not None else
            "INT8 GEMVs via the oracle's C restatement of the reference GEMV")
    return {
        "value": round(1.0 / per_token, 4), "unit": "tok/s", "cores": cores,
        "cores_available": available, "kind": "reference" if ref is not None else "port",
        "sample": (f"{n_layers_sample} decoder layers of the 8B shape ({what}; all-CPU fp32 "
                   f"attention over {ctx} tokens as the oracle restates kv_cache.py:376-380) "
                   f"x{reps} + 1/8 of the fp16 lm_head x{reps}, median per layer scaled to "
                   f"{sh.n_layers} layers + full lm_head"),
    }


def sweep_gemv() -> None:
    """INT8 weight-only GEMV at the Qwen3-8B layer shapes (K->N: 4096->4096 q/o,
    4096->1024 k/v, 4096->12288 gate/up, 12288->4096 down) for M in {1, 4, 16}
    tokens: x ~ N(0,1) fp16, q ~ U{-127..127}, s ~ U[1e-3, 1e-2].  Each launch
    reads the next of >= 1.2 GB of distinct weight buffers (no cache reuse);
    time per launch from HIP events over graph replays.  Through helm_int8_gemv_ws
    (the split-K form's partial sums in a workspace where the shape takes it),
    as int8_linear calls it."""
    import torch
    from helm_amd import _native
    dev = torch.device("cuda")
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    for K, N in [(4096, 4096), (4096, 1024), (4096, 12288), (12288, 4096)]:
        nb = max(2, math.ceil(1.2e9 / (N * K)))
        g = torch.Generator(device=dev).manual_seed(K + N)
        qs = [torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
              for _ in range(nb)]
        sc = (torch.rand(N, device=dev, generator=g) * 9e-3 + 1e-3).half()
        for M in (1, 4, 16):
            x = torch.randn(M, K, device=dev, generator=g).half()
            y = torch.empty(M, N, device=dev).half()
            wsb = int(_native.lib().helm_int8_gemv_workspace_bytes(M, N, K))
            ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)

            def fn(i):
                _native.call("helm_int8_gemv_ws", x.data_ptr(), K, qs[i % nb].data_ptr(), K,
                             sc.data_ptr(), None, None, y.data_ptr(), N, M, N, K, ws.data_ptr(),
                             wsb, st())
            us = time_graph(fn, 10, nb)
            nbytes = N * K + 2 * N + 2 * M * K + 2 * M * N
            print(json.dumps({"sweep": "int8_gemv", "K": K, "N": N, "M": M, "us": round(us, 3),
                              "bytes": nbytes, "gbps": round(nbytes / us / 1e3, 1),
                              "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBPS, 4)}), flush=True)
        del qs


def sweep_attention() -> None:
    """Paged GQA decode attention at the Qwen3-8B shape (32 q / 8 kv heads, D 128,
    page 16, fp16 N(0,1) Q/K/V, scale 1/sqrt(128)) for context {4096, 16384, 32768}
    x batch {1, 8}: page tables are a seeded random permutation of a shared pool;
    split-K partials + reduce timed over >= 1.2 GB of distinct pools.  Then the
    same with the oldest 50% of each sequence's pages in pinned host memory,
    streamed back per step through perform_streaming_attention (host-link bound)."""
    import numpy as np
    import torch
    from helm_amd.kernels import attention as ka
    from helm_amd.runtime import KVAllocator, KVCacheManager, perform_streaming_attention
    dev = torch.device("cuda")
    Hq, Hkv, D, P = 32, 8, 128, 16
    scale = 1.0 / math.sqrt(D)
    for ctx in (4096, 16384, 32768):
        for B in (1, 8):
            pages = B * ctx // P
            kv_bytes = pages * Hkv * P * D * 2 * 2
            nrot = max(1, math.ceil(1.2e9 / kv_bytes))
            rng = np.random.default_rng(ctx + B)
            pools, tables = [], []
            for _ in range(nrot):
                k = torch.randn(pages, Hkv, P, D, device=dev).half()
                v = ka.alloc_v((pages, Hkv, P, D), device=dev)
                v.normal_()
                pools.append(ka.PoolView.of_pool(k, v))
                tables.append(torch.from_numpy(rng.permutation(pages).astype(np.int32)
                                               .reshape(B, ctx // P)).to(dev))
            q = torch.randn(B, Hq, D, device=dev).half()
            sl = torch.full((B,), ctx, dtype=torch.int32, device=dev)
            S = ka.choose_num_splits(B, Hkv, ctx // P, P)
            ws = ka.AttnWorkspace(dev)
            po, pml = ws.get(B, Hq, D, S)
            out = torch.empty(B, Hq, D, dtype=torch.float16, device=dev)

            def part(i):
                ka.paged_decode_attention_partial(q, pools[i % nrot], tables[i % nrot], sl, P,
                                                  scale, po, pml, S)

            def both(i):
                part(i)
                ka.paged_attn_reduce(po, pml, out, S)
            us_p = time_graph(part, 10, nrot * 2)
            us_t = time_graph(both, 10, nrot * 2)
            nbytes = kv_bytes + B * Hq * D * 2 + B * Hq * S * (D + 2) * 4
            print(json.dumps({"sweep": "paged_attention", "ctx": ctx, "batch": B, "splits": S,
                              "partial_us": round(us_p, 3), "with_reduce_us": round(us_t, 3),
                              "bytes": nbytes, "gbps": round(nbytes / us_p / 1e3, 1),
                              "frac_hbm": round(nbytes / us_p / 1e3 / HBM_PEAK_GBPS, 4)}),
                  flush=True)
            del pools, tables
            torch.cuda.empty_cache()
    # 50% of each sequence's pages host-resident (watermark), streamed back every
    # call; batch 8 runs the reference's per-item path (kv_offload.py:163-167)
    for ctx in (4096, 16384, 32768):
        for B in (1, 8):
            n = ctx // P
            alloc = KVAllocator(1, Hkv, D, P, torch.float16, gpu_capacity_pages=B * (n + 8),
                                cpu_capacity_pages=B * (n // 2 + 16))
            ms = [KVCacheManager(alloc, gpu_high_watermark_bytes=10 ** 15) for _ in range(B)]
            for m in ms:
                m.initialize_layer_caches(1)
                m.reserve_prefill(0, ctx, dev)
            alloc.pool(dev).k.normal_()
            alloc.pool(dev).v_store.normal_()
            for m in ms:
                m.evict_pages((n // 2) * alloc.page_bytes())
            alloc.synchronize()
            page_lists = [m.iterate_layer_pages(0) for m in ms]
            n_host = sum(p.state == "CPU" for pl in page_lists for p in pl)
            q = torch.randn(B, Hq, 1, D, device=dev).half()

            def step():
                return torch.cat([perform_streaming_attention(q[i:i + 1], page_lists[i], scale,
                                                              allocator=alloc) for i in range(B)])
            step()
            torch.cuda.synchronize()
            reps = 5
            t0 = time.perf_counter()
            for _ in range(reps):
                step()
            torch.cuda.synchronize()
            us = (time.perf_counter() - t0) / reps * 1e6
            host_bytes = n_host * alloc.page_bytes()
            print(json.dumps({"sweep": "paged_attention_50pct_host", "ctx": ctx, "batch": B,
                              "host_pages": n_host, "us": round(us, 1), "host_bytes": host_bytes,
                              "host_link_gbps": round(host_bytes / us / 1e3, 2)}), flush=True)
            del ms, page_lists, alloc
            torch.cuda.empty_cache()


def sweep_prefill() -> None:
    """Prefill at Qwen3-14B shapes (hidden 5120, 40 q / 8 kv heads, D 128, FFN
    17408), prompt M = 2048 tokens: the INT8 GEMMs (x ~ N(0,1) fp16, q ~
    U{-127..127}, per-channel fp16 scales) and the causal prefill attention, in
    TFLOP/s against the 2.5 PFLOP/s dense fp16 MFMA peak; torch SDPA (is_causal,
    fp16) on the same inputs is timed beside the attention."""
    import torch
    from helm_amd import _native
    from helm_amd.kernels import attention as ka
    dev = torch.device("cuda")
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    M = 2048
    peak = 2500.0
    for K, N in [(5120, 5120), (5120, 1024), (5120, 17408), (17408, 5120)]:
        g = torch.Generator(device=dev).manual_seed(K + N)
        nb = max(2, math.ceil(0.5e9 / (N * K)))
        qs = [torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
              for _ in range(nb)]
        sc = (torch.rand(N, device=dev, generator=g) * 9e-3 + 1e-3).half()
        x = torch.randn(M, K, device=dev, generator=g).half()
        y = torch.empty(M, N, device=dev).half()

        def fn(i):
            _native.call("helm_int8_gemm", x.data_ptr(), K, qs[i % nb].data_ptr(), K,
                         sc.data_ptr(), None, y.data_ptr(), N, M, N, K, st())
        # the vendor library's fp16 GEMM (torch.matmul -> hipBLASLt) on the same
        # shape with fp16 weights, for scale (it reads twice the weight bytes);
        # the two are timed alternately, three rounds each, best of each (the
        # first round of a shape runs while the clocks settle)
        nbf = max(2, math.ceil(0.5e9 / (2 * N * K)))
        ws = [torch.randn(N, K, device=dev, generator=g).half() for _ in range(nbf)]
        ours, blas = [], []
        for _ in range(3):
            ours.append(time_graph(fn, 5, nb))
            blas.append(time_graph(lambda i: torch.matmul(x, ws[i % nbf].t(), out=y), 5, nbf))
        del qs, ws
        us, us_blas = min(ours), min(blas)
        tf = 2.0 * M * N * K / us / 1e6
        print(json.dumps({"sweep": "int8_gemm_prefill", "M": M, "K": K, "N": N, "us": round(us, 2),
                          "tflops": round(tf, 1), "frac_mfma": round(tf / peak, 4),
                          "torch_fp16_matmul_us": round(us_blas, 2),
                          "torch_fp16_matmul_tflops": round(2.0 * M * N * K / us_blas / 1e6, 1),
                          "ours_over_torch": round(us_blas / us, 3),
                          "rounds_us": [round(v, 2) for v in ours],
                          "torch_rounds_us": [round(v, 2) for v in blas]}),
              flush=True)
    T, Hq, Hkv, D = 2048, 40, 8, 128
    g = torch.Generator(device=dev).manual_seed(7)
    q = torch.randn(T, Hq, D, device=dev, generator=g).half()
    k = torch.randn(T, Hkv, D, device=dev, generator=g).half()
    v = torch.randn(T, Hkv, D, device=dev, generator=g).half()
    pool, pt = ka.dense_prefill_kv(k, v, 16)
    out = torch.empty(T, Hq, D, device=dev).half()
    scale = 1.0 / math.sqrt(D)
    us = time_graph(lambda i: ka.prefill_attention(q, pool, pt, 16, 0, scale, out=out), 10, 10)
    flops = 4.0 * Hq * D * T * (T + 1) / 2            # QK^T and PV over the causal triangle
    qt = q.transpose(0, 1).contiguous()[None]
    kt = k.transpose(0, 1).repeat_interleave(Hq // Hkv, 0).contiguous()[None]
    vt = v.transpose(0, 1).repeat_interleave(Hq // Hkv, 0).contiguous()[None]
    us_sdpa = time_graph(lambda i: torch.nn.functional.scaled_dot_product_attention(
        qt, kt, vt, is_causal=True, scale=scale), 10, 10)
    print(json.dumps({"sweep": "prefill_attention_causal", "T": T, "Hq": Hq, "Hkv": Hkv, "D": D,
                      "us": round(us, 2), "tflops": round(flops / us / 1e6, 1),
                      "frac_mfma": round(flops / us / 1e6 / peak, 4),
                      "torch_sdpa_us": round(us_sdpa, 2),
                      "torch_sdpa_tflops": round(flops / us_sdpa / 1e6, 1)}), flush=True)
    # a left-padded prompt (first 256 positions padding): the masked kernel sees
    # every key of every row, so the flops are the full square
    pad = 256
    pos = torch.arange(T, device=dev)
    keep = (pos[None, :] <= pos[:, None]) & (pos[None, :] >= pad)
    km, m_sh, ke = ka.kernel_mask(keep[None], T, T, Hq)   # the kernel's form, built once
    us_m = time_graph(lambda i: _native.call(
        "helm_prefill_attn_mask", q.data_ptr(), q.stride(0), q.stride(1), pool.c_ref(), pt.data_ptr(),
        T, T, Hq, Hkv, D, 16, float(scale), km.data_ptr(), m_sh, km.stride(1), ke.data_ptr(),
        out.data_ptr(), out.stride(0), out.stride(1), st()), 10, 10)
    # the same without the per-row key ends: every step of every row
    us_full = time_graph(lambda i: _native.call(
        "helm_prefill_attn_mask", q.data_ptr(), q.stride(0), q.stride(1), pool.c_ref(), pt.data_ptr(),
        T, T, Hq, Hkv, D, 16, float(scale), km.data_ptr(), m_sh, km.stride(1), None,
        out.data_ptr(), out.stride(0), out.stride(1), st()), 10, 10)
    flops_vis = 4.0 * Hq * D * float(keep.sum())    # QK^T and PV over the visible pairs
    us_sdpa_m = time_graph(lambda i: torch.nn.functional.scaled_dot_product_attention(
        qt, kt, vt, attn_mask=keep[None, None], scale=scale), 10, 10)
    print(json.dumps({"sweep": "prefill_attention_masked", "T": T, "Hq": Hq, "Hkv": Hkv, "D": D,
                      "mask": f"left padding of {pad}", "us": round(us_m, 2),
                      "visible_tflops": round(flops_vis / us_m / 1e6, 1),
                      "frac_mfma": round(flops_vis / us_m / 1e6 / peak, 4),
                      "us_without_key_ends": round(us_full, 2),
                      "torch_sdpa_us": round(us_sdpa_m, 2)}), flush=True)


def _timed_steps(engine, steps: int, warmup: int):
    """ms per decode_step over `steps` steps after `warmup` (HIP events)."""
    import torch
    for _ in range(warmup):
        engine.decode_step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        engine.decode_step()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def _kv_bytes(sh, ctx: int) -> int:
    return ctx * 2 * sh.n_kv_heads * sh.head_dim * 2 * sh.n_layers


def _host_pages(engine) -> int:
    return sum(1 for li in range(engine.shape.n_layers)
               for p in engine.kvcm.layers[li].pages if p.state == "CPU")


def _offload_run(sh, w, ctx: int, steps: int, warmup: int, frac: float, seed: int = 1) -> dict:
    """Decode at `ctx` with the watermark at `frac` of the context's KV bytes (the
    oldest pages go to pinned host memory and stream back every step)."""
    import torch
    from helm_amd.runtime.decode_engine import DecodeEngine
    wm = None if frac >= 1.0 else int(frac * _kv_bytes(sh, ctx))
    eng = DecodeEngine(w, max_context=ctx + warmup + steps + 64, page_size=16, gpu_watermark_bytes=wm)
    eng.fill_synthetic_context(ctx, seed=seed)
    torch.cuda.synchronize()
    host_pages = _host_pages(eng)
    ms = _timed_steps(eng, steps, warmup)
    page_bytes = eng.allocator.page_bytes()
    out = {"ctx": ctx, "kv_on_host_frac": round(host_pages / max(1, ctx // 16 * sh.n_layers), 3),
           "ms_per_step": round(ms, 3), "tok_s": round(1e3 / ms, 2), "graph": bool(eng.all_gpu)}
    if host_pages:
        out["host_bytes_per_step"] = host_pages * page_bytes
        out["host_link_gbps"] = round(host_pages * page_bytes / (ms * 1e-3) / 1e9, 2)
    del eng
    torch.cuda.empty_cache()
    return out


def bench_offload8b(args) -> None:
    """The headline step with the oldest 50% of KV pages on the host: every step
    streams them back (host-link bound)."""
    import torch
    from helm_amd.runtime.decode_engine import QWEN3_8B, Int8Qwen3Weights
    torch.cuda.set_device(0)
    w = Int8Qwen3Weights.random(QWEN3_8B, torch.device("cuda:0"), seed=0)
    r = _offload_run(QWEN3_8B, w, args.ctx, min(args.steps, 10), min(args.warmup, 2), 0.5)
    print(json.dumps({"metric": "decode tok/s Qwen3-8B-shape INT8 bs1, 50% of KV pages offloaded to host",
                      "value": r["tok_s"], "unit": "tok/s", "n_gpus": 1, "dtype": "int8w-fp16a",
                      "data": "synthetic (random-init N(0,0.02) INT8 weights, N(0,1) KV context)",
                      "config": {"workload": "Qwen3-8B-shape INT8 decode, batch 1, page 16, "
                                             "watermark at 50% of the context's KV"}, **r}), flush=True)


def bench_dropin8b(args) -> None:
    """The reference's own API path at the headline shape: transformers
    Qwen3ForCausalLM (8B shape, random-init N(0, 0.02), fp16) with every decoder
    nn.Linear replaced by Int8Linear (patch_linears) and the lm_head by
    FP16Linear (patch_cpu_linears: its fp16 weights through the fp16 GEMV), the
    patched Qwen3Attention.forward of KVOffloadManager (page 16), and
    PipelineRuntime's greedy loop over a `--ctx`-token random prompt, timed as
    the reference times decode (new tokens / decode wall time, synchronized on
    both sides).  KV: every page in HBM (Path 2, one kernel over the page
    table) and the contiguous buffer (Path 1, the reference's default on a GPU
    model); manager: the reference's API surface (only the attention class
    patched) and with fuse_decoder_layers (MLP, RMSNorm and decoder-layer
    classes patched too).  PipelineRuntime replays each planned decode step
    from a HIP graph.  Last, DecodeEngine over the same weights (shared
    storage) at the same context, for the ratio."""
    import torch
    from transformers import Qwen3Config, Qwen3ForCausalLM
    from helm_amd.kernels import patch_cpu_linears, patch_linears
    from helm_amd.runtime import KVOffloadConfig, KVOffloadManager, PipelineRuntime
    from helm_amd.runtime.decode_engine import QWEN3_8B as sh, DecodeEngine, Int8Qwen3Weights
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = Qwen3Config(vocab_size=sh.vocab, hidden_size=sh.hidden, intermediate_size=sh.ffn,
                      num_hidden_layers=sh.n_layers, num_attention_heads=sh.n_heads,
                      num_key_value_heads=sh.n_kv_heads, head_dim=sh.head_dim,
                      rms_norm_eps=sh.eps, rope_theta=sh.rope_theta, initializer_range=0.02,
                      max_position_embeddings=40960, tie_word_embeddings=False,
                      attention_bias=False)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    t0 = time.perf_counter()
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float16)
    try:
        with torch.device(dev), torch.no_grad():
            model = Qwen3ForCausalLM(cfg).eval()
            gen = torch.Generator(device=dev).manual_seed(0)
            for p in model.parameters():   # matrices N(0, 0.02), norm weights 1
                if p.dim() == 2:
                    p.normal_(0.0, 0.02, generator=gen)
                else:
                    p.fill_(1.0)
    finally:
        torch.set_default_dtype(prev)
    n_patched = patch_linears(model, exclude=("lm_head",))
    n_fp16 = patch_cpu_linears(model)
    torch.cuda.synchronize()
    print(f"[bench] HF 8B-shape model, {n_patched} Int8Linear + {n_fp16} FP16Linear, built in "
          f"{time.perf_counter() - t0:.1f}s", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(1)
    prompt = torch.randint(0, sh.vocab, (1, args.ctx), generator=g).to(dev)
    steps = max(args.steps, 1)
    results = []
    for path, cont in (("paged, every page in HBM", 0), ("contiguous buffer", None)):
        for fused in (False, True):
            name = ("paged" if cont == 0 else "contiguous") + ("-fused" if fused else "")
            if args.dropin_config not in ("all", name):
                continue
            kw = {} if cont is None else {"cont_capacity": cont}
            kcfg = KVOffloadConfig.from_model(model, page_size=16, gpu_watermark_bytes=10 ** 15,
                                              fuse_decoder_layers=fused, **kw)
            mgr = KVOffloadManager(model, kcfg, batch_size=1)
            try:
                rt = PipelineRuntime(model, kv_offload_mgr=mgr)
                mgr.reset()
                with torch.no_grad():
                    torch.cuda.synchronize()
                    tp = time.perf_counter()
                    logits = rt.prefill(prompt)
                    torch.cuda.synchronize()
                    prefill_s = time.perf_counter() - tp
                    tok = torch.argmax(logits[:, -1, :], dim=-1, keepdim=True)
                    del logits
                    warm = max(args.warmup, 3)
                    for i in range(warm):
                        logits = rt.decode_step(tok, args.ctx + i)
                        tok = torch.argmax(logits[:, -1, :], dim=-1, keepdim=True)
                    torch.cuda.synchronize()
                    td = time.perf_counter()
                    for i in range(steps):
                        logits = rt.decode_step(tok, args.ctx + warm + i)
                        tok = torch.argmax(logits[:, -1, :], dim=-1, keepdim=True)
                    torch.cuda.synchronize()
                    dec_s = time.perf_counter() - td
                graphs = rt.decode_graphs and rt._graphs is not None
            finally:
                mgr.restore()
                del mgr
                torch.cuda.empty_cache()
            line = {"metric": "decode tok/s Qwen3-8B-shape INT8 bs1, HF drop-in path",
                    "value": round(steps / dec_s, 2), "unit": "tok/s", "n_gpus": 1,
                    "dtype": "int8w-fp16a", "kv": path,
                    "patches": "attention, MLP, RMSNorm, decoder layer" if fused else "attention",
                    "graph_replay": graphs, "ctx": args.ctx, "steps": steps,
                    "ms_per_step": round(dec_s * 1e3 / steps, 3), "prefill_s": round(prefill_s, 3),
                    "data": "synthetic (random-init N(0,0.02) weights, random prompt ids)",
                    "config": {"workload": "transformers Qwen3-8B shape + patch_linears + "
                                           "KVOffloadManager + PipelineRuntime, batch 1, page 16"}}
            results.append(line)
            print(json.dumps(line), flush=True)
    if args.dropin_config != "all":
        return
    # DecodeEngine over the same weights (q|k|v packed, the modules re-pointed at views)
    w = Int8Qwen3Weights.from_hf(model)
    eng = DecodeEngine(w, max_context=args.ctx + 2 * steps + 64, page_size=16)
    eng.fill_synthetic_context(args.ctx)
    eng.tok.fill_(1)
    ms = _timed_steps(eng, steps, max(args.warmup, 3))
    eng_tps = 1000.0 / ms
    best = max(r["value"] for r in results)
    print(json.dumps({"metric": "decode tok/s Qwen3-8B-shape INT8 bs1, DecodeEngine on the drop-in "
                                "model's weights", "value": round(eng_tps, 2), "unit": "tok/s",
                      "ctx": args.ctx, "steps": steps,
                      "dropin_best_over_engine": round(best / eng_tps, 4)}), flush=True)


def bench_batch8b(args) -> None:
    """Qwen3-8B shape decoding `--batch` sequences of `--ctx` synthetic tokens each
    in one graph-replayed step (BatchDecodeEngine; every page in HBM): tokens/s
    over all sequences, and the step's algorithmic bytes (the INT8 linears and
    the fp16 lm_head once, every sequence's KV) per second."""
    import torch
    from helm_amd.runtime.batch_engine import BatchDecodeEngine
    from helm_amd.runtime.decode_engine import QWEN3_8B as sh, Int8Qwen3Weights
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B = args.batch
    w = Int8Qwen3Weights.random(sh, dev, seed=0)
    eng = BatchDecodeEngine(w, B, max_context=args.ctx + args.steps + args.warmup + 16)
    eng.fill_synthetic_context(args.ctx)
    for _ in range(max(args.warmup, 2)):
        eng.decode_step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        eng.decode_step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    step_bytes = sh.linear_bytes() + 2 * sh.vocab * sh.hidden + B * _kv_bytes(sh, args.ctx)
    print(json.dumps({"metric": f"decode tok/s Qwen3-8B-shape INT8 batch {B} @{args.ctx // 1024}K ctx",
                      "value": round(B * 1000.0 / ms, 2), "unit": "tok/s", "n_gpus": 1,
                      "steps": args.steps, "ms_per_step": round(ms, 4), "dtype": "int8w-fp16a",
                      "data": "synthetic (random-init N(0,0.02) INT8 weights, N(0,1) KV context)",
                      "config": {"workload": f"Qwen3-8B-shape INT8 decode, batch {B}, "
                                             f"{args.ctx}-token contexts, page 16",
                                 "global_batch": B},
                      "step_hbm_bytes": step_bytes,
                      "step_hbm_gbps": round(step_bytes / (ms * 1e-3) / 1e9, 1),
                      "frac_hbm": round(step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}),
          flush=True)


def bench_e2e32b(args) -> None:
    """Qwen3-32B shape (64 layers, hidden 5120, 64/8 heads, FFN 25600, vocab 151936):
    a real 1024-token random prompt through prefill, greedy decode of
    `--steps` tokens, then decode rate at 16K and 32K context with every page in
    HBM and with the oldest 50% of pages offloaded to host memory."""
    import torch
    from helm_amd.runtime.decode_engine import QWEN3_32B as sh, DecodeEngine, Int8Qwen3Weights
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    t0 = time.perf_counter()
    w = Int8Qwen3Weights.random(sh, dev, seed=0)
    torch.cuda.synchronize()
    print(f"[bench] 32B weights {sh.linear_bytes() / 1e9:.2f} GB int8 linears in "
          f"{time.perf_counter() - t0:.1f}s", file=sys.stderr, flush=True)
    base = {"n_gpus": 1, "dtype": "int8w-fp16a", "unit": "tok/s",
            "data": "synthetic (random-init N(0,0.02) INT8 weights; random prompt ids)",
            "config": {"workload": "Qwen3-32B-shape INT8, batch 1, page 16", "layers": sh.n_layers,
                       "hidden": sh.hidden, "ffn": sh.ffn}}
    steps = max(args.steps, 1)
    g = torch.Generator().manual_seed(1)
    prompt = torch.randint(0, sh.vocab, (1024,), generator=g).to(dev)
    # warm-up prefill on a throwaway engine (first-use kernel loads, allocator
    # growth), so that prefill_s is the steady-state time of one prompt
    warm = DecodeEngine(w, max_context=1024 + 64, page_size=16)
    warm.prefill(prompt)
    del warm
    torch.cuda.synchronize()
    eng = DecodeEngine(w, max_context=1024 + steps + 64, page_size=16)
    torch.cuda.synchronize()
    tp = time.perf_counter()
    logits = eng.prefill(prompt)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - tp
    eng.tok.copy_(torch.argmax(logits, dim=-1, keepdim=True))
    td = time.perf_counter()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    toks = [eng.decode_step().clone() for _ in range(steps)]
    e1.record()
    torch.cuda.synchronize()
    dec_wall = time.perf_counter() - td
    ms = e0.elapsed_time(e1) / steps
    print(json.dumps({"metric": "e2e Qwen3-32B-shape: 1024-token prefill + greedy decode", **base,
                      "value": round(1e3 / ms, 2), "prefill_s": round(prefill_s, 3),
                      "prefill_tok_s": round(1024 / prefill_s, 1), "decode_steps": steps,
                      "ms_per_step": round(ms, 3), "decode_wall_s": round(dec_wall, 3),
                      "ctx_end": eng.seq, "first_tokens": [int(t) for t in torch.cat(toks[:8]).cpu()]}),
          flush=True)
    del eng
    torch.cuda.empty_cache()
    for ctx in (16384, 32768):
        for frac in (1.0, 0.5):
            r = _offload_run(sh, w, ctx, 10 if frac >= 1.0 else 4, 2 if frac >= 1.0 else 1, frac)
            print(json.dumps({"metric": "decode tok/s Qwen3-32B-shape INT8 bs1", **base,
                              "value": r["tok_s"], **r}), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; multi-GPU runs are not part of it",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    if args.sweep == "gemv":
        return sweep_gemv()
    if args.sweep == "attention":
        return sweep_attention()
    if args.sweep == "prefill":
        return sweep_prefill()
    if args.workload == "offload8b":
        return bench_offload8b(args)
    if args.workload == "batch8b":
        return bench_batch8b(args)
    if args.workload == "dropin8b":
        return bench_dropin8b(args)
    if args.workload == "e2e32b":
        return bench_e2e32b(args)
    import torch
    from helm_amd.runtime.decode_engine import QWEN3_8B, DecodeEngine, Int8Qwen3Weights

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    t_setup = time.perf_counter()
    w = Int8Qwen3Weights.random(QWEN3_8B, dev, seed=0)
    engine = DecodeEngine(w, max_context=args.ctx + args.warmup + args.steps + 64, page_size=16,
                          int8_lm_head=args.int8_lm_head)
    engine.fill_synthetic_context(args.ctx, seed=1)
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t_setup
    print(f"[bench] setup {setup_s:.1f}s: {QWEN3_8B.linear_bytes() / 1e9:.2f} GB int8 linears, "
          f"ctx {engine.seq} tokens", file=sys.stderr, flush=True)

    if args.probe:
        engine.decode_step()        # one step: page tables and step parameters in place
        torch.cuda.synchronize()
        probe(engine, args.probe, args.probe_iters)
        return
    for _ in range(args.warmup):
        engine.decode_step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    host = 0.0
    for _ in range(args.steps):
        th = time.perf_counter()
        engine.decode_step()
        host += time.perf_counter() - th
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = e0.elapsed_time(e1) / args.steps
    tok_s = 1e3 / ms_step
    print(f"[bench] {args.steps} steps: {ms_step:.3f} ms/step (wall {wall * 1e3 / args.steps:.3f}, "
          f"host {host * 1e3 / args.steps:.3f} per decode_step call)", file=sys.stderr, flush=True)

    kr = kernel_rooflines(engine)
    # dominant kernel: the largest share of the step's GPU time
    dom_name = max(kr, key=lambda k: kr[k]["us"] * kr[k]["launches_per_step"])
    dom = kr[dom_name]
    ach = dom["bytes"] / dom["us"] / 1e3
    kv_bytes = engine.seq * 2 * QWEN3_8B.n_kv_heads * QWEN3_8B.head_dim * 2 * QWEN3_8B.n_layers
    head_bytes = (1 if args.int8_lm_head else 2) * QWEN3_8B.vocab * QWEN3_8B.hidden
    step_bytes = QWEN3_8B.linear_bytes() + head_bytes + kv_bytes
    line = {
        "metric": METRIC + (", INT8 lm_head" if args.int8_lm_head else ""),
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8w-fp16a",
        "data": "synthetic (random-init N(0,0.02) INT8 weights, N(0,1) KV context)",
        "config": {"workload": "Qwen3-8B-shape INT8 decode, batch 1, 16K context, page 16",
                   "layers": QWEN3_8B.n_layers, "hidden": QWEN3_8B.hidden, "ctx": args.ctx,
                   "global_batch": 1, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "kernel": dom_name, "achieved": round(ach, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBPS, 4),
                     "traffic": measured_traffic(dom_name)},
        "host_ms_per_step": round(host * 1e3 / args.steps, 4),
        "step_hbm_bytes": step_bytes,
        "step_hbm_gbps": round(step_bytes / (ms_step * 1e-3) / 1e9, 1),
        "kernels": kr,
    }
    if not args.no_cpu_baseline:
        t_cpu = time.perf_counter()
        line["cpu_baseline"] = cpu_baseline(args.ctx, args.cpu_layers)
        print(f"[bench] cpu baseline {time.perf_counter() - t_cpu:.1f}s", file=sys.stderr, flush=True)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
