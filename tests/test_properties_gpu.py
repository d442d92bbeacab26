"""Size-independent properties of the decode hot path, checked bit for bit at the
benchmark's full sizes (the Qwen3-8B layer linears and the fp16 lm_head at one
and four tokens, the prefill GEMM and causal prefill attention at 2048 tokens,
paged and fused decode attention over 16K and 32K tokens), where a CPU
restatement would take too long.  Each property is exact in the arithmetic the
kernels use, so any difference is an indexing or addressing mistake:

* attention reads a page only through its table entry: moving every page to
  another pool slot (the table rewritten to match) gives the same bits;
* attention is linear in V at a power-of-two scale: every product, sum and
  quotient of the V side scales exactly, so V x 2 gives exactly twice the fp32
  split partials (the fp16 output only to within the fp16 subnormal spacing);
* a GEMV output row depends on its weight row (and scale) only: permuting the
  rows permutes the outputs exactly;
* a GEMV without the SwiGLU epilogue is odd in x: y(-x) = -y(x), exactly for the
  INT8 linears (the RMSNorm prologue is odd too; a residual is negated with x).
  For the fp16 lm_head it holds to the larger of one fp16 ulp of the output and
  2^-20 (the fp32 spacing of its running sums, which stay below 8): the matrix
  units' fp16 x fp16 dot products (v_dot2_f32_f16 and the fp16 MFMA) drop the
  lowest aligned bits toward minus infinity, measured as a difference in about
  one output in 3000 (1 fp16 ulp; up to 2.4e-7 on outputs near 1e-4, where the
  sum cancels); INT8 weights give products short enough to be summed exactly.
"""
import math

import pytest
import torch

from helm_amd.kernels import attention as ka
from helm_amd.kernels import fused

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
Hq, Hkv, D, P = 32, 8, 128, 16


def _attention_case(B, ctx, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    npg = (ctx + P - 1) // P
    n_slots = B * npg + 9
    k = torch.randn(n_slots, Hkv, P, D, device=DEV, generator=g).half()
    v = torch.randn(n_slots, Hkv, P, D, device=DEV, generator=g).half()
    pt = torch.randperm(n_slots, device=DEV, generator=g)[:B * npg].int().view(B, npg).contiguous()
    q = torch.randn(B, Hq, D, device=DEV, generator=g).half()
    sl = torch.full((B,), ctx, dtype=torch.int32, device=DEV)
    sl[-1] = ctx - 5                                   # a partial last page
    return q, k, v, pt, sl


def _pool(k, v):
    """Pool view of [slots, Hkv, P, D] K / V (V stored token-contiguous)."""
    vs = v.transpose(2, 3).contiguous().transpose(2, 3)
    return ka.PoolView.of_pool(k, vs)


@pytest.mark.parametrize("B,ctx", [(1, 16384), (1, 32768), (8, 16384)])
def test_attention_is_invariant_to_where_pages_sit(B, ctx):
    q, k, v, pt, sl = _attention_case(B, ctx, seed=ctx + B)
    scale = 1.0 / math.sqrt(D)
    out = ka.paged_decode_attention(q, _pool(k, v), pt, sl, P, scale)
    perm = torch.randperm(k.shape[0], device=DEV, generator=torch.Generator(device=DEV).manual_seed(7))
    k2, v2 = torch.empty_like(k), torch.empty_like(v)
    k2[perm.long()] = k                                # slot s moves to perm[s]
    v2[perm.long()] = v
    pt2 = perm[pt.long()].int().contiguous()
    out2 = ka.paged_decode_attention(q, _pool(k2, v2), pt2, sl, P, scale)
    torch.cuda.synchronize()
    print(f"B={B} ctx={ctx}: moved pages, same bits: {torch.equal(out, out2)}", flush=True)
    assert torch.equal(out, out2)


@pytest.mark.parametrize("B,ctx", [(1, 16384), (8, 32768)])
def test_attention_is_linear_in_v_at_scale_two(B, ctx):
    q, k, v, pt, sl = _attention_case(B, ctx, seed=3 * ctx + B)
    scale = 1.0 / math.sqrt(D)
    S = ka.choose_num_splits(B, Hkv, pt.shape[1], P)
    ws = ka.AttnWorkspace(DEV)
    po, pml = (t.clone() for t in ws.get(B, Hq, D, S))
    po2, pml2 = torch.zeros_like(po), torch.zeros_like(pml)
    ka.paged_decode_attention_partial(q, _pool(k, v), pt, sl, P, scale, po, pml, S)
    ka.paged_decode_attention_partial(q, _pool(k, v * 2), pt, sl, P, scale, po2, pml2, S)
    torch.cuda.synchronize()
    assert torch.isfinite(po).all() and (po != 0).any()
    assert torch.equal(pml2, pml) and torch.equal(po2, po * 2)


# (N, K, kind): the Qwen3-8B decode step's linears and the fp16 lm_head
SHAPES = [(6144, 4096, "norm"), (4096, 4096, "residual"), (12288, 4096, "swiglu"),
          (4096, 12288, "residual"), (151936, 4096, "lm_head")]


def _linear(kind, x, w, s, w2=None, s2=None, ln=None, res=None):
    if kind == "norm":
        return fused.int8_gemv_fused(x, w, s, norm_weight=ln)
    if kind == "residual":
        return fused.int8_gemv_fused(x, w, s, residual=res)
    return fused.int8_gemv_swiglu(x, w, s, w2, s2, norm_weight=ln)


def _linear_case(N, K, kind, M, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(M, K, device=DEV, generator=g).half()
    ln = (1 + 0.2 * torch.randn(K, device=DEV, generator=g)).half()
    if kind == "lm_head":
        w = (torch.randn(N, K, device=DEV, generator=g) * 0.02).half()
        return dict(x=x, w=w, s=None, ln=ln)
    w = torch.randint(-127, 128, (N, K), device=DEV, dtype=torch.int8, generator=g)
    s = (torch.rand(N, device=DEV, generator=g) * 2e-3 + 1e-4).half()
    w2 = torch.randint(-127, 128, (N, K), device=DEV, dtype=torch.int8, generator=g)
    s2 = (torch.rand(N, device=DEV, generator=g) * 2e-3 + 1e-4).half()
    res = torch.randn(M, N, device=DEV, generator=g).half()
    return dict(x=x, w=w, s=s, w2=w2, s2=s2, ln=ln, res=res)


def _run(kind, c):
    if kind == "lm_head":   # final RMSNorm + fp16 lm_head, the head of the decode step
        from helm_amd import _native
        M, K = c["x"].shape
        N = c["w"].shape[0]
        y = torch.empty(M, N, dtype=torch.float16, device=DEV)
        _native.call("helm_fp16_gemv_rmsnorm", c["x"].data_ptr(), K, c["ln"].data_ptr(), 1e-6,
                     c["w"].data_ptr(), K, y.data_ptr(), N, M, N, K, _native.stream_ptr(DEV))
        return y
    return _linear(kind, c["x"], c["w"], c["s"], c.get("w2"), c.get("s2"), c["ln"], c.get("res"))


@pytest.mark.parametrize("M", [1, 4])
@pytest.mark.parametrize("N,K,kind", SHAPES)
def test_gemv_row_permutation_permutes_outputs(N, K, kind, M):
    c = _linear_case(N, K, kind, M, seed=N + K + M)
    y = _run(kind, c)
    perm = torch.randperm(N, device=DEV, generator=torch.Generator(device=DEV).manual_seed(11))
    c2 = dict(c)
    c2["w"] = c["w"][perm].contiguous()
    if kind != "lm_head":
        c2["s"] = c["s"][perm].contiguous()
        c2["w2"] = c["w2"][perm].contiguous()
        c2["s2"] = c["s2"][perm].contiguous()
        c2["res"] = c["res"][:, perm].contiguous()
    y2 = _run(kind, c2)
    torch.cuda.synchronize()
    print(f"{kind} {K}->{N} M={M}: permuted rows", flush=True)
    assert torch.equal(y2, y[:, perm])


@pytest.mark.parametrize("M", [1, 4])
@pytest.mark.parametrize("N,K,kind", [s for s in SHAPES if s[2] != "swiglu"])
def test_gemv_is_odd_in_x(N, K, kind, M):
    c = _linear_case(N, K, kind, M, seed=2 * N + K + M)
    y = _run(kind, c)
    c2 = dict(c)
    c2["x"] = -c["x"]
    if kind == "residual":
        c2["res"] = -c["res"]
    y2 = _run(kind, c2)
    torch.cuda.synchronize()
    if kind != "lm_head":
        assert torch.equal(y2, -y)
    else:   # fp16 x fp16 products: the bound above, rarely reached
        ya = torch.maximum(y.float().abs(), y2.float().abs())   # the binade of the larger one
        ulp = torch.where(ya < 2.0 ** -14, torch.full_like(ya, 2.0 ** -24),
                          2.0 ** (torch.floor(torch.log2(ya)) - 10))
        assert ((y2.float() + y.float()).abs() <= torch.clamp(ulp, min=2.0 ** -20)).all()
        assert (y2 != -y).float().mean() < 1e-3


@pytest.mark.parametrize("B", [1, 8])
def test_fused_decode_attention_is_invariant_to_where_pages_sit(B):
    """The decode step's attention launch (q/k norm, RoPE, the new token's K/V
    write, split partials) at 16K tokens: moving every page to another slot (table
    and the new token's slot rewritten to match) gives the same partials, and the
    new token's K/V lands in the moved slot."""
    from helm_amd import _native
    ctx = 16384
    q_unused, k, v, pt, sl = _attention_case(B, ctx, seed=5 * ctx + B)
    g = torch.Generator(device=DEV).manual_seed(17 + B)
    qkv = (torch.randn(B, (Hq + 2 * Hkv) * D, device=DEV, generator=g) * 2).half()
    qn = (1 + 0.1 * torch.randn(D, device=DEV, generator=g)).half()
    kn = (1 + 0.1 * torch.randn(D, device=DEV, generator=g)).half()
    pos = (sl + 3).contiguous()
    slots = pt.gather(1, ((sl.long() - 1) // P).view(B, 1)).view(B).contiguous()
    offs = ((sl - 1) % P).int().contiguous()
    inv = fused.rope_inv_freq(D, 1e6, DEV)
    S = ka.choose_num_splits(B, Hkv, pt.shape[1], P)
    ws = ka.AttnWorkspace(DEV)
    po, pml = (t.clone() for t in ws.get(B, Hq, D, S))
    po2, pml2 = torch.zeros_like(po), torch.zeros_like(pml)
    perm = torch.randperm(k.shape[0], device=DEV, generator=torch.Generator(device=DEV).manual_seed(9))
    k2, v2 = torch.empty_like(k), torch.empty_like(v)
    k2[perm.long()] = k
    v2[perm.long()] = v
    pt2, slots2 = perm[pt.long()].int().contiguous(), perm[slots.long()].int().contiguous()
    pools = []
    for kk, vv, table, sls, o, ml in ((k, v, pt, slots, po, pml), (k2, v2, pt2, slots2, po2, pml2)):
        pool = _pool(kk, vv)
        _native.call("helm_decode_attn_fused", qkv.data_ptr(), qkv.stride(0), qn.data_ptr(),
                     kn.data_ptr(), 1e-6, pos.data_ptr(), inv.data_ptr(), sls.data_ptr(),
                     offs.data_ptr(), pool.c_ref(), table.data_ptr(), table.stride(0), sl.data_ptr(),
                     o.data_ptr(), ml.data_ptr(), B, Hq, Hkv, D, P, table.shape[1], S,
                     1.0 / math.sqrt(D), _native.stream_ptr(DEV))
        pools.append(pool)
    torch.cuda.synchronize()
    assert torch.equal(po2, po) and torch.equal(pml2, pml)
    assert torch.equal(pools[1].k[perm.long()], pools[0].k)
    assert torch.equal(pools[1].v[perm.long()], pools[0].v)


@pytest.mark.parametrize("K,N", [(5120, 17408), (17408, 5120), (4096, 12288)])
def test_gemm_permutations_permute_outputs(K, N):
    """The prefill INT8 GEMM at 2048 tokens (Qwen3-14B / 8B shapes): permuting the
    weight rows (with scales and bias) permutes the output columns, and permuting
    the tokens permutes the output rows, exactly."""
    from helm_amd import kernels as hk
    M = 2048
    g = torch.Generator(device=DEV).manual_seed(K + N)
    x = torch.randn(M, K, device=DEV, generator=g).half()
    w = torch.randint(-127, 128, (N, K), device=DEV, dtype=torch.int8, generator=g)
    s = (torch.rand(N, device=DEV, generator=g) * 2e-3 + 1e-4).half()
    b = (torch.randn(N, device=DEV, generator=g) * 0.1).half()
    y = hk.int8_linear(x, w, s, b)
    pn = torch.randperm(N, device=DEV, generator=torch.Generator(device=DEV).manual_seed(3))
    pm = torch.randperm(M, device=DEV, generator=torch.Generator(device=DEV).manual_seed(4))
    y_n = hk.int8_linear(x, w[pn].contiguous(), s[pn].contiguous(), b[pn].contiguous())
    y_m = hk.int8_linear(x[pm].contiguous(), w, s, b)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    assert torch.equal(y_n, y[:, pn])
    assert torch.equal(y_m, y[pm])


@pytest.mark.parametrize("Hq_", [40, 32])
def test_prefill_attention_pages_and_chunks(Hq_):
    """Causal prefill attention over 2048 prompt tokens (the Qwen3-14B / 8B head
    layouts): moving every page to another slot gives the same bits, and a prompt
    attended in two chunks (queries 0..c-1, then c..2047 with q_start = c, at a
    split that is a multiple of the 32-row wave tile and at one that is not) gives
    the same rows as one call: key steps a query cannot see add exactly nothing."""
    T = 2048
    npg = T // P
    g = torch.Generator(device=DEV).manual_seed(Hq_)
    n_slots = npg + 11
    k = torch.randn(n_slots, Hkv, P, D, device=DEV, generator=g).half()
    v = torch.randn(n_slots, Hkv, P, D, device=DEV, generator=g).half()
    pt = torch.randperm(n_slots, device=DEV, generator=g)[:npg].int().contiguous()
    q = torch.randn(T, Hq_, D, device=DEV, generator=g).half()
    scale = 1.0 / math.sqrt(D)
    out = ka.prefill_attention(q, _pool(k, v), pt, P, 0, scale)
    perm = torch.randperm(n_slots, device=DEV, generator=torch.Generator(device=DEV).manual_seed(2))
    k2, v2 = torch.empty_like(k), torch.empty_like(v)
    k2[perm.long()] = k
    v2[perm.long()] = v
    out_moved = ka.prefill_attention(q, _pool(k2, v2), perm[pt.long()].int().contiguous(), P, 0, scale)
    chunks = {}
    for c in (1024, 777):
        a = ka.prefill_attention(q[:c].contiguous(), _pool(k, v), pt, P, 0, scale)
        b = ka.prefill_attention(q[c:].contiguous(), _pool(k, v), pt, P, c, scale)
        chunks[c] = torch.cat([a, b])
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    assert torch.equal(out_moved, out)
    for c, o in chunks.items():
        assert torch.equal(o, out), f"chunked at {c}"
