"""GPU parity of the INT8 / fp16 decode GEMV and the INT8 prefill GEMM.

Bar (written here, from the task's tolerance): every output element satisfies
|y - exact| <= 1e-2 * max(1, |exact|), exact being the fp64 closed form
scale * (x @ q.T) + bias before rounding (oracle.linear.int8_linear_exact).

A tighter check follows from the error analysis of fp32 accumulation: y is
within 1 fp16 ulp of exact plus 2^-22 * scale * sum_k |q x| (the accumulated
rounding error scales with the absolute sum, not with the result, so outputs
that cancel to near zero are held to the absolute bound).  The same bound
compares the kernel with the C restatement of the reference GEMV.
"""
import numpy as np
import pytest
import torch

from helm_amd import kernels as hk
from helm_amd.kernels import fused
from oracle import linear as ol

pytestmark = pytest.mark.gpu

# Qwen3-8B decode shapes (K -> N) and token counts
SHAPES_8B = [(4096, 4096), (4096, 1024), (4096, 12288), (12288, 4096)]


def make_inputs(M, N, K, seed, bias=False):
    g = np.random.default_rng(seed)
    x = g.standard_normal((M, K)).astype(np.float16)
    q = g.integers(-127, 128, size=(N, K), dtype=np.int8)
    s = g.uniform(1e-3, 1e-2, size=N).astype(np.float16)
    b = g.standard_normal(N).astype(np.float16) if bias else None
    return x, q, s, b


def ulp16(v):
    a = np.abs(np.asarray(v, np.float64)).astype(np.float16)
    return np.spacing(a).astype(np.float64)


def accumulation_bound(x, q, s):
    """2^-22 * s[n] * sum_k |q[n,k] x[m,k]| (fp32 accumulation error budget)."""
    a = np.abs(np.asarray(x, np.float64)) @ np.abs(np.asarray(q, np.float64)).T
    return a * np.asarray(s, np.float64)[None, :] * 2.0 ** -22


def assert_linear_ok(y_gpu, exact, what, acc_bound):
    y = y_gpu.astype(np.float64)
    ok, worst = ol.gemv_tolerance_ok(y, exact)
    assert ok, f"{what}: normalised error {worst:.3e} > 1e-2"
    err = np.abs(y - exact)
    tight = err <= ulp16(exact) + acc_bound
    assert tight.all(), (f"{what}: {np.count_nonzero(~tight)} outputs beyond 1 fp16 ulp + "
                         f"accumulation bound (max err {err.max():.3e})")


def swiglu_within_bar(a, gate, up):
    """SwiGLU output `a` against the exact fp16(fp16(silu(gate)) * up), gate and
    up the fp16-rounded exact projections: the GEMV bar (1e-2 * max(1, |exact|))
    on each projection propagated through the product, since errors e_g, e_u move
    silu(gate) * up by up to 1.1 |up| e_g + |silu(gate)| e_u (an up projection
    that cancels to a small value can carry the whole bar of the inputs it sums:
    a fused RMSNorm whose rsqrt differs from numpy's in the last bit changes a few
    normalised activations by one ulp), plus the bar on the product itself."""
    a = np.asarray(a, np.float64)
    silu = (gate / (1.0 + np.exp(-gate))).astype(np.float16).astype(np.float64)
    exact = silu * up
    e_g = 1e-2 * np.maximum(1.0, np.abs(gate))
    e_u = 1e-2 * np.maximum(1.0, np.abs(up))
    allowed = 1e-2 * np.maximum(1.0, np.abs(exact)) + 1.1 * np.abs(up) * e_g + np.abs(silu) * e_u
    return bool((np.abs(a - exact) <= allowed).all())


def to_dev(*arrs):
    return [None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in arrs]


@pytest.mark.parametrize("K,N", SHAPES_8B)
@pytest.mark.parametrize("M", [1, 4, 16])
def test_int8_gemv_qwen3_8b_shapes(M, N, K):
    x, q, s, _ = make_inputs(M, N, K, seed=1000 * M + N + K)
    xd, qd, sd = to_dev(x, q, s)
    y = hk.int8_linear(xd, qd, sd).cpu().numpy()
    exact = ol.int8_linear_exact(x, q, s)
    bound = accumulation_bound(x, q, s)
    assert_linear_ok(y, exact, f"int8 gemv M={M} K={K} N={N}", bound)
    if M == 1:
        ref = ol.int8_gemv(x, q, s).astype(np.float64)  # the reference GEMV's loop order
        assert (np.abs(y - ref) <= ulp16(ref) + 2 * bound).all()


@pytest.mark.parametrize("M,N,K", [(1, 1, 16), (2, 7, 32), (3, 1000, 1040), (5, 333, 4112),
                                   (7, 4095, 2064), (9, 64, 16384), (13, 129, 528), (16, 17, 64),
                                   (16, 17, 256), (11, 33, 768),
                                   # 3 <= M <= 16 with K % 1024 == 0: the matrix-core small-M path
                                   # (4 and 8 waves per K split; odd unit counts); 3-4 tokens
                                   # otherwise: the two-rows-per-wave streaming path
                                   (3, 1000, 1024), (4, 999, 4096), (7, 4095, 2048), (16, 17, 4096),
                                   (4, 999, 4112),
                                   # two 16-row tiles per workgroup (M >= 9, N >= 8192), ragged
                                   (5, 8200, 1024), (16, 8224, 2048), (9, 8200, 1024),
                                   (5, 200, 3072), (9, 1040, 5120), (16, 64, 12288),
                                   # the ring form over 1024-k units (K other than 4096 / 12288)
                                   (4, 300, 17408), (16, 70, 25600), (9, 1100, 17408),
                                   # the resident form: x rows of all of K in LDS, every token
                                   # bucket (4 / 8 / 12 / 16 rows), three row tiles per workgroup
                                   # (N = 12288) or one, ragged N, K = 12288 up to 4 tokens
                                   (3, 12288, 4096), (7, 12288, 4096), (11, 12288, 4096),
                                   (13, 4100, 4096), (8, 1000, 4096), (3, 4096, 12288),
                                   (4, 1030, 12288),
                                   # 257-512 row tiles at 5-8 tokens: four waves sharing
                                   # one x copy, two workgroups per CU (q|k|v at 6144 rows)
                                   (8, 6144, 4096), (5, 5000, 4096), (6, 4113, 4096)])
def test_int8_gemv_ragged_shapes_with_bias(M, N, K):
    x, q, s, b = make_inputs(M, N, K, seed=M * 7 + N, bias=True)
    xd, qd, sd, bd = to_dev(x, q, s, b)
    y = hk.int8_linear(xd, qd, sd, bd).cpu().numpy()
    assert_linear_ok(y, ol.int8_linear_exact(x, q, s, b), f"ragged M={M} N={N} K={K}",
                     accumulation_bound(x, q, s))


def test_int8_gemv_strided_input_and_batch_dims():
    x, q, s, _ = make_inputs(6, 256, 512, seed=3)
    xd, qd, sd = to_dev(x, q, s)
    big = torch.zeros(6, 1024, dtype=torch.float16, device="cuda")
    big[:, 256:768] = xd
    view = big[:, 256:768]                      # row stride 1024, offset 512 B
    y = hk.int8_linear(view.view(2, 3, 512), qd, sd)
    assert y.shape == (2, 3, 256)
    assert_linear_ok(y.reshape(6, 256).cpu().numpy(), ol.int8_linear_exact(x, q, s), "strided",
                     accumulation_bound(x, q, s))


def test_int8_gemv_extreme_values():
    """Saturated weights and large activations stay within the bar (no fp16 overflow in
    the dequant path: |q| <= 127 is exact in fp16, accumulation is fp32)."""
    M, N, K = 2, 64, 4096
    x = np.full((M, K), 4.0, np.float16)
    x[1] = -2.0
    q = np.full((N, K), 127, np.int8)
    q[::2] = -127
    s = np.full(N, 1e-4, np.float16)
    xd, qd, sd = to_dev(x, q, s)
    y = hk.int8_linear(xd, qd, sd).cpu().numpy()
    assert_linear_ok(y, ol.int8_linear_exact(x, q, s), "extreme", accumulation_bound(x, q, s))


@pytest.mark.parametrize("M,bias", [(17, True), (40, False), (300, True)])
def test_fp16_linear_prefill_branch(M, bias):
    """More than 16 tokens: the fp16 product accumulated and returned in fp32,
    the bias added in fp32, one rounding (the arithmetic of the reference's
    prefill branch, helm/kernels/__init__.py:84-86), against that branch as
    written (F.linear on fp32 copies) within one fp16 ulp plus the fp32
    accumulation bound, and against the exact product at the GEMV bar."""
    g = np.random.default_rng(61 + M)
    N, K = 1000, 4096
    x = g.standard_normal((M, K)).astype(np.float16)
    w = (g.standard_normal((N, K)) * 0.02).astype(np.float16)
    b = g.standard_normal(N).astype(np.float16) if bias else None
    xd, wd, bd = to_dev(x, w, b)
    y = hk.fp16_linear(xd.view(1, M, K), wd, bd)
    assert y.shape == (1, M, N) and y.dtype == torch.float16
    y = y.view(M, N).cpu().numpy().astype(np.float64)
    ref = torch.nn.functional.linear(xd.float(), wd.float(), bd.float() if bias else None).half()
    ref = ref.cpu().numpy().astype(np.float64)
    bound = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T * 2.0 ** -22
    assert (np.abs(y - ref) <= ulp16(ref) + 2 * bound).all()
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    if bias:
        exact = exact + b.astype(np.float64)
    assert ol.gemv_tolerance_ok(y, exact)[0]


@pytest.mark.parametrize("M", [1, 3, 16])
def test_fp16_gemv_matches_reference_order(M):
    g = np.random.default_rng(11 + M)
    N, K = 3000, 4096
    x = g.standard_normal((M, K)).astype(np.float16)
    w = (g.standard_normal((N, K)) * 0.02).astype(np.float16)
    b = g.standard_normal(N).astype(np.float16)
    xd, wd, bd = to_dev(x, w, b)
    y = hk.fp16_linear(xd, wd, bd).cpu().numpy().astype(np.float64)
    ref = ol.fp16_gemv(x, w, b).astype(np.float64)  # helm_fp16_linear restated
    exact = x.astype(np.float64) @ w.astype(np.float64).T + b.astype(np.float64)
    bound = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T * 2.0 ** -22
    assert (np.abs(y - ref) <= ulp16(ref) + 2 * bound).all()
    assert ol.gemv_tolerance_ok(y, exact)[0]


@pytest.mark.parametrize("M,N,K,bias", [(3, 1000, 4096, True), (4, 77, 128, False),
                                        (5, 3001, 1024, True), (8, 2000, 5120, False),
                                        (9, 16, 4096, True), (12, 4099, 2048, False),
                                        (16, 999, 4096, True), (16, 300, 8192, False)])
def test_fp16_gemv_small_m_matrix_cores(M, N, K, bias):
    """fp16 weights at 3-16 tokens (the matrix-core kernel from 4 tokens; at 3
    tokens the streaming kernel, at 16 tokens and K = 8192, whose x rows exceed
    LDS, the tiled kernel): ragged N
    (partial 16-row tiles), K from one 128-k half unit up, against the
    reference's loop order and the fp64 closed form."""
    g = np.random.default_rng(K + N + M)
    x = g.standard_normal((M, K)).astype(np.float16)
    w = (g.standard_normal((N, K)) * 0.02).astype(np.float16)
    b = g.standard_normal(N).astype(np.float16) if bias else None
    xd, wd, bd = to_dev(x, w, b)
    y = hk.fp16_linear(xd, wd, bd).cpu().numpy().astype(np.float64)
    ref = ol.fp16_gemv(x, w, b).astype(np.float64)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    if bias:
        exact = exact + b.astype(np.float64)
    bound = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T * 2.0 ** -22
    assert (np.abs(y - ref) <= ulp16(ref) + 2 * bound).all()
    assert ol.gemv_tolerance_ok(y, exact)[0]


@pytest.mark.parametrize("M", [3, 8, 16])
def test_fp16_gemv_rmsnorm_small_m_lm_head_shape(M):
    """The fused final RMSNorm + fp16 lm_head at a Qwen3-8B-sized vocabulary
    (151936 x 4096, 1.2 GB of weights: 9496 row tiles walked by 2048 waves),
    checked on 3000 sampled rows against the fp64 form of the normalised
    activations; the norm's rounding steps as RMSNorm's fp16 forward."""
    K, N = 4096, 151936
    gen = torch.Generator(device="cuda").manual_seed(M)
    wd = (torch.randn(N, K, device="cuda", generator=gen) * 0.02).half()
    g = np.random.default_rng(77 + M)
    x = (g.standard_normal((M, K)) * 2).astype(np.float16)
    nw = (1 + 0.1 * g.standard_normal(K)).astype(np.float16)
    xd, nwd = to_dev(x, nw)
    y = fused.fp16_gemv_rmsnorm(xd, nwd, 1e-6, wd).cpu().numpy().astype(np.float64)
    rows = np.sort(g.choice(N, 3000, replace=False))
    rows[-1] = N - 1
    ws = wd[torch.from_numpy(rows).cuda()].cpu().numpy().astype(np.float64)
    x32 = x.astype(np.float32)
    rstd = 1.0 / np.sqrt((x32 ** 2).mean(-1, keepdims=True) + 1e-6)
    xr = (nw.astype(np.float32) * (x32 * rstd).astype(np.float16).astype(np.float32)).astype(np.float16)
    assert ol.gemv_tolerance_ok(y[:, rows], xr.astype(np.float64) @ ws.T)[0]
    del wd


@pytest.mark.parametrize("M,N,K", [(17, 64, 64), (64, 256, 512), (130, 200, 320),
                                   (300, 1000, 1024), (2048, 384, 5120)])
def test_int8_gemm_prefill(M, N, K):
    x, q, s, b = make_inputs(M, N, K, seed=M + N + K, bias=True)
    xd, qd, sd, bd = to_dev(x, q, s, b)
    y = hk.int8_linear(xd, qd, sd, bd).cpu().numpy()
    assert_linear_ok(y, ol.int8_linear_exact(x, q, s, b), f"gemm M={M} N={N} K={K}",
                     accumulation_bound(x, q, s))


@pytest.mark.parametrize("tn", [4, 5])
@pytest.mark.parametrize("M,N,K", [(130, 200, 320), (300, 1000, 1024), (257, 700, 2048)])
def test_int8_gemm_wide_tiles_ragged(M, N, K, tn, monkeypatch):
    """The 128 x 32TN tiles with the k-split wave pairs (TN = 4, 5; the automatic
    choice takes them only for large M N), over ragged M and N."""
    monkeypatch.setenv("HELM_GEMM_TN", str(tn))
    x, q, s, b = make_inputs(M, N, K, seed=M + N + K + tn, bias=True)
    xd, qd, sd, bd = to_dev(x, q, s, b)
    y = hk.int8_linear(xd, qd, sd, bd).cpu().numpy()
    assert_linear_ok(y, ol.int8_linear_exact(x, q, s, b), f"gemm tn={tn} M={M} N={N} K={K}",
                     accumulation_bound(x, q, s))


@pytest.mark.parametrize("K,N", [(5120, 5120), (5120, 1024), (5120, 17408), (17408, 5120)])
def test_int8_gemm_qwen3_14b_shapes_row_sample(K, N):
    """Qwen3-14B prefill shapes at M=2048; the exact product is checked on a seeded
    sample of 48 rows (the fp64 product of the full matrix is slow on the host)."""
    M = 2048
    x, q, s, _ = make_inputs(M, N, K, seed=K + N)
    xd, qd, sd = to_dev(x, q, s)
    y = hk.int8_linear(xd, qd, sd).cpu().numpy()
    rows = np.random.default_rng(5).choice(M, 48, replace=False)
    assert_linear_ok(y[rows], ol.int8_linear_exact(x[rows], q, s), f"gemm14b K={K} N={N}",
                     accumulation_bound(x[rows], q, s))


def test_int8_linear_module_and_patch():
    torch.manual_seed(0)
    lin = torch.nn.Linear(512, 300, bias=True).half().cuda()
    mod = hk.Int8Linear.from_linear(lin)
    x = torch.randn(2, 1, 512, dtype=torch.float16, device="cuda")
    y = mod(x)
    assert y.shape == (2, 1, 300) and y.dtype == torch.float16
    exact = ol.int8_linear_exact(x.view(2, 512).cpu().numpy(), mod.qweight.cpu().numpy(),
                                 mod.scale.cpu().numpy(), mod.bias.cpu().numpy())
    xn = x.view(2, 512).cpu().numpy()
    assert_linear_ok(y.view(2, 300).cpu().numpy(), exact, "module",
                     accumulation_bound(xn, mod.qweight.cpu().numpy(), mod.scale.cpu().numpy()))
    seq = torch.nn.Sequential(torch.nn.Linear(64, 64), torch.nn.ReLU(),
                              torch.nn.Sequential(torch.nn.Linear(64, 32))).half().cuda()
    assert hk.patch_linears(seq) == 2
    out = seq(torch.randn(3, 64, dtype=torch.float16, device="cuda"))
    assert out.shape == (3, 32)


@pytest.mark.parametrize("M,N,K", [(1, 1536, 4096), (3, 1001, 4096), (4, 1536, 4096),
                                   # 13-16 x-vectors per thread in the prologue (M K > 24576),
                                   # 5-chunk steps (K = 5120) and a partial last step
                                   (4, 700, 8192), (2, 513, 16384), (3, 300, 5120), (1, 640, 25600),
                                   (4, 257, 7168),
                                   # the matrix-core forms with the norm prologue (K = 4096):
                                   # three row tiles, four waves at 257-512 tiles, eight
                                   # waves, a partial grid
                                   (8, 12288, 4096), (6, 6144, 4096), (16, 4096, 4096),
                                   (12, 500, 4096), (5, 12288, 4096), (4, 6144, 4096),
                                   (3, 4113, 4096)])
def test_fused_norm_residual_and_swiglu(M, N, K):
    """RMSNorm prologue + residual / SwiGLU epilogues: the streaming kernel at 1-2
    tokens and where K is not 4096 (two rows per wave at 3-4 tokens; ragged N
    leaves a wave's second row past the end), the matrix-core forms with the
    norm applied to their x copy in LDS at 3-16 tokens and K = 4096."""
    g = np.random.default_rng(21 + M)
    x = g.standard_normal((M, K)).astype(np.float16)
    nw = (1.0 + 0.1 * g.standard_normal(K)).astype(np.float16)
    _, q, s, _ = make_inputs(M, N, K, seed=22)
    _, q2, s2, _ = make_inputs(M, N, K, seed=23)
    res = g.standard_normal((M, N)).astype(np.float16)
    xd, nwd, qd, sd, q2d, s2d, resd = to_dev(x, nw, q, s, q2, s2, res)
    eps = 1e-6
    # RMSNorm as Qwen3RMSNorm computes it for fp16 activations
    x32 = x.astype(np.float32)
    rstd = 1.0 / np.sqrt((x32 ** 2).mean(-1, keepdims=True) + eps)
    xn = (nw.astype(np.float32) * (x32 * rstd).astype(np.float16).astype(np.float32)).astype(np.float16)
    # norm + residual
    y = fused.int8_gemv_fused(xd, qd, sd, norm_weight=nwd, eps=eps, residual=resd).cpu().numpy()
    lin = ol.int8_linear_exact(xn, q, s).astype(np.float16).astype(np.float64)
    exp_y = res.astype(np.float64) + lin
    assert ol.gemv_tolerance_ok(y.astype(np.float64), exp_y)[0]
    # swiglu
    a = fused.int8_gemv_swiglu(xd, qd, sd, q2d, s2d, norm_weight=nwd, eps=eps).cpu().numpy()
    gt = ol.int8_linear_exact(xn, q, s).astype(np.float16).astype(np.float64)
    up = ol.int8_linear_exact(xn, q2, s2).astype(np.float16).astype(np.float64)
    assert swiglu_within_bar(a, gt, up)
    # the norm in the prologue against the RMSNorm kernel followed by the same
    # projection: equal up to the norms' last-bit differences
    xk = fused.rmsnorm(xd, nwd, eps)
    two = fused.int8_gemv_swiglu(xk, qd, sd, q2d, s2d).cpu().numpy()
    assert np.mean(a == two) > 0.99
    y2 = fused.int8_gemv_fused(xk, qd, sd, residual=resd).cpu().numpy()
    assert np.mean(y == y2) > 0.99


@pytest.mark.parametrize("M,N", [(1, 6144), (2, 6144), (4, 6144), (8, 6144), (16, 6144),
                                 (5, 4608)])
def test_norm_prologue_with_bias(M, N):
    """RMSNorm prologue and a bias together at K = 4096 (a Qwen2-style q|k|v
    projection, which carries biases): the streaming kernel at 1-2 tokens, the
    matrix-core forms with the norm applied to their x copy at 3-16 tokens.
    Against the fp64 projection of the normalised x plus the bias, at the
    GEMV bar, and against the RMSNorm kernel followed by the same projection."""
    K = 4096
    g = np.random.default_rng(51 + M)
    x = g.standard_normal((M, K)).astype(np.float16)
    nw = (1.0 + 0.1 * g.standard_normal(K)).astype(np.float16)
    _, q, s, _ = make_inputs(M, N, K, seed=52)
    b = (0.5 * g.standard_normal(N)).astype(np.float16)
    xd, nwd, qd, sd, bd = to_dev(x, nw, q, s, b)
    eps = 1e-6
    x32 = x.astype(np.float32)
    rstd = 1.0 / np.sqrt((x32 ** 2).mean(-1, keepdims=True) + eps)
    xn = (nw.astype(np.float32) * (x32 * rstd).astype(np.float16).astype(np.float32)).astype(np.float16)
    y = fused.int8_gemv_fused(xd, qd, sd, norm_weight=nwd, eps=eps, bias=bd).cpu().numpy()
    exp_y = ol.int8_linear_exact(xn, q, s, b)
    assert ol.gemv_tolerance_ok(y.astype(np.float64), exp_y)[0]
    # against the RMSNorm kernel and the same projection: the norms' fp32 sums of
    # squares run in another order, so a normalised element may move by an ulp and
    # a few outputs round the other way; both are inside the bar
    xk = fused.rmsnorm(xd, nwd, eps)
    y2 = fused.int8_gemv_fused(xk, qd, sd, bias=bd).cpu().numpy()
    assert ol.gemv_tolerance_ok(y2.astype(np.float64), exp_y)[0]
    assert np.mean(y == y2) > 0.95


@pytest.mark.parametrize("M,N", [(3, 12288), (4, 12288), (8, 12288), (16, 12288), (5, 1000),
                                 (12, 130), (8, 49)])
def test_small_m_swiglu_one_launch(M, N):
    """Gate / up + SwiGLU at 3-16 tokens without a norm prologue (K = 4096): one
    matrix-core launch pairing gate and up row tiles; N = 12288 fills the 256-CU
    grid, smaller N (partial 48-row groups) take the small-grid variant.  Against
    the fp64 projections with the epilogue's rounding steps
    fp16(fp16(silu(fp16 g)) * fp16 u); the bar as in the fused test above."""
    K = 4096
    g = np.random.default_rng(31 + M + N)
    x = g.standard_normal((M, K)).astype(np.float16)
    _, q, s, _ = make_inputs(M, N, K, seed=40 + N)
    _, q2, s2, _ = make_inputs(M, N, K, seed=41 + N)
    xd, qd, sd, q2d, s2d = to_dev(x, q, s, q2, s2)
    a = fused.int8_gemv_swiglu(xd, qd, sd, q2d, s2d).cpu().numpy().astype(np.float64)
    gt = ol.int8_linear_exact(x, q, s).astype(np.float16).astype(np.float64)
    up = ol.int8_linear_exact(x, q2, s2).astype(np.float16).astype(np.float64)
    assert swiglu_within_bar(a, gt, up)
    # against two GEMVs and the SwiGLU kernel (same rounding steps; the fp32 sums
    # run in another order, so a gate output may round one fp16 ulp apart)
    gd = hk.int8_linear(xd, qd, sd)
    ud = hk.int8_linear(xd, q2d, s2d)
    two = fused.silu_mul(gd, ud).cpu().numpy().astype(np.float64)
    assert swiglu_within_bar(two, gt, up)
    assert np.mean(a == two) > 0.99


@pytest.mark.parametrize("M", [5, 16])
def test_small_m_residual_and_bias(M):
    """The small-M path's epilogue: fp16(residual + fp16(s * acc + bias))."""
    g = np.random.default_rng(31 + M)
    N, K = 600, 2048
    x, q, s, b = make_inputs(M, N, K, seed=40 + M, bias=True)
    res = g.standard_normal((M, N)).astype(np.float16)
    xd, qd, sd, bd, resd = to_dev(x, q, s, b, res)
    y = fused.int8_gemv_fused(xd, qd, sd, bias=bd, residual=resd).cpu().numpy()
    lin = ol.int8_linear_exact(x, q, s, b).astype(np.float16).astype(np.float64)
    assert ol.gemv_tolerance_ok(y.astype(np.float64), res.astype(np.float64) + lin)[0]


@pytest.mark.parametrize("M,N,K", [(7, 4096, 12288), (8, 4096, 12288), (12, 4096, 12288),
                                   (16, 4096, 12288), (16, 1000, 6144), (9, 68, 24576),
                                   (16, 4098, 9216)])
def test_small_m_split_k_workspace(M, N, K):
    """Long K at 8-16 tokens through helm_int8_gemv_ws: k split over workgroups
    (3072 each), fp32 partial sums in the caller's workspace, then one reduce with
    scale, bias and the residual aliasing y.  The workspace is filled with NaN
    first (its contents on entry must not matter); 64-row groups past N (N = 1000,
    68), a grid below the CU count (N = 68), and 7 tokens or N % 4 != 0 (no
    workspace, one-pass forms) are covered.  Checked against the fp64 closed form and against the
    one-pass form without a workspace (fp32 summation order only)."""
    from helm_amd import _native
    g = np.random.default_rng(K + N + M)
    x, q, s, b = make_inputs(M, N, K, seed=K + 7 * N + M, bias=True)
    res = g.standard_normal((M, N)).astype(np.float16)
    xd, qd, sd, bd, resd = to_dev(x, q, s, b, res)
    wsb = hk.gemv_workspace_bytes(M, N, K)
    assert (wsb > 0) == (N % 4 == 0 and M >= 8)
    ws = torch.full((max(wsb, 4) // 4,), float("nan"), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    y = resd.clone()
    _native.call("helm_int8_gemv_ws", xd.data_ptr(), K, qd.data_ptr(), K, sd.data_ptr(),
                 bd.data_ptr(), y.data_ptr(), y.data_ptr(), N, M, N, K, ws.data_ptr(), wsb, stream)
    y1 = resd.clone()
    _native.call("helm_int8_gemv_fused", xd.data_ptr(), K, None, 0.0, qd.data_ptr(), K,
                 sd.data_ptr(), bd.data_ptr(), y1.data_ptr(), y1.data_ptr(), N, M, N, K, stream)
    y, y1 = y.cpu().numpy().astype(np.float64), y1.cpu().numpy().astype(np.float64)
    lin = ol.int8_linear_exact(x, q, s, b)
    exp = res.astype(np.float64) + lin.astype(np.float16).astype(np.float64)
    assert ol.gemv_tolerance_ok(y, exp)[0]
    # both forms round the same fp32 sum up to its summation order: within one
    # fp16 ulp of the linear part, the accumulation bound and one ulp of the sum
    slack = 2 * ulp16(lin) + 2 * accumulation_bound(x, q, s) + 2 * ulp16(exp)
    assert (np.abs(y - y1) <= slack).all(), np.abs(y - y1).max()
    # the plain form through the Python wrapper (workspace from the allocator)
    yp = hk.int8_linear(xd, qd, sd, bd).cpu().numpy()
    assert_linear_ok(yp, lin, f"split K M={M} N={N} K={K}", accumulation_bound(x, q, s))


@pytest.mark.parametrize("M,N,K", [(1, 5120, 25600), (2, 600, 25600), (1, 300, 30000), (2, 77, 20000)])
def test_streaming_long_k_residual(M, N, K):
    """Long rows on the streaming kernel (x of K up to 32768 held through the
    prologue: the Qwen3-32B down projection, K = 25600, and ragged K whose last
    step is partial), with the residual epilogue: fp16(residual + fp16(s * acc))."""
    g = np.random.default_rng(K + M)
    x, q, s, _ = make_inputs(M, N, K, seed=K + N)
    res = g.standard_normal((M, N)).astype(np.float16)
    xd, qd, sd, resd = to_dev(x, q, s, res)
    y = fused.int8_gemv_fused(xd, qd, sd, residual=resd).cpu().numpy()
    lin = ol.int8_linear_exact(x, q, s).astype(np.float16).astype(np.float64)
    assert ol.gemv_tolerance_ok(y.astype(np.float64), res.astype(np.float64) + lin)[0]
    yp = hk.int8_linear(xd, qd, sd).cpu().numpy()
    assert_linear_ok(yp, ol.int8_linear_exact(x, q, s), f"long K M={M} N={N} K={K}",
                     accumulation_bound(x, q, s))


@pytest.mark.parametrize("M,K", [(3, 4096), (8, 5120), (2, 16384), (5, 1000), (1, 20000), (4, 24)])
def test_rmsnorm_kernel(M, K):
    """Vector form (K % 8 == 0 up to 16384) and scalar form (other K)."""
    g = np.random.default_rng(4 + K)
    x = (g.standard_normal((M, K)) * 3).astype(np.float16)
    w = (1 + 0.1 * g.standard_normal(K)).astype(np.float16)
    xd, wd = to_dev(x, w)
    y = fused.rmsnorm(xd, wd, 1e-6).cpu().numpy().astype(np.float64)
    x32 = x.astype(np.float32)
    rstd = 1.0 / np.sqrt((x32 ** 2).mean(-1, keepdims=True) + 1e-6)
    ref = (w.astype(np.float32) * (x32 * rstd).astype(np.float16).astype(np.float32)).astype(np.float16)
    assert np.abs(y - ref.astype(np.float64)).max() <= 2 * ulp16(ref).max()


@pytest.mark.parametrize("n", [8 * 12288, 8 * 3072 + 5, 7, 16])
def test_silu_mul_matches_swiglu_rounding(n):
    """fp16(fp16(silu(g)) * u) with silu in fp32, against numpy (tails past the
    last 8-element vector and an unaligned view included)."""
    g = np.random.default_rng(n)
    a = (g.standard_normal(n + 1) * 4).astype(np.float16)
    b = g.standard_normal(n + 1).astype(np.float16)
    ad, bd = to_dev(a, b)
    for sl in (slice(0, n), slice(1, n + 1)):       # aligned, then 2 bytes off
        gt, up = ad[sl].contiguous() if sl.start == 0 else ad[sl], bd[sl]
        out = fused.silu_mul(gt, up).cpu().numpy().astype(np.float64)
        g32 = a[sl].astype(np.float32)
        silu = (g32 / (1 + np.exp(-g32))).astype(np.float16).astype(np.float32)
        ref = (silu * b[sl].astype(np.float32)).astype(np.float16).astype(np.float64)
        assert np.abs(out - ref).max() <= ulp16(ref).max(), sl


def test_fp16_gemv_rmsnorm_matches_norm_then_gemv():
    g = np.random.default_rng(51)
    K, N = 4096, 3000
    x = (g.standard_normal((1, K)) * 2).astype(np.float16)
    nw = (1 + 0.1 * g.standard_normal(K)).astype(np.float16)
    w = (g.standard_normal((N, K)) * 0.02).astype(np.float16)
    xd, nwd, wd = to_dev(x, nw, w)
    y = fused.fp16_gemv_rmsnorm(xd, nwd, 1e-6, wd).cpu().numpy().astype(np.float64)
    xn = fused.rmsnorm(xd, nwd, 1e-6)                       # the separate kernels
    y2 = hk.fp16_linear(xn, wd).cpu().numpy().astype(np.float64)
    assert np.array_equal(y, y2)                            # same rounding steps
    x32 = x.astype(np.float32)
    rstd = 1.0 / np.sqrt((x32 ** 2).mean(-1, keepdims=True) + 1e-6)
    xr = (nw.astype(np.float32) * (x32 * rstd).astype(np.float16).astype(np.float32)).astype(np.float16)
    assert ol.gemv_tolerance_ok(y, xr.astype(np.float64) @ w.astype(np.float64).T)[0]


@pytest.mark.parametrize("single", [False, True])
def test_argmax_matches_torch_first_max(single):
    """Both forms (64 workgroups per row + merge, and one workgroup per row)."""
    g = np.random.default_rng(52)
    x = g.standard_normal((6, 151936)).astype(np.float16)
    x[1, [7, 90000, 151935]] = 30.0            # ties: the first index wins
    x[2, -1] = 40.0                            # maximum in the last element
    x[3, 12345] = np.nan                       # NaN counts as the maximum
    x[4] = -np.inf
    x[5, [2375, 2376, 4750]] = 60.0            # a tie across the boundary of two parts
    xd = torch.from_numpy(x).cuda()
    got = fused.argmax(xd, single_workgroup=single).cpu().numpy()
    exp = torch.argmax(torch.from_numpy(x).float(), dim=-1).numpy()
    assert got.tolist() == exp.tolist() == [int(np.argmax(x[0])), 7, 151935, 12345, 0, 2375]
    odd = torch.from_numpy(g.standard_normal((2, 1001)).astype(np.float16)).cuda()
    assert fused.argmax(odd, single_workgroup=single).tolist() == torch.argmax(odd.float(), -1).tolist()
    # unaligned rows (scalar loads), the maximum in the second batch of 16K vectors
    # (one vector into it), past the last whole vector, or rows shorter than one
    # part or one batch
    big = torch.from_numpy(g.standard_normal((1, 4099)).astype(np.float16)).cuda()
    assert fused.argmax(big[:, 1:], single_workgroup=single).tolist() == \
        torch.argmax(big[:, 1:].float(), -1).tolist()
    for n, at in ((131080, 131075), (131080, 3), (16, 9), (8200, 8199), (151939, 151938), (1, 0)):
        r = g.standard_normal((1, n)).astype(np.float16)
        r[0, at] = 50.0
        assert fused.argmax(torch.from_numpy(r).cuda(), single_workgroup=single).tolist() == [at], (n, at)


def test_fp16_module_patch_and_disable_flag(monkeypatch):
    """patch_cpu_linears / patch_fp16_linears (helm/kernels/__init__.py:107-157):
    fp16 GPU linears are wrapped by reference (same weight tensor), decode calls
    run the fp16 GEMV within its bar, non-fp16 linears are left alone, and
    HELM_DISABLE_GEMV routes decode calls through the fp32 prefill branch."""
    torch.manual_seed(3)
    seq = torch.nn.Sequential(torch.nn.Linear(512, 300, bias=True),
                              torch.nn.Sequential(torch.nn.Linear(300, 64, bias=False)),
                              torch.nn.Linear(64, 8)).cuda()
    seq[0].half()
    seq[1][0].half()                      # seq[2] stays fp32: not patched
    w0 = seq[0].weight
    assert hk.patch_cpu_linears(seq) == 2
    assert isinstance(seq[0], hk.FP16Linear) and seq[0].weight is w0
    assert isinstance(seq[2], torch.nn.Linear) and "fp16_gemv=True" in repr(seq[0])
    x = torch.randn(3, 512, dtype=torch.float16, device="cuda")
    with torch.no_grad():
        y = seq[0](x)
        exact = x.double() @ w0.double().t() + seq[0].bias.double()
        assert ol.gemv_tolerance_ok(y.double().cpu().numpy(), exact.cpu().numpy())[0]
        monkeypatch.setenv("HELM_DISABLE_GEMV", "1")
        y32 = seq[0](x)
        ref32 = torch.nn.functional.linear(x.float(), w0.float(), seq[0].bias.float()).half()
        assert torch.equal(y32, ref32)
