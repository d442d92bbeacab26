"""Pins the linear oracle (oracle/linear.py): the fp64 closed form, the C
restatement of the reference GEMV (gemv_ref.c) — against the reference's own
fp16_gemv.cpp built from its source (oracle/build_ref.py) — and the quantiser."""
import numpy as np
import pytest
import torch

from oracle import linear as ol


def data(M, N, K, seed=0):
    g = np.random.default_rng(seed)
    return (g.standard_normal((M, K)).astype(np.float16), g.integers(-127, 128, (N, K), dtype=np.int8),
            g.uniform(1e-3, 1e-2, N).astype(np.float16), g.standard_normal(N).astype(np.float16))


def test_exact_matches_brute_force():
    x, q, s, b = data(2, 5, 24)
    y = ol.int8_linear_exact(x, q, s, b)
    for m in range(2):
        for n in range(5):
            acc = sum(float(x[m, k]) * int(q[n, k]) for k in range(24))
            assert abs(y[m, n] - (acc * float(s[n]) + float(b[n]))) < 1e-12


def test_exact_special_case_is_torch_linear():
    """scale == 1 with an fp16-exact integer weight: the int8 linear is F.linear."""
    x, q, _, _ = data(3, 64, 256, seed=1)
    ones = np.ones(64, np.float16)
    y = ol.int8_linear_exact(x, q, ones)
    t = torch.nn.functional.linear(torch.from_numpy(x).double(), torch.from_numpy(q).double()).numpy()
    assert np.array_equal(y, t)


def test_exact_linearity_and_scale_doubling():
    x, q, s, _ = data(2, 16, 64, seed=2)
    x2 = np.random.default_rng(9).standard_normal((2, 64)).astype(np.float16)
    y = ol.int8_linear_exact(x, q, s) + ol.int8_linear_exact(x2, q, s)
    assert np.allclose(ol.int8_linear_exact(x.astype(np.float64) + x2, q, s), y, atol=1e-9)
    assert np.array_equal(ol.int8_linear_exact(x, q, (s.astype(np.float64) * 2)),
                          2 * ol.int8_linear_exact(x, q, s))


def test_c_gemv_matches_closed_form():
    for (M, N, K) in [(1, 300, 4096), (3, 17, 520), (2, 8, 40)]:   # includes the 8-wide and scalar tails
        x, q, s, b = data(M, N, K, seed=M + N)
        y = ol.int8_gemv(x, q, s, b).astype(np.float64)
        ex = ol.int8_linear_exact(x, q, s, b)
        bound = (np.abs(x.astype(np.float64)) @ np.abs(q.astype(np.float64)).T) * s.astype(np.float64) * 2.0 ** -20
        assert (np.abs(y - ex) <= np.spacing(np.abs(ex).astype(np.float16)).astype(np.float64) + bound).all()
        f32 = ol.int8_gemv_f32(x, q, s)
        assert np.allclose(f32, ex - b.astype(np.float64), rtol=1e-4, atol=1e-3)


def test_c_fp16_gemv_matches_torch_fp32():
    g = np.random.default_rng(7)
    x = g.standard_normal((2, 1000)).astype(np.float16)     # K not a multiple of 32 or 8
    w = (g.standard_normal((50, 1000)) * 0.05).astype(np.float16)
    b = g.standard_normal(50).astype(np.float16)
    y = ol.fp16_gemv(x, w, b).astype(np.float32)
    t = (torch.from_numpy(x).float() @ torch.from_numpy(w).float().T + torch.from_numpy(b).float()).half().float().numpy()
    assert np.allclose(y, t, atol=2e-3)


def test_c_fp16_gemv_summation_order():
    """With all-equal rows, the 4-accumulator order gives a result that differs
    from a sequential fp32 sum in the low bits; the C code reproduces the
    reference's association: lanes (acc0+acc1)+(acc2+acc3), then lo+hi halves,
    then pairwise."""
    K = 64
    x = np.full((1, K), 1.0, np.float16)
    w = np.zeros((1, K), np.float16)
    w[0, ::7] = 1.0009765625  # 1 + 2^-10
    w[0, 3] = 2048.0
    y = ol.fp16_gemv(x, w)
    acc = np.zeros((4, 8), np.float32)
    for j in range(0, K, 32):
        for a in range(4):
            acc[a] += w[0, j + 8 * a:j + 8 * a + 8].astype(np.float32) * x[0, j + 8 * a:j + 8 * a + 8].astype(np.float32)
    v = (acc[0] + acc[1]) + (acc[2] + acc[3])
    lo = v[:4] + v[4:]
    r = np.float32((lo[0] + lo[1]) + (lo[2] + lo[3]))
    assert y[0, 0] == np.float16(r)


def test_quantizer_properties():
    g = np.random.default_rng(3)
    w = (g.standard_normal((40, 300)) * 0.02).astype(np.float32)
    w[5] = 0.0
    q, s = ol.quantize_per_channel(w)
    assert q.dtype == np.int8 and s.dtype == np.float16
    assert s[5] == 0 and (q[5] == 0).all()
    nz = np.arange(40) != 5
    assert (np.abs(q[nz]).max(1) == 127).all()
    err = np.abs(w[nz] - q[nz].astype(np.float32) * s[nz].astype(np.float32)[:, None])
    assert (err <= s[nz].astype(np.float32)[:, None] * 0.5 * (1 + 1e-3) + 1e-9).all()


def test_product_quantizer_matches_oracle():
    from helm_amd.kernels import quantize_per_channel
    g = np.random.default_rng(4)
    w = (g.standard_normal((64, 256)) * 0.02).astype(np.float32)
    qp, sp = quantize_per_channel(torch.from_numpy(w))
    qo, so = ol.quantize_per_channel(w)
    assert np.array_equal(qp.numpy(), qo) and np.array_equal(sp.numpy(), so)


# ── the reference's own GEMV (helm/kernels/fp16_gemv.cpp, built by oracle/build_ref.py) ──
def _ref_module(strict):
    from oracle import build_ref
    m = build_ref.load(strict=strict)
    if m is None:
        pytest.skip("the reference GEMV is not built (oracle/build_ref.py needs the reference tree)")
    return m


GEMV_SHAPES = [(4096, 4096), (1024, 4096), (333, 12288), (77, 4104), (64, 4100), (5, 13), (3, 7),
               (12288, 4096)]


@pytest.mark.parametrize("N,K", GEMV_SHAPES)
@pytest.mark.parametrize("bias", [False, True])
def test_c_restatement_is_bit_exact_with_the_reference_gemv(N, K, bias):
    """oracle_fp16_gemv (gemv_ref.c) against the reference's helm_fp16_linear
    compiled from fp16_gemv.cpp without -ffast-math (the summation order as the
    source writes it): bit-identical fp16 outputs, for K with a 32-wide body, an
    8-wide tail and a scalar tail."""
    import torch
    m = _ref_module(strict=True)
    g = np.random.default_rng(N + K + bias)
    w = (g.standard_normal((N, K)) * 0.02).astype(np.float16)
    x = g.standard_normal((1, K)).astype(np.float16)
    b = g.standard_normal(N).astype(np.float16) if bias else None
    ref = m.helm_fp16_linear(torch.from_numpy(x), torch.from_numpy(w),
                             None if b is None else torch.from_numpy(b)).numpy()
    got = ol.fp16_gemv(x, w, b)
    assert ref.dtype == np.float16 and ref.shape == (1, N)
    assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} outputs differ"


@pytest.mark.parametrize("N,K", GEMV_SHAPES)
def test_c_restatement_against_the_reference_gemv_as_the_reference_builds_it(N, K):
    """The same with the reference's own -ffast-math build: the compiler may
    reassociate the four accumulators and the horizontal sum, so the fp32 sums
    may differ by their rounding error (a few 2^-24 of sum |w x|) and the
    outputs then round apart by an fp16 ulp; at most 1% of outputs differ."""
    import torch
    m = _ref_module(strict=False)
    g = np.random.default_rng(7 * N + K)
    w = (g.standard_normal((N, K)) * 0.02).astype(np.float16)
    x = g.standard_normal((1, K)).astype(np.float16)
    ref = m.helm_fp16_linear(torch.from_numpy(x), torch.from_numpy(w), None).numpy()
    got = ol.fp16_gemv(x, w, None)
    diff = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    sum_abs = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    assert (diff <= ulp + 2.0 ** -21 * sum_abs).all()
    assert np.mean(got != ref) <= 0.01


def test_reference_gemv_argument_errors_are_runtime_errors():
    """The reference op's TORCH_CHECKs raise RuntimeError (fp16_gemv.cpp:110-126),
    the error type the build's C ABI wrapper raises too."""
    import torch
    m = _ref_module(strict=False)
    w = torch.zeros(4, 8, dtype=torch.float16)
    with pytest.raises(RuntimeError):
        m.helm_fp16_linear(torch.zeros(1, 7, dtype=torch.float16), w, None)   # K mismatch
    with pytest.raises(RuntimeError):
        m.helm_fp16_linear(torch.zeros(1, 8, dtype=torch.float16), w.float(), None)   # not fp16
    with pytest.raises(RuntimeError):
        m.helm_fp16_linear(torch.zeros(1, 8, dtype=torch.float16), w.t(), None)   # K mismatch / layout
