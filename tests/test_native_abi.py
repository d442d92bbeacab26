"""The C ABI library loads and exports every entry point the header declares.

CPU only: argument validation happens before anything touches the GPU, so the
error paths (negative return codes + helm_last_error) are exercised here too —
the counterpart of the reference's TORCH_CHECK errors (fp16_gemv.cpp:110-126).
"""
import ctypes
import pathlib
import re

import pytest

from helm_amd import _native

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "helm_mi355x.h"


def header_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(helm_[a-z0-9_]+)\s*\(", text)))


def test_library_loads():
    assert _native.is_available(), _native.load_error()
    assert _native.load_error() is None
    assert "gfx950" in _native.version()


def test_every_declared_symbol_is_exported():
    lib = ctypes.CDLL(str(_native.LIB_PATH))
    declared = header_functions()
    assert len(declared) >= 12
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, f"declared in helm_mi355x.h but not exported: {missing}"


def test_binding_matches_header():
    assert sorted(_native.exported_symbols()) == header_functions()


def test_ceiling_probes_are_a_library_of_their_own():
    """The benchmark's ceiling probes (plain MFMA loop, streaming read, empty launch)
    live in probes/libhelm_ceilings.so; none of them is part of the C ABI, and the
    argument checks reject bad calls before any launch."""
    from helm_amd import build as hb
    if not hb.PROBES_LIB.exists():
        pytest.skip("probe library not built")
    lib = ctypes.CDLL(str(hb.PROBES_LIB))
    for name in ("ceil_mfma_loop", "ceil_stream_read", "ceil_empty"):
        assert hasattr(lib, name)
        assert not hasattr(_native.lib(), name)
    lib.ceil_mfma_loop.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_int, ctypes.c_void_p]
    lib.ceil_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_void_p, ctypes.c_void_p]
    fake = ctypes.c_void_p(16)
    assert lib.ceil_mfma_loop(fake, 256, 10, 16, 3, None) == -1      # no 3-chain form
    assert lib.ceil_mfma_loop(fake, 256, 10, 8, 8, None) == -1       # no 8x8 shape
    assert lib.ceil_mfma_loop(None, 256, 10, 16, 8, None) == -1
    assert lib.ceil_stream_read(fake, 100, 1024, 1, fake, None) == -1   # not a multiple of 16
    assert lib.ceil_stream_read(ctypes.c_void_p(24), 4096, 1024, 0, fake, None) == -1  # unaligned


def _last_error():
    return _native.lib().helm_last_error().decode()


def test_gemv_rejects_null_pointer():
    rc = _native.lib().helm_int8_gemv(None, 16, None, 16, None, None, None, 16, 1, 16, 16, None)
    assert rc == -1
    assert "null pointer" in _last_error()


def test_gemv_rejects_large_m():
    fake = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    rc = _native.lib().helm_int8_gemv(fake, 16, fake, 16, fake, None, fake, 16, 17, 16, 16, None)
    assert rc == -2
    assert "M <= 16" in _last_error()


def test_gemv_rejects_unaligned_k():
    fake = ctypes.c_void_p(16)
    rc = _native.lib().helm_int8_gemv(fake, 24, fake, 24, fake, None, fake, 16, 1, 16, 24, None)
    assert rc == -2
    assert "multiple of 16" in _last_error()


def test_check_raises_runtime_error():
    _native.lib().helm_int8_gemv(None, 16, None, 16, None, None, None, 16, 1, 16, 16, None)
    with pytest.raises(RuntimeError, match="null pointer"):
        _native.check(-1)


def _fake_pool(D=128, P=16, Hkv=8):
    from helm_amd.kernels.attention import KvPoolStruct
    return KvPoolStruct(16, 16, Hkv * P * D, P * D, Hkv * D * P, D * P, P, 8)


def test_attention_rejects_bad_head_dim():
    fake = ctypes.c_void_p(16)
    pool = _fake_pool(D=96)
    rc = _native.lib().helm_paged_decode_attn(fake, 96, 96, ctypes.byref(pool), fake, 4, fake,
                                              fake, fake, 0, 4, 1, 8, 8, 96, 16, 4, 4, 0.1, None)
    assert rc == -2
    assert "head_dim" in _last_error()


def test_attention_rejects_split_overflow():
    fake = ctypes.c_void_p(16)
    pool = _fake_pool()
    rc = _native.lib().helm_paged_decode_attn(fake, 128, 128, ctypes.byref(pool), fake, 4, fake,
                                              fake, fake, 3, 4, 1, 8, 8, 128, 16, 4, 2, 0.1, None)
    assert rc == -1
    assert "total_splits" in _last_error()


def test_reduce_rejects_misaligned_max_sum_pairs():
    fake = ctypes.c_void_p(16)
    rc = _native.lib().helm_paged_attn_reduce(fake, ctypes.c_void_p(20), fake, 1, 8, 128, 4, None)
    assert rc == -2
    assert "8-byte aligned" in _last_error()


def test_attention_rejects_null_pool():
    fake = ctypes.c_void_p(16)
    rc = _native.lib().helm_paged_decode_attn(fake, 128, 128, None, fake, 4, fake, fake, fake,
                                              0, 1, 1, 8, 8, 128, 16, 4, 1, 0.1, None)
    assert rc == -1
    assert "null" in _last_error()


def test_attention_rejects_too_many_pages_per_split():
    from helm_amd.kernels.attention import MAX_SPLIT_PAGES, choose_num_splits
    assert _native.lib().helm_paged_attn_max_split_pages() == MAX_SPLIT_PAGES
    fake = ctypes.c_void_p(16)
    pool = _fake_pool()
    n = MAX_SPLIT_PAGES + 1
    rc = _native.lib().helm_paged_decode_attn(fake, 128, 128, ctypes.byref(pool), fake, n, fake,
                                              fake, fake, 0, 1, 1, 8, 8, 128, 16, n, 1, 0.1, None)
    assert rc == -2
    assert "pages per split" in _last_error()
    # the split chooser never asks for that
    assert -(-n // choose_num_splits(64, 8, n, 16)) <= MAX_SPLIT_PAGES


@pytest.mark.parametrize("batch,P", [(1, 16), (8, 16), (1, 32), (3, 64), (4, 16), (16, 32)])
def test_split_partition_covers_the_table_in_whole_wave_rounds(batch, P):
    """choose_num_splits / split_pages (the kernel's partition rule): the splits
    cover every page, each full split is a whole number of rounds of the four
    32-token waves, no split exceeds the LDS page-table budget, and about 256
    workgroups run."""
    from helm_amd.kernels.attention import MAX_SPLIT_PAGES, choose_num_splits, split_pages
    unit = max(1, 128 // P)
    for n in list(range(1, 300)) + [1024, 1042, 1088, 2048, 2112, 4097, 65536, 200000]:
        S = choose_num_splits(batch, 8, n, P)
        pps = split_pages(n, S, P)
        assert pps % unit == 0 and pps <= MAX_SPLIT_PAGES
        assert S * pps >= n   # every page is covered
        want = max(1, 256 // (batch * 8))
        if n <= want * (MAX_SPLIT_PAGES - unit):
            assert batch * 8 * S <= max(256, batch * 8), (n, S)
        if n * P >= 256 * 64 and n <= want * (MAX_SPLIT_PAGES - unit):
            assert batch * 8 * S >= 128, (n, S)
    # the Qwen3-8B decode shapes: 16K context gives 32 splits of 32 pages (4 steps per wave)
    assert choose_num_splits(1, 8, 1024, 16) == 32 and split_pages(1024, 32, 16) == 32
    assert choose_num_splits(1, 8, 1042, 16) == 32 and split_pages(1042, 32, 16) == 40


def test_kv_append_rejects_small_pool_strides():
    fake = ctypes.c_void_p(16)
    from helm_amd.kernels.attention import KvPoolStruct
    pool = KvPoolStruct(16, 16, 128, 64, 128, 64, 8, 4)   # head strides below P*D
    rc = _native.lib().helm_kv_append(fake, fake, ctypes.byref(pool), fake, fake, 1, 1, 1, 8, 16,
                                      None)
    assert rc == -1
    assert "strides too small" in _last_error()


def test_gemm_rejects_k_not_multiple_of_64():
    fake = ctypes.c_void_p(16)
    rc = _native.lib().helm_int8_gemm(fake, 96, fake, 96, fake, None, fake, 16, 32, 16, 96, None)
    assert rc == -2


def test_workspace_size():
    assert _native.workspace_floats(1, 32, 128, 64) == 32 * 64 * 130
    assert _native.workspace_floats(0, 32, 128, 64) == 0


def test_ops_refuse_cpu_tensors():
    import torch
    from helm_amd.kernels import int8_linear
    x = torch.zeros(1, 16, dtype=torch.float16)
    q = torch.zeros(16, 16, dtype=torch.int8)
    s = torch.ones(16, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="GPU"):
        int8_linear(x, q, s)


def test_noalloc_attention_rejects_sizes_beyond_its_scratch():
    """The allocation-free attention entry point checks its scratch limit before
    touching the device (16 MiB of partials: B * Hq * splits * (D + 2) floats)."""
    limit = int(_native.lib().helm_paged_attn_noalloc_max_floats())
    assert limit == 4 << 20
    fake = ctypes.c_void_p(16)
    pool = _fake_pool()
    splits = limit // (8 * 32 * 130) + 1
    rc = _native.lib().helm_paged_decode_attn_noalloc(fake, 128, 128 * 32, ctypes.byref(pool),
                                                      fake, 4, fake, fake, 8, 32, 8, 128, 16, 4,
                                                      splits, 0.1, None)
    assert rc == -2
    assert "exceeds the scratch buffer" in _last_error()
    rc = _native.lib().helm_paged_decode_attn_noalloc(None, 128, 128, ctypes.byref(pool), fake, 4,
                                                      fake, fake, 1, 32, 8, 128, 16, 4, 1, 0.1, None)
    assert rc == -1


def test_masked_prefill_rejects_null_mask_and_short_mask_rows():
    fake = ctypes.c_void_p(16)
    pool = _fake_pool()
    lib = _native.lib()
    # (q, q_st, q_sh, pool, page_table, T, kv_len, Hq, Hkv, D, P, scale,
    #  mask, mask_sh, mask_st, key_end, out, o_st, o_sh, stream)
    rc = lib.helm_prefill_attn_mask(fake, 1024, 128, ctypes.byref(pool), fake, 10, 40, 8, 8, 128,
                                    16, 0.1, None, 0, 64, None, fake, 1024, 128, None)
    assert rc == -1 and "null mask" in _last_error()
    rc = lib.helm_prefill_attn_mask(fake, 1024, 128, ctypes.byref(pool), fake, 10, 40, 8, 8, 128,
                                    16, 0.1, fake, 0, 48, None, fake, 1024, 128, None)
    assert rc == -1 and "rounded up to a multiple of 32" in _last_error()


def test_argmax_workspace_size_and_rejection():
    lib = _native.lib()
    assert lib.helm_argmax_workspace_bytes(3) == 3 * 64 * 8
    assert lib.helm_argmax_workspace_bytes(0) == 0
    fake = ctypes.c_void_p(16)
    rc = lib.helm_argmax_f16_ws(fake, 1024, 3, 1000, fake, fake, 3 * 64 * 8 - 4, None)
    assert rc == -1 and "workspace smaller" in _last_error()
    rc = lib.helm_argmax_f16_ws(fake, 1024, 3, 1000, fake, None, 3 * 64 * 8, None)
    assert rc == -1 and "null pointer" in _last_error()


def test_int8_gemv_workspace_size_and_rejection():
    """The split-K form's workspace: S = K / 3072 slices of fp32 partial sums [M, N]
    for 8-16 tokens over K a multiple of 3072 above 4096 with N % 4 == 0; every
    other shape needs none.  Argument checks come before any launch."""
    lib = _native.lib()
    assert lib.helm_int8_gemv_workspace_bytes(16, 4096, 12288) == 4 * 16 * 4096 * 4
    assert lib.helm_int8_gemv_workspace_bytes(8, 1000, 6144) == 2 * 8 * 1000 * 4
    for M, N, K in [(7, 4096, 12288), (17, 4096, 12288), (16, 4096, 4096), (16, 4098, 12288),
                    (8, 4096, 10240), (1, 4096, 12288)]:
        assert lib.helm_int8_gemv_workspace_bytes(M, N, K) == 0, (M, N, K)
    fake = ctypes.c_void_p(256)
    need = 8 * 4096 * 4 * 4
    rc = lib.helm_int8_gemv_ws(fake, 12288, fake, 12288, fake, None, None, fake, 4096, 8, 4096,
                               12288, fake, need - 16, None)
    assert rc == -1 and "workspace smaller" in _last_error()
    rc = lib.helm_int8_gemv_ws(fake, 12288, fake, 12288, fake, None, None, fake, 4096, 8, 4096,
                               12288, None, need, None)
    assert rc == -1 and "workspace is null" in _last_error()
    rc = lib.helm_int8_gemv_ws(fake, 12288, fake, 12288, fake, None, None, fake, 4096, 8, 4096,
                               12288, ctypes.c_void_p(264), need, None)
    assert rc == -1 and "16-byte aligned" in _last_error()
    rc = lib.helm_int8_gemv_ws(fake, 12288, fake, 12288, fake, None, None, fake, 4096, 17, 4096,
                               12288, fake, need, None)
    assert rc == -2 and "M <= 16" in _last_error()
