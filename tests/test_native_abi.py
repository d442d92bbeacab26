"""The C ABI library loads and exports every entry point the header declares.

CPU only: argument validation happens before anything touches the GPU, so the
error paths (negative return codes + helm_last_error) are exercised here too —
the counterpart of the reference's TORCH_CHECK errors (fp16_gemv.cpp:110-126).
"""
import ctypes
import pathlib
import re

import numpy as np
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


def _kernel_partition(max_pages, S, P, pool_tokens):
    """paged_attn_kernel's index arithmetic for one item, restated: which tokens
    each (split, wave, step, lane group) attends, which page-table entries it
    stages and reads.  Returns per-token visit counts and per-split step counts."""
    from helm_amd.kernels.attention import MAX_SPLIT_PAGES, split_pages
    k_step, k_waves = 32, 4
    upp = max(1, k_step // P)
    max_steps = -(-max_pages * P // k_step)
    live = min(-(-pool_tokens // k_step), max_steps)
    seen = np.zeros(max(pool_tokens, 1), np.int64)
    per_split = []
    for split in range(S):
        n_local = (max_steps - 1 - split) // S + 1 if max_steps > split else 0
        p_cnt = n_local * upp
        assert p_cnt <= split_pages(max_pages, S, P) <= MAX_SPLIT_PAGES
        staged = []
        for i in range(p_cnt):
            j = i // upp
            pg = (split + j * S) * k_step // P + (i - j * upp)
            staged.append(pg if pg < max_pages else -1)
        nsteps = (live - 1 - split) // S + 1 if live > split else 0
        per_split.append(nsteps)
        assert nsteps <= n_local
        for wave in range(k_waves):
            if n_local > wave:   # the first step's entries read straight from the table
                t0 = (split + wave * S) * k_step
                for off in range(k_step):
                    assert 0 <= min((t0 + off) // P, max_pages - 1) < max_pages
            my = (nsteps - 1 - wave) // k_waves + 1 if nsteps > wave else 0
            for it in range(my):
                j = wave + k_waves * it
                tok0 = (split + j * S) * k_step
                for off in range(k_step):          # every lane's K row lies in its run's page
                    e = min(j * upp + ((tok0 % P) + off) // P, max(p_cnt - 1, 0))
                    assert staged[e] in (-1, (tok0 + off) // P)
                for grp in range(4):
                    tv = tok0 + grp * 8
                    e = min(j * upp + ((tok0 % P) + grp * 8) // P, max(p_cnt - 1, 0))
                    nvalid = max(0, min(8, pool_tokens - tv)) if staged[e] >= 0 else 0
                    seen[tv:tv + nvalid] += 1
    return seen[:pool_tokens], per_split


@pytest.mark.parametrize("P", [16, 32, 64])
def test_split_partition_attends_every_token_once(P):
    """The kernel's round-robin partition (split s takes the table's 32-token steps
    s, s + S, ...): every live token is attended exactly once, every page-table
    entry read lies in the table, each split stages at most
    helm_paged_attn_max_split_pages() entries, and the splits' step counts differ
    by at most one whatever the live length."""
    from helm_amd.kernels.attention import split_steps
    g = np.random.default_rng(P)
    cases = [(1, 1, 1), (1, 3, 5), (7, 4, 100), (64, 32, 1000), (1088, 32, 16400),
             (1088, 32, 16385), (320, 32, 4097), (33, 8, 33 * P), (2048, 32, 32768)]
    cases += [(int(m), int(s), int(t)) for m, s, t in
              zip(g.integers(1, 400, 30), g.integers(1, 40, 30), g.integers(0, 6000, 30))]
    for max_pages, S, tokens in cases:
        tokens = min(tokens, max_pages * P)
        seen, per_split = _kernel_partition(max_pages, S, P, tokens)
        assert (seen == 1).all(), (max_pages, S, P, tokens)
        assert max(per_split) - min(per_split) <= 1
        assert per_split == [len(split_steps(tokens, max_pages, S, s, P)) for s in range(S)]


@pytest.mark.parametrize("batch,P", [(1, 16), (8, 16), (1, 32), (3, 64), (4, 16), (16, 32)])
def test_split_count_rule(batch, P):
    """choose_num_splits / split_pages: no split stages more than the LDS budget,
    about 256 workgroups run, and none falls below the token floor of the full
    table."""
    from helm_amd.kernels.attention import MAX_SPLIT_PAGES, choose_num_splits, split_pages
    for n in list(range(1, 300)) + [1024, 1042, 1088, 2048, 2112, 4097, 65536, 200000]:
        S = choose_num_splits(batch, 8, n, P)
        assert split_pages(n, S, P) <= MAX_SPLIT_PAGES
        want = max(1, 256 // (batch * 8))
        if split_pages(n, want, P) <= MAX_SPLIT_PAGES:
            assert batch * 8 * S <= max(256, batch * 8), (n, S)
            if n * P >= 256 * 64:
                assert batch * 8 * S >= 128, (n, S)
    # the Qwen3-8B decode shapes: 16K context gives 32 splits of 16 steps
    assert choose_num_splits(1, 8, 1024, 16) == 32 and split_pages(1024, 32, 16) == 32
    assert choose_num_splits(1, 8, 1042, 16) == 32 and split_pages(1042, 32, 16) == 34


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
