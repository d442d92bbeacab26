"""helm_paged_decode_attn_noalloc: the allocation-free decode attention entry
point, called through the C ABI, against helm_paged_decode_attn +
helm_paged_attn_reduce with a caller workspace on the same inputs (the same
kernels, so the outputs are bit-identical), and against the oracle's paged
decode attention at the attention bar (2e-3).  Two calls in a row, the second
with a smaller input, so the second call runs over the scratch the first one
left behind."""
import ctypes
import math

import numpy as np
import pytest
import torch

from helm_amd import _native
from helm_amd.kernels import attention as ka
from oracle import attention as oa

pytestmark = pytest.mark.gpu


def _case(g, dev, B, Hq, Hkv, D, P, n_slots, seq_lens):
    max_pages = max(1, max(-(-n // P) for n in seq_lens))
    kp = g.standard_normal((n_slots, Hkv, P, D)).astype(np.float16)
    vp = g.standard_normal((n_slots, Hkv, P, D)).astype(np.float16)
    pt = np.full((B, max_pages), -1, np.int32)
    perm = g.permutation(n_slots)
    used = 0
    for b, n in enumerate(seq_lens):
        k = -(-n // P)
        pt[b, :k] = perm[used:used + k]
        used += k
    q = g.standard_normal((B, Hq, D)).astype(np.float16)
    vdev = ka.alloc_v(vp.shape, device=dev)
    vdev.copy_(torch.from_numpy(vp))
    pool = ka.PoolView.of_pool(torch.from_numpy(kp).to(dev), vdev)
    return dict(kp=kp, vp=vp, pt=pt, q=q, pool=pool, max_pages=max_pages,
                pt_d=torch.from_numpy(pt).to(dev), q_d=torch.from_numpy(q).to(dev),
                sl_d=torch.tensor(seq_lens, dtype=torch.int32, device=dev))


def _noalloc(c, B, Hq, Hkv, D, P, splits, scale, dev):
    out = torch.empty(B, Hq, D, dtype=torch.float16, device=dev)
    pool_struct = c["pool"].c_struct()
    rc = _native.lib().helm_paged_decode_attn_noalloc(
        c["q_d"].data_ptr(), c["q_d"].stride(0), c["q_d"].stride(1), ctypes.byref(pool_struct),
        c["pt_d"].data_ptr(), c["pt_d"].stride(0), c["sl_d"].data_ptr(), out.data_ptr(),
        B, Hq, Hkv, D, P, c["max_pages"], splits, scale, _native.stream_ptr(dev))
    _native.check(rc)
    return out


def _with_workspace(c, B, Hq, Hkv, D, P, splits, scale, dev):
    return ka.paged_decode_attention(c["q_d"], c["pool"], c["pt_d"], c["sl_d"], P, scale,
                                     num_splits=splits)


@pytest.mark.parametrize("D,P", [(128, 16), (64, 16)])
def test_noalloc_matches_workspace_entry_point_twice(cuda, D, P):
    g = np.random.default_rng(1234 + D)
    Hq, Hkv = 32, 8
    scale = 1.0 / math.sqrt(D)
    cases = [
        # first call: batch 4, ragged lengths up to 4000 tokens, 16 splits
        (4, [4000, 1, 777, 2049], 16, 1200),
        # second call: smaller (batch 2, fewer splits) over the scratch left behind
        (2, [300, 45], 4, 60),
    ]
    for B, seq_lens, splits, n_slots in cases:
        print(f"[noalloc] D={D} P={P} B={B} seq_lens={seq_lens} splits={splits}", flush=True)
        c = _case(g, cuda, B, Hq, Hkv, D, P, n_slots, seq_lens)
        got = _noalloc(c, B, Hq, Hkv, D, P, splits, scale, cuda)
        want = _with_workspace(c, B, Hq, Hkv, D, P, splits, scale, cuda)
        torch.cuda.synchronize()
        assert torch.equal(got, want), "noalloc output differs from the workspace entry point"
        ref = oa.paged_decode_reference(c["q"], c["kp"], c["vp"], c["pt"],
                                        np.asarray(seq_lens), P, scale)
        err = float(np.abs(got.float().cpu().numpy() - ref).max())
        assert err <= 2e-3, err


def test_noalloc_rejects_sizes_beyond_scratch(cuda):
    limit = int(_native.lib().helm_paged_attn_noalloc_max_floats())
    assert limit == 4 << 20
    D, Hq, Hkv = 128, 32, 8
    B, splits = 8, (limit // (Hq * (D + 2) * 8)) + 1     # one split past the limit
    g = np.random.default_rng(7)
    # inputs of the full batch, so every buffer matches the sizes passed
    c = _case(g, cuda, B, Hq, Hkv, D, 16, 64, [100] * B)
    out = torch.empty(B, Hq, D, dtype=torch.float16, device=cuda)
    rc = _native.lib().helm_paged_decode_attn_noalloc(
        c["q_d"].data_ptr(), c["q_d"].stride(0), c["q_d"].stride(1),
        ctypes.byref(c["pool"].c_struct()), c["pt_d"].data_ptr(),
        c["pt_d"].stride(0), c["sl_d"].data_ptr(), out.data_ptr(), B, Hq, Hkv, D, 16,
        c["max_pages"], splits, 1.0, _native.stream_ptr(cuda))
    assert rc == -2
    assert "exceeds the scratch buffer" in _native.lib().helm_last_error().decode()
