"""Paged GQA decode attention and KV page writes on the GPU (functional layer).

Thin typed wrappers over helm_paged_decode_attn / helm_paged_attn_reduce /
helm_kv_append / helm_stage_pages_h2d.  The page pool layout is
[slots, Hkv, P, D] fp16 (a slot view is the reference's per-page tensor
(1, Hkv, P, D), helm/runtime/kv_allocator.py:26-28); a contiguous per-layer
buffer [1, Hkv, cap, D] (helm/runtime/kv_cache.py:219-222) is addressed with
slot_stride = P*D, head_stride = cap*D.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch

from .. import _native

# Target workgroups (4 waves each) for one attention launch: ~2 per CU on 256 CUs.
_TARGET_WGS = 512


def choose_num_splits(batch: int, num_kv_heads: int, max_pages: int, blocks_per_page: int = 1,
                      target_wgs: int = _TARGET_WGS, min_blocks_per_split: int = 16) -> int:
    """Pages of one (item, kv head) are split so that batch*Hkv*splits ~ target_wgs
    workgroups, keeping at least `min_blocks_per_split` 16-token blocks per split
    (four per wave of the workgroup)."""
    max_pages = max(1, int(max_pages))
    base = max(1, batch * num_kv_heads)
    want = max(1, target_wgs // base)
    cap = max(1, (max_pages * blocks_per_page) // min_blocks_per_split)
    return int(max(1, min(want, cap, max_pages)))


@dataclass
class PoolView:
    """Where a layer's K/V live: pools plus strides in elements."""
    k: torch.Tensor
    v: torch.Tensor
    slot_stride: int
    head_stride: int
    num_slots: int

    @staticmethod
    def of_pool(k_pool: torch.Tensor, v_pool: torch.Tensor) -> "PoolView":
        """k_pool/v_pool [slots, Hkv, P, D]."""
        s, hkv, p, d = k_pool.shape
        return PoolView(k_pool, v_pool, hkv * p * d, p * d, s)

    @staticmethod
    def of_contiguous(k_buf: torch.Tensor, v_buf: torch.Tensor, page_size: int) -> "PoolView":
        """k_buf/v_buf [1, Hkv, cap, D]: page i = tokens [i*P, (i+1)*P)."""
        _, hkv, cap, d = k_buf.shape
        return PoolView(k_buf, v_buf, page_size * d, cap * d, cap // page_size)


class AttnWorkspace:
    """Reusable fp32 split-K workspace (part_o + part_ml), grown on demand."""

    def __init__(self, device: torch.device):
        self.device = device
        self.buf = torch.empty(0, dtype=torch.float32, device=device)

    def get(self, B: int, Hq: int, D: int, total_splits: int):
        n_o = B * Hq * total_splits * D
        n = n_o + B * Hq * total_splits * 2
        if self.buf.numel() < n:
            self.buf = torch.empty(n, dtype=torch.float32, device=self.device)
        return self.buf[:n_o], self.buf[n_o:n]


def paged_decode_attention_partial(q: torch.Tensor, pool: PoolView, page_table: torch.Tensor,
                                   seq_lens: torch.Tensor, page_size: int, scale: float,
                                   part_o: torch.Tensor, part_ml: torch.Tensor,
                                   num_splits: int, split_offset: int = 0,
                                   total_splits: Optional[int] = None) -> None:
    """Launch the split-K partial kernel; q [B, Hq, D] (any strides with unit last dim)."""
    _native.require_cuda(q, pool.k, pool.v, page_table, seq_lens, what="paged_decode_attention")
    if q.dtype != torch.float16 or pool.k.dtype != torch.float16 or pool.v.dtype != torch.float16:
        raise RuntimeError("paged_decode_attention: q and KV pools must be fp16")
    if page_table.dtype != torch.int32 or seq_lens.dtype != torch.int32:
        raise RuntimeError("paged_decode_attention: page_table and seq_lens must be int32")
    if q.dim() != 3 or q.stride(-1) != 1:
        raise RuntimeError("paged_decode_attention: q must be [B, Hq, D] with unit stride on D")
    if page_table.dim() != 2 or page_table.stride(1) != 1:
        raise RuntimeError("paged_decode_attention: page_table must be [B, max_pages], row-major")
    B, Hq, D = q.shape
    Hkv = pool.k.shape[1]
    max_pages = page_table.shape[1]
    total = num_splits if total_splits is None else total_splits
    _native.call("helm_paged_decode_attn", q.data_ptr(), q.stride(0), q.stride(1),
                 pool.k.data_ptr(), pool.v.data_ptr(), pool.slot_stride, pool.head_stride,
                 page_table.data_ptr(), page_table.stride(0), seq_lens.data_ptr(), pool.num_slots,
                 part_o.data_ptr(), part_ml.data_ptr(), split_offset, total, B, Hq, Hkv, D,
                 page_size, max_pages, num_splits, float(scale), _native.stream_ptr(q.device))


def paged_attn_reduce(part_o: torch.Tensor, part_ml: torch.Tensor, out: torch.Tensor,
                      total_splits: int) -> torch.Tensor:
    B, Hq, D = out.shape
    _native.call("helm_paged_attn_reduce", part_o.data_ptr(), part_ml.data_ptr(), out.data_ptr(),
                 B, Hq, D, total_splits, _native.stream_ptr(out.device))
    return out


def paged_decode_attention(q: torch.Tensor, pool: PoolView, page_table: torch.Tensor,
                           seq_lens: torch.Tensor, page_size: int, scale: Optional[float] = None,
                           num_splits: Optional[int] = None,
                           workspace: Optional[AttnWorkspace] = None,
                           out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out[b, h] = softmax(scale q[b,h] K_b^T) V_b over the paged KV of item b.

    q [B, Hq, D] fp16; page_table [B, max_pages] int32 slots; seq_lens [B] int32.
    Returns out [B, Hq, D] fp16 (zeros for an empty item)."""
    B, Hq, D = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if num_splits is None:
        num_splits = choose_num_splits(B, pool.k.shape[1], page_table.shape[1],
                                       max(1, page_size // 16))
    ws = workspace if workspace is not None else AttnWorkspace(q.device)
    part_o, part_ml = ws.get(B, Hq, D, num_splits)
    paged_decode_attention_partial(q, pool, page_table, seq_lens, page_size, scale, part_o,
                                   part_ml, num_splits)
    if out is None:
        out = torch.empty(B, Hq, D, dtype=torch.float16, device=q.device)
    return paged_attn_reduce(part_o, part_ml, out, num_splits)


def kv_append(k_new: torch.Tensor, v_new: torch.Tensor, pool: PoolView, slots: torch.Tensor,
              offsets: torch.Tensor, page_size: int) -> None:
    """Write k_new/v_new [B, Hkv, n_tok, D] at (slots[b], offsets[b] + t) of the pool."""
    _native.require_cuda(k_new, v_new, pool.k, slots, offsets, what="kv_append")
    k_new = k_new.contiguous()
    v_new = v_new.contiguous()
    B, Hkv, n_tok, D = k_new.shape
    _native.call("helm_kv_append", k_new.data_ptr(), v_new.data_ptr(), pool.k.data_ptr(),
                 pool.v.data_ptr(), pool.slot_stride, pool.head_stride, pool.num_slots,
                 slots.data_ptr(), offsets.data_ptr(), B, Hkv, n_tok, D, page_size,
                 _native.stream_ptr(k_new.device))


def stage_pages_h2d(host_pool: torch.Tensor, dev_staging: torch.Tensor, host_slots,
                    dev_first_slot: int, copy_stream: torch.cuda.Stream,
                    done_event: Optional[torch.cuda.Event] = None) -> None:
    """Copy pages host_pool[host_slots[i]] -> dev_staging[dev_first_slot + i] on
    `copy_stream` (pinned host pool; runs of consecutive slots become one copy)."""
    import numpy as np

    hs = np.ascontiguousarray(np.asarray(host_slots, dtype=np.int32))
    page_bytes = host_pool[0].numel() * host_pool.element_size()
    _native.call("helm_stage_pages_h2d", host_pool.data_ptr(), dev_staging.data_ptr(),
                 hs.ctypes.data, int(hs.size), int(dev_first_slot), int(page_bytes),
                 copy_stream.cuda_stream, None)
    if done_event is not None:
        # torch creates its event lazily on record, so it is recorded here
        done_event.record(copy_stream)
