"""Paged GQA decode attention and KV page writes on the GPU (functional layer).

Thin typed wrappers over helm_paged_decode_attn / helm_paged_attn_reduce /
helm_kv_append / helm_stage_pages_h2d.

KV layout.  A page of the reference is a pair of (1, Hkv, P, D) tensors
(helm/runtime/kv_allocator.py:26-28).  Here every page is a slot of a pool: K is
stored [slots, Hkv, P, D] (token rows of D), V is stored token-contiguous per
dim, [slots, Hkv, D, P], and handed around as its transposed view, so the
logical shape of both is still [slots, Hkv, P, D] and a slot view is the
reference's page tensor.  `alloc_v` makes such V storage; `PoolView` carries
the strides the kernels need (see helm_kv_pool in include/helm_mi355x.h).
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from .. import _native

# Target workgroups (4 waves each) for one attention launch: one per CU on 256 CUs.
# Measured at batch 1 (Qwen3-8B shape, 16K and 32K context): 256 workgroups stream
# the pages as fast as 512 and halve the partials the reduce has to merge.
_TARGET_WGS = 256
# Pages one split may cover (helm_paged_attn_max_split_pages(): the split's page
# table slice is staged in LDS).
MAX_SPLIT_PAGES = 4096
# Fewest tokens a split is cut to (one 32-token step for each of its four
# waves): below this the split overhead outweighs the parallelism.  Measured at
# batch 1 (8 kv heads): 128 against 256 gives 8.9 vs 10.0 us at 4K context, 7.9
# vs 9.6 us at 2K (partials + reduce), the same from 8K on.
MIN_SPLIT_TOKENS = 128


STEP_TOKENS = 32   # tokens of one wave step of the decode attention kernel


def table_steps(max_pages: int, page_size: int = 16) -> int:
    """32-token steps of a page table of `max_pages` columns."""
    return -(-max(1, int(max_pages)) * int(page_size) // STEP_TOKENS)


def split_pages(max_pages: int, num_splits: int, page_size: int = 16) -> int:
    """Page-table entries one split stages in helm_paged_decode_attn /
    helm_decode_attn_fused (at most helm_paged_attn_max_split_pages()): the
    table's 32-token steps are dealt to the splits round robin (split s takes
    steps s, s + S, s + 2S, ...), so a split holds ceil(steps / S) of them, each
    covering max(1, 32 // page_size) entries."""
    upp = max(1, STEP_TOKENS // int(page_size))
    return -(-table_steps(max_pages, page_size) // max(1, int(num_splits))) * upp


def split_steps(num_tokens: int, max_pages: int, num_splits: int, split: int,
                page_size: int = 16) -> list:
    """Global step indices split `split` attends for `num_tokens` live tokens (the
    kernel's rule: round robin over the live steps of the table)."""
    live = min(-(-max(0, int(num_tokens)) // STEP_TOKENS), table_steps(max_pages, page_size))
    return list(range(split, live, max(1, int(num_splits))))


def choose_num_splits(batch: int, num_kv_heads: int, max_pages: int, page_size: int = 16,
                      target_wgs: int = _TARGET_WGS, min_tokens: int = MIN_SPLIT_TOKENS) -> int:
    """Split count for a page table of `max_pages` columns: at most target_wgs
    workgroups of batch * num_kv_heads * splits (more than one per CU measured
    slower at batch 1, idle workgroups included), each split at least
    `min_tokens` tokens of the full table and at most
    helm_paged_attn_max_split_pages() staged entries.  The kernel deals the live
    32-token steps to the splits round robin (split_steps), so every split gets
    within one step of the same share of whatever length is live."""
    max_pages = max(1, int(max_pages))
    want = max(1, target_wgs // max(1, batch * num_kv_heads))
    cap = max(1, (max_pages * page_size) // int(min_tokens))
    n = int(max(1, min(want, cap, max_pages)))
    while split_pages(max_pages, n, page_size) > MAX_SPLIT_PAGES:
        n += 1
    return n


def alloc_v(shape, dtype=torch.float16, device=None, pin_memory: bool = False,
            zero: bool = False) -> torch.Tensor:
    """V storage for `shape` = (..., T, D): allocated as (..., D, T) and returned as
    its (..., T, D) transposed view (tokens contiguous per dim)."""
    *lead, t, d = shape
    kw = dict(dtype=dtype, device=device)
    if pin_memory:
        kw["pin_memory"] = True
    store = torch.zeros(*lead, d, t, **kw) if zero else torch.empty(*lead, d, t, **kw)
    return store.transpose(-1, -2)


def v_storage(v: torch.Tensor) -> torch.Tensor:
    """The (..., D, T) storage behind a V view made by alloc_v."""
    return v.transpose(-1, -2)


class KvPoolStruct(ctypes.Structure):
    """helm_kv_pool (include/helm_mi355x.h)."""
    _fields_ = [("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
                ("k_slot_stride", ctypes.c_int64), ("k_head_stride", ctypes.c_int64),
                ("v_slot_stride", ctypes.c_int64), ("v_head_stride", ctypes.c_int64),
                ("v_dim_stride", ctypes.c_int64), ("num_slots", ctypes.c_int64)]


@dataclass
class PoolView:
    """Where K/V pages live, in the kernels' terms: page `slot` of kv head h holds
    K at k[slot*k_slot_stride + h*k_head_stride + t*D + d] and V at
    v[slot*v_slot_stride + h*v_head_stride + d*v_dim_stride + t] (elements)."""
    k: torch.Tensor
    v: torch.Tensor
    k_slot_stride: int
    k_head_stride: int
    v_slot_stride: int
    v_head_stride: int
    v_dim_stride: int
    num_slots: int
    num_kv_heads: int

    def c_struct(self) -> KvPoolStruct:
        return KvPoolStruct(self.k.data_ptr(), self.v.data_ptr(), self.k_slot_stride,
                            self.k_head_stride, self.v_slot_stride, self.v_head_stride,
                            self.v_dim_stride, self.num_slots)

    def c_ref(self):
        """A pointer to a helm_kv_pool for one call (kept alive by the caller's frame)."""
        return ctypes.byref(self.c_struct())

    @staticmethod
    def _check(k: torch.Tensor, v: torch.Tensor) -> None:
        d = k.shape[-1]
        if k.stride(-1) != 1 or k.stride(-2) != d:
            raise RuntimeError("PoolView: K pages must be token rows of D contiguous elements")
        if v.stride(-2) != 1:
            raise RuntimeError("PoolView: V must be stored token-contiguous per dim "
                               "(allocate it with helm_amd.kernels.attention.alloc_v)")

    @staticmethod
    def of_pool(k_pool: torch.Tensor, v_pool: torch.Tensor) -> "PoolView":
        """k_pool / v_pool: [slots, Hkv, P, D] (v_pool a view made by alloc_v)."""
        PoolView._check(k_pool, v_pool)
        s, hkv, _, _ = k_pool.shape
        return PoolView(k_pool, v_pool, k_pool.stride(0), k_pool.stride(1), v_pool.stride(0),
                        v_pool.stride(1), v_pool.stride(3), s, hkv)

    @staticmethod
    def of_sequences(k_seq: torch.Tensor, v_seq: torch.Tensor, page_size: int) -> "PoolView":
        """k_seq / v_seq: [n, Hkv, cap, D] views of n sequences' contiguous K/V with
        the sequence dim strided (see alloc_sequences); page i of sequence b is slot
        b * (cap // page_size) + i."""
        PoolView._check(k_seq, v_seq)
        n, hkv, cap, d = k_seq.shape
        if cap % page_size:
            raise RuntimeError("PoolView: capacity must be a multiple of the page size")
        if n > 1 and (k_seq.stride(0) != cap * d or v_seq.stride(0) != cap):
            raise RuntimeError("PoolView: sequences must be adjacent in the token dimension")
        return PoolView(k_seq, v_seq, page_size * d, k_seq.stride(1), page_size, v_seq.stride(1),
                        v_seq.stride(3), n * (cap // page_size), hkv)

    # back-compat name: a single contiguous [1, Hkv, cap, D] buffer
    of_contiguous = of_sequences

    @staticmethod
    def of_blocked_sequences(k_seq: torch.Tensor, v_blocks: torch.Tensor,
                             page_size: int) -> "PoolView":
        """k_seq [n, Hkv, cap, D] as for of_sequences; v_blocks [Hkv, n, cap / P,
        D, P], V in page blocks (alloc_blocked_sequences, or rows of it): page i
        of sequence b is slot b * (cap // P) + i, its V a D x P block like a pool
        page's."""
        n, hkv, cap, d = k_seq.shape
        P = page_size
        if k_seq.stride(-1) != 1 or k_seq.stride(-2) != d:
            raise RuntimeError("PoolView: K pages must be token rows of D contiguous elements")
        if cap % P:
            raise RuntimeError("PoolView: capacity must be a multiple of the page size")
        if n > 1 and k_seq.stride(0) != cap * d:
            raise RuntimeError("PoolView: sequences must be adjacent in the token dimension")
        if tuple(v_blocks.shape) != (hkv, n, cap // P, d, P):
            raise RuntimeError(f"PoolView: V blocks {tuple(v_blocks.shape)} do not match K "
                               f"{tuple(k_seq.shape)} at page size {P}")
        if (v_blocks.stride(4) != 1 or v_blocks.stride(3) != P or v_blocks.stride(2) != d * P
                or (n > 1 and v_blocks.stride(1) != (cap // P) * d * P)):
            raise RuntimeError("PoolView: V blocks must be D x P page blocks, sequences adjacent")
        return PoolView(k_seq, v_blocks, P * d, k_seq.stride(1), d * P, v_blocks.stride(0), P,
                        n * (cap // P), hkv)

    @staticmethod
    def of_whole_sequences(k_seq: torch.Tensor, v_seq: torch.Tensor) -> "PoolView":
        """k_seq / v_seq: [n, Hkv, cap, D] as for of_sequences, addressed with one
        slot per sequence and a page size of `cap` tokens: helm_kv_append with
        slots[b] = b, offsets[b] = position and P = cap writes token `position`
        of sequence b."""
        PoolView._check(k_seq, v_seq)
        n, hkv, _, _ = k_seq.shape
        return PoolView(k_seq, v_seq, k_seq.stride(0), k_seq.stride(1), v_seq.stride(0),
                        v_seq.stride(1), v_seq.stride(3), n, hkv)


def alloc_sequences(n: int, num_kv_heads: int, cap: int, head_dim: int, dtype=torch.float16,
                    device=None, zero: bool = True):
    """K/V buffers for n sequences of `cap` tokens: K stored [Hkv, n, cap, D], V
    stored [Hkv, D, n, cap], returned as [n, Hkv, cap, D] views (k, v); a
    sequence's [1, Hkv, cap, D] slice is the reference's contiguous per-layer buffer
    (helm/runtime/kv_cache.py:219-222) and PoolView.of_sequences addresses all n."""
    mk = torch.zeros if zero else torch.empty
    ks = mk(num_kv_heads, n, cap, head_dim, dtype=dtype, device=device)
    vs = mk(num_kv_heads, head_dim, n, cap, dtype=dtype, device=device)
    return ks.permute(1, 0, 2, 3), vs.permute(2, 0, 3, 1)


def alloc_blocked_sequences(n: int, num_kv_heads: int, cap: int, head_dim: int, page_size: int,
                            dtype=torch.float16, device=None, zero: bool = True):
    """K/V buffers for n sequences of `cap` tokens (a multiple of page_size) with V
    in page blocks: K stored [Hkv, n, cap, D] and returned as its [n, Hkv, cap,
    D] view (as alloc_sequences); V stored [Hkv, n, cap / P, D, P], each P-token
    page a D x P block (tokens contiguous per dim), as the page pools hold V, so
    a decode step's V reads are whole 4 KB blocks rather than 32-byte pieces of
    each dim's row.  PoolView.of_blocked_sequences addresses both."""
    if cap % page_size:
        raise ValueError(f"capacity {cap} is not a multiple of the page size {page_size}")
    mk = torch.zeros if zero else torch.empty
    ks = mk(num_kv_heads, n, cap, head_dim, dtype=dtype, device=device)
    vb = mk(num_kv_heads, n, cap // page_size, head_dim, page_size, dtype=dtype, device=device)
    return ks.permute(1, 0, 2, 3), vb


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
    max_pages = page_table.shape[1]
    total = num_splits if total_splits is None else total_splits
    _native.call("helm_paged_decode_attn", q.data_ptr(), q.stride(0), q.stride(1), pool.c_ref(),
                 page_table.data_ptr(), page_table.stride(0), seq_lens.data_ptr(),
                 part_o.data_ptr(), part_ml.data_ptr(), split_offset, total, B, Hq,
                 pool.num_kv_heads, D, page_size, max_pages, num_splits, float(scale),
                 _native.stream_ptr(q.device))


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
        num_splits = choose_num_splits(B, pool.num_kv_heads, page_table.shape[1], page_size)
    ws = workspace if workspace is not None else AttnWorkspace(q.device)
    part_o, part_ml = ws.get(B, Hq, D, num_splits)
    paged_decode_attention_partial(q, pool, page_table, seq_lens, page_size, scale, part_o,
                                   part_ml, num_splits)
    if out is None:
        out = torch.empty(B, Hq, D, dtype=torch.float16, device=q.device)
    return paged_attn_reduce(part_o, part_ml, out, num_splits)


def decode_attention_fused_cs(qkv: torch.Tensor, q_norm_w: Optional[torch.Tensor],
                              k_norm_w: Optional[torch.Tensor], eps: float, cos: torch.Tensor,
                              sin: torch.Tensor, pool: PoolView, slots: torch.Tensor,
                              offsets: torch.Tensor, page_table: torch.Tensor,
                              seq_lens: torch.Tensor, page_size: int, scale: float,
                              part_o: torch.Tensor, part_ml: torch.Tensor, num_splits: int,
                              n_heads: int, n_kv_heads: int, head_dim: int) -> None:
    """One launch of a decode layer's attention half (helm_decode_attn_fused_cs):
    q / k RMSNorm (when the norm weights are given) and RoPE with the model's
    fp16 cos / sin rows [B, D] on the projection output qkv [B, (Hq + 2 Hkv) D],
    the new token's k / v into page slot (slots[b], offsets[b]) of `pool`, and the
    split-K partials over page_table [B, max_pages] with seq_lens[b] tokens
    (the new one included).  helm_paged_attn_reduce merges the partials."""
    _native.require_cuda(qkv, q_norm_w, k_norm_w, cos, sin, pool.k, slots, offsets, page_table,
                         seq_lens, what="decode_attention_fused_cs")
    if qkv.dtype != torch.float16 or cos.dtype != torch.float16 or sin.dtype != torch.float16:
        raise RuntimeError("decode_attention_fused_cs: qkv and cos / sin must be fp16")
    B = qkv.shape[0]
    if qkv.dim() != 2 or qkv.stride(1) != 1 or qkv.shape[1] != (n_heads + 2 * n_kv_heads) * head_dim:
        raise RuntimeError("decode_attention_fused_cs: qkv must be [B, (Hq + 2 Hkv) * D], unit stride")
    if (cos.shape[0] != B or cos.shape[-1] != head_dim or cos.stride(-1) != 1
            or sin.stride() != cos.stride() or sin.shape != cos.shape):
        raise RuntimeError("decode_attention_fused_cs: cos / sin must be [B, D] rows with unit stride")
    if page_table.dim() != 2 or page_table.stride(1) != 1 or page_table.dtype != torch.int32:
        raise RuntimeError("decode_attention_fused_cs: page_table must be int32 [B, max_pages], row-major")
    _native.call("helm_decode_attn_fused_cs", qkv.data_ptr(), qkv.stride(0), _native.ptr(q_norm_w),
                 _native.ptr(k_norm_w), float(eps), cos.data_ptr(), sin.data_ptr(), cos.stride(0),
                 slots.data_ptr(), offsets.data_ptr(), pool.c_ref(), page_table.data_ptr(),
                 page_table.stride(0), seq_lens.data_ptr(), part_o.data_ptr(), part_ml.data_ptr(),
                 B, n_heads, n_kv_heads, head_dim, page_size, page_table.shape[1], num_splits,
                 float(scale), _native.stream_ptr(qkv.device))


def kv_append(k_new: torch.Tensor, v_new: torch.Tensor, pool: PoolView, slots: torch.Tensor,
              offsets: torch.Tensor, page_size: int) -> None:
    """Write k_new/v_new [B, Hkv, n_tok, D] at (slots[b], offsets[b] + t) of the pool."""
    _native.require_cuda(k_new, v_new, pool.k, slots, offsets, what="kv_append")
    k_new = k_new.contiguous()
    v_new = v_new.contiguous()
    B, Hkv, n_tok, D = k_new.shape
    _native.call("helm_kv_append", k_new.data_ptr(), v_new.data_ptr(), pool.c_ref(),
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


def gather_pages_h2d(host_k: torch.Tensor, host_v: torch.Tensor, dev_k: torch.Tensor,
                     dev_v: torch.Tensor, slots: torch.Tensor, dev_first_slot: int,
                     stream: torch.cuda.Stream) -> None:
    """dev_k/dev_v page dev_first_slot + i <- pinned host_k/host_v page slots[i]
    (slots: device int32), by one kernel on `stream` that reads host memory
    directly.  Pools are [slots, ...] tensors with whole pages contiguous (V
    storage from alloc_v: pass the transposed views; their data pointers are the
    storage)."""
    if not (host_k.is_pinned() and host_v.is_pinned()):
        raise RuntimeError("gather_pages_h2d: host pools must be pinned")
    _native.require_cuda(dev_k, dev_v, slots, what="gather_pages_h2d")
    if slots.dtype != torch.int32 or not slots.is_contiguous():
        raise RuntimeError("gather_pages_h2d: slots must be a contiguous int32 tensor")
    page_bytes = host_k[0].numel() * host_k.element_size()
    _native.call("helm_gather_pages_h2d", host_k.data_ptr(), host_v.data_ptr(), dev_k.data_ptr(),
                 dev_v.data_ptr(), slots.data_ptr(), int(slots.numel()), int(dev_first_slot),
                 int(page_bytes), int(host_k.shape[0]), stream.cuda_stream)


def kernel_mask(mask: torch.Tensor, T: int, kv_len: int, Hq: int):
    """A [Hm, T, kv_len] attention mask (Hm 1 or Hq; bool True = attend, or
    additive float) as the fp16 additive mask helm_prefill_attn_mask reads: rows
    padded to a multiple of 32 keys, False -> -inf (SDPA's reading of a boolean
    mask), floats cast to fp16 (as the fp16 SDPA adds them).  Returns (mask, head
    stride, key_end): stride 0 when one mask serves every head; key_end int32
    [T], per row one past the last key that is not -inf in some head (0 for a
    row with none)."""
    if mask.dim() != 3 or mask.shape[1] != T or mask.shape[2] != kv_len or mask.shape[0] not in (1, Hq):
        raise RuntimeError(f"prefill_attention: mask must be [1 or {Hq}, {T}, {kv_len}], got "
                           f"{list(mask.shape)}")
    pitch = -(-kv_len // 32) * 32
    m = torch.full((mask.shape[0], T, pitch), float("-inf"), dtype=torch.float16, device=mask.device)
    if mask.dtype == torch.bool:
        m[:, :, :kv_len].masked_fill_(mask, 0.0)
    else:
        m[:, :, :kv_len].copy_(mask)
    vis = (m[:, :, :kv_len] > float("-inf")).any(0)                      # [T, kv_len]
    last = kv_len - vis.flip(-1).to(torch.int8).argmax(-1)
    key_end = torch.where(vis.any(-1), last, torch.zeros_like(last)).to(torch.int32)
    return m, (0 if mask.shape[0] == 1 else T * pitch), key_end


def prefill_attention(q: torch.Tensor, pool: PoolView, page_table: torch.Tensor, page_size: int,
                      q_start: int = 0, scale: Optional[float] = None,
                      out: Optional[torch.Tensor] = None,
                      mask: Optional[torch.Tensor] = None, key_ranges: bool = True) -> torch.Tensor:
    """Causal attention of the T queries q [T, Hq, D] (positions q_start ..
    q_start+T-1) over the keys 0 .. q_start+T-1 of one sequence's pages
    (page_table [>= ceil((q_start+T)/P)] int32 slots).  Returns [T, Hq, D] fp16.

    With `mask` ([Hm, T, kv_len], Hm 1 or Hq, bool or additive; q_start must be 0)
    every query sees keys 0 .. kv_len-1 instead, with the mask added to its scaled
    scores (SDPA's attn_mask, kv_offload.py:253-265); with key_ranges a workgroup
    stops after the last key any of its rows sees (the mask is -inf beyond)."""
    _native.require_cuda(q, pool.k, pool.v, page_table, what="prefill_attention")
    if q.dtype != torch.float16 or q.dim() != 3 or q.stride(-1) != 1:
        raise RuntimeError("prefill_attention: q must be fp16 [T, Hq, D] with unit stride on D")
    if page_table.dtype != torch.int32 or page_table.stride(-1) != 1:
        raise RuntimeError("prefill_attention: page_table must be a contiguous int32 vector")
    T, Hq, D = q.shape
    kv_len = q_start + T if mask is None else int(mask.shape[-1])
    if mask is not None and q_start != 0:
        raise RuntimeError("prefill_attention: a mask covers the keys itself (q_start must be 0)")
    if page_table.numel() * page_size < kv_len:
        raise RuntimeError("prefill_attention: page table does not cover the keys")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if out is None:
        out = torch.empty(T, Hq, D, dtype=torch.float16, device=q.device)
    if mask is None:
        _native.call("helm_prefill_attn", q.data_ptr(), q.stride(0), q.stride(1), pool.c_ref(),
                     page_table.data_ptr(), int(q_start), T, Hq, pool.num_kv_heads, D, page_size,
                     float(scale), out.data_ptr(), out.stride(0), out.stride(1),
                     _native.stream_ptr(q.device))
        return out
    _native.require_cuda(mask, what="prefill_attention")
    m, m_sh, ke = kernel_mask(mask, T, kv_len, Hq)
    _native.call("helm_prefill_attn_mask", q.data_ptr(), q.stride(0), q.stride(1), pool.c_ref(),
                 page_table.data_ptr(), T, kv_len, Hq, pool.num_kv_heads, D, page_size,
                 float(scale), m.data_ptr(), m_sh, m.stride(1), ke.data_ptr() if key_ranges else None,
                 out.data_ptr(), out.stride(0), out.stride(1), _native.stream_ptr(q.device))
    return out


def dense_prefill_pool(S: int, num_kv_heads: int, head_dim: int, page_size: int, device):
    """An empty page-layout buffer for one sequence of S tokens (ceil(S/P) pages,
    zero-filled) with its identity page table: (PoolView, page_table); the
    PoolView's k / v are the sequence's [1, Hkv, cap, D] views."""
    cap = -(-S // page_size) * page_size
    kb, vb = alloc_sequences(1, num_kv_heads, cap, head_dim, torch.float16, device, zero=True)
    pt = torch.arange(cap // page_size, dtype=torch.int32, device=device)
    return PoolView.of_sequences(kb, vb, page_size), pt


def dense_prefill_kv(k: torch.Tensor, v: torch.Tensor, page_size: int = 16):
    """Scratch copies of one sequence's prompt K/V [S, Hkv, D] in the kernels'
    page layout (K token rows per head, V token-contiguous per dim), as a pool of
    ceil(S/P) pages with an identity page table: (PoolView, page_table)."""
    S, Hkv, D = k.shape
    cap = -(-S // page_size) * page_size
    kb, vb = alloc_sequences(1, Hkv, cap, D, torch.float16, k.device, zero=True)
    kb[0, :, :S].copy_(k.transpose(0, 1))
    vb[0, :, :S].copy_(v.transpose(0, 1))
    pt = torch.arange(cap // page_size, dtype=torch.int32, device=k.device)
    return PoolView.of_sequences(kb, vb, page_size), pt
