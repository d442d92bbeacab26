/*
 * helm_mi355x.h — C ABI of libhelm_mi355x.so, the gfx950 (MI355X) decode hot path:
 * INT8 weight-only linear (GEMV for decode, MFMA GEMM for prefill) and paged GQA
 * decode attention with split-K online-softmax partials.
 *
 * Conventions (every entry point):
 *   - Plain pointers and sizes only.  Every pointer is a device pointer unless its
 *     name says `host`.  The caller owns every buffer; no entry point allocates or
 *     frees device memory, and none synchronises the host with the device.
 *   - Work is enqueued on the `stream` argument (a hipStream_t passed as void*;
 *     NULL = the legacy default stream).  Ordering is by stream only.
 *   - fp16 data is IEEE binary16 passed as void*.  Strides are in elements.
 *   - Return value: HELM_OK (0) on success, a negative HELM_ERR_* code otherwise.
 *     helm_last_error() returns a message for the last failure on the calling
 *     thread.  Argument checks happen before anything is enqueued.
 *   - Stateless and thread-safe: calls on different streams may run concurrently,
 *     except helm_paged_decode_attn_noalloc, whose partials live in one per-GPU
 *     array of the library, so its calls that overlap on one GPU race (see its
 *     declaration).
 *
 * The reference binds its one native op through pybind11
 * (helm/kernels/fp16_gemv.cpp:159-163) and raises RuntimeError via TORCH_CHECK
 * (fp16_gemv.cpp:110-126); the Python layer of this library turns a non-zero
 * return into RuntimeError(helm_last_error()) in the same way.
 */
#ifndef HELM_MI355X_H
#define HELM_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HELM_OK               0
#define HELM_ERR_INVALID_ARG -1  /* null pointer, non-positive size, bad stride      */
#define HELM_ERR_UNSUPPORTED -2  /* shape/alignment outside what the kernels handle */
#define HELM_ERR_HIP         -3  /* a HIP runtime call failed                        */

/* Message for the last non-zero return on this thread ("" if none). */
const char* helm_last_error(void);

/* Library version string, e.g. "helm_mi355x 0.1 gfx950". */
const char* helm_version(void);

/* ------------------------------------------------------------------------ */
/* Linear: INT8 weight-only, per-output-channel symmetric scales            */
/*   y[m,n] = fp16( scale[n] * sum_k q[n,k] * x[m,k]  (+ bias[n]) )         */
/* fp32 accumulation; bias added in fp32 before the single rounding, as the */
/* reference does for its fp16 GEMV (fp16_gemv.cpp:146-151).               */
/* ------------------------------------------------------------------------ */

/* Decode GEMV, 1 <= M <= 16 tokens.  Replaces the decode fast path of
 * helm_fp16_linear (helm/kernels/fp16_gemv.cpp:105-157, dispatch at
 * helm/kernels/__init__.py:72-82) with an int8-weight GPU kernel.
 *   x     [M, K] fp16, row stride ldx        q     [N, K] int8, row stride ldq
 *   scale [N] fp16                           bias  [N] fp16 or NULL
 *   y     [M, N] fp16, row stride ldy
 * Requirements: K % 16 == 0, ldq % 16 == 0, ldx % 8 == 0, q and x 16-byte aligned. */
int helm_int8_gemv(const void* x, int64_t ldx, const int8_t* q, int64_t ldq,
                   const void* scale, const void* bias, void* y, int64_t ldy,
                   int M, int N, int K, void* stream);

/* fp16-weight decode GEMV, 1 <= M <= 16: the GPU counterpart of the reference's
 * own op helm_fp16_linear (fp16_gemv.cpp:45-157): y = fp16(W x + bias), fp32
 * accumulate.  W [N, K] fp16 row stride ldw.  Same requirements as above with
 * K % 8 == 0 and ldw % 8 == 0.  Used for the fp16 lm_head. */
int helm_fp16_gemv(const void* x, int64_t ldx, const void* w, int64_t ldw,
                   const void* bias, void* y, int64_t ldy,
                   int M, int N, int K, void* stream);

/* Fused decode variants of helm_int8_gemv (no counterpart in the reference, which
 * runs these steps as separate torch ops inside the HF decoder layer,
 * helm/runtime/kv_offload.py:241-271 and transformers' Qwen3DecoderLayer).
 *   norm_w != NULL: x is first RMS-normalised per token,
 *       xn = fp16( norm_w * fp16( x * rsqrt(mean(x^2) + eps) ) )
 *       (at 3-16 tokens and K = 4096 inside the matrix-core kernel, each
 *       workgroup normalising its own copy: from 5 tokens on, helm_rmsnorm and
 *       the call without norm_w are faster for the plain linear)
 *   residual != NULL: y = fp16( residual + fp16(linear(x)) ), residual [M, N] row
 *       stride ldy (may alias y). */
int helm_int8_gemv_fused(const void* x, int64_t ldx, const void* norm_w, float eps,
                         const int8_t* q, int64_t ldq, const void* scale,
                         const void* bias, const void* residual,
                         void* y, int64_t ldy, int M, int N, int K, void* stream);

/* helm_int8_gemv_fused without the norm prologue, with a caller-owned workspace
 * of helm_int8_gemv_workspace_bytes(M, N, K) bytes (16-byte aligned; its contents
 * on entry do not matter).  Shapes whose activations of 8-16 tokens exceed the
 * kernel's LDS (K a multiple of 3072 above 4096, N % 4 == 0, e.g. the Qwen3-8B
 * down projection 12288 -> 4096) then split K over workgroups, keep fp32 partial
 * sums there and reduce them in a second kernel; every other shape (workspace
 * bytes 0) runs as helm_int8_gemv_fused and may pass workspace NULL.  Same results
 * up to the fp32 summation order.  Replaces the same decode fast path as
 * helm_int8_gemv (helm/kernels/fp16_gemv.cpp:105-157). */
int64_t helm_int8_gemv_workspace_bytes(int M, int N, int K);
int helm_int8_gemv_ws(const void* x, int64_t ldx, const int8_t* q, int64_t ldq,
                      const void* scale, const void* bias, const void* residual,
                      void* y, int64_t ldy, int M, int N, int K,
                      void* workspace, int64_t workspace_bytes, void* stream);

/* Fused gate/up projection with SwiGLU (Qwen3MLP: down(silu(gate(x)) * up(x))):
 *   g = fp16(sg[n] * q_gate[n,:].xn),  u = fp16(su[n] * q_up[n,:].xn),
 *   y[m,n] = fp16( fp16(silu(g)) * u ),  xn as above when norm_w != NULL. */
int helm_int8_gemv_swiglu(const void* x, int64_t ldx, const void* norm_w, float eps,
                          const int8_t* q_gate, const void* s_gate,
                          const int8_t* q_up, const void* s_up, int64_t ldq,
                          void* y, int64_t ldy, int M, int N, int K, void* stream);

/* Prefill GEMM (M > 16): int8 weights are dequantised into LDS as fp16 (|q| <= 127
 * is exact in fp16) and contracted on MFMA with fp32 accumulation; scale and bias
 * in the epilogue.  Replaces the prefill branch of fp16_linear
 * (helm/kernels/__init__.py:83-86: fp32 F.linear on the CPU) and torch::linear
 * (fp16_gemv.cpp:130-134).  Same operand layout as helm_int8_gemv, any M >= 1.
 * Requirements: K % 64 == 0, ldq % 16 == 0, ldx % 8 == 0, 16-byte aligned. */
int helm_int8_gemm(const void* x, int64_t ldx, const int8_t* q, int64_t ldq,
                   const void* scale, const void* bias, void* y, int64_t ldy,
                   int M, int N, int K, void* stream);

/* ------------------------------------------------------------------------ */
/* Paged GQA decode attention                                               */
/* ------------------------------------------------------------------------ */
/* KV storage.  One pool (or one contiguous per-layer buffer) of fp16 pages:
 *   K element (slot s, kv head h, token t, dim d) at
 *       k[s*k_slot_stride + h*k_head_stride + t*D + d]        (token rows of D)
 *   V element (s, h, t, d) at
 *       v[s*v_slot_stride + h*v_head_stride + d*v_dim_stride + t]  (tokens contiguous)
 * V is kept token-contiguous per dim so that the attention kernel's P.V product
 * reads 8 consecutive tokens of one dim with one 16-byte load.  The reference's
 * per-page tensors (1, Hkv, P, D) (helm/runtime/kv_allocator.py:26-28) are slot
 * views of such a pool: k_slot_stride = Hkv*P*D, k_head_stride = P*D,
 * v_slot_stride = Hkv*D*P, v_head_stride = D*P, v_dim_stride = P.  A contiguous
 * per-layer buffer (1, Hkv, cap, D) (helm/runtime/kv_cache.py:206-234) is the same
 * with slot i = page i: k_slot_stride = P*D, k_head_stride = cap*D,
 * v_slot_stride = P, v_head_stride = D*cap, v_dim_stride = cap.
 * num_slots: pool size in pages; page-table entries / slots outside
 * [0, num_slots) are never dereferenced.  All strides are in elements. */
typedef struct helm_kv_pool {
  void* k;
  void* v;
  int64_t k_slot_stride, k_head_stride;
  int64_t v_slot_stride, v_head_stride, v_dim_stride;
  int64_t num_slots;
} helm_kv_pool;

/* page_table [B, pt_stride] int32: slot of the i-th page (token order) of item b.
 * seq_lens [B] int32: tokens of item b; page i holds min(P, seq_len - i*P) tokens.
 * A page-table entry outside [0, num_slots) contributes no tokens, and pages past
 * max_pages are ignored.
 *
 * out[b, h, :] = softmax(scale * q[b,h] . K_b^T) V_b over kv head h / (Hq/Hkv)
 * (the GQA mapping of repeat_interleave, helm/runtime/kv_cache.py:356-363), fp32
 * online softmax, fp16 out; an item with seq_len 0 yields zeros
 * (kv_cache.py:353-354).  Replaces perform_streaming_attention
 * (helm/runtime/kv_cache.py:318-442) and the decode SDPA calls of
 * _decode_batched (helm/runtime/kv_offload.py:126,160).
 *
 * Split-K: the 32-token steps of each (b, kv head)'s page table are dealt to
 * num_splits splits round robin (split s takes steps s, s + num_splits, ...; a
 * split stages ceil(steps/num_splits) steps' page-table entries, at most
 * helm_paged_attn_max_split_pages()), so the live tokens of any seq_len are
 * shared to within one step; split s writes an fp32 partial (o[D] normalised by its own sum, and (max, sum)
 * in the log2 domain) at split index split_offset + s of
 *   part_o  [B, Hq, total_splits, D] fp32,  part_ml [B, Hq, total_splits, 2] fp32,
 * so several launches (e.g. device-resident pages, then staged host pages) can
 * fill disjoint split ranges of one buffer.  helm_paged_attn_reduce merges all
 * total_splits partials into out.  q [B, Hq, D] fp16 with strides
 * (q_stride_b, q_stride_h); out [B, Hq, D] fp16 contiguous.
 * Supported: D in {64, 128}, P in {16, 32, 64}, Hq % Hkv == 0, Hq/Hkv <= 16. */
int helm_paged_decode_attn(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                           const helm_kv_pool* pool,
                           const int32_t* page_table, int64_t pt_stride,
                           const int32_t* seq_lens,
                           float* part_o, float* part_ml, int split_offset, int total_splits,
                           int B, int Hq, int Hkv, int D, int P, int max_pages,
                           int num_splits, float scale, void* stream);

/* The attention half of one decode step for Qwen3-style layers, in one launch:
 * q/k RMSNorm (q_norm_w / k_norm_w over head_dim, eps) and RoPE (rotate_half,
 * angle inv_freq[i] * positions[b], cos/sin rounded to fp16) of the fused
 * projection output qkv [B, (Hq + 2*Hkv) * D] (q | k | v, row stride
 * qkv_stride_b), computed with the operations and order of
 * helm_qk_norm_rope_append; the new token's k and v are written into page slot
 * slots[b] at offset offsets[b] of `pool` (skipped when outside the pool or the
 * page); then the split-K partials (as helm_paged_decode_attn, total_splits =
 * num_splits) of the rotated q over the seq_lens[b] - 1 cached tokens of the
 * page table plus the new token, which is folded in by the last split instead
 * of being read back from the pool.  helm_paged_attn_reduce then merges the
 * partials.  Same math as helm_qk_norm_rope_append + helm_paged_decode_attn
 * (kv_offload.py:244-251, kv_cache.py:103-107 and :318-442). */
int helm_decode_attn_fused(const void* qkv, int64_t qkv_stride_b,
                           const void* q_norm_w, const void* k_norm_w, float eps,
                           const int32_t* positions, const float* inv_freq,
                           const int32_t* slots, const int32_t* offsets,
                           const helm_kv_pool* pool,
                           const int32_t* page_table, int64_t pt_stride,
                           const int32_t* seq_lens, float* part_o, float* part_ml,
                           int B, int Hq, int Hkv, int D, int P, int max_pages,
                           int num_splits, float scale, void* stream);

/* helm_decode_attn_fused with the RoPE rows a transformers model hands its
 * attention layer (position_embeddings: cos / sin [B, D] fp16, row stride
 * cs_stride_b, whatever RoPE scaling the model configures) instead of
 * positions and inv_freq, and the q / k RMSNorm optional (both norm weights
 * null for Qwen2 / Llama-style attention).  Per element the same roundings as
 * helm_qk_norm_rope_cs followed by the K/V page write and
 * helm_paged_decode_attn: fp16(w * fp16(x * rstd)), then
 * fp16(fp16(x * cos[d]) + fp16(rotate_half(x)[d] * sin[d])).  The patched
 * attention forward's decode half in one launch (kv_offload.py:241-251 and
 * :266-267 -> _decode_batched, kv_cache.py:87-113 and :318-442). */
int helm_decode_attn_fused_cs(const void* qkv, int64_t qkv_stride_b,
                              const void* q_norm_w, const void* k_norm_w, float eps,
                              const void* cos_rows, const void* sin_rows, int64_t cs_stride_b,
                              const int32_t* slots, const int32_t* offsets,
                              const helm_kv_pool* pool,
                              const int32_t* page_table, int64_t pt_stride,
                              const int32_t* seq_lens, float* part_o, float* part_ml,
                              int B, int Hq, int Hkv, int D, int P, int max_pages,
                              int num_splits, float scale, void* stream);

/* Causal prefill attention of one sequence: the T queries q [T, Hq, D] (strides
 * q_stride_t, q_stride_h; positions q_start .. q_start+T-1) attend keys
 * 0 .. q_start+i of the pages page_table[0 .. ceil((q_start+T)/P)) of `pool`
 * (whose K/V must already hold those tokens); out [T, Hq, D] fp16 (strides
 * out_stride_t, out_stride_h).  fp32 online softmax on the matrix cores.  The
 * prefill SDPA of kv_offload.py:253-265 with the causal mask of
 * pipeline_runtime.py:25-29.  Supported: D in {64, 128}, P in {16, 32, 64},
 * Hq a multiple of Hkv, ceil((q_start + T)/P) <= 4096 pages. */
int helm_prefill_attn(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                      const helm_kv_pool* pool, const int32_t* page_table,
                      int q_start, int T, int Hq, int Hkv, int D, int P, float scale,
                      void* out, int64_t out_stride_t, int64_t out_stride_h, void* stream);

/* Prefill attention of one sequence under an arbitrary additive mask: the T
 * queries q [T, Hq, D] attend keys 0 .. kv_len-1 of the pages page_table[0 ..
 * ceil(kv_len/P)) with softmax(scale * q.k + mask[h, t, key]).  mask is fp16,
 * element (h, t, key) at mask[h*mask_stride_h + t*mask_stride_t + key]
 * (mask_stride_h 0 broadcasts one mask over the heads; -inf removes a key; a row
 * with every key at -inf gives zeros); its rows must hold kv_len rounded up to
 * a multiple of 32 elements (the padding is read and ignored).  key_end
 * (int32 [T], or null): for each row one past the last key whose mask is not
 * -inf in some head (0 for a row with none); a workgroup then stops at the last
 * key step any of its rows can see.  The prefill SDPA of kv_offload.py:253-265 with the
 * attention_mask it is handed (padding or any other 4-D mask; the plain causal
 * mask takes helm_prefill_attn).  Same support limits as helm_prefill_attn;
 * mask 16-byte aligned, strides multiples of 8. */
int helm_prefill_attn_mask(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                           const helm_kv_pool* pool, const int32_t* page_table, int T,
                           int kv_len, int Hq, int Hkv, int D, int P, float scale,
                           const void* mask, int64_t mask_stride_h, int64_t mask_stride_t,
                           const int32_t* key_end, void* out, int64_t out_stride_t, int64_t out_stride_h, void* stream);

/* Largest number of page-table entries one split of helm_paged_decode_attn may
 * stage. */
int helm_paged_attn_max_split_pages(void);

/* part_ml must be 8-byte aligned (each split's (max, sum) pair is read as one). */
int helm_paged_attn_reduce(const float* part_o, const float* part_ml, void* out,
                           int B, int Hq, int D, int total_splits, void* stream);

/* Workspace floats needed by the split-K partials (part_o + part_ml). */
int64_t helm_paged_attn_workspace_floats(int B, int Hq, int D, int total_splits);

/* Allocation-free decode attention.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Computes exactly
 * helm_paged_decode_attn (split_offset 0, total_splits = num_splits) followed by
 * helm_paged_attn_reduce into out [B, Hq, D] fp16, with the split-K partials in a
 * library-owned device array of helm_paged_attn_noalloc_max_floats() floats
 * (16 MiB) per GPU instead of a caller workspace; it allocates and frees nothing.
 * Rejects (HELM_ERR_UNSUPPORTED) B * Hq * num_splits * (D + 2) above that limit.
 * The array belongs to the device current on the calling thread (the stream must
 * be on it) and is shared by every call on that GPU: calls that overlap on one
 * GPU race.  Same requirements as helm_paged_decode_attn otherwise. */
int helm_paged_decode_attn_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                   const helm_kv_pool* pool,
                                   const int32_t* page_table, int64_t pt_stride,
                                   const int32_t* seq_lens, void* out,
                                   int B, int Hq, int Hkv, int D, int P, int max_pages,
                                   int num_splits, float scale, void* stream);

/* Size limit of helm_paged_decode_attn_noalloc's scratch, in floats. */
int64_t helm_paged_attn_noalloc_max_floats(void);

/* ------------------------------------------------------------------------ */
/* KV page movement                                                         */
/* ------------------------------------------------------------------------ */

/* Write n_tok new tokens of every item into their page slots: K/V element
 * (slots[b], h, offsets[b] + t, d) of the pool = k_new/v_new[b, h, t, d]
 * (layout of helm_kv_pool), k_new/v_new [B, Hkv, n_tok, D] fp16 contiguous;
 * offsets[b] + n_tok must not exceed the page size P, and slots outside
 * [0, num_slots) are skipped.  Replaces the per-item copies of append_decode
 * (helm/runtime/kv_cache.py:103-107) and write_decode_contiguous
 * (kv_cache.py:245-249). */
int helm_kv_append(const void* k_new, const void* v_new, const helm_kv_pool* pool,
                   const int32_t* slots, const int32_t* offsets,
                   int B, int Hkv, int n_tok, int D, int P, void* stream);

/* Stage host-resident pages to the device by a kernel that reads pinned host
 * memory directly: K and V page slots[i] of the pinned host pools host_k / host_v
 * (page_bytes each, host_slots pages) are copied to pages dev_first_slot + i of
 * dev_k / dev_v, on `stream`.  slots is a DEVICE array of n int32; slots outside
 * [0, host_slots) are skipped.  The host pools must be pinned allocations the
 * runtime maps for the device (hipHostMalloc); anything else is refused before
 * launch.  One launch per chunk instead of a copy per run of adjacent host slots,
 * so pages scattered over the host pool stream at the host link's rate.
 * Replaces the per-page non_blocking .to(device) loop of
 * perform_streaming_attention (helm/runtime/kv_cache.py:412-423). */
int helm_gather_pages_h2d(const void* host_k, const void* host_v, void* dev_k, void* dev_v,
                          const int32_t* slots, int n, int64_t dev_first_slot, int64_t page_bytes,
                          int64_t host_slots, void* stream);

/* Stage host-resident pages to the device for attention: page host_slots[i] of the
 * pinned host pool (page_bytes each, contiguous pages) is copied to page
 * dev_first_slot + i of dev_staging, by hipMemcpyAsync on copy_stream, merging runs
 * of consecutive host slots into one copy.  When done_event != NULL it is recorded
 * on copy_stream after the last copy.  host_slots is a HOST array.  Replaces the
 * per-page non_blocking .to(device) + Event loop of perform_streaming_attention
 * (helm/runtime/kv_cache.py:412-423). */
int helm_stage_pages_h2d(const void* host_pool, void* dev_staging,
                         const int32_t* host_slots, int n, int64_t dev_first_slot,
                         size_t page_bytes, void* copy_stream, void* done_event);

/* ------------------------------------------------------------------------ */
/* Decode-step glue (widening around the path; no single reference counterpart) */
/* ------------------------------------------------------------------------ */

/* Per-head RMSNorm of q and k (Qwen3 q_norm/k_norm over head_dim), RoPE with the
 * rotate_half convention at position positions[b] (angle = inv_freq[i] * pos in
 * fp32, cos/sin rounded to fp16, products and sum rounded to fp16 as the fp16
 * torch ops of transformers' apply_rotary_pos_emb do), then the new k and v are
 * written into their page slots (slots[b], offsets[b]) of `pool` and the rotated q to
 * q_out [B, Hq, D].  qkv [B, (Hq + 2*Hkv) * D] fp16 is the fused projection output
 * (q | k | v); inv_freq [D/2] fp32.  Follows helm/runtime/kv_offload.py:244-249
 * and the page write of kv_cache.py:103-107.  Slots outside [0, num_slots) and
 * offsets outside [0, P) are not written. */
int helm_qk_norm_rope_append(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                             float eps, const int32_t* positions, const float* inv_freq,
                             void* q_out, const helm_kv_pool* pool,
                             const int32_t* slots, const int32_t* offsets,
                             int B, int Hq, int Hkv, int D, int P, void* stream);

/* The q / k half of helm_qk_norm_rope_append for callers that hold the model's
 * own RoPE tables (the patched attention forward of the drop-in path): per-head
 * RMSNorm of q and k when q_norm_w and k_norm_w are given (Qwen3; both null for
 * models without them), then RoPE with the rotate_half convention from the fp16
 * rows cos_t[b], sin_t[b] (row stride cs_stride_b, 0 for one row shared by
 * every item; head_dim values each: the
 * position_embeddings transformers hands every attention layer, any RoPE
 * scaling already applied), products and sum rounded to fp16 as
 * apply_rotary_pos_emb's fp16 ops round.  qkv [B, (Hq + 2*Hkv) * D] fp16
 * contiguous (q | k | v); writes q_out [B, Hq, D] and k_out [B, Hkv, D].
 * Follows helm/runtime/kv_offload.py:244-249 (the q_norm / k_norm calls and
 * apply_rotary_pos_emb of the patched Qwen3 forward). */
int helm_qk_norm_rope_cs(const void* qkv, const void* q_norm_w, const void* k_norm_w, float eps,
                         const void* cos_t, const void* sin_t, int64_t cs_stride_b,
                         void* q_out, void* k_out, int B, int Hq, int Hkv, int D, void* stream);

/* fp16 GEMV of RMS-normalised activations: y = fp16(W . rmsnorm(x)) with the
 * normalisation of helm_rmsnorm applied on the way in (the final norm + lm_head
 * of a decode step in one launch).  W [N, K] fp16, M <= 16. */
int helm_fp16_gemv_rmsnorm(const void* x, int64_t ldx, const void* norm_w, float eps,
                           const void* w, int64_t ldw, void* y, int64_t ldy,
                           int M, int N, int K, void* stream);

/* Greedy token: out[m] = first index of the maximum of x[m, 0:N] (fp16 rows of
 * stride ldx), as torch.argmax (a NaN counts as the maximum).  Replaces the
 * argmax of pipeline_runtime.py:160 on the device. */
int helm_argmax_f16(const void* x, int64_t ldx, int M, int N, int64_t* out, void* stream);

/* The same argmax spread over 64 workgroups per row, whose partial (value,
 * index) pairs go to a caller-owned workspace of helm_argmax_workspace_bytes(M)
 * bytes (4-byte aligned), merged by a second kernel on the same stream (the
 * single-workgroup form above is VALU-bound on one CU for a 151936-entry
 * vocabulary row).  Same result as helm_argmax_f16; M <= 65535.  Replaces the
 * argmax of pipeline_runtime.py:160 in the decode step. */
int64_t helm_argmax_workspace_bytes(int M);
int helm_argmax_f16_ws(const void* x, int64_t ldx, int M, int N, int64_t* out,
                       void* workspace, int64_t workspace_bytes, void* stream);

/* RMSNorm: y = fp16(w * fp16(x * rsqrt(mean(x^2) + eps))), x/y [M, K] fp16. */
int helm_rmsnorm(const void* x, const void* w, float eps, void* y,
                 int M, int K, void* stream);

/* out[i] = fp16(fp16(silu(gate[i])) * up[i]) over n fp16 elements, silu in fp32:
 * the SwiGLU of helm_int8_gemv_swiglu's epilogue for gate / up projections
 * computed apart (the MLP of transformers' Qwen3MLP, reached through the
 * patched decoder layer of kv_offload.py:225-273; batched decode). */
int helm_silu_mul(const void* gate, const void* up, void* out, int64_t n, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* HELM_MI355X_H */
