// paged_attention.hip — paged GQA decode attention, split-K over pages.
//
// Restates the mixed-residency path of perform_streaming_attention
// (helm/runtime/kv_cache.py:387-442): fp32 online softmax over pages in token
// order, m' = max(m, blockmax), alpha = exp(m - m') (0 when m = -inf),
// o = o*alpha + sum_t exp(s_t - m') v_t, l = l*alpha + sum_t exp(s_t - m'),
// out = o / max(l, 1e-12).  GQA: q head h reads kv head h / (Hq/Hkv) (the
// repeat_interleave mapping of kv_cache.py:356-363).
//
// gfx950 design: both contractions run on the matrix cores.  One 256-thread
// workgroup per (item, kv head, split); its four waves take 32-token steps of
// the split round robin.  Per step a wave computes
//   S[32 tok x 16 col] = K[32 x D] . Q^T[D x 16]      (2 x D/32 v_mfma_f32_16x16x32_f16)
//   O^T[D x 16]       += V^T[D x 32] . P^T[32 x 16]   (D/16 x 2 MFMAs, P = hi + lo fp16)
// where the 16 columns are the G = Hq/Hkv query heads of the kv head (zero
// padded), so every K/V byte is read once for the whole group.  The token order
// inside the score tiles is permuted so that each lane ends up holding the
// scores of exactly the 8 consecutive tokens whose V^T it feeds to the second
// MFMA: no data moves between lanes except two butterflies for the row max.
// V pages are stored token-contiguous per dim ([slot, Hkv, D, P]) so a lane's
// V operand (8 tokens of one dim) is one 16-byte load; K pages are [slot, Hkv,
// P, D] and a lane's K operand is 8 dims of one token.  Probabilities are split
// into fp16 hi + lo parts so the PV product keeps fp32-level accuracy.  The
// split's page-table slice is staged in LDS once, so address computation never
// waits on a global load inside the pipelined step loop.  The four waves' (max,
// sum, o) are merged through LDS and the split writes one normalised fp32
// partial + (max, sum); helm_paged_attn_reduce merges the splits.
#include "helm_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kStep = 32;             // tokens per wave step
constexpr int kMaxSplitPages = 4096;  // page-table entries of one split staged in LDS

// The kStep-token steps of a page table are dealt to the splits round robin:
// split s takes steps s, s + S, s + 2S, ... (S = num_splits) and wave w of the
// split its local steps w, w + 4, ...  A step covers kUpp<P> page-table entries
// (two pages at P = 16, one page or half of one above).
template <int P>
constexpr int kUpp = kStep >= P ? kStep / P : 1;
__host__ __device__ inline int table_steps(int max_pages, int P) {
  return (max_pages * P + kStep - 1) / kStep;
}
// Page-table entries one split stages in LDS: its share of the table's steps.
__host__ __device__ inline int split_pages(int max_pages, int num_splits, int P) {
  const int upp = kStep >= P ? kStep / P : 1;
  return (table_steps(max_pages, P) + num_splits - 1) / num_splits * upp;
}

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

struct AttnArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const uint16_t* k;
  int64_t k_ss, k_hs;          // K element (slot, h, t, d): slot*k_ss + h*k_hs + t*D + d
  const uint16_t* v;
  int64_t v_ss, v_hs, v_ds;    // V element (slot, h, t, d): slot*v_ss + h*v_hs + d*v_ds + t
  int64_t num_slots;           // page-table entries outside [0, num_slots) are skipped
  const int32_t* page_table;
  int64_t pt_stride;
  const int32_t* seq_lens;
  float* part_o;
  float* part_ml;
  int B, Hq, Hkv, max_pages, num_splits;
  int split_offset, total_splits;  // partial index of split s is split_offset + s of total_splits
  float qk_scale_log2;             // scale * log2(e)
  // fused decode step only (helm_decode_attn_fused)
  const uint16_t* qkv;             // [B, (Hq + 2 Hkv) * D] projection output (q | k | v)
  int64_t qkv_sb;
  const uint16_t* q_norm_w;
  const uint16_t* k_norm_w;
  float eps;
  const int32_t* positions;        // RoPE position of the new token
  const float* inv_freq;           // [D/2]
  const int32_t* new_slots;        // page slot / in-page offset of the new token
  const int32_t* new_offsets;
  // helm_decode_attn_fused_cs: the model's fp16 RoPE rows [B, D] (row stride
  // cs_sb) instead of positions / inv_freq; null in helm_decode_attn_fused
  const uint16_t* cos_rows;
  const uint16_t* sin_rows;
  int64_t cs_sb;
};


__device__ __forceinline__ h8_t ld_h8(const uint16_t* p) {
  return __builtin_bit_cast(h8_t, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p)));
}

template <int D>
struct StepBuf {
  h8_t k[2][D / 32];   // A operands of the two score tiles
  h8_t v[D / 16];      // A operands of the D/16 output tiles (V^T rows)
};

// fp16(w * fp16(x * rstd)), the fp16 rounding of Qwen3RMSNorm in fp16 models
__device__ __forceinline__ float norm_h(float x, float rstd, float w) {
  return h2f(f2h(w * h2f(f2h(x * rstd))));
}
// RoPE rotate_half output: fp16(fp16(x * cos) + fp16(rot * sin)) as fp16 torch ops round
__device__ __forceinline__ _Float16 rope_h(float x, float rot, float c, float s) {
  return (_Float16)(h2f(f2h(x * c)) + h2f(f2h(rot * s)));
}

// FUSED = the decode-step variant (helm_decode_attn_fused): q/k RMSNorm + RoPE
// from the raw projection, and the new token's K/V written to its page and
// folded in by the last split (not read back from the pool).
//
// Splits take the table's steps round robin (table_steps), so the live tokens of
// any length are shared to within one step by all splits, and by all XCDs
// (workgroup s of a kv head runs on XCD s mod 8 when S is a multiple of 8): a
// decode launch ends when its busiest XCD has streamed its share, and a block
// partition of the pages left whole splits, and so whole XCDs, idle or short
// whenever the live length was not a multiple of the block.  Addresses depend
// only on max_pages, so the page-table reads go out in parallel with the
// seq_len read; the live length sets loop counts and masks only.

// MODE 0: partials of a given q (helm_paged_decode_attn); 1: the fused decode step
// with the RoPE angle from positions / inv_freq and both q / k norms
// (helm_decode_attn_fused); 2: the same with the model's cos / sin rows and
// optional norms (helm_decode_attn_fused_cs).  Modes 1 and 2 are separate
// instances so that mode 1 keeps its own (smaller) prologue.
template <int D, int P, int GMAX, int MODE>
__global__ __launch_bounds__(kThreads, 2) void paged_attn_kernel(AttnArgs a) {
  constexpr bool FUSED = MODE != 0;
  constexpr bool CS = MODE == 2;
  constexpr int KT = D / 32;
  constexpr int DT = D / 16;
  constexpr int HALF = D / 2;
  static_assert(P % 16 == 0, "page size must be a multiple of 16");

  __shared__ int s_slot[kMaxSplitPages];
  __shared__ float s_m[kWaves][GMAX], s_l[kWaves][GMAX];
  __shared__ __attribute__((aligned(16))) float s_o[kWaves][GMAX][D];
  // fused-only state (small)
  // RoPE factors: one per dim from the cos / sin rows (mode 2), one per angle
  // (dims d and d + D/2 share it) from inv_freq (mode 1)
  constexpr int kCs = CS ? D : (FUSED ? HALF : 1);
  __shared__ float s_cos[kCs], s_sin[kCs];
  __shared__ __attribute__((aligned(16))) uint16_t s_qh[FUSED ? GMAX : 1][FUSED ? D : 1];
  __shared__ float s_kv[FUSED ? 2 : 1][FUSED ? D : 1];
  __shared__ float s_snew[GMAX];
  __shared__ int s_newok;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int col = lane & 15;   // MFMA row/column index held by this lane
  const int grp = lane >> 4;   // MFMA k-group (8 consecutive k) held by this lane
  const int split = blockIdx.x;   // grid.x == num_splits; every wave reaches the barriers
  const int hk = blockIdx.y;
  const int b = blockIdx.z;
  const int G = a.Hq / a.Hkv;
  const bool designated = FUSED && split == a.num_splits - 1;   // folds in the new token

  // fused step: wave w normalises and rotates the group's q heads w, w + 4, ...
  // with lane holding dims lane + 64 j (the layout of helm_qk_norm_rope_append),
  // so only the G real heads are computed, once per workgroup.  Every small load
  // of the prologue is issued first, and consumed before the first K/V loads go
  // out (a wait on a load issued after them would wait for them too).
  constexpr int J = D / 64;
  constexpr int GPW = (GMAX + kWaves - 1) / kWaves;
  const bool new_wave = designated && wave == kWaves - 1;   // computes the new token
  // raw fp16 bits, one per 32-bit register (packing two into one would wait for
  // the loads right away); converted after the page-table loads are issued so
  // that all of them share one round trip
  uint32_t qx_h[FUSED ? GPW : 1][J], qw_h[J], kx_h[J], kw_h[J], vh[J];
  float qx[FUSED ? GPW : 1][J], qw[J], kx[J], kw[J];
  int new_slot = -1, new_off = -1, pos = 0;
  float inv_f = 0.f;
  uint32_t cos_h = 0, sin_h = 0;
  // q / k norms are optional (both given, or neither: Qwen2 / Llama attention)
  const bool has_norm = FUSED && (!CS || a.q_norm_w != nullptr);   // a constant in mode 1
  auto cs_at = [](int d) { return CS ? d : d % HALF; };
  h8_t qb[KT];
  // Q^T as the B operand of the score MFMA: lane holds q[head col][kk*32 + grp*8, +8].
  // Columns >= G repeat head G-1 (zeros in the fused step); their scores and
  // outputs are never published.
  const int hq = hk * G + min(col, G - 1);
  if constexpr (FUSED) {
#pragma unroll
    for (int j = 0; j < J; ++j) qw_h[j] = has_norm ? a.q_norm_w[lane + 64 * j] : 0u;
#pragma unroll
    for (int t = 0; t < GPW; ++t) {
      const int g = min(wave + t * kWaves, G - 1);   // clamped; rows past G are not used
      const uint16_t* src = a.qkv + (int64_t)b * a.qkv_sb + (int64_t)(hk * G + g) * D;
#pragma unroll
      for (int j = 0; j < J; ++j) qx_h[t][j] = src[lane + 64 * j];
    }
    if (new_wave) {   // the new token's k and v rows of kv head hk
      const uint16_t* kr = a.qkv + (int64_t)b * a.qkv_sb + (int64_t)(a.Hq + hk) * D;
      const uint16_t* vr = kr + (int64_t)a.Hkv * D;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        kx_h[j] = kr[lane + 64 * j];
        kw_h[j] = has_norm ? a.k_norm_w[lane + 64 * j] : 0u;
        vh[j] = vr[lane + 64 * j];
      }
      new_slot = a.new_slots[b];
      new_off = a.new_offsets[b];
    }
    if constexpr (CS) {
      if (tid < D) {
        cos_h = a.cos_rows[(int64_t)b * a.cs_sb + tid];
        sin_h = a.sin_rows[(int64_t)b * a.cs_sb + tid];
      }
    } else {
      pos = a.positions[b];
      if (tid < HALF) inv_f = a.inv_freq[tid];
    }
  }

  const int seq = a.seq_lens[b];
  // this split's steps of the table (independent of seq_len, so the page-table
  // reads load in parallel with it): global step split + j * S for local step j
  constexpr int UPP = kUpp<P>;
  const int S = a.num_splits;
  const int max_steps = table_steps(a.max_pages, P);
  const int n_local = max_steps > split ? (max_steps - 1 - split) / S + 1 : 0;
  const int p_cnt = n_local * UPP;   // staged entries: UPP per local step
  const int p_last = max(p_cnt - 1, 0);
  const int32_t* ptab = a.page_table + (int64_t)b * a.pt_stride;
  // first token of local step j, and the staged entry of token offset `off` in it
  auto step_tok = [&](int j) { return (split + j * S) * kStep; };
  auto entry = [&](int j, int off) { return min(j * UPP + ((step_tok(j) % P) + off) / P, p_last); };
  // This lane's two page slots of the wave's first step (its score-tile token
  // and its V^T token run), read straight from the page table, so that the
  // first K/V loads go out as soon as the small loads land instead of after the
  // prologue's arithmetic and barrier.  No entry is read for a wave without a
  // staged step.
  int first_k = -1, first_v = -1;
  if (n_local > wave) {
    const int t0 = step_tok(wave);
    first_k = ptab[min((t0 + (col >> 2) * 8 + (col & 3)) / P, a.max_pages - 1)];
    first_v = ptab[min((t0 + grp * 8) / P, a.max_pages - 1)];
  }
  for (int i = tid; i < p_cnt; i += kThreads) {
    const int j = i / UPP;
    const int pg = step_tok(j) / P + (i - j * UPP);
    const int slot = pg < a.max_pages ? ptab[pg] : -1;
    s_slot[i] = (slot >= 0 && slot < a.num_slots) ? slot : -1;
  }
  if constexpr (!FUSED) {
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) qb[kk] = ld_h8(a.q + (int64_t)b * a.q_sb + (int64_t)hq * a.q_sh + kk * 32 + grp * 8);
  }

  // pool tokens [0, pool_tokens); in the fused step the new token (position
  // seq - 1) is not read from the pool but folded in directly
  const int pool_tokens = max(FUSED ? seq - 1 : seq, 0);
  const int live_steps = min((pool_tokens + kStep - 1) / kStep, max_steps);
  const int nsteps = live_steps > split ? (live_steps - 1 - split) / S + 1 : 0;
  const int my_steps = nsteps > wave ? (nsteps - 1 - wave) / kWaves + 1 : 0;

  const uint16_t* kbase = a.k + (int64_t)hk * a.k_hs;
  const uint16_t* vbase = a.v + (int64_t)hk * a.v_hs + (int64_t)col * a.v_ds;

  // Loads of the i-th step of this wave (step index wave + 4 i) from the pool
  // slots slot_k / slot_v (each in [0, num_slots)).  Addresses stay inside the
  // slot's page, so a step's loads need no per-lane guard (lanes past the last
  // token read in-range memory, masked in compute).
  auto load_slots = [&](StepBuf<D>& bf, int i, int slot_k, int slot_v) {
    const int tok0 = step_tok(wave + kWaves * i);
    // score-tile row `col` of tile t is token tok0 + (col/4)*8 + t*4 + col%4
    const int tk = tok0 + (col >> 2) * 8 + (col & 3);
    const uint16_t* kp = kbase + (int64_t)slot_k * a.k_ss + (int64_t)(tk % P) * D + grp * 8;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) bf.k[t][kk] = ld_h8(kp + t * 4 * D + kk * 32);
    // V^T rows: dim i*16 + col, tokens tok0 + grp*8 .. +8 (one page: 8 | P)
    const int tv = tok0 + grp * 8;
    const uint16_t* vp = vbase + (int64_t)slot_v * a.v_ss + (tv % P);
#pragma unroll
    for (int d = 0; d < DT; ++d) bf.v[d] = ld_h8(vp + (int64_t)(d * 16) * a.v_ds);
  };
  // later steps take their slots from the staged slice (unused entries -> slot 0)
  auto load = [&](StepBuf<D>& bf, int i) {
    const int j = wave + kWaves * i;
    const int slot_k = max(s_slot[entry(j, (col >> 2) * 8 + (col & 3))], 0);
    const int slot_v = max(s_slot[entry(j, grp * 8)], 0);
    load_slots(bf, i, slot_k, slot_v);
  };

  // The first step is issued unconditionally (a wave without steps reads slot 0
  // and never uses it), so every later wait on an earlier small load can count
  // these loads as outstanding instead of waiting for them.
  StepBuf<D> bufA, bufB;
  load_slots(bufA, 0, (first_k >= 0 && first_k < a.num_slots) ? first_k : 0,
             (first_v >= 0 && first_v < a.num_slots) ? first_v : 0);
  __builtin_amdgcn_sched_barrier(0);   // keep them ahead of the prologue

  float q_rstd[FUSED ? GPW : 1], k_rstd = 0.f;
  if constexpr (FUSED) {
    if constexpr (CS) {   // the model's own RoPE rows
      if (tid < D) {
        s_cos[tid] = h2f((uint16_t)cos_h);
        s_sin[tid] = h2f((uint16_t)sin_h);
      }
    } else if (tid < HALF) {   // RoPE table of this position, rounded to fp16 as the torch ops do
      const float ang = inv_f * (float)pos;
      s_cos[tid] = h2f(f2h(cosf(ang)));
      s_sin[tid] = h2f(f2h(sinf(ang)));
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
      qw[j] = h2f((uint16_t)qw_h[j]);
      kx[j] = h2f((uint16_t)kx_h[j]);
      kw[j] = h2f((uint16_t)kw_h[j]);
    }
#pragma unroll
    for (int t = 0; t < GPW; ++t)
#pragma unroll
      for (int j = 0; j < J; ++j) qx[t][j] = h2f((uint16_t)qx_h[t][j]);
    if (has_norm) {
#pragma unroll
      for (int t = 0; t < GPW; ++t) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < J; ++j) ss = fmaf(qx[t][j], qx[t][j], ss);
        q_rstd[t] = rsqrtf(wave_sum(ss) / (float)D + a.eps);
      }
      if (new_wave) {
        float kss = 0.f;
#pragma unroll
        for (int j = 0; j < J; ++j) kss = fmaf(kx[j], kx[j], kss);
        k_rstd = rsqrtf(wave_sum(kss) / (float)D + a.eps);
      }
    }
  }
  lds_barrier();   // s_slot (and the RoPE table); the first K/V loads stay in flight

  if constexpr (FUSED) {
    // q RMSNorm + RoPE per real head (the operations and order of
    // helm_qk_norm_rope_append), fp16 into LDS, then each lane reads its B operand
#pragma unroll
    for (int t = 0; t < GPW; ++t) {
      const int g = wave + t * kWaves;
      if (g < G) {   // uniform per wave
        float xn[J];
#pragma unroll
        for (int j = 0; j < J; ++j) xn[j] = has_norm ? norm_h(qx[t][j], q_rstd[t], qw[j]) : qx[t][j];
#pragma unroll
        for (int j = 0; j < J; ++j) {
          const int d = lane + 64 * j;
          float partner;
          if constexpr (J == 2) {
            partner = xn[1 - j];
          } else {
            partner = __shfl_xor(xn[j], HALF, 64);
          }
          const float rot = d < HALF ? -partner : partner;
          s_qh[g][d] = __builtin_bit_cast(uint16_t, rope_h(xn[j], rot, s_cos[cs_at(d)], s_sin[cs_at(d)]));
        }
      }
    }
    if (new_wave) {
      // the new token: k RMSNorm + RoPE of kv head hk (same operations), v as is;
      // both written to the token's page slot and kept for the merge
      if (has_norm) {
#pragma unroll
        for (int j = 0; j < J; ++j) kx[j] = norm_h(kx[j], k_rstd, kw[j]);
      }
      const int slot = new_slot;
      const int off = new_off;
      const bool ok = slot >= 0 && slot < a.num_slots && off >= 0 && off < P;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int d = lane + 64 * j;
        float partner;
        if constexpr (J == 2) {
          partner = kx[1 - j];
        } else {
          partner = __shfl_xor(kx[j], HALF, 64);
        }
        const float rot = d < HALF ? -partner : partner;
        const _Float16 kh = rope_h(kx[j], rot, s_cos[cs_at(d)], s_sin[cs_at(d)]);
        s_kv[0][d] = (float)kh;
        s_kv[1][d] = h2f((uint16_t)vh[j]);
        if (ok) {
          const_cast<uint16_t*>(a.k)[(int64_t)slot * a.k_ss + (int64_t)hk * a.k_hs + (int64_t)off * D + d] =
              __builtin_bit_cast(uint16_t, kh);
          const_cast<uint16_t*>(a.v)[(int64_t)slot * a.v_ss + (int64_t)hk * a.v_hs + (int64_t)d * a.v_ds + off] = (uint16_t)vh[j];
        }
      }
      if (lane == 0) s_newok = (ok && seq >= 1) ? 1 : 0;
    }
    lds_barrier();
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) {
      const h8_t v = *reinterpret_cast<const h8_t*>(&s_qh[min(col, G - 1)][kk * 32 + grp * 8]);
      qb[kk] = col < G ? v : h8_t{};
    }
  }

  float m_run = -INFINITY, l_run = 0.f;   // per query head `col` (same in every grp)
  f4_t o[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) o[d] = f4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const StepBuf<D>& bf, int i) {
    const int j = wave + kWaves * i;
    const int tv = step_tok(j) + grp * 8;
    const bool page_ok = s_slot[entry(j, grp * 8)] >= 0;
    // this lane's 8 tokens tv .. tv+7: the first nvalid are real
    const int nvalid = page_ok ? max(0, min(8, pool_tokens - tv)) : 0;

    f4_t sc0 = {0.f, 0.f, 0.f, 0.f}, sc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) {
      sc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf.k[0][kk], qb[kk], sc0, 0, 0, 0);
      sc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf.k[1][kk], qb[kk], sc1, 0, 0, 0);
    }
    // lane holds S[token tv + j][head col], j = t*4 + r
    float s[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s[r] = r < nvalid ? sc0[r] * a.qk_scale_log2 : -INFINITY;
      s[4 + r] = 4 + r < nvalid ? sc1[r] * a.qk_scale_log2 : -INFINITY;
    }
    float mx = s[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) mx = fmaxf(mx, s[j]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    // reference point of the exponentials; 0 while nothing has been seen so that
    // exp2(-inf - ref) = 0 never becomes exp2(NaN)
    const float ref = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = exp2f(m_run - ref);
    h8_t phi, plo;
    float lsum = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float p = exp2f(s[j] - ref);   // masked tokens: exp2(-inf) = 0
      const _Float16 h = (_Float16)p;
      phi[j] = h;
      plo[j] = (_Float16)(p - (float)h);
      lsum += p;
    }
    l_run = l_run * alpha + lsum;
    m_run = m_new;
    // Unwritten page slots hold arbitrary bits (possibly NaN/Inf); a masked token
    // has p = 0 and 0 * NaN would poison the sum, so its V entries are zeroed.
    uint32_t vmask[4];
#pragma unroll
    for (int q2 = 0; q2 < 4; ++q2)
      vmask[q2] = (2 * q2 < nvalid ? 0x0000ffffu : 0u) | (2 * q2 + 1 < nvalid ? 0xffff0000u : 0u);
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      u32x4_t vw = __builtin_bit_cast(u32x4_t, bf.v[d]);
      vw.x &= vmask[0];
      vw.y &= vmask[1];
      vw.z &= vmask[2];
      vw.w &= vmask[3];
      const h8_t vv = __builtin_bit_cast(h8_t, vw);
      o[d] *= alpha;
      o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vv, phi, o[d], 0, 0, 0);
      o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vv, plo, o[d], 0, 0, 0);
    }
  };

  // ---- pipelined walk over this wave's steps, ping-pong buffers ----
  int i = 0;
  for (; i + 2 < my_steps; i += 2) {
    load(bufB, i + 1);
    compute(bufA, i);
    load(bufA, i + 2);
    compute(bufB, i + 1);
  }
  if (i + 1 < my_steps) {
    load(bufB, i + 1);
    compute(bufA, i);
    compute(bufB, i + 1);
  } else if (i < my_steps) {
    compute(bufA, i);
  }

  // ---- merge the k-groups of the wave, publish to LDS ----
  float l = l_run;
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (col < G) {
    // o[d][r] = O^T[dim d*16 + grp*4 + r][head col]
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      *reinterpret_cast<float4*>(&s_o[wave][col][d * 16 + grp * 4]) =
          make_float4(o[d][0], o[d][1], o[d][2], o[d][3]);
    }
    if (grp == 0) {
      s_m[wave][col] = m_run;
      s_l[wave][col] = l;
    }
  }
  __syncthreads();

  if (designated) {
    // score of the new token for each query head of the group (log2 units)
    for (int g = wave; g < G; g += kWaves) {
      float t = 0.f;
      for (int d = lane; d < D; d += 64) t = fmaf(h2f(s_qh[g][d]), s_kv[0][d], t);
      t = wave_sum(t);
      if (lane == 0) s_snew[g] = s_newok ? t * a.qk_scale_log2 : -INFINITY;
    }
    __syncthreads();
  }

  // merge the four waves (and the new token) and write this split's partial:
  // one thread per 4 dims of a head (one pass for G * D <= 1024), the waves'
  // weights computed once per thread, 16-byte LDS reads and stores
  for (int idx = tid; idx < G * (D / 4); idx += kThreads) {
    const int g = idx / (D / 4);
    const int d = (idx - g * (D / 4)) * 4;
    float mx = s_m[0][g];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) mx = fmaxf(mx, s_m[w][g]);
    if (designated) mx = fmaxf(mx, s_snew[g]);
    const float ref = (mx == -INFINITY) ? 0.f : mx;
    float num[4] = {0.f, 0.f, 0.f, 0.f}, den = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float sc = exp2f(s_m[w][g] - ref);
      const float4 ow = *reinterpret_cast<const float4*>(&s_o[w][g][d]);
      num[0] = fmaf(sc, ow.x, num[0]);
      num[1] = fmaf(sc, ow.y, num[1]);
      num[2] = fmaf(sc, ow.z, num[2]);
      num[3] = fmaf(sc, ow.w, num[3]);
      den = fmaf(sc, s_l[w][g], den);
    }
    if (designated) {
      const float sc = exp2f(s_snew[g] - ref);
#pragma unroll
      for (int e = 0; e < 4; ++e) num[e] = fmaf(sc, s_kv[1][d + e], num[e]);
      den += sc;
    }
    const int64_t pidx = ((int64_t)b * a.Hq + hk * G + g) * a.total_splits + a.split_offset + split;
    float4 out = make_float4(0.f, 0.f, 0.f, 0.f);
    if (den > 0.f) out = make_float4(num[0] / den, num[1] / den, num[2] / den, num[3] / den);
    *reinterpret_cast<float4*>(&a.part_o[pidx * D + d]) = out;
    if (d == 0) {
      a.part_ml[pidx * 2] = mx;
      a.part_ml[pidx * 2 + 1] = den;
    }
  }
}

// out[b,h,:] = sum_s w_s o_s / sum_s w_s with w_s = exp2(m_s - M) l_s: one
// 256-thread block per (item, q head); the splits' weights go through LDS in
// chunks and the weighted sum runs over (dim, split-group) threads.
constexpr int kReduceChunk = 2048;

template <int D>
__global__ __launch_bounds__(256) void attn_reduce_kernel(const float* __restrict__ part_o,
                                                          const float* __restrict__ part_ml,
                                                          uint16_t* __restrict__ out, int S) {
  constexpr int GR = 256 / D;   // split groups
  __shared__ float w_s[kReduceChunk];
  __shared__ float red[4];
  __shared__ float acc_s[GR][D];
  const int bh = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const float* ml = part_ml + (int64_t)bh * S * 2;
  const float* po = part_o + (int64_t)bh * S * D;

  float mx = -INFINITY;
  for (int s = tid; s < S; s += 256) {
    if (ml[2 * s + 1] > 0.f) mx = fmaxf(mx, ml[2 * s]);
  }
  mx = wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();

  const int g = tid / D, d = tid - (tid / D) * D;
  float acc = 0.f, den = 0.f;
  for (int c0 = 0; c0 < S; c0 += kReduceChunk) {
    const int cn = min(kReduceChunk, S - c0);
    for (int s = tid; s < cn; s += 256) {
      const float l = ml[2 * (c0 + s) + 1];
      const float w = (l > 0.f) ? exp2f(ml[2 * (c0 + s)] - mx) * l : 0.f;
      w_s[s] = w;
      den += w;
    }
    __syncthreads();
    const float* pc = po + (int64_t)c0 * D + d;
    int s = g;
    for (; s + 3 * GR < cn; s += 4 * GR) {
      const float o0 = pc[(int64_t)s * D], o1 = pc[(int64_t)(s + GR) * D];
      const float o2 = pc[(int64_t)(s + 2 * GR) * D], o3 = pc[(int64_t)(s + 3 * GR) * D];
      acc = fmaf(w_s[s], o0, acc);
      acc = fmaf(w_s[s + GR], o1, acc);
      acc = fmaf(w_s[s + 2 * GR], o2, acc);
      acc = fmaf(w_s[s + 3 * GR], o3, acc);
    }
    for (; s < cn; s += GR) acc = fmaf(w_s[s], pc[(int64_t)s * D], acc);
    __syncthreads();
  }
  den = wave_sum(den);
  if (lane == 0) red[wave] = den;
  acc_s[g][d] = acc;
  __syncthreads();
  if (tid < D) {
    const float tot = red[0] + red[1] + red[2] + red[3];
    float a = 0.f;
#pragma unroll
    for (int k = 0; k < GR; ++k) a += acc_s[k][tid];
    out[(int64_t)bh * D + tid] = f2h(tot > 0.f ? a / fmaxf(tot, 1e-12f) : 0.f);
  }
}

// Same merge for up to PER * (NT / D) splits with one round trip to memory: every
// thread loads the partials of its splits (thread (g, d) takes splits g, g + GR,
// ... of dim d) and their (max, sum) pairs at once; the block maximum and the
// group sums go through LDS.  The block widens with the split count (256 / 512 /
// 1024 threads, four splits per thread): at 32 splits 2.92 -> 2.58 us against
// 256 threads with sixteen each, whose 48 loads per thread took longer to issue.
template <int D, int PER, int NT>
__global__ __launch_bounds__(NT) void attn_reduce_small_kernel(const float* __restrict__ part_o,
                                                                const float* __restrict__ part_ml,
                                                                uint16_t* __restrict__ out, int S) {
  constexpr int GR = NT / D;
  __shared__ float mx_s[GR], den_s[GR];
  __shared__ float acc_s[GR][D];
  const int bh = blockIdx.x;
  const int tid = threadIdx.x;
  const int g = tid / D, d = tid - (tid / D) * D;
  const float* ml = part_ml + (int64_t)bh * S * 2;
  const float* po = part_o + (int64_t)bh * S * D;
  float o[PER], m[PER], l[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int s = min(g + j * GR, S - 1);   // clamped in range; entries past S are dropped below
    o[j] = po[(int64_t)s * D + d];
    const float2 mlj = *reinterpret_cast<const float2*>(ml + 2 * s);   // (max, sum), 8-byte aligned
    m[j] = mlj.x;
    l[j] = mlj.y;
  }
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < PER; ++j)
    if (g + j * GR < S && l[j] > 0.f) mx = fmaxf(mx, m[j]);
  if (d == 0) mx_s[g] = mx;
  __syncthreads();
#pragma unroll
  for (int k = 0; k < GR; ++k) mx = fmaxf(mx, mx_s[k]);
  float acc = 0.f, den = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const bool ok = g + j * GR < S && l[j] > 0.f;
    const float w = ok ? exp2f(m[j] - mx) * l[j] : 0.f;
    acc = fmaf(w, o[j], acc);
    den += w;
  }
  acc_s[g][d] = acc;
  if (d == 0) den_s[g] = den;
  __syncthreads();
  if (tid < D) {
    float a = 0.f, tot = 0.f;
#pragma unroll
    for (int k = 0; k < GR; ++k) {
      a += acc_s[k][tid];
      tot += den_s[k];
    }
    out[(int64_t)bh * D + tid] = f2h(tot > 0.f ? a / fmaxf(tot, 1e-12f) : 0.f);
  }
}

template <int D>
void launch_reduce(const float* part_o, const float* part_ml, uint16_t* out, int BH, int S,
                   hipStream_t s) {
  constexpr int GR = 256 / D;
  const int per = (S + GR - 1) / GR;
  if (per <= 4)
    hipLaunchKernelGGL((attn_reduce_small_kernel<D, 4, 256>), dim3(BH), dim3(256), 0, s, part_o, part_ml, out, S);
  else if (per <= 8)
    hipLaunchKernelGGL((attn_reduce_small_kernel<D, 4, 512>), dim3(BH), dim3(512), 0, s, part_o, part_ml, out, S);
  else if (per <= 16)
    hipLaunchKernelGGL((attn_reduce_small_kernel<D, 4, 1024>), dim3(BH), dim3(1024), 0, s, part_o, part_ml, out, S);
  else   // more splits: the register-resident form loses to the chunked loop (measured)
    hipLaunchKernelGGL((attn_reduce_kernel<D>), dim3(BH), dim3(256), 0, s, part_o, part_ml, out, S);
}

template <int D, int P, int MODE>
void launch_attn_dp(const AttnArgs& a, int G, hipStream_t s) {
  dim3 grid(a.num_splits, a.Hkv, a.B);
  if (G <= 4) hipLaunchKernelGGL((paged_attn_kernel<D, P, 4, MODE>), grid, dim3(kThreads), 0, s, a);
  else if (G <= 8) hipLaunchKernelGGL((paged_attn_kernel<D, P, 8, MODE>), grid, dim3(kThreads), 0, s, a);
  else hipLaunchKernelGGL((paged_attn_kernel<D, P, 16, MODE>), grid, dim3(kThreads), 0, s, a);
}

template <int MODE>
void launch_attn(const AttnArgs& a, int D, int P, int G, hipStream_t s) {
  if (D == 64) {
    if (P == 16) launch_attn_dp<64, 16, MODE>(a, G, s);
    else if (P == 32) launch_attn_dp<64, 32, MODE>(a, G, s);
    else launch_attn_dp<64, 64, MODE>(a, G, s);
  } else {
    if (P == 16) launch_attn_dp<128, 16, MODE>(a, G, s);
    else if (P == 32) launch_attn_dp<128, 32, MODE>(a, G, s);
    else launch_attn_dp<128, 64, MODE>(a, G, s);
  }
}

// Checks shared by both entry points; fills the pool / table / split fields.
int check_attn(const helm_kv_pool* pool, const int32_t* page_table, int64_t pt_stride,
               const int32_t* seq_lens, float* part_o, float* part_ml, int B, int Hq, int Hkv,
               int D, int P, int max_pages, int num_splits, const char* fn, AttnArgs& a) {
  const std::string f(fn);
  HELM_CHECK_ARG(pool && page_table && seq_lens && part_o && part_ml, f + ": null pointer");
  HELM_CHECK_ARG(pool->k && pool->v, f + ": null pool pointer");
  HELM_CHECK_ARG(B >= 1 && Hq >= 1 && Hkv >= 1 && max_pages >= 1 && num_splits >= 1,
                 f + ": sizes must be positive");
  HELM_CHECK_ARG(Hq % Hkv == 0, f + ": Hq must be a multiple of Hkv");
  HELM_CHECK_SUPPORTED(Hq / Hkv <= 16, f + ": at most 16 query heads per kv head");
  HELM_CHECK_SUPPORTED(D == 64 || D == 128, f + ": head_dim must be 64 or 128");
  HELM_CHECK_SUPPORTED(P == 16 || P == 32 || P == 64, f + ": page size must be 16, 32 or 64");
  HELM_CHECK_ARG(pt_stride >= max_pages, f + ": page-table stride < max_pages");
  HELM_CHECK_ARG(pool->num_slots >= 1, f + ": num_slots must be positive");
  HELM_CHECK_SUPPORTED(split_pages(max_pages, num_splits, P) <= kMaxSplitPages,
                       f + ": more than " + std::to_string(kMaxSplitPages) +
                           " pages per split (raise num_splits)");
  HELM_CHECK_ARG(pool->k_head_stride >= (int64_t)P * D && pool->v_dim_stride >= P &&
                     pool->v_head_stride >= (int64_t)P * D,
                 f + ": pool strides too small for the page");
  HELM_CHECK_SUPPORTED(pool->k_slot_stride % 8 == 0 && pool->k_head_stride % 8 == 0 &&
                           pool->v_slot_stride % 8 == 0 && pool->v_head_stride % 8 == 0 &&
                           pool->v_dim_stride % 8 == 0,
                       f + ": strides must be multiples of 8 elements");
  HELM_CHECK_SUPPORTED(helm::aligned16(pool->k) && helm::aligned16(pool->v) && helm::aligned16(part_o),
                       f + ": pools and part_o must be 16-byte aligned");
  a.k = static_cast<const uint16_t*>(pool->k);
  a.k_ss = pool->k_slot_stride; a.k_hs = pool->k_head_stride;
  a.v = static_cast<const uint16_t*>(pool->v);
  a.v_ss = pool->v_slot_stride; a.v_hs = pool->v_head_stride; a.v_ds = pool->v_dim_stride;
  a.num_slots = pool->num_slots;
  a.page_table = page_table; a.pt_stride = pt_stride; a.seq_lens = seq_lens;
  a.part_o = part_o; a.part_ml = part_ml;
  a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.max_pages = max_pages; a.num_splits = num_splits;
  return HELM_OK;
}

}  // namespace

extern "C" int64_t helm_paged_attn_workspace_floats(int B, int Hq, int D, int num_splits) {
  if (B < 1 || Hq < 1 || D < 1 || num_splits < 1) return 0;
  return (int64_t)B * Hq * num_splits * (D + 2);
}

extern "C" int helm_paged_attn_max_split_pages(void) { return kMaxSplitPages; }

extern "C" int helm_paged_decode_attn(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                      const helm_kv_pool* pool, const int32_t* page_table,
                                      int64_t pt_stride, const int32_t* seq_lens, float* part_o,
                                      float* part_ml, int split_offset, int total_splits, int B,
                                      int Hq, int Hkv, int D, int P, int max_pages, int num_splits,
                                      float scale, void* stream) {
  AttnArgs a{};
  int rc = check_attn(pool, page_table, pt_stride, seq_lens, part_o, part_ml, B, Hq, Hkv, D, P,
                      max_pages, num_splits, "helm_paged_decode_attn", a);
  if (rc != HELM_OK) return rc;
  HELM_CHECK_ARG(q, "helm_paged_decode_attn: null pointer");
  HELM_CHECK_ARG(split_offset >= 0 && split_offset + num_splits <= total_splits,
                 "helm_paged_decode_attn: splits [split_offset, split_offset+num_splits) exceed total_splits");
  HELM_CHECK_SUPPORTED(q_stride_h % 8 == 0 && q_stride_b % 8 == 0 && helm::aligned16(q),
                       "helm_paged_decode_attn: q strides must be multiples of 8 and q 16-byte aligned");
  a.q = static_cast<const uint16_t*>(q); a.q_sb = q_stride_b; a.q_sh = q_stride_h;
  a.split_offset = split_offset; a.total_splits = total_splits;
  a.qk_scale_log2 = scale * kLog2e;
  launch_attn<0>(a, D, P, Hq / Hkv, static_cast<hipStream_t>(stream));
  HELM_CHECK_LAUNCH("helm_paged_decode_attn launch");
  return HELM_OK;
}

extern "C" int helm_decode_attn_fused(const void* qkv, int64_t qkv_stride_b, const void* q_norm_w,
                                      const void* k_norm_w, float eps, const int32_t* positions,
                                      const float* inv_freq, const int32_t* slots,
                                      const int32_t* offsets, const helm_kv_pool* pool,
                                      const int32_t* page_table, int64_t pt_stride,
                                      const int32_t* seq_lens, float* part_o, float* part_ml,
                                      int B, int Hq, int Hkv, int D, int P, int max_pages,
                                      int num_splits, float scale, void* stream) {
  AttnArgs a{};
  int rc = check_attn(pool, page_table, pt_stride, seq_lens, part_o, part_ml, B, Hq, Hkv, D, P,
                      max_pages, num_splits, "helm_decode_attn_fused", a);
  if (rc != HELM_OK) return rc;
  HELM_CHECK_ARG(qkv && q_norm_w && k_norm_w && positions && inv_freq && slots && offsets,
                 "helm_decode_attn_fused: null pointer");
  HELM_CHECK_SUPPORTED(qkv_stride_b % 8 == 0 && helm::aligned16(qkv),
                       "helm_decode_attn_fused: qkv rows must be 16-byte aligned");
  HELM_CHECK_ARG(qkv_stride_b >= (int64_t)(Hq + 2 * Hkv) * D, "helm_decode_attn_fused: qkv row stride too small");
  a.qkv = static_cast<const uint16_t*>(qkv); a.qkv_sb = qkv_stride_b;
  a.q_norm_w = static_cast<const uint16_t*>(q_norm_w);
  a.k_norm_w = static_cast<const uint16_t*>(k_norm_w);
  a.eps = eps; a.positions = positions; a.inv_freq = inv_freq;
  a.new_slots = slots; a.new_offsets = offsets;
  a.split_offset = 0; a.total_splits = num_splits;
  a.qk_scale_log2 = scale * kLog2e;
  launch_attn<1>(a, D, P, Hq / Hkv, static_cast<hipStream_t>(stream));
  HELM_CHECK_LAUNCH("helm_decode_attn_fused launch");
  return HELM_OK;
}

extern "C" int helm_decode_attn_fused_cs(const void* qkv, int64_t qkv_stride_b, const void* q_norm_w,
                                         const void* k_norm_w, float eps, const void* cos_rows,
                                         const void* sin_rows, int64_t cs_stride_b,
                                         const int32_t* slots, const int32_t* offsets,
                                         const helm_kv_pool* pool, const int32_t* page_table,
                                         int64_t pt_stride, const int32_t* seq_lens, float* part_o,
                                         float* part_ml, int B, int Hq, int Hkv, int D, int P,
                                         int max_pages, int num_splits, float scale, void* stream) {
  AttnArgs a{};
  int rc = check_attn(pool, page_table, pt_stride, seq_lens, part_o, part_ml, B, Hq, Hkv, D, P,
                      max_pages, num_splits, "helm_decode_attn_fused_cs", a);
  if (rc != HELM_OK) return rc;
  HELM_CHECK_ARG(qkv && cos_rows && sin_rows && slots && offsets,
                 "helm_decode_attn_fused_cs: null pointer");
  HELM_CHECK_ARG((q_norm_w == nullptr) == (k_norm_w == nullptr),
                 "helm_decode_attn_fused_cs: give both q / k norm weights or neither");
  HELM_CHECK_SUPPORTED(qkv_stride_b % 8 == 0 && helm::aligned16(qkv),
                       "helm_decode_attn_fused_cs: qkv rows must be 16-byte aligned");
  HELM_CHECK_ARG(qkv_stride_b >= (int64_t)(Hq + 2 * Hkv) * D,
                 "helm_decode_attn_fused_cs: qkv row stride too small");
  HELM_CHECK_ARG(cs_stride_b >= 0, "helm_decode_attn_fused_cs: negative cos / sin row stride");
  a.qkv = static_cast<const uint16_t*>(qkv); a.qkv_sb = qkv_stride_b;
  a.q_norm_w = static_cast<const uint16_t*>(q_norm_w);
  a.k_norm_w = static_cast<const uint16_t*>(k_norm_w);
  a.eps = eps;
  a.cos_rows = static_cast<const uint16_t*>(cos_rows);
  a.sin_rows = static_cast<const uint16_t*>(sin_rows);
  a.cs_sb = cs_stride_b;
  a.new_slots = slots; a.new_offsets = offsets;
  a.split_offset = 0; a.total_splits = num_splits;
  a.qk_scale_log2 = scale * kLog2e;
  launch_attn<2>(a, D, P, Hq / Hkv, static_cast<hipStream_t>(stream));
  HELM_CHECK_LAUNCH("helm_decode_attn_fused_cs launch");
  return HELM_OK;
}

extern "C" int helm_paged_attn_reduce(const float* part_o, const float* part_ml, void* out, int B,
                                      int Hq, int D, int num_splits, void* stream) {
  HELM_CHECK_ARG(part_o && part_ml && out, "helm_paged_attn_reduce: null pointer");
  HELM_CHECK_ARG(B >= 1 && Hq >= 1 && num_splits >= 1, "helm_paged_attn_reduce: sizes must be positive");
  HELM_CHECK_SUPPORTED(D == 64 || D == 128, "helm_paged_attn_reduce: head_dim must be 64 or 128");
  HELM_CHECK_SUPPORTED(reinterpret_cast<uintptr_t>(part_ml) % 8 == 0,
                       "helm_paged_attn_reduce: part_ml must be 8-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (D == 64)
    launch_reduce<64>(part_o, part_ml, static_cast<uint16_t*>(out), B * Hq, num_splits, s);
  else
    launch_reduce<128>(part_o, part_ml, static_cast<uint16_t*>(out), B * Hq, num_splits, s);
  HELM_CHECK_LAUNCH("helm_paged_attn_reduce launch");
  return HELM_OK;
}

// ---------------------------------------------------------------------------
// Allocation-free decode attention (helm_paged_decode_attn_noalloc)
// ---------------------------------------------------------------------------
// The split-K partials of helm_paged_decode_attn + helm_paged_attn_reduce live
// in this file-scope device array instead of a caller-supplied workspace, so the
// call needs no device allocation at all.  Each GPU the library runs on holds
// its own copy (kNoAllocScratchFloats * 4 bytes) until the process ends.  Host
// code never uses the array's name as an address: its per-device address comes
// from hipGetSymbolAddress, looked up once per device on the first call there.
// Every split writes its whole partial (empty splits write max = -inf, sum = 0),
// so nothing in the array has to start at zero; calls that overlap on one GPU
// (different streams) share the array and race.
#include <mutex>

namespace {

constexpr int64_t kNoAllocScratchFloats = int64_t(4) << 20;   // 16 MiB
constexpr int kNoAllocMaxDevices = 64;

}  // namespace

static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

namespace {

std::mutex g_scratch_mu;
float* g_scratch_ptr[kNoAllocMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on first use).
int scratch_ptr(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return helm::hip_fail(e, "helm_paged_decode_attn_noalloc: hipGetDevice");
  if (dev < 0 || dev >= kNoAllocMaxDevices)
    return helm::fail(HELM_ERR_UNSUPPORTED, "helm_paged_decode_attn_noalloc: device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess)
      return helm::hip_fail(e, "helm_paged_decode_attn_noalloc: hipGetSymbolAddress(scratch)");
    if (p == nullptr)
      return helm::fail(HELM_ERR_HIP, "helm_paged_decode_attn_noalloc: null scratch address");
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return HELM_OK;
}

}  // namespace

extern "C" int64_t helm_paged_attn_noalloc_max_floats(void) { return kNoAllocScratchFloats; }

extern "C" int helm_paged_decode_attn_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                              const helm_kv_pool* pool, const int32_t* page_table,
                                              int64_t pt_stride, const int32_t* seq_lens, void* out,
                                              int B, int Hq, int Hkv, int D, int P, int max_pages,
                                              int num_splits, float scale, void* stream) {
  HELM_CHECK_ARG(q && out, "helm_paged_decode_attn_noalloc: null pointer");
  HELM_CHECK_ARG(B >= 1 && Hq >= 1 && num_splits >= 1 && D >= 1,
                 "helm_paged_decode_attn_noalloc: sizes must be positive");
  const int64_t n_o = (int64_t)B * Hq * num_splits * D;
  const int64_t need = n_o + (int64_t)B * Hq * num_splits * 2;
  HELM_CHECK_SUPPORTED(need <= kNoAllocScratchFloats,
                       "helm_paged_decode_attn_noalloc: B * Hq * num_splits * (D + 2) = " +
                           std::to_string(need) + " floats exceeds the scratch buffer (" +
                           std::to_string(kNoAllocScratchFloats) + " floats)");
  float* ws = nullptr;
  int rc = scratch_ptr(&ws);
  if (rc != HELM_OK) return rc;
  // part_o first, then part_ml: n_o is a multiple of D (even), so part_ml stays
  // 8-byte aligned; `scratch` itself is 256-byte aligned.
  float* part_o = ws;
  float* part_ml = ws + n_o;
  AttnArgs a{};
  rc = check_attn(pool, page_table, pt_stride, seq_lens, part_o, part_ml, B, Hq, Hkv, D, P,
                  max_pages, num_splits, "helm_paged_decode_attn_noalloc", a);
  if (rc != HELM_OK) return rc;
  HELM_CHECK_SUPPORTED(q_stride_h % 8 == 0 && q_stride_b % 8 == 0 && helm::aligned16(q),
                       "helm_paged_decode_attn_noalloc: q strides must be multiples of 8 and q 16-byte aligned");
  a.q = static_cast<const uint16_t*>(q); a.q_sb = q_stride_b; a.q_sh = q_stride_h;
  a.split_offset = 0; a.total_splits = num_splits;
  a.qk_scale_log2 = scale * kLog2e;
  hipStream_t s = static_cast<hipStream_t>(stream);
  launch_attn<0>(a, D, P, Hq / Hkv, s);
  HELM_CHECK_LAUNCH("helm_paged_decode_attn_noalloc launch");
  if (D == 64)
    launch_reduce<64>(part_o, part_ml, static_cast<uint16_t*>(out), B * Hq, num_splits, s);
  else
    launch_reduce<128>(part_o, part_ml, static_cast<uint16_t*>(out), B * Hq, num_splits, s);
  HELM_CHECK_LAUNCH("helm_paged_decode_attn_noalloc reduce launch");
  return HELM_OK;
}
