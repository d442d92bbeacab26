// paged_attention.hip — paged GQA decode attention, split-K over pages.
//
// Restates the mixed-residency path of perform_streaming_attention
// (helm/runtime/kv_cache.py:387-442): fp32 online softmax over pages in token
// order, m' = max(m, blockmax), alpha = exp(m - m') (0 when m = -inf),
// o = o*alpha + sum_t exp(s_t - m') v_t, l = l*alpha + sum_t exp(s_t - m'),
// out = o / max(l, 1e-12).  GQA: q head h reads kv head h / (Hq/Hkv) (the
// repeat_interleave mapping of kv_cache.py:356-363).
//
// gfx950 layout: one 256-thread workgroup per (item, kv head, split).  Its four
// waves take the split's 16-token blocks round robin, so the workgroup streams
// four adjacent blocks at a time.  A token row of D fp16 is read by D/8 lanes
// with one 16-byte load each; a wave covers 64/(D/8) tokens per load
// instruction, coalesced.  Each wave keeps the G = Hq/Hkv query heads of its kv
// head in registers, so every K/V byte is read from HBM exactly once for the
// whole group.  Scores are fp32 FMAs over the lane's 8 dims plus a butterfly
// across the D/8 lanes of the row; the exponentials run in the log2 domain (q
// pre-multiplied by scale*log2(e)).  The next block is loaded while the current
// one is consumed.  The four waves' (max, sum, o) are merged through LDS and the
// split writes one normalised fp32 partial + (max, sum); a second kernel merges
// the splits with a block-parallel reduction.
#include "helm_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;

struct AttnArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const uint16_t* k_pool;
  const uint16_t* v_pool;
  int64_t slot_stride, head_stride;
  const int32_t* page_table;
  int64_t pt_stride;
  const int32_t* seq_lens;
  int64_t num_slots;  // pool size in slots; page-table entries outside [0, num_slots) are skipped
  float* part_o;
  float* part_ml;
  int B, Hq, Hkv, max_pages, num_splits;
  int split_offset, total_splits;  // partial index of split s is split_offset + s of total_splits
  float qk_scale_log2;  // scale * log2(e)
};

template <int D, int P, int GMAX>
__global__ __launch_bounds__(kThreads) void paged_attn_kernel(AttnArgs a) {
  constexpr int LPT = D / 8;        // lanes per token row
  constexpr int TPW = 64 / LPT;     // tokens per wave load
  constexpr int BT = 16;            // tokens per block (pages are walked in 16-token blocks)
  constexpr int NT = BT / TPW;      // tokens per lane per block
  constexpr int BPP = P / BT;       // blocks per page
  static_assert(P % BT == 0 && BT % TPW == 0, "page size must be a multiple of 16");

  __shared__ float s_m[kWaves][GMAX], s_l[kWaves][GMAX];
  __shared__ __attribute__((aligned(16))) float s_o[kWaves][GMAX][D];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int split = blockIdx.x;   // grid.x == num_splits; every wave reaches the barrier
  const int hk = blockIdx.y;
  const int b = blockIdx.z;

  const int G = a.Hq / a.Hkv;
  const int tg = lane / LPT;  // token group within a wave step
  const int dc = lane % LPT;  // 8-dim column chunk

  const int seq = a.seq_lens[b];
  const int n_pages = min((seq + P - 1) / P, a.max_pages);
  const int pps = (a.max_pages + a.num_splits - 1) / a.num_splits;
  const int p_begin = split * pps;
  const int p_end = min(n_pages, p_begin + pps);
  const int blk_begin = p_begin * BPP;
  const int blk_end = max(p_end * BPP, blk_begin);

  // Query heads of this kv head, 8 dims per lane, pre-scaled into log2 units.
  float qf[GMAX][8];
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    if (g < G) {
      const uint16_t* qp = a.q + (int64_t)b * a.q_sb + (int64_t)(hk * G + g) * a.q_sh + dc * 8;
      const uint4 v = *reinterpret_cast<const uint4*>(qp);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        qf[g][2 * j] = lo_h(w[j]) * a.qk_scale_log2;
        qf[g][2 * j + 1] = hi_h(w[j]) * a.qk_scale_log2;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) qf[g][j] = 0.f;
    }
  }

  float m_run[GMAX], l_run[GMAX], o[GMAX][8];
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    m_run[g] = -INFINITY;
    l_run[g] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[g][j] = 0.f;
  }

  const int64_t head_off = (int64_t)hk * a.head_stride + dc * 8;
  uint4 kc[NT], vc[NT], kn[NT], vn[NT];

  // A slot outside the pool is read as slot 0 and its tokens are masked.
  auto page_slot = [&](int p) -> int {
    const int slot = a.page_table[(int64_t)b * a.pt_stride + p];
    return (slot >= 0 && slot < a.num_slots) ? slot : -1;
  };
  auto load_block = [&](int blk, uint4* kk, uint4* vv) {
    const int p = blk / BPP;
    const int t0 = (blk - p * BPP) * BT;
    const int slot = max(page_slot(p), 0);
    const int64_t base = (int64_t)slot * a.slot_stride + head_off + (int64_t)t0 * D;
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      const int64_t off = base + (int64_t)(tg + i * TPW) * D;
      kk[i] = ld_nt16((a.k_pool + off));
      vv[i] = ld_nt16((a.v_pool + off));
    }
  };

  // wave w takes blocks blk_begin + w, + kWaves, ...
  if (blk_begin + wave < blk_end) load_block(blk_begin + wave, kc, vc);

  for (int blk = blk_begin + wave; blk < blk_end; blk += kWaves) {
    if (blk + kWaves < blk_end) load_block(blk + kWaves, kn, vn);
    const int p = blk / BPP;
    const int t0 = (blk - p * BPP) * BT;
    // valid tokens of this block (may be <= 0 for the tail blocks of the last page)
    const int ntok = page_slot(p) < 0 ? 0 : min(BT, seq - p * P - t0);

    // scores s[g][i] (log2 units) for this lane's NT tokens
    float s[GMAX][NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      const uint32_t kw[4] = {kc[i].x, kc[i].y, kc[i].z, kc[i].w};
      float kf[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        kf[2 * j] = lo_h(kw[j]);
        kf[2 * j + 1] = hi_h(kw[j]);
      }
#pragma unroll
      for (int g = 0; g < GMAX; ++g) {
        float t = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) t = fmaf(qf[g][j], kf[j], t);
        s[g][i] = t;
      }
    }
    // reduce the partial dots over the LPT lanes of a token row
#pragma unroll
    for (int off = LPT / 2; off >= 1; off >>= 1) {
#pragma unroll
      for (int g = 0; g < GMAX; ++g)
#pragma unroll
        for (int i = 0; i < NT; ++i) s[g][i] += __shfl_xor(s[g][i], off, 64);
    }
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      if (tg + i * TPW >= ntok) {
#pragma unroll
        for (int g = 0; g < GMAX; ++g) s[g][i] = -INFINITY;
      }
    }

    // Unwritten page slots hold arbitrary bits (possibly NaN/Inf); a masked token
    // has p = 0, and 0 * NaN would poison the sum, so its V row is zeroed.
    float vf[NT][8];
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      const bool valid = tg + i * TPW < ntok;
      const uint32_t vw[4] = {vc[i].x, vc[i].y, vc[i].z, vc[i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        vf[i][2 * j] = valid ? lo_h(vw[j]) : 0.f;
        vf[i][2 * j + 1] = valid ? hi_h(vw[j]) : 0.f;
      }
    }

#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      if (g < G) {
        float pm = s[g][0];
#pragma unroll
        for (int i = 1; i < NT; ++i) pm = fmaxf(pm, s[g][i]);
#pragma unroll
        for (int off = LPT; off < 64; off <<= 1) pm = fmaxf(pm, __shfl_xor(pm, off, 64));
        const float m_new = fmaxf(m_run[g], pm);
        // reference point for the exponentials; 0 while nothing has been seen so
        // that exp2(-inf - ref) = 0 never becomes exp2(NaN)
        const float ref = (m_new == -INFINITY) ? 0.f : m_new;
        const float alpha = exp2f(m_run[g] - ref);
        float lsum = 0.f;
        float pv[NT];
#pragma unroll
        for (int i = 0; i < NT; ++i) {
          pv[i] = exp2f(s[g][i] - ref);  // masked tokens: exp2(-inf) = 0
          lsum += pv[i];
        }
        l_run[g] = l_run[g] * alpha + lsum;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          float t = o[g][j] * alpha;
#pragma unroll
          for (int i = 0; i < NT; ++i) t = fmaf(pv[i], vf[i][j], t);
          o[g][j] = t;
        }
        m_run[g] = m_new;
      }
    }

#pragma unroll
    for (int i = 0; i < NT; ++i) {
      kc[i] = kn[i];
      vc[i] = vn[i];
    }
  }

  // merge the token groups of the wave (lanes with the same dc), publish to LDS
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    if (g < G) {
      float l = l_run[g];
#pragma unroll
      for (int off = LPT; off < 64; off <<= 1) l += __shfl_xor(l, off, 64);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float t = o[g][j];
#pragma unroll
        for (int off = LPT; off < 64; off <<= 1) t += __shfl_xor(t, off, 64);
        o[g][j] = t;
      }
      if (tg == 0) {
        float4* dst = reinterpret_cast<float4*>(&s_o[wave][g][dc * 8]);
        dst[0] = make_float4(o[g][0], o[g][1], o[g][2], o[g][3]);
        dst[1] = make_float4(o[g][4], o[g][5], o[g][6], o[g][7]);
      }
      if (lane == 0) {
        s_m[wave][g] = m_run[g];
        s_l[wave][g] = l;
      }
    }
  }
  __syncthreads();

  // merge the four waves and write this split's partial
  for (int idx = threadIdx.x; idx < G * D; idx += kThreads) {
    const int g = idx / D;
    const int d = idx - g * D;
    float mx = s_m[0][g];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) mx = fmaxf(mx, s_m[w][g]);
    const float ref = (mx == -INFINITY) ? 0.f : mx;
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float sc = exp2f(s_m[w][g] - ref);
      num = fmaf(sc, s_o[w][g][d], num);
      den = fmaf(sc, s_l[w][g], den);
    }
    const int64_t pidx = ((int64_t)b * a.Hq + hk * G + g) * a.total_splits + a.split_offset + split;
    a.part_o[pidx * D + d] = den > 0.f ? num / den : 0.f;
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

template <int D, int P>
int launch_attn_dp(const AttnArgs& a, int G, hipStream_t s) {
  dim3 grid(a.num_splits, a.Hkv, a.B);
  if (G <= 2) hipLaunchKernelGGL((paged_attn_kernel<D, P, 2>), grid, dim3(kThreads), 0, s, a);
  else if (G <= 4) hipLaunchKernelGGL((paged_attn_kernel<D, P, 4>), grid, dim3(kThreads), 0, s, a);
  else hipLaunchKernelGGL((paged_attn_kernel<D, P, 8>), grid, dim3(kThreads), 0, s, a);
  return HELM_OK;
}

template <int D>
int launch_attn_d(const AttnArgs& a, int P, int G, hipStream_t s) {
  if (P == 16) return launch_attn_dp<D, 16>(a, G, s);
  if (P == 32) return launch_attn_dp<D, 32>(a, G, s);
  return launch_attn_dp<D, 64>(a, G, s);
}

}  // namespace

extern "C" int64_t helm_paged_attn_workspace_floats(int B, int Hq, int D, int num_splits) {
  if (B < 1 || Hq < 1 || D < 1 || num_splits < 1) return 0;
  return (int64_t)B * Hq * num_splits * (D + 2);
}

extern "C" int helm_paged_decode_attn(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                      const void* k_pool, const void* v_pool, int64_t slot_stride,
                                      int64_t head_stride, const int32_t* page_table,
                                      int64_t pt_stride, const int32_t* seq_lens,
                                      int64_t num_slots, float* part_o, float* part_ml,
                                      int split_offset, int total_splits, int B, int Hq, int Hkv,
                                      int D, int P, int max_pages, int num_splits, float scale,
                                      void* stream) {
  HELM_CHECK_ARG(q && k_pool && v_pool && page_table && seq_lens && part_o && part_ml,
                 "helm_paged_decode_attn: null pointer");
  HELM_CHECK_ARG(B >= 1 && Hq >= 1 && Hkv >= 1 && max_pages >= 1 && num_splits >= 1,
                 "helm_paged_decode_attn: sizes must be positive");
  HELM_CHECK_ARG(Hq % Hkv == 0, "helm_paged_decode_attn: Hq must be a multiple of Hkv");
  HELM_CHECK_SUPPORTED(Hq / Hkv <= 8, "helm_paged_decode_attn: at most 8 query heads per kv head");
  HELM_CHECK_SUPPORTED(D == 64 || D == 128, "helm_paged_decode_attn: head_dim must be 64 or 128");
  HELM_CHECK_SUPPORTED(P == 16 || P == 32 || P == 64, "helm_paged_decode_attn: page size must be 16, 32 or 64");
  HELM_CHECK_ARG(pt_stride >= max_pages, "helm_paged_decode_attn: page-table stride < max_pages");
  HELM_CHECK_ARG(num_slots >= 1, "helm_paged_decode_attn: num_slots must be positive");
  HELM_CHECK_ARG(split_offset >= 0 && split_offset + num_splits <= total_splits,
                 "helm_paged_decode_attn: splits [split_offset, split_offset+num_splits) exceed total_splits");
  HELM_CHECK_ARG(head_stride >= (int64_t)P * D, "helm_paged_decode_attn: head stride too small");
  HELM_CHECK_SUPPORTED(q_stride_h % 8 == 0 && q_stride_b % 8 == 0 && slot_stride % 8 == 0 &&
                           head_stride % 8 == 0,
                       "helm_paged_decode_attn: strides must be multiples of 8 elements");
  HELM_CHECK_SUPPORTED(helm::aligned16(q) && helm::aligned16(k_pool) && helm::aligned16(v_pool) &&
                           helm::aligned16(part_o),
                       "helm_paged_decode_attn: q, pools and part_o must be 16-byte aligned");
  AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q); a.q_sb = q_stride_b; a.q_sh = q_stride_h;
  a.k_pool = static_cast<const uint16_t*>(k_pool);
  a.v_pool = static_cast<const uint16_t*>(v_pool);
  a.slot_stride = slot_stride; a.head_stride = head_stride;
  a.page_table = page_table; a.pt_stride = pt_stride; a.seq_lens = seq_lens;
  a.num_slots = num_slots;
  a.part_o = part_o; a.part_ml = part_ml;
  a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.max_pages = max_pages; a.num_splits = num_splits;
  a.split_offset = split_offset; a.total_splits = total_splits;
  a.qk_scale_log2 = scale * kLog2e;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int G = Hq / Hkv;
  if (D == 64) launch_attn_d<64>(a, P, G, s);
  else launch_attn_d<128>(a, P, G, s);
  HELM_CHECK_LAUNCH("helm_paged_decode_attn launch");
  return HELM_OK;
}

extern "C" int helm_paged_attn_reduce(const float* part_o, const float* part_ml, void* out, int B,
                                      int Hq, int D, int num_splits, void* stream) {
  HELM_CHECK_ARG(part_o && part_ml && out, "helm_paged_attn_reduce: null pointer");
  HELM_CHECK_ARG(B >= 1 && Hq >= 1 && num_splits >= 1, "helm_paged_attn_reduce: sizes must be positive");
  HELM_CHECK_SUPPORTED(D == 64 || D == 128, "helm_paged_attn_reduce: head_dim must be 64 or 128");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (D == 64)
    hipLaunchKernelGGL((attn_reduce_kernel<64>), dim3(B * Hq), dim3(256), 0, s, part_o, part_ml,
                       static_cast<uint16_t*>(out), num_splits);
  else
    hipLaunchKernelGGL((attn_reduce_kernel<128>), dim3(B * Hq), dim3(256), 0, s, part_o, part_ml,
                       static_cast<uint16_t*>(out), num_splits);
  HELM_CHECK_LAUNCH("helm_paged_attn_reduce launch");
  return HELM_OK;
}
