// prefill_attention.hip — causal prefill attention over the paged KV pool.
//
// The prefill half of the patched Qwen3 attention (helm/runtime/kv_offload.py:
// 253-265: SDPA with a causal mask over the prompt) for one sequence whose
// prompt K/V already sit in their pages: query token i (position q_start + i)
// attends keys 0 .. q_start + i of the page table.  Same MFMA scheme as the
// decode kernel (paged_attention.hip): per 32-key step a wave computes
//   S^T[32 keys x 16 queries] = K . Q^T       (2 x D/32 v_mfma_f32_16x16x32_f16)
//   O^T[D x 16 queries]     += V^T . P^T      (D/16 x 2 MFMAs, P = fp16 hi + lo)
// for two 16-query column tiles; the key order inside the score tiles is
// permuted so that each lane holds the probabilities of exactly the 8
// consecutive keys whose V^T it feeds to the second MFMA.  A workgroup is the G
// query heads of one kv head (one wave each) x a 32-query block, so the waves
// stream the same K/V rows (shared through L1).  fp32 online softmax per query
// in the log2 domain; keys past the query's position are masked; blocks with
// the most keys are launched first.
#include "helm_common.h"

namespace {

constexpr int kKS = 32;                 // keys per step
constexpr int kMaxPages = 4096;         // page-table entries staged in LDS

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_st, q_sh;                   // query element (t, h, d): t*q_st + h*q_sh + d
  uint16_t* out;
  int64_t o_st, o_sh;
  const uint16_t* k;
  int64_t k_ss, k_hs;
  const uint16_t* v;
  int64_t v_ss, v_hs, v_ds;
  int64_t num_slots;
  const int32_t* page_table;
  int T, q_start, Hq, Hkv;
  float qk_scale_log2;
};

__device__ __forceinline__ h8_t ld_h8(const uint16_t* p) {
  return __builtin_bit_cast(h8_t, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p)));
}

template <int D>
struct KStep {
  h8_t k[2][D / 32];
  h8_t v[D / 16];
};

// NC: 16-query column tiles per wave (2 when a group has at most 4 query heads,
// so the 256-thread workgroup may use up to 512 registers per lane; 1 for 5-8
// heads, 512 threads); a workgroup covers QB = 16 * NC queries.
template <int D, int P, int NC>
__global__ __launch_bounds__(NC == 2 ? 256 : 512) void prefill_attn_kernel(PrefillArgs a) {
  constexpr int KT = D / 32;
  constexpr int DT = D / 16;
  constexpr int kQB = 16 * NC;
  static_assert(P % 16 == 0, "page size must be a multiple of 16");
  __shared__ int s_slot[kMaxPages];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;                      // query head g of the group
  const int lane = tid & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int G = a.Hq / a.Hkv;
  const int hk = blockIdx.y;
  const int nqb = (a.T + kQB - 1) / kQB;
  const int qb = nqb - 1 - (int)blockIdx.x;       // heaviest (latest) blocks first
  const int q0 = qb * kQB;                         // first query index of the block
  const int h = hk * G + wave;

  const int key_end = a.q_start + min(q0 + kQB, a.T);   // keys [0, key_end) can be seen
  const int npages = (key_end + P - 1) / P;
  for (int i = tid; i < npages; i += blockDim.x) {
    const int slot = a.page_table[i];
    s_slot[i] = (slot >= 0 && slot < a.num_slots) ? slot : -1;
  }
  // Q^T operands of the two column tiles: lane holds q[query col][kk*32 + grp*8, +8]
  h8_t qb_op[NC][KT];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int qi = min(q0 + c * 16 + col, a.T - 1);
#pragma unroll
    for (int kk = 0; kk < KT; ++kk)
      qb_op[c][kk] = ld_h8(a.q + (int64_t)qi * a.q_st + (int64_t)h * a.q_sh + kk * 32 + grp * 8);
  }
  __syncthreads();

  const int nsteps = (key_end + kKS - 1) / kKS;
  const int p_last = max(npages - 1, 0);
  const uint16_t* kbase = a.k + (int64_t)hk * a.k_hs;
  const uint16_t* vbase = a.v + (int64_t)hk * a.v_hs + (int64_t)col * a.v_ds;

  auto load = [&](KStep<D>& bf, int s) {
    const int tok0 = s * kKS;
    const int tk = tok0 + (col >> 2) * 8 + (col & 3);   // score-tile row `col` of tile 0
    const int slot_k = max(s_slot[min(tk / P, p_last)], 0);
    const uint16_t* kp = kbase + (int64_t)slot_k * a.k_ss + (int64_t)(tk % P) * D + grp * 8;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) bf.k[t][kk] = ld_h8(kp + t * 4 * D + kk * 32);
    const int tv = tok0 + grp * 8;
    const int slot_v = max(s_slot[min(tv / P, p_last)], 0);
    const uint16_t* vp = vbase + (int64_t)slot_v * a.v_ss + (tv % P);
#pragma unroll
    for (int d = 0; d < DT; ++d) bf.v[d] = ld_h8(vp + (int64_t)(d * 16) * a.v_ds);
  };

  float m_run[NC], l_run[NC];
  f4_t o[NC][DT];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    m_run[c] = -INFINITY;
    l_run[c] = 0.f;
#pragma unroll
    for (int d = 0; d < DT; ++d) o[c][d] = f4_t{0.f, 0.f, 0.f, 0.f};
  }

  auto compute = [&](KStep<D>& bf, int s) {
    const int tok0 = s * kKS;
    const int tv = tok0 + grp * 8;                     // this lane's 8 keys tv .. tv+7
    const bool page_ok = s_slot[min(tv / P, p_last)] >= 0 && tv / P < npages;
    // V entries of keys that no query of the block may see are zeroed (their
    // bytes may be unwritten)
    const int nvis = page_ok ? max(0, min(8, key_end - tv)) : 0;
    uint32_t vmask[4];
#pragma unroll
    for (int q2 = 0; q2 < 4; ++q2)
      vmask[q2] = (2 * q2 < nvis ? 0x0000ffffu : 0u) | (2 * q2 + 1 < nvis ? 0xffff0000u : 0u);
#pragma unroll
    for (int d = 0; d < DT; ++d) {   // in place: the buffer is reloaded before its next use
      u32x4_t vw = __builtin_bit_cast(u32x4_t, bf.v[d]);
      vw.x &= vmask[0];
      vw.y &= vmask[1];
      vw.z &= vmask[2];
      vw.w &= vmask[3];
      bf.v[d] = __builtin_bit_cast(h8_t, vw);
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int qi = q0 + c * 16 + col;                // query index of this lane's column
      const int qpos = a.q_start + qi;
      // keys visible to this query: tv + j <= qpos (and inside valid pages)
      const int nvalid = (page_ok && qi < a.T) ? max(0, min(8, qpos + 1 - tv)) : 0;
      f4_t sc0 = {0.f, 0.f, 0.f, 0.f}, sc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) {
        sc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf.k[0][kk], qb_op[c][kk], sc0, 0, 0, 0);
        sc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf.k[1][kk], qb_op[c][kk], sc1, 0, 0, 0);
      }
      float sv[8];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sv[r] = r < nvalid ? sc0[r] * a.qk_scale_log2 : -INFINITY;
        sv[4 + r] = 4 + r < nvalid ? sc1[r] * a.qk_scale_log2 : -INFINITY;
      }
      float mx = sv[0];
#pragma unroll
      for (int j = 1; j < 8; ++j) mx = fmaxf(mx, sv[j]);
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run[c], mx);
      const float ref = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = exp2f(m_run[c] - ref);
      h8_t phi, plo;
      float lsum = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float p = exp2f(sv[j] - ref);
        const _Float16 hp = (_Float16)p;
        phi[j] = hp;
        plo[j] = (_Float16)(p - (float)hp);
        lsum += p;
      }
      l_run[c] = l_run[c] * alpha + lsum;
      m_run[c] = m_new;
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        o[c][d] *= alpha;
        o[c][d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf.v[d], phi, o[c][d], 0, 0, 0);
        o[c][d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf.v[d], plo, o[c][d], 0, 0, 0);
      }
    }
  };

  // every wave walks all key steps of the block (ping-pong register buffers)
  KStep<D> bufA, bufB;
  if (wave < G && nsteps > 0) load(bufA, 0);
  int s = 0;
  if (wave < G) {
    for (; s + 2 < nsteps; s += 2) {
      load(bufB, s + 1);
      compute(bufA, s);
      load(bufA, s + 2);
      compute(bufB, s + 1);
    }
    if (s + 1 < nsteps) {
      load(bufB, s + 1);
      compute(bufA, s);
      compute(bufB, s + 1);
    } else if (s < nsteps) {
      compute(bufA, s);
    }
  }

  // normalise and store: o[c][d][r] = O^T[dim d*16 + grp*4 + r][query col of tile c]
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float l = l_run[c];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const int qi = q0 + c * 16 + col;
    if (wave < G && qi < a.T) {
      const float inv = l > 0.f ? 1.f / fmaxf(l, 1e-12f) : 0.f;
      uint16_t* dst = a.out + (int64_t)qi * a.o_st + (int64_t)h * a.o_sh + grp * 4;
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        const uint32_t lo = pack_h2(o[c][d][0] * inv, o[c][d][1] * inv);
        const uint32_t hi = pack_h2(o[c][d][2] * inv, o[c][d][3] * inv);
        *reinterpret_cast<uint2*>(dst + d * 16) = make_uint2(lo, hi);
      }
    }
  }
}

}  // namespace

extern "C" int helm_prefill_attn(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                                 const helm_kv_pool* pool, const int32_t* page_table,
                                 int q_start, int T, int Hq, int Hkv, int D, int P, float scale,
                                 void* out, int64_t out_stride_t, int64_t out_stride_h,
                                 void* stream) {
  HELM_CHECK_ARG(q && pool && pool->k && pool->v && page_table && out, "helm_prefill_attn: null pointer");
  HELM_CHECK_ARG(T >= 1 && q_start >= 0 && Hq >= 1 && Hkv >= 1, "helm_prefill_attn: bad sizes");
  HELM_CHECK_ARG(Hq % Hkv == 0, "helm_prefill_attn: Hq must be a multiple of Hkv");
  HELM_CHECK_SUPPORTED(Hq / Hkv <= 8, "helm_prefill_attn: at most 8 query heads per kv head");
  HELM_CHECK_SUPPORTED(D == 64 || D == 128, "helm_prefill_attn: head_dim must be 64 or 128");
  HELM_CHECK_SUPPORTED(P == 16 || P == 32 || P == 64, "helm_prefill_attn: page size must be 16, 32 or 64");
  HELM_CHECK_SUPPORTED(((int64_t)q_start + T + P - 1) / P <= kMaxPages,
                       "helm_prefill_attn: more than " + std::to_string(kMaxPages) + " pages");
  HELM_CHECK_ARG(pool->num_slots >= 1 && pool->k_head_stride >= (int64_t)P * D &&
                     pool->v_dim_stride >= P && pool->v_head_stride >= (int64_t)P * D,
                 "helm_prefill_attn: pool strides too small for the page");
  HELM_CHECK_SUPPORTED(q_stride_t % 8 == 0 && q_stride_h % 8 == 0 && out_stride_t % 4 == 0 &&
                           out_stride_h % 4 == 0 && pool->k_slot_stride % 8 == 0 &&
                           pool->k_head_stride % 8 == 0 && pool->v_slot_stride % 8 == 0 &&
                           pool->v_head_stride % 8 == 0 && pool->v_dim_stride % 8 == 0,
                       "helm_prefill_attn: strides must be multiples of 8 (q, pool) / 4 (out) elements");
  HELM_CHECK_SUPPORTED(helm::aligned16(q) && helm::aligned16(pool->k) && helm::aligned16(pool->v) &&
                           (reinterpret_cast<uintptr_t>(out) & 7u) == 0,
                       "helm_prefill_attn: q and pools must be 16-byte aligned, out 8-byte aligned");
  PrefillArgs a{};
  a.q = static_cast<const uint16_t*>(q); a.q_st = q_stride_t; a.q_sh = q_stride_h;
  a.out = static_cast<uint16_t*>(out); a.o_st = out_stride_t; a.o_sh = out_stride_h;
  a.k = static_cast<const uint16_t*>(pool->k); a.k_ss = pool->k_slot_stride; a.k_hs = pool->k_head_stride;
  a.v = static_cast<const uint16_t*>(pool->v);
  a.v_ss = pool->v_slot_stride; a.v_hs = pool->v_head_stride; a.v_ds = pool->v_dim_stride;
  a.num_slots = pool->num_slots;
  a.page_table = page_table;
  a.T = T; a.q_start = q_start; a.Hq = Hq; a.Hkv = Hkv;
  a.qk_scale_log2 = scale * kLog2e;
  const int G = Hq / Hkv;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto go = [&](auto kern, int qb) {
    hipLaunchKernelGGL(kern, dim3((T + qb - 1) / qb, Hkv), dim3(64 * G), 0, s, a);
  };
  if (G <= 4) {
    if (D == 64) {
      if (P == 16) go(prefill_attn_kernel<64, 16, 2>, 32);
      else if (P == 32) go(prefill_attn_kernel<64, 32, 2>, 32);
      else go(prefill_attn_kernel<64, 64, 2>, 32);
    } else {
      if (P == 16) go(prefill_attn_kernel<128, 16, 2>, 32);
      else if (P == 32) go(prefill_attn_kernel<128, 32, 2>, 32);
      else go(prefill_attn_kernel<128, 64, 2>, 32);
    }
  } else {
    if (D == 64) {
      if (P == 16) go(prefill_attn_kernel<64, 16, 1>, 16);
      else if (P == 32) go(prefill_attn_kernel<64, 32, 1>, 16);
      else go(prefill_attn_kernel<64, 64, 1>, 16);
    } else {
      if (P == 16) go(prefill_attn_kernel<128, 16, 1>, 16);
      else if (P == 32) go(prefill_attn_kernel<128, 32, 1>, 16);
      else go(prefill_attn_kernel<128, 64, 1>, 16);
    }
  }
  HELM_CHECK_LAUNCH("helm_prefill_attn launch");
  return HELM_OK;
}
