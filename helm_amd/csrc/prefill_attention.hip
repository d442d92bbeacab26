// prefill_attention.hip — causal prefill attention over the paged KV pool.
//
// The prefill half of the patched Qwen3 attention (helm/runtime/kv_offload.py:
// 253-265: SDPA with a causal mask over the prompt) for one sequence whose
// prompt K/V already sit in their pages: query token i (position q_start + i)
// attends keys 0 .. q_start + i of the page table.  Same MFMA scheme as the
// decode kernel (paged_attention.hip): per 32-key step a wave computes
//   S^T[32 keys x 16 queries] = K . Q^T       (2 x D/32 v_mfma_f32_16x16x32_f16)
//   O^T[D x 16 queries]     += V^T . P^T      (D/16 MFMAs, P rounded to fp16 as in
//                                               the reference's fp16 SDPA)
// for NC 16-query column tiles; the key order inside the score tiles is
// permuted so that each lane holds the probabilities of exactly the 8
// consecutive keys whose V^T it feeds to the second MFMA.
//
// A workgroup is one query head x a block of 4 * 16 * NC queries, one wave per
// 16 * NC queries.  The four waves need the same K/V tiles, so the workgroup
// fetches each 32-key tile once, straight into LDS (global_load_lds_dwordx4:
// every lane moves 16 bytes, a wave 1 KiB of contiguous pool memory), double
// buffered: tile s+1 is copied while tile s is computed, and the waves read
// their MFMA operands from LDS.  The copy of tile s+1 is issued only after the
// operand reads of tile s (the compiler makes LDS reads wait for outstanding
// copies, so this order keeps the copy in flight across the whole step).  LDS layouts (16-byte chunks) are chosen so
// that both the copies and the operand reads are conflict free:
//   K: row-major [32 keys][D/8 chunks], chunk index XOR-swizzled by key bits
//      {0,1,3,4}, so the 16 rows one operand read touches hit 16 distinct banks;
//   V: [D/16 dim groups][4 key chunks][16 dims] — one operand read is 16
//      consecutive chunks; one copy instruction is 16 dims x 32 keys.
// Each wave computes up to its own causal end; the workgroup keeps copying
// until its last wave's end.  The kv head is the fastest-varying workgroup
// index: workgroups are dealt round-robin to the 8 XCDs, so with 8 kv heads
// each XCD serves one kv head and its K/V stays in that XCD's L2.  fp32 online
// softmax per query in the log2 domain; keys past the query's position are
// masked; blocks with the most keys are launched first.
#include <type_traits>

#include "helm_common.h"

namespace {

constexpr int kKS = 32;                 // keys per step
constexpr float kLazy = 8.f;            // lazy-rescale slack of the running maximum (log2)
constexpr int kMaxPages = 4096;         // page-table entries staged in LDS
#ifndef PF_NC
#define PF_NC 2
#endif
constexpr int kNS = 2;                  // K/V stages in LDS

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;

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
  // MASK form: additive fp16 mask element (h, t, key) at mask[h*m_sh + t*m_si + key]
  // over keys 0 .. kv_len - 1; rows padded to m_si >= kv_len rounded up to 32
  const uint16_t* mask;
  int64_t m_sh, m_si;
  int kv_len;
  float inv_scale;
  // optional per query row t: keys from key_end[t] on are -inf in every head's
  // mask, so a wave (workgroup) stops at the last key step any of its rows sees
  const int32_t* key_end;
};

// Workgroup barrier for the K/V stages: this wave's copies into LDS have landed
// and its LDS reads have returned (s_waitcnt vmcnt(0) lgkmcnt(0); gfx9
// encoding, expcnt left at its maximum), then s_barrier.
__device__ __forceinline__ void stage_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (0 << 8));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// q is read once (non-temporal)
__device__ __forceinline__ h8_t ld_h8_nt(const uint16_t* p) {
  return __builtin_bit_cast(h8_t, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p)));
}

template <int D>
struct KStep {
  h8_t k[2][D / 32];
  h8_t v[D / 16];
  bool page_ok;     // the page of this lane's 8 keys is valid
};

// XOR swizzle of K chunk columns: key row r -> bits {0,1} and {3,4} of r, so the
// rows (col>>2)*8 + t*4 + (col&3) of the 16 lanes of one operand read differ
// in their swizzle (limited to the chunk count of a row)
template <int CPR>
__device__ __forceinline__ int kswz(int r) {
  return ((r & 3) | (((r >> 3) & 3) << 2)) & (CPR - 1);
}

// NC: 16-query column tiles per wave; a workgroup covers QB = 64 * NC queries.
// MASK: every query sees keys 0 .. kv_len - 1 with the additive mask added to its
// scaled scores (the reference's SDPA with attn_mask); otherwise causal.
template <int D, int P, int NC, bool MASK>
#ifndef PF_WPE
#define PF_WPE 2
#endif
__global__ __launch_bounds__(256, PF_WPE) void prefill_attn_kernel(PrefillArgs a) {
  constexpr int KT = D / 32;
  constexpr int DT = D / 16;
  constexpr int CPR = D / 8;                      // 16-byte chunks per K row
  constexpr int kWQ = 16 * NC;                    // queries per wave
  constexpr int kQB = 4 * kWQ;                    // queries per workgroup
  constexpr int kKC = kKS * CPR;                  // K chunks per stage
  constexpr int kVC = D * (kKS / 8);              // V chunks per stage
  constexpr int kIssue = (kKC + kVC) / 256;       // copy instructions per thread per stage
  static_assert(P % 16 == 0, "page size must be a multiple of 16");
  static_assert(kKC % 256 == 0 && kVC % 256 == 0, "stage must split evenly over 256 threads");
  __shared__ int s_slot[kMaxPages];
  __shared__ int s_bad;                           // some staged page is invalid
  __shared__ int s_kr;                            // MASK: one past the workgroup's last key
  __shared__ __attribute__((aligned(16))) u32x4_t s_kv[kNS][kKC + kVC];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int G = a.Hq / a.Hkv;
  const int nqb = (a.T + kQB - 1) / kQB;
  const int hk = (int)blockIdx.x % a.Hkv;
  const int r = (int)blockIdx.x / a.Hkv;
  const int h = hk * G + r % G;
  const int q0 = (nqb - 1 - r / G) * kQB;         // heaviest (latest) blocks first
  const int qw = q0 + wave * kWQ;                  // this wave's first query

  const int wg_key_end = MASK ? a.kv_len : a.q_start + min(q0 + kQB, a.T);
  const int npages = (wg_key_end + P - 1) / P;
  if (tid == 0) {
    s_bad = 0;
    s_kr = 0;
  }
  __syncthreads();
  for (int i = tid; i < npages; i += blockDim.x) {
    const int slot = a.page_table[i];
    const bool ok = slot >= 0 && slot < a.num_slots;
    s_slot[i] = ok ? slot : -1;
    if (!ok) s_bad = 1;
  }
  // Q^T operands of the column tiles: lane holds q[query col][kk*32 + grp*8, +8]
  h8_t qb_op[NC][KT];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int qi = min(qw + c * 16 + col, a.T - 1);
#pragma unroll
    for (int kk = 0; kk < KT; ++kk)
      qb_op[c][kk] = ld_h8_nt(a.q + (int64_t)qi * a.q_st + (int64_t)h * a.q_sh + kk * 32 + grp * 8);
  }
  // MASK: keys [0, w_hi) hold every key some query of this wave can see
  int w_hi = a.kv_len;
  if constexpr (MASK) {
    if (a.key_end) {
      w_hi = 0;
      for (int i = lane; i < kWQ; i += 64) {
        const int t = qw + i;
        if (t < a.T) w_hi = max(w_hi, a.key_end[t]);
      }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) w_hi = max(w_hi, __shfl_xor(w_hi, off, 64));
      // wave-uniform after the butterfly: held in a scalar register
      w_hi = __builtin_amdgcn_readfirstlane(min(w_hi, a.kv_len));
    }
    if (qw >= a.T) w_hi = 0;
    if (lane == 0) atomicMax(&s_kr, w_hi);
  }
  __syncthreads();

  // keys [0, key_end) can be seen by some query of this wave
  const int key_end = qw < a.T ? (MASK ? w_hi : a.q_start + min(qw + kWQ, a.T)) : 0;
  const int nsteps = (key_end + kKS - 1) / kKS;
  // the workgroup's steps [step0, wg_steps)
  // the workgroup's steps [0, wg_steps): with MASK up to the last key any of its
  // rows sees (an LDS value, uniform over the workgroup).  Steps below a row's
  // first visible key are visited anyway (their keys are -inf for it): a loop
  // starting at a run-time step measured spills at every form tried.
  const int wg_steps = MASK ? (__builtin_amdgcn_readfirstlane(s_kr) + kKS - 1) / kKS
                            : (wg_key_end + kKS - 1) / kKS;
  // steps whose keys every query of the wave sees (all below the diagonal, valid
  // pages): no masking
  const int nfull = (s_bad || MASK) ? 0 : min(nsteps, (a.q_start + qw + 1) / kKS);
  const int p_last = max(npages - 1, 0);
  const uint16_t* kbase = a.k + (int64_t)hk * a.k_hs;
  const uint16_t* vbase = a.v + (int64_t)hk * a.v_hs;

  // Copies key tile `st` into stage `b`: thread tid moves chunk i*256 + tid of
  // the stage for i < kIssue (K chunks first, then V); a wave's 64 lanes fill 64
  // consecutive chunks.  Invalid pages read slot 0 (masked in compute).
  // Each thread's chunks sit at the same token row of every 32-key step: the
  // row and its element offset inside a page are computed once.  When P divides
  // the step (P = 16, 32) a step starts on a page boundary, so only the page's
  // slot changes from step to step; with P = 64 odd steps start half way in.
  constexpr bool kStepOnPage = kKS % P == 0;
  int c_row[kIssue];     // token row of chunk i inside the step
  int c_off[kIssue];     // its element offset inside a page at in-page row c_row (K) / token c_row (V)
#pragma unroll
  for (int i = 0; i < kIssue; ++i) {
    const int pos = i * 256 + tid;
    if (i * 256 < kKC) {                             // K chunk (wave-uniform branch)
      const int row = pos / CPR;
      const int c = (pos % CPR) ^ kswz<CPR>(row);
      c_row[i] = row;
      c_off[i] = (row % P) * D + c * 8;
    } else {                                         // V chunk
      const int qv = pos - kKC;
      const int dim = (qv >> 6) * 16 + (qv & 15);
      const int row = ((qv >> 4) & 3) * 8;
      c_row[i] = row;
      c_off[i] = dim * (int)a.v_ds + row % P;
    }
  }
  auto issue = [&](int st, int b) {
    const int tok0 = st * kKS;
    const int in0 = kStepOnPage ? 0 : tok0 % P;       // the step's start inside its page
#pragma unroll
    for (int i = 0; i < kIssue; ++i) {
      const bool is_k = i * 256 < kKC;                // compile-time per i
      const int slot = max(s_slot[min((tok0 + c_row[i]) / P, p_last)], 0);
      const uint16_t* src =
          is_k ? kbase + (int64_t)slot * a.k_ss + c_off[i] + in0 * D
               : vbase + (int64_t)slot * a.v_ss + c_off[i] + in0;
      __builtin_amdgcn_global_load_lds(src, (lds_void_t*)&s_kv[b][i * 256 + wave * 64], 16, 0, 0);
    }
  };

  // MFMA operands of key tile s (in stage b), and the validity of its page
  auto read = [&](KStep<D>& bf, int s, int b) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int row = (col >> 2) * 8 + t * 4 + (col & 3);
#pragma unroll
      for (int kk = 0; kk < KT; ++kk)
        bf.k[t][kk] = __builtin_bit_cast(h8_t, s_kv[b][row * CPR + ((kk * 4 + grp) ^ kswz<CPR>(row))]);
    }
#pragma unroll
    for (int d = 0; d < DT; ++d) bf.v[d] = __builtin_bit_cast(h8_t, s_kv[b][kKC + d * 64 + grp * 16 + col]);
    const int tv = s * kKS + grp * 8;
    bf.page_ok = s_slot[min(tv / P, p_last)] >= 0 && tv / P < npages;
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

  // One key step for the NC column tiles.  FULL: every key of the step is
  // visible to every query of the wave.  Otherwise keys past a query's position
  // or in invalid pages are masked, and V entries of keys no query of the wave
  // may see are zeroed in place (their bytes may be unwritten).  The running maximum is raised lazily: while
  // no column's step maximum exceeds it by more than kLazy (log2 units) the
  // stale maximum stays the exponent reference (p <= 2^kLazy: fp32 sums, and
  // fp16 P keeps its relative precision), which skips rescaling O on most steps.
  auto compute = [&](auto full_tag, KStep<D>& bf, int s) {
    constexpr bool FULL = decltype(full_tag)::value;
    const int tok0 = s * kKS;
    const int tv = tok0 + grp * 8;                     // this lane's 8 keys tv .. tv+7
    const bool page_ok = bf.page_ok;
    if constexpr (!FULL) {
      const int nvis = page_ok ? max(0, min(8, key_end - tv)) : 0;
      uint32_t vmask[4];
#pragma unroll
      for (int q2 = 0; q2 < 4; ++q2)
        vmask[q2] = (2 * q2 < nvis ? 0x0000ffffu : 0u) | (2 * q2 + 1 < nvis ? 0xffff0000u : 0u);
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        u32x4_t vw = __builtin_bit_cast(u32x4_t, bf.v[d]);
        vw.x &= vmask[0];
        vw.y &= vmask[1];
        vw.z &= vmask[2];
        vw.w &= vmask[3];
        bf.v[d] = __builtin_bit_cast(h8_t, vw);
      }
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      f4_t sc0 = {0.f, 0.f, 0.f, 0.f}, sc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) {
        sc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf.k[0][kk], qb_op[c][kk], sc0, 0, 0, 0);
        sc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf.k[1][kk], qb_op[c][kk], sc1, 0, 0, 0);
      }
      float sv[8];                                     // raw scores of keys tv .. tv+7
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sv[r] = sc0[r];
        sv[4 + r] = sc1[r];
      }
      if constexpr (MASK) {
        // mask of this lane's query row at keys tv .. tv+7 (loaded after the score
        // MFMAs: fewer registers live across them); scores are scaled at the
        // exponent, so the mask enters divided by the scale
        const int qm = min(qw + c * 16 + col, a.T - 1);
        const u32x4_t mraw =
            *reinterpret_cast<const u32x4_t*>(a.mask + (int64_t)h * a.m_sh + (int64_t)qm * a.m_si + tv);
        const h8_t mh = __builtin_bit_cast(h8_t, mraw);
#pragma unroll
        for (int j = 0; j < 8; ++j) sv[j] = __builtin_fmaf((float)mh[j], a.inv_scale, sv[j]);
      }
      if constexpr (!FULL) {
        const int qi = qw + c * 16 + col;              // query index of this lane's column
        // keys visible to this query: tv + j <= q_start + qi, or < kv_len with a mask
        // (and inside valid pages)
        const int kend = MASK ? a.kv_len : a.q_start + qi + 1;
        const int nvalid = (page_ok && qi < a.T) ? max(0, min(8, kend - tv)) : 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) sv[j] = j < nvalid ? sv[j] : -INFINITY;
      }
      // this lane's maximum over its 8 keys; some lane of a column exceeds the
      // column's running maximum by more than kLazy exactly when the column's
      // maximum does, so the lanes combine (two butterflies over the column's
      // four lane groups) only on the rare steps that rescale
      float mx = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                       fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
      if (__ballot(mx * a.qk_scale_log2 > m_run[c] + kLazy)) {   // wave-uniform; the scale is positive
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m_run[c], mx * a.qk_scale_log2);
        const float alpha = __builtin_amdgcn_exp2f(m_run[c] - (m_new == -INFINITY ? 0.f : m_new));
        l_run[c] *= alpha;
#pragma unroll
        for (int d = 0; d < DT; ++d) o[c][d] *= alpha;
        m_run[c] = m_new;
      }
      const float nref = m_run[c] == -INFINITY ? 0.f : -m_run[c];
      // P enters the PV product rounded to fp16, as the fp16 SDPA of the
      // reference's prefill keeps it (the row sums stay fp32)
      h8_t ph;
      float lsum = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[j], a.qk_scale_log2, nref));
        ph[j] = (_Float16)p;
        lsum += p;
      }
      l_run[c] += lsum;
#pragma unroll
      for (int d = 0; d < DT; ++d)
        o[c][d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf.v[d], ph, o[c][d], 0, 0, 0);
    }
  };
  auto step = [&](KStep<D>& bf, int s) {
    if (s < nfull) compute(std::true_type{}, bf, s);
    else compute(std::false_type{}, bf, s);
  };

  issue(0, 0);
  for (int s = 0; s < wg_steps; ++s) {
    stage_barrier();                 // tile s is in stage s&1; stage (s+1)&1 is no longer read
    KStep<D> bf;
    if (s < nsteps) read(bf, s, s & 1);
    if (s + 1 < wg_steps) issue(s + 1, (s + 1) & 1);
    if (s < nsteps) step(bf, s);
  }

  // normalise and store: o[c][d][r] = O^T[dim d*16 + grp*4 + r][query col of tile c]
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float l = l_run[c];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const int qi = qw + c * 16 + col;
    if (qi < a.T) {
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

namespace {

// Checks shared by both entry points, argument set-up and the launch.
int prefill_launch(const char* fn, const void* q, int64_t q_stride_t, int64_t q_stride_h,
                   const helm_kv_pool* pool, const int32_t* page_table, int q_start, int T, int Hq,
                   int Hkv, int D, int P, float scale, void* out, int64_t out_stride_t,
                   int64_t out_stride_h, const void* mask, int64_t mask_stride_h,
                   int64_t mask_stride_t, int kv_len, const int32_t* key_end, void* stream) {
  const std::string f(fn);
  HELM_CHECK_ARG(q && pool && pool->k && pool->v && page_table && out, f + ": null pointer");
  HELM_CHECK_ARG(T >= 1 && q_start >= 0 && Hq >= 1 && Hkv >= 1, f + ": bad sizes");
  HELM_CHECK_ARG(Hq % Hkv == 0, f + ": Hq must be a multiple of Hkv");
  HELM_CHECK_SUPPORTED(D == 64 || D == 128, f + ": head_dim must be 64 or 128");
  HELM_CHECK_SUPPORTED(P == 16 || P == 32 || P == 64, f + ": page size must be 16, 32 or 64");
  const int64_t keys = mask ? (int64_t)kv_len : (int64_t)q_start + T;
  HELM_CHECK_SUPPORTED((keys + P - 1) / P <= kMaxPages,
                       f + ": more than " + std::to_string(kMaxPages) + " pages");
  HELM_CHECK_ARG(pool->num_slots >= 1 && pool->k_head_stride >= (int64_t)P * D &&
                     pool->v_dim_stride >= P && pool->v_head_stride >= (int64_t)P * D,
                 f + ": pool strides too small for the page");
  HELM_CHECK_SUPPORTED(pool->v_dim_stride * D < (1ll << 31),
                       f + ": V dim stride too large (in-page offsets are 32-bit)");
  HELM_CHECK_SUPPORTED(q_stride_t % 8 == 0 && q_stride_h % 8 == 0 && out_stride_t % 4 == 0 &&
                           out_stride_h % 4 == 0 && pool->k_slot_stride % 8 == 0 &&
                           pool->k_head_stride % 8 == 0 && pool->v_slot_stride % 8 == 0 &&
                           pool->v_head_stride % 8 == 0 && pool->v_dim_stride % 8 == 0,
                       f + ": strides must be multiples of 8 (q, pool) / 4 (out) elements");
  HELM_CHECK_SUPPORTED(helm::aligned16(q) && helm::aligned16(pool->k) && helm::aligned16(pool->v) &&
                           (reinterpret_cast<uintptr_t>(out) & 7u) == 0,
                       f + ": q and pools must be 16-byte aligned, out 8-byte aligned");
  if (mask) {
    HELM_CHECK_ARG(kv_len >= 1, f + ": kv_len must be positive");
    HELM_CHECK_ARG(mask_stride_h >= 0 && mask_stride_t >= ((int64_t)kv_len + 31) / 32 * 32,
                   f + ": mask rows must hold kv_len rounded up to a multiple of 32");
    HELM_CHECK_SUPPORTED(mask_stride_h % 8 == 0 && mask_stride_t % 8 == 0 && helm::aligned16(mask),
                         f + ": mask must be 16-byte aligned with strides multiples of 8");
  }
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
  a.mask = static_cast<const uint16_t*>(mask); a.m_sh = mask_stride_h; a.m_si = mask_stride_t;
  a.kv_len = kv_len;
  a.inv_scale = 1.f / scale;
  a.key_end = key_end;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto go = [&](auto kern) {
    constexpr int qb = 64 * PF_NC;
    hipLaunchKernelGGL(kern, dim3(((T + qb - 1) / qb) * Hq), dim3(256), 0, s, a);
  };
  auto by_page = [&](auto d_tag, auto m_tag) {
    constexpr int Dc = decltype(d_tag)::value;
    constexpr bool Mc = decltype(m_tag)::value;
    if (P == 16) go(prefill_attn_kernel<Dc, 16, PF_NC, Mc>);
    else if (P == 32) go(prefill_attn_kernel<Dc, 32, PF_NC, Mc>);
    else go(prefill_attn_kernel<Dc, 64, PF_NC, Mc>);
  };
  auto by_mask = [&](auto d_tag) {
    if (mask) by_page(d_tag, std::true_type{});
    else by_page(d_tag, std::false_type{});
  };
  if (D == 64) by_mask(std::integral_constant<int, 64>{});
  else by_mask(std::integral_constant<int, 128>{});
  HELM_CHECK_LAUNCH(fn);
  return HELM_OK;
}

}  // namespace

extern "C" int helm_prefill_attn(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                                 const helm_kv_pool* pool, const int32_t* page_table,
                                 int q_start, int T, int Hq, int Hkv, int D, int P, float scale,
                                 void* out, int64_t out_stride_t, int64_t out_stride_h,
                                 void* stream) {
  return prefill_launch("helm_prefill_attn", q, q_stride_t, q_stride_h, pool, page_table, q_start,
                        T, Hq, Hkv, D, P, scale, out, out_stride_t, out_stride_h, nullptr, 0, 0, 0,
                        nullptr, stream);
}

extern "C" int helm_prefill_attn_mask(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                                      const helm_kv_pool* pool, const int32_t* page_table, int T,
                                      int kv_len, int Hq, int Hkv, int D, int P, float scale,
                                      const void* mask, int64_t mask_stride_h,
                                      int64_t mask_stride_t, const int32_t* key_end, void* out,
                                      int64_t out_stride_t,
                                      int64_t out_stride_h, void* stream) {
  HELM_CHECK_ARG(mask, "helm_prefill_attn_mask: null mask");
  return prefill_launch("helm_prefill_attn_mask", q, q_stride_t, q_stride_h, pool, page_table, 0,
                        T, Hq, Hkv, D, P, scale, out, out_stride_t, out_stride_h, mask,
                        mask_stride_h, mask_stride_t, kv_len, key_end, stream);
}
