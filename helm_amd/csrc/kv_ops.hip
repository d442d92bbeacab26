// kv_ops.hip — KV page writes, host-page staging and the decode-step glue that
// sits between the projections and the paged attention.
#include <vector>

#include "helm_common.h"

namespace {

// Layout of one pool (strides in elements; see helm_kv_pool).
struct PoolArgs {
  uint16_t* k;
  uint16_t* v;
  int64_t k_ss, k_hs, v_ss, v_hs, v_ds, num_slots;
};

PoolArgs pool_args(const helm_kv_pool* p) {
  return PoolArgs{static_cast<uint16_t*>(p->k), static_cast<uint16_t*>(p->v), p->k_slot_stride,
                  p->k_head_stride, p->v_slot_stride, p->v_head_stride, p->v_dim_stride,
                  p->num_slots};
}

// ---------------------------------------------------------------------------
// helm_kv_append: one thread per 8 fp16 (16 bytes) of the new tokens; K rows are
// stored as one 16-byte write, V (token-contiguous per dim) as 8 fp16 writes.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void kv_append_kernel(
    const uint4* __restrict__ k_new, const uint4* __restrict__ v_new, PoolArgs pa,
    const int32_t* __restrict__ slots, const int32_t* __restrict__ offsets, int B, int Hkv,
    int n_tok, int D, int P) {
  const int vec_per_tok = D / 8;
  const int64_t total = (int64_t)B * Hkv * n_tok * vec_per_tok;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(i % vec_per_tok);
    int64_t r = i / vec_per_tok;
    const int t = (int)(r % n_tok);
    r /= n_tok;
    const int h = (int)(r % Hkv);
    const int b = (int)(r / Hkv);
    const int slot = slots[b];
    const int pos = offsets[b] + t;
    if (slot < 0 || slot >= pa.num_slots || pos < 0 || pos >= P) continue;
    *reinterpret_cast<uint4*>(pa.k + (int64_t)slot * pa.k_ss + (int64_t)h * pa.k_hs +
                              (int64_t)pos * D + c * 8) = k_new[i];
    const uint4 vv = v_new[i];
    const uint32_t w[4] = {vv.x, vv.y, vv.z, vv.w};
    uint16_t* vd = pa.v + (int64_t)slot * pa.v_ss + (int64_t)h * pa.v_hs + (int64_t)(c * 8) * pa.v_ds + pos;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      vd[(int64_t)(2 * e) * pa.v_ds] = (uint16_t)(w[e] & 0xffffu);
      vd[(int64_t)(2 * e + 1) * pa.v_ds] = (uint16_t)(w[e] >> 16);
    }
  }
}

// ---------------------------------------------------------------------------
// helm_qk_norm_rope_append: one wave per (item, head) of the fused qkv output.
// Lane l holds elements d = l + 64*j, j < D/64.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void qk_norm_rope_append_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ q_norm_w,
    const uint16_t* __restrict__ k_norm_w, float eps, const int32_t* __restrict__ positions,
    const float* __restrict__ inv_freq, uint16_t* __restrict__ q_out, PoolArgs pa,
    const int32_t* __restrict__ slots, const int32_t* __restrict__ offsets, int B, int Hq, int Hkv,
    int P) {
  constexpr int J = D / 64;
  constexpr int HALF = D / 2;
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int heads = Hq + 2 * Hkv;
  if (item >= B * heads) return;
  const int b = item / heads;
  const int hh = item - b * heads;
  const uint16_t* src = qkv + (int64_t)b * heads * D + (int64_t)hh * D;

  float x[J];
#pragma unroll
  for (int j = 0; j < J; ++j) x[j] = h2f(src[lane + 64 * j]);

  const int slot = slots[b];
  const int off = offsets[b];
  const bool slot_ok = slot >= 0 && slot < pa.num_slots && off >= 0 && off < P;

  if (hh >= Hq + Hkv) {  // value head: copy into the page (token-contiguous per dim)
    if (!slot_ok) return;
    const int h = hh - Hq - Hkv;
    uint16_t* dst = pa.v + (int64_t)slot * pa.v_ss + (int64_t)h * pa.v_hs + off;
#pragma unroll
    for (int j = 0; j < J; ++j) dst[(int64_t)(lane + 64 * j) * pa.v_ds] = src[lane + 64 * j];
    return;
  }

  // RMSNorm over the head: fp16(w * fp16(x * rsqrt(mean(x^2) + eps)))
  const uint16_t* nw = hh < Hq ? q_norm_w : k_norm_w;
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < J; ++j) ss = fmaf(x[j], x[j], ss);
  ss = wave_sum(ss);
  const float rstd = rsqrtf(ss / (float)D + eps);
  float xn[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const float t = h2f(f2h(x[j] * rstd));
    xn[j] = h2f(f2h(h2f(nw[lane + 64 * j]) * t));
  }

  // RoPE, rotate_half: d < D/2 pairs with -x[d + D/2], d >= D/2 with x[d - D/2]
  const float pos = (float)positions[b];
  float out[J];
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
    const float ang = inv_freq[d % HALF] * pos;
    const float c = h2f(f2h(cosf(ang)));
    const float s = h2f(f2h(sinf(ang)));
    const float t1 = h2f(f2h(xn[j] * c));
    const float t2 = h2f(f2h(rot * s));
    out[j] = t1 + t2;
  }

  if (hh < Hq) {
    uint16_t* dst = q_out + ((int64_t)b * Hq + hh) * D;
#pragma unroll
    for (int j = 0; j < J; ++j) dst[lane + 64 * j] = f2h(out[j]);
  } else if (slot_ok) {
    const int h = hh - Hq;
    uint16_t* dst = pa.k + (int64_t)slot * pa.k_ss + (int64_t)h * pa.k_hs + (int64_t)off * D;
#pragma unroll
    for (int j = 0; j < J; ++j) dst[lane + 64 * j] = f2h(out[j]);
  }
}

// helm_qk_norm_rope_cs: one wave per (item, q or k head) of the fused qkv
// output: the per-head RMSNorm when norm weights are given, then RoPE with the
// caller's cos / sin rows (transformers' position embeddings, so every RoPE
// scaling the model configures is already in them), rounded as the fp16 torch
// ops round; q to q_out [B, Hq, D], k to k_out [B, Hkv, D].
template <int D>
__global__ __launch_bounds__(256) void qk_norm_rope_cs_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ q_norm_w,
    const uint16_t* __restrict__ k_norm_w, float eps, const uint16_t* __restrict__ cos_t,
    const uint16_t* __restrict__ sin_t, int64_t cs_b, uint16_t* __restrict__ q_out,
    uint16_t* __restrict__ k_out, int B, int Hq, int Hkv) {
  constexpr int J = D / 64;
  constexpr int HALF = D / 2;
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int qk_heads = Hq + Hkv;
  if (item >= B * qk_heads) return;
  const int b = item / qk_heads;
  const int hh = item - b * qk_heads;
  const uint16_t* src = qkv + (int64_t)b * (qk_heads + Hkv) * D + (int64_t)hh * D;
  float xn[J];
#pragma unroll
  for (int j = 0; j < J; ++j) xn[j] = h2f(src[lane + 64 * j]);
  const uint16_t* nw = hh < Hq ? q_norm_w : k_norm_w;
  if (nw != nullptr) {   // fp16(w * fp16(x * rsqrt(mean(x^2) + eps)))
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j) ss = fmaf(xn[j], xn[j], ss);
    const float rstd = rsqrtf(wave_sum(ss) / (float)D + eps);
#pragma unroll
    for (int j = 0; j < J; ++j) xn[j] = h2f(f2h(h2f(nw[lane + 64 * j]) * h2f(f2h(xn[j] * rstd))));
  }
  const uint16_t* cr = cos_t + (int64_t)b * cs_b;
  const uint16_t* sr = sin_t + (int64_t)b * cs_b;
  uint16_t* dst = hh < Hq ? q_out + ((int64_t)b * Hq + hh) * D : k_out + ((int64_t)b * Hkv + hh - Hq) * D;
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
    const float t1 = h2f(f2h(xn[j] * h2f(cr[d])));
    const float t2 = h2f(f2h(rot * h2f(sr[d])));
    dst[d] = f2h(t1 + t2);
  }
}

// ---------------------------------------------------------------------------
// helm_rmsnorm: one workgroup per row.  Rows of up to 8 * 256 * 8 elements with
// 16-byte aligned data take the vector form: each thread loads its 16-byte
// pieces of x and of the weight once, up front, and keeps them in registers
// through the reduction (one round trip instead of a loop of 2-byte loads, then
// a second pass); other rows the scalar form.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float rms_block_sum(float ss, float* red) {
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                      const uint16_t* __restrict__ w, float eps,
                                                      uint16_t* __restrict__ y, int K) {
  __shared__ float red[4];
  const int row = blockIdx.x;
  const uint16_t* xr = x + (int64_t)row * K;
  float ss = 0.f;
  for (int k = threadIdx.x; k < K; k += 256) {
    const float f = h2f(xr[k]);
    ss = fmaf(f, f, ss);
  }
  const float tot = rms_block_sum(ss, red);
  const float rstd = rsqrtf(tot / (float)K + eps);
  for (int k = threadIdx.x; k < K; k += 256) {
    const float t = h2f(f2h(h2f(xr[k]) * rstd));
    y[(int64_t)row * K + k] = f2h(h2f(w[k]) * t);
  }
}

constexpr int kRmsVec = 8;   // most 16-byte pieces per thread of the vector form

__global__ __launch_bounds__(256) void rmsnorm_vec_kernel(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ w, float eps,
                                                          uint16_t* __restrict__ y, int K) {
  __shared__ float red[4];
  const int row = blockIdx.x;
  const int nv = K / 8;
  const uint4* xr = reinterpret_cast<const uint4*>(x + (int64_t)row * K);
  const uint4* wr = reinterpret_cast<const uint4*>(w);
  uint4 xv[kRmsVec], wv[kRmsVec];
#pragma unroll
  for (int i = 0; i < kRmsVec; ++i) {
    const int v = min(threadIdx.x + i * 256, nv - 1);   // clamped in range; extra pieces unused
    xv[i] = xr[v];
    wv[i] = wr[v];
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kRmsVec; ++i) {
    if ((int)threadIdx.x + i * 256 < nv) {
      const uint32_t q[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float a = lo_h(q[j]), b = hi_h(q[j]);
        ss = fmaf(a, a, ss);
        ss = fmaf(b, b, ss);
      }
    }
  }
  const float tot = rms_block_sum(ss, red);
  const float rstd = rsqrtf(tot / (float)K + eps);
  uint4* yr = reinterpret_cast<uint4*>(y + (int64_t)row * K);
#pragma unroll
  for (int i = 0; i < kRmsVec; ++i) {
    const int v = threadIdx.x + i * 256;
    if (v < nv) {
      const uint32_t q[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
      const uint32_t g[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
      uint32_t o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float t0 = h2f(f2h(lo_h(q[j]) * rstd)), t1 = h2f(f2h(hi_h(q[j]) * rstd));
        o[j] = pack_h2(lo_h(g[j]) * t0, hi_h(g[j]) * t1);
      }
      yr[v] = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
}

// ---------------------------------------------------------------------------
// helm_silu_mul: out = fp16(fp16(silu(gate)) * up) elementwise (silu in fp32),
// the SwiGLU of the fused GEMV epilogue, for gate / up computed by separate
// GEMVs; 8 elements per thread where the tensors are 16-byte aligned.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float silu_f16(float g) { return h2f(f2h(g / (1.0f + expf(-g)))); }

__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ gate,
                                                       const uint16_t* __restrict__ up,
                                                       uint16_t* __restrict__ out, int64_t n,
                                                       bool vec) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (vec) {
    if (t * 8 + 8 <= n) {
      const uint4 g = reinterpret_cast<const uint4*>(gate)[t];
      const uint4 u = reinterpret_cast<const uint4*>(up)[t];
      const uint32_t gq[4] = {g.x, g.y, g.z, g.w}, uq[4] = {u.x, u.y, u.z, u.w};
      uint32_t o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = pack_h2(silu_f16(lo_h(gq[j])) * lo_h(uq[j]), silu_f16(hi_h(gq[j])) * hi_h(uq[j]));
      reinterpret_cast<uint4*>(out)[t] = make_uint4(o[0], o[1], o[2], o[3]);
      return;
    }
    for (int64_t i = t * 8; i < n; ++i) out[i] = f2h(silu_f16(h2f(gate[i])) * h2f(up[i]));   // tail
  } else if (t < n) {
    out[t] = f2h(silu_f16(h2f(gate[t])) * h2f(up[t]));
  }
}

// ---------------------------------------------------------------------------
// helm_argmax_f16: one 1024-thread workgroup per row; 16-byte loads, every
// thread keeps the first index of its largest value, then a tree over lanes and
// waves keeps the smaller index on ties (torch.argmax returns the first maximum;
// a NaN counts as larger than any number, as there).
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool argmax_better(float v, int i, float bv, int bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

__global__ __launch_bounds__(1024) void argmax_f16_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                          int N, bool vec, int64_t* __restrict__ out) {
  __shared__ float s_v[16];
  __shared__ int s_i[16];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const uint16_t* xr = x + (int64_t)row * ldx;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  const int nvec = vec ? N / 8 : 0;   // rows not 16-byte aligned: scalar loads only
  // 16 loads per thread issued before any compare (one round trip per 16K
  // vectors: a 151936-entry vocabulary row in two); argmax_better is a total
  // order, so the scan order does not change the result
  constexpr int U = 16;
  for (int v0 = tid; v0 < nvec; v0 += 1024 * U) {
    uint4 q[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int v = min(v0 + u * 1024, nvec - 1);   // clamped in range; extra lanes skipped below
      q[u] = *reinterpret_cast<const uint4*>(xr + (int64_t)v * 8);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int v = v0 + u * 1024;
      if (v < nvec) {
        const uint32_t w[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float a = lo_h(w[j]), b = hi_h(w[j]);
          if (argmax_better(a, v * 8 + 2 * j, bv, bi)) { bv = a; bi = v * 8 + 2 * j; }
          if (argmax_better(b, v * 8 + 2 * j + 1, bv, bi)) { bv = b; bi = v * 8 + 2 * j + 1; }
        }
      }
    }
  }
  for (int i = nvec * 8 + tid; i < N; i += 1024) {   // tail (or all of an unaligned row)
    const float a = h2f(xr[i]);
    if (argmax_better(a, i, bv, bi)) { bv = a; bi = i; }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    if (argmax_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  if ((tid & 63) == 0) {
    s_v[tid >> 6] = bv;
    s_i[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 16; ++w)
      if (argmax_better(s_v[w], s_i[w], bv, bi)) { bv = s_v[w]; bi = s_i[w]; }
    out[row] = bi == 0x7fffffff ? 0 : bi;
  }
}

// Workspace form: kArgmaxParts workgroups per row each reduce one contiguous
// range (a wave per 64 vectors, 4 loads per thread issued together) to its first
// best (value, index); one wave per row then merges the parts in the same order.
// The per-element compares, serial on one CU in the single-workgroup form (about
// 20 us for a 151936-entry row), spread over the parts' CUs.
constexpr int kArgmaxParts = 64;

__device__ __forceinline__ void argmax_wave_reduce(float& bv, int& bi) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    if (argmax_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
}

__global__ __launch_bounds__(256) void argmax_part_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                          int N, bool vec, float* __restrict__ pv,
                                                          int* __restrict__ pi) {
  __shared__ float s_v[4];
  __shared__ int s_i[4];
  const int part = blockIdx.x;
  const int row = blockIdx.y;
  const int tid = threadIdx.x;
  const uint16_t* xr = x + (int64_t)row * ldx;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  if (vec) {
    const int nvec = N / 8;
    const int per = (nvec + kArgmaxParts - 1) / kArgmaxParts;
    const int lo = part * per, hi = min(nvec, lo + per);
    constexpr int U = 4;
    for (int v0 = lo + tid; v0 < hi; v0 += 256 * U) {
      uint4 q[U];
#pragma unroll
      for (int u = 0; u < U; ++u)   // clamped into [v0, hi): extra lanes skipped below
        q[u] = *reinterpret_cast<const uint4*>(xr + (int64_t)min(v0 + u * 256, hi - 1) * 8);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int v = v0 + u * 256;
        if (v < hi) {
          const uint32_t w[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float a = lo_h(w[j]), b = hi_h(w[j]);
            if (argmax_better(a, v * 8 + 2 * j, bv, bi)) { bv = a; bi = v * 8 + 2 * j; }
            if (argmax_better(b, v * 8 + 2 * j + 1, bv, bi)) { bv = b; bi = v * 8 + 2 * j + 1; }
          }
        }
      }
    }
    if (part == kArgmaxParts - 1) {   // elements past the last whole vector
      for (int i = nvec * 8 + tid; i < N; i += 256) {
        const float a = h2f(xr[i]);
        if (argmax_better(a, i, bv, bi)) { bv = a; bi = i; }
      }
    }
  } else {   // rows not 16-byte aligned: scalar loads over an element range
    const int per = (N + kArgmaxParts - 1) / kArgmaxParts;
    const int lo = part * per, hi = min(N, lo + per);
    for (int i = lo + tid; i < hi; i += 256) {
      const float a = h2f(xr[i]);
      if (argmax_better(a, i, bv, bi)) { bv = a; bi = i; }
    }
  }
  argmax_wave_reduce(bv, bi);
  if ((tid & 63) == 0) {
    s_v[tid >> 6] = bv;
    s_i[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w)
      if (argmax_better(s_v[w], s_i[w], bv, bi)) { bv = s_v[w]; bi = s_i[w]; }
    pv[row * kArgmaxParts + part] = bv;
    pi[row * kArgmaxParts + part] = bi;
  }
}

__global__ __launch_bounds__(64) void argmax_merge_kernel(const float* __restrict__ pv,
                                                          const int* __restrict__ pi,
                                                          int64_t* __restrict__ out) {
  const int row = blockIdx.x;
  const int lane = threadIdx.x;
  float bv = pv[row * kArgmaxParts + lane];
  int bi = pi[row * kArgmaxParts + lane];
  argmax_wave_reduce(bv, bi);
  if (lane == 0) out[row] = bi == 0x7fffffff ? 0 : bi;
}

// ---------------------------------------------------------------------------
// helm_gather_pages_h2d: one workgroup per (page, K or V) reads the page straight
// out of pinned host memory (through its device mapping, over the host link)
// and writes it to its staging slot; 8 independent 16-byte loads per thread in
// flight.  Slots outside [0, host_slots) leave their staging page untouched.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gather_pages_kernel(
    const u32x4_t* __restrict__ host_k, const u32x4_t* __restrict__ host_v,
    u32x4_t* __restrict__ dev_k, u32x4_t* __restrict__ dev_v, const int32_t* __restrict__ slots, int64_t first, int64_t vec_per_page,
    int64_t host_slots) {
  const int page = blockIdx.x >> 1;
  const int slot = slots[page];
  if (slot < 0 || slot >= host_slots) return;
  const u32x4_t* src = ((blockIdx.x & 1) ? host_v : host_k) + (int64_t)slot * vec_per_page;
  u32x4_t* dst = ((blockIdx.x & 1) ? dev_v : dev_k) + (first + page) * vec_per_page;
  constexpr int kUnroll = 8;
  for (int64_t base = 0; base < vec_per_page; base += (int64_t)kUnroll * blockDim.x) {
    u32x4_t r[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + (int64_t)u * blockDim.x + threadIdx.x;
      if (i < vec_per_page) r[u] = __builtin_nontemporal_load(src + i);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + (int64_t)u * blockDim.x + threadIdx.x;
      if (i < vec_per_page) dst[i] = r[u];
    }
  }
}

}  // namespace

static int check_pool(const helm_kv_pool* p, int D, int P, const char* fn) {
  const std::string f(fn);
  HELM_CHECK_ARG(p && p->k && p->v, f + ": null pool pointer");
  HELM_CHECK_ARG(p->num_slots >= 1, f + ": num_slots must be positive");
  HELM_CHECK_ARG(p->k_head_stride >= (int64_t)P * D && p->v_dim_stride >= P &&
                     p->v_head_stride >= (int64_t)P * D,
                 f + ": pool strides too small for the page");
  HELM_CHECK_SUPPORTED(p->k_slot_stride % 8 == 0 && p->k_head_stride % 8 == 0 && helm::aligned16(p->k),
                       f + ": K pool strides must be multiples of 8 and the pool 16-byte aligned");
  return HELM_OK;
}

extern "C" int helm_kv_append(const void* k_new, const void* v_new, const helm_kv_pool* pool,
                              const int32_t* slots, const int32_t* offsets, int B, int Hkv,
                              int n_tok, int D, int P, void* stream) {
  HELM_CHECK_ARG(k_new && v_new && slots && offsets, "helm_kv_append: null pointer");
  HELM_CHECK_ARG(B >= 1 && Hkv >= 1 && n_tok >= 1 && D >= 8 && P >= 1,
                 "helm_kv_append: sizes must be positive");
  HELM_CHECK_SUPPORTED(D % 8 == 0, "helm_kv_append: D must be a multiple of 8");
  const int rc = check_pool(pool, D, P, "helm_kv_append");
  if (rc != HELM_OK) return rc;
  HELM_CHECK_SUPPORTED(helm::aligned16(k_new) && helm::aligned16(v_new),
                       "helm_kv_append: buffers must be 16-byte aligned");
  const int64_t total = (int64_t)B * Hkv * n_tok * (D / 8);
  const int blocks = (int)std::min<int64_t>((total + 255) / 256, 4096);
  hipLaunchKernelGGL(kv_append_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint4*>(k_new), static_cast<const uint4*>(v_new),
                     pool_args(pool), slots, offsets, B, Hkv, n_tok, D, P);
  HELM_CHECK_LAUNCH("helm_kv_append launch");
  return HELM_OK;
}

extern "C" int helm_gather_pages_h2d(const void* host_k, const void* host_v, void* dev_k,
                                     void* dev_v, const int32_t* slots, int n,
                                     int64_t dev_first_slot, int64_t page_bytes,
                                     int64_t host_slots, void* stream) {
  HELM_CHECK_ARG(host_k && host_v && dev_k && dev_v && (n == 0 || slots),
                 "helm_gather_pages_h2d: null pointer");
  HELM_CHECK_ARG(n >= 0 && page_bytes > 0 && dev_first_slot >= 0 && host_slots >= 0,
                 "helm_gather_pages_h2d: bad sizes");
  HELM_CHECK_SUPPORTED(page_bytes % 16 == 0 && helm::aligned16(host_k) && helm::aligned16(host_v) &&
                           helm::aligned16(dev_k) && helm::aligned16(dev_v),
                       "helm_gather_pages_h2d: pages must be 16-byte multiples, pools 16-byte aligned");
  if (n == 0) return HELM_OK;
  // the kernel reads the host pools through their device mappings; memory the
  // runtime does not map for the device is refused here, never dereferenced
  void* dk = nullptr;
  void* dv = nullptr;
  hipError_t e = hipHostGetDevicePointer(&dk, const_cast<void*>(host_k), 0);
  if (e != hipSuccess || !dk)
    return helm::hip_fail(e == hipSuccess ? hipErrorInvalidValue : e,
                          "helm_gather_pages_h2d: host K pool is not device-mapped pinned memory");
  e = hipHostGetDevicePointer(&dv, const_cast<void*>(host_v), 0);
  if (e != hipSuccess || !dv)
    return helm::hip_fail(e == hipSuccess ? hipErrorInvalidValue : e,
                          "helm_gather_pages_h2d: host V pool is not device-mapped pinned memory");
  hipLaunchKernelGGL(gather_pages_kernel, dim3(2 * n), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4_t*>(dk), static_cast<const u32x4_t*>(dv),
                     static_cast<u32x4_t*>(dev_k), static_cast<u32x4_t*>(dev_v), slots, dev_first_slot, page_bytes / 16, host_slots);
  HELM_CHECK_LAUNCH("helm_gather_pages_h2d launch");
  return HELM_OK;
}

extern "C" int helm_stage_pages_h2d(const void* host_pool, void* dev_staging,
                                    const int32_t* host_slots, int n, int64_t dev_first_slot,
                                    size_t page_bytes, void* copy_stream, void* done_event) {
  HELM_CHECK_ARG(host_pool && dev_staging && (n == 0 || host_slots), "helm_stage_pages_h2d: null pointer");
  HELM_CHECK_ARG(n >= 0 && page_bytes > 0 && dev_first_slot >= 0, "helm_stage_pages_h2d: bad sizes");
  hipStream_t s = static_cast<hipStream_t>(copy_stream);
  const char* src = static_cast<const char*>(host_pool);
  char* dst = static_cast<char*>(dev_staging);
  int i = 0;
  while (i < n) {
    HELM_CHECK_ARG(host_slots[i] >= 0, "helm_stage_pages_h2d: negative host slot");
    int j = i + 1;
    while (j < n && host_slots[j] == host_slots[j - 1] + 1) ++j;  // merge a run of slots
    const size_t bytes = (size_t)(j - i) * page_bytes;
    hipError_t e = hipMemcpyAsync(dst + (size_t)(dev_first_slot + i) * page_bytes,
                                  src + (size_t)host_slots[i] * page_bytes, bytes,
                                  hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return helm::hip_fail(e, "helm_stage_pages_h2d: hipMemcpyAsync");
    i = j;
  }
  if (done_event) {
    hipError_t e = hipEventRecord(static_cast<hipEvent_t>(done_event), s);
    if (e != hipSuccess) return helm::hip_fail(e, "helm_stage_pages_h2d: hipEventRecord");
  }
  return HELM_OK;
}

extern "C" int helm_qk_norm_rope_append(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                                        float eps, const int32_t* positions, const float* inv_freq,
                                        void* q_out, const helm_kv_pool* pool, const int32_t* slots,
                                        const int32_t* offsets, int B, int Hq, int Hkv, int D,
                                        int P, void* stream) {
  HELM_CHECK_ARG(qkv && q_norm_w && k_norm_w && positions && inv_freq && q_out && slots && offsets,
                 "helm_qk_norm_rope_append: null pointer");
  HELM_CHECK_ARG(B >= 1 && Hq >= 1 && Hkv >= 1 && P >= 1, "helm_qk_norm_rope_append: sizes must be positive");
  HELM_CHECK_SUPPORTED(D == 64 || D == 128, "helm_qk_norm_rope_append: head_dim must be 64 or 128");
  const int rc = check_pool(pool, D, P, "helm_qk_norm_rope_append");
  if (rc != HELM_OK) return rc;
  const int items = B * (Hq + 2 * Hkv);
  const int blocks = (items + 3) / 4;
  const PoolArgs pa = pool_args(pool);
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto args = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), 0, s, static_cast<const uint16_t*>(qkv),
                       static_cast<const uint16_t*>(q_norm_w), static_cast<const uint16_t*>(k_norm_w),
                       eps, positions, inv_freq, static_cast<uint16_t*>(q_out), pa, slots,
                       offsets, B, Hq, Hkv, P);
  };
  if (D == 64) args(qk_norm_rope_append_kernel<64>);
  else args(qk_norm_rope_append_kernel<128>);
  HELM_CHECK_LAUNCH("helm_qk_norm_rope_append launch");
  return HELM_OK;
}

extern "C" int helm_qk_norm_rope_cs(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                                    float eps, const void* cos_t, const void* sin_t,
                                    int64_t cs_stride_b, void* q_out, void* k_out, int B, int Hq,
                                    int Hkv, int D, void* stream) {
  HELM_CHECK_ARG(qkv && cos_t && sin_t && q_out && k_out, "helm_qk_norm_rope_cs: null pointer");
  HELM_CHECK_ARG((q_norm_w == nullptr) == (k_norm_w == nullptr),
                 "helm_qk_norm_rope_cs: give both norm weights or neither");
  HELM_CHECK_ARG(B >= 1 && Hq >= 1 && Hkv >= 1, "helm_qk_norm_rope_cs: sizes must be positive");
  HELM_CHECK_SUPPORTED(D == 64 || D == 128, "helm_qk_norm_rope_cs: head_dim must be 64 or 128");
  HELM_CHECK_ARG(cs_stride_b == 0 || cs_stride_b >= D || B == 1,
                 "helm_qk_norm_rope_cs: cos / sin row stride must be 0 (one row for all) or >= head_dim");
  const int items = B * (Hq + Hkv);
  const int blocks = (items + 3) / 4;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto args = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), 0, s, static_cast<const uint16_t*>(qkv),
                       static_cast<const uint16_t*>(q_norm_w), static_cast<const uint16_t*>(k_norm_w),
                       eps, static_cast<const uint16_t*>(cos_t), static_cast<const uint16_t*>(sin_t),
                       cs_stride_b, static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_out), B,
                       Hq, Hkv);
  };
  if (D == 64) args(qk_norm_rope_cs_kernel<64>);
  else args(qk_norm_rope_cs_kernel<128>);
  HELM_CHECK_LAUNCH("helm_qk_norm_rope_cs launch");
  return HELM_OK;
}

extern "C" int helm_rmsnorm(const void* x, const void* w, float eps, void* y, int M, int K,
                            void* stream) {
  HELM_CHECK_ARG(x && w && y, "helm_rmsnorm: null pointer");
  HELM_CHECK_ARG(M >= 1 && K >= 1, "helm_rmsnorm: sizes must be positive");
  const bool vec = K % 8 == 0 && K <= kRmsVec * 256 * 8 && helm::aligned16(x) && helm::aligned16(w) &&
                   helm::aligned16(y);
  if (vec)
    hipLaunchKernelGGL(rmsnorm_vec_kernel, dim3(M), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), eps,
                       static_cast<uint16_t*>(y), K);
  else
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(M), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), eps,
                       static_cast<uint16_t*>(y), K);
  HELM_CHECK_LAUNCH("helm_rmsnorm launch");
  return HELM_OK;
}

extern "C" int helm_silu_mul(const void* gate, const void* up, void* out, int64_t n, void* stream) {
  HELM_CHECK_ARG(gate && up && out, "helm_silu_mul: null pointer");
  HELM_CHECK_ARG(n >= 1, "helm_silu_mul: n must be positive");
  const bool vec = helm::aligned16(gate) && helm::aligned16(up) && helm::aligned16(out);
  const int64_t threads = vec ? (n + 7) / 8 : n;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(gate),
                     static_cast<const uint16_t*>(up), static_cast<uint16_t*>(out), n, vec);
  HELM_CHECK_LAUNCH("helm_silu_mul launch");
  return HELM_OK;
}

extern "C" int64_t helm_argmax_workspace_bytes(int M) {
  return M < 1 ? 0 : (int64_t)M * kArgmaxParts * (sizeof(float) + sizeof(int));
}

extern "C" int helm_argmax_f16_ws(const void* x, int64_t ldx, int M, int N, int64_t* out,
                                  void* workspace, int64_t workspace_bytes, void* stream) {
  HELM_CHECK_ARG(x && out && workspace, "helm_argmax_f16_ws: null pointer");
  HELM_CHECK_ARG(M >= 1 && N >= 1 && ldx >= N, "helm_argmax_f16_ws: bad sizes");
  HELM_CHECK_ARG(M <= 65535, "helm_argmax_f16_ws: at most 65535 rows");
  HELM_CHECK_ARG(workspace_bytes >= helm_argmax_workspace_bytes(M),
                 "helm_argmax_f16_ws: workspace smaller than helm_argmax_workspace_bytes(M)");
  HELM_CHECK_ARG((reinterpret_cast<uintptr_t>(workspace) & 3u) == 0,
                 "helm_argmax_f16_ws: workspace must be 4-byte aligned");
  const bool vec = ldx % 8 == 0 && helm::aligned16(x);
  float* pv = static_cast<float*>(workspace);
  int* pi = reinterpret_cast<int*>(pv + (int64_t)M * kArgmaxParts);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(argmax_part_kernel, dim3(kArgmaxParts, M), dim3(256), 0, s,
                     static_cast<const uint16_t*>(x), ldx, N, vec, pv, pi);
  hipLaunchKernelGGL(argmax_merge_kernel, dim3(M), dim3(64), 0, s, pv, pi, out);
  HELM_CHECK_LAUNCH("helm_argmax_f16_ws launch");
  return HELM_OK;
}

extern "C" int helm_argmax_f16(const void* x, int64_t ldx, int M, int N, int64_t* out, void* stream) {
  HELM_CHECK_ARG(x && out, "helm_argmax_f16: null pointer");
  HELM_CHECK_ARG(M >= 1 && N >= 1 && ldx >= N, "helm_argmax_f16: bad sizes");
  const bool vec = ldx % 8 == 0 && helm::aligned16(x);
  hipLaunchKernelGGL(argmax_f16_kernel, dim3(M), dim3(1024), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(x), ldx, N, vec, out);
  HELM_CHECK_LAUNCH("helm_argmax_f16 launch");
  return HELM_OK;
}
