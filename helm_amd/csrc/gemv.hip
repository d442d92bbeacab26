// gemv.hip — decode GEMV (1 <= M <= 16 tokens) with int8 or fp16 weights.
//
// Counterpart of the reference's only native op, the AVX2/F16C fp16 GEMV
// (helm/kernels/fp16_gemv.cpp:45-157): one output row = one dot product over K
// with fp32 accumulation.  gfx950 design:
//   * a wave64 owns R output rows and walks the whole K; every lane streams one
//     16-byte chunk of each row per step (coalesced dwordx4, non-temporal), so a
//     wave reads 1 KiB of a row per step and U steps are issued before any math;
//   * the activations x (optionally RMS-normalised on the way in) are staged once
//     per workgroup in LDS and read back as packed fp16;
//   * int8 -> fp16 dequant in registers with a bias trick (exact), then
//     v_dot2_f32_f16 (2 MACs/lane, fp32 accumulate); no MFMA;
//   * cross-lane sums with a wave butterfly; the per-channel scale, bias and the
//     fused epilogues (residual add, SwiGLU) are applied once per output.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "helm_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kLdsBytes = 32768;  // x tile budget per workgroup

enum Epi { EPI_PLAIN = 0, EPI_RESIDUAL = 1, EPI_SWIGLU = 2 };

struct GemvArgs {
  const uint16_t* x;
  int64_t ldx;
  const uint16_t* norm_w;  // RMSNorm weight [K] or null
  float eps;
  const void* w;           // [N, K] int8 or fp16
  const void* w2;          // up-projection for SwiGLU
  int64_t ldw;             // row stride in elements
  const uint16_t* scale;   // [N] (int8 only)
  const uint16_t* scale2;
  const uint16_t* bias;    // [N] or null
  const uint16_t* residual;
  uint16_t* y;
  int64_t ldy;
  int M, N, K;
  int kt;                  // K elements staged per LDS pass
};

// Elements of x covered by one 16-byte weight chunk.
template <bool I8> struct Chunk { static constexpr int kElems = I8 ? 16 : 8; };

template <int MB, int R, bool I8, int EPI, bool NORM>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs a) {
  extern __shared__ uint4 smem_u4[];
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem_u4);
  __shared__ float red_s[kWaves][MB];
  __shared__ float rstd_s[MB];

  constexpr int NW = (EPI == EPI_SWIGLU) ? 2 : 1;
  constexpr int EPC = Chunk<I8>::kElems;
  constexpr int U = (16 / (NW * R)) < 1 ? 1 : ((16 / (NW * R)) > 4 ? 4 : (16 / (NW * R)));

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int M = a.M;
  const int n0 = (blockIdx.x * kWaves + wave) * R;

  // ---- optional RMSNorm statistics (per token, over the full K) ----
  if constexpr (NORM) {
    float ss[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m) ss[m] = 0.f;
    for (int k = tid * 8; k < a.K; k += kThreads * 8) {
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        if (m < M) {
          const uint4 v = *reinterpret_cast<const uint4*>(a.x + (int64_t)m * a.ldx + k);
          const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float f0 = lo_h(wd[j]), f1 = hi_h(wd[j]);
            ss[m] = fmaf(f0, f0, ss[m]);
            ss[m] = fmaf(f1, f1, ss[m]);
          }
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      const float t = wave_sum(ss[m]);
      if (lane == 0) red_s[wave][m] = t;
    }
    __syncthreads();
    if (tid < MB) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) t += red_s[w][tid];
      rstd_s[tid] = rsqrtf(t / (float)a.K + a.eps);
    }
    __syncthreads();
  }

  float acc[NW][R][MB];
#pragma unroll
  for (int w = 0; w < NW; ++w)
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < MB; ++m) acc[w][r][m] = 0.f;

  // Row pointers (rows past N are clamped to a valid row and discarded).
  const uint8_t* wrow[NW][R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int n = min(n0 + r, a.N - 1);
    const int64_t off = (int64_t)n * a.ldw * (I8 ? 1 : 2);
    wrow[0][r] = reinterpret_cast<const uint8_t*>(a.w) + off;
    if constexpr (NW == 2) wrow[1][r] = reinterpret_cast<const uint8_t*>(a.w2) + off;
  }

  for (int k0 = 0; k0 < a.K; k0 += a.kt) {
    const int klen = min(a.kt, a.K - k0);
    // ---- stage x[:, k0:k0+klen] in LDS (normalised when NORM) ----
    __syncthreads();
    const int vec_per_row = klen / 8;
    for (int idx = tid; idx < M * vec_per_row; idx += kThreads) {
      const int m = idx / vec_per_row;
      const int c = idx - m * vec_per_row;
      uint4 v = *reinterpret_cast<const uint4*>(a.x + (int64_t)m * a.ldx + k0 + c * 8);
      if constexpr (NORM) {
        const uint4 g = *reinterpret_cast<const uint4*>(a.norm_w + k0 + c * 8);
        const float rs = rstd_s[m];
        uint32_t xv[4] = {v.x, v.y, v.z, v.w};
        const uint32_t gv[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // fp16(w * fp16(x * rstd)), as Qwen3RMSNorm computes it in fp16 models
          const float a0 = h2f(f2h(lo_h(xv[j]) * rs));
          const float a1 = h2f(f2h(hi_h(xv[j]) * rs));
          xv[j] = pack_h2(lo_h(gv[j]) * a0, hi_h(gv[j]) * a1);
        }
        v = make_uint4(xv[0], xv[1], xv[2], xv[3]);
      }
      *reinterpret_cast<uint4*>(xs + m * klen + c * 8) = v;
    }
    __syncthreads();

    // ---- stream weight chunks of this tile ----
    const int nchunk = klen / EPC;
    const int64_t kbyte0 = (int64_t)k0 * (I8 ? 1 : 2);
    for (int c0 = 0; c0 < nchunk; c0 += 64 * U) {
      uint4 wv[U][NW][R];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u * 64 + lane;
        const bool ok = c < nchunk;
#pragma unroll
        for (int w = 0; w < NW; ++w)
#pragma unroll
          for (int r = 0; r < R; ++r) {
            if (ok) {
              wv[u][w][r] = ld_nt16((wrow[w][r] + kbyte0 + (int64_t)c * 16));
            } else {
              wv[u][w][r] = make_uint4(0u, 0u, 0u, 0u);
            }
          }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u * 64 + lane;
        if (c >= nchunk) break;
        if constexpr (I8) {
          // dequantise each row's 16 int8 into 8 packed-fp16 dwords
          h2_t dq[NW][R][8];
#pragma unroll
          for (int w = 0; w < NW; ++w)
#pragma unroll
            for (int r = 0; r < R; ++r) {
              i8x4_to_h2x2(wv[u][w][r].x, dq[w][r][0], dq[w][r][1]);
              i8x4_to_h2x2(wv[u][w][r].y, dq[w][r][2], dq[w][r][3]);
              i8x4_to_h2x2(wv[u][w][r].z, dq[w][r][4], dq[w][r][5]);
              i8x4_to_h2x2(wv[u][w][r].w, dq[w][r][6], dq[w][r][7]);
            }
#pragma unroll
          for (int m = 0; m < MB; ++m) {
            if (m < M) {
              const uint4* xp = reinterpret_cast<const uint4*>(xs + m * klen + c * 16);
              const uint4 xa = xp[0], xb = xp[1];
              const uint32_t xw[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
              for (int w = 0; w < NW; ++w)
#pragma unroll
                for (int r = 0; r < R; ++r) {
                  float s = acc[w][r][m];
#pragma unroll
                  for (int j = 0; j < 8; ++j) s = dot2h(dq[w][r][j], xw[j], s);
                  acc[w][r][m] = s;
                }
            }
          }
        } else {
#pragma unroll
          for (int m = 0; m < MB; ++m) {
            if (m < M) {
              const uint4 xa = *reinterpret_cast<const uint4*>(xs + m * klen + c * 8);
#pragma unroll
              for (int w = 0; w < NW; ++w)
#pragma unroll
                for (int r = 0; r < R; ++r) {
                  float s = acc[w][r][m];
                  s = dot2(wv[u][w][r].x, xa.x, s);
                  s = dot2(wv[u][w][r].y, xa.y, s);
                  s = dot2(wv[u][w][r].z, xa.z, s);
                  s = dot2(wv[u][w][r].w, xa.w, s);
                  acc[w][r][m] = s;
                }
            }
          }
        }
      }
    }
  }

  // ---- cross-lane sums and epilogue ----
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int n = n0 + r;
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      const float s0 = wave_sum(acc[0][r][m]);
      float s1 = 0.f;
      if constexpr (NW == 2) s1 = wave_sum(acc[1][r][m]);
      if (lane == ((r * MB + m) & 63) && m < M && n < a.N) {
        uint16_t out;
        if constexpr (EPI == EPI_SWIGLU) {
          const float g = h2f(f2h(s0 * h2f(a.scale[n])));
          const float u = h2f(f2h(s1 * h2f(a.scale2[n])));
          const float sg = h2f(f2h(g / (1.0f + expf(-g))));
          out = f2h(sg * u);
        } else {
          float v = I8 ? s0 * h2f(a.scale[n]) : s0;
          if (a.bias) v += h2f(a.bias[n]);
          if constexpr (EPI == EPI_RESIDUAL) {
            const float t = h2f(f2h(v));
            out = f2h(h2f(a.residual[(int64_t)m * a.ldy + n]) + t);
          } else {
            out = f2h(v);
          }
        }
        a.y[(int64_t)m * a.ldy + n] = out;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Streaming variant for the decode case where all of x fits in LDS.
//
// Work unit of a wave: R output rows (NW weight rows each) of a row tile; a
// workgroup walks tiles blockIdx.x, +gridDim.x, ... (grid sized so every
// workgroup gets the same number of tiles).  A wave's sequence of (tile, K-step)
// loads is software pipelined: the loads of the next step — also across the
// tile boundary — are issued before the current step's math, and the very first
// loads are issued before the RMSNorm statistics / x staging prologue, so HBM
// is busy from the first cycle to the last.
// ---------------------------------------------------------------------------
// Per-step buffer of one wave: weight chunks plus the epilogue operands of the
// step's rows (scale, up-scale, bias, residual), fetched together so that the
// epilogue never waits behind a later prefetch (vector loads retire in order).
template <int U, int NW, int R, int MB>
struct StreamBuf {
  uint4 w[U][NW][R];
  uint16_t sc[NW][R];
  uint16_t bias[R];
  uint16_t res[R][MB];
};

constexpr int kStreamXRegs = 16;   // most x / norm-weight uint4 per thread held through the prologue

// XR: x (and norm-weight) 16-byte vectors per thread in the prologue,
// ceil(M*K / (8*256)).  BIAS: a bias vector is read.  FULLK: K is a multiple of
// one step (64 lanes x U chunks), so no chunk of a step lies past K.  The load
// ring holds NB = 2 register buffers: one step in flight while one is consumed
// (deeper rings measured slower at every decode shape).
template <int MB, int R, bool I8, int EPI, bool NORM, int XR, bool BIAS, bool FULLK, int U>
__global__ __launch_bounds__(kThreads) void gemv_stream_kernel(GemvArgs a, int ntiles) {
  constexpr int NB = 2;
  extern __shared__ uint4 smem_u4[];
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem_u4);   // [M][K]
  __shared__ float red_s[kWaves][MB];
  __shared__ float rstd_s[MB];

  constexpr int NW = (EPI == EPI_SWIGLU) ? 2 : 1;
  constexpr int EPC = Chunk<I8>::kElems;
  using Buf = StreamBuf<U, NW, R, MB>;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int M = a.M;
  const int K = a.K;
  const int nchunk = K / EPC;
  const int steps = (nchunk + 64 * U - 1) / (64 * U);
  const int64_t row_bytes = a.ldw * (I8 ? 1 : 2);
  const uint8_t* wbase[2] = {reinterpret_cast<const uint8_t*>(a.w),
                             reinterpret_cast<const uint8_t*>(NW == 2 ? a.w2 : a.w)};
  const uint16_t* scp[2] = {I8 ? a.scale : a.x, (NW == 2) ? a.scale2 : (I8 ? a.scale : a.x)};
  // steps this workgroup walks: its tiles blockIdx.x, +gridDim.x, ... times K-steps
  const int my_tiles = blockIdx.x < ntiles ? (ntiles - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
  const int total = my_tiles * steps;

  // Loads are unconditional (addresses clamped in range) so the compiler can count
  // them: a consumer then waits only for its own buffer, not for the prefetch.
  // A step index past this workgroup's last one (the ring's prefetches at the
  // end) reads the first KiB of row 0 instead, shared by every wave, so the tail
  // costs no HBM traffic.
  auto load = [&](Buf& buf, int it) {
    const bool real = it < total;
    const int tile = blockIdx.x + (it / steps) * gridDim.x;
    const int ks = it - (it / steps) * steps;
    const int n0 = (tile * kWaves + wave) * R;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = min(real ? ks * 64 * U + u * 64 + lane : u * 64 + lane, nchunk - 1);
#pragma unroll
      for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int n = real ? min(n0 + r, a.N - 1) : 0;
          buf.w[u][w][r] = ld_nt16(wbase[w] + (int64_t)n * row_bytes + (int64_t)c * 16);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int n = real ? min(n0 + r, a.N - 1) : 0;
#pragma unroll
      for (int w = 0; w < NW; ++w) buf.sc[w][r] = scp[w][I8 ? n : 0];
      if constexpr (BIAS) buf.bias[r] = a.bias[n];
      if constexpr (EPI == EPI_RESIDUAL) {
#pragma unroll
        for (int m = 0; m < MB; ++m) buf.res[r][m] = a.residual[(int64_t)min(m, M - 1) * a.ldy + n];
      }
    }
  };

  float acc[NW][R][MB];
#pragma unroll
  for (int w = 0; w < NW; ++w)
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < MB; ++m) acc[w][r][m] = 0.f;

  auto compute = [&](const Buf& buf, int it) {
    const int ks = it - (it / steps) * steps;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c_raw = ks * 64 * U + u * 64 + lane;
      const bool ok = FULLK || c_raw < nchunk;   // past K: weights zeroed, x index clamped
      const int c = ok ? c_raw : 0;
      if constexpr (I8) {
        h2_t dq[NW][R][8];
#pragma unroll
        for (int w = 0; w < NW; ++w)
#pragma unroll
          for (int r = 0; r < R; ++r) {
            // past K the chunk is replaced by int8 zeros (bytes 0x00)
            const uint4 v = buf.w[u][w][r];
            i8x4_to_h2x2(ok ? v.x : 0u, dq[w][r][0], dq[w][r][1]);
            i8x4_to_h2x2(ok ? v.y : 0u, dq[w][r][2], dq[w][r][3]);
            i8x4_to_h2x2(ok ? v.z : 0u, dq[w][r][4], dq[w][r][5]);
            i8x4_to_h2x2(ok ? v.w : 0u, dq[w][r][6], dq[w][r][7]);
          }
#pragma unroll
        for (int m = 0; m < MB; ++m) {
          if (m < M) {
            const uint4* xp = reinterpret_cast<const uint4*>(xs + m * K + c * 16);
            const uint4 xa = xp[0], xb = xp[1];
            const uint32_t xw[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
            for (int w = 0; w < NW; ++w)
#pragma unroll
              for (int r = 0; r < R; ++r) {
                float s = acc[w][r][m];
#pragma unroll
                for (int j = 0; j < 8; ++j) s = dot2h(dq[w][r][j], xw[j], s);
                acc[w][r][m] = s;
              }
          }
        }
      } else {
#pragma unroll
        for (int m = 0; m < MB; ++m) {
          if (m < M) {
            const uint4 xa = *reinterpret_cast<const uint4*>(xs + m * K + c * 8);
#pragma unroll
            for (int w = 0; w < NW; ++w)
#pragma unroll
              for (int r = 0; r < R; ++r) {
                const uint4 v = buf.w[u][w][r];
                float s = acc[w][r][m];
                s = dot2(ok ? v.x : 0u, xa.x, s);
                s = dot2(ok ? v.y : 0u, xa.y, s);
                s = dot2(ok ? v.z : 0u, xa.z, s);
                s = dot2(ok ? v.w : 0u, xa.w, s);
                acc[w][r][m] = s;
              }
          }
        }
      }
    }
  };

  auto epilogue = [&](const Buf& buf, int it) {
    const int tile = blockIdx.x + (it / steps) * gridDim.x;
    const int n0 = (tile * kWaves + wave) * R;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int n = n0 + r;
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        const float s0 = wave_sum_uniform(acc[0][r][m]);
        float s1 = 0.f;
        if constexpr (NW == 2) s1 = wave_sum_uniform(acc[NW - 1][r][m]);
        if (lane == ((r * MB + m) & 63) && m < M && n < a.N) {
          uint16_t out;
          if constexpr (EPI == EPI_SWIGLU) {
            const float g = h2f(f2h(s0 * h2f(buf.sc[0][r])));
            const float u = h2f(f2h(s1 * h2f(buf.sc[NW - 1][r])));
            const float sg = h2f(f2h(g / (1.0f + expf(-g))));
            out = f2h(sg * u);
          } else {
            float v = I8 ? s0 * h2f(buf.sc[0][r]) : s0;
            if constexpr (BIAS) v += h2f(buf.bias[r]);
            if constexpr (EPI == EPI_RESIDUAL) {
              const float t = h2f(f2h(v));
              out = f2h(h2f(buf.res[r][m]) + t);
            } else {
              out = f2h(v);
            }
          }
          a.y[(int64_t)m * a.ldy + n] = out;
        }
#pragma unroll
        for (int w = 0; w < NW; ++w) acc[w][r][m] = 0.f;
      }
    }
  };

  // ---- prologue: x (and the norm weight) into registers, THEN the first weight
  // loads, so waiting for x never waits for weights ----
  const int vec_per_row = K / 8;
  const int n_vec = M * vec_per_row;
  uint4 xr[XR], gr[XR];
#pragma unroll
  for (int i = 0; i < XR; ++i) {
    const int idx = min(tid + i * kThreads, n_vec - 1);
    const int m = idx / vec_per_row;
    const int c = idx - m * vec_per_row;
    xr[i] = *reinterpret_cast<const uint4*>(a.x + (int64_t)m * a.ldx + c * 8);
    if constexpr (NORM) gr[i] = *reinterpret_cast<const uint4*>(a.norm_w + c * 8);
  }
  // keep the x loads ahead of the weight loads in issue order (in-order retirement
  // means the prologue then waits for x only)
  __builtin_amdgcn_sched_barrier(0);
  Buf buf[NB];
#pragma unroll
  for (int j = 0; j < NB - 1; ++j) load(buf[j], j);   // the ring's first NB-1 steps

  if constexpr (NORM) {
    float ss[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m) ss[m] = 0.f;
#pragma unroll
    for (int i = 0; i < XR; ++i) {   // branch-free: out-of-range entries add 0
      const int idx = tid + i * kThreads;
      const int m = min(idx, n_vec - 1) / vec_per_row;
      const uint32_t wd[4] = {xr[i].x, xr[i].y, xr[i].z, xr[i].w};
      float t = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float f0 = lo_h(wd[j]), f1 = hi_h(wd[j]);
        t = fmaf(f0, f0, t);
        t = fmaf(f1, f1, t);
      }
      t = idx < n_vec ? t : 0.f;
#pragma unroll
      for (int mm = 0; mm < MB; ++mm) ss[mm] += (mm == m) ? t : 0.f;
    }
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      const float t = wave_sum(ss[m]);
      if (lane == 0) red_s[wave][m] = t;
    }
    lds_barrier();
    if (tid < MB) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) t += red_s[w][tid];
      rstd_s[tid] = rsqrtf(t / (float)K + a.eps);
    }
    lds_barrier();
  }
  // Branch-free staging: out-of-range entries were loaded from the clamped index
  // n_vec - 1 and store that same value to the same place again.
#pragma unroll
  for (int i = 0; i < XR; ++i) {
    {
      const int idx = min(tid + i * kThreads, n_vec - 1);
      const int m = idx / vec_per_row;
      const int c = idx - m * vec_per_row;
      uint4 v = xr[i];
      if constexpr (NORM) {
        const float rs = rstd_s[m];
        uint32_t xv[4] = {v.x, v.y, v.z, v.w};
        const uint32_t gv[4] = {gr[i].x, gr[i].y, gr[i].z, gr[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // fp16(w * fp16(x * rstd)), as Qwen3RMSNorm computes it in fp16 models
          const float a0 = h2f(f2h(lo_h(xv[j]) * rs));
          const float a1 = h2f(f2h(hi_h(xv[j]) * rs));
          xv[j] = pack_h2(lo_h(gv[j]) * a0, hi_h(gv[j]) * a1);
        }
        v = make_uint4(xv[0], xv[1], xv[2], xv[3]);
      }
      *reinterpret_cast<uint4*>(xs + m * K + c * 8) = v;
    }
  }
  // LDS-only barriers in this prologue: the first weight step stays in flight, so
  // the second is requested as soon as the loop starts rather than after the
  // first has landed (one memory round trip less for waves of two or three steps)
  lds_barrier();

  // ---- pipelined walk: a ring of NB register buffers, NB-1 steps in flight while
  // one is consumed (unrolled by NB so every buffer index is a constant; no copy
  // of in-flight registers) ----
  for (int it = 0; it < total; it += NB) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int cur = it + j;
      load(buf[(j + NB - 1) % NB], cur + NB - 1);
      if (cur < total) {
        compute(buf[j], cur);
        if ((cur + 1) % steps == 0) epilogue(buf[j], cur);
      }
    }
  }
}

constexpr int kStreamLdsBytes = 65536;

int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v ? atoi(v) : dflt;
}

template <int MB, int R, bool I8, int EPI, bool NORM, bool BIAS, bool FULLK, int U>
void launch_stream_xr(const GemvArgs& a, hipStream_t s, int grid, int tiles, size_t lds, int xr) {
#define HELM_STREAM(XR_) \
  hipLaunchKernelGGL((gemv_stream_kernel<MB, R, I8, EPI, NORM, XR_, BIAS, FULLK, U>), dim3(grid), dim3(kThreads), lds, s, a, tiles)
  if constexpr (MB <= 2) {
    if (xr <= 2) { HELM_STREAM(2); return; }
    if (xr <= 4) { HELM_STREAM(4); return; }
  }
  if (xr <= 6) HELM_STREAM(6);
  else if (xr <= 12) HELM_STREAM(12);
  else HELM_STREAM(kStreamXRegs);   // K up to 32768 at one token (the Qwen3-32B down projection, K = 25600)
#undef HELM_STREAM
}

// R output rows per wave (each two weight rows for SwiGLU: gate and up); tiles of
// 4R rows; grid =
// ceil(tiles / per) with per = ceil(tiles / (256 * wgs_per_cu)) so that every
// workgroup walks the same number of tiles (to within one).  Measured at the
// Qwen3-8B decode shapes: matrices of >= 40 MB stream fastest with one workgroup
// per CU (gate/up + SwiGLU, down, the fp16 lm_head), smaller ones with two.
// HELM_GEMV_WGS_PER_CU overrides.
template <int MB, int R, bool I8, int EPI, bool NORM>
void launch_stream(const GemvArgs& a, hipStream_t s) {
  static const int wpc_env = env_int("HELM_GEMV_WGS_PER_CU", 0);
  const double wbytes = (double)a.N * a.K * (I8 ? 1 : 2) * (EPI == EPI_SWIGLU ? 2 : 1);
  // one row of a plain int8 matrix with K <= 4096 is a single step per wave: there
  // a 50 MB matrix (4096 -> 12288) measured 10% faster with two workgroups per CU
  const bool short_rows = I8 && EPI != EPI_SWIGLU && a.K <= 4096;
  const int wpc = wpc_env > 0 ? std::min(wpc_env, 8) : ((wbytes >= 40e6 && !short_rows) ? 1 : 2);
  const int tiles = (a.N + kWaves * R - 1) / (kWaves * R);
  const int slots = 256 * wpc;
  const int per = (tiles + slots - 1) / slots;
  const int grid = (tiles + per - 1) / per;
  const size_t lds = (size_t)a.M * a.K * 2;
  const int xr = (int)(((size_t)a.M * a.K / 8 + kThreads - 1) / kThreads);
  // a step is U chunks per lane: 4, or 5 where rows are whole steps of 5 but not
  // of 4 (K = 5120 int8 or fp16, 25600 int8: the Qwen3-14B / 32B widths), so no
  // step runs with idle lanes
  const int nch = a.K / Chunk<I8>::kElems;
  const bool u5 = nch % (64 * 5) == 0 && nch % (64 * 4) != 0;
  const bool fullk = nch % (64 * 4) == 0;
  auto go = [&](auto bias_tag) {
    constexpr bool B = decltype(bias_tag)::value;
    if constexpr (MB <= 2) {   // (3-4 tokens keep 4-chunk steps: fewer instances)
      if (u5) return launch_stream_xr<MB, R, I8, EPI, NORM, B, true, 5>(a, s, grid, tiles, lds, xr);
    }
    if (fullk) launch_stream_xr<MB, R, I8, EPI, NORM, B, true, 4>(a, s, grid, tiles, lds, xr);
    else launch_stream_xr<MB, R, I8, EPI, NORM, B, false, 4>(a, s, grid, tiles, lds, xr);
  };
  if (a.bias) go(std::true_type{});
  else go(std::false_type{});
}

template <int MB, int R, bool I8, int EPI, bool NORM>
void launch_one(const GemvArgs& a, int blocks, hipStream_t s) {
  const size_t lds = (size_t)a.M * a.kt * 2;
  hipLaunchKernelGGL((gemv_kernel<MB, R, I8, EPI, NORM>), dim3(blocks), dim3(kThreads), lds, s, a);
}

template <int MB, bool I8, int EPI, bool NORM>
void launch_r(const GemvArgs& a, hipStream_t s) {
  // Rows per wave: the largest R in {4,2,1} that still gives >= 512 workgroups
  // (two per CU on 256 CUs); small N falls back to one row per wave.
  int R = 1;
  for (int cand : {4, 2}) {
    if ((a.N + kWaves * cand - 1) / (kWaves * cand) >= 512) { R = cand; break; }
  }
  const int blocks = (a.N + kWaves * R - 1) / (kWaves * R);
  if (R == 4) launch_one<MB, 4, I8, EPI, NORM>(a, blocks, s);
  else if (R == 2) launch_one<MB, 2, I8, EPI, NORM>(a, blocks, s);
  else launch_one<MB, 1, I8, EPI, NORM>(a, blocks, s);
}

// Decode shapes whose activations fit in LDS (and in the prologue's registers)
// take the streaming kernel: one row per wave for 1-2 tokens, two rows per wave
// for 3-4 tokens (each x chunk read from LDS then feeds two rows; with the norm
// prologue or the SwiGLU epilogue 1.1-1.6x faster than the tiled kernel there).
bool stream_fits(const GemvArgs& a) {
  static const int no_stream = env_int("HELM_GEMV_NO_STREAM", 0);
  return (size_t)a.M * a.K * 2 + 1024 <= (size_t)kStreamLdsBytes &&
         (size_t)a.M * a.K <= (size_t)kStreamXRegs * kThreads * 8 && a.M <= 4 && !no_stream;
}

template <bool I8, int EPI, bool NORM>
void launch_m(const GemvArgs& a, hipStream_t s) {
  if (stream_fits(a)) {
    if (a.M == 1) launch_stream<1, 1, I8, EPI, NORM>(a, s);
    else if (a.M == 2) launch_stream<2, 1, I8, EPI, NORM>(a, s);
    else launch_stream<4, 2, I8, EPI, NORM>(a, s);
    return;
  }
  if (a.M <= 1) launch_r<1, I8, EPI, NORM>(a, s);
  else if (a.M <= 2) launch_r<2, I8, EPI, NORM>(a, s);
  else if (a.M <= 4) launch_r<4, I8, EPI, NORM>(a, s);
  else if (a.M <= 8) launch_r<8, I8, EPI, NORM>(a, s);
  else launch_r<16, I8, EPI, NORM>(a, s);
}

int choose_kt(int M, int K) {
  int kt = kLdsBytes / (2 * M);
  kt = (kt / 1024) * 1024;
  if (kt < 1024) kt = 1024;
  return std::min(kt, K);
}

int check_common(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* y,
                 int64_t ldy, int M, int N, int K, int elem_align, const char* fn) {
  std::string f(fn);
  HELM_CHECK_ARG(x && w && y, f + ": null pointer");
  HELM_CHECK_ARG(M >= 1 && N >= 1 && K >= 1, f + ": M, N, K must be positive");
  HELM_CHECK_SUPPORTED(M <= 16, f + ": decode GEMV handles M <= 16 (use helm_int8_gemm)");
  HELM_CHECK_ARG(ldx >= K && ldw >= K && ldy >= N, f + ": leading dimension too small");
  HELM_CHECK_SUPPORTED(K % elem_align == 0, f + ": K must be a multiple of " + std::to_string(elem_align));
  HELM_CHECK_SUPPORTED(ldw % elem_align == 0, f + ": weight row stride must be a multiple of " + std::to_string(elem_align));
  HELM_CHECK_SUPPORTED(ldx % 8 == 0, f + ": x row stride must be a multiple of 8");
  HELM_CHECK_SUPPORTED(helm::aligned16(x) && helm::aligned16(w), f + ": x and weights must be 16-byte aligned");
  return HELM_OK;
}

}  // namespace

// The int8 decode linear behind helm_int8_gemv, _fused and _ws: `part` null, or a
// workspace the 3-16 token kernel may use for its split form.
static int int8_gemv_impl(const void* x, int64_t ldx, const void* norm_w, float eps,
                          const int8_t* q, int64_t ldq, const void* scale, const void* bias,
                          const void* residual, void* y, int64_t ldy, int M, int N, int K,
                          float* part, int64_t part_bytes, void* stream) {
  int rc = check_common(x, ldx, q, ldq, y, ldy, M, N, K, 16, "helm_int8_gemv");
  if (rc) return rc;
  HELM_CHECK_ARG(scale != nullptr, "helm_int8_gemv: scale is null");
  if (norm_w) HELM_CHECK_SUPPORTED(helm::aligned16(norm_w), "helm_int8_gemv: norm weight must be 16-byte aligned");
  GemvArgs a{};
  a.x = static_cast<const uint16_t*>(x); a.ldx = ldx;
  a.norm_w = static_cast<const uint16_t*>(norm_w); a.eps = eps;
  a.w = q; a.w2 = nullptr; a.ldw = ldq;
  a.scale = static_cast<const uint16_t*>(scale); a.scale2 = nullptr;
  a.bias = static_cast<const uint16_t*>(bias);
  a.residual = static_cast<const uint16_t*>(residual);
  a.y = static_cast<uint16_t*>(y); a.ldy = ldy;
  a.M = M; a.N = N; a.K = K; a.kt = choose_kt(M, K);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // 3-16 tokens: the matrix-core small-M kernel where it takes the shape (with a
  // norm prologue at K = 4096; measured faster than the streaming kernel at 3-4
  // tokens too)
  if (helm::launch_int8_small_m(x, ldx, norm_w, eps, q, ldq, scale, bias, residual, y, ldy, M, N,
                                K, part, part_bytes, s)) {
    HELM_CHECK_LAUNCH("helm_int8_gemv launch");
    return HELM_OK;
  }
  if (residual) {
    if (norm_w) launch_m<true, EPI_RESIDUAL, true>(a, s);
    else launch_m<true, EPI_RESIDUAL, false>(a, s);
  } else {
    if (norm_w) launch_m<true, EPI_PLAIN, true>(a, s);
    else launch_m<true, EPI_PLAIN, false>(a, s);
  }
  HELM_CHECK_LAUNCH("helm_int8_gemv launch");
  return HELM_OK;
}

extern "C" int helm_int8_gemv_fused(const void* x, int64_t ldx, const void* norm_w, float eps,
                                    const int8_t* q, int64_t ldq, const void* scale,
                                    const void* bias, const void* residual, void* y, int64_t ldy,
                                    int M, int N, int K, void* stream) {
  return int8_gemv_impl(x, ldx, norm_w, eps, q, ldq, scale, bias, residual, y, ldy, M, N, K,
                        nullptr, 0, stream);
}

extern "C" int64_t helm_int8_gemv_workspace_bytes(int M, int N, int K) {
  return helm::int8_small_m_workspace_bytes(M, N, K);
}

extern "C" int helm_int8_gemv_ws(const void* x, int64_t ldx, const int8_t* q, int64_t ldq,
                                 const void* scale, const void* bias, const void* residual,
                                 void* y, int64_t ldy, int M, int N, int K, void* workspace,
                                 int64_t workspace_bytes, void* stream) {
  const int64_t need = helm::int8_small_m_workspace_bytes(M, N, K);
  if (need > 0) {
    HELM_CHECK_ARG(workspace != nullptr, "helm_int8_gemv_ws: workspace is null");
    HELM_CHECK_ARG(workspace_bytes >= need,
                   "helm_int8_gemv_ws: workspace smaller than helm_int8_gemv_workspace_bytes(M, N, K)");
    HELM_CHECK_ARG(helm::aligned16(workspace), "helm_int8_gemv_ws: workspace must be 16-byte aligned");
  }
  return int8_gemv_impl(x, ldx, nullptr, 0.f, q, ldq, scale, bias, residual, y, ldy, M, N, K,
                        need > 0 ? static_cast<float*>(workspace) : nullptr, workspace_bytes, stream);
}

extern "C" int helm_int8_gemv(const void* x, int64_t ldx, const int8_t* q, int64_t ldq,
                              const void* scale, const void* bias, void* y, int64_t ldy,
                              int M, int N, int K, void* stream) {
  return helm_int8_gemv_fused(x, ldx, nullptr, 0.f, q, ldq, scale, bias, nullptr, y, ldy, M, N, K,
                              stream);
}

extern "C" int helm_fp16_gemv(const void* x, int64_t ldx, const void* w, int64_t ldw,
                              const void* bias, void* y, int64_t ldy, int M, int N, int K,
                              void* stream) {
  int rc = check_common(x, ldx, w, ldw, y, ldy, M, N, K, 8, "helm_fp16_gemv");
  if (rc) return rc;
  GemvArgs a{};
  a.x = static_cast<const uint16_t*>(x); a.ldx = ldx;
  a.w = w; a.ldw = ldw;
  a.bias = static_cast<const uint16_t*>(bias);
  a.y = static_cast<uint16_t*>(y); a.ldy = ldy;
  a.M = M; a.N = N; a.K = K; a.kt = choose_kt(M, K);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (!helm::launch_fp16_small_m(x, ldx, nullptr, 0.f, w, ldw, bias, y, ldy, M, N, K, s))
    launch_m<false, EPI_PLAIN, false>(a, s);
  HELM_CHECK_LAUNCH("helm_fp16_gemv launch");
  return HELM_OK;
}

extern "C" int helm_fp16_gemv_rmsnorm(const void* x, int64_t ldx, const void* norm_w, float eps,
                                      const void* w, int64_t ldw, void* y, int64_t ldy, int M,
                                      int N, int K, void* stream) {
  int rc = check_common(x, ldx, w, ldw, y, ldy, M, N, K, 8, "helm_fp16_gemv_rmsnorm");
  if (rc) return rc;
  HELM_CHECK_ARG(norm_w != nullptr, "helm_fp16_gemv_rmsnorm: norm weight is null");
  HELM_CHECK_SUPPORTED(helm::aligned16(norm_w), "helm_fp16_gemv_rmsnorm: norm weight must be 16-byte aligned");
  GemvArgs a{};
  a.x = static_cast<const uint16_t*>(x); a.ldx = ldx;
  a.norm_w = static_cast<const uint16_t*>(norm_w); a.eps = eps;
  a.w = w; a.ldw = ldw;
  a.y = static_cast<uint16_t*>(y); a.ldy = ldy;
  a.M = M; a.N = N; a.K = K; a.kt = choose_kt(M, K);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (!helm::launch_fp16_small_m(x, ldx, norm_w, eps, w, ldw, nullptr, y, ldy, M, N, K, s))
    launch_m<false, EPI_PLAIN, true>(a, s);
  HELM_CHECK_LAUNCH("helm_fp16_gemv_rmsnorm launch");
  return HELM_OK;
}

extern "C" int helm_int8_gemv_swiglu(const void* x, int64_t ldx, const void* norm_w, float eps,
                                     const int8_t* q_gate, const void* s_gate, const int8_t* q_up,
                                     const void* s_up, int64_t ldq, void* y, int64_t ldy, int M,
                                     int N, int K, void* stream) {
  int rc = check_common(x, ldx, q_gate, ldq, y, ldy, M, N, K, 16, "helm_int8_gemv_swiglu");
  if (rc) return rc;
  HELM_CHECK_ARG(q_up && s_gate && s_up, "helm_int8_gemv_swiglu: null pointer");
  HELM_CHECK_SUPPORTED(helm::aligned16(q_up), "helm_int8_gemv_swiglu: up weights must be 16-byte aligned");
  if (norm_w) HELM_CHECK_SUPPORTED(helm::aligned16(norm_w), "helm_int8_gemv_swiglu: norm weight must be 16-byte aligned");
  GemvArgs a{};
  a.x = static_cast<const uint16_t*>(x); a.ldx = ldx;
  a.norm_w = static_cast<const uint16_t*>(norm_w); a.eps = eps;
  a.w = q_gate; a.w2 = q_up; a.ldw = ldq;
  a.scale = static_cast<const uint16_t*>(s_gate); a.scale2 = static_cast<const uint16_t*>(s_up);
  a.y = static_cast<uint16_t*>(y); a.ldy = ldy;
  a.M = M; a.N = N; a.K = K; a.kt = choose_kt(M, K);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // 3-16 tokens at K = 4096: norm, gate and up on the matrix cores in one launch
  if (helm::launch_int8_small_m_swiglu(x, ldx, norm_w, eps, q_gate, s_gate, q_up, s_up, ldq, y, ldy,
                                       M, N, K, s)) {
    HELM_CHECK_LAUNCH("helm_int8_gemv_swiglu launch");
    return HELM_OK;
  }
  if (norm_w) launch_m<true, EPI_SWIGLU, true>(a, s);
  else launch_m<true, EPI_SWIGLU, false>(a, s);
  HELM_CHECK_LAUNCH("helm_int8_gemv_swiglu launch");
  return HELM_OK;
}
