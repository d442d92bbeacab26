// gemv_small_m.hip — INT8 weight-only linear for 3 <= M <= 16 tokens.
//
// Same contract as the decode GEMV (y = fp16(s * (x . q^T) + bias), fp32
// accumulation; optional residual add), for a few tokens at once (small-batch
// or multi-token decode).  With M tokens every weight byte feeds M products, so
// at M = 16 the packed-fp16 dot products of the M <= 2 kernel would be VALU
// bound well below the HBM rate; here the products run on the matrix cores and
// the VALU only dequantises:
//   * a workgroup owns 16 RT output rows (RT = 2 from 9 tokens on when N leaves
//     >= 256 such workgroups, so each x^T operand read feeds two row tiles); its
//     W waves (4, or 8 for long K) split K into slices;
//   * weights stream in units of 256 k per row: one load instruction covers 4
//     rows x 256 contiguous bytes, so a unit of 16 rows is four instructions and
//     two units are in flight per wave;
//   * each unit goes through the wave's own LDS region (rows padded to 272 bytes,
//     so the reads below are bank-conflict free) and is read back in the MFMA
//     operand layout: per 64-k step a lane takes 16 int8 of row `lane % 16`,
//     turns them into two fp16x8 A operands (exact bias trick) and multiplies them
//     with two fp16x8 B operands of x^T (16 tokens, token columns past M zeroed,
//     their loads masked off) read from L2: two v_mfma_f32_16x16x32_f16;
//   * the waves' 16x16 partial tiles are summed through LDS, then scale, bias,
//     residual, one rounding to fp16.
// The k order inside an MFMA is a permutation of the true k order (the same on
// both operands), which only changes the fp32 summation order.
#include <algorithm>
#include <cstdlib>

#include "helm_common.h"

namespace {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int kUnitK = 256;              // k per row of one unit
constexpr int kRowPitch = kUnitK + 16;    // LDS bytes per row (padding spreads banks)
constexpr int kUnitLds = 16 * kRowPitch;  // one unit of one wave in LDS

struct SmallMArgs {
  const uint16_t* x;
  int64_t ldx;
  const int8_t* q;
  int64_t ldq;
  const uint16_t* scale;
  const uint16_t* bias;
  const uint16_t* residual;
  uint16_t* y;
  int64_t ldy;
  int M, N, K;
  float* part;   // split form: fp32 partial sums [K slices][M][N]
  const int8_t* q2;          // SwiGLU form: up weights (q holds gate) ...
  const uint16_t* scale2;    // ... and their scales
  const uint16_t* norm_w;    // NORM: RMSNorm weight [K] ...
  float eps;                 // ... and epsilon
};

// One unit in registers: 4 RT weight chunks (rows 4t + lane/16, bytes
// 16*(lane%16) .. +16 of the unit) and the x operands of its four 64-k steps
// (shared by the RT row tiles).
template <int RT>
struct Unit {
  uint4 w[4 * RT];
  uint4 xa[4], xb[4];
};

// RT: 16-row tiles per workgroup (each x^T operand read from L2 feeds RT tiles).
template <int W, int RT>
__global__ __launch_bounds__(W * 64) void int8_small_m_kernel(SmallMArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t s_w[W][RT * kUnitLds];
  __shared__ __attribute__((aligned(16))) float s_c[W][RT][64][4];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int col = lane & 15;   // MFMA row (weights) / column (token) of this lane
  const int grp = lane >> 4;   // MFMA k-group of this lane
  const int row0 = blockIdx.x * 16 * RT;
  const bool tok_ok = col < a.M;
  const int kw = a.K / W;                  // this wave's K slice (a multiple of kUnitK)
  const int k_begin = wave * kw;
  const int units = kw / kUnitK;

  // Buffer loads: an offset outside the buffer returns zeros without touching
  // memory, which serves rows past N, token columns past M and the ring's loads
  // past this wave's last unit (the instruction stream stays unconditional, so
  // every wait covers exactly the loads it needs).
  constexpr uint32_t kOob = 0x80000000u;
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t*>(a.q), (short)0, (int)((int64_t)a.N * a.ldq), 0x00020000);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.x), (short)0, (int)(((int64_t)(a.M - 1) * a.ldx + a.K) * 2), 0x00020000);
  // load rows 4t + grp (t = 0..3) of the unit: bytes 16*col .. +16 of 256
  uint32_t woff[4 * RT];
#pragma unroll
  for (int t = 0; t < 4 * RT; ++t) {
    const int r = row0 + 4 * t + grp;
    woff[t] = r < a.N ? (uint32_t)((int64_t)r * a.ldq + k_begin + col * 16) : kOob;
  }
  const uint32_t xoff = tok_ok ? (uint32_t)(((int64_t)col * a.ldx + k_begin + grp * 16) * 2) : kOob;
  uint8_t* lds = s_w[wave];

  auto load = [&](Unit<RT>& u, int i) {
    const bool real = i < units;
#pragma unroll
    for (int t = 0; t < 4 * RT; ++t) {
      const uint32_t o = real && woff[t] != kOob ? woff[t] + (uint32_t)(i * kUnitK) : kOob;
      const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rq, o, 0, 2);   // non-temporal
      u.w[t] = make_uint4(v.x, v.y, v.z, v.w);
    }
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const uint32_t o = real && xoff != kOob ? xoff + (uint32_t)((i * kUnitK + st * 64) * 2) : kOob;
      const u32x4_t va = __builtin_amdgcn_raw_buffer_load_b128(rx, o, 0, 0);
      const u32x4_t vb = __builtin_amdgcn_raw_buffer_load_b128(rx, o == kOob ? kOob : o + 16, 0, 0);
      u.xa[st] = make_uint4(va.x, va.y, va.z, va.w);
      u.xb[st] = make_uint4(vb.x, vb.y, vb.z, vb.w);
    }
  };

  f4_t acc[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) acc[rt] = f4_t{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const Unit<RT>& u) {
    // registers -> LDS (row-major, padded), then back in the MFMA layout
#pragma unroll
    for (int t = 0; t < 4 * RT; ++t)
      *reinterpret_cast<uint4*>(lds + (4 * t + grp) * kRowPitch + col * 16) = u.w[t];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      uint4 wv[4];
#pragma unroll
      for (int st = 0; st < 4; ++st)
        wv[st] = *reinterpret_cast<const uint4*>(lds + (16 * rt + col) * kRowPitch + st * 64 + grp * 16);
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        h2_t d[8];
        i8x4_to_h2x2(wv[st].x, d[0], d[1]);
        i8x4_to_h2x2(wv[st].y, d[2], d[3]);
        i8x4_to_h2x2(wv[st].z, d[4], d[5]);
        i8x4_to_h2x2(wv[st].w, d[6], d[7]);
        const h8_t a0 = {d[0][0], d[0][1], d[1][0], d[1][1], d[2][0], d[2][1], d[3][0], d[3][1]};
        const h8_t a1 = {d[4][0], d[4][1], d[5][0], d[5][1], d[6][0], d[6][1], d[7][0], d[7][1]};
        acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, __builtin_bit_cast(h8_t, u.xa[st]), acc[rt], 0, 0, 0);
        acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, __builtin_bit_cast(h8_t, u.xb[st]), acc[rt], 0, 0, 0);
      }
    }
  };

  // two units in flight: the loads of unit i + 2 go out once unit i is in LDS
  Unit<RT> ua, ub;
  load(ua, 0);
  load(ub, 1);
  for (int i = 0; i < units; i += 2) {
    compute(ua);
    load(ua, i + 2);
    if (i + 1 < units) compute(ub);
    load(ub, i + 3);
  }

  // acc[rt][r] = partial C[row 16 rt + grp*4 + r][token col] of this wave's K slice
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int r = 0; r < 4; ++r) s_c[wave][rt][lane][r] = acc[rt][r];
  __syncthreads();
  if (wave < RT) {   // wave rt finishes row tile rt
    const int rt = wave;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < W; ++w) v += s_c[w][rt][lane][r];
      const int n = row0 + 16 * rt + grp * 4 + r;
      if (tok_ok && n < a.N) {
        float o = v * h2f(a.scale[n]);
        if (a.bias) o += h2f(a.bias[n]);
        const int64_t yi = (int64_t)col * a.ldy + n;
        if (a.residual) o = h2f(a.residual[yi]) + h2f(f2h(o));
        a.y[yi] = f2h(o);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Resident form (used for K = 4096, and K = 12288 up to 4 tokens; the ring form
// above serves every other shape).  Reading x^T from L2 for every 16-row tile
// costs more than the weights themselves (at 4096 -> 12288 with 16 tokens:
// 19.4 us with the operand loads from L2, 11.0 us with the same operands read
// from LDS; with 4 tokens 13.8 vs 10.5 us), so here x^T stays in LDS:
//   * the x rows (XR >= M token rows, row pitch 2 KS + 16 bytes so the 16 token
//     rows of one operand read fall in different banks; KS = all of K, or one
//     wave's slice of it, PRIV below) are loaded first, coalesced, and the
//     wave's weights after them: in-order returns make x arrive first; a shared
//     copy is published by one barrier that orders LDS only, so it waits for x
//     while every unit's weights stay in flight;
//   * the workgroup owns RT row tiles x all of K; the KQ waves of a row tile
//     split K, NU units of 256 k each, LA half units of a wave in flight (the
//     next one requested as soon as one is in LDS);
//   * weights travel in half units (16 rows x 128 k: two loads of 8 rows x 128
//     contiguous bytes) transposed through a 2.3 KB LDS region of the wave into
//     the MFMA operand layout; B operands (x^T, token columns past M zero) come
//     from the resident x rows;
//   * the KQ partial tiles of a row tile are summed through LDS.
// ---------------------------------------------------------------------------
// The shared-x forms publish the copy with lds_barrier (helm_common.h), which
// keeps the weight loads in flight (__syncthreads would wait for them: measured
// 2.3-3.8 us of the kernel at the Qwen3-8B shapes).

constexpr int kHalfK = 128;                     // k of one half unit
constexpr int kHalfPitch = kHalfK + 16;         // LDS bytes per weight row of a half unit
constexpr int kHalfLds = 16 * kHalfPitch;

// PRIV: each wave keeps only its own K slice of the x rows, in its own LDS
// region, so no workgroup barrier is needed (even a bare s_barrier here cost
// 2-2.5 us of a 13 us kernel at the Qwen3-8B shapes: the waves wait for the
// slowest one's x); with RT > 1 the RT waves of one slice each load their own
// copy.  Always with RT = 1 (no copy is duplicated); with RT = 3 up to 4 tokens,
// where the copies are small (4096 -> 12288 at M = 4: 13.5 -> 12.1 us); from 5
// tokens on RT = 3 shares one copy of all of K behind one LDS-only barrier (RT = 1
// with private slices measured 18.2 us against 15.1 at M = 16).
// SWI: the first RT/2 row tiles are gate rows, the last RT/2 the same rows of
// the up projection; the epilogue writes fp16(fp16(silu(g)) * u) (the SwiGLU of
// helm_int8_gemv_swiglu).
// NORM (shared x copy only): the x rows are RMS-normalised in LDS before use,
// xn = fp16(w * fp16(x * rsqrt(mean(x^2) + eps))) per token, the rounding steps of
// RMSNorm on fp16 activations.
template <int RT, int KQ, int NU, int XR, bool PRIV, int LA, bool PART, bool SWI = false,
          bool NORM = false>
__global__ __launch_bounds__(RT * KQ * 64) void int8_small_m_resident_kernel(SmallMArgs a) {
  constexpr int NW = RT * KQ;
  constexpr int NT = NW * 64;
  constexpr int K = KQ * NU * kUnitK;
  constexpr int KS = PRIV ? NU * kUnitK : K;      // k of the x rows one LDS region holds
  constexpr int kXPitch = 2 * KS + 16;
  constexpr int kXRegions = PRIV ? NW : 1;
  constexpr int kXChunks = XR * KS / 8;           // 16-byte pieces of one region's x rows
  constexpr int kXLoaders = PRIV ? 64 : NT;       // threads that load one region
  constexpr int kXPer = (kXChunks + kXLoaders - 1) / kXLoaders;
  constexpr int kHalves = 2 * NU;
  static_assert(NW * 64 * 4 * sizeof(float) <= NW * kHalfLds, "partials fit the weight staging");
  __shared__ __attribute__((aligned(16))) uint8_t s_x[kXRegions][XR * kXPitch];
  __shared__ __attribute__((aligned(16))) uint8_t s_w[NW][kHalfLds];
  __shared__ float s_rstd[NORM ? XR : 1];
  static_assert(!NORM || !PRIV, "the norm needs every k of a token in one LDS copy");

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int rt = wave / KQ;
  const int kq = wave - rt * KQ;
  constexpr int RTO = SWI ? RT / 2 : RT;          // row tiles of output rows
  static_assert(!SWI || (RT % 2 == 0 && !PART), "SwiGLU pairs gate and up tiles");
  const int row0 = blockIdx.x * 16 * RTO + (rt % RTO) * 16;
  const bool up_tile = SWI && rt >= RTO;
  const int M = a.M;

  // split form: workgroup column blockIdx.y takes k slice blockIdx.y * K .. + K
  const int ks = PART ? (int)blockIdx.y : 0;
  constexpr uint32_t kOob = 0x80000000u;
  const int8_t* qsrc = up_tile ? a.q2 : a.q;
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t*>(qsrc + (int64_t)ks * K), (short)0, (int)((int64_t)a.N * a.ldq), 0x00020000);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.x + (int64_t)ks * K), (short)0, (int)(((int64_t)(M - 1) * a.ldx + K) * 2), 0x00020000);
  const int kw0 = kq * NU * kUnitK;
  // x rows first: piece c is token c / (KS/8), k 8 (c % (KS/8)) .. +8 of the region
  // (all of K, or this wave's slice kw0 .. kw0 + KS)
  const int xt = PRIV ? lane : tid;
  const int xk0 = PRIV ? kw0 : 0;
  uint4 xr[kXPer];
#pragma unroll
  for (int i = 0; i < kXPer; ++i) {
    const int c = xt + i * kXLoaders;
    const int tok = c / (KS / 8);
    const uint32_t o = (c < kXChunks && tok < M)
        ? (uint32_t)(((int64_t)tok * a.ldx + xk0 + (c % (KS / 8)) * 8) * 2) : kOob;
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rx, o, 0, 0);
    xr[i] = make_uint4(v.x, v.y, v.z, v.w);
  }
  // NORM: the norm-weight pieces of the same k, also ahead of the weight loads
  uint4 nwr[NORM ? kXPer : 1];
  if constexpr (NORM) {
#pragma unroll
    for (int i = 0; i < kXPer; ++i) {
      const int c = xt + i * kXLoaders;
      nwr[i] = *reinterpret_cast<const uint4*>(a.norm_w + (c % (KS / 8)) * 8);
    }
  }
  // then the first LA half units of this wave: rows 8 j + lane / 8, bytes 16 (lane % 8) .. +16
  uint4 w[kHalves][2];
  auto issue = [&](int h) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int r = row0 + 8 * j + (lane >> 3);
      const uint32_t o = r < a.N ? (uint32_t)((int64_t)r * a.ldq + kw0 + h * kHalfK + (lane & 7) * 16) : kOob;
      const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rq, o, 0, 2);   // non-temporal
      w[h][j] = make_uint4(v.x, v.y, v.z, v.w);
    }
  };
  constexpr int kAhead = LA < kHalves ? LA : kHalves;
#pragma unroll
  for (int h = 0; h < kAhead; ++h) issue(h);
  __builtin_amdgcn_sched_barrier(0);
  uint8_t* xs = s_x[PRIV ? wave : 0];
#pragma unroll
  for (int i = 0; i < kXPer; ++i) {
    const int c = xt + i * kXLoaders;
    if (c < kXChunks)   // rows past M hold the zeros their loads returned
      *reinterpret_cast<uint4*>(xs + (c / (KS / 8)) * kXPitch + (c % (KS / 8)) * 16) = xr[i];
  }
  // a wave reads back its own LDS writes in order; a shared copy needs the barrier
  if constexpr (!PRIV) lds_barrier();
  if constexpr (NORM) {
    // per token: the waves sum x^2 over the LDS row, then every thread
    // normalises the pieces it loaded and writes them back in place
    // (all reads of a row issued together, eight independent accumulators: a
    // single fma chain over the row measured 2-4 us of latency before the first
    // product)
    constexpr int kRowIt = KS / 8 / 64;
    static_assert(KS % 512 == 0, "a row is whole 64-lane rounds of 16-byte pieces");
    for (int t = wave; t < M; t += NW) {
      uint4 v[kRowIt];
#pragma unroll
      for (int it = 0; it < kRowIt; ++it)
        v[it] = *reinterpret_cast<const uint4*>(xs + t * kXPitch + (it * 64 + lane) * 16);
      float acc8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int it = 0; it < kRowIt; ++it) {
        const uint32_t wd[4] = {v[it].x, v[it].y, v[it].z, v[it].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float f0 = lo_h(wd[j]), f1 = hi_h(wd[j]);
          acc8[2 * j] = fmaf(f0, f0, acc8[2 * j]);
          acc8[2 * j + 1] = fmaf(f1, f1, acc8[2 * j + 1]);
        }
      }
      float ss = ((acc8[0] + acc8[1]) + (acc8[2] + acc8[3])) + ((acc8[4] + acc8[5]) + (acc8[6] + acc8[7]));
      ss = wave_sum(ss);
      if (lane == 0) s_rstd[t] = rsqrtf(ss / (float)K + a.eps);
    }
    lds_barrier();
#pragma unroll
    for (int i = 0; i < kXPer; ++i) {
      const int c = xt + i * kXLoaders;
      const int tok = c / (KS / 8);
      if (c < kXChunks && tok < M) {
        const float rs = s_rstd[tok];
        const uint32_t xv[4] = {xr[i].x, xr[i].y, xr[i].z, xr[i].w};
        const uint32_t gv[4] = {nwr[i].x, nwr[i].y, nwr[i].z, nwr[i].w};
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float a0 = h2f(f2h(lo_h(xv[j]) * rs));
          const float a1 = h2f(f2h(hi_h(xv[j]) * rs));
          o[j] = pack_h2(lo_h(gv[j]) * a0, hi_h(gv[j]) * a1);
        }
        *reinterpret_cast<uint4*>(xs + tok * kXPitch + (c % (KS / 8)) * 16) =
            make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
    lds_barrier();
  }

  uint8_t* lds = s_w[wave];
  const bool tok_ok = col < M;
  const uint8_t* xb = xs + (tok_ok ? col : 0) * kXPitch + ((PRIV ? 0 : kw0) + grp * 16) * 2;
  f4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int h = 0; h < kHalves; ++h) {
    *reinterpret_cast<uint4*>(lds + (lane >> 3) * kHalfPitch + (lane & 7) * 16) = w[h][0];
    *reinterpret_cast<uint4*>(lds + (8 + (lane >> 3)) * kHalfPitch + (lane & 7) * 16) = w[h][1];
    if (h + kAhead < kHalves) {   // half h's registers are free: request half h + LA
      __builtin_amdgcn_sched_barrier(0);
      issue(h + kAhead);
      __builtin_amdgcn_sched_barrier(0);
    }
    uint4 wv[2];
#pragma unroll
    for (int st = 0; st < 2; ++st)
      wv[st] = *reinterpret_cast<const uint4*>(lds + col * kHalfPitch + st * 64 + grp * 16);
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const uint8_t* xp = xb + (h * kHalfK + st * 64) * 2;
      uint4 b0 = *reinterpret_cast<const uint4*>(xp);
      uint4 b1 = *reinterpret_cast<const uint4*>(xp + 16);
      if (!tok_ok) b0 = b1 = make_uint4(0u, 0u, 0u, 0u);   // token columns past M
      h2_t d[8];
      i8x4_to_h2x2(wv[st].x, d[0], d[1]);
      i8x4_to_h2x2(wv[st].y, d[2], d[3]);
      i8x4_to_h2x2(wv[st].z, d[4], d[5]);
      i8x4_to_h2x2(wv[st].w, d[6], d[7]);
      const h8_t a0 = {d[0][0], d[0][1], d[1][0], d[1][1], d[2][0], d[2][1], d[3][0], d[3][1]};
      const h8_t a1 = {d[4][0], d[4][1], d[5][0], d[5][1], d[6][0], d[6][1], d[7][0], d[7][1]};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, __builtin_bit_cast(h8_t, b0), acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, __builtin_bit_cast(h8_t, b1), acc, 0, 0, 0);
    }
  }

  // partial tiles through the (no longer used) weight staging
  __syncthreads();
  float (*s_c)[64][4] = reinterpret_cast<float (*)[64][4]>(&s_w[0][0]);
#pragma unroll
  for (int i = 0; i < 4; ++i) s_c[wave][lane][i] = acc[i];
  __syncthreads();
  if constexpr (SWI) {
    if (kq == 0 && !up_tile) {   // gate tile rt and up tile rt + RTO: the same rows
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float vg = 0.f, vu = 0.f;
#pragma unroll
        for (int q = 0; q < KQ; ++q) {
          vg += s_c[rt * KQ + q][lane][i];
          vu += s_c[(rt + RTO) * KQ + q][lane][i];
        }
        const int n = row0 + grp * 4 + i;
        if (tok_ok && n < a.N) {
          const float g = h2f(f2h(vg * h2f(a.scale[n])));
          const float u = h2f(f2h(vu * h2f(a.scale2[n])));
          const float sg = h2f(f2h(g / (1.0f + expf(-g))));
          a.y[(int64_t)col * a.ldy + n] = f2h(sg * u);
        }
      }
    }
    return;
  }
  if (kq == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = 0.f;
#pragma unroll
      for (int q = 0; q < KQ; ++q) v += s_c[rt * KQ + q][lane][i];
      const int n = row0 + grp * 4 + i;
      if constexpr (PART) {
        if (tok_ok && n < a.N) a.part[((int64_t)ks * M + col) * a.N + n] = v;
      } else if (tok_ok && n < a.N) {
        float o = v * h2f(a.scale[n]);
        if (a.bias) o += h2f(a.bias[n]);
        const int64_t yi = (int64_t)col * a.ldy + n;
        if (a.residual) o = h2f(a.residual[yi]) + h2f(f2h(o));
        a.y[yi] = f2h(o);
      }
    }
  }
}

// Split form, second pass: sums the K-slice partials of four consecutive outputs
// per thread and applies the one-pass forms' epilogue (scale, bias, residual,
// one rounding to fp16).
__global__ __launch_bounds__(256) void small_m_split_reduce_kernel(SmallMArgs a, int slices) {
  const int n4 = a.N / 4;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= a.M * n4) return;
  const int m = i / n4;
  const int n0 = (i - m * n4) * 4;
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < slices; ++s) {
    const float4 p = *reinterpret_cast<const float4*>(a.part + ((int64_t)s * a.M + m) * a.N + n0);
    v[0] += p.x; v[1] += p.y; v[2] += p.z; v[3] += p.w;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = n0 + j;
    float o = v[j] * h2f(a.scale[n]);
    if (a.bias) o += h2f(a.bias[n]);
    const int64_t yi = (int64_t)m * a.ldy + n;
    if (a.residual) o = h2f(a.residual[yi]) + h2f(f2h(o));
    a.y[yi] = f2h(o);
  }
}

// ---------------------------------------------------------------------------
// fp16 weights, 4-16 tokens (helm_fp16_gemv / helm_fp16_gemv_rmsnorm: the fp16
// lm_head of a batched decode step).  With fp16 weights every weight byte feeds
// M/2 products, so packed dot products would be VALU bound from 4 tokens on; the
// products run on the matrix cores instead:
//   * persistent: one workgroup per CU loads the x rows once into LDS (rows past
//     M zero; RMS-normalised in place for the fused form);
//   * each wave walks whole 16-row tiles over all of K (no cross-wave sum);
//     per 128-k half unit the 16 rows arrive as four loads of 4 rows x 256
//     contiguous bytes, two half units in flight, each transposed through the
//     wave's LDS region into the MFMA operand layout (lane: row lane % 16, k
//     32 st + 8 (lane / 16) .. +8) and multiplied with x^T on
//     v_mfma_f32_16x16x32_f16;
//   * fp32 accumulation, bias added in fp32, one rounding to fp16.
// ---------------------------------------------------------------------------
struct F16SmallMArgs {
  const uint16_t* x;
  int64_t ldx;
  const uint16_t* norm_w;
  float eps;
  const uint16_t* w;
  int64_t ldw;
  const uint16_t* bias;
  uint16_t* y;
  int64_t ldy;
  int M, N, K;
};

constexpr int kF16Pitch = 256 + 16;          // LDS bytes per staged weight row (128 k)
constexpr int kF16Stage = 16 * kF16Pitch;    // one half unit of one wave

__host__ __device__ constexpr int f16_small_m_lds(int XR, int NWV, int K) {
  return XR * (2 * K + 16) + NWV * kF16Stage;
}

template <int XR, int NWV, bool NORM>
__global__ __launch_bounds__(NWV * 64) void fp16_small_m_kernel(F16SmallMArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t f16_smem[];
  __shared__ float s_rstd[XR];
  constexpr int NT = NWV * 64;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int M = a.M, N = a.N, K = a.K;
  const int xpitch = 2 * K + 16;     // token rows 16 bytes apart in bank order
  const int cpr = K / 8;             // 16-byte pieces per x row
  uint8_t* xs = f16_smem;
  uint8_t* stg = f16_smem + XR * xpitch + wave * kF16Stage;

  // x rows into LDS, coalesced; rows M .. XR-1 zero
  for (int c = tid; c < XR * cpr; c += NT) {
    const int t = c / cpr;
    const int k8 = c - t * cpr;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (t < M) v = *reinterpret_cast<const uint4*>(a.x + (int64_t)t * a.ldx + k8 * 8);
    *reinterpret_cast<uint4*>(xs + t * xpitch + k8 * 16) = v;
  }
  __syncthreads();
  if constexpr (NORM) {
    // xn = fp16(w * fp16(x * rsqrt(mean(x^2) + eps))), in place
    for (int t = wave; t < M; t += NWV) {
      float ss = 0.f;
      for (int k8 = lane; k8 < cpr; k8 += 64) {
        const uint4 v = *reinterpret_cast<const uint4*>(xs + t * xpitch + k8 * 16);
        const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float f0 = lo_h(wd[j]), f1 = hi_h(wd[j]);
          ss = fmaf(f0, f0, ss);
          ss = fmaf(f1, f1, ss);
        }
      }
      ss = wave_sum(ss);
      if (lane == 0) s_rstd[t] = rsqrtf(ss / (float)K + a.eps);
    }
    __syncthreads();
    for (int c = tid; c < M * cpr; c += NT) {
      const int t = c / cpr;
      const int k8 = c - t * cpr;
      const float rs = s_rstd[t];
      uint4* p = reinterpret_cast<uint4*>(xs + t * xpitch + k8 * 16);
      const uint4 v = *p;
      const uint4 g = *reinterpret_cast<const uint4*>(a.norm_w + k8 * 8);
      const uint32_t xv[4] = {v.x, v.y, v.z, v.w};
      const uint32_t gv[4] = {g.x, g.y, g.z, g.w};
      uint32_t o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float a0 = h2f(f2h(lo_h(xv[j]) * rs));
        const float a1 = h2f(f2h(hi_h(xv[j]) * rs));
        o[j] = pack_h2(lo_h(gv[j]) * a0, hi_h(gv[j]) * a1);
      }
      *p = make_uint4(o[0], o[1], o[2], o[3]);
    }
    __syncthreads();
  }

  constexpr uint32_t kOob = 0x80000000u;
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.w), (short)0, (int)((int64_t)N * a.ldw * 2), 0x00020000);
  const int ntiles = (N + 15) / 16;
  const int halves = K / 128;
  const int gw = (int)blockIdx.x * NWV + wave;      // this wave's first tile
  const int nwv = (int)gridDim.x * NWV;
  const int my_tiles = gw < ntiles ? (ntiles - 1 - gw) / nwv + 1 : 0;
  const int total = my_tiles * halves;

  // load stream position (tile, half unit), two half units ahead of compute;
  // positions past the wave's last one load nothing (out-of-range offsets)
  int l_cnt = 0, l_h = 0, l_tile = gw;
  auto load = [&](uint4 (&b)[4]) {
    const bool real = l_cnt < total;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = l_tile * 16 + 4 * j + (lane >> 4);
      const uint32_t o = (real && r < N)
          ? (uint32_t)(((int64_t)r * a.ldw + l_h * 128 + (lane & 15) * 8) * 2) : kOob;
      const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rw, o, 0, 2);   // non-temporal
      b[j] = make_uint4(v.x, v.y, v.z, v.w);
    }
    ++l_cnt;
    if (++l_h == halves) {
      l_h = 0;
      l_tile += nwv;
    }
  };

  f4_t acc = {0.f, 0.f, 0.f, 0.f};
  int c_h = 0, c_tile = gw;
  auto process = [&](uint4 (&b)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<uint4*>(stg + (4 * j + (lane >> 4)) * kF16Pitch + (lane & 15) * 16) = b[j];
    __builtin_amdgcn_sched_barrier(0);
    load(b);   // b's registers are free once staged: the half unit two ahead
    __builtin_amdgcn_sched_barrier(0);
    // token columns past XR read row XR - 1 (zero, or a real row whose products
    // land in discarded columns): every read stays inside the x rows
    const uint8_t* xb = xs + min(col, XR - 1) * xpitch + (c_h * 128 + grp * 8) * 2;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const h8_t wa = *reinterpret_cast<const h8_t*>(stg + col * kF16Pitch + st * 64 + grp * 16);
      const h8_t xbv = *reinterpret_cast<const h8_t*>(xb + st * 64);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, xbv, acc, 0, 0, 0);
    }
    if (++c_h == halves) {   // tile done: rows 16 tile + 4 grp + i, token col
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = c_tile * 16 + grp * 4 + i;
        if (col < M && n < N) {
          float o = acc[i];
          if (a.bias) o += h2f(a.bias[n]);
          a.y[(int64_t)col * a.ldy + n] = f2h(o);
        }
      }
      acc = f4_t{0.f, 0.f, 0.f, 0.f};
      c_h = 0;
      c_tile += nwv;
    }
  };

  uint4 b0[4], b1[4];
  load(b0);
  load(b1);
  for (int it = 0; it < total; it += 2) {
    process(b0);
    if (it + 1 < total) process(b1);
  }
}

}  // namespace

namespace helm {

// Split form for long K (a multiple of kSplitK above 4096) at 8-16 tokens, whose
// x rows do not fit LDS: 4 row tiles x kSplitK of k per workgroup, the x slice
// shared in LDS, fp32 partials per k slice, then one reduce kernel.  12288 ->
// 4096: 16 tokens 18.4 -> 15.0 us, 12 tokens 16.4 -> 14.6, 8 tokens 14.9 -> 14.3
// against the ring form; at 5 tokens the reduce's launch makes it slower (14.0 ->
// 14.4), so fewer tokens keep the one-pass forms.
constexpr int kSplitK = 3072;

int64_t int8_small_m_workspace_bytes(int M, int N, int K) {
  if (M < 8 || M > 16 || N < 1 || N % 4 != 0 || K <= 4096 || K % kSplitK != 0) return 0;
  return (int64_t)(K / kSplitK) * M * N * (int64_t)sizeof(float);
}

// Launches the small-M kernel when the shape suits it (3 <= M <= 16, K a
// multiple of 1024, 16-byte aligned rows, operands below 2 GiB); returns false
// otherwise.  `part` (part_bytes >= int8_small_m_workspace_bytes, 16-byte
// aligned) enables the split form where it applies; null keeps the one-pass forms.
// With `norm_w` only K = 4096 is taken (a shared x copy with the norm prologue).
bool launch_int8_small_m(const void* x, int64_t ldx, const void* norm_w, float eps,
                         const int8_t* q, int64_t ldq, const void* scale, const void* bias,
                         const void* residual, void* y, int64_t ldy, int M, int N, int K,
                         float* part, int64_t part_bytes, hipStream_t stream) {
  if (M < 3 || M > 16 || K % 1024 != 0 || ldx % 8 != 0 || ldq % 16 != 0) return false;
  if (!aligned16(x) || !aligned16(q)) return false;
  if (norm_w && (K != 4096 || !aligned16(norm_w))) return false;
  // buffer offsets are 32-bit: weights and activations below 2 GiB
  if ((int64_t)N * ldq >= (1ll << 31) || ((int64_t)(M - 1) * ldx + K) * 2 >= (1ll << 31)) return false;
  SmallMArgs a{static_cast<const uint16_t*>(x), ldx, q, ldq, static_cast<const uint16_t*>(scale),
               static_cast<const uint16_t*>(bias), static_cast<const uint16_t*>(residual),
               static_cast<uint16_t*>(y), ldy, M, N, K, part, nullptr, nullptr,
               static_cast<const uint16_t*>(norm_w), eps};
  const int xr = M <= 4 ? 4 : M <= 8 ? 8 : M <= 12 ? 12 : 16;
  const int64_t ws = int8_small_m_workspace_bytes(M, N, K);
  if (!norm_w && ws > 0 && part && part_bytes >= ws && aligned16(part)) {
    // 4 row tiles (64 rows) x 3072 k per workgroup, 16 waves (4 per row tile,
    // each 768 k), the workgroup's x slice in LDS behind one LDS-only barrier
    const int slices = K / kSplitK;
    const dim3 grid((N + 63) / 64, slices);
#define HELM_SPLIT(XR_) \
    do { \
      if (grid.x * grid.y >= 256) \
        hipLaunchKernelGGL((int8_small_m_resident_kernel<4, 4, 3, XR_, false, 2, true>), grid, dim3(1024), 0, stream, a); \
      else \
        hipLaunchKernelGGL((int8_small_m_resident_kernel<4, 4, 3, XR_, false, 6, true>), grid, dim3(1024), 0, stream, a); \
    } while (0)
    if (xr == 8) HELM_SPLIT(8);
    else if (xr == 12) HELM_SPLIT(12);
    else HELM_SPLIT(16);
#undef HELM_SPLIT
    hipLaunchKernelGGL(small_m_split_reduce_kernel, dim3((M * (N / 4) + 255) / 256), dim3(256), 0, stream,
                       a, slices);
    return true;
  }
  // resident form for the K it is built for (x rows of all of K in LDS): K = 4096
  // with three row tiles per workgroup when that gives whole rounds of 256
  // workgroups, else one; K = 12288 with one row tile and at most 4 tokens (the
  // x of more tokens exceeds LDS).  HELM_SMALLM_RESIDENT=0 turns it off.
  static const int res_env = [] { const char* v = getenv("HELM_SMALLM_RESIDENT"); return v ? atoi(v) : 1; }();
  if (norm_w) {   // K = 4096: every form with one x copy per workgroup
    const int tiles = (N + 15) / 16;
    const bool rt3 = tiles % 3 == 0 && (tiles / 3) % 256 == 0;
#define HELM_RESIDENT_N(RT_, KQ_, NU_, XR_) \
    do { \
      const int blocks = rt3 && RT_ == 3 ? tiles / 3 : tiles; \
      if (blocks >= 256) \
        hipLaunchKernelGGL((int8_small_m_resident_kernel<RT_, KQ_, NU_, XR_, false, 2, false, false, true>), \
                           dim3(blocks), dim3(RT_ * KQ_ * 64), 0, stream, a); \
      else \
        hipLaunchKernelGGL((int8_small_m_resident_kernel<RT_, KQ_, NU_, XR_, false, 2 * NU_, false, false, true>), \
                           dim3(blocks), dim3(RT_ * KQ_ * 64), 0, stream, a); \
    } while (0)
    if (rt3) {   // whole rounds of 256 workgroups: two half units in flight
#define HELM_RT3_N(XR_) \
      hipLaunchKernelGGL((int8_small_m_resident_kernel<3, 4, 4, XR_, false, 2, false, false, true>), \
                         dim3(tiles / 3), dim3(768), 0, stream, a)
      if (xr == 4) HELM_RT3_N(4);
      else if (xr == 8) HELM_RT3_N(8);
      else if (xr == 12) HELM_RT3_N(12);
      else HELM_RT3_N(16);
#undef HELM_RT3_N
    } else if (xr <= 8 && tiles > 256 && tiles <= 512) {
      if (xr == 4) HELM_RESIDENT_N(1, 4, 4, 4);
      else HELM_RESIDENT_N(1, 4, 4, 8);
    } else {
      if (xr == 4) HELM_RESIDENT_N(1, 8, 2, 4);
      else if (xr == 8) HELM_RESIDENT_N(1, 8, 2, 8);
      else if (xr == 12) HELM_RESIDENT_N(1, 8, 2, 12);
      else HELM_RESIDENT_N(1, 8, 2, 16);
    }
#undef HELM_RESIDENT_N
    return true;
  }
  if (res_env) {
    const int tiles = (N + 15) / 16;
    const bool rt3 = tiles % 3 == 0 && (tiles / 3) % 256 == 0;
    // Weight loads in flight per wave: two half units when the grid fills the
    // 256 CUs (4096 -> 12288 at 16 tokens 15.1 -> 12.3 us, 12288 -> 4096 at 4
    // tokens 12.4 -> 11.4 us, 4096 -> 4096 7-9% faster than requesting a wave's
    // whole share at the launch's start; one half unit or three measured equal
    // or slower), all of them when the grid leaves CUs idle (4096 -> 1024: 64
    // workgroups, each CU then needs more bytes in flight).
#define HELM_RESIDENT(RT_, KQ_, NU_, XR_, PRIV_) \
    do { \
      const int blocks = rt3 && RT_ == 3 ? tiles / 3 : tiles; \
      if (blocks >= 256) \
        hipLaunchKernelGGL((int8_small_m_resident_kernel<RT_, KQ_, NU_, XR_, PRIV_, 2, false>), dim3(blocks), \
                           dim3(RT_ * KQ_ * 64), 0, stream, a); \
      else \
        hipLaunchKernelGGL((int8_small_m_resident_kernel<RT_, KQ_, NU_, XR_, PRIV_, 2 * NU_, false>), dim3(blocks), \
                           dim3(RT_ * KQ_ * 64), 0, stream, a); \
    } while (0)
    if (K == 4096 && rt3) {
      if (xr == 4) HELM_RESIDENT(3, 4, 4, 4, true);
      else if (xr == 8) HELM_RESIDENT(3, 4, 4, 8, false);
      else if (xr == 12) HELM_RESIDENT(3, 4, 4, 12, false);
      else HELM_RESIDENT(3, 4, 4, 16, false);
      return true;
    }
    if (K == 4096) {
      // 257-512 row tiles at 5-8 tokens: four waves sharing one x copy (75 KB of
      // LDS) so two workgroups fit a CU and the grid runs in one round; the
      // eight-wave private-x form (85 KB) leaves half the CUs idle in a second
      // round (4096 -> 6144 at 8 tokens 9.84 -> 8.0 us, 4096 -> 5120 9.56 -> 7.5 us)
      if (xr == 8 && tiles > 256 && tiles <= 512) {
        HELM_RESIDENT(1, 4, 4, 8, false);
        return true;
      }
      if (xr == 4) HELM_RESIDENT(1, 8, 2, 4, true);
      else if (xr == 8) HELM_RESIDENT(1, 8, 2, 8, true);
      else if (xr == 12) HELM_RESIDENT(1, 8, 2, 12, true);
      else HELM_RESIDENT(1, 8, 2, 16, true);
      return true;
    }
    if (K == 12288 && M <= 4) {
      HELM_RESIDENT(1, 8, 6, 4, true);
      return true;
    }
#undef HELM_RESIDENT
  }
  // four waves per K split measured fastest, eight once a wave's slice would
  // exceed 2048 k (Qwen3-8B down projection); HELM_SMALLM_WAVES overrides.
  // Two row tiles per workgroup (x^T read once for 32 rows) from 9 tokens on,
  // when that still leaves at least 256 workgroups (measured: 4096 -> 12288 at
  // M = 16 7% faster, at M = 4 4% slower); HELM_SMALLM_ROWTILES overrides.
  static const int w_env = [] { const char* v = getenv("HELM_SMALLM_WAVES"); return v ? atoi(v) : 0; }();
  static const int rt_env = [] { const char* v = getenv("HELM_SMALLM_ROWTILES"); return v ? atoi(v) : 0; }();
  int w = (K >= 8192 && K % (8 * kUnitK) == 0) ? 8 : 4;
  if ((w_env == 4 || w_env == 8 || w_env == 16) && K % (w_env * kUnitK) == 0) w = w_env;
  int rt = (M >= 9 && (N + 31) / 32 >= 256) ? 2 : 1;
  if (rt_env == 1 || rt_env == 2) rt = rt_env;
  if (w == 16) rt = 1;   // LDS: 16 waves hold one 16-row tile each
  const int tiles = (N + 16 * rt - 1) / (16 * rt);
  if (rt == 2) {
    if (w == 4) hipLaunchKernelGGL((int8_small_m_kernel<4, 2>), dim3(tiles), dim3(4 * 64), 0, stream, a);
    else hipLaunchKernelGGL((int8_small_m_kernel<8, 2>), dim3(tiles), dim3(8 * 64), 0, stream, a);
  } else {
    if (w == 4) hipLaunchKernelGGL((int8_small_m_kernel<4, 1>), dim3(tiles), dim3(4 * 64), 0, stream, a);
    else if (w == 8) hipLaunchKernelGGL((int8_small_m_kernel<8, 1>), dim3(tiles), dim3(8 * 64), 0, stream, a);
    else hipLaunchKernelGGL((int8_small_m_kernel<16, 1>), dim3(tiles), dim3(16 * 64), 0, stream, a);
  }
  return true;
}

// fp16-weight linear for 4 <= M <= 16 on the matrix cores; false when the shape
// is not one it takes (K % 128 != 0, x rows beyond LDS, weights above 2 GiB,
// unaligned operands).  Qwen3-8B lm_head (151936 x 4096, fused norm): 8 tokens
// 386 -> 231 us, 16 tokens 882 -> 244 us, 4 tokens 249 -> 231 us against the
// tiled / streaming dot-product kernels; at 3 tokens the streaming kernel stays
// (216-226 against 233 us).
bool launch_fp16_small_m(const void* x, int64_t ldx, const void* norm_w, float eps,
                         const void* w, int64_t ldw, const void* bias, void* y, int64_t ldy,
                         int M, int N, int K, hipStream_t stream) {
  if (M < 4 || M > 16 || K % 128 != 0 || ldx % 8 != 0 || ldw % 8 != 0) return false;
  if (!aligned16(x) || !aligned16(w) || (norm_w && !aligned16(norm_w))) return false;
  if ((int64_t)N * ldw * 2 >= (1ll << 31)) return false;
  constexpr int kLdsMax = 160 * 1024;
  const int xr = M <= 4 ? 4 : M <= 8 ? 8 : M <= 12 ? 12 : 16;
  const int nwv = f16_small_m_lds(xr, 8, K) <= kLdsMax ? 8 : 4;
  const int lds = f16_small_m_lds(xr, nwv, K);
  if (lds > kLdsMax) return false;
  F16SmallMArgs a{static_cast<const uint16_t*>(x), ldx, static_cast<const uint16_t*>(norm_w), eps,
                  static_cast<const uint16_t*>(w), ldw, static_cast<const uint16_t*>(bias),
                  static_cast<uint16_t*>(y), ldy, M, N, K};
  const int ntiles = (N + 15) / 16;
  const int grid = std::min(256, (ntiles + nwv - 1) / nwv);
#define HELM_F16SM(XR_, NWV_)                                                                    \
  do {                                                                                           \
    if (norm_w)                                                                                  \
      hipLaunchKernelGGL((fp16_small_m_kernel<XR_, NWV_, true>), dim3(grid), dim3(NWV_ * 64), lds, \
                         stream, a);                                                             \
    else                                                                                         \
      hipLaunchKernelGGL((fp16_small_m_kernel<XR_, NWV_, false>), dim3(grid), dim3(NWV_ * 64), lds, \
                         stream, a);                                                             \
  } while (0)
  if (nwv == 8) {
    if (xr == 4) HELM_F16SM(4, 8);
    else if (xr == 8) HELM_F16SM(8, 8);
    else if (xr == 12) HELM_F16SM(12, 8);
    else HELM_F16SM(16, 8);
  } else {
    if (xr == 4) HELM_F16SM(4, 4);
    else if (xr == 8) HELM_F16SM(8, 4);
    else if (xr == 12) HELM_F16SM(12, 4);
    else HELM_F16SM(16, 4);
  }
#undef HELM_F16SM
  return true;
}

// Gate / up projections with the SwiGLU epilogue for 3 <= M <= 16 (K = 4096, with
// the RMSNorm prologue when norm_w is given): one launch instead of a norm, two
// GEMVs and a SwiGLU kernel.  A
// workgroup takes 3 gate row tiles and the same 3 up row tiles (12 waves, two
// per tile splitting K) with one x copy in LDS; false when the shape is not one
// it takes.
bool launch_int8_small_m_swiglu(const void* x, int64_t ldx, const void* norm_w, float eps,
                                const int8_t* q_gate, const void* s_gate, const int8_t* q_up,
                                const void* s_up, int64_t ldq, void* y, int64_t ldy, int M,
                                int N, int K, hipStream_t stream) {
  if (M < 3 || M > 16 || K != 4096 || ldx % 8 != 0 || ldq % 16 != 0) return false;
  if (!aligned16(x) || !aligned16(q_gate) || !aligned16(q_up)) return false;
  if (norm_w && !aligned16(norm_w)) return false;
  if ((int64_t)N * ldq >= (1ll << 31) || ((int64_t)(M - 1) * ldx + K) * 2 >= (1ll << 31)) return false;
  SmallMArgs a{static_cast<const uint16_t*>(x), ldx, q_gate, ldq, static_cast<const uint16_t*>(s_gate),
               nullptr, nullptr, static_cast<uint16_t*>(y), ldy, M, N, K, nullptr, q_up,
               static_cast<const uint16_t*>(s_up), static_cast<const uint16_t*>(norm_w), eps};
  const int blocks = (N + 47) / 48;
  const int xr = M <= 4 ? 4 : M <= 8 ? 8 : M <= 12 ? 12 : 16;
  // two half units in flight per wave when the grid fills the CUs, four below
  // (more would spill at 768 threads per workgroup)
#define HELM_SWI1(XR_, NORM_)                                                                       \
  do {                                                                                              \
    if (blocks >= 256)                                                                              \
      hipLaunchKernelGGL((int8_small_m_resident_kernel<6, 2, 8, XR_, false, 2, false, true, NORM_>), \
                         dim3(blocks), dim3(768), 0, stream, a);                                    \
    else                                                                                            \
      hipLaunchKernelGGL((int8_small_m_resident_kernel<6, 2, 8, XR_, false, 4, false, true, NORM_>), \
                         dim3(blocks), dim3(768), 0, stream, a);                                    \
  } while (0)
#define HELM_SWI(XR_)                 \
  do {                                \
    if (norm_w) HELM_SWI1(XR_, true); \
    else HELM_SWI1(XR_, false);       \
  } while (0)
  if (xr == 4) HELM_SWI(4);
  else if (xr == 8) HELM_SWI(8);
  else if (xr == 12) HELM_SWI(12);
  else HELM_SWI(16);
#undef HELM_SWI
#undef HELM_SWI1
  return true;
}

}  // namespace helm
