// gemm.hip — INT8 weight-only prefill GEMM on MFMA.
//
// y[m,n] = fp16( scale[n] * sum_k x[m,k] * q[n,k] + bias[n] ), fp32 accumulate.
// Replaces the prefill branch of the reference's linear dispatch (fp32 F.linear on
// the CPU, helm/kernels/__init__.py:83-86; torch::linear, fp16_gemv.cpp:130-134).
//
// gfx950 design: a 256-thread workgroup computes a 128x128 tile of y; its four
// waves own 64x64 quadrants made of 4x4 v_mfma_f32_16x16x32_f16 tiles.  Per
// K-step of 64, x (fp16) and q (int8, dequantised to fp16 on the way in — exact
// since |q| <= 127) are staged in LDS with padded rows; the next K-step's global
// loads are issued before the current step's MFMAs so HBM latency overlaps math.
// The per-channel scale and bias are applied once in the epilogue.
#include "helm_common.h"

namespace {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int kThreads = 256;
constexpr int LDA = BK + 8;  // padded LDS row (halves): 144 B keeps 16-byte reads spread over banks

__global__ __launch_bounds__(kThreads) void int8_gemm_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const int8_t* __restrict__ q, int64_t ldq,
    const uint16_t* __restrict__ scale, const uint16_t* __restrict__ bias, uint16_t* __restrict__ y,
    int64_t ldy, int M, int N, int K) {
  __shared__ __attribute__((aligned(16))) uint16_t As[BM * LDA];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[BN * LDA];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;
  const int wm = (wave >> 1) * 64;
  const int wn = (wave & 1) * 64;

  // global -> register staging assignments
  // A: 128 rows x 8 uint4 per row; thread handles idx = tid + 256*i, i < 4
  // B: 128 rows x 4 uint4 (int8) per row; thread handles idx = tid + 256*i, i < 2
  uint4 ra[4], rb[2];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + kThreads * i;
      const int r = idx >> 3, c = idx & 7;
      const int gm = m0 + r;
      ra[i] = gm < M ? *reinterpret_cast<const uint4*>(x + (int64_t)gm * ldx + k0 + c * 8)
                     : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int idx = tid + kThreads * i;
      const int r = idx >> 2, c = idx & 3;
      const int gn = n0 + r;
      rb[i] = gn < N ? ld_nt16((q + (int64_t)gn * ldq + k0 + c * 16))
                     : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  auto sstore = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + kThreads * i;
      const int r = idx >> 3, c = idx & 7;
      *reinterpret_cast<uint4*>(As + r * LDA + c * 8) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int idx = tid + kThreads * i;
      const int r = idx >> 2, c = idx & 3;
      const uint32_t w[4] = {rb[i].x, rb[i].y, rb[i].z, rb[i].w};
      h2_t d[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) i8x4_to_h2x2(w[j], d[2 * j], d[2 * j + 1]);
      uint4 lo, hi;
      lo.x = __builtin_bit_cast(uint32_t, d[0]); lo.y = __builtin_bit_cast(uint32_t, d[1]);
      lo.z = __builtin_bit_cast(uint32_t, d[2]); lo.w = __builtin_bit_cast(uint32_t, d[3]);
      hi.x = __builtin_bit_cast(uint32_t, d[4]); hi.y = __builtin_bit_cast(uint32_t, d[5]);
      hi.z = __builtin_bit_cast(uint32_t, d[6]); hi.w = __builtin_bit_cast(uint32_t, d[7]);
      uint4* dst = reinterpret_cast<uint4*>(Bs + r * LDA + c * 16);
      dst[0] = lo;
      dst[1] = hi;
    }
  };

  f4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

  // MFMA 16x16x32 operand layout: lane l supplies row (A) / column (B) l % 16 and
  // 8 consecutive k starting at (l / 16) * 8; the same k for A and B.
  const int fr = lane & 15;
  const int fk = (lane >> 4) * 8;

  gload(0);
  for (int k0 = 0; k0 < K; k0 += BK) {
    __syncthreads();
    sstore();
    __syncthreads();
    if (k0 + BK < K) gload(k0 + BK);
#pragma unroll
    for (int ks = 0; ks < BK; ks += 32) {
      h8_t af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = *reinterpret_cast<const h8_t*>(As + (wm + i * 16 + fr) * LDA + ks + fk);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bf[j] = *reinterpret_cast<const h8_t*>(Bs + (wn + j * 16 + fr) * LDA + ks + fk);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  }

  // epilogue: C tile layout — lane l holds column l % 16, rows (l / 16) * 4 + r
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = n0 + wn + j * 16 + (lane & 15);
    if (n >= N) continue;
    const float sc = h2f(scale[n]);
    const float bs = bias ? h2f(bias[n]) : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm + i * 16 + (lane >> 4) * 4 + r;
        if (m < M) y[(int64_t)m * ldy + n] = f2h(acc[i][j][r] * sc + bs);
      }
    }
  }
}

}  // namespace

extern "C" int helm_int8_gemm(const void* x, int64_t ldx, const int8_t* q, int64_t ldq,
                              const void* scale, const void* bias, void* y, int64_t ldy, int M,
                              int N, int K, void* stream) {
  HELM_CHECK_ARG(x && q && scale && y, "helm_int8_gemm: null pointer");
  HELM_CHECK_ARG(M >= 1 && N >= 1 && K >= 1, "helm_int8_gemm: M, N, K must be positive");
  HELM_CHECK_ARG(ldx >= K && ldq >= K && ldy >= N, "helm_int8_gemm: leading dimension too small");
  HELM_CHECK_SUPPORTED(K % BK == 0, "helm_int8_gemm: K must be a multiple of 64");
  HELM_CHECK_SUPPORTED(ldq % 16 == 0 && ldx % 8 == 0, "helm_int8_gemm: row strides must be multiples of 16 (q) and 8 (x)");
  HELM_CHECK_SUPPORTED(helm::aligned16(x) && helm::aligned16(q), "helm_int8_gemm: x and q must be 16-byte aligned");
  dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
  hipLaunchKernelGGL(int8_gemm_kernel, grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(x), ldx, q, ldq, static_cast<const uint16_t*>(scale),
                     static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y), ldy, M, N, K);
  HELM_CHECK_LAUNCH("helm_int8_gemm launch");
  return HELM_OK;
}
