// gemv_small_m.hip — INT8 weight-only linear for 3 <= M <= 16 tokens.
//
// Same contract as the decode GEMV (y = fp16(s * (x . q^T) + bias), fp32
// accumulation; optional residual add), for a few tokens at once (small-batch
// or multi-token decode).  With M tokens every weight byte feeds M products, so
// at M = 16 the packed-fp16 dot products of the M <= 2 kernel would be VALU
// bound well below the HBM rate; here the products run on the matrix cores and
// the VALU only dequantises:
//   * a workgroup owns 16 output rows; its four waves split K into quarters
//     (eight waves measured slower);
//   * per 64-k step a lane loads 16 int8 of one row (a 16-row x 64-byte block per
//     wave, non-temporal), turns them into two fp16x8 A operands (exact bias
//     trick), and multiplies them with two fp16x8 B operands of x^T (16 tokens,
//     zero padded past M) read straight from L2: two v_mfma_f32_16x16x32_f16;
//   * a 4-deep ring of register buffers keeps 3 steps in flight per wave (deeper
//     rings measured slower; what limits this kernel is that the MFMA operand
//     layout gives each row only a 64-byte run per load instruction);
//   * the waves' 16x16 partial tiles are summed through LDS, then scale, bias,
//     residual, one rounding to fp16.
// The k order inside an MFMA is a permutation of the true k order (the same on
// both operands), which only changes the fp32 summation order.
#include "helm_common.h"

namespace {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int kRing = 4;

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
};

struct Step {
  uint4 w;        // 16 int8 of row `col`
  uint4 xa, xb;   // x[token col][k .. k+8), [k+8 .. k+16)
};

template <int W>
__global__ __launch_bounds__(W * 64) void int8_small_m_kernel(SmallMArgs a) {
  __shared__ __attribute__((aligned(16))) float s_c[W][64][4];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int row0 = blockIdx.x * 16;
  const int row = min(row0 + col, a.N - 1);           // rows past N: clamped, never stored
  const int tok = min(col, a.M - 1);                  // tokens past M: operand zeroed
  const bool tok_ok = col < a.M;
  const int kq = a.K / W;                             // this wave's K range
  const int k_begin = wave * kq;
  const int steps = kq / 64;

  const int8_t* wp = a.q + (int64_t)row * a.ldq + k_begin + grp * 16;
  const uint16_t* xp = a.x + (int64_t)tok * a.ldx + k_begin + grp * 16;

  auto load = [&](Step& st, int i) {
    const int s = min(i, steps - 1);   // past the end: re-read the last step (L2)
    st.w = ld_nt16(wp + (int64_t)s * 64);
    st.xa = *reinterpret_cast<const uint4*>(xp + s * 64);
    st.xb = *reinterpret_cast<const uint4*>(xp + s * 64 + 8);
  };

  f4_t acc = {0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const Step& st) {
    h2_t d[8];
    i8x4_to_h2x2(st.w.x, d[0], d[1]);
    i8x4_to_h2x2(st.w.y, d[2], d[3]);
    i8x4_to_h2x2(st.w.z, d[4], d[5]);
    i8x4_to_h2x2(st.w.w, d[6], d[7]);
    const h8_t a0 = {d[0][0], d[0][1], d[1][0], d[1][1], d[2][0], d[2][1], d[3][0], d[3][1]};
    const h8_t a1 = {d[4][0], d[4][1], d[5][0], d[5][1], d[6][0], d[6][1], d[7][0], d[7][1]};
    const uint4 zero = make_uint4(0u, 0u, 0u, 0u);
    const h8_t b0 = __builtin_bit_cast(h8_t, tok_ok ? st.xa : zero);
    const h8_t b1 = __builtin_bit_cast(h8_t, tok_ok ? st.xb : zero);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b0, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b1, acc, 0, 0, 0);
  };

  Step ring[kRing];
#pragma unroll
  for (int j = 0; j < kRing - 1; ++j) load(ring[j], j);
  for (int i = 0; i < steps; i += kRing) {
#pragma unroll
    for (int j = 0; j < kRing; ++j) {
      load(ring[(j + kRing - 1) % kRing], i + j + kRing - 1);
      if (i + j < steps) compute(ring[j]);
    }
  }

  // acc[r] = partial C[row (grp*4 + r)][token col] of this wave's K range
#pragma unroll
  for (int r = 0; r < 4; ++r) s_c[wave][lane][r] = acc[r];
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < W; ++w) v += s_c[w][lane][r];
      const int n = row0 + grp * 4 + r;
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

}  // namespace

namespace helm {

// Launches the small-M kernel when the shape suits it (3 <= M <= 16, K a
// multiple of 256, 16-byte aligned rows); returns false otherwise.
bool launch_int8_small_m(const void* x, int64_t ldx, const int8_t* q, int64_t ldq,
                         const void* scale, const void* bias, const void* residual, void* y,
                         int64_t ldy, int M, int N, int K, hipStream_t stream) {
  if (M < 3 || M > 16 || K % 256 != 0 || ldx % 8 != 0 || ldq % 16 != 0) return false;
  if (!aligned16(x) || !aligned16(q)) return false;
  SmallMArgs a{static_cast<const uint16_t*>(x), ldx, q, ldq, static_cast<const uint16_t*>(scale),
               static_cast<const uint16_t*>(bias), static_cast<const uint16_t*>(residual),
               static_cast<uint16_t*>(y), ldy, M, N, K};
  hipLaunchKernelGGL((int8_small_m_kernel<4>), dim3((N + 15) / 16), dim3(256), 0, stream, a);
  return true;
}

}  // namespace helm
