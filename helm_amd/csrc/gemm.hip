// gemm.hip — INT8 weight-only prefill GEMM on MFMA.
//
// y[m,n] = fp16( scale[n] * sum_k x[m,k] * q[n,k] + bias[n] ), fp32 accumulate.
// Replaces the prefill branch of the reference's linear dispatch (fp32 F.linear on
// the CPU, helm/kernels/__init__.py:83-86; torch::linear, fp16_gemv.cpp:130-134).
//
// gfx950 design: a 256-thread workgroup computes a 128 x BN tile of y (BN = 32 TN);
// its four waves own 64 x 16TN quadrants made of 4 x TN v_mfma_f32_16x16x32_f16
// tiles (from TN = 4 on, 128 x 16TN halves of the tile over one k half of every
// K-step, so each int8 weight fragment is dequantised by one wave only).  Both operands of a K-step of 64 go straight from global memory into LDS
// (global_load_lds_dwordx4: one wave instruction moves 1 KiB, each lane picking the
// 16-byte chunk that belongs at its LDS position), x as fp16 and the weights as
// int8 (dequantised to fp16 after the LDS read, exact bias trick).  A ring of three
// LDS stages keeps two K-steps in flight while one is consumed; one barrier per
// K-step.  LDS rows are XOR-swizzled in 16-byte chunks so that the operand reads
// (16 rows at one k offset per instruction) hit every bank once.  The per-channel
// scale and bias are applied once in the epilogue.
#include <cstdlib>
#include <type_traits>

#include "helm_common.h"

namespace {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int BM = 128, BK = 64;
constexpr int kThreads = 256;
constexpr int kStages = 3;
constexpr int kABytes = BM * BK * 2;        // fp16 x tile of one stage (16 KiB)
constexpr int kAWaveCopies = kABytes / 1024 / 4;   // 1 KiB copies per wave (4)

// LDS swizzles (16-byte chunks): an operand read takes one chunk of 16 consecutive
// rows (one 256-byte pass of the 64 4-byte banks); these make the 16 chunks
// distinct in their bank positions.
__device__ __forceinline__ int aswz(int r) { return (r >> 1) & 7; }   // 128-byte rows
__device__ __forceinline__ int bswz(int n) { return (n >> 2) & 3; }   // 64-byte rows

template <int TN>
struct GemmCfg {
  static constexpr int BN = 32 * TN;
  static constexpr int kBBytes = BN * BK;                // int8 weight tile of one stage
  static constexpr int kStageBytes = kABytes + kBBytes;
  static constexpr int kBCopies = kBBytes / 1024;        // 1 KiB copies of the B tile
  static constexpr int kBWaveMax = (kBCopies + 3) / 4;   // most B copies of one wave
  static constexpr int kCopiesMin = kAWaveCopies + kBCopies / 4;   // fewest copies of any wave
};

// s_waitcnt vmcnt(N) only (expcnt / lgkmcnt fields at their maxima = no wait)
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// One wave's 1 KiB global -> LDS copy: lane l moves 16 bytes from `src` to LDS
// byte lds + 16 l.  Written as inline assembly so the compiler does not track it:
// its own bookkeeping would wait for every copy in flight (vmcnt(0)) before each
// LDS read, which serialises the ring; the kernel waits for its copies itself.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"   // m0 is named as clobbered on purpose
__device__ __forceinline__ void copy_to_lds(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(src)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Workgroup barrier after this wave's LDS reads have completed (the copies are
// waited for separately, by count).
__device__ __forceinline__ void lds_read_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// KSPLIT: the two waves that share B columns split each K-step (k half kh =
// wave / 2) instead of the rows, so every int8 B fragment is dequantised once;
// each wave then holds the partial sums of all 128 rows, and the pair adds them
// through LDS after the last step.
template <int TN, bool KSPLIT>
__global__ __launch_bounds__(kThreads, 2) void int8_gemm_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const int8_t* __restrict__ q, int64_t ldq,
    const uint16_t* __restrict__ scale, const uint16_t* __restrict__ bias, uint16_t* __restrict__ y,
    int64_t ldy, int M, int N, int K) {
  using C = GemmCfg<TN>;
  constexpr int kRing = kStages * C::kStageBytes;
  constexpr int kRed = KSPLIT ? 4 * 4 * TN * 64 * 16 : 0;   // partial tiles handed to the partner
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kRing > kRed ? kRing : kRed];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * C::BN;
  constexpr int RI = KSPLIT ? 8 : 4;     // 16-row tiles of one wave
  const int kh = wave >> 1;              // KSPLIT: k half of every K-step
  const int wm = KSPLIT ? 0 : (wave >> 1) * 64;
  const int wn = (wave & 1) * (16 * TN);
  const int nk = K / BK;

  // Copy sources.  A stage: row r (128 B) holds logical chunk g (8 halves) in slot
  // g ^ aswz(r).  B stage: row n (64 B) holds logical chunk g (16 int8) in slot
  // g ^ bswz(n).  Copy j moves LDS bytes [1024 j, 1024 j + 1024) of its
  // part; lane l fills 16 bytes at 1024 j + 16 l.  Rows past M / N read the last
  // row (their results are not stored).
  const uint16_t* asrc[kAWaveCopies];
#pragma unroll
  for (int i = 0; i < kAWaveCopies; ++i) {
    const int c = (wave * kAWaveCopies + i) * 64 + lane;
    const int r = c >> 3;
    const int g = (c & 7) ^ aswz(r);
    asrc[i] = x + (int64_t)min(m0 + r, M - 1) * ldx + g * 8;
  }
  const int8_t* bsrc[C::kBWaveMax];
#pragma unroll
  for (int i = 0; i < C::kBWaveMax; ++i) {
    const int j = min(wave + 4 * i, C::kBCopies - 1);
    const int c = j * 64 + lane;
    const int n = c >> 2;
    const int g = (c & 3) ^ bswz(n);
    bsrc[i] = q + (int64_t)min(n0 + n, N - 1) * ldq + g * 16;
  }
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t*)smem;
  auto copy = [&](int kb, int st) {
    const uint32_t base = lds0 + st * C::kStageBytes;
#pragma unroll
    for (int i = 0; i < kAWaveCopies; ++i)
      copy_to_lds(asrc[i] + kb * BK, base + (wave * kAWaveCopies + i) * 1024);
#pragma unroll
    for (int i = 0; i < C::kBWaveMax; ++i) {
      const int j = wave + 4 * i;
      if (j < C::kBCopies)   // uniform per wave
        copy_to_lds(bsrc[i] + kb * BK, base + kABytes + j * 1024);
    }
  };

  f4_t acc[RI][TN];
#pragma unroll
  for (int i = 0; i < RI; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

  // MFMA 16x16x32 operand layout: lane l supplies row (A) / column (B) l % 16 and
  // 8 k values; here lane group grp = l / 16 takes k 16 grp + 8 h .. + 8 for the
  // h-th MFMA of a K-step (the same k on both operands), so one 16-byte B read
  // serves both MFMAs.
  // KSPLIT: the wave takes k 32 kh .. 32 kh + 32 of each K-step, lane group grp
  // the 8 k from 32 kh + 8 grp: its B piece is half (grp & 1) of 16-byte chunk
  // 2 kh + grp / 2, so the 32 lanes of one 8-byte read pass (two lane groups)
  // fill both halves of 16 distinct chunks: every bank once.
  auto compute_ks = [&](int st) {
    const uint8_t* As = smem + st * C::kStageBytes;
    const uint8_t* Bs = As + kABytes;
    uint2 braw[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = wn + 16 * j + col;
      braw[j] = *reinterpret_cast<const uint2*>(Bs + n * 64 + (((2 * kh + (grp >> 1)) ^ bswz(n)) << 4) +
                                                (grp & 1) * 8);
    }
    h8_t af[RI];
#pragma unroll
    for (int i = 0; i < RI; ++i) {
      const int r = 16 * i + col;
      af[i] = *reinterpret_cast<const h8_t*>(As + r * 128 + (((4 * kh + grp) ^ aswz(r)) << 4));
    }
    h8_t bf[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      h2_t d[4];
      i8x4_to_h2x2(braw[j].x, d[0], d[1]);
      i8x4_to_h2x2(braw[j].y, d[2], d[3]);
      bf[j] = h8_t{d[0][0], d[0][1], d[1][0], d[1][1], d[2][0], d[2][1], d[3][0], d[3][1]};
    }
#pragma unroll
    for (int i = 0; i < RI; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
  };

  auto compute = [&](int st) {
    const uint8_t* As = smem + st * C::kStageBytes;
    const uint8_t* Bs = As + kABytes;
    uint4 braw[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = wn + 16 * j + col;
      braw[j] = *reinterpret_cast<const uint4*>(Bs + n * 64 + ((grp ^ bswz(n)) << 4));
    }
    h8_t af[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = wm + 16 * i + col;
        af[h][i] = *reinterpret_cast<const h8_t*>(As + r * 128 + (((2 * grp + h) ^ aswz(r)) << 4));
      }
    h8_t bf[TN][2];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      h2_t d[8];
      i8x4_to_h2x2(braw[j].x, d[0], d[1]);
      i8x4_to_h2x2(braw[j].y, d[2], d[3]);
      i8x4_to_h2x2(braw[j].z, d[4], d[5]);
      i8x4_to_h2x2(braw[j].w, d[6], d[7]);
      bf[j][0] = h8_t{d[0][0], d[0][1], d[1][0], d[1][1], d[2][0], d[2][1], d[3][0], d[3][1]};
      bf[j][1] = h8_t{d[4][0], d[4][1], d[5][0], d[5][1], d[6][0], d[6][1], d[7][0], d[7][1]};
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[h][i], bf[j][h], acc[i][j], 0, 0, 0);
  };

  // Three-stage ring: copies of steps kb + 1 and kb + 2 are in flight while kb is
  // consumed.  Before the barrier of step kb each wave waits until only its copies
  // of step kb + 1 may still be outstanding (vector memory operations retire in
  // order); after it, stage (kb + 2) % 3, last read in step kb - 1, is refilled.
  copy(0, 0);
  if (nk > 1) copy(1, 1);
  for (int kb = 0; kb < nk; ++kb) {
    if (kb + 1 < nk) wait_vm<C::kCopiesMin>();
    else wait_vm<0>();
    lds_read_barrier();
    if (kb + 2 < nk) copy(kb + 2, (kb + 2) % kStages);
    if constexpr (KSPLIT) compute_ks(kb % kStages);
    else compute(kb % kStages);
  }

  if constexpr (KSPLIT) {
    // wave (kh, side) keeps row tiles 4 kh .. 4 kh + 3 and hands the other four
    // to its partner (wave ^ 2) through LDS, one f4 per lane and tile
    // (the tile indices stay compile-time constants: registers are not indexable)
    __syncthreads();   // every wave is past its last LDS read of the ring
    f4_t* red = reinterpret_cast<f4_t*>(smem);
    auto finish = [&](auto keep_c) {
      constexpr int keep = decltype(keep_c)::value;
      constexpr int give = 4 - keep;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) red[((wave * 4 + i) * TN + j) * 64 + lane] = acc[give + i][j];
      __syncthreads();
      const int partner = wave ^ 2;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = n0 + wn + j * 16 + col;
        if (n >= N) continue;
        const float sc = h2f(scale[n]);
        const float bs = bias ? h2f(bias[n]) : 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f4_t o = red[((partner * 4 + i) * TN + j) * 64 + lane];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = m0 + (keep + i) * 16 + grp * 4 + r;
            if (m < M) y[(int64_t)m * ldy + n] = f2h((acc[keep + i][j][r] + o[r]) * sc + bs);
          }
        }
      }
    };
    if (kh == 0) finish(std::integral_constant<int, 0>{});
    else finish(std::integral_constant<int, 4>{});
    return;
  }

  // epilogue: C tile layout — lane l holds column l % 16, rows (l / 16) * 4 + r
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = n0 + wn + j * 16 + col;
    if (n >= N) continue;
    const float sc = h2f(scale[n]);
    const float bs = bias ? h2f(bias[n]) : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm + i * 16 + grp * 4 + r;
        if (m < M) y[(int64_t)m * ldy + n] = f2h(acc[i][j][r] * sc + bs);
      }
    }
  }
}

template <int TN>
void launch_gemm(const void* x, int64_t ldx, const int8_t* q, int64_t ldq, const void* scale,
                 const void* bias, void* y, int64_t ldy, int M, int N, int K, hipStream_t s) {
  dim3 grid((N + GemmCfg<TN>::BN - 1) / GemmCfg<TN>::BN, (M + BM - 1) / BM);
  // K split from TN = 4 on (14B shapes, same-run A/B: 5120->5120 127.4 -> 120.3 us,
  // 17408->5120 364.2 -> 336.5 us); with TN = 2 the grid holds one workgroup per
  // CU and the split measured 3% slower.  HELM_GEMM_KSPLIT=0 turns it off.
  static const int ks_env = [] { const char* v = getenv("HELM_GEMM_KSPLIT"); return v ? atoi(v) : 1; }();
  if (ks_env && TN >= 4)
    hipLaunchKernelGGL((int8_gemm_kernel<TN, true>), grid, dim3(kThreads), 0, s,
                       static_cast<const uint16_t*>(x), ldx, q, ldq, static_cast<const uint16_t*>(scale),
                       static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y), ldy, M, N, K);
  else
    hipLaunchKernelGGL((int8_gemm_kernel<TN, false>), grid, dim3(kThreads), 0, s,
                       static_cast<const uint16_t*>(x), ldx, q, ldq, static_cast<const uint16_t*>(scale),
                       static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y), ldy, M, N, K);
}

int env_tn() {
  const char* v = getenv("HELM_GEMM_TN");
  return v ? atoi(v) : 0;
}

// Tile width: the N extent per workgroup that fills the GPU's 2 x 256 workgroup
// slots most evenly (two workgroups fit per CU), wider tiles preferred on ties.
int pick_tn(int M, int N) {
  const int env = env_tn();
  if (env == 2 || env == 4 || env == 5) return env;
  const int mt = (M + BM - 1) / BM;
  int best = 4;
  double best_eff = -1.0;
  for (int tn : {5, 4, 2}) {
    const int tiles = mt * ((N + 32 * tn - 1) / (32 * tn));
    const int rounds = (tiles + 511) / 512;
    // useful work over slots spent, with the narrower tile's lower per-step rate
    const double fill = (double)M * N / ((double)rounds * 512 * BM * 32 * tn);
    const double eff = fill * (tn == 2 ? 0.8 : 1.0);
    if (eff > best_eff + 1e-9) {
      best_eff = eff;
      best = tn;
    }
  }
  return best;
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
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (pick_tn(M, N)) {
    case 2: launch_gemm<2>(x, ldx, q, ldq, scale, bias, y, ldy, M, N, K, s); break;
    case 5: launch_gemm<5>(x, ldx, q, ldq, scale, bias, y, ldy, M, N, K, s); break;
    default: launch_gemm<4>(x, ldx, q, ldq, scale, bias, y, ldy, M, N, K, s); break;
  }
  HELM_CHECK_LAUNCH("helm_int8_gemm launch");
  return HELM_OK;
}
