// helm_common.h — shared device helpers and host-side error plumbing for the
// gfx950 kernels of libhelm_mi355x.so.  Wave64 throughout.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/helm_mi355x.h"

// ---------------------------------------------------------------------------
// Host-side error reporting (thread-local last error, negative return codes)
// ---------------------------------------------------------------------------
namespace helm {

void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int hip_fail(hipError_t e, const char* what);

#define HELM_CHECK_ARG(cond, msg)                                   \
  do {                                                              \
    if (!(cond)) return ::helm::fail(HELM_ERR_INVALID_ARG, msg);    \
  } while (0)
#define HELM_CHECK_SUPPORTED(cond, msg)                             \
  do {                                                              \
    if (!(cond)) return ::helm::fail(HELM_ERR_UNSUPPORTED, msg);    \
  } while (0)
#define HELM_CHECK_LAUNCH(what)                                     \
  do {                                                              \
    hipError_t e_ = hipGetLastError();                              \
    if (e_ != hipSuccess) return ::helm::hip_fail(e_, what);        \
  } while (0)

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// INT8 linear for 3 <= M <= 16 tokens on the matrix cores (gemv_small_m.hip),
// with the RMSNorm prologue when norm_w is given; false when the shape is not one
// it takes.  `part` (null, or at least int8_small_m_workspace_bytes) holds the
// split form's partial sums.
bool launch_int8_small_m(const void* x, int64_t ldx, const void* norm_w, float eps,
                         const int8_t* q, int64_t ldq, const void* scale, const void* bias,
                         const void* residual, void* y, int64_t ldy, int M, int N, int K,
                         float* part, int64_t part_bytes, hipStream_t stream);
int64_t int8_small_m_workspace_bytes(int M, int N, int K);
// Gate / up projections with the SwiGLU epilogue, 3 <= M <= 16 tokens (RMSNorm
// prologue when norm_w is given), on the matrix cores; false when the shape is
// not one it takes.
bool launch_int8_small_m_swiglu(const void* x, int64_t ldx, const void* norm_w, float eps,
                                const int8_t* q_gate, const void* s_gate, const int8_t* q_up,
                                const void* s_up, int64_t ldq, void* y, int64_t ldy, int M,
                                int N, int K, hipStream_t stream);
// fp16-weight linear for 4 <= M <= 16 tokens on the matrix cores, with the
// RMSNorm prologue when norm_w is given; false when the shape is not one it takes.
bool launch_fp16_small_m(const void* x, int64_t ldx, const void* norm_w, float eps,
                         const void* w, int64_t ldw, const void* bias, void* y, int64_t ldy,
                         int M, int N, int K, hipStream_t stream);

}  // namespace helm

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte streaming load (non-temporal: data read once should not displace
// reusable lines in L2 / MALL).
__device__ __forceinline__ uint4 ld_nt16(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float h2f(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}
__device__ __forceinline__ uint16_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);  // round to nearest even
}
__device__ __forceinline__ float lo_h(uint32_t w) { return h2f((uint16_t)(w & 0xffffu)); }
__device__ __forceinline__ float hi_h(uint32_t w) { return h2f((uint16_t)(w >> 16)); }
__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
  return (uint32_t)f2h(a) | ((uint32_t)f2h(b) << 16);
}

// Four signed int8 in one dword -> two packed-fp16 dwords holding the exact
// integer values (q0,q1) and (q2,q3).  Bias trick: flip the sign bit so each byte
// is u = q + 128 in [1, 255]; the fp16 bit pattern 0x6400 | u is 1024 + u exactly
// (ulp(1024) = 1), and subtracting 1152 = 1024 + 128 leaves q exactly.
__device__ __forceinline__ void i8x4_to_h2x2(uint32_t w, h2_t& lo, h2_t& hi) {
  const uint32_t u = w ^ 0x80808080u;
  // v_perm_b32 selector bytes: 0..3 pick from `u`, 4..7 from 0x64646464.
  const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
  const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
  const h2_t off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  lo = __builtin_bit_cast(h2_t, a) + off;
  hi = __builtin_bit_cast(h2_t, b) + off;
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a), __builtin_bit_cast(h2_t, b), c, false);
}
__device__ __forceinline__ float dot2h(h2_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(a, __builtin_bit_cast(h2_t, b), c, false);
}

// Workgroup barrier that orders LDS only: the fences cover the local address
// space, so the wait before the barrier is for LDS traffic (lgkmcnt) and global
// loads in flight (prefetched weights or K/V) stay in flight across it, where
// __syncthreads would wait for them too.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Full-wave (64 lane) butterfly sum; every lane ends with the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
// Full-wave sum with DPP row operations (no LDS round trips): quad swaps and the
// two row mirrors leave each 16-lane row holding its row sum, and four lane reads
// add the rows.  The result is wave-uniform.  Every lane of the wave must be
// active (uniform control flow).
#define HELM_DPP_ADD(v, ctrl)                                                                    \
  ((v) + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (v)), \
                                                               (ctrl), 0xF, 0xF, true)))
__device__ __forceinline__ float wave_sum_uniform(float v) {
  v = HELM_DPP_ADD(v, 0xB1);   // quad_perm [1,0,3,2]
  v = HELM_DPP_ADD(v, 0x4E);   // quad_perm [2,3,0,1]
  v = HELM_DPP_ADD(v, 0x141);  // row_half_mirror
  v = HELM_DPP_ADD(v, 0x140);  // row_mirror
  const int iv = __builtin_bit_cast(int, v);
  return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16))) +
         (__builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48)));
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

constexpr float kLog2e = 1.4426950408889634f;
