// Shared device helpers for the MoE SwiGLU kernels (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hmoe.h"

namespace hmoe {

constexpr int kWave = 64;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf2f(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// float -> bf16, round to nearest even, NaN -> 0x7fc0 (the rule torch uses for c10::BFloat16).
__device__ __forceinline__ uint32_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) { return f2bf(lo) | (f2bf(hi) << 16); }

// exp for x <= 0 by Cody-Waite reduction (Cephes split of ln 2) + degree-7 Taylor polynomial (Horner, fma) +
// exponent scaling.  Bit-identical to the host restatement used by the tests: every step is an explicitly rounded
// IEEE operation.  Arguments below -87 return 0 (results above that are normal floats).
__device__ __forceinline__ float hexp(float x) {
  if (x < -87.0f) return 0.0f;
  if (x > 88.0f) return __builtin_inff();
  float n = __builtin_rintf(__fmul_rn(x, 0x1.715476p+0f));
  float r = __builtin_fmaf(-n, 0x1.63p-1f, x);
  r = __builtin_fmaf(-n, -0x1.bd0106p-13f, r);
  float p = 0x1.a01a02p-13f;
  p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
  p = __builtin_fmaf(p, r, 0x1.111112p-7f);
  p = __builtin_fmaf(p, r, 0x1.555556p-5f);
  p = __builtin_fmaf(p, r, 0x1.555556p-3f);
  p = __builtin_fmaf(p, r, 0x1.0p-1f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_ldexpf(p, (int)n);
}

// logistic sigmoid and SiLU with the hardware reciprocal (v_rcp_f32, ~1 ulp) instead of an IEEE division; the
// forward and backward epilogues use these same two functions, so the backward sees exactly the bf16(silu(g)) the
// forward stored.
__device__ __forceinline__ float sigmoid_f(float g) { return __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }
__device__ __forceinline__ float silu_f(float g) { return g * sigmoid_f(g); }

// xor-butterfly sum over the 64 lanes; every lane ends with the same value (fp add is commutative).
__device__ __forceinline__ float wave_sum_butterfly(float v) {
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) v = __fadd_rn(v, __shfl_xor(v, s, 64));
  return v;
}

__device__ __forceinline__ int wave_lane() { return __lane_id(); }

template <typename T>
__device__ __forceinline__ T ldg(const T* p) { return __builtin_nontemporal_load(p); }

// Read a device `counts` array of either int32 or int64 (the reference's torch.bincount gives int64).
__device__ __forceinline__ int64_t read_count(const void* counts, int is64, int e) {
  return is64 ? reinterpret_cast<const int64_t*>(counts)[e] : (int64_t) reinterpret_cast<const int32_t*>(counts)[e];
}

}  // namespace hmoe

#define HMOE_CHECK_LAUNCH()                                \
  do {                                                     \
    hipError_t _e = hipGetLastError();                     \
    if (_e != hipSuccess) return HMOE_ERR_LAUNCH;          \
  } while (0)
