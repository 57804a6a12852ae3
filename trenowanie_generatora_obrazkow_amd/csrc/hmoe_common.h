// Shared device helpers for the MoE SwiGLU kernels (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hmoe.h"

namespace hmoe {

constexpr int kWave = 64;

// Row-group tiles of the sorted rows (the layout is described in gemm_common.h): groups of 128 rows, 32-wide k
// slices of 8 KB.  Bytes needed for M sorted rows of width d over E experts: at most ceil(M / 128) + E groups.
constexpr int kTileGroupRows = 128;
constexpr int kTileK = 32;
inline int64_t tiles_groups_max(int64_t M, int64_t E) { return (M + kTileGroupRows - 1) / kTileGroupRows + E; }
inline int64_t tiles_bytes(int64_t M, int64_t E, int64_t d) {
  return tiles_groups_max(M, E) * ((d + kTileK - 1) / kTileK) * (int64_t)(kTileGroupRows * kTileK * 2);
}

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

// Two floats -> packed bf16 pair with the gfx950 conversion instruction (v_cvt_pk_bf16_f32, round to nearest even).
// Identical to pack_bf2 for every non-NaN input; a NaN becomes a quiet NaN that keeps its sign (pack_bf2 gives
// 0x7fc0).
typedef __bf16 bf16x2_hw __attribute__((ext_vector_type(2)));
typedef float f32x2_hw __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt_bf2(float lo, float hi) {
  const f32x2_hw v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_hw));
}

// Two floats -> packed fp16 pair, round to nearest even (the conversion torch applies to fp16 tensors).
typedef _Float16 f16x2_hw __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt_h2(float lo, float hi) {
  const f32x2_hw v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_hw));
}
__device__ __forceinline__ float h_lo(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu)); }
__device__ __forceinline__ float h_hi(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16)); }

// The 16-bit element type of activations, 16-bit weights, row scales and outputs: bf16 (F16 = false) or fp16.
// pack2 rounds two floats to a packed pair (nearest even), lo / hi widen the halves of a pair exactly.
template <bool F16>
struct Elt {
  __device__ __forceinline__ static uint32_t pack2(float lo, float hi) { return cvt_bf2(lo, hi); }
  __device__ __forceinline__ static float lo(uint32_t w) { return bf_lo(w); }
  __device__ __forceinline__ static float hi(uint32_t w) { return bf_hi(w); }
  __device__ __forceinline__ static float one(uint16_t b) { return bf2f(b); }
};
template <>
struct Elt<true> {
  __device__ __forceinline__ static uint32_t pack2(float lo, float hi) { return cvt_h2(lo, hi); }
  __device__ __forceinline__ static float lo(uint32_t w) { return h_lo(w); }
  __device__ __forceinline__ static float hi(uint32_t w) { return h_hi(w); }
  __device__ __forceinline__ static float one(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
};

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

// ---- cross-lane exchange without LDS: the value of lane (l ^ S) ----
// S = 1, 2: DPP quad permutations; S = 8: DPP rotation of each 16-lane row by 8 (= xor 8); S = 4: row rotations
// (row_ror:n reads lane (l - n) mod 16 of the row): lanes with bit 2 set read l - 4 (ror 4), the others l + 4
// (ror 12).  S = 16, 32 are served by the permlane swaps below.
template <int S>
__device__ __forceinline__ float lane_xor(float v) {
  static_assert(S == 1 || S == 2 || S == 4 || S == 8, "lane_xor: S in {1, 2, 4, 8}");
  const int b = __float_as_int(v);
  if constexpr (S == 1) return __int_as_float(__builtin_amdgcn_mov_dpp(b, 0xB1, 0xF, 0xF, false));  // [1,0,3,2]
  if constexpr (S == 2) return __int_as_float(__builtin_amdgcn_mov_dpp(b, 0x4E, 0xF, 0xF, false));  // [2,3,0,1]
  if constexpr (S == 8) return __int_as_float(__builtin_amdgcn_mov_dpp(b, 0x128, 0xF, 0xF, false)); // row_ror:8
  if constexpr (S == 4) {
    const int from_below = __builtin_amdgcn_mov_dpp(b, 0x124, 0xF, 0xF, false);  // row_ror:4:  lane l - 4
    const int from_above = __builtin_amdgcn_mov_dpp(b, 0x12C, 0xF, 0xF, false);  // row_ror:12: lane l + 4
    return __int_as_float((__lane_id() & 4) ? from_below : from_above);
  }
  return v;
}
template <int S>
__device__ __forceinline__ int lane_xor_i(int v) {
  return __float_as_int(lane_xor<S>(__int_as_float(v)));
}

// Pair exchange across 32 / 16 lanes (gfx950 v_permlane32_swap / v_permlane16_swap).  With lo = the value lanes
// whose bit S is clear keep and hi = the value lanes whose bit S is set keep, returns {own, partner}: lanes with bit S
// clear get (lo[l], lo[l ^ S]), lanes with it set get (hi[l ^ S], hi[l]).  With lo = hi = v this is (v[l], v[l ^ S])
// in some order, i.e. one xor-butterfly step.
template <int S>
__device__ __forceinline__ void lane_swap(float lo, float hi, float& a, float& b) {
  static_assert(S == 16 || S == 32, "lane_swap: S in {16, 32}");
  if constexpr (S == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
  }
}

// one xor-butterfly step of a sum: v[l] + v[l ^ S] (fp addition is commutative, so every lane pair gets the same sum)
template <int S>
__device__ __forceinline__ float bfly_add(float v) {
  if constexpr (S >= 16) {
    float a, b;
    lane_swap<S>(v, v, a, b);
    return __fadd_rn(a, b);
  } else {
    return __fadd_rn(v, lane_xor<S>(v));
  }
}
template <int S>
__device__ __forceinline__ float bfly_max(float v) {
  if constexpr (S >= 16) {
    float a, b;
    lane_swap<S>(v, v, a, b);
    return fmaxf(a, b);
  } else {
    return fmaxf(v, lane_xor<S>(v));
  }
}

// xor-butterfly sum over the 64 lanes (s = 32, 16, ..., 1); every lane ends with the same value.
__device__ __forceinline__ float wave_sum_butterfly(float v) {
  v = bfly_add<32>(v);
  v = bfly_add<16>(v);
  v = bfly_add<8>(v);
  v = bfly_add<4>(v);
  v = bfly_add<2>(v);
  v = bfly_add<1>(v);
  return v;
}
__device__ __forceinline__ float wave_max_butterfly(float v) {
  v = bfly_max<32>(v);
  v = bfly_max<16>(v);
  v = bfly_max<8>(v);
  v = bfly_max<4>(v);
  v = bfly_max<2>(v);
  v = bfly_max<1>(v);
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
