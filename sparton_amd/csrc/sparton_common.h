// Shared device helpers for the SpartonHead HIP kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/sparton.h"

namespace sparton {

typedef __bf16 bf16;
typedef _Float16 f16;

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(4))) _Float16 f16x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(4))) int32_t i32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

constexpr int kWave = 64;

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(f16 x) { return (float)x; }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) { return (bf16)x; }
template <> __device__ __forceinline__ f16 from_f32<f16>(float x) { return (f16)x; }

// log1p(x) for x >= 0 (inf and NaN pass through), in ~20 VALU instructions and within a few
// ulp (the library's log1pf, an extended-precision evaluation, takes ~110):
//   x < 1:  log1p(x) = 2 atanh(t), t = x / (2 + x) < 1/3, by its odd series
//           2t (1 + t^2/3 + t^4/5 + ... + t^14/15); the next term is below 2^-29 relative.
//           t carries the roundings of 2 + x and of the reciprocal (about 2.5 ulp).
//   x >= 1: ln(1 + x) = log2(1 + x) ln 2 with the hardware base-2 logarithm; rounding 1 + x
//           costs at most 2^-24 / ln 2 relative.
// Every forward kernel rounds reps through this function, so their outputs agree bitwise.
__device__ __forceinline__ float log1p_pos(float x) {
  const float t = x * __builtin_amdgcn_rcpf(2.0f + x);
  const float t2 = t * t;
  float p = 1.0f / 15.0f;
  p = __builtin_fmaf(p, t2, 1.0f / 13.0f);
  p = __builtin_fmaf(p, t2, 1.0f / 11.0f);
  p = __builtin_fmaf(p, t2, 1.0f / 9.0f);
  p = __builtin_fmaf(p, t2, 1.0f / 7.0f);
  p = __builtin_fmaf(p, t2, 1.0f / 5.0f);
  p = __builtin_fmaf(p, t2, 1.0f / 3.0f);
  p = __builtin_fmaf(p, t2, 1.0f);
  const float small = 2.0f * t * p;
  const float large = __builtin_amdgcn_logf(1.0f + x) * 0.69314718055994531f;
  return x < 1.0f ? small : large;
}

// ---- wave-wide reductions in a fixed order (reproducible), result in every lane ----------
// Within each 16-lane row by DPP (swap neighbours, swap pairs, half-row mirror, row mirror:
// every lane of the row ends with the same value, as a + b == b + a and max is symmetric),
// then the four row results read out in lane order. Every lane of the wave must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                                               0xF, 0xF, false));
}
__device__ __forceinline__ float lane_f(float x, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}
__device__ __forceinline__ float wave_sum(float x) {
  x += dpp_f<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp_f<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp_f<0x141>(x);  // row_half_mirror
  x += dpp_f<0x140>(x);  // row_mirror
  return (lane_f(x, 0) + lane_f(x, 16)) + (lane_f(x, 32) + lane_f(x, 48));
}
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp_f<0xB1>(x));
  x = fmaxf(x, dpp_f<0x4E>(x));
  x = fmaxf(x, dpp_f<0x141>(x));
  x = fmaxf(x, dpp_f<0x140>(x));
  return fmaxf(fmaxf(lane_f(x, 0), lane_f(x, 16)), fmaxf(lane_f(x, 32), lane_f(x, 48)));
}

// Mask element (b,s) as float, whatever its storage type. `mask_dtype` is uniform
// across the launch, so the switch is a uniform branch.
__device__ __forceinline__ float load_mask(const void* mask, int mask_dtype, int64_t off) {
  switch (mask_dtype) {
    case SPARTON_MASK_I64: return (float)((const int64_t*)mask)[off];
    case SPARTON_MASK_I32: return (float)((const int32_t*)mask)[off];
    case SPARTON_MASK_U8: return (float)((const uint8_t*)mask)[off];
    case SPARTON_MASK_F32: return ((const float*)mask)[off];
    case SPARTON_MASK_BF16: return (float)((const bf16*)mask)[off];
    default: return (float)((const f16*)mask)[off];
  }
}

// Mask values at N element offsets: every load is issued before any is converted, so
// they take one round trip together (a conversion right after each load would make
// each wait for the previous one).
template <typename M, int N>
__device__ __forceinline__ void mask_vals(const void* mask, const int64_t* off, float* out) {
  M raw[N];
#pragma unroll
  for (int i = 0; i < N; ++i) raw[i] = ((const M*)mask)[off[i]];
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = (float)raw[i];
}
template <int N>
__device__ __forceinline__ void load_mask_n(const void* mask, int mask_dtype, const int64_t* off,
                                            float* out) {
  switch (mask_dtype) {  // uniform
    case SPARTON_MASK_I64: mask_vals<int64_t, N>(mask, off, out); break;
    case SPARTON_MASK_I32: mask_vals<int32_t, N>(mask, off, out); break;
    case SPARTON_MASK_U8: mask_vals<uint8_t, N>(mask, off, out); break;
    case SPARTON_MASK_F32: mask_vals<float, N>(mask, off, out); break;
    case SPARTON_MASK_BF16: mask_vals<bf16, N>(mask, off, out); break;
    default: mask_vals<f16, N>(mask, off, out); break;
  }
}

// Element `off` of a float tensor of dtype `dt` (enum sparton_dtype) as float.
__device__ __forceinline__ float load_float(const void* p, int dt, int64_t off) {
  switch (dt) {
    case SPARTON_BF16: return (float)((const bf16*)p)[off];
    case SPARTON_F16: return (float)((const f16*)p)[off];
    default: return ((const float*)p)[off];
  }
}

// Four consecutive elements of a row as float (8-byte load for 16-bit types,
// 16-byte load for fp32). `p` must be aligned to 4 elements.
__device__ __forceinline__ f32x4 load4(const float* p) { return *(const f32x4*)p; }
__device__ __forceinline__ f32x4 load4(const bf16* p) {
  bf16x4 v = *(const bf16x4*)p;
  return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}
__device__ __forceinline__ f32x4 load4(const f16* p) {
  f16x4 v = *(const f16x4*)p;
  return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}

__host__ __device__ constexpr int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
__host__ __device__ constexpr int64_t round_up(int64_t a, int64_t b) { return cdiv(a, b) * b; }

}  // namespace sparton
