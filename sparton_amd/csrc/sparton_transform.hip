// The MLM transform that produces the head's input, on gfx950:
//     H = LayerNorm(gelu(X W^T + b_d)) * gamma + beta        (per row over D)
// BERT's cls.predictions.transform and RoBERTa's lm_head dense/gelu/layer_norm
// (reference training/model.py:14-40); gelu is the exact erf form.
//
// The two D x D GEMMs of the forward and backward are plain library GEMMs (hipBLASLt,
// called by the Python op on the caller's stream). This file holds what fuses around them:
//   forward epilogue  Z (= X W^T) -> u = gelu(Z + b_d) -> LayerNorm -> H, and the row's
//                     mean and 1/std for the backward;
//   backward epilogue dH -> dZ = d/dZ through LayerNorm and gelu (recomputing u from Z),
//                     plus per-block column partial sums of dH * xhat, dH and dZ;
//   column reduction  those partials summed in block order into d gamma, d beta, d b_d.
// One wave per row; lane l holds elements 256 p + 4 l .. +3 of the row. All sums over a
// row or a column run in a fixed order, so results are bitwise reproducible.

#include <math.h>

#include "sparton_common.h"

namespace sparton {
namespace xf {

constexpr int MAX_NP = 12;          // D up to 12 * 256 (the backward's LDS: 4 waves x D floats)
constexpr int ROW_WAVES = 4;        // waves per workgroup
constexpr int ROWS_PER_WAVE = 8;    // backward: rows per wave (column partials per block)
constexpr int BLOCK_ROWS = ROW_WAVES * ROWS_PER_WAVE;
constexpr float kInvSqrt2 = 0.70710678118654752f;
constexpr float kInvSqrt2Pi = 0.39894228040143268f;

__device__ __forceinline__ float gelu(float x) { return 0.5f * x * (1.0f + erff(x * kInvSqrt2)); }
__device__ __forceinline__ float gelu_grad(float x) {
  return 0.5f * (1.0f + erff(x * kInvSqrt2)) + x * kInvSqrt2Pi * expf(-0.5f * x * x);
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// Four consecutive elements of a row (one 8- or 16-byte access; D % 4 == 0 keeps each
// group of four whole, and rows start 8- or 16-byte aligned) as float, zeros past D.
template <typename T> struct Vec4;
template <> struct Vec4<bf16> { typedef bf16x4 type; };
template <> struct Vec4<f16> { typedef f16x4 type; };
template <> struct Vec4<float> { typedef f32x4 type; };
template <typename T>
__device__ __forceinline__ f32x4 load4f(const T* p, int d, int D) {
  f32x4 r = f32x4{0.f, 0.f, 0.f, 0.f};
  if (d < D) {
    const typename Vec4<T>::type v = *(const typename Vec4<T>::type*)(p + d);
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = (float)v[e];
  }
  return r;
}
template <typename T>
__device__ __forceinline__ void store4t(T* p, int d, int D, f32x4 v) {
  if (d < D) {
    typename Vec4<T>::type o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = from_f32<T>(v[e]);
    *(typename Vec4<T>::type*)(p + d) = o;
  }
}
__device__ __forceinline__ f32x4 load4p(const float* p, int d, int D) {
  return d < D ? *(const f32x4*)(p + d) : f32x4{0.f, 0.f, 0.f, 0.f};
}

// ---- forward epilogue: one wave per row ------------------------------------------------
template <typename T, int NP>
__global__ __launch_bounds__(64 * ROW_WAVES) void xf_fwd_kernel(
    const T* __restrict__ Z, const float* __restrict__ bd, const float* __restrict__ gamma,
    const float* __restrict__ beta, float eps, T* __restrict__ Y, float* __restrict__ mean_out,
    float* __restrict__ rstd_out, int M, int D) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * ROW_WAVES + (threadIdx.x >> 6);
  if (row >= M) return;
  const T* z = Z + row * D;
  f32x4 u[NP];
  float s = 0.0f;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int d = p * 256 + lane * 4;
    const f32x4 zz = load4f(z, d, D), bb = load4p(bd, d, D);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      u[p][e] = d < D ? gelu(zz[e] + bb[e]) : 0.0f;
      s += u[p][e];
    }
  }
  const float mu = wave_sum(s) / (float)D;
  float q = 0.0f;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int d = p * 256 + lane * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float c = d < D ? u[p][e] - mu : 0.0f;
      q += c * c;
    }
  }
  const float rs = rsqrtf(wave_sum(q) / (float)D + eps);
  T* y = Y + row * D;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int d = p * 256 + lane * 4;
    const f32x4 g = load4p(gamma, d, D), bt = load4p(beta, d, D);
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = (u[p][e] - mu) * rs * g[e] + bt[e];
    store4t(y, d, D, o);
  }
  if (lane == 0) {
    mean_out[row] = mu;
    rstd_out[row] = rs;
  }
}

// ---- backward epilogue: ROWS_PER_WAVE rows per wave, column partials per block ----------
// Per row: xhat = (u - mean) * rstd, g = dY * gamma,
//          du = rstd * (g - mean_D(g) - xhat * mean_D(g * xhat)),   dZ = du * gelu'(Z + b_d).
// The block's rows add dY * xhat, dY and dZ into per-column partials in row order (each wave
// its rows, then the waves in order through LDS, one quantity at a time), written to
// part[block][3][D].
template <typename T, int NP>
__global__ __launch_bounds__(64 * ROW_WAVES) void xf_bwd_kernel(
    const T* __restrict__ dY, const T* __restrict__ Z, const float* __restrict__ bd,
    const float* __restrict__ gamma, const float* __restrict__ mean_in,
    const float* __restrict__ rstd_in, T* __restrict__ dZ, float* __restrict__ part, int M, int D) {
  extern __shared__ __attribute__((aligned(16))) float xf_smem[];  // [ROW_WAVES][D]
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  f32x4 pg[NP], pb[NP], pd[NP];  // partials of dY * xhat, dY, dZ
#pragma unroll
  for (int p = 0; p < NP; ++p) pg[p] = pb[p] = pd[p] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int r = 0; r < ROWS_PER_WAVE; ++r) {
    const int64_t row = (int64_t)blockIdx.x * BLOCK_ROWS + wave * ROWS_PER_WAVE + r;
    if (row >= M) break;
    const float mu = mean_in[row], rs = rstd_in[row];
    f32x4 xh[NP], gg[NP], dy[NP], zb[NP];
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int d = p * 256 + lane * 4;
      dy[p] = load4f(dY + row * D, d, D);
      const f32x4 zz = load4f(Z + row * D, d, D), bb = load4p(bd, d, D), ga = load4p(gamma, d, D);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        zb[p][e] = zz[e] + bb[e];
        xh[p][e] = d < D ? (gelu(zb[p][e]) - mu) * rs : 0.0f;
        gg[p][e] = dy[p][e] * ga[e];
        s1 += gg[p][e];
        s2 += gg[p][e] * xh[p][e];
      }
    }
    const float c1 = wave_sum(s1) / (float)D, c2 = wave_sum(s2) / (float)D;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int d = p * 256 + lane * 4;
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o[e] = rs * (gg[p][e] - c1 - xh[p][e] * c2) * gelu_grad(zb[p][e]);
        pg[p][e] += dy[p][e] * xh[p][e];
        pb[p][e] += dy[p][e];
        pd[p][e] += o[e];
      }
      store4t(dZ + row * D, d, D, o);
    }
  }
  float* mine = xf_smem + (size_t)wave * D;
  float* out = part + (size_t)blockIdx.x * 3 * D;
#pragma unroll
  for (int qn = 0; qn < 3; ++qn) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int d = p * 256 + lane * 4;
      if (d < D) *(f32x4*)(mine + d) = qn == 0 ? pg[p] : qn == 1 ? pb[p] : pd[p];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < D; i += 64 * ROW_WAVES) {
      float acc = 0.0f;
#pragma unroll
      for (int w = 0; w < ROW_WAVES; ++w) acc += xf_smem[(size_t)w * D + i];
      out[qn * D + i] = acc;
    }
    __syncthreads();  // the buffer is refilled with the next quantity
  }
}

// ---- column reduction: d gamma, d beta, d b_d = the blocks' partials summed in order ----
constexpr int COL_THREADS = 256;
__global__ __launch_bounds__(COL_THREADS) void xf_colsum_kernel(const float* __restrict__ part,
                                                               int nblk, int D,
                                                               float* __restrict__ dgamma,
                                                               float* __restrict__ dbeta,
                                                               float* __restrict__ dbd) {
  const int i = blockIdx.x * COL_THREADS + threadIdx.x;  // i in [0, 3D)
  if (i >= 3 * D) return;
  float acc = 0.0f;
  for (int k = 0; k < nblk; ++k) acc += part[(size_t)k * 3 * D + i];
  const int which = i / D, d = i - which * D;
  float* dst = which == 0 ? dgamma : which == 1 ? dbeta : dbd;
  if (dst != nullptr) dst[d] = acc;
}

static int passes(int64_t D) { return (int)cdiv(D, 256); }

template <typename T>
static int fwd(const void* z, const float* bd, const float* gamma, const float* beta, float eps,
               void* y, float* mean, float* rstd, int64_t M, int64_t D, hipStream_t st) {
  const dim3 grid((unsigned)cdiv(M, ROW_WAVES)), block(64 * ROW_WAVES);
#define XF_FWD(NP)                                                                          \
  hipLaunchKernelGGL((xf_fwd_kernel<T, NP>), grid, block, 0, st, (const T*)z, bd, gamma, beta, \
                     eps, (T*)y, mean, rstd, (int)M, (int)D)
  switch (passes(D)) {
    case 1: XF_FWD(1); break;
    case 2: XF_FWD(2); break;
    case 3: XF_FWD(3); break;
    case 4: XF_FWD(4); break;
    case 5: case 6: XF_FWD(6); break;
    case 7: case 8: XF_FWD(8); break;
    default: XF_FWD(12); break;
  }
#undef XF_FWD
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPARTON_OK : (int)e;
}

template <typename T>
static int bwd(const void* dy, const void* z, const float* bd, const float* gamma,
               const float* mean, const float* rstd, void* dz, float* part, float* dgamma,
               float* dbeta, float* dbd, int64_t M, int64_t D, hipStream_t st) {
  const int nblk = (int)cdiv(M, BLOCK_ROWS);
  const dim3 grid((unsigned)nblk), block(64 * ROW_WAVES);
  const size_t lds = (size_t)ROW_WAVES * D * sizeof(float);
#define XF_BWD(NP)                                                                              \
  hipLaunchKernelGGL((xf_bwd_kernel<T, NP>), grid, block, lds, st, (const T*)dy, (const T*)z, bd, \
                     gamma, mean, rstd, (T*)dz, part, (int)M, (int)D)
  switch (passes(D)) {
    case 1: XF_BWD(1); break;
    case 2: XF_BWD(2); break;
    case 3: XF_BWD(3); break;
    case 4: XF_BWD(4); break;
    case 5: case 6: XF_BWD(6); break;
    case 7: case 8: XF_BWD(8); break;
    default: XF_BWD(12); break;
  }
#undef XF_BWD
  hipLaunchKernelGGL(xf_colsum_kernel, dim3((unsigned)cdiv(3 * D, COL_THREADS)), dim3(COL_THREADS),
                     0, st, (const float*)part, nblk, (int)D, dgamma, dbeta, dbd);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPARTON_OK : (int)e;
}

}  // namespace xf
}  // namespace sparton

using namespace sparton;

static int xf_check(int64_t M, int64_t D, int dtype) {
  if (M < 0 || D < 0) return SPARTON_EINVAL;
  if (dtype < SPARTON_F32 || dtype > SPARTON_F16) return SPARTON_EINVAL;
  if (D % 4 != 0) return SPARTON_EINVAL;
  if (D > xf::MAX_NP * 256 || M > INT32_MAX) return SPARTON_EUNSUPPORTED;
  return SPARTON_OK;
}

extern "C" __attribute__((visibility("default"))) size_t sparton_transform_workspace_bytes(
    int64_t M, int64_t D) {
  if (M <= 0 || D <= 0) return 0;
  return (size_t)(cdiv(M, xf::BLOCK_ROWS) * 3 * D) * sizeof(float);
}

extern "C" __attribute__((visibility("default"))) int sparton_transform_fwd(
    const void* z, const float* dense_bias, const float* ln_weight, const float* ln_bias,
    float eps, void* y, float* mean, float* rstd, int64_t M, int64_t D, int dtype, void* stream) {
  const int rc = xf_check(M, D, dtype);
  if (rc != SPARTON_OK) return rc;
  if (M == 0 || D == 0) return SPARTON_OK;
  if (z == nullptr || y == nullptr || mean == nullptr || rstd == nullptr || dense_bias == nullptr ||
      ln_weight == nullptr || ln_bias == nullptr || !(eps >= 0.0f))
    return SPARTON_EINVAL;
  if (((uintptr_t)dense_bias | (uintptr_t)ln_weight | (uintptr_t)ln_bias) % 16 != 0)
    return SPARTON_EALIGN;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case SPARTON_BF16: return xf::fwd<bf16>(z, dense_bias, ln_weight, ln_bias, eps, y, mean, rstd, M, D, st);
    case SPARTON_F16: return xf::fwd<f16>(z, dense_bias, ln_weight, ln_bias, eps, y, mean, rstd, M, D, st);
    default: return xf::fwd<float>(z, dense_bias, ln_weight, ln_bias, eps, y, mean, rstd, M, D, st);
  }
}

extern "C" __attribute__((visibility("default"))) int sparton_transform_bwd(
    const void* dy, const void* z, const float* dense_bias, const float* ln_weight,
    const float* mean, const float* rstd, void* dz, float* d_ln_weight, float* d_ln_bias,
    float* d_dense_bias, void* workspace, size_t workspace_bytes, int64_t M, int64_t D, int dtype,
    void* stream) {
  const int rc = xf_check(M, D, dtype);
  if (rc != SPARTON_OK) return rc;
  if (M == 0 || D == 0) return SPARTON_OK;
  if (dy == nullptr || z == nullptr || dz == nullptr || mean == nullptr || rstd == nullptr ||
      dense_bias == nullptr || ln_weight == nullptr)
    return SPARTON_EINVAL;
  if (((uintptr_t)dense_bias | (uintptr_t)ln_weight) % 16 != 0) return SPARTON_EALIGN;
  if (workspace == nullptr || workspace_bytes < sparton_transform_workspace_bytes(M, D))
    return SPARTON_EWORKSPACE;
  if ((uintptr_t)workspace % 16 != 0) return SPARTON_EALIGN;
  hipStream_t st = (hipStream_t)stream;
  float* part = (float*)workspace;
  switch (dtype) {
    case SPARTON_BF16:
      return xf::bwd<bf16>(dy, z, dense_bias, ln_weight, mean, rstd, dz, part, d_ln_weight,
                           d_ln_bias, d_dense_bias, M, D, st);
    case SPARTON_F16:
      return xf::bwd<f16>(dy, z, dense_bias, ln_weight, mean, rstd, dz, part, d_ln_weight,
                          d_ln_bias, d_dense_bias, M, D, st);
    default:
      return xf::bwd<float>(dy, z, dense_bias, ln_weight, mean, rstd, dz, part, d_ln_weight,
                            d_ln_bias, d_dense_bias, M, D, st);
  }
}
