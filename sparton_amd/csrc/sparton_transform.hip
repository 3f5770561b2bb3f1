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
// A wave works on whole rows; lane l holds elements 256 p + 4 l .. +3 of a row. All sums
// over a row or a column run in a fixed order, so results are bitwise reproducible.

#include <math.h>

#include <algorithm>

#include "sparton_common.h"

namespace sparton {
namespace xf {

constexpr int MAX_NP = 12;          // D up to 12 * 256
constexpr int FWD_WAVES = 4;        // forward: one row per wave, 4 waves per workgroup
constexpr int BWD_WAVES_NARROW = 8; // backward waves per workgroup for D <= 1024
constexpr int BWD_WAVES_WIDE = 4;   // wider rows: 512 registers per wave (VGPRs + AGPRs)
constexpr int BWD_TARGET_BLOCKS = 256;  // enough backward workgroups for one per CU
constexpr int MAX_ROWS_PER_WAVE = 32;
constexpr int COL_WAVES = 16;       // column reduction: 64 columns x 16 waves per workgroup
constexpr float kInvSqrt2 = 0.70710678118654752f;
constexpr float kInvSqrt2Pi = 0.39894228040143268f;
constexpr float kLog2e = 1.44269504088896341f;

// ---- the normal CDF for exact (erf) gelu ------------------------------------------------
// gelu(x) = x Phi(x) and gelu'(x) = Phi(x) + x phi(x), with Phi(x) = erfc(-x / sqrt 2) / 2
// and phi(x) = exp(-x^2 / 2) / sqrt(2 pi). erfc comes from the Chebyshev fit of Numerical
// Recipes (Press et al., 2nd ed., section 6.2, erfcc):
//     erfc(z) = t exp(-z^2 + P(t)),  t = 1 / (1 + z / 2),  z >= 0,
// fractional error below 1.2e-7 for every z >= 0, so Phi keeps its relative accuracy in
// the lower tail. One v_rcp, one v_exp and a 9-term Horner polynomial: about a fifth of
// the VALU work of the library erff.
__device__ __forceinline__ float erfc_pos(float z) {
  const float t = __builtin_amdgcn_rcpf(fmaf(0.5f, z, 1.0f));
  float p = 0.17087277f;
  p = fmaf(t, p, -0.82215223f);
  p = fmaf(t, p, 1.48851587f);
  p = fmaf(t, p, -1.13520398f);
  p = fmaf(t, p, 0.27886807f);
  p = fmaf(t, p, -0.18628806f);
  p = fmaf(t, p, 0.09678418f);
  p = fmaf(t, p, 0.37409196f);
  p = fmaf(t, p, 1.00002368f);
  const float a = fmaf(t, p, fmaf(-z, z, -1.26551223f));
  return t * __builtin_amdgcn_exp2f(a * kLog2e);
}
__device__ __forceinline__ float norm_cdf(float x) {
  const float h = 0.5f * erfc_pos(fabsf(x) * kInvSqrt2);
  return x >= 0.0f ? 1.0f - h : h;
}
__device__ __forceinline__ float gelu(float x) { return x * norm_cdf(x); }
// x phi(x), the second term of gelu'(x)
__device__ __forceinline__ float x_pdf(float x) {
  return x * kInvSqrt2Pi * __builtin_amdgcn_exp2f((-0.5f * kLog2e) * (x * x));
}

// Four consecutive elements of a row (one 8- or 16-byte access; D % 4 == 0 keeps each
// group of four whole, and rows start 8- or 16-byte aligned). FULL: D == NP * 256, so every
// lane's groups are in range and the bounds tests compile away.
template <typename T> struct Vec4;
template <> struct Vec4<bf16> { typedef bf16x4 type; };
template <> struct Vec4<f16> { typedef f16x4 type; };
template <> struct Vec4<float> { typedef f32x4 type; };
template <typename T> using vec4_t = typename Vec4<T>::type;

template <bool FULL>
__device__ __forceinline__ bool in_row(int d, int D) { return FULL || d < D; }
// Past the row end a lane loads the row's last group instead (D >= 4): every load is
// unconditional, so a wave's loads are in flight together (a load under a per-lane condition,
// or one whose value is selected right away, is waited for before the next is issued). The
// values past the row end are not zeros: every use masks them with in_row.
template <typename T, bool FULL>
__device__ __forceinline__ vec4_t<T> load4(const T* p, int d, int D) {
  return *(const vec4_t<T>*)(p + (FULL ? d : min(d, D - 4)));
}
template <typename T>
__device__ __forceinline__ f32x4 to_f32(vec4_t<T> v) {
  f32x4 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) r[e] = (float)v[e];
  return r;
}
// The epilogues' row outputs (H forward, dZ backward) stream out with nontemporal stores:
// nothing re-reads them before the next kernel (8192 x 768 bf16: forward 9.0 -> 8.0 us,
// backward 17.6 -> 16.7 us).
template <typename T, bool FULL>
__device__ __forceinline__ void store4t(T* p, int d, int D, f32x4 v) {
  if (in_row<FULL>(d, D)) {
    vec4_t<T> o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = from_f32<T>(v[e]);
    __builtin_nontemporal_store(o, (vec4_t<T>*)(p + d));
  }
}
template <bool FULL>
__device__ __forceinline__ f32x4 load4p(const float* p, int d, int D) {
  return *(const f32x4*)(p + (FULL ? d : min(d, D - 4)));
}

// ---- forward epilogue: one wave per row ------------------------------------------------
// u = gelu(Z + b_d), mean and 1/std of u over the row, Y = (u - mean) / std * gamma + beta.
template <typename T, int NP, bool FULL>
__global__ __launch_bounds__(64 * FWD_WAVES) void xf_fwd_kernel(
    const T* __restrict__ Z, const float* __restrict__ bd, const float* __restrict__ gamma,
    const float* __restrict__ beta, float eps, T* __restrict__ Y, float* __restrict__ mean_out,
    float* __restrict__ rstd_out, int M, int D) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * FWD_WAVES + (threadIdx.x >> 6);
  if (row >= M) return;
  const T* z = Z + row * D;
  vec4_t<T> zr[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) zr[p] = load4<T, FULL>(z, p * 256 + lane * 4, D);
  f32x4 u[NP];
  float s = 0.0f;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int d = p * 256 + lane * 4;
    const f32x4 zz = to_f32<T>(zr[p]), bb = load4p<FULL>(bd, d, D);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      u[p][e] = in_row<FULL>(d, D) ? gelu(zz[e] + bb[e]) : 0.0f;
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
      const float c = in_row<FULL>(d, D) ? u[p][e] - mu : 0.0f;
      q += c * c;
    }
  }
  const float rs = rsqrtf(wave_sum(q) / (float)D + eps);
  T* y = Y + row * D;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int d = p * 256 + lane * 4;
    const f32x4 g = load4p<FULL>(gamma, d, D), bt = load4p<FULL>(beta, d, D);
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = (u[p][e] - mu) * rs * g[e] + bt[e];
    store4t<T, FULL>(y, d, D, o);
  }
  if (lane == 0) {
    mean_out[row] = mu;
    rstd_out[row] = rs;
  }
}

// ---- backward epilogue -----------------------------------------------------------------
// Per row: xhat = (u - mean) * rstd, g = dY * gamma,
//          du = rstd * (g - mean_D(g) - xhat * mean_D(g * xhat)),   dZ = du * gelu'(Z + b_d).
// Workgroup b owns rows [b R W, (b + 1) R W) (W waves, R rows per wave, each wave R
// consecutive rows); every wave adds dY * xhat, dY and dZ of its rows, in row order,
// into per-column register partials, and the workgroup sums its waves' partials in wave
// order through LDS, one quantity at a time, into part[b][3][D].
// KEEP (NP <= 4): the row's g, xhat and gelu' stay in registers between the two passes,
// b_d and gamma are held for the whole loop and the next row's dY and Z are loaded while
// the current one is computed. Wider rows reload b_d and gamma from cache and recompute
// xhat and gelu' in the second pass and run 4 waves per workgroup, so that each wave may
// hold 512 registers.
template <int NP> struct BwdCfg {
  static constexpr bool keep = NP <= 4;
  static constexpr int waves = NP <= 4 ? BWD_WAVES_NARROW : BWD_WAVES_WIDE;
  static constexpr int threads = 64 * waves;
};

template <typename T, int NP, bool FULL>
__global__ __launch_bounds__(BwdCfg<NP>::threads) void xf_bwd_kernel(
    const T* __restrict__ dY, const T* __restrict__ Z, const float* __restrict__ bd,
    const float* __restrict__ gamma, const float* __restrict__ mean_in,
    const float* __restrict__ rstd_in, T* __restrict__ dZ, float* __restrict__ part, int M, int D,
    int rows_per_wave) {
  constexpr bool KEEP = BwdCfg<NP>::keep;
  constexpr int W = BwdCfg<NP>::waves;
  extern __shared__ __attribute__((aligned(16))) float xf_smem[];  // [W][D]
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row0 = ((int64_t)blockIdx.x * W + wave) * rows_per_wave;
  const int nrows = (int)max((int64_t)0, min((int64_t)rows_per_wave, (int64_t)M - row0));

  f32x4 pg[NP], pb[NP], pd[NP];  // partials of dY * xhat, dY, dZ
#pragma unroll
  for (int p = 0; p < NP; ++p) pg[p] = pb[p] = pd[p] = f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 vb[KEEP ? NP : 1], vg[KEEP ? NP : 1];
  if constexpr (KEEP) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      vb[p] = load4p<FULL>(bd, p * 256 + lane * 4, D);
      vg[p] = load4p<FULL>(gamma, p * 256 + lane * 4, D);
    }
  }
  vec4_t<T> ny[NP], nz[NP];  // the next row's dY and Z
  if (nrows > 0) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      ny[p] = load4<T, FULL>(dY + row0 * D, p * 256 + lane * 4, D);
      nz[p] = load4<T, FULL>(Z + row0 * D, p * 256 + lane * 4, D);
    }
  }
  for (int r = 0; r < nrows; ++r) {
    const int64_t row = row0 + r;
    vec4_t<T> cy[NP], cz[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      cy[p] = ny[p];
      cz[p] = nz[p];
    }
    if (KEEP && r + 1 < nrows) {
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        ny[p] = load4<T, FULL>(dY + (row + 1) * D, p * 256 + lane * 4, D);
        nz[p] = load4<T, FULL>(Z + (row + 1) * D, p * 256 + lane * 4, D);
      }
    }
    const float mu = mean_in[row], rs = rstd_in[row];
    f32x4 xh[KEEP ? NP : 1], gg[KEEP ? NP : 1], gp[KEEP ? NP : 1];
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int d = p * 256 + lane * 4;
      const f32x4 dy = to_f32<T>(cy[p]), zz = to_f32<T>(cz[p]);
      const f32x4 bb = KEEP ? vb[p] : load4p<FULL>(bd, d, D);
      const f32x4 ga = KEEP ? vg[p] : load4p<FULL>(gamma, d, D);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float zb = zz[e] + bb[e];
        const float cdf = norm_cdf(zb);
        const float x = in_row<FULL>(d, D) ? (zb * cdf - mu) * rs : 0.0f;
        const float g = in_row<FULL>(d, D) ? dy[e] * ga[e] : 0.0f;
        s1 += g;
        s2 += g * x;
        pg[p][e] += dy[e] * x;
        pb[p][e] += dy[e];
        if constexpr (KEEP) {
          xh[p][e] = x;
          gg[p][e] = g;
          gp[p][e] = cdf + x_pdf(zb);
        }
      }
    }
    const float c1 = wave_sum(s1) / (float)D, c2 = wave_sum(s2) / (float)D;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int d = p * 256 + lane * 4;
      f32x4 o;
      if constexpr (KEEP) {
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = rs * (gg[p][e] - c1 - xh[p][e] * c2) * gp[p][e];
      } else {
        const f32x4 dy = to_f32<T>(cy[p]), zz = to_f32<T>(cz[p]);
        const f32x4 bb = load4p<FULL>(bd, d, D), ga = load4p<FULL>(gamma, d, D);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float zb = zz[e] + bb[e];
          const float cdf = norm_cdf(zb);
          const float x = in_row<FULL>(d, D) ? (zb * cdf - mu) * rs : 0.0f;
          o[e] = rs * (dy[e] * ga[e] - c1 - x * c2) * (cdf + x_pdf(zb));
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) pd[p][e] += o[e];
      store4t<T, FULL>(dZ + row * D, d, D, o);
    }
    if (!KEEP && r + 1 < nrows) {
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        ny[p] = load4<T, FULL>(dY + (row + 1) * D, p * 256 + lane * 4, D);
        nz[p] = load4<T, FULL>(Z + (row + 1) * D, p * 256 + lane * 4, D);
      }
    }
  }
  float* mine = xf_smem + (size_t)wave * D;
  float* out = part + (size_t)blockIdx.x * 3 * D;
#pragma unroll
  for (int qn = 0; qn < 3; ++qn) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int d = p * 256 + lane * 4;
      if (in_row<FULL>(d, D)) *(f32x4*)(mine + d) = qn == 0 ? pg[p] : qn == 1 ? pb[p] : pd[p];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < D; i += 64 * W) {
      float acc = 0.0f;
#pragma unroll
      for (int w = 0; w < W; ++w) acc += xf_smem[(size_t)w * D + i];
      out[qn * D + i] = acc;
    }
    __syncthreads();  // the buffer is refilled with the next quantity
  }
}

// ---- column reduction: d gamma, d beta, d b_d = the blocks' partials summed --------------
// Workgroup c owns columns [64 c, 64 c + 64) of part's 3D columns, one per lane; wave w sums
// blocks [w S, (w + 1) S) (S = ceil(nblk / COL_WAVES)) in block order, eight loads in flight,
// and lane i of wave 0 adds the 16 wave sums in wave order. Fixed order: reproducible.
__global__ __launch_bounds__(64 * COL_WAVES) void xf_colsum_kernel(const float* __restrict__ part,
                                                                   int nblk, int D,
                                                                   float* __restrict__ dgamma,
                                                                   float* __restrict__ dbeta,
                                                                   float* __restrict__ dbd) {
  __shared__ float wsum[COL_WAVES][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = blockIdx.x * 64 + lane;
  const int ncol = 3 * D;
  const int seg = (nblk + COL_WAVES - 1) / COL_WAVES;
  const int beg = min(nblk, wave * seg), end = min(nblk, beg + seg);
  float acc = 0.0f;
  if (col < ncol) {
    for (int k0 = beg; k0 < end; k0 += 8) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = part[(size_t)min(k0 + j, end - 1) * ncol + col];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc += k0 + j < end ? v[j] : 0.0f;
    }
  }
  wsum[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && col < ncol) {
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < COL_WAVES; ++w) t += wsum[w][lane];
    const int which = col / D, d = col - which * D;
    float* dst = which == 0 ? dgamma : which == 1 ? dbeta : dbd;
    if (dst != nullptr) dst[d] = t;
  }
}

// ---- weight gradient support: dW = dZ^T X as a batched GEMM over C row chunks -----------
// A plain dZ^T X GEMM has K = M (thousands of rows) and a D x D output of only a few dozen
// tiles, so a library GEMM leaves most CUs idle. Split into C chunks of L = M / C rows,
// dW = sum_c dZ_c^T X_c is a batched GEMM whose left operands dZ_c^T are K-contiguous
// [D, L] matrices (X_c are views of X, no copy). These two kernels write those operands
// and sum the C fp32 products in chunk order.

// dzt[c][i][l] = dz[c L + l][i] for 16-bit types, in registers: each wave takes a 64 x 64
// (row x column) tile of dz and each lane an 8 x 8 block of it -- eight 16-byte row loads,
// a transpose by 32 v_perm_b32 (output dword q of column j = the j-th halves of rows 2q and
// 2q + 1), eight 16-byte column stores. A wave's loads cover 8 rows x 128 contiguous bytes
// and its stores 8 columns x 128 contiguous bytes. L % 64 == 0 and D % 64 == 0, so a tile
// never straddles two chunks or the row end.
constexpr int TR_TILE = 64;
constexpr int TR_WAVES = 4;  // tiles side by side along D per workgroup
template <typename T>
__global__ __launch_bounds__(64 * TR_WAVES) void xf_chunk_transpose_kernel(const T* __restrict__ dz,
                                                                          T* __restrict__ dzt, int M,
                                                                          int D, int L) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int m0 = blockIdx.x * TR_TILE, i0 = (blockIdx.y * TR_WAVES + wave) * TR_TILE;
  if (i0 >= D) return;
  const int rb = lane >> 3, cb = lane & 7;  // the lane's 8-row and 8-column block
  u32x4 r[8];
#pragma unroll
  for (int e = 0; e < 8; ++e)
    r[e] = *(const u32x4*)(dz + (size_t)(m0 + 8 * rb + e) * D + i0 + 8 * cb);
  const int c = m0 / L, l = m0 - c * L + 8 * rb;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = __builtin_amdgcn_perm(r[2 * q + 1][j >> 1], r[2 * q][j >> 1], sel);
    *(u32x4*)(dzt + ((size_t)c * D + i0 + 8 * cb + j) * L + l) = o;
  }
}

// out[k] = sum_c part[c][k] in chunk order, cast to T; four entries per thread.
template <typename T>
__global__ __launch_bounds__(256) void xf_chunk_sum_kernel(const float* __restrict__ part,
                                                           T* __restrict__ out, int C,
                                                           int64_t n) {
  const int64_t k = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (k >= n) return;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int c = 0; c < C; ++c) acc += *(const f32x4*)(part + (size_t)c * n + k);
  vec4_t<T> o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = from_f32<T>(acc[e]);
  *(vec4_t<T>*)(out + k) = o;
}

static int passes(int64_t D) { return (int)cdiv(D, 256); }
static int bwd_waves(int64_t D) { return D <= 4 * 256 ? BWD_WAVES_NARROW : BWD_WAVES_WIDE; }
static int rows_per_wave(int64_t M, int64_t D) {
  return (int)std::min<int64_t>(
      MAX_ROWS_PER_WAVE, std::max<int64_t>(1, cdiv(M, (int64_t)bwd_waves(D) * BWD_TARGET_BLOCKS)));
}
static int64_t bwd_blocks(int64_t M, int64_t D) {
  return cdiv(M, (int64_t)bwd_waves(D) * rows_per_wave(M, D));
}

template <typename T>
static int fwd(const void* z, const float* bd, const float* gamma, const float* beta, float eps,
               void* y, float* mean, float* rstd, int64_t M, int64_t D, hipStream_t st) {
  const dim3 grid((unsigned)cdiv(M, FWD_WAVES)), block(64 * FWD_WAVES);
  const bool full = D % 256 == 0;
#define XF_FWD(NP)                                                                            \
  do {                                                                                        \
    if (full && D == NP * 256)                                                                \
      hipLaunchKernelGGL((xf_fwd_kernel<T, NP, true>), grid, block, 0, st, (const T*)z, bd,   \
                         gamma, beta, eps, (T*)y, mean, rstd, (int)M, (int)D);                \
    else                                                                                      \
      hipLaunchKernelGGL((xf_fwd_kernel<T, NP, false>), grid, block, 0, st, (const T*)z, bd,  \
                         gamma, beta, eps, (T*)y, mean, rstd, (int)M, (int)D);                \
  } while (0)
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
  const int rpw = rows_per_wave(M, D);
  const int nblk = (int)bwd_blocks(M, D);
  const dim3 grid((unsigned)nblk), block(64 * bwd_waves(D));
  const size_t lds = (size_t)bwd_waves(D) * D * sizeof(float);
  const bool full = D % 256 == 0;
#define XF_BWD(NP)                                                                               \
  do {                                                                                           \
    if (full && D == NP * 256)                                                                   \
      hipLaunchKernelGGL((xf_bwd_kernel<T, NP, true>), grid, block, lds, st, (const T*)dy,       \
                         (const T*)z, bd, gamma, mean, rstd, (T*)dz, part, (int)M, (int)D, rpw); \
    else                                                                                         \
      hipLaunchKernelGGL((xf_bwd_kernel<T, NP, false>), grid, block, lds, st, (const T*)dy,      \
                         (const T*)z, bd, gamma, mean, rstd, (T*)dz, part, (int)M, (int)D, rpw); \
  } while (0)
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
  hipLaunchKernelGGL(xf_colsum_kernel, dim3((unsigned)cdiv(3 * D, 64)), dim3(64 * COL_WAVES), 0, st,
                     (const float*)part, nblk, (int)D, dgamma, dbeta, dbd);
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
  return (size_t)(xf::bwd_blocks(M, D) * 3 * D) * sizeof(float);
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

extern "C" __attribute__((visibility("default"))) int sparton_transform_dz_chunks(
    const void* dz, void* dzt, int64_t M, int64_t D, int64_t C, int dtype, void* stream) {
  if ((dtype != SPARTON_BF16 && dtype != SPARTON_F16) || M < 0 || D < 0 || C < 1) return SPARTON_EINVAL;
  if (M == 0 || D == 0) return SPARTON_OK;
  if (dz == nullptr || dzt == nullptr || M % C != 0 || (M / C) % xf::TR_TILE != 0 ||
      D % xf::TR_TILE != 0)
    return SPARTON_EINVAL;
  if ((((uintptr_t)dz) | ((uintptr_t)dzt)) % 16 != 0) return SPARTON_EALIGN;
  if (M > INT32_MAX || D > INT32_MAX) return SPARTON_EUNSUPPORTED;
  const dim3 grid((unsigned)(M / xf::TR_TILE), (unsigned)cdiv(D, (int64_t)xf::TR_TILE * xf::TR_WAVES));
  hipStream_t st = (hipStream_t)stream;
  const int L = (int)(M / C);
  if (dtype == SPARTON_BF16)
    hipLaunchKernelGGL(xf::xf_chunk_transpose_kernel<bf16>, grid, dim3(64 * xf::TR_WAVES), 0, st,
                       (const bf16*)dz, (bf16*)dzt, (int)M, (int)D, L);
  else
    hipLaunchKernelGGL(xf::xf_chunk_transpose_kernel<f16>, grid, dim3(64 * xf::TR_WAVES), 0, st,
                       (const f16*)dz, (f16*)dzt, (int)M, (int)D, L);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPARTON_OK : (int)e;
}

extern "C" __attribute__((visibility("default"))) int sparton_transform_chunk_sum(
    const float* part, void* out, int64_t C, int64_t n, int dtype, void* stream) {
  if (dtype < SPARTON_F32 || dtype > SPARTON_F16 || C < 1 || n < 0) return SPARTON_EINVAL;
  if (n == 0) return SPARTON_OK;
  if (part == nullptr || out == nullptr || n % 4 != 0) return SPARTON_EINVAL;
  if ((((uintptr_t)part) | ((uintptr_t)out)) % 16 != 0) return SPARTON_EALIGN;
  const dim3 grid((unsigned)cdiv(n / 4, (int64_t)256));
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case SPARTON_BF16:
      hipLaunchKernelGGL(xf::xf_chunk_sum_kernel<bf16>, grid, dim3(256), 0, st, part, (bf16*)out, (int)C, n);
      break;
    case SPARTON_F16:
      hipLaunchKernelGGL(xf::xf_chunk_sum_kernel<f16>, grid, dim3(256), 0, st, part, (f16*)out, (int)C, n);
      break;
    default:
      hipLaunchKernelGGL(xf::xf_chunk_sum_kernel<float>, grid, dim3(256), 0, st, part, (float*)out, (int)C, n);
      break;
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPARTON_OK : (int)e;
}
