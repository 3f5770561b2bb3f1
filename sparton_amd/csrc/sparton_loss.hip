// The SPLADE training loss on the head's output, on gfx950 (reference training/train.py:73-88,
// combined at :164-197). For query reps Q [Bq,V] and document reps R [Bd,V] (row-major, the
// head's reps dtype):
//   S      = Q R^T / T                                   in-batch scores
//   CE     = mean_i ( logsumexp_j S[i,j] - S[i,i] )       InfoNCE with labels arange(Bq) (:73-77)
//   L1(X)  = mean_b sum_v |X[b,v]|                        (:80-82)
//   FL(X)  = mean_v ( sum_b X[b,v] )^2                    (:85-87)
//   total  = w_ce CE + w_l1 (L1(Q) + L1(R)) + w_fl (FL(Q) + FL(R))    (:196-197)
// R may be absent (Bd = 0): then CE, L1(R) and FL(R) are 0.
//
// Forward, three launches:
//   loss_partial_kernel   one workgroup per 64-column vocabulary slice: stages the slice of Q
//                         and R as fp32 in LDS and writes the slice's partial S (4x4 or 2x2
//                         register tiles), each row's partial sum |X| and the slice's
//                         sum_v (sum_b X)^2;
//   loss_slice_sum_kernel those partials summed over the slices in a fixed order;
//   loss_final_kernel     one workgroup: the rows' softmax, CE, the means, total, and
//                         P = (softmax(S) - I) / (Bq T), which the backward uses.
// Backward, one launch (loss_bwd_kernel, one workgroup per slice), with the upstream
// gradients g[0..5] of (total, CE, L1(Q), L1(R), FL(Q), FL(R)) read from device memory:
//   dQ = (g0 w_ce + g1) P R + (g0 w_l1 + g2) sign(Q) / Bq + (g0 w_fl + g4) 2 colsum(Q) / V
//   dR = (g0 w_ce + g1) P^T Q + (g0 w_l1 + g3) sign(R) / Bd + (g0 w_fl + g5) 2 colsum(R) / V
// Everything accumulates in fp32 in a fixed order, so results are bitwise reproducible.
// The whole loss moves each of Q and R once forward and once backward: HBM-bound, small.

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <type_traits>

#include "sparton_common.h"

namespace sparton {
namespace loss {

constexpr int SLICE = 64;            // vocabulary columns per workgroup, one per lane
constexpr int NWAVES = 4;
constexpr int NT = 64 * NWAVES;
constexpr int MAX_B = 64;            // rows of Q and of R (past it the GEMM kernels are faster)
constexpr int LD = SLICE + 4;        // LDS row stride (floats) of a staged slice
constexpr int SUM_WAVES = 16;        // slice reduction: 64 entries x 16 waves per workgroup

__host__ __device__ constexpr int round4(int x) { return (x + 3) & ~3; }

// Rows [0, Bq) of Q then [0, Bd) of R, columns [c0, c0 + 64), as fp32 into sq / sd, zeros past
// V and in the padding rows up to a multiple of 4. Wave w stages rows w, w + 4, ...; lane l
// column c0 + l (one 128-byte segment per row for 16-bit types). All of a wave's loads are
// issued before the first is used, so they share one round trip: every lane loads from a
// clamped, valid address and the values of padding rows and columns past V are replaced by
// zeros afterwards (a load under a per-lane condition is waited for before the next one is
// issued). Bq >= 1, and R is read only when Bd > 0. Then row_fn(isq, row, x) runs for every
// real row with the lane's value (wave-uniform control flow).
template <typename T, int MB, typename F>
__device__ __forceinline__ void stage_slice(const T* __restrict__ Q, const T* __restrict__ R, int Bq,
                                            int Bd, int V, int c0, float* sq, float* sd, F row_fn) {
  constexpr int RPW = 2 * MB / NWAVES;  // rows per wave at most (Q and R padded to MB each)
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = c0 + lane;
  const int cl = min(c, V - 1);
  const int Bqp = round4(Bq), Bdp = round4(Bd);
  T raw[RPW];
#pragma unroll
  for (int k = 0; k < RPW; ++k) {
    const int r = wave + k * NWAVES;
    const bool isq = r < Bqp || Bd == 0;
    const int row = isq ? min(r, Bq - 1) : min(r - Bqp, Bd - 1);
    raw[k] = (isq ? Q : R)[(size_t)row * V + cl];
  }
#pragma unroll
  for (int k = 0; k < RPW; ++k) {
    const int r = wave + k * NWAVES;
    if (r >= Bqp + Bdp) break;
    const bool isq = r < Bqp;
    const int row = isq ? r : r - Bqp;
    if (!(row < (isq ? Bq : Bd) && c < V)) raw[k] = T(0.0f);
    const float x = to_f32(raw[k]);
    (isq ? sq : sd)[row * LD + lane] = x;
    if (row < (isq ? Bq : Bd)) row_fn(isq, row, x);
  }
}

// Partials of one slice, at part + slice * K:
//   [0, Bq Bd)                     S without the 1/T (only when Bd > 0)
//   [o, o + Bq), [o + Bq, o + Bq + Bd)   sum over the slice of |Q[i,:]|, |R[j,:]|
//   o + Bq + Bd, o + Bq + Bd + 1   sum over the slice of colsum(Q)^2, colsum(R)^2
template <typename T, int MB, int TM>
__global__ __launch_bounds__(NT) void loss_partial_kernel(const T* __restrict__ Q,
                                                          const T* __restrict__ R, int Bq, int Bd,
                                                          int V, float* __restrict__ part, int K) {
  __shared__ __attribute__((aligned(16))) float sq[MB * LD];
  __shared__ __attribute__((aligned(16))) float sd[MB * LD];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float* out = part + (size_t)blockIdx.x * K;
  const int o = Bq * Bd;
  stage_slice<T, MB>(Q, R, Bq, Bd, V, blockIdx.x * SLICE, sq, sd, [&](bool isq, int row, float x) {
    const float s = wave_sum(fabsf(x));
    if (lane == 0) out[o + (isq ? 0 : Bq) + row] = s;
  });
  __syncthreads();
  if (wave < 2) {  // wave 0: Q's column sums, wave 1: R's
    const float* s = wave == 0 ? sq : sd;
    const int nrows = wave == 0 ? Bq : Bd;
    float cs = 0.0f;
    for (int r = 0; r < nrows; ++r) cs += s[r * LD + lane];
    const float t = wave_sum(cs * cs);
    if (lane == 0) out[o + Bq + Bd + wave] = t;
  }
  if (Bd == 0) return;
  // S tiles of TM x TM (TM = 2 when 4 x 4 tiles would leave threads idle)
  const int nbi = round4(Bq) / TM, nbj = round4(Bd) / TM;
  for (int blk = threadIdx.x; blk < nbi * nbj; blk += NT) {
    const int i0 = (blk / nbj) * TM, j0 = (blk % nbj) * TM;
    float acc[TM][TM];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int b = 0; b < TM; ++b) acc[a][b] = 0.0f;
#pragma unroll 4
    for (int cc = 0; cc < SLICE; cc += 4) {
      f32x4 qa[TM], rb[TM];
#pragma unroll
      for (int k = 0; k < TM; ++k) {
        qa[k] = *(const f32x4*)(sq + (i0 + k) * LD + cc);
        rb[k] = *(const f32x4*)(sd + (j0 + k) * LD + cc);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
          for (int b = 0; b < TM; ++b) acc[a][b] = fmaf(qa[a][e], rb[b][e], acc[a][b]);
    }
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int b = 0; b < TM; ++b)
        if (i0 + a < Bq && j0 + b < Bd) out[(i0 + a) * Bd + j0 + b] = acc[a][b];
  }
}

// sums[k] = sum over slices of part[slice][k]. Workgroup g owns entries [64 g, 64 g + 64), one
// per lane; wave w sums slices [w S, (w + 1) S) in order (S = ceil(nslice / 16)), eight loads
// in flight, and wave 0 adds the 16 wave sums in wave order.
__global__ __launch_bounds__(64 * SUM_WAVES) void loss_slice_sum_kernel(const float* __restrict__ part,
                                                                       int nslice, int K,
                                                                       float* __restrict__ sums) {
  __shared__ float wsum[SUM_WAVES][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int k = blockIdx.x * 64 + lane;
  const int seg = (nslice + SUM_WAVES - 1) / SUM_WAVES;
  const int beg = min(nslice, wave * seg), end = min(nslice, beg + seg);
  float acc = 0.0f;
  if (k < K) {
    for (int s0 = beg; s0 < end; s0 += 8) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = part[(size_t)min(s0 + j, end - 1) * K + k];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc += s0 + j < end ? v[j] : 0.0f;
    }
  }
  wsum[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && k < K) {
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < SUM_WAVES; ++w) t += wsum[w][lane];
    sums[k] = t;
  }
}

// One workgroup. Wave w takes score rows w, w + 4, ...; lane l holds columns l and l + 64.
// out = (total, CE, L1(Q), L1(R), FL(Q), FL(R)); probs[i][j] = (softmax_j(S[i,:]) - [i == j]) / (Bq T).
__global__ __launch_bounds__(NT) void loss_final_kernel(const float* __restrict__ sums, int Bq, int Bd,
                                                        int V, float inv_t, float w_ce, float w_l1,
                                                        float w_fl, float* __restrict__ out,
                                                        float* __restrict__ probs) {
  __shared__ float row_loss[MAX_B];
  __shared__ float tail[2 * MAX_B + 2];  // the row sums of |x| and the two FLOPS sums
  __shared__ float ss[MAX_B * MAX_B];     // S without the 1/T
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int o = Bq * Bd, n = o + Bq + Bd + 2;
  for (int k0 = 0; k0 < n; k0 += 8 * NT) {  // every load of a round issued before any store
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      v[u] = sums[min(k0 + u * NT + (int)threadIdx.x, n - 1)];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = k0 + u * NT + threadIdx.x;
      if (k < o) ss[k] = v[u];
      else if (k < n) tail[k - o] = v[u];
    }
  }
  __syncthreads();
  if (Bd > 0) {
    const float pscale = inv_t / (float)Bq;
    for (int i = wave; i < Bq; i += NWAVES) {
      const float* srow = ss + i * Bd;
      const bool h0 = lane < Bd, h1 = lane + 64 < Bd;
      const float x0 = h0 ? srow[lane] * inv_t : -INFINITY;
      const float x1 = h1 ? srow[lane + 64] * inv_t : -INFINITY;
      const float m = wave_max(fmaxf(x0, x1));
      const float e0 = h0 ? expf(x0 - m) : 0.0f, e1 = h1 ? expf(x1 - m) : 0.0f;
      const float s = wave_sum(e0 + e1);
      if (lane == 0) row_loss[i] = m + logf(s) - srow[i] * inv_t;
      const float rs = 1.0f / s;
      if (h0) probs[(size_t)i * Bd + lane] = (e0 * rs - (lane == i ? 1.0f : 0.0f)) * pscale;
      if (h1) probs[(size_t)i * Bd + lane + 64] = (e1 * rs - (lane + 64 == i ? 1.0f : 0.0f)) * pscale;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float ce = 0.0f, l1q = 0.0f, l1d = 0.0f;
    for (int i = 0; i < (Bd > 0 ? Bq : 0); ++i) ce += row_loss[i];
    for (int i = 0; i < Bq; ++i) l1q += tail[i];
    for (int j = 0; j < Bd; ++j) l1d += tail[Bq + j];
    ce = Bd > 0 ? ce / (float)Bq : 0.0f;
    l1q /= (float)Bq;
    l1d = Bd > 0 ? l1d / (float)Bd : 0.0f;
    const float flq = tail[Bq + Bd] / (float)V, fld = tail[Bq + Bd + 1] / (float)V;
    out[0] = w_ce * ce + w_l1 * (l1q + l1d) + w_fl * (flq + fld);
    out[1] = ce;
    out[2] = l1q;
    out[3] = l1d;
    out[4] = flq;
    out[5] = fld;
  }
}

// The upstream gradients of the six outputs: each a device fp32 scalar, or NULL for 0.
struct Grads6 {
  const float* p[6];
};
__device__ __forceinline__ float grad_of(const Grads6& g, int k) {
  return g.p[k] != nullptr ? *g.p[k] : 0.0f;
}

// One workgroup per slice: stages Q, R and P, the slice's column sums, then 4x4 tiles of
// dQ (rows i0..i0+3 x 4 columns) and dR (rows j0..j0+3 x 4 columns), each thread a tile.
template <typename T, int MB>
__global__ __launch_bounds__(NT) void loss_bwd_kernel(const T* __restrict__ Q, const T* __restrict__ R,
                                                      const float* __restrict__ P,
                                                      const Grads6 g, int Bq, int Bd,
                                                      int V, float w_ce, float w_l1, float w_fl,
                                                      T* __restrict__ GQ, T* __restrict__ GR) {
  constexpr int PLD = MB + 4;
  __shared__ __attribute__((aligned(16))) float sq[MB * LD];
  __shared__ __attribute__((aligned(16))) float sd[MB * LD];
  __shared__ __attribute__((aligned(16))) float sp[MB * PLD];
  __shared__ float colsum[2][SLICE];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c0 = blockIdx.x * SLICE;
  const int Bqp = round4(Bq), Bdp = round4(Bd);
  // P, zero-padded to Bqp x Bdp: its loads are issued first, so that they are in flight
  // together with the slice's (clamped addresses, padding zeroed afterwards; P exists only
  // when Bd > 0)
  constexpr int PPT = MB * MB / NT;  // P entries per thread at most
  float pr[PPT];
  if (Bdp > 0) {
#pragma unroll
    for (int u = 0; u < PPT; ++u) {
      const int e = u * NT + threadIdx.x;
      const int i = e / Bdp, j = e - i * Bdp;
      pr[u] = P[(size_t)min(i, Bq - 1) * Bd + min(j, Bd - 1)];
    }
#pragma unroll
    for (int u = 0; u < PPT; ++u) {
      const int e = u * NT + threadIdx.x;
      const int i = e / Bdp, j = e - i * Bdp;
      if (!(e < Bqp * Bdp && i < Bq && j < Bd)) pr[u] = 0.0f;
    }
  }
  stage_slice<T, MB>(Q, R, Bq, Bd, V, c0, sq, sd, [](bool, int, float) {});
#pragma unroll
  for (int u = 0; u < PPT; ++u) {
    const int e = u * NT + threadIdx.x;
    if (Bdp > 0 && e < Bqp * Bdp) sp[(e / Bdp) * PLD + e % Bdp] = pr[u];
  }
  __syncthreads();
  if (wave < 2) {
    const float* s = wave == 0 ? sq : sd;
    const int nrows = wave == 0 ? Bq : Bd;
    float cs = 0.0f;
    for (int r = 0; r < nrows; ++r) cs += s[r * LD + lane];
    colsum[wave][lane] = cs;
  }
  __syncthreads();
  const float g0 = grad_of(g, 0);
  const float c_ce = g0 * w_ce + grad_of(g, 1);
  const float c_sq = (g0 * w_l1 + grad_of(g, 2)) / (float)Bq;
  const float c_sd = Bd > 0 ? (g0 * w_l1 + grad_of(g, 3)) / (float)Bd : 0.0f;
  const float c_fq = 2.0f * (g0 * w_fl + grad_of(g, 4)) / (float)V;
  const float c_fd = 2.0f * (g0 * w_fl + grad_of(g, 5)) / (float)V;
  const int nbi = Bqp / 4, nbj = Bdp / 4;
  constexpr int CT = SLICE / 4;  // column tiles per slice
  for (int t = threadIdx.x; t < (nbi + nbj) * CT; t += NT) {
    const bool isq = t < nbi * CT;
    const int tt = isq ? t : t - nbi * CT;
    const int r0 = (tt / CT) * 4, cc = (tt % CT) * 4;
    float acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) acc[a][b] = 0.0f;
    if (isq) {  // sum_j P[i][j] R[j][c]
      for (int j = 0; j < Bd; ++j) {
        const f32x4 rv = *(const f32x4*)(sd + j * LD + cc);
        float p[4];
#pragma unroll
        for (int a = 0; a < 4; ++a) p[a] = sp[(r0 + a) * PLD + j];
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
          for (int b = 0; b < 4; ++b) acc[a][b] = fmaf(p[a], rv[b], acc[a][b]);
      }
    } else {  // sum_i P[i][j] Q[i][c]
      for (int i = 0; i < Bq; ++i) {
        const f32x4 qv = *(const f32x4*)(sq + i * LD + cc);
        const f32x4 p = *(const f32x4*)(sp + i * PLD + r0);
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
          for (int b = 0; b < 4; ++b) acc[a][b] = fmaf(p[a], qv[b], acc[a][b]);
      }
    }
    const float* own = isq ? sq : sd;
    const float* cs = colsum[isq ? 0 : 1];
    const float c_s = isq ? c_sq : c_sd, c_f = isq ? c_fq : c_fd;
    const int nrows = isq ? Bq : Bd;
    T* G = isq ? GQ : GR;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int row = r0 + a;
      if (row >= nrows) continue;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int c = c0 + cc + b;
        if (c >= V) continue;
        const float x = own[row * LD + cc + b];
        const float sg = x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f);
        G[(size_t)row * V + c] = from_f32<T>(c_ce * acc[a][b] + c_s * sg + c_f * cs[cc + b]);
      }
    }
  }
}

static int64_t slices(int64_t V) { return cdiv(V, (int64_t)SLICE); }
static int64_t entries(int64_t Bq, int64_t Bd) { return Bq * Bd + Bq + Bd + 2; }

template <typename T, int MB>
static void launch_fwd(const void* q, const void* d, int Bq, int Bd, int V, float* part, int K,
                       hipStream_t st) {
  const dim3 grid((unsigned)slices(V));
  if ((round4(Bq) / 4) * (round4(Bd) / 4) >= NT)
    hipLaunchKernelGGL((loss_partial_kernel<T, MB, 4>), grid, dim3(NT), 0, st, (const T*)q,
                       (const T*)d, Bq, Bd, V, part, K);
  else
    hipLaunchKernelGGL((loss_partial_kernel<T, MB, 2>), grid, dim3(NT), 0, st, (const T*)q,
                       (const T*)d, Bq, Bd, V, part, K);
}
template <typename T, int MB>
static void launch_bwd(const void* q, const void* d, const float* P, const Grads6& g, int Bq, int Bd,
                       int V, float w_ce, float w_l1, float w_fl, void* gq, void* gd, hipStream_t st) {
  hipLaunchKernelGGL((loss_bwd_kernel<T, MB>), dim3((unsigned)slices(V)), dim3(NT), 0, st,
                     (const T*)q, (const T*)d, P, g, Bq, Bd, V, w_ce, w_l1, w_fl, (T*)gq, (T*)gd);
}

template <typename T>
static void fwd_partial(const void* q, const void* d, int Bq, int Bd, int V, float* part, int K,
                        hipStream_t st) {
  const int mb = Bq > Bd ? Bq : Bd;
  if (mb <= 32) launch_fwd<T, 32>(q, d, Bq, Bd, V, part, K, st);
  else launch_fwd<T, MAX_B>(q, d, Bq, Bd, V, part, K, st);
}
template <typename T>
static void bwd_all(const void* q, const void* d, const float* P, const Grads6& g, int Bq, int Bd,
                    int V, float w_ce, float w_l1, float w_fl, void* gq, void* gd, hipStream_t st) {
  const int mb = Bq > Bd ? Bq : Bd;
  if (mb <= 32) launch_bwd<T, 32>(q, d, P, g, Bq, Bd, V, w_ce, w_l1, w_fl, gq, gd, st);
  else launch_bwd<T, MAX_B>(q, d, P, g, Bq, Bd, V, w_ce, w_l1, w_fl, gq, gd, st);
}

// ---- batches past MAX_B rows ---------------------------------------------------------------
//
// The kernels above stage every row of a 64-column slice and keep per-slice partials of all
// Bq x Bd scores; their per-thread work grows with the rows, and past 64 rows a side the
// kernels below are faster (V 30522, fwd+bwd device time: 96 rows 134 us against 81 us, 128
// rows 190 against 90; 64 rows 62 against 70). Larger batches take GEMM-shaped kernels on the
// fp32 matrix cores (v_mfma_f32_32x32x2f32: the products of any reps dtype are exact in fp32,
// and the sums accumulate in fp32, as above; 16-bit reps have the variants further down):
//   forward   loss_stats_kernel   per 64-column slice: each row's sum of |x| over the slice,
//                                 and sum_v (sum_b x)^2 of Q and of R;
//             loss_score_kernel   S = Q R^T in 128 x 128 tiles, the vocabulary split into
//                                 chunks (one partial S per chunk);
//             loss_slice_sum_kernel (above) sums both sets of partials in a fixed order;
//             loss_rows_kernel    one wave per query row: softmax, the row's CE term, P;
//             loss_final_large_kernel the six scalars.
//   backward  loss_bwd_large_kernel, one workgroup per 64 vocabulary columns: the columns'
//             sums over Q and R, then dQ = c P R + ... tile by tile over 128 query rows and
//             dR = c P^T Q + ... over 128 document rows, K (the other side's rows) streamed
//             through LDS in stages of 32. No workspace.
// Operand tiles sit in LDS as fp32 [k][m]; an MFMA takes A[m][k] from lane m + 32 k and B[k][n]
// from lane n + 32 k, so both reads are consecutive floats. The row strides 161 and 97 are
// 33 mod 64 banks, so the transposing stores and the two lane halves' reads barely conflict.
namespace big {
constexpr int TM = 128;   // score tile rows and columns; gradient rows per tile
constexpr int KS = 32;    // K per LDS stage
constexpr int LDA = 161;  // floats per k row of a [KS][128] tile
constexpr int NC = 64;    // backward: vocabulary columns per workgroup
constexpr int LDB = 97;   // floats per k row of a [KS][64] tile
constexpr int ST_ROWS = 32;  // stats: rows whose loads are in flight together per wave

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

// K-contiguous source X[m][k] (row stride ld): rows [m0, m0 + 128), k in [k0, k0 + KS); zero past
// M rows or past kend. Thread t holds k = t % 32 of rows t / 32 + 8 u.
template <typename T>
__device__ __forceinline__ void load_kc(const T* __restrict__ X, int64_t ld, int m0, int M, int k0,
                                        int kend, T (&v)[16]) {
  const int t = threadIdx.x, k = k0 + (t & 31), rb = t >> 5;
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int m = m0 + rb + 8 * u;
    v[u] = (m < M && k < kend) ? X[(int64_t)m * ld + k] : T(0.0f);
  }
}
template <typename T>
__device__ __forceinline__ void store_kc(float* s, const T (&v)[16]) {
  const int t = threadIdx.x, kk = t & 31, rb = t >> 5;
#pragma unroll
  for (int u = 0; u < 16; ++u) s[kk * LDA + rb + 8 * u] = to_f32(v[u]);
}

// N-contiguous source X[k][n] (row stride ld): k in [k0, k0 + KS) below kend, n in [n0, n0 + NN)
// below nend, into s[k][n] (row stride LD). Thread t holds n = t % NN of k rows t / NN + (NT/NN) u.
template <typename T, int NN>
__device__ __forceinline__ void load_nc(const T* __restrict__ X, int64_t ld, int k0, int kend, int n0,
                                        int nend, T (&v)[KS * NN / NT]) {
  constexpr int KSTEP = NT / NN;
  const int t = threadIdx.x, n = n0 + t % NN, kb = t / NN;
#pragma unroll
  for (int u = 0; u < KS / KSTEP; ++u) {
    const int k = k0 + kb + KSTEP * u;
    v[u] = (k < kend && n < nend) ? X[(int64_t)k * ld + n] : T(0.0f);
  }
}
template <typename T, int NN, int LD>
__device__ __forceinline__ void store_nc(float* s, const T (&v)[KS * NN / NT]) {
  constexpr int KSTEP = NT / NN;
  const int t = threadIdx.x, n = t % NN, kb = t / NN;
#pragma unroll
  for (int u = 0; u < KS / KSTEP; ++u) s[(kb + KSTEP * u) * LD + n] = to_f32(v[u]);
}

// acc[bi][bj] += A[am0 + 32 bi .., :] B[:, bn0 + 32 bj ..] over one stage (KS values of k).
template <int BI, int BJ, int LDa, int LDb>
__device__ __forceinline__ void mma_stage(const float* sA, int am0, const float* sB, int bn0,
                                          f32x16 (&acc)[BI][BJ]) {
  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
#pragma unroll 4
  for (int ks = 0; ks < KS / 2; ++ks) {
    const int k = 2 * ks + h;
    float a[BI], b[BJ];
#pragma unroll
    for (int i = 0; i < BI; ++i) a[i] = sA[k * LDa + am0 + 32 * i + l32];
#pragma unroll
    for (int j = 0; j < BJ; ++j) b[j] = sB[k * LDb + bn0 + 32 * j + l32];
#pragma unroll
    for (int i = 0; i < BI; ++i)
#pragma unroll
      for (int j = 0; j < BJ; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
  }
}

// Row of accumulator register r of a 32 x 32 block held by lane half h (the lane holds column
// lane % 32).
__device__ __forceinline__ int acc_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// Partial S = Q R^T over the vocabulary chunk blockIdx.y (columns [chunk y, chunk (y+1))) for
// the 128 x 128 tile blockIdx.x, at part + y Bq Bd. Four waves of 64 x 64 (2 x 2 blocks).
template <typename T>
__global__ __launch_bounds__(NT) void loss_score_kernel(const T* __restrict__ Q, const T* __restrict__ R,
                                                        int Bq, int Bd, int V, int chunk,
                                                        float* __restrict__ part) {
  __shared__ float sA[KS * LDA];
  __shared__ float sB[KS * LDA];
  const int tj = (Bd + TM - 1) / TM;
  const int i0 = (blockIdx.x / tj) * TM, j0 = (blockIdx.x % tj) * TM;
  const int kc0 = blockIdx.y * chunk, kc1 = min(V, kc0 + chunk);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, wm = wave >> 1, wn = wave & 1;
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = zero16();
  T ra[16], rb[16];
  load_kc(Q, V, i0, Bq, kc0, kc1, ra);
  load_kc(R, V, j0, Bd, kc0, kc1, rb);
  for (int k0 = kc0; k0 < kc1; k0 += KS) {
    __syncthreads();  // the previous stage is read
    store_kc(sA, ra);
    store_kc(sB, rb);
    __syncthreads();
    if (k0 + KS < kc1) {  // the next stage's loads run under this stage's MFMAs
      load_kc(Q, V, i0, Bq, k0 + KS, kc1, ra);
      load_kc(R, V, j0, Bd, k0 + KS, kc1, rb);
    }
    mma_stage<2, 2, LDA, LDA>(sA, wm * 64, sB, wn * 64, acc);
  }
  float* out = part + (size_t)blockIdx.y * Bq * Bd;
  const int l32 = lane & 31, h = lane >> 5;
#pragma unroll
  for (int bi = 0; bi < 2; ++bi)
#pragma unroll
    for (int bj = 0; bj < 2; ++bj) {
      const int j = j0 + wn * 64 + 32 * bj + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = i0 + wm * 64 + 32 * bi + acc_row(r, h);
        if (i < Bq && j < Bd) out[(size_t)i * Bd + j] = acc[bi][bj][r];
      }
    }
}

// Per 64-column slice (blockIdx.x), at part + slice K: entries [0, Bq) and [Bq, Bq + Bd) the
// rows' sums of |x| over the slice, Bq + Bd and Bq + Bd + 1 the slice's sum_v (sum_b x)^2 of Q
// and of R. Wave w takes rows w, w + 4, ...; column sums are added over the waves in order.
template <typename T>
__global__ __launch_bounds__(NT) void loss_stats_kernel(const T* __restrict__ Q, const T* __restrict__ R,
                                                        int Bq, int Bd, int V, float* __restrict__ part,
                                                        int K) {
  __shared__ float cpart[4][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = blockIdx.x * 64 + lane;
  const bool cv = c < V;
  float* out = part + (size_t)blockIdx.x * K;
  for (int side = 0; side < 2; ++side) {
    const T* X = side ? R : Q;
    const int rows = side ? Bd : Bq, o = side ? Bq : 0;
    float cs = 0.0f;
    for (int b0 = wave; b0 < rows; b0 += 4 * ST_ROWS) {  // uniform per wave
      // every load issued, from clamped indices, before any is used
      T v[ST_ROWS];
#pragma unroll
      for (int u = 0; u < ST_ROWS; ++u)
        v[u] = X[(int64_t)min(b0 + 4 * u, rows - 1) * V + min(c, V - 1)];
#pragma unroll
      for (int u = 0; u < ST_ROWS; ++u)
        if (!(b0 + 4 * u < rows && cv)) v[u] = T(0.0f);
#pragma unroll
      for (int u = 0; u < ST_ROWS; ++u) {
        const int b = b0 + 4 * u;
        if (b < rows) {
          const float x = to_f32(v[u]);
          cs += x;
          const float a = wave_sum(fabsf(x));
          if (lane == 0) out[o + b] = a;
        }
      }
    }
    cpart[wave][lane] = cs;
    __syncthreads();
    if (wave == 0) {
      const float tot = ((cpart[0][lane] + cpart[1][lane]) + cpart[2][lane]) + cpart[3][lane];
      const float sq = wave_sum(tot * tot);
      if (lane == 0) out[Bq + Bd + side] = sq;
    }
    __syncthreads();
  }
}

// One wave per query row i: x = S[i, :] / T, the row's CE term logsumexp(x) - x[i] and
// P[i, j] = (softmax(x)_j - [i == j]) / (Bq T).
__global__ __launch_bounds__(NT) void loss_rows_kernel(const float* __restrict__ S, int Bq, int Bd,
                                                       float inv_t, float* __restrict__ row_loss,
                                                       float* __restrict__ probs) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int i = blockIdx.x * 4 + wave;
  if (i >= Bq) return;
  const float* srow = S + (size_t)i * Bd;
  float m = -INFINITY;
  for (int j = lane; j < Bd; j += 64) m = fmaxf(m, srow[j] * inv_t);
  m = wave_max(m);
  float s = 0.0f;
  for (int j = lane; j < Bd; j += 64) s += expf(srow[j] * inv_t - m);
  s = wave_sum(s);
  if (lane == 0) row_loss[i] = m + logf(s) - srow[i] * inv_t;
  const float rs = 1.0f / s, pscale = inv_t / (float)Bq;
  for (int j = lane; j < Bd; j += 64)
    probs[(size_t)i * Bd + j] = (expf(srow[j] * inv_t - m) * rs - (j == i ? 1.0f : 0.0f)) * pscale;
}

// One wave: the six scalars from the row CE terms and the summed statistics.
__global__ __launch_bounds__(64) void loss_final_large_kernel(const float* __restrict__ row_loss,
                                                              const float* __restrict__ stats, int Bq,
                                                              int Bd, int V, float w_ce, float w_l1,
                                                              float w_fl, float* __restrict__ out) {
  const int lane = threadIdx.x;
  float ce = 0.0f, l1q = 0.0f, l1d = 0.0f;
  if (Bd > 0)
    for (int i = lane; i < Bq; i += 64) ce += row_loss[i];
  for (int i = lane; i < Bq; i += 64) l1q += stats[i];
  for (int j = lane; j < Bd; j += 64) l1d += stats[Bq + j];
  ce = wave_sum(ce);
  l1q = wave_sum(l1q);
  l1d = wave_sum(l1d);
  if (lane == 0) {
    ce = Bd > 0 ? ce / (float)Bq : 0.0f;
    l1q /= (float)Bq;
    l1d = Bd > 0 ? l1d / (float)Bd : 0.0f;
    const float flq = stats[Bq + Bd] / (float)V, fld = stats[Bq + Bd + 1] / (float)V;
    out[0] = w_ce * ce + w_l1 * (l1q + l1d) + w_fl * (flq + fld);
    out[1] = ce;
    out[2] = l1q;
    out[3] = l1d;
    out[4] = flq;
    out[5] = fld;
  }
}

// ---- 16-bit reps on 16-bit MFMAs ----
//
// A product of two bf16 (or two fp16) values is exact in fp32, so for 16-bit reps the score
// GEMM runs on v_mfma_f32_32x32x16_{bf16,f16}: 8 times the k per instruction of the fp32
// MFMA, in the same 32 x 32 output layout. The stage's operands are kept in LDS as [row][k]
// 16-bit values, rows LDH apart: 80 bytes, so the 16 rows of one ds_read_b128 phase fall in
// distinct banks. A lane's MFMA operand (8 consecutive k of one row) is one 16-byte read.
// The global loads are those of the fp32 path (element by element: a row of V elements is
// not 16-byte aligned in general).
// The gradients' products P R and P^T Q take P (fp32) as two bf16 parts, p = hi + lo + r
// with |r| <= 2^-18 |p| (both round to nearest even, p - hi is exact), against R or Q exact
// in bf16: two MFMAs per step, lo first. fp16 reps keep the fp32 MFMA there (P's range does
// not fit fp16).
constexpr int LDH = 40;

template <typename T> struct Mfma16;
template <> struct Mfma16<bf16> {
  static __device__ __forceinline__ f32x16 run(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma16<f16> {
  static __device__ __forceinline__ f32x16 run(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

template <typename T> __device__ __forceinline__ uint16_t bits16(T x) {
  return __builtin_bit_cast(uint16_t, x);
}

// load_kc's registers (thread t: k = t % 32 of rows t / 32 + 8 u) into a [rows][KS] tile.
template <typename T>
__device__ __forceinline__ void store_kc16(uint16_t* s, const T (&v)[16]) {
  const int t = threadIdx.x, kk = t & 31, rb = t >> 5;
#pragma unroll
  for (int u = 0; u < 16; ++u) s[(rb + 8 * u) * LDH + kk] = bits16(v[u]);
}

// The operand of lane (l32, h) for k step s of a stage: row `row`, k = 16 s + 8 h .. + 7.
__device__ __forceinline__ u32x4 frag16(const uint16_t* s, int row, int ks) {
  const int h = (threadIdx.x & 63) >> 5;
  return *(const u32x4*)(s + row * LDH + 16 * ks + 8 * h);
}

// acc[bi][bj] += A[am0 + 32 bi .., :] B[bn0 + 32 bj .., :]^T over one stage.
template <typename T, int BI, int BJ>
__device__ __forceinline__ void mma16_stage(const uint16_t* sA, int am0, const uint16_t* sB, int bn0,
                                            f32x16 (&acc)[BI][BJ]) {
  const int l32 = threadIdx.x & 31;
#pragma unroll
  for (int ks = 0; ks < KS / 16; ++ks) {
    u32x4 a[BI], b[BJ];
#pragma unroll
    for (int i = 0; i < BI; ++i) a[i] = frag16(sA, am0 + 32 * i + l32, ks);
#pragma unroll
    for (int j = 0; j < BJ; ++j) b[j] = frag16(sB, bn0 + 32 * j + l32, ks);
#pragma unroll
    for (int i = 0; i < BI; ++i)
#pragma unroll
      for (int j = 0; j < BJ; ++j) acc[i][j] = Mfma16<T>::run(a[i], b[j], acc[i][j]);
  }
}

// loss_score_kernel for 16-bit reps.
template <typename T>
__global__ __launch_bounds__(NT) void loss_score16_kernel(const T* __restrict__ Q,
                                                          const T* __restrict__ R, int Bq, int Bd,
                                                          int V, int chunk, float* __restrict__ part) {
  __shared__ __attribute__((aligned(16))) uint16_t sA[TM * LDH];
  __shared__ __attribute__((aligned(16))) uint16_t sB[TM * LDH];
  const int tj = (Bd + TM - 1) / TM;
  const int i0 = (blockIdx.x / tj) * TM, j0 = (blockIdx.x % tj) * TM;
  const int kc0 = blockIdx.y * chunk, kc1 = min(V, kc0 + chunk);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, wm = wave >> 1, wn = wave & 1;
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = zero16();
  T ra[16], rb[16];
  load_kc(Q, V, i0, Bq, kc0, kc1, ra);
  load_kc(R, V, j0, Bd, kc0, kc1, rb);
  for (int k0 = kc0; k0 < kc1; k0 += KS) {
    __syncthreads();  // the previous stage is read
    store_kc16(sA, ra);
    store_kc16(sB, rb);
    __syncthreads();
    if (k0 + KS < kc1) {  // the next stage's loads run under this stage's MFMAs
      load_kc(Q, V, i0, Bq, k0 + KS, kc1, ra);
      load_kc(R, V, j0, Bd, k0 + KS, kc1, rb);
    }
    mma16_stage<T, 2, 2>(sA, wm * 64, sB, wn * 64, acc);
  }
  float* out = part + (size_t)blockIdx.y * Bq * Bd;
  const int l32 = lane & 31, h = lane >> 5;
#pragma unroll
  for (int bi = 0; bi < 2; ++bi)
#pragma unroll
    for (int bj = 0; bj < 2; ++bj) {
      const int j = j0 + wn * 64 + 32 * bj + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = i0 + wm * 64 + 32 * bi + acc_row(r, h);
        if (i < Bq && j < Bd) out[(size_t)i * Bd + j] = acc[bi][bj][r];
      }
    }
}

// p as bf16 hi and lo bits.
__device__ __forceinline__ void split_bf16(float p, uint16_t& hi, uint16_t& lo) {
  const bf16 h = (bf16)p;
  hi = bits16(h);
  lo = bits16((bf16)(p - (float)h));
}

// ---- bf16 gradients as one tiled GEMM grid ----
//
// Both gradients are GEMMs over the other side's rows plus per-element terms:
//   dQ = c_ce P R + ...  (K = Bd),   dR = c_ce P^T Q + ...  (K = Bq).
// A workgroup owns GC columns and row tile t of both (dQ rows and dR rows 128 t ..
// 128 t + 127; either may be empty), four waves of 64 x 64 per tile. The dQ GEMM streams
// all of R's rows for its columns, so it also sums R's columns (the FLOPS term of dR), and
// the dR GEMM sums Q's (that of dQ); a workgroup with only one of the tiles streams the
// other side for its sums alone. No workspace: everything stays in the workgroup.
constexpr int GC = 128;

// One GEMM tile: acc += A B^T over k in [0, K), A = P rows m0.. (A_KC) or P columns m0..,
// B = X[k][c0 ..] (bf16). cs accumulates thread t's share of X's column sums (column
// t % GC, k rows of parity t / GC). With MM false only the sums are taken.
template <bool A_KC, bool MM>
__device__ __forceinline__ void gemm16(uint16_t* sAh, uint16_t* sAl, uint16_t* sB,
                                       const float* __restrict__ P, int Bq, int Bd,
                                       const bf16* __restrict__ X, int K, int m0, int c0, int V,
                                       f32x16 (&acc)[2][2], float& cs) {
  const int t = threadIdx.x, wave = t >> 6, l32 = t & 31, wm = wave >> 1, wn = wave & 1;
  if (K <= 0) return;
  float pa[16];
  bf16 rbv[KS * GC / NT];
  auto load = [&](int k0) {
    if (MM) {
      if (A_KC) load_kc(P, Bd, m0, Bq, k0, K, pa);         // A[m][k] = P[m0 + m][k]
      else load_nc<float, TM>(P, Bd, k0, K, m0, Bd, pa);   // A[m][k] = P[k][m0 + m]
    }
    load_nc<bf16, GC>(X, V, k0, K, c0, V, rbv);            // B[n][k] = X[k][c0 + n]
  };
  load(0);
  for (int k0 = 0; k0 < K; k0 += KS) {
#pragma unroll
    for (int u = 0; u < KS * GC / NT; ++u) cs += to_f32(rbv[u]);
    if (MM) {
      __syncthreads();  // the previous stage is read
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        // load_kc: k = t % 32 of rows t / 32 + 8 u; load_nc<TM>: m = t % 128 of k rows t / 128 + 2 u
        const int m = A_KC ? (t >> 5) + 8 * u : t % TM;
        const int k = A_KC ? (t & 31) : t / TM + 2 * u;
        uint16_t hi, lo;
        split_bf16(pa[u], hi, lo);
        sAh[m * LDH + k] = hi;
        sAl[m * LDH + k] = lo;
      }
#pragma unroll
      for (int u = 0; u < KS * GC / NT; ++u)  // load_nc<GC>: n = t % GC of k rows t / GC + 2 u
        sB[(t % GC) * LDH + t / GC + (NT / GC) * u] = bits16(rbv[u]);
      __syncthreads();
    }
    if (k0 + KS < K) load(k0 + KS);  // the next stage's loads run under this stage's MFMAs
    if (MM) {
#pragma unroll
      for (int ks = 0; ks < KS / 16; ++ks) {
        u32x4 ah[2], al[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          ah[i] = frag16(sAh, wm * 64 + 32 * i + l32, ks);
          al[i] = frag16(sAl, wm * 64 + 32 * i + l32, ks);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) b[j] = frag16(sB, wn * 64 + 32 * j + l32, ks);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            acc[i][j] = Mfma16<bf16>::run(al[i], b[j], acc[i][j]);
            acc[i][j] = Mfma16<bf16>::run(ah[i], b[j], acc[i][j]);
          }
      }
    }
  }
}

// G[i][c] = c_ce acc + c_s sign(X[i][c]) + c_f colsum[c] for the tile's rows below `rows`.
__device__ __forceinline__ void grad16_epilogue(const f32x16 (&acc)[2][2], const bf16* __restrict__ X,
                                                int rows, int m0, int c0, int V, float c_ce,
                                                float c_s, float c_f, const float* colsum,
                                                bf16* __restrict__ G) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;
#pragma unroll
  for (int bj = 0; bj < 2; ++bj) {
    const int cl = wn * 64 + 32 * bj + l32, c = c0 + cl;
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
      bf16 xv[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = m0 + wm * 64 + 32 * bi + acc_row(r, h);
        xv[r] = (i < rows && c < V) ? X[(int64_t)i * V + c] : bf16(0.0f);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = m0 + wm * 64 + 32 * bi + acc_row(r, h);
        if (i < rows && c < V) {
          const float x = to_f32(xv[r]);
          const float sg = x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f);
          G[(int64_t)i * V + c] = from_f32<bf16>(c_ce * acc[bi][bj][r] + c_s * sg + c_f * colsum[cl]);
        }
      }
    }
  }
}

__global__ __launch_bounds__(NT) void loss_grad16_kernel(const bf16* __restrict__ Q,
                                                         const bf16* __restrict__ R,
                                                         const float* __restrict__ P, const Grads6 g,
                                                         int Bq, int Bd, int V, float w_ce,
                                                         float w_l1, float w_fl,
                                                         bf16* __restrict__ GQ,
                                                         bf16* __restrict__ GR) {
  __shared__ __attribute__((aligned(16))) uint16_t sAh[TM * LDH];
  __shared__ __attribute__((aligned(16))) uint16_t sAl[TM * LDH];
  __shared__ __attribute__((aligned(16))) uint16_t sB[GC * LDH];
  __shared__ float csp[2][2][GC];   // [side][k parity][column]
  __shared__ float colsum[2][GC];
  const int t = threadIdx.x;
  const int c0 = blockIdx.x * GC, m0 = blockIdx.y * TM;
  const bool has_q = m0 < Bq, has_r = m0 < Bd;
  f32x16 accq[2][2], accr[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      accq[i][j] = zero16();
      accr[i][j] = zero16();
    }
  float csq = 0.0f, csr = 0.0f;
  // dQ streams R (K = Bd): R's column sums for dR
  if (has_q) gemm16<true, true>(sAh, sAl, sB, P, Bq, Bd, R, Bd, m0, c0, V, accq, csr);
  else if (has_r) gemm16<true, false>(sAh, sAl, sB, P, Bq, Bd, R, Bd, m0, c0, V, accq, csr);
  // dR streams Q (K = Bq): Q's column sums for dQ
  if (has_r) gemm16<false, true>(sAh, sAl, sB, P, Bq, Bd, Q, Bq, m0, c0, V, accr, csq);
  else if (has_q) gemm16<false, false>(sAh, sAl, sB, P, Bq, Bd, Q, Bq, m0, c0, V, accr, csq);
  csp[0][t / GC][t % GC] = csq;
  csp[1][t / GC][t % GC] = csr;
  __syncthreads();
  if (t < 2 * GC) colsum[t / GC][t % GC] = csp[t / GC][0][t % GC] + csp[t / GC][1][t % GC];
  __syncthreads();
  const float g0 = grad_of(g, 0);
  const float c_ce = g0 * w_ce + grad_of(g, 1);
  const float c_sq = (g0 * w_l1 + grad_of(g, 2)) / (float)Bq;
  const float c_sd = Bd > 0 ? (g0 * w_l1 + grad_of(g, 3)) / (float)Bd : 0.0f;
  const float c_fq = 2.0f * (g0 * w_fl + grad_of(g, 4)) / (float)V;
  const float c_fd = 2.0f * (g0 * w_fl + grad_of(g, 5)) / (float)V;
  if (has_q) grad16_epilogue(accq, Q, Bq, m0, c0, V, c_ce, c_sq, c_fq, colsum[0], GQ);
  if (has_r) grad16_epilogue(accr, R, Bd, m0, c0, V, c_ce, c_sd, c_fd, colsum[1], GR);
}

// 128 rows of one gradient over the workgroup's 64 columns: acc = sum_k A[m][k] B[k][n] with A
// from a K-contiguous (P rows, dQ) or N-contiguous (P columns, dR) source; wave w owns rows
// 32 w .. 32 w + 31 (two 32 x 32 blocks). Then G = c_ce acc + c_s sign(X) + c_f colsum, in T.
template <typename T, bool A_KC>
__device__ __forceinline__ void grad_tile(float* sA, float* sB, const float* __restrict__ P,
                                          int Bq, int Bd, const T* __restrict__ Bsrc, int K,
                                          const T* __restrict__ X, int rows, int m0, int c0, int V,
                                          float c_ce, float c_s, float c_f, const float* colsum,
                                          T* __restrict__ G) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
  f32x16 acc[1][2] = {{zero16(), zero16()}};
  if (K > 0) {
    float pa[16];
    T rbv[KS * NC / NT];
    auto load_a = [&](int k0) {
      if (A_KC) {  // A[m][k] = P[m0 + m][k]: rows of P (dQ)
        load_kc(P, Bd, m0, Bq, k0, K, pa);
      } else {     // A[m][k] = P[k][m0 + m]: columns of P (dR)
        load_nc<float, TM>(P, Bd, k0, K, m0, Bd, pa);
      }
    };
    load_a(0);
    load_nc<T, NC>(Bsrc, V, 0, K, c0, V, rbv);
    for (int k0 = 0; k0 < K; k0 += KS) {
      __syncthreads();
      if (A_KC) store_kc(sA, pa);
      else store_nc<float, TM, LDA>(sA, pa);
      store_nc<T, NC, LDB>(sB, rbv);
      __syncthreads();
      if (k0 + KS < K) {
        load_a(k0 + KS);
        load_nc<T, NC>(Bsrc, V, k0 + KS, K, c0, V, rbv);
      }
      mma_stage<1, 2, LDA, LDB>(sA, wave * 32, sB, 0, acc);
    }
  }
#pragma unroll
  for (int bj = 0; bj < 2; ++bj) {
    const int cl = 32 * bj + l32, c = c0 + cl;
    T xv[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = m0 + wave * 32 + acc_row(r, h);
      xv[r] = (i < rows && c < V) ? X[(int64_t)i * V + c] : T(0.0f);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = m0 + wave * 32 + acc_row(r, h);
      if (i < rows && c < V) {
        const float x = to_f32(xv[r]);
        const float sg = x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f);
        G[(int64_t)i * V + c] = from_f32<T>(c_ce * acc[0][bj][r] + c_s * sg + c_f * colsum[cl]);
      }
    }
  }
}

template <typename T>
__global__ __launch_bounds__(NT) void loss_bwd_large_kernel(const T* __restrict__ Q, const T* __restrict__ R,
                                                            const float* __restrict__ P, const Grads6 g,
                                                            int Bq, int Bd, int V, float w_ce, float w_l1,
                                                            float w_fl, T* __restrict__ GQ,
                                                            T* __restrict__ GR) {
  __shared__ float sA[KS * LDA];
  __shared__ float sB[KS * LDB];
  __shared__ float cpart[2][4][NC];
  __shared__ float colsum[2][NC];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c0 = blockIdx.x * NC;
  // the columns' sums over Q's and R's rows: wave w sums rows w, w + 4, ... in order
  {
    const int c = c0 + lane;
    const bool cv = c < V;
    for (int side = 0; side < 2; ++side) {
      const T* X = side ? R : Q;
      const int rows = side ? Bd : Bq;
      float cs = 0.0f;
      for (int b0 = wave; b0 < rows; b0 += 4 * ST_ROWS) {
        T v[ST_ROWS];
#pragma unroll
        for (int u = 0; u < ST_ROWS; ++u)
          v[u] = X[(int64_t)min(b0 + 4 * u, rows - 1) * V + min(c, V - 1)];
#pragma unroll
        for (int u = 0; u < ST_ROWS; ++u)
          if (!(b0 + 4 * u < rows && cv)) v[u] = T(0.0f);
#pragma unroll
        for (int u = 0; u < ST_ROWS; ++u) cs += to_f32(v[u]);
      }
      cpart[side][wave][lane] = cs;
    }
  }
  __syncthreads();
  if (threadIdx.x < 2 * NC) {
    const int side = threadIdx.x / NC, l = threadIdx.x % NC;
    colsum[side][l] = ((cpart[side][0][l] + cpart[side][1][l]) + cpart[side][2][l]) + cpart[side][3][l];
  }
  __syncthreads();
  const float g0 = grad_of(g, 0);
  const float c_ce = g0 * w_ce + grad_of(g, 1);
  const float c_sq = (g0 * w_l1 + grad_of(g, 2)) / (float)Bq;
  const float c_sd = Bd > 0 ? (g0 * w_l1 + grad_of(g, 3)) / (float)Bd : 0.0f;
  const float c_fq = 2.0f * (g0 * w_fl + grad_of(g, 4)) / (float)V;
  const float c_fd = 2.0f * (g0 * w_fl + grad_of(g, 5)) / (float)V;
  for (int i0 = 0; i0 < Bq; i0 += TM)  // dQ = c_ce P R + ...
    grad_tile<T, true>(sA, sB, P, Bq, Bd, R, Bd, Q, Bq, i0, c0, V, c_ce, c_sq, c_fq, colsum[0], GQ);
  for (int j0 = 0; j0 < Bd; j0 += TM)  // dR = c_ce P^T Q + ...
    grad_tile<T, false>(sA, sB, P, Bq, Bd, Q, Bq, R, Bd, j0, c0, V, c_ce, c_sd, c_fd, colsum[1], GR);
}

// Score chunking: about 512 workgroups, chunks of whole LDS stages.
struct ScorePlan {
  int tiles, chunk, nchunk;
};
static ScorePlan score_plan(int64_t Bq, int64_t Bd, int64_t V) {
  ScorePlan p;
  p.tiles = (int)(cdiv(Bq, TM) * cdiv(Bd, TM));
  const int64_t want = cdiv(512, p.tiles);
  const int64_t nc = want < 1 ? 1 : (want > cdiv(V, 256) ? cdiv(V, 256) : want);
  p.chunk = (int)round_up(cdiv(V, nc), KS);
  p.nchunk = (int)cdiv(V, p.chunk);
  return p;
}
static int64_t stats_entries(int64_t Bq, int64_t Bd) { return Bq + Bd + 2; }
// Workspace (floats): partial S per chunk, S, partial stats per slice, stats, row CE terms.
static int64_t workspace_floats(int64_t Bq, int64_t Bd, int64_t V) {
  const int64_t s = Bd > 0 ? (int64_t)score_plan(Bq, Bd, V).nchunk * Bq * Bd + Bq * Bd : 0;
  return s + (slices(V) + 1) * stats_entries(Bq, Bd) + Bq;
}

// SPARTON_LOSS_MFMA16=0 keeps 16-bit reps on the fp32 MFMA (tests compare the two).
static bool mfma16_on() {
  const char* e = getenv("SPARTON_LOSS_MFMA16");
  return e == nullptr || strcmp(e, "0") != 0;
}

template <typename T>
static void fwd(const void* q, const void* d, int Bq, int Bd, int V, float inv_t, float w_ce,
                float w_l1, float w_fl, float* out, float* probs, float* ws, hipStream_t st) {
  float* spart = ws;
  float* S = nullptr;
  if (Bd > 0) {
    const ScorePlan p = score_plan(Bq, Bd, V);
    S = spart + (size_t)p.nchunk * Bq * Bd;
    const dim3 grid((unsigned)p.tiles, (unsigned)p.nchunk);
    if constexpr (sizeof(T) == 2) {
      if (mfma16_on()) {
        hipLaunchKernelGGL((loss_score16_kernel<T>), grid, dim3(NT), 0, st, (const T*)q, (const T*)d,
                           Bq, Bd, V, p.chunk, spart);
      } else {
        hipLaunchKernelGGL((loss_score_kernel<T>), grid, dim3(NT), 0, st, (const T*)q, (const T*)d,
                           Bq, Bd, V, p.chunk, spart);
      }
    } else {
      hipLaunchKernelGGL((loss_score_kernel<T>), grid, dim3(NT), 0, st, (const T*)q, (const T*)d,
                         Bq, Bd, V, p.chunk, spart);
    }
    const int K = Bq * Bd;
    hipLaunchKernelGGL(loss_slice_sum_kernel, dim3((unsigned)cdiv(K, 64)), dim3(64 * SUM_WAVES), 0, st,
                       (const float*)spart, p.nchunk, K, S);
  }
  float* tpart = Bd > 0 ? S + (size_t)Bq * Bd : ws;
  const int KS2 = (int)stats_entries(Bq, Bd), ns = (int)slices(V);
  float* stats = tpart + (size_t)ns * KS2;
  float* row_loss = stats + KS2;
  hipLaunchKernelGGL((loss_stats_kernel<T>), dim3((unsigned)ns), dim3(NT), 0, st, (const T*)q,
                     (const T*)d, Bq, Bd, V, tpart, KS2);
  hipLaunchKernelGGL(loss_slice_sum_kernel, dim3((unsigned)cdiv(KS2, 64)), dim3(64 * SUM_WAVES), 0, st,
                     (const float*)tpart, ns, KS2, stats);
  if (Bd > 0)
    hipLaunchKernelGGL(loss_rows_kernel, dim3((unsigned)cdiv(Bq, 4)), dim3(NT), 0, st, (const float*)S,
                       Bq, Bd, inv_t, row_loss, probs);
  hipLaunchKernelGGL(loss_final_large_kernel, dim3(1), dim3(64), 0, st, (const float*)row_loss,
                     (const float*)stats, Bq, Bd, V, w_ce, w_l1, w_fl, out);
}

template <typename T>
static void bwd(const void* q, const void* d, const float* P, const Grads6& g, int Bq, int Bd, int V,
                float w_ce, float w_l1, float w_fl, void* gq, void* gd, hipStream_t st) {
  if constexpr (std::is_same<T, bf16>::value) {
    if (mfma16_on()) {
      const dim3 grid((unsigned)cdiv(V, GC), (unsigned)cdiv(std::max(Bq, Bd), TM));
      hipLaunchKernelGGL(loss_grad16_kernel, grid, dim3(NT), 0, st, (const bf16*)q, (const bf16*)d, P,
                         g, Bq, Bd, V, w_ce, w_l1, w_fl, (bf16*)gq, (bf16*)gd);
      return;
    }
  }
  hipLaunchKernelGGL((loss_bwd_large_kernel<T>), dim3((unsigned)cdiv(V, NC)), dim3(NT), 0, st,
                     (const T*)q, (const T*)d, P, g, Bq, Bd, V, w_ce, w_l1, w_fl, (T*)gq, (T*)gd);
}
}  // namespace big

// Batches with more than MAX_B rows on either side take the kernels in `big`.
static bool is_big(int64_t Bq, int64_t Bd) { return Bq > MAX_B || Bd > MAX_B; }

}  // namespace loss
}  // namespace sparton

using namespace sparton;

static int loss_check(int64_t Bq, int64_t Bd, int64_t V, int dtype) {
  if (dtype < SPARTON_F32 || dtype > SPARTON_F16) return SPARTON_EINVAL;
  if (Bq < 1 || Bd < 0 || V < 1) return SPARTON_EINVAL;
  // int offsets: the scores and their per-chunk partials, and row * V + column
  if (V > INT32_MAX || Bq > INT32_MAX / 8 || Bd > INT32_MAX / 8 ||
      (Bd > 0 && Bq * Bd * (int64_t)loss::big::score_plan(Bq, Bd, V).nchunk > INT32_MAX) ||
      (Bq + Bd) * V > ((int64_t)1 << 62))
    return SPARTON_EUNSUPPORTED;
  if (Bd > 0 && Bq > Bd) return SPARTON_EINVAL;  // labels arange(Bq) index R's rows
  return SPARTON_OK;
}

extern "C" __attribute__((visibility("default"))) size_t sparton_loss_workspace_bytes(int64_t Bq,
                                                                                      int64_t Bd,
                                                                                      int64_t V) {
  if (Bq < 1 || Bd < 0 || V < 1) return 0;
  if (loss::is_big(Bq, Bd)) return (size_t)loss::big::workspace_floats(Bq, Bd, V) * sizeof(float);
  return (size_t)((loss::slices(V) + 1) * loss::entries(Bq, Bd)) * sizeof(float);
}

extern "C" __attribute__((visibility("default"))) int sparton_loss_fwd(
    const void* q, const void* d, int64_t Bq, int64_t Bd, int64_t V, float temperature, float w_ce,
    float w_l1, float w_flops, float* out, float* probs, void* workspace, size_t workspace_bytes,
    int dtype, void* stream) {
  const int rc = loss_check(Bq, Bd, V, dtype);
  if (rc != SPARTON_OK) return rc;
  if (q == nullptr || out == nullptr || (Bd > 0 && (d == nullptr || probs == nullptr)))
    return SPARTON_EINVAL;
  if (Bd > 0 && !(temperature > 0.0f && temperature < INFINITY)) return SPARTON_EINVAL;
  if (workspace == nullptr || workspace_bytes < sparton_loss_workspace_bytes(Bq, Bd, V))
    return SPARTON_EWORKSPACE;
  if ((uintptr_t)workspace % 16 != 0) return SPARTON_EALIGN;
  hipStream_t st = (hipStream_t)stream;
  if (loss::is_big(Bq, Bd)) {
    const float inv_t = Bd > 0 ? 1.0f / temperature : 0.0f;
    float* ws = (float*)workspace;
    switch (dtype) {
      case SPARTON_BF16:
        loss::big::fwd<bf16>(q, d, (int)Bq, (int)Bd, (int)V, inv_t, w_ce, w_l1, w_flops, out, probs, ws, st);
        break;
      case SPARTON_F16:
        loss::big::fwd<f16>(q, d, (int)Bq, (int)Bd, (int)V, inv_t, w_ce, w_l1, w_flops, out, probs, ws, st);
        break;
      default:
        loss::big::fwd<float>(q, d, (int)Bq, (int)Bd, (int)V, inv_t, w_ce, w_l1, w_flops, out, probs, ws, st);
        break;
    }
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? SPARTON_OK : (int)e;
  }
  const int K = (int)loss::entries(Bq, Bd), ns = (int)loss::slices(V);
  float* part = (float*)workspace;
  float* sums = part + (size_t)ns * K;
  switch (dtype) {
    case SPARTON_BF16: loss::fwd_partial<bf16>(q, d, (int)Bq, (int)Bd, (int)V, part, K, st); break;
    case SPARTON_F16: loss::fwd_partial<f16>(q, d, (int)Bq, (int)Bd, (int)V, part, K, st); break;
    default: loss::fwd_partial<float>(q, d, (int)Bq, (int)Bd, (int)V, part, K, st); break;
  }
  hipLaunchKernelGGL(loss::loss_slice_sum_kernel, dim3((unsigned)cdiv((int64_t)K, (int64_t)64)),
                     dim3(64 * loss::SUM_WAVES), 0, st, (const float*)part, ns, K, sums);
  hipLaunchKernelGGL(loss::loss_final_kernel, dim3(1), dim3(loss::NT), 0, st, (const float*)sums,
                     (int)Bq, (int)Bd, (int)V, Bd > 0 ? 1.0f / temperature : 0.0f, w_ce, w_l1,
                     w_flops, out, probs);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPARTON_OK : (int)e;
}

static int loss_bwd_run(const void* q, const void* d, const float* probs, const loss::Grads6& grad_out,
                        int64_t Bq, int64_t Bd, int64_t V, float w_ce, float w_l1, float w_flops,
                        void* grad_q, void* grad_d, int dtype, void* stream) {
  const int rc = loss_check(Bq, Bd, V, dtype);
  if (rc != SPARTON_OK) return rc;
  if (q == nullptr || grad_q == nullptr ||
      (Bd > 0 && (d == nullptr || probs == nullptr || grad_d == nullptr)))
    return SPARTON_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  if (loss::is_big(Bq, Bd)) {
    switch (dtype) {
      case SPARTON_BF16:
        loss::big::bwd<bf16>(q, d, probs, grad_out, (int)Bq, (int)Bd, (int)V, w_ce, w_l1, w_flops, grad_q,
                             grad_d, st);
        break;
      case SPARTON_F16:
        loss::big::bwd<f16>(q, d, probs, grad_out, (int)Bq, (int)Bd, (int)V, w_ce, w_l1, w_flops, grad_q,
                            grad_d, st);
        break;
      default:
        loss::big::bwd<float>(q, d, probs, grad_out, (int)Bq, (int)Bd, (int)V, w_ce, w_l1, w_flops, grad_q,
                              grad_d, st);
        break;
    }
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? SPARTON_OK : (int)e;
  }
  switch (dtype) {
    case SPARTON_BF16:
      loss::bwd_all<bf16>(q, d, probs, grad_out, (int)Bq, (int)Bd, (int)V, w_ce, w_l1, w_flops, grad_q,
                          grad_d, st);
      break;
    case SPARTON_F16:
      loss::bwd_all<f16>(q, d, probs, grad_out, (int)Bq, (int)Bd, (int)V, w_ce, w_l1, w_flops, grad_q,
                         grad_d, st);
      break;
    default:
      loss::bwd_all<float>(q, d, probs, grad_out, (int)Bq, (int)Bd, (int)V, w_ce, w_l1, w_flops,
                           grad_q, grad_d, st);
      break;
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPARTON_OK : (int)e;
}

extern "C" __attribute__((visibility("default"))) int sparton_loss_bwd(
    const void* q, const void* d, const float* probs, const float* grad_out, int64_t Bq, int64_t Bd,
    int64_t V, float w_ce, float w_l1, float w_flops, void* grad_q, void* grad_d, int dtype,
    void* stream) {
  if (grad_out == nullptr) return SPARTON_EINVAL;
  const loss::Grads6 g{{grad_out, grad_out + 1, grad_out + 2, grad_out + 3, grad_out + 4, grad_out + 5}};
  return loss_bwd_run(q, d, probs, g, Bq, Bd, V, w_ce, w_l1, w_flops, grad_q, grad_d, dtype, stream);
}

extern "C" __attribute__((visibility("default"))) int sparton_loss_bwd_terms(
    const void* q, const void* d, const float* probs, const float* const* grad_terms, int64_t Bq,
    int64_t Bd, int64_t V, float w_ce, float w_l1, float w_flops, void* grad_q, void* grad_d,
    int dtype, void* stream) {
  if (grad_terms == nullptr) return SPARTON_EINVAL;
  loss::Grads6 g;
  for (int k = 0; k < 6; ++k) g.p[k] = grad_terms[k];
  return loss_bwd_run(q, d, probs, g, Bq, Bd, V, w_ce, w_l1, w_flops, grad_q, grad_d, dtype, stream);
}
