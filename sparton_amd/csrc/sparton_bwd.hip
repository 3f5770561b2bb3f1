// SpartonHead backward on gfx950: atomic-free, deterministic, HBM-bound.
//
// Only entries (b,v) with reps > 0, G != 0 and mask[b,I] != 0 carry gradient
// (g' = G*exp(-reps)*mask[b,I]). The reference scatters them with fp32 atomics into
// zero-filled dH/dW/dbias (src/sparton/sparton_kernel.py:473-565, :676-678). Here
// every output row is produced by exactly one wave, summed in a fixed order:
//
//   dW / dbias  (bwd_dw_kernel)     row v gathers H[b, I[b,v], :] for b ascending.
//   dH          (hist -> scan -> scatter -> bwd_dh_kernel)
//       1. hist:    per (b, chunk of CH vocab ids), count active entries per s.
//       2. scan:    per b, exclusive scan in (s, chunk) order -> each (b,s) segment
//                   start, and each chunk's first slot inside every segment.
//       3. scatter: per (b, chunk), write (v, g') to its slot; the rank among equal
//                   s inside a 64-lane step comes from ballots, so each segment is
//                   ordered by v ascending (a stable counting sort by s).
//       4. dh:      one wave per (b,s) row sums g' * W[v,:] over its segment.
// Integer counts are the only LDS atomics; they are order-independent.

#include "sparton_common.h"

extern __shared__ __attribute__((aligned(16))) unsigned char sparton_bwd_smem[];

namespace sparton {
namespace bwd {

constexpr int CH = 2048;          // vocab ids per histogram chunk (one wave)
constexpr int MAX_S = 16384;      // per-wave LDS counters: S ints
constexpr int MAX_B = 8192;       // dW kernel stages g' for B x vblk entries in LDS
constexpr int DW_LDS_ENTRIES = 8192;  // B * vblk (8 bytes each -> 64 KB)
constexpr int VBLK_MAX = 16;      // vocab rows per dW workgroup
constexpr int PASS = 256;         // hidden elements per wave pass (4 per lane)

struct Layout {
  int64_t nch;
  size_t hist, seg_start, seg_cnt, list, total;
};

static Layout layout(int64_t B, int64_t S, int64_t V) {
  Layout L;
  L.nch = cdiv(V, CH);
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off += (size_t)round_up((int64_t)bytes, 256); return o; };
  L.hist = take((size_t)(B * L.nch * S) * 4);
  L.seg_start = take((size_t)(B * S) * 4);
  L.seg_cnt = take((size_t)(B * S) * 4);
  L.list = take((size_t)(B * V) * 8);
  L.total = off;
  return L;
}

static int waves_for(int64_t S) { return S <= 4096 ? 4 : 1; }

// ---- 1. histogram ----------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void bwd_hist_kernel(
    const T* __restrict__ grad, const void* __restrict__ reps, int reps_dtype,
    const int32_t* __restrict__ idx,
    const void* __restrict__ mask, int mask_dtype, int S, int V, int nch, int* __restrict__ hist) {
  int* lds = (int*)sparton_bwd_smem;
  const int wpb = blockDim.x >> 6, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int b = blockIdx.y, c = blockIdx.x * wpb + wave;
  int* h = lds + wave * S;
  for (int s = lane; s < S; s += 64) h[s] = 0;
  __syncthreads();
  if (c < nch) {
    const int vend = min(V, (c + 1) * CH);
    for (int v = c * CH + lane; v < vend; v += 64) {
      int s;
      float g;
      if (grad_entry(grad, reps, reps_dtype, idx, mask, mask_dtype, b, S, (int64_t)b * V + v, &g, &s))
        atomicAdd(&h[s], 1);
    }
  }
  __syncthreads();
  if (c < nch) {
    int* out = hist + ((int64_t)b * nch + c) * S;
    for (int s = lane; s < S; s += 64) out[s] = h[s];
  }
}

// Exclusive scan of one int per thread over a 256-thread block.
__device__ __forceinline__ int block_excl_scan(int x, int* tmp4) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int v = x;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(v, off);
    if (lane >= off) v += y;
  }
  if (lane == 63) tmp4[wave] = v;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += tmp4[w];
  __syncthreads();
  return base + v - x;
}

// ---- 2. scan ---------------------------------------------------------------
__global__ __launch_bounds__(256) void bwd_scan_kernel(int* __restrict__ hist, int* __restrict__ seg_start,
                                                       int* __restrict__ seg_cnt, int S, int nch) {
  int* tot = (int*)sparton_bwd_smem;  // [S]
  __shared__ int tmp4[4];
  const int b = blockIdx.x, tid = threadIdx.x;
  int* hb = hist + (int64_t)b * nch * S;
  for (int s = tid; s < S; s += 256) {
    int t = 0;
    for (int c = 0; c < nch; ++c) t += hb[(int64_t)c * S + s];
    tot[s] = t;
  }
  __syncthreads();
  const int per = (S + 255) / 256, beg = min(S, tid * per), end = min(S, beg + per);
  int local = 0;
  for (int s = beg; s < end; ++s) local += tot[s];
  int run = block_excl_scan(local, tmp4);
  for (int s = beg; s < end; ++s) {
    const int t = tot[s];
    tot[s] = run;
    seg_start[(int64_t)b * S + s] = run;
    seg_cnt[(int64_t)b * S + s] = t;
    run += t;
  }
  __syncthreads();
  for (int s = tid; s < S; s += 256) {
    int r = tot[s];
    for (int c = 0; c < nch; ++c) {
      int* p = hb + (int64_t)c * S + s;
      const int cnt = *p;
      *p = r;
      r += cnt;
    }
  }
}

// ---- 3. scatter ------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void bwd_scatter_kernel(
    const T* __restrict__ grad, const void* __restrict__ reps, int reps_dtype,
    const int32_t* __restrict__ idx,
    const void* __restrict__ mask, int mask_dtype, int S, int V, int nch,
    const int* __restrict__ hist_base, int2* __restrict__ list) {
  int* lds = (int*)sparton_bwd_smem;
  const int wpb = blockDim.x >> 6, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int b = blockIdx.y, c = blockIdx.x * wpb + wave;
  int* cur = lds + wave * S;
  if (c < nch) {
    const int* in = hist_base + ((int64_t)b * nch + c) * S;
    for (int s = lane; s < S; s += 64) cur[s] = in[s];
  }
  __syncthreads();
  if (c >= nch) return;
  int2* lb = list + (int64_t)b * V;
  const uint64_t lt = (1ull << lane) - 1ull;
  const int vend = min(V, (c + 1) * CH);
  for (int vs = c * CH; vs < vend; vs += 64) {
    const int v = vs + lane;
    float g = 0.0f;
    int s = 0;
    const bool act =
        v < vend && grad_entry(grad, reps, reps_dtype, idx, mask, mask_dtype, b, S, (int64_t)b * V + v, &g, &s);
    uint64_t pending = __ballot(act);
    while (pending) {
      const int leader = __ffsll((unsigned long long)pending) - 1;
      const int ls = __builtin_amdgcn_readlane(s, leader);
      const bool mine = act && s == ls;
      const uint64_t grp = __ballot(mine);
      const int base = cur[ls];
      if (mine) lb[base + __popcll(grp & lt)] = make_int2(v, __float_as_int(g));
      if (lane == leader) cur[ls] = base + __popcll(grp);
      pending &= ~grp;
    }
  }
}

// ---- 4. dH -----------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void bwd_dh_kernel(
    const T* __restrict__ W, const int2* __restrict__ list, const int* __restrict__ seg_start,
    const int* __restrict__ seg_cnt, float* __restrict__ dH, int B, int S, int D, int V) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= (int64_t)B * S) return;
  const int64_t b = row / S;
  const int start = seg_start[row], cnt = seg_cnt[row];
  const int2* seg = list + b * V + start;
  float* out = dH + row * D;
  for (int d0 = 0; d0 < D; d0 += PASS) {
    const int d = d0 + lane * 4;
    const bool dv = d < D;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int e0 = 0; e0 < cnt; e0 += 64) {
      const int2 ent = e0 + lane < cnt ? seg[e0 + lane] : make_int2(0, 0);
      const int n = min(64, cnt - e0);
      if (dv) {
        for (int j = 0; j < n; ++j) {
          const int v = __builtin_amdgcn_readlane(ent.x, j);
          const float g = __int_as_float(__builtin_amdgcn_readlane(ent.y, j));
          acc += g * load4(W + (int64_t)v * D + d);
        }
      }
    }
    if (dv) *(f32x4*)(out + d) = acc;
  }
}

// ---- 5. dW and dbias ---------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void bwd_dw_kernel(
    const T* __restrict__ grad, const void* __restrict__ reps, int reps_dtype,
    const int32_t* __restrict__ idx,
    const void* __restrict__ mask, int mask_dtype, const T* __restrict__ H,
    float* __restrict__ dW, float* __restrict__ dbias, int B, int S, int D, int V, int vblk) {
  float* gp = (float*)sparton_bwd_smem;   // [B][vblk]
  int* si = (int*)(gp + (int64_t)B * vblk);  // [B][vblk]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int v0 = blockIdx.x * vblk;
  for (int i = tid; i < B * vblk; i += 256) {
    const int bb = i / vblk, j = i - bb * vblk, v = v0 + j;
    float g = 0.0f;
    int s = 0;
    if (v < V) grad_entry(grad, reps, reps_dtype, idx, mask, mask_dtype, bb, S, (int64_t)bb * V + v, &g, &s);
    gp[i] = g;   // 0 for inactive entries, which the gather loop skips
    si[i] = s;
  }
  __syncthreads();
  if (dbias != nullptr && tid < vblk && v0 + tid < V) {
    float sum = 0.0f;
    for (int bb = 0; bb < B; ++bb) sum += gp[bb * vblk + tid];
    dbias[v0 + tid] = sum;
  }
  if (dW == nullptr) return;
  for (int j = wave; j < vblk; j += 4) {
    const int v = v0 + j;
    if (v >= V) break;
    for (int d0 = 0; d0 < D; d0 += PASS) {
      const int d = d0 + lane * 4;
      if (d < D) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int bb = 0; bb < B; ++bb) {
          const float g = gp[bb * vblk + j];
          if (g != 0.0f) {
            const int s = si[bb * vblk + j];
            acc += g * load4(H + ((int64_t)bb * S + s) * D + d);
          }
        }
        *(f32x4*)(dW + (int64_t)v * D + d) = acc;
      }
    }
  }
}

template <typename T>
static int launch(const void* grad, const void* r, int rdt, const int32_t* idx, const void* mask,
                  int mdt, const void* H, const void* W, float* dH, float* dW, float* dbias,
                  void* ws, int64_t B, int64_t S, int64_t D, int64_t V, hipStream_t st) {
  const T* g = (const T*)grad;
  if (dH != nullptr && B * S > 0 && D > 0) {
    const Layout L = layout(B, S, V);
    int* hist = (int*)((char*)ws + L.hist);
    int* seg_start = (int*)((char*)ws + L.seg_start);
    int* seg_cnt = (int*)((char*)ws + L.seg_cnt);
    int2* list = (int2*)((char*)ws + L.list);
    const int wpb = waves_for(S);
    const dim3 cgrid((unsigned)cdiv(L.nch, wpb), (unsigned)B);
    const size_t cl = (size_t)wpb * S * 4;
    if (L.nch > 0)
      hipLaunchKernelGGL(bwd_hist_kernel<T>, cgrid, dim3(64 * wpb), cl, st, g, r, rdt, idx, mask, mdt,
                         (int)S, (int)V, (int)L.nch, hist);
    hipLaunchKernelGGL(bwd_scan_kernel, dim3((unsigned)B), dim3(256), (size_t)S * 4, st, hist,
                       seg_start, seg_cnt, (int)S, (int)L.nch);
    if (L.nch > 0)
      hipLaunchKernelGGL(bwd_scatter_kernel<T>, cgrid, dim3(64 * wpb), cl, st, g, r, rdt, idx, mask,
                         mdt, (int)S, (int)V, (int)L.nch, (const int*)hist, list);
    hipLaunchKernelGGL(bwd_dh_kernel<T>, dim3((unsigned)cdiv(B * S, 4)), dim3(256), 0, st,
                       (const T*)W, (const int2*)list, (const int*)seg_start, (const int*)seg_cnt,
                       dH, (int)B, (int)S, (int)D, (int)V);
  }
  if ((dW != nullptr || dbias != nullptr) && V > 0) {
    const int vblk = B > 0 ? (int)std::min<int64_t>(VBLK_MAX, DW_LDS_ENTRIES / B) : VBLK_MAX;
    hipLaunchKernelGGL(bwd_dw_kernel<T>, dim3((unsigned)cdiv(V, vblk)), dim3(256),
                       (size_t)B * vblk * 8, st, g, r, rdt, idx, mask, mdt, (const T*)H, dW, dbias,
                       (int)B, (int)S, (int)D, (int)V, vblk);
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPARTON_OK : (int)e;
}

}  // namespace bwd
}  // namespace sparton

using namespace sparton;

extern "C" __attribute__((visibility("default"))) size_t sparton_bwd_workspace_bytes(
    int64_t B, int64_t S, int64_t D, int64_t V) {
  if (B <= 0 || S <= 0 || D <= 0 || V < 0) return 0;
  return bwd::layout(B, S, V).total;
}

extern "C" __attribute__((visibility("default"))) int sparton_bwd(
    const void* grad_reps, const void* reps, int reps_dtype, const int32_t* argmax,
    const void* mask, int mask_dtype, const void* hidden, const void* weight, float* d_hidden,
    float* d_weight, float* d_bias, void* workspace, size_t workspace_bytes, int64_t B, int64_t S,
    int64_t D, int64_t V, int dtype, void* stream) {
  if (B < 0 || S < 0 || D < 0 || V < 0) return SPARTON_EINVAL;
  if (dtype < SPARTON_F32 || dtype > SPARTON_F16) return SPARTON_EINVAL;
  if (reps_dtype < SPARTON_F32 || reps_dtype > SPARTON_F16) return SPARTON_EINVAL;
  if (mask_dtype < SPARTON_MASK_I64 || mask_dtype > SPARTON_MASK_F16) return SPARTON_EINVAL;
  if (B * V > 0 && (grad_reps == nullptr || reps == nullptr || argmax == nullptr || mask == nullptr))
    return SPARTON_EINVAL;
  const bool need_dh = d_hidden != nullptr && B * S > 0 && D > 0;
  const bool need_dw = (d_weight != nullptr || d_bias != nullptr) && V > 0;
  if (need_dh && weight == nullptr) return SPARTON_EINVAL;
  if (need_dw && d_weight != nullptr && D > 0 && B * S > 0 && hidden == nullptr) return SPARTON_EINVAL;
  const int64_t esz = dtype == SPARTON_F32 ? 4 : 2;
  if ((D * esz) % 16 != 0) return SPARTON_EINVAL;
  if (((uintptr_t)hidden | (uintptr_t)weight | (uintptr_t)d_hidden | (uintptr_t)d_weight) % 16 != 0)
    return SPARTON_EALIGN;
  if (B > bwd::MAX_B || S > bwd::MAX_S) return SPARTON_EUNSUPPORTED;
  if (D > INT32_MAX || V > INT32_MAX || B * S > INT32_MAX || B * V > INT32_MAX)
    return SPARTON_EUNSUPPORTED;
  if (need_dh) {
    if (workspace == nullptr) return SPARTON_EWORKSPACE;
    if (workspace_bytes < bwd::layout(B, S, V).total) return SPARTON_EWORKSPACE;
    if ((uintptr_t)workspace % 256 != 0) return SPARTON_EALIGN;
  }
  if (!need_dh && !need_dw) return SPARTON_OK;
  hipStream_t st = (hipStream_t)stream;
  float* dh = need_dh ? d_hidden : nullptr;
  switch (dtype) {
    case SPARTON_BF16:
      return bwd::launch<bf16>(grad_reps, reps, reps_dtype, argmax, mask, mask_dtype, hidden, weight, dh,
                               d_weight, d_bias, workspace, B, S, D, V, st);
    case SPARTON_F16:
      return bwd::launch<f16>(grad_reps, reps, reps_dtype, argmax, mask, mask_dtype, hidden, weight, dh,
                              d_weight, d_bias, workspace, B, S, D, V, st);
    default:
      return bwd::launch<float>(grad_reps, reps, reps_dtype, argmax, mask, mask_dtype, hidden, weight, dh,
                                d_weight, d_bias, workspace, B, S, D, V, st);
  }
}
