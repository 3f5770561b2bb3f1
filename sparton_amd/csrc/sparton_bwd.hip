// SpartonHead backward on gfx950: atomic-free on floating-point data, deterministic,
// HBM-bound.
//
// Only entries (b,v) with reps > 0, G != 0 and mask[b,I] != 0 carry gradient
// (g' = G*exp(-reps)*mask[b,I]). The reference scatters them with fp32 atomics into
// zero-filled dH/dW/dbias (src/sparton/sparton_kernel.py:473-565, :676-678). Here
// every output row is produced by exactly one wave and summed in a fixed order:
//
//   dW / dbias  (bwd_dw_kernel)   row v gathers H[b, I[b,v], :] for b ascending.
//   dH          (count -> scan -> scatter -> bwd_dh_kernel)
//       1. count:   per (b, wave chunk of CHW vocab ids), active entries per s,
//                   stored as hist[b][chunk][s]; the active entries (v, g') are also
//                   compacted, in v order, into the chunk's slice of the workspace.
//       2. scan:    per b, the exclusive scan of hist[b] in (s, chunk) order -> each
//                   (b,s) segment start and each chunk's first slot inside it (one
//                   thread per s sums its chunks; a block scan over s gives the bases).
//       3. scatter: per (b, chunk), write its compacted entries to their slots, ranked
//                   among equal s with one ballot per bit of s, so each segment lists
//                   its vocab ids in ascending order (a stable counting sort).
//       4. dh:      one wave per (b,s) row sums g' * W[v,:] over its segment,
//                   gathering several W rows per batch before accumulating.
//   dW / dbias for B <= 128 and S <= 65536 (bwd_dw_staged_kernel): a workgroup stages g'
//   and I of all batch rows for 64 consecutive vocab ids in LDS (coalesced loads), then
//   each wave gathers the H rows of one id at a time.
//   The fused path (B <= 128, S <= 1024, V <= 65536; configs 2 and 3) is two launches:
//   bwd_compact_kernel lists each (b, 64-id block)'s active entries sorted by 16-row
//   range, and bwd_fused_kernel runs the dH workgroups (one per (b, 8 rows), which
//   gather the entries of their rows from every block) and the staged dW workgroups
//   side by side.
// The only atomics are integer counts in LDS, which are order-independent.
//
// Gradients are written as fp32 (what the reference returns) or in the input dtype
// (what autograd would cast them to for bf16/fp16 parameters), rounded once from
// the fp32 sums.

#include <stdlib.h>
#include <string.h>

#include "sparton_common.h"

extern __shared__ __attribute__((aligned(16))) unsigned char sparton_bwd_smem[];

namespace sparton {
namespace bwd {

constexpr int CHW = 1024;          // vocab ids per wave chunk (16 rounds of 64 lanes)
constexpr int ROUNDS = CHW / 64;
constexpr int MAX_S = 16384;       // positions per dH window (LDS: S mask floats + S counters per wave)
constexpr int MAX_B = 8192;        // batch rows per dH chunk
constexpr int MAX_NP = 16;         // D up to 16 * 256 per register pass

struct Layout {
  int64_t nch;
  size_t hist, seg_start, seg_cnt, list, comp, ccount, cnt64, off64, hot, total;  // hist: [B][nch][S] int32
};

static Layout layout(int64_t B, int64_t S, int64_t V) {
  Layout L;
  L.nch = cdiv(V, CHW);
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off += (size_t)round_up((int64_t)bytes, 256); return o; };
  L.hist = take((size_t)(B * L.nch * S) * 4);
  L.seg_start = take((size_t)(B * S) * 4);
  L.seg_cnt = take((size_t)(B * S) * 4);
  // [B][V] segment lists; the fused path keeps [B][V/64][64] compacted entries here
  L.list = take((size_t)(B * round_up(V, 64)) * 8);
  L.comp = take((size_t)(B * L.nch * CHW) * 8);  // [B][nch][CHW] active (v, g') per chunk
  L.ccount = take((size_t)(B * L.nch) * 4);      // [B][nch] their number
  L.hot = take((size_t)(B * S + 1) * 4);          // [0]: hot rows; [1 ..]: their (b * S + s)
  L.cnt64 = take((size_t)(B * cdiv(V, 64)) * 4);  // fused path: [B][V/64] entries per block
  L.off64 = take((size_t)(B * cdiv(V, 64) * cdiv(std::min<int64_t>(S, 1024), 16)) * 4);  // and per row range
  L.total = off;
  return L;
}

// The workspace of one dH pass (at most MAX_B batch rows x MAX_S positions); the fused
// path's layout (B <= DW_STAGE_B, S <= FUSE_MAX_S) is the same.
static Layout pass_layout(int64_t B, int64_t S, int64_t V) {
  return layout(std::min<int64_t>(B, MAX_B), std::min<int64_t>(S, MAX_S), V);
}

// Waves per block of the count/scatter kernels: LDS holds S mask floats plus S
// counters per wave (at most 40 KB with 4 waves, 128 KB with one wave at MAX_S).
static int waves_for(int64_t S) { return S <= 2048 ? 4 : 1; }

// Stage the S mask entries from element `off` on as floats in LDS.
__device__ __forceinline__ void stage_mask(float* maskf, const void* mask, int mdt, int64_t off,
                                           int S) {
  for (int s = threadIdx.x; s < S; s += blockDim.x) maskf[s] = load_mask(mask, mdt, off + s);
}

// Entry (b, v): whether it carries gradient, its coefficient g' and index s.
// Activity is decided by comparisons of loaded values only (never by the float
// product), so the count and scatter kernels agree on every entry; an index outside
// [0, S) makes the entry inactive, so it can never turn into an out-of-bounds access.
// g' = G * exp(-reps) (src/sparton/sparton_kernel.py:531) times mask[b, I], the torch
// head's d x / d logits (training/model.py:60); 1 for a 0/1 mask.
template <typename T, typename RT>
__device__ __forceinline__ bool entry(T g_raw, RT r_raw, int s, const float* maskf, int S,
                                      float* g_out) {
  *g_out = 0.0f;
  const float r = to_f32(r_raw);
  if (!(r > 0.0f) || s < 0 || s >= S) return false;
  const float g = to_f32(g_raw);
  if (g == 0.0f) return false;
  const float m = maskf[s];
  if (m == 0.0f) return false;
  *g_out = g * expf(-r) * m;
  return true;
}

// This wave's chunk of row b: round j, lane l holds entry v = base + j*64 + l, so every
// load instruction reads consecutive elements. All 3 * ROUNDS loads are issued up front
// and unconditionally (ids past V re-read id V-1 and are marked inactive): no value is
// converted or tested until every load is in flight, so they overlap instead of each
// waiting for the previous one.
template <typename T, typename RT>
struct ChunkData {
  T g[ROUNDS];
  RT r[ROUNDS];
  int s[ROUNDS];
  __device__ __forceinline__ void load(const T* grad, const RT* reps, const int32_t* idx,
                                       int64_t row, int base, int V, int lane) {
#pragma unroll
    for (int j = 0; j < ROUNDS; ++j) {
      const int64_t o = row + min(base + j * 64 + lane, V - 1);
      g[j] = grad[o];
      r[j] = reps[o];
      s[j] = idx[o];
    }
  }
  // Entry j of this lane (v = base + j*64 + lane): active, with coefficient *g.
  __device__ __forceinline__ bool get(int j, int base, int V, int lane, const float* maskf,
                                      int S, float* gout) const {
    if (base + j * 64 + lane >= V) {
      *gout = 0.0f;
      return false;
    }
    return entry(g[j], r[j], s[j], maskf, S, gout);
  }
};

// ---- 1. count ----------------------------------------------------------------
template <typename T, typename RT>
__global__ __launch_bounds__(256) void bwd_count_kernel(
    const T* __restrict__ grad, const RT* __restrict__ reps, const int32_t* __restrict__ idx,
    const void* __restrict__ mask, int mdt, int S, int V, int nch, int* __restrict__ hist,
    int2* __restrict__ comp, int* __restrict__ ccount, int s0, int64_t mrow0, int S_row,
    int* __restrict__ hot) {
  float* maskf = (float*)sparton_bwd_smem;
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) hot[0] = 0;  // the scan lists them
  const int wpb = blockDim.x >> 6, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  int* h = (int*)(maskf + S) + wave * S;
  const int b = blockIdx.y, c = blockIdx.x * wpb + wave;
  stage_mask(maskf, mask, mdt, (mrow0 + b) * S_row + s0, S);
  for (int s = lane; s < S; s += 64) h[s] = 0;
  __syncthreads();
  if (c < nch) {
    ChunkData<T, RT> d;
    d.load(grad, reps, idx, (int64_t)b * V, c * CHW, V, lane);
    // Positions relative to the window (wrapping: an index outside it lands outside
    // [0, S) and the entry is inactive).
#pragma unroll
    for (int j = 0; j < ROUNDS; ++j) d.s[j] = (int)((unsigned)d.s[j] - (unsigned)s0);
    // Active entries are also compacted, in v order, into the chunk's slice of comp.
    int2* cb = comp + ((int64_t)b * nch + c) * CHW;
    const uint64_t lt = (1ull << lane) - 1ull;
    int n = 0;
#pragma unroll
    for (int j = 0; j < ROUNDS; ++j) {
      float g;
      const bool act = d.get(j, c * CHW, V, lane, maskf, S, &g);
      const uint64_t am = __ballot(act);
      if (act) {
        atomicAdd(&h[d.s[j]], 1);
        cb[n + __popcll(am & lt)] = make_int2(c * CHW + j * 64 + lane, __float_as_int(g));
      }
      n += __popcll(am);
    }
    if (lane == 0) ccount[(int64_t)b * nch + c] = n;
  }
  __syncthreads();
  if (c < nch) {
    int* out = hist + ((int64_t)b * nch + c) * S;
    for (int s = lane; s < S; s += 64) out[s] = h[s];
  }
}

// ---- 2. scan -----------------------------------------------------------------
constexpr int SCAN_THREADS = 1024;
constexpr int SCAN_BATCH = 8;  // chunk counts loaded together

// One workgroup per batch row, threads over s: thread s sums its chunks' counts
// hist[b][c][s] (coalesced across threads), a block scan over s gives the segment
// starts, and a second pass rewrites each count as its chunk's first slot.
// Both scans also list the rows with more than hot_min entries (hot[0] counts them, set
// to 0 by the count kernel; integer atomics, so only the list's order varies).
__device__ __forceinline__ void list_hot_row(int* hot, int hot_min, int64_t row, int cnt) {
  if (cnt > hot_min) hot[1 + atomicAdd(&hot[0], 1)] = (int)row;
}

__global__ __launch_bounds__(SCAN_THREADS) void bwd_scan_kernel(int* __restrict__ hist,
                                                                int* __restrict__ seg_start,
                                                                int* __restrict__ seg_cnt, int S,
                                                                int nch, int* __restrict__ hot,
                                                                int hot_min) {
  __shared__ int wsum[SCAN_THREADS / 64];
  __shared__ int carry;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t b = blockIdx.x;
  int* hb = hist + b * nch * S;
  if (tid == 0) carry = 0;
  __syncthreads();
  for (int s0 = 0; s0 < S; s0 += blockDim.x) {
    const int s = s0 + tid;
    const bool in = s < S;
    int tot = 0;
    for (int c0 = 0; c0 < nch; c0 += SCAN_BATCH) {
      int x[SCAN_BATCH];
#pragma unroll
      for (int i = 0; i < SCAN_BATCH; ++i)
        x[i] = (in && c0 + i < nch) ? hb[(int64_t)(c0 + i) * S + s] : 0;
#pragma unroll
      for (int i = 0; i < SCAN_BATCH; ++i) tot += x[i];
    }
    int incl = tot;  // inclusive scan over s: within the wave, then across waves
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(incl, d);
      if (lane >= d) incl += y;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int run = carry + incl - tot;
    for (int w = 0; w < wave; ++w) run += wsum[w];
    if (in) {
      seg_start[b * S + s] = run;
      seg_cnt[b * S + s] = tot;
      list_hot_row(hot, hot_min, b * S + s, tot);
    }
    for (int c0 = 0; c0 < nch; c0 += SCAN_BATCH) {
      int x[SCAN_BATCH];
#pragma unroll
      for (int i = 0; i < SCAN_BATCH; ++i)
        x[i] = (in && c0 + i < nch) ? hb[(int64_t)(c0 + i) * S + s] : 0;
#pragma unroll
      for (int i = 0; i < SCAN_BATCH; ++i) {
        if (in && c0 + i < nch) hb[(int64_t)(c0 + i) * S + s] = run;
        run += x[i];
      }
    }
    __syncthreads();
    if (tid == (int)blockDim.x - 1) carry = run;
    __syncthreads();
  }
}

// S <= 512: one workgroup of SCAN_THREADS per batch row, as P = floor(SCAN_THREADS / Sr)
// parts of Sr = round_up(S, 64) positions (the remaining threads idle); part p sums and rewrites chunks [p n / P, (p + 1) n / P)
// of every position, so every thread works instead of S of them. Part 0 scans the
// positions' totals; each part then starts its chunks at the position's segment start
// plus the counts of the parts before it (integer sums: the same offsets as above).
__global__ __launch_bounds__(SCAN_THREADS) void bwd_scan_parts_kernel(int* __restrict__ hist,
                                                                      int* __restrict__ seg_start,
                                                                      int* __restrict__ seg_cnt,
                                                                      int S, int nch, int Sr,
                                                                      int* __restrict__ hot,
                                                                      int hot_min) {
  __shared__ int ptot[SCAN_THREADS];
  __shared__ int base[SCAN_THREADS];
  __shared__ int wsum[SCAN_THREADS / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int P = SCAN_THREADS / Sr;            // Sr need not divide SCAN_THREADS:
  const int part = tid / Sr, s = tid - part * Sr;
  const bool in = s < S && part < P;          // threads past P * Sr take no chunks
  const int c_beg = part < P ? (int)((int64_t)nch * part / P) : 0;
  const int c_end = part < P ? (int)((int64_t)nch * (part + 1) / P) : 0;
  const int64_t b = blockIdx.x;
  int* hb = hist + b * nch * S;
  int tot = 0;
  for (int c0 = c_beg; c0 < c_end; c0 += SCAN_BATCH) {
    int x[SCAN_BATCH];
#pragma unroll
    for (int i = 0; i < SCAN_BATCH; ++i)
      x[i] = (in && c0 + i < c_end) ? hb[(int64_t)(c0 + i) * S + s] : 0;
#pragma unroll
    for (int i = 0; i < SCAN_BATCH; ++i) tot += x[i];
  }
  ptot[tid] = tot;
  __syncthreads();
  int t = 0, incl = 0;
  if (part == 0) {  // waves 0 .. Sr/64 - 1: the positions' totals and their inclusive scan
    for (int q = 0; q < P; ++q) t += ptot[q * Sr + s];
    incl = t;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(incl, d);
      if (lane >= d) incl += y;
    }
    if (lane == 63) wsum[wave] = incl;
  }
  __syncthreads();
  if (part == 0) {
    int run = incl - t;
    for (int w = 0; w < wave; ++w) run += wsum[w];
    if (in) {
      seg_start[b * S + s] = run;
      seg_cnt[b * S + s] = t;
      list_hot_row(hot, hot_min, b * S + s, t);
    }
    base[s] = run;
  }
  __syncthreads();
  int off = base[s];
  for (int q = 0; q < part; ++q) off += ptot[q * Sr + s];
  for (int c0 = c_beg; c0 < c_end; c0 += SCAN_BATCH) {
    int x[SCAN_BATCH];
#pragma unroll
    for (int i = 0; i < SCAN_BATCH; ++i)
      x[i] = (in && c0 + i < c_end) ? hb[(int64_t)(c0 + i) * S + s] : 0;
#pragma unroll
    for (int i = 0; i < SCAN_BATCH; ++i) {
      if (in && c0 + i < c_end) hb[(int64_t)(c0 + i) * S + s] = off;
      off += x[i];
    }
  }
}

// ---- 3. scatter ----------------------------------------------------------------
// One wave per chunk: its compacted entries (in v order) are ranked among equal s and
// written to their segments. Lanes with equal s are found with one ballot per bit of
// s: `same` keeps the lanes that agree with this lane on every bit. An entry's slot is
// the cursor of its s plus the lower lanes of its group; all lanes read the cursor,
// then each group's lowest lane advances it (one wave's LDS accesses complete in
// program order), so each segment lists its vocab ids in ascending order.
__global__ __launch_bounds__(256) void bwd_scatter_kernel(
    const int32_t* __restrict__ idx, int S, int V, int nch, const int* __restrict__ hist_base,
    const int2* __restrict__ comp, const int* __restrict__ ccount, int2* __restrict__ list,
    int s0) {
  int* cur = (int*)sparton_bwd_smem + (threadIdx.x >> 6) * S;
  const int wpb = blockDim.x >> 6, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int b = blockIdx.y, c = blockIdx.x * wpb + wave;
  if (c >= nch) return;  // no workgroup barrier below: waves are independent
  const int* in = hist_base + ((int64_t)b * nch + c) * S;
  for (int s = lane; s < S; s += 64) cur[s] = in[s];
  const int n = ccount[(int64_t)b * nch + c];
  const int2* cb = comp + ((int64_t)b * nch + c) * CHW;
  int2* lb = list + (int64_t)b * V;
  const int32_t* ib = idx + (int64_t)b * V;
  const uint64_t lt = (1ull << lane) - 1ull;
  const int sbits = S > 1 ? 32 - __builtin_clz((unsigned)(S - 1)) : 0;
  // SCATTER_AHEAD rounds of 64 entries at a time: their entries, then their indices
  // (one dependent round trip each, all rounds' loads in flight together).
  constexpr int SCATTER_AHEAD = 4;
  for (int i0 = 0; i0 < n; i0 += 64 * SCATTER_AHEAD) {
    int2 e[SCATTER_AHEAD];
    int s[SCATTER_AHEAD];
#pragma unroll
    for (int r = 0; r < SCATTER_AHEAD; ++r) e[r] = cb[min(i0 + r * 64 + lane, max(n - 1, 0))];
#pragma unroll
    for (int r = 0; r < SCATTER_AHEAD; ++r) s[r] = ib[e[r].x] - s0;  // entries lie in the window
#pragma unroll
    for (int r = 0; r < SCATTER_AHEAD; ++r) {
      const bool act = i0 + r * 64 + lane < n;
      uint64_t same = __ballot(act);
      if (same == 0) break;  // uniform: no entries left
      const int sr = act ? s[r] : 0;
      for (int k = 0; k < sbits; ++k) {
        const bool bit = ((sr >> k) & 1) != 0;
        const uint64_t ones = __ballot(bit);
        same &= bit ? ones : ~ones;
      }
      const int base = act ? cur[sr] : 0;
      if (act) lb[base + __popcll(same & lt)] = e[r];
      if (act && (same & lt) == 0) cur[sr] = base + __popcll(same);
    }
  }
}

// Store four fp32 values as O. The gradients are written once and read by nothing in the
// backward, so the stores are nontemporal: they stream to memory instead of evicting from
// L2 the W and H rows that the gathers re-read (cfg 4 backward 342 -> 320 us, cfg 5
// 535 -> 482 us).
__device__ __forceinline__ void store4(float* p, const f32x4& a) {
  __builtin_nontemporal_store(a, (f32x4*)p);
}
__device__ __forceinline__ void store4(bf16* p, const f32x4& a) {
  const bf16x4 v = bf16x4{(bf16)a[0], (bf16)a[1], (bf16)a[2], (bf16)a[3]};
  __builtin_nontemporal_store(__builtin_bit_cast(uint64_t, v), (uint64_t*)p);
}
__device__ __forceinline__ void store4(f16* p, const f32x4& a) {
  const f16x4 v = f16x4{(f16)a[0], (f16)a[1], (f16)a[2], (f16)a[3]};
  __builtin_nontemporal_store(__builtin_bit_cast(uint64_t, v), (uint64_t*)p);
}

// Four consecutive elements of a row, loaded raw (8 bytes for 16-bit types, 16 for
// fp32) so that a batch of loads is issued before any conversion.
template <typename T> struct Raw4;
template <> struct Raw4<float> {
  f32x4 v;
  __device__ __forceinline__ void load(const float* p) { v = *(const f32x4*)p; }
  __device__ __forceinline__ void zero() { v = f32x4{0.f, 0.f, 0.f, 0.f}; }
  __device__ __forceinline__ f32x4 f() const { return v; }
};
template <> struct Raw4<bf16> {
  bf16x4 v;
  __device__ __forceinline__ void load(const bf16* p) { v = *(const bf16x4*)p; }
  __device__ __forceinline__ void zero() { v = bf16x4{(bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f}; }
  __device__ __forceinline__ f32x4 f() const { return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]}; }
};
template <> struct Raw4<f16> {
  f16x4 v;
  __device__ __forceinline__ void load(const f16* p) { v = *(const f16x4*)p; }
  __device__ __forceinline__ void zero() { v = f16x4{(f16)0.f, (f16)0.f, (f16)0.f, (f16)0.f}; }
  __device__ __forceinline__ f32x4 f() const { return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]}; }
};

// The order every dH kernel (except the few-rows split kernel) sums a row in: the row's
// entries, in v order, are taken DH_BATCH at a time (the last batch may hold fewer); a
// batch's partial is P = fma(g_u, W[v_u], P) over its entries from P = 0, and the row is
// ((0 + P_0) + P_1) + ... So the fused path, whose waves share one workgroup's batches,
// and the five-kernel path agree bitwise.
constexpr int DH_BATCH = 4;

// P = fma(g, w, P) per element, written out so that every dH kernel rounds the same way.
__device__ __forceinline__ void fma4(f32x4& P, float g, const f32x4& w) {
  P[0] = __builtin_fmaf(g, w[0], P[0]);
  P[1] = __builtin_fmaf(g, w[1], P[1]);
  P[2] = __builtin_fmaf(g, w[2], P[2]);
  P[3] = __builtin_fmaf(g, w[3], P[3]);
}

// Rows gathered per batch: all their loads are in flight together (about 24 per lane).
template <int NP> struct Batch { static constexpr int U = NP <= 3 ? 8 : NP <= 6 ? 4 : NP <= 8 ? 3 : 2; };
// bwd_dh_kernel takes at most DH_MAX_NP register passes (wider rows loop over D) and
// whole DH_BATCH-entry batches per load group: U rows while at least U entries are left
// in the 64-entry chunk, US rows otherwise. Its gathers are chains of round trips, so
// for long rows more rows in flight beat occupancy; LONG is chosen for large vocabularies
// (V > FUSE_V_FAST), where rows hold many entries. Measured (dH alone incl. its bucketing):
// config 4 (V = 250002, 16-bit D = 768, ~49 entries per row) U = 8 vs 32: 279 vs 233 us
// with every row here; with rows past HOT_MIN entries in bwd_dh_hot_kernel, U = 8 / 16 /
// 32: 187 / 181 / 187 us. Config 5 (D = 4096, 8 passes) U = 4 vs 8: 233 vs 218 us; short
// rows (config 2 on this path) lose 3 us with U = 32 (fewer waves in flight).
constexpr int DH_MAX_NP = 8;
template <int NP> struct DhPasses { static constexpr int value = NP < DH_MAX_NP ? NP : DH_MAX_NP; };
template <typename T, int NP, bool LONG> struct DhBatch {
  static constexpr bool B16 = sizeof(T) == 2;
  static constexpr int U = NP <= 3 ? (LONG && B16 ? 16 : 8) : (LONG && B16 ? 8 : 4);
  static constexpr int US = NP <= 3 ? 8 : 4;
};
static_assert(DhBatch<bf16, 1, true>::US % DH_BATCH == 0 && DhBatch<float, DH_MAX_NP, false>::U % DH_BATCH == 0,
              "whole batches");

// One load group of bwd_dh_kernel: entries j .. j + U - 1 of the chunk held one per lane
// in ent (n of them valid), their W rows loaded together, then summed as DH_BATCH-entry
// partials, one pass at a time (so that only one pass of a partial is held in registers).
template <typename T, int NP, int U>
__device__ __forceinline__ void dh_group(const T* __restrict__ W, int2 ent, int j, int n, int d0,
                                         int D, int lane, f32x4* acc) {
  Raw4<T> w[U][NP];
  float g[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    // past the segment end: reload the last entry's row (a cache hit) with g' = 0,
    // which keeps the batch free of branches so all its loads issue together
    const int jj = min(j + u, n - 1);
    const int v = __builtin_amdgcn_readlane(ent.x, jj);
    g[u] = j + u < n ? __int_as_float(__builtin_amdgcn_readlane(ent.y, jj)) : 0.0f;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int d = d0 + p * 256 + lane * 4;
      if (d < D) w[u][p].load(W + (int64_t)v * D + d);
      else w[u][p].zero();
    }
  }
#pragma unroll
  for (int p = 0; p < NP; ++p) {
#pragma unroll
    for (int a = 0; a < U; a += DH_BATCH) {
      if (j + a < n) {  // uniform: the batch exists
        f32x4 P = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = a; u < a + DH_BATCH; ++u)
          if (j + u < n) fma4(P, g[u], w[u][p].f());
        acc[p] += P;
      }
    }
  }
}


// The staged dW kernel gathers the rows of IDC of a wave's ids together, U rows at a
// time. For 16-bit rows of up to 768 elements one id and 4 rows keep it within 64 VGPRs:
// two 16-wave workgroups per CU, so config 2's 477 workgroups run in one round instead
// of two (measured: 4 ids x 6 rows at 128 VGPRs, 55.0 us for the backward; 1 x 4, 49.8).
template <typename T, int NP> struct DwBatch {
  static constexpr int IDC = sizeof(T) == 2 ? 1 : NP > 3 ? 1 : 2;
  static constexpr int U = sizeof(T) == 2 && NP <= 3 ? 4 : IDC > 1 ? 6 : Batch<NP>::U;
};
// Register passes of the staged dW kernel: at most 8 (16-bit) or 4 (fp32), so that one
// id's accumulators and a batch of rows fit 128 VGPRs; longer rows loop over D.
template <typename T, int NP> struct DwPasses {
  static constexpr int CAP = sizeof(T) == 2 ? 8 : 4;
  static constexpr int value = NP < CAP ? NP : CAP;
};

// ---- 4. dH ---------------------------------------------------------------------
// One wave per (b,s) row; lane l owns elements d0 + p*256 + 4l .. +3 for p < NP. The
// segment's entries sit one per lane; they are taken U (or US) at a time (a uniform
// loop, so the summation order is the segment's v order), all loads of a group are
// issued, then its rows are accumulated.
template <typename T, typename O, int NP, bool LONG>
__device__ __forceinline__ void dh_rows_body(const T* __restrict__ W, const int2* __restrict__ list,
                                             const int* __restrict__ seg_start,
                                             const int* __restrict__ seg_cnt, O* __restrict__ dH,
                                             int B, int S, int D, int V, int S_row, int hot_min,
                                             int blk) {
  constexpr int U = DhBatch<T, NP, LONG>::U, US = DhBatch<T, NP, LONG>::US;
  static_assert(NP <= DH_MAX_NP, "register passes");
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blk * 4 + wave;
  if (row >= (int64_t)B * S) return;
  const int64_t b = row / S;
  const int start = __builtin_amdgcn_readfirstlane(seg_start[row]);
  const int cnt = __builtin_amdgcn_readfirstlane(seg_cnt[row]);
  if (cnt > hot_min) return;  // bwd_dh_hot_kernel writes this row
  const int2* seg = list + b * V + start;
  for (int d0 = 0; d0 < D; d0 += NP * 256) {
    f32x4 acc[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) acc[p] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int e0 = 0; e0 < cnt; e0 += 64) {
      const int2 ent = e0 + lane < cnt ? seg[e0 + lane] : make_int2(0, 0);
      const int n = min(64, cnt - e0);
      // j stays a multiple of DH_BATCH (chunks of 64 too): whole batches per group.
      int j = 0;
      if constexpr (U > US) {
        for (; j + U <= n; j += U) dh_group<T, NP, U>(W, ent, j, n, d0, D, lane, acc);
      }
      for (; j < n; j += US) dh_group<T, NP, US>(W, ent, j, n, d0, D, lane, acc);
    }
    O* out = dH + (b * S_row + (row - b * S)) * D;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int d = d0 + p * 256 + lane * 4;
      if (d < D) store4(out + d, acc[p]);
    }
  }
}
template <typename T, typename O, int NP, bool LONG>
__global__ __launch_bounds__(256) void bwd_dh_kernel(
    const T* __restrict__ W, const int2* __restrict__ list, const int* __restrict__ seg_start,
    const int* __restrict__ seg_cnt, O* __restrict__ dH, int B, int S, int D, int V, int S_row,
    int hot_min) {
  dh_rows_body<T, O, NP, LONG>(W, list, seg_start, seg_cnt, dH, B, S, D, V, S_row, hot_min,
                               (int)blockIdx.x);
}

// Hot rows (more than hot_min entries, e.g. a position that wins most vocab ids; at
// config 4, V = 250002, rows hold ~49 entries and up to 776): one wave per row would
// gather them alone. Measured at config 4, backward with HOT_MIN = 64 / 128 / 256 / 512 /
// off: 341 / 342 / 369 / 398 / 390 us; configs 1, 2, 3 (five-kernel) and 5 unchanged. Here a workgroup of HOT_WAVES waves takes one
// (hot row, 256-column slice) at a time from the list the scan built (a grid of fixed
// size walks the list). Each step its waves compute HOT_PER_WAVE consecutive batch
// partials each (the DH_BATCH-entry partials of bwd_dh_kernel, over the slice) into LDS,
// and wave 0 adds them in batch order: the same sums as bwd_dh_kernel, bitwise.
constexpr int HOT_MIN = 128;
constexpr int HOT_WAVES = 16;
constexpr int HOT_PER_WAVE = 2;
constexpr int HOT_STEP = HOT_WAVES * HOT_PER_WAVE;  // batches per step
constexpr int HOT_GRID = 512;
template <typename T, typename O>
__global__ __launch_bounds__(64 * HOT_WAVES) void bwd_dh_hot_kernel(
    const T* __restrict__ W, const int2* __restrict__ list, const int* __restrict__ seg_start,
    const int* __restrict__ seg_cnt, const int* __restrict__ hot, O* __restrict__ dH, int S,
    int D, int V, int S_row, int ns) {
  __shared__ f32x4 part[HOT_STEP][64];
  constexpr int U = HOT_PER_WAVE * DH_BATCH;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n_items = __builtin_amdgcn_readfirstlane(hot[0]) * ns;
  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int64_t row = __builtin_amdgcn_readfirstlane(hot[1 + item / ns]);
    const int d = (item % ns) * 256 + lane * 4;
    const int64_t b = row / S;
    const int start = __builtin_amdgcn_readfirstlane(seg_start[row]);
    const int cnt = __builtin_amdgcn_readfirstlane(seg_cnt[row]);
    const int2* seg = list + b * V + start;
    const int nbat = (cnt + DH_BATCH - 1) / DH_BATCH;
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int t0 = 0; t0 < nbat; t0 += HOT_STEP) {
      const int e0 = (t0 + wave * HOT_PER_WAVE) * DH_BATCH;  // this wave's first entry
      if (e0 < cnt) {  // uniform
        const int2 ent = lane < U ? seg[min(e0 + lane, cnt - 1)] : make_int2(0, 0);
        Raw4<T> w[U];
        float g[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          // past the row's last entry: reload that entry's row (a cache hit), unused
          const int v = __builtin_amdgcn_readlane(ent.x, u);
          g[u] = __int_as_float(__builtin_amdgcn_readlane(ent.y, u));
          if (d < D) w[u].load(W + (int64_t)v * D + d);
          else w[u].zero();
        }
#pragma unroll
        for (int h = 0; h < HOT_PER_WAVE; ++h) {
          f32x4 P = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int u = h * DH_BATCH; u < (h + 1) * DH_BATCH; ++u)
            if (e0 + u < cnt) fma4(P, g[u], w[u].f());  // uniform condition
          part[wave * HOT_PER_WAVE + h][lane] = P;
        }
      }
      __syncthreads();
      if (wave == 0) {
        const int m = min(HOT_STEP, nbat - t0);
        for (int j = 0; j < m; ++j) acc += part[j][lane];
      }
      __syncthreads();  // the partials are rewritten next step
    }
    if (wave == 0 && d < D) store4(dH + (b * S_row + (row - b * S)) * D + d, acc);
  }
}

// Few rows (B*S < SPLIT_ROWS, e.g. 2 x 32 with every v active): one workgroup of
// SPLIT_WAVES waves per (row, 256-column slice of D) instead of one wave per row, so that
// even a handful of rows keeps thousands of waves gathering. Wave w sums entries
// [w c, (w + 1) c) of the row's segment (c = ceil(cnt / SPLIT_WAVES)) in v order over its
// slice, and wave 0 adds the partial slices in wave order through LDS: deterministic
// (each element's sum does not depend on the slicing).
constexpr int SPLIT_WAVES = 8;
constexpr int SPLIT_ROWS = 1024;
constexpr int SPLIT_U = 16;  // rows gathered per batch (one 256-column slice each)
template <typename T, typename O>
__device__ __forceinline__ void dh_split_body(float (*red)[256], const T* __restrict__ W,
                                              const int2* __restrict__ list,
                                              const int* __restrict__ seg_start,
                                              const int* __restrict__ seg_cnt, O* __restrict__ dH,
                                              int S, int D, int V, int S_row, int ns, int blk) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = blk / ns;  // workgroups = B * S * ns exactly
  const int d = (int)(blk % ns) * 256 + lane * 4;
  const int64_t b = row / S;
  const int start = __builtin_amdgcn_readfirstlane(seg_start[row]);
  const int cnt = __builtin_amdgcn_readfirstlane(seg_cnt[row]);
  const int per = (cnt + SPLIT_WAVES - 1) / SPLIT_WAVES;
  const int e_beg = min(cnt, wave * per), e_end = min(cnt, e_beg + per);
  const int2* seg = list + b * V + start;
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int e0 = e_beg; e0 < e_end; e0 += 64) {
    const int2 ent = e0 + lane < e_end ? seg[e0 + lane] : make_int2(0, 0);
    const int n = min(64, e_end - e0);
    for (int j = 0; j < n; j += SPLIT_U) {
      Raw4<T> w[SPLIT_U];
      float g[SPLIT_U];
#pragma unroll
      for (int u = 0; u < SPLIT_U; ++u) {
        const int jj = min(j + u, n - 1);
        const int v = __builtin_amdgcn_readlane(ent.x, jj);
        g[u] = j + u < n ? __int_as_float(__builtin_amdgcn_readlane(ent.y, jj)) : 0.0f;
        if (d < D) w[u].load(W + (int64_t)v * D + d);
        else w[u].zero();
      }
#pragma unroll
      for (int u = 0; u < SPLIT_U; ++u) acc += g[u] * w[u].f();
    }
  }
  *(f32x4*)&red[wave][lane * 4] = acc;
  __syncthreads();
  if (wave == 0) {
    f32x4 t = *(const f32x4*)&red[0][lane * 4];
#pragma unroll
    for (int w = 1; w < SPLIT_WAVES; ++w) t += *(const f32x4*)&red[w][lane * 4];
    if (d < D) store4(dH + (b * S_row + (row - b * S)) * D + d, t);
  }
}
template <typename T, typename O>
__global__ __launch_bounds__(64 * SPLIT_WAVES) void bwd_dh_split_kernel(
    const T* __restrict__ W, const int2* __restrict__ list, const int* __restrict__ seg_start,
    const int* __restrict__ seg_cnt, O* __restrict__ dH, int B, int S, int D, int V, int S_row,
    int ns) {
  __shared__ __attribute__((aligned(16))) float red[SPLIT_WAVES][256];
  dh_split_body<T, O>(red, W, list, seg_start, seg_cnt, dH, S, D, V, S_row, ns, (int)blockIdx.x);
}

// Entries (b_i, v) for N batch rows (b_i >= B or v >= V: inactive): g' (0 if inactive) and
// s. Three raw loads per row, issued together; then the mask of the candidates, issued
// together; then the coefficients. Inactive entries get s = 0.
template <typename T, typename RT, int N>
__device__ __forceinline__ void entries_n(const T* grad, const RT* reps, const int32_t* idx,
                                          const void* mask, int mdt, const int* bs, int v, int B,
                                          int S, int V, float* g, int* s) {
  T gr[N];
  RT rr[N];
  int ss[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int64_t o = (int64_t)min(bs[i], B - 1) * V + min(v, V - 1);
    gr[i] = grad[o];
    rr[i] = reps[o];
    ss[i] = idx[o];
  }
  bool cand[N];
  int64_t moff[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    cand[i] = bs[i] < B && v < V && to_f32(rr[i]) > 0.0f && ss[i] >= 0 && ss[i] < S &&
              to_f32(gr[i]) != 0.0f;
    moff[i] = cand[i] ? (int64_t)bs[i] * S + ss[i] : 0;
  }
  float mv[N];
  load_mask_n<N>(mask, mdt, moff, mv);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const bool act = cand[i] && mv[i] != 0.0f;
    g[i] = act ? to_f32(gr[i]) * expf(-to_f32(rr[i])) * mv[i] : 0.0f;
    s[i] = act ? ss[i] : 0;
  }
}

// ---- 5. dW and dbias -------------------------------------------------------------
// One wave per vocab row v: lanes hold batch rows b (64 per pass), a ballot lists the
// active ones, and their H rows are gathered in ascending b, two at a time. Lanes past the
// row end load the row's last group (D >= 4 whenever D > 0), so the loads carry no per-lane
// condition and are in flight together; those lanes' sums are never stored.
template <typename T, typename O, int NP, typename RT>
__global__ __launch_bounds__(256) void bwd_dw_kernel(
    const T* __restrict__ grad, const RT* __restrict__ reps,
    const int32_t* __restrict__ idx, const void* __restrict__ mask, int mdt,
    const T* __restrict__ H, O* __restrict__ dW, O* __restrict__ dbias, int B, int S, int D,
    int V) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int v = blockIdx.x * 4 + wave;
  if (v >= V) return;
  const int dend = max(D, 1);  // one pass even when D == 0, for dbias
  for (int d0 = 0; d0 < dend; d0 += NP * 256) {
    f32x4 acc[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) acc[p] = f32x4{0.f, 0.f, 0.f, 0.f};
    float bsum = 0.0f;
    for (int b0 = 0; b0 < B; b0 += 64) {
      const int bb = b0 + lane;
      float g;
      int s;
      entries_n<T, RT, 1>(grad, reps, idx, mask, mdt, &bb, v, B, S, V, &g, &s);
      uint64_t pending = __ballot(g != 0.0f);
      while (pending) {
        const int l0 = __ffsll((unsigned long long)pending) - 1;
        pending &= pending - 1;
        const int s0 = __builtin_amdgcn_readlane(s, l0);
        const float g0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(g), l0));
        const T* h0 = H + ((int64_t)(b0 + l0) * S + s0) * D;
        bsum += g0;
        if (pending) {
          const int l1 = __ffsll((unsigned long long)pending) - 1;
          pending &= pending - 1;
          const int s1 = __builtin_amdgcn_readlane(s, l1);
          const float g1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(g), l1));
          const T* h1 = H + ((int64_t)(b0 + l1) * S + s1) * D;
          bsum += g1;
          if (D > 0) {  // (H may be null without columns)
            f32x4 x0[NP], x1[NP];
#pragma unroll
            for (int p = 0; p < NP; ++p) {
              const int d = min(d0 + p * 256 + lane * 4, D - 4);
              x0[p] = load4(h0 + d);
              x1[p] = load4(h1 + d);
            }
#pragma unroll
            for (int p = 0; p < NP; ++p) acc[p] += g0 * x0[p] + g1 * x1[p];
          }
        } else if (D > 0) {
          f32x4 x0[NP];
#pragma unroll
          for (int p = 0; p < NP; ++p) x0[p] = load4(h0 + min(d0 + p * 256 + lane * 4, D - 4));
#pragma unroll
          for (int p = 0; p < NP; ++p) acc[p] += g0 * x0[p];
        }
      }
    }
    if (d0 == 0 && dbias != nullptr && lane == 0) dbias[v] = from_f32<O>(bsum);
    if (dW != nullptr) {
      O* out = dW + (int64_t)v * D;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const int d = d0 + p * 256 + lane * 4;
        if (d < D) store4(out + d, acc[p]);
      }
    }
  }
}

// ---- 5b. dW and dbias, staged (B <= DW_STAGE_B) ---------------------------------
constexpr int DW_STAGE_B = 128;
// The fused dH path (B <= DW_STAGE_B, S <= FUSE_MAX_S, V <= 2^FUSE_V_BITS, D in one
// register pass): an entry packs v and s into one int.
constexpr int FUSE_V_BITS = 18;
constexpr int FUSE_MAX_S = 1024;
constexpr int FUSE_ROWS = 16;                          // rows per range (one workgroup)
constexpr int FUSE_V_FAST = 1 << 16;    // above this the five-kernel path is faster
constexpr int FUSE_MAX_NVB = FUSE_V_FAST / 64;         // 64-id blocks the fused path takes
constexpr int FUSE_MIN_RANGES = 64;     // below this too (too few workgroups)
constexpr int FUSE_MAX_NR = FUSE_MAX_S / FUSE_ROWS;    // ranges (<= 64: one lane each)

// The staged dW: a workgroup of NW waves owns NIDS consecutive vocab ids (NIDS / NW per
// wave). It loads G, reps and I of all batch rows for them (each load instruction reads
// NIDS consecutive elements of 64 / NIDS rows) and keeps g' (0 = inactive) and I in LDS;
// then each wave handles its ids: lanes scan the batch rows, ballots list the active
// ones, and their H rows are gathered up to U at a time and accumulated, each id in
// ascending b. I is kept as 16 bits: the staged kernels take S <= DW_STAGE_S.
constexpr int DW_WAVES = 16;
constexpr int DW_LD = DW_STAGE_B + 1;  // odd row stride: conflict-free column and row access
constexpr int DW_STAGE_S = 1 << 16;

template <typename T, typename RT, int NIDS, int NW, int LD = DW_LD>
__device__ __forceinline__ void dw_stage(float* gl, uint16_t* sl, const T* __restrict__ grad,
                                         const RT* __restrict__ reps,
                                         const int32_t* __restrict__ idx,
                                         const void* __restrict__ mask, int mdt, int B, int S,
                                         int V, int v0, int wave, int lane) {
  constexpr int RPL = 64 / NIDS;  // batch rows per load instruction
  const int idl = lane % NIDS, rsub = lane / NIDS;
  // Each wave takes 2 * RPL batch rows at a time, their loads in flight together.
  for (int b0 = wave * 2 * RPL; b0 < B; b0 += NW * 2 * RPL) {
    const int bs[2] = {b0 + rsub, b0 + RPL + rsub};
    float g[2];
    int s[2];
    entries_n<T, RT, 2>(grad, reps, idx, mask, mdt, bs, v0 + idl, B, S, V, g, s);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (bs[i] < B) {
        gl[idl * LD + bs[i]] = g[i];
        sl[idl * LD + bs[i]] = (uint16_t)s[i];
      }
    }
  }
}

template <typename T, typename O, int NP, typename RT, int NIDS, int NW, int LD = DW_LD>
__device__ __forceinline__ void dw_gather(const float* gl, const uint16_t* sl,
                                          const T* __restrict__ H, O* __restrict__ dW,
                                          O* __restrict__ dbias, int B, int S, int D, int V,
                                          int v0, int wave, int lane) {
  // IDC of the wave's ids at a time are gathered together: batches of U rows are taken
  // from their active (id, b) pairs in (id, b) order, so each id still sums its rows in
  // ascending b.
  constexpr int IDS = NIDS / NW;  // ids per wave
  constexpr int IDC = DwBatch<T, NP>::IDC;
  constexpr int U = DwBatch<T, NP>::U;
  static_assert(IDS % IDC == 0, "ids per wave");
  const int dend = max(D, 1);  // one pass even when D == 0, for dbias
  for (int i0 = 0; i0 < IDS; i0 += IDC) {
    if (v0 + wave * IDS + i0 >= V) break;
    for (int d0 = 0; d0 < dend; d0 += NP * 256) {
      f32x4 acc[IDC][NP];
      float bsum[IDC];
#pragma unroll
      for (int i = 0; i < IDC; ++i) {
        bsum[i] = 0.0f;
#pragma unroll
        for (int p = 0; p < NP; ++p) acc[i][p] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      for (int b0 = 0; b0 < B; b0 += 64) {
        const int bb = b0 + lane;
        float g[IDC];
        int s[IDC];
        uint64_t pend[IDC];
        int left = 0;
#pragma unroll
        for (int i = 0; i < IDC; ++i) {
          const int vl = wave * IDS + i0 + i;
          const bool in = bb < B && v0 + vl < V;
          g[i] = in ? gl[vl * LD + bb] : 0.0f;
          s[i] = in ? (int)sl[vl * LD + bb] : 0;
          pend[i] = __ballot(g[i] != 0.0f);
          left += __popcll(pend[i]);
        }
        while (left > 0) {
          const int nb = min(U, left);  // rows in this batch (uniform)
          left -= nb;
          Raw4<T> x[U][NP];
          float gu[U];
          int iu[U];
#pragma unroll
          for (int u = 0; u < U; ++u) {
            gu[u] = 0.0f;
            iu[u] = -1;
            if (u < nb) {
              int l = 0, su = 0;
              float gg = 0.0f;
              bool taken = false;
#pragma unroll
              for (int i = 0; i < IDC; ++i) {  // the first id with rows left (uniform)
                if (!taken && pend[i] != 0) {
                  taken = true;
                  iu[u] = i;
                  l = __ffsll((unsigned long long)pend[i]) - 1;
                  pend[i] &= pend[i] - 1;
                  gg = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(g[i]), l));
                  su = __builtin_amdgcn_readlane(s[i], l);
                }
              }
              gu[u] = gg;
              const T* hr = H + ((int64_t)(b0 + l) * S + su) * D;
#pragma unroll
              for (int p = 0; p < NP; ++p) {
                const int d = d0 + p * 256 + lane * 4;
                if (d < D) x[u][p].load(hr + d);
                else x[u][p].zero();
              }
            }
          }
#pragma unroll
          for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int i = 0; i < IDC; ++i) {
              if (iu[u] == i) {
                bsum[i] += gu[u];
#pragma unroll
                for (int p = 0; p < NP; ++p) acc[i][p] += gu[u] * x[u][p].f();
              }
            }
          }
        }
      }
#pragma unroll
      for (int i = 0; i < IDC; ++i) {
        const int v = v0 + wave * IDS + i0 + i;
        if (v >= V) break;
        if (d0 == 0 && dbias != nullptr && lane == 0) dbias[v] = from_f32<O>(bsum[i]);
        if (dW != nullptr) {
          O* out = dW + (int64_t)v * D;
#pragma unroll
          for (int p = 0; p < NP; ++p) {
            const int d = d0 + p * 256 + lane * 4;
            if (d < D) store4(out + d, acc[i][p]);
          }
        }
      }
    }
  }
}

// dW / dbias for B <= DW_STAGE_B and S <= DW_STAGE_S (the five-kernel path's).
template <typename T, typename O, int NP, typename RT>
__global__ __launch_bounds__(64 * DW_WAVES) void bwd_dw_staged_kernel(
    const T* __restrict__ grad, const RT* __restrict__ reps,
    const int32_t* __restrict__ idx, const void* __restrict__ mask, int mdt,
    const T* __restrict__ H, O* __restrict__ dW, O* __restrict__ dbias, int B, int S, int D,
    int V) {
  __shared__ float gl[64 * DW_LD];
  __shared__ uint16_t sl[64 * DW_LD];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int v0 = blockIdx.x * 64;
  dw_stage<T, RT, 64, DW_WAVES>(gl, sl, grad, reps, idx, mask, mdt, B, S, V, v0, wave, lane);
  __syncthreads();
  dw_gather<T, O, NP, RT, 64, DW_WAVES>(gl, sl, H, dW, dbias, B, S, D, V, v0, wave, lane);
}

// dW / dbias for DW_STAGE_B < B <= DW_WIDE_B and S <= DW_STAGE_S: the staged kernel with
// fewer ids per workgroup, so that every batch row of them fits LDS (NIDS ids x (ROWS + 1)
// x 6 bytes, ~99 KB: 64 ids up to 256 rows, 32 up to 512, 16 up to 1024). The rows are
// staged once and each id sums its rows in ascending b, as above.
constexpr int DW_WIDE_IDS_ROWS = 16384;  // NIDS x ROWS
constexpr int DW_WIDE_B = 1024;
template <typename T, typename O, int NP, typename RT, int NIDS>
__global__ __launch_bounds__(64 * DW_WAVES) void bwd_dw_wide_kernel(
    const T* __restrict__ grad, const RT* __restrict__ reps,
    const int32_t* __restrict__ idx, const void* __restrict__ mask, int mdt,
    const T* __restrict__ H, O* __restrict__ dW, O* __restrict__ dbias, int B, int S, int D,
    int V) {
  constexpr int LD = DW_WIDE_IDS_ROWS / NIDS + 1;  // odd: conflict-free
  __shared__ float gl[NIDS * LD];
  __shared__ uint16_t sl[NIDS * LD];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int v0 = blockIdx.x * NIDS;
  dw_stage<T, RT, NIDS, DW_WAVES, LD>(gl, sl, grad, reps, idx, mask, mdt, B, S, V, v0, wave, lane);
  __syncthreads();
  dw_gather<T, O, NP, RT, NIDS, DW_WAVES, LD>(gl, sl, H, dW, dbias, B, S, D, V, v0, wave, lane);
}

// dH and the staged dW in one launch, for the five-kernel path when it makes one pass
// (B <= MAX_B, S <= MAX_S), dW is staged (B <= DW_STAGE_B, S <= DW_STAGE_S) and the rows
// are wide (the launch rule is at the host dispatch): the dH workgroups first, then dW
// workgroups of 4 ids per wave. dW reads only the inputs, so its workgroups fill the CUs
// that the dH rows leave idle, and its own launch (about 4.5 us of dispatch and cache
// work at each kernel boundary) is saved. The sums are those of the separate kernels.
template <typename T, typename O, int NP, bool LONG, int DNP, typename RT>
__global__ __launch_bounds__(256) void bwd_dh_dw_kernel(
    const T* __restrict__ W, const int2* __restrict__ list, const int* __restrict__ seg_start,
    const int* __restrict__ seg_cnt, O* __restrict__ dH, int B, int S, int D, int V,
    int hot_min, int n_dh, const T* __restrict__ grad, const RT* __restrict__ reps,
    const int32_t* __restrict__ idx, const void* __restrict__ mask, int mdt,
    const T* __restrict__ H, O* __restrict__ dW, O* __restrict__ dbias) {
  constexpr int NW = 4, NIDS = 4 * NW;
  __shared__ float gl[NIDS * DW_LD];
  __shared__ uint16_t sl[NIDS * DW_LD];
  if ((int)blockIdx.x < n_dh) {  // workgroup-uniform
    dh_rows_body<T, O, NP, LONG>(W, list, seg_start, seg_cnt, dH, B, S, D, V, S, hot_min,
                                 (int)blockIdx.x);
    return;
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int v0 = ((int)blockIdx.x - n_dh) * NIDS;
  dw_stage<T, RT, NIDS, NW>(gl, sl, grad, reps, idx, mask, mdt, B, S, V, v0, wave, lane);
  __syncthreads();
  dw_gather<T, O, DNP, RT, NIDS, NW>(gl, sl, H, dW, dbias, B, S, D, V, v0, wave, lane);
}

// The same for few rows: the split dH workgroups, then dW workgroups of 4 ids per wave.
template <typename T, typename O, int DNP, typename RT>
__global__ __launch_bounds__(64 * SPLIT_WAVES) void bwd_dh_split_dw_kernel(
    const T* __restrict__ W, const int2* __restrict__ list, const int* __restrict__ seg_start,
    const int* __restrict__ seg_cnt, O* __restrict__ dH, int B, int S, int D, int V, int ns,
    int n_dh, const T* __restrict__ grad, const RT* __restrict__ reps,
    const int32_t* __restrict__ idx, const void* __restrict__ mask, int mdt,
    const T* __restrict__ H, O* __restrict__ dW, O* __restrict__ dbias) {
  constexpr int NW = SPLIT_WAVES, NIDS = 4 * NW;
  struct DwSmem {
    float gl[NIDS * DW_LD];
    uint16_t sl[NIDS * DW_LD];
  };
  union Smem {
    float red[SPLIT_WAVES][256];
    DwSmem w;
  };
  __shared__ __attribute__((aligned(16))) Smem sm;
  if ((int)blockIdx.x < n_dh) {  // workgroup-uniform
    dh_split_body<T, O>(sm.red, W, list, seg_start, seg_cnt, dH, S, D, V, S, ns, (int)blockIdx.x);
    return;
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int v0 = ((int)blockIdx.x - n_dh) * NIDS;
  dw_stage<T, RT, NIDS, NW>(sm.w.gl, sm.w.sl, grad, reps, idx, mask, mdt, B, S, V, v0, wave, lane);
  __syncthreads();
  dw_gather<T, O, DNP, RT, NIDS, NW>(sm.w.gl, sm.w.sl, H, dW, dbias, B, S, D, V, v0, wave, lane);
}

// The fused path's compaction, for the dH workgroups: for batch row b and 64-id block
// blk, the active entries sorted by row range k = s / FUSE_ROWS and then by v, as
// (v | s << FUSE_V_BITS, g') at comp[(b * nvb + blk) * 64 + rank]; their number
// cnt[b * nvb + blk], and the first rank of each range (offs[(b * nvb + blk) * nr + k],
// lane k). Ranks come from one pass over the active lanes (a handful per block). One
// wave per (block, two batch rows b, b + 4).
template <typename T, typename RT>
__global__ __launch_bounds__(256) void bwd_compact_kernel(
    const T* __restrict__ grad, const RT* __restrict__ reps, const int32_t* __restrict__ idx,
    const void* __restrict__ mask, int mdt, int B, int S, int V, int2* __restrict__ comp,
    int* __restrict__ cnt, int* __restrict__ offs) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nvb = gridDim.x, blk = blockIdx.x, v0 = blk * 64;
  const int nr = (S + FUSE_ROWS - 1) / FUSE_ROWS;
  const int bs[2] = {(int)blockIdx.y * 8 + wave, (int)blockIdx.y * 8 + 4 + wave};
  float g[2];
  int sv[2];
  entries_n<T, RT, 2>(grad, reps, idx, mask, mdt, bs, v0 + lane, B, S, V, g, sv);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (bs[i] >= B) break;  // wave-uniform
    const bool on = g[i] != 0.0f;
    const int k = sv[i] / FUSE_ROWS;
    const uint64_t bal = __ballot(on);
    uint64_t act = bal;
    const int64_t base = (int64_t)bs[i] * nvb + blk;
    int rank = 0, first = 0;  // this entry's rank; the first rank of range `lane`
    while (act) {
      const int j = __ffsll((unsigned long long)act) - 1;
      act &= act - 1;
      const int kj = __builtin_amdgcn_readlane(k, j);
      rank += (kj < k || (kj == k && j < lane)) ? 1 : 0;
      first += kj < lane ? 1 : 0;
    }
    if (on) comp[base * 64 + rank] = make_int2((v0 + lane) | (sv[i] << FUSE_V_BITS), __float_as_int(g[i]));
    if (lane < nr) offs[base * nr + lane] = first;
    if (lane == 0) cnt[base] = __popcll(bal);
  }
}

// ---- 4b. dH from the staged dW kernel's compacted entries (the fused path) -------------
// FUSE_HALVES workgroups per (b, range of FUSE_ROWS consecutive rows); wave w of
// workgroup h owns row s = FUSE_ROWS * range + FUSE_WAVES * h + w. Each 64-id block of row b lists its active
// entries sorted by row range, then v, so a range's entries are one contiguous run per
// block: thread t copies the t-th of them into LDS (its block found by binary search over
// the runs' prefix sums), 64 * FUSE_WAVES per round, in block (= v) order. Each wave
// appends the entries of its row to its own list, keeping v order.
// The workgroup's waves then share the gathering: the rows' DH_BATCH-entry batches, in
// (row, batch) order, are taken FUSE_SLOTS at a time, one per wave; each wave gathers its
// batch's W rows and writes the batch partial to LDS, and each row's own wave adds its
// rows' partials in batch order. A row with many entries is gathered by all the waves of
// its workgroup, and the sums are exactly those of bwd_dh_kernel.
// With the compaction in the dW kernel this replaces the count, scan and scatter passes.
constexpr int FUSE_CAP = 120;  // a wave's list; the lists are gathered before one could overflow
constexpr int FUSE_WAVES = 8;  // rows per workgroup (one 16-wave workgroup per range measured
                               // slower: 56.5 vs 49.4 us at config 2)
constexpr int FUSE_HALVES = FUSE_ROWS / FUSE_WAVES;  // workgroups per row range
static_assert(FUSE_ROWS % FUSE_WAVES == 0, "whole workgroups per row range");
// Register passes the fused path takes (a batch of rows and the accumulators in ~64 VGPRs).
template <typename T> struct FuseMaxNp { static constexpr int value = sizeof(T) == 2 ? 6 : 3; };
// W rows loaded at a time by the fused dH gather (a divisor of DH_BATCH): fewer for wide
// rows, so that the kernel stays near 64 VGPRs (8 waves per SIMD: four workgroups per CU).
template <int NP> struct FuseBatch { static constexpr int U = NP <= 3 ? 4 : 2; };
// Batches gathered per step (one per wave; half the waves for wide rows, whose partials
// take twice the LDS).
template <int NP> struct FuseSlots { static constexpr int value = NP <= 3 ? FUSE_WAVES : FUSE_WAVES / 2; };
static_assert(DH_BATCH % FuseBatch<1>::U == 0 && DH_BATCH % FuseBatch<6>::U == 0, "whole batches");

// PER: 64-id blocks per thread in the prefix (nvb <= PER * 64 * FUSE_WAVES).
template <int PER, int NP>
struct DhSmem {
  static constexpr int NT = 64 * FUSE_WAVES;
  static constexpr int SLOTS = FuseSlots<NP>::value;
  static_assert(PER * NT <= FUSE_MAX_NVB, "prefix arrays");
  int pre[PER * NT];    // prefix of the runs' lengths
  int lo_of[PER * NT];  // each run's first rank in its block
  int2 stage[NT];
  int2 lst[FUSE_WAVES][FUSE_CAP];
  f32x4 part[SLOTS][NP * 64];  // one step's batch partials, [slot][p * 64 + lane]
  int wsum[FUSE_WAVES];
  int nlist[FUSE_WAVES];       // entries in each row's list
  int nbat[FUSE_WAVES];        // batches of each row to gather now
  int full[2][FUSE_WAVES];     // a row's list could overflow (two buffers: no WAR barrier)
};
static_assert(sizeof(DhSmem<1, 3>) <= 40 * 1024, "four dH workgroups per CU at config 2's widths");

// One batch's partial (entries e0 .. e0 + m - 1 of `list`), pass by pass: pass p goes to
// dst[p * 64 + lane] (ADD = false) or is added to acc[p] (ADD = true).
template <typename T, int NP, bool ADD>
__device__ __forceinline__ void dh_batch(const T* __restrict__ W, const int2* list, int e0, int m,
                                         int D, int lane, f32x4* dst, f32x4* acc) {
  constexpr int U = FuseBatch<NP>::U;
  constexpr int VMASK = (1 << FUSE_V_BITS) - 1;
  f32x4 Pr[NP];  // ADD with two load groups: the partial between them
#pragma unroll
  for (int u0 = 0; u0 < DH_BATCH; u0 += U) {
    Raw4<T> w[U][NP];
    float g[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      // past the batch's last entry: reload that entry's row (a cache hit), unused
      const int2 ent = list[e0 + min(u0 + u, m - 1)];
      const int v = __builtin_amdgcn_readfirstlane(ent.x) & VMASK;  // uniform
      g[u] = __int_as_float(__builtin_amdgcn_readfirstlane(ent.y));
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const int d = p * 256 + lane * 4;
        if (d < D) w[u][p].load(W + (int64_t)v * D + d);
        else w[u][p].zero();
      }
    }
    // One pass at a time, so that only one pass of the partial is held in registers when
    // the batch is one load group.
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      f32x4 P = u0 == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : (ADD ? Pr[p] : dst[p * 64 + lane]);
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (u0 + u < m) fma4(P, g[u], w[u][p].f());  // uniform condition
      if (!ADD) dst[p * 64 + lane] = P;
      else if (u0 + U >= DH_BATCH) acc[p] += P;
      else Pr[p] = P;
    }
  }
}

// The workgroup's gather of every listed batch of its rows (only the complete ones unless
// `last`); row `wave`'s partials are added to acc in batch order, and the gathered entries
// leave the lists (a row keeps its incomplete last batch). When one row holds more than
// `share` times the batches per wave, the waves share them: SLOTS per step, each wave's
// partial through LDS to the row's wave. Otherwise each wave gathers its own row.
template <typename T, int NP, int PER>
__device__ __forceinline__ void dh_gather(DhSmem<PER, NP>& sm, const T* __restrict__ W, int D,
                                          int wave, int lane, int& n, bool last, int share,
                                          f32x4* acc) {
  constexpr int SLOTS = DhSmem<PER, NP>::SLOTS;
  const int mine = last ? (n + DH_BATCH - 1) / DH_BATCH : n / DH_BATCH;
  if (lane == 0) {
    sm.nlist[wave] = n;
    sm.nbat[wave] = mine;
  }
  __syncthreads();
  int st[FUSE_WAVES + 1];  // first batch of each row in the workgroup's order (uniform)
  st[0] = 0;
  int most = 0;
#pragma unroll
  for (int w = 0; w < FUSE_WAVES; ++w) {
    const int c = __builtin_amdgcn_readfirstlane(sm.nbat[w]);
    st[w + 1] = st[w] + c;
    most = max(most, c);
  }
  const int nb = st[FUSE_WAVES];
  if (most > share * ((nb + SLOTS - 1) / SLOTS)) {
    for (int t0 = 0; t0 < nb; t0 += SLOTS) {
      const int q = t0 + wave;  // this wave's batch
      if (wave < SLOTS && q < nb) {
        int r = 0;
#pragma unroll
        for (int w = 1; w < FUSE_WAVES; ++w) r += q >= st[w] ? 1 : 0;
        const int e0 = (q - st[r]) * DH_BATCH;
        const int m = min(DH_BATCH, __builtin_amdgcn_readfirstlane(sm.nlist[r]) - e0);
        dh_batch<T, NP, false>(W, sm.lst[r], e0, m, D, lane, sm.part[wave], acc);
      }
      __syncthreads();
      // This wave's row: its batches among this step's, in order.
      const int b0 = max(st[wave], t0), b1 = min(st[wave + 1], t0 + SLOTS);
      for (int q2 = b0; q2 < b1; ++q2)
#pragma unroll
        for (int p = 0; p < NP; ++p) acc[p] += sm.part[q2 - t0][p * 64 + lane];
      __syncthreads();  // the partials are rewritten next step
    }
  } else {
    for (int k = 0; k < mine; ++k)
      dh_batch<T, NP, true>(W, sm.lst[wave], k * DH_BATCH, min(DH_BATCH, n - k * DH_BATCH), D,
                            lane, nullptr, acc);
  }
  // The row keeps only its incomplete batch (at most DH_BATCH - 1 entries).
  const int taken = mine * DH_BATCH;
  const int keep = max(0, n - taken);
  int2 e = make_int2(0, 0);
  if (lane < keep) e = sm.lst[wave][taken + lane];
  if (lane < keep) sm.lst[wave][lane] = e;
  n = keep;
}

// The workgroup for batch row b and xb = FUSE_HALVES * range + half.
template <typename T, typename O, int NP, int PER>
__device__ __forceinline__ void dh_fused_body(DhSmem<PER, NP>& sm, const T* __restrict__ W,
                                              const int2* __restrict__ comp,
                                              const int* __restrict__ cnt,
                                              const int* __restrict__ offs, O* __restrict__ dH,
                                              int S, int D, int nvb, int64_t b, int xb,
                                              int share) {
  constexpr int NT = DhSmem<PER, NP>::NT;
  int* pre = sm.pre;
  int* lo_of = sm.lo_of;
  int2* stage = sm.stage;
  int* wsum = sm.wsum;
  auto& lst = sm.lst;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int k = xb / FUSE_HALVES, nr = (S + FUSE_ROWS - 1) / FUSE_ROWS;
  // >= S: no row (the wave still keeps the barriers and helps gather)
  const int s = k * FUSE_ROWS + (xb % FUSE_HALVES) * FUSE_WAVES + wave;
  // Run of block `blk`: ranks [offs[k], offs[k+1]) (the last range ends at the count).
  int c[PER], sum = 0;
  {
    int lo[PER], hi[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int blk = min(PER * tid + q, nvb - 1);
      const int64_t o = (b * nvb + blk) * nr + k;
      lo[q] = offs[o];
      hi[q] = k + 1 < nr ? offs[o + 1] : cnt[b * nvb + blk];
    }
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int blk = PER * tid + q;
      c[q] = blk < nvb ? hi[q] - lo[q] : 0;
      if (blk < nvb) lo_of[blk] = lo[q];
      sum += c[q];
    }
  }
  int x = sum;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d);
    if (lane >= d) x += y;
  }
  if (lane == 63) wsum[wave] = x;
  __syncthreads();
  int before = 0, total = 0;
#pragma unroll
  for (int w = 0; w < FUSE_WAVES; ++w) {
    before += w < wave ? wsum[w] : 0;
    total += wsum[w];
  }
  int run = before + x - sum;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    pre[PER * tid + q] = run;
    run += c[q];
  }
  __syncthreads();
  f32x4 acc[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) acc[p] = f32x4{0.f, 0.f, 0.f, 0.f};
  int n = 0;  // entries in this wave's list (uniform)
  int par = 0;
  for (int t0 = 0; t0 < total; t0 += NT) {
    const int t = t0 + tid;
    if (t < total) {
      int lo = 0, hi = nvb;  // pre[lo] <= t < pre[hi]
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (pre[mid] <= t) lo = mid;
        else hi = mid;
      }
      stage[tid] = comp[(b * nvb + lo) * 64 + lo_of[lo] + (t - pre[lo])];
    }
    __syncthreads();
    const int here = min(NT, total - t0);
    for (int i = 0; i * 64 < here; ++i) {
      const int j = i * 64 + lane;
      const int2 e = j < here ? stage[j] : make_int2(-1, 0);
      const bool mine = j < here && (e.x >> FUSE_V_BITS) == s;
      const uint64_t bal = __ballot(mine);
      if (mine) lst[wave][n + __popcll(bal & ((1ull << lane) - 1ull))] = e;
      n += __popcll(bal);
      // If any row's list could overflow on the next 64 entries, gather the complete
      // batches listed (workgroup-uniform decision).
      if (i * 64 + 64 < here || t0 + NT < total) {
        if (lane == 0) sm.full[par][wave] = n > FUSE_CAP - 64 ? 1 : 0;
        __syncthreads();
        int any = 0;
#pragma unroll
        for (int w = 0; w < FUSE_WAVES; ++w) any |= sm.full[par][w];
        par ^= 1;
        if (any) dh_gather<T, NP, PER>(sm, W, D, wave, lane, n, false, share, acc);
      }
    }
    __syncthreads();  // stage is refilled next round
  }
  dh_gather<T, NP, PER>(sm, W, D, wave, lane, n, true, share, acc);
  if (s < S) {
    O* out = dH + (b * S + s) * D;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int d = p * 256 + lane * 4;
      if (d < D) store4(out + d, acc[p]);
    }
  }
}

// The fused path after the compaction: the dH workgroups (the first n_dh_x * B; the
// long rows start first) and the staged dW workgroups (FUSE_DW_IDS ids each) in one
// launch. The two read only the compaction and the inputs, so the dW work fills the
// CUs while the dH workgroups with long rows finish.
constexpr int FUSE_DW_IDS = 4 * FUSE_WAVES;
template <typename T, typename O, int NP, typename RT, int PER>
__global__ __launch_bounds__(64 * FUSE_WAVES) void bwd_fused_kernel(
    const T* __restrict__ grad, const RT* __restrict__ reps, const int32_t* __restrict__ idx,
    const void* __restrict__ mask, int mdt, const T* __restrict__ H, const T* __restrict__ W,
    const int2* __restrict__ comp, const int* __restrict__ cnt, const int* __restrict__ offs,
    O* __restrict__ dH, O* __restrict__ dW, O* __restrict__ dbias, int B, int S, int D, int V,
    int nvb, int n_dh_x, int share) {
  struct DwSmem {
    float gl[FUSE_DW_IDS * DW_LD];
    uint16_t sl[FUSE_DW_IDS * DW_LD];
  };
  union Smem {
    DhSmem<PER, NP> h;
    DwSmem w;
  };
  __shared__ Smem sm;
  const int n_dh = n_dh_x * B;
  if ((int)blockIdx.x < n_dh) {  // workgroup-uniform
    dh_fused_body<T, O, NP, PER>(sm.h, W, comp, cnt, offs, dH, S, D, nvb, blockIdx.x / n_dh_x,
                                 blockIdx.x % n_dh_x, share);
  } else {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int v0 = ((int)blockIdx.x - n_dh) * FUSE_DW_IDS;
    dw_stage<T, RT, FUSE_DW_IDS, FUSE_WAVES>(sm.w.gl, sm.w.sl, grad, reps, idx, mask, mdt, B, S,
                                             V, v0, wave, lane);
    __syncthreads();
    dw_gather<T, O, NP, RT, FUSE_DW_IDS, FUSE_WAVES>(sm.w.gl, sm.w.sl, H, dW, dbias, B, S, D, V,
                                                     v0, wave, lane);
  }
}

// Register passes for a row of D elements (4 per lane, 256 per pass), capped at MAX_NP
// (longer rows loop over D in chunks of MAX_NP * 256).
static int passes_for(int64_t D) {
  return (int)std::min<int64_t>(MAX_NP, std::max<int64_t>(1, cdiv(D, 256)));
}

// Fused dH: a workgroup's waves share the gathering when one row holds more than this
// many times the batches per wave (SPARTON_BWD_SHARE overrides it; tests use 0, always).
static int dh_share() {
  const char* e = getenv("SPARTON_BWD_SHARE");
  return e != nullptr ? atoi(e) : 2;
}
// Rows with more entries than this go to bwd_dh_hot_kernel (SPARTON_BWD_HOT_MIN overrides
// it; tests compare both).
static int dh_hot_min() {
  const char* e = getenv("SPARTON_BWD_HOT_MIN");
  return e != nullptr ? atoi(e) : HOT_MIN;
}
// The five-kernel dH takes its long-row load groups for large vocabularies
// (SPARTON_BWD_DH_LONG=1 forces them; tests compare the two).
static bool dh_long_rows(int64_t V) {
  const char* e = getenv("SPARTON_BWD_DH_LONG");
  return V > FUSE_V_FAST || (e != nullptr && strcmp(e, "1") == 0);
}
// Register passes from which the many-rows dH launch also takes dW's workgroups.
constexpr int DH_MERGE_NP = 6;
// ---- few dH rows (B * S <= FEW_ROWS) ------------------------------------------------------
//
// With few dH rows every W row serves several of them (config 1: each of the 30522 ids is
// active in both batch rows), so gathering W rows per dH row reads W once per batch row.
// Here one launch does all of the backward: a workgroup owns a range of vocabulary ids and
// a 256-column slice of D, and walks the range tile by tile (FEW_TILE ids), reading each W
// row of its slice once.
//   dH: wave w holds dH rows FEW_RPW w .. FEW_RPW w + FEW_RPW - 1 of the slice in registers
//   (lane l: columns 4 l .. 4 l + 3), indexed statically. A row b S + s takes the tile's
//   ids whose entry (b, id) is active with index s (one ballot), in ascending v, so its
//   partial sum runs over the range in ascending v; bwd_few_sum_kernel adds the ranges'
//   partials in range order. These sums are this path's own order (they agree with every
//   other path to fp32 rounding, not bitwise).
//   dW, dbias: wave w also owns the tile's ids 8 w .. 8 w + 7 and sums their active entries'
//   H rows (the slice of all B S rows sits in LDS) in ascending b, exactly as the staged dW
//   kernel does (same operations in the same order: the results are bitwise the same).
//
// The tile's W rows travel HBM -> registers -> LDS: they are loaded during the previous
// tile and written to LDS at the start of this one, so the loads overlap a whole tile's
// work. (Direct-to-LDS copies would not: the compiler cannot tell the copy's target from
// the buffer being read and waits for every copy before each LDS read.)
constexpr int FEW_ROWS = 64;                          // dH rows held per workgroup
constexpr int FEW_TILE = 64;                          // vocabulary ids per tile (one per lane)
constexpr int FEW_WAVES = 8;
constexpr int FEW_THREADS = 64 * FEW_WAVES;
constexpr int FEW_COLS = 256;                         // columns of D per slice (4 per lane)
constexpr int FEW_RPW = FEW_ROWS / FEW_WAVES;         // dH rows per wave
constexpr int FEW_IPW = FEW_TILE / FEW_WAVES;         // dW ids per wave
constexpr int FEW_IDC = 8;                            // dW ids summed together
constexpr int FEW_NJ = FEW_ROWS * FEW_TILE / FEW_THREADS;  // entry rounds: batch rows per wave
constexpr int FEW_ES_LD = 68;   // bytes per id of the index table: 17 words, odd, so a wave's
                                // 64 ids fall in 64 different banks
constexpr uint8_t FEW_NONE = 0xff;  // index table: inactive entry (S <= FEW_ROWS < 255)

// SPARTON_BWD_FEW=0 sends few-row batches down the count/scan/scatter path instead (tests
// compare the two).
static bool few_enabled() {
  const char* e = getenv("SPARTON_BWD_FEW");
  return e == nullptr || strcmp(e, "0") != 0;
}

struct FewPlan {
  bool fits;       // the shape qualifies (the workspace is sized for it whatever the switch)
  int slices, ranges, range_len;
  size_t part_bytes;
};
static FewPlan few_plan(int64_t B, int64_t S, int64_t D, int64_t V) {
  FewPlan p{};
  p.fits = B * S > 0 && B * S <= FEW_ROWS && D > 0 && V > 0;
  if (!p.fits) return p;
  p.slices = (int)cdiv(D, FEW_COLS);
  // about one workgroup per CU: each reads range_len W rows of its slice once
  const int64_t want = std::max<int64_t>(1, 256 / p.slices);
  p.range_len = (int)(cdiv(cdiv(V, FEW_TILE), want) * FEW_TILE);
  p.ranges = (int)cdiv(V, p.range_len);
  p.part_bytes = (size_t)p.ranges * (size_t)(B * S) * (size_t)D * 4;
  return p;
}

// Workgroup barrier once this wave's LDS operations are complete. Global loads in flight
// (the next tile's, into registers) are not waited for; the memory clobber keeps the
// compiler from moving memory accesses across it.
__device__ __forceinline__ void few_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Rows of a matrix with row stride D, slice columns c0 .. c0 + FEW_COLS - 1, in 16-byte
// chunks: chunk q = i * FEW_THREADS + thread is row q / CPR, chunk q % CPR of the row, so
// consecutive threads read consecutive bytes. Chunks past D re-read the slice's first chunk
// (those columns are never stored); D * sizeof(T) is a multiple of 16.
template <typename T>
struct FewChunks {
  static constexpr int CPR = FEW_COLS * (int)sizeof(T) / 16;  // chunks per row
  static constexpr int PER = 16 / (int)sizeof(T);             // elements per chunk
  static __device__ __forceinline__ u32x4 load(const T* __restrict__ M, int row, int q, int D,
                                               int c0) {
    const int col = c0 + (q % CPR) * PER;
    return *(const u32x4*)(M + (int64_t)row * D + (col < D ? col : c0));
  }
};

// One tile's W rows (ids past V re-read id V-1: their entries are inactive), held in
// registers between their load and their store to LDS.
template <typename T>
struct FewStage {
  static constexpr int NL = FEW_TILE * FewChunks<T>::CPR / FEW_THREADS;  // chunks per thread
  u32x4 c[NL];
  __device__ __forceinline__ void load(const T* __restrict__ W, int v0, int V, int D, int c0,
                                       int t) {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int q = i * FEW_THREADS + t;
      c[i] = FewChunks<T>::load(W, min(v0 + q / FewChunks<T>::CPR, V - 1), q, D, c0);
    }
  }
  __device__ __forceinline__ void store(T* wt, int t) const {
#pragma unroll
    for (int i = 0; i < NL; ++i) ((u32x4*)wt)[i * FEW_THREADS + t] = c[i];
  }
};

template <typename T, typename O, typename RT>
__global__ __launch_bounds__(FEW_THREADS) void bwd_few_kernel(
    const T* __restrict__ grad, const RT* __restrict__ reps, const int32_t* __restrict__ idx,
    const void* __restrict__ mask, int mdt, const T* __restrict__ H, const T* __restrict__ W,
    float* __restrict__ part, O* __restrict__ dW, O* __restrict__ dbias, int B, int S, int D,
    int V, int slices, int range_len) {
  // Each table has one more row, of zeros (row FEW_TILE, FEW_ROWS): a pass points a row or
  // id with no entry left at it, and adding g' * w = +0 * +0 changes no sum.
  __shared__ __attribute__((aligned(16))) T wt[FEW_TILE + 1][FEW_COLS];  // the tile's W rows
  __shared__ __attribute__((aligned(16))) T hs[FEW_ROWS + 1][FEW_COLS];  // H's B*S rows, this slice
  __shared__ float eg[FEW_ROWS][FEW_TILE + 1];  // g' of entry (b, v0 + id) at [b][id], 0 = inactive
  __shared__ uint8_t es[FEW_TILE][FEW_ES_LD];       // its index s, FEW_NONE = inactive
  __shared__ float maskf[FEW_ROWS];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // uniform: scalar registers, branches
  const int range = (int)blockIdx.x / slices, slice = (int)blockIdx.x - range * slices;
  const int c0 = slice * FEW_COLS;
  const int BS = B * S;
  const int v_beg = range * range_len, v_end = min(V, v_beg + range_len);
  const bool dw_on = dW != nullptr || dbias != nullptr;
  for (int i = t; i < BS; i += FEW_THREADS) maskf[i] = load_mask(mask, mdt, i);
  for (int i = t; i < FEW_COLS; i += FEW_THREADS) {
    wt[FEW_TILE][i] = T(0.0f);
    hs[FEW_ROWS][i] = T(0.0f);
  }
  for (int i = t; i < FEW_ROWS; i += FEW_THREADS) eg[i][FEW_TILE] = 0.0f;
  if (dW != nullptr) {  // (H may be absent when only dbias is asked for)
    for (int q = t; q < BS * FewChunks<T>::CPR; q += FEW_THREADS)
      ((u32x4*)&hs[0][0])[q] = FewChunks<T>::load(H, q / FewChunks<T>::CPR, q, D, c0);
  }
  // This wave's dH rows: batch row and index of each (rows past B*S take none).
  int rb[FEW_RPW], rs[FEW_RPW];
#pragma unroll
  for (int r = 0; r < FEW_RPW; ++r) {
    const int row = wave * FEW_RPW + r;
    rb[r] = row < BS ? row / S : 0;
    rs[r] = row < BS ? row - rb[r] * S : -1;
  }
  f32x4 acc[FEW_RPW];
#pragma unroll
  for (int r = 0; r < FEW_RPW; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
  // The tile's W rows and entries (b, v0 + lane), loaded one tile ahead; round j of wave w
  // holds batch row b = FEW_WAVES j + w (B <= FEW_ROWS).
  FewStage<T> stage;
  T gr[FEW_NJ];
  RT rr[FEW_NJ];
  int sr[FEW_NJ];
  auto load_entries = [&](int v0) {
    const int v = min(v0 + lane, V - 1);
#pragma unroll
    for (int j = 0; j < FEW_NJ; ++j) {
      const int b = FEW_WAVES * j + wave;
      if (b < B) {  // uniform per wave
        const int64_t o = (int64_t)b * V + v;
        gr[j] = grad[o];
        rr[j] = reps[o];
        sr[j] = idx[o];
      }
    }
  };
  stage.load(W, v_beg, V, D, c0, t);
  load_entries(v_beg);
  const T* wcol = &wt[0][lane * 4];
  const int c = c0 + lane * 4;
  for (int v0 = v_beg; v0 < v_end; v0 += FEW_TILE) {
    // the previous tile's rows and ids are done: wt, eg and es are free
    few_barrier();
    stage.store(&wt[0][0], t);
    const bool more = v0 + FEW_TILE < v_end;
    // The next tile's W rows load under all of this tile's work; its entries load once
    // this tile's are used, below. (The next tile's first wait is for all of them, and for
    // this tile's dW stores: stores and loads share one counter.)
    if (more) stage.load(W, v0 + FEW_TILE, V, D, c0, t);
    const int v = v0 + lane;
#pragma unroll
    for (int j = 0; j < FEW_NJ; ++j) {
      const int b = FEW_WAVES * j + wave;
      if (b < B) {  // uniform per wave
        float gp;
        const int si = sr[j];
        const bool act = v < v_end && entry(gr[j], rr[j], si, maskf + b * S, S, &gp) &&
                         gp != 0.0f;
        eg[b][lane] = act ? gp : 0.0f;
        es[lane][b] = act ? (uint8_t)si : FEW_NONE;
      }
    }
    if (more) load_entries(v0 + FEW_TILE);
    few_barrier();
    // dW, dbias: this wave's ids, FEW_IDC at a time, pass k taking each id's k-th active
    // batch row (ascending); an id with none left takes the zero rows.
    if (dw_on) {
#pragma unroll 1
      for (int i0 = 0; i0 < FEW_IPW; i0 += FEW_IDC) {
        uint64_t p[FEW_IDC];
        int npass = 0;
#pragma unroll
        for (int i = 0; i < FEW_IDC; ++i) {
          const int il = wave * FEW_IPW + i0 + i;
          // eg holds +0.0 for every inactive entry
          p[i] = __ballot(lane < B && __float_as_int(eg[min(lane, FEW_ROWS - 1)][il]) != 0);
          npass = max(npass, __popcll(p[i]));
        }
        f32x4 ad[FEW_IDC];
        float bsum[FEW_IDC];
#pragma unroll
        for (int i = 0; i < FEW_IDC; ++i) {
          ad[i] = f32x4{0.f, 0.f, 0.f, 0.f};
          bsum[i] = 0.0f;
        }
        for (int k = 0; k < npass; ++k) {
          float g[FEW_IDC];
          f32x4 h[FEW_IDC];
#pragma unroll
          for (int i = 0; i < FEW_IDC; ++i) {
            const bool on = p[i] != 0;  // uniform
            const int b = on ? (int)__builtin_ctzll(p[i]) : 0;
            p[i] &= ~(1ull << b);
            const int iv = wave * FEW_IPW + i0 + i;
            g[i] = eg[b][on ? iv : FEW_TILE];
            const int hr = on ? b * S + (int)es[iv][b] : FEW_ROWS;
            h[i] = load4(&hs[hr][lane * 4]);
          }
#pragma unroll
          for (int i = 0; i < FEW_IDC; ++i) {
            ad[i] = f32x4{fmaf(g[i], h[i][0], ad[i][0]), fmaf(g[i], h[i][1], ad[i][1]),
                          fmaf(g[i], h[i][2], ad[i][2]), fmaf(g[i], h[i][3], ad[i][3])};
            bsum[i] += g[i];
          }
        }
#pragma unroll
        for (int i = 0; i < FEW_IDC; ++i) {
          const int vi = v0 + wave * FEW_IPW + i0 + i;
          if (vi < v_end) {
            if (dW != nullptr && c < D) store4(dW + (int64_t)vi * D + c, ad[i]);
            if (dbias != nullptr && slice == 0 && lane == 0) dbias[vi] = from_f32<O>(bsum[i]);
          }
        }
      }
    }
    // dH: this wave's rows, pass k taking each row's k-th id (ascending); a row with none
    // left takes the zero rows. Straight-line passes: the ids are scalar, the coefficients
    // come by broadcast LDS reads, and a pass's reads are independent of each other.
    {
      uint64_t m[FEW_RPW];
      int npass = 0;
#pragma unroll
      for (int r = 0; r < FEW_RPW; ++r) {
        m[r] = __ballot((int)es[lane][rb[r]] == rs[r]);
        npass = max(npass, __popcll(m[r]));
      }
      for (int k = 0; k < npass; ++k) {
        float g[FEW_RPW];
        f32x4 w[FEW_RPW];
#pragma unroll
        for (int r = 0; r < FEW_RPW; ++r) {
          const int id = m[r] != 0 ? (int)__builtin_ctzll(m[r]) : FEW_TILE;  // uniform
          m[r] &= ~(1ull << (id & 63));
          g[r] = eg[rb[r]][id];
          w[r] = load4(wcol + id * FEW_COLS);
        }
#pragma unroll
        for (int r = 0; r < FEW_RPW; ++r)
          acc[r] = f32x4{fmaf(g[r], w[r][0], acc[r][0]), fmaf(g[r], w[r][1], acc[r][1]),
                         fmaf(g[r], w[r][2], acc[r][2]), fmaf(g[r], w[r][3], acc[r][3])};
      }
    }
  }
  if (c < D) {
    float* out = part + (int64_t)range * BS * D + c;
#pragma unroll
    for (int r = 0; r < FEW_RPW; ++r) {
      const int row = wave * FEW_RPW + r;
      if (row < BS) *(f32x4*)(out + (int64_t)row * D) = acc[r];
    }
  }
}

// dH = the ranges' partial rows added in range order, in the output dtype. A workgroup
// takes 256 elements (4 per lane of a wave); its FEW_SUM_WAVES waves sum consecutive
// groups of the ranges, and the groups are added in order.
constexpr int FEW_SUM_WAVES = 8;
template <typename O>
__global__ __launch_bounds__(64 * FEW_SUM_WAVES) void bwd_few_sum_kernel(
    const float* __restrict__ part, O* __restrict__ dH, int64_t n, int ranges) {
  __shared__ f32x4 red[FEW_SUM_WAVES - 1][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t i = ((int64_t)blockIdx.x * 64 + lane) * 4;
  const int q = (ranges + FEW_SUM_WAVES - 1) / FEW_SUM_WAVES;
  const int k0 = min(ranges, wave * q), k1 = min(ranges, k0 + q);
  f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
  if (i < n) {  // n is a multiple of 4
    int k = k0;
    for (; k + 4 <= k1; k += 4) {
      f32x4 x[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = *(const f32x4*)(part + (int64_t)(k + j) * n + i);
#pragma unroll
      for (int j = 0; j < 4; ++j) s += x[j];
    }
    for (; k < k1; ++k) s += *(const f32x4*)(part + (int64_t)k * n + i);
  }
  if (wave > 0) red[wave - 1][lane] = s;
  __syncthreads();
  if (wave == 0 && i < n) {
#pragma unroll
    for (int w = 0; w < FEW_SUM_WAVES - 1; ++w) s += red[w][lane];
    store4(dH + i, s);
  }
}

// The five-kernel path runs dW in the dH launch where it can (SPARTON_BWD_DW_MERGE=0 keeps
// it a separate launch; tests compare the two).
static bool dw_merge_on() {
  const char* e = getenv("SPARTON_BWD_DW_MERGE");
  return e == nullptr || strcmp(e, "0") != 0;
}
// SPARTON_BWD_PATH=five forces the five-kernel path (tests compare the two paths).
static bool fused_path_enabled() {
  const char* e = getenv("SPARTON_BWD_PATH");
  return e == nullptr || strcmp(e, "five") != 0;
}

// The wide staged dW with 16 ids per workgroup (B <= DW_WIDE_B), for 16-bit types: fp32
// rows gather two ids at a time, which 16 ids over 16 waves cannot give. Returns whether it
// launched.
template <typename T, typename O, int DNP, typename RT>
static bool wide16(const T* g, const RT* r, const int32_t* idx, const void* mask, int mdt,
                   const T* H, O* dW, O* dbias, int64_t B, int64_t S, int64_t D, int64_t V,
                   hipStream_t st) {
  if constexpr (sizeof(T) == 2) {
    if (B <= DW_WIDE_B && S <= DW_STAGE_S) {
      hipLaunchKernelGGL((bwd_dw_wide_kernel<T, O, DNP, RT, 16>), dim3((unsigned)cdiv(V, 16)),
                         dim3(64 * DW_WAVES), 0, st, g, r, idx, mask, mdt, H, dW, dbias, (int)B,
                         (int)S, (int)D, (int)V);
      return true;
    }
  }
  return false;
}

template <typename T, typename O, int NP, typename RT>
static void launch_rows(const T* g, const RT* r, const int32_t* idx, const void* mask,
                        int mdt, const T* H, const T* W, O* dH, O* dW, O* dbias, void* ws,
                        int64_t B, int64_t S, int64_t D, int64_t V, hipStream_t st) {
  constexpr int FNP = NP <= FuseMaxNp<T>::value ? NP : FuseMaxNp<T>::value;
  // The fused path stages, per (b, 16-row range), a prefix over every 64-id block, and
  // gives each dH row one wave: it needs many ranges and few blocks. Measured on MI355X:
  // B = 32, S = 256, V = 30522: fused 61 us vs 65 us; B = 2, S = 32 (dense grads):
  // 1133 us vs 331 us; V = 250002: 753 us vs 460 us.
  const FewPlan few = few_plan(B, S, D, V);
  if (few.fits && few_enabled() && dH != nullptr) {
    float* part = (float*)ws;
    hipLaunchKernelGGL((bwd_few_kernel<T, O, RT>), dim3((unsigned)(few.ranges * few.slices)),
                       dim3(FEW_THREADS), 0, st, g, r, idx, mask, mdt, H, W, part, dW, dbias,
                       (int)B, (int)S, (int)D, (int)V, few.slices, few.range_len);
    const int64_t n = B * S * D;
    hipLaunchKernelGGL((bwd_few_sum_kernel<O>), dim3((unsigned)cdiv(n, 256)), dim3(64 * FEW_SUM_WAVES),
                       0, st,
                       (const float*)part, dH, n, few.ranges);
    return;
  }
  const bool fused = fused_path_enabled() && dH != nullptr && dW != nullptr && B * S > 0 &&
                     D > 0 && V > 0 &&
                     B <= DW_STAGE_B && S <= FUSE_MAX_S && V <= FUSE_V_FAST &&
                     B * cdiv(S, FUSE_ROWS) >= FUSE_MIN_RANGES &&
                     D <= (int64_t)FNP * 256;
  if (fused) {
    const Layout L = layout(B, S, V);
    int2* comp = (int2*)((char*)ws + L.list);
    int* cnt = (int*)((char*)ws + L.cnt64);
    int* offs = (int*)((char*)ws + L.off64);
    const int nvb = (int)cdiv(V, 64);
    hipLaunchKernelGGL((bwd_compact_kernel<T, RT>), dim3((unsigned)nvb, (unsigned)cdiv(B, 8)), dim3(256),
                       0, st, g, r, idx, mask, mdt, (int)B, (int)S, (int)V, comp, cnt, offs);
    const int n_dh_x = (int)(FUSE_HALVES * cdiv(S, FUSE_ROWS));
    const dim3 grid((unsigned)(n_dh_x * B + cdiv(V, FUSE_DW_IDS)));
#define FUSED(PER)                                                                                  \
  hipLaunchKernelGGL((bwd_fused_kernel<T, O, FNP, RT, PER>), grid, dim3(64 * FUSE_WAVES), 0, st, g,  \
                     r, idx, mask, mdt, H, W, (const int2*)comp, (const int*)cnt, (const int*)offs, \
                     dH, dW, dbias, (int)B, (int)S, (int)D, (int)V, nvb, n_dh_x, dh_share())
    if (nvb <= 64 * FUSE_WAVES) FUSED(1);
    else FUSED(FUSE_MAX_NVB / (64 * FUSE_WAVES));
#undef FUSED
    return;
  }
  bool merged_dw = false;
  if (dH != nullptr && B * S > 0 && D > 0) {
    // Batch rows in chunks of at most MAX_B and positions in windows of at most MAX_S:
    // each pass runs count -> scan -> scatter -> dH over rows [b0, b0 + nb) and
    // positions [s0, s0 + sw), with entries whose index lies outside the window
    // inactive, so every dH row is written by exactly one pass. The workspace holds
    // one pass; the passes reuse it in stream order.
    const int64_t Bc = std::min<int64_t>(B, MAX_B), Sc = std::min<int64_t>(S, MAX_S);
    const Layout L = layout(Bc, Sc, V);
    int* hist = (int*)((char*)ws + L.hist);
    int* seg_start = (int*)((char*)ws + L.seg_start);
    int* seg_cnt = (int*)((char*)ws + L.seg_cnt);
    int2* list = (int2*)((char*)ws + L.list);
    int2* comp = (int2*)((char*)ws + L.comp);
    int* ccount = (int*)((char*)ws + L.ccount);
    int* hot = (int*)((char*)ws + L.hot);
    const int hot_min = dh_hot_min();
    // One pass and a staged dW: dW's workgroups join the dH launch when that launch
    // does not take dW's occupancy away. Measured (backward, one box): few rows (config
    // 1, split dH) 78.9 -> 73.6 us; wide rows (config 5, D = 4096: 182 VGPRs for dH
    // against 107 for dW) 520 -> 504 us; but config 4 (D = 768, long rows: dH at 125
    // VGPRs, dW at 58) 328 -> 346 us, so rows under DH_MERGE_NP passes keep two launches.
    const bool few_rows = B * S < SPLIT_ROWS;
    merged_dw = (dW != nullptr || dbias != nullptr) && V > 0 && B <= Bc && S <= Sc &&
                B <= DW_STAGE_B && S <= DW_STAGE_S && L.nch > 0 && dw_merge_on() &&
                (few_rows || DhPasses<NP>::value >= DH_MERGE_NP);
    for (int64_t b0 = 0; b0 < B; b0 += Bc) {
      const int64_t nb = std::min(Bc, B - b0);
      const T* gb = g + b0 * V;
      const RT* rb = r + b0 * V;
      const int32_t* ib = idx + b0 * V;
      for (int64_t s0 = 0; s0 < S; s0 += Sc) {
        const int64_t sw = std::min(Sc, S - s0);
        O* dhb = dH + (b0 * S + s0) * D;
        const int wpb = waves_for(sw);
        const dim3 cgrid((unsigned)cdiv(L.nch, wpb), (unsigned)nb);
        const size_t cl = (size_t)sw * 4 * (1 + wpb);
        if (L.nch > 0)
          hipLaunchKernelGGL((bwd_count_kernel<T, RT>), cgrid, dim3(64 * wpb), cl, st, gb, rb, ib,
                             mask, mdt, (int)sw, (int)V, (int)L.nch, hist, comp, ccount, (int)s0,
                             b0, (int)S, hot);
        if (sw <= SCAN_THREADS / 2)
          hipLaunchKernelGGL(bwd_scan_parts_kernel, dim3((unsigned)nb), dim3(SCAN_THREADS), 0, st,
                             hist, seg_start, seg_cnt, (int)sw, (int)L.nch, (int)round_up(sw, 64),
                             hot, hot_min);
        else
          hipLaunchKernelGGL(bwd_scan_kernel, dim3((unsigned)nb),
                             dim3((unsigned)std::min<int64_t>(SCAN_THREADS, round_up(sw, 64))), 0, st,
                             hist, seg_start, seg_cnt, (int)sw, (int)L.nch, hot, hot_min);
        if (L.nch > 0)
          hipLaunchKernelGGL(bwd_scatter_kernel, cgrid, dim3(64 * wpb), (size_t)sw * 4 * wpb, st, ib,
                             (int)sw, (int)V, (int)L.nch, (const int*)hist, (const int2*)comp,
                             (const int*)ccount, list, (int)s0);
        if (nb * sw < SPLIT_ROWS) {
          const int64_t ns = cdiv(D, 256);
          if (merged_dw)
            hipLaunchKernelGGL((bwd_dh_split_dw_kernel<T, O, DwPasses<T, NP>::value, RT>),
                               dim3((unsigned)(nb * sw * ns + cdiv(V, 4 * SPLIT_WAVES))),
                               dim3(64 * SPLIT_WAVES), 0, st, W, (const int2*)list,
                               (const int*)seg_start, (const int*)seg_cnt, dhb, (int)B, (int)S,
                               (int)D, (int)V, (int)ns, (int)(nb * sw * ns), g, r, idx, mask, mdt,
                               H, dW, dbias);
          else
            hipLaunchKernelGGL((bwd_dh_split_kernel<T, O>), dim3((unsigned)(nb * sw * ns)),
                               dim3(64 * SPLIT_WAVES), 0, st, W, (const int2*)list,
                               (const int*)seg_start, (const int*)seg_cnt, dhb, (int)nb, (int)sw,
                               (int)D, (int)V, (int)S, (int)ns);
        } else if (merged_dw) {
          if constexpr (DhPasses<NP>::value >= DH_MERGE_NP) {
            const int n_dh = (int)cdiv(nb * sw, 4);
            const dim3 grid((unsigned)(n_dh + cdiv(V, 16)));
            if (dh_long_rows(V))
              hipLaunchKernelGGL((bwd_dh_dw_kernel<T, O, DhPasses<NP>::value, true, DwPasses<T, NP>::value, RT>),
                                 grid, dim3(256), 0, st, W, (const int2*)list, (const int*)seg_start,
                                 (const int*)seg_cnt, dhb, (int)B, (int)S, (int)D, (int)V, hot_min,
                                 n_dh, g, r, idx, mask, mdt, H, dW, dbias);
            else
              hipLaunchKernelGGL((bwd_dh_dw_kernel<T, O, DhPasses<NP>::value, false, DwPasses<T, NP>::value, RT>),
                                 grid, dim3(256), 0, st, W, (const int2*)list, (const int*)seg_start,
                                 (const int*)seg_cnt, dhb, (int)B, (int)S, (int)D, (int)V, hot_min,
                                 n_dh, g, r, idx, mask, mdt, H, dW, dbias);
          }
          if (L.nch > 0)
            hipLaunchKernelGGL((bwd_dh_hot_kernel<T, O>), dim3(HOT_GRID), dim3(64 * HOT_WAVES), 0, st, W,
                               (const int2*)list, (const int*)seg_start, (const int*)seg_cnt,
                               (const int*)hot, dhb, (int)sw, (int)D, (int)V, (int)S,
                               (int)cdiv(D, 256));
        } else {
          if (dh_long_rows(V))
            hipLaunchKernelGGL((bwd_dh_kernel<T, O, DhPasses<NP>::value, true>), dim3((unsigned)cdiv(nb * sw, 4)),
                               dim3(256), 0, st, W, (const int2*)list, (const int*)seg_start,
                               (const int*)seg_cnt, dhb, (int)nb, (int)sw, (int)D, (int)V, (int)S,
                               hot_min);
          else
            hipLaunchKernelGGL((bwd_dh_kernel<T, O, DhPasses<NP>::value, false>), dim3((unsigned)cdiv(nb * sw, 4)),
                               dim3(256), 0, st, W, (const int2*)list, (const int*)seg_start,
                               (const int*)seg_cnt, dhb, (int)nb, (int)sw, (int)D, (int)V, (int)S,
                               hot_min);
          // The rows bwd_dh_kernel left (listed by the scan; the count kernel zeroed the list).
          if (L.nch > 0)
            hipLaunchKernelGGL((bwd_dh_hot_kernel<T, O>), dim3(HOT_GRID), dim3(64 * HOT_WAVES), 0, st, W,
                               (const int2*)list, (const int*)seg_start, (const int*)seg_cnt,
                               (const int*)hot, dhb, (int)sw, (int)D, (int)V, (int)S,
                               (int)cdiv(D, 256));
        }
      }
    }
  }
  if ((dW != nullptr || dbias != nullptr) && V > 0 && !merged_dw) {
    constexpr int DNP = DwPasses<T, NP>::value;
    if (B <= DW_STAGE_B && S <= DW_STAGE_S)
      hipLaunchKernelGGL((bwd_dw_staged_kernel<T, O, DNP, RT>),
                         dim3((unsigned)cdiv(V, 64)), dim3(64 * DW_WAVES), 0,
                         st, g, r, idx, mask, mdt, H, dW, dbias, (int)B, (int)S, (int)D, (int)V);
    else if (B <= DW_WIDE_IDS_ROWS / 64 && S <= DW_STAGE_S)
      hipLaunchKernelGGL((bwd_dw_wide_kernel<T, O, DNP, RT, 64>), dim3((unsigned)cdiv(V, 64)),
                         dim3(64 * DW_WAVES), 0, st, g, r, idx, mask, mdt, H, dW, dbias, (int)B,
                         (int)S, (int)D, (int)V);
    else if (B <= DW_WIDE_IDS_ROWS / 32 && S <= DW_STAGE_S)
      hipLaunchKernelGGL((bwd_dw_wide_kernel<T, O, DNP, RT, 32>), dim3((unsigned)cdiv(V, 32)),
                         dim3(64 * DW_WAVES), 0, st, g, r, idx, mask, mdt, H, dW, dbias, (int)B,
                         (int)S, (int)D, (int)V);
    else if (!wide16<T, O, DNP, RT>(g, r, idx, mask, mdt, H, dW, dbias, B, S, D, V, st))
      hipLaunchKernelGGL((bwd_dw_kernel<T, O, NP, RT>), dim3((unsigned)cdiv(V, 4)), dim3(256), 0, st,
                         g, r, idx, mask, mdt, H, dW, dbias, (int)B, (int)S, (int)D, (int)V);
  }
}

template <typename T, typename O>
static int launch(const void* grad, const void* r, int rdt, const int32_t* idx, const void* mask,
                  int mdt, const void* H, const void* W, void* dH, void* dW, void* dbias,
                  void* ws, int64_t B, int64_t S, int64_t D, int64_t V, hipStream_t st) {
  const T* g = (const T*)grad;
  const T* h = (const T*)H;
  const T* w = (const T*)W;
#define SPARTON_ROWS(NP)                                                                        \
  (rdt == SPARTON_F32                                                                           \
       ? launch_rows<T, O, NP, float>(g, (const float*)r, idx, mask, mdt, h, w, (O*)dH, (O*)dW, \
                                      (O*)dbias, ws, B, S, D, V, st)                            \
       : launch_rows<T, O, NP, T>(g, (const T*)r, idx, mask, mdt, h, w, (O*)dH, (O*)dW,         \
                                  (O*)dbias, ws, B, S, D, V, st))
  switch (passes_for(D)) {
    case 1: SPARTON_ROWS(1); break;
    case 2: SPARTON_ROWS(2); break;
    case 3: SPARTON_ROWS(3); break;
    case 4: SPARTON_ROWS(4); break;
    case 5: case 6: SPARTON_ROWS(6); break;
    case 7: case 8: SPARTON_ROWS(8); break;
    case 9: case 10: case 11: case 12: SPARTON_ROWS(12); break;
    default: SPARTON_ROWS(16); break;
  }
#undef SPARTON_ROWS
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPARTON_OK : (int)e;
}

}  // namespace bwd
}  // namespace sparton

using namespace sparton;

extern "C" __attribute__((visibility("default"))) size_t sparton_bwd_workspace_bytes(
    int64_t B, int64_t S, int64_t D, int64_t V) {
  if (B <= 0 || S <= 0 || D <= 0 || V < 0) return 0;
  const bwd::FewPlan few = bwd::few_plan(B, S, D, V);
  return std::max(bwd::pass_layout(B, S, V).total, few.fits ? few.part_bytes : (size_t)0);
}

extern "C" __attribute__((visibility("default"))) int sparton_bwd(
    const void* grad_reps, const void* reps, int reps_dtype, const int32_t* argmax,
    const void* mask, int mask_dtype, const void* hidden, const void* weight, void* d_hidden,
    void* d_weight, void* d_bias, int grad_dtype, void* workspace, size_t workspace_bytes,
    int64_t B, int64_t S, int64_t D, int64_t V, int dtype, void* stream) {
  if (B < 0 || S < 0 || D < 0 || V < 0) return SPARTON_EINVAL;
  if (dtype < SPARTON_F32 || dtype > SPARTON_F16) return SPARTON_EINVAL;
  if (reps_dtype != SPARTON_F32 && reps_dtype != dtype) return SPARTON_EINVAL;
  if (grad_dtype != SPARTON_F32 && grad_dtype != dtype) return SPARTON_EINVAL;
  if (mask_dtype < SPARTON_MASK_I64 || mask_dtype > SPARTON_MASK_F16) return SPARTON_EINVAL;
  if (B * V > 0 && (grad_reps == nullptr || reps == nullptr || argmax == nullptr || mask == nullptr))
    return SPARTON_EINVAL;
  const bool need_dh = d_hidden != nullptr && B * S > 0 && D > 0;
  const bool need_dw = (d_weight != nullptr || d_bias != nullptr) && V > 0;
  if (need_dh && weight == nullptr) return SPARTON_EINVAL;
  if (need_dw && d_weight != nullptr && D > 0 && B * S > 0 && hidden == nullptr) return SPARTON_EINVAL;
  const int64_t esz = dtype == SPARTON_F32 ? 4 : 2;
  if ((D * esz) % 16 != 0) return SPARTON_EINVAL;
  if (((uintptr_t)hidden | (uintptr_t)weight) % 16 != 0) return SPARTON_EALIGN;
  // Outputs are written 4 elements at a time: 16 bytes (fp32) or 8 bytes (16-bit).
  const uintptr_t oalign = grad_dtype == SPARTON_F32 ? 16 : 8;
  if (((uintptr_t)d_hidden | (uintptr_t)d_weight) % oalign != 0) return SPARTON_EALIGN;
  if (D > INT32_MAX || V > INT32_MAX || B * S > INT32_MAX || B * V > INT32_MAX)
    return SPARTON_EUNSUPPORTED;
  if (need_dh) {
    if (workspace == nullptr) return SPARTON_EWORKSPACE;
    if (workspace_bytes < sparton_bwd_workspace_bytes(B, S, D, V)) return SPARTON_EWORKSPACE;
    if ((uintptr_t)workspace % 256 != 0) return SPARTON_EALIGN;
  }
  if (!need_dh && !need_dw) return SPARTON_OK;
  hipStream_t st = (hipStream_t)stream;
  void* dh = need_dh ? d_hidden : nullptr;
  const bool f32out = grad_dtype == SPARTON_F32;
#define SPARTON_BWD(T)                                                                           \
  (f32out ? bwd::launch<T, float>(grad_reps, reps, reps_dtype, argmax, mask, mask_dtype, hidden, \
                                  weight, dh, d_weight, d_bias, workspace, B, S, D, V, st)       \
          : bwd::launch<T, T>(grad_reps, reps, reps_dtype, argmax, mask, mask_dtype, hidden,     \
                              weight, dh, d_weight, d_bias, workspace, B, S, D, V, st))
  switch (dtype) {
    case SPARTON_BF16: return SPARTON_BWD(bf16);
    case SPARTON_F16: return SPARTON_BWD(f16);
    default: return SPARTON_BWD(float);
  }
#undef SPARTON_BWD
}
