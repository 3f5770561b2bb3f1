// SpartonHead forward on gfx950: a plan pass, one MFMA kernel with a fused reduction
// epilogue, and a small fixup pass.
//
// Math (reference src/sparton/sparton_kernel.py):
//     x[b,s,v] = (H[b,s,:] . W[v,:] + bias[v]) * mask[b,s]     bias :209-210/:245, mask :147
//     M[b,v]   = max(0, max_s x),  I[b,v] = lowest s attaining M (0 if M == 0)
//                                             init 0/0 :112-114, ties :151-156
//     reps     = log1p(M)                                        :159-161 (log(1+x) there)
// The [B,S,V] logits never reach HBM.
//
// Packing. Positions are grouped 16 at a time: group (b, j) = positions 16j..16j+15 of
// batch row b. A group whose mask is all zero contributes x = 0, which never beats the
// initial 0, so it is dropped. The plan pass lists the remaining ("active") groups in
// (b, j) order, and the main kernel multiplies them sixteen at a time: M-tile m holds
// active groups 16m..16m+15, i.e. 256 rows that may belong to several batch rows.
// Every tile except the last is full, so each decoder tile loaded from memory is used
// for 256 live rows instead of one batch row's (often partly padded) 256 positions,
// and a batch row wastes less than 16 rows of padding.
//
// Main kernel. A "unit" is one M-tile x one vocab tile of BN columns. The grid is
// persistent (one workgroup per CU) and each workgroup walks its units in rounds; for
// each it computes the 256 x BN logit tile with bf16/fp16 (or fp32) MFMA, K = D
// streamed through two LDS stages. The K slabs of all its units form one stream, and
// the next unit's metadata (group list, row mask, row offsets, bias) is fetched during
// the current unit's first K steps, so a unit starts while the previous one finishes.
// Eight compute waves run the MFMAs and the epilogue; four copy waves issue all copies
// and write the results. The epilogue folds each group into a per-column (max, argmax),
// merges consecutive groups of the same batch row in s order (larger value; on ties
// the lower s, which is the earlier group), and per batch-row segment either writes
// reps/argmax (segment complete in this tile) or, when the segment continues into a
// neighbouring tile, writes the partial (max, argmax) to the workspace.
//
// Fixup kernel. For each batch row whose groups span several M-tiles it merges those
// partials in tile order (= s order) and writes reps/argmax; for a batch row with no
// active group it writes reps = 0, argmax = 0.
//
// Data movement: K slabs of 128 bytes per row go straight from global memory into
// LDS (global_load_lds_dwordx4, no VGPR staging). LDS rows are 128 bytes with the
// 16-byte chunk index XOR-swizzled by f(row) = (row & 7) ^ ((row >> 3) & 1). The MFMA
// operand reads are ds_read_b128 of 32 consecutive rows at one logical chunk; gfx950's
// 64 banks serve 16 lanes (256 bytes) per cycle, and over any 16 aligned rows the
// pairs (row & 1, chunk ^ f(row)) are all distinct, so each read is conflict-free
// (and so is any 8-lane group, since f is distinct over 8 aligned rows).
// A K tail (D not a multiple of the slab) re-reads valid data and zeroes the W chunks
// past D in LDS; a unit always has at least two slabs (a second, all-zero slab is
// added when D fits in one), which keeps the two-stage stream uniform.

#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "sparton_common.h"

namespace sparton {
namespace fwd {

constexpr int BM = 256;              // rows per M-tile
constexpr int BN = 256;              // vocab columns per tile
constexpr int WAVES_M = 2;           // compute waves along M
constexpr int WAVES_N = 4;           // compute waves along N (vocab)
// Roles. Waves 0..7 compute (a 2 x 4 grid of 128 x 64 tiles). Waves 8..11, the copy
// waves (one per SIMD), move data: they issue every slab copy, fetch the next unit's
// metadata and write the previous unit's results. A wave waits while the address unit
// takes its copies; this way no compute wave ever does, and the matrix pipe of each
// SIMD is fed by its two compute waves. Three waves per SIMD leave 168 VGPRs each.
constexpr int COMPUTE_WAVES = WAVES_M * WAVES_N;
constexpr int COPY_WAVES = 4;
constexpr int COPY_THREADS = 64 * COPY_WAVES;
constexpr int NTHREADS = 64 * (COMPUTE_WAVES + COPY_WAVES);
constexpr int MBLK = BM / 32;        // 32-row MFMA blocks per M-tile (8)
constexpr int GROUP = 16;            // positions are packed into M-tiles 16 at a time
constexpr int NGRP = BM / GROUP;     // groups per M-tile (16); MFMA block j = groups 2j, 2j+1
constexpr int NB_PER_WAVE = BN / WAVES_N / 32;     // 2
constexpr int SLAB = 128;            // bytes of K per row per pipeline stage
constexpr int CHUNKS = SLAB / 16;    // 16-byte chunks per row slab (8)
constexpr int ROWS_PER_LOAD = 64 / CHUNKS;          // rows one wave-wide load covers (8)
constexpr int A_LOADS = BM / ROWS_PER_LOAD / COPY_WAVES;  // wave-wide copies per slab for A (8)
constexpr int B_LOADS = BN / ROWS_PER_LOAD / COPY_WAVES;  // and for B (8)
// The copy threads handle one tile row / one column each.
static_assert(BM == COPY_THREADS && BN == COPY_THREADS, "one copy thread per row and column");
constexpr int PLAN_THREADS = 1024;

// ---- workspace ------------------------------------------------------------------

// Device scratch of one launch, carved from the caller's workspace (256-byte aligned
// sections). ngrp = groups per batch row, n_mt_max = M-tiles if every group is active.
struct Work {
  int* meta;          // [0] active groups
  int* count;         // [B] active groups per batch row
  int* first;         // [B] index of its first active group in `list`
  uint8_t* flag;      // [B][ngrp] 1 = group has a nonzero mask entry
  int* list;          // [B*ngrp] active groups as b * ngrp + j, in (b, j) order
  float2* part;       // [n_mt_max][2][V] partial (max, argmax bits) of edge segments
  float* rowmask;     // [n_mt_max * 256] mask of each tile row, in list order (0 past S
                      // and past the last active group of the last tile)
  size_t total;
};

static Work carve(void* base, int64_t B, int64_t S, int64_t V) {
  const int64_t ngrp = cdiv(S, GROUP);
  const int64_t n_mt_max = cdiv(B * ngrp, NGRP);
  char* p = (char*)base;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += (size_t)round_up((int64_t)bytes, 256);
    return p != nullptr ? p + o : nullptr;
  };
  Work w;
  w.meta = (int*)take(16);
  w.count = (int*)take((size_t)B * 4);
  w.first = (int*)take((size_t)B * 4);
  w.flag = (uint8_t*)take((size_t)(B * ngrp));
  w.list = (int*)take((size_t)(B * ngrp) * 4);
  w.part = (float2*)take((size_t)(n_mt_max * 2 * V) * sizeof(float2));
  w.rowmask = (float*)take((size_t)(n_mt_max * 256) * sizeof(float));
  w.total = off;
  return w;
}

// ---- plan -------------------------------------------------------------------------

// Flags of the GROUP-position groups j .. j+3 that 64 consecutive positions (ballot
// `bal`, lane = position) cover: lane q < 4 gets group j + q's flag in *on; returns how
// many of them are active (the same in every lane).
__device__ __forceinline__ int group_flags(uint64_t bal, int j, int ngrp, int lane, bool* on) {
  static_assert(GROUP == 16, "four groups per 64-position ballot");
  int n = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) n += (j + q < ngrp && ((bal >> (16 * q)) & 0xffffull) != 0) ? 1 : 0;
  const int q = lane & 3;
  *on = lane < 4 && j + q < ngrp && ((bal >> (16 * q)) & 0xffffull) != 0;
  return n;
}

// Which groups of batch row b have a nonzero mask entry (one wave). Positions are read
// 8 x 64 at a time, all loads issued before the ballots.
__device__ __forceinline__ void plan_row(const void* __restrict__ mask, int mask_dtype, int b,
                                         int S, int ngrp, uint8_t* __restrict__ flag,
                                         int* __restrict__ count, int lane) {
  int n = 0;
  for (int t0 = 0; t0 < ngrp * GROUP; t0 += 8 * 64) {
    bool nz[8];
    int64_t off[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) off[u] = (int64_t)b * S + min(t0 + u * 64 + lane, S - 1);
    float mv[8];
    load_mask_n<8>(mask, mask_dtype, off, mv);
#pragma unroll
    for (int u = 0; u < 8; ++u) nz[u] = t0 + u * 64 + lane < S && mv[u] != 0.0f;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int j = (t0 + u * 64) / GROUP;
      if (j >= ngrp) break;
      bool on;
      n += group_flags(__ballot(nz[u]), j, ngrp, lane, &on);
      if (lane < 4 && j + lane < ngrp) flag[(int64_t)b * ngrp + j + lane] = (uint8_t)(on ? 1 : 0);
    }
  }
  if (lane == 0) count[b] = n;
}

// One wave per batch row.
__global__ __launch_bounds__(256) void fwd_plan_rows_kernel(const void* __restrict__ mask,
                                                            int mask_dtype, int B, int S, int ngrp,
                                                            uint8_t* __restrict__ flag,
                                                            int* __restrict__ count) {
  const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (b < B) plan_row(mask, mask_dtype, b, S, ngrp, flag, count, threadIdx.x & 63);
}

// Exclusive scan of the per-row counts, then the group list (one workgroup).
__device__ __forceinline__ void plan_list(int B, int ngrp, const uint8_t* __restrict__ flag,
                                          const int* __restrict__ count, int* __restrict__ first,
                                          int* __restrict__ list, int* __restrict__ meta) {
  __shared__ int wsum[PLAN_THREADS / 64];
  __shared__ int carry;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid == 0) carry = 0;
  __syncthreads();
  for (int b0 = 0; b0 < B; b0 += PLAN_THREADS) {
    const int b = b0 + tid;
    const int c = b < B ? count[b] : 0;
    int x = c;  // inclusive scan within the wave, then across waves
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(x, d);
      if (lane >= d) x += y;
    }
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    int before = carry;
    for (int w = 0; w < wave; ++w) before += wsum[w];
    const int start = before + x - c;
    if (b < B) first[b] = start;
    __syncthreads();
    if (tid == PLAN_THREADS - 1) carry = start + c;
    __syncthreads();
  }
  if (tid == 0) meta[0] = carry;
  // One wave per batch row: lane j takes group j (64 at a time); its slot is the row
  // start plus the active groups before it (a ballot prefix), so the list stays in
  // (b, j) order.
  const int nw = PLAN_THREADS / 64;
  for (int b = wave; b < B; b += nw) {
    int k = first[b];
    const uint8_t* f = flag + (int64_t)b * ngrp;
    for (int j0 = 0; j0 < ngrp; j0 += 64) {
      const int j = j0 + lane;
      const bool on = j < ngrp && f[j] != 0;
      const uint64_t bal = __ballot(on);
      if (on) list[k + __popcll(bal & ((1ull << lane) - 1ull))] = b * ngrp + j;
      k += __popcll(bal);
    }
  }
}

__global__ __launch_bounds__(PLAN_THREADS) void fwd_plan_list_kernel(
    int B, int ngrp, const uint8_t* __restrict__ flag, const int* __restrict__ count,
    int* __restrict__ first, int* __restrict__ list, int* __restrict__ meta) {
  plan_list(B, ngrp, flag, count, first, list, meta);
}

// Row mask in list order: tile row t = 16 e + r is position 16 j + r of batch row b,
// where list[e] = b * ngrp + j; rows of entries past the last active group are 0.
__device__ __forceinline__ void fill_rowmask(const void* __restrict__ mask, int mask_dtype, int S,
                                             int ngrp, int n_grp, const int* __restrict__ list,
                                             float* __restrict__ rowmask, int t) {
  const int e = t / GROUP;
  float v = 0.0f;
  if (e < n_grp) {
    const int code = list[e];
    const int b = code / ngrp;
    const int s = (code - b * ngrp) * GROUP + (t % GROUP);
    if (s < S) v = load_mask(mask, mask_dtype, (int64_t)b * S + s);
  }
  rowmask[t] = v;
}

__global__ __launch_bounds__(256) void fwd_plan_rowmask_kernel(
    const void* __restrict__ mask, int mask_dtype, int S, int ngrp, const int* __restrict__ meta,
    const int* __restrict__ list, float* __restrict__ rowmask) {
  const int n_grp = meta[0];
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t < (int64_t)(n_grp + NGRP - 1) / NGRP * BM)
    fill_rowmask(mask, mask_dtype, S, ngrp, n_grp, list, rowmask, (int)t);
}

// Both plan steps in one workgroup, for small batches (B * ngrp <= PLAN_FUSED_MAX):
// flags and counts stay in LDS, one launch instead of two.
constexpr int PLAN_FUSED_MAX = 1 << 14;  // groups (B * ngrp); also bounds B
__global__ __launch_bounds__(PLAN_THREADS) void fwd_plan_small_kernel(
    const void* __restrict__ mask, int mask_dtype, int B, int S, int ngrp, int* __restrict__ count,
    int* __restrict__ first, int* __restrict__ list, int* __restrict__ meta,
    float* __restrict__ rowmask) {
  __shared__ uint8_t fl[PLAN_FUSED_MAX];
  __shared__ int cnt[PLAN_FUSED_MAX];
  __shared__ int lst[PLAN_FUSED_MAX];  // the list, also kept here for the row mask
  __shared__ int wsum[PLAN_THREADS / 64];
  __shared__ int carry;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int NW = PLAN_THREADS / 64;
  for (int b = wave; b < B; b += NW) {
    int n = 0;
    for (int t0 = 0; t0 < ngrp * GROUP; t0 += 8 * 64) {
      bool nz[8];
      int64_t off[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) off[u] = (int64_t)b * S + min(t0 + u * 64 + lane, S - 1);
      float mv[8];
      load_mask_n<8>(mask, mask_dtype, off, mv);
#pragma unroll
      for (int u = 0; u < 8; ++u) nz[u] = t0 + u * 64 + lane < S && mv[u] != 0.0f;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int j = (t0 + u * 64) / GROUP;
        if (j >= ngrp) break;
        bool on;
        n += group_flags(__ballot(nz[u]), j, ngrp, lane, &on);
        if (lane < 4 && j + lane < ngrp) fl[b * ngrp + j + lane] = (uint8_t)(on ? 1 : 0);
      }
    }
    if (lane == 0) cnt[b] = n;
  }
  if (tid == 0) carry = 0;
  __syncthreads();
  for (int b0 = 0; b0 < B; b0 += PLAN_THREADS) {
    const int b = b0 + tid;
    const int c = b < B ? cnt[b] : 0;
    int x = c;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(x, d);
      if (lane >= d) x += y;
    }
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    int before = carry;
    for (int w = 0; w < wave; ++w) before += wsum[w];
    const int start = before + x - c;
    if (b < B) {
      first[b] = start;
      count[b] = c;
      cnt[b] = start;  // from here on: the row's first slot
    }
    __syncthreads();
    if (tid == PLAN_THREADS - 1) carry = start + c;
    __syncthreads();
  }
  if (tid == 0) meta[0] = carry;
  for (int b = wave; b < B; b += NW) {
    int k = cnt[b];
    for (int j0 = 0; j0 < ngrp; j0 += 64) {
      const int j = j0 + lane;
      const bool on = j < ngrp && fl[b * ngrp + j] != 0;
      const uint64_t bal = __ballot(on);
      if (on) {
        const int e = k + __popcll(bal & ((1ull << lane) - 1ull));
        list[e] = b * ngrp + j;
        lst[e] = b * ngrp + j;
      }
      k += __popcll(bal);
    }
  }
  __syncthreads();  // lst is complete
  // Row mask in list order, RM rows per thread with their mask loads in flight together.
  constexpr int RM = 8;
  const int n_grp = carry;
  const int n_rows = (n_grp + NGRP - 1) / NGRP * BM;
  for (int t0 = tid; t0 < n_rows; t0 += RM * PLAN_THREADS) {
    int64_t off[RM];
    bool ok[RM];
#pragma unroll
    for (int u = 0; u < RM; ++u) {
      const int t = t0 + u * PLAN_THREADS, e = t / GROUP;
      const int code = (t < n_rows && e < n_grp) ? lst[e] : -1;
      const int bb = code >= 0 ? code / ngrp : 0;
      const int ss = code >= 0 ? (code - bb * ngrp) * GROUP + (t % GROUP) : S;
      ok[u] = ss < S;
      off[u] = ok[u] ? (int64_t)bb * S + ss : 0;
    }
    float mv[RM];
    load_mask_n<RM>(mask, mask_dtype, off, mv);
#pragma unroll
    for (int u = 0; u < RM; ++u) {
      const int t = t0 + u * PLAN_THREADS;
      if (t < n_rows) rowmask[t] = ok[u] ? mv[u] : 0.0f;
    }
  }
}

// The whole plan in one workgroup with every mask value staged in LDS, for
// B * S <= PLAN_TINY_POS and B * ngrp <= PLAN_THREADS: one batch of mask loads, one
// prefix scan over the groups (thread g = group g, in (b, j) order), and the row mask
// filled from LDS.
constexpr int PLAN_TINY_POS = 1 << 14;  // positions (B * S)
__global__ __launch_bounds__(PLAN_THREADS) void fwd_plan_tiny_kernel(
    const void* __restrict__ mask, int mask_dtype, int B, int S, int ngrp, int* __restrict__ count,
    int* __restrict__ first, int* __restrict__ list, int* __restrict__ meta,
    float* __restrict__ rowmask) {
  __shared__ float mv[PLAN_TINY_POS];
  __shared__ int lst[PLAN_THREADS];          // the list
  __shared__ int slot_of[PLAN_THREADS + 1];  // list slot of group g (active or not); [n_g] = total
  __shared__ int wsum[PLAN_THREADS / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n_pos = B * S, n_g = B * ngrp;
  constexpr int PER = PLAN_TINY_POS / PLAN_THREADS;
  if (n_pos > 0) {
    int64_t off[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) off[u] = min(tid + u * PLAN_THREADS, n_pos - 1);
    float v[PER];
    load_mask_n<PER>(mask, mask_dtype, off, v);
#pragma unroll
    for (int u = 0; u < PER; ++u)
      if (tid + u * PLAN_THREADS < n_pos) mv[tid + u * PLAN_THREADS] = v[u];
  }
  __syncthreads();
  bool on = false;
  if (tid < n_g) {
    const int b = tid / ngrp, j = tid - b * ngrp;
    const int s1 = min(S, (j + 1) * GROUP);
    for (int s = j * GROUP; s < s1; ++s) on |= mv[b * S + s] != 0.0f;
  }
  const uint64_t bal = __ballot(on);
  if (lane == 0) wsum[wave] = __popcll(bal);
  __syncthreads();
  int before = 0, total = 0;
#pragma unroll
  for (int w = 0; w < PLAN_THREADS / 64; ++w) {
    before += w < wave ? wsum[w] : 0;
    total += wsum[w];
  }
  const int slot = before + __popcll(bal & ((1ull << lane) - 1ull));
  if (tid < n_g) slot_of[tid] = slot;
  if (on) {
    list[slot] = tid;  // b * ngrp + j
    lst[slot] = tid;
  }
  if (tid == 0) {
    slot_of[n_g] = total;
    meta[0] = total;
  }
  __syncthreads();
  for (int b = tid; b < B; b += PLAN_THREADS) {
    const int f = slot_of[b * ngrp];
    first[b] = f;
    count[b] = slot_of[(b + 1) * ngrp] - f;
  }
  const int n_rows = (total + NGRP - 1) / NGRP * BM;
  for (int t = tid; t < n_rows; t += PLAN_THREADS) {
    const int e = t / GROUP;
    float v = 0.0f;
    if (e < total) {
      const int code = lst[e], b = code / ngrp;
      const int s = (code - b * ngrp) * GROUP + t % GROUP;
      if (s < S) v = mv[b * S + s];
    }
    rowmask[t] = v;
  }
}

// ---- main kernel ------------------------------------------------------------------

// Metadata of one unit, double-buffered: the next unit's copy is filled while the
// current unit computes. 16-byte aligned: the epilogue reads the mask 4 rows at a time.
struct __align__(16) UnitMeta {
  float maskf[BM];           // mask of the tile's rows (0 past S or past the last block)
  int maskw[BM];             // the same as an AND mask for 0/1 masks: ~31 (kept) or 0
  int grp_b[NGRP + 2];       // batch row of each group; [NGRP], [NGRP+1]: rows of the
                             // groups just before / after the tile (-1 if none)
  int grp_s[NGRP];           // first position of each group (16 j)
  int mask_binary;           // every maskf value is 0 or 1
  float bias[BN];            // bias of the tile's columns (0 past V or without bias)
};

struct Smem {
  u32x4 a[2][BM * CHUNKS];   // [stage][row * 8 + (chunk ^ f(row))]
  u32x4 b[2][BN * CHUNKS];
  int key[NGRP][BN];         // per group, per column: the epilogue key of the group's
                             // maximum (value and row); a value that is not positive (0,
                             // negative or NaN) never wins the merge
  UnitMeta um[2];
};

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ int swz_key(int row) { return (row & 7) ^ ((row >> 3) & 1); }

// Byte offset, within a 128-byte row slab, of the 16-byte chunk that lane L copies in
// a wave-wide load of tile row `row` (= 8g + L/8): physical chunk L%8 holds logical
// chunk (L%8) ^ f(row), so the lane reads that logical chunk from global memory.
__device__ __forceinline__ uint32_t lane_chunk(int row, int lane) {
  return (uint32_t)(((lane & 7) ^ swz_key(row)) * 16);
}

// One MFMA "step" consumes 16 bytes of A and B per lane.
template <typename T> struct Mfma;
template <> struct Mfma<bf16> {
  static constexpr int kInsts = 1;
  static __device__ __forceinline__ void run(const u32x4& a, const u32x4& b, f32x16& c) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ void run_from(const u32x4& a, const u32x4& b, const f32x16& c,
                                                  f32x16& d) {
    d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma<f16> {
  static constexpr int kInsts = 1;
  static __device__ __forceinline__ void run(const u32x4& a, const u32x4& b, f32x16& c) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                               __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ void run_from(const u32x4& a, const u32x4& b, const f32x16& c,
                                                  f32x16& d) {
    d = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                               __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma<float> {
  static constexpr int kInsts = 4;
  // 4 floats per lane = four K=2 steps. Lane half h supplies k = 16h + 4p + j for
  // A and B alike, so every k of the slab is paired once. __uint_as_float takes the
  // element value: a bit_cast of a vector-element lvalue reads element 0 every time.
  static __device__ __forceinline__ void run(const u32x4& a, const u32x4& b, f32x16& c) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a[j]), __uint_as_float(b[j]), c,
                                               0, 0, 0);
  }
  static __device__ __forceinline__ void run_from(const u32x4& a, const u32x4& b, const f32x16& c,
                                                  f32x16& d) {
    d = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a[0]), __uint_as_float(b[0]), c, 0, 0, 0);
#pragma unroll
    for (int j = 1; j < 4; ++j)
      d = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a[j]), __uint_as_float(b[j]), d,
                                               0, 0, 0);
  }
};

// fp32 as two bf16 ("split" mode, torch's 'high' float32 matmul precision): x = hi + lo + r
// with hi = bf16(x) and lo = bf16(x - hi) (both round to nearest even; x - hi is exact), so
// |r| <= 2^-16 |x|. A product is taken as hi_a hi_b + hi_a lo_b + lo_a hi_b: the dropped
// lo_a lo_b and the residuals keep it within 3 * 2^-16 relative of the exact one.
// Non-finite values: x - hi is finite whenever hi is, and NaN or infinite when x is infinite
// or NaN (or a finite x rounds to an infinite bf16). Such a pair moves its values into the lo
// slot (hi = 0, lo = bf16(x)), so that of the three products only lo_a hi_b or hi_a lo_b sees
// the infinity: an infinite operand times a finite partner gives the exact product's
// infinity (or NaN where the partner's bf16 part is 0, as inf * 0 is), instead of adding
// inf - inf across the terms. Both operands infinite at the same k give 0 * inf = NaN where
// the exact product is infinite. A pair's two k belong to one dot product, which is infinite
// or NaN either way, so the finite neighbour of an infinite value may lose its lo part.
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(2))) float f32x2;
__device__ __forceinline__ void split_pair(float x0, float x1, uint32_t& hi, uint32_t& lo) {
  const f32x2 v = {x0, x1};
  hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  const f32x2 hf = {__uint_as_float(hi << 16), __uint_as_float(hi & 0xffff0000u)};
  const f32x2 d = v - hf;
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(d, bf16x2));
  if (!__builtin_isfinite(d.x + d.y)) {
    lo = hi;
    hi = 0u;
  }
}
// Eight floats (x0: k = 0..3, x1: k = 4..7) as bf16x8 hi and lo parts in k order.
__device__ __forceinline__ void split8(const u32x4& x0, const u32x4& x1, u32x4& hi, u32x4& lo) {
  uint32_t h0, h1, h2, h3, l0, l1, l2, l3;
  split_pair(__uint_as_float(x0[0]), __uint_as_float(x0[1]), h0, l0);
  split_pair(__uint_as_float(x0[2]), __uint_as_float(x0[3]), h1, l1);
  split_pair(__uint_as_float(x1[0]), __uint_as_float(x1[1]), h2, l2);
  split_pair(__uint_as_float(x1[2]), __uint_as_float(x1[3]), h3, l3);
  hi = u32x4{h0, h1, h2, h3};
  lo = u32x4{l0, l1, l2, l3};
}
// acc += a b over 16 k (8 per lane half), both as hi + lo: the two small terms first.
__device__ __forceinline__ void mfma_split(const u32x4& ahi, const u32x4& alo, const u32x4& bhi,
                                           const u32x4& blo, f32x16& c) {
  c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, alo),
                                               __builtin_bit_cast(bf16x8, bhi), c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ahi),
                                               __builtin_bit_cast(bf16x8, blo), c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ahi),
                                               __builtin_bit_cast(bf16x8, bhi), c, 0, 0, 0);
}

// ---- unit schedule ----
//
// The grid is persistent (about one workgroup per CU); the units (M-tile, vocab tile)
// are dealt out in rounds of gridDim.x. Workgroups are dispatched round-robin over the
// 8 XCDs, so in each round the workgroups of one XCD (w % 8 equal) take a contiguous
// range of unit numbers; unit numbers walk groups of GROUP_V vocab tiles x all M-tiles
// (vocab tile fastest), so the units running together on one XCD share a few decoder
// tiles and a few M-tiles' rows in its L2. In the last, partial round the ranges
// shrink evenly and workgroups past them stop.
constexpr int GROUP_V = 4;

// Unit number of workgroup w in round r, or -1 when it has none (it is done).
__device__ __forceinline__ int unit_at(int w, int r, int G, int n_units) {
  const int base = r * G;
  const int R = min(G, n_units - base);
  if (R <= 0) return -1;
  const int x = w & 7, local = w >> 3, q = R >> 3, rr = R & 7;
  if (local >= q + (x < rr ? 1 : 0)) return -1;
  return base + (x < rr ? x * (q + 1) : rr * (q + 1) + (x - rr) * q) + local;
}

__device__ __forceinline__ void unit_tile(int u, int n_mt, int n_vt, int* m, int* vt) {
  const int per_group = GROUP_V * n_mt;
  const int group = u / per_group;
  const int rem = u - group * per_group;
  const int gv = min(GROUP_V, n_vt - group * GROUP_V);
  const int mm = rem / gv;
  *m = mm;
  *vt = group * GROUP_V + rem - mm * gv;
}

// Launch-wide, wave-uniform parameters.
template <typename T>
struct Args {
  const char* H;      // H[0, 0, :]
  const char* W;
  const T* bias;
  const float* rowmask;  // [n_mt * BM] mask of each tile row
  const int* list;
  int n_grp;          // active groups
  int ngrp;           // groups per batch row
  int S;
  int row_bytes;      // D * sizeof(T)
  int nk_full;        // slabs lying entirely inside the row
  int nk;             // slabs per unit
  int V;
};

// One unit as the copy waves see it.
struct CopyUnit {
  int m, v0, n_valid;
  uint32_t a_off[A_LOADS];  // byte offset from H of the lane's A row and chunk, per copy
};

// ---- unit metadata (run by the copy threads, ct = 0..255; the ones named take part) ----

// Copy threads 0..NGRP+1: the tile's list entry (b * ngrp + j), or -1; threads NGRP
// and NGRP+1 take the entries just before and after the tile.
__device__ __forceinline__ int group_entry(int m, int ct) {
  return ct < NGRP ? m * NGRP + ct : (ct == NGRP ? m * NGRP - 1 : m * NGRP + NGRP);
}
__device__ __forceinline__ int group_code(const int* list, int n_grp, int m, int n_valid, int ct) {
  const int e = group_entry(m, ct);
  const bool ok = e >= 0 && e < n_grp && (ct >= NGRP || ct < n_valid);
  return ok ? list[e] : -1;
}

__device__ __forceinline__ void put_groups(UnitMeta& um, int code, int ngrp, int ct) {
  if (ct < NGRP + 2) {
    um.grp_b[ct] = code >= 0 ? code / ngrp : -1;
    if (ct < NGRP) um.grp_s[ct] = code >= 0 ? (code % ngrp) * GROUP : 0;
  }
}

// Given the mask value of tile row ct: the AND word, and clear mask_binary (set to 1
// before a barrier) on any value other than 0 / 1.
__device__ __forceinline__ void put_mask_words(UnitMeta& um, float mv, int ct, int lane) {
  um.maskw[ct] = mv != 0.0f ? ~31 : 0;
  if (__ballot(mv != 0.0f && mv != 1.0f) != 0 && lane == 0) um.mask_binary = 0;
}

// Per copy lane (after put_groups is visible): the byte offsets of its A rows. Rows of
// groups past n_valid get some valid row (their copies are skipped); positions past S
// any valid position of the row.
__device__ __forceinline__ void row_offsets(const UnitMeta& um, int n_valid, int S, int row_bytes,
                                            int c, int lane, uint32_t* a_off) {
#pragma unroll
  for (int i = 0; i < A_LOADS; ++i) {
    const int grp = i * COPY_WAVES + c;
    const int row = grp * ROWS_PER_LOAD + (lane >> 3);
    const int g = min(row / GROUP, n_valid - 1);
    const int s = min(um.grp_s[g] + row % GROUP, S - 1);
    a_off[i] = (uint32_t)(((int64_t)um.grp_b[g] * S + s) * row_bytes) + lane_chunk(row, lane);
  }
}

// Raw loads for the in-loop prefetch: the bits are loaded without any conversion or
// select, and converted two K steps later, after the steps' drains.
template <typename T> __device__ __forceinline__ uint32_t load_bits(const T* p, int64_t i);
template <> __device__ __forceinline__ uint32_t load_bits(const bf16* p, int64_t i) {
  return ((const uint16_t*)p)[i];
}
template <> __device__ __forceinline__ uint32_t load_bits(const f16* p, int64_t i) {
  return ((const uint16_t*)p)[i];
}
template <> __device__ __forceinline__ uint32_t load_bits(const float* p, int64_t i) {
  return ((const uint32_t*)p)[i];
}
template <typename T> __device__ __forceinline__ float bits_to_f32(uint32_t x);
template <> __device__ __forceinline__ float bits_to_f32<bf16>(uint32_t x) { return __uint_as_float(x << 16); }
template <> __device__ __forceinline__ float bits_to_f32<f16>(uint32_t x) {
  return (float)__builtin_bit_cast(f16, (uint16_t)x);
}
template <> __device__ __forceinline__ float bits_to_f32<float>(uint32_t x) { return __uint_as_float(x); }

// ---- K stream ----

// Issue the direct global -> LDS copies of K slab k of a unit into stage buf. Copy
// wave c, copy i covers the 8-row group g = i * COPY_WAVES + c (rows 8g..8g+7 of the
// tile, in group g / 2); lane L lands at LDS chunk g*64 + L. A chunk past the row end
// (tail or padding slabs) re-reads the row's first chunk -- valid, finite data inside
// the row, so nothing outside H or W is read -- and its W copy is zeroed by zero_tail()
// before use (a zero W times a finite H adds exactly 0). W rows past V re-read row V-1
// (never stored). Rows of groups past the last active one (n_valid) re-read a row of the
// last active group (their keys are never used), so every copy is issued unconditionally.
template <typename T, bool TAIL>
__device__ __forceinline__ void issue_slab_k(Smem& sm, const Args<T>& a, const CopyUnit& cu, int k,
                                             int buf, int c, int lane) {
  const uint32_t kb = (uint32_t)k * SLAB;
#pragma unroll
  for (int i = 0; i < A_LOADS; ++i) {
    const int grp = i * COPY_WAVES + c;
    const uint32_t c16 = lane_chunk(grp * ROWS_PER_LOAD + (lane >> 3), lane);
    // a_off includes c16: adding 0 - c16 (mod 2^32) lands on the row's first chunk.
    const uint32_t step = (!TAIL || kb + c16 < (uint32_t)a.row_bytes) ? kb : 0u - c16;
    __builtin_amdgcn_global_load_lds((const void*)(a.H + (cu.a_off[i] + step)),
                                     (lds_void*)&sm.a[buf][grp * 64], 16, 0, 0);
  }
  const char* bb = a.W + (int64_t)cu.v0 * a.row_bytes;
  const int b_last = a.V - 1 - cu.v0;
#pragma unroll
  for (int i = 0; i < B_LOADS; ++i) {
    const int grp = i * COPY_WAVES + c;
    const int row = grp * ROWS_PER_LOAD + (lane >> 3);
    const uint32_t c16 = lane_chunk(row, lane);
    const uint32_t step = (!TAIL || kb + c16 < (uint32_t)a.row_bytes) ? kb : 0u - c16;
    const uint32_t off = (uint32_t)min(row, b_last) * (uint32_t)a.row_bytes + c16 + step;
    __builtin_amdgcn_global_load_lds((const void*)(bb + off), (lds_void*)&sm.b[buf][grp * 64], 16, 0, 0);
  }
}
template <typename T>
__device__ __forceinline__ void issue_slab(Smem& sm, const Args<T>& a, const CopyUnit& cu, int k,
                                           int buf, int c, int lane) {
  if (k >= a.nk_full) issue_slab_k<T, true>(sm, a, cu, k, buf, c, lane);
  else issue_slab_k<T, false>(sm, a, cu, k, buf, c, lane);
}

// Zero the W chunks of slab k (in stage buf) that lie past D; each copy wave clears the
// chunks it copied itself, after its copies landed and before the step's barrier.
__device__ __forceinline__ void zero_tail(Smem& sm, int row_bytes, int k, int buf, int c, int lane) {
  const uint32_t kb = (uint32_t)k * SLAB;
#pragma unroll
  for (int i = 0; i < B_LOADS; ++i) {
    const int grp = i * COPY_WAVES + c;
    if (kb + lane_chunk(grp * ROWS_PER_LOAD + (lane >> 3), lane) >= (uint32_t)row_bytes)
      sm.b[buf][grp * 64 + lane] = u32x4{0, 0, 0, 0};
  }
}

// Workgroup barrier once this wave's LDS operations are complete; its global loads
// (direct-to-LDS copies included) may still be in flight. (__syncthreads() would also
// wait for every outstanding direct-to-LDS copy.) The memory clobber keeps the compiler
// from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Wait for all of this wave's memory operations (copies, loads, stores).
__device__ __forceinline__ void wait_all() {
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
}


// ---- the workgroup's unit sequence ----
//
// Both roles walk the same sequence and pass the same barriers:
//   start of the first unit, and of every unit when the metadata is not prefetched
//   (nk < PREFETCH_MIN_NK): 2 barriers;
//   each K step k = 0..nk-1: 1 barrier (B_k); after the epilogue: 1 barrier (E).
// Slab j of a unit lives in stage buf ^ (j & 1), where buf is the unit's first stage.
// The copy waves issue slab k+1 at the start of step k (k >= 1; slab 1 is issued before
// step 0), into the stage that slab k-1 left at B_(k-1), and wait for it before B_k.
// With prefetch the next unit's slab 0 is issued at step nk-1 and its slab 1 after
// B_(nk-1). Its metadata is loaded into registers one unit ahead (with the unit's slab 1)
// and written to the metadata buffer at steps 2 and 3: step 1 writes the previous unit's
// results, which read that buffer.
constexpr int PREFETCH_MIN_NK = 5;

struct Unit {
  int u, m, v0, n_valid;
};
__device__ __forceinline__ Unit unit_of(int w, int r, int G, int n_units, int n_mt, int n_vt,
                                        int n_grp) {
  Unit x;
  x.u = unit_at(w, r, G, n_units);
  x.m = 0;
  x.v0 = 0;
  x.n_valid = 0;
  if (x.u >= 0) {
    int vt;
    unit_tile(x.u, n_mt, n_vt, &x.m, &vt);
    x.v0 = vt * BN;
    x.n_valid = min(NGRP, n_grp - x.m * NGRP);
  }
  return x;
}

// ---- copy waves ----

// Merge the groups of each batch-row segment of the tile (copy thread = column) and
// write reps/argmax for complete segments, or the partial for a segment that continues
// into the previous M-tile (slot 0) or the next one (slot 1). A group's key holds its
// maximum x (5 low mantissa bits cleared) and its row r in the 32-row block (as
// 31 - r); the row's position is the group's first position plus r mod 16.
// The segment boundaries are wave-uniform: lane g of every copy wave compares group g's
// batch row with group g+1's, and one ballot gives the bitmask of segment ends (lanes
// NGRP, NGRP + 1 hold the rows of the groups just before and after the tile). The merge
// is unrolled with scalar branches and keeps, per column, the best value and the group
// and row that hold it; a segment end reads that group's first position (one LDS read),
// so no LDS read waits inside the per-group merge.
template <typename T>
__device__ __forceinline__ void write_unit(const Smem& sm, const UnitMeta& um, int m, int v0, int V,
                                           int n_valid, int ct, T* reps, int32_t* argmax,
                                           float* reps_f32, float2* part) {
  const int lane = ct & 63;
  const int gbv = um.grp_b[min(lane, NGRP + 1)];
  const int gbn = um.grp_b[min(lane + 1, NGRP + 1)];
  const uint64_t ends = __ballot(lane < n_valid && (lane + 1 == n_valid || gbn != gbv));
  const int b_prev = __builtin_amdgcn_readlane(gbv, NGRP);
  const int b_next = __builtin_amdgcn_readlane(gbv, NGRP + 1);
  const int b_first = __builtin_amdgcn_readlane(gbv, 0);
  const bool live = v0 + ct < V;
  const int v = min(v0 + ct, V - 1);
  int kr[NGRP];
#pragma unroll
  for (int g = 0; g < NGRP; ++g) kr[g] = sm.key[g][ct];  // all loads first (groups past n_valid are unused)
  float bv = 0.0f;
  int bk = 0;  // (group << 5) | (31 - row in the 32-row block) of the best value
  // A rolled loop (kr indexed through M0): unrolled, the copy path's registers and SGPR
  // spills outgrow the kernel's 168-VGPR budget.
#pragma unroll 1
  for (int g = 0; g < n_valid; ++g) {  // uniform
    {
      const int key = kr[g];
      const float x = __int_as_float(key & ~31);
      const bool gt = x > bv;  // earlier groups hold lower s: strict '>' keeps them on ties
      bv = gt ? x : bv;
      bk = gt ? ((g << 5) | (key & 31)) : bk;
      if ((ends >> g) & 1) {  // uniform: the segment of batch row b ends
        const int b = __builtin_amdgcn_readlane(gbv, g);
        const bool cont_prev = b == b_first && b == b_prev;
        const bool cont_next = g + 1 == n_valid && b == b_next;
        // the best row's position (0 when no value is positive)
        const int bi = bv > 0.0f ? um.grp_s[bk >> 5] + ((31 - (bk & 31)) & (GROUP - 1)) : 0;
        if (live) {
          if (cont_prev || cont_next) {
            part[((int64_t)m * 2 + (cont_prev ? 0 : 1)) * V + v] = make_float2(bv, __int_as_float(bi));
          } else {
            const int64_t o = (int64_t)b * V + v;
            const float rv = log1p_pos(bv);
            reps[o] = from_f32<T>(rv);
            if (argmax != nullptr) argmax[o] = bi;
            if (reps_f32 != nullptr) reps_f32[o] = rv;
          }
        }
        bv = 0.0f;
        bk = 0;
      }
    }
  }
}

template <typename T>
struct Outputs {
  T* reps;
  int32_t* argmax;
  float* reps_f32;
  float2* part;
};

// Start a unit without prefetch: fetch its metadata into um, write the previous unit's
// results (prev.u >= 0, metadata in um_prev), and land its first two slabs. Two barriers.
template <typename T>
__device__ __forceinline__ void copy_start(Smem& sm, const Args<T>& a, const Outputs<T>& o,
                                           UnitMeta& um, CopyUnit& cu, int buf,
                                           const Unit& prev, const UnitMeta& um_prev, int ct,
                                           int c, int lane) {
  const int code = ct < NGRP + 2 ? group_code(a.list, a.n_grp, cu.m, cu.n_valid, ct) : -1;
  const float mv = a.rowmask[(int64_t)cu.m * BM + ct];
  const int col = cu.v0 + ct;
  const float bv = (a.bias != nullptr && col < a.V) ? to_f32(a.bias[col]) : 0.0f;
  put_groups(um, code, a.ngrp, ct);
  um.maskf[ct] = mv;
  um.bias[ct] = bv;
  if (ct == 0) um.mask_binary = 1;
  lds_barrier();  // S1
  row_offsets(um, cu.n_valid, a.S, a.row_bytes, c, lane, cu.a_off);
  if (a.nk > 0) {
    issue_slab(sm, a, cu, 0, buf, c, lane);
    issue_slab(sm, a, cu, 1, buf ^ 1, c, lane);
  }
  put_mask_words(um, mv, ct, lane);
  if (prev.u >= 0)
    write_unit<T>(sm, um_prev, prev.m, prev.v0, a.V, prev.n_valid, ct, o.reps, o.argmax,
                  o.reps_f32, o.part);
  wait_all();
  if (a.nk > 0) {
    if (0 >= a.nk_full) zero_tail(sm, a.row_bytes, 0, buf, c, lane);
    if (1 >= a.nk_full) zero_tail(sm, a.row_bytes, 1, buf ^ 1, c, lane);
  }
  lds_barrier();  // S2
}

template <typename T>
__device__ void copy_path(Smem& sm, const Args<T>& a, const Outputs<T>& o, int w, int G,
                          int n_units, int n_mt, int n_vt, int ct, int c, int lane) {
  const int nk = a.nk;
  Unit cur = unit_of(w, 0, G, n_units, n_mt, n_vt, a.n_grp);
  if (cur.u < 0) return;
  Unit prev;
  prev.u = -1;
  int par = 0, buf = 0;
  CopyUnit cu;
  cu.m = cur.m;
  cu.v0 = cur.v0;
  cu.n_valid = cur.n_valid;
  copy_start(sm, a, o, sm.um[0], cu, buf, prev, sm.um[1], ct, c, lane);

  // The metadata of a prefetched unit (this copy thread's mask row, group-list entry and
  // bias bits) is loaded into registers one unit ahead, with the unit's slab 1 (before E),
  // so step 0's wait covers it; steps 2 and 3 write it to the metadata buffer.
  struct MetaRegs {
    float mv;
    int code;
    uint32_t bias;
  };
  auto load_meta = [&](const Unit& x) {
    MetaRegs mr{0.0f, 0, 0u};
    if (x.u >= 0 && nk >= PREFETCH_MIN_NK) {
      mr.mv = a.rowmask[(int64_t)x.m * BM + ct];
      mr.code = a.list[min(max(group_entry(x.m, min(ct, NGRP + 1)), 0), a.n_grp - 1)];
      if (a.bias != nullptr) mr.bias = load_bits(a.bias + min(x.v0 + ct, a.V - 1), 0);
    }
    return mr;
  };
  Unit next = unit_of(w, 1, G, n_units, n_mt, n_vt, a.n_grp);
  MetaRegs meta = load_meta(next);
  for (int r = 1;; ++r) {
    const bool pre = next.u >= 0 && nk >= PREFETCH_MIN_NK;
    UnitMeta& um_next = sm.um[par ^ 1];
    const int buf_next = buf ^ (nk & 1);
    CopyUnit nx;
    nx.m = next.m;
    nx.v0 = next.v0;
    nx.n_valid = next.n_valid;
    for (int k = 0; k < nk; ++k) {
      if (k >= 1) {
        if (k + 1 < nk)
          issue_slab(sm, a, cu, k + 1, buf ^ ((k + 1) & 1), c, lane);
        else if (pre)
          issue_slab(sm, a, nx, 0, buf_next, c, lane);
      }
      if (pre) {
        if (k == 1) {
          if (ct == 0) um_next.mask_binary = 1;  // cleared at step 2 by any other value
        } else if (k == 2) {
          const int e = group_entry(nx.m, ct);
          const bool ok = e >= 0 && e < a.n_grp && (ct >= NGRP || ct < nx.n_valid);
          put_groups(um_next, ok ? meta.code : -1, a.ngrp, ct);
          um_next.maskf[ct] = meta.mv;
          put_mask_words(um_next, meta.mv, ct, lane);
          const int col = nx.v0 + ct;
          um_next.bias[ct] = (a.bias != nullptr && col < a.V) ? bits_to_f32<T>(meta.bias) : 0.0f;
        } else if (k == 3) {
          row_offsets(um_next, nx.n_valid, a.S, a.row_bytes, c, lane, nx.a_off);
        }
      }
      if (k == 1 && prev.u >= 0) {
        write_unit<T>(sm, um_next, prev.m, prev.v0, a.V, prev.n_valid, ct, o.reps, o.argmax,
                      o.reps_f32, o.part);
        prev.u = -1;
      }
      wait_all();
      if (k + 1 < nk) {
        if (k + 1 >= a.nk_full) zero_tail(sm, a.row_bytes, k + 1, buf ^ ((k + 1) & 1), c, lane);
      } else if (pre && 0 >= a.nk_full) {
        zero_tail(sm, a.row_bytes, 0, buf_next, c, lane);
      }
      lds_barrier();  // B_k
    }
    if (pre) issue_slab(sm, a, nx, 1, buf_next ^ 1, c, lane);
    // the unit after next, worked out while the compute waves run their epilogue, and its
    // metadata loads
    const Unit next2 = next.u >= 0 ? unit_of(w, r + 1, G, n_units, n_mt, n_vt, a.n_grp) : next;
    if (pre) meta = load_meta(next2);
    lds_barrier();  // E: the compute waves' keys are written
    if (next.u < 0) {
      write_unit<T>(sm, sm.um[par], cur.m, cur.v0, a.V, cur.n_valid, ct, o.reps, o.argmax,
                    o.reps_f32, o.part);
      return;
    }
    if (pre) {
      prev = cur;  // written during the next unit's step 1
    } else {
      copy_start(sm, a, o, um_next, nx, buf_next, cur, sm.um[par], ct, c, lane);
    }
    cur = next;
    cu = nx;
    next = next2;
    par ^= 1;
    buf = buf_next;
  }
}

// ---- compute waves ----

// Mainloop + block epilogue of one unit for a compute wave with JM blocks (JM = 0: the
// wave only keeps the barrier schedule). Stage buf holds the unit's slab 0.
template <typename T, int JM>
__device__ __forceinline__ void compute_unit(Smem& sm, const UnitMeta& um, int nk, int buf,
                                             int lane, int wm, int wn) {
  constexpr int JA = JM > 0 ? JM : 1;
  const int l32 = lane & 31, h = lane >> 5;
  // Accumulators start at the bias of their column. Only the last block's are set here: the
  // unit's first MFMA of every other block takes them as its C operand, so each block still
  // sums bias + products in the same order, with 32 register moves instead of 16 JA.
  f32x16 acc[JA][NB_PER_WAVE];
#pragma unroll
  for (int nb = 0; nb < NB_PER_WAVE; ++nb) {
    const float bv = um.bias[wn * 64 + nb * 32 + l32];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[JA - 1][nb][i] = bv;
    if (nk == 0) {  // no MFMAs: x = bias
#pragma unroll
      for (int j = 0; j < JA - 1; ++j) acc[j][nb] = acc[JA - 1][nb];
    }
  }

  // Every operand row is (multiple of 32) + l32, so its swizzle key is key(l32): a
  // fragment's LDS index is a per-lane offset plus a compile-time row offset.
  const u32x4* abase = sm.a[0] + (wm * 32) * CHUNKS;
  const u32x4* bbase = sm.b[0] + (wn * 64) * CHUNKS;
  constexpr int A_STAGE = BM * CHUNKS, B_STAGE = BN * CHUNKS;
  const int kx = swz_key(l32), off0 = l32 * CHUNKS;
  auto chunk = [&](int p) { return off0 + ((h * (CHUNKS / 2) + p) ^ kx); };  // lane half h: K chunks 4h..4h+3
  // One buffer of operand fragments (the 168-VGPR budget holds the 128 accumulator
  // registers and 24 more): each fragment for the next K step is read right after the
  // last MFMA that uses it. MFMAs run B-fragment-major, so B fragment 0 frees first,
  // then A fragments 0..JM-1, then B fragment 1.
  u32x4 bf[NB_PER_WAVE], af[JA];
  // MFMAs of the fragments at hand; rolling reads of K step p of stage st. With `first`
  // (the unit's first K step), blocks 0..JM-2 start from block JM-1's bias registers, which
  // block JM-1 itself overwrites only after them.
  auto step_x = [&](int st, int p, auto first) {
    const u32x4* an = abase + st * A_STAGE;
    const u32x4* bn = bbase + st * B_STAGE;
    const int cn = chunk(p);
#pragma unroll
    for (int j = 0; j < JM; ++j) {
      if (decltype(first)::value && j < JM - 1) Mfma<T>::run_from(af[j], bf[0], acc[JM - 1][0], acc[j][0]);
      else Mfma<T>::run(af[j], bf[0], acc[j][0]);
    }
    bf[0] = bn[cn];
#pragma unroll
    for (int j = 0; j < JM; ++j) {
      if (decltype(first)::value && j < JM - 1) Mfma<T>::run_from(af[j], bf[1], acc[JM - 1][1], acc[j][1]);
      else Mfma<T>::run(af[j], bf[1], acc[j][1]);
      af[j] = an[j * WAVES_M * 32 * CHUNKS + cn];
    }
    bf[1] = bn[32 * CHUNKS + cn];
  };
  auto step = [&](int st, int p) { step_x(st, p, std::false_type{}); };
  // Keep that order: each read right after the MFMA that frees its registers.
  auto order = [&](int steps) {
    constexpr int KI = Mfma<T>::kInsts;
#pragma unroll
    for (int p = 0; p < steps; ++p) {
      __builtin_amdgcn_sched_group_barrier(0x008, JM * KI, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
      for (int j = 0; j < JM; ++j) {
        __builtin_amdgcn_sched_group_barrier(0x008, KI, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
  };
  if (JM > 0) {
#pragma unroll
    for (int nb = 0; nb < NB_PER_WAVE; ++nb) bf[nb] = bbase[buf * B_STAGE + nb * 32 * CHUNKS + chunk(0)];
#pragma unroll
    for (int j = 0; j < JM; ++j) af[j] = abase[buf * A_STAGE + j * WAVES_M * 32 * CHUNKS + chunk(0)];
  }
  // Software-pipelined over the step barrier: K steps 0..2 of slab k, then B_k, then
  // K step 3 of slab k with the reads of slab k+1's first K step, whose latency the
  // MFMAs hide. (After the last slab those reads fetch stale data, never used.)
  if (nk > 0) {  // slab 0, peeled: it holds the unit's first MFMAs
    if (JM > 0) {
      step_x(buf, 1, std::true_type{});
#pragma unroll
      for (int p = 2; p < CHUNKS / 2; ++p) step(buf, p);
      order(CHUNKS / 2 - 1);
    }
    lds_barrier();  // B_0
    if (JM > 0) {
      step(buf ^ 1, 0);
      order(1);
    }
  }
  for (int k = 1; k < nk; ++k) {
    const int cur = buf ^ (k & 1);
    if (JM > 0) {
#pragma unroll
      for (int p = 1; p < CHUNKS / 2; ++p) step(cur, p);
      order(CHUNKS / 2 - 1);
    }
    lds_barrier();  // B_k: slab k read (the last fragments are in registers); slab k+1 landed
    if (JM > 0) {
      step(cur ^ 1, 0);
      order(1);
    }
  }

  // Block epilogue. 32x32 accumulator layout: lane holds column l32, and register
  // i = 4q + e the row 8q + 4h + e of the block. Each candidate becomes one integer key:
  //     key = (bits(x) & ~31) | (31 - row),   x = acc * mask
  // i.e. x with its 5 lowest mantissa bits replaced by the inverted row. For x > 0 the
  // float bits order like the values, so the largest key has the largest x and, among
  // x equal to 2^-18 relative, the lowest row -- the lowest-s rule, applied at the
  // precision the key keeps (the reference compares bf16-rounded logits, 2^-8). Keys of
  // x <= 0 are never positive-valued. With a 0/1 mask, bits(x) & ~31 is one AND with
  // the row's mask word. Rows 0..15 of block b are group 2b (registers q = 0, 1) and rows
  // 16..31 group 2b + 1 (q = 2, 3): one key per group and column.
  const int binary = um.mask_binary;
  const float* mrow = &um.maskf[wm * 32 + 4 * h];
  const int* wrow = &um.maskw[wm * 32 + 4 * h];
  int* kw = &sm.key[2 * wm][wn * 64 + l32];
#pragma unroll
  for (int j = 0; j < JM; ++j) {
    int kmax[2][NB_PER_WAVE];
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int nb = 0; nb < NB_PER_WAVE; ++nb) kmax[g][nb] = INT32_MIN;
    if (binary) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const i32x4 w4 = *(const i32x4*)(wrow + j * WAVES_M * 32 + 8 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int nb = 0; nb < NB_PER_WAVE; ++nb)
            kmax[q >> 1][nb] = max(kmax[q >> 1][nb],
                                   (__float_as_int(acc[j][nb][q * 4 + e]) & w4[e]) | (31 - 8 * q - e));
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 m4 = *(const f32x4*)(mrow + j * WAVES_M * 32 + 8 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int nb = 0; nb < NB_PER_WAVE; ++nb)
            kmax[q >> 1][nb] = max(kmax[q >> 1][nb],
                                   (__float_as_int(acc[j][nb][q * 4 + e] * m4[e]) & ~31) | (31 - 8 * q - e));
      }
    }
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int nb = 0; nb < NB_PER_WAVE; ++nb) {
        // The keys above encode rows 8q + e; lanes of half 1 hold rows 4 higher. Then
        // v_permlane32_swap exchanges the halves: element 1 of the result holds, in
        // lanes 0..31, the keys of lanes 32..63 (the only lanes that store below).
        const int k = kmax[g][nb] - 4 * h;
        const int ko = (int)__builtin_amdgcn_permlane32_swap((unsigned)k, (unsigned)k, false, false)[1];
        const int kb = max(k, ko);
        if (h == 0) kw[(j * 2 * WAVES_M + g) * BN + nb * 32] = kb;
      }
  }
  lds_barrier();  // E
}

template <typename T>
__device__ void compute_path(Smem& sm, const Args<T>& a, int w, int G, int n_units, int n_mt,
                             int n_vt, int wave, int lane) {
  const int nk = a.nk;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  Unit cur = unit_of(w, 0, G, n_units, n_mt, n_vt, a.n_grp);
  if (cur.u < 0) return;
  lds_barrier();  // S1
  lds_barrier();  // S2
  int par = 0, buf = 0;
  for (int r = 1;; ++r) {
    const UnitMeta& um = sm.um[par];
    const int n_blocks = (cur.n_valid + 1) / 2;  // 32-row blocks with an active group
    const int jm = n_blocks <= wm ? 0 : min(4, (n_blocks - wm + 1) / WAVES_M);
    switch (jm) {
      case 0: compute_unit<T, 0>(sm, um, nk, buf, lane, wm, wn); break;
      case 1: compute_unit<T, 1>(sm, um, nk, buf, lane, wm, wn); break;
      case 2: compute_unit<T, 2>(sm, um, nk, buf, lane, wm, wn); break;
      case 3: compute_unit<T, 3>(sm, um, nk, buf, lane, wm, wn); break;
      default: compute_unit<T, 4>(sm, um, nk, buf, lane, wm, wn); break;
    }
    const Unit next = unit_of(w, r, G, n_units, n_mt, n_vt, a.n_grp);
    if (next.u < 0) return;
    if (nk < PREFETCH_MIN_NK) {
      lds_barrier();  // S1
      lds_barrier();  // S2
    }
    cur = next;
    par ^= 1;
    buf ^= nk & 1;
  }
}

template <typename T>
__global__ __launch_bounds__(NTHREADS, 1) void sparton_fwd_kernel(
    const T* __restrict__ H, const T* __restrict__ W, const T* __restrict__ bias,
    const float* __restrict__ rowmask, T* __restrict__ reps, int32_t* __restrict__ argmax,
    float* __restrict__ reps_f32, int S, int D, int V, int n_vt, int ngrp,
    const int* __restrict__ meta, const int* __restrict__ list, float2* __restrict__ part) {
  __shared__ Smem sm;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: keep it scalar

  Args<T> a;
  a.H = (const char*)H;
  a.W = (const char*)W;
  a.bias = bias;
  a.rowmask = rowmask;
  a.list = list;
  a.n_grp = __builtin_amdgcn_readfirstlane(meta[0]);
  a.ngrp = ngrp;
  a.S = S;
  a.row_bytes = D * (int)sizeof(T);
  const int slab_elems = SLAB / (int)sizeof(T);
  a.nk_full = D / slab_elems;
  // At least two slabs per unit (a padding slab contributes zero); none when D == 0,
  // where x = bias * mask and nothing is loaded.
  a.nk = D == 0 ? 0 : max(2, (int)cdiv(D, slab_elems));
  a.V = V;

  const int n_mt = (a.n_grp + NGRP - 1) / NGRP;
  const int n_units = n_mt * n_vt;
  if (wave < COMPUTE_WAVES) {
    compute_path<T>(sm, a, blockIdx.x, gridDim.x, n_units, n_mt, n_vt, wave, lane);
  } else {
    Outputs<T> o{reps, argmax, reps_f32, part};
    copy_path<T>(sm, a, o, blockIdx.x, gridDim.x, n_units, n_mt, n_vt, tid - 64 * COMPUTE_WAVES,
                 wave - COMPUTE_WAVES, lane);
  }
}

// ---- fixup ------------------------------------------------------------------------

// Per batch row: no active group -> reps = 0, argmax = 0; groups spread over several
// M-tiles -> merge their partials in tile order (= s order). A workgroup covers 1024
// vocab ids (4 per thread) of one batch row and exits at once if the main kernel
// completed that row.
constexpr int FIX_COLS = 1024;
template <typename T>
__global__ __launch_bounds__(256) void fwd_fixup_kernel(int V, const int* __restrict__ count,
                                                        const int* __restrict__ first,
                                                        const float2* __restrict__ part,
                                                        T* __restrict__ reps,
                                                        int32_t* __restrict__ argmax,
                                                        float* __restrict__ reps_f32) {
  const int b = blockIdx.y;
  const int n = count[b];
  int ms = 0, me = 0;
  if (n > 0) {
    ms = first[b] / NGRP;
    me = (first[b] + n - 1) / NGRP;
    if (ms == me) return;  // written by the main kernel
  }
  constexpr int CPT = FIX_COLS / 256;  // columns per thread; each round's loads go together
  int col[CPT];
  float bv[CPT];
  int bi[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    col[k] = min(blockIdx.x * FIX_COLS + k * 256 + (int)threadIdx.x, V - 1);
    bv[k] = 0.0f;
    bi[k] = 0;
  }
  if (n > 0) {
    float2 p[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) p[k] = part[((int64_t)ms * 2 + 1) * V + col[k]];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      bv[k] = p[k].x;
      bi[k] = __float_as_int(p[k].y);
    }
    for (int mm = ms + 1; mm <= me; ++mm) {
#pragma unroll
      for (int k = 0; k < CPT; ++k) p[k] = part[((int64_t)mm * 2 + 0) * V + col[k]];
#pragma unroll
      for (int k = 0; k < CPT; ++k)
        if (p[k].x > bv[k]) {  // later tiles hold higher s: strict '>' keeps the lower on ties
          bv[k] = p[k].x;
          bi[k] = __float_as_int(p[k].y);
        }
    }
  }
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int v = blockIdx.x * FIX_COLS + k * 256 + threadIdx.x;
    if (v >= V) break;
    const int64_t o = (int64_t)b * V + v;
    const float rv = log1p_pos(bv[k]);
    reps[o] = from_f32<T>(rv);
    if (argmax != nullptr) argmax[o] = bi[k];
    if (reps_f32 != nullptr) reps_f32[o] = rv;
  }
}

// ---- small batches --------------------------------------------------------------
//
// B * S <= SMALL_MAX_ROWS: one kernel, no plan or fixup. The 256-column unit gives only
// cdiv(V, 256) units to 256 CUs (config 1: 120) and leaves most of its 256 rows empty;
// an fp32 batch is then bound by MFMA issue (fp32 MFMAs are 16x slower than bf16 ones)
// and a 16-bit one by the latency of its few units' W streams. Here every wave owns
// 32 vocab columns and all the batch's rows (RB blocks of 32): cdiv(V, 32) waves, about
// one per SIMD, and W is read once.
// K runs in 128-byte slabs. Each wave loads its W rows straight into registers through
// a ring of four slabs (three in flight while one is multiplied). The workgroup's four
// waves share the H rows: each slab of them is copied once into LDS (double-buffered,
// the main kernel's swizzled layout, one barrier per slab), so H is read from L2 once
// per workgroup instead of once per wave. Lane (l32, h) takes bytes 64h + 16p of each
// slab in step p, the main kernel's K order, and the accumulators start at the bias:
// every logit is summed exactly as the main kernel sums it. Bytes past D enter as
// zeros, and rows past B * S repeat the last row and are never reduced.
// Epilogue: x = acc * mask[row] goes to LDS, and lane pairs (batch row b, column) scan
// the b's S positions in order keeping the largest x with its 5 lowest mantissa bits
// cleared and, on ties, the lowest s -- the main kernel's key order.
constexpr int SMALL_MAX_ROWS = 128;
constexpr int SMALL_WAVES = 4;
// 16-bit batches take this kernel up to B * S * V = 2^24 (measured against the main path:
// 64-128 rows at V = 30522 and 32 rows at V = 128256 win by 7-36%, 128 rows at V = 250002
// loses by 15%); fp32 ones always (1.8-2x faster at every measured shape).
constexpr int64_t SMALL_MAX_WORK_16 = (int64_t)1 << 24;
// W slabs in each wave's register ring (SMALL_RING - 1 in flight). Deeper rings did not
// stream W faster: 6 and 8 slots measured 0-8% slower (1 x 16 bf16 rows at config-2
// widths 13.7 / 14.9 / 14.8 us; config 1, fp32, 40.9 / 41.1 / 42.4 us).
constexpr int SMALL_RING = 4;
// The same depth for the split mode (fp32 as bf16 hi/lo): 6, 8 and 10 slots measured 2-10%
// slower at config 1 (25.1 / 25.5 / 26.2 / 27.2 us).
constexpr int SMALL_RING_SPLIT = 4;

// The lane's W row, slab k: four 16-byte chunks (lane half h: bytes 64h + 16p), the
// offsets clamped into the row (chunks past D are cleared at use).
__device__ __forceinline__ void small_w_load(u32x4 (&f)[4], const char* wrow, int k, int h,
                                             int row_bytes) {
#pragma unroll
  for (int p = 0; p < 4; ++p) f[p] = *(const u32x4*)(wrow + min(k * 128 + h * 64 + p * 16, row_bytes - 16));
}

// This thread's RB chunks of the H slab k (thread t: row 32 r + t / 8, chunk t % 8),
// the offset clamped into the row.
template <int RB>
__device__ __forceinline__ void small_h_load(u32x4 (&hv)[RB], const char* const (&hrow)[RB], int k,
                                             int hc, int row_bytes) {
  const int off = min(k * 128 + hc * 16, row_bytes - 16);
#pragma unroll
  for (int r = 0; r < RB; ++r) hv[r] = *(const u32x4*)(hrow[r] + off);
}

// Into LDS, chunks past D as zeros. (The select sits here, after the slab's MFMAs, so
// that the wait for these loads does not hold the MFMAs back.)
template <int RB>
__device__ __forceinline__ void small_h_store(u32x4* buf, const u32x4 (&hv)[RB], int k, int hr, int hc,
                                              int row_bytes) {
  const bool ok = k * 128 + hc * 16 < row_bytes;
#pragma unroll
  for (int r = 0; r < RB; ++r)
    buf[(r * 32 + hr) * CHUNKS + (hc ^ swz_key(hr))] = ok ? hv[r] : u32x4{0u, 0u, 0u, 0u};
}

// Split mode (fp32): the slab's row holds its 32 floats as bf16 hi parts in logical chunks
// 0..3 and lo parts in chunks 4..7 (chunk c: k = 8c..8c+7 of the slab), under the same
// XOR swizzle. Thread chunk hc (k = 4hc..4hc+3) fills half hc & 1 of chunks hc / 2 and
// 4 + hc / 2; chunks past D hold zeros.
template <int RB>
__device__ __forceinline__ void small_h_store_split(u32x4* buf, const u32x4 (&hv)[RB], int k, int hr,
                                                    int hc, int row_bytes) {
  const bool ok = k * 128 + hc * 16 < row_bytes;
  u32x2* b2 = (u32x2*)buf;
  const int kx = swz_key(hr);
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    uint32_t h0, l0, h1, l1;
    split_pair(__uint_as_float(hv[r][0]), __uint_as_float(hv[r][1]), h0, l0);
    split_pair(__uint_as_float(hv[r][2]), __uint_as_float(hv[r][3]), h1, l1);
    const int row = (r * 32 + hr) * CHUNKS;
    b2[(row + ((hc >> 1) ^ kx)) * 2 + (hc & 1)] = ok ? u32x2{h0, h1} : u32x2{0u, 0u};
    b2[(row + ((4 + (hc >> 1)) ^ kx)) * 2 + (hc & 1)] = ok ? u32x2{l0, l1} : u32x2{0u, 0u};
  }
}

// Split-mode MFMAs of slab k: lane half h takes k = 16h..16h+15 of the slab, in two
// MFMA steps q of 8 (W chunks 2q, 2q + 1 of the lane; H chunks 2h + q and 4 + 2h + q).
template <int RB>
__device__ __forceinline__ void small_slab_split(const u32x4* buf, const u32x4 (&f)[4],
                                                 f32x16 (&acc)[RB], int k, int l32, int h,
                                                 int row_bytes) {
  const int kx = swz_key(l32);
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int b0 = k * 128 + h * 64 + q * 32;
    const u32x4 w0 = b0 < row_bytes ? f[2 * q] : u32x4{0u, 0u, 0u, 0u};
    const u32x4 w1 = b0 + 16 < row_bytes ? f[2 * q + 1] : u32x4{0u, 0u, 0u, 0u};
    u32x4 bhi, blo;
    split8(w0, w1, bhi, blo);
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const u32x4* row = buf + (r * 32 + l32) * CHUNKS;
      mfma_split(row[(2 * h + q) ^ kx], row[(4 + 2 * h + q) ^ kx], bhi, blo, acc[r]);
    }
  }
}

// The MFMAs of slab k: A from the LDS slab, B from the W registers.
template <typename T, int RB>
__device__ __forceinline__ void small_slab(const u32x4* buf, const u32x4 (&f)[4], f32x16 (&acc)[RB],
                                           int k, int l32, int h, int row_bytes) {
  const int kx = swz_key(l32);
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const bool ok = k * 128 + h * 64 + p * 16 < row_bytes;
    const u32x4 bq = ok ? f[p] : u32x4{0u, 0u, 0u, 0u};
    const int c = (h * 4 + p) ^ kx;
#pragma unroll
    for (int r = 0; r < RB; ++r) Mfma<T>::run(buf[(r * 32 + l32) * CHUNKS + c], bq, acc[r]);
  }
}

template <typename T, int RB, bool SPLIT>
__global__ __launch_bounds__(64 * SMALL_WAVES) void fwd_small_kernel(
    const T* __restrict__ H, const T* __restrict__ W, const T* __restrict__ bias,
    const void* __restrict__ mask, int mask_dtype, T* __restrict__ reps,
    int32_t* __restrict__ argmax, float* __restrict__ reps_f32, int B, int S, int D, int V) {
  static_assert(SMALL_WAVES * 64 == 32 * CHUNKS, "one thread per 16-byte chunk of 32 H rows");
  union Smem {
    u32x4 h[2][RB * 32 * CHUNKS];             // H slabs k and k + 1
    float xs[SMALL_WAVES][RB * 32][33];      // epilogue, per wave: x[row][column] (+1: no conflicts)
  };
  __shared__ Smem sm;
  __shared__ float mk[RB * 32];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, h = lane >> 5;
  const int rows = B * S;
  if (tid < RB * 32) mk[tid] = tid < rows ? load_mask(mask, mask_dtype, tid) : 0.0f;
  const int v0 = (blockIdx.x * SMALL_WAVES + wave) * 32;
  const bool live = v0 < V;  // waves past V stage H and keep the barriers
  const int row_bytes = D * (int)sizeof(T);
  const int nk = (row_bytes + 127) >> 7;  // slabs (the last may be partial)
  f32x16 acc[RB];
  const float bv = bias != nullptr ? to_f32(bias[min(v0 + l32, V - 1)]) : 0.0f;
#pragma unroll
  for (int r = 0; r < RB; ++r)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[r][i] = bv;
  const char* wrow = (const char*)(W + (int64_t)min(v0 + l32, V - 1) * D);
  const int hr = tid / CHUNKS, hc = tid % CHUNKS;
  const char* hrow[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) hrow[r] = (const char*)(H + (int64_t)min(r * 32 + hr, rows - 1) * D);
  if (nk > 0) {
    // Slab j: W from ring slot j % R (R - 1 slabs in flight while one is multiplied), H
    // from LDS buffer j % 2. Loads past the last slab re-read it (unused), so every step
    // issues the same loads; the scheduling barriers keep the loads in issue order (H's
    // first), so each wait counts only what it needs.
    constexpr int R = SPLIT ? SMALL_RING_SPLIT : SMALL_RING;
    u32x4 f[R][4], hv[RB];
    small_h_load<RB>(hv, hrow, 0, hc, row_bytes);
#pragma unroll
    for (int i = 0; i + 1 < R; ++i) small_w_load(f[i], wrow, min(i, nk - 1), h, row_bytes);
    if constexpr (SPLIT) small_h_store_split<RB>(sm.h[0], hv, 0, hr, hc, row_bytes);
    else small_h_store<RB>(sm.h[0], hv, 0, hr, hc, row_bytes);
    __syncthreads();
    auto step = [&](int j, const u32x4 (&fc)[4], u32x4 (&fn)[4]) {
      small_h_load<RB>(hv, hrow, min(j + 1, nk - 1), hc, row_bytes);
      small_w_load(fn, wrow, min(j + R - 1, nk - 1), h, row_bytes);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (SPLIT) small_slab_split<RB>(sm.h[j & 1], fc, acc, j, l32, h, row_bytes);
      else small_slab<T, RB>(sm.h[j & 1], fc, acc, j, l32, h, row_bytes);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (SPLIT)
        small_h_store_split<RB>(sm.h[(j + 1) & 1], hv, min(j + 1, nk - 1), hr, hc, row_bytes);
      else
        small_h_store<RB>(sm.h[(j + 1) & 1], hv, min(j + 1, nk - 1), hr, hc, row_bytes);
      __syncthreads();
    };
    int k = 0;
    for (; k + R - 1 < nk; k += R) {
#pragma unroll
      for (int i = 0; i < R; ++i) step(k + i, f[i], f[(i + R - 1) % R]);
    }
    // slots 0 .. R - 2 hold slabs k .. k + R - 2 (loads clamped to the last slab)
#pragma unroll
    for (int i = 0; i + 1 < R; ++i)
      if (k + i < nk) step(k + i, f[i], f[(i + R - 1) % R]);
  }
  // (the last step's barrier: every wave is done with the H slabs, sm.xs may be written)
  __syncthreads();  // mk is staged (also when nk == 0)
  if (live) {
    // 32x32 accumulator layout: lane holds column l32, register 4q + e row 8q + 4h + e.
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = r * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
        sm.xs[wave][row][l32] = acc[r][i] * mk[row];
      }
  }
  __syncthreads();
  if (!live) return;
  for (int t = lane; t < B * 32; t += 64) {
    const int b = t >> 5, c = t & 31, v = v0 + c;
    if (v >= V) continue;
    float bvx = 0.0f;
    int bi = 0;
    for (int s = 0; s < S; ++s) {
      const float x = __int_as_float(__float_as_int(sm.xs[wave][b * S + s][c]) & ~31);
      if (x > bvx) {  // strict: the lowest s keeps a tie
        bvx = x;
        bi = s;
      }
    }
    const int64_t o = (int64_t)b * V + v;
    const float rv = log1p_pos(bvx);
    reps[o] = from_f32<T>(rv);
    if (argmax != nullptr) argmax[o] = bi;
    if (reps_f32 != nullptr) reps_f32[o] = rv;
  }
}

// SPARTON_FWD_PATH=main sends small fp32 batches through the plan / main / fixup kernels
// too, and SPARTON_FWD_PATH=small sends small 16-bit batches through the small-batch kernel
// (tests compare the paths; measurements).
static int fwd_path_override() {
  const char* e = getenv("SPARTON_FWD_PATH");
  if (e == nullptr) return 0;
  if (strcmp(e, "main") == 0) return 1;
  if (strcmp(e, "small") == 0) return 2;
  return 0;
}

template <typename T, bool SPLIT>
static void launch_small(const void* H, const void* W, const void* bias, const void* mask,
                         int mask_dtype, void* reps, int32_t* argmax, float* reps_f32, int64_t B,
                         int64_t S, int64_t D, int64_t V, hipStream_t stream) {
  const dim3 grid((unsigned)cdiv(cdiv(V, 32), SMALL_WAVES)), block(64 * SMALL_WAVES);
#define SMALL(RB)                                                                                   \
  hipLaunchKernelGGL((fwd_small_kernel<T, RB, SPLIT>), grid, block, 0, stream, (const T*)H,        \
                     (const T*)W, (const T*)bias, mask, mask_dtype, (T*)reps, argmax, reps_f32,    \
                     (int)B, (int)S, (int)D, (int)V)
  switch (cdiv(B * S, 32)) {
    case 1: SMALL(1); break;
    case 2: SMALL(2); break;
    case 3: SMALL(3); break;
    default: SMALL(4); break;
  }
#undef SMALL
}

// Persistent grid: one workgroup per CU (the kernel's LDS allows one per CU), or
// fewer when there are fewer units. SPARTON_FWD_GRID overrides the workgroup count
// (tests use it to give each workgroup many units).
static int64_t persistent_grid(int64_t n_units_max) {
  int64_t g = 0;
  if (const char* env = getenv("SPARTON_FWD_GRID")) g = atoll(env);
  if (g <= 0) {
    int dev = 0, n_cu = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        n_cu > 0) {
      g = n_cu;
    } else {
      (void)hipGetLastError();  // clear the failed query; size for MI355X
      g = 256;
    }
  }
  return std::min<int64_t>(g, n_units_max);
}

// ev_main: if non-null, two events recorded on `stream` just before and after the main
// kernel (profiling).
// split: fp32 products as bf16 hi/lo parts (SPARTON_F32_SPLIT) in the small-batch kernel;
// the main kernel computes fp32 exactly either way.
template <typename T>
static int launch(const void* H, const void* W, const void* bias, const void* mask,
                  int mask_dtype, void* reps, int32_t* argmax, float* reps_f32, int64_t B,
                  int64_t S, int64_t D, int64_t V, const Work& w, hipStream_t stream,
                  hipEvent_t* ev_main, bool split) {
  const int64_t ngrp = cdiv(S, GROUP);
  const int64_t n_vt = cdiv(V, BN);
  const int64_t n_mt_max = cdiv(B * ngrp, NGRP);
  // Unit numbers (and one round past them) must fit in int.
  if (n_mt_max * n_vt > INT32_MAX / 2) return SPARTON_EUNSUPPORTED;
  const int ovr = fwd_path_override();
  if (B * S > 0 && B * S <= SMALL_MAX_ROWS && ovr != 1 &&
      (sizeof(T) == 4 || B * S * V <= SMALL_MAX_WORK_16 || ovr == 2)) {
    if (ev_main != nullptr) (void)hipEventRecord(ev_main[0], stream);
    bool done = false;
    if constexpr (sizeof(T) == 4) {
      if (split) {
        launch_small<T, true>(H, W, bias, mask, mask_dtype, reps, argmax, reps_f32, B, S, D, V, stream);
        done = true;
      }
    }
    if (!done)
      launch_small<T, false>(H, W, bias, mask, mask_dtype, reps, argmax, reps_f32, B, S, D, V, stream);
    if (ev_main != nullptr) (void)hipEventRecord(ev_main[1], stream);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? SPARTON_OK : (int)e;
  }
  const int64_t grid = persistent_grid(n_mt_max * n_vt);
  if (B * S <= PLAN_TINY_POS && B * ngrp <= PLAN_THREADS) {
    hipLaunchKernelGGL(fwd_plan_tiny_kernel, dim3(1), dim3(PLAN_THREADS), 0, stream, mask,
                       mask_dtype, (int)B, (int)S, (int)ngrp, w.count, w.first, w.list, w.meta,
                       w.rowmask);
  } else if (B <= PLAN_FUSED_MAX && B * ngrp <= PLAN_FUSED_MAX) {
    hipLaunchKernelGGL(fwd_plan_small_kernel, dim3(1), dim3(PLAN_THREADS), 0, stream, mask,
                       mask_dtype, (int)B, (int)S, (int)ngrp, w.count, w.first, w.list, w.meta,
                       w.rowmask);
  } else {
    hipLaunchKernelGGL(fwd_plan_rows_kernel, dim3((unsigned)cdiv(B, 4)), dim3(256), 0, stream,
                       mask, mask_dtype, (int)B, (int)S, (int)ngrp, w.flag, w.count);
    hipLaunchKernelGGL(fwd_plan_list_kernel, dim3(1), dim3(PLAN_THREADS), 0, stream, (int)B,
                       (int)ngrp, (const uint8_t*)w.flag, (const int*)w.count, w.first, w.list,
                       w.meta);
    hipLaunchKernelGGL(fwd_plan_rowmask_kernel, dim3((unsigned)cdiv(n_mt_max * BM, 256)), dim3(256),
                       0, stream, mask, mask_dtype, (int)S, (int)ngrp, (const int*)w.meta,
                       (const int*)w.list, w.rowmask);
  }
  if (ev_main != nullptr) (void)hipEventRecord(ev_main[0], stream);
  if (grid > 0)  // S == 0: no blocks, the fixup writes every row
    hipLaunchKernelGGL(sparton_fwd_kernel<T>, dim3((unsigned)grid), dim3(NTHREADS), 0, stream,
                       (const T*)H, (const T*)W, (const T*)bias, (const float*)w.rowmask, (T*)reps,
                       argmax, reps_f32, (int)S, (int)D, (int)V, (int)n_vt, (int)ngrp,
                       (const int*)w.meta, (const int*)w.list, w.part);
  if (ev_main != nullptr) (void)hipEventRecord(ev_main[1], stream);
  hipLaunchKernelGGL(fwd_fixup_kernel<T>, dim3((unsigned)cdiv(V, FIX_COLS), (unsigned)B), dim3(256), 0,
                     stream, (int)V, (const int*)w.count, (const int*)w.first,
                     (const float2*)w.part, (T*)reps, argmax, reps_f32);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPARTON_OK : (int)e;
}

// Batch rows per launch: byte offsets into H inside a launch stay below 2^31 (which also
// keeps every group code b * ngrp + j and tile-row index an int), and the fixup grid's
// y dimension (one per batch row) stays within 32768.
constexpr int64_t MAX_ROWS_PER_LAUNCH = 32768;
static int64_t rows_per_launch(int64_t B, int64_t S, int64_t D, int64_t esz) {
  const int64_t per_row = std::max<int64_t>(1, S * D * esz);
  const int64_t cap = std::min<int64_t>(MAX_ROWS_PER_LAUNCH, ((int64_t)1 << 31) / per_row);
  return std::max<int64_t>(1, std::min<int64_t>(B, cap));
}

static int64_t mask_elem_bytes(int mask_dtype) {
  switch (mask_dtype) {
    case SPARTON_MASK_I64: return 8;
    case SPARTON_MASK_I32:
    case SPARTON_MASK_F32: return 4;
    case SPARTON_MASK_U8: return 1;
    default: return 2;
  }
}

}  // namespace fwd
}  // namespace sparton

using namespace sparton;

extern "C" __attribute__((visibility("default"))) size_t sparton_fwd_workspace_bytes(
    int64_t B, int64_t S, int64_t D, int64_t V, int dtype) {
  if (B <= 0 || S < 0 || D < 0 || V <= 0) return 0;
  const int64_t esz = (dtype & ~SPARTON_F32_SPLIT) == SPARTON_F32 ? 4 : 2;
  return fwd::carve(nullptr, fwd::rows_per_launch(B, S, D, esz), S, V).total;
}

// dtype: an enum sparton_dtype, or SPARTON_F32 | SPARTON_F32_SPLIT.
static bool fwd_dtype_ok(int dtype) {
  const int base = dtype & ~SPARTON_F32_SPLIT;
  if (base < SPARTON_F32 || base > SPARTON_F16) return false;
  return (dtype & SPARTON_F32_SPLIT) == 0 || base == SPARTON_F32;
}

// The forward over row chunks; with main_ms, each chunk's main kernel is bracketed by
// HIP events and its device time added to *main_ms (synchronizing on each chunk).
static int fwd_run(const void* hidden, const void* weight, const void* bias, const void* mask,
                   int mask_dtype, void* reps, int32_t* argmax, float* reps_f32, int64_t B,
                   int64_t S, int64_t D, int64_t V, int dtype, void* workspace,
                   size_t workspace_bytes, void* stream, float* main_ms) {
  if (B < 0 || S < 0 || D < 0 || V < 0) return SPARTON_EINVAL;
  if (!fwd_dtype_ok(dtype)) return SPARTON_EINVAL;
  const bool split = (dtype & SPARTON_F32_SPLIT) != 0;
  dtype &= ~SPARTON_F32_SPLIT;
  if (mask_dtype < SPARTON_MASK_I64 || mask_dtype > SPARTON_MASK_F16) return SPARTON_EINVAL;
  if (B == 0 || V == 0) return SPARTON_OK;
  // Only pointers that will be dereferenced must be non-null (empty tensors may
  // carry a null data pointer).
  if (reps == nullptr) return SPARTON_EINVAL;
  if (S > 0 && D > 0 && (hidden == nullptr || weight == nullptr)) return SPARTON_EINVAL;
  if (S > 0 && mask == nullptr) return SPARTON_EINVAL;
  const int64_t esz = dtype == SPARTON_F32 ? 4 : 2;
  if ((D * esz) % 16 != 0) return SPARTON_EINVAL;
  if (((uintptr_t)hidden | (uintptr_t)weight) % 16 != 0) return SPARTON_EALIGN;
  if (B > INT32_MAX || V > INT32_MAX) return SPARTON_EUNSUPPORTED;
  if (S * D * esz >= ((int64_t)1 << 31) || (int64_t)fwd::BN * D * esz >= ((int64_t)1 << 31))
    return SPARTON_EUNSUPPORTED;
  const size_t need = sparton_fwd_workspace_bytes(B, S, D, V, dtype);
  if (workspace == nullptr || workspace_bytes < need) return SPARTON_EWORKSPACE;
  if ((uintptr_t)workspace % 256 != 0) return SPARTON_EALIGN;
  hipStream_t st = (hipStream_t)stream;
  const int64_t Bc = fwd::rows_per_launch(B, S, D, esz);
  for (int64_t b0 = 0; b0 < B; b0 += Bc) {
    const int64_t nb = std::min(Bc, B - b0);
    const fwd::Work w = fwd::carve(workspace, nb, S, V);
    const char* h = (const char*)hidden + b0 * S * D * esz;
    const char* mk = mask == nullptr ? nullptr : (const char*)mask + b0 * S * fwd::mask_elem_bytes(mask_dtype);
    char* r = (char*)reps + b0 * V * esz;
    int32_t* am = argmax == nullptr ? nullptr : argmax + b0 * V;
    float* r32 = reps_f32 == nullptr ? nullptr : reps_f32 + b0 * V;
    hipEvent_t ev[2] = {nullptr, nullptr};
    if (main_ms != nullptr) {
      if (hipEventCreate(&ev[0]) != hipSuccess || hipEventCreate(&ev[1]) != hipSuccess) {
        if (ev[0] != nullptr) (void)hipEventDestroy(ev[0]);
        return (int)hipGetLastError();
      }
    }
    hipEvent_t* evp = main_ms != nullptr ? ev : nullptr;
    int rc;
    switch (dtype) {
      case SPARTON_BF16:
        rc = fwd::launch<bf16>(h, weight, bias, mk, mask_dtype, r, am, r32, nb, S, D, V, w, st, evp, false);
        break;
      case SPARTON_F16:
        rc = fwd::launch<f16>(h, weight, bias, mk, mask_dtype, r, am, r32, nb, S, D, V, w, st, evp, false);
        break;
      default:
        rc = fwd::launch<float>(h, weight, bias, mk, mask_dtype, r, am, r32, nb, S, D, V, w, st, evp, split);
        break;
    }
    if (main_ms != nullptr) {
      float ms = 0.0f;
      hipError_t e = hipEventSynchronize(ev[1]);
      if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev[0], ev[1]);
      (void)hipEventDestroy(ev[0]);
      (void)hipEventDestroy(ev[1]);
      if (rc == SPARTON_OK && e != hipSuccess) rc = (int)e;
      *main_ms += ms;
    }
    if (rc != SPARTON_OK) return rc;
  }
  return SPARTON_OK;
}

extern "C" __attribute__((visibility("default"))) int sparton_fwd(
    const void* hidden, const void* weight, const void* bias, const void* mask,
    int mask_dtype, void* reps, int32_t* argmax, float* reps_f32, int64_t B, int64_t S,
    int64_t D, int64_t V, int dtype, void* workspace, size_t workspace_bytes, void* stream) {
  return fwd_run(hidden, weight, bias, mask, mask_dtype, reps, argmax, reps_f32, B, S, D, V,
                 dtype, workspace, workspace_bytes, stream, nullptr);
}

// ---- no-allocation entry point ----------------------------------------------------
//
// sparton_fwd_noalloc runs the same kernels as sparton_fwd with the workspace taken from
// `scratch`, a file-scope device array: one copy per GPU, created when the library's code
// object is loaded there and held until the process ends. Its device address on the
// current GPU comes from hipGetSymbolAddress, once per device (the array's name in host
// code is only a stand-in for the symbol). Nothing in the workspace has to start at zero:
// the plan kernels write every count, list entry and row-mask value they use, and the
// fixup reads only partials the main kernel wrote in the same launch. Every call on one
// GPU shares the array, so calls that overlap on that GPU (other streams, other threads)
// race and must be serialised by the caller.
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device, once resolved
}  // namespace

// Device address of `scratch` on the current device (resolved on its first call there).
static int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return SPARTON_EUNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (p == nullptr || (uintptr_t)p % 256 != 0) return SPARTON_EALIGN;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SPARTON_OK;
}

extern "C" __attribute__((visibility("default"))) size_t sparton_fwd_noalloc_max_workspace(void) {
  return kNoAllocScratchBytes;
}

extern "C" __attribute__((visibility("default"))) int sparton_fwd_noalloc(
    const void* hidden, const void* weight, const void* bias, const void* mask,
    int mask_dtype, void* reps, int32_t* argmax, float* reps_f32, int64_t B, int64_t S,
    int64_t D, int64_t V, int dtype, void* stream) {
  if (B < 0 || S < 0 || D < 0 || V < 0) return SPARTON_EINVAL;
  if (!fwd_dtype_ok(dtype)) return SPARTON_EINVAL;
  if (mask_dtype < SPARTON_MASK_I64 || mask_dtype > SPARTON_MASK_F16) return SPARTON_EINVAL;
  const size_t need = sparton_fwd_workspace_bytes(B, S, D, V, dtype);
  if (need > kNoAllocScratchBytes) return SPARTON_ESCRATCH;
  void* ws = nullptr;
  if (need > 0) {
    const int rc = scratch_address(&ws);
    if (rc != SPARTON_OK) return rc;
  }
  return fwd_run(hidden, weight, bias, mask, mask_dtype, reps, argmax, reps_f32, B, S, D, V,
                 dtype, ws, need > 0 ? kNoAllocScratchBytes : 0, stream, nullptr);
}

extern "C" __attribute__((visibility("default"))) int sparton_fwd_profile(
    const void* hidden, const void* weight, const void* bias, const void* mask,
    int mask_dtype, void* reps, int32_t* argmax, float* reps_f32, int64_t B, int64_t S,
    int64_t D, int64_t V, int dtype, void* workspace, size_t workspace_bytes, void* stream,
    float* main_ms) {
  if (main_ms == nullptr) return SPARTON_EINVAL;
  *main_ms = 0.0f;
  return fwd_run(hidden, weight, bias, mask, mask_dtype, reps, argmax, reps_f32, B, S, D, V,
                 dtype, workspace, workspace_bytes, stream, main_ms);
}
