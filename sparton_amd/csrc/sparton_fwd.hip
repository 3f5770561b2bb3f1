// SpartonHead forward on gfx950: one kernel, MFMA mainloop + fused reduction epilogue.
//
// A workgroup owns one batch row b and P consecutive vocab tiles of BN columns. It
// sweeps the sequence in chunks of BM positions; one (vocab tile, chunk) pair is a
// "unit". For each unit it computes the BM x BN logit tile
//     H[b, s0:s0+BM, :] . W[v0:v0+BN, :]^T
// with bf16/fp16 (or fp32) MFMA, K = D streamed through double-buffered LDS, then folds
// the tile into a running (max, argmax) per column in registers:
//     x = (acc + bias[v]) * mask[b, s];  take x if x > best (strict, s ascending)
// so the [B,S,V] logits never reach HBM. After the last chunk of a vocab tile the
// per-column winners of the two M-waves are merged (larger value, ties -> lower s) and
// the workgroup writes reps[b, v] = log1p(max(0, best)) and argmax[b, v].
//
// Reference semantics followed (src/sparton/sparton_kernel.py):
//   bias added to the GEMM output            :209-210, :245
//   logits multiplied by mask                :147
//   running max initialised to 0, idx to 0   :112-114
//   lowest s wins ties (tl.argmax + strict >) :151-156
//   reps = log(1 + relu(max))                :159-161 (log1p here)
//
// Pipeline: the K slabs of all units of a workgroup form one stream through the two
// LDS stages, so the first two slabs of a unit are loaded while the previous unit
// finishes its last slab and runs its epilogue (no per-tile load latency on the
// critical path). The mask row of b is scanned once per workgroup: all-zero 32-row
// blocks contribute x = 0, which never beats the initial 0, so chunks without an
// active block are skipped and, inside a chunk, a wave only multiplies its blocks up
// to the last active one and A rows past it are not loaded.
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

#include "sparton_common.h"

namespace sparton {
namespace fwd {

constexpr int BM = 256;              // sequence positions per chunk
constexpr int BN = 256;              // vocab columns per tile
constexpr int WAVES_M = 2;           // waves along M (sequence)
constexpr int WAVES_N = 4;           // waves along N (vocab)
constexpr int NWAVES = WAVES_M * WAVES_N;
constexpr int NTHREADS = 64 * NWAVES;
constexpr int MBLK = BM / 32;        // 32-row MFMA blocks per chunk (8)
constexpr int NB_PER_WAVE = BN / WAVES_N / 32;     // 2
constexpr int SLAB = 128;            // bytes of K per row per pipeline stage
constexpr int CHUNKS = SLAB / 16;    // 16-byte chunks per row slab (8)
constexpr int ROWS_PER_LOAD = 64 / CHUNKS;          // rows one wave-wide load covers (8)
constexpr int A_LOADS = BM / ROWS_PER_LOAD / NWAVES;  // wave-wide loads per slab for A (4)
constexpr int B_LOADS = BN / ROWS_PER_LOAD / NWAVES;  // and for B (4)
constexpr int GROUP_V = 4;           // vocab-tile groups per scheduling group (L2 reuse)
constexpr int MAX_CHUNKS = 64;       // S <= MAX_CHUNKS * BM
constexpr int MAX_P = 16;            // vocab tiles per workgroup

struct Smem {
  u32x4 a[2][BM * CHUNKS];   // [stage][row * 8 + (chunk ^ f(row))]
  u32x4 b[2][BN * CHUNKS];
  float maskf[BM];           // mask of the current unit's chunk
  float biasf[MAX_P * BN];   // bias of the workgroup's vocab tiles
  float red_v[WAVES_M][BN];  // cross-wave merge of the per-column winners
  int red_i[WAVES_M][BN];
  uint8_t chunk_fl[MAX_CHUNKS];  // per chunk: bit j = block j has a nonzero mask entry
  uint8_t chunk_list[MAX_CHUNKS];
  int n_active;                  // chunks with an active block
};

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ int swz_key(int row) { return (row & 7) ^ ((row >> 3) & 1); }

// One MFMA "step" consumes 16 bytes of A and B per lane.
template <typename T> struct Mfma;
template <> struct Mfma<bf16> {
  static constexpr int kInsts = 1;
  static __device__ __forceinline__ void run(const u32x4& a, const u32x4& b, f32x16& c) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma<f16> {
  static constexpr int kInsts = 1;
  static __device__ __forceinline__ void run(const u32x4& a, const u32x4& b, f32x16& c) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
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
};

// Map the hardware workgroup id to (b, vocab-tile group). Workgroups are dispatched
// round-robin over the 8 XCDs; first make ids that share an XCD consecutive, then
// walk groups of GROUP_V vocab-tile groups x all batch rows so the workgroups
// resident on one XCD at a time share a few W tiles and a few H rows in its L2.
__device__ __forceinline__ void tile_of(int wg, int grid, int B, int n_vg, int* b, int* vg) {
  const int xcd = wg & 7, local = wg >> 3, q = grid >> 3, r = grid & 7;
  const int lin = (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + local;
  const int group = lin / (GROUP_V * B);
  const int rem = lin - group * GROUP_V * B;
  const int gv = min(GROUP_V, n_vg - group * GROUP_V);
  *b = rem / gv;
  *vg = group * GROUP_V + rem % gv;
}

__device__ __forceinline__ void merge(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}

// One (vocab tile, chunk) unit: workgroup-uniform scalars.
struct Unit {
  int v0, s0;
  int last_blk;   // highest 32-row block of the chunk with a nonzero mask entry
};

// Wave w, load i covers the 8-row group g = i * NWAVES + w; lane L lands at LDS chunk
// g*64 + L, i.e. row 8g + L/8, physical chunk L%8, which holds logical chunk (L%8) ^ f(row).
__device__ __forceinline__ void load_rows(int i, int wave, int lane, int* row, int* chunk) {
  const int g = i * NWAVES + wave;
  *row = g * ROWS_PER_LOAD + (lane >> 3);
  *chunk = (lane & 7) ^ swz_key(*row);
}

struct Geo {
  const char* H;      // row (b, 0) of H
  const char* W;
  int row_bytes;      // D * sizeof(T)
  int nk_full;        // slabs lying entirely inside the row
  int S, V;
};

// Issue the direct global -> LDS copies of K slab k of unit u into stage buf. Chunks
// past the row end (tail or padding slabs) re-read slab 0 -- valid, finite data -- and
// their W copies are zeroed by zero_tail() before use. Rows past S or V re-read the
// last row (their results are masked out or never stored).
__device__ __forceinline__ void issue_slab(Smem& sm, const Geo& g, const Unit& u, int k, int buf,
                                           int wave, int lane) {
  const uint32_t kb = (uint32_t)k * SLAB;
  const bool tail = k >= g.nk_full;
  const char* ab = g.H + (int64_t)u.s0 * g.row_bytes;
  const char* bb = g.W + (int64_t)u.v0 * g.row_bytes;
  const int a_groups = (u.last_blk + 1) * (32 / ROWS_PER_LOAD);
#pragma unroll
  for (int i = 0; i < A_LOADS; ++i) {
    const int grp = i * NWAVES + wave;
    if (grp < a_groups) {
      int row, c;
      load_rows(i, wave, lane, &row, &c);
      uint32_t off = (uint32_t)min(row, g.S - 1 - u.s0) * (uint32_t)g.row_bytes + c * 16;
      off += (!tail || kb + c * 16 < (uint32_t)g.row_bytes) ? kb : 0u;
      __builtin_amdgcn_global_load_lds((const void*)(ab + off), (lds_void*)&sm.a[buf][grp * 64], 16, 0, 0);
    }
  }
#pragma unroll
  for (int i = 0; i < B_LOADS; ++i) {
    const int grp = i * NWAVES + wave;
    int row, c;
    load_rows(i, wave, lane, &row, &c);
    uint32_t off = (uint32_t)min(row, g.V - 1 - u.v0) * (uint32_t)g.row_bytes + c * 16;
    off += (!tail || kb + c * 16 < (uint32_t)g.row_bytes) ? kb : 0u;
    __builtin_amdgcn_global_load_lds((const void*)(bb + off), (lds_void*)&sm.b[buf][grp * 64], 16, 0, 0);
  }
}

// Zero the W chunks of slab k (in stage buf) that lie past D; run after its copies
// landed and before any wave reads the stage.
__device__ __forceinline__ void zero_tail(Smem& sm, int row_bytes, int k, int buf, int wave, int lane) {
  const uint32_t kb = (uint32_t)k * SLAB;
#pragma unroll
  for (int i = 0; i < B_LOADS; ++i) {
    int row, c;
    load_rows(i, wave, lane, &row, &c);
    if (kb + c * 16 >= (uint32_t)row_bytes)
      sm.b[buf][(i * NWAVES + wave) * 64 + lane] = u32x4{0, 0, 0, 0};
  }
}

// Wait for all of this thread's outstanding memory operations (the direct-to-LDS
// loads included), then the workgroup barrier.
__device__ __forceinline__ void drain_and_sync() {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

// Workgroup barrier for data exchanged through ordinary LDS reads/writes only: waits
// for this wave's LDS operations, not for its global loads. (__syncthreads() implies a
// workgroup fence, which on gfx950 also waits for every outstanding direct-to-LDS
// load -- here the next unit's slabs, which must stay in flight.) The memory clobber
// keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Wait until at most n (0..8, wave-uniform) direct loads of this wave are in flight.
// s_waitcnt takes an immediate: simm16 = vmcnt[15:14,3:0] | lgkmcnt[11:8] | expcnt[6:4];
// 0x0F70 | n is vmcnt(n) with lgkmcnt and expcnt at their no-wait maxima.
__device__ __forceinline__ void wait_loads_at_most(int n) {
  switch (n) {
    case 0: __builtin_amdgcn_s_waitcnt(0x0F70 | 0); break;
    case 1: __builtin_amdgcn_s_waitcnt(0x0F70 | 1); break;
    case 2: __builtin_amdgcn_s_waitcnt(0x0F70 | 2); break;
    case 3: __builtin_amdgcn_s_waitcnt(0x0F70 | 3); break;
    case 4: __builtin_amdgcn_s_waitcnt(0x0F70 | 4); break;
    case 5: __builtin_amdgcn_s_waitcnt(0x0F70 | 5); break;
    case 6: __builtin_amdgcn_s_waitcnt(0x0F70 | 6); break;
    case 7: __builtin_amdgcn_s_waitcnt(0x0F70 | 7); break;
    default: __builtin_amdgcn_s_waitcnt(0x0F70 | 8); break;
  }
}

// Prefetched state for the next unit.
struct Next {
  bool valid;
  bool new_tile;      // next unit starts another vocab tile
  Unit u;
};

// Mainloop + chunk epilogue of one unit, for a wave with JM blocks to multiply.
// On entry slab 0 of the unit has landed in stage `buf` (and is visible) and slab 1 is
// in flight or landed in the other stage. On exit slab 0 of the next unit has landed
// and its slab 1 is in flight. Returns the stage of the next unit's slab 0.
template <typename T, int JM>
__device__ __forceinline__ int run_unit(Smem& sm, const Geo& g, const Unit& u, const Next& nx,
                                        int nk, int buf, int wave, int lane, int wm, int wn,
                                        const void* mask, int mask_dtype, int64_t mrow,
                                        int S, int btile, float* best, int* bidx) {
  constexpr int JA = JM > 0 ? JM : 1;
  const int tid = threadIdx.x;
  const int l32 = lane & 31, h = lane >> 5;
  f32x16 acc[JA][NB_PER_WAVE];
#pragma unroll
  for (int nb = 0; nb < NB_PER_WAVE; ++nb) {
    const float bc = sm.biasf[btile * BN + wn * 64 + nb * 32 + l32];
#pragma unroll
    for (int j = 0; j < JA; ++j)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[j][nb][i] = bc;
  }

  // This unit's mask: loaded at step 0, stored at step 1 (the previous unit's
  // epilogue is done with maskf by then), read by the epilogue below.
  float mv = 0.0f;
  if (nk == 0) {  // D == 0: no slabs; store the mask between two barriers
    lds_barrier();
    if (tid < BM) sm.maskf[tid] = u.s0 + tid < S ? load_mask(mask, mask_dtype, mrow + u.s0 + tid) : 0.0f;
    lds_barrier();
  }
  for (int k = 0; k < nk; ++k) {
    const int cur = buf ^ (k & 1);
    if (k >= g.nk_full) {  // tail / padding slab: clear W past D before use
      zero_tail(sm, g.row_bytes, k, cur, wave, lane);
      lds_barrier();
    }
    if (k == 0 && tid < BM) {
      const int s = u.s0 + tid;
      mv = s < S ? load_mask(mask, mask_dtype, mrow + s) : 0.0f;
    }
    if (k == 1 && tid < BM) sm.maskf[tid] = mv;
    if (JM > 0) {
      // Every operand row is (multiple of 32) + l32, so its swizzle key is key(l32):
      // a fragment's LDS index is a per-lane offset plus a compile-time row offset.
      const u32x4* abuf = sm.a[cur] + (wm * 32) * CHUNKS;
      const u32x4* bbuf = sm.b[cur] + (wn * 64) * CHUNKS;
      const int kx = swz_key(l32);
      // Operand fragments for K step p+1 are read while step p's MFMAs run.
      u32x4 bf[2][NB_PER_WAVE], af[2][JA];
      auto read = [&](int p, int slot) {
        const int off = l32 * CHUNKS + ((h * (CHUNKS / 2) + p) ^ kx);  // lane half h: K chunks 4h..4h+3
#pragma unroll
        for (int nb = 0; nb < NB_PER_WAVE; ++nb) bf[slot][nb] = bbuf[nb * 32 * CHUNKS + off];
#pragma unroll
        for (int j = 0; j < JM; ++j) af[slot][j] = abuf[j * WAVES_M * 32 * CHUNKS + off];
      };
      read(0, 0);
#pragma unroll
      for (int p = 0; p < CHUNKS / 2; ++p) {
        if (p + 1 < CHUNKS / 2) read(p + 1, (p + 1) & 1);
#pragma unroll
        for (int j = 0; j < JM; ++j)
#pragma unroll
          for (int nb = 0; nb < NB_PER_WAVE; ++nb)
            Mfma<T>::run(af[p & 1][j], bf[p & 1][nb], acc[j][nb]);
      }
      // Schedule: the first step's reads, then each step's MFMAs with the next
      // step's LDS reads slotted one by one between them.
      constexpr int NREAD = NB_PER_WAVE + JM;
      constexpr int NMFMA = NB_PER_WAVE * JM * Mfma<T>::kInsts;
      __builtin_amdgcn_sched_group_barrier(0x100, NREAD, 0);
#pragma unroll
      for (int p = 0; p < CHUNKS / 2; ++p) {
#pragma unroll
        for (int i = 0; i < NMFMA; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if (p + 1 < CHUNKS / 2 && i < NREAD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
      }
    }
    drain_and_sync();
    // Stage `cur` is free: refill it with the slab two ahead in the stream.
    const bool own = k + 2 < nk;
    if (own || nx.valid) {
      Unit t;
      t.v0 = own ? u.v0 : nx.u.v0;
      t.s0 = own ? u.s0 : nx.u.s0;
      t.last_blk = own ? u.last_blk : nx.u.last_blk;
      issue_slab(sm, g, t, own ? k + 2 : k + 2 - nk, cur, wave, lane);
    }
  }

  // Chunk epilogue: 32x32 accumulator layout -- lane holds column l32, and for
  // register i the row 8*(i/4) + 4*h + (i%4). Rows rise with i, blocks rise with j,
  // chunks rise with s0, so a strict '>' keeps the lowest s within the lane.
#pragma unroll
  for (int j = 0; j < JM; ++j) {
    const int rbase = (wm + WAVES_M * j) * 32 + 4 * h;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x4 m4 = *(const f32x4*)(&sm.maskf[rbase + 8 * q]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int s = u.s0 + rbase + 8 * q + e;
#pragma unroll
        for (int nb = 0; nb < NB_PER_WAVE; ++nb) {
          const float x = acc[j][nb][q * 4 + e] * m4[e];
          if (x > best[nb]) { best[nb] = x; bidx[nb] = s; }
        }
      }
    }
  }
  return buf ^ (nk & 1);
}

// Merge the per-column winners of all waves and write reps / argmax for vocab tile v0.
template <typename T>
__device__ __forceinline__ void write_tile(Smem& sm, int v0, int64_t orow, int V, int wm, int wn,
                                           int lane, float* best, int* bidx, T* reps,
                                           int32_t* argmax, float* reps_f32) {
  const int tid = threadIdx.x, l32 = lane & 31, h = lane >> 5;
  // Lanes l and l^32 hold the same column (different rows): merge them.
#pragma unroll
  for (int nb = 0; nb < NB_PER_WAVE; ++nb) {
    const float ov = __shfl_xor(best[nb], 32);
    const int oi = __shfl_xor(bidx[nb], 32);
    merge(best[nb], bidx[nb], ov, oi);
  }
  if (h == 0) {
#pragma unroll
    for (int nb = 0; nb < NB_PER_WAVE; ++nb) {
      const int col = wn * 64 + nb * 32 + l32;
      sm.red_v[wm][col] = best[nb];
      sm.red_i[wm][col] = bidx[nb];
    }
  }
  lds_barrier();
  if (tid < BN) {
    const int v = v0 + tid;
    if (v < V) {
      float bv = sm.red_v[0][tid];
      int bi = sm.red_i[0][tid];
#pragma unroll
      for (int w = 1; w < WAVES_M; ++w) merge(bv, bi, sm.red_v[w][tid], sm.red_i[w][tid]);
      const int64_t o = orow + v;
      const float r = log1pf(bv);
      reps[o] = from_f32<T>(r);
      if (argmax != nullptr) argmax[o] = bi;
      if (reps_f32 != nullptr) reps_f32[o] = r;
    }
  }
  lds_barrier();  // red_v/red_i are reused by the next tile
}

template <typename T>
__global__ __launch_bounds__(NTHREADS, 1) void sparton_fwd_kernel(
    const T* __restrict__ H, const T* __restrict__ W, const T* __restrict__ bias,
    const void* __restrict__ mask, int mask_dtype, T* __restrict__ reps,
    int32_t* __restrict__ argmax, float* __restrict__ reps_f32, int B, int S, int D, int V,
    int n_vt, int P) {
  __shared__ Smem sm;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: keep it scalar
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int l32 = lane & 31;

  const int n_vg = (n_vt + P - 1) / P;
  int b, vg;
  tile_of(blockIdx.x, gridDim.x, B, n_vg, &b, &vg);
  const int vt_lo = vg * P, n_tiles = min(P, n_vt - vt_lo);
  const int64_t mrow = (int64_t)b * S;

  Geo g;
  g.row_bytes = D * (int)sizeof(T);
  g.H = (const char*)(H + mrow * D);
  g.W = (const char*)W;
  const int slab_elems = SLAB / (int)sizeof(T);
  g.nk_full = D / slab_elems;
  g.S = S;
  g.V = V;
  // At least two slabs per unit (a padding slab contributes zero); none when D == 0,
  // where x = bias * mask and nothing is loaded.
  const int nk = D == 0 ? 0 : max(2, (int)cdiv(D, slab_elems));

  // Slab 0 of the first unit is started before anything else, on the guess that the
  // first unit is chunk 0 of the first vocab tile (reloaded below if it is not); all
  // A rows are loaded, as the active blocks are not known yet.
  Unit u0;
  u0.v0 = vt_lo * BN;
  u0.s0 = 0;
  u0.last_blk = MBLK - 1;
  if (nk > 0 && S > 0) issue_slab(sm, g, u0, 0, 0, wave, lane);

  // Scan the mask row once: per 32-row block, whether any entry is nonzero.
  const int n_chunks = (int)cdiv(S, BM);
  if (tid < MAX_CHUNKS) sm.chunk_fl[tid] = 0;
  lds_barrier();
  for (int s_base = 0; s_base < n_chunks * BM; s_base += NTHREADS) {
    const int s = s_base + tid;
    const bool nz = s < S && load_mask(mask, mask_dtype, mrow + s) != 0.0f;
    const uint64_t bal = __ballot(nz);
    if (lane == 0 && bal != 0) {
      const int blk0 = (s_base + wave * 64) / 32;  // two 32-row blocks per wave
      const uint32_t bits = ((bal & 0xffffffffull) != 0 ? 1u : 0u) << (blk0 & 7) |
                            ((bal >> 32) != 0 ? 1u : 0u) << ((blk0 + 1) & 7);
      atomicOr((unsigned*)&sm.chunk_fl[0] + (blk0 / 8) / 4, bits << (8 * ((blk0 / 8) & 3)));
    }
  }
  for (int i = tid; i < n_tiles * BN; i += NTHREADS) {
    const int col = vt_lo * BN + i;
    sm.biasf[i] = (bias != nullptr && col < V) ? to_f32(bias[col]) : 0.0f;
  }
  lds_barrier();
  if (tid == 0) {
    int n = 0;
    for (int c = 0; c < n_chunks; ++c)
      if (sm.chunk_fl[c] != 0) sm.chunk_list[n++] = (uint8_t)c;
    sm.n_active = n;
  }
  lds_barrier();
  const int n_active = __builtin_amdgcn_readfirstlane(sm.n_active);

  if (n_active == 0) {  // fully masked row: M = 0, I = 0 for every column
    __builtin_amdgcn_s_waitcnt(0);  // no direct load may land after the workgroup ends
    for (int t = 0; t < n_tiles; ++t) {
      if (tid < BN) {
        const int v = (vt_lo + t) * BN + tid;
        if (v < V) {
          const int64_t o = (int64_t)b * V + v;
          reps[o] = from_f32<T>(0.0f);
          if (argmax != nullptr) argmax[o] = 0;
          if (reps_f32 != nullptr) reps_f32[o] = 0.0f;
        }
      }
    }
    return;
  }

  // Unit descriptors are read from LDS: readfirstlane keeps them in SGPRs (they are
  // workgroup-uniform), so the loads use the SGPR-base + VGPR-offset form.
  auto unit_at = [&](int idx) {
    Unit u;
    const int t = idx / n_active;
    const int c = __builtin_amdgcn_readfirstlane(sm.chunk_list[idx - t * n_active]);
    const uint32_t fl = __builtin_amdgcn_readfirstlane(sm.chunk_fl[c]);
    u.v0 = (vt_lo + t) * BN;
    u.s0 = c * BM;
    u.last_blk = 31 - __builtin_clz(fl);
    return u;
  };
  const int n_units = n_tiles * n_active;

  Unit u = unit_at(0);
  if (nk > 0) {
    if (u.s0 != 0) {  // the guess was wrong: drain it and load the right rows
      __builtin_amdgcn_s_waitcnt(0);
      issue_slab(sm, g, u, 0, 0, wave, lane);
    }
    issue_slab(sm, g, u, 1, 1, wave, lane);
    // Slab 0 must have landed everywhere; slab 1 stays in flight.
    const int a_groups = (u.last_blk + 1) * (32 / ROWS_PER_LOAD);
    int n1 = B_LOADS;
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) n1 += (i * NWAVES + wave < a_groups) ? 1 : 0;
    wait_loads_at_most(n1);
  }
  float best[NB_PER_WAVE];
  int bidx[NB_PER_WAVE];
#pragma unroll
  for (int nb = 0; nb < NB_PER_WAVE; ++nb) {
    best[nb] = 0.0f;
    bidx[nb] = 0;
  }
  lds_barrier();

  int buf = 0;
  for (int idx = 0; idx < n_units; ++idx) {
    Next nx;
    nx.valid = idx + 1 < n_units;
    nx.new_tile = nx.valid && ((idx + 1) % n_active == 0);
    if (nx.valid) nx.u = unit_at(idx + 1);
    // Blocks of this wave are wm, wm+2, ...: multiply those up to the last active
    // one (masked rows below it give x = 0 and cannot win).
    const int jm = u.last_blk < wm ? 0 : (u.last_blk - wm) / WAVES_M + 1;
    switch (jm) {
      case 0: buf = run_unit<T, 0>(sm, g, u, nx, nk, buf, wave, lane, wm, wn, mask, mask_dtype, mrow, S, idx / n_active, best, bidx); break;
      case 1: buf = run_unit<T, 1>(sm, g, u, nx, nk, buf, wave, lane, wm, wn, mask, mask_dtype, mrow, S, idx / n_active, best, bidx); break;
      case 2: buf = run_unit<T, 2>(sm, g, u, nx, nk, buf, wave, lane, wm, wn, mask, mask_dtype, mrow, S, idx / n_active, best, bidx); break;
      case 3: buf = run_unit<T, 3>(sm, g, u, nx, nk, buf, wave, lane, wm, wn, mask, mask_dtype, mrow, S, idx / n_active, best, bidx); break;
      default: buf = run_unit<T, 4>(sm, g, u, nx, nk, buf, wave, lane, wm, wn, mask, mask_dtype, mrow, S, idx / n_active, best, bidx); break;
    }
    if (!nx.valid || nx.new_tile) {
      write_tile<T>(sm, u.v0, (int64_t)b * V, V, wm, wn, lane, best, bidx, reps, argmax, reps_f32);
#pragma unroll
      for (int nb = 0; nb < NB_PER_WAVE; ++nb) {
        best[nb] = 0.0f;
        bidx[nb] = 0;
      }
    }
    if (nx.valid) u = nx.u;
  }
}

template <typename T>
static int launch(const void* H, const void* W, const void* bias, const void* mask,
                  int mask_dtype, void* reps, int32_t* argmax, float* reps_f32, int64_t B,
                  int64_t S, int64_t D, int64_t V, int P, hipStream_t stream) {
  const int64_t n_vt = cdiv(V, BN);
  const int64_t grid = cdiv(n_vt, P) * B;
  hipLaunchKernelGGL(sparton_fwd_kernel<T>, dim3((unsigned)grid), dim3(NTHREADS), 0, stream,
                     (const T*)H, (const T*)W, (const T*)bias, mask, mask_dtype, (T*)reps,
                     argmax, reps_f32, (int)B, (int)S, (int)D, (int)V, (int)n_vt, P);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPARTON_OK : (int)e;
}

// Vocab tiles per workgroup: enough workgroups to keep every CU busy for several
// rounds (the dispatcher balances rows of different length), as few as that allows
// (each workgroup pays its prologue once). SPARTON_FWD_TILES_PER_GROUP (1..16)
// overrides the choice, for tests and tuning.
static int tiles_per_group(int64_t B, int64_t n_vt) {
  if (const char* env = getenv("SPARTON_FWD_TILES_PER_GROUP")) {
    const int p = atoi(env);
    if (p >= 1 && p <= MAX_P) return p;
  }
  const int64_t target = 256 * 6;  // CUs x rounds
  int P = 1;
  while (P < MAX_P && cdiv(n_vt, 2 * P) * B >= target) P *= 2;
  return P;
}

}  // namespace fwd
}  // namespace sparton

using namespace sparton;

extern "C" __attribute__((visibility("default"))) int sparton_fwd(
    const void* hidden, const void* weight, const void* bias, const void* mask,
    int mask_dtype, void* reps, int32_t* argmax, float* reps_f32, int64_t B, int64_t S,
    int64_t D, int64_t V, int dtype, void* stream) {
  if (B < 0 || S < 0 || D < 0 || V < 0) return SPARTON_EINVAL;
  if (dtype < SPARTON_F32 || dtype > SPARTON_F16) return SPARTON_EINVAL;
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
  // 32-bit sizes inside the kernel; per-tile byte offsets (256 rows) in 32 bits.
  if (B > INT32_MAX || S > INT32_MAX || V > INT32_MAX) return SPARTON_EUNSUPPORTED;
  if (S > fwd::MAX_CHUNKS * fwd::BM) return SPARTON_EUNSUPPORTED;
  if (D * esz * fwd::BM >= ((int64_t)1 << 32)) return SPARTON_EUNSUPPORTED;
  if (cdiv(V, fwd::BN) * B > INT32_MAX) return SPARTON_EUNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  const int P = fwd::tiles_per_group(B, cdiv(V, fwd::BN));
  switch (dtype) {
    case SPARTON_BF16:
      return fwd::launch<bf16>(hidden, weight, bias, mask, mask_dtype, reps, argmax, reps_f32, B, S, D, V, P, st);
    case SPARTON_F16:
      return fwd::launch<f16>(hidden, weight, bias, mask, mask_dtype, reps, argmax, reps_f32, B, S, D, V, P, st);
    default:
      return fwd::launch<float>(hidden, weight, bias, mask, mask_dtype, reps, argmax, reps_f32, B, S, D, V, P, st);
  }
}
