// SpartonHead forward on gfx950: one kernel, MFMA mainloop + fused reduction epilogue.
//
// A workgroup owns one batch row b and a tile of BN vocab columns, and sweeps the
// sequence in chunks of BM positions. For each chunk it computes the BM x BN logit
// tile  H[b, s0:s0+BM, :] . W[v0:v0+BN, :]^T  with bf16/fp16 (or fp32) MFMA, K = D
// streamed through double-buffered LDS, then folds the tile into a running
// (max, argmax) per column in registers:
//     x = (acc + bias[v]) * mask[b, s];  take x if x > best (strict, s ascending)
// so the [B,S,V] logits never reach HBM. At the end the per-column winners of the
// two M-waves are merged (larger value, ties -> lower s) and the workgroup writes
// reps[b, v] = log1p(max(0, best)) and argmax[b, v].
//
// Reference semantics followed (src/sparton/sparton_kernel.py):
//   bias added to the GEMM output            :209-210, :245
//   logits multiplied by mask                :147
//   running max initialised to 0, idx to 0   :112-114
//   lowest s wins ties (tl.argmax + strict >) :151-156
//   reps = log(1 + relu(max))                :159-161 (log1p here)
//
// Data movement: K slabs of 128 bytes per row go straight from global memory into
// LDS (global_load_lds_dwordx4, no VGPR staging). LDS rows are 128 bytes with the
// 16-byte chunk index XOR-swizzled by f(row) = (row & 7) ^ ((row >> 3) & 1). The MFMA
// operand reads are ds_read_b128 of 32 consecutive rows at one logical chunk; gfx950's
// 64 banks serve 16 lanes (256 bytes) per cycle, and over any 16 aligned rows the
// pairs (row & 1, chunk ^ f(row)) are all distinct, so each read is conflict-free
// (and so is any 8-lane group, since f is distinct over 8 aligned rows).
// A K tail (D not a multiple of the slab) is staged through VGPRs with zero fill.
//
// Skipping: 32-row blocks whose mask is all zero contribute x = 0, which never beats
// the initial 0, so a wave only multiplies its blocks up to the last active one and
// A rows past that block are not loaded.

#include "sparton_common.h"

namespace sparton {
namespace fwd {

constexpr int BM = 256;              // sequence positions per chunk
constexpr int BN = 256;              // vocab columns per workgroup
constexpr int WAVES_M = 2;           // waves along M (sequence)
constexpr int WAVES_N = 4;           // waves along N (vocab)
constexpr int NWAVES = WAVES_M * WAVES_N;
constexpr int NTHREADS = 64 * NWAVES;
constexpr int MBLK = BM / 32;        // 32-row MFMA blocks per chunk (8)
constexpr int MB_PER_WAVE = MBLK / WAVES_M;        // 4, interleaved: wm, wm+2, ...
constexpr int NB_PER_WAVE = BN / WAVES_N / 32;     // 2
constexpr int SLAB = 128;            // bytes of K per row per pipeline stage
constexpr int CHUNKS = SLAB / 16;    // 16-byte chunks per row slab (8)
constexpr int ROWS_PER_LOAD = 64 / CHUNKS;          // rows one wave-wide load covers (8)
constexpr int A_LOADS = BM / ROWS_PER_LOAD / NWAVES;  // wave-wide loads per slab for A (4)
constexpr int B_LOADS = BN / ROWS_PER_LOAD / NWAVES;  // and for B (4)
constexpr int GROUP_V = 4;           // vocab tiles per scheduling group (L2 reuse)

struct Smem {
  u32x4 a[2][BM * CHUNKS];   // [stage][row * 8 + (chunk ^ f(row))]
  u32x4 b[2][BN * CHUNKS];
  float maskf[BM];
  int blockflag[MBLK];
};

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ int swz_key(int row) { return (row & 7) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int swz(int row, int chunk) { return row * CHUNKS + (chunk ^ swz_key(row)); }

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

// Map the hardware workgroup id to (b, vocab tile). Workgroups are dispatched
// round-robin over the 8 XCDs; first make ids that share an XCD consecutive, then
// walk groups of GROUP_V vocab tiles x all batch rows so the workgroups resident on
// one XCD at a time share a few W tiles and a few H rows in that XCD's L2.
__device__ __forceinline__ void tile_of(int wg, int grid, int B, int n_vt, int* b, int* vt) {
  const int xcd = wg & 7, local = wg >> 3, q = grid >> 3, r = grid & 7;
  const int lin = (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + local;
  const int group = lin / (GROUP_V * B);
  const int rem = lin - group * GROUP_V * B;
  const int gv = min(GROUP_V, n_vt - group * GROUP_V);
  *b = rem / gv;
  *vt = group * GROUP_V + rem % gv;
}

__device__ __forceinline__ void merge(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}

// Per-workgroup addressing of the direct loads. Every lane keeps one 32-bit byte
// offset per wave-wide load; the 64-bit bases are workgroup-uniform and advance by one
// slab per K step, so the loads use the SGPR-base + VGPR-offset form.
struct Loads {
  const char* a_base;   // H row (b, s0) at K = 0
  const char* b_base;   // W row v0 at K = 0
  uint32_t a_off[A_LOADS], b_off[B_LOADS];
  int a_groups;         // 8-row groups of A to load (rows past the last active block are skipped)
  int row_bytes;        // D * sizeof(T)
};

// Wave w, load i covers the 8-row group g = i * NWAVES + w; lane L lands at LDS chunk
// g*64 + L, i.e. row 8g + L/8, physical chunk L%8, which holds logical chunk (L%8) ^ f(row).
__device__ __forceinline__ void load_rows(int i, int wave, int lane, int* row, int* chunk) {
  const int g = i * NWAVES + wave;
  *row = g * ROWS_PER_LOAD + (lane >> 3);
  *chunk = (lane & 7) ^ swz_key(*row);
}

// Issue the direct global -> LDS copies of K slab kt into stage buf. In a tail slab
// (K past D in some chunks), those chunks re-read slab 0 (valid, finite data) and the
// W copies are zeroed afterwards by zero_tail(), so they add nothing.
__device__ __forceinline__ void issue_slab(Smem& sm, const Loads& L, int kt, bool tail, int buf,
                                           int wave, int lane) {
  const uint32_t kb = (uint32_t)kt * SLAB;
  const char* ab = L.a_base + (tail ? 0 : kb);
  const char* bb = L.b_base + (tail ? 0 : kb);
#pragma unroll
  for (int i = 0; i < A_LOADS; ++i) {
    const int g = i * NWAVES + wave;
    if (g < L.a_groups) {
      uint32_t off = L.a_off[i];
      if (tail) {
        int row, c;
        load_rows(i, wave, lane, &row, &c);
        off += (kb + c * 16 < (uint32_t)L.row_bytes) ? kb : 0;
      }
      __builtin_amdgcn_global_load_lds((const void*)(ab + off), (lds_void*)&sm.a[buf][g * 64], 16, 0, 0);
    }
  }
#pragma unroll
  for (int i = 0; i < B_LOADS; ++i) {
    const int g = i * NWAVES + wave;
    uint32_t off = L.b_off[i];
    if (tail) {
      int row, c;
      load_rows(i, wave, lane, &row, &c);
      off += (kb + c * 16 < (uint32_t)L.row_bytes) ? kb : 0;
    }
    __builtin_amdgcn_global_load_lds((const void*)(bb + off), (lds_void*)&sm.b[buf][g * 64], 16, 0, 0);
  }
}

// Zero the W chunks of tail slab kt that lie past D (run after its copies landed).
__device__ __forceinline__ void zero_tail(Smem& sm, const Loads& L, int kt, int buf, int wave, int lane) {
  const uint32_t kb = (uint32_t)kt * SLAB;
#pragma unroll
  for (int i = 0; i < B_LOADS; ++i) {
    int row, c;
    load_rows(i, wave, lane, &row, &c);
    if (kb + c * 16 >= (uint32_t)L.row_bytes)
      sm.b[buf][(i * NWAVES + wave) * 64 + lane] = u32x4{0, 0, 0, 0};
  }
}

// Wait for all of this thread's outstanding memory operations (the direct-to-LDS
// loads included), then the workgroup barrier.
__device__ __forceinline__ void drain_and_sync() {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

// Mainloop + epilogue of one sequence chunk for a wave with JM blocks to multiply.
template <typename T, int JM>
__device__ __forceinline__ void chunk(Smem& sm, const Loads& L, int s0, int nk, int nk_full,
                                      int wave, int lane, int wm, int wn, const float* bcol,
                                      float* best, int* bidx) {
  constexpr int JA = JM > 0 ? JM : 1;
  const int l32 = lane & 31, h = lane >> 5;
  f32x16 acc[JA][NB_PER_WAVE];
#pragma unroll
  for (int j = 0; j < JA; ++j)
#pragma unroll
    for (int nb = 0; nb < NB_PER_WAVE; ++nb)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[j][nb][i] = bcol[nb];

  issue_slab(sm, L, 0, nk_full == 0, 0, wave, lane);
  drain_and_sync();
  if (nk_full == 0) {
    zero_tail(sm, L, 0, 0, wave, lane);
    __syncthreads();
  }
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) issue_slab(sm, L, kt + 1, kt + 1 >= nk_full, cur ^ 1, wave, lane);
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
    if (kt + 1 < nk && kt + 1 >= nk_full) {
      zero_tail(sm, L, kt + 1, cur ^ 1, wave, lane);
      __syncthreads();
    }
  }

  // Epilogue: 32x32 accumulator layout -- lane holds column l32, and for register i
  // the row 8*(i/4) + 4*h + (i%4). Rows rise with i, blocks rise with j, chunks rise
  // with s0, so a strict '>' keeps the lowest s within the lane.
#pragma unroll
  for (int j = 0; j < JM; ++j) {
    const int rbase = (wm + WAVES_M * j) * 32 + 4 * h;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x4 m4 = *(const f32x4*)(&sm.maskf[rbase + 8 * q]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int s = s0 + rbase + 8 * q + e;
#pragma unroll
        for (int nb = 0; nb < NB_PER_WAVE; ++nb) {
          const float x = acc[j][nb][q * 4 + e] * m4[e];
          if (x > best[nb]) { best[nb] = x; bidx[nb] = s; }
        }
      }
    }
  }
}

template <typename T>
__global__ __launch_bounds__(NTHREADS, 1) void sparton_fwd_kernel(
    const T* __restrict__ H, const T* __restrict__ W, const T* __restrict__ bias,
    const void* __restrict__ mask, int mask_dtype, T* __restrict__ reps,
    int32_t* __restrict__ argmax, float* __restrict__ reps_f32, int B, int S, int D, int V,
    int n_vt) {
  __shared__ Smem sm;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int l32 = lane & 31, h = lane >> 5;

  int b, vt;
  tile_of(blockIdx.x, gridDim.x, B, n_vt, &b, &vt);
  const int v0 = vt * BN;
  const int64_t hrow0 = (int64_t)b * S;
  const int slab_elems = SLAB / (int)sizeof(T);
  const int nk = (int)cdiv(D, slab_elems);
  const int nk_full = D / slab_elems;

  Loads L;
  L.row_bytes = D * (int)sizeof(T);
  L.b_base = (const char*)(W + (int64_t)v0 * D);
#pragma unroll
  for (int i = 0; i < B_LOADS; ++i) {
    int row, c;
    load_rows(i, wave, lane, &row, &c);
    const int vr = min(v0 + row, V - 1) - v0;  // columns past V are never stored
    L.b_off[i] = (uint32_t)vr * (uint32_t)L.row_bytes + c * 16;
  }

  float bcol[NB_PER_WAVE], best[NB_PER_WAVE];
  int bidx[NB_PER_WAVE];
#pragma unroll
  for (int nb = 0; nb < NB_PER_WAVE; ++nb) {
    const int col = v0 + wn * 64 + nb * 32 + l32;
    bcol[nb] = (bias != nullptr && col < V) ? to_f32(bias[col]) : 0.0f;
    best[nb] = 0.0f;
    bidx[nb] = 0;
  }

  for (int s0 = 0; s0 < S; s0 += BM) {
    __syncthreads();  // previous chunk's epilogue is done with maskf
    if (tid < BM) {
      const int s = s0 + tid;
      const float mv = s < S ? load_mask(mask, mask_dtype, hrow0 + s) : 0.0f;
      sm.maskf[tid] = mv;
      const uint64_t bal = __ballot(mv != 0.0f);
      if (lane == 0) {
        sm.blockflag[2 * wave] = (bal & 0xffffffffull) != 0;
        sm.blockflag[2 * wave + 1] = (bal >> 32) != 0;
      }
    }
    __syncthreads();
    uint32_t fl = 0;
#pragma unroll
    for (int j = 0; j < MBLK; ++j) fl |= (uint32_t)(sm.blockflag[j] != 0) << j;
    fl = __builtin_amdgcn_readfirstlane(fl);
    if (fl == 0) continue;  // whole chunk masked: contributes nothing
    const int last_blk = 31 - __builtin_clz(fl);
    L.a_groups = (last_blk + 1) * (32 / ROWS_PER_LOAD);
    L.a_base = (const char*)(H + (hrow0 + s0) * D);
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      int row, c;
      load_rows(i, wave, lane, &row, &c);
      const int sr = min(s0 + row, S - 1) - s0;  // rows past S are masked out; any finite data will do
      L.a_off[i] = (uint32_t)sr * (uint32_t)L.row_bytes + c * 16;
    }
    // Blocks of this wave are wm, wm+2, ...: multiply those up to the last active
    // one (masked rows below it give x = 0 and cannot win).
    const int jm = last_blk < wm ? 0 : (last_blk - wm) / WAVES_M + 1;
    switch (jm) {
      case 0: chunk<T, 0>(sm, L, s0, nk, nk_full, wave, lane, wm, wn, bcol, best, bidx); break;
      case 1: chunk<T, 1>(sm, L, s0, nk, nk_full, wave, lane, wm, wn, bcol, best, bidx); break;
      case 2: chunk<T, 2>(sm, L, s0, nk, nk_full, wave, lane, wm, wn, bcol, best, bidx); break;
      case 3: chunk<T, 3>(sm, L, s0, nk, nk_full, wave, lane, wm, wn, bcol, best, bidx); break;
      default: chunk<T, 4>(sm, L, s0, nk, nk_full, wave, lane, wm, wn, bcol, best, bidx); break;
    }
  }

  // Lanes l and l^32 hold the same column (different rows): merge them.
#pragma unroll
  for (int nb = 0; nb < NB_PER_WAVE; ++nb) {
    const float ov = __shfl_xor(best[nb], 32);
    const int oi = __shfl_xor(bidx[nb], 32);
    merge(best[nb], bidx[nb], ov, oi);
  }
  __syncthreads();  // operand buffers are free: reuse them for the cross-wave merge
  float* red_v = (float*)&sm.a[0][0];
  int* red_i = (int*)(red_v + WAVES_M * BN);
  if (h == 0) {
#pragma unroll
    for (int nb = 0; nb < NB_PER_WAVE; ++nb) {
      const int col = wn * 64 + nb * 32 + l32;
      red_v[wm * BN + col] = best[nb];
      red_i[wm * BN + col] = bidx[nb];
    }
  }
  __syncthreads();
  if (tid < BN) {
    const int v = v0 + tid;
    if (v < V) {
      float bv = red_v[tid];
      int bi = red_i[tid];
#pragma unroll
      for (int w = 1; w < WAVES_M; ++w) merge(bv, bi, red_v[w * BN + tid], red_i[w * BN + tid]);
      const int64_t o = (int64_t)b * V + v;
      const float r = log1pf(bv);
      reps[o] = from_f32<T>(r);
      if (argmax != nullptr) argmax[o] = bi;
      if (reps_f32 != nullptr) reps_f32[o] = r;
    }
  }
}

template <typename T>
static int launch(const void* H, const void* W, const void* bias, const void* mask,
                  int mask_dtype, void* reps, int32_t* argmax, float* reps_f32, int64_t B,
                  int64_t S, int64_t D, int64_t V, hipStream_t stream) {
  const int64_t n_vt = cdiv(V, BN);
  const int64_t grid = n_vt * B;
  hipLaunchKernelGGL(sparton_fwd_kernel<T>, dim3((unsigned)grid), dim3(NTHREADS), 0, stream,
                     (const T*)H, (const T*)W, (const T*)bias, mask, mask_dtype, (T*)reps,
                     argmax, reps_f32, (int)B, (int)S, (int)D, (int)V, (int)n_vt);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPARTON_OK : (int)e;
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
  // 32-bit sizes inside the kernel; 64-bit element offsets.
  if (B > INT32_MAX || S > INT32_MAX || D > INT32_MAX || V > INT32_MAX) return SPARTON_EUNSUPPORTED;
  if (cdiv(V, fwd::BN) * B > INT32_MAX) return SPARTON_EUNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case SPARTON_BF16:
      return fwd::launch<bf16>(hidden, weight, bias, mask, mask_dtype, reps, argmax, reps_f32, B, S, D, V, st);
    case SPARTON_F16:
      return fwd::launch<f16>(hidden, weight, bias, mask, mask_dtype, reps, argmax, reps_f32, B, S, D, V, st);
    default:
      return fwd::launch<float>(hidden, weight, bias, mask, mask_dtype, reps, argmax, reps_f32, B, S, D, V, st);
  }
}
