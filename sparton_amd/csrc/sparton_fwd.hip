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
// Positions whose whole 32-row MFMA block is masked out are skipped (no loads, no
// MFMA): they would contribute x = 0, which never beats the initial 0.

#include "sparton_common.h"

namespace sparton {
namespace fwd {

constexpr int BM = 256;              // sequence positions per chunk
constexpr int BN = 256;              // vocab columns per workgroup
constexpr int WAVES_M = 2;           // waves along M (sequence)
constexpr int WAVES_N = 4;           // waves along N (vocab)
constexpr int NTHREADS = 64 * WAVES_M * WAVES_N;
constexpr int MBLK = BM / 32;        // 32-row MFMA blocks per chunk (8)
constexpr int MB_PER_WAVE = MBLK / WAVES_M;        // 4, interleaved: wm, wm+2, ...
constexpr int NB_PER_WAVE = BN / WAVES_N / 32;     // 2
constexpr int SLAB = 128;            // bytes of K per row per pipeline stage
constexpr int ROW = SLAB + 16;       // padded LDS row pitch (conflict-free b128 reads)
constexpr int CHUNKS = SLAB / 16;    // 16-byte chunks per row slab
constexpr int ROWS_PER_PASS = NTHREADS / CHUNKS;   // 64 rows loaded per pass
constexpr int A_PASSES = BM / ROWS_PER_PASS;       // 4
constexpr int B_PASSES = BN / ROWS_PER_PASS;       // 4
constexpr int GROUP_V = 4;           // vocab tiles per scheduling group (L2 reuse)

struct Smem {
  uint8_t a[2][BM * ROW];
  uint8_t b[2][BN * ROW];
  float maskf[BM];
  int blockflag[MBLK];
};

// One MFMA "step" consumes 16 bytes of A and B per lane.
template <typename T> struct Mfma;
template <> struct Mfma<bf16> {
  static __device__ __forceinline__ void run(const u32x4& a, const u32x4& b, f32x16& c) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma<f16> {
  static __device__ __forceinline__ void run(const u32x4& a, const u32x4& b, f32x16& c) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                               __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma<float> {
  // 4 floats per lane = four K=2 steps. Lane half h supplies k = 16h + 4p + j for
  // A and B alike, so every k of the slab is paired once.
  static __device__ __forceinline__ void run(const u32x4& a, const u32x4& b, f32x16& c) {
    // __uint_as_float on the element value: a bit_cast of a vector-element lvalue
    // would read element 0 every time.
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

  const int nk = (int)cdiv((int64_t)D * sizeof(T), SLAB);
  const int64_t hrow0 = (int64_t)b * S;

  float bcol[NB_PER_WAVE], best[NB_PER_WAVE];
  int bidx[NB_PER_WAVE];
#pragma unroll
  for (int nb = 0; nb < NB_PER_WAVE; ++nb) {
    const int col = v0 + wn * 64 + nb * 32 + l32;
    bcol[nb] = (bias != nullptr && col < V) ? to_f32(bias[col]) : 0.0f;
    best[nb] = 0.0f;
    bidx[nb] = 0;
  }

  // Loader coordinates: each thread moves one 16-byte chunk of 4 A rows and 4 B rows.
  const int ld_c = tid % CHUNKS, ld_r = tid / CHUNKS;

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
    uint32_t wfl = 0;
#pragma unroll
    for (int j = 0; j < MB_PER_WAVE; ++j) wfl |= ((fl >> (wm + WAVES_M * j)) & 1u) << j;

    f32x16 acc[MB_PER_WAVE][NB_PER_WAVE];
#pragma unroll
    for (int j = 0; j < MB_PER_WAVE; ++j)
#pragma unroll
      for (int nb = 0; nb < NB_PER_WAVE; ++nb) acc[j][nb] = f32x16{};

    u32x4 ra[A_PASSES], rb[B_PASSES];
    auto load_slab = [&](int kt) {
      const int k = (kt * SLAB + ld_c * 16) / (int)sizeof(T);
      const bool kin = k < D;
#pragma unroll
      for (int i = 0; i < A_PASSES; ++i) {
        const int row = ld_r + i * ROWS_PER_PASS;
        const int s = s0 + row;
        const bool ok = kin && s < S && ((fl >> (row / 32)) & 1u);
        ra[i] = ok ? *(const u32x4*)(H + (hrow0 + s) * D + k) : u32x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int i = 0; i < B_PASSES; ++i) {
        const int row = ld_r + i * ROWS_PER_PASS;
        const int v = v0 + row;
        const bool ok = kin && v < V;
        rb[i] = ok ? *(const u32x4*)(W + (int64_t)v * D + k) : u32x4{0, 0, 0, 0};
      }
    };
    auto store_slab = [&](int buf) {
#pragma unroll
      for (int i = 0; i < A_PASSES; ++i)
        *(u32x4*)(sm.a[buf] + (ld_r + i * ROWS_PER_PASS) * ROW + ld_c * 16) = ra[i];
#pragma unroll
      for (int i = 0; i < B_PASSES; ++i)
        *(u32x4*)(sm.b[buf] + (ld_r + i * ROWS_PER_PASS) * ROW + ld_c * 16) = rb[i];
    };

    load_slab(0);
    store_slab(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < nk) load_slab(kt + 1);
      const uint8_t* abuf = sm.a[cur];
      const uint8_t* bbuf = sm.b[cur];
#pragma unroll
      for (int p = 0; p < SLAB / 32; ++p) {
        const int koff = h * (SLAB / 2) + p * 16;
        u32x4 bf[NB_PER_WAVE];
#pragma unroll
        for (int nb = 0; nb < NB_PER_WAVE; ++nb)
          bf[nb] = *(const u32x4*)(bbuf + (wn * 64 + nb * 32 + l32) * ROW + koff);
#pragma unroll
        for (int j = 0; j < MB_PER_WAVE; ++j) {
          if ((wfl >> j) & 1u) {
            const int row = (wm + WAVES_M * j) * 32 + l32;
            const u32x4 af = *(const u32x4*)(abuf + row * ROW + koff);
#pragma unroll
            for (int nb = 0; nb < NB_PER_WAVE; ++nb) Mfma<T>::run(af, bf[nb], acc[j][nb]);
          }
        }
      }
      if (kt + 1 < nk) store_slab(cur ^ 1);
      __syncthreads();
    }

    // Epilogue: 32x32 accumulator layout -- lane holds column l32, and for register
    // i the row 8*(i/4) + 4*h + (i%4). Rows rise with i, blocks rise with j, chunks
    // rise with s0, so a strict '>' keeps the lowest s within the lane.
#pragma unroll
    for (int j = 0; j < MB_PER_WAVE; ++j) {
      if ((wfl >> j) & 1u) {
        const int rbase = (wm + WAVES_M * j) * 32 + 4 * h;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 m4 = *(const f32x4*)(&sm.maskf[rbase + 8 * q]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int i = q * 4 + e;
            const int s = s0 + rbase + 8 * q + e;
#pragma unroll
            for (int nb = 0; nb < NB_PER_WAVE; ++nb) {
              const float x = (acc[j][nb][i] + bcol[nb]) * m4[e];
              if (x > best[nb]) { best[nb] = x; bidx[nb] = s; }
            }
          }
        }
      }
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
  float* red_v = (float*)sm.a[0];
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
