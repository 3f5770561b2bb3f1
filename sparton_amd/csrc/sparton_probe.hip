// Measurement probe: the bf16/fp16 MFMA throughput every CU of the GPU sustains at once
// on data-like operands, and the shader clock it runs at. It bounds what the forward's
// main kernel (v_mfma_f32_32x32x16_*) can reach on this GPU: under a full MFMA load the
// chip is power-limited, so its sustained rate on random operands is well below the
// nominal 2.5 PFLOP/s (a clock of ~2.4 GHz), which only constant operands approach.
//
// One workgroup of 4 waves per CU; each wave runs `iters` rounds of 16 independent
// 32x32x16 MFMAs (a 4 x 4 block of accumulators, as the forward's compute waves keep)
// whose A and B registers hold random 16-bit values (a hash of lane and slot: random
// sign and mantissa, small normal exponents, like the head's data). Each workgroup
// records its shader-clock cycles (s_memtime) and 100 MHz real time (s_memrealtime)
// between two barriers.
#include "sparton_common.h"

namespace sparton {
namespace probe {

__device__ __forceinline__ uint32_t hash32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// Two random normal 16-bit values: random sign and mantissa, exponent 2^-8 .. 2^-5 (bf16)
// or 2^-4 .. 2^-1 (fp16).
__device__ __forceinline__ uint32_t rand_pair(uint32_t seed, bool is_bf16) {
  const uint32_t h = hash32(seed);
  uint32_t lo, hi;
  if (is_bf16) {
    lo = (h & 0x807fu) | ((119u + ((h >> 8) & 3u)) << 7);
    hi = ((h >> 16) & 0x807fu) | ((119u + ((h >> 24) & 3u)) << 7);
  } else {
    lo = (h & 0x83ffu) | ((11u + ((h >> 10) & 3u)) << 10);
    hi = ((h >> 16) & 0x83ffu) | ((11u + ((h >> 26) & 3u)) << 10);
  }
  return lo | (hi << 16);
}

template <bool BF16>
__global__ __launch_bounds__(256, 1) void mfma_probe_kernel(int iters, float* __restrict__ out,
                                                           long long* __restrict__ clk) {
  const int tid = threadIdx.x;
  const uint32_t seed = (blockIdx.x * 256u + tid) * 64u;
  u32x4 a[4], b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      a[i][j] = rand_pair(seed + i * 4 + j, BF16);
      b[i][j] = rand_pair(seed + 32 + i * 4 + j, BF16);
    }
  f32x16 acc[16];
#pragma unroll
  for (int k = 0; k < 16; ++k)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[k][e] = 0.0f;
  __syncthreads();
  const long long c0 = __builtin_amdgcn_s_memtime();
  const long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        if (BF16)
          acc[rb * 4 + cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8, a[rb]), __builtin_bit_cast(bf16x8, b[cb]), acc[rb * 4 + cb], 0, 0, 0);
        else
          acc[rb * 4 + cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
              __builtin_bit_cast(f16x8, a[rb]), __builtin_bit_cast(f16x8, b[cb]), acc[rb * 4 + cb], 0, 0, 0);
      }
  }
  __syncthreads();
  const long long c1 = __builtin_amdgcn_s_memtime();
  const long long r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < 16; ++k)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += acc[k][e];
  out[blockIdx.x * 256 + tid] = s;  // keeps the MFMAs live
  if (tid == 0) {
    clk[blockIdx.x * 2] = c1 - c0;
    clk[blockIdx.x * 2 + 1] = r1 - r0;
  }
}

}  // namespace probe
}  // namespace sparton

using namespace sparton;

extern "C" __attribute__((visibility("default"))) int sparton_mfma_probe(
    int dtype, int grid, int iters, float* out, long long* clk, void* stream) {
  if ((dtype != SPARTON_BF16 && dtype != SPARTON_F16) || grid <= 0 || iters <= 0 ||
      out == nullptr || clk == nullptr)
    return SPARTON_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == SPARTON_BF16)
    hipLaunchKernelGGL(probe::mfma_probe_kernel<true>, dim3((unsigned)grid), dim3(256), 0, st, iters, out, clk);
  else
    hipLaunchKernelGGL(probe::mfma_probe_kernel<false>, dim3((unsigned)grid), dim3(256), 0, st, iters, out, clk);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPARTON_OK : (int)e;
}
