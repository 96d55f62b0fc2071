// Matrix-core ceiling probe: one wavefront per SIMD issues nothing but independent
// v_mfma_f32_32x32x16_f16 (four accumulator chains, operands fixed in registers, no memory
// traffic), and records its shader-clock cycles (s_memtime) and wall ticks (s_memrealtime, a
// constant 100 MHz) around the loop. (With eight 16x16x32 chains of f32x4 accumulators in a
// loop the compiler rotates the accumulators through moves every iteration; the 16-register
// accumulators of the 32x32x16 form stay in place.) Over a few milliseconds of load this gives the rate the part
// sustains for f16 MFMAs, the shader clock it settles at, and the issue cycles per MFMA: the
// ceiling the GEMM's efficiency is judged against (the dense-peak figure assumes 2.4 GHz).
#include "../launch.hpp"
#include "common.hpp"

namespace uk::kern {

// Pseudo-random binary16 value in [-1, 1) from a 32-bit hash (operand bits toggle like the
// BASELINE GEMM's uniform inputs, which matters for the part's power draw).
__device__ __forceinline__ _Float16 probe_half(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352dU;
  x ^= x >> 15;
  x *= 0x846ca68bU;
  x ^= x >> 16;
  return (_Float16)((float)(x >> 8) * (1.0f / 8388608.0f) - 1.0f);
}

__global__ void __launch_bounds__(256) mfma_probe_kernel(int iters, unsigned long long* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const uint32_t seed = (blockIdx.x * 256u + threadIdx.x) * 256u;
  // A different operand pair per chain, so consecutive MFMAs switch operands as a GEMM's do.
  f16x8 a[kProbeChains], b[kProbeChains];
#pragma unroll
  for (int j = 0; j < kProbeChains; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a[j][i] = probe_half(seed + 64u * j + i);
      b[j][i] = probe_half(seed + 64u * j + 8 + i);
    }
  f32x16 acc[kProbeChains];
#pragma unroll
  for (int j = 0; j < kProbeChains; ++j) {
    acc[j] = f32x16{};
    acc[j][0] = float(j);  // distinct chains: equal ones could be merged into one
  }
  const unsigned long long c0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < kProbeChains; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[j], b[j], acc[j], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kProbeChains; ++j) s += acc[j][0];
  const unsigned long long c1 = __builtin_amdgcn_s_memtime();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (lane == 0) {
    out[3 * w] = c1 - c0;
    out[3 * w + 1] = r1 - r0;
    out[3 * w + 2] = (unsigned long long)(s != s);  // keeps the sums live; 0 unless NaN
  }
}

}  // namespace uk::kern

namespace uk {

hipError_t launch_mfma_probe(int workgroups, int iters, unsigned long long* out, hipStream_t s) {
  if (workgroups <= 0 || iters <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(kern::mfma_probe_kernel, dim3((unsigned)workgroups), dim3(256), 0, s, iters, out);
  return hipGetLastError();
}

}  // namespace uk
