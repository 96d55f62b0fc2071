// Q8_0 skinny GEMM on gfx950: Y[M][N] f32 = X[M][K] f16 . dequant(W)^T, W in GGUF Q8_0 blocks.
//
// The reference has no Q8_0 kernel (src/codegen_hip.cpp:87-88 refuses int8); this is new.
// Weight layout: N rows, each K/32 blocks of 34 bytes {binary16 d (little endian), int8 q[32]}.
// Dequantised value w = float(d) * float(q) is exact in binary32 (11 + 7 significant bits).
//
// One v_mfma_f32_16x16x32_f16 covers exactly one block of 16 weight rows against 16 activation
// rows: A = the block's quants as f16 (integers in [-128, 127] are exact in binary16), B = the
// matching 32 activations. The MFMA sums q*x with products exact and an f32 accumulator; the
// block scale then multiplies that block sum in f32 and the result is accumulated in f32:
//   y[m][n] = sum_b float(d[n][b]) * (sum_{i<32} q[n][b][i] * x[m][32b+i])
// i.e. the dequantised weight d*q enters as the exact product of its two factors.
//
// Memory path: a block pair is 68 bytes, so every pair starts 4-byte aligned; lanes read the
// quants of both blocks with aligned dword loads and realign the even block's (2-byte shifted)
// bytes with a funnel shift. Each lane converts 8 quants to f16 with the 1024-bias trick
// (0x6400 | (q ^ 0x80) is the binary16 value 1024 + q + 128; subtracting 1152 is exact). The
// scales of the 16 rows arrive in lanes 0-15 (even block) and 48-63 (odd block) as a side
// effect of those loads and are moved to the lanes that hold each row's outputs with ds_bpermute.
//
// K must be a multiple of 64 (whole block pairs per row).
// Work split: a workgroup owns 16 weight rows (and 16 activation rows per grid.y); its WAVES
// wavefronts split the K blocks and fold their 16x16 partials in LDS in wavefront order
// (deterministic). Rows past N and activation rows past M are masked, never read.
#include "../launch.hpp"
#include "../variants.hpp"
#include "common.hpp"

namespace uk::kern {

typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));

// Four int8 quants packed in a dword -> four binary16 values (exact).
__device__ __forceinline__ u32x2 q4_to_f16(uint32_t dw) {
  const uint32_t u = dw ^ 0x80808080u;  // q + 128 as unsigned bytes
  const uint32_t lo = (u & 0xffu) | ((u & 0xff00u) << 8) | 0x64006400u;
  const uint32_t hi = ((u >> 16) & 0xffu) | ((u >> 8) & 0xff0000u) | 0x64006400u;
  const f16x2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  const f16x2v l = __builtin_bit_cast(f16x2v, lo) - bias;
  const f16x2v h = __builtin_bit_cast(f16x2v, hi) - bias;
  return u32x2{__builtin_bit_cast(uint32_t, l), __builtin_bit_cast(uint32_t, h)};
}

__device__ __forceinline__ f16x8 q8_to_f16x8(uint32_t lo_dw, uint32_t hi_dw) {
  const u32x2 a = q4_to_f16(lo_dw), b = q4_to_f16(hi_dw);
  return __builtin_bit_cast(f16x8, u32x4{a.x, a.y, b.x, b.y});
}

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xffffu));
}

template <int WAVES>
__global__ void __launch_bounds__(WAVES * 64)
    q8_0_gemm_kernel(const _Float16* __restrict__ X, const uint8_t* __restrict__ Wq, float* __restrict__ Y, int M,
                     int N, int K) {
  __shared__ float red[WAVES][256];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int i = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16, m0 = blockIdx.y * 16;
  const int nblk = K >> 5, npairs = nblk >> 1;
  const int per = (npairs + WAVES - 1) / WAVES;
  const int pb = wave * per;
  const int pe = (pb + per) < npairs ? (pb + per) : npairs;

  const int row = n0 + i;
  const bool rok = row < N;
  const uint8_t* wrow = Wq + (int64_t)(rok ? row : 0) * nblk * 34;
  const int m = m0 + i;
  const bool mok = m < M;
  const _Float16* xrow = X + (int64_t)(mok ? m : 0) * K + 8 * g;

  f32x4 yacc = f32x4{0.f, 0.f, 0.f, 0.f};
  const f32x4 zero = f32x4{0.f, 0.f, 0.f, 0.f};
  // The wavefront's pairs are processed in chunks of kU: all loads of a chunk are issued
  // before any of its math, so a wavefront keeps kU * 16 rows * 68 B in flight.
  constexpr int kU = 4;
  for (int pc = pb; pc < pe; pc += kU) {
    uint32_t a0[kU], a1[kU], a2[kU], b0[kU], b1[kU];
    f16x8 xa[kU], xb[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int p = pc + u;
      const bool ok = rok && p < pe;
      const uint32_t* pw = reinterpret_cast<const uint32_t*>(wrow + 68 * (ok ? p : 0));
      a0[u] = pw[2 * g];
      a1[u] = pw[2 * g + 1];
      a2[u] = pw[2 * g + 2];  // dword 8 also carries the odd block's scale (lanes g = 3)
      b0[u] = pw[9 + 2 * g];
      b1[u] = pw[10 + 2 * g];
      if (!ok) a0[u] = a1[u] = a2[u] = b0[u] = b1[u] = 0;
      const bool xok = mok && p < pe;
      const _Float16* xp = xrow + 64 * (xok ? p : 0);
      xa[u] = *reinterpret_cast<const f16x8*>(xp);
      xb[u] = *reinterpret_cast<const f16x8*>(xp + 32);
      if (!xok) xa[u] = xb[u] = f16x8{};
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      // Even block: quant bytes 2..9 of this lane's 12-byte window; odd block: aligned.
      const f16x8 qa = q8_to_f16x8(__builtin_amdgcn_alignbyte(a1[u], a0[u], 2),
                                   __builtin_amdgcn_alignbyte(a2[u], a1[u], 2));
      const f16x8 qb = q8_to_f16x8(b0[u], b1[u]);
      const f32x4 s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa, xa[u], zero, 0, 0, 0);
      const f32x4 s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(qb, xb[u], zero, 0, 0, 0);
      // Scales: d_even of row r sits in the low half of a0 in lane r (g = 0); d_odd of row r in
      // the high half of a2 in lane 48 + r (g = 3). This lane's outputs are rows 4g + {0..3}.
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int src = 4 * g + r;
        const float d0 = half_bits_to_float((uint32_t)__shfl((int)a0[u], src));
        const float d1 = half_bits_to_float((uint32_t)__shfl((int)a2[u], 48 + src) >> 16);
        yacc[r] = fmaf(d0, s0[r], yacc[r]);
        yacc[r] = fmaf(d1, s1[r], yacc[r]);
      }
    }
  }

  // Fold the wavefronts' partials in wavefront order.
#pragma unroll
  for (int r = 0; r < 4; ++r) red[wave][lane * 4 + r] = yacc[r];
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float s = red[0][lane * 4 + r];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) s += red[w][lane * 4 + r];
    const int n = n0 + 4 * g + r;  // MFMA output row = weight row
    if (n < N && mok) Y[(int64_t)m * N + n] = s;
  }
}

}  // namespace uk::kern

namespace uk {

namespace {
template <int WAVES>
hipError_t q8_go(const void* X, const void* Wq, float* Y, int64_t M, int64_t N, int64_t K, hipStream_t s) {
  const dim3 grid((unsigned)((N + 15) / 16), (unsigned)((M + 15) / 16));
  hipLaunchKernelGGL((kern::q8_0_gemm_kernel<WAVES>), grid, dim3(WAVES * 64), 0, s, static_cast<const _Float16*>(X),
                     static_cast<const uint8_t*>(Wq), Y, (int)M, (int)N, (int)K);
  return hipGetLastError();
}
}  // namespace

hipError_t launch_q8_gemm(const Plan& p, const void* X, const void* Wq, float* Y, int64_t M, int64_t N, int64_t K,
                          hipStream_t s) {
  if (p.family != Family::Q8Gemm || p.variant < 0 || p.variant >= kNumQ8Variants) return hipErrorInvalidValue;
  // Whole block pairs per row keep every row (34*K/32 bytes) and pair 4-byte aligned.
  if (M <= 0 || N <= 0 || K <= 0 || K % 64) return hipErrorInvalidValue;
  // Row byte offsets and element indices are formed in 32/64-bit as above; grid limits.
  if ((N + 15) / 16 > INT32_MAX || (M + 15) / 16 > 65535 || K > INT32_MAX / 2 || N > INT32_MAX) return hipErrorInvalidValue;
  // Activation rows are read as 16-byte vectors at 2*(m*K + 32b + 8g) bytes; rows of the weight
  // stream are 34*K/32 bytes, pairs 68 bytes: both need 4-byte alignment, X 16-byte.
  if ((((uintptr_t)X) & 15) || (((uintptr_t)Wq) & 3) || (((uintptr_t)Y) & 3)) return hipErrorInvalidValue;
  switch (kQ8Variants[p.variant].waves) {
    case 4: return q8_go<4>(X, Wq, Y, M, N, K, s);
    case 8: return q8_go<8>(X, Wq, Y, M, N, K, s);
    case 16: return q8_go<16>(X, Wq, Y, M, N, K, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace uk
