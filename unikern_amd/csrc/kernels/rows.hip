// Row family on gfx950: row-sum, RMSNorm and softmax over X[L][C] f32.
//
// Replaces the reference's one-thread-per-row kernels (src/codegen_hip.cpp:1985-1996 softmax,
// :2154-2164 rmsnorm) and its two-pass scalar reduce (:818-833, used here per row).
// Design: tpr threads own one row; each thread keeps nv float4 of it in registers, loaded
// with 128-bit coalesced loads (for a fixed register index the wavefront reads 1 KiB of
// contiguous HBM). Reductions run inside the wavefront with DPP/swizzle/readlane; when a row
// spans several wavefronts, one LDS slot per wavefront carries the partial and every thread
// folds the slots in wavefront order (deterministic). X is read once and Y written once, so
// the kernels are HBM-bound: algorithmic bytes are read(X) + write(Y) (+ W for RMSNorm).
//
// Semantics kept from the reference CPU loops: rmsnorm y = (x * rms) * W with
// rms = 1/sqrt(sum(x^2)/C + eps) (correctly rounded divide and sqrt); softmax
// y = exp(x - max) / sum(exp(x - max)), here as 2^((x - max) log2 e) * (1 / sum) on v_exp_f32
// (exp_sub below): within about 2e-6 of the reference wherever the 1e-5 relative gate can see an
// element, and a fifth of the vector instructions of a libm exp and a divide per element.
#include <math.h>

#include <mutex>

#include "../launch.hpp"
#include "../variants.hpp"
#include "common.hpp"

namespace uk::kern {

// Loads and stores of the row stream; NT adds the non-temporal hint.
template <bool NT>
__device__ __forceinline__ f32x4 ld4(const f32x4* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}
template <bool NT>
__device__ __forceinline__ void st4(f32x4* p, f32x4 v) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// e^(x - m) for the softmax numerators of a row with maximum m: 2^((x - m) log2 e) as a subtract,
// a multiply by the binary32 log2(e) and v_exp_f32. Error in the exponent t = (x - m) log2 e: the
// subtract's rounding (at most |x - m| 2^-24, none when x is within a factor of two of m), the
// product's (|t| 2^-24) and the binary32 log2(e)'s (|t| 2^-27). Only elements with
// e^(x - m) >= 1e-6 * sum (so t >= -20) can move the 1e-5 relative gate, whose denominator is
// max(|r|, 1e-6): for them the numerator is within 20 (2^-23 + 2^-27) ln 2 + 2^-23 of e^(x - m),
// about 1.9e-6 relative (measured: 8.8e-7 against binary64). It holds for any finite maximum;
// padding (-inf) gives 0, and a row holding +inf or only -inf gives NaN, as the reference's
// exp(x - max) does. (A libm expf and an IEEE divide per element cost twice the vector
// instructions, which did not hide behind the row stream.)
constexpr float kLog2eF = 1.44269502f;  // log2(e) rounded to binary32
__device__ __forceinline__ float exp_sub(float x, float m) { return __builtin_amdgcn_exp2f((x - m) * kLog2eF); }

// TPR threads own one row at a time and each keeps NV float4 of it in registers; a workgroup
// walks RPB rows (RPB > 1: the next row's loads are issued before the current row's reduction,
// so the reduction's latency hides behind HBM traffic). GS (one wavefront per row, RPB = 1): the
// workgroup's four rows store together after one barrier, and a gain vector (RMSNorm's W,
// channelscale's S, softmax's unit gain) is staged in LDS once per workgroup, after the row's
// loads, by a loop whose every load is waited for before the next is issued. That staging is
// part of what makes the form fast, and not only for its gain reads: in standalone copies at
// 4096 x 4096 the same softmax took 23.5 us without it and 21.8 us with it (a table of ones), and
// neither one extra load, four loads under one wait, nor pauses of 0.25-4 us before or after the
// compute reproduced the gain. RMSNorm runs 7% faster in this form than in the two-row walk (and
// faster than a plain copy of one row per workgroup). Row-sum runs slower in it. Rows beyond L
// are masked, never skipped: every thread reaches every barrier.
// FULL (grouped-store launches whose rows all exist and are exactly TPR NV 4 floats long, every
// row of a 4096 x 4096 launch): loads and stores carry no guards. The guards compile to an
// exec-masked branch around each load and store; at 4096 x 4096 on one box the FULL instantiation
// of the grouped-store softmax ran 21.77-21.84 against 22.13-22.27 us, RMSNorm 21.77-21.83 against
// 22.29-22.34 us and channelscale 21.69-21.70 against 22.39-22.47 us, with the same bits. The
// 512-thread row-sum without guards ran 4% slower (11.5 against 11.1 us), so only the grouped-store
// launches take it. (Both paths in one kernel, chosen by a uniform branch, gained nothing.)
template <int TPR, int NV, int OP, bool NT, int RPB, bool GS = false, bool FULL = false>
__global__ void __launch_bounds__(TPR < 256 ? 256 : TPR)
    rows_kernel(const float* __restrict__ X, const float* __restrict__ Wg, float* __restrict__ Y, int L, int C,
                float eps) {
  static_assert(!GS || (TPR == 64 && RPB == 1), "grouped stores: one wavefront per row, one row per wavefront");
  // All arguments in scalar registers before anything else (one wait for their loads, not one per
  // argument between the computations that need them).
  asm volatile("" ::"s"(X), "s"(Wg), "s"(Y), "s"(L), "s"(C), "s"(eps));
  constexpr int WG = TPR < 256 ? 256 : TPR;
  constexpr int RPW = WG / TPR;  // rows per workgroup at a time
  constexpr int WPR = TPR / 64;  // wavefronts per row
  // Reduction slots, alternating between consecutive rows: a fast wavefront may publish row
  // k+1's partial while a slow one still reads row k's.
  __shared__ float red0[2][WG / 64];
  __shared__ float red1[2][WG / 64];
  // OP 3 (channelscale) scales by S[c] the way RMSNorm applies its gain, with no row statistic;
  // softmax takes a gain in the grouped-store form only (the launcher passes ones: x * 1 is x).
  constexpr bool kGain = OP == 1 || OP == 3 || (OP == 2 && GS);
  __shared__ f32x4 gain_lds[(kGain && GS) ? TPR * NV : 1];

  const int tid = threadIdx.x;
  const int rloc = tid / TPR;
  const int t = tid % TPR;
  const int wave = tid >> 6;
  const int C4 = C >> 2;
  auto row_of = [&](int k) -> int64_t { return ((int64_t)blockIdx.x * RPB + k) * RPW + rloc; };

  const float fill = (OP == 2) ? -INFINITY : 0.f;
  auto load_row = [&](f32x4 (&v)[NV], int k) {
    const int64_t row = row_of(k);
    const bool active = FULL || row < L;
    const f32x4* x4 = reinterpret_cast<const f32x4*>(X + (active ? row : 0) * (int64_t)C);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int j = i * TPR + t;
      if constexpr (FULL) {
        v[i] = ld4<NT>(x4 + j);
      } else {
        v[i] = (active && j < C4) ? ld4<NT>(x4 + j) : f32x4{fill, fill, fill, fill};
      }
    }
  };

  // Row reduction: wave-level, then (when the row spans wavefronts) an LDS fold in wave order.
  auto row_reduce_sum = [&](float s, float* slots) -> float {
    s = wave_sum(s);
    if constexpr (WPR == 1) {
      return s;
    } else {
      if ((tid & 63) == 0) slots[wave] = s;
      __syncthreads();
      float r = slots[rloc * WPR];
#pragma unroll
      for (int w = 1; w < WPR; ++w) r += slots[rloc * WPR + w];
      return r;
    }
  };
  auto row_reduce_max = [&](float m, float* slots) -> float {
    m = wave_max(m);
    if constexpr (WPR == 1) {
      return m;
    } else {
      if ((tid & 63) == 0) slots[wave] = m;
      __syncthreads();
      float r = slots[rloc * WPR];
#pragma unroll
      for (int w = 1; w < WPR; ++w) r = fmaxf(r, slots[rloc * WPR + w]);
      return r;
    }
  };

  // RMSNorm gain, read once per workgroup (L2 hits under the row's HBM latency). Where it is
  // requested was measured per geometry at 4096 x 4096: rows of 512 threads run 1.5% faster with
  // the gain before the first row's loads, rows of up to 256 threads 0.3-3% faster with it after.
  f32x4 g[NV];
  auto load_gain = [&]() __attribute__((always_inline)) {
    const f32x4* w4 = reinterpret_cast<const f32x4*>(Wg);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int j = i * TPR + t;
      g[i] = (FULL || j < C4) ? w4[j] : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  constexpr bool kGainFirst = TPR >= 512;
  if constexpr (kGain && !GS && kGainFirst) load_gain();
  f32x4 va[NV], vb[NV];
  load_row(va, 0);
  if constexpr (kGain && !GS && !kGainFirst) load_gain();
  if constexpr (kGain && GS) {
    const f32x4* w4 = reinterpret_cast<const f32x4*>(Wg);
    for (int j = tid; j < C4; j += WG) gain_lds[j] = w4[j];
  }

#pragma unroll
  for (int k = 0; k < RPB; ++k) {
    f32x4(&v)[NV] = (k & 1) ? vb : va;
    if (k + 1 < RPB) load_row((k & 1) ? va : vb, k + 1);
    const int64_t row = row_of(k);
    const bool active = FULL || row < L;
    f32x4* y4 = reinterpret_cast<f32x4*>(Y + (active ? row : 0) * (int64_t)C);

    if constexpr (OP == 0) {  // row-sum
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < NV; ++i) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
      s = row_reduce_sum(s, red0[k & 1]);
      if (active && t == 0) Y[row] = s;
    } else if constexpr (OP == 1) {  // RMSNorm
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        // The compiler may contract a square with the following add (one rounding fewer).
        ss += (v[i].x * v[i].x + v[i].y * v[i].y) + (v[i].z * v[i].z + v[i].w * v[i].w);
      }
      ss = row_reduce_sum(ss, red0[k & 1]);
      // Correctly rounded divide and square root, as the reference's 1.0f / std::sqrt(...).
      const float rms = 1.0f / sqrtf(ss / (float)C + eps);
      if constexpr (GS) __syncthreads();
      if (active) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          const int j = i * TPR + t;
          if (FULL || j < C4) {
            const f32x4 gi = GS ? gain_lds[j] : g[i];
            f32x4 o;
            o.x = (v[i].x * rms) * gi.x;
            o.y = (v[i].y * rms) * gi.y;
            o.z = (v[i].z * rms) * gi.z;
            o.w = (v[i].w * rms) * gi.w;
            st4<NT>(y4 + j, o);
          }
        }
      }
    } else if constexpr (OP == 3) {  // channelscale: one correctly rounded multiply per element
      if constexpr (GS) __syncthreads();
      if (active) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          const int j = i * TPR + t;
          if (FULL || j < C4) {
            const f32x4 gi = GS ? gain_lds[j] : g[i];
            st4<NT>(y4 + j, f32x4{v[i].x * gi.x, v[i].y * gi.y, v[i].z * gi.z, v[i].w * gi.w});
          }
        }
      }
    } else {  // softmax
      float m = -INFINITY;
#pragma unroll
      for (int i = 0; i < NV; ++i) m = fmaxf(m, fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w)));
      m = row_reduce_max(m, red0[k & 1]);
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        v[i].x = exp_sub(v[i].x, m);
        v[i].y = exp_sub(v[i].y, m);
        v[i].z = exp_sub(v[i].z, m);
        v[i].w = exp_sub(v[i].w, m);
        s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
      }
      s = row_reduce_sum(s, red1[k & 1]);
      // One correctly rounded reciprocal per row, then a multiply per element: within one
      // rounding of the reference's per-element divide.
      const float inv = 1.0f / s;
      if constexpr (GS) __syncthreads();
      if (active) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          const int j = i * TPR + t;
          if (FULL || j < C4) {
            if constexpr (GS) {
              const f32x4 gi = gain_lds[j];
              st4<NT>(y4 + j, f32x4{(v[i].x * inv) * gi.x, (v[i].y * inv) * gi.y, (v[i].z * inv) * gi.z,
                                    (v[i].w * inv) * gi.w});
            } else {
              st4<NT>(y4 + j, f32x4{v[i].x * inv, v[i].y * inv, v[i].z * inv, v[i].w * inv});
            }
          }
        }
      }
    }
  }
}

// Any row length: the row is streamed (twice for RMSNorm, three times for softmax) with
// scalar coalesced loads. Used only when C is not a multiple of 4 or does not fit registers.
template <int OP>
__global__ void __launch_bounds__(256)
    rows_stream_kernel(const float* __restrict__ X, const float* __restrict__ Wg, float* __restrict__ Y, int L,
                       int C, float eps) {
  __shared__ float red0[4];
  __shared__ float red1[4];
  const int tid = threadIdx.x, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  if (row >= L) return;  // uniform per workgroup: one row per workgroup
  const float* x = X + row * (int64_t)C;
  auto block_sum = [&](float s, float* slots) {
    s = wave_sum(s);
    if ((tid & 63) == 0) slots[wave] = s;
    __syncthreads();
    return ((slots[0] + slots[1]) + slots[2]) + slots[3];
  };
  auto block_max = [&](float m, float* slots) {
    m = wave_max(m);
    if ((tid & 63) == 0) slots[wave] = m;
    __syncthreads();
    return fmaxf(fmaxf(slots[0], slots[1]), fmaxf(slots[2], slots[3]));
  };
  if constexpr (OP == 0) {
    float s = 0.f;
    for (int c = tid; c < C; c += 256) s += x[c];
    s = block_sum(s, red0);
    if (tid == 0) Y[row] = s;
  } else if constexpr (OP == 1) {
    float ss = 0.f;
    for (int c = tid; c < C; c += 256) ss += __fmul_rn(x[c], x[c]);
    ss = block_sum(ss, red0);
    const float rms = 1.0f / sqrtf(ss / (float)C + eps);
    float* y = Y + row * (int64_t)C;
    for (int c = tid; c < C; c += 256) y[c] = __fmul_rn(__fmul_rn(x[c], rms), Wg[c]);
  } else {
    float m = -INFINITY;
    for (int c = tid; c < C; c += 256) m = fmaxf(m, x[c]);
    m = block_max(m, red0);
    float s = 0.f;
    for (int c = tid; c < C; c += 256) s += expf(x[c] - m);
    s = block_sum(s, red1);
    float* y = Y + row * (int64_t)C;
    for (int c = tid; c < C; c += 256) y[c] = expf(x[c] - m) / s;
  }
}

// Standalone channelscale (reference src/codegen_hip.cpp:2329-2335): Y[i*C+c] = X[i*C+c]*S[c].
__global__ void __launch_bounds__(256)
    channelscale4_kernel(const f32x4* __restrict__ X, const float* __restrict__ S, f32x4* __restrict__ Y,
                         int64_t n4, int C) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) {
    const int c = (int)((i * 4) % C);
    const f32x4 x = X[i];
    Y[i] = f32x4{x.x * S[c], x.y * S[c + 1], x.z * S[c + 2], x.w * S[c + 3]};
  }
}
__global__ void __launch_bounds__(256)
    channelscale1_kernel(const float* __restrict__ X, const float* __restrict__ S, float* __restrict__ Y, int64_t n,
                         int C) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) Y[i] = X[i] * S[i % C];
}

// 1-D reduce, pass 1: partial p sums the contiguous chunk [p*chunk, min((p+1)*chunk, n)).
__global__ void __launch_bounds__(kReduceThreads)
    reduce_part_kernel(const float* __restrict__ X, float* __restrict__ P, int64_t n, int64_t chunk) {
  __shared__ float slots[kReduceThreads / 64];
  const int tid = threadIdx.x;
  const int64_t b = (int64_t)blockIdx.x * chunk;
  const int64_t e = b + chunk < n ? b + chunk : n;
  float s = 0.f;
  if ((chunk & 3) == 0 && (((uintptr_t)X) & 15) == 0) {
    const f32x4* x4 = reinterpret_cast<const f32x4*>(X + b);
    const int64_t full4 = (e - b) >> 2;
    for (int64_t i = tid; i < full4; i += kReduceThreads) {
      const f32x4 v = x4[i];
      s += (v.x + v.y) + (v.z + v.w);
    }
    for (int64_t i = b + (full4 << 2) + tid; i < e; i += kReduceThreads) s += X[i];
  } else {
    for (int64_t i = b + tid; i < e; i += kReduceThreads) s += X[i];
  }
  s = wave_sum(s);
  if ((tid & 63) == 0) slots[tid >> 6] = s;
  __syncthreads();
  if (tid == 0) {
    float r = slots[0];
    for (int w = 1; w < kReduceThreads / 64; ++w) r += slots[w];
    P[blockIdx.x] = r;
  }
}
// Pass 2: one workgroup folds the partials (thread t takes t, t+256, ...), then in wave order.
__global__ void __launch_bounds__(kReduceThreads)
    reduce_fold_kernel(const float* __restrict__ P, float* __restrict__ Y, int np) {
  __shared__ float slots[kReduceThreads / 64];
  const int tid = threadIdx.x;
  float s = 0.f;
  for (int i = tid; i < np; i += kReduceThreads) s += P[i];
  s = wave_sum(s);
  if ((tid & 63) == 0) slots[tid >> 6] = s;
  __syncthreads();
  if (tid == 0) {
    float r = slots[0];
    for (int w = 1; w < kReduceThreads / 64; ++w) r += slots[w];
    Y[0] = r;
  }
}

// The grouped-store softmax's gain: ones for the widest row the form holds (4096 floats).
constexpr int kUnitGainFloats = 64 * 16 * 4;
struct UnitGain {
  float v[kUnitGainFloats];
};
constexpr UnitGain unit_gain_ones() {
  UnitGain u{};
  for (int i = 0; i < kUnitGainFloats; ++i) u.v[i] = 1.0f;
  return u;
}
__device__ __align__(16) UnitGain unit_gain = unit_gain_ones();

}  // namespace uk::kern

namespace uk {

namespace {
// Device address of the unit gain on the current device, looked up once per device (the host
// name of a __device__ variable is a stand-in, not its address).
const float* unit_gain_device() {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static const float* addr[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lk(mu);
  if (!addr[dev]) {
    void* q = nullptr;
    if (hipGetSymbolAddress(&q, HIP_SYMBOL(kern::unit_gain)) != hipSuccess) return nullptr;
    addr[dev] = static_cast<const float*>(q);
  }
  return addr[dev];
}

template <int TPR, int NV, bool NT, int RPB, bool GS, bool FULL>
hipError_t rows_go(RowOp op, const float* X, const float* W, float* Y, int64_t L, int64_t C, float eps, int64_t grid,
                   hipStream_t s) {
  constexpr int WG = TPR < 256 ? 256 : TPR;
  switch (op) {
    case RowOp::Sum:
      hipLaunchKernelGGL((kern::rows_kernel<TPR, NV, 0, NT, RPB, GS, FULL>), dim3((unsigned)grid), dim3(WG), 0, s, X, W,
                         Y, (int)L, (int)C, eps);
      break;
    case RowOp::RmsNorm:
      hipLaunchKernelGGL((kern::rows_kernel<TPR, NV, 1, NT, RPB, GS, FULL>), dim3((unsigned)grid), dim3(WG), 0, s, X, W,
                         Y, (int)L, (int)C, eps);
      break;
    case RowOp::Softmax:
      hipLaunchKernelGGL((kern::rows_kernel<TPR, NV, 2, NT, RPB, GS, FULL>), dim3((unsigned)grid), dim3(WG), 0, s, X, W,
                         Y, (int)L, (int)C, eps);
      break;
  }
  return hipGetLastError();
}

template <int TPR, int NV, bool NT, int RPB, bool GS>
hipError_t rows_dispatch_op(RowOp op, const float* X, const float* W, float* Y, int64_t L, int64_t C, float eps,
                            hipStream_t s) {
  constexpr int WG = TPR < 256 ? 256 : TPR;
  constexpr int RPW = WG / TPR;
  const int64_t grid = (L + RPW * RPB - 1) / (RPW * RPB);
  if constexpr (GS) {
    if (C == int64_t(TPR) * NV * 4 && L % (RPW * RPB) == 0) return rows_go<TPR, NV, NT, RPB, GS, true>(op, X, W, Y, L, C, eps, grid, s);
  }
  return rows_go<TPR, NV, NT, RPB, GS, false>(op, X, W, Y, L, C, eps, grid, s);
}
}  // namespace

hipError_t launch_rows(const Plan& p, RowOp op, const float* X, const float* W, float* Y, int64_t L, int64_t C,
                       float eps, hipStream_t s) {
  if (L <= 0 || C <= 0 || L > INT32_MAX || C > INT32_MAX) return hipErrorInvalidValue;
  if (op == RowOp::RmsNorm && !W) return hipErrorInvalidValue;
  if (p.family == Family::RowsStream) {
    if (L > 0x7fffffff) return hipErrorInvalidValue;
    switch (op) {
      case RowOp::Sum:
        hipLaunchKernelGGL(kern::rows_stream_kernel<0>, dim3((unsigned)L), dim3(256), 0, s, X, W, Y, (int)L, (int)C,
                           eps);
        break;
      case RowOp::RmsNorm:
        hipLaunchKernelGGL(kern::rows_stream_kernel<1>, dim3((unsigned)L), dim3(256), 0, s, X, W, Y, (int)L, (int)C,
                           eps);
        break;
      case RowOp::Softmax:
        hipLaunchKernelGGL(kern::rows_stream_kernel<2>, dim3((unsigned)L), dim3(256), 0, s, X, W, Y, (int)L, (int)C,
                           eps);
        break;
    }
    return hipGetLastError();
  }
  if (p.family != Family::Rows || p.variant < 0 || p.variant >= kNumRowsVariants) return hipErrorInvalidValue;
  const RowsVariant v = kRowsVariants[p.variant];
  if (op == RowOp::Softmax && v.grp) {
    W = unit_gain_device();
    if (!W) return hipErrorInvalidSymbol;
  }
  // The register-resident kernel reads float4 at row*C + 4j: rows must be 16-byte aligned and
  // the row must fit the variant's capacity.
  if ((C & 3) != 0 || C > (int64_t)v.tpr * v.nv * 4) return hipErrorInvalidValue;
  if ((((uintptr_t)X) & 15) || (((uintptr_t)Y) & 15) || (W && (((uintptr_t)W) & 15))) return hipErrorInvalidValue;
  switch (p.variant) {
  static_assert(kNumRowsVariants == 25, "every rows variant needs a case below");
#define UK_ROWS_CASE(I)                                                                                   \
  case I:                                                                                                 \
    return rows_dispatch_op<kRowsVariants[I].tpr, kRowsVariants[I].nv, kRowsVariants[I].nt != 0,         \
                            kRowsVariants[I].rpb, kRowsVariants[I].grp != 0>(op, X, W, Y, L, C, eps, s);
    UK_ROWS_CASE(0)
    UK_ROWS_CASE(1)
    UK_ROWS_CASE(2)
    UK_ROWS_CASE(3)
    UK_ROWS_CASE(4)
    UK_ROWS_CASE(5)
    UK_ROWS_CASE(6)
    UK_ROWS_CASE(7)
    UK_ROWS_CASE(8)
    UK_ROWS_CASE(9)
    UK_ROWS_CASE(10)
    UK_ROWS_CASE(11)
    UK_ROWS_CASE(12)
    UK_ROWS_CASE(13)
    UK_ROWS_CASE(14)
    UK_ROWS_CASE(15)
    UK_ROWS_CASE(16)
    UK_ROWS_CASE(17)
    UK_ROWS_CASE(18)
    UK_ROWS_CASE(19)
    UK_ROWS_CASE(20)
    UK_ROWS_CASE(21)
    UK_ROWS_CASE(22)
    UK_ROWS_CASE(23)
    UK_ROWS_CASE(24)
#undef UK_ROWS_CASE
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_channelscale(const float* X, const float* S, float* Y, int64_t L, int64_t C, hipStream_t s) {
  if (L <= 0 || C <= 0 || C > INT32_MAX) return hipErrorInvalidValue;
  if (channelscale_rows_form(L, C) && !((((uintptr_t)X) | ((uintptr_t)Y) | ((uintptr_t)S)) & 15)) {
    // One wavefront per row, four rows per workgroup, S staged in LDS, the rows stored together;
    // unguarded when every workgroup holds four whole 4096-float rows.
    if (C == 4096 && L % 4 == 0)
      hipLaunchKernelGGL((kern::rows_kernel<64, 16, 3, true, 1, true, true>), dim3((unsigned)(L / 4)), dim3(256), 0, s,
                         X, S, Y, (int)L, (int)C, 0.f);
    else
      hipLaunchKernelGGL((kern::rows_kernel<64, 16, 3, true, 1, true>), dim3((unsigned)((L + 3) / 4)), dim3(256), 0,
                         s, X, S, Y, (int)L, (int)C, 0.f);
    return hipGetLastError();
  }
  const int64_t n = L * C;
  const bool v4 = (C & 3) == 0 && !(((uintptr_t)X) & 15) && !(((uintptr_t)Y) & 15);
  const int64_t units = v4 ? n / 4 : n;
  int64_t grid = (units + 255) / 256;
  if (grid > 256 * 32) grid = 256 * 32;  // grid-stride beyond 32 workgroups per CU
  if (v4)
    hipLaunchKernelGGL(kern::channelscale4_kernel, dim3((unsigned)grid), dim3(256), 0, s,
                       reinterpret_cast<const kern::f32x4*>(X), S, reinterpret_cast<kern::f32x4*>(Y), units, (int)C);
  else
    hipLaunchKernelGGL(kern::channelscale1_kernel, dim3((unsigned)grid), dim3(256), 0, s, X, S, Y, n, (int)C);
  return hipGetLastError();
}

hipError_t launch_reduce1d(const float* X, float* partials, float* Y, int64_t n, hipStream_t s) {
  if (n < 0 || !partials) return hipErrorInvalidValue;
  int64_t chunk = (n + kReduceParts - 1) / kReduceParts;
  chunk = (chunk + 3) & ~int64_t(3);
  if (chunk < 4) chunk = 4;
  const int64_t np = n == 0 ? 1 : (n + chunk - 1) / chunk;  // <= kReduceParts
  hipLaunchKernelGGL(kern::reduce_part_kernel, dim3((unsigned)np), dim3(kReduceThreads), 0, s, X, partials, n, chunk);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern::reduce_fold_kernel, dim3(1), dim3(kReduceThreads), 0, s, partials, Y, (int)np);
  return hipGetLastError();
}

}  // namespace uk
