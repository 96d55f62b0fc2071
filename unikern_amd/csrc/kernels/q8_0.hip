// Q8_0 skinny GEMM on gfx950: Y[M][N] f32 = X[M][K] f16 . dequant(W)^T, W in GGUF Q8_0 blocks.
//
// The reference has no Q8_0 kernel (src/codegen_hip.cpp:87-88 refuses int8); this is new.
// Weight layout: N rows, each K/32 blocks of 34 bytes {binary16 d (little endian), int8 q[32]}.
// Dequantised value w = float(d) * float(q) is exact in binary32 (11 + 7 significant bits).
//
// One v_mfma_f32_16x16x32_f16 covers exactly one block of 16 weight rows against 16 activation
// rows: A = the matching 32 activations, B = the block's quants as f16 (integers in [-128, 127]
// are exact in binary16). The MFMA sums q*x with products exact and an f32 accumulator; the
// block scale then multiplies that block sum in f32 and the result is accumulated in f32:
//   y[m][n] = sum_b float(d[n][b]) * (sum_{i<32} q[n][b][i] * x[m][32b+i])
// i.e. the dequantised weight d*q enters as the exact product of its two factors.
//
// Memory path: a workgroup owns 16 consecutive weight rows. Each wavefront owns P consecutive
// block pairs (68 bytes per row) of those rows per round; for one row they are P * 68 contiguous
// bytes. It copies them into its own LDS area as [row][17 P dwords] with direct-to-LDS DMA of VEC
// dwords per lane (global_load_lds_dword, or global_load_lds_dwordx4 when every segment is 16-byte
// aligned: K a multiple of 64 P, P a multiple of 4), activation loads and copies all issued
// before one wait.
// No workgroup barrier is needed until the final fold; other wavefronts of the SIMD overlap it.
// From LDS, lane (i = row, g) reads the quants of both blocks of a pair with five dword reads and
// realigns the even block's (2-byte shifted) bytes with a funnel shift. Each lane converts 8
// quants to f16 with the 1024-bias trick (0x6400 | (q ^ 0x80) is the binary16 value 1024 + q +
// 128; subtracting 1152 is exact). The MFMA takes the activations as A and the quants as B, so a
// lane's outputs all belong to one weight row and its two block scales are one LDS broadcast.
//
// K must be a multiple of 64 (whole block pairs per row).
// Two kernel forms: q8_0_gemm_kernel (MFMA tiles of 16 weight rows, any M) below, and
// q8_0_gemv_kernel (M = 1: one weight row per wavefront on the vector ALUs) further down.
// Work split of q8_0_gemm_kernel: grid.x = groups of 16 NT weight rows, grid.y = 16-row groups of activations. With
// NT > 1 each activation fragment (read from global memory per workgroup) feeds NT MFMA tiles of
// weights: every workgroup reads all of its activation rows over K, so for M = 16 the activation
// reads (M K 2 bytes per workgroup, from L2) exceed the workgroup's weight bytes at NT = 1. A round
// covers WAVES * P pairs; wavefront w takes pairs [w * P, w * P + P) of it. Each wavefront
// accumulates in registers across rounds; the partials fold in LDS in wavefront order
// (deterministic). Weight rows past N read row n0 (valid memory) and are never stored;
// activation rows past M read row 0 and feed only output rows past M, which are never stored;
// pairs past K/64 are copied from pair 0 and skipped.
#include "../launch.hpp"
#include "../variants.hpp"
#include "common.hpp"

namespace uk::kern {

typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;

// Four int8 quants packed in a dword -> four binary16 values (exact): with u = q ^ 0x80 = q + 128
// as an unsigned byte, the binary16 pattern 0x64uu is 1024 + u; v_perm_b32 places the bytes
// under 0x64 high bytes (selector byte 4 picks the first operand's low byte, 0..3 the second's)
// and one packed subtract of 1152 leaves q.
__device__ __forceinline__ u32x2 q4_to_f16(uint32_t dw) {
  const uint32_t u = dw ^ 0x80808080u;
  const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
  const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
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

// s_waitcnt vmcnt(N), other counters unconstrained (gfx9 encoding: vmcnt bits 3:0 and 15:14).
template <int N>
__device__ __forceinline__ void q8_wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// XL (activations through LDS, one-round-at-a-time kernels of 4 pairs per wavefront, M <= 8): each
// wavefront copies the 512-byte slices of its pairs of the XL real activation rows (XL = 1: row
// 0; XL = 8: rows m0 .. M - 1) into LDS with 16-byte direct-to-LDS copies, one instruction per
// two rows, and reads the operands from there (rows past M read row 0 as an LDS broadcast). The
// register form issues 2 P loads per lane for the same bytes, and each 16-lane row group of
// them requests the same addresses. Same bits either way; bench.py (rotating activation and
// weight sets) on one box: N = K = 4096, M = 1 5.94 -> 5.67 us, M = 8 6.54 -> 6.47 us;
// N = 11008, M = 1 12.00 -> 11.72 us (XL = 8 is used by the one-tile kernels only).
// FL (whole lines, used for M > 8 in the one-tile kernels): the activation loads of a pair cover
// whole 128-byte lines, rows 0-7 in one load (lanes i < 8: row i's even block, lanes i >= 8: row
// i - 8's odd block, bytes 16 g of the block) and rows 8-15 in the other, and two masked DPP row
// shifts per dword rebuild the two MFMA operands after the wait. The operand layout itself (lane (i, g): row i,
// 16 bytes of one block) touches 16 half lines per load, which the memory path serves about
// 1.7 times slower for the same bytes. Same load count per round either way. (A/B on one box at
// M = 16: 2% faster at N = 4096 with one tile; 1% slower at N = 11008 with three, where each
// rebuilt operand feeds three MFMA tiles and the moves are not worth it.)
template <int WAVES, int P, int VEC, bool DB, int NT, bool FL, int XL = 0>
__global__ void __launch_bounds__(WAVES * 64)
    q8_0_gemm_kernel(const _Float16* __restrict__ X, const uint8_t* __restrict__ Wq, float* __restrict__ Y, int M,
                     int N, int K) {
  // All arguments in scalar registers before anything else (one wait for their loads, not one per
  // argument between the computations that need them).
  asm volatile("" ::"s"(X), "s"(Wq), "s"(Y), "s"(M), "s"(N), "s"(K));
  static_assert(VEC == 1 || (VEC == 4 && P % 4 == 0), "16-byte copies need 16-byte aligned segments");
  constexpr int kRowDw = 17 * P;                   // one row's P block pairs, in dwords
  constexpr int kWaveDw = NT * 16 * kRowDw;        // this wavefront's staging area
  constexpr int kUnits = kWaveDw / VEC;            // copy units of VEC dwords
  constexpr int kInst = (kUnits + 63) / 64;        // DMA instructions per round
  static_assert(2 * (2 * P + kInst) <= 63, "two rounds of loads must fit the vmcnt counter");
  static_assert(WAVES * kWaveDw >= WAVES * 256 * NT, "the partials fold reuses the staging buffer");
  static_assert(XL == 0 || ((XL == 1 || XL == 8) && P == 4 && !DB && !FL),
                "activation copies: 512-byte slices of 1 or up to 8 rows, each round waited for in full");
  __shared__ uint32_t wl[WAVES * kWaveDw * (DB ? 2 : 1)];
  __shared__ __attribute__((aligned(16))) _Float16 xs[XL ? WAVES * XL * 64 * P : 8];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int i = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16 * NT, m0 = blockIdx.y * 16;
  const int npairs = K >> 6;
  const int64_t row_bytes = (int64_t)npairs * 68;
  uint32_t* mine = wl + wave * kWaveDw * (DB ? 2 : 1);

  // DMA lane geometry (the same for every round): unit u = t * 64 + lane starts at flattened
  // dword f = VEC u of the [row][17 P] image, dword d of row r's segment, i.e. dword d % 17 of
  // its pair d / 17. (With VEC = 4 a unit may straddle two pairs of the segment; the segment is
  // contiguous in the weight stream, so the copy is still of consecutive bytes.)
  // With one weight tile (NT = 1) computed unit by unit beside the first round's copies (below),
  // not all before them: the first copy then leaves after one unit's arithmetic instead of every
  // unit's (4-6% faster at N = 4096 in A/B runs on one box). With three tiles the same order
  // measured 3% slower at M = 1 and 2% faster at M = 16, so NT > 1 computes them all first.
  constexpr bool kGeomBesideCopies = NT == 1;
  int src_row[kInst], src_pair[kInst], src_dw[kInst];
  auto geom = [&](int t) __attribute__((always_inline)) {
    const int u = t * 64 + lane;
    const int f = u * VEC;
    const int r = f / kRowDw, d = f - (f / kRowDw) * kRowDw;
    src_row[t] = (u < kUnits && n0 + r < N) ? n0 + r : n0;
    src_pair[t] = u < kUnits ? d / 17 : 0;
    src_dw[t] = u < kUnits ? d - (d / 17) * 17 : 0;
  };
  if constexpr (!kGeomBesideCopies) {
#pragma unroll
    for (int t = 0; t < kInst; ++t) geom(t);
  }

  const int m = m0 + i;
  const bool mok = m < M;
  // Rows past M read row 0 (finite values that feed only output rows that are never stored).
  const int mlo = m0 + (i & 7), mhi = m0 + 8 + (i & 7);
  const _Float16* xrow = FL ? X + (int64_t)(mlo < M ? mlo : 0) * K + 8 * g + 32 * (i >> 3)
                            : X + (int64_t)(mok ? m : 0) * K + 8 * g;
  const _Float16* xrow_hi = X + (int64_t)(mhi < M ? mhi : 0) * K + 8 * g + 32 * (i >> 3);

  f32x4 yacc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) yacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const f32x4 zero = f32x4{0.f, 0.f, 0.f, 0.f};
  // Round issue: the activations of this wavefront's pairs p0 .. p0 + P - 1 and the weight
  // copies into `buf`. Pairs past K/64 read pair 0 (valid memory) and are skipped below. Every
  // round issues the same 2 P + kInst loads, which the explicit vmcnt waits below count.
  // XL: rows staged (the MFMA operand's rows past them take row 0's slice).
  const int xr = XL == 1 ? 1 : (M - m0 < XL ? M - m0 : XL);
  auto issue_x = [&](int p0, f16x8 (&xa)[P], f16x8 (&xb)[P]) __attribute__((always_inline)) {
    if constexpr (XL > 0) {
      // Lanes 0-31 copy row 2t's slice, lanes 32-63 row 2t + 1's (16 bytes each, in order).
      const int64_t po = 64 * (p0 < npairs ? p0 : 0) + (lane & 31) * 8;
      for (int t = 0; 2 * t < xr; ++t) {
        const int r = 2 * t + (lane >> 5);
        if (r < xr)
          __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint32_t*>(X + (int64_t)(m0 + r) * K + po),
                                           (lds_void*)(xs + (wave * XL + 2 * t) * 64 * P), 16, 0, 0);
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < P; ++j) {
      const int p = p0 + j;
      const int64_t po = 64 * (p < npairs ? p : 0);
      if constexpr (FL) {  // raw whole-line loads: rows 0-7 in xa, rows 8-15 in xb
        xa[j] = *reinterpret_cast<const f16x8*>(xrow + po);
        xb[j] = *reinterpret_cast<const f16x8*>(xrow_hi + po);
      } else {
        xa[j] = *reinterpret_cast<const f16x8*>(xrow + po);
        xb[j] = *reinterpret_cast<const f16x8*>(xrow + po + 32);
      }
    }
  };
  // FIRST: the first round, which computes each unit's geometry just before its copy.
  auto issue_w = [&]<bool FIRST>(int p0, uint32_t* buf) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < kInst; ++t) {
      if constexpr (FIRST) geom(t);
      const int p = p0 + src_pair[t];
      const uint32_t* src = reinterpret_cast<const uint32_t*>(Wq + (int64_t)src_row[t] * row_bytes +
                                                              (int64_t)(p < npairs ? p : 0) * 68) + src_dw[t];
      lds_void* dst = (lds_void*)(buf + t * 64 * VEC);
      if (t * 64 + lane < kUnits) {
        if constexpr (VEC == 4) __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
        else __builtin_amdgcn_global_load_lds(src, dst, 4, 0, 0);
      }
      if constexpr (FIRST) __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto issue = [&](int p0, uint32_t* buf, f16x8 (&xa)[P], f16x8 (&xb)[P]) __attribute__((always_inline)) {
    __asm__ volatile("" ::: "memory");  // the buffer's previous reads stay before its refill
    issue_x(p0, xa, xb);
    issue_w.template operator()<false>(p0, buf);
  };
  auto compute = [&](int p0, const uint32_t* buf, const f16x8 (&xa)[P], const f16x8 (&xb)[P]) {
#pragma unroll
    for (int j = 0; j < P; ++j) {
      const int p = p0 + j;
      if (p >= npairs) break;  // wave-uniform: the last round's tail
      // Lanes of activation rows past M hold row 0's values (finite): they only feed output
      // rows past M, which are never stored, so no select is spent on them.
      f16x8 x0 = xa[j];
      f16x8 x1 = xb[j];
      if constexpr (XL > 0) {
        const int xrow_l = XL == 1 ? 0 : (i < xr ? i : 0);
        const _Float16* xl = xs + (wave * XL + xrow_l) * 64 * P + 64 * j + 8 * g;
        x0 = *reinterpret_cast<const f16x8*>(xl);
        x1 = *reinterpret_cast<const f16x8*>(xl + 32);
      }
      if constexpr (FL) {
        // Even-block operand: lanes 8-15 of each 16-lane row take rows 8-15's even blocks from
        // lanes 0-7 of the second load (row_shr:8); odd-block operand: lanes 0-7 take rows 0-7's
        // odd blocks from lanes 8-15 of the first load (row_shl:8).
        const u32x4 lo = __builtin_bit_cast(u32x4, xa[j]), hi = __builtin_bit_cast(u32x4, xb[j]);
        u32x4 e, o;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          e[d] = (uint32_t)__builtin_amdgcn_update_dpp((int)lo[d], (int)hi[d], 0x118, 0xf, 0xc, false);
          o[d] = (uint32_t)__builtin_amdgcn_update_dpp((int)hi[d], (int)lo[d], 0x108, 0xf, 0x3, false);
        }
        x0 = __builtin_bit_cast(f16x8, e);
        x1 = __builtin_bit_cast(f16x8, o);
      }
      // The pair's activations serve the NT 16-row tiles of weights.
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint32_t* pw = buf + (t * 16 + i) * kRowDw + 17 * j;
        const uint32_t a0 = pw[2 * g], a1 = pw[2 * g + 1];
        const uint32_t a2 = pw[2 * g + 2];  // dword 8 also carries the odd block's scale (lanes g = 3)
        const uint32_t b0 = pw[9 + 2 * g], b1 = pw[10 + 2 * g];
        // Even block: quant bytes 2..9 of this lane's 12-byte window; odd block: aligned.
        const f16x8 qa = q8_to_f16x8(__builtin_amdgcn_alignbyte(a1, a0, 2), __builtin_amdgcn_alignbyte(a2, a1, 2));
        const f16x8 qb = q8_to_f16x8(b0, b1);
        // A = activations (row m = i), B = quants (column n = i): the output lanes (i, g) hold
        // C[m = 4g + r][n = i], so every lane's four outputs belong to weight row i and need only
        // that row's two block scales, read as an LDS broadcast (dword 0: d_even in the low half,
        // dword 8: d_odd in the high half).
        const f32x4 s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(x0, qa, zero, 0, 0, 0);
        const f32x4 s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(x1, qb, zero, 0, 0, 0);
        const float d0 = half_bits_to_float(pw[0]);
        const float d1 = half_bits_to_float(pw[8] >> 16);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          yacc[t][r] = fmaf(d0, s0[r], yacc[t][r]);
          yacc[t][r] = fmaf(d1, s1[r], yacc[t][r]);
        }
      }
    }
  };

  // Rounds: wavefront w takes pairs [w P, w P + P) of each round of WAVES * P pairs. With DB the
  // next round's loads are in flight while this round is computed (two LDS buffers, two
  // activation register sets); the wait then leaves exactly the next round outstanding.
  constexpr int kRoundLoads = 2 * P + kInst;
  const int stride = WAVES * P;
  f16x8 xa0[P], xb0[P], xa1[P], xb1[P];
  uint32_t* buf0 = mine;
  uint32_t* buf1 = mine + (DB ? kWaveDw : 0);
  int p0 = wave * P;
  if (p0 < npairs) {
    issue_x(p0, xa0, xb0);
    issue_w.template operator()<kGeomBesideCopies>(p0, buf0);
  }
  while (p0 < npairs) {
    const int p1 = p0 + stride;
    if (DB && p1 < npairs) {
      issue(p1, buf1, xa1, xb1);
      q8_wait_vmcnt<kRoundLoads>();
    } else {
      q8_wait_vmcnt<0>();
    }
    compute(p0, buf0, xa0, xb0);
    if (p1 >= npairs) break;
    if constexpr (!DB) {
      issue(p1, buf0, xa0, xb0);
      p0 = p1;
      continue;
    }
    const int p2 = p1 + stride;
    if (p2 < npairs) {
      issue(p2, buf0, xa0, xb0);
      q8_wait_vmcnt<kRoundLoads>();
    } else {
      q8_wait_vmcnt<0>();
    }
    compute(p1, buf1, xa1, xb1);
    p0 = p2;
  }

  // Fold the wavefronts' partials in wavefront order (in the staging buffer, once every
  // wavefront is done reading it). Every thread folds outputs: thread o takes output row
  // o / (16 NT), column o % (16 NT) of the tile, so consecutive threads store consecutive columns.
  // (Folding in wavefront 0 alone read 64 LDS values per lane in sequence and took about as long
  // as the compute of a round.)
  float* red = reinterpret_cast<float*>(wl);
  __syncthreads();
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[(wave * NT + t) * 256 + lane * 4 + r] = yacc[t][r];
  __syncthreads();
  constexpr int kCols = 16 * NT;
  for (int o = threadIdx.x; o < 16 * kCols; o += WAVES * 64) {
    const int row = o / kCols, col = o - row * kCols;  // activation row, weight row in the tile
    const int t = col >> 4, c = col & 15;
    // The MFMA output lane that held (row, col): lane c + 16 (row / 4), register row % 4.
    const int e = t * 256 + (c + 16 * (row >> 2)) * 4 + (row & 3);
    float sum = red[e];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) sum += red[w * NT * 256 + e];
    const int n = n0 + col, mr = m0 + row;
    if (n < N && mr < M) Y[(int64_t)mr * N + n] = sum;
  }
}

// ---------------------------------------------------------------------------------------
// M = 1 (one activation row): q8_0_gemv_kernel. Without 16 activation rows the MFMA tile buys
// nothing, so each wavefront owns one whole weight row and reduces it on the vector ALUs: the
// row is K/32 * 34 contiguous bytes (4352 at K = 4096), copied into the wavefront's LDS area with
// 1 KiB direct-to-LDS instructions (whole 128-byte lines except at the ends, where the tile
// kernels copy 272-byte row segments), lane l takes block pair l, and a DPP wavefront sum replaces
// the tile kernels' LDS fold and its barrier.
// The activation row is copied into LDS once per workgroup (WAVES rows share it), 128 bytes per
// block pair, with the eight 16-byte chunks of pair p rotated by p (slot s holds chunk
// (s - p) mod 8): a lane reading chunk k of its pair reads slot (k + p) mod 8, so the 64 lanes'
// 16-byte reads, 128 bytes apart, spread over the LDS banks instead of falling on two bank
// groups (the unrotated layout measured 5.45 against 5.12 us at N = K = 4096).
// Per block: 16 v_dot2_f32_f16 of the quants (as binary16, exact, by the 1024-bias trick of
// q4_to_f16) with the activations, f32 accumulation; the pair adds d_odd * s_odd + d_even * s_even
// and the wavefront sum is a fixed DPP tree (deterministic).
// K: a multiple of 256 (16-byte aligned rows of whole block-pair quadruples), at most 4096 (one
// pair per lane; with two, at K = 4608-8192, the 16-wavefront tile kernel measured faster at four
// of five shapes). Rows past N copy row N - 1 (valid memory) and are never stored. FULL: K = 4096,
// every count a compile-time constant (the general form's run-time copy counts and wait cost 5.49
// against 5.12 us at N = K = 4096).
// Four quants (one dword) -> binary16 -> s + q . x over four activations (two dwords).
// The two f16 pairs enter __builtin_amdgcn_fdot2 as separate values: this compiler, given the
// pairs packed into a two-dword vector (as q4_to_f16 returns them) and extracted again, fed the
// low pair to both products (seen in its output for gfx950; the MFMA operands are not affected).
__device__ __forceinline__ float q4_dot(uint32_t dw, uint32_t xa, uint32_t xb, float s) {
  const uint32_t u = dw ^ 0x80808080u;
  const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
  const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
  const f16x2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  const f16x2v l = __builtin_bit_cast(f16x2v, lo) - bias, h = __builtin_bit_cast(f16x2v, hi) - bias;
  s = __builtin_amdgcn_fdot2(l, __builtin_bit_cast(f16x2v, xa), s, false);
  return __builtin_amdgcn_fdot2(h, __builtin_bit_cast(f16x2v, xb), s, false);
}

// s_waitcnt vmcnt(n) for a wave-uniform n known only at run time (n > 15: vmcnt(0), which waits
// for more than asked and is still correct).
__device__ __forceinline__ void q8_wait_vmcnt_rt(int n) {
  switch (n) {
    case 15: q8_wait_vmcnt<15>(); break;
    case 14: q8_wait_vmcnt<14>(); break;
    case 13: q8_wait_vmcnt<13>(); break;
    case 12: q8_wait_vmcnt<12>(); break;
    case 11: q8_wait_vmcnt<11>(); break;
    case 10: q8_wait_vmcnt<10>(); break;
    case 9: q8_wait_vmcnt<9>(); break;
    case 8: q8_wait_vmcnt<8>(); break;
    case 7: q8_wait_vmcnt<7>(); break;
    case 6: q8_wait_vmcnt<6>(); break;
    case 5: q8_wait_vmcnt<5>(); break;
    case 4: q8_wait_vmcnt<4>(); break;
    case 3: q8_wait_vmcnt<3>(); break;
    case 2: q8_wait_vmcnt<2>(); break;
    case 1: q8_wait_vmcnt<1>(); break;
    default: q8_wait_vmcnt<0>(); break;
  }
}

// Workgroup barrier without the memory fence of __syncthreads(), which would also wait for the
// wavefront's weight copies; the activation copies are waited for explicitly before it.
__device__ __forceinline__ void q8_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __asm__ volatile("s_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

template <int WAVES, bool FULL>
__global__ void __launch_bounds__(WAVES * 64)
    q8_0_gemv_kernel(const _Float16* __restrict__ X, const uint8_t* __restrict__ Wq, float* __restrict__ Y, int N,
                     int K) {
  asm volatile("" ::"s"(X), "s"(Wq), "s"(Y), "s"(N), "s"(K));
  constexpr int kMaxPairs = 64;
  constexpr int kRowDw = 17 * kMaxPairs;                        // the longest row, in dwords
  constexpr int kInstMax = (kMaxPairs * 68 / 16 + 63) / 64;      // its 16-byte copy instructions
  static_assert(kInstMax <= 15, "the weight copies fit the explicit vmcnt waits");
  __shared__ __attribute__((aligned(16))) unsigned char xs[kMaxPairs * 128];
  __shared__ __attribute__((aligned(16))) uint32_t wl[WAVES * kRowDw];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int npairs = FULL ? kMaxPairs : K >> 6;
  const int units = npairs / 4 * 17;      // 16-byte units of a row (npairs is a multiple of 4)
  const int ninst = (units + 63) >> 6;
  const int n = blockIdx.x * WAVES + wave;
  const int nn = n < N ? n : N - 1;

  // Activation copies: instruction q covers pairs 8q .. 8q + 7, lanes 8j .. 8j + 7 pair 8q + j.
  for (int q = wave; 8 * q < npairs; q += WAVES) {
    const int pr = 8 * q + (lane >> 3);
    const int ch = ((lane & 7) - pr) & 7;
    if (pr < npairs)
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint32_t*>(X + pr * 64 + ch * 8),
                                       (lds_void*)(xs + q * 1024), 16, 0, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
  uint32_t* mine = wl + wave * kRowDw;
  const uint8_t* row = Wq + (int64_t)nn * npairs * 68;
#pragma unroll
  for (int t = 0; t < kInstMax; ++t) {
    if (t < ninst) {
      const int u = t * 64 + lane;
      if (u < units)
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint32_t*>(row + 16 * u),
                                         (lds_void*)(mine + t * 256), 16, 0, 0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  q8_wait_vmcnt_rt(ninst);  // this wavefront's activation copies have landed
  q8_barrier();             // and every wavefront's
  q8_wait_vmcnt<0>();

  float y = 0.f;
  const int p = lane;  // this lane's block pair
  if (p < npairs) {
    const uint32_t* pw = mine + 17 * p;
    uint32_t dw[17];
#pragma unroll
    for (int d = 0; d < 17; ++d) dw[d] = pw[d];
    const unsigned char* xl = xs + 128 * p;
    u32x4 xv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) xv[k] = *reinterpret_cast<const u32x4*>(xl + 16 * ((k + p) & 7));
    // Even block: quant dword k is bytes 2 + 4k .. 5 + 4k of the pair; odd block: dwords 9-16.
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      s0 = q4_dot(__builtin_amdgcn_alignbyte(dw[k + 1], dw[k], 2), xv[k >> 1][(k & 1) * 2],
                  xv[k >> 1][(k & 1) * 2 + 1], s0);
#pragma unroll
    for (int k = 0; k < 8; ++k)
      s1 = q4_dot(dw[9 + k], xv[4 + (k >> 1)][(k & 1) * 2], xv[4 + (k >> 1)][(k & 1) * 2 + 1], s1);
    const float d0 = half_bits_to_float(dw[0]), d1 = half_bits_to_float(dw[8] >> 16);
    y = fmaf(d1, s1, d0 * s0);
  }
  y = wave_sum(y);
  if (lane == 0 && n < N) Y[n] = y;
}

}  // namespace uk::kern

namespace uk {

namespace {
template <int WAVES>
hipError_t q8_gemv_go(const void* X, const void* Wq, float* Y, int64_t N, int64_t K, hipStream_t s) {
  const dim3 grid((unsigned)((N + WAVES - 1) / WAVES));
  if (K == 4096)
    hipLaunchKernelGGL((kern::q8_0_gemv_kernel<WAVES, true>), grid, dim3(WAVES * 64), 0, s,
                       static_cast<const _Float16*>(X), static_cast<const uint8_t*>(Wq), Y, (int)N, (int)K);
  else
    hipLaunchKernelGGL((kern::q8_0_gemv_kernel<WAVES, false>), grid, dim3(WAVES * 64), 0, s,
                       static_cast<const _Float16*>(X), static_cast<const uint8_t*>(Wq), Y, (int)N, (int)K);
  return hipGetLastError();
}

// LDS bytes of an instantiation: the weight staging plus the activation slices of XL rows.
constexpr int q8_lds_bytes(int waves, int p, int vec, bool db, int nt, int xl) {
  return waves * nt * 16 * 17 * p * 4 * (db ? 2 : 1) + (xl ? waves * xl * 64 * p * 2 : 16);
}
constexpr int kQ8LdsLimit = 160 * 1024;

template <int WAVES, int P, int VEC, bool DB, int NT>
hipError_t q8_go(const void* X, const void* Wq, float* Y, int64_t M, int64_t N, int64_t K, hipStream_t s) {
  const dim3 grid((unsigned)((N + 16 * NT - 1) / (16 * NT)), (unsigned)((M + 15) / 16));
  // Activations through LDS at M <= 8 where the instantiation's LDS allows it.
  if constexpr (P == 4 && !DB) {
    if constexpr (q8_lds_bytes(WAVES, P, VEC, DB, NT, 1) <= kQ8LdsLimit) {
      if (M == 1) {
        hipLaunchKernelGGL((kern::q8_0_gemm_kernel<WAVES, P, VEC, DB, NT, false, 1>), grid, dim3(WAVES * 64), 0, s,
                           static_cast<const _Float16*>(X), static_cast<const uint8_t*>(Wq), Y, (int)M, (int)N,
                           (int)K);
        return hipGetLastError();
      }
    }
    // Eight rows only in the one-tile kernels: the three-tile kernel at N = 11008, M = 8 measured
    // 12.83 us with them against 12.63 us without.
    if constexpr (NT == 1 && q8_lds_bytes(WAVES, P, VEC, DB, NT, 8) <= kQ8LdsLimit) {
      if (M <= 8) {
        hipLaunchKernelGGL((kern::q8_0_gemm_kernel<WAVES, P, VEC, DB, NT, false, 8>), grid, dim3(WAVES * 64), 0, s,
                           static_cast<const _Float16*>(X), static_cast<const uint8_t*>(Wq), Y, (int)M, (int)N,
                           (int)K);
        return hipGetLastError();
      }
    }
  }
  // Whole-line activation loads in the one-tile kernels when more than 8 rows are real (at most
  // 8, the operand layout's half lines of the rows past M all fall on row 0).
  if constexpr (NT == 1) {
    if (M > 8) {
      hipLaunchKernelGGL((kern::q8_0_gemm_kernel<WAVES, P, VEC, DB, NT, true>), grid, dim3(WAVES * 64), 0, s,
                         static_cast<const _Float16*>(X), static_cast<const uint8_t*>(Wq), Y, (int)M, (int)N,
                         (int)K);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((kern::q8_0_gemm_kernel<WAVES, P, VEC, DB, NT, false>), grid, dim3(WAVES * 64), 0, s,
                     static_cast<const _Float16*>(X), static_cast<const uint8_t*>(Wq), Y, (int)M, (int)N, (int)K);
  return hipGetLastError();
}
}  // namespace

hipError_t launch_q8_gemm(const Plan& p, const void* X, const void* Wq, float* Y, int64_t M, int64_t N, int64_t K,
                          hipStream_t s) {
  if (p.family != Family::Q8Gemm || p.variant < 0 || p.variant >= kNumQ8Variants) return hipErrorInvalidValue;
  // Whole block pairs per row keep every row (34*K/32 bytes) and pair 4-byte aligned.
  if (M <= 0 || N <= 0 || K <= 0 || K % 64) return hipErrorInvalidValue;
  // Row byte offsets are 64-bit, element indices 32-bit; grid limits.
  if ((N + 15) / 16 > INT32_MAX || (M + 15) / 16 > 65535 || K > INT32_MAX / 2 || N > INT32_MAX ||
      M * K > INT32_MAX)
    return hipErrorInvalidValue;
  // Activation rows are read as 16-byte vectors at 2*(m*K + 64p + 8g [+ 32]) bytes (16-byte
  // aligned when X is); the weight stream is copied as dwords (4-byte aligned rows and pairs).
  if ((((uintptr_t)X) & 15) || (((uintptr_t)Wq) & 3) || (((uintptr_t)Y) & 3)) return hipErrorInvalidValue;
  const Q8Variant v = kQ8Variants[p.variant];
  if (v.gemv) {
    // One activation row; rows of whole block-pair quadruples (16-byte aligned), one pair per lane.
    if (M != 1 || K % 256 != 0 || K > 4096 || (((uintptr_t)Wq) & 15)) return hipErrorInvalidValue;
    if (v.waves == 4) return q8_gemv_go<4>(X, Wq, Y, N, K, s);
    return hipErrorInvalidValue;
  }
  // 16-byte copies: every wavefront segment (64 P elements of K) starts 16-byte aligned.
  if (v.vec == 4 && ((K % (64 * v.pairs)) != 0 || (((uintptr_t)Wq) & 15))) return hipErrorInvalidValue;
#define UK_Q8_CASE(W, PV, VV, DBV, NTV)                                                          \
  if (v.waves == W && v.pairs == PV && v.vec == VV && v.db == DBV && v.nt == NTV) \
    return q8_go<W, PV, VV, DBV != 0, NTV>(X, Wq, Y, M, N, K, s);
  UK_Q8_CASE(16, 4, 4, 0, 1)
  UK_Q8_CASE(16, 4, 1, 0, 1)
  UK_Q8_CASE(8, 8, 4, 0, 1)
  UK_Q8_CASE(8, 4, 1, 0, 1)
  UK_Q8_CASE(8, 4, 4, 1, 1)
  UK_Q8_CASE(4, 4, 4, 1, 1)
  UK_Q8_CASE(4, 8, 4, 1, 1)
  UK_Q8_CASE(8, 4, 4, 0, 4)
  UK_Q8_CASE(8, 4, 4, 0, 1)
  UK_Q8_CASE(8, 4, 4, 0, 3)
#undef UK_Q8_CASE
  return hipErrorInvalidValue;
}

}  // namespace uk
