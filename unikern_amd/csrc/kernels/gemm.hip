// GEMM on gfx950 matrix cores.
//
// Replaces the reference's SIMT uk_gemm / uk_gemm_h (src/codegen_hip.cpp:1089-1120,
// :1777-1808), which convert to f32 in LDS and run scalar FMAs. Eight kernels:
//
// gemm_f16_tn_kernel — the hot path: C[M][N] f16 = A[M][K] f16 . B^T, B stored [N][K]
//   (column-major B: both operands K-contiguous), f32 accumulate in v_mfma_f32_32x32x16_f16.
//   * BM x BN x BK macro tile per workgroup, WM x WN wavefronts, each a (BM/WM) x (BN/WN)
//     block of 32x32 MFMA tiles with accumulators resident in AGPR/VGPR.
//   * global -> LDS with buffer_load_dwordx4 ... lds (no VGPR staging): one instruction moves
//     1 KiB (16 rows x 64 B at BK = 32) into LDS. The buffer form takes a scalar resource and
//     one 32-bit offset per lane, which keeps the texture addresser's queues short (the 64-bit
//     per-lane global form backed them up and stalled the issuing wave); the resource's record
//     count covers exactly the tile's rows, so no offset can reach past the operand. The
//     16-byte chunk index is XOR-swizzled by row on the global side, so the MFMA fragment reads
//     (ds_read_b128, 32 rows at one k offset) hit distinct banks.
//   * STAGES-deep LDS ring (4 x 32 KiB for 256x256x32): the DMA runs STAGES-1 k-tiles ahead,
//     with partial vmcnt waits, and one barrier per k-tile. Each k-step issues its share of the
//     next tile's copies, spread evenly between the MFMAs (a burst at the start of the tile
//     filled the addresser's queues); MFMA fragments are double buffered in registers so LDS
//     reads for the next k-step overlap the current MFMAs.
//   * workgroup -> tile mapping is XCD-aware: workgroup i runs on XCD i % 8, so ids are
//     regrouped so each XCD owns a compact block of tiles and shares A/B panels in its L2.
//   * the MFMA computes C^T tiles (B fragment as the first operand), so each lane holds four
//     consecutive output columns per row; the epilogue converts to f16 (round to nearest
//     even), stages the tile in LDS and writes rows with 128-bit stores.
//
// gemm_f16_pp_kernel — the same 256x256 tile and LDS ring, scheduled as "ping-pong": the eight
//   wavefronts form two groups of four, one wavefront of each group per SIMD. While one group
//   issues MFMAs (v_mfma_f32_16x16x32_f16, a k-tile's worth from registers) the other reads its
//   next fragments from LDS and issues its share of the DMA copies; the groups swap at every
//   workgroup barrier. A wavefront issuing LDS reads or DMA copies stalls its own MFMA stream
//   (about 16 and 40-60 cycles per instruction, measured), so separating the roles keeps each
//   SIMD's matrix pipe fed by a wavefront that issues nothing else. The 16x16x32 form moves half
//   the accumulator bytes per flop of the 32x32x16 form; this chip runs the GEMM at its power
//   limit, so the saving shows up as a higher sustained clock.
//
// gemm_f16_w4_kernel — the same 256x256 tile with four wavefronts of 128x128 (one per SIMD, the
//   largest wave tile: a third fewer LDS bytes per flop than 128x64), copies sharing one M0 per
//   four, a barrier without a memory fence and a branch-free loop body.
//
// gemm_f16_w4s_kernel — that tiling on v_mfma_f32_16x16x32_f16 with a rolling A fragment.
//
// gemm_f16_w4k_kernel — that tiling with 64-deep k-tiles in five operand slots: each row's
//   k-segment is one whole 128-byte L2 line, so the L2 serves half the requests for the same bytes.
//
// gemm_f16_w4k16_kernel — the same on v_mfma_f32_16x16x32_f16, which sustains a higher clock at
//   the part's power limit.
//
// gemm_f32_kernel — f32 C = A . B (B stored [K][N] or [N][K]) on v_mfma_f32_32x32x2f32 for
//   M, N, K multiples of 64: a 64x64 tile per workgroup of eight wavefronts. Each k-tile of 64
//   moves into LDS by direct-to-LDS copies issued one tile ahead (rows of 256 bytes, 16-byte
//   chunks rotated by row so the fragment reads of eight lanes hit distinct bank groups; the
//   register-staged form with float4 stores into padded rows took 24.2-24.3 us at 1024^3 NN
//   against 21.9-22.2, same bits) and split between two wavefronts per SIMD: waves
//   0-3 multiply its first 32 k, waves 4-7 its last 32, each a 32x32 quarter of the tile, so one
//   wavefront's LDS reads and waits overlap the other's MFMAs. A lane's float4 of A (and of B
//   when B is [N][K]) feeds four MFMAs: MFMA (q, e) pairs k = 8q + e on lanes 0-31 with
//   k = 8q + 4 + e on lanes 32-63 (any assignment of k to MFMA steps gives the same sum when A
//   and B agree). The two halves' accumulators add in LDS in a fixed order.
//
// gemm_generic_kernel — any M, N, K, either B layout, f16 or f32 inputs: 64x64 tiles,
//   bounds-checked element loads, MFMA 32x32x16 f16 or 32x32x2 f32. Used for shapes the
//   fast kernels' divisibility predicates reject.
#include <type_traits>
#include <utility>

#include "../launch.hpp"
#include "../variants.hpp"
#include "common.hpp"

namespace uk::kern {

typedef __attribute__((address_space(3))) void lds_void;

template <int BM, int BN, int BK, int WM, int WN, int STAGES>
struct GemmF16Cfg {
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreads = kWaves * 64;
  static constexpr int kWTM = BM / WM;  // wave tile rows (M)
  static constexpr int kWTN = BN / WN;  // wave tile cols (N)
  static constexpr int kFM = kWTM / 32;
  static constexpr int kFN = kWTN / 32;
  static constexpr int kKK = BK / 16;   // MFMA k-steps per k-tile
  static constexpr int kRowBytes = BK * 2;
  static constexpr int kChunks = kRowBytes / 16;  // 16-byte chunks per LDS row
  static constexpr int kRowsPerInst = 1024 / kRowBytes;
  static constexpr int kStageBytes = (BM + BN) * kRowBytes;
  static constexpr int kInstsA = BM / kRowsPerInst / kWaves;  // DMA instructions per wave per k-tile
  static constexpr int kInstsB = BN / kRowsPerInst / kWaves;
  static constexpr int kInsts = kInstsA + kInstsB;
  static constexpr int kInstsPerStep = kInsts / kKK;  // copies issued per k-step
  static constexpr int kPitch = kWTN * 2 + 16;  // epilogue staging row pitch (bytes)
  static constexpr int kEpiBytes = kWaves * kWTM * kPitch;
  static constexpr int kLdsBytes = (STAGES * kStageBytes > kEpiBytes) ? STAGES * kStageBytes : kEpiBytes;
  static_assert(kWTM % 32 == 0 && kWTN % 32 == 0, "wave tile must be whole 32x32 MFMA tiles");
  static_assert(BK % 32 == 0 && kChunks <= 8 && 1024 % kRowBytes == 0, "BK must be 32 or 64");
  static_assert(kKK % 2 == 0, "fragment double buffering alternates k-steps");
  static_assert(BM % (kRowsPerInst * kWaves) == 0 && BN % (kRowsPerInst * kWaves) == 0,
                "DMA instructions must split evenly over the wavefronts");
  static_assert(STAGES >= 3, "the ring prefetches at least two k-tiles ahead");
  static_assert((STAGES - 2) * kInsts <= 63, "outstanding DMA must fit the vmcnt counter");
  static_assert(kInsts % kKK == 0, "copies must split evenly over the k-steps");
};

// One 1 KiB copy to LDS: lane offset voff and scalar offset soff (bytes) into the buffer of
// nbytes at base; offsets at or past nbytes read zero. A plain device function: the resource
// type is device-only, and kernel-template lambdas that name it lose their host launch stub.
__device__ __forceinline__ void copy_to_lds(const void* base, int nbytes, char* dst, int voff, int soff) {
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, nbytes, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)dst, 16, voff, soff, 0, 0);
}

// Scheduling pattern of one k-step: NM MFMAs with NR LDS reads and ND copies spread evenly
// between them (after MFMA m: the reads and copies whose even share falls due there).
template <int NM, int NR, int ND, int M = 0>
__device__ __forceinline__ void sched_spread() {
  if constexpr (M < NM) {
    constexpr int dr = ((M + 1) * NR + NM - 1) / NM - (M * NR + NM - 1) / NM;
    constexpr int dv = ((M + 1) * ND) / NM - (M * ND) / NM;
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
    if constexpr (dr > 0) __builtin_amdgcn_sched_group_barrier(0x100, dr, 0);  // DS reads
    if constexpr (dv > 0) __builtin_amdgcn_sched_group_barrier(0x020, dv, 0);  // VMEM (copies)
    sched_spread<NM, NR, ND, M + 1>();
  }
}

// Physical 16-byte chunk of logical chunk c in LDS row r: c ^ f(r). SWZ picks f for the bank
// geometry (0: r, 1: r >> 1, 2: r >> 2, each masked to the chunk count).
template <int SWZ, int CHUNKS>
__device__ __forceinline__ int swz(int r) {
  if constexpr (SWZ == 0) return r & (CHUNKS - 1);
  else if constexpr (SWZ == 1) return (r >> 1) & (CHUNKS - 1);
  else return (r >> 2) & (CHUNKS - 1);
}

// s_waitcnt vmcnt(N) with expcnt/lgkmcnt left unconstrained (gfx9 encoding: vmcnt in bits
// 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int BM, int BN, int BK, int WM, int WN, int STAGES, int SWZ>
__global__ void __launch_bounds__(WM* WN * 64, 1)
    gemm_f16_tn_kernel(const _Float16* __restrict__ A, const _Float16* __restrict__ B, _Float16* __restrict__ C,
                       int M, int N, int K, int tiles_m, int tiles_n) {
  using Cfg = GemmF16Cfg<BM, BN, BK, WM, WN, STAGES>;
  __shared__ __attribute__((aligned(1024))) char lds[Cfg::kLdsBytes];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;

  // XCD-aware tile mapping: make ids that share an XCD consecutive, then walk tiles in
  // groups of 4 tile-rows so consecutive ids share A panels (rows) and B panels (columns).
  const int G = gridDim.x;
  int lin = blockIdx.x;
  if ((G & 7) == 0) lin = (lin & 7) * (G >> 3) + (lin >> 3);
  constexpr int kGroupM = 4;
  const int per_group = kGroupM * tiles_n;
  const int group = lin / per_group;
  const int first_m = group * kGroupM;
  const int gm = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
  const int in_group = lin - group * per_group;
  const int tm = first_m + in_group % gm;
  const int tn = in_group / gm;

  const int m0 = tm * BM, n0 = tn * BN;
  const _Float16* Ag = A + (int64_t)m0 * K;
  const _Float16* Bg = B + (int64_t)n0 * K;

  const int wm = wave / WN, wn = wave % WN;
  f32x16 acc[Cfg::kFM][Cfg::kFN];
#pragma unroll
  for (int i = 0; i < Cfg::kFM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::kFN; ++j) acc[i][j] = f32x16{};

  // Copies of one k-tile: this wave's instruction q (q < kInstsA: A, else B) is copy
  // ins = (q mod kInstsA) * kWaves + w, which moves rows ins * kRowsPerInst + l / kChunks of the
  // operand's row block (lane l fills physical chunk l % kChunks, fetching the logical chunk
  // that lands there). The row term is a wave-uniform scalar offset. The swizzle term depends
  // on the row only through ins modulo kPeriod, and kPeriod divides kWaves, so it is the same
  // for every copy of this wave: one lane offset serves them all.
  constexpr int kPeriod = (Cfg::kChunks == 4 || SWZ == 0) ? 1 : (SWZ == 1 ? 2 : 4);
  static_assert(Cfg::kWaves % kPeriod == 0, "the swizzle period must divide the wave count");
  const int w = __builtin_amdgcn_readfirstlane(wave);
  const int vrow = lane / Cfg::kChunks;
  const int vchunk = (lane % Cfg::kChunks) ^ swz<SWZ, Cfg::kChunks>((w % kPeriod) * Cfg::kRowsPerInst + vrow);
  const int voff = (vrow * K + vchunk * 8) * 2;
  // Copies [part * kInstsPerStep, (part + 1) * kInstsPerStep) of k-tile t into its ring slot.
  // The tile index is clamped to the last tile, so the ring is issued without branches: a
  // clamped issue refills a slot nobody reads again.
  const int KT = K / BK;
  auto issue = [&](int t, int part) {
    char* st = lds + (t % STAGES) * Cfg::kStageBytes;
    const int tc = t < KT ? t : KT - 1;
#pragma unroll
    for (int u = 0; u < Cfg::kInstsPerStep; ++u) {
      const int q = part * Cfg::kInstsPerStep + u;
      const bool isA = q < Cfg::kInstsA;
      const int ins = (isA ? q : q - Cfg::kInstsA) * Cfg::kWaves + w;
      const int so = (ins * Cfg::kRowsPerInst * K + tc * BK) * 2;
      if (isA)
        copy_to_lds(Ag, BM * K * 2, st + ins * 1024, voff, so);
      else
        copy_to_lds(Bg, BN * K * 2, st + BM * Cfg::kRowBytes + ins * 1024, voff, so);
    }
  };

  // Fragment registers, double buffered across k-steps (and across k-tiles).
  const int frow = lane & 31;    // row within a 32-row MFMA tile
  const int fhalf = lane >> 5;   // which 8-element half of the 16-wide k-step
  f16x8 fa[2][Cfg::kFM], fb[2][Cfg::kFN];
  auto load_frags = [&](f16x8 (&a)[Cfg::kFM], f16x8 (&b)[Cfg::kFN], int t, int kk) {
    const char* As = lds + (t % STAGES) * Cfg::kStageBytes;
    const char* Bs = As + BM * Cfg::kRowBytes;
    const int c = kk * 2 + fhalf;
#pragma unroll
    for (int i = 0; i < Cfg::kFM; ++i) {
      const int r = wm * Cfg::kWTM + i * 32 + frow;
      a[i] = *reinterpret_cast<const f16x8*>(As + r * Cfg::kRowBytes + ((c ^ swz<SWZ, Cfg::kChunks>(r)) << 4));
    }
#pragma unroll
    for (int j = 0; j < Cfg::kFN; ++j) {
      const int r = wn * Cfg::kWTN + j * 32 + frow;
      b[j] = *reinterpret_cast<const f16x8*>(Bs + r * Cfg::kRowBytes + ((c ^ swz<SWZ, Cfg::kChunks>(r)) << 4));
    }
  };
  auto mfmas = [&](const f16x8 (&a)[Cfg::kFM], const f16x8 (&b)[Cfg::kFN]) {
#pragma unroll
    for (int i = 0; i < Cfg::kFM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::kFN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b[j], a[i], acc[i][j], 0, 0, 0);
  };
  constexpr int kMfmaPerStep = Cfg::kFM * Cfg::kFN;
  constexpr int kReadsPerStep = Cfg::kFM + Cfg::kFN;

  // Prologue: tiles 0 .. STAGES-2 in flight; wait for tile 0 only.
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
#pragma unroll
    for (int part = 0; part < Cfg::kKK; ++part) issue(s, part);
  wait_vmcnt<(STAGES - 2) * Cfg::kInsts>();
  __syncthreads();
  load_frags(fa[0], fb[0], 0, 0);

  for (int kt = 0; kt < KT; ++kt) {
    // Tile kt+1 has landed for this wave (tiles kt+2 .. kt+STAGES-2 may still fly) and, after
    // the barrier, for every wave; the barrier also retires all reads of tile kt-1, whose
    // slot the DMA below refills.
    wait_vmcnt<(STAGES - 3) * Cfg::kInsts>();
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < Cfg::kKK; ++kk) {
      const int cur = kk & 1;
      // Next k-step's fragments: the rest of this tile, then the first step of tile kt+1
      // (re-reading tile kt on the last iteration keeps the code branch-free).
      if (kk + 1 < Cfg::kKK)
        load_frags(fa[cur ^ 1], fb[cur ^ 1], kt, kk + 1);
      else
        load_frags(fa[cur ^ 1], fb[cur ^ 1], kt + 1 < KT ? kt + 1 : kt, 0);
      issue(kt + STAGES - 1, kk);
      mfmas(fa[cur], fb[cur]);
      // Spread the LDS reads and this step's copies between the MFMAs so the matrix pipe
      // never drains while they issue.
      sched_spread<kMfmaPerStep, kReadsPerStep, Cfg::kInstsPerStep>();
    }
  }
  wait_vmcnt<0>();  // clamped refills still in flight must land before LDS is reused
  __syncthreads();

  // Epilogue. acc[i][j] holds C^T: lane -> row m = i*32 + (lane & 31) of the wave tile and
  // columns n = j*32 + 8*g + 4*(lane >> 5) + {0..3} for register group g = r / 4.
  char* stage = lds + wave * (Cfg::kWTM * Cfg::kPitch);
#pragma unroll
  for (int i = 0; i < Cfg::kFM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::kFN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f16x4 h;
        h[0] = (_Float16)acc[i][j][g * 4 + 0];
        h[1] = (_Float16)acc[i][j][g * 4 + 1];
        h[2] = (_Float16)acc[i][j][g * 4 + 2];
        h[3] = (_Float16)acc[i][j][g * 4 + 3];
        const int m = i * 32 + (lane & 31);
        const int n = j * 32 + g * 8 + (lane >> 5) * 4;
        *reinterpret_cast<f16x4*>(stage + m * Cfg::kPitch + n * 2) = h;
      }
  __syncthreads();
  constexpr int kRowChunks = Cfg::kWTN * 2 / 16;
  constexpr int kTotal = Cfg::kWTM * kRowChunks;
  _Float16* Cw = C + (int64_t)(m0 + wm * Cfg::kWTM) * N + n0 + wn * Cfg::kWTN;
#pragma unroll 4
  for (int id = lane; id < kTotal; id += 64) {
    const int r = id / kRowChunks, q = id % kRowChunks;
    const u32x4 v = *reinterpret_cast<const u32x4*>(stage + r * Cfg::kPitch + q * 16);
    *reinterpret_cast<u32x4*>(Cw + (int64_t)r * N + q * 8) = v;
  }
}

// ---------------------------------------------------------------------------------------
// Ping-pong f16 GEMM: 256x256x32 macro tile, 8 wavefronts in two groups (g = wave / 4), wave
// tile 128 x 64 (rows g*128.., columns (wave % 4)*64..), STAGES-deep LDS ring of k-tiles.
//
// Phases p = 0, 1, 2, ... are separated by workgroup barriers b_p. Group 0 reads k-tile t's
// fragments in phase 2t and multiplies them in phase 2t+1; group 1 does the same one phase later
// (2t+1, 2t+2). In its read phase of tile t a wavefront also issues its quarter of one operand's
// copies of tile t + STAGES - 1 (group 0 copies A, group 1 copies B) into the slot tile t - 1
// left: its last reader, group 1, finished with it before b_2t. Before b_{2t+2} every wavefront
// waits until its own copies of tile t + 1 have landed, so after that barrier tile t + 1 is
// visible to all. Both groups execute the same number of barriers (2 KT after the prologue's).
// ---------------------------------------------------------------------------------------
constexpr int kPpBM = 256, kPpBN = 256, kPpBK = 32;
constexpr int kPpRow = kPpBK * 2;             // 64-byte LDS rows (4 chunks of 16 bytes)
constexpr int kPpOp = 256 * kPpRow;           // 16 KiB per operand per stage
constexpr int kPpStage = 2 * kPpOp;
constexpr int kPpWTM = 128, kPpWTN = 64;
constexpr int kPpPitch = kPpWTN * 2 + 16;     // epilogue staging row pitch (bytes)
constexpr int kPpEpi = 8 * kPpWTM * kPpPitch;
template <int STAGES>
constexpr int pp_lds_bytes() { return STAGES * kPpStage > kPpEpi ? STAGES * kPpStage : kPpEpi; }

// Workgroup barrier without the memory fence __syncthreads() implies: the fence would make every
// barrier wait for all outstanding copies, and each wait this kernel needs is issued explicitly.
__device__ __forceinline__ void barrier_nofence() {
  __builtin_amdgcn_sched_barrier(0);
  __asm__ volatile("s_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);  // nothing (an MFMA included) moves across the barrier
}

// Wait until at most 4 * n copies of this wavefront are outstanding (n = 0..3).
__device__ __forceinline__ void wait_copies(int n) {
  if (n >= 3) wait_vmcnt<12>();
  else if (n == 2) wait_vmcnt<8>();
  else if (n == 1) wait_vmcnt<4>();
  else wait_vmcnt<0>();
}

template <int STAGES, int SWZ>
__global__ void __launch_bounds__(512, 1)
    gemm_f16_pp_kernel(const _Float16* __restrict__ A, const _Float16* __restrict__ B, _Float16* __restrict__ C,
                       int M, int N, int K, int tiles_m, int tiles_n) {
  static_assert(STAGES >= 2 && STAGES - 2 <= 3, "copies in flight must fit wait_copies");
  typedef float f32x4v __attribute__((ext_vector_type(4)));
  __shared__ __attribute__((aligned(1024))) char lds[pp_lds_bytes<STAGES>()];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = w >> 2, q = w & 3;

  // XCD-aware tile order, as in gemm_f16_tn_kernel.
  const int G = gridDim.x;
  int lin = blockIdx.x;
  if ((G & 7) == 0) lin = (lin & 7) * (G >> 3) + (lin >> 3);
  constexpr int kGroupM = 4;
  const int per_group = kGroupM * tiles_n;
  const int group = lin / per_group;
  const int first_m = group * kGroupM;
  const int gm = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
  const int in_group = lin - group * per_group;
  const int tm = first_m + in_group % gm;
  const int tn = in_group / gm;
  const int m0 = tm * kPpBM, n0 = tn * kPpBN;

  // Copies: operand g's row block; instruction ins = 4u + q (u < 4) moves rows ins*16 .. +16.
  // Lane l fills row l / 4, physical chunk l % 4 with logical chunk (l % 4) ^ swz(row); rows of
  // an instruction start at multiples of 16, so swz(row) = swz(l / 4) and one lane offset serves
  // all four. SWZ 2 (row >> 2) conflicts two ways on the fragment reads below, SWZ 1 (row >> 1)
  // does not (gfx950 LDS, measured).
  const _Float16* op = g == 0 ? A + (int64_t)m0 * K : B + (int64_t)n0 * K;
  const int vrow = lane >> 2;
  const int voff = (vrow * K + (((lane & 3) ^ swz<SWZ, 4>(vrow)) * 8)) * 2;
  const int KT = K / kPpBK;
  auto issue = [&](int t) {
    char* st = lds + (t % STAGES) * kPpStage + g * kPpOp;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int ins = u * 4 + q;
      copy_to_lds(op, 256 * K * 2, st + ins * 1024, voff, (ins * 16 * K + t * kPpBK) * 2);
    }
  };

  // v_mfma_f32_16x16x32_f16 fragments: lane l supplies row l & 15 of a 16-row group at k-group
  // (logical chunk) l >> 4; one fragment per 16-row group covers the whole k-tile.
  const int frow = lane & 15, fk = lane >> 4;
  f16x8 fa[8], fb[4];
  auto read_frags = [&](int t) {
    const char* As = lds + (t % STAGES) * kPpStage;
    const char* Bs = As + kPpOp;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = g * kPpWTM + i * 16 + frow;
      fa[i] = *reinterpret_cast<const f16x8*>(As + r * kPpRow + ((fk ^ swz<SWZ, 4>(r)) << 4));
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = q * kPpWTN + j * 16 + frow;
      fb[j] = *reinterpret_cast<const f16x8*>(Bs + r * kPpRow + ((fk ^ swz<SWZ, 4>(r)) << 4));
    }
  };
  // acc[i][j] = C^T block: lane l holds C[i*16 + (l & 15)][j*16 + 4*(l >> 4) + r], r < 4.
  f32x4v acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};
  auto multiply = [&]() {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fb[j], fa[i], acc[i][j], 0, 0, 0);
  };
  // Copies of tiles issued after tile t+1 by this wavefront (they may stay in flight).
  auto after = [&](int t) {
    const int last = (t + STAGES - 1 < KT - 1) ? t + STAGES - 1 : KT - 1;
    return last - (t + 1);
  };

  // Prologue: tiles 0 .. STAGES-2 (those that exist), then wait for tile 0.
  for (int t = 0; t < STAGES - 1; ++t)
    if (t < KT) issue(t);
  wait_copies((STAGES - 2 < KT - 1) ? STAGES - 2 : KT - 1);
  barrier_nofence();  // b0

  if (g == 0) {
    for (int t = 0; t < KT; ++t) {
      read_frags(t);  // phase 2t
      if (t + STAGES - 1 < KT) issue(t + STAGES - 1);
      // No wait for the fragment reads here: slot t is refilled only after b_{2t+2S-2}, which
      // follows this group's MFMAs (and so its reads); the MFMAs wait for their fragments.
      barrier_nofence();  // b_{2t+1}
      multiply();  // phase 2t+1
      wait_copies(after(t));
      barrier_nofence();  // b_{2t+2}
    }
  } else {
    barrier_nofence();  // b1 (phase 0: nothing to multiply yet)
    for (int t = 0; t < KT; ++t) {
      read_frags(t);  // phase 2t+1
      if (t + STAGES - 1 < KT) issue(t + STAGES - 1);
      wait_copies(after(t));
      // After b_{2t+2} group 0 issues the copies of tile t + STAGES into tile t's slot (after the
      // last barrier it stages its epilogue over the ring): this group's reads of tile t must
      // have returned first, since the barrier does not order LDS requests of different
      // wavefronts. The reads went out at the start of the phase, so the wait costs little.
      __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      barrier_nofence();  // b_{2t+2}
      multiply();  // phase 2t+2
      if (t < KT - 1) barrier_nofence();  // b_{2t+3}
    }
  }
  // After b_{2KT} no wavefront reads the ring and no copy is in flight (every wavefront waited
  // for all of its copies before that barrier): each wavefront stages its tile in its own region.
  char* stage = lds + w * (kPpWTM * kPpPitch);
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f16x4 h;
      h[0] = (_Float16)acc[i][j][0];
      h[1] = (_Float16)acc[i][j][1];
      h[2] = (_Float16)acc[i][j][2];
      h[3] = (_Float16)acc[i][j][3];
      const int m = i * 16 + (lane & 15);
      const int n = j * 16 + 4 * (lane >> 4);
      *reinterpret_cast<f16x4*>(stage + m * kPpPitch + n * 2) = h;
    }
  // The region is private to this wavefront: its own LDS writes must land before its reads.
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  constexpr int kRowChunks = kPpWTN * 2 / 16;
  _Float16* Cw = C + (int64_t)(m0 + g * kPpWTM) * N + n0 + q * kPpWTN;
#pragma unroll 4
  for (int id = lane; id < kPpWTM * kRowChunks; id += 64) {
    const int r = id / kRowChunks, c = id % kRowChunks;
    const u32x4 v = *reinterpret_cast<const u32x4*>(stage + r * kPpPitch + c * 16);
    *reinterpret_cast<u32x4*>(Cw + (int64_t)r * N + c * 8) = v;
  }
}

// ---------------------------------------------------------------------------------------
// Four-wavefront f16 GEMM: 256x256x32 macro tile, 2 x 2 wavefronts of 128 x 128 (one per SIMD),
// v_mfma_f32_32x32x16_f16 with the 16 accumulator tiles of a wavefront in its 256 AGPRs.
//
// Why one wavefront per SIMD with the largest wave tile: a 128 x 128 wave tile reads 16 KiB of
// fragments per 32-deep k-tile for 1024 MFMA cycles, a third fewer LDS bytes per flop than the
// ping-pong kernel's 128 x 64, and one wavefront sustains about 52 B/ns of LDS reads (measured),
// so its reads of the next k-step fit in about half of the current k-step's MFMA time and
// overlap it. (With v_mfma_f32_16x16x32_f16 the 64 accumulator tuples fill the AGPR file and the
// register allocator rotates tuples through VGPRs every iteration; the 16 tuples of the 32x32
// form stay put.)
//
// Per k-tile: wait for this wavefront's copies of tile t+1, one barrier without a memory fence
// (tile t+1 is then visible to all; every wavefront has read its last fragments of tile t-1, whose
// slot the copies refill), then two k-steps of 16 MFMAs, each with the next k-step's 8 fragment
// reads (fragments double buffered in VGPRs) and 4 copies spread between them. No read is
// waited for at the barrier: the MFMAs wait for their own fragments.
//
// LDS rows are 64 bytes (32 halfs); chunk c of row r sits at c ^ ((r >> 2) & 3), for which the
// 32x32x16 fragment reads (32 rows x 2 k-groups per ds_read_b128) are free of bank conflicts on
// gfx950 (measured). Copies: wavefront w moves A rows 64w..64w+63 and B rows 64w..64w+63 of a
// k-tile as four 1 KiB buffer_load_dwordx4 ... lds per operand sharing one M0: the instruction
// offset steps both the LDS and the global address and the scalar offset corrects the global one.
constexpr int kW4BM = 256, kW4BN = 256, kW4BK = 32;
constexpr int kW4Row = kW4BK * 2;        // 64-byte LDS rows
constexpr int kW4Op = 256 * kW4Row;      // 16 KiB per operand per stage
constexpr int kW4Stage = 2 * kW4Op;
constexpr int kW4WT = 128;               // wave tile (both dimensions)
constexpr int kW4Pitch = kW4WT * 2 + 16; // epilogue staging row pitch (bytes)
constexpr int kW4Epi = 4 * kW4WT * kW4Pitch;
template <int STAGES>
constexpr int w4_lds_bytes() { return STAGES * kW4Stage > kW4Epi ? STAGES * kW4Stage : kW4Epi; }

// Four 1 KiB copies into consecutive LDS blocks dst, dst + 1 KiB, .. from global offsets
// soff, soff + step, soff + 2 step, soff + 3 step (bytes, plus the lane offset voff) of the
// buffer of nbytes at base; one M0 for all four. The buffer range check covers the lane offset
// (plus the instruction offset), not the scalar one: a lane offset of kCopyNone makes every copy
// return zeros without a memory access.
constexpr int kCopyNone = int(0x80000000u);
__device__ __forceinline__ void copy4_to_lds(const void* base, int nbytes, char* dst, int voff, int soff, int step) {
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, nbytes, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)dst, 16, voff, soff, 0, 0);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)dst, 16, voff, soff + step - 1024, 1024, 0);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)dst, 16, voff, soff + 2 * step - 2048, 2048, 0);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)dst, 16, voff, soff + 3 * step - 3072, 3072, 0);
}

template <int STAGES>
__global__ void __launch_bounds__(256, 1)
    gemm_f16_w4_kernel(const _Float16* __restrict__ A, const _Float16* __restrict__ B, _Float16* __restrict__ C,
                       int M, int N, int K, int tiles_m, int tiles_n) {
  static_assert(STAGES >= 3 && (STAGES - 2) * 8 <= 63, "copies in flight must fit vmcnt");
  __shared__ __attribute__((aligned(1024))) char lds[w4_lds_bytes<STAGES>()];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w >> 1, wn = w & 1;

  // XCD-aware tile order, as in gemm_f16_tn_kernel.
  const int G = gridDim.x;
  int lin = blockIdx.x;
  if ((G & 7) == 0) lin = (lin & 7) * (G >> 3) + (lin >> 3);
  constexpr int kGroupM = 4;
  const int per_group = kGroupM * tiles_n;
  const int group = lin / per_group;
  const int first_m = group * kGroupM;
  const int gm = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
  const int in_group = lin - group * per_group;
  const int tm = first_m + in_group % gm;
  const int tn = in_group / gm;
  const int m0 = tm * kW4BM, n0 = tn * kW4BN;

  // Copy lanes: lane l fills row l / 4 of a 16-row block, physical chunk l % 4 with logical
  // chunk (l % 4) ^ ((row >> 2) & 3) = (l % 4) ^ ((l >> 4) & 3) (blocks start at multiples of 16).
  const _Float16* Ab = A + (int64_t)m0 * K;
  const _Float16* Bb = B + (int64_t)n0 * K;
  const int panel = 256 * K * 2;
  const int voff = ((lane >> 2) * K + (((lane & 3) ^ ((lane >> 4) & 3)) * 8)) * 2;
  const int step = 16 * K * 2;
  const int KT = K / kW4BK;
  // One operand's four copies of tile t into its slot; past the last tile the lane offset is
  // out of range, so the copies return zeros without a memory access and the body stays the same.
  auto issue = [&](int t, int slot, int op) {
    char* st = lds + slot * kW4Stage + op * kW4Op + w * 4096;
    const bool live = t < KT;
    const int soff = (w * 64 * K + (live ? t : 0) * kW4BK) * 2;
    copy4_to_lds(op == 0 ? Ab : Bb, panel, st, live ? voff : kCopyNone, soff, step);
  };

  // Fragments of v_mfma_f32_32x32x16_f16: lane l supplies row l & 31 of a 32-row tile at the
  // k-group (chunk) 2 kk + (l >> 5) of k-step kk. Rows of a tile start at multiples of 32, so the
  // swizzle term (r >> 2) & 3 depends on the lane only.
  const int frow = lane & 31, fhalf = lane >> 5;
  const int fsw = (frow >> 2) & 3;
  const int a_row = (wm * kW4WT + frow) * kW4Row, b_row = kW4Op + (wn * kW4WT + frow) * kW4Row;
  f16x8 fa[2][4], fb[2][4];
  auto read_frags = [&](int slot, int kk, int buf) {
    const char* st = lds + slot * kW4Stage;
    const int c = ((2 * kk + fhalf) ^ fsw) << 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) fa[buf][i] = *reinterpret_cast<const f16x8*>(st + a_row + i * 32 * kW4Row + c);
#pragma unroll
    for (int j = 0; j < 4; ++j) fb[buf][j] = *reinterpret_cast<const f16x8*>(st + b_row + j * 32 * kW4Row + c);
  };
  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};
  auto mfmas = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[buf][j], fa[buf][i], acc[i][j], 0, 0, 0);
  };

  // Prologue: tiles 0 .. STAGES-2 in flight, wait for tile 0, read its first k-step.
#pragma unroll
  for (int t = 0; t < STAGES - 1; ++t) {
    issue(t, t, 0);
    issue(t, t, 1);
  }
  wait_vmcnt<(STAGES - 2) * 8>();
  barrier_nofence();
  read_frags(0, 0, 0);

  int slot = 0;  // slot of tile t
  for (int t = 0; t < KT; ++t) {
    const int nslot = slot + 1 == STAGES ? 0 : slot + 1;  // tile t+1 (read in k-step 1; past the
    const int islot = slot == 0 ? STAGES - 1 : slot - 1;  // end a set nobody uses); copies refill t-1's slot
    wait_vmcnt<(STAGES - 3) * 8>();  // this wavefront's copies of tile t+1 have landed
    barrier_nofence();
    // k-step 0: multiply set 0, read k-step 1 of tile t into set 1, copy A of tile t+STAGES-1.
    read_frags(slot, 1, 1);
    issue(t + STAGES - 1, islot, 0);
    mfmas(0);
    sched_spread<16, 8, 4>();
    // k-step 1: multiply set 1, read k-step 0 of tile t+1 into set 0, copy B of tile t+STAGES-1.
    read_frags(nslot, 0, 0);
    issue(t + STAGES - 1, islot, 1);
    mfmas(1);
    sched_spread<16, 8, 4>();
    slot = nslot;
  }
  wait_vmcnt<0>();  // copies past the last tile still land in the ring

  // Every wavefront has consumed its last fragments (its MFMAs waited for them) and no copy is
  // in flight: after this barrier the ring is free for the epilogue staging.
  barrier_nofence();
  // acc[i][j] holds C^T: lane -> row m = i*32 + (lane & 31) of the wave tile and columns
  // n = j*32 + 8 g + 4 (lane >> 5) + {0..3} for register group g = r / 4.
  char* stage = lds + w * (kW4WT * kW4Pitch);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f16x4 h;
        h[0] = (_Float16)acc[i][j][g * 4 + 0];
        h[1] = (_Float16)acc[i][j][g * 4 + 1];
        h[2] = (_Float16)acc[i][j][g * 4 + 2];
        h[3] = (_Float16)acc[i][j][g * 4 + 3];
        const int m = i * 32 + (lane & 31);
        const int n = j * 32 + g * 8 + (lane >> 5) * 4;
        *reinterpret_cast<f16x4*>(stage + m * kW4Pitch + n * 2) = h;
      }
  // The region is private to this wavefront: its own LDS writes must land before its reads.
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  constexpr int kRowChunks = kW4WT * 2 / 16;
  _Float16* Cw = C + (int64_t)(m0 + wm * kW4WT) * N + n0 + wn * kW4WT;
#pragma unroll 4
  for (int id = lane; id < kW4WT * kRowChunks; id += 64) {
    const int r = id / kRowChunks, c = id % kRowChunks;
    const u32x4 v = *reinterpret_cast<const u32x4*>(stage + r * kW4Pitch + c * 16);
    *reinterpret_cast<u32x4*>(Cw + (int64_t)r * N + c * 8) = v;
  }
}

// gemm_f16_w4s_kernel: the four-wavefront 128 x 128 tiling of gemm_f16_w4_kernel on
// v_mfma_f32_16x16x32_f16, which moves half the accumulator bytes per flop of the 32x32x16 form
// (on a part that runs the GEMM at its power limit, less energy per flop is a higher clock). The
// 64 accumulator tuples fill the 256 AGPRs; A fragments are reloaded row by row as their MFMAs
// finish (one set), B fragments are double buffered (every row uses them). LDS rows of 64 bytes
// with chunk c of row r at c ^ ((r >> 1) & 3): conflict-free for 16-row fragment reads (measured).
template <int STAGES>
__global__ void __launch_bounds__(256, 1)
    gemm_f16_w4s_kernel(const _Float16* __restrict__ A, const _Float16* __restrict__ B, _Float16* __restrict__ C,
                        int M, int N, int K, int tiles_m, int tiles_n) {
  static_assert(STAGES >= 3 && (STAGES - 2) * 8 <= 63, "copies in flight must fit vmcnt");
  typedef float f32x4v __attribute__((ext_vector_type(4)));
  __shared__ __attribute__((aligned(1024))) char lds[w4_lds_bytes<STAGES>()];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w >> 1, wn = w & 1;

  const int G = gridDim.x;
  int lin = blockIdx.x;
  if ((G & 7) == 0) lin = (lin & 7) * (G >> 3) + (lin >> 3);
  constexpr int kGroupM = 4;
  const int per_group = kGroupM * tiles_n;
  const int group = lin / per_group;
  const int first_m = group * kGroupM;
  const int gm = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
  const int in_group = lin - group * per_group;
  const int tm = first_m + in_group % gm;
  const int tn = in_group / gm;
  const int m0 = tm * kW4BM, n0 = tn * kW4BN;

  // Copy lanes: row l / 4 of a 16-row block, physical chunk l % 4 holding logical chunk
  // (l % 4) ^ ((row >> 1) & 3) = (l % 4) ^ ((l >> 3) & 3).
  const _Float16* Ab = A + (int64_t)m0 * K;
  const _Float16* Bb = B + (int64_t)n0 * K;
  const int panel = 256 * K * 2;
  const int voff = ((lane >> 2) * K + (((lane & 3) ^ ((lane >> 3) & 3)) * 8)) * 2;
  const int step = 16 * K * 2;
  const int KT = K / kW4BK;
  auto issue = [&](int t, int slot) {
    char* st = lds + slot * kW4Stage + w * 4096;
    const bool live = t < KT;
    const int soff = (w * 64 * K + (live ? t : 0) * kW4BK) * 2;
    copy4_to_lds(Ab, panel, st, live ? voff : kCopyNone, soff, step);
    copy4_to_lds(Bb, panel, st + kW4Op, live ? voff : kCopyNone, soff, step);
  };
  const int frow = lane & 15, fk = lane >> 4;
  const int fo = frow * kW4Row + ((fk ^ ((frow >> 1) & 3)) << 4);
  const int a_off = wm * kW4WT * kW4Row + fo, b_off = kW4Op + wn * kW4WT * kW4Row + fo;
  f16x8 fa[8], fb[2][8];
  auto read_a = [&](int slot, int i) {
    fa[i] = *reinterpret_cast<const f16x8*>(lds + slot * kW4Stage + a_off + i * 16 * kW4Row);
  };
  auto read_b = [&](int slot, int buf, int j) {
    fb[buf][j] = *reinterpret_cast<const f16x8*>(lds + slot * kW4Stage + b_off + j * 16 * kW4Row);
  };
  // acc[i][j] = C^T block: lane l holds C[i*16 + (l & 15)][j*16 + 4*(l >> 4) + r], r < 4.
  f32x4v acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int t = 0; t < STAGES - 1; ++t) issue(t, t);
  wait_vmcnt<(STAGES - 2) * 8>();
  barrier_nofence();
#pragma unroll
  for (int j = 0; j < 8; ++j) read_b(0, 0, j);
#pragma unroll
  for (int i = 0; i < 8; ++i) read_a(0, i);

  int slot = 0;
  auto body = [&](int t, auto cur_c) {
    constexpr int cur = decltype(cur_c)::value, nxt = cur ^ 1;
    const int nslot = slot + 1 == STAGES ? 0 : slot + 1;
    const int islot = slot == 0 ? STAGES - 1 : slot - 1;
    wait_vmcnt<(STAGES - 3) * 8>();
    barrier_nofence();
#pragma unroll
    for (int j = 0; j < 8; ++j) read_b(nslot, nxt, j);
    issue(t + STAGES - 1, islot);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fb[cur][j], fa[i], acc[i][j], 0, 0, 0);
      read_a(nslot, i);
    }
    sched_spread<64, 16, 8>();
    slot = nslot;
  };
  int t = 0;
  for (; t + 1 < KT; t += 2) {
    body(t, std::integral_constant<int, 0>{});
    body(t + 1, std::integral_constant<int, 1>{});
  }
  if (t < KT) body(t, std::integral_constant<int, 0>{});
  wait_vmcnt<0>();
  barrier_nofence();
  char* stage = lds + w * (kW4WT * kW4Pitch);
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      f16x4 h;
      h[0] = (_Float16)acc[i][j][0];
      h[1] = (_Float16)acc[i][j][1];
      h[2] = (_Float16)acc[i][j][2];
      h[3] = (_Float16)acc[i][j][3];
      const int m = i * 16 + (lane & 15);
      const int n = j * 16 + 4 * (lane >> 4);
      *reinterpret_cast<f16x4*>(stage + m * kW4Pitch + n * 2) = h;
    }
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  constexpr int kRowChunks = kW4WT * 2 / 16;
  _Float16* Cw = C + (int64_t)(m0 + wm * kW4WT) * N + n0 + wn * kW4WT;
#pragma unroll 4
  for (int id = lane; id < kW4WT * kRowChunks; id += 64) {
    const int r = id / kRowChunks, c = id % kRowChunks;
    const u32x4 v = *reinterpret_cast<const u32x4*>(stage + r * kW4Pitch + c * 16);
    *reinterpret_cast<u32x4*>(Cw + (int64_t)r * N + c * 8) = v;
  }
}

// ---------------------------------------------------------------------------------------
// gemm_f16_w4k_kernel: the four-wavefront 128 x 128 tiling of gemm_f16_w4_kernel with 64-deep
// k-tiles. A copy lane moves 16 bytes of a row's 128-byte k-segment, so every segment is one
// whole L2 line: half the L2 requests of 32-deep tiles for the same bytes (64-byte segments make
// the L2 look up each line twice).
//
// LDS: two 32 KiB slots for A tiles and three for B tiles (160 KiB); tile t sits in A slot t % 2
// and B slot t % 3. Rows are 128 bytes, chunk c of row r at c ^ ((r >> 1) & 7), for which the
// 32x32x16 fragment reads (32 rows x 2 k-groups per ds_read_b128) are free of bank conflicts
// (measured). A copy fills eight rows (1 KiB); its lanes' swizzle depends on the block's parity
// only, so a wavefront keeps one lane offset per parity and four copies share one M0.
//
// Schedule, k-step s = 4t + kk of tile t (fragments double buffered in VGPRs, k-step s reads
// those of s + 1): the one barrier of tile t sits between its k-steps 2 and 3. Before it every
// wavefront waits for its own copies of tile t + 1 and for its reads of tile t (k-step 2 read the
// last of them); after it tile t + 1 is visible to all and nobody reads tile t's slots. k-step 3
// reads tile t + 1's first fragments and issues the A copies of tile t + 2 into tile t's A slot.
// The B copies of tile t + 2 go to the B slot tile t - 1 left at the previous barrier, spread
// over k-steps 0-2: the copies of a 64-deep tile are 64 KiB per CU, twice what the texture
// addresser takes in one k-step, and in one burst they stalled the issuing wavefront's MFMAs
// (about 60 cycles per copy, measured). Every copy has at least four k-steps to land.
// ---------------------------------------------------------------------------------------
constexpr int kW4kBK = 64;
constexpr int kW4kRow = kW4kBK * 2;   // 128-byte LDS rows
constexpr int kW4kOp = 256 * kW4kRow; // 32 KiB: one operand tile
constexpr int kW4kB0 = 2 * kW4kOp;    // B slots after the two A slots
constexpr int kW4kLds = 5 * kW4kOp > kW4Epi ? 5 * kW4kOp : kW4Epi;

// Copy U (< 4) of a group of four sharing one M0: the LDS block dst + U KiB from global offset
// soff + U step (plus the lane offset voff) of the buffer of nbytes at base.
template <int U>
__device__ __forceinline__ void copy_u_to_lds(const void* base, int nbytes, char* dst, int voff, int soff, int step) {
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, nbytes, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)dst, 16, voff, soff + U * step - U * 1024, U * 1024, 0);
}

// Copy q (< 8) of an operand tile issued after MFMA m of k-step kk, or -1: the B copies of tile
// t + 2 after MFMAs 1, 6, 11 of k-steps 0 and 1 and 9, 13 of k-step 2; the A copies after every
// even MFMA of k-step 3.
template <int KK, int M>
constexpr int w4k_copy() {
  if constexpr (KK == 3) return M % 2 == 0 ? M / 2 : -1;
  else if constexpr (KK < 2) return M == 1 ? 3 * KK : M == 6 ? 3 * KK + 1 : M == 11 ? 3 * KK + 2 : -1;
  else return M == 9 ? 6 : M == 13 ? 7 : -1;
}

__global__ void __launch_bounds__(256, 1)
    gemm_f16_w4k_kernel(const _Float16* __restrict__ A, const _Float16* __restrict__ B, _Float16* __restrict__ C,
                        int M, int N, int K, int tiles_m, int tiles_n) {
  __shared__ __attribute__((aligned(1024))) char lds[kW4kLds];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w >> 1, wn = w & 1;

  const int G = gridDim.x;
  int lin = blockIdx.x;
  if ((G & 7) == 0) lin = (lin & 7) * (G >> 3) + (lin >> 3);
  constexpr int kGroupM = 4;
  const int per_group = kGroupM * tiles_n;
  const int group = lin / per_group;
  const int first_m = group * kGroupM;
  const int gm = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
  const int in_group = lin - group * per_group;
  const int tm = first_m + in_group % gm;
  const int tn = in_group / gm;
  const int m0 = tm * kW4BM, n0 = tn * kW4BN;

  // Copy lanes: lane l fills row 8b + l / 8 of block b, physical chunk l % 8 with logical chunk
  // (l % 8) ^ (((8b + l / 8) >> 1) & 7) = (l % 8) ^ (l >> 4) ^ 4 (b & 1). Wavefront w moves
  // blocks 8w .. 8w + 7 (rows 64w .. 64w + 63) of each operand tile: copy q < 8 is block 8w + q.
  const _Float16* Ab = A + (int64_t)m0 * K;
  const _Float16* Bb = B + (int64_t)n0 * K;
  const int panel = 256 * K * 2;
  const int lrow = (lane >> 3) * K * 2;
  const int ve = lrow + (((lane & 7) ^ (lane >> 4)) << 4);
  const int vo = lrow + (((lane & 7) ^ (lane >> 4) ^ 4) << 4);
  const int step = 8 * K * 2;
  const int KT = K / kW4kBK;
  // Copy q of tile t of one operand into the slot at dst (past the last tile: zeros, no access).
  auto copy_q = [&](auto q_c, const void* base, char* dst, int t) {
    constexpr int q = decltype(q_c)::value, half = q >> 2, u = q & 3;
    const bool live = t < KT;
    const int voff = live ? ((u & 1) ? vo : ve) : kCopyNone;
    const int soff = ((w * 64 + half * 32) * K + (live ? t : 0) * kW4kBK) * 2;
    copy_u_to_lds<u>(base, panel, dst + w * 8 * 1024 + half * 4096, voff, soff, step);
  };

  // Fragments of v_mfma_f32_32x32x16_f16: lane l supplies row l & 31 of a 32-row tile at logical
  // chunk 2 kk + (l >> 5) of k-step kk; tiles start at multiples of 32, so the swizzle term
  // ((r >> 1) & 7) depends on the lane only.
  const int frow = lane & 31, fhalf = lane >> 5;
  const int fsw = (frow >> 1) & 7;
  const int a_row = (wm * kW4WT + frow) * kW4kRow, b_row = (wn * kW4WT + frow) * kW4kRow;
  f16x8 fa[2][4], fb[2][4];
  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  // Read r < 8 of a k-step's fragments in the order the MFMAs consume them: A0, B0..B3, A1..A3.
  auto read = [&](auto buf_c, auto r_c, const char* ab, const char* bb) {
    constexpr int buf = decltype(buf_c)::value, r = decltype(r_c)::value;
    if constexpr (r == 0) fa[buf][0] = *reinterpret_cast<const f16x8*>(ab);
    else if constexpr (r <= 4) fb[buf][r - 1] = *reinterpret_cast<const f16x8*>(bb + (r - 1) * 32 * kW4kRow);
    else fa[buf][r - 4] = *reinterpret_cast<const f16x8*>(ab + (r - 4) * 32 * kW4kRow);
  };
  // MFMA m of k-step KK on fragment set CUR, then (every RS-th MFMA, eight in all) the next read
  // into the other set and the copy that falls due. Each group is fenced, so issue order is
  // program order: left to itself the compiler hoists every read above every copy (it cannot tell
  // that the LDS slots differ) and the copies end up in one burst.
  auto mstep = [&](auto cur_c, auto kk_c, auto m_c, auto rs_c, const char* ab, const char* bb, char* cdst, int tc) {
    constexpr int cur = decltype(cur_c)::value, KK = decltype(kk_c)::value, m = decltype(m_c)::value;
    constexpr int RS = decltype(rs_c)::value, q = w4k_copy<KK, m>();
    acc[m >> 2][m & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[cur][m & 3], fa[cur][m >> 2], acc[m >> 2][m & 3], 0, 0, 0);
    if constexpr (m % RS == 0 && m / RS < 8)
      read(std::integral_constant<int, cur ^ 1>{}, std::integral_constant<int, m / RS>{}, ab, bb);
    if constexpr (q >= 0)
      copy_q(std::integral_constant<int, q>{}, KK == 3 ? static_cast<const void*>(Ab) : static_cast<const void*>(Bb),
             cdst, tc);
    __builtin_amdgcn_sched_barrier(0);
  };
  // One k-step: 16 MFMAs on set CUR; the next k-step's fragments from k-step kr of the tile in
  // A slot as and B slot bs; the copies due in k-step KK (of tile tc, into the slot at cdst).
  auto kstep = [&](auto cur_c, auto kk_c, auto rs_c, int as, int bs, int kr, char* cdst, int tc) {
    const int c = ((2 * kr + fhalf) ^ fsw) << 4;
    const char* ab = lds + as * kW4kOp + a_row + c;
    const char* bb = lds + kW4kB0 + bs * kW4kOp + b_row + c;
    [&]<int... Ms>(std::integer_sequence<int, Ms...>) {
      (mstep(cur_c, kk_c, std::integral_constant<int, Ms>{}, rs_c, ab, bb, cdst, tc), ...);
    }(std::make_integer_sequence<int, 16>{});
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;

  // Prologue: B0, A0, B1, A1 in flight (the loop waits on this order), wait for tile 0, read its
  // first k-step.
  [&]<int... Qs>(std::integer_sequence<int, Qs...>) {
    (copy_q(std::integral_constant<int, Qs>{}, Bb, lds + kW4kB0, 0), ...);
    (copy_q(std::integral_constant<int, Qs>{}, Ab, lds, 0), ...);
    (copy_q(std::integral_constant<int, Qs>{}, Bb, lds + kW4kB0 + kW4kOp, 1), ...);
    (copy_q(std::integral_constant<int, Qs>{}, Ab, lds + kW4kOp, 1), ...);
  }(std::make_integer_sequence<int, 8>{});
  wait_vmcnt<16>();
  barrier_nofence();
  {
    const int c = (fhalf ^ fsw) << 4;
    [&]<int... Rs>(std::integer_sequence<int, Rs...>) {
      (read(I0{}, std::integral_constant<int, Rs>{}, lds + a_row + c, lds + kW4kB0 + b_row + c), ...);
    }(std::make_integer_sequence<int, 8>{});
  }

  int as = 0, bs = 0;  // slots of tile t: t % 2, t % 3
  for (int t = 0; t < KT; ++t) {
    const int as1 = as ^ 1, bs1 = bs == 2 ? 0 : bs + 1, bs2 = bs == 0 ? 2 : bs - 1;  // t+1; t+2 = t-1
    char* bfill = lds + kW4kB0 + bs2 * kW4kOp;
    kstep(I0{}, I0{}, I2{}, as, bs, 1, bfill, t + 2);
    kstep(I1{}, I1{}, I2{}, as, bs, 2, bfill, t + 2);
    kstep(I0{}, I2{}, I1{}, as, bs, 3, bfill, t + 2);  // reads early: they are waited for at the barrier
    // Tiles t + 1 (A and B) have landed for this wavefront (the B copies of t + 2 may still be in
    // flight) and its reads of tile t have returned.
    wait_vmcnt<8>();
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    barrier_nofence();
    // Past the last tile the reads see zeros that are never multiplied.
    kstep(I1{}, I3{}, I1{}, as1, bs1, 0, lds + as * kW4kOp, t + 2);
    as = as1;
    bs = bs1;
  }
  wait_vmcnt<0>();
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  // No copy is in flight and no wavefront reads the slots after this barrier: the epilogue
  // stages each wavefront's tile over them.
  barrier_nofence();
  char* stage = lds + w * (kW4WT * kW4Pitch);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f16x4 h;
        h[0] = (_Float16)acc[i][j][g * 4 + 0];
        h[1] = (_Float16)acc[i][j][g * 4 + 1];
        h[2] = (_Float16)acc[i][j][g * 4 + 2];
        h[3] = (_Float16)acc[i][j][g * 4 + 3];
        const int m = i * 32 + (lane & 31);
        const int n = j * 32 + g * 8 + (lane >> 5) * 4;
        *reinterpret_cast<f16x4*>(stage + m * kW4Pitch + n * 2) = h;
      }
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  constexpr int kRowChunks = kW4WT * 2 / 16;
  _Float16* Cw = C + (int64_t)(m0 + wm * kW4WT) * N + n0 + wn * kW4WT;
#pragma unroll 4
  for (int id = lane; id < kW4WT * kRowChunks; id += 64) {
    const int r = id / kRowChunks, c = id % kRowChunks;
    const u32x4 v = *reinterpret_cast<const u32x4*>(stage + r * kW4Pitch + c * 16);
    *reinterpret_cast<u32x4*>(Cw + (int64_t)r * N + c * 8) = v;
  }
}

// ---------------------------------------------------------------------------------------
// gemm_f16_w4k16_kernel: gemm_f16_w4k_kernel's tiling, slots and copies on
// v_mfma_f32_16x16x32_f16. With no memory traffic at all, back-to-back 16x16x32 MFMAs sustain
// 73% of the dense peak against 67% for 32x32x16 (measured: the part holds 2.0 GHz instead of
// 1.66 GHz at its power limit, for 18 instead of 16 issue cycles per MFMA), and the 64-deep
// kernel runs at that power limit. The 64 accumulator tuples fill the 256 AGPRs; the MFMAs are
// issued from inline assembly with the accumulators bound to AGPRs so that the register
// allocator keeps each tuple in place (left to itself it rotated them through VGPRs).
//
// Per 64-deep tile two k-steps of 32, each 64 MFMAs with 16 fragment reads for the next k-step
// (double buffered) and 8 copies: the B copies of tile t + 2 in k-step 0 (into the B slot tile
// t - 1 left), the A copies in k-step 1 after the tile's barrier (into tile t's A slot).
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256, 1)
    gemm_f16_w4k16_kernel(const _Float16* __restrict__ A, const _Float16* __restrict__ B, _Float16* __restrict__ C,
                          int M, int N, int K, int tiles_m, int tiles_n) {
  // All arguments in scalar registers before anything else (one wait for their loads, not one per
  // argument between the computations that need them).
  asm volatile("" ::"s"(A), "s"(B), "s"(C), "s"(M), "s"(N), "s"(K), "s"(tiles_m), "s"(tiles_n));
  typedef float f32x4v __attribute__((ext_vector_type(4)));
  __shared__ __attribute__((aligned(1024))) char lds[kW4kLds];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w >> 1, wn = w & 1;

  const int G = gridDim.x;
  int lin = blockIdx.x;
  if ((G & 7) == 0) lin = (lin & 7) * (G >> 3) + (lin >> 3);
  constexpr int kGroupM = 4;
  const int per_group = kGroupM * tiles_n;
  const int group = lin / per_group;
  const int first_m = group * kGroupM;
  const int gm = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
  const int in_group = lin - group * per_group;
  const int tm = first_m + in_group % gm;
  const int tn = in_group / gm;
  const int m0 = tm * kW4BM, n0 = tn * kW4BN;

  // Copies as in gemm_f16_w4k_kernel.
  const _Float16* Ab = A + (int64_t)m0 * K;
  const _Float16* Bb = B + (int64_t)n0 * K;
  const int panel = 256 * K * 2;
  const int lrow = (lane >> 3) * K * 2;
  const int ve = lrow + (((lane & 7) ^ (lane >> 4)) << 4);
  const int vo = lrow + (((lane & 7) ^ (lane >> 4) ^ 4) << 4);
  const int step = 8 * K * 2;
  const int KT = K / kW4kBK;
  auto copy_q = [&](auto q_c, const void* base, char* dst, int t) {
    constexpr int q = decltype(q_c)::value, half = q >> 2, u = q & 3;
    const bool live = t < KT;
    const int voff = live ? ((u & 1) ? vo : ve) : kCopyNone;
    const int soff = ((w * 64 + half * 32) * K + (live ? t : 0) * kW4kBK) * 2;
    copy_u_to_lds<u>(base, panel, dst + w * 8 * 1024 + half * 4096, voff, soff, step);
  };

  // Fragments of v_mfma_f32_16x16x32_f16: lane l supplies row l & 15 of a 16-row group at
  // logical chunk 4 ks + (l >> 4) of k-step ks; groups start at multiples of 16, so the swizzle
  // term ((r >> 1) & 7) depends on the lane only (conflict-free, measured).
  const int frow = lane & 15, fk = lane >> 4;
  const int fsw = (frow >> 1) & 7;
  const int a_row = (wm * kW4WT + frow) * kW4kRow, b_row = (wn * kW4WT + frow) * kW4kRow;
  f16x8 fa[2][8], fb[2][8];
  // acc[i][j] = C^T block: lane l holds C[i*16 + (l & 15)][j*16 + 4*(l >> 4) + r], r < 4.
  f32x4v acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};

  // Read r < 16 of a k-step's fragments in the order the MFMAs consume them: A0, B0..B7, A1..A7.
  auto read = [&](auto buf_c, auto r_c, const char* ab, const char* bb) {
    constexpr int buf = decltype(buf_c)::value, r = decltype(r_c)::value;
    if constexpr (r == 0) fa[buf][0] = *reinterpret_cast<const f16x8*>(ab);
    else if constexpr (r <= 8) fb[buf][r - 1] = *reinterpret_cast<const f16x8*>(bb + (r - 1) * 16 * kW4kRow);
    else fa[buf][r - 8] = *reinterpret_cast<const f16x8*>(ab + (r - 8) * 16 * kW4kRow);
  };
  // MFMA m of a k-step on fragment set CUR; read m / RS after every RS-th MFMA (sixteen in all);
  // copy q after MFMA 8q + 3. Fenced groups keep issue order = program order. The 8 x 8 tuples
  // are visited in serpentine order (odd A fragments walk the B fragments backwards), so each
  // MFMA changes one operand from the one before it; the part runs this kernel at its power
  // limit, and fewer operand changes measured 0.3-0.9% faster (same sums, same bits).
  auto mstep = [&](auto cur_c, auto m_c, auto rs_c, auto op_c, const char* ab, const char* bb, char* cdst, int tc) {
    constexpr int cur = decltype(cur_c)::value, m = decltype(m_c)::value, RS = decltype(rs_c)::value;
    constexpr int i = m >> 3, j = (i & 1) ? 7 - (m & 7) : (m & 7);
    __asm__ volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(acc[i][j]) : "v"(fb[cur][j]), "v"(fa[cur][i]));
    if constexpr (m % RS == 0 && m / RS < 16)
      read(std::integral_constant<int, cur ^ 1>{}, std::integral_constant<int, m / RS>{}, ab, bb);
    if constexpr (m % 8 == 3)
      copy_q(std::integral_constant<int, m / 8>{},
             decltype(op_c)::value == 0 ? static_cast<const void*>(Ab) : static_cast<const void*>(Bb), cdst, tc);
    __builtin_amdgcn_sched_barrier(0);
  };
  // One k-step: 64 MFMAs on set CUR; the next fragments from k-step ks of the tile in A slot as
  // and B slot bs; eight copies of operand OP (0: A, 1: B) of tile tc into the slot at cdst.
  auto kstep = [&](auto cur_c, auto rs_c, auto op_c, int as, int bs, int ks, char* cdst, int tc) {
    const int c = ((4 * ks + fk) ^ fsw) << 4;
    const char* ab = lds + as * kW4kOp + a_row + c;
    const char* bb = lds + kW4kB0 + bs * kW4kOp + b_row + c;
    [&]<int... Ms>(std::integer_sequence<int, Ms...>) {
      (mstep(cur_c, std::integral_constant<int, Ms>{}, rs_c, op_c, ab, bb, cdst, tc), ...);
    }(std::make_integer_sequence<int, 64>{});
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I4 = std::integral_constant<int, 4>;

  [&]<int... Qs>(std::integer_sequence<int, Qs...>) {
    (copy_q(std::integral_constant<int, Qs>{}, Bb, lds + kW4kB0, 0), ...);
    (copy_q(std::integral_constant<int, Qs>{}, Ab, lds, 0), ...);
    (copy_q(std::integral_constant<int, Qs>{}, Bb, lds + kW4kB0 + kW4kOp, 1), ...);
    (copy_q(std::integral_constant<int, Qs>{}, Ab, lds + kW4kOp, 1), ...);
  }(std::make_integer_sequence<int, 8>{});
  wait_vmcnt<16>();
  barrier_nofence();
  {
    const int c = (fk ^ fsw) << 4;
    [&]<int... Rs>(std::integer_sequence<int, Rs...>) {
      (read(I0{}, std::integral_constant<int, Rs>{}, lds + a_row + c, lds + kW4kB0 + b_row + c), ...);
    }(std::make_integer_sequence<int, 16>{});
  }

  int as = 0, bs = 0;  // slots of tile t: t % 2, t % 3
  for (int t = 0; t < KT; ++t) {
    const int as1 = as ^ 1, bs1 = bs == 2 ? 0 : bs + 1, bs2 = bs == 0 ? 2 : bs - 1;
    // k-step 0: reads of k-step 1 early (waited for at the barrier); B copies of tile t + 2.
    kstep(I0{}, I2{}, I1{}, as, bs, 1, lds + kW4kB0 + bs2 * kW4kOp, t + 2);
    wait_vmcnt<8>();
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    barrier_nofence();
    // k-step 1: tile t + 1's first fragments (zeros past the last tile); A copies of tile t + 2.
    kstep(I1{}, I4{}, I0{}, as1, bs1, 0, lds + as * kW4kOp, t + 2);
    as = as1;
    bs = bs1;
  }
  // The MFMAs above are inline assembly: let the last ones retire before their accumulators are
  // read (the compiler inserts no wait states for them).
  __asm__ volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  wait_vmcnt<0>();
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  barrier_nofence();
  char* stage = lds + w * (kW4WT * kW4Pitch);
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      f16x4 h;
      h[0] = (_Float16)acc[i][j][0];
      h[1] = (_Float16)acc[i][j][1];
      h[2] = (_Float16)acc[i][j][2];
      h[3] = (_Float16)acc[i][j][3];
      const int m = i * 16 + (lane & 15);
      const int n = j * 16 + 4 * (lane >> 4);
      *reinterpret_cast<f16x4*>(stage + m * kW4Pitch + n * 2) = h;
    }
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  constexpr int kRowChunks = kW4WT * 2 / 16;
  _Float16* Cw = C + (int64_t)(m0 + wm * kW4WT) * N + n0 + wn * kW4WT;
#pragma unroll 4
  for (int id = lane; id < kW4WT * kRowChunks; id += 64) {
    const int r = id / kRowChunks, c = id % kRowChunks;
    const u32x4 v = *reinterpret_cast<const u32x4*>(stage + r * kW4Pitch + c * 16);
    // Non-temporal: C (32 MiB at 4096^2, the size of all eight L2s) is not read back here, and
    // streaming it past the L2 measured 1.3% faster than ordinary stores.
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(Cw + (int64_t)r * N + c * 8));
  }
}

// ---------------------------------------------------------------------------------------
// gemm_f16_w8k16_kernel: the 256x256x64 tile, slots and copy schedule of gemm_f16_w4k16_kernel
// with eight wavefronts, two per SIMD, each a 128x64 wave tile (8 x 4 accumulator tuples, 128
// AGPRs, so that two wavefronts share a SIMD's registers); per 64-deep tile each wavefront issues
// two k-steps of 32 MFMAs, 12 fragment reads for the next k-step and four copies. Kept beside the
// pick as the measured answer to whether a second wavefront per SIMD, multiplying while the other
// reads and copies, hides the data movement: it reads 1.5 times the LDS bytes per flop, and at
// 4096^3 it ran 104.3-106.0 us against 97.1-98.9 us for gemm_f16_w4k16_kernel (same bits, one box).
// ---------------------------------------------------------------------------------------
constexpr int kW8WM = 128, kW8WN = 64;
constexpr int kW8Pitch = kW8WN * 2 + 16;
static_assert(8 * kW8WM * kW8Pitch <= kW4kLds, "epilogue staging fits");

__global__ void __launch_bounds__(512, 1)
    gemm_f16_w8k16_kernel(const _Float16* __restrict__ A, const _Float16* __restrict__ B, _Float16* __restrict__ C,
                          int M, int N, int K, int tiles_m, int tiles_n) {
  asm volatile("" ::"s"(A), "s"(B), "s"(C), "s"(M), "s"(N), "s"(K), "s"(tiles_m), "s"(tiles_n));
  typedef float f32x4v __attribute__((ext_vector_type(4)));
  __shared__ __attribute__((aligned(1024))) char lds[kW4kLds];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w >> 2, wn = w & 3;

  const int G = gridDim.x;
  int lin = blockIdx.x;
  if ((G & 7) == 0) lin = (lin & 7) * (G >> 3) + (lin >> 3);
  constexpr int kGroupM = 4;
  const int per_group = kGroupM * tiles_n;
  const int group = lin / per_group;
  const int first_m = group * kGroupM;
  const int gm = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
  const int in_group = lin - group * per_group;
  const int tm = first_m + in_group % gm;
  const int tn = in_group / gm;
  const int m0 = tm * kW4BM, n0 = tn * kW4BN;

  const _Float16* Ab = A + (int64_t)m0 * K;
  const _Float16* Bb = B + (int64_t)n0 * K;
  const int panel = 256 * K * 2;
  const int lrow = (lane >> 3) * K * 2;
  const int ve = lrow + (((lane & 7) ^ (lane >> 4)) << 4);
  const int vo = lrow + (((lane & 7) ^ (lane >> 4) ^ 4) << 4);
  const int step = 8 * K * 2;
  const int KT = K / kW4kBK;
  // Copy u (< 4) of this wavefront's 32 rows of an operand tile: rows w 32 + 8 u .. + 8.
  auto copy_q = [&](auto q_c, const void* base, char* dst, int t) {
    constexpr int u = decltype(q_c)::value;
    const bool live = t < KT;
    const int voff = live ? ((u & 1) ? vo : ve) : kCopyNone;
    const int soff = ((w * 32) * K + (live ? t : 0) * kW4kBK) * 2;
    copy_u_to_lds<u>(base, panel, dst + w * 4 * 1024, voff, soff, step);
  };

  const int frow = lane & 15, fk = lane >> 4;
  const int fsw = (frow >> 1) & 7;
  const int a_row = (wm * kW8WM + frow) * kW4kRow, b_row = (wn * kW8WN + frow) * kW4kRow;
  f16x8 fa[2][8], fb[2][4];
  f32x4v acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};

  // Read r < 12 in the order the MFMAs consume them: A0, B0..B3, A1..A7.
  auto read = [&](auto buf_c, auto r_c, const char* ab, const char* bb) {
    constexpr int buf = decltype(buf_c)::value, r = decltype(r_c)::value;
    if constexpr (r == 0) fa[buf][0] = *reinterpret_cast<const f16x8*>(ab);
    else if constexpr (r <= 4) fb[buf][r - 1] = *reinterpret_cast<const f16x8*>(bb + (r - 1) * 16 * kW4kRow);
    else fa[buf][r - 4] = *reinterpret_cast<const f16x8*>(ab + (r - 4) * 16 * kW4kRow);
  };
  // MFMA m (< 32) on set CUR, serpentine over the 8 x 4 tuples; read r of the next set after MFMA
  // (8 r) / 3; copy q after MFMA 8 q + 3.
  auto mstep = [&](auto cur_c, auto m_c, auto op_c, const char* ab, const char* bb, char* cdst, int tc) {
    constexpr int cur = decltype(cur_c)::value, m = decltype(m_c)::value;
    constexpr int i = m >> 2, j = (i & 1) ? 3 - (m & 3) : (m & 3);
    __asm__ volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(acc[i][j]) : "v"(fb[cur][j]), "v"(fa[cur][i]));
    [&]<int... Rs>(std::integer_sequence<int, Rs...>) {
      ((((8 * Rs) / 3 == m) ? (read(std::integral_constant<int, cur ^ 1>{}, std::integral_constant<int, Rs>{}, ab, bb), 0)
                            : 0),
       ...);
    }(std::make_integer_sequence<int, 12>{});
    if constexpr (m % 8 == 3)
      copy_q(std::integral_constant<int, m / 8>{},
             decltype(op_c)::value == 0 ? static_cast<const void*>(Ab) : static_cast<const void*>(Bb), cdst, tc);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto kstep = [&](auto cur_c, auto op_c, const char* ab, const char* bb, char* cdst, int tc) {
    [&]<int... Ms>(std::integer_sequence<int, Ms...>) {
      (mstep(cur_c, std::integral_constant<int, Ms>{}, op_c, ab, bb, cdst, tc), ...);
    }(std::make_integer_sequence<int, 32>{});
  };
  auto frag_ptrs = [&](int as, int bs, int ks, const char** ab, const char** bb) {
    const int c = ((4 * ks + fk) ^ fsw) << 4;
    *ab = lds + as * kW4kOp + a_row + c;
    *bb = lds + kW4kB0 + bs * kW4kOp + b_row + c;
  };
  auto read_all = [&](auto buf_c, const char* ab, const char* bb) {
    [&]<int... Rs>(std::integer_sequence<int, Rs...>) { (read(buf_c, std::integral_constant<int, Rs>{}, ab, bb), ...); }(
        std::make_integer_sequence<int, 12>{});
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;

  [&]<int... Qs>(std::integer_sequence<int, Qs...>) {
    (copy_q(std::integral_constant<int, Qs>{}, Bb, lds + kW4kB0, 0), ...);
    (copy_q(std::integral_constant<int, Qs>{}, Ab, lds, 0), ...);
    (copy_q(std::integral_constant<int, Qs>{}, Bb, lds + kW4kB0 + kW4kOp, 1), ...);
    (copy_q(std::integral_constant<int, Qs>{}, Ab, lds + kW4kOp, 1), ...);
  }(std::make_integer_sequence<int, 4>{});
  wait_vmcnt<8>();
  barrier_nofence();
  {
    const char *ab, *bb;
    frag_ptrs(0, 0, 0, &ab, &bb);
    read_all(I0{}, ab, bb);
  }
  int as = 0, bs = 0;
  for (int t = 0; t < KT; ++t) {
    const int as1 = as ^ 1, bs1 = bs == 2 ? 0 : bs + 1, bs2 = bs == 0 ? 2 : bs - 1;
    const char *ab, *bb;
    frag_ptrs(as, bs, 1, &ab, &bb);  // k-step 1's fragments, read during k-step 0
    kstep(I0{}, I1{}, ab, bb, lds + kW4kB0 + bs2 * kW4kOp, t + 2);
    wait_vmcnt<4>();
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    barrier_nofence();
    frag_ptrs(as1, bs1, 0, &ab, &bb);  // tile t + 1's first fragments
    kstep(I1{}, I0{}, ab, bb, lds + as * kW4kOp, t + 2);
    as = as1;
    bs = bs1;
  }
  __asm__ volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  wait_vmcnt<0>();
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  barrier_nofence();
  char* stage = lds + w * (kW8WM * kW8Pitch);
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f16x4 h;
      h[0] = (_Float16)acc[i][j][0];
      h[1] = (_Float16)acc[i][j][1];
      h[2] = (_Float16)acc[i][j][2];
      h[3] = (_Float16)acc[i][j][3];
      const int m = i * 16 + (lane & 15);
      const int n = j * 16 + 4 * (lane >> 4);
      *reinterpret_cast<f16x4*>(stage + m * kW8Pitch + n * 2) = h;
    }
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  constexpr int kRowChunks = kW8WN * 2 / 16;
  _Float16* Cw = C + (int64_t)(m0 + wm * kW8WM) * N + n0 + wn * kW8WN;
#pragma unroll 4
  for (int id = lane; id < kW8WM * kRowChunks; id += 64) {
    const int r = id / kRowChunks, c = id % kRowChunks;
    const u32x4 v = *reinterpret_cast<const u32x4*>(stage + r * kW8Pitch + c * 16);
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(Cw + (int64_t)r * N + c * 8));
  }
}

// ---------------------------------------------------------------------------------------
// f32 GEMM, 64x64x64 tiles, eight wavefronts (two k halves x 2x2 quarters).
// ---------------------------------------------------------------------------------------
template <bool BT>
__global__ void __launch_bounds__(512)
    gemm_f32_kernel(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N,
                    int K, int tiles_m, int tiles_n) {
  // All arguments in scalar registers before anything else (one wait for their loads, not one per
  // argument between the computations that need them).
  asm volatile("" ::"s"(A), "s"(B), "s"(C), "s"(M), "s"(N), "s"(K), "s"(tiles_m), "s"(tiles_n), "s"(gridDim.x));
  constexpr int kOp = 64 * 64;  // floats of one operand's k-tile: 64 rows of 256 bytes
  __shared__ __attribute__((aligned(16))) float lds[2 * 2 * kOp];  // two slots of (A, B)
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kh = w >> 2, wm = (w >> 1) & 1, wn = w & 1;
  // XCD-aware tile order (one-dimensional grid): consecutive workgroup ids run on different
  // XCDs, so ids are regrouped to give each XCD a contiguous range, walked in groups of 4
  // tile-rows; an XCD's 32 tiles at 1024^3 are then 4 tile-rows x 8 tile-columns sharing 4 A and
  // 8 B panels in its L2, instead of every XCD fetching every A panel.
  const int G = gridDim.x;
  int lin = blockIdx.x;
  if ((G & 7) == 0) lin = (lin & 7) * (G >> 3) + (lin >> 3);
  constexpr int kGroupM = 4;
  const int per_group = kGroupM * tiles_n;
  const int group = lin / per_group;
  const int first_m = group * kGroupM;
  const int gm = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
  const int in_group = lin - group * per_group;
  const int m0 = (first_m + in_group % gm) * 64, n0 = (in_group / gm) * 64;
  // Copies: an operand's k-tile is 16 instructions of four 256-byte rows; wavefront w issues
  // instructions 2w and 2w + 1, and lane l fills 16-byte slot l & 15 of row 4 (2w + i) + (l >> 4).
  // Rows read down a column of chunks (A's m rows; B's n rows when B is [N][K]) hold chunk c of
  // row r in slot c ^ (r & 7); B's k rows ([K][N]) are read along the row and keep chunk order.
  const float* a_src[2];
  const float* b_src[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = 4 * (2 * w + i) + (lane >> 4), sl = lane & 15;
    a_src[i] = A + (int64_t)(m0 + r) * K + 4 * (sl ^ (r & 7));
    b_src[i] = BT ? B + (int64_t)(n0 + r) * K + 4 * (sl ^ (r & 7)) : B + (int64_t)r * N + n0 + 4 * sl;
  }
  auto copy = [&](int t, int slot) __attribute__((always_inline)) {
    float* as = lds + slot * 2 * kOp;
    float* bs = as + kOp;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint32_t*>(a_src[i] + t * 64),
                                       (lds_void*)(as + (2 * w + i) * 256), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < 2; ++i)
      __builtin_amdgcn_global_load_lds(
          reinterpret_cast<const uint32_t*>(BT ? b_src[i] + t * 64 : b_src[i] + (int64_t)t * 64 * N),
          (lds_void*)(bs + (2 * w + i) * 256), 16, 0, 0);
  };
  const int fi = lane & 31, fh = lane >> 5;
  const int ra = wm * 32 + fi, rb = wn * 32 + fi;
  f32x16 acc = f32x16{};
  auto multiply = [&](int slot) __attribute__((always_inline)) {
    const float* as = lds + slot * 2 * kOp;
    const float* bs = as + kOp;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = 8 * kh + fh + 2 * q;  // the 16-byte chunk of k = 32 kh + 4 fh + 8 q
      const f32x4 av = *reinterpret_cast<const f32x4*>(as + ra * 64 + 4 * (c ^ (ra & 7)));
      f32x4 bv;
      if constexpr (BT) {
        bv = *reinterpret_cast<const f32x4*>(bs + rb * 64 + 4 * (c ^ (rb & 7)));
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[e] = bs[(4 * c + e) * 64 + rb];
      }
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, bv.x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, bv.y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, bv.z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, bv.w, acc, 0, 0, 0);
    }
  };
  // Tile t + 1's copies go into the slot tile t - 1 left (every wavefront passed the barrier
  // after reading it) before tile t's MFMAs, and each wavefront waits for its own copies before
  // the barrier that publishes the tile. The barrier carries no memory fence (that would also
  // wait for the copies in flight); this wavefront's LDS reads are complete by then, since the
  // MFMAs consumed them.
  const int KT = K / 64;
  copy(0, 0);
  wait_vmcnt<0>();
  barrier_nofence();
  for (int t = 0; t < KT; ++t) {
    if (t + 1 < KT) copy(t + 1, (t + 1) & 1);
    __builtin_amdgcn_sched_barrier(0);
    multiply(t & 1);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<0>();
    barrier_nofence();
  }
  // D[i][j]: lane -> column j = lane & 31, rows i = 8 (r / 4) + 4 (lane >> 5) + r % 4. The k
  // halves add in LDS (first half + second half) and the first half stores.
  float* red = lds;  // every wavefront passed the last barrier and every copy landed
  const int q4 = w & 3;
  if (kh == 1) {
#pragma unroll
    for (int r = 0; r < 16; ++r) red[(q4 * 16 + r) * 64 + lane] = acc[r];
  }
  __syncthreads();
  if (kh == 1) return;
  const int j = n0 + rb;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int i = m0 + wm * 32 + (r >> 2) * 8 + fh * 4 + (r & 3);
    C[(int64_t)i * N + j] = acc[r] + red[(q4 * 16 + r) * 64 + lane];
  }
}

// ---------------------------------------------------------------------------------------
// Generic MFMA GEMM: 64x64 tile, 4 wavefronts (2x2 of 32x32), BK = 16, bounds-checked.
// T = _Float16 or float inputs; TO = output type; BT: B stored [N][K] (TN) else [K][N] (NT).
// ---------------------------------------------------------------------------------------
template <typename T, typename TO, bool BT>
__global__ void __launch_bounds__(256)
    gemm_generic_kernel(const T* __restrict__ A, const T* __restrict__ B, TO* __restrict__ C, int M, int N, int K) {
  constexpr int BKg = 16;
  __shared__ __attribute__((aligned(16))) T As[64][BKg];
  __shared__ __attribute__((aligned(16))) T Bs[64][BKg];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  const int wm = wave >> 1, wn = wave & 1;
  f32x16 acc = f32x16{};
  for (int k0 = 0; k0 < K; k0 += BKg) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int idx = tid * 4 + e;
      const int r = idx / BKg, kk = idx % BKg;
      const int gm = m0 + r, gk = k0 + kk;
      As[r][kk] = (gm < M && gk < K) ? A[(int64_t)gm * K + gk] : T(0);
      if (BT) {
        const int gn = n0 + r;
        Bs[r][kk] = (gn < N && gk < K) ? B[(int64_t)gn * K + gk] : T(0);
      } else {
        const int kr = idx / 64, nn = idx % 64;
        const int gk2 = k0 + kr, gn = n0 + nn;
        Bs[nn][kr] = (gn < N && gk2 < K) ? B[(int64_t)gk2 * N + gn] : T(0);
      }
    }
    __syncthreads();
    if constexpr (sizeof(T) == 2) {
      const f16x8 a = *reinterpret_cast<const f16x8*>(&As[wm * 32 + (lane & 31)][(lane >> 5) * 8]);
      const f16x8 b = *reinterpret_cast<const f16x8*>(&Bs[wn * 32 + (lane & 31)][(lane >> 5) * 8]);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
    } else {
#pragma unroll
      for (int s = 0; s < BKg / 2; ++s) {
        const float a = As[wm * 32 + (lane & 31)][2 * s + (lane >> 5)];
        const float b = Bs[wn * 32 + (lane & 31)][2 * s + (lane >> 5)];
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
      }
    }
    __syncthreads();
  }
  // D[i][j]: lane -> column j = lane & 31, rows i = 8*(r/4) + 4*(lane>>5) + r%4.
  const int n = n0 + wn * 32 + (lane & 31);
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int m = m0 + wm * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
    if (m < M && n < N) C[(int64_t)m * N + n] = (TO)acc[r];
  }
}

}  // namespace uk::kern

namespace uk {

namespace {
template <int I>
hipError_t gemm_f16_variant(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, hipStream_t s) {
  constexpr GemmF16Variant v = kGemmF16Variants[I];
  if constexpr (v.pp == 6) {
    static_assert(v.bm == kern::kW4BM && v.bn == kern::kW4BN && v.bk == kern::kW4kBK && v.wm == 2 && v.wn == 4,
                  "the eight-wavefront variant is 256x256x64 with 2x4 wavefronts");
    const int tiles_m = int(M / v.bm), tiles_n = int(N / v.bn);
    hipLaunchKernelGGL(kern::gemm_f16_w8k16_kernel, dim3((unsigned)(tiles_m * tiles_n)), dim3(512), 0, s,
                       static_cast<const _Float16*>(A), static_cast<const _Float16*>(B), static_cast<_Float16*>(C),
                       (int)M, (int)N, (int)K, tiles_m, tiles_n);
    return hipGetLastError();
  } else if constexpr (v.pp == 4 || v.pp == 5) {
    static_assert(v.bm == kern::kW4BM && v.bn == kern::kW4BN && v.bk == kern::kW4kBK && v.wm * v.wn == 4 &&
                      v.stages == 2,
                  "the 64-deep four-wavefront variants are 256x256x64 with two A slots");
    const int tiles_m = int(M / v.bm), tiles_n = int(N / v.bn);
    hipLaunchKernelGGL(v.pp == 4 ? kern::gemm_f16_w4k_kernel : kern::gemm_f16_w4k16_kernel,
                       dim3((unsigned)(tiles_m * tiles_n)), dim3(256), 0, s, static_cast<const _Float16*>(A),
                       static_cast<const _Float16*>(B), static_cast<_Float16*>(C), (int)M, (int)N, (int)K, tiles_m,
                       tiles_n);
    return hipGetLastError();
  } else if constexpr (v.pp == 2 || v.pp == 3) {
    static_assert(v.bm == kern::kW4BM && v.bn == kern::kW4BN && v.bk == kern::kW4BK && v.wm * v.wn == 4,
                  "four-wavefront variants are 256x256x32 with 2x2 wavefronts");
    const int tiles_m = int(M / v.bm), tiles_n = int(N / v.bn);
    if constexpr (v.pp == 2)
      hipLaunchKernelGGL((kern::gemm_f16_w4_kernel<v.stages>), dim3((unsigned)(tiles_m * tiles_n)), dim3(256), 0, s,
                         static_cast<const _Float16*>(A), static_cast<const _Float16*>(B), static_cast<_Float16*>(C),
                         (int)M, (int)N, (int)K, tiles_m, tiles_n);
    else
      hipLaunchKernelGGL((kern::gemm_f16_w4s_kernel<v.stages>), dim3((unsigned)(tiles_m * tiles_n)), dim3(256), 0, s,
                         static_cast<const _Float16*>(A), static_cast<const _Float16*>(B), static_cast<_Float16*>(C),
                         (int)M, (int)N, (int)K, tiles_m, tiles_n);
    return hipGetLastError();
  } else if constexpr (v.pp) {
    static_assert(v.bm == kern::kPpBM && v.bn == kern::kPpBN && v.bk == kern::kPpBK && v.wm * v.wn == 8,
                  "ping-pong variants are 256x256x32 with 8 wavefronts");
    const int tiles_m = int(M / v.bm), tiles_n = int(N / v.bn);
    hipLaunchKernelGGL((kern::gemm_f16_pp_kernel<v.stages, v.swz>), dim3((unsigned)(tiles_m * tiles_n)), dim3(512), 0, s,
                       static_cast<const _Float16*>(A), static_cast<const _Float16*>(B), static_cast<_Float16*>(C),
                       (int)M, (int)N, (int)K, tiles_m, tiles_n);
    return hipGetLastError();
  } else {
    using Cfg = kern::GemmF16Cfg<v.bm, v.bn, v.bk, v.wm, v.wn, v.stages>;
    const int tiles_m = int(M / v.bm), tiles_n = int(N / v.bn);
    hipLaunchKernelGGL((kern::gemm_f16_tn_kernel<v.bm, v.bn, v.bk, v.wm, v.wn, v.stages, v.swz>),
                       dim3((unsigned)(tiles_m * tiles_n)), dim3(Cfg::kThreads), 0, s,
                       static_cast<const _Float16*>(A), static_cast<const _Float16*>(B), static_cast<_Float16*>(C),
                       (int)M, (int)N, (int)K, tiles_m, tiles_n);
    return hipGetLastError();
  }
}
}  // namespace

hipError_t launch_gemm_f16(const Plan& p, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                           hipStream_t s) {
  if (p.family != Family::GemmF16 || p.variant < 0 || p.variant >= kNumGemmF16Variants) return hipErrorInvalidValue;
  const GemmF16Variant v = kGemmF16Variants[p.variant];
  // The kernel has no bounds checks: every tile must be whole, and the DMA reads 16-byte
  // chunks of K-contiguous rows.
  if (M <= 0 || N <= 0 || K <= 0 || M % v.bm || N % v.bn || K % v.bk) return hipErrorInvalidValue;
  if (M > INT32_MAX / 2 || N > INT32_MAX / 2 || K > INT32_MAX / 2) return hipErrorInvalidValue;
  // Copy offsets are 32-bit byte offsets within a row block of the operand.
  if (int64_t(v.bm > v.bn ? v.bm : v.bn) * K * 2 > INT32_MAX) return hipErrorInvalidValue;
  if ((((uintptr_t)A) | ((uintptr_t)B) | ((uintptr_t)C)) & 15) return hipErrorInvalidValue;
  if ((M / v.bm) * (N / v.bn) > INT32_MAX) return hipErrorInvalidValue;
  static_assert(kNumGemmF16Variants == 20, "every GEMM variant needs a case below");
  switch (p.variant) {
#define UK_GEMM_CASE(I) \
  case I:                 \
    return gemm_f16_variant<I>(A, B, C, M, N, K, s);
    UK_GEMM_CASE(0)
    UK_GEMM_CASE(1)
    UK_GEMM_CASE(2)
    UK_GEMM_CASE(3)
    UK_GEMM_CASE(4)
    UK_GEMM_CASE(5)
    UK_GEMM_CASE(6)
    UK_GEMM_CASE(7)
    UK_GEMM_CASE(8)
    UK_GEMM_CASE(9)
    UK_GEMM_CASE(10)
    UK_GEMM_CASE(11)
    UK_GEMM_CASE(12)
    UK_GEMM_CASE(13)
    UK_GEMM_CASE(14)
    UK_GEMM_CASE(15)
    UK_GEMM_CASE(16)
    UK_GEMM_CASE(17)
    UK_GEMM_CASE(18)
    UK_GEMM_CASE(19)
#undef UK_GEMM_CASE
    default: return hipErrorInvalidValue;
  }
}

bool gemm_f32_tiled_supported(int64_t M, int64_t N, int64_t K) {
  return M > 0 && N > 0 && K > 0 && M % 64 == 0 && N % 64 == 0 && K % 64 == 0;
}

hipError_t launch_gemm_generic(int variant, DType dt, Layout lay, const void* A, const void* B, void* C, int64_t M,
                               int64_t N, int64_t K, hipStream_t s) {
  if (M <= 0 || N <= 0 || K <= 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return hipErrorInvalidValue;
  if (lay != Layout::NT && lay != Layout::TN) return hipErrorInvalidValue;
  if ((M + 63) / 64 > 65535) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
  const bool bt = lay == Layout::TN;
  if (variant == 1) {  // gemm_f32_kernel: f32, 64-multiples, 16-byte aligned operands
    if (dt != DType::F32 || !gemm_f32_tiled_supported(M, N, K)) return hipErrorInvalidValue;
    if ((((uintptr_t)A) | ((uintptr_t)B) | ((uintptr_t)C)) & 15) return hipErrorInvalidValue;
    auto a = static_cast<const float*>(A);
    auto b = static_cast<const float*>(B);
    auto c = static_cast<float*>(C);
    const int tm = int(M / 64), tn = int(N / 64);
    if (int64_t(tm) * tn > INT32_MAX) return hipErrorInvalidValue;
    const dim3 g1((unsigned)(tm * tn));
    if (bt)
      hipLaunchKernelGGL((kern::gemm_f32_kernel<true>), g1, dim3(512), 0, s, a, b, c, (int)M, (int)N, (int)K, tm, tn);
    else
      hipLaunchKernelGGL((kern::gemm_f32_kernel<false>), g1, dim3(512), 0, s, a, b, c, (int)M, (int)N, (int)K, tm, tn);
    return hipGetLastError();
  }
  if (variant != 0) return hipErrorInvalidValue;
  if (dt == DType::F16) {
    auto a = static_cast<const _Float16*>(A);
    auto b = static_cast<const _Float16*>(B);
    auto c = static_cast<_Float16*>(C);
    if (bt)
      hipLaunchKernelGGL((kern::gemm_generic_kernel<_Float16, _Float16, true>), grid, dim3(256), 0, s, a, b, c,
                         (int)M, (int)N, (int)K);
    else
      hipLaunchKernelGGL((kern::gemm_generic_kernel<_Float16, _Float16, false>), grid, dim3(256), 0, s, a, b, c,
                         (int)M, (int)N, (int)K);
  } else if (dt == DType::F32) {
    auto a = static_cast<const float*>(A);
    auto b = static_cast<const float*>(B);
    auto c = static_cast<float*>(C);
    if (bt)
      hipLaunchKernelGGL((kern::gemm_generic_kernel<float, float, true>), grid, dim3(256), 0, s, a, b, c, (int)M,
                         (int)N, (int)K);
    else
      hipLaunchKernelGGL((kern::gemm_generic_kernel<float, float, false>), grid, dim3(256), 0, s, a, b, c, (int)M,
                         (int)N, (int)K);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace uk
