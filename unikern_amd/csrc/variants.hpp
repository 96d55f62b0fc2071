// Compiled kernel variant tables. The solver enumerates exactly these (its candidate set is
// what was compiled, so a plan can never name a kernel that does not exist) and the kernel
// files instantiate exactly these.
#pragma once

namespace uk {

// Row family (row-sum, RMSNorm, softmax with the row held in registers).
// tpr: threads per row (whole wavefronts), nv: float4 registers per thread.
// A workgroup is max(tpr, 256) threads, i.e. 256/tpr rows per workgroup when tpr < 256.
// nt: loads and stores carry the non-temporal hint (streamed data bypasses cache retention).
// rpb: rows a workgroup walks in turn, the next row's loads in flight during this row's reduction.
// grp: one wavefront per row (tpr = 64, rpb = 1), the workgroup's rows stored together after one
// barrier, a row-length vector staged in LDS per workgroup (the RMSNorm or channelscale gain; for
// softmax a library-owned vector of ones, which the stores multiply by).
// eff: calibrated fraction of the HBM peak the variant sustains for row-sum, RMSNorm and softmax
// (kernel-only median at 4096 x 4096 f32 on one MI355X, rotating buffers > 512 MiB); 0 where the
// variant cannot hold a 4096-wide row, and the solver's bytes-in-flight model prices it alone.
struct RowsVariant {
  int tpr, nv, nt, rpb;
  double eff_sum, eff_rms, eff_softmax;
  int grp = 0;
};
constexpr RowsVariant kRowsVariants[] = {
    {64, 1, 0, 1, 0, 0, 0},
    {64, 2, 0, 1, 0, 0, 0},
    {64, 4, 0, 1, 0, 0, 0},
    {64, 8, 0, 1, 0, 0, 0},
    {64, 16, 0, 1, 0.653, 0.622, 0.625},
    {128, 4, 0, 1, 0, 0, 0},
    {128, 8, 0, 1, 0.697, 0.658, 0.661},
    {256, 1, 0, 1, 0, 0, 0},
    {256, 2, 0, 1, 0, 0, 0},
    {256, 4, 0, 1, 0.707, 0.679, 0.690},
    {256, 8, 0, 1, 0.706, 0.683, 0.681},
    {512, 2, 0, 1, 0.715, 0.694, 0.698},
    {512, 4, 0, 1, 0.715, 0.690, 0.684},
    {1024, 1, 0, 1, 0.549, 0.585, 0.672},
    {1024, 2, 0, 1, 0.552, 0.583, 0.639},
    {1024, 4, 0, 1, 0.544, 0.597, 0.526},
    {256, 4, 1, 1, 0.754, 0.717, 0.718},
    {512, 2, 1, 1, 0.762, 0.713, 0.735},
    {1024, 1, 1, 1, 0.558, 0.598, 0.683},
    {512, 4, 1, 1, 0.759, 0.702, 0.717},
    {1024, 2, 1, 1, 0.562, 0.606, 0.642},
    {128, 8, 1, 1, 0.740, 0.704, 0.709},
    {256, 4, 1, 2, 0.731, 0.718, 0.698},
    {512, 2, 1, 2, 0.742, 0.700, 0.681},
    {64, 16, 1, 1, 0.707, 0.771, 0.759, 1},
};
constexpr int kNumRowsVariants = sizeof(kRowsVariants) / sizeof(kRowsVariants[0]);

// Standalone channelscale in the grouped-store row form (one wavefront per row of at most 4096
// floats, more than half of its lanes busy); other shapes take the float4 grid-stride kernel.
inline bool channelscale_rows_form(long L, long C) { return C % 4 == 0 && C > 2048 && C <= 4096 && L <= 0x7fffffffL; }
constexpr int kRowsStreamThreads = 256;

// 1-D reduce: pass-1 partial count and threads.
constexpr int kReduceParts = 2048;
constexpr int kReduceThreads = 256;

// f16 MFMA GEMM, layout TN (A[M][K], B stored [N][K]).
// bm x bn x bk macro tile; wm x wn waves; stages of LDS buffering; swz selects the LDS
// XOR swizzle (0: row, 1: row >> 1, 2: row >> 2) for the bank geometry. pp = 0: every wavefront
// interleaves copies, fragment reads and v_mfma_f32_32x32x16_f16 (gemm_f16_tn_kernel); pp = 1:
// ping-pong wavefront groups on v_mfma_f32_16x16x32_f16 (gemm_f16_pp_kernel, 256x256x32 with 8
// wavefronts); pp = 2: four wavefronts of 128x128 on v_mfma_f32_32x32x16_f16 with copies sharing
// one M0 and a fence-free barrier (gemm_f16_w4_kernel, 256x256x32); pp = 3: the same four
// wavefronts on v_mfma_f32_16x16x32_f16 with a rolling A fragment (gemm_f16_w4s_kernel); pp = 4:
// the pp = 2 tiling with 64-deep k-tiles in 128-byte rows, two A and three B tile slots
// (gemm_f16_w4k_kernel; stages counts the A slots); pp = 5: the same on v_mfma_f32_16x16x32_f16
// (gemm_f16_w4k16_kernel); pp = 6: that tile with eight wavefronts of 128x64, two per SIMD
// (gemm_f16_w8k16_kernel). eff is
// the calibrated fraction of the dense f16 MFMA peak the variant sustains when every CU holds a
// tile (kernel-only median at M = N = K = 4096 on one MI355X, clocks settled); the solver's cost
// model scales it by wave quantisation for other shapes.
struct GemmF16Variant {
  int bm, bn, bk, wm, wn, stages, swz;
  double eff;
  int pp;
};
constexpr GemmF16Variant kGemmF16Variants[] = {
    {256, 256, 32, 2, 2, 4, 1, 0.431, 0},
    {256, 256, 32, 2, 2, 4, 2, 0.436, 0},
    {256, 256, 32, 2, 2, 4, 0, 0.432, 0},
    {256, 256, 32, 2, 4, 4, 2, 0.446, 0},
    {256, 128, 32, 2, 2, 4, 2, 0.354, 0},
    {256, 128, 64, 2, 2, 3, 1, 0.336, 0},
    {128, 128, 64, 2, 2, 3, 1, 0.231, 0},
    {128, 128, 32, 2, 2, 4, 2, 0.314, 0},
    {256, 256, 32, 2, 4, 5, 2, 0.445, 0},
    {256, 256, 32, 2, 2, 5, 2, 0.425, 0},
    {256, 256, 32, 2, 4, 4, 2, 0.479, 1},
    {256, 256, 32, 2, 4, 5, 2, 0.475, 1},
    {256, 256, 32, 2, 2, 4, 2, 0.448, 2},
    {256, 256, 32, 2, 2, 5, 2, 0.446, 2},
    {256, 256, 32, 2, 4, 4, 1, 0.477, 1},
    {256, 256, 32, 2, 4, 5, 1, 0.473, 1},
    {256, 256, 32, 2, 2, 4, 1, 0.440, 3},
    {256, 256, 64, 2, 2, 2, 1, 0.487, 4},
    {256, 256, 64, 2, 2, 2, 1, 0.545, 5},
    {256, 256, 64, 2, 4, 2, 1, 0.517, 6},
};
constexpr int kNumGemmF16Variants = sizeof(kGemmF16Variants) / sizeof(kGemmF16Variants[0]);

// Generic MFMA GEMM (any M, N, K; NT or TN; fp16 or fp32 inputs): 64x64 tiles, 4 waves.
constexpr int kGemmGenericTile = 64;

// Q8_0 skinny GEMM: a workgroup owns 16 nt weight rows; each of its wavefronts copies `pairs`
// block pairs of those rows per round into its own LDS area (nt * pairs * 1088 bytes) and
// computes them; a round covers waves * pairs block pairs. vec: dwords per lane per copy
// instruction (4 needs K divisible by 64 * pairs). db: two LDS buffers per wavefront, the next
// round's copies in flight while the current round is computed. nt: 16-row weight tiles that
// share each activation fragment.
// gemv: the M = 1 kernel instead (one weight row per wavefront, vector-ALU dot products, `waves`
// rows per workgroup sharing the activation row in LDS, one block pair per lane: K <= 4096).
struct Q8Variant {
  int waves, pairs, vec, db, nt, gemv;
};
constexpr Q8Variant kQ8Variants[] = {{16, 4, 4, 0, 1}, {16, 4, 1, 0, 1}, {8, 8, 4, 0, 1}, {8, 4, 1, 0, 1},
                                     {8, 4, 4, 1, 1},  {4, 4, 4, 1, 1},  {4, 8, 4, 1, 1}, {8, 4, 4, 0, 4},
                                     {8, 4, 4, 0, 1},  {8, 4, 4, 0, 3},  {4, 1, 4, 0, 1, 1}};
constexpr int kNumQ8Variants = sizeof(kQ8Variants) / sizeof(kQ8Variants[0]);

// Implicit-GEMM conv on f32 MFMA (v_mfma_f32_32x32x2f32). Wide kernel (tile_strips 0): a
// wavefront owns 32 output pixels x 64 output channels, `waves` wavefronts per workgroup, and
// bk_bytes is the LDS budget of one staged weight chunk (channels = budget / (taps * 64 * 4 B),
// even). Tile kernel (tile_strips S > 0, 3x3 and 1x1 only): wavefronts of 32 pixels x 32 output
// channels, S strips x 2 channel halves per workgroup, bk_bytes channels per weight chunk. LDS
// kernel (tile_strips -T for T = 1, 2, NCHW 3x3 stride 1 only, see conv_lds_supported): 64 T
// pixels x 64 output channels per workgroup of 4 T wavefronts, input rows and weights of 8
// channels staged in LDS. 16-pixel-group kernel (tile_strips kConvL16, see conv_l16_geom): runs of
// 16-pixel groups x 64 output channels per workgroup of 8 wavefronts on v_mfma_f32_16x16x4f32,
// bk_bytes channels per staged chunk. eff is the calibrated fraction of the f32 MFMA rate the
// busiest SIMD sustains (kernel-only median at the BASELINE conv shape on one MI355X).
struct ConvVariant {
  int waves;
  int bk_bytes;
  int tile_strips;
  double eff;
};
constexpr ConvVariant kConvVariants[] = {
    {4, 147456, 0, 0.273}, {2, 73728, 0, 0.175}, {4, 73728, 0, 0.260}, {2, 36864, 0, 0.170},
    {4, 16, 2, 0.130},     {4, 8, 2, 0.130},     {8, 8, 4, 0.310},     {4, 8, -1, 0.472},
    {8, 8, -2, 0.619},     {8, 16, -16, 0.696},
};
// LDS kernel geometry: input rows and padded columns one staged tile holds.
constexpr int kConvLdsRows = 8;
constexpr int kConvLdsCols = 64;
// The LDS kernel covers NCHW, 3x3, stride 1, pad 0 or 1, W + 2 pad <= kConvLdsCols, W a multiple
// of 4 and C of 8 (16-byte staging loads, whole channel chunks), and pix (64 or 128) consecutive
// output pixels spanning at most kConvLdsRows - 2 output rows.
inline bool conv_lds_supported(bool nchw, long kh, long kw, long stride, long pad, long W, long Ho, long Wo, long C,
                               long pix) {
  if (!nchw || kh != 3 || kw != 3 || stride != 1 || (pad != 0 && pad != 1)) return false;
  if (W + 2 * pad > kConvLdsCols || W % 4 != 0 || C % 8 != 0 || C <= 0 || Wo <= 0 || Ho <= 0) return false;
  return (pix - 1 + Wo - 1) / Wo + 1 + 2 <= kConvLdsRows;
}
constexpr int kNumConvVariants = sizeof(kConvVariants) / sizeof(kConvVariants[0]);

// 16-pixel-group kernel (conv_lds16_kernel, tile_strips kConvL16): the output pixels of an image
// (flattened Ho*Wo order) cut into gp groups of 16, and each image's groups into wpi contiguous
// runs, run j of gp / wpi + (j < gp % wpi) <= kConvL16MaxGroups groups, one workgroup (x 64
// output channels) each. wpi aims the launch at kConvL16Target workgroups (the CU count of
// MI355X: one workgroup per CU, runs balanced to within one group). rows: the most output rows
// a run spans; the kernel stages rows + 2 input rows per channel chunk, at most kConvL16Rows.
constexpr int kConvL16 = -16;
constexpr int kConvL16Target = 256;
constexpr int kConvL16MaxGroups = 8;
constexpr int kConvL16Rows = 6;
constexpr int kConvL16Pitch = 72;  // 16-byte entries per staged input row (8 mod 16: see the kernel)
constexpr int kConvL16WQuad = 68;  // 16-byte weight entries per channel quad (64 oc + 4: see the kernel)
struct ConvL16Geom {
  long gp, wpi, gmax, rows;
};
inline ConvL16Geom conv_l16_geom(long N, long Ho, long Wo, long oc_blocks) {
  ConvL16Geom g{0, 0, 0, 0};
  if (N <= 0 || Ho <= 0 || Wo <= 0 || oc_blocks <= 0) return g;
  const long P = Ho * Wo;
  g.gp = (P + 15) / 16;
  long wpi = (kConvL16Target + N * oc_blocks - 1) / (N * oc_blocks);
  const long least = (g.gp + kConvL16MaxGroups - 1) / kConvL16MaxGroups;
  if (wpi < least) wpi = least;
  if (wpi > g.gp) wpi = g.gp;
  g.wpi = wpi;
  const long q = g.gp / wpi, r = g.gp % wpi;
  for (long j = 0; j < wpi; ++j) {
    const long a = j * q + (j < r ? j : r), b = a + q + (j < r ? 1 : 0);
    const long pend = (16 * b < P ? 16 * b : P) - 1;
    const long rows = pend / Wo - (16 * a) / Wo + 1;
    if (b - a > g.gmax) g.gmax = b - a;
    if (rows > g.rows) g.rows = rows;
  }
  return g;
}
// NCHW, 3x3, stride 1, pad 0 or 1, W + 2 pad <= kConvL16Pitch, W a multiple of 4 and C of 16
// (16-byte staging loads, whole 16-channel chunks), every run within kConvL16Rows - 2 rows, and
// the kernel's index quotients (pixel indices up to 16 (gp + 4), workgroup indices up to N wpi)
// below kConvL16IndexLimit, where its reciprocal division is exact.
constexpr long kConvL16IndexLimit = 1L << 21;
inline bool conv_l16_supported(bool nchw, long kh, long kw, long stride, long pad, long N, long W, long Ho, long Wo,
                               long C, long Oc) {
  if (!nchw || kh != 3 || kw != 3 || stride != 1 || (pad != 0 && pad != 1)) return false;
  if (W + 2 * pad > kConvL16Pitch || W % 4 != 0 || C % 16 != 0 || C <= 0 || Oc <= 0) return false;
  const ConvL16Geom g = conv_l16_geom(N, Ho, Wo, (Oc + 63) / 64);
  return g.wpi > 0 && g.gmax <= kConvL16MaxGroups && g.rows + 2 <= kConvL16Rows &&
         16 * (g.gp + 4) < kConvL16IndexLimit && N * g.wpi < kConvL16IndexLimit;
}

// Sustained shader clock (GHz) of the matrix-core probe (uk_probe_mfma: one wavefront per SIMD
// issuing only v_mfma_f32_16x16x32_f16 on switching random operands, its primary form) on the
// parts where the GEMM and conv efficiencies above were fitted (2.01-2.03 GHz measured; the same
// parts settle at 1.66 GHz under the 32x32x16 form). A part whose probe sustains less under that
// load runs every MFMA-bound kernel proportionally slower; calibration uses the ratio when no
// measured MFMA-bound row is available.
constexpr double kEffFitProbeClockGhz = 2.02;

}  // namespace uk
