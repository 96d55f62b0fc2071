// Seeded synthetic inputs, number formats and the self-verification references used by
// uk_run (the library's counterpart of the CPU reference every emitted reference program
// embeds, src/codegen_hip.cpp:24-26).
//
// The self-check computes in binary64 and applies the north-star gates; it checks a GPU
// result, it never produces one.
#pragma once
#include <cstddef>
#include <cstdint>
#include <vector>

namespace uk {

// SplitMix64 (Steele, Lea, Flood, OOPSLA 2014); one stream per tensor.
uint64_t splitmix64(uint64_t* state);
void fill_uniform(float* out, size_t n, uint64_t seed, float lo, float hi);
void fill_normal(float* out, size_t n, uint64_t seed, float mu, float sigma);
// Sawtooth of the reference's exact-mode inputs (src/codegen_hip.cpp:1122-1123, :2166-2167):
// bias + ((idx % period) - offset) * unit, in binary32.
void fill_sawtooth(float* out, size_t n, int period, int offset, float unit, float bias);

uint16_t f32_to_f16(float f);  // IEEE binary16, round to nearest even
float f16_to_f32(uint16_t h);

// GGUF Q8_0 block: binary16 d (little endian) then int8 qs[32]; 34 bytes.
constexpr int kQ8Block = 34;
void q8_0_pack(const int8_t* q, const uint16_t* d, uint8_t* blocks, int N, int K);

// Seed offsets per tensor (base seed + offset).
enum SeedOffset : uint64_t {
  kSeedGemmF32A = 0, kSeedGemmF32B = 1,
  kSeedRowsX = 10, kSeedRmsW = 11, kSeedSoftmaxX = 12,
  kSeedGemmF16A = 20, kSeedGemmF16B = 21,
  kSeedConvX = 30, kSeedConvW = 31, kSeedConvS = 32,
  kSeedQ8X = 40, kSeedQ8Q = 41, kSeedQ8D = 42,
};

// ---- binary64 references for the self-check ----
// Host threads the reference loops below run on for n independent units (rows, columns,
// planes): min(hardware threads, 32), or 1 below 64 units.
int ref_threads(int64_t n);
void ref_rowsum(const float* X, double* Y, double* Yabs, int64_t L, int64_t C);
void ref_rmsnorm(const float* X, const float* W, double* Y, int64_t L, int64_t C, double eps);
void ref_softmax(const float* X, double* Y, int64_t L, int64_t C);
// rows[] lists the output rows to compute (all rows when empty). B layout: bt -> [N][K].
void ref_gemm(const float* A, const float* B, double* C, int64_t M, int64_t N, int64_t K, bool bt,
              const std::vector<int64_t>& rows);
void ref_conv_nchw(const float* x, const float* w, const float* scale, double* y, int64_t Nb, int64_t C, int64_t H,
                   int64_t W, int64_t Oc, int64_t Kh, int64_t Kw, int64_t pad, int64_t stride,
                   const std::vector<int64_t>& images);
void ref_conv_hwc(const float* x, const float* wt, const float* scale, double* y, int64_t H, int64_t W, int64_t C,
                  int64_t Kh, int64_t Kw, int64_t Oc);
void ref_q8_0(const uint16_t* X, const uint8_t* blocks, double* Y, int64_t M, int64_t N, int64_t K);

// ---- metrics ----
double max_rel(const float* got, const double* ref, size_t n, double floor);
double frobenius_rel(const float* got, const double* ref, size_t n);

}  // namespace uk
