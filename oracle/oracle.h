/* CPU oracle for the UNIKERN kernel hot path — TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the reference's CPU loops. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it, and only as
 * the checker (or as the timed CPU baseline). The product library
 * (unikern_amd/libunikern_hip.so) never links, loads or calls it.
 *
 * Each function names the reference file:line it follows. Pinning status:
 *   or_cpu_conv, or_cpu_reduce, or_cpu_reduce_blocked      pinned (oracle/_ref build of src/reference.cpp,
 *                                                              golden fixtures, hand cases of tests/acceptance.cpp:1322-1357)
 *   or_gemm_f32, or_gemm_f16q, or_softmax, or_rmsnorm,
 *   or_channelscale                                          pinned (oracle/_ref build of the stored emitted
 *                                                              programs, golden fixtures, closed forms)
 *   or_rowsum_blocked                                        pinned (per-row or_cpu_reduce_blocked, fixtures)
 *   or_conv_nchw                                             pinned (reduces to cpu_conv under a layout transpose
 *                                                              at batch 1, pad 0; zero-padding closed forms)
 *   or_q8_0_*                                                pinned by the block definition and closed forms
 *                                                              (no reference implementation exists)
 *   or_f32_to_f16 / or_f16_to_f32                            pinned (exhaustive vs numpy float16)
 *   or_splitmix64 / or_fill_*                                pinned (published SplitMix64 vectors)
 */
#ifndef UK_ORACLE_H
#define UK_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- number formats ---- */
uint16_t or_f32_to_f16(float f);      /* IEEE binary16, round to nearest even */
float or_f16_to_f32(uint16_t h);
void or_f32_to_f16_n(const float* in, uint16_t* out, size_t n);
void or_f16_to_f32_n(const uint16_t* in, float* out, size_t n);

/* ---- seeded inputs (SplitMix64; uniform = top 24 bits * 2^-24; normal = Box-Muller) ---- */
uint64_t or_splitmix64(uint64_t* state);
void or_fill_uniform(float* out, size_t n, uint64_t seed, float lo, float hi);
void or_fill_normal(float* out, size_t n, uint64_t seed, float mu, float sigma);
void or_fill_sawtooth(float* out, size_t n, int period, int offset, float unit, float bias);

/* ---- reference.cpp restatements ---- */
void or_cpu_conv(const float* x, const float* wt, float* y, int H, int W, int C, int Kh, int Kw, int Oc);
void or_cpu_reduce(const float* x, float* y, int64_t n);
void or_cpu_reduce_blocked(const float* x, float* y, int64_t n, int width);

/* ---- emitted-program CPU references (codegen_hip.cpp) ---- */
void or_gemm_f32(const float* A, const float* B, float* C, int M, int N, int K, int b_colmajor);
void or_gemm_f16q(const uint16_t* A, const uint16_t* B, float* C, int M, int N, int K, int b_colmajor);
void or_softmax(const float* X, float* Y, int L, int C);
void or_rmsnorm(const float* X, const float* W, float* Y, int L, int C, float eps);
void or_channelscale(const float* X, const float* S, float* Y, int L, int C);

/* ---- extensions of the op surface ---- */
void or_rowsum_blocked(const float* X, float* Y, int L, int C, int width);
void or_rowsum_f64(const float* X, double* Y, double* Yabs, int L, int C);
void or_conv_nchw(const float* x, const float* w, const float* scale, float* y, int N, int C, int H, int W,
                  int Oc, int Kh, int Kw, int pad, int stride);
void or_q8_0_dequant(const uint8_t* blocks, float* out, int N, int K);
void or_q8_0_gemm_f64(const uint16_t* X, const uint8_t* blocks, double* Y, int M, int N, int K);
void or_q8_0_pack(const int8_t* q, const uint16_t* d, uint8_t* blocks, int N, int K);

/* ---- verification metrics ---- */
double or_max_rel(const float* got, const float* ref, size_t n, double floor);
double or_frobenius_rel(const float* got, const float* ref, size_t n);

/* ---- multi-threaded wrappers for the timed CPU baseline (same per-output order) ---- */
void or_softmax_mt(const float* X, float* Y, int L, int C, int threads);
void or_rmsnorm_mt(const float* X, const float* W, float* Y, int L, int C, float eps, int threads);
void or_rowsum_blocked_mt(const float* X, float* Y, int L, int C, int width, int threads);
void or_gemm_f16q_mt(const uint16_t* A, const uint16_t* B, float* C, int M, int N, int K, int b_colmajor,
                     int threads);
void or_gemm_f32_mt(const float* A, const float* B, float* C, int M, int N, int K, int b_colmajor, int threads);
void or_conv_nchw_mt(const float* x, const float* w, const float* scale, float* y, int N, int C, int H, int W,
                     int Oc, int Kh, int Kw, int pad, int stride, int threads);
void or_q8_0_gemm_f64_mt(const uint16_t* X, const uint8_t* blocks, double* Y, int M, int N, int K, int threads);

#ifdef __cplusplus
}
#endif
#endif
