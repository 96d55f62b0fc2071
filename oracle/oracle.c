/* CPU oracle for the UNIKERN kernel hot path — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU loops (src/reference.cpp and
 * the CPU references that src/codegen_hip.cpp embeds in every emitted
 * program). It is the checker for the HIP kernels and the timed CPU baseline;
 * the product library never links or calls it. Build: oracle/Makefile
 * (gcc -O2 -ffp-contract=off, no -march flags, so every float operation is the
 * plain IEEE binary32 operation the reference's host code performs).
 *
 * Pinning of each function is listed in oracle.h.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* binary16 <-> binary32 (IEEE 754-2008, round to nearest, ties to even).     */
/* The reference converts with __float2half / __half2float on the host        */
/* (codegen_hip.cpp:1852-1858); both are the IEEE conversions restated here.  */
/* ------------------------------------------------------------------------- */
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t or_f32_to_f16(float f) {
  const uint32_t x = f2u(f);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) {                       /* inf / nan */
    if (ax == 0x7f800000u) return sign | 0x7c00u;
    return sign | 0x7e00u | (uint16_t)((ax >> 13) & 0x3ffu);
  }
  if (ax >= 0x477ff000u) return sign | 0x7c00u;  /* >= 65520 rounds to inf */
  if (ax >= 0x38800000u) {                       /* normal half */
    uint32_t h = (ax - 0x38000000u) >> 13;
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return sign | (uint16_t)h;
  }
  if (ax < 0x33000000u) return sign;             /* <= 2^-25 rounds to (signed) zero */
  {                                              /* subnormal half: units of 2^-24 */
    const uint32_t e = ax >> 23;
    const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - e;             /* 14..24 */
    uint32_t h = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) ++h;
    return sign | (uint16_t)h;
  }
}

float or_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  const uint32_t m = h & 0x3ffu;
  if (e == 0) {
    const float v = (float)m * 5.9604644775390625e-08f; /* m * 2^-24, exact */
    return (sign ? -v : v);
  }
  if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
  return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

void or_f32_to_f16_n(const float* in, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = or_f32_to_f16(in[i]);
}
void or_f16_to_f32_n(const uint16_t* in, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = or_f16_to_f32(in[i]);
}

/* ------------------------------------------------------------------------- */
/* Seeded inputs. SplitMix64 (Steele, Lea, Flood, "Fast splittable           */
/* pseudorandom number generators", OOPSLA 2014), one stream per tensor.     */
/* ------------------------------------------------------------------------- */
uint64_t or_splitmix64(uint64_t* s) {
  uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

void or_fill_uniform(float* out, size_t n, uint64_t seed, float lo, float hi) {
  uint64_t s = seed;
  for (size_t i = 0; i < n; ++i) {
    const double u = (double)(or_splitmix64(&s) >> 40) * (1.0 / 16777216.0);
    out[i] = (float)((double)lo + ((double)hi - (double)lo) * u);
  }
}

void or_fill_normal(float* out, size_t n, uint64_t seed, float mu, float sigma) {
  /* Box-Muller: u1 in (0,1], u2 in [0,1), both with 53-bit resolution. */
  uint64_t s = seed;
  const double two_pi = 6.283185307179586476925286766559;
  for (size_t i = 0; i < n; i += 2) {
    const double u1 = (double)((or_splitmix64(&s) >> 11) + 1) * (1.0 / 9007199254740992.0);
    const double u2 = (double)(or_splitmix64(&s) >> 11) * (1.0 / 9007199254740992.0);
    const double r = sqrt(-2.0 * log(u1));
    out[i] = (float)((double)mu + (double)sigma * (r * cos(two_pi * u2)));
    if (i + 1 < n) out[i + 1] = (float)((double)mu + (double)sigma * (r * sin(two_pi * u2)));
  }
}

/* initA/initB/initX/initW/initS of the emitted programs (codegen_hip.cpp:1122-1123, :1998,
 * :2166-2167, :2337-2338): bias + ((idx % period) - offset) * unit, all in binary32. */
void or_fill_sawtooth(float* out, size_t n, int period, int offset, float unit, float bias) {
  for (size_t i = 0; i < n; ++i) {
    const int idx = (int)i;
    const float t = (float)((idx % period) - offset) * unit;
    out[i] = bias == 0.0f ? t : bias + t;
  }
}

/* ------------------------------------------------------------------------- */
/* src/reference.cpp                                                          */
/* ------------------------------------------------------------------------- */

/* src/reference.cpp:6-22 — valid conv, X[H][W][C], Wt[Oc][Kh][Kw][C], Y[Oc][Ho][Wo],
 * accumulation c -> kh -> kw ascending in binary32. */
void or_cpu_conv(const float* x, const float* wt, float* y, int H, int W, int C, int Kh, int Kw, int Oc) {
  const int Ho = H - Kh + 1, Wo = W - Kw + 1;
  for (int oc = 0; oc < Oc; ++oc)
    for (int ho = 0; ho < Ho; ++ho)
      for (int wo = 0; wo < Wo; ++wo) {
        float acc = 0.f;
        for (int c = 0; c < C; ++c)
          for (int kh = 0; kh < Kh; ++kh)
            for (int kw = 0; kw < Kw; ++kw)
              acc += x[((size_t)(ho + kh) * W + (size_t)(wo + kw)) * C + c] *
                     wt[((size_t)(oc * Kh + kh) * Kw + kw) * C + c];
        y[((size_t)oc * Ho + ho) * Wo + wo] = acc;
      }
}

/* src/reference.cpp:24-28 — index-order binary32 sum. */
void or_cpu_reduce(const float* x, float* y, int64_t n) {
  float acc = 0.f;
  for (int64_t i = 0; i < n; ++i) acc += x[i];
  y[0] = acc;
}

/* src/reference.cpp:36-48 — `width` strided partials, folded in index order. */
void or_cpu_reduce_blocked(const float* x, float* y, int64_t n, int width) {
  if (width <= 0) { or_cpu_reduce(x, y, n); return; }
  float acc = 0.f;
  for (int b = 0; b < width; ++b) {
    float part = 0.f;
    for (int64_t i = b; i < n; i += width) part += x[i];
    acc += part;
  }
  y[0] = acc;
}

/* ------------------------------------------------------------------------- */
/* CPU references embedded in the emitted programs                            */
/* ------------------------------------------------------------------------- */

/* src/codegen_hip.cpp:1124-1132 — f32 GEMM, k-ascending binary32 dot. The reference
 * indexes B[k*N+j] (layout NT); b_colmajor=1 reads B[j*K+k] (layout TN extension). */
static void gemm_f32_rows(const float* A, const float* B, float* C, int r0, int r1, int N, int K, int bcm) {
  for (int i = r0; i < r1; ++i)
    for (int j = 0; j < N; ++j) {
      float s = 0.f;
      const float* a = A + (size_t)i * K;
      if (bcm) {
        const float* b = B + (size_t)j * K;
        for (int k = 0; k < K; ++k) s += a[k] * b[k];
      } else {
        for (int k = 0; k < K; ++k) s += a[k] * B[(size_t)k * N + j];
      }
      C[(size_t)i * N + j] = s;
    }
}
void or_gemm_f32(const float* A, const float* B, float* C, int M, int N, int K, int b_colmajor) {
  gemm_f32_rows(A, B, C, 0, M, N, K, b_colmajor);
}

/* src/codegen_hip.cpp:1854-1862 with :1814-1822 — the fp16 program rounds its inputs to
 * half, widens them back to float, and runs the same binary32 loop on the quantized values. */
void or_gemm_f16q(const uint16_t* A, const uint16_t* B, float* C, int M, int N, int K, int b_colmajor) {
  or_gemm_f16q_mt(A, B, C, M, N, K, b_colmajor, 1);
}

/* src/codegen_hip.cpp:1999-2009 — per row: max, then sum of expf(x-max) in index order,
 * then y = expf(x-max)/sum (expf evaluated again, as the reference does). */
static void softmax_rows(const float* X, float* Y, int r0, int r1, int C) {
  for (int l = r0; l < r1; ++l) {
    const float* x = X + (size_t)l * C;
    float* y = Y + (size_t)l * C;
    float maxv = -INFINITY;
    for (int c = 0; c < C; ++c) if (x[c] > maxv) maxv = x[c];
    float sum = 0.0f;
    for (int c = 0; c < C; ++c) sum += expf(x[c] - maxv);
    for (int c = 0; c < C; ++c) y[c] = expf(x[c] - maxv) / sum;
  }
}
void or_softmax(const float* X, float* Y, int L, int C) { softmax_rows(X, Y, 0, L, C); }

/* src/codegen_hip.cpp:2168-2178 — sum of squares in index order, rms = 1/sqrt(ss/C + eps),
 * y = (x * rms) * W. The reference fixes eps = 1e-6f. */
static void rmsnorm_rows(const float* X, const float* W, float* Y, int r0, int r1, int C, float eps) {
  for (int l = r0; l < r1; ++l) {
    const float* x = X + (size_t)l * C;
    float* y = Y + (size_t)l * C;
    float sum_sq = 0.0f;
    for (int c = 0; c < C; ++c) sum_sq += x[c] * x[c];
    const float rms = 1.0f / sqrtf(sum_sq / (float)C + eps);
    for (int c = 0; c < C; ++c) y[c] = x[c] * rms * W[c];
  }
}
void or_rmsnorm(const float* X, const float* W, float* Y, int L, int C, float eps) {
  rmsnorm_rows(X, W, Y, 0, L, C, eps);
}

/* src/codegen_hip.cpp:2339-2344 — Y[i*C+c] = X[i*C+c] * S[c]. */
void or_channelscale(const float* X, const float* S, float* Y, int L, int C) {
  for (int i = 0; i < L; ++i)
    for (int c = 0; c < C; ++c) Y[(size_t)i * C + c] = X[(size_t)i * C + c] * S[c];
}

/* ------------------------------------------------------------------------- */
/* Extensions                                                                 */
/* ------------------------------------------------------------------------- */

/* Row-sum: src/reference.cpp:36-48 applied to each row of X[L][C] (kRefReduceWidth=1024,
 * include/unikern/core.hpp:124, is the reference's own basis width). */
static void rowsum_rows(const float* X, float* Y, int r0, int r1, int C, int width) {
  for (int l = r0; l < r1; ++l) or_cpu_reduce_blocked(X + (size_t)l * C, Y + l, C, width);
}
void or_rowsum_blocked(const float* X, float* Y, int L, int C, int width) {
  rowsum_rows(X, Y, 0, L, C, width);
}

/* binary64 row sums and sums of |x| (the condition scale of the row-sum gate). */
void or_rowsum_f64(const float* X, double* Y, double* Yabs, int L, int C) {
  for (int l = 0; l < L; ++l) {
    double s = 0.0, a = 0.0;
    for (int c = 0; c < C; ++c) { s += (double)X[(size_t)l * C + c]; a += fabs((double)X[(size_t)l * C + c]); }
    Y[l] = s;
    if (Yabs) Yabs[l] = a;
  }
}

/* Batched NCHW conv with zero padding and stride, weights OIHW [Oc][C][Kh][Kw],
 * accumulation order c -> kh -> kw as src/reference.cpp:13-18, taps that fall in the
 * padding are skipped (they would add +0), then one multiply by scale[oc] — the
 * channelscale epilogue of src/codegen_hip.cpp:2339-2344 applied per output channel. */
static void conv_nchw_planes(const float* x, const float* w, const float* scale, float* y, int p0, int p1,
                             int C, int H, int W, int Oc, int Kh, int Kw, int pad, int stride) {
  const int Ho = (H + 2 * pad - Kh) / stride + 1, Wo = (W + 2 * pad - Kw) / stride + 1;
  for (int p = p0; p < p1; ++p) {           /* p = n*Oc + oc */
    const int n = p / Oc, oc = p % Oc;
    for (int ho = 0; ho < Ho; ++ho)
      for (int wo = 0; wo < Wo; ++wo) {
        float acc = 0.f;
        for (int c = 0; c < C; ++c)
          for (int kh = 0; kh < Kh; ++kh) {
            const int hi = ho * stride + kh - pad;
            if (hi < 0 || hi >= H) continue;
            for (int kw = 0; kw < Kw; ++kw) {
              const int wi = wo * stride + kw - pad;
              if (wi < 0 || wi >= W) continue;
              acc += x[(((size_t)n * C + c) * H + hi) * W + wi] * w[(((size_t)oc * C + c) * Kh + kh) * Kw + kw];
            }
          }
        y[(((size_t)n * Oc + oc) * Ho + ho) * Wo + wo] = scale ? acc * scale[oc] : acc;
      }
  }
}
void or_conv_nchw(const float* x, const float* w, const float* scale, float* y, int N, int C, int H, int W,
                  int Oc, int Kh, int Kw, int pad, int stride) {
  conv_nchw_planes(x, w, scale, y, 0, N * Oc, C, H, W, Oc, Kh, Kw, pad, stride);
}

/* Q8_0 block (GGUF type 8, probe/phase63_gguf_header.py:91): 34 bytes = binary16 scale d
 * (little endian) followed by 32 int8 quants; value = float(d) * float(q), exact in binary32
 * (11 + 7 significant bits). Weights are N rows of K/32 blocks. */
void or_q8_0_pack(const int8_t* q, const uint16_t* d, uint8_t* blocks, int N, int K) {
  const int nb = K / 32;
  for (int n = 0; n < N; ++n)
    for (int b = 0; b < nb; ++b) {
      uint8_t* blk = blocks + ((size_t)n * nb + b) * 34;
      const uint16_t dv = d[(size_t)n * nb + b];
      blk[0] = (uint8_t)(dv & 0xff);
      blk[1] = (uint8_t)(dv >> 8);
      memcpy(blk + 2, q + ((size_t)n * K + (size_t)b * 32), 32);
    }
}

void or_q8_0_dequant(const uint8_t* blocks, float* out, int N, int K) {
  const int nb = K / 32;
  for (int n = 0; n < N; ++n)
    for (int b = 0; b < nb; ++b) {
      const uint8_t* blk = blocks + ((size_t)n * nb + b) * 34;
      const float d = or_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
      for (int i = 0; i < 32; ++i) out[(size_t)n * K + (size_t)b * 32 + i] = d * (float)(int8_t)blk[2 + i];
    }
}

/* Y[m][n] = sum_k deq(W)[n][k] * X[m][k] in binary64. Every product is exact in binary64
 * (18 + 11 significant bits), so the only rounding is the binary64 accumulation. */
static void q8_rows(const uint16_t* X, const uint8_t* blocks, double* Y, int n0, int n1, int M, int N, int K) {
  const int nb = K / 32;
  for (int n = n0; n < n1; ++n)
    for (int m = 0; m < M; ++m) {
      double s = 0.0;
      for (int b = 0; b < nb; ++b) {
        const uint8_t* blk = blocks + ((size_t)n * nb + b) * 34;
        const float d = or_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        for (int i = 0; i < 32; ++i) {
          const float wv = d * (float)(int8_t)blk[2 + i];
          s += (double)wv * (double)or_f16_to_f32(X[(size_t)m * K + (size_t)b * 32 + i]);
        }
      }
      Y[(size_t)m * N + n] = s;
    }
}
void or_q8_0_gemm_f64(const uint16_t* X, const uint8_t* blocks, double* Y, int M, int N, int K) {
  q8_rows(X, blocks, Y, 0, N, M, N, K);
}

/* ------------------------------------------------------------------------- */
/* Verification metrics                                                       */
/* ------------------------------------------------------------------------- */

/* src/codegen_hip.cpp:1410-1416: max |y-r| / max(|r|, floor) (floor 1e-6 in the reference). */
double or_max_rel(const float* got, const float* ref, size_t n, double floor) {
  double worst = 0.0;
  for (size_t i = 0; i < n; ++i) {
    double den = fabs((double)ref[i]);
    if (den < floor) den = floor;
    const double r = fabs((double)got[i] - (double)ref[i]) / den;
    if (r > worst || r != r) worst = r;
  }
  return worst;
}

/* ||got - ref||_F / ||ref||_F in binary64. */
double or_frobenius_rel(const float* got, const float* ref, size_t n) {
  double num = 0.0, den = 0.0;
  for (size_t i = 0; i < n; ++i) {
    const double d = (double)got[i] - (double)ref[i];
    num += d * d;
    den += (double)ref[i] * (double)ref[i];
  }
  return den > 0.0 ? sqrt(num / den) : sqrt(num);
}

/* ------------------------------------------------------------------------- */
/* Threaded wrappers: rows (or output planes) split across threads; each      */
/* output keeps the single-thread accumulation order, so results are bitwise  */
/* identical to the one-thread functions.                                      */
/* ------------------------------------------------------------------------- */
typedef struct {
  int kind, r0, r1;
  const void *a, *b, *c;
  void* out;
  int i0, i1, i2, i3, i4, i5, i6, i7, i8;
  float f0;
} job_t;

static void run_job(job_t* j) {
  switch (j->kind) {
    case 0: softmax_rows(j->a, j->out, j->r0, j->r1, j->i0); break;
    case 1: rmsnorm_rows(j->a, j->b, j->out, j->r0, j->r1, j->i0, j->f0); break;
    case 2: rowsum_rows(j->a, j->out, j->r0, j->r1, j->i0, j->i1); break;
    case 3: {
      const uint16_t* A = j->a;
      const uint16_t* B = j->b;
      const int N = j->i0, K = j->i1, bcm = j->i2;
      float* arow = malloc(sizeof(float) * (size_t)K);
      float* bq = j->c ? (float*)j->c : NULL;
      for (int i = j->r0; i < j->r1; ++i) {
        for (int k = 0; k < K; ++k) arow[k] = or_f16_to_f32(A[(size_t)i * K + k]);
        for (int c = 0; c < N; ++c) {
          float s = 0.f;
          if (bcm) {
            const float* bb = bq + (size_t)c * K;
            for (int k = 0; k < K; ++k) s += arow[k] * bb[k];
          } else {
            for (int k = 0; k < K; ++k) s += arow[k] * bq[(size_t)k * N + c];
          }
          ((float*)j->out)[(size_t)i * N + c] = s;
        }
      }
      free(arow);
      (void)B;
      break;
    }
    case 4: gemm_f32_rows(j->a, j->b, j->out, j->r0, j->r1, j->i0, j->i1, j->i2); break;
    case 5:
      conv_nchw_planes(j->a, j->b, j->c, j->out, j->r0, j->r1, j->i0, j->i1, j->i2, j->i3, j->i4, j->i5,
                       j->i6, j->i7);
      break;
    case 6: q8_rows(j->a, j->b, j->out, j->r0, j->r1, j->i0, j->i1, j->i2); break;
  }
}

static void* job_entry(void* p) { run_job((job_t*)p); return NULL; }

static void run_split(job_t proto, int total, int threads) {
  if (threads < 1) threads = 1;
  if (threads > total) threads = total > 0 ? total : 1;
  job_t* jobs = calloc((size_t)threads, sizeof(job_t));
  pthread_t* tids = calloc((size_t)threads, sizeof(pthread_t));
  for (int t = 0; t < threads; ++t) {
    jobs[t] = proto;
    jobs[t].r0 = (int)((long long)total * t / threads);
    jobs[t].r1 = (int)((long long)total * (t + 1) / threads);
  }
  for (int t = 1; t < threads; ++t) pthread_create(&tids[t], NULL, job_entry, &jobs[t]);
  run_job(&jobs[0]);
  for (int t = 1; t < threads; ++t) pthread_join(tids[t], NULL);
  free(jobs);
  free(tids);
}

void or_softmax_mt(const float* X, float* Y, int L, int C, int threads) {
  job_t j = {0}; j.kind = 0; j.a = X; j.out = Y; j.i0 = C;
  run_split(j, L, threads);
}
void or_rmsnorm_mt(const float* X, const float* W, float* Y, int L, int C, float eps, int threads) {
  job_t j = {0}; j.kind = 1; j.a = X; j.b = W; j.out = Y; j.i0 = C; j.f0 = eps;
  run_split(j, L, threads);
}
void or_rowsum_blocked_mt(const float* X, float* Y, int L, int C, int width, int threads) {
  job_t j = {0}; j.kind = 2; j.a = X; j.out = Y; j.i0 = C; j.i1 = width;
  run_split(j, L, threads);
}
void or_gemm_f16q_mt(const uint16_t* A, const uint16_t* B, float* C, int M, int N, int K, int b_colmajor,
                     int threads) {
  /* widen B once (exact), then every output is the binary32 loop of codegen_hip.cpp:1818-1820 */
  const size_t nb = (size_t)N * K;
  float* bq = malloc(sizeof(float) * nb);
  for (size_t i = 0; i < nb; ++i) bq[i] = or_f16_to_f32(B[i]);
  job_t j = {0}; j.kind = 3; j.a = A; j.b = B; j.c = bq; j.out = C; j.i0 = N; j.i1 = K; j.i2 = b_colmajor;
  run_split(j, M, threads);
  free(bq);
}
void or_gemm_f32_mt(const float* A, const float* B, float* C, int M, int N, int K, int b_colmajor, int threads) {
  job_t j = {0}; j.kind = 4; j.a = A; j.b = B; j.out = C; j.i0 = N; j.i1 = K; j.i2 = b_colmajor;
  run_split(j, M, threads);
}
void or_conv_nchw_mt(const float* x, const float* w, const float* scale, float* y, int N, int C, int H, int W,
                     int Oc, int Kh, int Kw, int pad, int stride, int threads) {
  job_t j = {0}; j.kind = 5; j.a = x; j.b = w; j.c = scale; j.out = y;
  j.i0 = C; j.i1 = H; j.i2 = W; j.i3 = Oc; j.i4 = Kh; j.i5 = Kw; j.i6 = pad; j.i7 = stride;
  run_split(j, N * Oc, threads);
}
void or_q8_0_gemm_f64_mt(const uint16_t* X, const uint8_t* blocks, double* Y, int M, int N, int K, int threads) {
  job_t j = {0}; j.kind = 6; j.a = X; j.b = blocks; j.out = Y; j.i0 = M; j.i1 = N; j.i2 = K;
  run_split(j, N, threads);
}
