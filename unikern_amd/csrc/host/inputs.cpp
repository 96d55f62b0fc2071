#include "inputs.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>

namespace uk {

uint64_t splitmix64(uint64_t* s) {
  uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// uniform = lo + (hi - lo) * u with u = top 24 bits * 2^-24, evaluated in binary64.
void fill_uniform(float* out, size_t n, uint64_t seed, float lo, float hi) {
  uint64_t s = seed;
  const double span = double(hi) - double(lo);
  for (size_t i = 0; i < n; ++i) {
    const double u = double(splitmix64(&s) >> 40) * (1.0 / 16777216.0);
    out[i] = float(double(lo) + span * u);
  }
}

// Box-Muller over pairs: u1 in (0,1], u2 in [0,1), 53-bit resolution.
void fill_normal(float* out, size_t n, uint64_t seed, float mu, float sigma) {
  uint64_t s = seed;
  constexpr double kTwoPi = 6.283185307179586476925286766559;
  for (size_t i = 0; i < n; i += 2) {
    const double u1 = double((splitmix64(&s) >> 11) + 1) * (1.0 / 9007199254740992.0);
    const double u2 = double(splitmix64(&s) >> 11) * (1.0 / 9007199254740992.0);
    const double r = std::sqrt(-2.0 * std::log(u1));
    out[i] = float(double(mu) + double(sigma) * (r * std::cos(kTwoPi * u2)));
    if (i + 1 < n) out[i + 1] = float(double(mu) + double(sigma) * (r * std::sin(kTwoPi * u2)));
  }
}

void fill_sawtooth(float* out, size_t n, int period, int offset, float unit, float bias) {
  for (size_t i = 0; i < n; ++i) {
    const int idx = int(i);
    const float t = float((idx % period) - offset) * unit;
    out[i] = bias == 0.0f ? t : bias + t;
  }
}

uint16_t f32_to_f16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint16_t sign = uint16_t((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return ax == 0x7f800000u ? uint16_t(sign | 0x7c00u) : uint16_t(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
  if (ax >= 0x477ff000u) return uint16_t(sign | 0x7c00u);
  if (ax >= 0x38800000u) {
    uint32_t h = (ax - 0x38000000u) >> 13;
    const uint32_t rem = ax & 0x1fffu;
    h += (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ? 1u : 0u;
    return uint16_t(sign | h);
  }
  if (ax < 0x33000000u) return sign;
  const uint32_t e = ax >> 23;
  const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
  const uint32_t sh = 126u - e;
  uint32_t h = mant >> sh;
  const uint32_t rem = mant & ((1u << sh) - 1u), half = 1u << (sh - 1u);
  h += (rem > half || (rem == half && (h & 1u))) ? 1u : 0u;
  return uint16_t(sign | h);
}

float f16_to_f32(uint16_t h) {
  const uint32_t sign = uint32_t(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  uint32_t bits;
  if (e == 0) {
    const float v = float(m) * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  bits = e == 31 ? (sign | 0x7f800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

void q8_0_pack(const int8_t* q, const uint16_t* d, uint8_t* blocks, int N, int K) {
  const int nb = K / 32;
  for (int n = 0; n < N; ++n)
    for (int b = 0; b < nb; ++b) {
      uint8_t* blk = blocks + (size_t(n) * nb + b) * kQ8Block;
      const uint16_t dv = d[size_t(n) * nb + b];
      blk[0] = uint8_t(dv & 0xff);
      blk[1] = uint8_t(dv >> 8);
      std::memcpy(blk + 2, q + size_t(n) * K + size_t(b) * 32, 32);
    }
}

int ref_threads(int64_t n) {
  if (n < 64) return 1;
  return int(std::min<unsigned>(std::max(1u, std::thread::hardware_concurrency()), 32u));
}

namespace {
template <typename F>
void parallel_for(int64_t n, F&& f) {
  const int th = ref_threads(n);
  std::vector<std::thread> ts;
  for (int t = 1; t < th; ++t) ts.emplace_back([&, t] { f(n * t / th, n * (t + 1) / th); });
  f(0, n / th);
  for (auto& x : ts) x.join();
}
}  // namespace

void ref_rowsum(const float* X, double* Y, double* Yabs, int64_t L, int64_t C) {
  parallel_for(L, [&](int64_t a, int64_t b) {
    for (int64_t l = a; l < b; ++l) {
      double s = 0, q = 0;
      for (int64_t c = 0; c < C; ++c) {
        s += X[l * C + c];
        q += std::fabs(double(X[l * C + c]));
      }
      Y[l] = s;
      if (Yabs) Yabs[l] = q;
    }
  });
}

void ref_rmsnorm(const float* X, const float* W, double* Y, int64_t L, int64_t C, double eps) {
  parallel_for(L, [&](int64_t a, int64_t b) {
    for (int64_t l = a; l < b; ++l) {
      double ss = 0;
      for (int64_t c = 0; c < C; ++c) ss += double(X[l * C + c]) * double(X[l * C + c]);
      const double rms = 1.0 / std::sqrt(ss / double(C) + eps);
      for (int64_t c = 0; c < C; ++c) Y[l * C + c] = double(X[l * C + c]) * rms * double(W[c]);
    }
  });
}

void ref_softmax(const float* X, double* Y, int64_t L, int64_t C) {
  parallel_for(L, [&](int64_t a, int64_t b) {
    for (int64_t l = a; l < b; ++l) {
      double m = -INFINITY;
      for (int64_t c = 0; c < C; ++c) m = std::max(m, double(X[l * C + c]));
      double s = 0;
      for (int64_t c = 0; c < C; ++c) s += std::exp(double(X[l * C + c]) - m);
      for (int64_t c = 0; c < C; ++c) Y[l * C + c] = std::exp(double(X[l * C + c]) - m) / s;
    }
  });
}

void ref_gemm(const float* A, const float* B, double* C, int64_t M, int64_t N, int64_t K, bool bt,
              const std::vector<int64_t>& rows) {
  std::vector<int64_t> rs = rows;
  if (rs.empty())
    for (int64_t i = 0; i < M; ++i) rs.push_back(i);
  parallel_for(int64_t(rs.size()), [&](int64_t a, int64_t b) {
    std::vector<double> acc(static_cast<size_t>(N));
    for (int64_t ii = a; ii < b; ++ii) {
      const int64_t i = rs[size_t(ii)];
      std::fill(acc.begin(), acc.end(), 0.0);
      for (int64_t k = 0; k < K; ++k) {
        const double av = A[i * K + k];
        if (bt) {
          for (int64_t j = 0; j < N; ++j) acc[size_t(j)] += av * double(B[j * K + k]);
        } else {
          const float* brow = B + k * N;
          for (int64_t j = 0; j < N; ++j) acc[size_t(j)] += av * double(brow[j]);
        }
      }
      for (int64_t j = 0; j < N; ++j) C[ii * N + j] = acc[size_t(j)];
    }
  });
}

void ref_conv_nchw(const float* x, const float* w, const float* scale, double* y, int64_t Nb, int64_t C, int64_t H,
                   int64_t W, int64_t Oc, int64_t Kh, int64_t Kw, int64_t pad, int64_t stride,
                   const std::vector<int64_t>& images) {
  const int64_t Ho = (H + 2 * pad - Kh) / stride + 1, Wo = (W + 2 * pad - Kw) / stride + 1;
  std::vector<int64_t> ims = images;
  if (ims.empty())
    for (int64_t n = 0; n < Nb; ++n) ims.push_back(n);
  const int64_t planes = int64_t(ims.size()) * Oc;
  parallel_for(planes, [&](int64_t a, int64_t b) {
    for (int64_t p = a; p < b; ++p) {
      const int64_t n = ims[size_t(p / Oc)], oc = p % Oc;
      for (int64_t ho = 0; ho < Ho; ++ho)
        for (int64_t wo = 0; wo < Wo; ++wo) {
          double acc = 0;
          for (int64_t c = 0; c < C; ++c)
            for (int64_t kh = 0; kh < Kh; ++kh) {
              const int64_t hi = ho * stride + kh - pad;
              if (hi < 0 || hi >= H) continue;
              for (int64_t kw = 0; kw < Kw; ++kw) {
                const int64_t wi = wo * stride + kw - pad;
                if (wi < 0 || wi >= W) continue;
                acc += double(x[((n * C + c) * H + hi) * W + wi]) * double(w[((oc * C + c) * Kh + kh) * Kw + kw]);
              }
            }
          y[((p / Oc * Oc + oc) * Ho + ho) * Wo + wo] = scale ? acc * double(scale[oc]) : acc;
        }
    }
  });
}

void ref_conv_hwc(const float* x, const float* wt, const float* scale, double* y, int64_t H, int64_t W, int64_t C,
                  int64_t Kh, int64_t Kw, int64_t Oc) {
  const int64_t Ho = H - Kh + 1, Wo = W - Kw + 1;
  parallel_for(Oc, [&](int64_t a, int64_t b) {
    for (int64_t oc = a; oc < b; ++oc)
      for (int64_t ho = 0; ho < Ho; ++ho)
        for (int64_t wo = 0; wo < Wo; ++wo) {
          double acc = 0;
          for (int64_t c = 0; c < C; ++c)
            for (int64_t kh = 0; kh < Kh; ++kh)
              for (int64_t kw = 0; kw < Kw; ++kw)
                acc += double(x[((ho + kh) * W + (wo + kw)) * C + c]) * double(wt[((oc * Kh + kh) * Kw + kw) * C + c]);
          y[(oc * Ho + ho) * Wo + wo] = scale ? acc * double(scale[oc]) : acc;
        }
  });
}

void ref_q8_0(const uint16_t* X, const uint8_t* blocks, double* Y, int64_t M, int64_t N, int64_t K) {
  const int64_t nb = K / 32;
  std::vector<float> xf(size_t(M * K));
  for (size_t i = 0; i < xf.size(); ++i) xf[i] = f16_to_f32(X[i]);
  parallel_for(N, [&](int64_t a, int64_t b) {
    std::vector<double> acc(static_cast<size_t>(M));
    for (int64_t n = a; n < b; ++n) {
      std::fill(acc.begin(), acc.end(), 0.0);
      for (int64_t bb = 0; bb < nb; ++bb) {
        const uint8_t* blk = blocks + (n * nb + bb) * kQ8Block;
        const float d = f16_to_f32(uint16_t(blk[0] | (blk[1] << 8)));
        for (int i = 0; i < 32; ++i) {
          const double wv = double(d * float(int8_t(blk[2 + i])));
          for (int64_t m = 0; m < M; ++m) acc[size_t(m)] += wv * double(xf[size_t(m * K + bb * 32 + i)]);
        }
      }
      for (int64_t m = 0; m < M; ++m) Y[m * N + n] = acc[size_t(m)];
    }
  });
}

double max_rel(const float* got, const double* ref, size_t n, double floor) {
  double worst = 0;
  for (size_t i = 0; i < n; ++i) {
    const double den = std::max(std::fabs(ref[i]), floor);
    const double r = std::fabs(double(got[i]) - ref[i]) / den;
    if (r > worst || std::isnan(r)) worst = std::isnan(r) ? INFINITY : r;
  }
  return worst;
}

double frobenius_rel(const float* got, const double* ref, size_t n) {
  double num = 0, den = 0;
  for (size_t i = 0; i < n; ++i) {
    const double d = double(got[i]) - ref[i];
    num += d * d;
    den += ref[i] * ref[i];
  }
  if (std::isnan(num)) return INFINITY;
  return den > 0 ? std::sqrt(num / den) : std::sqrt(num);
}

}  // namespace uk
