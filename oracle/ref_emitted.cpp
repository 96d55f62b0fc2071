// Entry points into the CPU references of the reference's stored, emitted HIP programs —
// TEST INFRASTRUCTURE ONLY.
//
// The reference's gemm/softmax/rmsnorm/channelscale CPU references exist only inside the
// programs src/codegen_hip.cpp emits; the reference keeps emitted copies under
// docs/evidence/phase64/emit/*/uk_amd.cpp and docs/evidence/phase15/emit/uk_amd_gemm.cpp.
// (The later stored gemm programs, phase45-65, target Windows: they pass unsigned long long*
// to hipMemGetInfo, which does not compile against the Linux HIP headers, so the gemm entry
// points use the phase15 program, whose cpu_ref is the same loop as codegen_hip.cpp:1124-1132
// and :1814-1822.) oracle/Makefile compiles this file once
// per stored program, host-only, with UK_EMITTED_FILE naming the program where it lies and
// UK_EMITTED_KIND selecting the entry point below. The program's main() is renamed so the
// static CPU reference in the same translation unit can be called directly; nothing in the
// program runs except that function.
#define UK_CAT2(a, b) a##b
#define UK_CAT(a, b) UK_CAT2(a, b)
#define main UK_CAT(uk_emitted_program_main_, UK_EMITTED_KIND)
#include UK_EMITTED_FILE
#undef main

#include <cstring>
#include <vector>

#if UK_EMITTED_KIND == 1  // phase64/emit/softmax: cpu_softmax (codegen_hip.cpp:1999-2009)
extern "C" void ref_emit_softmax(const float* x, float* y, int L, int C) {
  std::vector<float> X(x, x + (size_t)L * C), Y((size_t)L * C);
  cpu_softmax(X, Y, L, C);
  std::memcpy(y, Y.data(), Y.size() * sizeof(float));
}
#elif UK_EMITTED_KIND == 2  // phase64/emit/rmsnorm: cpu_rmsnorm (codegen_hip.cpp:2168-2178)
extern "C" void ref_emit_rmsnorm(const float* x, const float* w, float* y, int L, int C) {
  std::vector<float> X(x, x + (size_t)L * C), W(w, w + C), Y((size_t)L * C);
  cpu_rmsnorm(X, W, Y, L, C);
  std::memcpy(y, Y.data(), Y.size() * sizeof(float));
}
#elif UK_EMITTED_KIND == 3  // phase64/emit/channelscale: cpu_channelscale (codegen_hip.cpp:2339-2344)
extern "C" void ref_emit_channelscale(const float* x, const float* s, float* y, int L, int C) {
  std::vector<float> X(x, x + (size_t)L * C), S(s, s + C), Y((size_t)L * C);
  cpu_channelscale(X, S, Y, L, C);
  std::memcpy(y, Y.data(), Y.size() * sizeof(float));
}
#elif UK_EMITTED_KIND == 4  // phase15/emit/uk_amd_gemm.cpp: cpu_ref (codegen_hip.cpp:1124-1132)
#include <hip/hip_fp16.h>  // the header the fp16 program includes for __float2half/__half2float
extern "C" void ref_emit_gemm_f32(const float* a, const float* b, float* c, int M, int N, int K) {
  std::vector<float> A(a, a + (size_t)M * K), B(b, b + (size_t)K * N), Cv((size_t)M * N);
  cpu_ref(A, B, Cv, M, N, K);
  std::memcpy(c, Cv.data(), Cv.size() * sizeof(float));
}
// The fp16 program (codegen_hip.cpp:1852-1862) rounds the inputs with __float2half, widens them
// with __half2float and runs the same cpu_ref loop on the quantized values.
extern "C" void ref_emit_gemm_f16(const float* a, const float* b, float* c, int M, int N, int K) {
  std::vector<float> qA((size_t)M * K), qB((size_t)K * N), Cv((size_t)M * N);
  for (size_t i = 0; i < qA.size(); ++i) qA[i] = __half2float(__float2half(a[i]));
  for (size_t i = 0; i < qB.size(); ++i) qB[i] = __half2float(__float2half(b[i]));
  cpu_ref(qA, qB, Cv, M, N, K);
  std::memcpy(c, Cv.data(), Cv.size() * sizeof(float));
}
// The program's own half conversion, exposed so the oracle's binary16 rounding can be
// checked against it value by value.
extern "C" void ref_emit_float2half(const float* in, unsigned short* out, long long n) {
  for (long long i = 0; i < n; ++i) {
    const __half h = __float2half(in[i]);
    std::memcpy(&out[i], &h, 2);
  }
}
extern "C" void ref_emit_sawtooth_ab(float* a, float* b, int n) {
  for (int i = 0; i < n; ++i) {
    a[i] = initA(i);
    b[i] = initB(i);
  }
}
#else
#error "UK_EMITTED_KIND must be 1..4"
#endif
