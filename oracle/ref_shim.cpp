// C-ABI glue around the reference's own CPU functions — TEST INFRASTRUCTURE ONLY.
//
// oracle/Makefile compiles this file together with the reference sources where they lie
// (/root/reference/src/{reference,kml,kml_front,json_flat,hcs,solver,runtime,codegen_hip}.cpp)
// into oracle/_ref/libukref.so. Tests use it to check the oracle restatement and the host
// front end against the reference's real behaviour, and tests/golden/make_golden.py uses it
// to write fixtures. Nothing here is shipped; the GPU box never builds it.
#include <cstdint>
#include <cstring>
#include <string>

#include "unikern/codegen.hpp"
#include "unikern/components.hpp"
#include "unikern/core.hpp"

using namespace unikern;

namespace {
int put(const std::string& s, char* out, int cap) {
  if (!out || cap <= 0) return (int)s.size();
  const size_t n = s.size() < (size_t)cap - 1 ? s.size() : (size_t)cap - 1;
  std::memcpy(out, s.data(), n);
  out[n] = 0;
  return (int)s.size();
}
}  // namespace

extern "C" {

// src/reference.cpp:6-48
void ref_cpu_conv(const float* x, const float* wt, float* y, int H, int W, int C, int Kh, int Kw, int Oc) {
  cpu_conv(x, wt, y, H, W, C, Kh, Kw, Oc);
}
void ref_cpu_reduce(const float* x, float* y, long long n) { cpu_reduce(x, y, n); }
void ref_cpu_reduce_blocked(const float* x, float* y, long long n, int width) {
  cpu_reduce_blocked(x, y, n, width);
}
int ref_kref_reduce_width() { return kRefReduceWidth; }

// src/kml_front.cpp:203-217 kml_import; returns 1 on accept. Fields are written only on accept.
int ref_kml_import(const char* json, int* op, int* dtype, int* dims6, int* tile_m, int* tile_n, char* layout,
                   int layout_cap, int* n_children, char* err, int err_cap) {
  std::string e;
  const auto t = kml_import(json, &e);
  if (!t) {
    put(e, err, err_cap);
    return 0;
  }
  *op = (int)t->op;
  *dtype = (int)t->dtype;
  for (int i = 0; i < 6; ++i) dims6[i] = t->dims[i];
  *tile_m = t->tile_m;
  *tile_n = t->tile_n;
  put(t->layout, layout, layout_cap);
  *n_children = (int)t->children.size();
  return 1;
}

// src/kml.cpp:57-122 over an imported tree; returns -1 when the import is rejected.
int ref_kml_canonical(const char* json, char* out, int cap) {
  const auto t = kml_import(json, nullptr);
  return t ? put(canonical_form(*t), out, cap) : -1;
}
int ref_kml_signature(const char* json, char* out, int cap) {
  const auto t = kml_import(json, nullptr);
  return t ? put(op_signature(*t), out, cap) : -1;
}
int ref_kml_export(const char* json, char* out, int cap) {
  const auto t = kml_import(json, nullptr);
  return t ? put(kml_export(*t), out, cap) : -1;
}
int ref_kml_tree_hash(const char* json, char* out, int cap) {
  const auto t = kml_import(json, nullptr);
  return t ? put(fnv1a_hex(canonical_form(*t)), out, cap) : -1;
}
// src/kml.cpp:125-177
int ref_workload(const char* json, long long* ops, long long* bytes) {
  const auto t = kml_import(json, nullptr);
  if (!t) return 0;
  const Workload w = workload_of(*t);
  *ops = w.ops;
  *bytes = w.bytes;
  return 1;
}
int ref_fnv1a(const char* data, char* out, int cap) { return put(fnv1a_hex(data), out, cap); }

// src/hcs.cpp:52-115
int ref_hcs_fingerprint(const char* json, char* out, int cap) {
  std::string e;
  const auto h = hcs_import(json, &e);
  if (!h) {
    put(e, out, cap);
    return 0;
  }
  put(hcs_fingerprint(*h), out, cap);
  return 1;
}
int ref_hcs_export(const char* json, char* out, int cap) {
  const auto h = hcs_import(json, nullptr);
  return h ? put(hcs_export(*h), out, cap) : -1;
}

// src/solver.cpp:141-186
int ref_solve(const char* hcs_json, const char* kml_json, int* tile_m, int* tile_n, int* path, double* c_ms,
              int* feasible_count) {
  const auto h = hcs_import(hcs_json, nullptr);
  const auto t = kml_import(kml_json, nullptr);
  if (!h || !t) return 0;
  const Solution s = solve(*h, *t);
  *tile_m = s.best.tile_m;
  *tile_n = s.best.tile_n;
  *path = (int)s.best.path;
  *c_ms = s.c_ms;
  *feasible_count = s.feasible_count;
  return 1;
}

// src/runtime.cpp:182-213
double ref_tolerance_for(int dtype) { return tolerance_for((DType)dtype); }
int ref_verify_fp32(const float* got, const float* ref, int n, double fp32_rel, double* max_rel) {
  const std::vector<float> g(got, got + n), r(ref, ref + n);
  Tolerance tol;
  tol.fp32_rel = fp32_rel;
  const Verdict v = verify_fp32(g, r, tol);
  *max_rel = v.max_rel_err;
  return v.ok ? 1 : 0;
}

// src/codegen_hip.cpp:124-130
int ref_op_support_gap(const char* kml_json, char* out, int cap) {
  const auto t = kml_import(kml_json, nullptr);
  if (!t) return -1;
  return put(op_support_gap(*t), out, cap);
}

}  // extern "C"
