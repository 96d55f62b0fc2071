// Hardware description (HCS) import/export/fingerprint, plus the built-in MI355X description.
//
// Reference behaviour kept (src/hcs.cpp:52-148): the same fields, tiers with a legacy flat
// form, unknown keys ignored, rejection with the complete missing-field list, and a
// fingerprint over the modelled capability fields that is byte-identical to the reference's
// for a file without CDNA4 fields. CDNA4 fields (wave size, LDS, XCDs, MFMA shapes, clocks,
// HBM bandwidth) are optional keys; when present they enter the fingerprint under schema=3.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <sstream>

#include "json.hpp"
#include "uk_core.hpp"

namespace uk {

int64_t Hcs::tier_bytes(const std::string& name) const {
  for (const auto& t : tiers)
    if (t.name == name) return t.bytes;
  return 0;
}
double Hcs::tier_bw(const std::string& name) const {
  for (const auto& t : tiers)
    if (t.name == name) return t.bw_gbps;
  return 0;
}
int64_t Hcs::device_capacity() const { return unified_memory ? tier_bytes("unified") : tier_bytes("vram"); }

namespace {

std::string str_of(const json::Value* v) { return v ? (v->is_string() ? v->text : v->scalar_text()) : ""; }
double num_of(const json::Value* v, double dflt = 0) {
  if (!v) return dflt;
  if (v->is_number()) return v->num;
  if (v->is_string()) {
    char* end = nullptr;
    const double d = std::strtod(v->text.c_str(), &end);
    return (end && end != v->text.c_str()) ? d : dflt;
  }
  return dflt;
}
int64_t int_of(const json::Value* v, int64_t dflt = 0) {
  if (!v) return dflt;
  long long x = 0;
  if (json::as_int64(*v, &x)) return x;
  return int64_t(num_of(v, double(dflt)));
}
Confidence conf_of(const std::string& s) {
  return s == "measured" ? Confidence::Measured : s == "predicted" ? Confidence::Predicted : Confidence::Official;
}
const char* conf_name(Confidence c) {
  return c == Confidence::Measured ? "measured" : c == Confidence::Predicted ? "predicted" : "official";
}
// std::ostream's default formatting of a double (6 significant digits, %g), which the
// reference's fingerprint string uses (src/hcs.cpp:106-113).
std::string g6(double v) {
  char b[64];
  std::snprintf(b, sizeof b, "%g", v);
  return b;
}
std::string g17(double v) {
  char b[64];
  std::snprintf(b, sizeof b, "%.17g", v);
  return b;
}

}  // namespace

std::optional<Hcs> hcs_import(const std::string& text, std::string* err) {
  std::string perr;
  const auto jv = json::parse(text, &perr);
  if (!jv || jv->kind != json::Value::Kind::Object) {
    if (err) *err = jv ? "HCS must be a JSON object" : perr;
    return std::nullopt;
  }
  const json::Value& j = *jv;
  Hcs h;
  h.vendor = str_of(j.get("vendor"));
  h.device = str_of(j.get("device"));
  if (const auto* u = j.get("unified_memory")) h.unified_memory = u->kind == json::Value::Kind::Bool ? u->b : str_of(u) == "true";
  h.link_bw_gbps = num_of(j.get("link_bw_gbps"));
  h.flops_gflops = num_of(j.get("flops_gflops"));
  h.compute_units = int(int_of(j.get("compute_units")));
  h.toolchain = str_of(j.get("toolchain"));
  if (const auto* tiers = j.get("tiers"); tiers && tiers->kind == json::Value::Kind::Array) {
    for (const auto& tb : tiers->arr) {
      StorageTier t;
      t.name = str_of(tb.get("name"));
      if (t.name.empty()) continue;  // a tier without a name cannot be addressed (src/hcs.cpp:21)
      t.bytes = int_of(tb.get("bytes"));
      t.bw_gbps = num_of(tb.get("bw_gbps"));
      t.confidence = conf_of(tb.get("confidence") ? str_of(tb.get("confidence")) : "official");
      h.tiers.push_back(t);
    }
  }
  if (h.tiers.empty()) {  // legacy flat form (src/hcs.cpp:63-74)
    if (h.unified_memory)
      h.tiers.push_back({"unified", int_of(j.get("unified_bytes")), num_of(j.get("mem_bw_gbps")), Confidence::Official});
    else
      h.tiers.push_back({"vram", int_of(j.get("vram_bytes")), num_of(j.get("mem_bw_gbps")), Confidence::Official});
  }
  h.confidence = conf_of(j.get("confidence") ? str_of(j.get("confidence")) : "official");
  h.constants_version = int(int_of(j.get("constants_version"), 1));
  if (h.constants_version < 1) h.constants_version = 1;

  // CDNA4 extension
  h.arch = str_of(j.get("arch"));
  h.wave_size = int(int_of(j.get("wave_size")));
  h.simds_per_cu = int(int_of(j.get("simds_per_cu")));
  h.xcds = int(int_of(j.get("xcds")));
  h.max_waves_per_simd = int(int_of(j.get("max_waves_per_simd")));
  h.vgprs_per_lane = int(int_of(j.get("vgprs_per_lane")));
  h.lds_bytes_per_cu = int_of(j.get("lds_bytes_per_cu"));
  h.lds_bytes_per_block = int_of(j.get("lds_bytes_per_block"));
  h.l2_bytes_per_xcd = int_of(j.get("l2_bytes_per_xcd"));
  h.mall_bytes = int_of(j.get("mall_bytes"));
  h.clock_mhz = num_of(j.get("clock_mhz"));
  h.hbm_bw_gbps = num_of(j.get("hbm_bw_gbps"));
  h.peak_f16_mfma_tflops = num_of(j.get("peak_f16_mfma_tflops"));
  h.peak_f32_mfma_tflops = num_of(j.get("peak_f32_mfma_tflops"));
  h.peak_f32_valu_tflops = num_of(j.get("peak_f32_valu_tflops"));
  h.launch_overhead_us = num_of(j.get("launch_overhead_us"));
  if (const auto* mf = j.get("mfma"); mf && mf->kind == json::Value::Kind::Array) {
    for (const auto& e : mf->arr) {
      MfmaShape m;
      m.name = str_of(e.get("name"));
      m.in = str_of(e.get("in"));
      m.m = int(int_of(e.get("m")));
      m.n = int(int_of(e.get("n")));
      m.k = int(int_of(e.get("k")));
      m.cycles = int(int_of(e.get("cycles")));
      if (!m.name.empty()) h.mfma.push_back(m);
    }
  }

  std::vector<std::string> missing;  // src/hcs.cpp:83-99
  if (h.vendor.empty()) missing.push_back("vendor");
  if (h.device.empty()) missing.push_back("device");
  if (h.device_capacity() <= 0) missing.push_back(h.unified_memory ? "tiers[unified].bytes" : "tiers[vram].bytes");
  if (h.tier_bw(h.unified_memory ? "unified" : "vram") <= 0) missing.push_back("tiers[device].bw_gbps");
  if (h.link_bw_gbps <= 0) missing.push_back("link_bw_gbps");
  if (h.flops_gflops <= 0) missing.push_back("flops_gflops");
  if (h.compute_units <= 0) missing.push_back("compute_units");
  if (h.cdna4()) {  // a CDNA4 description must carry what the solver's predicates read
    if (h.wave_size <= 0) missing.push_back("wave_size");
    if (h.simds_per_cu <= 0) missing.push_back("simds_per_cu");
    if (h.lds_bytes_per_cu <= 0) missing.push_back("lds_bytes_per_cu");
    if (h.vgprs_per_lane <= 0) missing.push_back("vgprs_per_lane");
    if (h.clock_mhz <= 0) missing.push_back("clock_mhz");
    if (h.hbm_bw_gbps <= 0) missing.push_back("hbm_bw_gbps");
  }
  if (!missing.empty()) {
    std::ostringstream os;
    os << "missing required fields:";
    for (const auto& m : missing) os << " " << m;
    if (err) *err = os.str();
    return std::nullopt;
  }
  if (h.cdna4()) {
    if (h.lds_bytes_per_block <= 0) h.lds_bytes_per_block = h.lds_bytes_per_cu;
    if (h.xcds <= 0) h.xcds = 1;
    if (h.max_waves_per_simd <= 0) h.max_waves_per_simd = 8;
  }
  return h;
}

std::string hcs_fingerprint(const Hcs& h) {
  std::ostringstream os;
  os << "vendor=" << h.vendor << ";device=" << h.device << ";unified=" << (h.unified_memory ? 1 : 0)
     << ";linkbw=" << g6(h.link_bw_gbps) << ";flops=" << g6(h.flops_gflops) << ";cu=" << h.compute_units;
  for (const auto& t : h.tiers) os << ";tier=" << t.name << ":" << t.bytes << ":" << g6(t.bw_gbps);
  if (!h.cdna4()) {
    os << ";schema=2";
  } else {
    os << ";arch=" << h.arch << ";wave=" << h.wave_size << ";simd=" << h.simds_per_cu << ";xcd=" << h.xcds
       << ";waves=" << h.max_waves_per_simd << ";vgpr=" << h.vgprs_per_lane << ";lds=" << h.lds_bytes_per_cu
       << ":" << h.lds_bytes_per_block << ";l2=" << h.l2_bytes_per_xcd << ";mall=" << h.mall_bytes
       << ";clk=" << g6(h.clock_mhz) << ";hbm=" << g6(h.hbm_bw_gbps) << ";f16=" << g6(h.peak_f16_mfma_tflops)
       << ";f32=" << g6(h.peak_f32_mfma_tflops) << ";valu=" << g6(h.peak_f32_valu_tflops);
    for (const auto& m : h.mfma) os << ";mfma=" << m.name << ":" << m.m << "x" << m.n << "x" << m.k << ":" << m.cycles;
    os << ";schema=3";
  }
  return fnv1a_hex(os.str());
}

std::string hcs_export(const Hcs& h) {
  std::ostringstream os;
  os << "{\n"
     << "  \"vendor\": \"" << h.vendor << "\",\n"
     << "  \"device\": \"" << h.device << "\",\n"
     << "  \"unified_memory\": " << (h.unified_memory ? "true" : "false") << ",\n"
     << "  \"link_bw_gbps\": " << g17(h.link_bw_gbps) << ",\n"
     << "  \"flops_gflops\": " << g17(h.flops_gflops) << ",\n"
     << "  \"compute_units\": " << h.compute_units << ",\n"
     << "  \"toolchain\": \"" << h.toolchain << "\",\n"
     << "  \"constants_version\": " << h.constants_version << ",\n"
     << "  \"confidence\": \"" << conf_name(h.confidence) << "\",\n";
  if (h.cdna4()) {
    os << "  \"arch\": \"" << h.arch << "\",\n"
       << "  \"wave_size\": " << h.wave_size << ",\n"
       << "  \"simds_per_cu\": " << h.simds_per_cu << ",\n"
       << "  \"xcds\": " << h.xcds << ",\n"
       << "  \"max_waves_per_simd\": " << h.max_waves_per_simd << ",\n"
       << "  \"vgprs_per_lane\": " << h.vgprs_per_lane << ",\n"
       << "  \"lds_bytes_per_cu\": " << h.lds_bytes_per_cu << ",\n"
       << "  \"lds_bytes_per_block\": " << h.lds_bytes_per_block << ",\n"
       << "  \"l2_bytes_per_xcd\": " << h.l2_bytes_per_xcd << ",\n"
       << "  \"mall_bytes\": " << h.mall_bytes << ",\n"
       << "  \"clock_mhz\": " << g17(h.clock_mhz) << ",\n"
       << "  \"hbm_bw_gbps\": " << g17(h.hbm_bw_gbps) << ",\n"
       << "  \"peak_f16_mfma_tflops\": " << g17(h.peak_f16_mfma_tflops) << ",\n"
       << "  \"peak_f32_mfma_tflops\": " << g17(h.peak_f32_mfma_tflops) << ",\n"
       << "  \"peak_f32_valu_tflops\": " << g17(h.peak_f32_valu_tflops) << ",\n"
       << "  \"launch_overhead_us\": " << g17(h.launch_overhead_us) << ",\n"
       << "  \"mfma\": [\n";
    for (size_t i = 0; i < h.mfma.size(); ++i) {
      const MfmaShape& m = h.mfma[i];
      os << "    { \"name\": \"" << m.name << "\", \"in\": \"" << m.in << "\", \"m\": " << m.m << ", \"n\": " << m.n
         << ", \"k\": " << m.k << ", \"cycles\": " << m.cycles << " }" << (i + 1 < h.mfma.size() ? "," : "") << "\n";
    }
    os << "  ],\n";
  }
  os << "  \"tiers\": [\n";
  for (size_t i = 0; i < h.tiers.size(); ++i) {
    const StorageTier& t = h.tiers[i];
    os << "    { \"name\": \"" << t.name << "\", \"bytes\": " << t.bytes << ", \"bw_gbps\": " << g17(t.bw_gbps)
       << ", \"confidence\": \"" << conf_name(t.confidence) << "\" }" << (i + 1 < h.tiers.size() ? "," : "") << "\n";
  }
  os << "  ]\n}\n";
  return os.str();
}

// One MI355X (AMD public specifications; the CU count, clock and LDS limits are re-read on
// the device by uk_device_check). Same text as samples/hcs_mi355x.json.
const char* hcs_mi355x_json() {
  return R"JSON({
  "vendor": "amd",
  "device": "AMD Instinct MI355X (gfx950, CDNA4)",
  "unified_memory": false,
  "link_bw_gbps": 64,
  "flops_gflops": 2516582.4,
  "compute_units": 256,
  "toolchain": "rocm-7.2.0",
  "constants_version": 1,
  "confidence": "official",
  "arch": "gfx950",
  "wave_size": 64,
  "simds_per_cu": 4,
  "xcds": 8,
  "max_waves_per_simd": 8,
  "vgprs_per_lane": 512,
  "lds_bytes_per_cu": 163840,
  "lds_bytes_per_block": 163840,
  "l2_bytes_per_xcd": 4194304,
  "mall_bytes": 268435456,
  "clock_mhz": 2400,
  "hbm_bw_gbps": 8000,
  "peak_f16_mfma_tflops": 2516.5824,
  "peak_f32_mfma_tflops": 157.2864,
  "peak_f32_valu_tflops": 157.2864,
  "launch_overhead_us": 2.0,
  "mfma": [
    { "name": "f32_32x32x16_f16", "in": "fp16", "m": 32, "n": 32, "k": 16, "cycles": 32 },
    { "name": "f32_16x16x32_f16", "in": "fp16", "m": 16, "n": 16, "k": 32, "cycles": 16 },
    { "name": "f32_32x32x2_f32", "in": "fp32", "m": 32, "n": 32, "k": 2, "cycles": 64 },
    { "name": "f32_16x16x4_f32", "in": "fp32", "m": 16, "n": 16, "k": 4, "cycles": 32 }
  ],
  "tiers": [
    { "name": "vram", "bytes": 309237645312, "bw_gbps": 8000, "confidence": "official" },
    { "name": "ram", "bytes": 1649267441664, "bw_gbps": 200, "confidence": "predicted" }
  ]
}
)JSON";
}

const Hcs& hcs_mi355x() {
  static const Hcs h = [] {
    std::string e;
    auto v = hcs_import(hcs_mi355x_json(), &e);
    if (!v) {
      std::fprintf(stderr, "UNIKERN_ERROR what=builtin_hcs msg=%s\n", e.c_str());
      std::abort();
    }
    return *v;
  }();
  return h;
}

}  // namespace uk
