// KML op-spec front end: import with a complete violation list, export, canonical form,
// op signature, workload model and the capability gate.
//
// Behaviour follows the reference's src/kml_front.cpp:75-217 and src/kml.cpp:57-177:
// the same keys, the same per-field checks and messages, every violation reported at once,
// children validated with a path prefix and composed only when clean. Reference files parse
// unchanged and give the same canonical form, signature and tree hash. The extensions needed
// by the MI355X configs are additive (see uk_core.hpp): reduce with 2 dims (row-sum), layout
// TN (column-major B), conv layout NCHW with batch/pad/stride, a fused channelscale epilogue,
// an explicit rmsnorm eps, and dtype q8_0.
#include <climits>
#include <cmath>
#include <cstdio>
#include <algorithm>
#include <sstream>

#include "json.hpp"
#include "uk_core.hpp"

namespace uk {

const char* to_string(OpKind k) {
  switch (k) {
    case OpKind::Gemm: return "gemm";
    case OpKind::Conv: return "conv";
    case OpKind::Reduction: return "reduce";
    case OpKind::Softmax: return "softmax";
    case OpKind::RmsNorm: return "rmsnorm";
    case OpKind::ChannelScale: return "channelscale";
  }
  return "?";
}
const char* to_string(DType d) {
  switch (d) {
    case DType::F32: return "fp32";
    case DType::F16: return "fp16";
    case DType::I8: return "int8";
    case DType::Q8_0: return "q8_0";
  }
  return "?";
}
const char* to_string(Layout l) {
  switch (l) {
    case Layout::NT: return "NT";
    case Layout::TN: return "TN";
    case Layout::NCHW: return "NCHW";
  }
  return "?";
}
const char* to_string(Epilogue e) { return e == Epilogue::ChannelScale ? "channelscale" : "none"; }

std::optional<OpKind> op_from_string(const std::string& s) {
  if (s == "gemm") return OpKind::Gemm;
  if (s == "conv") return OpKind::Conv;
  if (s == "reduce") return OpKind::Reduction;
  if (s == "softmax") return OpKind::Softmax;
  if (s == "rmsnorm") return OpKind::RmsNorm;
  if (s == "channelscale") return OpKind::ChannelScale;
  return std::nullopt;
}
std::optional<DType> dtype_from_string(const std::string& s) {
  if (s == "fp32") return DType::F32;
  if (s == "fp16") return DType::F16;
  if (s == "int8") return DType::I8;
  if (s == "q8_0") return DType::Q8_0;
  return std::nullopt;
}
std::optional<Layout> layout_from_string(const std::string& s) {
  if (s == "NT") return Layout::NT;
  if (s == "TN") return Layout::TN;
  if (s == "NCHW") return Layout::NCHW;
  return std::nullopt;
}
size_t dtype_size(DType d) {
  switch (d) {
    case DType::F32: return 4;
    case DType::F16: return 2;
    case DType::I8: return 1;
    case DType::Q8_0: return 1;
  }
  return 4;
}

// Arity per op (reference kml_arity, src/kml.cpp:97-107); reduce also accepts [L, C].
int kml_arity_min(OpKind op) {
  switch (op) {
    case OpKind::Gemm: return 3;
    case OpKind::Conv: return 6;
    case OpKind::Reduction: return 1;
    default: return 2;
  }
}
int kml_arity_max(OpKind op) { return op == OpKind::Reduction ? 2 : kml_arity_min(op); }

const char* kml_dim_spec(OpKind op) {
  switch (op) {
    case OpKind::Gemm: return "3 dims (M,N,K)";
    case OpKind::Conv: return "6 dims (H,W,C,Kh,Kw,outC)";
    case OpKind::Reduction: return "1 dim (L) or 2 dims (L,C)";
    case OpKind::Softmax:
    case OpKind::RmsNorm:
    case OpKind::ChannelScale: return "2 dims (L,C)";
  }
  return "3 dims (M,N,K)";
}

namespace {

bool layout_valid_for(OpKind op, Layout l) {
  if (l == Layout::NT) return true;
  if (l == Layout::TN) return op == OpKind::Gemm;
  if (l == Layout::NCHW) return op == OpKind::Conv;
  return false;
}

void parse_node(const json::Value& v, const std::string& path, KmlTree* t, std::vector<std::string>* errs) {
  auto bad = [&](const std::string& m) { errs->push_back(path + m); };
  if (v.kind != json::Value::Kind::Object) {
    bad("node is not a JSON object");
    return;
  }
  static const char* allowed[] = {"op",    "dtype", "dims",   "tile_m",   "tile_n", "layout",
                                  "batch", "pad",   "stride", "epilogue", "eps",    "children"};
  for (const auto& kv : v.obj) {
    bool known = false;
    for (const char* a : allowed)
      if (kv.first == a) known = true;
    if (!known) bad("unknown field '" + kv.first + "' (typo would otherwise be ignored)");
  }

  bool op_ok = false;
  if (const json::Value* op = v.get("op"); !op) {
    bad("missing op (one of gemm|conv|reduce|softmax|rmsnorm|channelscale)");
  } else if (const auto k = op_from_string(op->scalar_text()); !k || !op->is_string()) {
    bad("op='" + op->scalar_text() + "' not one of gemm|conv|reduce|softmax|rmsnorm|channelscale");
  } else {
    t->op = *k;
    op_ok = true;
  }

  if (const json::Value* dt = v.get("dtype"); !dt) {
    bad("missing dtype (one of fp32|fp16|int8|q8_0)");
  } else if (const auto d = dtype_from_string(dt->scalar_text()); !d || !dt->is_string()) {
    bad("dtype='" + dt->scalar_text() + "' not one of fp32|fp16|int8|q8_0");
  } else {
    t->dtype = *d;
  }

  if (const json::Value* dims = v.get("dims"); !dims) {
    bad("missing dims");
  } else if (dims->kind != json::Value::Kind::Array) {
    bad("dims must be an array of positive integers");
  } else {
    const auto& toks = dims->arr;
    bool values_ok = true;
    int vals[6] = {0, 0, 0, 0, 0, 0};
    if (toks.size() > 6) {
      bad("dims has " + std::to_string(toks.size()) + " entries, max 6");
      values_ok = false;
    }
    for (size_t i = 0; i < toks.size() && i < 6; ++i) {
      long long wide = 0;
      if (!json::as_int64(toks[i], &wide)) {
        bad("dims[" + std::to_string(i) + "]='" + toks[i].scalar_text() + "' is not an integer");
        values_ok = false;
        continue;
      }
      if (wide > INT_MAX) {
        bad("dims[" + std::to_string(i) + "]=" + toks[i].text + " exceeds " + std::to_string(INT_MAX) +
            ", the largest element index the generated kernels can address");
        values_ok = false;
        continue;
      }
      if (wide <= 0) {
        bad("dims[" + std::to_string(i) + "]=" + std::to_string(wide) + " must be positive");
        values_ok = false;
        continue;
      }
      vals[i] = int(wide);
    }
    if (op_ok && values_ok) {
      const int n = int(toks.size());
      if (n < kml_arity_min(t->op) || n > kml_arity_max(t->op)) {
        bad("dims: " + std::string(to_string(t->op)) + " needs " + kml_dim_spec(t->op) + ", got " +
            std::to_string(n));
      } else {
        t->ndims = n;
        for (int i = 0; i < 6; ++i) t->dims[i] = vals[i];
      }
    }
  }

  for (const char* key : {"tile_m", "tile_n"}) {
    const json::Value* f = v.get(key);
    if (!f) continue;
    long long n = 0;
    if (!json::as_int64(*f, &n) || n <= 0 || n > INT_MAX)
      bad(std::string(key) + "='" + f->scalar_text() + "' must be a positive integer");
    else if (key == std::string("tile_m"))
      t->tile_m = int(n);
    else
      t->tile_n = int(n);
  }

  if (const json::Value* lay = v.get("layout")) {
    const auto l = layout_from_string(lay->scalar_text());
    if (!l || !lay->is_string()) {
      bad("layout='" + lay->scalar_text() + "' is not implemented (NT: A/B/C row-major; TN: gemm with "
          "column-major B; NCHW: batched conv)");
    } else if (op_ok && !layout_valid_for(t->op, *l)) {
      bad("layout='" + lay->scalar_text() + "' does not apply to op=" + to_string(t->op));
    } else {
      t->layout = *l;
    }
  }

  auto int_field = [&](const char* key, int lo, int* out) {
    const json::Value* f = v.get(key);
    if (!f) return false;
    long long n = 0;
    if (!json::as_int64(*f, &n) || n < lo || n > INT_MAX) {
      bad(std::string(key) + "='" + f->scalar_text() + "' must be an integer >= " + std::to_string(lo));
      return false;
    }
    *out = int(n);
    return true;
  };
  const bool has_batch = int_field("batch", 1, &t->batch);
  const bool has_pad = int_field("pad", 0, &t->pad);
  const bool has_stride = int_field("stride", 1, &t->stride);
  if (op_ok && (has_batch || has_pad || has_stride) &&
      !(t->op == OpKind::Conv && t->layout == Layout::NCHW))
    bad("batch/pad/stride apply to op=conv with layout NCHW only");

  if (const json::Value* e = v.get("epilogue")) {
    const std::string s = e->scalar_text();
    if (!e->is_string() || (s != "channelscale" && s != "none"))
      bad("epilogue='" + s + "' not one of none|channelscale");
    else if (op_ok && s == "channelscale" && t->op != OpKind::Conv)
      bad("epilogue=channelscale applies to op=conv only (standalone channelscale is its own op)");
    else
      t->epilogue = s == "channelscale" ? Epilogue::ChannelScale : Epilogue::None;
  }

  if (const json::Value* e = v.get("eps")) {
    if (!e->is_number() || !(e->num > 0) || !std::isfinite(e->num) || float(e->num) <= 0.f)
      bad("eps='" + e->scalar_text() + "' must be a positive finite number");
    else if (op_ok && t->op != OpKind::RmsNorm)
      bad("eps applies to op=rmsnorm only");
    else {
      t->eps = float(e->num);
      t->has_eps = true;
    }
  }

  if (op_ok && t->op == OpKind::Conv && t->ndims == 6) {
    // The output must be non-empty: the reference's valid conv needs Kh <= H and Kw <= W.
    const int H = t->dims[0], W = t->dims[1], Kh = t->dims[3], Kw = t->dims[4];
    if (H + 2 * t->pad < Kh || W + 2 * t->pad < Kw)
      bad("conv kernel " + std::to_string(Kh) + "x" + std::to_string(Kw) + " exceeds the padded input " +
          std::to_string(H + 2 * t->pad) + "x" + std::to_string(W + 2 * t->pad));
  }

  if (const json::Value* kids = v.get("children")) {
    if (kids->kind != json::Value::Kind::Array) {
      bad("children must be an array of nodes");
    } else {
      for (size_t i = 0; i < kids->arr.size(); ++i) {
        KmlTree child;
        const size_t before = errs->size();
        parse_node(kids->arr[i], path + "children[" + std::to_string(i) + "].", &child, errs);
        if (errs->size() == before) t->children.push_back(child);
      }
    }
  }
}

std::string fmt_eps(float e) {
  char b[32];
  std::snprintf(b, sizeof b, "%.9g", double(e));
  return b;
}

void export_node(std::ostringstream& os, const KmlTree& t, bool nested) {
  // Byte layout of the reference export (src/kml_front.cpp:220-244): top-level fields indented
  // by two spaces, every child (at any depth) and its fields by four, a child list closed by
  // "]" on the last child's line. Extension fields follow "layout" with the same indentation.
  const char* in = nested ? "    " : "  ";
  os << (nested ? "    {" : "{") << "\n";
  os << in << "\"op\": \"" << to_string(t.op) << "\",\n";
  os << in << "\"dtype\": \"" << to_string(t.dtype) << "\",\n";
  os << in << "\"dims\": [";
  for (int i = 0; i < t.ndims; ++i) os << (i ? "," : "") << t.dims[i];
  os << "],\n";
  os << in << "\"tile_m\": " << t.tile_m << ",\n";
  os << in << "\"tile_n\": " << t.tile_n << ",\n";
  os << in << "\"layout\": \"" << to_string(t.layout) << "\"";
  if (t.op == OpKind::Conv && t.layout == Layout::NCHW)
    os << ",\n" << in << "\"batch\": " << t.batch << ",\n" << in << "\"pad\": " << t.pad << ",\n" << in
       << "\"stride\": " << t.stride;
  if (t.epilogue != Epilogue::None) os << ",\n" << in << "\"epilogue\": \"" << to_string(t.epilogue) << "\"";
  if (t.has_eps) os << ",\n" << in << "\"eps\": " << fmt_eps(t.eps);
  if (!t.children.empty()) {
    os << ",\n" << in << "\"children\": [";
    for (size_t i = 0; i < t.children.size(); ++i) {
      os << (i ? "," : "") << "\n";
      export_node(os, t.children[i], true);
    }
    os << "]\n";
  } else {
    os << "\n";
  }
  os << (nested ? "    " : "") << "}";
}

}  // namespace

std::optional<KmlTree> kml_import(const std::string& text, std::string* err) {
  std::string perr;
  const auto v = json::parse(text, &perr);
  KmlTree t;
  std::vector<std::string> errs;
  if (!v)
    errs.push_back(perr);
  else
    parse_node(*v, "", &t, &errs);
  if (!errs.empty()) {
    if (err) {
      std::ostringstream os;
      os << "rejected (" << errs.size() << " violations):";
      for (const auto& e : errs) os << "\n  " << e;
      *err = os.str();
    }
    return std::nullopt;
  }
  return t;
}

std::string kml_export(const KmlTree& t) {
  std::ostringstream os;
  export_node(os, t, false);
  os << "\n";
  return os.str();
}

// Reference src/kml.cpp:57-84: fixed field order, exactly the declared dims, children
// sorted. Extension fields are appended only when they differ from reference semantics, so
// every reference tree keeps its reference canonical form (and therefore its tree hash).
std::string canonical_form(const KmlTree& t) {
  std::string s = "(";
  s += to_string(t.op);
  s += ":";
  s += to_string(t.dtype);
  s += " dims=";
  for (int i = 0; i < t.ndims; ++i) {
    if (i) s += ",";
    s += std::to_string(t.dims[i]);
  }
  s += " tile=" + std::to_string(t.tile_m) + "x" + std::to_string(t.tile_n);
  s += std::string(" layout=") + to_string(t.layout);
  if (t.op == OpKind::Conv && t.layout == Layout::NCHW)
    s += " batch=" + std::to_string(t.batch) + " pad=" + std::to_string(t.pad) + " stride=" +
         std::to_string(t.stride);
  if (t.epilogue != Epilogue::None) s += std::string(" epilogue=") + to_string(t.epilogue);
  if (t.has_eps) s += " eps=" + fmt_eps(t.eps);
  std::vector<std::string> kids;
  for (const auto& c : t.children) kids.push_back(canonical_form(c));
  std::sort(kids.begin(), kids.end());
  for (const auto& k : kids) s += " " + k;
  s += ")";
  return s;
}

// Reference src/kml.cpp:86-95 (64-bit FNV-1a, 16 hex digits).
std::string fnv1a_hex(const std::string& data) {
  uint64_t h = 1469598103934665603ull;
  for (unsigned char c : data) {
    h ^= c;
    h *= 1099511628211ull;
  }
  char buf[19];
  std::snprintf(buf, sizeof buf, "%016llx", (unsigned long long)h);
  return buf;
}

// Reference src/kml.cpp:109-122 ("gemm:fp32:4096x4096x4096"); extensions add suffixes.
std::string op_signature(const KmlTree& t) {
  std::string s = std::string(to_string(t.op)) + ":" + to_string(t.dtype) + ":";
  for (int i = 0; i < t.ndims; ++i) {
    if (i) s += "x";
    s += std::to_string(t.dims[i]);
  }
  if (t.layout != Layout::NT) s += std::string(":") + to_string(t.layout);
  if (t.op == OpKind::Conv && t.layout == Layout::NCHW)
    s += ":n" + std::to_string(t.batch) + ":p" + std::to_string(t.pad) + ":s" + std::to_string(t.stride);
  if (t.epilogue != Epilogue::None) s += ":cs";
  if (t.has_eps) s += ":eps" + fmt_eps(t.eps);
  return s;
}

Shape shape_of(const KmlTree& t) {
  Shape s;
  switch (t.op) {
    case OpKind::Gemm:
      s.M = t.dims[0];
      s.N = t.dims[1];
      s.K = t.dims[2];
      break;
    case OpKind::Conv:
      s.H = t.dims[0];
      s.W = t.dims[1];
      s.Ci = t.dims[2];
      s.Kh = t.dims[3];
      s.Kw = t.dims[4];
      s.Co = t.dims[5];
      if (t.layout == Layout::NCHW) {
        s.Nb = t.batch;
        s.pad = t.pad;
        s.stride = t.stride;
      }
      s.Ho = (s.H + 2 * s.pad - s.Kh) / s.stride + 1;
      s.Wo = (s.W + 2 * s.pad - s.Kw) / s.stride + 1;
      break;
    case OpKind::Reduction:
      if (t.ndims == 2) {
        s.L = t.dims[0];
        s.C = t.dims[1];
      } else {
        s.L = 1;
        s.C = t.dims[0];
      }
      break;
    default:
      s.L = t.dims[0];
      s.C = t.dims[1];
      break;
  }
  return s;
}

// Algorithmic work: arithmetic, and the bytes each operand must cross HBM once (the
// reference's src/kml.cpp:125-177 over-counts softmax/rmsnorm/channelscale as 3*L*C and the
// 1-D reduce as 2*L; these are the corrected roofline numerators).
Workload workload_of(const KmlTree& t) {
  const Shape s = shape_of(t);
  const int64_t es = int64_t(dtype_size(t.dtype));
  Workload w;
  switch (t.op) {
    case OpKind::Gemm:
      w.ops = 2 * s.M * s.N * s.K;
      if (t.dtype == DType::Q8_0) {
        w.weight_bytes = s.N * (s.K / 32) * 34;
        w.bytes = w.weight_bytes + s.M * s.K * 2 + s.M * s.N * 4;
      } else {
        w.bytes = (s.M * s.K + s.K * s.N + s.M * s.N) * es;
      }
      break;
    case OpKind::Conv:
      w.ops = 2 * s.Nb * s.Co * s.Ho * s.Wo * s.Ci * s.Kh * s.Kw;
      w.bytes = (s.Nb * s.Ci * s.H * s.W + s.Co * s.Ci * s.Kh * s.Kw + s.Nb * s.Co * s.Ho * s.Wo +
                 (t.epilogue == Epilogue::ChannelScale ? s.Co : 0)) * es;
      break;
    case OpKind::Reduction:
      w.ops = s.L * s.C;
      w.bytes = (s.L * s.C + s.L) * es;
      break;
    case OpKind::Softmax:
      w.ops = 5 * s.L * s.C;
      w.bytes = 2 * s.L * s.C * es;
      break;
    case OpKind::RmsNorm:
      w.ops = 4 * s.L * s.C;
      w.bytes = (2 * s.L * s.C + s.C) * es;
      break;
    case OpKind::ChannelScale:
      w.ops = s.L * s.C;
      w.bytes = (2 * s.L * s.C + s.C) * es;
      break;
  }
  return w;
}

// Capability gate (reference src/codegen_hip.cpp:81-130: a refusal names the field).
std::string support_gap(const KmlTree& t) {
  const std::string dt = to_string(t.dtype);
  switch (t.op) {
    case OpKind::Gemm:
      if (t.dtype == DType::F32 || t.dtype == DType::F16) return "";
      if (t.dtype == DType::Q8_0) {
        if (t.layout != Layout::TN)
          return "dtype=q8_0 weights are stored one row per output column (layout TN); layout=" +
                 std::string(to_string(t.layout)) + " has no q8_0 kernel";
        if (t.dims[2] % 64 != 0)
          return "dtype=q8_0 needs K divisible by 64 (whole pairs of 32-element blocks per row); K=" +
                 std::to_string(t.dims[2]);
        return "";
      }
      return "dtype=" + dt + " has no gemm kernel (int8 results are refused, as in the reference)";
    case OpKind::Conv:
      if (t.dtype != DType::F32) return "dtype=" + dt + " has no conv kernel; conv runs in fp32";
      return "";
    default:
      if (t.dtype != DType::F32)
        return "dtype=" + dt + " has no " + std::string(to_string(t.op)) + " kernel; op=" + to_string(t.op) +
               " runs in fp32";
      return "";
  }
}

const char* to_string(Family f) {
  switch (f) {
    case Family::None: return "none";
    case Family::Rows: return "rows";
    case Family::RowsStream: return "rows_stream";
    case Family::ChannelScale: return "channelscale";
    case Family::Reduce1D: return "reduce1d";
    case Family::GemmF16: return "gemm_f16_mfma";
    case Family::GemmGeneric: return "gemm_generic_mfma";
    case Family::ConvIgemm: return "conv_igemm_mfma";
    case Family::Q8Gemm: return "q8_0_gemm";
    case Family::ConvDirect: return "conv_direct";
  }
  return "?";
}

}  // namespace uk

namespace uk {

// Inverse of op_signature: "op:dtype:d0xd1x...[:layout][:nB:pP:sS][:cs][:epsE]". Used by
// calibration to recover a ledger row's workload (reference src/solver.cpp:194-225 parses the
// same way). Returns nullopt for a malformed signature.
std::optional<KmlTree> tree_from_signature(const std::string& sig) {
  std::vector<std::string> parts;
  size_t p = 0;
  while (true) {
    const size_t c = sig.find(':', p);
    parts.push_back(sig.substr(p, c == std::string::npos ? std::string::npos : c - p));
    if (c == std::string::npos) break;
    p = c + 1;
  }
  if (parts.size() < 3) return std::nullopt;
  const auto op = op_from_string(parts[0]);
  const auto dt = dtype_from_string(parts[1]);
  if (!op || !dt) return std::nullopt;
  KmlTree t;
  t.op = *op;
  t.dtype = *dt;
  t.ndims = 0;
  try {
    size_t q = 0;
    while (t.ndims < 6) {
      const size_t x = parts[2].find('x', q);
      size_t used = 0;
      const std::string tok = parts[2].substr(q, x == std::string::npos ? std::string::npos : x - q);
      const long v = std::stol(tok, &used);
      if (used != tok.size() || v <= 0 || v > INT32_MAX) return std::nullopt;
      t.dims[t.ndims++] = int(v);
      if (x == std::string::npos) break;
      q = x + 1;
    }
    for (size_t i = 3; i < parts.size(); ++i) {
      const std::string& s = parts[i];
      if (const auto l = layout_from_string(s)) t.layout = *l;
      else if (s == "cs") t.epilogue = Epilogue::ChannelScale;
      else if (s.size() > 1 && s[0] == 'n') t.batch = std::stoi(s.substr(1));
      else if (s.size() > 1 && s[0] == 'p') t.pad = std::stoi(s.substr(1));
      else if (s.size() > 1 && s[0] == 's') t.stride = std::stoi(s.substr(1));
      else if (s.rfind("eps", 0) == 0) {
        t.eps = std::stof(s.substr(3));
        t.has_eps = true;
      } else {
        return std::nullopt;
      }
    }
  } catch (...) {
    return std::nullopt;
  }
  if (t.ndims < kml_arity_min(t.op) || t.ndims > kml_arity_max(t.op)) return std::nullopt;
  return t;
}

}  // namespace uk
