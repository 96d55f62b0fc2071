// A small strict JSON reader for KML op specs and HCS hardware descriptions.
//
// The reference reads both formats with a flat text scanner (src/json_flat.cpp); this reader
// builds a value tree instead, so nested CDNA4 fields (the MFMA shape table) and children are
// read structurally. Numbers keep their source text, so integer fields can be validated the
// way the reference does (digits only, range-checked; src/kml_front.cpp:29-46).
#pragma once
#include <optional>
#include <string>
#include <utility>
#include <vector>

namespace uk::json {

struct Value {
  enum class Kind { Null, Bool, Number, String, Array, Object };
  Kind kind = Kind::Null;
  bool b = false;
  double num = 0;
  std::string text;  // number source text, or string contents
  std::vector<Value> arr;
  std::vector<std::pair<std::string, Value>> obj;

  const Value* get(const std::string& key) const;
  bool is_string() const { return kind == Kind::String; }
  bool is_number() const { return kind == Kind::Number; }
  // Scalar rendered as text (string contents, number text, true/false/null).
  std::string scalar_text() const;
};

std::optional<Value> parse(const std::string& text, std::string* err);

// Integer with the reference's rules: optional '-', then digits only.
bool as_int64(const Value& v, long long* out);

}  // namespace uk::json
