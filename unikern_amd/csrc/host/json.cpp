#include "json.hpp"

#include <cctype>
#include <cerrno>
#include <cstdlib>

namespace uk::json {

const Value* Value::get(const std::string& key) const {
  if (kind != Kind::Object) return nullptr;
  for (const auto& kv : obj)
    if (kv.first == key) return &kv.second;
  return nullptr;
}

std::string Value::scalar_text() const {
  switch (kind) {
    case Kind::String:
    case Kind::Number: return text;
    case Kind::Bool: return b ? "true" : "false";
    case Kind::Null: return "null";
    case Kind::Array: return "[...]";
    case Kind::Object: return "{...}";
  }
  return "";
}

namespace {

struct Parser {
  const std::string& s;
  size_t p = 0;
  std::string err;

  explicit Parser(const std::string& src) : s(src) {}

  void ws() {
    while (p < s.size() && (s[p] == ' ' || s[p] == '\t' || s[p] == '\n' || s[p] == '\r')) ++p;
  }
  bool fail(const std::string& m) {
    if (err.empty()) err = m + " at offset " + std::to_string(p);
    return false;
  }
  bool lit(const char* w) {
    size_t n = 0;
    while (w[n]) ++n;
    if (s.compare(p, n, w) != 0) return false;
    p += n;
    return true;
  }
  static void put_utf8(std::string* out, unsigned cp) {
    if (cp < 0x80) {
      out->push_back(char(cp));
    } else if (cp < 0x800) {
      out->push_back(char(0xC0 | (cp >> 6)));
      out->push_back(char(0x80 | (cp & 0x3F)));
    } else if (cp < 0x10000) {
      out->push_back(char(0xE0 | (cp >> 12)));
      out->push_back(char(0x80 | ((cp >> 6) & 0x3F)));
      out->push_back(char(0x80 | (cp & 0x3F)));
    } else {
      out->push_back(char(0xF0 | (cp >> 18)));
      out->push_back(char(0x80 | ((cp >> 12) & 0x3F)));
      out->push_back(char(0x80 | ((cp >> 6) & 0x3F)));
      out->push_back(char(0x80 | (cp & 0x3F)));
    }
  }
  bool hex4(unsigned* cp) {
    if (p + 4 > s.size()) return fail("truncated \\u escape");
    unsigned v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = s[p++];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= unsigned(c - '0');
      else if (c >= 'a' && c <= 'f') v |= unsigned(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= unsigned(c - 'A' + 10);
      else return fail("bad \\u escape");
    }
    *cp = v;
    return true;
  }
  bool str(std::string* out) {
    if (p >= s.size() || s[p] != '"') return fail("expected string");
    ++p;
    while (p < s.size()) {
      const char c = s[p++];
      if (c == '"') return true;
      if (c == '\\') {
        if (p >= s.size()) return fail("truncated escape");
        const char e = s[p++];
        switch (e) {
          case '"': out->push_back('"'); break;
          case '\\': out->push_back('\\'); break;
          case '/': out->push_back('/'); break;
          case 'b': out->push_back('\b'); break;
          case 'f': out->push_back('\f'); break;
          case 'n': out->push_back('\n'); break;
          case 'r': out->push_back('\r'); break;
          case 't': out->push_back('\t'); break;
          case 'u': {
            unsigned cp = 0;
            if (!hex4(&cp)) return false;
            if (cp >= 0xD800 && cp < 0xDC00 && p + 1 < s.size() && s[p] == '\\' && s[p + 1] == 'u') {
              p += 2;
              unsigned lo = 0;
              if (!hex4(&lo)) return false;
              cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
            }
            put_utf8(out, cp);
            break;
          }
          default: return fail("bad escape");
        }
      } else {
        out->push_back(c);
      }
    }
    return fail("unterminated string");
  }
  bool number(Value* v) {
    const size_t a = p;
    if (p < s.size() && s[p] == '-') ++p;
    if (p >= s.size() || !std::isdigit(static_cast<unsigned char>(s[p]))) return fail("bad number");
    while (p < s.size() && std::isdigit(static_cast<unsigned char>(s[p]))) ++p;
    if (p < s.size() && s[p] == '.') {
      ++p;
      if (p >= s.size() || !std::isdigit(static_cast<unsigned char>(s[p]))) return fail("bad number");
      while (p < s.size() && std::isdigit(static_cast<unsigned char>(s[p]))) ++p;
    }
    if (p < s.size() && (s[p] == 'e' || s[p] == 'E')) {
      ++p;
      if (p < s.size() && (s[p] == '+' || s[p] == '-')) ++p;
      if (p >= s.size() || !std::isdigit(static_cast<unsigned char>(s[p]))) return fail("bad number");
      while (p < s.size() && std::isdigit(static_cast<unsigned char>(s[p]))) ++p;
    }
    v->kind = Value::Kind::Number;
    v->text = s.substr(a, p - a);
    v->num = std::strtod(v->text.c_str(), nullptr);
    return true;
  }
  bool value(Value* v, int depth) {
    if (depth > 64) return fail("nesting too deep");
    ws();
    if (p >= s.size()) return fail("unexpected end");
    const char c = s[p];
    if (c == '{') {
      ++p;
      v->kind = Value::Kind::Object;
      ws();
      if (p < s.size() && s[p] == '}') { ++p; return true; }
      for (;;) {
        ws();
        std::string k;
        if (!str(&k)) return false;
        ws();
        if (p >= s.size() || s[p] != ':') return fail("expected ':'");
        ++p;
        Value child;
        if (!value(&child, depth + 1)) return false;
        v->obj.emplace_back(std::move(k), std::move(child));
        ws();
        if (p < s.size() && s[p] == ',') { ++p; continue; }
        if (p < s.size() && s[p] == '}') { ++p; return true; }
        return fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      ++p;
      v->kind = Value::Kind::Array;
      ws();
      if (p < s.size() && s[p] == ']') { ++p; return true; }
      for (;;) {
        Value child;
        if (!value(&child, depth + 1)) return false;
        v->arr.push_back(std::move(child));
        ws();
        if (p < s.size() && s[p] == ',') { ++p; continue; }
        if (p < s.size() && s[p] == ']') { ++p; return true; }
        return fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v->kind = Value::Kind::String;
      return str(&v->text);
    }
    if (lit("true")) { v->kind = Value::Kind::Bool; v->b = true; return true; }
    if (lit("false")) { v->kind = Value::Kind::Bool; v->b = false; return true; }
    if (lit("null")) { v->kind = Value::Kind::Null; return true; }
    return number(v);
  }
};

}  // namespace

std::optional<Value> parse(const std::string& text, std::string* err) {
  Parser ps(text);
  Value v;
  if (!ps.value(&v, 0)) {
    if (err) *err = "invalid JSON: " + ps.err;
    return std::nullopt;
  }
  ps.ws();
  if (ps.p != text.size()) {
    if (err) *err = "invalid JSON: trailing characters at offset " + std::to_string(ps.p);
    return std::nullopt;
  }
  return v;
}

bool as_int64(const Value& v, long long* out) {
  if (v.kind != Value::Kind::Number) return false;
  const std::string& t = v.text;
  size_t i = (!t.empty() && t[0] == '-') ? 1 : 0;
  if (i >= t.size()) return false;
  for (; i < t.size(); ++i)
    if (!std::isdigit(static_cast<unsigned char>(t[i]))) return false;
  errno = 0;
  char* end = nullptr;
  const long long x = std::strtoll(t.c_str(), &end, 10);
  if (errno == ERANGE || end == t.c_str()) return false;
  *out = x;
  return true;
}

}  // namespace uk::json
