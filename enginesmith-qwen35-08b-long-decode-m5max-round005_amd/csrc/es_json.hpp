// Minimal JSON value and parser (objects, arrays, strings with escapes,
// numbers, literals), shared by the protocol server and the checkpoint loader.
#pragma once
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

namespace es {

struct Json {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  double num = 0;
  bool is_int = false;
  long long i = 0;
  bool neg = false;
  std::string s;            // string value, or raw text of a number
  std::vector<Json> arr;
  std::map<std::string, Json> obj;
  const Json* get(const std::string& k) const {
    auto it = obj.find(k);
    return it == obj.end() ? nullptr : &it->second;
  }
};

struct Parser {
  const char* p;
  const char* e;
  std::string err;
  void ws() {
    while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool fail(const char* m) {
    if (err.empty()) err = m;
    return false;
  }
  bool lit(const char* w) {
    size_t n = std::strlen(w);
    if ((size_t)(e - p) < n || std::strncmp(p, w, n) != 0) return fail("invalid literal");
    p += n;
    return true;
  }
  bool str(std::string& out) {
    if (p >= e || *p != '"') return fail("expected string");
    ++p;
    while (p < e && *p != '"') {
      if (*p == '\\') {
        ++p;
        if (p >= e) return fail("bad escape");
        char c = *p++;
        switch (c) {
          case '"': out += '"'; break;
          case '\\': out += '\\'; break;
          case '/': out += '/'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'n': out += '\n'; break;
          case 'r': out += '\r'; break;
          case 't': out += '\t'; break;
          case 'u': {
            if (e - p < 4) return fail("bad unicode escape");
            unsigned v = (unsigned)std::strtoul(std::string(p, p + 4).c_str(), nullptr, 16);
            p += 4;
            if (v < 0x80) out += (char)v;
            else if (v < 0x800) { out += (char)(0xC0 | (v >> 6)); out += (char)(0x80 | (v & 0x3F)); }
            else { out += (char)(0xE0 | (v >> 12)); out += (char)(0x80 | ((v >> 6) & 0x3F)); out += (char)(0x80 | (v & 0x3F)); }
            break;
          }
          default: return fail("bad escape");
        }
      } else {
        out += *p++;
      }
    }
    if (p >= e) return fail("unterminated string");
    ++p;
    return true;
  }
  bool number(Json& v) {
    const char* st = p;
    if (p < e && *p == '-') ++p;
    bool frac = false;
    while (p < e && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '+' || *p == '-')) {
      if (*p == '.' || *p == 'e' || *p == 'E') frac = true;
      ++p;
    }
    if (p == st) return fail("expected value");
    v.kind = Json::Num;
    v.s.assign(st, p);
    v.num = std::strtod(v.s.c_str(), nullptr);
    v.neg = v.s[0] == '-';
    v.is_int = !frac;
    if (v.is_int) v.i = std::strtoll(v.s.c_str(), nullptr, 10);
    return true;
  }
  bool value(Json& v, int depth) {
    if (depth > 64) return fail("nesting too deep");
    ws();
    if (p >= e) return fail("unexpected end");
    char c = *p;
    if (c == '{') {
      ++p;
      v.kind = Json::Obj;
      ws();
      if (p < e && *p == '}') { ++p; return true; }
      while (true) {
        ws();
        std::string k;
        if (!str(k)) return false;
        ws();
        if (p >= e || *p != ':') return fail("expected ':'");
        ++p;
        Json child;
        if (!value(child, depth + 1)) return false;
        v.obj[k] = std::move(child);
        ws();
        if (p < e && *p == ',') { ++p; continue; }
        if (p < e && *p == '}') { ++p; return true; }
        return fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      ++p;
      v.kind = Json::Arr;
      ws();
      if (p < e && *p == ']') { ++p; return true; }
      while (true) {
        Json child;
        if (!value(child, depth + 1)) return false;
        v.arr.push_back(std::move(child));
        ws();
        if (p < e && *p == ',') { ++p; continue; }
        if (p < e && *p == ']') { ++p; return true; }
        return fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind = Json::Str;
      return str(v.s);
    }
    if (c == 't') { v.kind = Json::Bool; v.b = true; return lit("true"); }
    if (c == 'f') { v.kind = Json::Bool; v.b = false; return lit("false"); }
    if (c == 'n') { v.kind = Json::Null; return lit("null"); }
    return number(v);
  }
};

inline bool parse_json(const std::string& text, Json& out, std::string& err) {
  Parser ps{text.data(), text.data() + text.size(), {}};
  if (!ps.value(out, 0)) {
    err = ps.err;
    return false;
  }
  ps.ws();
  if (ps.p != ps.e) {
    err = "trailing characters";
    return false;
  }
  return true;
}

}  // namespace es
