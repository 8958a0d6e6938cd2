#include "json.h"

#include <cctype>
#include <cerrno>
#include <cstdio>
#include <cstdlib>

namespace yalm {

const Json* Json::find(const std::string& key) const {
  if (kind != Kind::Object) return nullptr;
  for (const auto& kv : obj)
    if (kv.first == key) return &kv.second;
  return nullptr;
}

namespace {

struct Parser {
  const std::string& s;
  size_t i = 0;
  std::string err;
  int depth = 0;

  explicit Parser(const std::string& t) : s(t) {}

  void ws() {
    while (i < s.size() && (s[i] == ' ' || s[i] == '\t' || s[i] == '\n' || s[i] == '\r')) ++i;
  }
  bool fail(const char* m) {
    if (err.empty()) err = std::string(m) + " at offset " + std::to_string(i);
    return false;
  }
  bool lit(const char* w) {
    size_t n = 0;
    while (w[n]) ++n;
    if (s.compare(i, n, w) != 0) return fail("bad literal");
    i += n;
    return true;
  }
  static void put_utf8(std::string& o, uint32_t cp) {
    if (cp < 0x80) {
      o += (char)cp;
    } else if (cp < 0x800) {
      o += (char)(0xC0 | (cp >> 6));
      o += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      o += (char)(0xE0 | (cp >> 12));
      o += (char)(0x80 | ((cp >> 6) & 0x3F));
      o += (char)(0x80 | (cp & 0x3F));
    } else {
      o += (char)(0xF0 | (cp >> 18));
      o += (char)(0x80 | ((cp >> 12) & 0x3F));
      o += (char)(0x80 | ((cp >> 6) & 0x3F));
      o += (char)(0x80 | (cp & 0x3F));
    }
  }
  bool hex4(uint32_t& v) {
    if (i + 4 > s.size()) return fail("short \\u escape");
    v = 0;
    for (int k = 0; k < 4; ++k) {
      char c = s[i++];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= c - '0';
      else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
      else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
      else return fail("bad hex digit");
    }
    return true;
  }
  bool string(std::string& o) {
    if (i >= s.size() || s[i] != '"') return fail("expected string");
    ++i;
    while (true) {
      if (i >= s.size()) return fail("unterminated string");
      char c = s[i++];
      if (c == '"') return true;
      if ((unsigned char)c < 0x20) return fail("control character in string");
      if (c != '\\') {
        o += c;
        continue;
      }
      if (i >= s.size()) return fail("bad escape");
      char e = s[i++];
      switch (e) {
        case '"': o += '"'; break;
        case '\\': o += '\\'; break;
        case '/': o += '/'; break;
        case 'b': o += '\b'; break;
        case 'f': o += '\f'; break;
        case 'n': o += '\n'; break;
        case 'r': o += '\r'; break;
        case 't': o += '\t'; break;
        case 'u': {
          uint32_t cp = 0;
          if (!hex4(cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
            uint32_t lo = 0;
            if (i + 2 > s.size() || s[i] != '\\' || s[i + 1] != 'u') return fail("lone surrogate");
            i += 2;
            if (!hex4(lo) || lo < 0xDC00 || lo > 0xDFFF) return fail("bad surrogate");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          put_utf8(o, cp);
          break;
        }
        default: return fail("bad escape");
      }
    }
  }
  bool number(Json& v) {
    size_t st = i;
    if (i < s.size() && s[i] == '-') ++i;
    if (i >= s.size() || !isdigit((unsigned char)s[i])) return fail("bad number");
    while (i < s.size() && isdigit((unsigned char)s[i])) ++i;
    bool integer = true;
    if (i < s.size() && s[i] == '.') {
      integer = false;
      ++i;
      if (i >= s.size() || !isdigit((unsigned char)s[i])) return fail("bad fraction");
      while (i < s.size() && isdigit((unsigned char)s[i])) ++i;
    }
    if (i < s.size() && (s[i] == 'e' || s[i] == 'E')) {
      integer = false;
      ++i;
      if (i < s.size() && (s[i] == '+' || s[i] == '-')) ++i;
      if (i >= s.size() || !isdigit((unsigned char)s[i])) return fail("bad exponent");
      while (i < s.size() && isdigit((unsigned char)s[i])) ++i;
    }
    std::string lit_s = s.substr(st, i - st);
    v.kind = Json::Kind::Number;
    v.num = strtod(lit_s.c_str(), nullptr);
    v.is_integer = integer;
    if (integer) {
      errno = 0;
      long long x = strtoll(lit_s.c_str(), nullptr, 10);
      if (errno == ERANGE) return fail("integer out of range");
      v.i64 = x;
    }
    return true;
  }
  bool value(Json& v) {
    if (++depth > 64) return fail("nesting too deep");
    ws();
    if (i >= s.size()) return fail("unexpected end");
    char c = s[i];
    bool ok;
    if (c == '{') {
      v.kind = Json::Kind::Object;
      ++i;
      ws();
      if (i < s.size() && s[i] == '}') {
        ++i;
        ok = true;
      } else {
        ok = true;
        while (true) {
          ws();
          std::string k;
          if (!string(k)) { ok = false; break; }
          ws();
          if (i >= s.size() || s[i] != ':') { ok = fail("expected ':'"); break; }
          ++i;
          Json child;
          if (!value(child)) { ok = false; break; }
          v.obj.emplace_back(std::move(k), std::move(child));
          ws();
          if (i < s.size() && s[i] == ',') { ++i; continue; }
          if (i < s.size() && s[i] == '}') { ++i; break; }
          ok = fail("expected ',' or '}'");
          break;
        }
      }
    } else if (c == '[') {
      v.kind = Json::Kind::Array;
      ++i;
      ws();
      if (i < s.size() && s[i] == ']') {
        ++i;
        ok = true;
      } else {
        ok = true;
        while (true) {
          Json child;
          if (!value(child)) { ok = false; break; }
          v.arr.push_back(std::move(child));
          ws();
          if (i < s.size() && s[i] == ',') { ++i; continue; }
          if (i < s.size() && s[i] == ']') { ++i; break; }
          ok = fail("expected ',' or ']'");
          break;
        }
      }
    } else if (c == '"') {
      v.kind = Json::Kind::String;
      ok = string(v.str);
    } else if (c == 't') {
      v.kind = Json::Kind::Bool;
      v.b = true;
      ok = lit("true");
    } else if (c == 'f') {
      v.kind = Json::Kind::Bool;
      ok = lit("false");
    } else if (c == 'n') {
      ok = lit("null");
    } else {
      ok = number(v);
    }
    --depth;
    return ok;
  }
};

}  // namespace

bool json_parse(const std::string& text, Json& out, std::string& err) {
  Parser p(text);
  out = Json();
  if (!p.value(out)) {
    err = p.err;
    return false;
  }
  p.ws();
  if (p.i != text.size()) {
    err = "trailing characters after JSON value at offset " + std::to_string(p.i);
    return false;
  }
  return true;
}

std::string json_quote(const std::string& s) {
  std::string o = "\"";
  for (unsigned char c : s) {
    switch (c) {
      case '"': o += "\\\""; break;
      case '\\': o += "\\\\"; break;
      case '\n': o += "\\n"; break;
      case '\r': o += "\\r"; break;
      case '\t': o += "\\t"; break;
      default:
        if (c < 0x20) {
          char buf[8];
          snprintf(buf, sizeof(buf), "\\u%04x", c);
          o += buf;
        } else {
          o += (char)c;
        }
    }
  }
  return o + "\"";
}

}  // namespace yalm
