// JSON reader (see json.h): recursive descent over RFC 8259's grammar.
#include "json.h"

#include <cerrno>
#include <cstdio>
#include <cstdlib>

namespace llrs {

const JsonValue *JsonValue::get(const std::string &key) const {
  if (kind != OBJECT) return nullptr;
  const JsonValue *found = nullptr;
  for (const auto &m : members)
    if (m.first == key) found = &m.second;
  return found;
}

bool JsonValue::as_u64(uint64_t &out) const {
  if (kind != NUMBER || text.empty() || text[0] == '-') return false;
  uint64_t v = 0;
  for (char c : text) {
    if (c < '0' || c > '9') return false;  // a fraction or an exponent
    const uint64_t d = (uint64_t)(c - '0');
    if (v > (UINT64_MAX - d) / 10) return false;
    v = v * 10 + d;
  }
  out = v;
  return true;
}

bool JsonValue::as_f64(double &out) const {
  if (kind != NUMBER) return false;
  errno = 0;
  out = strtod(text.c_str(), nullptr);  // the lexeme already matched JSON's grammar
  return true;
}

namespace {

constexpr int kMaxDepth = 128;

struct Parser {
  const char *p, *end, *begin;
  std::string err;

  bool fail(const char *what) {
    if (err.empty()) {
      char buf[96];
      snprintf(buf, sizeof buf, "%s at byte %zu", what, (size_t)(p - begin));
      err = buf;
    }
    return false;
  }
  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
  }
  bool lit(const char *s, size_t n) {
    if ((size_t)(end - p) < n) return false;
    for (size_t i = 0; i < n; i++)
      if (p[i] != s[i]) return false;
    p += n;
    return true;
  }
  static void put_utf8(std::string &o, uint32_t c) {
    if (c < 0x80) {
      o += (char)c;
    } else if (c < 0x800) {
      o += (char)(0xc0 | (c >> 6));
      o += (char)(0x80 | (c & 0x3f));
    } else if (c < 0x10000) {
      o += (char)(0xe0 | (c >> 12));
      o += (char)(0x80 | ((c >> 6) & 0x3f));
      o += (char)(0x80 | (c & 0x3f));
    } else {
      o += (char)(0xf0 | (c >> 18));
      o += (char)(0x80 | ((c >> 12) & 0x3f));
      o += (char)(0x80 | ((c >> 6) & 0x3f));
      o += (char)(0x80 | (c & 0x3f));
    }
  }
  bool hex4(uint32_t &v) {
    if (end - p < 4) return fail("truncated \\u escape");
    v = 0;
    for (int i = 0; i < 4; i++, p++) {
      const char c = *p;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
      else return fail("invalid \\u escape");
    }
    return true;
  }
  bool string(std::string &o) {
    p++;  // the opening quote
    o.clear();
    while (true) {
      if (p >= end) return fail("unterminated string");
      const unsigned char c = (unsigned char)*p;
      if (c == '"') {
        p++;
        return true;
      }
      if (c < 0x20) return fail("control character in string");
      if (c != '\\') {
        o += (char)c;
        p++;
        continue;
      }
      if (++p >= end) return fail("unterminated escape");
      const char e = *p++;
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
          uint32_t u;
          if (!hex4(u)) return false;
          if (u >= 0xdc00 && u < 0xe000) return fail("unpaired low surrogate");
          if (u >= 0xd800 && u < 0xdc00) {
            uint32_t lo;
            if (!lit("\\u", 2) || !hex4(lo) || lo < 0xdc00 || lo >= 0xe000)
              return fail("unpaired high surrogate");
            u = 0x10000 + ((u - 0xd800) << 10) + (lo - 0xdc00);
          }
          put_utf8(o, u);
          break;
        }
        default: return fail("invalid escape");
      }
    }
  }
  bool number(JsonValue &v) {
    const char *s = p;
    if (p < end && *p == '-') p++;
    if (p >= end) return fail("invalid number");
    if (*p == '0') {
      p++;
    } else if (*p >= '1' && *p <= '9') {
      while (p < end && *p >= '0' && *p <= '9') p++;
    } else {
      return fail("invalid number");
    }
    if (p < end && *p == '.') {
      p++;
      if (p >= end || *p < '0' || *p > '9') return fail("invalid number");
      while (p < end && *p >= '0' && *p <= '9') p++;
    }
    if (p < end && (*p == 'e' || *p == 'E')) {
      p++;
      if (p < end && (*p == '+' || *p == '-')) p++;
      if (p >= end || *p < '0' || *p > '9') return fail("invalid number");
      while (p < end && *p >= '0' && *p <= '9') p++;
    }
    v.kind = JsonValue::NUMBER;
    v.text.assign(s, p);
    return true;
  }
  bool value(JsonValue &v, int depth) {
    if (depth > kMaxDepth) return fail("nesting too deep");
    ws();
    if (p >= end) return fail("unexpected end of input");
    switch (*p) {
      case '{': {
        p++;
        v.kind = JsonValue::OBJECT;
        ws();
        if (p < end && *p == '}') {
          p++;
          return true;
        }
        while (true) {
          ws();
          if (p >= end || *p != '"') return fail("expected a string key");
          std::string key;
          if (!string(key)) return false;
          ws();
          if (p >= end || *p != ':') return fail("expected ':'");
          p++;
          v.members.emplace_back(std::move(key), JsonValue());
          if (!value(v.members.back().second, depth + 1)) return false;
          ws();
          if (p < end && *p == ',') {
            p++;
            continue;
          }
          if (p < end && *p == '}') {
            p++;
            return true;
          }
          return fail("expected ',' or '}'");
        }
      }
      case '[': {
        p++;
        v.kind = JsonValue::ARRAY;
        ws();
        if (p < end && *p == ']') {
          p++;
          return true;
        }
        while (true) {
          v.items.emplace_back();
          if (!value(v.items.back(), depth + 1)) return false;
          ws();
          if (p < end && *p == ',') {
            p++;
            continue;
          }
          if (p < end && *p == ']') {
            p++;
            return true;
          }
          return fail("expected ',' or ']'");
        }
      }
      case '"':
        v.kind = JsonValue::STRING;
        return string(v.text);
      case 't':
        if (!lit("true", 4)) return fail("invalid literal");
        v.kind = JsonValue::BOOL;
        v.b = true;
        return true;
      case 'f':
        if (!lit("false", 5)) return fail("invalid literal");
        v.kind = JsonValue::BOOL;
        v.b = false;
        return true;
      case 'n':
        if (!lit("null", 4)) return fail("invalid literal");
        v.kind = JsonValue::NUL;
        return true;
      default:
        return number(v);
    }
  }
};

}  // namespace

bool json_parse(const char *data, size_t n, JsonValue &out, std::string &error) {
  Parser ps{data, data + n, data, {}};
  out = JsonValue();
  if (!ps.value(out, 0)) {
    error = ps.err;
    return false;
  }
  ps.ws();
  if (ps.p != ps.end) {
    ps.fail("trailing characters");
    error = ps.err;
    return false;
  }
  return true;
}

}  // namespace llrs
