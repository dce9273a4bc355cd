#include "json.hpp"

#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>

#include "common.hpp"

namespace tsa {
namespace {

constexpr int kMaxDepth = 64;

struct Parser {
  const std::string& s;
  size_t i = 0;

  [[noreturn]] void bad(const std::string& what) const {
    fail(SS_E_DESC, "json: " + what + " at offset " + std::to_string(i));
  }
  void ws() {
    while (i < s.size() && (s[i] == ' ' || s[i] == '\t' || s[i] == '\n' || s[i] == '\r')) ++i;
  }
  bool eat(char c) {
    ws();
    if (i < s.size() && s[i] == c) {
      ++i;
      return true;
    }
    return false;
  }
  void expect(char c) {
    if (!eat(c)) bad(std::string("expected '") + c + "'");
  }
  static void put_utf8(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
      out += char(cp);
    } else if (cp < 0x800) {
      out += char(0xC0 | (cp >> 6));
      out += char(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      out += char(0xE0 | (cp >> 12));
      out += char(0x80 | ((cp >> 6) & 0x3F));
      out += char(0x80 | (cp & 0x3F));
    } else {
      out += char(0xF0 | (cp >> 18));
      out += char(0x80 | ((cp >> 12) & 0x3F));
      out += char(0x80 | ((cp >> 6) & 0x3F));
      out += char(0x80 | (cp & 0x3F));
    }
  }
  uint32_t hex4() {
    if (i + 4 > s.size()) bad("short \\u escape");
    uint32_t v = 0;
    for (int k = 0; k < 4; ++k) {
      const char c = s[i++];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= uint32_t(c - '0');
      else if (c >= 'a' && c <= 'f') v |= uint32_t(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= uint32_t(c - 'A' + 10);
      else bad("bad \\u escape");
    }
    return v;
  }
  std::string str() {
    ws();
    if (i >= s.size() || s[i] != '"') bad("expected a string");
    ++i;
    std::string out;
    while (true) {
      if (i >= s.size()) bad("unterminated string");
      const char c = s[i++];
      if (c == '"') break;
      if (static_cast<unsigned char>(c) < 0x20) bad("control character in a string");
      if (c != '\\') {
        out += c;
        continue;
      }
      if (i >= s.size()) bad("unterminated escape");
      const char e = s[i++];
      switch (e) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          uint32_t cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00) {
            if (i + 2 > s.size() || s[i] != '\\' || s[i + 1] != 'u') bad("lone surrogate");
            i += 2;
            const uint32_t lo = hex4();
            if (lo < 0xDC00 || lo >= 0xE000) bad("bad surrogate pair");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          put_utf8(out, cp);
          break;
        }
        default: bad("bad escape");
      }
    }
    return out;
  }
  Json value(int depth) {
    if (depth > kMaxDepth) bad("nesting too deep");
    ws();
    if (i >= s.size()) bad("unexpected end");
    const char c = s[i];
    if (c == '{') {
      ++i;
      Json o = Json::object();
      if (eat('}')) return o;
      do {
        std::string k = str();
        expect(':');
        if (o.obj.count(k)) bad("duplicate key \"" + k + "\"");
        o.obj.emplace(std::move(k), value(depth + 1));
      } while (eat(','));
      expect('}');
      return o;
    }
    if (c == '[') {
      ++i;
      Json a = Json::array();
      if (eat(']')) return a;
      do a.arr.push_back(value(depth + 1));
      while (eat(','));
      expect(']');
      return a;
    }
    if (c == '"') return Json::string(str());
    if (s.compare(i, 4, "true") == 0) {
      i += 4;
      return Json::boolean(true);
    }
    if (s.compare(i, 5, "false") == 0) {
      i += 5;
      return Json::boolean(false);
    }
    if (s.compare(i, 4, "null") == 0) {
      i += 4;
      return Json{};
    }
    // number: -?(0|[1-9][0-9]*)(\.[0-9]+)?([eE][+-]?[0-9]+)?
    const size_t start = i;
    if (s[i] == '-') ++i;
    if (i >= s.size() || !isdigit(static_cast<unsigned char>(s[i]))) bad("bad value");
    if (s[i] == '0') ++i;
    else
      while (i < s.size() && isdigit(static_cast<unsigned char>(s[i]))) ++i;
    if (i < s.size() && s[i] == '.') {
      ++i;
      if (i >= s.size() || !isdigit(static_cast<unsigned char>(s[i]))) bad("bad number");
      while (i < s.size() && isdigit(static_cast<unsigned char>(s[i]))) ++i;
    }
    if (i < s.size() && (s[i] == 'e' || s[i] == 'E')) {
      ++i;
      if (i < s.size() && (s[i] == '+' || s[i] == '-')) ++i;
      if (i >= s.size() || !isdigit(static_cast<unsigned char>(s[i]))) bad("bad exponent");
      while (i < s.size() && isdigit(static_cast<unsigned char>(s[i]))) ++i;
    }
    Json n;
    n.kind = Json::Number;
    n.text = s.substr(start, i - start);
    return n;
  }
};

void dump_string(std::string& out, const std::string& v) {
  out += '"';
  for (unsigned char c : v) {
    switch (c) {
      case '"': out += "\\\""; break;
      case '\\': out += "\\\\"; break;
      case '\n': out += "\\n"; break;
      case '\r': out += "\\r"; break;
      case '\t': out += "\\t"; break;
      case '\b': out += "\\b"; break;
      case '\f': out += "\\f"; break;
      default:
        if (c < 0x20) {
          char buf[8];
          std::snprintf(buf, sizeof buf, "\\u%04x", c);
          out += buf;
        } else {
          out += char(c);
        }
    }
  }
  out += '"';
}

void dump(std::string& out, const Json& j) {
  switch (j.kind) {
    case Json::Null: out += "null"; break;
    case Json::Bool: out += j.b ? "true" : "false"; break;
    case Json::Number: out += j.text; break;
    case Json::String: dump_string(out, j.text); break;
    case Json::Array: {
      out += '[';
      for (size_t k = 0; k < j.arr.size(); ++k) {
        if (k) out += ',';
        dump(out, j.arr[k]);
      }
      out += ']';
      break;
    }
    case Json::Object: {
      out += '{';
      bool first = true;
      for (const auto& kv : j.obj) {
        if (!first) out += ',';
        first = false;
        dump_string(out, kv.first);
        out += ':';
        dump(out, kv.second);
      }
      out += '}';
      break;
    }
  }
}

bool is_integer_literal(const std::string& t) {
  size_t i = t[0] == '-' ? 1 : 0;
  if (i >= t.size()) return false;
  for (; i < t.size(); ++i)
    if (!isdigit(static_cast<unsigned char>(t[i]))) return false;
  return true;
}

}  // namespace

Json Json::number_f(double v) {
  Json j;
  j.kind = Number;
  char buf[40];
  std::snprintf(buf, sizeof buf, "%.17g", v);
  j.text = buf;
  return j;
}

Json json_parse(const std::string& text) {
  Parser p{text};
  Json v = p.value(0);
  p.ws();
  if (p.i != text.size()) p.bad("trailing characters");
  return v;
}

std::string json_dump(const Json& j) {
  std::string out;
  dump(out, j);
  return out;
}

uint64_t json_u64(const Json& j, const std::string& where) {
  require(j.kind == Json::Number && is_integer_literal(j.text) && j.text[0] != '-', SS_E_DESC,
          where + ": expected a non-negative integer");
  errno = 0;
  char* end = nullptr;
  const unsigned long long v = std::strtoull(j.text.c_str(), &end, 10);
  require(errno == 0 && end && *end == '\0', SS_E_DESC, where + ": integer out of range");
  return uint64_t(v);
}

int64_t json_i64(const Json& j, const std::string& where) {
  require(j.kind == Json::Number && is_integer_literal(j.text), SS_E_DESC, where + ": expected an integer");
  errno = 0;
  char* end = nullptr;
  const long long v = std::strtoll(j.text.c_str(), &end, 10);
  require(errno == 0 && end && *end == '\0', SS_E_DESC, where + ": integer out of range");
  return int64_t(v);
}

double json_f64(const Json& j, const std::string& where) {
  require(j.kind == Json::Number, SS_E_DESC, where + ": expected a number");
  const double v = std::strtod(j.text.c_str(), nullptr);
  require(std::isfinite(v), SS_E_DESC, where + ": number out of range");
  return v;
}

const std::string& json_str(const Json& j, const std::string& where) {
  require(j.kind == Json::String, SS_E_DESC, where + ": expected a string");
  return j.text;
}

bool json_bool(const Json& j, const std::string& where) {
  require(j.kind == Json::Bool, SS_E_DESC, where + ": expected true or false");
  return j.b;
}

}  // namespace tsa
