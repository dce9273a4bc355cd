#include "json.hpp"

#include <cmath>
#include <cstdio>
#include <cstdlib>

#include "common.hpp"

namespace tsa {
namespace {

constexpr size_t kNestLimit = 64;                  // containers below the top value
constexpr size_t kTextLimit = size_t(256) << 20;   // bytes of text

bool digit(char c) { return c >= '0' && c <= '9'; }

int hex_value(char c) {
  if (digit(c)) return c - '0';
  if (c >= 'a' && c <= 'f') return c - 'a' + 10;
  if (c >= 'A' && c <= 'F') return c - 'A' + 10;
  return -1;
}

// Appends code point cp (at most 0x10FFFF) as UTF-8: the lead byte carries the length, continuation bytes 6 bits each.
void append_utf8(std::string& out, uint32_t cp) {
  if (cp < 0x80) {
    out.push_back(char(cp));
    return;
  }
  const int n = cp < 0x800 ? 2 : cp < 0x10000 ? 3 : 4;
  static const unsigned char lead[5] = {0, 0, 0xC0, 0xE0, 0xF0};
  char buf[4];
  for (int k = n - 1; k > 0; --k, cp >>= 6) buf[k] = char(0x80 | (cp & 0x3F));
  buf[0] = char(lead[n] | cp);
  out.append(buf, size_t(n));
}

// The text and a read position, and the pieces of the grammar that do not nest.
class Reader {
 public:
  explicit Reader(const std::string& t) : t_(t) {}

  [[noreturn]] void reject(const std::string& why) const {
    fail(SS_E_DESC, "json: " + why + " (byte " + std::to_string(pos_) + ")");
  }
  void space() {
    while (pos_ < t_.size()) {
      const char c = t_[pos_];
      if (c != ' ' && c != '\t' && c != '\n' && c != '\r') return;
      ++pos_;
    }
  }
  bool done() const { return pos_ >= t_.size(); }
  char peek() const { return t_[pos_]; }
  bool skip(char c) {  // after whitespace
    space();
    if (done() || peek() != c) return false;
    ++pos_;
    return true;
  }
  size_t pos() const { return pos_; }

  std::string string_body() {  // at the opening quote
    if (done() || peek() != '"') reject("a string must start here");
    ++pos_;
    std::string out;
    for (;;) {
      if (done()) reject("the string never ends");
      const char c = t_[pos_++];
      if (c == '"') return out;
      if (static_cast<unsigned char>(c) < 0x20) reject("a raw control byte inside a string");
      if (c != '\\') {
        out.push_back(c);
        continue;
      }
      if (done()) reject("the string ends inside an escape");
      const char e = t_[pos_++];
      switch (e) {
        case '"': case '\\': case '/': out.push_back(e); break;
        case 'b': out.push_back('\b'); break;
        case 'f': out.push_back('\f'); break;
        case 'n': out.push_back('\n'); break;
        case 'r': out.push_back('\r'); break;
        case 't': out.push_back('\t'); break;
        case 'u': append_utf8(out, code_point()); break;
        default: reject(std::string("unknown escape \\") + e);
      }
    }
  }

  Json scalar() {  // at a non-container value
    const char c = peek();
    if (c == '"') return Json::string(string_body());
    if (word("true")) return Json::boolean(true);
    if (word("false")) return Json::boolean(false);
    if (word("null")) return Json{};
    return number();
  }

 private:
  uint32_t hex_quad() {
    if (t_.size() - pos_ < 4) reject("a \\u escape needs four hex digits");
    uint32_t v = 0;
    for (int k = 0; k < 4; ++k) {
      const int h = hex_value(t_[pos_++]);
      if (h < 0) reject("a \\u escape needs four hex digits");
      v = v << 4 | uint32_t(h);
    }
    return v;
  }
  // After "\u": one code point; a high surrogate must be followed at once by an escaped low one.
  uint32_t code_point() {
    const uint32_t u = hex_quad();
    if (u >= 0xDC00 && u <= 0xDFFF) reject("a low surrogate with no high one before it");
    if (u < 0xD800 || u > 0xDBFF) return u;
    if (t_.size() - pos_ < 2 || t_[pos_] != '\\' || t_[pos_ + 1] != 'u') reject("a high surrogate with no low one");
    pos_ += 2;
    const uint32_t lo = hex_quad();
    if (lo < 0xDC00 || lo > 0xDFFF) reject("a high surrogate followed by a non-low escape");
    return 0x10000 + ((u - 0xD800) << 10 | (lo - 0xDC00));
  }
  bool word(const char* w) {
    size_t n = 0;
    while (w[n]) ++n;
    if (t_.compare(pos_, n, w) != 0) return false;
    pos_ += n;
    return true;
  }
  void digits() {
    while (!done() && digit(peek())) ++pos_;
  }
  // -?(0|[1-9][0-9]*)(.[0-9]+)?([eE][+-]?[0-9]+)?, kept as text
  Json number() {
    const size_t from = pos_;
    if (peek() == '-') ++pos_;
    if (done() || !digit(peek())) reject("not a value");
    if (peek() == '0') ++pos_;
    else digits();
    if (!done() && peek() == '.') {
      ++pos_;
      if (done() || !digit(peek())) reject("a fraction needs digits");
      digits();
    }
    if (!done() && (peek() == 'e' || peek() == 'E')) {
      ++pos_;
      if (!done() && (peek() == '+' || peek() == '-')) ++pos_;
      if (done() || !digit(peek())) reject("an exponent needs digits");
      digits();
    }
    Json j;
    j.kind = Json::Number;
    j.text = t_.substr(from, pos_ - from);
    return j;
  }

  const std::string& t_;
  size_t pos_ = 0;
};

// The next object key and its colon; *slot becomes the key's (new) value.
Json* open_member(Reader& r, Json& o) {
  r.space();
  if (r.done()) r.reject("the text ends inside an object");
  std::string key = r.string_body();
  if (!r.skip(':')) r.reject("a key needs a ':'");
  if (o.obj.count(key)) r.reject("key \"" + key + "\" appears twice");
  return &o.obj[key];
}

// Iterative: `open` holds the containers being filled (never more than kNestLimit + 1), so deep text cannot exhaust
// the native stack. A pointer to an open container stays valid: its parent is not touched while it is open.
Json parse_text(Reader& r) {
  Json root;
  std::vector<Json*> open;
  Json* slot = &root;  // where the next value goes
  for (;;) {
    if (open.size() > kNestLimit) r.reject("containers nested more than 64 deep");
    r.space();
    if (r.done()) r.reject("the text ends where a value should start");
    const char c = r.peek();
    bool filled = true;
    if (c == '{' || c == '[') {
      r.skip(c);
      *slot = c == '{' ? Json::object() : Json::array();
      open.push_back(slot);
      if (r.skip(c == '{' ? '}' : ']')) {
        open.pop_back();
      } else {
        slot = c == '{' ? open_member(r, *slot) : (slot->arr.emplace_back(), &slot->arr.back());
        filled = false;
      }
    } else {
      *slot = r.scalar();
    }
    // after a complete value: a separator opens the next one, a bracket closes the innermost container
    while (filled && !open.empty()) {
      Json& top = *open.back();
      if (r.skip(',')) {
        slot = top.is_object() ? open_member(r, top) : (top.arr.emplace_back(), &top.arr.back());
        filled = false;
      } else if (r.skip(top.is_object() ? '}' : ']')) {
        open.pop_back();
      } else {
        r.reject(top.is_object() ? "expected ',' or '}'" : "expected ',' or ']'");
      }
    }
    if (filled) return root;
  }
}

void write_string(std::string& out, const std::string& v) {
  static const char hex[] = "0123456789abcdef";
  out.push_back('"');
  for (const char ch : v) {
    const unsigned char c = static_cast<unsigned char>(ch);
    const char* named = c == '"' ? "\\\"" : c == '\\' ? "\\\\" : c == '\n' ? "\\n" : c == '\r' ? "\\r" : c == '\t' ? "\\t" : nullptr;
    if (named) {
      out += named;
    } else if (c < 0x20) {
      out += "\\u00";
      out.push_back(hex[c >> 4]);
      out.push_back(hex[c & 15]);
    } else {
      out.push_back(ch);
    }
  }
  out.push_back('"');
}

void write_value(std::string& out, const Json& j) {
  switch (j.kind) {
    case Json::Null: out += "null"; return;
    case Json::Bool: out += j.b ? "true" : "false"; return;
    case Json::Number: out += j.text; return;
    case Json::String: write_string(out, j.text); return;
    case Json::Array: {
      out.push_back('[');
      const char* sep = "";
      for (const Json& e : j.arr) {
        out += sep;
        write_value(out, e);
        sep = ",";
      }
      out.push_back(']');
      return;
    }
    case Json::Object: {
      out.push_back('{');
      const char* sep = "";
      for (const auto& kv : j.obj) {
        out += sep;
        write_string(out, kv.first);
        out.push_back(':');
        write_value(out, kv.second);
        sep = ",";
      }
      out.push_back('}');
      return;
    }
  }
}

// The magnitude of an all-digit literal of at most 20 digits; false when it is not one or does not fit 64 bits.
bool magnitude(const std::string& t, size_t from, uint64_t* out) {
  if (from >= t.size() || t.size() - from > 20) return false;
  uint64_t v = 0;
  for (size_t i = from; i < t.size(); ++i) {
    if (!digit(t[i])) return false;
    const uint64_t d = uint64_t(t[i] - '0');
    if (v > (UINT64_MAX - d) / 10) return false;
    v = v * 10 + d;
  }
  *out = v;
  return true;
}

}  // namespace

Json Json::number_f(double v) {
  char buf[40];
  std::snprintf(buf, sizeof buf, "%.17g", v);
  Json j = of(Number);
  j.text = buf;
  return j;
}

Json json_parse(const std::string& text) {
  require(text.size() <= kTextLimit, SS_E_DESC, "json: more than 256 MiB of text");
  Reader r(text);
  Json v = parse_text(r);
  r.space();
  if (!r.done()) r.reject("text after the value");
  return v;
}

std::string json_dump(const Json& j) {
  std::string out;
  write_value(out, j);
  return out;
}

uint64_t json_u64(const Json& j, const std::string& where) {
  uint64_t v = 0;
  require(j.kind == Json::Number, SS_E_DESC, where + ": not a number");
  require(magnitude(j.text, 0, &v), SS_E_DESC, where + ": " + j.text + " is not an integer in 0..2^64-1");
  return v;
}

int64_t json_i64(const Json& j, const std::string& where) {
  require(j.kind == Json::Number, SS_E_DESC, where + ": not a number");
  const bool minus = !j.text.empty() && j.text[0] == '-';
  uint64_t v = 0;
  require(magnitude(j.text, minus ? 1 : 0, &v) && v <= uint64_t(INT64_MAX), SS_E_DESC,
          where + ": " + j.text + " is not an integer of magnitude below 2^63");
  return minus ? -int64_t(v) : int64_t(v);
}

double json_f64(const Json& j, const std::string& where) {
  require(j.kind == Json::Number, SS_E_DESC, where + ": not a number");
  char* end = nullptr;
  const double v = std::strtod(j.text.c_str(), &end);
  require(end && *end == '\0' && std::isfinite(v), SS_E_DESC, where + ": " + j.text + " is not a finite double");
  return v;
}

const std::string& json_str(const Json& j, const std::string& where) {
  require(j.kind == Json::String, SS_E_DESC, where + ": not a string");
  return j.text;
}

bool json_bool(const Json& j, const std::string& where) {
  require(j.kind == Json::Bool, SS_E_DESC, where + ": not true or false");
  return j.b;
}

}  // namespace tsa
