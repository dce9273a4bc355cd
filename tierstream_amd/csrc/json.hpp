// A small JSON DOM for the descriptor / plan documents: objects keep their keys sorted (canonical output), numbers keep
// their source text (an integer never passes through a double).
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace tsa {

struct Json {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  std::string text;  // Number: the literal; String: the value
  std::vector<Json> arr;
  std::map<std::string, Json> obj;

  static Json object() { Json j; j.kind = Object; return j; }
  static Json array() { Json j; j.kind = Array; return j; }
  static Json string(const std::string& s) { Json j; j.kind = String; j.text = s; return j; }
  static Json number(uint64_t v) { Json j; j.kind = Number; j.text = std::to_string(v); return j; }
  static Json number_i(int64_t v) { Json j; j.kind = Number; j.text = std::to_string(v); return j; }
  static Json number_f(double v);
  static Json boolean(bool v) { Json j; j.kind = Bool; j.b = v; return j; }

  bool is_object() const { return kind == Object; }
  bool is_array() const { return kind == Array; }
  const Json* find(const std::string& k) const {
    if (kind != Object) return nullptr;
    auto it = obj.find(k);
    return it == obj.end() ? nullptr : &it->second;
  }
  Json& operator[](const std::string& k) { return obj[k]; }
  void push(const Json& v) { arr.push_back(v); }
};

// Throws Error(SS_E_DESC) on malformed text (depth-limited).
Json json_parse(const std::string& text);
std::string json_dump(const Json& j);  // canonical: sorted keys, no whitespace

uint64_t json_u64(const Json& j, const std::string& where);
int64_t json_i64(const Json& j, const std::string& where);
double json_f64(const Json& j, const std::string& where);
const std::string& json_str(const Json& j, const std::string& where);
bool json_bool(const Json& j, const std::string& where);

}  // namespace tsa
