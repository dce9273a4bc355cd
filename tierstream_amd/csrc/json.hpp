// JSON for the descriptor, plan and stats documents. The DOM keeps each number's literal text (an integer never passes
// through a double) and each object's keys in byte order, so writing a document back gives its canonical form: keys
// sorted, no whitespace, numbers as read.
//
// Accepted text (the desc-v1 / plan-v1 rules of reference src/json.cpp): RFC 8259 values with whitespace limited to
// space, tab, LF and CR; at most 64 containers nested below the top value; no duplicate keys; \u escapes decoded to
// UTF-8 with surrogates only as a high-low pair; raw bytes 0x80 and above passed through; at most 256 MiB of text.
// Written strings escape '"', '\\', LF, CR and tab by name and every other byte below 0x20 as \u00xx.
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace tsa {

struct Json {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  std::string text;  // Number: its literal; String: its decoded bytes
  std::vector<Json> arr;
  std::map<std::string, Json> obj;

  static Json object() { return of(Object); }
  static Json array() { return of(Array); }
  static Json string(const std::string& s) {
    Json j = of(String);
    j.text = s;
    return j;
  }
  static Json number(uint64_t v) {
    Json j = of(Number);
    j.text = std::to_string(v);
    return j;
  }
  static Json number_i(int64_t v) {
    Json j = of(Number);
    j.text = std::to_string(v);
    return j;
  }
  static Json number_f(double v);  // shortest round-trip form is not promised: 17 significant digits
  static Json boolean(bool v) {
    Json j = of(Bool);
    j.b = v;
    return j;
  }

  bool is_object() const { return kind == Object; }
  bool is_array() const { return kind == Array; }
  const Json* find(const std::string& k) const {
    if (kind != Object) return nullptr;
    const auto it = obj.find(k);
    return it == obj.end() ? nullptr : &it->second;
  }
  Json& operator[](const std::string& k) { return obj[k]; }
  void push(const Json& v) { arr.push_back(v); }

 private:
  static Json of(Kind k) {
    Json j;
    j.kind = k;
    return j;
  }
};

Json json_parse(const std::string& text);  // SS_E_DESC naming the byte offset of the first fault
std::string json_dump(const Json& j);       // canonical form

// Typed reads of a parsed value; SS_E_DESC naming `where` when the value is not of that type or out of range.
uint64_t json_u64(const Json& j, const std::string& where);  // digits only
int64_t json_i64(const Json& j, const std::string& where);   // digits with an optional '-'
double json_f64(const Json& j, const std::string& where);    // any number that is finite as a double
const std::string& json_str(const Json& j, const std::string& where);
bool json_bool(const Json& j, const std::string& where);

}  // namespace tsa
