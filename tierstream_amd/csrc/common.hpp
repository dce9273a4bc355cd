// Shared host-side helpers: the library's error type, checks, and the C ABI guard that turns exceptions into an
// ss_status plus a thread-local message.
#pragma once

#include <cstdint>
#include <cstring>
#include <new>
#include <stdexcept>
#include <string>

#include "strix_stream/ss.h"

namespace tsa {

class Error : public std::runtime_error {
 public:
  Error(ss_status s, const std::string& m) : std::runtime_error(m), status_(s) {}
  ss_status status() const { return status_; }

 private:
  ss_status status_;
};

[[noreturn]] inline void fail(ss_status s, const std::string& m) { throw Error(s, m); }
inline void require(bool ok, ss_status s, const std::string& m) {
  if (!ok) fail(s, m);
}
inline void require(bool ok, ss_status s, const char* m) {
  if (!ok) fail(s, m);
}

void set_last_error(const char* msg) noexcept;
void clear_last_error() noexcept;

// Runs f, mapping every exception to a status (the message is kept for ss_last_error).
template <class F>
ss_status guard(F&& f) noexcept {
  try {
    f();
    clear_last_error();
    return SS_OK;
  } catch (const Error& e) {
    set_last_error(e.what());
    return e.status();
  } catch (const std::bad_alloc&) {
    set_last_error("out of host memory");
    return SS_E_NOMEM;
  } catch (const std::exception& e) {
    set_last_error(e.what());
    return SS_E_BACKEND;
  } catch (...) {
    set_last_error("unknown exception");
    return SS_E_BACKEND;
  }
}

inline uint64_t round_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }
inline char* at(void* base, uint64_t off) { return static_cast<char*>(base) + off; }
inline const char* at(const void* base, uint64_t off) { return static_cast<const char*>(base) + off; }

// XXH64, seed 0 (host). Streaming, so file reads can hash chunk by chunk; checkpoints() exposes the accumulators.
class Xxh64 {
 public:
  Xxh64();
  void update(const void* data, size_t len);
  uint64_t digest() const;
  // The four accumulators; meaningful when every update so far was a multiple of 32 bytes (no buffered bytes).
  const uint64_t* acc() const { return v_; }
  uint64_t buffered() const { return buf_len_; }

 private:
  uint64_t v_[4];
  uint64_t total_ = 0;
  unsigned char buf_[32];
  size_t buf_len_ = 0;
};
uint64_t xxh64(const void* data, size_t len);

}  // namespace tsa
