// SHA-256 (FIPS 180-4): the digest that binds a scored-eviction profile to its model and checks its bytes.
#pragma once

#include <cstddef>
#include <string>

namespace tsa {

// The 32 raw digest bytes of data[0..n).
std::string sha256(const void* data, size_t n);

}  // namespace tsa
