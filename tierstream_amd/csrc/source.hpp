// A descriptor source file, read with positional reads. O_DIRECT when asked and the file system allows it (else
// buffered, reported by ss_source_direct); unaligned ranges are read through an aligned covering buffer by the caller.
#pragma once

#include <atomic>
#include <cstdint>
#include <string>

namespace tsa {

class SourceFile {
 public:
  SourceFile(const std::string& path, bool direct);
  ~SourceFile();
  SourceFile(const SourceFile&) = delete;
  SourceFile& operator=(const SourceFile&) = delete;

  uint64_t size() const { return size_; }
  bool direct() const { return direct_; }
  const std::string& path() const { return path_; }
  // Reads exactly n bytes at off (short reads retried; EOF or an error throws SS_E_IO). With direct(), dst, n and off
  // must be multiples of the device alignment (the caller covers unaligned ranges).
  void pread_all(void* dst, uint64_t n, uint64_t off) const;
  // Up to n bytes at off (returns the count; stops early only at EOF).
  uint64_t pread_some(void* dst, uint64_t n, uint64_t off) const;

 private:
  std::string path_;
  int fd_ = -1;
  bool direct_ = false;
  uint64_t size_ = 0;
  mutable std::atomic<bool> bounce_{false};  // direct reads into pinned memory failed: bounce through pageable memory
};

}  // namespace tsa
