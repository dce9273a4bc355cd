#include "source.hpp"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>

#include "common.hpp"

namespace tsa {

SourceFile::SourceFile(const std::string& path, bool direct) : path_(path) {
  if (direct) {
    fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC | O_DIRECT);
    direct_ = fd_ >= 0;
  }
  if (fd_ < 0) fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);  // buffered: the file system refused O_DIRECT
  require(fd_ >= 0, SS_E_IO, "open source " + path + ": " + std::strerror(errno));
  struct stat st;
  if (::fstat(fd_, &st) != 0) {
    const int e = errno;
    ::close(fd_);
    fail(SS_E_IO, "stat source " + path + ": " + std::strerror(e));
  }
  size_ = uint64_t(st.st_size);
}

SourceFile::~SourceFile() {
  if (fd_ >= 0) ::close(fd_);
}

namespace {
// Unbuffered reads cannot land in hipHostMalloc memory (the kernel cannot pin those pages for the DMA: EFAULT). Such
// reads go through a page-aligned pageable buffer of the reading thread, then a memcpy.
constexpr uint64_t kBounce = 8ull << 20;
struct Bounce {
  void* p = nullptr;
  ~Bounce() { std::free(p); }
};
thread_local Bounce t_bounce;
}  // namespace

uint64_t SourceFile::pread_some(void* dst, uint64_t n, uint64_t off) const {
  uint64_t got = 0;
  bool bounced = false;
  while (got < n) {
    char* out = static_cast<char*>(dst) + got;
    const uint64_t want = n - got;
    ssize_t r;
    if (direct_ && (bounced || bounce_.load(std::memory_order_relaxed))) {
      if (!t_bounce.p) {
        t_bounce.p = std::aligned_alloc(4096, kBounce);
        require(t_bounce.p != nullptr, SS_E_NOMEM, "read bounce buffer");
      }
      r = ::pread(fd_, t_bounce.p, size_t(std::min(want, kBounce)), off_t(off + got));
      if (r > 0) std::memcpy(out, t_bounce.p, size_t(r));
    } else {
      r = ::pread(fd_, out, size_t(want), off_t(off + got));
    }
    if (r < 0) {
      if (errno == EINTR) continue;
      if (errno == EFAULT && direct_ && !bounced) {  // (another reader may have switched already: retry anyway)
        bounce_.store(true, std::memory_order_relaxed);
        bounced = true;
        continue;
      }
      fail(SS_E_IO, "read " + path_ + " at " + std::to_string(off + got) + ": " + std::strerror(errno));
    }
    if (r == 0) break;
    got += uint64_t(r);
  }
  return got;
}

void SourceFile::pread_all(void* dst, uint64_t n, uint64_t off) const {
  require(pread_some(dst, n, off) == n, SS_E_IO, "short read of " + path_ + " at " + std::to_string(off));
}

}  // namespace tsa
