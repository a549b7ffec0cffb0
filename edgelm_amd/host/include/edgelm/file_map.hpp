// A read-only mapping of a whole file (a model's .elm container or its device image), unmapped when
// the last owner lets go.
#pragma once
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <stdexcept>
#include <string>

namespace edgelm {

// A read-only private mapping of a whole file.
class FileMap {
 public:
  explicit FileMap(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) throw std::runtime_error("edgelm: cannot open file " + path);
    struct stat st {};
    const bool sized = ::fstat(fd, &st) == 0 && st.st_size > 0;
    if (sized) {
      len_ = static_cast<size_t>(st.st_size);
      void* p = ::mmap(nullptr, len_, PROT_READ, MAP_PRIVATE, fd, 0);
      base_ = p == MAP_FAILED ? nullptr : static_cast<const uint8_t*>(p);
    }
    ::close(fd);
    if (!base_) throw std::runtime_error("edgelm: cannot map file " + path + (sized ? "" : " (empty)"));
  }
  ~FileMap() { ::munmap(const_cast<uint8_t*>(base_), len_); }
  FileMap(const FileMap&) = delete;
  FileMap& operator=(const FileMap&) = delete;
  const uint8_t* base() const { return base_; }
  size_t size() const { return len_; }

 private:
  const uint8_t* base_ = nullptr;
  size_t len_ = 0;
};

}  // namespace edgelm
