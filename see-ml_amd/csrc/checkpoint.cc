// checkpoint.cc — the SEKP container (runtime/custodian/checkpoint.cc:39-83).
#include "checkpoint.h"

#include <fcntl.h>
#include <unistd.h>

#include <cerrno>
#include <cstdio>
#include <cstring>
#include <vector>

namespace seeml_hip {

namespace {

struct CheckpointHeader {
  uint32_t magic;
  uint32_t version;
  uint64_t plan_hash;
  uint64_t step;
  uint64_t persistent_size;
  uint64_t payload_hash;
};
static_assert(sizeof(CheckpointHeader) == 40, "the SEKP header is 40 bytes");

Status Fail(const std::string& m) { return Status::Fail(kUnitCheckpoint, m); }

// Writes all of [p, p + n) to fd, retrying short writes and EINTR.
bool WriteAll(int fd, const uint8_t* p, uint64_t n) {
  while (n > 0) {
    const ssize_t w = ::write(fd, p, n > (1u << 30) ? (1u << 30) : static_cast<size_t>(n));
    if (w < 0 && errno == EINTR) continue;
    if (w <= 0) return false;
    p += w;
    n -= static_cast<uint64_t>(w);
  }
  return true;
}

// Reads exactly n bytes; false on a short file or an error.
bool ReadAll(int fd, uint8_t* p, uint64_t n) {
  while (n > 0) {
    const ssize_t r = ::read(fd, p, n > (1u << 30) ? (1u << 30) : static_cast<size_t>(n));
    if (r < 0 && errno == EINTR) continue;
    if (r <= 0) return false;
    p += r;
    n -= static_cast<uint64_t>(r);
  }
  return true;
}

std::string DirOf(const std::string& path) {
  const size_t slash = path.find_last_of('/');
  if (slash == std::string::npos) return ".";
  return slash == 0 ? "/" : path.substr(0, slash);
}

}  // namespace

Status WriteCheckpoint(const std::string& path, uint64_t plan_hash, uint64_t step,
                       const uint8_t* payload, uint64_t size) {
  const CheckpointHeader h{kCheckpointMagic, kCheckpointVersion, plan_hash, step, size,
                           ContentHash64(payload, size)};
  const std::string tmp = path + ".tmp";
  const int fd = ::open(tmp.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
  if (fd < 0) return Fail("cannot write '" + path + "': " + std::strerror(errno));
  const bool ok = WriteAll(fd, reinterpret_cast<const uint8_t*>(&h), sizeof h) &&
                  WriteAll(fd, payload, size) && ::fsync(fd) == 0;
  const int err = errno;
  if (::close(fd) != 0 || !ok) {
    ::unlink(tmp.c_str());
    return Fail("short write to '" + path + "': " + std::strerror(ok ? errno : err));
  }
  if (::rename(tmp.c_str(), path.c_str()) != 0) {
    const int e = errno;
    ::unlink(tmp.c_str());
    return Fail("cannot replace '" + path + "': " + std::strerror(e));
  }
  // The rename is durable only once the directory entry is on disk.
  const int dfd = ::open(DirOf(path).c_str(), O_RDONLY | O_DIRECTORY | O_CLOEXEC);
  if (dfd >= 0) {
    (void)::fsync(dfd);
    ::close(dfd);
  }
  return Status::Ok();
}

Status ReadCheckpoint(const std::string& path, uint64_t plan_hash, uint64_t size, uint8_t* dst,
                      uint64_t* step) {
  const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) return Fail("no checkpoint at '" + path + "'");
  CheckpointHeader h{};
  Status s = Status::Ok();
  std::vector<uint8_t> payload;
  if (!ReadAll(fd, reinterpret_cast<uint8_t*>(&h), sizeof h) || h.magic != kCheckpointMagic ||
      h.version != kCheckpointVersion) {
    s = Fail("not a v3 checkpoint: '" + path + "'");
  } else if (h.plan_hash != plan_hash) {
    // The segment's layout is one plan's: any other plan would misread it.
    s = Fail("checkpoint belongs to a different plan");
  } else if (h.persistent_size != size) {
    s = Fail("checkpoint incompatible with plan");
  } else {
    payload.resize(size);
    if (!ReadAll(fd, payload.data(), size))
      s = Fail("truncated checkpoint");
    else if (ContentHash64(payload.data(), size) != h.payload_hash)
      s = Fail("checkpoint payload is corrupt");
  }
  ::close(fd);
  if (!s) return s;
  std::memcpy(dst, payload.data(), size);
  *step = h.step;
  return Status::Ok();
}

}  // namespace seeml_hip
