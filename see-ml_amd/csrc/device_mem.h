// device_mem.h — device allocation and graph capture, serialised across
// engines.
//
// On this runtime a stream capture is invalidated when another thread makes
// a call that waits on the capturing stream: a copy on the legacy stream, or
// a free that synchronises the device. Engines on one GPU capture their
// graphs on their own streams from their own threads, so every allocation,
// free and capture in this library holds one process-wide lock: no engine
// allocates or frees while another captures. Copies are issued on the
// engine's own (non-blocking) stream.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <mutex>

namespace seeml_hip {

std::recursive_mutex& DeviceMemMutex();

template <typename T>
inline hipError_t LockedMalloc(T** p, size_t bytes) {
  std::lock_guard<std::recursive_mutex> lock(DeviceMemMutex());
  return hipMalloc(reinterpret_cast<void**>(p), bytes);
}
inline hipError_t LockedFree(void* p) {
  std::lock_guard<std::recursive_mutex> lock(DeviceMemMutex());
  return hipFree(p);
}
template <typename T>
inline hipError_t LockedHostMalloc(T** p, size_t bytes) {
  std::lock_guard<std::recursive_mutex> lock(DeviceMemMutex());
  return hipHostMalloc(reinterpret_cast<void**>(p), bytes, hipHostMallocDefault);
}
inline hipError_t LockedHostFree(void* p) {
  std::lock_guard<std::recursive_mutex> lock(DeviceMemMutex());
  return hipHostFree(p);
}

}  // namespace seeml_hip
