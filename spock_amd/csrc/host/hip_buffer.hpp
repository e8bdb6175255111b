// hip_buffer.hpp -- RAII device memory and status checks for the C++ host side.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <stdexcept>
#include <string>
#include <utility>

#include "../../../include/spock_hip.h"

namespace spock::hip {

// Throws std::runtime_error for a failed HIP call (the reference's session
// reports device failures as exceptions too).
inline void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// Throws std::runtime_error for a non-zero C-ABI status, with the library's message.
inline void spk_check(int rc, const char* what) {
  if (rc != SPK_OK) throw std::runtime_error(std::string(what) + ": " + spk_last_error());
}

// Owning device allocation (hipMalloc / hipFree), move-only.
class DeviceBuffer {
 public:
  DeviceBuffer() = default;
  explicit DeviceBuffer(std::size_t bytes) : bytes_(bytes) {
    if (bytes_) hip_check(hipMalloc(&ptr_, bytes_), "hipMalloc");
  }
  ~DeviceBuffer() {
    if (ptr_) (void)hipFree(ptr_);
  }
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  DeviceBuffer(DeviceBuffer&& o) noexcept : ptr_(std::exchange(o.ptr_, nullptr)), bytes_(std::exchange(o.bytes_, 0)) {}
  DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
    if (this != &o) {
      if (ptr_) (void)hipFree(ptr_);
      ptr_ = std::exchange(o.ptr_, nullptr);
      bytes_ = std::exchange(o.bytes_, 0);
    }
    return *this;
  }
  template <typename T = void>
  T* get() const { return static_cast<T*>(ptr_); }
  std::size_t bytes() const { return bytes_; }

  void upload(const void* src, std::size_t n, std::size_t offset = 0) {
    if (offset + n > bytes_) throw std::runtime_error("DeviceBuffer::upload out of range");
    hip_check(hipMemcpy(static_cast<char*>(ptr_) + offset, src, n, hipMemcpyHostToDevice), "hipMemcpy H2D");
  }
  void download(void* dst, std::size_t n, std::size_t offset = 0) const {
    if (offset + n > bytes_) throw std::runtime_error("DeviceBuffer::download out of range");
    hip_check(hipMemcpy(dst, static_cast<const char*>(ptr_) + offset, n, hipMemcpyDeviceToHost), "hipMemcpy D2H");
  }
  void zero(hipStream_t s = nullptr) {
    if (bytes_) hip_check(hipMemsetAsync(ptr_, 0, bytes_, s), "hipMemsetAsync");
  }

 private:
  void* ptr_ = nullptr;
  std::size_t bytes_ = 0;
};

}  // namespace spock::hip
