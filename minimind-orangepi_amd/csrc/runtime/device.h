// device.h -- HIP runtime plumbing: status checks and RAII device memory.
//
// Counterpart of the reference's AscendRuntime / DeviceBuffer
// (ascend_matmul.h:18-54): one explicit stream per decode state instead of a
// process-wide singleton, and buffers that never regrow implicitly.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <stdexcept>
#include <string>

namespace minimind::model {

[[noreturn]] void throw_hip(hipError_t status, const char* what);

inline void check_hip(hipError_t status, const char* what) {
  if (status != hipSuccess) throw_hip(status, what);
}

class DeviceBuffer {
 public:
  DeviceBuffer() = default;
  explicit DeviceBuffer(std::size_t bytes) { reset(bytes); }
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  DeviceBuffer(DeviceBuffer&& o) noexcept : data_(o.data_), bytes_(o.bytes_) {
    o.data_ = nullptr;
    o.bytes_ = 0;
  }
  DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
    if (this != &o) {
      release();
      data_ = o.data_;
      bytes_ = o.bytes_;
      o.data_ = nullptr;
      o.bytes_ = 0;
    }
    return *this;
  }
  ~DeviceBuffer() { release(); }

  void* data() const noexcept { return data_; }
  std::size_t bytes() const noexcept { return bytes_; }
  void reset(std::size_t bytes);

 private:
  void release() noexcept;
  void* data_ = nullptr;
  std::size_t bytes_ = 0;
};

// Bump allocator over one DeviceBuffer; every slice is 256-byte aligned.
class Arena {
 public:
  static constexpr std::size_t kAlign = 256;
  static std::size_t round_up(std::size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }
  void plan(std::size_t bytes) { planned_ += round_up(bytes); }
  void allocate() { buffer_.reset(planned_); }
  template <typename T>
  T* take(std::size_t count) {
    const std::size_t bytes = round_up(count * sizeof(T));
    if (used_ + bytes > buffer_.bytes()) throw std::logic_error("arena overflow");
    T* p = reinterpret_cast<T*>(static_cast<char*>(buffer_.data()) + used_);
    used_ += bytes;
    return p;
  }
  std::size_t bytes() const { return buffer_.bytes(); }
  void* base() const { return buffer_.data(); }

 private:
  DeviceBuffer buffer_;
  std::size_t planned_ = 0;
  std::size_t used_ = 0;
};

}  // namespace minimind::model
