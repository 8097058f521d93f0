#include "device.h"

namespace minimind::model {

void throw_hip(hipError_t status, const char* what) {
  throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(status) + " (" +
                           std::to_string(static_cast<int>(status)) + ")");
}

void DeviceBuffer::reset(std::size_t bytes) {
  release();
  if (bytes == 0) return;
  check_hip(hipMalloc(&data_, bytes), "hipMalloc");
  bytes_ = bytes;
}

void DeviceBuffer::release() noexcept {
  if (data_) (void)hipFree(data_);
  data_ = nullptr;
  bytes_ = 0;
}

}  // namespace minimind::model
