/*
 * The minimal raft::resources of this library: the HIP device and stream a call runs on (the
 * reference's API takes a raft::resources, octex.hpp:214-253; RAFT itself is CUDA-only).
 */
#pragma once

#include <hip/hip_runtime_api.h>

namespace raft {

class resources {
 public:
  resources()
  {
    if (hipGetDevice(&device_) != hipSuccess) device_ = 0;
  }
  explicit resources(hipStream_t s) : resources() { stream_ = s; }
  [[nodiscard]] auto get_stream() const noexcept -> hipStream_t { return stream_; }
  void set_stream(hipStream_t s) noexcept { stream_ = s; }
  [[nodiscard]] auto device() const noexcept -> int { return device_; }

 private:
  hipStream_t stream_ = nullptr;
  int device_         = 0;
};

namespace resource {
inline auto get_cuda_stream(resources const& r) -> hipStream_t { return r.get_stream(); }
}  // namespace resource

}  // namespace raft
