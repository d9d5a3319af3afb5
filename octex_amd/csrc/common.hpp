// Shared host-side helpers of the octex MI355X library: error checks, device and pinned buffers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <utility>

namespace cuvs::neighbors::octex::detail {

/** An "octex: ..." exception (the reference's RAFT_EXPECTS / RAFT_FAIL texts). */
[[noreturn]] inline void fail(const char* fmt, ...)
{
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  throw std::runtime_error(buf);
}

#define OCTEX_EXPECTS(cond, ...)                                  \
  do {                                                            \
    if (!(cond)) ::cuvs::neighbors::octex::detail::fail(__VA_ARGS__); \
  } while (0)

#define OCTEX_HIP(call)                                                                        \
  do {                                                                                         \
    hipError_t e_ = (call);                                                                    \
    if (e_ != hipSuccess)                                                                      \
      ::cuvs::neighbors::octex::detail::fail("octex: HIP error %s (%s) at %s:%d", hipGetErrorName(e_), \
                                             hipGetErrorString(e_), __FILE__, __LINE__);      \
  } while (0)

/** Device memory of one allocation (freed on destruction). */
struct dbuf {
  void* ptr   = nullptr;
  size_t size = 0;
  dbuf()      = default;
  explicit dbuf(size_t bytes) : size(bytes)
  {
    if (bytes > 0) OCTEX_HIP(hipMalloc(&ptr, bytes));
  }
  dbuf(dbuf const&)                    = delete;
  auto operator=(dbuf const&) -> dbuf& = delete;
  dbuf(dbuf&& o) noexcept { *this = std::move(o); }
  auto operator=(dbuf&& o) noexcept -> dbuf&
  {
    std::swap(ptr, o.ptr);
    std::swap(size, o.size);
    return *this;
  }
  ~dbuf()
  {
    if (ptr != nullptr) (void)hipFree(ptr);
  }
  template <typename T>
  [[nodiscard]] auto as() const -> T*
  {
    return static_cast<T*>(ptr);
  }
};

/** Pinned, device-mapped host memory (hipHostMalloc); kernels read it in place through dptr. */
struct hbuf {
  void* ptr   = nullptr;
  void* dptr  = nullptr;
  size_t size = 0;
  hbuf()      = default;
  explicit hbuf(size_t bytes) : size(bytes)
  {
    if (bytes > 0) {
      OCTEX_HIP(hipHostMalloc(&ptr, bytes, hipHostMallocMapped | hipHostMallocPortable));
      OCTEX_HIP(hipHostGetDevicePointer(&dptr, ptr, 0));
    }
  }
  hbuf(hbuf const&)                    = delete;
  auto operator=(hbuf const&) -> hbuf& = delete;
  hbuf(hbuf&& o) noexcept { *this = std::move(o); }
  auto operator=(hbuf&& o) noexcept -> hbuf&
  {
    std::swap(ptr, o.ptr);
    std::swap(dptr, o.dptr);
    std::swap(size, o.size);
    return *this;
  }
  ~hbuf()
  {
    if (ptr != nullptr) (void)hipHostFree(ptr);
  }
  template <typename T>
  [[nodiscard]] auto as() const -> T*
  {
    return static_cast<T*>(ptr);
  }
};

/**
 * A host-to-device copy that is on the device when this returns and ordered before later work on s.  A
 * plain hipMemcpy from pageable memory may return before its DMA lands, and a non-blocking stream does
 * not wait for the null stream, so a kernel on s could read the old bytes.
 */
inline void upload(void* dst, const void* src, size_t bytes, hipStream_t s)
{
  if (bytes == 0) return;
  OCTEX_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s));
  OCTEX_HIP(hipStreamSynchronize(s));
}

/**
 * Allow a kernel `bytes` of dynamic LDS on the current device.  The attribute is set only when a launch needs more
 * than any earlier one of the same kernel on that device, so repeated launches of a plan (including launches under
 * stream capture) make no other runtime call than the launch itself.
 */
inline void allow_lds(const void* kernel, size_t bytes)
{
  static std::mutex mu;
  static std::map<std::pair<const void*, int>, size_t> set_to;
  int dev = 0;
  OCTEX_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(mu);
  auto& cur = set_to[{kernel, dev}];
  if (bytes <= cur) return;
  OCTEX_HIP(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes)));
  cur = bytes;
}

inline auto grid_for(int64_t total, int threads) -> unsigned
{
  return static_cast<unsigned>((total + threads - 1) / threads);
}

inline auto log2_ceil(int64_t v) -> int
{
  int e = 0;
  while ((int64_t{1} << e) < v)
    e++;
  return e;
}

}  // namespace cuvs::neighbors::octex::detail
