/*
 * Minimal row-major matrix views with the names and accessors of RAFT's host/device mdspans
 * (data_handle(), extent(i), size()), which the reference's C++ API takes (octex.hpp:214-253).
 */
#pragma once

#include <cstdint>

namespace raft {

struct row_major {};

namespace detail {
template <typename T, typename I, bool Device>
class matrix_view {
 public:
  using value_type = T;
  using index_type = I;
  static constexpr bool is_device_accessible = Device;
  static constexpr int rank() { return 2; }
  matrix_view() = default;
  matrix_view(T* p, I rows, I cols) : p_(p), rows_(rows), cols_(cols) {}
  [[nodiscard]] auto data_handle() const noexcept -> T* { return p_; }
  [[nodiscard]] auto extent(int i) const noexcept -> I { return i == 0 ? rows_ : cols_; }
  [[nodiscard]] auto size() const noexcept -> I { return rows_ * cols_; }

 private:
  T* p_    = nullptr;
  I rows_  = 0;
  I cols_  = 0;
};
}  // namespace detail

template <typename T, typename I = int64_t, typename L = row_major>
using host_matrix_view = detail::matrix_view<T, I, false>;
template <typename T, typename I = int64_t, typename L = row_major>
using device_matrix_view = detail::matrix_view<T, I, true>;

template <typename T, typename I>
auto make_host_matrix_view(T* p, I rows, I cols) -> host_matrix_view<T, I>
{
  return host_matrix_view<T, I>(p, rows, cols);
}
template <typename T, typename I>
auto make_device_matrix_view(T* p, I rows, I cols) -> device_matrix_view<T, I>
{
  return device_matrix_view<T, I>(p, rows, cols);
}

}  // namespace raft
