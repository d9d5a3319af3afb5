// The search of device queries without a device allocation (octexSearchNoAlloc): the per-batch buffers of a
// plan (queries, projections, segments, candidates, kept lists, results) are laid out in `scratch`, a file-scope
// device array of kScratchBytes that every GPU the library runs on holds until the process ends, instead of a
// cached plan's hipMalloc'ed block; the kernels of the batch run directly on the caller's stream (no graph).
//
// In host code `scratch` names a host-side stand-in, not a device address: its device address on the current
// GPU comes from hipGetSymbolAddress, once per device, and only that address is passed to kernels and copies.
// Every call on one GPU shares its array and leaves its contents behind; a batch writes every buffer before it
// reads it, so nothing needs clearing between calls.  Calls that overlap on one GPU race on the array.

#include "common.hpp"
#include "index_impl.hpp"
#include "kernels.hpp"
#include "search.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>

namespace cuvs::neighbors::octex::detail {

namespace {

constexpr size_t kScratchBytes = size_t{256} << 20;
constexpr int kMaxDevices      = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex scratch_mu;
void* scratch_at[kMaxDevices] = {};  // the array's device address on each GPU

/** The device address of `scratch` on `device`, looked up the first time with that device current. */
auto scratch_on(int device) -> void*
{
  OCTEX_EXPECTS(device >= 0 && device < kMaxDevices, "octex: device %d out of range", device);
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (scratch_at[device] == nullptr) {
    void* p = nullptr;
    OCTEX_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    OCTEX_EXPECTS(p != nullptr, "octex: no device address for the search scratch on device %d", device);
    scratch_at[device] = p;
  }
  return scratch_at[device];
}

}  // namespace

void search_no_alloc(search_params const& sp, index const& idx, const float* queries, int64_t nq, int64_t dim,
                     int64_t k, int64_t* neighbors, float* distances, hipStream_t s)
{
  auto& ix = idx.impl();
  OCTEX_EXPECTS(dim == ix.dim, "octex: query dimension differs from the index");
  OCTEX_EXPECTS(k >= 1 && k <= kMaxSketchKO, "octex: k in [1, %d] for a search without allocations", kMaxSketchKO);
  OCTEX_EXPECTS(nq >= 0, "octex: a negative number of queries");
  if (nq == 0) return;
  OCTEX_EXPECTS(queries != nullptr && neighbors != nullptr && distances != nullptr, "octex: NULL tensor");
  const int m   = static_cast<int>(std::min<int64_t>(std::max(sp.batch, 1), nq));
  const auto sh = make_shape(ix, sp, m, static_cast<int>(k));
  const size_t need = carve_buffers(ix, sh, nullptr, nullptr);
  OCTEX_EXPECTS(need <= kScratchBytes,
                "octex: a search without allocations needs %zu bytes of scratch for a batch of %d queries with these "
                "parameters; the scratch holds %zu bytes: lower search_params.batch",
                need, m, kScratchBytes);
  int cur = 0;
  OCTEX_HIP(hipGetDevice(&cur));
  OCTEX_HIP(hipSetDevice(ix.device));
  try {
    batch_buffers b;
    carve_buffers(ix, sh, scratch_on(ix.device), &b);
    const int64_t D = ix.dim;
    for (int64_t b0 = 0; b0 < nq; b0 += m) {
      const int n = static_cast<int>(std::min<int64_t>(m, nq - b0));
      OCTEX_HIP(hipMemcpyAsync(b.qbuf, queries + b0 * D, sizeof(float) * n * D, hipMemcpyDeviceToDevice, s));
      if (n < m) launch_pad_rows(b.qbuf, n, m, static_cast<int>(D), s);
      launch_batch(ix, sh, b, s);
      OCTEX_HIP(hipMemcpyAsync(neighbors + b0 * k, b.bi, sizeof(int64_t) * n * k, hipMemcpyDeviceToDevice, s));
      OCTEX_HIP(hipMemcpyAsync(distances + b0 * k, b.bd, sizeof(float) * n * k, hipMemcpyDeviceToDevice, s));
    }
  } catch (...) {
    (void)hipSetDevice(cur);
    throw;
  }
  OCTEX_HIP(hipSetDevice(cur));
}

}  // namespace cuvs::neighbors::octex::detail
