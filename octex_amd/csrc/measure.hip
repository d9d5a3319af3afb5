// The random-row read ceiling of the GPU: the access pattern of every search gather (short rows at random
// addresses of a many-GB array, many rows in flight) with no other work, so that a gather's achieved rate can be
// set against what the memory system delivers for the same rows.  Measurement only: no search path calls it.

#include "common.hpp"

#include <cuvs/core/c_api.h>
#include <octex_amd/octex_amd.h>

#include <exception>

namespace {

using namespace cuvs::neighbors::octex::detail;

/** splitmix64 finalizer: a well-mixed 64-bit value of j. */
__device__ __forceinline__ uint64_t mix64(uint64_t z)
{
  z += 0x9e3779b97f4a7c15ULL;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}

/**
 * n random rows of `pieces` 16-byte pieces each (row r at base + r * pitch, r uniform in [0, rows)), read by
 * LR-lane groups, one 16-byte load per lane (lanes past the row's pieces read its first piece, as the sketch
 * gather does), R rows of a group in flight before any is used.  The XOR of every word a group read goes to
 * out[group] so that no load is dropped.  The grid strides over the rows; every wavefront leaves after its last.
 */
template <int LR, int R>
__global__ __launch_bounds__(256) void row_read_kernel(const unsigned char* __restrict__ base, uint64_t rows,
                                                       int pitch, int pieces, int64_t n, uint64_t seed,
                                                       unsigned* __restrict__ out)
{
  const int sub        = threadIdx.x & (LR - 1);
  const int64_t grp    = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / LR;
  const int64_t ngrp   = static_cast<int64_t>(gridDim.x) * blockDim.x / LR;
  const int64_t piece  = sub < pieces ? 16 * sub : 0;
  unsigned acc         = 0;
  for (int64_t j0 = grp * R; j0 < n; j0 += ngrp * R) {
    uint4 w[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int64_t j  = min(j0 + r, n - 1);
      const uint64_t v = __umul64hi(mix64(seed + static_cast<uint64_t>(j)), rows);
      w[r]             = *reinterpret_cast<const uint4*>(base + v * static_cast<uint64_t>(pitch) + piece);
    }
#pragma unroll
    for (int r = 0; r < R; r++)
      acc ^= w[r].x ^ w[r].y ^ w[r].z ^ w[r].w;
  }
  if (sub == 0) out[grp] = acc;
}

template <int LR>
void launch_rows(int R, unsigned blocks, const unsigned char* base, uint64_t rows, int pitch, int pieces, int64_t n,
                 uint64_t seed, unsigned* out, hipStream_t s)
{
  switch (R) {
    case 1: row_read_kernel<LR, 1><<<blocks, 256, 0, s>>>(base, rows, pitch, pieces, n, seed, out); break;
    case 2: row_read_kernel<LR, 2><<<blocks, 256, 0, s>>>(base, rows, pitch, pieces, n, seed, out); break;
    case 4: row_read_kernel<LR, 4><<<blocks, 256, 0, s>>>(base, rows, pitch, pieces, n, seed, out); break;
    default: row_read_kernel<LR, 8><<<blocks, 256, 0, s>>>(base, rows, pitch, pieces, n, seed, out); break;
  }
}

}  // namespace

extern "C" cuvsError_t octexMeasureRowReads(const void* base, int64_t rows, int32_t pitch, int32_t row_bytes,
                                            int64_t n, int32_t in_flight, int32_t blocks, uint64_t seed,
                                            uint32_t* out, void* stream)
{
  try {
    OCTEX_EXPECTS(base != nullptr && out != nullptr, "octex: row reads need a base array and an output");
    OCTEX_EXPECTS(rows >= 1 && n >= 1, "octex: row reads need rows");
    OCTEX_EXPECTS(row_bytes >= 16 && row_bytes <= 512 && row_bytes % 16 == 0,
                  "octex: row_bytes must be a multiple of 16 in [16, 512]");
    OCTEX_EXPECTS(pitch >= row_bytes && pitch % 16 == 0, "octex: pitch must be a multiple of 16 >= row_bytes");
    OCTEX_EXPECTS(in_flight == 1 || in_flight == 2 || in_flight == 4 || in_flight == 8,
                  "octex: in_flight must be 1, 2, 4 or 8");
    OCTEX_EXPECTS(blocks >= 1, "octex: blocks must be positive");
    const int pieces = row_bytes / 16;
    int lr           = 1;
    while (lr < pieces)
      lr <<= 1;
    // out holds one word per group: blocks * 256 / lr words
    auto s   = static_cast<hipStream_t>(stream);
    auto b   = static_cast<const unsigned char*>(base);
    auto r   = static_cast<uint64_t>(rows);
    auto nb  = static_cast<unsigned>(blocks);
    auto* o  = reinterpret_cast<unsigned*>(out);
    switch (lr) {
      case 1: launch_rows<1>(in_flight, nb, b, r, pitch, pieces, n, seed, o, s); break;
      case 2: launch_rows<2>(in_flight, nb, b, r, pitch, pieces, n, seed, o, s); break;
      case 4: launch_rows<4>(in_flight, nb, b, r, pitch, pieces, n, seed, o, s); break;
      case 8: launch_rows<8>(in_flight, nb, b, r, pitch, pieces, n, seed, o, s); break;
      case 16: launch_rows<16>(in_flight, nb, b, r, pitch, pieces, n, seed, o, s); break;
      default: launch_rows<32>(in_flight, nb, b, r, pitch, pieces, n, seed, o, s); break;
    }
    OCTEX_HIP(hipGetLastError());
    cuvsSetLastErrorText(nullptr);
    return CUVS_SUCCESS;
  } catch (std::exception const& e) {
    cuvsSetLastErrorText(e.what());
  } catch (...) {
    cuvsSetLastErrorText("unknown exception");
  }
  return CUVS_ERROR;
}
