// E8 closest-point decoding and the 64-bit cell id on the device (the reference: detail/e8.cuh:13-85),
// shared by the search kernels and the index builder.  D8 rounding with the parity fix, the nearer
// of D8 and D8 + 1/2 (ties: D8) with distances t = x - a, acc = fma(t, t, acc), and the hash of
// 2 p over the primes with the 64-bit mixer.
#pragma once

#include <hip/hip_runtime.h>

namespace cuvs::neighbors::octex::detail {

namespace {

__constant__ long long kPrimes[8] = {1000003LL,
                                     998244353LL,
                                     1000000007LL,
                                     2147483647LL,
                                     1099511627791LL,
                                     4398042316799LL,
                                     70368744177643LL,
                                     1125899906842597LL};  // e8.cuh:13-20
constexpr unsigned long long kMix = 0x9E3779B97F4A7C15ULL;  // e8.cuh:21

// ------------------------------------------------------------------ E8 (e8.cuh:24-85)

/**
 * Nearest point of D8: round every coordinate, then fix the parity at the worst-rounded one, the first index
 * whose |x - rint(x)| is the largest (the reference's strict-greater scan from -1 picks the same one; a NaN error
 * is never picked, and when every error is NaN the reference's fix lands on a coordinate that is NaN or infinite
 * already).  The fix moves that coordinate one step towards x: copysign(1, e), e never being -0 here.
 */
__device__ __forceinline__ void d8(const float (&x)[8], float (&f)[8])
{
  float s = 0.f, m = -1.f, e[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    f[i] = rintf(x[i]);
    s    = s + f[i];
    e[i] = x[i] - f[i];
    m    = fmaxf(m, fabsf(e[i]));
  }
  // fmodf(s, 2) != 0, with the integer parity for |s| < 2^24 (every such s here is an integer, and fmodf's
  // general reduction loop is costly); larger, infinite or NaN sums take fmodf itself
  const bool odd = fabsf(s) < 16777216.f ? (static_cast<int>(s) & 1) != 0 : fmodf(s, 2.f) != 0.f;
  bool seen      = false;
#pragma unroll
  for (int i = 0; i < 8; i++) {  // selects, not branches: the fixed coordinate differs between lanes
    const bool pick = !seen && fabsf(e[i]) == m;
    seen            = seen || pick;
    f[i]            = (odd && pick) ? f[i] + copysignf(1.f, e[i]) : f[i];
  }
}

/** Nearest point of E8 = D8 u (D8 + 1/2): the nearer of the two cosets' points (ties: D8). */
__device__ __forceinline__ void e8_point(const float (&x)[8], float (&p)[8])
{
  float a[8], c[8], xs[8];
#pragma unroll
  for (int i = 0; i < 8; i++)
    xs[i] = x[i] - 0.5f;
  d8(x, a);
  d8(xs, c);
  float da = 0.f, dc = 0.f;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    c[i]     = c[i] + 0.5f;
    float ta = x[i] - a[i];
    float tc = x[i] - c[i];
    da       = fmaf(ta, ta, da);
    dc       = fmaf(tc, tc, dc);
  }
  const bool useA = da <= dc;
#pragma unroll
  for (int i = 0; i < 8; i++)
    p[i] = useA ? a[i] : c[i];
}

/** The i-th prime as a signed low word and a high word with P = hi 2^32 + lo (mod 2^64), for 32 x 32 products. */
struct prime_split {
  int lo, hi;
};
constexpr auto split_prime(unsigned long long P) -> prime_split
{
  const unsigned lo = static_cast<unsigned>(P & 0xffffffffULL);
  const unsigned hi = static_cast<unsigned>(P >> 32) + (lo >= 0x80000000u ? 1u : 0u);
  return {static_cast<int>(lo), static_cast<int>(hi)};
}
constexpr prime_split kPrimeSplit[8] = {split_prime(1000003ULL),          split_prime(998244353ULL),
                                        split_prime(1000000007ULL),       split_prime(2147483647ULL),
                                        split_prime(1099511627791ULL),    split_prime(4398042316799ULL),
                                        split_prime(70368744177643ULL),   split_prime(1125899906842597ULL)};

/**
 * Block hash: sum of 2 p_i times the i-th prime (64-bit wraparound).  When every |2 p_i| < 2^31, 2 p_i is a 32-bit
 * integer q and q P = q lo + (q hi mod 2^32) 2^32 (mod 2^64) with lo, hi of kPrimeSplit: a 32 x 32 -> 64 signed
 * multiply-add, plus a 32-bit product into the high word for the primes above 2^31.  Otherwise 2 p_i goes through
 * the int64 conversion itself.
 */
__device__ __forceinline__ unsigned long long block_hash(const float (&p)[8])
{
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; i++)
    amax = fmaxf(amax, fabsf(2.f * p[i]));
  unsigned long long hb = 0;
  if (amax < 2147483648.f) {
    unsigned long long lo = 0;  // each product fits in int64; their sum wraps mod 2^64
    unsigned hi           = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int q = static_cast<int>(2.f * p[i]);
      lo += static_cast<unsigned long long>(static_cast<long long>(q) * static_cast<long long>(kPrimeSplit[i].lo));
      if (kPrimeSplit[i].hi != 0) hi += static_cast<unsigned>(q) * static_cast<unsigned>(kPrimeSplit[i].hi);
    }
    hb = lo + (static_cast<unsigned long long>(hi) << 32);
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const long long p2 = static_cast<long long>(2.f * p[i]);
      hb += static_cast<unsigned long long>(p2) * static_cast<unsigned long long>(kPrimes[i]);
    }
  }
  return hb;
}

__device__ __forceinline__ long long finish_hash(unsigned long long h)
{
  long long hs = static_cast<long long>(h);
  hs           = static_cast<long long>(static_cast<unsigned long long>(hs ^ (hs >> 31)) * kMix);
  return hs ^ (hs >> 29);
}

/** 64-bit cell id of the E8^B point nearest to y * inv_f; coord(i) gives y[i] as a float. */
template <int B, typename Coord>
__device__ __forceinline__ long long e8b_hash64_of(Coord const& coord, float inv_f)
{
  unsigned long long h = 0;
#pragma unroll
  for (int j = 0; j < B; j++) {
    float x[8], p[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
      x[i] = coord(8 * j + i) * inv_f;
    e8_point(x, p);
    unsigned long long hb = block_hash(p);
    h                     = (j == 0) ? hb : h * kMix + hb;
  }
  return finish_hash(h);
}

/** 64-bit cell id of the E8^B point nearest to y * inv_f. */
template <int B>
__device__ __forceinline__ long long e8b_hash64(const float (&y)[8 * B], float inv_f)
{
  return e8b_hash64_of<B>([&](int i) { return y[i]; }, inv_f);
}

}  // namespace

}  // namespace cuvs::neighbors::octex::detail
