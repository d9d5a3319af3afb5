/*
 * CPU oracle of the octex batched search path: TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it.  Every function cites
 * the reference file:line it restates; the arithmetic pins are listed in octex_oracle.h.
 */
#include "octex_oracle.h"

#include <algorithm>
#include <atomic>
#include <charconv>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <exception>
#include <fstream>
#include <immintrin.h>
#include <numeric>
#include <random>
#include <sstream>
#include <stdexcept>
#include <string>
#include <sys/stat.h>
#include <thread>
#include <vector>

namespace {

thread_local std::string g_err;

// ---------------------------------------------------------------- fp16

uint16_t f2h(float f)
{
  uint32_t x;
  std::memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ex   = (x >> 23) & 0xffu;
  uint32_t man  = x & 0x7fffffu;
  if (ex == 0xffu) return static_cast<uint16_t>(sign | 0x7c00u | (man ? 0x200u | (man >> 13) : 0u));
  int e = static_cast<int>(ex) - 127 + 15;
  if (e >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return static_cast<uint16_t>(sign);
    uint32_t M     = man | 0x800000u;
    int sh         = 14 - e;
    uint32_t hm    = M >> sh;
    uint32_t rem   = M & ((1u << sh) - 1u);
    uint32_t halfw = 1u << (sh - 1);
    if (rem > halfw || (rem == halfw && (hm & 1u))) hm++;
    return static_cast<uint16_t>(sign | hm);
  }
  uint32_t h   = sign | (static_cast<uint32_t>(e) << 10) | (man >> 13);
  uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return static_cast<uint16_t>(h);
}

float h2f(uint16_t h)
{
  uint32_t sign = (h & 0x8000u) ? 1u : 0u;
  uint32_t ex   = (h >> 10) & 0x1fu;
  uint32_t man  = h & 0x3ffu;
  float v;
  if (ex == 0) {
    v = std::ldexp(static_cast<float>(man), -24);
  } else if (ex == 31) {
    uint32_t x = (sign << 31) | 0x7f800000u | (man << 13);
    std::memcpy(&v, &x, 4);
    return v;
  } else {
    uint32_t x = ((ex + 112u) << 23) | (man << 13);
    std::memcpy(&v, &x, 4);
  }
  return sign ? -v : v;
}

inline uint32_t fbits(float f)
{
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}

/**
 * fp64 -> fp16 with a single rounding to nearest even.  The value is first taken to fp32 by rounding to
 * odd (truncate toward zero, then set the last significand bit when inexact); fp32 keeps 13 more bits than
 * fp16, so the second rounding sees every tie and every sticky bit the direct rounding would.
 */
uint16_t d2h(double d)
{
  float f = static_cast<float>(d);
  if (std::isfinite(f) && static_cast<double>(f) != d) {
    if (std::fabs(static_cast<double>(f)) > std::fabs(d)) f = std::nextafter(f, 0.0f);
    uint32_t u = fbits(f) | 1u;
    std::memcpy(&f, &u, 4);
  }
  return f2h(f);
}
inline float bitsf(uint32_t u)
{
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// ---------------------------------------------------------------- E8 (e8.cuh)

const int64_t kPrimes[8] = {1000003LL,
                            998244353LL,
                            1000000007LL,
                            2147483647LL,
                            1099511627791LL,
                            4398042316799LL,
                            70368744177643LL,
                            1125899906842597LL};  // e8.cuh:13-20
const uint64_t kMix      = 0x9E3779B97F4A7C15ULL;  // e8.cuh:21

/** Nearest point of D8 (e8.cuh:24-41). */
void d8(const float* x, float* f)
{
  float s  = 0.f;
  int im   = 0;
  float em = -1.f, ei = 0.f;
  for (int i = 0; i < 8; i++) {
    f[i] = std::nearbyint(x[i]);
    s    = s + f[i];
    float e = x[i] - f[i];
    if (std::fabs(e) > em) {
      em = std::fabs(e);
      im = i;
      ei = e;
    }
  }
  if (std::fmod(s, 2.f) != 0.f) f[im] = f[im] + (ei >= 0.f ? 1.f : -1.f);
}

/** Nearest point of E8 = D8 u (D8 + 1/2) (e8.cuh:44-62). */
void e8_point(const float* x, float* p)
{
  float a[8], c[8], xs[8];
  for (int i = 0; i < 8; i++)
    xs[i] = x[i] - 0.5f;
  d8(x, a);
  d8(xs, c);
  float da = 0.f, dc = 0.f;
  for (int i = 0; i < 8; i++) {
    c[i]     = c[i] + 0.5f;
    float ta = x[i] - a[i];
    float tc = x[i] - c[i];
    da       = std::fma(ta, ta, da);
    dc       = std::fma(tc, tc, dc);
  }
  for (int i = 0; i < 8; i++)
    p[i] = da <= dc ? a[i] : c[i];
}

/** e8.cuh:65-85. */
int64_t e8b_hash64(const float* y, int b, float inv_f)
{
  uint64_t h = 0;
  for (int j = 0; j < b; j++) {
    float x[8], p[8];
    for (int i = 0; i < 8; i++)
      x[i] = y[8 * j + i] * inv_f;
    e8_point(x, p);
    uint64_t hb = 0;
    for (int i = 0; i < 8; i++) {
      int64_t p2 = static_cast<int64_t>(2.f * p[i]);
      hb += static_cast<uint64_t>(p2) * static_cast<uint64_t>(kPrimes[i]);
    }
    h = (j == 0) ? hb : h * kMix + hb;
  }
  int64_t hs = static_cast<int64_t>(h);
  hs         = static_cast<int64_t>(static_cast<uint64_t>(hs ^ (hs >> 31)) * kMix);
  return hs ^ (hs >> 29);
}

// ---------------------------------------------------------------- scores

/** search_kernels.cuh:227-251: Lr-lane chunks, then the xor butterfly. */
float sketch_dist(const int8_t* x, const float* sc, const float* qv, int S)
{
  int Lr = 1;
  while (Lr < S / 16 && Lr < 32)
    Lr <<= 1;
  float part[32];
  for (int sub = 0; sub < Lr; sub++) {
    float d = 0.f;
    for (int k = sub * 16; k < S; k += Lr * 16)
      for (int t = 0; t < 16; t++) {
        float u = std::fma(static_cast<float>(x[k + t]), sc[k + t], -qv[k + t]);
        d       = std::fma(u, u, d);
      }
    part[sub] = d;
  }
  for (int o = Lr >> 1; o; o >>= 1) {
    float nx[32];
    for (int i = 0; i < Lr; i++)
      nx[i] = part[i] + part[i ^ o];
    std::memcpy(part, nx, sizeof(float) * Lr);
  }
  return part[0];
}

/**
 * search_kernels.cuh:325-342 with the lane split of the HIP kernel: LX lanes per row (the next power
 * of two >= D / 8, at most 32), lane sub summing the 8-element chunks sub, sub + LX, ... in order with
 * t = x - q, acc = fma(t, t, acc), then the xor butterfly over the LX lanes.
 */
float exact_dist(const uint16_t* x, const float* q, int D)
{
  const int nch = (D + 7) / 8;
  int LX        = 1;
  while (LX < nch && LX < 32)
    LX <<= 1;
  float part[32];
  for (int sub = 0; sub < LX; sub++) {
    float acc = 0.f;
    for (int c = sub; c < nch; c += LX)
      for (int e = 0; e < 8 && 8 * c + e < D; e++) {
        const float t = h2f(x[8 * c + e]) - q[8 * c + e];
        acc           = std::fma(t, t, acc);
      }
    part[sub] = acc;
  }
  for (int o = LX >> 1; o; o >>= 1) {
    float nx[32];
    for (int i = 0; i < LX; i++)
      nx[i] = part[i] + part[i ^ o];
    std::memcpy(part, nx, sizeof(float) * LX);
  }
  return part[0];
}

inline uint64_t dist_key(float d, int64_t id)  // search_kernels.cuh:365-368
{
  return (static_cast<uint64_t>(fbits(d)) << 32) | static_cast<uint32_t>(id);
}
const uint64_t kEmpty = ~0ULL;

// ---------------------------------------------------------------- per-query stages

inline int row_of(const orc_index& ix, int64_t c, int j) { return ix.base[c * ix.levels + j]; }

/** probe_kernel (search_kernels.cuh:84-127) for one (query, copy). */
void probe_one(const orc_index& ix, const uint16_t* yrow, int c, int lr, int32_t* sg)
{
  const int B = ix.blocks, L = ix.levels;
  float y[64];
  for (int i = 0; i < 8 * B; i++)
    y[i] = h2f(yrow[i]);
  sg[0] = 0;
  sg[1] = 0;
  for (int j = 0; j < L; j++) {
    int64_t h       = e8b_hash64(y, B, ix.inv_f[j]);
    int bk          = static_cast<int>(h & ((int64_t{1} << ix.log_buckets) - 1));
    const int32_t* o = ix.offsets + (int64_t{c} * L + j) * ix.T1 + bk;
    const int64_t* kk = ix.keys + (int64_t{c} * L + j) * ix.mmax;
    for (int p = o[0]; p < o[1]; p++)
      if (kk[p] == h) {
        sg[0] = (row_of(ix, c, j) + p) * ix.list_len;
        sg[1] = lr;
        return;
      }
  }
}

/** gather_kernel (search_kernels.cuh:138-253) as a set: distinct ids ascending with sketch scores. */
int gather(const orc_index& ix, const int32_t* seg, int nseg, bool rows, const float* qs,
           std::vector<int32_t>& ids, int32_t* cand, float* dist, int cap)
{
  ids.clear();
  for (int c = 0; c < nseg; c++) {
    int st = seg[2 * c], len = seg[2 * c + 1];
    for (int i = 0; i < len; i++) {
      int v = rows ? ix.table[int64_t{st} * ix.table_len + i] : ix.lists[c * ix.stride + st + i];
      if (v < 0) continue;  // padding of a table row (search_kernels.cuh:213)
      ids.push_back(v);
    }
  }
  std::sort(ids.begin(), ids.end());
  ids.erase(std::unique(ids.begin(), ids.end()), ids.end());
  int n = std::min<int>(static_cast<int>(ids.size()), cap);
  const int S = ix.sketch_width;
  for (int j = 0; j < n; j++) {
    cand[j] = ids[j];
    dist[j] = sketch_dist(ix.sketch + int64_t{ids[j]} * S, ix.scale, qs, S);
  }
  return n;
}

int select_smallest(const int32_t* cand, const float* dist, int n, int R, int32_t* sid, float* sd)
{
  std::vector<uint64_t> k(n);
  for (int i = 0; i < n; i++)
    k[i] = (static_cast<uint64_t>(fbits(dist[i])) << 32) | static_cast<uint32_t>(cand[i]);
  int r = std::min(R, n);
  std::partial_sort(k.begin(), k.begin() + r, k.end());
  for (int i = 0; i < r; i++) {
    sid[i] = static_cast<int32_t>(k[i] & 0xffffffffULL);
    if (sd) sd[i] = bitsf(static_cast<uint32_t>(k[i] >> 32));
  }
  return r;
}

void merge_keep(int64_t* si, float* sd, int KO, bool fresh, const int32_t* nid, const float* nd,
                int nn)
{
  std::vector<uint64_t> key;
  key.reserve(KO + nn);
  if (!fresh)
    for (int i = 0; i < KO; i++)
      if (si[i] >= 0) key.push_back(dist_key(sd[i], si[i]));
  for (int i = 0; i < nn; i++)
    key.push_back(dist_key(nd[i], nid[i]));
  std::sort(key.begin(), key.end());
  int o         = 0;
  uint64_t prev = kEmpty - 1;
  for (size_t i = 0; i < key.size() && o < KO; i++) {
    if (key[i] == prev) continue;
    prev  = key[i];
    si[o] = static_cast<int64_t>(static_cast<uint32_t>(key[i] & 0xffffffffULL));
    sd[o] = bitsf(static_cast<uint32_t>(key[i] >> 32));
    o++;
  }
  for (; o < KO; o++) {
    si[o] = -1;
    sd[o] = INFINITY;
  }
}

void rerank_keep(const orc_index& ix, const int32_t* cand, const float* dist, int n, const float* q,
                 int R, int KO, bool fresh, int64_t* si, float* sd)
{
  std::vector<int32_t> sid(std::max(1, std::min(R, n)));
  std::vector<float> ex(sid.size());
  int ns       = select_smallest(cand, dist, n, R, sid.data(), nullptr);
  const int D  = static_cast<int>(ix.dim);
  for (int j = 0; j < ns; j++)
    ex[j] = exact_dist(ix.vectors + int64_t{sid[j]} * D, q, D);
  merge_keep(si, sd, KO, fresh, sid.data(), ex.data(), ns);
}

void sketch_keep(const int32_t* cand, const float* dist, int n, int KO, bool fresh, int64_t* si,
                 float* sd)
{
  std::vector<int32_t> sid(std::max(1, std::min(KO, n)));
  std::vector<float> sdv(sid.size());
  int ns = select_smallest(cand, dist, n, KO, sid.data(), sdv.data());
  merge_keep(si, sd, KO, fresh, sid.data(), sdv.data(), ns);
}

int pick_starts(const int64_t* si, int KO, int64_t* done, int off, int S, int rowlen, int32_t* seg2)
{
  std::vector<int64_t> prev(done, done + off);
  std::sort(prev.begin(), prev.end());
  int o = 0;
  for (int i = 0; i < KO && o < S; i++) {
    int64_t v = si[i];
    if (v < 0) continue;
    if (std::binary_search(prev.begin(), prev.end(), v)) continue;
    done[off + o]  = v;
    seg2[2 * o]    = static_cast<int32_t>(v);
    seg2[2 * o + 1] = rowlen;
    o++;
  }
  int got = o;
  for (; o < S; o++) {
    done[off + o]   = -1;
    seg2[2 * o]     = 0;
    seg2[2 * o + 1] = 0;
  }
  return got;
}

void final_rerank(const orc_index& ix, const int64_t* si, int R, const float* q, int k, int64_t* bi,
                  float* bd)
{
  const int D = static_cast<int>(ix.dim);
  std::vector<int32_t> sid;
  std::vector<float> ex;
  for (int i = 0; i < R; i++)
    if (si[i] >= 0) {
      sid.push_back(static_cast<int32_t>(si[i]));
      ex.push_back(exact_dist(ix.vectors + si[i] * D, q, D));
    }
  merge_keep(bi, bd, k, true, sid.data(), ex.data(), static_cast<int>(sid.size()));
}

// ---------------------------------------------------------------- projections

void project_rows(const uint16_t* qh, int64_t r0, int64_t r1, int D, const uint16_t* ucat, int wdt,
                  const uint16_t* shift, uint16_t* Y, double* Yd)
{
  std::vector<float> uf(static_cast<size_t>(D) * wdt);
  for (size_t i = 0; i < uf.size(); i++)
    uf[i] = h2f(ucat[i]);
  std::vector<double> acc(wdt);
  for (int64_t q = r0; q < r1; q++) {
    for (int j = 0; j < wdt; j++)
      acc[j] = h2f(shift[j]);
    for (int d = 0; d < D; d++) {
      double a     = h2f(qh[q * D + d]);
      const float* u = uf.data() + static_cast<size_t>(d) * wdt;
      for (int j = 0; j < wdt; j++)
        acc[j] += a * u[j];
    }
    for (int j = 0; j < wdt; j++) {
      Y[q * wdt + j] = d2h(acc[j]);  // one rounding of the fp64 value
      if (Yd) Yd[q * wdt + j] = acc[j];
    }
  }
}

template <typename F>
void parallel_rows(int64_t n, int threads, F&& f)
{
  threads = std::max(1, std::min<int>(threads, static_cast<int>(std::max<int64_t>(n, 1))));
  if (threads == 1) {
    f(0, n, 0);
    return;
  }
  std::vector<std::thread> th;
  for (int t = 0; t < threads; t++)
    th.emplace_back([&, t] { f(n * t / threads, n * (t + 1) / threads, t); });
  for (auto& x : th)
    x.join();
}

// ---------------------------------------------------------------- the search

int log2_ceil(int64_t v)  // search.cu:85-91
{
  int e = 0;
  while ((int64_t{1} << e) < v)
    e++;
  return e;
}

struct searcher {
  const orc_index& ix;
  const orc_search_params& sp;
  int k, KO, lr, W, W2, FR;
  std::vector<int32_t> ids, cand, seg, seg2;
  std::vector<float> dist;
  std::vector<int64_t> done;

  searcher(const orc_index& ix_, const orc_search_params& sp_, int k_)
    : ix(ix_), sp(sp_), k(k_)
  {
    KO = std::max(sp.starts, k);                    // search.cu:626
    lr = std::min(sp.read, ix.list_len);            // search.cu:627
    FR = std::min(sp.final_rerank, KO);             // search.cu:630
    W  = 1 << std::clamp(log2_ceil(static_cast<int64_t>(std::ceil(ix.copies * lr * 1.5f))), 11, 15);
    W2 = 1 << std::clamp(log2_ceil(static_cast<int64_t>(std::ceil(sp.starts * ix.table_len * 1.5f))), 11, 15);
    int cap = std::max(W, W2);
    cand.resize(cap);
    dist.resize(cap);
    seg.resize(2 * ix.copies);
    seg2.resize(2 * std::max(1, sp.starts));
    done.resize(std::max(1, sp.starts * sp.waves));
  }

  /** first_round + wave_round (search.cu:294-518) of one query. */
  void run(const float* q, const uint16_t* yrow, const float* qs, int64_t* I, float* Dout,
           int64_t* si, float* sd, int32_t* tseg, int32_t* n1, int64_t* si1, float* sd1, int32_t* n2)
  {
    const int C = ix.copies;
    for (int c = 0; c < C; c++)
      probe_one(ix, yrow + int64_t{c} * 8 * ix.blocks, c, lr, seg.data() + 2 * c);
    if (tseg) std::memcpy(tseg, seg.data(), sizeof(int32_t) * 2 * C);
    int n = gather(ix, seg.data(), C, false, qs, ids, cand.data(), dist.data(), W);
    if (n1) *n1 = n;
    if (sp.sketch_rank)
      sketch_keep(cand.data(), dist.data(), n, KO, true, si, sd);
    else
      rerank_keep(ix, cand.data(), dist.data(), n, q, sp.rerank, KO, true, si, sd);
    if (si1) std::memcpy(si1, si, sizeof(int64_t) * KO);
    if (sd1) std::memcpy(sd1, sd, sizeof(float) * KO);
    const int S = sp.starts;
    for (int wv = 0; wv < sp.waves; wv++) {
      pick_starts(si, KO, done.data(), wv * S, S, ix.table_len, seg2.data());
      int m2 = gather(ix, seg2.data(), S, true, qs, ids, cand.data(), dist.data(), W2);
      if (n2) n2[wv] = m2;
      if (sp.sketch_rank)
        sketch_keep(cand.data(), dist.data(), m2, KO, false, si, sd);
      else
        rerank_keep(ix, cand.data(), dist.data(), m2, q, sp.wave_rerank, KO, false, si, sd);
    }
    if (sp.sketch_rank && FR > 0) {
      final_rerank(ix, si, FR, q, k, I, Dout);
    } else {
      for (int j = 0; j < k; j++) {  // take_k_kernel (search_kernels.cuh:672-685)
        I[j]    = si[j];
        Dout[j] = sd[j];
      }
    }
  }
};

void check_params(const orc_index& ix, const orc_search_params& sp, int k)
{
  // search.cu:638-656, 681-692
  const int KO = std::max(sp.starts, k);
  auto expect  = [](bool ok, const char* msg) {
    if (!ok) throw std::runtime_error(msg);
  };
  expect(k >= 1, "octex: k >= 1");
  expect(sp.read >= 1 && sp.starts >= 1 && sp.waves >= 0, "octex: read, starts >= 1 and waves >= 0");
  expect(sp.waves == 0 || ix.table_len > 0, "octex: waves need the neighbor table");
  expect(KO <= (sp.sketch_rank ? 1024 : 512),
         "octex: max(starts, k) must be <= 512 (1024 with sketch_rank)");
  expect(sp.sketch_rank || (sp.rerank >= 1 && sp.rerank <= 512 && KO + sp.rerank <= 1024),
         "octex: rerank in [1, 512] and max(starts, k) + rerank <= 1024");
  expect(sp.sketch_rank || sp.waves == 0 ||
           (sp.wave_rerank >= 1 && sp.wave_rerank <= 512 && KO + sp.wave_rerank <= 1024),
         "octex: wave_rerank in [1, 512] and max(starts, k) + wave_rerank <= 1024");
  const int FR = std::min(sp.final_rerank, KO);
  expect(!sp.sketch_rank || FR == 0 || (k <= FR && FR <= 512),
         "octex: final_rerank 0 (sketch order) or k <= final_rerank <= 512");
  expect(sp.waves <= 1 || sp.starts * (sp.waves - 1) <= 6144, "octex: starts * (waves - 1) <= 6144");
  const int lr = std::min(sp.read, ix.list_len);
  expect(int64_t{ix.copies} * lr <= 32768,
         "octex: copies x read too large for the shared-memory hash set");
  expect(sp.waves == 0 || int64_t{sp.starts} * ix.table_len <= 32768,
         "octex: starts x table_len too large for the shared-memory hash set");
}

// ---------------------------------------------------------------- npy / builder helpers

template <typename T>
const char* descr();
template <>
const char* descr<float>() { return "<f4"; }
template <>
const char* descr<int8_t>() { return "|i1"; }
template <>
const char* descr<int32_t>() { return "<i4"; }
template <>
const char* descr<int64_t>() { return "<i8"; }
template <>
const char* descr<uint16_t>() { return "<f2"; }

/** .npy format 1.0 writer (the header layout numpy itself writes). */
template <typename T>
void write_npy(const std::string& path, const T* data, std::vector<int64_t> const& shape)
{
  std::string sh = "(";
  int64_t n      = 1;
  for (size_t i = 0; i < shape.size(); i++) {
    sh += std::to_string(shape[i]);
    if (shape.size() == 1 || i + 1 < shape.size()) sh += ",";
    if (i + 1 < shape.size()) sh += " ";
    n *= shape[i];
  }
  sh += ")";
  std::string hdr = std::string("{'descr': '") + descr<T>() + "', 'fortran_order': False, 'shape': " + sh + ", }";
  size_t total = 10 + hdr.size() + 1;
  hdr.append((64 - total % 64) % 64, ' ');
  hdr += '\n';
  std::ofstream f(path, std::ios::binary);
  if (!f) throw std::runtime_error("octex: cannot write " + path);
  f.write("\x93NUMPY\x01\x00", 8);
  uint16_t hl = static_cast<uint16_t>(hdr.size());
  f.write(reinterpret_cast<const char*>(&hl), 2);
  f.write(hdr.data(), static_cast<std::streamsize>(hdr.size()));
  f.write(reinterpret_cast<const char*>(data), static_cast<std::streamsize>(n * sizeof(T)));
}

uint64_t splitmix64(uint64_t z)  // build_setup.cuh:105-111
{
  z += 0x9E3779B97F4A7C15ULL;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

/** Symmetric eigen decomposition by cyclic Jacobi: values descending, vectors as columns of V [d, d]. */
void jacobi_eig(std::vector<double>& A, int d, std::vector<double>& vals, std::vector<double>& V)
{
  V.assign(static_cast<size_t>(d) * d, 0.0);
  for (int i = 0; i < d; i++)
    V[static_cast<size_t>(i) * d + i] = 1.0;
  for (int sweep = 0; sweep < 100; sweep++) {
    double off = 0, diag = 0;
    for (int i = 0; i < d; i++)
      for (int j = 0; j < d; j++)
        (i == j ? diag : off) += A[static_cast<size_t>(i) * d + j] * A[static_cast<size_t>(i) * d + j];
    if (off <= 1e-30 * std::max(diag, 1e-300)) break;
    for (int p = 0; p < d; p++)
      for (int q = p + 1; q < d; q++) {
        double apq = A[static_cast<size_t>(p) * d + q];
        if (std::fabs(apq) < 1e-300) continue;
        double app = A[static_cast<size_t>(p) * d + p], aqq = A[static_cast<size_t>(q) * d + q];
        double theta = (aqq - app) / (2 * apq);
        double t = (theta >= 0 ? 1.0 : -1.0) / (std::fabs(theta) + std::sqrt(theta * theta + 1));
        double c = 1 / std::sqrt(t * t + 1), s = t * c;
        for (int r = 0; r < d; r++) {
          double arp = A[static_cast<size_t>(r) * d + p], arq = A[static_cast<size_t>(r) * d + q];
          A[static_cast<size_t>(r) * d + p] = c * arp - s * arq;
          A[static_cast<size_t>(r) * d + q] = s * arp + c * arq;
        }
        for (int r = 0; r < d; r++) {
          double apr = A[static_cast<size_t>(p) * d + r], aqr = A[static_cast<size_t>(q) * d + r];
          A[static_cast<size_t>(p) * d + r] = c * apr - s * aqr;
          A[static_cast<size_t>(q) * d + r] = s * apr + c * aqr;
        }
        for (int r = 0; r < d; r++) {
          double vrp = V[static_cast<size_t>(r) * d + p], vrq = V[static_cast<size_t>(r) * d + q];
          V[static_cast<size_t>(r) * d + p] = c * vrp - s * vrq;
          V[static_cast<size_t>(r) * d + q] = s * vrp + c * vrq;
        }
      }
  }
  std::vector<int> order(d);
  std::iota(order.begin(), order.end(), 0);
  std::sort(order.begin(), order.end(), [&](int a, int b) {
    return A[static_cast<size_t>(a) * d + a] > A[static_cast<size_t>(b) * d + b];
  });
  std::vector<double> V2(static_cast<size_t>(d) * d);
  vals.resize(d);
  for (int k = 0; k < d; k++) {
    vals[k] = A[static_cast<size_t>(order[k]) * d + order[k]];
    for (int r = 0; r < d; r++)
      V2[static_cast<size_t>(r) * d + k] = V[static_cast<size_t>(r) * d + order[k]];
  }
  V.swap(V2);
}

/** Shortest text that reads back as the same float (build.cu:39-46). */
std::string json_float(float v)
{
  char b[64];
  auto r = std::to_chars(b, b + sizeof(b), v);
  std::string s(b, r.ptr);
  if (s.find_first_of(".en") == std::string::npos) s += ".0";
  return s;
}

}  // namespace

// ==================================================================== C interface

extern "C" {

uint16_t orc_f2h(float f) { return f2h(f); }
float orc_h2f(uint16_t h) { return h2f(h); }
void orc_f2h_n(const float* x, int64_t n, uint16_t* out)
{
  for (int64_t i = 0; i < n; i++)
    out[i] = f2h(x[i]);
}
void orc_h2f_n(const uint16_t* x, int64_t n, float* out)
{
  for (int64_t i = 0; i < n; i++)
    out[i] = h2f(x[i]);
}

void orc_e8_point(const float* x, float* p) { e8_point(x, p); }
int64_t orc_e8b_hash64(const float* y, int b, float inv_f) { return e8b_hash64(y, b, inv_f); }

void orc_e8_batch(const float* y, int64_t n, int b, float inv_f, float* p, int64_t* h)
{
  for (int64_t i = 0; i < n; i++) {
    for (int j = 0; j < b; j++) {
      float x[8];
      for (int k = 0; k < 8; k++)
        x[k] = y[i * 8 * b + 8 * j + k] * inv_f;
      e8_point(x, p + i * 8 * b + 8 * j);
    }
    h[i] = e8b_hash64(y + i * 8 * b, b, inv_f);
  }
}

void orc_center(const float* q, const float* mu, int64_t m, int D, float* qc, uint16_t* qh)
{
  for (int64_t t = 0; t < m * D; t++) {  // search_kernels.cuh:57-69
    float v = q[t] - mu[t % D];
    qc[t]   = v;
    qh[t]   = f2h(v);
  }
}

void orc_project(const uint16_t* qh, int64_t m, int D, const uint16_t* ucat, int wdt,
                 const uint16_t* shift, uint16_t* Y, double* Yd)
{
  project_rows(qh, 0, m, D, ucat, wdt, shift, Y, Yd);
}

void orc_sketch_query(const float* qc, int64_t m, int D, const float* basis, int S, float* qs)
{
  for (int64_t q = 0; q < m; q++)
    for (int s = 0; s < S; s++) {
      double acc = 0;
      for (int d = 0; d < D; d++)
        acc += double(qc[q * D + d]) * double(basis[int64_t{d} * S + s]);
      qs[q * S + s] = static_cast<float>(acc);
    }
}

void orc_probe(const orc_index* ix, const uint16_t* Y, int64_t m, int lr, int32_t* seg)
{
  const int C = ix->copies, w = 8 * ix->blocks;
  for (int64_t q = 0; q < m; q++)
    for (int c = 0; c < C; c++)
      probe_one(*ix, Y + (q * C + c) * w, c, lr, seg + 2 * (q * C + c));
}

int orc_gather(const orc_index* ix, const int32_t* seg, int nseg, int rows, const float* qs,
               int32_t* cand, float* dist, int cap)
{
  std::vector<int32_t> ids;
  return gather(*ix, seg, nseg, rows != 0, qs, ids, cand, dist, cap);
}

float orc_sketch_dist(const int8_t* code, const float* scale, const float* qs, int S)
{
  return sketch_dist(code, scale, qs, S);
}

float orc_exact_dist(const uint16_t* x, const float* q, int D) { return exact_dist(x, q, D); }

int orc_select(const int32_t* cand, const float* dist, int n, int R, int32_t* sid, float* sd)
{
  return select_smallest(cand, dist, n, R, sid, sd);
}

void orc_merge_keep(int64_t* si, float* sd, int KO, int fresh, const int32_t* nid, const float* nd,
                    int nn)
{
  merge_keep(si, sd, KO, fresh != 0, nid, nd, nn);
}

void orc_rerank_keep(const orc_index* ix, const int32_t* cand, const float* dist, int n,
                     const float* q, int R, int KO, int fresh, int64_t* si, float* sd)
{
  rerank_keep(*ix, cand, dist, n, q, R, KO, fresh != 0, si, sd);
}

void orc_sketch_keep(const int32_t* cand, const float* dist, int n, int KO, int fresh, int64_t* si,
                     float* sd)
{
  sketch_keep(cand, dist, n, KO, fresh != 0, si, sd);
}

int orc_pick_starts(const int64_t* si, int KO, int64_t* done, int off, int S, int rowlen,
                    int32_t* seg2)
{
  return pick_starts(si, KO, done, off, S, rowlen, seg2);
}

void orc_final_rerank(const orc_index* ix, const int64_t* si, int R, const float* q, int k,
                      int64_t* bi, float* bd)
{
  final_rerank(*ix, si, R, q, k, bi, bd);
}

const char* orc_last_error(void) { return g_err.c_str(); }

int orc_search(const orc_index* ix, const orc_search_params* sp, const float* q, int64_t nq, int k,
               const uint16_t* Y, const float* qs, int64_t* I, float* D, int threads,
               const orc_trace* trace)
{
  try {
    if (k < 1) throw std::runtime_error("octex: k >= 1");
    check_params(*ix, *sp, k);
    if (nq == 0) return 0;
    const int Dm = static_cast<int>(ix->dim), C = ix->copies, w = 8 * ix->blocks, S = ix->sketch_width;
    const int KO = std::max(sp->starts, k);
    std::vector<std::string> errs(std::max(1, threads));
    parallel_rows(nq, threads, [&](int64_t r0, int64_t r1, int t) {
      try {
        searcher s(*ix, *sp, k);
        std::vector<float> qc(Dm), qsb(S);
        std::vector<uint16_t> qh(Dm), yb(static_cast<size_t>(C) * w);
        std::vector<int64_t> si(KO);
        std::vector<float> sd(KO);
        for (int64_t r = r0; r < r1; r++) {
          const float* qr = q + r * Dm;
          const uint16_t* yrow;
          const float* qsr;
          if (Y == nullptr || qs == nullptr) orc_center(qr, ix->mean, 1, Dm, qc.data(), qh.data());
          if (Y) {
            yrow = Y + r * C * w;
          } else {
            project_rows(qh.data(), 0, 1, Dm, ix->ucat, C * w, ix->shift, yb.data(), nullptr);
            yrow = yb.data();
          }
          if (qs) {
            qsr = qs + r * S;
          } else {
            orc_sketch_query(qc.data(), 1, Dm, ix->basis, S, qsb.data());
            qsr = qsb.data();
          }
          const orc_trace* tr = trace;
          s.run(qr, yrow, qsr, I + r * k, D + r * k, si.data(), sd.data(),
                tr && tr->seg ? tr->seg + r * 2 * C : nullptr, tr && tr->n1 ? tr->n1 + r : nullptr,
                tr && tr->si1 ? tr->si1 + r * KO : nullptr, tr && tr->sd1 ? tr->sd1 + r * KO : nullptr,
                tr && tr->n2 ? tr->n2 + r * std::max(1, sp->waves) : nullptr);
          if (tr && tr->si) std::memcpy(tr->si + r * KO, si.data(), sizeof(int64_t) * KO);
          if (tr && tr->sd) std::memcpy(tr->sd + r * KO, sd.data(), sizeof(float) * KO);
        }
      } catch (std::exception const& e) {
        errs[t] = e.what();
      }
    });
    for (auto& e : errs)
      if (!e.empty()) throw std::runtime_error(e);
    return 0;
  } catch (std::exception const& e) {
    g_err = e.what();
    return -1;
  }
}

void orc_bruteforce(const float* x, int64_t n, const float* q, int64_t m, int64_t d, int k,
                    int64_t* I, float* D, int threads)
{
  // blocks of kQ queries share each pass over the rows, their fp64 sums four to an AVX register (a multiply, then
  // an add: the same roundings as one query at a time); every query keeps its k smallest (distance, id) pairs in a
  // max-heap, which holds what a partial sort of all n pairs puts first (the pairs are distinct by id)
  constexpr int kQ     = 16;
  const int kk         = static_cast<int>(std::min<int64_t>(k, n));
  const int64_t blocks = (m + kQ - 1) / kQ;
  parallel_rows(blocks, threads, [&](int64_t b0, int64_t b1, int) {
    std::vector<std::pair<double, int64_t>> best[kQ];
    std::vector<double> qb(static_cast<size_t>(d) * kQ);  // [d][kQ]
    alignas(32) double acc[kQ];
    for (int64_t bq = b0; bq < b1; bq++) {
      const int64_t r0 = bq * kQ;
      const int nr     = static_cast<int>(std::min<int64_t>(kQ, m - r0));
      for (int t = 0; t < kQ; t++) {
        const float* qt = q + (r0 + std::min(t, nr - 1)) * d;
        for (int64_t j = 0; j < d; j++)
          qb[j * kQ + t] = double(qt[j]);
        best[t].clear();
      }
      for (int64_t i = 0; i < n; i++) {
        const float* xi = x + i * d;
        __m256d a0 = _mm256_setzero_pd(), a1 = _mm256_setzero_pd();
        __m256d a2 = _mm256_setzero_pd(), a3 = _mm256_setzero_pd();
        for (int64_t j = 0; j < d; j++) {
          const __m256d xj = _mm256_set1_pd(double(xi[j]));
          const double* qj = qb.data() + j * kQ;
          const __m256d u0 = _mm256_sub_pd(xj, _mm256_loadu_pd(qj));
          const __m256d u1 = _mm256_sub_pd(xj, _mm256_loadu_pd(qj + 4));
          const __m256d u2 = _mm256_sub_pd(xj, _mm256_loadu_pd(qj + 8));
          const __m256d u3 = _mm256_sub_pd(xj, _mm256_loadu_pd(qj + 12));
          a0 = _mm256_add_pd(a0, _mm256_mul_pd(u0, u0));
          a1 = _mm256_add_pd(a1, _mm256_mul_pd(u1, u1));
          a2 = _mm256_add_pd(a2, _mm256_mul_pd(u2, u2));
          a3 = _mm256_add_pd(a3, _mm256_mul_pd(u3, u3));
        }
        _mm256_store_pd(acc, a0);
        _mm256_store_pd(acc + 4, a1);
        _mm256_store_pd(acc + 8, a2);
        _mm256_store_pd(acc + 12, a3);
        for (int t = 0; t < nr; t++) {
          auto& h = best[t];
          const std::pair<double, int64_t> e{acc[t], i};
          if (static_cast<int>(h.size()) < kk) {
            h.push_back(e);
            std::push_heap(h.begin(), h.end());
          } else if (kk > 0 && e < h.front()) {
            std::pop_heap(h.begin(), h.end());
            h.back() = e;
            std::push_heap(h.begin(), h.end());
          }
        }
      }
      for (int t = 0; t < nr; t++) {
        auto& h = best[t];
        std::sort_heap(h.begin(), h.end());
        const int64_t r = r0 + t;
        for (int j = 0; j < k; j++) {
          I[r * k + j] = j < kk ? h[j].second : -1;
          D[r * k + j] = j < kk ? static_cast<float>(h[j].first) : INFINITY;
        }
      }
    }
  });
}

/*
 * The small builder (build.cu:104-426; build_setup.cuh:40-175; build_cells.cuh:61-613;
 * build_table.cuh:157-554), its copies and table rows over host threads, for test indexes and the host build of
 * the 100k-row CPU workload.
 * Lists: exact (brute force in the projection) or from cell members (build_cells.cuh:176-250); the
 * reference's IVF-Flat default is approximate, exact lists stand in for it here.
 */
int orc_build(const float* xin, int64_t n, int64_t d, const orc_build_params* p, const char* path)
{
  try {
    const int C = p->copies, b = p->blocks, w = 8 * b, l = p->list_len;
    std::vector<float> spac(p->spacings, p->spacings + p->n_spacings);
    if (spac.empty()) spac = {2.0f, 2.5f, 3.2f, 4.0f, 5.0f};
    const int L     = static_cast<int>(spac.size());
    const int64_t T = int64_t{1} << p->log_buckets;
    const int S     = p->sketch_width > 0
                        ? static_cast<int>(std::min<int64_t>(p->sketch_width, d))
                        : static_cast<int>(std::max<int64_t>(std::min<int64_t>(d / 16 * 16, 128),
                                                         std::min<int64_t>(d, 16)));
    const int k = p->table_len;
    if (n < l || n < 2) throw std::runtime_error("octex: fewer vectors than the list length");
    mkdir(path, 0755);
    std::string dir(path);
    auto file = [&](const char* name) { return dir + "/" + name; };
    // the index is built from (and reranks with) the fp16 vectors (build.cu:434-441)
    std::vector<uint16_t> xh(static_cast<size_t>(n) * d);
    std::vector<float> x(xh.size());
    for (size_t i = 0; i < xh.size(); i++) {
      xh[i] = f2h(xin[i]);
      x[i]  = h2f(xh[i]);
    }
    // PCA of every max(1, n / 200000)-th row (build_setup.cuh:40-103)
    int64_t step = std::max<int64_t>(1, n / 200000), ns = (n + step - 1) / step;
    std::vector<double> mu(d, 0.0);
    for (int64_t i = 0; i < ns; i++)
      for (int64_t j = 0; j < d; j++)
        mu[j] += x[i * step * d + j];
    std::vector<float> mean(d);
    for (int64_t j = 0; j < d; j++)
      mean[j] = static_cast<float>(mu[j] / double(ns));
    std::vector<double> G(static_cast<size_t>(d) * d, 0.0);
    for (int64_t i = 0; i < ns; i++)
      for (int64_t a = 0; a < d; a++) {
        double va = double(x[i * step * d + a] - mean[a]);
        for (int64_t c2 = 0; c2 < d; c2++)
          G[a * d + c2] += va * double(x[i * step * d + c2] - mean[c2]);
      }
    std::vector<double> vals, V;
    jacobi_eig(G, static_cast<int>(d), vals, V);
    // projections and shifts (build_setup.cuh:119-175)
    int pd = std::min<int>(p->pca_dims, static_cast<int>(d));
    if (pd < w) throw std::runtime_error("octex: pca_dims must be at least 8 * blocks");
    std::vector<float> proj(static_cast<size_t>(C) * d * w), shift(static_cast<size_t>(C) * w);
    std::vector<double> qm(static_cast<size_t>(pd) * w);
    for (int c = 0; c < C; c++) {
      std::mt19937_64 gen(splitmix64(p->seed * 0x100000001B3ULL + uint64_t(c)));
      std::normal_distribution<double> normal(0.0, 1.0);
      std::uniform_real_distribution<double> uni(0.0, 2.0);
      for (auto& v : qm)
        v = normal(gen);
      for (int s = 0; s < w; s++) {
        for (int t = 0; t < s; t++) {
          double dot = 0;
          for (int r = 0; r < pd; r++)
            dot += qm[r * w + s] * qm[r * w + t];
          for (int r = 0; r < pd; r++)
            qm[r * w + s] -= dot * qm[r * w + t];
        }
        double nrm = 0;
        for (int r = 0; r < pd; r++)
          nrm += qm[r * w + s] * qm[r * w + s];
        nrm = std::sqrt(nrm);
        for (int r = 0; r < pd; r++)
          qm[r * w + s] /= nrm;
      }
      double sd = 0;
      for (int s = 0; s < w; s++) {
        double v = 0;
        for (int r = 0; r < pd; r++)
          v += vals[r] * qm[r * w + s] * qm[r * w + s];
        sd += std::sqrt(v / double(std::max<int64_t>(ns - 1, 1)));
      }
      sd /= w;
      for (int64_t kk = 0; kk < d; kk++)
        for (int s = 0; s < w; s++) {
          double v = 0;
          for (int r = 0; r < pd; r++)
            v += double(static_cast<float>(V[kk * d + r])) * qm[r * w + s];
          proj[(static_cast<size_t>(c) * d + kk) * w + s] = static_cast<float>(v / sd);
        }
      for (int s = 0; s < w; s++)
        shift[static_cast<size_t>(c) * w + s] = static_cast<float>(uni(gen));
    }
    // cells of every copy (build_cells.cuh:451-613, finish_level :387-448)
    std::vector<std::vector<int32_t>> lists(C);
    std::vector<std::vector<int64_t>> keys(C);
    std::vector<std::vector<int32_t>> offs(C);
    std::vector<int32_t> base(static_cast<size_t>(C) * L);
    std::vector<int64_t> ncells(static_cast<size_t>(C) * L);
    // the copies are independent (each writes its own lists, keys, offsets, bases and counts): threads take
    // contiguous ranges of them, and the files are the same for any thread count
    const int nth = std::max(1, p->threads);
    std::vector<std::exception_ptr> fail(nth);
    parallel_rows(C, nth, [&](int64_t c0, int64_t c1, int th) {
      try {
        std::vector<float> y(static_cast<size_t>(n) * w);
        std::vector<float> xc(d);
        for (int c = static_cast<int>(c0); c < c1; c++) {
          const float* u = proj.data() + static_cast<size_t>(c) * d * w;
          for (int64_t i = 0; i < n; i++) {
            for (int64_t j = 0; j < d; j++)
              xc[j] = x[i * d + j] - mean[j];
            for (int s = 0; s < w; s++) {
              float acc = 0.f;
              for (int64_t j = 0; j < d; j++)
                acc = std::fma(xc[j], u[j * w + s], acc);
              y[i * w + s] = acc + shift[static_cast<size_t>(c) * w + s];
            }
          }
          int64_t row = 0;
          offs[c].assign(static_cast<size_t>(L) * (T + 1), 0);
          for (int j = 0; j < L; j++) {
            const float f = spac[j];
            std::vector<std::pair<int64_t, int32_t>> hv(n);
            std::vector<float> yf(w);
            for (int64_t i = 0; i < n; i++) {
              for (int s = 0; s < w; s++)
                yf[s] = y[i * w + s] / f;  // division, as build_cells.cuh:69-71
              hv[i] = {e8b_hash64(yf.data(), b, 1.0f), static_cast<int32_t>(i)};
            }
            std::sort(hv.begin(), hv.end());
            struct cell {
              int64_t key;
              int32_t start, pop;
            };
            std::vector<cell> cells;
            for (int64_t i = 0; i < n;) {
              int64_t e = i;
              while (e < n && hv[e].first == hv[i].first)
                e++;
              int32_t pop = static_cast<int32_t>(e - i);
              if (!(p->min_cell > 1 && j < L - 1 && pop < p->min_cell))
                cells.push_back({hv[i].first, static_cast<int32_t>(i), pop});
              i = e;
            }
            const int64_t M = static_cast<int64_t>(cells.size());
            std::vector<int32_t> lst(static_cast<size_t>(M) * l);
            std::vector<float> z(w);
            std::vector<std::pair<float, int32_t>> cand;
            for (int64_t ci = 0; ci < M; ci++) {
              // center: f times the E8 point of the first member / f (build_cells.cuh:86-103)
              const float* r0 = y.data() + int64_t{hv[cells[ci].start].second} * w;
              for (int jb = 0; jb < b; jb++) {
                float xx[8], pp[8];
                for (int kk = 0; kk < 8; kk++)
                  xx[kk] = r0[8 * jb + kk] / f;
                e8_point(xx, pp);
                for (int kk = 0; kk < 8; kk++)
                  z[8 * jb + kk] = pp[kk] * f;
              }
              cand.clear();
              auto dist_to = [&](int32_t r) {
                float dd = 0.f;
                for (int s = 0; s < w; s++) {
                  float e = y[int64_t{r} * w + s] - z[s];
                  dd      = std::fma(e, e, dd);
                }
                return dd;
              };
              if (p->member_lists || !p->exact_lists) {
                for (int32_t t = 0; t < cells[ci].pop; t++) {
                  int32_t r = hv[cells[ci].start + t].second;
                  cand.push_back({dist_to(r), r});
                }
              } else {
                for (int32_t r = 0; r < n; r++)
                  cand.push_back({dist_to(r), r});
              }
              int kk = std::min<int>(l, static_cast<int>(cand.size()));
              std::partial_sort(cand.begin(), cand.begin() + kk, cand.end());
              for (int t = 0; t < l; t++)  // fewer than l members: the nearest repeats (octex.hpp:62-68)
                lst[ci * l + t] = cand[t < kk ? t : 0].second;
            }
            // (bucket, hash) order, CSR over buckets (build_cells.cuh:387-448)
            std::vector<int64_t> order(M);
            std::iota(order.begin(), order.end(), 0);
            std::stable_sort(order.begin(), order.end(), [&](int64_t a2, int64_t b2) {
              return (cells[a2].key & (T - 1)) < (cells[b2].key & (T - 1));
            });
            int32_t* o = offs[c].data() + static_cast<size_t>(j) * (T + 1);
            std::vector<int64_t> cnt(T + 1, 0);
            for (int64_t ci = 0; ci < M; ci++) {
              keys[c].push_back(cells[order[ci]].key);
              for (int t = 0; t < l; t++)
                lists[c].push_back(lst[order[ci] * l + t]);
              cnt[(cells[order[ci]].key & (T - 1)) + 1]++;
            }
            for (int64_t t = 0; t < T; t++)
              cnt[t + 1] += cnt[t];
            for (int64_t t = 0; t <= T; t++)
              o[t] = static_cast<int32_t>(cnt[t]);
            base[static_cast<size_t>(c) * L + j]   = static_cast<int32_t>(row);
            ncells[static_cast<size_t>(c) * L + j] = M;
            row += M;
          }
        }
      } catch (...) {
        fail[th] = std::current_exception();
      }
    });
    for (auto& e : fail)
      if (e) std::rethrow_exception(e);
    int64_t lmax = 0, mmax = 0;
    for (int c = 0; c < C; c++) {
      lmax = std::max<int64_t>(lmax, lists[c].size());
      for (int j = 0; j < L; j++)
        mmax = std::max(mmax, ncells[static_cast<size_t>(c) * L + j]);
    }
    std::vector<int32_t> lall(static_cast<size_t>(C) * lmax, 0);
    std::vector<int64_t> kall(static_cast<size_t>(C) * L * mmax, 0);
    std::vector<int32_t> oall(static_cast<size_t>(C) * L * (T + 1));
    for (int c = 0; c < C; c++) {
      std::copy(lists[c].begin(), lists[c].end(), lall.begin() + static_cast<size_t>(c) * lmax);
      int64_t at = 0;
      for (int j = 0; j < L; j++) {
        int64_t M = ncells[static_cast<size_t>(c) * L + j];
        std::copy(keys[c].begin() + at, keys[c].begin() + at + M,
                  kall.begin() + (static_cast<size_t>(c) * L + j) * mmax);
        at += M;
      }
      std::copy(offs[c].begin(), offs[c].end(), oall.begin() + static_cast<size_t>(c) * L * (T + 1));
    }
    write_npy(file("mean.npy"), mean.data(), {d});
    write_npy(file("proj.npy"), proj.data(), {C, d, w});
    write_npy(file("shift.npy"), shift.data(), {C, w});
    write_npy(file("base.npy"), base.data(), {C, L});
    write_npy(file("cells.npy"), ncells.data(), {C, L});
    write_npy(file("keys.npy"), kall.data(), {C, L, mmax});
    write_npy(file("offsets.npy"), oall.data(), {C, L, T + 1});
    write_npy(file("lists.npy"), lall.data(), {C, lmax});
    // sketch (build.cu:286-305; build_setup.cuh:177-264)
    std::vector<float> basis(static_cast<size_t>(d) * S);
    for (int64_t r = 0; r < d; r++)
      for (int s = 0; s < S; s++)
        basis[r * S + s] = static_cast<float>(V[r * d + s]);
    std::vector<float> v(static_cast<size_t>(n) * S);
    std::vector<float> scale(S, 0.f);
    for (int64_t i = 0; i < n; i++)
      for (int s = 0; s < S; s++) {
        float acc = 0.f;
        for (int64_t j = 0; j < d; j++)
          acc = std::fma(x[i * d + j] - mean[j], basis[j * S + s], acc);
        v[i * S + s] = acc;
        scale[s]     = std::max(scale[s], std::fabs(acc));
      }
    for (int s = 0; s < S; s++)
      scale[s] = scale[s] > 0.f ? scale[s] / 127.f : 1.f;
    std::vector<int8_t> codes(static_cast<size_t>(n) * S);
    for (int64_t i = 0; i < n; i++)
      for (int s = 0; s < S; s++) {
        float qv       = std::nearbyint(v[i * S + s] / scale[s]);
        codes[i * S + s] = static_cast<int8_t>(std::fmin(127.f, std::fmax(-127.f, qv)));
      }
    write_npy(file("sketch_basis.npy"), basis.data(), {d, int64_t{S}});
    write_npy(file("sketch_scale.npy"), scale.data(), {int64_t{S}});
    write_npy(file("sketch.npy"), codes.data(), {n, int64_t{S}});
    write_npy(file("vectors.npy"), xh.data(), {n, d});
    // exact neighbor table, reverse edges by the half rule (build_table.cuh:529-554, 166-253)
    if (k > 0) {
      if (k >= n) throw std::runtime_error("octex: table_len must be in [1, n)");
      std::vector<int32_t> fid(static_cast<size_t>(n) * k);
      std::vector<float> fd(static_cast<size_t>(n) * k);
      std::vector<int64_t> I(static_cast<size_t>(n) * (k + 1));
      std::vector<float> Dd(static_cast<size_t>(n) * (k + 1));
      orc_bruteforce(x.data(), n, x.data(), n, d, k + 1, I.data(), Dd.data(), nth);
      for (int64_t i = 0; i < n; i++) {  // drop_self_kernel (build_table.cuh:60-74)
        int t = 0;
        for (int j = 0; j <= k && t < k; j++) {
          int64_t vv = I[i * (k + 1) + j];
          if (vv == i) continue;
          fid[i * k + t] = vv < 0 ? -1 : static_cast<int32_t>(vv);
          fd[i * k + t]  = vv < 0 ? INFINITY : std::max(Dd[i * (k + 1) + j], 0.f);
          t++;
        }
      }
      std::vector<int32_t> table(static_cast<size_t>(n) * k);
      if (!p->reverse_edges) {
        table = fid;
      } else {
        const int h = std::max(1, k / 2), kin = k, kf = h, ks = h, kr = h, kout = k;
        // reverse entries of row u: (rank, v) for v listing u at rank < ks, sorted by (rank, v)
        std::vector<std::vector<std::pair<int, int32_t>>> rev(n);
        for (int64_t vv = 0; vv < n; vv++)
          for (int r = 0; r < ks; r++) {
            int32_t u = fid[vv * kin + r];
            if (u >= 0 && u != vv) rev[u].push_back({r, static_cast<int32_t>(vv)});
          }
        for (int64_t u = 0; u < n; u++) {
          auto& rv = rev[u];
          std::sort(rv.begin(), rv.end());
          // candidates in priority order with their distances (merge_rows_kernel :166-252)
          std::vector<std::pair<int32_t, float>> pri;
          for (int t = 0; t < kf; t++)
            pri.push_back({fid[u * kin + t], fd[u * kin + t]});
          for (int t = 0; t < kr; t++)
            if (t < static_cast<int>(rv.size())) {
              int32_t vv = rv[t].second;
              // the distance of a reverse entry is the forward distance of v's row at that rank
              pri.push_back({vv, fd[int64_t{vv} * kin + rv[t].first]});
            } else {
              pri.push_back({-1, 0.f});
            }
          for (int t = kf; t < kin; t++)
            pri.push_back({fid[u * kin + t], fd[u * kin + t]});
          std::vector<std::pair<int32_t, float>> kept;
          for (auto& e : pri) {
            if (e.first < 0 || e.first == u) continue;
            bool dup = false;
            for (auto& q2 : kept)
              dup |= q2.first == e.first;
            if (!dup) kept.push_back(e);
          }
          if (static_cast<int>(kept.size()) > kout) kept.resize(kout);
          std::vector<std::pair<uint32_t, int32_t>> byd;
          for (auto& e : kept)
            byd.push_back({fbits(std::max(e.second, 0.f)), e.first});
          std::sort(byd.begin(), byd.end());
          for (int t = 0; t < kout; t++)
            table[u * kout + t] = t < static_cast<int>(byd.size()) ? byd[t].second : -1;
        }
      }
      write_npy(file("table.npy"), table.data(), {n, int64_t{k}});
    }
    // meta.json last (build.cu:67-98, 423-424)
    std::ostringstream m;
    m << "{\n \"format\": 1,\n \"n\": " << n << ",\n \"dim\": " << d << ",\n \"copies\": " << C
      << ",\n \"blocks\": " << b << ",\n \"spacings\": [";
    for (int j = 0; j < L; j++)
      m << (j ? ", " : "") << json_float(spac[j]);
    m << "],\n \"list_len\": " << l << ",\n \"log_buckets\": " << p->log_buckets
      << ",\n \"sketch_width\": " << S << ",\n \"table_len\": " << k
      << ",\n \"metric\": \"sqeuclidean\",\n \"files\": {}\n}\n";
    std::ofstream(file("meta.json")) << m.str();
    return 0;
  } catch (std::exception const& e) {
    g_err = e.what();
    return -1;
  }
}

}  // extern "C"
