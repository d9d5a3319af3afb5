// octex::build on one MI355X (the reference: build.cu:104-454, build_setup.cuh:40-175,
// build_cells.cuh:451-613, build_table.cuh:557-843).  The index is built in HBM:
//   - PCA of every max(1, n / 200000)-th row: fp64 scatter matrix on the GPU, cyclic Jacobi on the host;
//   - per copy the seeded rotation of the top pca_dims directions (the reference's generator scheme),
//     then per spacing the cells (GPU sort of the cell ids) and their member lists;
//   - the int8 sketch of the top sketch_width directions;
//   - the neighbor table searched by this library's own search over every base vector (first round,
//     then 2 and 3 waves over the previous table), with reverse edges merged on the host.
// build() writes the format-1 directory; build_and_load() keeps the index in HBM as well.

#include "build_kernels.hpp"
#include "build.hpp"
#include "common.hpp"
#include "directory.hpp"
#include "index_impl.hpp"
#include "meta.hpp"
#include "npy.hpp"
#include "search.hpp"

#include <hip/hip_fp16.h>

#include <algorithm>
#include <atomic>
#include <exception>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <memory>
#include <numeric>
#include <random>
#include <sstream>
#include <thread>

namespace cuvs::neighbors::octex {

namespace detail {

namespace {

auto seconds_since(std::chrono::steady_clock::time_point t) -> double
{
  return std::chrono::duration<double>(std::chrono::steady_clock::now() - t).count();
}

void build_log(const char* fmt, ...)
{
  static const bool on = std::getenv("OCTEX_VERBOSE") != nullptr;
  if (!on) return;
  va_list ap;
  va_start(ap, fmt);
  std::vfprintf(stderr, fmt, ap);
  va_end(ap);
}

template <typename F>
void parallel_for(int64_t n, F&& f)
{
  const int threads = static_cast<int>(std::clamp<int64_t>(n / 4096, 1, 16));
  if (threads == 1) {
    f(0, n);
    return;
  }
  std::vector<std::thread> th;
  for (int t = 0; t < threads; t++)
    th.emplace_back([&, t] { f(n * t / threads, n * (t + 1) / threads); });
  for (auto& x : th)
    x.join();
}

/** Symmetric eigen decomposition by cyclic Jacobi rotations: values descending, vectors as columns. */
void jacobi(std::vector<double>& A, int d, std::vector<double>& vals, std::vector<double>& V)
{
  V.assign(static_cast<size_t>(d) * d, 0.0);
  for (int i = 0; i < d; i++)
    V[static_cast<size_t>(i) * d + i] = 1.0;
  auto at = [&](int i, int j) -> double& { return A[static_cast<size_t>(i) * d + j]; };
  for (int sweep = 0; sweep < 60; sweep++) {
    double off = 0, tot = 0;
    for (int i = 0; i < d; i++)
      for (int j = 0; j < d; j++) {
        double v = at(i, j) * at(i, j);
        tot += v;
        if (i != j) off += v;
      }
    if (off <= 1e-26 * tot) break;
    for (int p = 0; p < d; p++)
      for (int q = p + 1; q < d; q++) {
        double apq = at(p, q);
        if (std::fabs(apq) <= 1e-300) continue;
        double theta = (at(q, q) - at(p, p)) / (2 * apq);
        double t     = (theta >= 0 ? 1.0 : -1.0) / (std::fabs(theta) + std::sqrt(theta * theta + 1));
        double c = 1 / std::sqrt(t * t + 1), s = t * c;
        for (int r = 0; r < d; r++) {  // columns p, q
          double arp = at(r, p), arq = at(r, q);
          at(r, p)   = c * arp - s * arq;
          at(r, q)   = s * arp + c * arq;
        }
        for (int r = 0; r < d; r++) {  // rows p, q
          double apr = at(p, r), aqr = at(q, r);
          at(p, r)   = c * apr - s * aqr;
          at(q, r)   = s * apr + c * aqr;
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
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return at(a, a) > at(b, b); });
  std::vector<double> V2(static_cast<size_t>(d) * d);
  vals.resize(d);
  for (int k = 0; k < d; k++) {
    vals[k] = at(order[k], order[k]);
    for (int r = 0; r < d; r++)
      V2[static_cast<size_t>(r) * d + k] = V[static_cast<size_t>(r) * d + order[k]];
  }
  V.swap(V2);
}

auto splitmix64(uint64_t z) -> uint64_t  // build_setup.cuh:105-111
{
  z += 0x9E3779B97F4A7C15ULL;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

/**
 * Projections [C, d, w] and shifts [C, w] (build_setup.cuh:119-175): copy c draws a Gaussian [p, w]
 * matrix from mt19937_64(splitmix64(seed * 0x100000001B3 + c)), orthonormalizes its columns
 * (Gram-Schmidt), rotates the top-p principal directions with it and divides by the mean projected
 * standard deviation; its shift is uniform in [0, 2) from the same generator.
 */
void make_projections(std::vector<float> const& vectors, std::vector<double> const& values, int64_t samples,
                      int64_t d, int p, int w, int copies, uint64_t seed, std::vector<float>& proj,
                      std::vector<float>& shift)
{
  OCTEX_EXPECTS(p >= w, "octex: pca_dims must be at least 8 * blocks");
  OCTEX_EXPECTS(p <= d, "octex: pca_dims exceeds the dimension");
  proj.assign(static_cast<size_t>(copies) * d * w, 0.f);
  shift.assign(static_cast<size_t>(copies) * w, 0.f);
  std::vector<double> q(static_cast<size_t>(p) * w);
  for (int c = 0; c < copies; c++) {
    std::mt19937_64 gen(splitmix64(seed * 0x100000001B3ULL + static_cast<uint64_t>(c)));
    std::normal_distribution<double> normal(0.0, 1.0);
    std::uniform_real_distribution<double> uni(0.0, 2.0);
    for (auto& v : q)
      v = normal(gen);
    for (int s = 0; s < w; s++) {
      for (int t = 0; t < s; t++) {
        double dot = 0;
        for (int r = 0; r < p; r++)
          dot += q[r * w + s] * q[r * w + t];
        for (int r = 0; r < p; r++)
          q[r * w + s] -= dot * q[r * w + t];
      }
      double nrm = 0;
      for (int r = 0; r < p; r++)
        nrm += q[r * w + s] * q[r * w + s];
      nrm = std::sqrt(nrm);
      for (int r = 0; r < p; r++)
        q[r * w + s] /= nrm;
    }
    double sd = 0;
    for (int s = 0; s < w; s++) {
      double v = 0;
      for (int r = 0; r < p; r++)
        v += values[r] * q[r * w + s] * q[r * w + s];
      sd += std::sqrt(v / static_cast<double>(std::max<int64_t>(samples - 1, 1)));
    }
    sd /= w;
    float* u = proj.data() + static_cast<size_t>(c) * d * w;
    for (int64_t k = 0; k < d; k++)
      for (int s = 0; s < w; s++) {
        double v = 0;
        for (int r = 0; r < p; r++)
          v += static_cast<double>(vectors[k * d + r]) * q[r * w + s];
        u[k * w + s] = static_cast<float>(v / sd);
      }
    for (int s = 0; s < w; s++)
      shift[static_cast<size_t>(c) * w + s] = static_cast<float>(uni(gen));
  }
}

/** The rule of a merged table row (build_table.cuh:157-164): its first kf forward entries, up to kr
 * reverse entries (lowest rank first, then lowest id), then its other forward entries; duplicates,
 * -1 and the row itself dropped; the first kout kept, in that priority order. */
struct reverse_rule {
  int kin, kf, ks, kr, kout;
};

void merge_reverse(std::vector<int32_t> const& fwd, int64_t n, reverse_rule const& rr, std::vector<int32_t>& table,
                   const float* fdist = nullptr)
{
  // Every reverse entry (u <- v at forward rank r) goes to the block of 2^16 u's that holds u, by
  // sequential appends per thread (threads own ascending v ranges, so a block's entries arrive in v
  // order); each block is then bucketed by u, and each u's entries stably by r: (r, v) order.
  const int kin = rr.kin, ks = rr.ks;
  OCTEX_EXPECTS(ks <= 256, "octex: the reverse-edge merge takes forward rows of at most 256 entries");
  constexpr int kLogBlock = 16;
  const int64_t B = (n >> kLogBlock) + 1;
  const int T     = static_cast<int>(std::clamp<int64_t>(n / 4096, 1, 16));
  auto v_range   = [&](int t) { return std::make_pair(n * t / T, n * (t + 1) / T); };
  auto run       = [&](auto&& body) {
    std::vector<std::thread> th;
    for (int t = 0; t < T; t++)
      th.emplace_back(body, t);
    for (auto& x : th)
      x.join();
  };
  std::vector<int64_t> pos(static_cast<size_t>(T) * B, 0);  // [t][block]
  run([&](int t) {
    auto [v0, v1] = v_range(t);
    std::vector<int64_t> c(B, 0);
    for (int64_t v = v0; v < v1; v++)
      for (int r = 0; r < ks; r++) {
        const int32_t u = fwd[v * kin + r];
        if (u >= 0 && u != v) c[u >> kLogBlock]++;
      }
    std::copy(c.begin(), c.end(), pos.begin() + static_cast<int64_t>(t) * B);
  });
  std::vector<int64_t> boff(B + 1, 0);  // block-major, thread-minor
  int64_t acc = 0;
  for (int64_t b = 0; b < B; b++) {
    boff[b] = acc;
    for (int t = 0; t < T; t++) {
      int64_t& p = pos[static_cast<size_t>(t) * B + b];
      const int64_t c = p;
      p = acc;
      acc += c;
    }
  }
  boff[B] = acc;
  std::unique_ptr<uint64_t[]> ent(new uint64_t[std::max<int64_t>(acc, 1)]);  // (u % 2^16) << 40 | r << 32 | v
  run([&](int t) {
    auto [v0, v1] = v_range(t);
    int64_t* p = pos.data() + static_cast<int64_t>(t) * B;
    for (int64_t v = v0; v < v1; v++)
      for (int r = 0; r < ks; r++) {
        const int32_t u = fwd[v * kin + r];
        if (u >= 0 && u != v)
          ent[p[u >> kLogBlock]++] = (static_cast<uint64_t>(u & ((1 << kLogBlock) - 1)) << 40) |
                                     (static_cast<uint64_t>(r) << 32) | static_cast<uint32_t>(v);
      }
  });
  table.assign(static_cast<size_t>(n) * rr.kout, -1);
  std::atomic<int64_t> next{0};
  run([&](int) {
    std::vector<int32_t> cu, tmp, tmpr;
    std::vector<uint64_t> srt;
    std::vector<std::pair<uint32_t, int32_t>> kd;  // (distance bits, id) of the kept entries
    std::vector<int32_t> rc(ks + 1);
    const int log_hs = std::max(8, log2_ceil(4 * int64_t{rr.kout}));  // at most a quarter full
    const unsigned hmask = (1u << log_hs) - 1;
    std::vector<uint32_t> stamp(hmask + 1, 0);
    std::vector<int32_t> slot(hmask + 1);
    uint32_t epoch = 0;
    for (int64_t b; (b = next.fetch_add(1)) < B;) {
      const int64_t u0 = b << kLogBlock, nu = std::min<int64_t>(int64_t{1} << kLogBlock, n - u0);
      const int64_t e0 = boff[b], ne = boff[b + 1] - e0;
      cu.assign(nu + 1, 0);
      srt.resize(ne);
      for (int64_t i = 0; i < ne; i++)
        cu[(ent[e0 + i] >> 40) + 1]++;
      for (int64_t u = 0; u < nu; u++)
        cu[u + 1] += cu[u];
      std::vector<int32_t> at(cu.begin(), cu.end() - 1);
      for (int64_t i = 0; i < ne; i++) {
        const uint64_t e = ent[e0 + i];
        srt[at[e >> 40]++] = e;
      }
      for (int64_t ul = 0; ul < nu; ul++) {
        const int64_t u    = u0 + ul;
        const uint64_t* eu = srt.data() + cu[ul];
        const int m        = cu[ul + 1] - cu[ul];
        std::fill(rc.begin(), rc.end(), 0);
        for (int i = 0; i < m; i++)
          rc[((eu[i] >> 32) & 0xff) + 1]++;
        for (int r = 0; r < ks; r++)
          rc[r + 1] += rc[r];
        if (static_cast<int>(tmp.size()) < m) {
          tmp.resize(m);
          tmpr.resize(m);
        }
        for (int i = 0; i < m; i++) {
          const int at2 = rc[(eu[i] >> 32) & 0xff]++;
          tmp[at2]      = static_cast<int32_t>(eu[i] & 0xffffffffULL);
          tmpr[at2]     = static_cast<int32_t>((eu[i] >> 32) & 0xff);
        }
        // kf forward, up to kr reverse, the other forward entries: the first kout distinct
        int o         = 0;
        int32_t* row  = table.data() + u * rr.kout;
        epoch++;
        kd.clear();
        auto add = [&](int32_t v, float dv) {
          if (v < 0 || v == u || o >= rr.kout) return;
          unsigned h = (static_cast<uint32_t>(v) * 2654435761u) >> (32 - log_hs);
          for (; stamp[h] == epoch; h = (h + 1) & hmask)
            if (slot[h] == v) return;
          stamp[h] = epoch;
          slot[h]  = v;
          row[o++] = v;
          if (fdist != nullptr) {
            uint32_t bits;
            const float c = dv > 0.f ? dv : 0.f;
            std::memcpy(&bits, &c, sizeof(bits));
            kd.emplace_back(bits, v);
          }
        };
        auto fd = [&](int64_t r, int t) { return fdist != nullptr ? fdist[r * kin + t] : 0.f; };
        for (int t = 0; t < rr.kf; t++)
          add(fwd[u * kin + t], fd(u, t));
        for (int t = 0; t < std::min(m, rr.kr); t++)  // a reverse entry's distance: v's forward one to u
          add(tmp[t], fd(tmp[t], tmpr[t]));
        for (int t = rr.kf; t < kin && o < rr.kout; t++)
          add(fwd[u * kin + t], fd(u, t));
        if (fdist != nullptr) {  // the kept entries nearest first, ties by id (build_table.cuh:240-251)
          std::sort(kd.begin(), kd.end());
          for (size_t t = 0; t < kd.size(); t++)
            row[t] = kd[t].second;
        }
      }
    }
  });
}

/** What one copy of a streamed build with exact or IVF lists works with (the projection of copy U, shift). */
struct stream_copy {
  row_source* rsrc    = nullptr;
  const __half* xd    = nullptr;  // the same rows, device-readable (pinned host memory's device alias)
  int64_t n           = 0;
  int d = 0, b = 0, l = 0, log_buckets = 0, min_cell = 1, probes = 0, lpp = 1;
  bool exact          = false;
  const float *mean = nullptr, *U = nullptr, *shift = nullptr;
  int64_t chunk       = 0;  // rows of y
  float* y            = nullptr;
  std::vector<dbuf>* skey  = nullptr;
  std::vector<dbuf>* sdist = nullptr;
};

/**
 * The exact or IVF lists of one copy without its whole projection on the device (build_cells.cuh:1074-1335).
 * Every level's cells come from each row's cell id (lpp levels per pass over the rows), each cell's center from its
 * first row, re-projected.  Then the rows go in ranges: each range is projected once, and the l nearest rows of every
 * center are found among its rows (brute force, or the range's own IVF index searched with `probes` probes) and
 * merged into the center's list.  Exact lists come out the same as from one search over all rows; IVF lists from one
 * range the same as the whole-projection build's.  Level j's arrays go to keys_out[j] / lists_out[j] / offs + j (T + 1);
 * returns the cells of every level.
 */
auto streamed_center_lists(cell_builder& cb, stream_copy const& sc, std::vector<float> const& spacings, int* offs,
                           std::vector<dbuf>& keys_out, std::vector<dbuf>& lists_out, hipStream_t s)
  -> std::vector<int64_t>
{
  const int L = static_cast<int>(spacings.size()), w = 8 * sc.b, l = sc.l;
  const int64_t n = sc.n, T1 = (int64_t{1} << sc.log_buckets) + 1;
  std::vector<dbuf> ck(L), z(L), zn(L), bd(L), bi(L);
  std::vector<int64_t> M(L, 0);
  dbuf stage;
  for (int j0 = 0; j0 < L; j0 += sc.lpp) {
    const int j1 = std::min(L, j0 + sc.lpp);
    for (int64_t r0 = 0; r0 < n; r0 += sc.chunk) {  // one pass: every row's cell id at levels j0 .. j1 - 1
      const int64_t m = std::min(sc.chunk, n - r0);
      project_rows(sc.rsrc->rows(r0, m, s), m, sc.d, sc.mean, sc.U, sc.shift, w, sc.y, s);
      for (int j = j0; j < j1; j++)
        stream_keys(sc.y, m, sc.b, spacings[j], (*sc.skey)[j - j0].as<long long>() + r0,
                    (*sc.sdist)[j - j0].as<float>() + r0, s);
    }
    for (int j = j0; j < j1; j++) {
      const int mc = (sc.min_cell > 1 && j < L - 1) ? sc.min_cell : 1;  // the coarsest level keeps every cell
      dbuf crow;
      M[j]  = cb.cells_of_keys((*sc.skey)[j - j0].as<long long>(), mc, ck[j], crow);
      z[j]  = dbuf(static_cast<size_t>(std::max<int64_t>(M[j], 1)) * w * sizeof(float));
      zn[j] = dbuf(static_cast<size_t>(std::max<int64_t>(M[j], 1)) * sizeof(float));
      bd[j] = dbuf(static_cast<size_t>(std::max<int64_t>(M[j] * l, 1)) * sizeof(float));
      bi[j] = dbuf(static_cast<size_t>(std::max<int64_t>(M[j] * l, 1)) * sizeof(int));
      if (M[j] > 0) {
        cell_centers(sc.xd, crow.as<int>(), M[j], sc.d, sc.mean, sc.U, sc.shift, sc.b, spacings[j], sc.chunk, stage,
                     sc.y, z[j].as<float>(), s);
        row_norms<float>(z[j].as<float>(), M[j], w, zn[j].as<float>(), s);
        init_lists(bd[j].as<float>(), bi[j].as<int>(), M[j] * l, s);
      }
      OCTEX_HIP(hipStreamSynchronize(s));
    }
  }
  stage = dbuf();
  // the row ranges (build_cells.cuh:1233-1245): OCTEX_BUILD_RANGES of them, else as many rows as 0.6 of the free
  // memory holds at the range's bytes a row (its projection, and for IVF lists the index's copy of it, labels and
  // sort scratch), at most 2^26; at least l rows a range; ranges over 2^18 rows end at multiples of 2^18 rows
  int64_t K = 0;
  if (const char* er = std::getenv("OCTEX_BUILD_RANGES"); er != nullptr && std::atoi(er) > 0) {
    K = std::atoi(er);
  } else {
    size_t fr = 0, tot = 0;
    OCTEX_HIP(hipMemGetInfo(&fr, &tot));
    const double per_row = sc.exact ? 4.0 * w + 8 : 8.0 * w + 40;
    const int64_t rmax   = std::clamp<int64_t>(static_cast<int64_t>(0.6 * static_cast<double>(fr) / per_row), 1,
                                               int64_t{1} << 26);
    K = (n + rmax - 1) / rmax;
  }
  K = std::clamp<int64_t>(K, 1, std::max<int64_t>(1, n / std::max(l, 1)));
  constexpr int64_t kRangeStep = int64_t{1} << 18;
  int64_t rlen = (n + K - 1) / K;
  if (rlen > kRangeStep) rlen = std::min(n, (rlen + kRangeStep - 1) / kRangeStep * kRangeStep);
  int64_t Mmax = 1;
  for (auto m : M)
    Mmax = std::max(Mmax, m);
  const int64_t zc = std::min<int64_t>(int64_t{1} << 20, Mmax);  // centers per search
  dbuf nd(static_cast<size_t>(zc) * l * sizeof(float)), ni(static_cast<size_t>(zc) * l * sizeof(int)),
    od(static_cast<size_t>(zc) * l * sizeof(float)), oi(static_cast<size_t>(zc) * l * sizeof(int));
  ivf_index ivf;
  build_log("streamed lists: %lld row ranges of %lld rows\n", static_cast<long long>((n + rlen - 1) / rlen),
            static_cast<long long>(rlen));
  for (int64_t a = 0; a < n; a += rlen) {
    const int64_t R = std::min(rlen, n - a);
    dbuf yr(static_cast<size_t>(R) * w * sizeof(float)), yn;
    for (int64_t r0 = 0; r0 < R; r0 += sc.chunk) {
      const int64_t m = std::min(sc.chunk, R - r0);
      project_rows(sc.rsrc->rows(a + r0, m, s), m, sc.d, sc.mean, sc.U, sc.shift, w, yr.as<float>() + r0 * w, s);
    }
    if (sc.exact) {
      yn = dbuf(static_cast<size_t>(R) * sizeof(float));
      row_norms<float>(yr.as<float>(), R, w, yn.as<float>(), s);
    } else {  // the whole-projection build's IVF settings (build_cells.cuh:513-515, 1275-1279), for this range
      const int nlist = static_cast<int>(std::max<int64_t>(64, static_cast<int64_t>(4 * std::sqrt(static_cast<double>(R)))));
      ivf.build(yr.as<float>(), R, w, nlist, R <= 4000000 ? 0.5 : 0.1, 20, s);
      yr = dbuf();  // the index holds its own copy of the rows
    }
    for (int j = 0; j < L; j++)
      for (int64_t z0 = 0; z0 < M[j]; z0 += zc) {
        const int64_t mz = std::min(zc, M[j] - z0);
        const float* zj  = z[j].as<float>() + z0 * w;
        if (sc.exact)
          knn_rows<float>(zj, zn[j].as<float>() + z0, mz, yr.as<float>(), yn.as<float>(), R, w, l, nd.as<float>(),
                          ni.as<int>(), s);
        else
          ivf.lists(zj, zn[j].as<float>() + z0, mz, sc.probes, l, ni.as<int>(), s, nd.as<float>());
        float* bdj = bd[j].as<float>() + z0 * l;
        int* bij   = bi[j].as<int>() + z0 * l;
        merge_lists(bdj, bij, nd.as<float>(), ni.as<int>(), mz, l, a, od.as<float>(), oi.as<int>(), s);
        OCTEX_HIP(hipMemcpyAsync(bdj, od.ptr, static_cast<size_t>(mz) * l * sizeof(float), hipMemcpyDeviceToDevice, s));
        OCTEX_HIP(hipMemcpyAsync(bij, oi.ptr, static_cast<size_t>(mz) * l * sizeof(int), hipMemcpyDeviceToDevice, s));
      }
    OCTEX_HIP(hipStreamSynchronize(s));
  }
  for (int j = 0; j < L; j++) {
    cb.finish_level(ck[j].as<long long>(), bi[j].as<int>(), M[j], l, sc.log_buckets, offs + j * T1, keys_out[j],
                    lists_out[j]);
    ck[j] = dbuf(), z[j] = dbuf(), zn[j] = dbuf(), bd[j] = dbuf(), bi[j] = dbuf();
  }
  return M;
}

}  // namespace

/** The neighbor rows [n, k] of an in-memory index, replacing its table (the reference's set_table). */
void set_table(index_impl& ix, std::vector<int32_t> const& rows, int k)
{
  std::lock_guard<std::mutex> run(ix.stream_mu);
  {
    std::lock_guard<std::mutex> lock(ix.mu);
    ix.plans.clear();
  }
  const size_t bytes = static_cast<size_t>(ix.n) * k * sizeof(int32_t);
  if (ix.table.size != bytes) {
    ix.bytes -= static_cast<int64_t>(ix.table.size);
    ix.table = dbuf();
    ix.table = dbuf(bytes);
    ix.bytes += static_cast<int64_t>(bytes);
  }
  upload(ix.table.ptr, rows.data(), bytes, ix.stream);
  ix.table_len = k;
}

void drop_table(index_impl& ix)
{
  std::lock_guard<std::mutex> run(ix.stream_mu);
  {
    std::lock_guard<std::mutex> lock(ix.mu);
    ix.plans.clear();
  }
  ix.bytes -= static_cast<int64_t>(ix.table.size);
  ix.table     = dbuf();
  ix.table_len = 0;
}

/**
 * The exact neighbor table (build_table.cuh:57-142, 529-554): the k + 1 nearest rows of every row by
 * brute force on the GPU (knn_rows over the fp16 vectors), the row itself dropped and distances
 * clamped at zero (drop_self_kernel, :60-74), then reverse edges merged by the half rule (kf = ks =
 * kr = k / 2) with the kept entries ordered nearest first (merge_rows_kernel, :166-252).
 */
void exact_table(index_impl& ix, int k, bool reverse_edges, std::vector<int32_t>& table)
{
  const int64_t n = ix.n, d = ix.dim;
  OCTEX_EXPECTS(k >= 1 && k < n, "octex: table_len must be in [1, n)");
  OCTEX_EXPECTS(k + 1 <= 128, "octex: the exact neighbor table takes table_len <= 127");
  const int K = k + 1;
  hipStream_t s = ix.stream;
  const __half* xd = ix.vecs();
  dbuf norms(static_cast<size_t>(n) * sizeof(float));
  row_norms(xd, n, static_cast<int>(d), norms.as<float>(), s);
  const int64_t chunk = std::min<int64_t>(n, int64_t{1} << 18);
  dbuf od(static_cast<size_t>(chunk) * K * sizeof(float)), oi(static_cast<size_t>(chunk) * K * sizeof(int32_t));
  std::vector<float> hd(static_cast<size_t>(chunk) * K);
  std::vector<int32_t> hi(static_cast<size_t>(chunk) * K);
  std::vector<int32_t> fid(static_cast<size_t>(n) * k);
  std::vector<float> fdist(static_cast<size_t>(n) * k);
  const auto t0 = std::chrono::steady_clock::now();
  for (int64_t r0 = 0; r0 < n; r0 += chunk) {
    const int64_t m = std::min(chunk, n - r0);
    knn_rows(xd + r0 * d, norms.as<float>() + r0, m, xd, norms.as<float>(), n, static_cast<int>(d), K, od.as<float>(),
             oi.as<int32_t>(), s);
    OCTEX_HIP(hipMemcpyAsync(hd.data(), od.ptr, static_cast<size_t>(m) * K * sizeof(float), hipMemcpyDeviceToHost, s));
    OCTEX_HIP(hipMemcpyAsync(hi.data(), oi.ptr, static_cast<size_t>(m) * K * sizeof(int32_t), hipMemcpyDeviceToHost,
                             s));
    OCTEX_HIP(hipStreamSynchronize(s));
    parallel_for(m, [&](int64_t i0, int64_t i1) {
      for (int64_t i = i0; i < i1; i++) {
        int t = 0;
        for (int j = 0; j < K && t < k; j++) {
          const int32_t v = hi[i * K + j];
          if (v == r0 + i) continue;
          const float dv                 = hd[i * K + j];
          fid[(r0 + i) * k + t]          = v;
          fdist[(r0 + i) * k + t]        = v < 0 ? INFINITY : (dv > 0.f ? dv : 0.f);
          t++;
        }
        for (; t < k; t++) {
          fid[(r0 + i) * k + t]   = -1;
          fdist[(r0 + i) * k + t] = INFINITY;
        }
      }
    });
    build_log("exact table: %lld of %lld rows, %.1f s\n", static_cast<long long>(r0 + m), static_cast<long long>(n),
              seconds_since(t0));
  }
  if (reverse_edges) {
    const int h = std::max(1, k / 2);
    merge_reverse(fid, n, reverse_rule{k, h, h, h, k}, table, fdist.data());
  } else {
    table = std::move(fid);
  }
}

/**
 * The searched neighbor table (build_table.cuh:557-843): forward rows of 3k/2 from a search of every
 * base vector (the vector itself dropped), passes with 0, 2 and 3 waves over the previous table,
 * reverse edges merged by the rule kf = k/4 forward first, then up to k - kf reverse entries.
 */
void searched_table(index_impl& ix, index const& idx, int k, bool reverse_edges, int passes, bool sketch_order,
                    std::vector<int32_t>& table)
{
  const int64_t n = ix.n, d = ix.dim;
  const int kin = k + k / 2, kq = kin + 1;
  OCTEX_EXPECTS(k >= 1 && kq < n, "octex: table_len too large for the dataset");
  const int kf = std::max(1, k / 4);
  reverse_rule rr{kin, kf, kin, std::max(1, k - kf), k};
  struct pass_t {
    int waves, starts;
  };
  std::vector<pass_t> plan{{0, 64}, {2, 128}, {3, 128}};
  plan.resize(std::clamp(passes, 1, 3));
  for (auto& p : plan)
    p.starts = std::max(p.starts, kin + 1);
  search_params sp;
  sp.read         = 64;
  sp.batch        = 10000;
  sp.sketch_rank  = true;
  sp.final_rerank = sketch_order ? 0 : std::max(64, kin + 1);
  std::vector<int32_t> fwd(static_cast<size_t>(n) * kin);
  const int64_t chunk = std::min<int64_t>(n, int64_t{1} << 20);
  dbuf qf(static_cast<size_t>(chunk) * d * sizeof(float));
  dbuf nb(static_cast<size_t>(chunk) * kq * sizeof(int64_t)), nd(static_cast<size_t>(chunk) * kq * sizeof(float));
  std::vector<int64_t> hnb(static_cast<size_t>(chunk) * kq);
  raft::resources res;
  res.set_stream(ix.stream);
  for (size_t v = 0; v < plan.size(); v++) {
    auto t0 = std::chrono::steady_clock::now();
    if (plan[v].waves > 0) set_table(ix, table, k);
    sp.starts = plan[v].starts;
    sp.waves  = plan[v].waves;
    for (int64_t r0 = 0; r0 < n; r0 += chunk) {
      const int64_t m = std::min(chunk, n - r0);
      half_to_float(ix.vecs() + r0 * d, m * d, qf.as<float>(), ix.stream);
      search_impl(res, sp, idx, qf.as<float>(), m, d, nb.as<int64_t>(), nd.as<float>(), kq, false, false);
      OCTEX_HIP(hipStreamSynchronize(ix.stream));
      OCTEX_HIP(hipMemcpy(hnb.data(), nb.ptr, sizeof(int64_t) * m * kq, hipMemcpyDeviceToHost));
      parallel_for(m, [&](int64_t i0, int64_t i1) {  // drop the vector itself, keep the first kin
        for (int64_t i = i0; i < i1; i++) {
          int32_t* o = fwd.data() + (r0 + i) * kin;
          int t      = 0;
          for (int j = 0; j < kq && t < kin; j++) {
            int64_t u = hnb[i * kq + j];
            if (u == r0 + i) continue;
            o[t++] = u < 0 ? -1 : static_cast<int32_t>(u);
          }
          for (; t < kin; t++)
            o[t] = -1;
        }
      });
      if ((r0 / chunk + 1) % 8 == 0)
        build_log("table pass %zu: %lld of %lld rows, %.1f s\n", v + 1, static_cast<long long>(r0 + m),
                  static_cast<long long>(n), seconds_since(t0));
    }
    if (plan[v].waves > 0) drop_table(ix);
    if (reverse_edges) {
      build_log("table pass %zu: searched in %.1f s, merging reverse edges\n", v + 1, seconds_since(t0));
      merge_reverse(fwd, n, rr, table);
    } else {
      table.assign(static_cast<size_t>(n) * k, -1);
      parallel_for(n, [&](int64_t i0, int64_t i1) {
        for (int64_t i = i0; i < i1; i++)
          std::copy_n(fwd.data() + i * kin, k, table.data() + i * k);
      });
    }
    build_log("table pass %zu (%d waves): %.2f s\n", v + 1, plan[v].waves, seconds_since(t0));
  }
}

auto build_in_memory(index_params const& params, dataset_view const& x, build_record& rec,
                     std::function<void(std::shared_ptr<index_impl> const&)> const& before_table)
  -> std::shared_ptr<index_impl>
{
  const int64_t n = x.n, d = x.d;
  const auto t_all = std::chrono::steady_clock::now();
  const int C = params.copies, b = params.blocks, w = 8 * b, l = params.list_len;
  const int L     = static_cast<int>(params.spacings.size());
  const int64_t T = int64_t{1} << params.log_buckets;
  const int S     = params.sketch_width > 0
                      ? static_cast<int>(std::min<int64_t>(params.sketch_width, d))
                      : static_cast<int>(std::max<int64_t>(std::min<int64_t>(d / 16 * 16, 128), std::min<int64_t>(d, 16)));
  const int k = params.table_len;
  // the loader's rule for a directory (load.cu:236): the sketch is scored in 16-code chunks
  OCTEX_EXPECTS(S % 16 == 0 && S >= 16 && S <= 512,
                "octex: sketch_width %d: the sketch width must be a multiple of 16 in [16, 512]", S);
  OCTEX_EXPECTS(C >= 1, "octex: at least one copy");
  OCTEX_EXPECTS(n >= 2 && d >= 1, "octex: empty dataset");
  OCTEX_EXPECTS(b >= 1 && b <= 8 && b != 7, "octex: blocks must be 1-6 or 8");
  OCTEX_EXPECTS(L >= 1, "octex: at least one spacing");
  OCTEX_EXPECTS(n >= l && l >= 1, "octex: fewer vectors than the list length");
  OCTEX_EXPECTS(n < (int64_t{1} << 31), "octex: at most 2^31 - 1 vectors");
  OCTEX_EXPECTS(params.log_buckets >= 1 && params.log_buckets <= 30, "octex: log_buckets in [1, 30]");
  OCTEX_EXPECTS(d % 2 == 0, "octex: the dimension must be even");
  OCTEX_EXPECTS(S % 16 == 0 && S <= 512, "octex: sketch width: a multiple of 16, <= 512");
  // member lists first, then exact, else the IVF lists of the reference's default (build_cells.cuh:505-516)
  const bool exact_lists = params.exact_lists && !params.member_lists;
  const bool ivf_lists   = !params.exact_lists && !params.member_lists;
  OCTEX_EXPECTS(!exact_lists || l <= 128, "octex: exact lists take list_len <= 128");
  OCTEX_EXPECTS(!ivf_lists || l <= 128, "octex: IVF lists take list_len <= 128");
  OCTEX_EXPECTS(!ivf_lists || params.list_probes >= 1, "octex: list_probes must be positive");
  int cur = 0;
  OCTEX_HIP(hipGetDevice(&cur));
  auto impl = std::make_shared<index_impl>();
  auto& ix  = *impl;
  ix.device = params.devices.empty() ? cur : params.devices.front();
  ix.devices = {ix.device};
  OCTEX_HIP(hipSetDevice(ix.device));
  OCTEX_HIP(hipStreamCreateWithFlags(&ix.stream, hipStreamNonBlocking));
  hipStream_t s = ix.stream;
  ix.n = n, ix.dim = d, ix.copies = C, ix.blocks = b, ix.list_len = l, ix.log_buckets = params.log_buckets;
  ix.sketch_width = S;
  ix.spacings     = params.spacings;
  auto t = std::chrono::steady_clock::now();
  auto phase = [&](const char* name) {
    rec.phases.emplace_back(name, seconds_since(t));
    build_log("%s: %.2f s\n", name, rec.phases.back().second);
    t = std::chrono::steady_clock::now();
  };

  // Streamed build (build_cells.cuh:756-1393, 1351-1393): when the whole-projection build's device arrays (fp16 rows,
  // one copy's fp32 projection, the cell sorts' scratch, and for IVF lists the index's copy of the projection: about
  // 2d + 4w + 64 bytes a row, 2d + 8w + 96 with IVF lists) would take more than half of the free device memory, the
  // vectors stay in pinned host memory and every copy's projection is made in chunks.  Member lists come from each
  // row's cell id and distance to its cell center; exact and IVF lists from row ranges, merged.  OCTEX_BUILD_STREAM=1
  // forces the streamed build, =0 the whole-projection one.
  size_t free_b = 0, total_b = 0;
  OCTEX_HIP(hipMemGetInfo(&free_b, &total_b));
  const char* stream_env   = std::getenv("OCTEX_BUILD_STREAM");
  const double whole_bytes = static_cast<double>(n) * (ivf_lists ? 2.0 * d + 8.0 * w + 96 : 2.0 * d + 4.0 * w + 64);
  const bool streamed      = (stream_env != nullptr && *stream_env != '\0')
                               ? std::atoi(stream_env) != 0
                               : whole_bytes > 0.5 * static_cast<double>(free_b);
  if (streamed) build_log("streamed build: vectors in pinned host memory, projections in chunks\n");

  // the fp16 vectors: the index's own, read by every step of the build (pinned host memory when streamed)
  __half* vdst = nullptr;
  if (streamed) {
    ix.host_vectors = hbuf(static_cast<size_t>(n) * d * sizeof(__half));
    vdst            = static_cast<__half*>(ix.host_vectors.dptr);
  } else {
    ix.vectors = dbuf(static_cast<size_t>(n) * d * sizeof(__half));
    ix.bytes += static_cast<int64_t>(ix.vectors.size);
    vdst = ix.vectors.as<__half>();
  }
  if (!x.f32) {
    OCTEX_HIP(hipMemcpyAsync(vdst, x.data, static_cast<size_t>(n) * d * sizeof(__half), hipMemcpyDefault, s));
  } else if (x.device) {
    float_to_half(static_cast<const float*>(x.data), n * d, vdst, s);
  } else {  // fp32 rows from the host in pieces, rounded on the GPU
    const int64_t piece = std::min<int64_t>(n * d, int64_t{1} << 26);
    dbuf tmp(static_cast<size_t>(piece) * sizeof(float));
    for (int64_t o = 0; o < n * d; o += piece) {  // tmp is rewritten only after the previous piece's kernel
      const int64_t m = std::min(piece, n * d - o);
      upload(tmp.ptr, static_cast<const float*>(x.data) + o, m * sizeof(float), s);
      float_to_half(tmp.as<float>(), m, vdst + o, s);
      OCTEX_HIP(hipStreamSynchronize(s));
    }
  }
  OCTEX_HIP(hipStreamSynchronize(s));
  const __half* xd = ix.vecs();
  row_source rsrc;
  rsrc.d = static_cast<int>(d);
  if (streamed)
    rsrc.host = static_cast<const __half*>(ix.host_vectors.ptr);
  else
    rsrc.dev = xd;

  // PCA of a sample (build_setup.cuh:40-103): every step-th row
  const int64_t step = std::max<int64_t>(1, n / 200000), ns = (n + step - 1) / step;
  std::vector<__half> sample(static_cast<size_t>(ns) * d);
  sample_rows(xd, ns, step, static_cast<int>(d), sample.data(), s);
  std::vector<double> mu(d, 0.0);
  for (int64_t i = 0; i < ns; i++)
    for (int64_t j = 0; j < d; j++)
      mu[j] += static_cast<double>(__half2float(sample[i * d + j]));
  rec.mean.resize(d);
  for (int64_t j = 0; j < d; j++)
    rec.mean[j] = static_cast<float>(mu[j] / static_cast<double>(ns));
  ix.mean = dbuf(d * sizeof(float));
  upload(ix.mean.ptr, rec.mean.data(), d * sizeof(float), s);
  std::vector<double> G(static_cast<size_t>(d) * d);
  {
    dbuf dG(G.size() * sizeof(double));
    pca_scatter(xd, n, static_cast<int>(d), step, ns, ix.mean.as<float>(), dG.as<double>(), s);
    OCTEX_HIP(hipMemcpy(G.data(), dG.ptr, dG.size, hipMemcpyDeviceToHost));
  }
  std::vector<double> vals, V;
  jacobi(G, static_cast<int>(d), vals, V);
  std::vector<float> pvec(static_cast<size_t>(d) * d);
  for (size_t i = 0; i < pvec.size(); i++)
    pvec[i] = static_cast<float>(V[i]);
  const int p = std::min<int>(params.pca_dims, static_cast<int>(d));
  make_projections(pvec, vals, ns, d, p, w, C, params.seed, rec.proj, rec.shift);
  {
    double msum = 0, vsum = 0;
    for (auto v : rec.mean)
      msum += v;
    for (auto v : vals)
      vsum += v;
    build_log("pca: %lld sampled rows, mean sum %.6g, eigenvalue sum %.6g, top %.6g\n", static_cast<long long>(ns),
              msum, vsum, vals.empty() ? 0.0 : vals[0]);
  }
  phase("setup");

  // cells of every copy
  ix.offsets = dbuf(static_cast<size_t>(C) * L * (T + 1) * sizeof(int32_t));
  ix.bytes += static_cast<int64_t>(ix.offsets.size);
  ix.T1 = T + 1;
  rec.base.assign(static_cast<size_t>(C) * L, 0);
  rec.cells.assign(static_cast<size_t>(C) * L, 0);
  std::vector<std::vector<dbuf>> level_keys(C);
  ix.copy_lists.resize(C);
  ix.list_rows.resize(C);
  {
    cell_builder cb;
    cb.reserve(n, w, s, !streamed);
    ivf_index ivf;
    // the reference's IVF parameters (build_cells.cuh:513-515): max(64, 4 sqrt(n)) lists, trained on half the rows
    // up to 4M rows, a tenth above; 20 rounds of k-means (cuVS's default)
    const int nlist = static_cast<int>(std::max<int64_t>(64, static_cast<int64_t>(4 * std::sqrt(static_cast<double>(n)))));
    const double train_fraction = n <= 4000000 ? 0.5 : 0.1;
    // streamed: rows per projected chunk, and levels per pass over the rows (12 bytes a row per level: cell id and
    // distance), within a quarter of the free memory
    const int64_t chunk = std::min<int64_t>(n, int64_t{1} << 22);
    int lpp             = L;
    if (streamed) {
      size_t fr = 0, tot = 0;
      OCTEX_HIP(hipMemGetInfo(&fr, &tot));
      lpp = static_cast<int>(std::clamp<int64_t>(static_cast<int64_t>(fr / 4) / (n * 12), 1, L));
      build_log("streamed build: %d levels per pass over the rows\n", lpp);
    }
    dbuf y(static_cast<size_t>(streamed ? chunk : n) * w * sizeof(float)), U(static_cast<size_t>(d) * w * sizeof(float)),
      sh(w * sizeof(float));
    std::vector<dbuf> skey(streamed ? lpp : 0), sdist(streamed ? lpp : 0);
    for (auto& v : skey)
      v = dbuf(static_cast<size_t>(n) * sizeof(long long));
    for (auto& v : sdist)
      v = dbuf(static_cast<size_t>(n) * sizeof(float));
    for (int c = 0; c < C; c++) {
      upload(U.ptr, rec.proj.data() + static_cast<size_t>(c) * d * w, U.size, s);
      upload(sh.ptr, rec.shift.data() + static_cast<size_t>(c) * w, sh.size, s);
      if (!streamed) {
        project_rows(xd, n, static_cast<int>(d), ix.mean.as<float>(), U.as<float>(), sh.as<float>(), w, y.as<float>(),
                     s);
        if (ivf_lists) ivf.build(y.as<float>(), n, w, nlist, train_fraction, 20, s);
      }
      std::vector<dbuf> level_lists(L);
      level_keys[c].resize(L);
      int64_t row = 0;
      if (streamed && !params.member_lists) {
        stream_copy sc;
        sc.rsrc = &rsrc, sc.xd = xd, sc.n = n, sc.d = static_cast<int>(d), sc.b = b, sc.l = l;
        sc.log_buckets = params.log_buckets, sc.min_cell = params.min_cell, sc.probes = params.list_probes;
        sc.lpp = lpp, sc.exact = exact_lists, sc.mean = ix.mean.as<float>(), sc.U = U.as<float>();
        sc.shift = sh.as<float>(), sc.chunk = chunk, sc.y = y.as<float>(), sc.skey = &skey, sc.sdist = &sdist;
        const auto Ms = streamed_center_lists(cb, sc, params.spacings,
                                              ix.offsets.as<int32_t>() + static_cast<int64_t>(c) * L * (T + 1),
                                              level_keys[c], level_lists, s);
        for (int j = 0; j < L; j++) {
          rec.base[static_cast<size_t>(c) * L + j]  = static_cast<int32_t>(row);
          rec.cells[static_cast<size_t>(c) * L + j] = Ms[j];
          row += Ms[j];
        }
      }
      for (int j0 = 0; j0 < L && !(streamed && !params.member_lists); j0 += lpp) {
        const int j1 = std::min(L, j0 + lpp);
        if (streamed)  // one pass over the rows: every row's cell id and center distance at levels j0 .. j1 - 1
          for (int64_t r0 = 0; r0 < n; r0 += chunk) {
            const int64_t m = std::min(chunk, n - r0);
            project_rows(rsrc.rows(r0, m, s), m, static_cast<int>(d), ix.mean.as<float>(), U.as<float>(),
                         sh.as<float>(), w, y.as<float>(), s);
            for (int j = j0; j < j1; j++)
              stream_keys(y.as<float>(), m, b, params.spacings[j], skey[j - j0].as<long long>() + r0,
                          sdist[j - j0].as<float>() + r0, s);
          }
        for (int j = j0; j < j1; j++) {
          const int mc = (params.min_cell > 1 && j < L - 1) ? params.min_cell : 1;
          int* offs    = ix.offsets.as<int32_t>() + (static_cast<int64_t>(c) * L + j) * (T + 1);
          int64_t M    = streamed
                           ? cb.level_streamed(skey[j - j0].as<long long>(), sdist[j - j0].as<float>(), mc, l,
                                               params.log_buckets, offs, level_keys[c][j], level_lists[j])
                           : cb.level(y.as<float>(), b, params.spacings[j], mc, l, params.log_buckets, exact_lists,
                                      offs, level_keys[c][j], level_lists[j], ivf_lists ? &ivf : nullptr,
                                      params.list_probes);
          rec.base[static_cast<size_t>(c) * L + j]  = static_cast<int32_t>(row);
          rec.cells[static_cast<size_t>(c) * L + j] = M;
          row += M;
        }
      }
      OCTEX_EXPECTS(row * l < (int64_t{1} << 31), "octex: a copy holds more than 2^31 list entries");
      ix.list_rows[c]     = row;
      ix.copy_lists[c]    = dbuf(static_cast<size_t>(std::max<int64_t>(row * l, 1)) * sizeof(int32_t));
      int64_t at          = 0;
      for (int j = 0; j < L; j++) {
        const int64_t M = rec.cells[static_cast<size_t>(c) * L + j];
        if (M > 0)
          OCTEX_HIP(hipMemcpyAsync(ix.copy_lists[c].as<int32_t>() + at * l, level_lists[j].ptr,
                                   static_cast<size_t>(M) * l * sizeof(int32_t), hipMemcpyDeviceToDevice, s));
        at += M;
      }
      OCTEX_HIP(hipStreamSynchronize(s));
      ix.bytes += static_cast<int64_t>(ix.copy_lists[c].size);
      if (c == 0 || (c + 1) % 25 == 0 || c + 1 == C || exact_lists) {
        size_t fr = 0, tot = 0;
        OCTEX_HIP(hipMemGetInfo(&fr, &tot));
        std::string cells;
        for (int j = 0; j < L; j++)
          cells += " " + std::to_string(rec.cells[static_cast<size_t>(c) * L + j]);
        build_log("copy %d: cells%s, %.3f GB of lists, %.1f GB free\n", c + 1, cells.c_str(),
                  static_cast<double>(ix.copy_lists[c].size) / 1e9, static_cast<double>(fr) / 1e9);
      }
    }
  }
  // keys [C, L, mmax], zero padded; the per-copy list pointers
  int64_t mmax = 1;
  for (auto v : rec.cells)
    mmax = std::max(mmax, v);
  ix.mmax = mmax;
  build_log("keys: [%d, %d, %lld], %.2f GB\n", C, L, static_cast<long long>(mmax),
            static_cast<double>(C) * L * mmax * 8 / 1e9);
  ix.keys = dbuf(static_cast<size_t>(C) * L * mmax * sizeof(int64_t));
  ix.bytes += static_cast<int64_t>(ix.keys.size);
  OCTEX_HIP(hipMemsetAsync(ix.keys.ptr, 0, ix.keys.size, s));
  for (int c = 0; c < C; c++)
    for (int j = 0; j < L; j++) {
      const int64_t M = rec.cells[static_cast<size_t>(c) * L + j];
      if (M > 0)
        OCTEX_HIP(hipMemcpyAsync(ix.keys.as<int64_t>() + (static_cast<int64_t>(c) * L + j) * mmax,
                                 level_keys[c][j].ptr, M * sizeof(int64_t), hipMemcpyDeviceToDevice, s));
    }
  OCTEX_HIP(hipStreamSynchronize(s));
  level_keys.clear();
  {
    std::vector<long long> hp(C);
    for (int c = 0; c < C; c++)
      hp[c] = reinterpret_cast<long long>(ix.copy_lists[c].ptr);
    ix.list_ptr = dbuf(hp.size() * sizeof(long long));
    upload(ix.list_ptr.ptr, hp.data(), ix.list_ptr.size, s);
    ix.base = dbuf(rec.base.size() * sizeof(int32_t));
    upload(ix.base.ptr, rec.base.data(), ix.base.size, s);
  }
  // the search-side arrays of the loader (load.cu:385-402): fp16 ucatT and shift, inv_f of the JSON text
  {
    std::vector<__half> uc(static_cast<size_t>(C) * w * d), shh(static_cast<size_t>(C) * w);
    for (int c = 0; c < C; c++)
      for (int sI = 0; sI < w; sI++) {
        for (int64_t k2 = 0; k2 < d; k2++)
          uc[(static_cast<size_t>(c) * w + sI) * d + k2] = __float2half(rec.proj[(static_cast<size_t>(c) * d + k2) * w + sI]);
        shh[static_cast<size_t>(c) * w + sI] = __float2half(rec.shift[static_cast<size_t>(c) * w + sI]);
      }
    std::vector<float> inv(L);
    for (int j = 0; j < L; j++)
      inv[j] = static_cast<float>(1.0 / std::strtod(json_float(params.spacings[j]).c_str(), nullptr));
    ix.ucatT = dbuf(uc.size() * sizeof(__half));
    ix.shift = dbuf(shh.size() * sizeof(__half));
    ix.inv_f = dbuf(inv.size() * sizeof(float));
    upload(ix.ucatT.ptr, uc.data(), ix.ucatT.size, s);
    upload(ix.shift.ptr, shh.data(), ix.shift.size, s);
    upload(ix.inv_f.ptr, inv.data(), ix.inv_f.size, s);
  }
  phase("copies");

  // sketch (build.cu:286-305)
  rec.basis.resize(static_cast<size_t>(d) * S);
  for (int64_t r = 0; r < d; r++)
    for (int sI = 0; sI < S; sI++)
      rec.basis[r * S + sI] = pvec[r * d + sI];
  ix.basis  = dbuf(rec.basis.size() * sizeof(float));
  ix.sketch_pitch = sketch_pitch_for(S, n, device_memory_bytes());
  ix.sketch       = dbuf(static_cast<size_t>(n) * ix.sketch_pitch);
  ix.bytes += static_cast<int64_t>(ix.sketch.size);
  upload(ix.basis.ptr, rec.basis.data(), ix.basis.size, s);
  make_sketch(rsrc, n, static_cast<int>(d), ix.mean.as<float>(), ix.basis.as<float>(), S, ix.sketch_pitch, rec.scale,
              ix.sketch.as<signed char>(), s);
  ix.scale = dbuf(S * sizeof(float));
  upload(ix.scale.ptr, rec.scale.data(), ix.scale.size, s);
  phase("sketch");

  // the probe's bucket lines, before the table phase's searches, keeping room for the table and the searches
  make_bucket_lines(ix, kSearchReserve + (k > 0 ? static_cast<size_t>(n) * k * sizeof(int32_t) : 0));
  build_log("bucket lines: %s\n", ix.lines.ptr != nullptr ? "in HBM" : "left out (memory)");

  if (before_table) before_table(impl);  // a hook that outlives this call (a writer thread) keeps its own reference

  // neighbor table: exact up to exact_table_max rows (build.cu:354-360), else searched by this library's search
  if (k > 0) {
    std::vector<int32_t> table;
    if (n <= params.exact_table_max) {
      exact_table(ix, k, params.reverse_edges, table);
    } else {
      index idx(impl);
      searched_table(ix, idx, k, params.reverse_edges, params.table_passes, params.table_sketch_order, table);
    }
    set_table(ix, table, k);
    phase("table");
  }
  OCTEX_HIP(hipSetDevice(cur));
  rec.phases.emplace_back("total", seconds_since(t_all));
  return impl;
}

namespace {

/** Device bytes appended to an .npy file through a host buffer of at most 64 MB. */
void put_device(npy_writer& w, const void* p, size_t bytes)
{
  constexpr size_t kChunk = size_t{64} << 20;
  std::vector<char> h(std::min(bytes, kChunk));
  for (size_t o = 0; o < bytes; o += kChunk) {
    const size_t m = std::min(kChunk, bytes - o);
    OCTEX_HIP(hipMemcpy(h.data(), static_cast<const char*>(p) + o, m, hipMemcpyDefault));  // device or pinned host
    w.put(h.data(), m);
  }
}

/** Rows of `row_bytes` stored `pitch` bytes apart on the device, appended back to back. */
void put_device_rows(npy_writer& w, const void* p, int64_t rows, size_t row_bytes, size_t pitch)
{
  if (pitch == row_bytes) {
    put_device(w, p, static_cast<size_t>(rows) * row_bytes);
    return;
  }
  const int64_t chunk = std::max<int64_t>(1, (int64_t{64} << 20) / static_cast<int64_t>(pitch));
  std::vector<char> h(static_cast<size_t>(std::min(chunk, rows)) * pitch);
  for (int64_t r0 = 0; r0 < rows; r0 += chunk) {
    const int64_t m = std::min(chunk, rows - r0);
    OCTEX_HIP(hipMemcpy(h.data(), static_cast<const char*>(p) + r0 * pitch, static_cast<size_t>(m) * pitch,
                        hipMemcpyDeviceToHost));
    for (int64_t r = 0; r < m; r++)
      w.put(h.data() + r * pitch, row_bytes);
  }
}

/** Every array of the directory but table.npy and meta.json (the arrays final before the neighbor table). */
void write_arrays(index_impl const& ix, build_record const& rec, index_params const& params, std::string const& path)
{
  namespace fs = std::filesystem;
  fs::create_directories(path);
  auto file = [&](const char* name) { return (fs::path(path) / name).string(); };
  const int C = ix.copies, L = ix.levels(), w = 8 * ix.blocks, l = ix.list_len, S = ix.sketch_width;
  const int64_t n = ix.n, d = ix.dim, T1 = ix.T1;
  OCTEX_HIP(hipSetDevice(ix.device));
  write_npy(file("mean.npy"), rec.mean.data(), {d});
  write_npy(file("proj.npy"), rec.proj.data(), {C, d, w});
  write_npy(file("shift.npy"), rec.shift.data(), {C, w});
  write_npy(file("base.npy"), rec.base.data(), {C, L});
  write_npy(file("cells.npy"), rec.cells.data(), {C, L});
  {
    npy_writer k(file("keys.npy"), "<i8", {C, L, ix.mmax});
    put_device(k, ix.keys.ptr, ix.keys.size);
    k.close();
  }
  {
    npy_writer o(file("offsets.npy"), "<i4", {C, L, T1});
    put_device(o, ix.offsets.ptr, ix.offsets.size);
    o.close();
  }
  {
    int64_t lmax = 0;
    for (auto r : ix.list_rows)
      lmax = std::max(lmax, r * l);
    npy_writer ls(file("lists.npy"), "<i4", {C, lmax});
    for (int c = 0; c < C; c++) {
      const size_t bytes = static_cast<size_t>(ix.list_rows[c] * l) * sizeof(int32_t);
      put_device(ls, ix.copy_lists[c].ptr, bytes);
      ls.zeros(static_cast<size_t>(lmax) * sizeof(int32_t) - bytes);
    }
    ls.close();
  }
  write_npy(file("sketch_basis.npy"), rec.basis.data(), {d, int64_t{S}});
  write_npy(file("sketch_scale.npy"), rec.scale.data(), {int64_t{S}});
  {
    npy_writer sk(file("sketch.npy"), "|i1", {n, int64_t{S}});
    put_device_rows(sk, ix.sketch.ptr, n, S, ix.sketch_pitch);
    sk.close();
  }
  {
    npy_writer v(file("vectors.npy"), "<f2", {n, d});
    put_device(v, ix.host_vectors.ptr != nullptr ? ix.host_vectors.ptr : ix.vectors.ptr,
               static_cast<size_t>(n) * d * sizeof(__half));
    v.close();
  }
}

/** The format-1 meta.json text of an index with the given table_len (build.cu:67-98). */
auto meta_text(index_impl const& ix, index_params const& params, int table_len,
               std::vector<std::pair<std::string, double>> const& phases) -> std::string
{
  const int C = ix.copies, L = ix.levels(), l = ix.list_len, S = ix.sketch_width;
  const int64_t n = ix.n, d = ix.dim;
  std::ostringstream m;
  m << "{\n \"format\": 1,\n \"n\": " << n << ",\n \"dim\": " << d << ",\n \"copies\": " << C
    << ",\n \"blocks\": " << ix.blocks << ",\n \"spacings\": [";
  for (int j = 0; j < L; j++)
    m << (j ? ", " : "") << json_float(params.spacings[j]);
  m << "],\n \"list_len\": " << l << ",\n \"log_buckets\": " << ix.log_buckets << ",\n \"sketch_width\": " << S
    << ",\n \"table_len\": " << table_len << ",\n \"metric\": \"sqeuclidean\",\n \"files\": {}";
  if (!phases.empty()) {
    m << ",\n \"build_seconds\": {";
    for (size_t i = 0; i < phases.size(); i++) {
      char buf[64];
      std::snprintf(buf, sizeof(buf), "%.3f", phases[i].second);
      m << (i ? ", " : "") << "\"" << phases[i].first << "\": " << buf;
    }
    m << "}";
  }
  m << "\n}\n";
  return m.str();
}

/** table.npy, then meta.json last: a directory without meta.json is incomplete (build.cu:67-98, 423-424). */
void write_table_meta(index_impl const& ix, index_params const& params,
                      std::vector<std::pair<std::string, double>> const& phases, std::string const& path)
{
  namespace fs = std::filesystem;
  OCTEX_HIP(hipSetDevice(ix.device));
  if (ix.table_len > 0) {
    npy_writer t((fs::path(path) / "table.npy").string(), "<i4", {ix.n, int64_t{ix.table_len}});
    put_device(t, ix.table.ptr, static_cast<size_t>(ix.n) * ix.table_len * sizeof(int32_t));
    t.close();
  }
  std::ofstream((fs::path(path) / "meta.json").string()) << meta_text(ix, params, ix.table_len, phases);
}

}  // namespace

void write_index(index_impl const& ix, build_record const& rec, index_params const& params, std::string const& path)
{
  write_arrays(ix, rec, params, path);
  write_table_meta(ix, params, rec.phases, path);
}

namespace {

/** A writer thread that is joined whatever happens: its exception is rethrown by join(). */
struct writer_thread {
  std::thread t;
  std::exception_ptr err;
  template <typename F>
  void start(F f)
  {
    t = std::thread([this, f] {
      try {
        f();
      } catch (...) {
        err = std::current_exception();
      }
    });
  }
  void join()
  {
    if (t.joinable()) t.join();
    if (err) std::rethrow_exception(std::exchange(err, nullptr));
  }
  ~writer_thread()
  {
    if (t.joinable()) t.join();
  }
};

/**
 * The neighbor table of a directory holding every other array (OCTEX_TABLE_ONLY: build.cu:153-169): the arrays
 * loaded under a meta.json text made in memory with no table, the table built over them as build_in_memory builds
 * it, then table.npy and meta.json written.
 */
auto resume_table(index_params const& params, dataset_view const& x, std::string const& path, build_record& rec)
  -> std::shared_ptr<index_impl>
{
  namespace fs = std::filesystem;
  for (const char* f : {"mean.npy", "proj.npy", "shift.npy", "base.npy", "cells.npy", "keys.npy", "offsets.npy",
                        "lists.npy", "sketch_basis.npy", "sketch_scale.npy", "sketch.npy", "vectors.npy"})
    OCTEX_EXPECTS(fs::exists(fs::path(path) / f), "octex: OCTEX_TABLE_ONLY needs %s",
                  (fs::path(path) / f).string().c_str());
  const auto t0 = std::chrono::steady_clock::now();
  npy_file basis((fs::path(path) / "sketch_basis.npy").string());
  npy_file vec((fs::path(path) / "vectors.npy").string());
  OCTEX_EXPECTS(vec.rank() == 2 && vec.dim(0) == x.n && vec.dim(1) == x.d,
                "octex: OCTEX_TABLE_ONLY: vectors.npy does not hold the dataset's shape");
  index_impl shape;  // the fields meta_text reads
  shape.n = x.n, shape.dim = x.d, shape.copies = params.copies, shape.blocks = params.blocks;
  shape.list_len = params.list_len, shape.log_buckets = params.log_buckets;
  shape.sketch_width = static_cast<int>(basis.dim(1));
  shape.spacings     = params.spacings;
  load_params lp;
  auto dir  = open_directory(path, lp, meta_text(shape, params, 0, {}));
  auto impl = load_directory(dir, path, lp);
  auto& ix  = *impl;
  const int k = params.table_len;
  if (k > 0) {
    std::vector<int32_t> table;
    if (x.n <= params.exact_table_max) {
      exact_table(ix, k, params.reverse_edges, table);
    } else {
      index idx(impl);
      searched_table(ix, idx, k, params.reverse_edges, params.table_passes, params.table_sketch_order, table);
    }
    set_table(ix, table, k);
  }
  rec.phases.emplace_back("table", seconds_since(t0));
  build_log("table: %.2f s\n", rec.phases.back().second);
  write_table_meta(ix, params, rec.phases, path);
  return impl;
}

}  // namespace

auto build_to_directory(index_params const& params, dataset_view const& x, std::string const& path,
                        build_record& rec) -> std::shared_ptr<index_impl>
{
  if (std::getenv("OCTEX_TABLE_ONLY") != nullptr)  // set at all, as build.cu:148 reads it
    return resume_table(params, x, path, rec);
  if (!params.write_behind) {
    auto impl = build_in_memory(params, x, rec);
    write_index(*impl, rec, params, path);
    return impl;
  }
  // write_behind (build.cu:146-178): the arrays final before the table go out while the table is built
  // The writer holds its own reference to the index: when the table phase throws, build_in_memory drops its
  // reference while the writer may still copy from the index's device buffers, and `w` is joined only as this
  // frame unwinds (rec, params and path outlive it).
  writer_thread w;
  auto impl = build_in_memory(params, x, rec, [&](std::shared_ptr<index_impl> const& ixp) {
    w.start([ixp, &rec, &params, &path] { write_arrays(*ixp, rec, params, path); });
  });
  w.join();
  write_table_meta(*impl, params, rec.phases, path);
  return impl;
}

}  // namespace detail

namespace {

void build_to(index_params const& params, detail::dataset_view const& x, std::string const& path)
{
  detail::build_record rec;
  detail::build_to_directory(params, x, path, rec);
}

}  // namespace

void build(raft::resources const&, index_params const& params,
           raft::host_matrix_view<const float, int64_t, raft::row_major> dataset, std::string const& path)
{
  build_to(params, {dataset.data_handle(), dataset.extent(0), dataset.extent(1), true, false}, path);
}

void build(raft::resources const&, index_params const& params,
           raft::host_matrix_view<const half, int64_t, raft::row_major> dataset, std::string const& path)
{
  build_to(params, {dataset.data_handle(), dataset.extent(0), dataset.extent(1), false, false}, path);
}

}  // namespace cuvs::neighbors::octex
