// octex search kernels for MI355X (gfx950, wave64).  One workgroup per query for every per-query
// step, as the reference's kernels (cpp/src/neighbors/octex/detail/search_kernels.cuh), written for
// 64-lane wavefronts: wave-aggregated LDS appends (ballot / popcount), 64-lane scans and butterflies.
//
// Arithmetic pins shared with the CPU oracle: E8 distances t = x - a, acc = fma(t, t, acc); the
// sketch score u = fma(code, scale, -qs), d = fma(u, u, d) over Lr-lane chunks then an xor butterfly;
// the exact distance over LX-lane groups (8-element chunks sub, sub + LX, ...), acc = fma(t, t, acc),
// then an xor butterfly; selections by (distance bits, id).  Built with -ffp-contract=off so that no other
// operation is contracted.

#include "common.hpp"
#include "e8_device.hpp"
#include "kernels.hpp"

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

namespace cuvs::neighbors::octex::detail {

namespace {

constexpr unsigned kIdHash = 2654435761u;
constexpr uint64_t kEmpty  = ~0ULL;

// ------------------------------------------------------------------ query preparation

__global__ void center_kernel(const float* __restrict__ q, const float* __restrict__ mu,
                              int64_t total, int D, float* __restrict__ qc, __half* __restrict__ qh)
{
  int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= total) return;
  float v = q[t] - mu[t % D];
  qc[t]   = v;
  qh[t]   = __float2half(v);
}

__global__ void pad_rows_kernel(float* __restrict__ q, int from, int m, int D)
{
  int64_t t     = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  int64_t total = static_cast<int64_t>(m - from) * D;
  if (t >= total) return;
  q[static_cast<int64_t>(from) * D + t] = q[t % D];
}

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

/**
 * Four consecutive fp16 at columns k..k+3 of `row` (a row pointer, or row 0 of the matrix when the row is past
 * its end: `ok` false), zeros when !ok.  FULL: every column read lies inside the row (K a multiple of 16), so
 * it is one unconditional 8-byte load and a select; otherwise each element is checked against K.  No load is
 * under a per-lane branch: that made the compiler wait for every earlier load before the next one.
 */
template <bool FULL>
__device__ __forceinline__ half4_t load_h4(const __half* __restrict__ row, bool ok, int K, int k)
{
  if constexpr (FULL) {
    uint2 u         = *reinterpret_cast<const uint2*>(row + k);
    const half4_t v = *reinterpret_cast<half4_t*>(&u);
    const half4_t z = {0, 0, 0, 0};
    return ok ? v : z;
  } else {
    half4_t v;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const bool in  = ok && k + j < K;
      const __half h = row[in ? k + j : 0];
      v[j]           = in ? static_cast<_Float16>(__half2float(h)) : static_cast<_Float16>(0.f);
    }
    return v;
  }
}

/**
 * Y [m, N] = qh [m, K] @ ucatT [N, K]^T + shift (search.cu:305-320 as one MFMA kernel): every wave
 * computes a 64-query x 64-output tile as 4 x 4 v_mfma_f32_16x16x16_f16 tiles (A = 16 outputs x 16 k
 * of ucatT, B = 16 k x 16 queries of qh), so each fragment it loads feeds four MFMAs; fp32
 * accumulation over k in steps of 16, the fp16 shift added in fp32 and one rounding to fp16.  Lane l
 * holds D[4 (l / 16) + r][l % 16]: 4 consecutive outputs of one query, written to an LDS tile and
 * stored by rows, 16 bytes per lane.  A workgroup is 4 waves along the outputs (64 queries x 256
 * outputs), held to 3 waves per SIMD (the registers allow it without spills; measured faster than 2).  The
 * fragments of 2 k steps are loaded before their MFMAs, so a wave's loads overlap; the shift is read after the
 * products.
 */
template <bool FULL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) void project_kernel(const __half* __restrict__ qh,
                                                      const __half* __restrict__ ucatT,
                                                      const __half* __restrict__ shift, int m, int K,
                                                      int N, __half* __restrict__ Y)
{
  __shared__ __align__(16) __half tile[4][64][72];  // a wave's 64 x 64 outputs, rows padded to 144 bytes
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int q0   = blockIdx.x * 64;
  const int n0   = (blockIdx.y * 4 + wid) * 64;
  const bool active = n0 < N;  // a wave past the outputs computes nothing but meets the barrier
  const int kq      = (lane >> 4) * 4;
  // this lane's rows of qh and ucatT: pointers (row 0 past the end) and validity, the same for every k step
  const __half* qrow[4];
  const __half* urow[4];
  bool qok[4], uok[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = q0 + i * 16 + (lane & 15);
    qok[i]      = r < m;
    qrow[i]     = qh + static_cast<int64_t>(qok[i] ? r : 0) * K;
  }
#pragma unroll
  for (int t = 0; t < 4; t++) {
    const int r = n0 + t * 16 + (lane & 15);
    uok[t]      = r < N;
    urow[t]     = ucatT + static_cast<int64_t>(uok[t] ? r : 0) * K;
  }
  float4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int t = 0; t < 4; t++)
      acc[i][t] = float4_t{0.f, 0.f, 0.f, 0.f};
  // k in chunks of 2 steps of 16: a chunk's 16 fragment loads are issued back to back, so a wave waits
  // for memory once per chunk rather than once per step (2, not 4: the registers of 3 waves per SIMD)
  constexpr int kChunk = 2;
  for (int c0 = 0; active && c0 < K; c0 += 16 * kChunk) {
    half4_t a[kChunk][4], b[kChunk][4];
#pragma unroll
    for (int j = 0; j < kChunk; j++) {
      if (c0 + 16 * j >= K) break;  // uniform: the steps past K of a partial last chunk
      const int k = c0 + 16 * j + kq;
#pragma unroll
      for (int i = 0; i < 4; i++)
        b[j][i] = load_h4<FULL>(qrow[i], qok[i], K, k);
#pragma unroll
      for (int t = 0; t < 4; t++)
        a[j][t] = load_h4<FULL>(urow[t], uok[t], K, k);
    }
#pragma unroll
    for (int j = 0; j < kChunk; j++) {
      if (c0 + 16 * j >= K) break;
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int t = 0; t < 4; t++)
          acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x16f16(a[j][t], b[j][i], acc[i][t], 0, 0, 0);
    }
  }
  // the tile through LDS: lane l holds 4 consecutive outputs of query l % 16 per MFMA tile, so direct
  // stores would write every 128-byte line of Y in four 32-byte pieces; read back by rows, a lane
  // stores 16 bytes and 8 lanes a whole line
  if (active) {
    float sh[4][4];  // the shift of this lane's 16 outputs
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int nb  = n0 + t * 16 + kq + r;
        const float v = __half2float(shift[nb < N ? nb : 0]);  // unconditional load, then a select
        sh[t][r]      = nb < N ? v : 0.f;
      }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int t = 0; t < 4; t++) {
        __half o[4];
#pragma unroll
        for (int r = 0; r < 4; r++)
          o[r] = __float2half(acc[i][t][r] + sh[t][r]);
        *reinterpret_cast<uint2*>(&tile[wid][i * 16 + (lane & 15)][t * 16 + kq]) = *reinterpret_cast<uint2*>(o);
      }
  }
  __syncthreads();
  if (!active) return;
#pragma unroll
  for (int pass = 0; pass < 8; pass++) {
    const int row = pass * 8 + (lane >> 3), col = (lane & 7) * 8;
    const int q = q0 + row, nb = n0 + col;
    if (q < m && nb < N)  // N is a multiple of 8: a lane's 8 outputs are all in or all out
      *reinterpret_cast<uint4*>(Y + static_cast<int64_t>(q) * N + nb) =
        *reinterpret_cast<const uint4*>(&tile[wid][row][col]);
  }
}

/**
 * qs [m, S] = qc [m, D] @ basis [D, S] with one sequential fma chain over d per output (fp32; the
 * reference uses a TF32 GEMM here).  A workgroup takes 16 queries (their rows staged in LDS) by 64
 * sketch coordinates; a thread keeps 4 queries' chains for one coordinate, so every basis load feeds
 * four fmas.
 */
__global__ __launch_bounds__(256) void sketch_query_kernel(const float* __restrict__ qc,
                                                           const float* __restrict__ basis, int m, int D,
                                                           int S, float* __restrict__ qs)
{
  extern __shared__ float qrows[];  // [16, D]
  const int q0 = blockIdx.y * 16, s = blockIdx.x * 64 + (threadIdx.x & 63), ty = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < 16 * D; i += blockDim.x) {
    const int q = q0 + i / D;
    qrows[i]     = q < m ? qc[static_cast<int64_t>(q) * D + i % D] : 0.f;
  }
  __syncthreads();
  if (s >= S) return;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int d = 0; d < D; d++) {
    const float b = basis[static_cast<int64_t>(d) * S + s];
#pragma unroll
    for (int r = 0; r < 4; r++)
      acc[r] = fmaf(qrows[(4 * ty + r) * D + d], b, acc[r]);
  }
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int q = q0 + 4 * ty + r;
    if (q < m) qs[static_cast<int64_t>(q) * S + s] = acc[r];
  }
}

template <int B>
__global__ __launch_bounds__(256) void e8_kernel(const float* __restrict__ y, int64_t n, float inv_f, float* __restrict__ p,
                          long long* __restrict__ h)
{
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float yv[8 * B];
#pragma unroll
  for (int k = 0; k < 8 * B; k++)
    yv[k] = y[i * 8 * B + k];
#pragma unroll
  for (int j = 0; j < B; j++) {
    float x[8], pp[8];
#pragma unroll
    for (int k = 0; k < 8; k++)
      x[k] = yv[8 * j + k] * inv_f;
    e8_point(x, pp);
#pragma unroll
    for (int k = 0; k < 8; k++)
      p[i * 8 * B + 8 * j + k] = pp[k];
  }
  h[i] = e8b_hash64<B>(yv, inv_f);
}

// ------------------------------------------------------------------ probe (search_kernels.cuh:84-127)

/**
 * Cell id of the E8^B point nearest to y * inv for the fp16 row yv (B 16-byte pieces): the blocks are
 * decoded one after another, a scheduling barrier between blocks keeping one decode live at a time
 * (interleaved decodes need 2-3x the registers, and the wavefronts per SIMD hide the bucket lookups).
 */
template <int B>
__device__ __forceinline__ long long probe_cell_id(const uint4 (&yv)[B], float inv)
{
  unsigned long long hh = 0;
#pragma unroll
  for (int jb = 0; jb < B; jb++) {
    const __half* hv = reinterpret_cast<const __half*>(&yv[jb]);
    float x[8], pt[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
      x[i] = __half2float(hv[i]) * inv;
    e8_point(x, pt);
    const unsigned long long hb = block_hash(pt);
    hh                          = jb == 0 ? hb : hh * kMix + hb;
    __builtin_amdgcn_sched_barrier(0);
  }
  return finish_hash(hh);
}

/**
 * The bucket lines of the CSR offsets off [CL, T1] into keys [CL, Mmax] (one thread a bucket): the first key and the
 * range of every bucket.  The loader has checked that the offsets of a level rise to at most its cell count.
 */
__global__ __launch_bounds__(256) void bucket_lines_kernel(const int* __restrict__ off, int64_t T1,
                                                           const long long* __restrict__ keys, int64_t Mmax,
                                                           int64_t total, bucket_line* __restrict__ lines)
{
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t T = T1 - 1, cl = i / T, b = i - cl * T;
  const int* o    = off + cl * T1 + b;
  bucket_line e;
  e.p0   = o[0];
  e.p1   = o[1];
  e.key0 = e.p1 > e.p0 ? keys[cl * Mmax + e.p0] : 0;
  lines[i] = e;
}

/**
 * Levels fine to coarse for every (query, copy) item, stopping at the first level whose bucket holds
 * the cell id (search_kernels.cuh:84-127).  A wavefront owns `chunk` consecutive items (item t: copy
 * t / m, query t % m, so a wavefront's lookups stay in one copy's tables); each lane holds one item and
 * its next level, and runs one level per step: the cell id of y * inv_f[level], the bucket's bounds,
 * its keys four loads at a time.  With kLines the bucket's line (its first key and bounds, one 16-byte load)
 * replaces the bounds, and the keys are read only past a first key that is not the cell's.  A lane whose item is
 * decided (a hit: seg = ((base + p) * l, lr); no level left: (0, 0)) takes the wavefront's next item, so lanes stay
 * busy until the chunk runs out instead of every item paying for all L levels.  The loop ends for the whole
 * wavefront together.
 */
template <int B, bool kLines>
__global__ __launch_bounds__(256) void probe_kernel(const __half* __restrict__ Y, int m, int C,
                                                    int L, const float* __restrict__ inv_f,
                                                    const int* __restrict__ off,
                                                    const bucket_line* __restrict__ lines, int64_t T1,
                                                    const long long* __restrict__ keys,
                                                    int64_t Mmax, const int* __restrict__ base,
                                                    int l, int lr, int logT, int64_t chunk,
                                                    int2* __restrict__ seg)
{
  const int lane         = threadIdx.x & 63;
  const int64_t total    = static_cast<int64_t>(m) * C;
  const int64_t wave     = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  const int64_t first    = wave * chunk;
  const int64_t last     = min(first + chunk, total);
  const unsigned long long below = (1ULL << lane) - 1ULL;
  int64_t next = first;  // the wavefront's next unassigned item (uniform)
  int64_t item = first + lane < last ? first + lane : -1;
  next += 64;
  int lvl = 0, c = 0;
  int64_t u = 0;
  uint4 yv[B];
  // item / m as (item + 1/2) * fl(1 / m), truncated: exact when item + 1/2 < 2^22 (the relative error of the
  // product, at most 2^-23 (1 + 2^-24), stays under the 1/(2 m) between the quotient and an integer); larger
  // batches divide in 64 bits
  const bool by_recip = total < (int64_t{1} << 22);
  const float inv_m   = 1.f / static_cast<float>(m);
  auto start = [&]() {  // a new item: its copy, its output slot, its fp16 row
    c = by_recip ? static_cast<int>((static_cast<float>(item) + 0.5f) * inv_m) : static_cast<int>(item / m);
    u = (item - static_cast<int64_t>(c) * m) * C + c;
    const uint4* yp   = reinterpret_cast<const uint4*>(Y + u * 8 * B);
#pragma unroll
    for (int jb = 0; jb < B; jb++)
      yv[jb] = yp[jb];
    lvl = 0;
  };
  if (item >= 0) start();
  while (__ballot(item >= 0) != 0) {
    bool done = false;
    if (item >= 0) {
      const long long h   = probe_cell_id<B>(yv, inv_f[lvl]);
      const int bk        = static_cast<int>(h & ((1LL << logT) - 1));
      const long long* kk = keys + (static_cast<int64_t>(c) * L + lvl) * Mmax;
      int p0 = 0, p1 = 0, hit = -1;
      if constexpr (kLines) {
        const bucket_line e = lines[(static_cast<int64_t>(c) * L + lvl) * (T1 - 1) + bk];
        p1                  = e.p1;
        if (e.p1 > e.p0 && e.key0 == h) hit = e.p0;
        p0 = e.p0 + 1;  // the first key is checked
      } else {
        const int* o = off + (static_cast<int64_t>(c) * L + lvl) * T1 + bk;
        p0           = o[0];
        p1           = o[1];
      }
      for (int p = p0; p < p1 && hit < 0; p += 4) {  // keys of the bucket, four loads in flight
        long long k4[4];
#pragma unroll
        for (int i = 0; i < 4; i++)
          k4[i] = kk[min(p + i, p1 - 1)];
#pragma unroll
        for (int i = 0; i < 4; i++)
          if (hit < 0 && p + i < p1 && k4[i] == h) hit = p + i;
      }
      if (hit >= 0) {
        seg[u] = make_int2((base[c * L + lvl] + hit) * l, lr);
        done   = true;
      } else if (lvl + 1 == L) {
        seg[u] = make_int2(0, 0);
        done   = true;
      } else {
        lvl++;
      }
    }
    // decided lanes (and idle ones) take the next items in lane order
    const unsigned long long fr = __ballot(done || item < 0);
    if (done || item < 0) {
      const int64_t t = next + __popcll(fr & below);
      item            = t < last ? t : -1;
      if (item >= 0) start();
    }
    next += __popcll(fr);
  }
}

// ------------------------------------------------------------------ gather (search_kernels.cuh:138-253)

__device__ __forceinline__ int hash_log_dev(int total, int log_cap)
{
  if (total <= 0) return kMinLogHash;
  int want = static_cast<int>((3 * static_cast<int64_t>(total) + 1) / 2);
  int e    = 32 - __clz(want - 1);  // smallest e with 2^e >= want (want >= 1)
  if (want == 1) e = 0;
  return e < kMinLogHash ? kMinLogHash : (e > log_cap ? log_cap : e);
}

/**
 * Sketch scores of a query's candidates 0..n-1 (search_kernels.cuh:227-251): an LR-lane group (LR = the
 * next power of two >= S / 16, at most 32) scores a candidate, lane `sub` reducing the 16-element chunks
 * sub, sub + LR, ... as u = fma(code, scale, -qs), d = fma(u, u, d), then an xor butterfly over the
 * group; the group's lane 0 hands (j, id, score) to put.  id_of(j) gives candidate j's id.  A
 * candidate's row is read by one load instruction of its group (one address translation per row: rows
 * lie anywhere in a sketch of many GB), and every group has kRows candidates' loads in flight before it
 * computes.
 */
template <int LR, typename IdOf, typename Put>
__device__ __forceinline__ void sketch_scores(int n, IdOf const& id_of, const signed char* __restrict__ code, int S,
                                              int pitch, const float2* sq, Put const& put)
{
  constexpr int kRows = 4;        // candidates per group in flight
  constexpr int GPW   = 64 / LR;  // groups per wavefront
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int sub = lane & (LR - 1), grp = lane / LR;
  const int k = sub * 16;         // this lane's chunk (S <= 512 = 32 chunks: one chunk per lane)
  const bool has = k < S;
  float s16[16], q16[16];         // the chunk's scale and query sketch, held in registers
#pragma unroll
  for (int e = 0; e < 16; e++) {
    const float2 v = has ? sq[k + e] : make_float2(0.f, 0.f);
    s16[e]         = v.x;
    q16[e]         = v.y;
  }
  const int per_wave = GPW * kRows;
  // Loads are unconditional (past-the-end candidates read row 0, chunkless lanes chunk 0) so that every row of
  // the group is requested before the first one is used.  A past-the-end candidate's id is row 0 whatever id_of
  // returns for the clamped index n - 1: that entry belongs to another group, which may already have replaced
  // what id_of reads there (the slot list kept in `cand` is overwritten by ids as candidates are scored), so its
  // value is no row id.
  const int stride = nw * per_wave;
  auto id_at = [&](int j) {
    const int v = id_of(min(j, n - 1));
    return j < n ? v : 0;
  };
  int id[kRows];
  if (wid * per_wave < n) {
#pragma unroll
    for (int r = 0; r < kRows; r++)  // candidate j0 + r * GPW + grp
      id[r] = id_at(wid * per_wave + r * GPW + grp);
  }
  for (int j0 = wid * per_wave; j0 < n; j0 += stride) {
    int4 w[kRows];
#pragma unroll
    for (int r = 0; r < kRows; r++)
      w[r] = *reinterpret_cast<const int4*>(code + static_cast<int64_t>(id[r]) * pitch + (has ? k : 0));
    int idn[kRows];  // the next rows' ids, read while these rows are in flight
#pragma unroll
    for (int r = 0; r < kRows; r++)
      idn[r] = j0 + stride < n ? id_at(j0 + stride + r * GPW + grp) : 0;
    float d[kRows];
#pragma unroll
    for (int r = 0; r < kRows; r++) {
      const signed char* bb = reinterpret_cast<const signed char*>(&w[r]);
      float acc             = 0.f;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        float u = fmaf(static_cast<float>(bb[e]), s16[e], -q16[e]);
        acc     = fmaf(u, u, acc);
      }
      d[r] = acc;
    }
#pragma unroll
    for (int r = 0; r < kRows; r++) {
      if (!has) d[r] = 0.f;
#pragma unroll
      for (int o = LR >> 1; o; o >>= 1)
        d[r] += __shfl_xor(d[r], o);
      const int j = j0 + r * GPW + grp;
      if (j < n && sub == 0) put(j, id[r], d[r]);
    }
#pragma unroll
    for (int r = 0; r < kRows; r++)
      id[r] = idn[r];
  }
}

/** Per-query state of collect_candidates (LDS). */
struct collect_state {
  int cnt, nsp, ulen;
  int hts;       // the hash set's slots
  int known;     // candidates whose scores came from earlier rows (row gathers)
  int wsum[16];  // a prefix sum's per-wavefront totals
};

/**
 * The distinct ids of a query's segments (search_kernels.cuh:138-222).  Wavefront 0 compacts the
 * non-empty segments (entry pointer sp and exclusive prefix pre of the lengths) into LDS; the entries
 * are then split evenly over the workgroup, kUnroll per thread with their loads issued together (entry
 * i of a query whose non-empty segments all have one length len lies in segment i / len, otherwise a
 * binary search over the prefix finds it); an LDS open-addressing set ht (of up to W slots) drops
 * duplicates, and each new id gets the next number by one atomic per wavefront: add(slot, id, h) with
 * h its hash-set slot, for slot < cap.  Returns min(distinct count, cap) in every thread.
 *
 * kRows = false: segment c = (first entry, length) in the lists of copy c (at list_ptr[c]).
 * kRows = true:  segment = (row, length) of the neighbor table [N, table_len]; -1 entries skipped.
 */
template <bool kRows, typename Add>
__device__ int collect_candidates(const int2* __restrict__ seg, int nseg, const long long* __restrict__ list_ptr,
                                  const int* __restrict__ table, int table_len, int64_t N, int logW, int cap,
                                  const int** sp, int* pre, int* ht, collect_state& cs, Add const& add)
{
  constexpr int kUnroll = 4;
  const int q = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  if (tid == 0) cs.cnt = 0;
  if (wid == 0) {
    int carry = 0, at = 0, lmin = 0x7fffffff, lmax = 0;
    for (int c0 = 0; c0 < nseg; c0 += 64) {
      const int c = c0 + lane;
      int2 sl     = c < nseg ? seg[static_cast<int64_t>(q) * nseg + c] : make_int2(0, 0);
      if (sl.y < 0) sl.y = 0;
      const bool keep               = sl.y > 0;
      const unsigned long long mask = __ballot(keep);
      const int o                   = at + __popcll(mask & ((1ULL << lane) - 1ULL));
      int v                         = sl.y;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        int u = __shfl_up(v, d);
        if (lane >= d) v += u;
      }
      if (keep) {
        pre[o] = carry + v - sl.y;
        if constexpr (kRows)
          sp[o] = table + static_cast<int64_t>(sl.x) * table_len;
        else
          sp[o] = reinterpret_cast<const int*>(list_ptr[c]) + sl.x;
        lmin = min(lmin, sl.y);
        lmax = max(lmax, sl.y);
      }
      carry += __shfl(v, 63);
      at += __popcll(mask);
    }
#pragma unroll
    for (int d = 32; d; d >>= 1) {
      lmin = min(lmin, __shfl_xor(lmin, d));
      lmax = max(lmax, __shfl_xor(lmax, d));
    }
    if (lane == 0) {
      pre[at] = carry;
      cs.nsp  = at;
      cs.ulen = at > 0 && lmin == lmax ? lmax : 0;  // one length for every non-empty segment
    }
  }
  __syncthreads();
  const int ns = cs.nsp, len = cs.ulen;
  const int total = pre[ns];
  const int HT    = 1 << hash_log_dev(total, logW);
  for (int i = tid; i < HT; i += blockDim.x)
    ht[i] = -1;
  if (tid == 0) cs.hts = HT;
  __syncthreads();
  const int step = blockDim.x;
  // i / len as (i + 1/2) * fl(1 / len), truncated: the product's relative error is at most 2^-23 (1 + 2^-24), under
  // the 1/(2 len) between (i + 1/2) / len and an integer when i + 1/2 < 2^22 (a search reads at most kMaxHash
  // entries per query); larger totals divide
  const float inv_len = len > 0 ? 1.f / static_cast<float>(len) : 0.f;
  const bool by_recip = total < (1 << 22);
  for (int i0 = 0; i0 < total; i0 += step * kUnroll) {
    int v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {  // kUnroll entries' loads issued together (past the end: the last)
      const int i = min(i0 + u * step + tid, total - 1);
      int sg;
      if (len > 0) {
        sg = by_recip ? static_cast<int>((static_cast<float>(i) + 0.5f) * inv_len) : i / len;
      } else {
        int lo = 0, hi = ns - 1;
        while (lo < hi) {
          int mid = (lo + hi + 1) >> 1;
          if (pre[mid] <= i)
            lo = mid;
          else
            hi = mid - 1;
        }
        sg = lo;
      }
      v[u] = sp[sg][i - pre[sg]];
    }
#pragma unroll
    for (int u = 0; u < kUnroll; u++)
      if (i0 + u * step + tid >= total) v[u] = -1;
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
      bool fresh = false;
      unsigned h = 0;
      if (v[u] >= 0 && v[u] < N) {  // -1: padding of a table row (search_kernels.cuh:213)
        h = (static_cast<unsigned>(v[u]) * kIdHash) & (HT - 1);
        for (int p = 0; p < HT; p++) {
          int prev = atomicCAS(&ht[h], -1, v[u]);
          if (prev == -1) {
            fresh = true;
            break;
          }
          if (prev == v[u]) break;
          h = (h + 1) & (HT - 1);
        }
      }
      const unsigned long long mask = __ballot(fresh);
      if (mask != 0) {
        const int leader = __ffsll(static_cast<long long>(mask)) - 1;
        int at           = 0;
        if (lane == leader) at = atomicAdd(&cs.cnt, __popcll(mask));
        at = __shfl(at, leader);
        if (fresh) {
          const int slot = at + __popcll(mask & ((1ULL << lane) - 1ULL));
          if (slot < cap) add(slot, v[u], h);
        }
      }
    }
  }
  __syncthreads();
  return min(cs.cnt, cap);
}

/**
 * Slot of this lane's item in a list appended to by several wavefronts: one atomic per wavefront on
 * *count, the lanes with pred set numbered in lane order (-1 for the others).  Every lane of the
 * wavefront calls it.
 */
__device__ __forceinline__ int wave_append(bool pred, int* count)
{
  const int lane                = threadIdx.x & 63;
  const unsigned long long mask = __ballot(pred);
  if (mask == 0) return -1;
  const int leader = __ffsll(static_cast<long long>(mask)) - 1;
  int base         = 0;
  if (lane == leader) base = atomicAdd(count, __popcll(mask));
  base = __shfl(base, leader);
  return pred ? base + __popcll(mask & ((1ULL << lane) - 1ULL)) : -1;
}

/** Exclusive prefix sum of one int per thread over the workgroup (<= 16 wavefronts); *total gets the sum. */
__device__ __forceinline__ int block_exclusive_sum(int v, int* wsum, int* total)
{
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
  int incl = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int u = __shfl_up(incl, d);
    if (lane >= d) incl += u;
  }
  if (lane == 63) wsum[wid] = incl;
  __syncthreads();
  int before = 0, all = 0;
  for (int w = 0; w < nw; w++) {
    before += w < wid ? wsum[w] : 0;
    all += wsum[w];
  }
  *total = all;
  __syncthreads();  // wsum may be reused by the caller
  return before + incl - v;
}

/**
 * collect_candidates without the load balance (the reference's ablation, gather_warp_kernel of
 * search_kernels.cuh:687-760): wavefront w reads the segments w, w + wavefronts, ... whole, one entry per
 * lane, so a query's longest segments set its time.  The same hash set, the same distinct ids and the same
 * add(slot, id, h) calls (slot numbers in another order).
 */
template <bool kRows, typename Add>
__device__ int collect_segments_whole(const int2* __restrict__ seg, int nseg, const long long* __restrict__ list_ptr,
                                      const int* __restrict__ table, int table_len, int64_t N, int logW, int cap,
                                      int* ht, collect_state& cs, Add const& add)
{
  const int q = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, nw = blockDim.x >> 6;
  if (tid == 0) {
    cs.cnt  = 0;
    cs.ulen = 0;
  }
  __syncthreads();
  int part = 0;
  for (int c = tid; c < nseg; c += blockDim.x)
    part += max(seg[static_cast<int64_t>(q) * nseg + c].y, 0);
  if (part > 0) atomicAdd(&cs.ulen, part);
  __syncthreads();
  const int HT = 1 << hash_log_dev(cs.ulen, logW);
  for (int i = tid; i < HT; i += blockDim.x)
    ht[i] = -1;
  if (tid == 0) cs.hts = HT;
  __syncthreads();
  for (int c = wid; c < nseg; c += nw) {
    const int2 sl = seg[static_cast<int64_t>(q) * nseg + c];
    const int* src = kRows ? table + static_cast<int64_t>(sl.x) * table_len
                           : reinterpret_cast<const int*>(list_ptr[c]) + sl.x;
    for (int e0 = 0; e0 < sl.y; e0 += 64) {  // uniform over the wavefront
      const int e = e0 + lane;
      const int v = e < sl.y ? src[e] : -1;
      bool fresh  = false;
      unsigned h  = 0;
      if (v >= 0 && v < N) {
        h = (static_cast<unsigned>(v) * kIdHash) & (HT - 1);
        for (int p = 0; p < HT; p++) {
          const int prev = atomicCAS(&ht[h], -1, v);
          if (prev == -1) {
            fresh = true;
            break;
          }
          if (prev == v) break;
          h = (h + 1) & (HT - 1);
        }
      }
      const int slot = wave_append(fresh, &cs.cnt);
      if (fresh && slot < cap) add(slot, v, h);
    }
  }
  __syncthreads();
  return min(cs.cnt, cap);
}

// ------------------------------------------------------------------ selection (search_kernels.cuh:259-322)

constexpr int kBins     = 2048;  // histogram of the selection's passes
constexpr int kTieCap   = 256;   // keys of the threshold bin ranked directly
constexpr int kSelCache = 8;     // keys per thread held in registers

struct bin_select_state {
  unsigned kmin, kmax;
  int bstar, below, ntb, nsel;
  int wtot[16];
};

static_assert(kMaxHash <= 65535, "a selection's bin counts are 16-bit");

struct bin_select_lds {
  unsigned hist[kBins / 2];  // two 16-bit bin counts a word (a query has at most 2^15 candidates: no carry)
  unsigned tkey[kTieCap];
  int tid[kTieCap];
  bin_select_state bs;
};

/** An id as the selections order it (ids are non-negative). */
__device__ __forceinline__ unsigned plain_id(int v) { return static_cast<unsigned>(v); }

/** Bin b's count in the packed histogram. */
__device__ __forceinline__ unsigned bin_count(bin_select_lds const& sh, int b)
{
  return (sh.hist[b >> 1] >> (16 * (b & 1))) & 0xffffu;
}

/**
 * The bin where the running count of the histogram reaches `need` (1 <= need <= the total count): bs.bstar, and in
 * bs.below the count of the bins before it.  Thread t scans bins [t per, (t + 1) per) after a 64-lane scan of the
 * per-thread sums.  Every thread calls it; it ends with a barrier.
 */
__device__ __forceinline__ void threshold_bin(bin_select_lds& sh, unsigned need)
{
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, nthr = blockDim.x;
  auto& bs      = sh.bs;
  const int per = kBins / nthr;
  unsigned s    = 0;
  for (int b = 0; b < per; b++)
    s += bin_count(sh, tid * per + b);
  unsigned incl = s;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const unsigned u = __shfl_up(incl, o);
    if (lane >= o) incl += u;
  }
  if (lane == 63) bs.wtot[wid] = static_cast<int>(incl);
  __syncthreads();
  unsigned excl = incl - s;
  for (int w = 0; w < wid; w++)
    excl += static_cast<unsigned>(bs.wtot[w]);
  if (excl < need && need <= excl + s) {
    unsigned cum = excl;
    for (int b = 0; b < per; b++) {
      const unsigned h = bin_count(sh, tid * per + b);
      if (cum + h >= need) {
        bs.bstar = tid * per + b;
        bs.below = static_cast<int>(cum);
        break;
      }
      cum += h;
    }
  }
  __syncthreads();
}

/**
 * The R smallest of n (distance, id) pairs of a query by (distance bits, id) (search_kernels.cuh:259-322 with a
 * deterministic tie rule) in passes over the keys, kSelCache per thread
 * held in registers (the rest are read again).
 * - First pass: a kBins-bin histogram of (key - kmin) >> shift, shift fitting the keys' range into the bins, gives
 *   the bin b* where the count reaches R.  Keys of lower bins are taken.
 * - When b* holds at most kTieCap keys, they are ranked by (key, id) among themselves and the R - (count below b*)
 *   smallest taken.
 * - Otherwise (many equal or nearly equal distances) the (key, id) pairs of b* are narrowed by further histogram
 *   passes over the 64-bit values key 2^32 + id, each over a range 2^11 times smaller, until the threshold bin holds
 *   at most kTieCap pairs (ids being distinct, at most 6 passes): linear in n, as the reference's radix passes.
 * Selected ids and their keys (skey, when not null) go to sid / skey in any order; their count (at most R) is returned
 * in every thread.  All threads of the workgroup call it.
 */
template <int kCache = kSelCache>
__device__ __forceinline__ int select_by_bins(const unsigned* __restrict__ kd, const int* cid, int n, int R, int* sid,
                                              float* skey, bin_select_lds& sh)
{
  const int tid = threadIdx.x, lane = tid & 63, nthr = blockDim.x;
  auto& bs = sh.bs;
  if (n <= R) {
    for (int i = tid; i < n; i += nthr) {
      sid[i] = cid[i];
      if (skey) skey[i] = __uint_as_float(kd[i]);
    }
    __syncthreads();
    return n;
  }
  if (tid == 0) {
    bs.kmin = ~0u;
    bs.kmax = 0u;
    bs.ntb  = 0;
    bs.nsel = 0;
  }
  constexpr unsigned kNone = ~0u;  // an empty register slot (valid keys are finite non-negative floats)
  unsigned kr[kCache];
  unsigned lo = ~0u, hi = 0u;
#pragma unroll
  for (int j = 0; j < kCache; j++) {
    const int i = tid + j * nthr;
    kr[j]       = i < n ? kd[i] : kNone;
    if (kr[j] != kNone) {
      lo = min(lo, kr[j]);
      hi = max(hi, kr[j]);
    }
  }
#pragma unroll
  for (int o = 32; o; o >>= 1) {
    lo = min(lo, static_cast<unsigned>(__shfl_xor(static_cast<int>(lo), o)));
    hi = max(hi, static_cast<unsigned>(__shfl_xor(static_cast<int>(hi), o)));
  }
  for (int i = tid; i < kBins / 2; i += nthr)
    sh.hist[i] = 0;
  __syncthreads();
  if (lane == 0) {
    atomicMin(&bs.kmin, lo);
    atomicMax(&bs.kmax, hi);
  }
  __syncthreads();
  // the range of the register-held keys (all keys when n <= kCache nthr): keys past the cache outside it fall into
  // the first or the last bin, which keeps the bins in key order
  const unsigned kmin = bs.kmin, kmax = bs.kmax, range = kmax - kmin;
  const int shift = range < static_cast<unsigned>(kBins) ? 0 : (32 - __clz(static_cast<int>(range))) - 11;
  auto bin_of     = [&](unsigned k) {
    return k < kmin ? 0u : min((k - kmin) >> shift, static_cast<unsigned>(kBins - 1));
  };
  for (int j = 0; j < kCache; j++) {  // the histogram: register-held keys, then the rest
    if (kr[j] != kNone) {
      const unsigned b = bin_of(kr[j]);
      atomicAdd(&sh.hist[b >> 1], 1u << (16 * (b & 1)));
    }
  }
  // keys past the cache, kPast a thread in flight together (unconditional loads of clamped indices, then a select:
  // one key at a time waited for each load in turn)
  constexpr int kPast = 4;
  for (int i0 = tid + kCache * nthr; i0 < n; i0 += kPast * nthr) {
    unsigned kv[kPast];
#pragma unroll
    for (int u = 0; u < kPast; u++)
      kv[u] = kd[min(i0 + u * nthr, n - 1)];
#pragma unroll
    for (int u = 0; u < kPast; u++) {
      if (i0 + u * nthr < n) {
        const unsigned b = bin_of(kv[u]);
        atomicAdd(&sh.hist[b >> 1], 1u << (16 * (b & 1)));
      }
    }
  }
  __syncthreads();
  threshold_bin(sh, static_cast<unsigned>(R));
  const unsigned bstar = static_cast<unsigned>(bs.bstar);
  int need             = R - bs.below;
  auto take = [&](bool pred, int id, unsigned key) {  // append to the selection (every lane calls it)
    const int at = wave_append(pred, &bs.nsel);
    if (pred && at < R) {
      sid[at] = id;
      if (skey) skey[at] = __uint_as_float(key);
    }
  };
  auto to_tie = [&](bool pred, int id, unsigned key) {  // into the ranked buffer (every lane calls it)
    const int t = wave_append(pred, &bs.ntb);
    if (pred && t < kTieCap) {
      sh.tkey[t] = key;
      sh.tid[t]  = id;
    }
  };
  // the candidate ids of the cached keys, loaded together before they are placed (unconditional loads of
  // clamped indices: an id read under the per-lane "selected" branch waited for the previous one)
  int ci[kCache];
#pragma unroll
  for (int j = 0; j < kCache; j++) {
    const int i = tid + j * nthr;
    ci[j]       = cid[i < n ? i : 0];
  }
#pragma unroll
  for (int j = 0; j < kCache; j++) {
    const bool ok    = kr[j] != kNone;
    const unsigned b = bin_of(kr[j]);
    take(ok && b < bstar, ci[j], kr[j]);
    to_tie(ok && b == bstar, ci[j], kr[j]);
  }
  for (int i0 = kCache * nthr; i0 < n; i0 += kPast * nthr) {  // keys past the cache: kPast keys and ids in flight
    unsigned kv[kPast];
    int id[kPast];
#pragma unroll
    for (int u = 0; u < kPast; u++) {
      const int ii = min(i0 + u * nthr + tid, n - 1);
      kv[u]        = kd[ii];
      id[u]        = cid[ii];
    }
#pragma unroll
    for (int u = 0; u < kPast; u++) {  // uniform trip counts: the appends use ballots
      const bool in    = i0 + u * nthr + tid < n;
      const unsigned b = bin_of(kv[u]);
      take(in && b < bstar, id[u], kv[u]);
      to_tie(in && b == bstar, id[u], kv[u]);
    }
  }
  __syncthreads();
  // every thread reads the count before the passes below reset it (a wave that read it after thread 0's reset would
  // skip the passes, and its barriers would pair with the other waves' barriers inside them)
  const bool many = bs.ntb > kTieCap;
  __syncthreads();
  if (many) {
    // more keys in bin b* than the ranked buffer holds: narrow the (key, id) values of b* by histogram passes
    // the key range of bin b*: the first bin also holds the keys below kmin, the last those above kmax
    const uint64_t blo = bstar == 0 ? 0 : static_cast<uint64_t>(kmin) + (static_cast<uint64_t>(bstar) << shift);
    const uint64_t bhi = bstar == kBins - 1
                           ? uint64_t{0xffffffffu}
                           : static_cast<uint64_t>(kmin) + ((static_cast<uint64_t>(bstar) + 1) << shift) - 1;
    uint64_t vlo = blo << 32, vhi = (bhi << 32) | 0x7fffffffu;
    for (;;) {  // uniform: every bound comes from LDS after a barrier
      const uint64_t vr = vhi - vlo;
      const int sh2     = vr < static_cast<uint64_t>(kBins) ? 0 : (64 - __clzll(static_cast<long long>(vr))) - 11;
      for (int i = tid; i < kBins / 2; i += nthr)
        sh.hist[i] = 0;
      if (tid == 0) bs.ntb = 0;
      __syncthreads();
      for (int i = tid; i < n; i += nthr) {
        const uint64_t v = (static_cast<uint64_t>(kd[i]) << 32) | plain_id(cid[i]);
        if (v >= vlo && v <= vhi) {
          const unsigned b = static_cast<unsigned>((v - vlo) >> sh2);
          atomicAdd(&sh.hist[b >> 1], 1u << (16 * (b & 1)));
        }
      }
      __syncthreads();
      threshold_bin(sh, static_cast<unsigned>(need));
      const int b2        = bs.bstar;
      const int below2    = bs.below;
      const bool last     = bin_count(sh, b2) <= static_cast<unsigned>(kTieCap) || sh2 == 0;
      const uint64_t nlo  = vlo + (static_cast<uint64_t>(b2) << sh2);
      const uint64_t nhi  = min(vhi, nlo + ((uint64_t{1} << sh2) - 1));
      for (int i0 = 0; i0 < n; i0 += nthr) {  // uniform trip count: the appends use ballots
        const int i      = i0 + tid;
        const int ii     = i < n ? i : 0;
        const unsigned k = kd[ii];
        const int id     = cid[ii];
        const uint64_t v = (static_cast<uint64_t>(k) << 32) | plain_id(id);
        take(i < n && v >= vlo && v < nlo, id, k);
        to_tie(last && i < n && v >= nlo && v <= nhi, id, k);
      }
      __syncthreads();
      need -= below2;
      vlo = nlo;
      vhi = nhi;
      if (last) break;
    }
  }
  const int ntb = min(bs.ntb, kTieCap);
  for (int i = tid; i < ntb; i += nthr) {  // rank of each ranked-buffer key by (key, id) among them
    const unsigned ki = sh.tkey[i], ii = plain_id(sh.tid[i]);
    int rank          = 0;
    for (int j = 0; j < ntb; j++) {
      const unsigned kj = sh.tkey[j], ij = plain_id(sh.tid[j]);
      rank += (kj < ki || (kj == ki && ij < ii)) ? 1 : 0;
    }
    if (rank < need) {
      const int at = atomicAdd(&bs.nsel, 1);
      if (at < R) {
        sid[at] = sh.tid[i];
        if (skey) skey[at] = __uint_as_float(ki);
      }
    }
  }
  __syncthreads();
  const int ns = min(bs.nsel, R);
  __syncthreads();
  return ns;
}

/**
 * Distinct ids of all segments of a query with their sketch scores (collect_candidates, then
 * sketch_scores with LR = the reference's lanes per candidate for this S), written to the query's rows of
 * cand / dist and their count to nout.  The candidates are kept as hash-set slot numbers: 16-bit in LDS
 * (kLdsSlots), or, when they do not fit in LDS beside a large hash set, in the query's own row of cand,
 * where candidate j's slot is read and then overwritten by its id by the one lane group that scores it.  A list
 * gather runs on kGatherListThreads, a row gather on kGatherRowThreads: the row gather's larger hash set leaves room
 * for fewer workgroups per CU, so each gets more threads.
 */
constexpr int kKnown = static_cast<int>(0x80000000u);  // a hash-set entry whose id's score came from an earlier row

/**
 * The entries of a query's earlier rows (earlier_rows, one or two) as one sequence: entry e is row 0's e-th while
 * e < no0, then row 1's.  load() reads entry e from an in-bounds address whatever e is (a row's W slots exist whatever
 * its count) and returns whether the entry exists; nothing derived from the loaded values is computed before the
 * caller uses them, so the loads stay in flight.
 */
struct earlier_entries {
  const int* c0;
  const int* c1;
  const float* d0;
  const float* d1;
  int W0, W1, no0, no1;

  __device__ earlier_entries(earlier_rows const& er, int q)
  {
    const int r1 = er.count > 1 ? 1 : 0;  // one row: row 1 is row 0, never taken (no1 = 0)
    c0  = er.cand[0] + static_cast<int64_t>(q) * er.W[0];
    d0  = er.dist[0] + static_cast<int64_t>(q) * er.W[0];
    c1  = er.cand[r1] + static_cast<int64_t>(q) * er.W[r1];
    d1  = er.dist[r1] + static_cast<int64_t>(q) * er.W[r1];
    W0  = er.W[0];
    W1  = er.W[r1];
    no0 = min(er.n[0][q], W0);
    no1 = er.count > 1 ? min(er.n[1][q], W1) : 0;
  }
  [[nodiscard]] __device__ int total() const { return no0 + no1; }
  __device__ bool load(int e, int& id, float& sc) const
  {
    const bool first = e < no0;
    const int Wr     = first ? W0 : W1;
    const int i      = min(max(first ? e : e - no0, 0), Wr - 1);
    id               = (first ? c0 : c1)[i];
    sc               = (first ? d0 : d1)[i];
    return e < no0 + no1;
  }
};

constexpr int kKnownPre = 4;  // earlier entries a row-gather thread loads before collecting

/**
 * Looks up an earlier entry (id, score) in a row gather's hash set ht (HT slots) after collecting; the first lookup to
 * find an id marks its slot kKnown and writes (id, score) to crow / drow from position n - 1 down.
 */
__device__ __forceinline__ void take_entry(int id, float sc, int64_t N, int n, int* ht, int HT, int* crow,
                                           float* drow, collect_state& cs)
{
  if (id < 0 || id >= N) return;
  unsigned h = (static_cast<unsigned>(id) * kIdHash) & (HT - 1);
  int at     = -1;
  for (int p = 0; p < HT; p++) {
    const int v = ht[h];
    if (v == -1) break;
    if ((v & ~kKnown) == id) {
      at = static_cast<int>(h);
      break;
    }
    h = (h + 1) & (HT - 1);
  }
  if (at >= 0 && (atomicOr(&ht[at], kKnown) & kKnown) == 0) {
    const int pos = n - 1 - atomicAdd(&cs.known, 1);
    if (pos >= 0) {
      crow[pos] = id;
      drow[pos] = sc;
    }
  }
}

/**
 * A row gather's candidates found in earlier rows of the batch (the same query's, so the same scores), after
 * collecting: the entries the thread loaded before collecting (pid / psc, entries tid + u NT), then the rest, are
 * looked up (take_entry).  Then the slot list cl keeps only the unmarked candidates, in order, at its front.  Returns
 * their count: candidates 0 .. returned - 1 are scored, the others are the copied ones.  Requires every inserted id
 * listed (cnt <= cap).  Every thread calls it; it ends with a barrier.
 */
template <int NT>
__device__ int take_known(earlier_entries const& ee, int const (&pid)[kKnownPre], float const (&psc)[kKnownPre],
                          bool const (&pok)[kKnownPre], int64_t N, int n, int* ht, int HT, unsigned short* cl,
                          int* crow, float* drow, collect_state& cs)
{
  constexpr int kU = 4;  // entries past the preloaded ones a thread loads together
  const int tid = threadIdx.x;
#pragma unroll
  for (int u = 0; u < kKnownPre; u++)
    take_entry(pok[u] ? pid[u] : -1, psc[u], N, n, ht, HT, crow, drow, cs);
  const int total = ee.total();
  for (int e0 = kKnownPre * NT; e0 < total; e0 += NT * kU) {
    int id[kU];
    float sc[kU];
    bool ok[kU];
#pragma unroll
    for (int u = 0; u < kU; u++)
      ok[u] = ee.load(e0 + u * NT + tid, id[u], sc[u]);
#pragma unroll
    for (int u = 0; u < kU; u++)
      take_entry(ok[u] ? id[u] : -1, sc[u], N, n, ht, HT, crow, drow, cs);
  }
  __syncthreads();
  // the unmarked candidates' slots to the front of cl, in order: each chunk read whole before any of it is written
  constexpr int kE = 8;
  int kept = 0;
  for (int j0 = 0; j0 < n; j0 += NT * kE) {
    unsigned short sl[kE];
    bool keep[kE];
    int mine = 0;
#pragma unroll
    for (int e = 0; e < kE; e++) {
      const int j = j0 + tid * kE + e;
      sl[e]       = cl[j < n ? j : 0];
      keep[e]     = j < n && (ht[sl[e]] & kKnown) == 0;
      mine += keep[e] ? 1 : 0;
    }
    int tot = 0;
    int at  = kept + block_exclusive_sum(mine, cs.wsum, &tot);
#pragma unroll
    for (int e = 0; e < kE; e++)
      if (keep[e]) cl[at++] = sl[e];
    kept += tot;
  }
  __syncthreads();
  return kept;
}

template <bool kRows, int LR, bool kLdsSlots, bool kBalanced>
__global__ __launch_bounds__(kRows ? kGatherRowThreads : kGatherListThreads) void gather_kernel(
  const int2* __restrict__ seg, int nseg, const long long* __restrict__ list_ptr,
  const int* __restrict__ table, int table_len, int64_t N, const signed char* __restrict__ code,
  const float* __restrict__ scale, const float* __restrict__ qs, int S, int pitch, int W, int logW, int cap,
  int* __restrict__ cand, float* __restrict__ dist, int* __restrict__ nout, earlier_rows er, int* __restrict__ nknown)
{
  const int q = blockIdx.x;
  extern __shared__ long long smq[];
  const int** sp = reinterpret_cast<const int**>(smq);  // [nseg] first entry of every non-empty segment
  float2* sq     = reinterpret_cast<float2*>(smq + nseg);  // [S] (scale, query sketch) per coordinate
  int* pre       = reinterpret_cast<int*>(sq + S);  // [nseg + 1] exclusive prefix of the compacted lengths
  int* ht        = pre + nseg + 1;                  // [W] hash set
  auto* cl       = reinterpret_cast<unsigned short*>(ht + W);  // [cap] slots of the candidates (kLdsSlots)
  __shared__ collect_state cs;
  int* crow   = cand + static_cast<int64_t>(q) * W;
  float* drow = dist + static_cast<int64_t>(q) * W;
  for (int i = threadIdx.x; i < S; i += blockDim.x)
    sq[i] = make_float2(scale[i], qs[static_cast<int64_t>(q) * S + i]);
  auto keep_slot = [&](int slot, int, unsigned h) {
    if constexpr (kLdsSlots)
      cl[slot] = static_cast<unsigned short>(h);
    else
      crow[slot] = static_cast<int>(h);
  };
  if (threadIdx.x == 0) cs.known = 0;  // the collection's barriers order this before take_known
  // the earlier rows' first entries, loaded now and not used before the collection ends: their latency passes under
  // the collection's (pid / psc are left unset without earlier rows, so that no value of them waits for the loads)
  const bool reuse = kRows && kLdsSlots && er.count > 0;
  int pid[kKnownPre];
  float psc[kKnownPre];
  bool pok[kKnownPre] = {};
  if constexpr (kRows && kLdsSlots) {
    if (reuse) {  // uniform
      const earlier_entries ee(er, q);
#pragma unroll
      for (int u = 0; u < kKnownPre; u++)
        pok[u] = ee.load(threadIdx.x + u * kGatherRowThreads, pid[u], psc[u]);
    }
  }
  int n = 0;
  if constexpr (kBalanced)
    n = collect_candidates<kRows>(seg, nseg, list_ptr, table, table_len, N, logW, cap, sp, pre, ht, cs, keep_slot);
  else
    n = collect_segments_whole<kRows>(seg, nseg, list_ptr, table, table_len, N, logW, cap, ht, cs, keep_slot);
  int nu = n;  // the candidates scored here
  if constexpr (kRows && kLdsSlots) {
    if (reuse && cs.cnt <= cap)  // uniform (read after the collection's last barrier)
      nu = take_known<kGatherRowThreads>(earlier_entries(er, q), pid, psc, pok, N, n, ht, cs.hts, cl, crow, drow, cs);
  }
  if (nknown != nullptr && threadIdx.x == 0) nknown[q] = n - nu;
  sketch_scores<LR>(
    nu,
    [&](int j) {
      if constexpr (kLdsSlots)
        return ht[cl[j]];
      else
        return ht[crow[j] & (W - 1)];  // a slot (< W), or an id when another group has scored j: kept inside ht
    },
    code, S, pitch, sq,
    [&](int j, int id, float d) {
      crow[j] = id;
      drow[j] = d;
    });
  if (threadIdx.x == 0) nout[q] = n;
}

// ------------------------------------------------------------------ selection and merges


/**
 * Squared distances of the fp16 rows sid[0, ns) to the fp32 query sq (search_kernels.cuh:325-342 with
 * another lane split): an LX-lane group scores a row (LX = the next power of two >= D / 8, at most
 * 32), lane sub reducing the 8-element chunks sub, sub + LX, ... in order as t = x - q,
 * acc = fma(t, t, acc), then an xor butterfly over the group.  A chunk is one 16-byte load when rows are
 * 16-byte aligned (D a multiple of 8), and every group has kRows rows in flight.
 */
template <int LX, bool VEC>
__device__ __forceinline__ void exact_distances_rows(const int* sid, int ns, const __half* __restrict__ vectors, int D,
                                     const float* sq, float* sd)
{
  constexpr int kRows = VEC ? 4 : 1, GPW = 64 / LX;  // rows in flight per group (one for the rare unaligned D)
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int sub = lane & (LX - 1), grp = lane / LX;
  const int nch = (D + 7) / 8;
  for (int j0 = wid * GPW * kRows; j0 < ns; j0 += nw * GPW * kRows) {
    const __half* x[kRows];
    float acc[kRows];
#pragma unroll
    for (int r = 0; r < kRows; r++) {  // past-the-end rows read the last row (results dropped)
      acc[r] = 0.f;
      x[r]   = vectors + static_cast<int64_t>(sid[min(j0 + r * GPW + grp, ns - 1)]) * D;
    }
    for (int c = sub; c < nch; c += LX) {
      const int k0 = 8 * c;
      uint4 w[kRows];
#pragma unroll
      for (int r = 0; r < kRows; r++) {  // every row's chunk first, all kRows loads in flight together
        if constexpr (VEC) {
          w[r] = *reinterpret_cast<const uint4*>(x[r] + k0);
        } else {
          __half h[8];
#pragma unroll
          for (int e = 0; e < 8; e++) {  // unconditional loads of clamped columns, then a select
            const __half v = x[r][k0 + e < D ? k0 + e : 0];
            h[e]           = k0 + e < D ? v : __float2half(0.f);
          }
          w[r] = *reinterpret_cast<const uint4*>(h);
        }
      }
      float qk[8];
#pragma unroll
      for (int e = 0; e < 8; e++)
        qk[e] = (VEC || k0 + e < D) ? sq[k0 + e] : 0.f;
#pragma unroll
      for (int r = 0; r < kRows; r++) {
        const __half* h = reinterpret_cast<const __half*>(&w[r]);
#pragma unroll
        for (int e = 0; e < 8; e++) {
          if (VEC || k0 + e < D) {
            const float t = __half2float(h[e]) - qk[e];
            acc[r]        = fmaf(t, t, acc[r]);
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < kRows; r++) {
#pragma unroll
      for (int o = LX >> 1; o; o >>= 1)
        acc[r] += __shfl_xor(acc[r], o);
      const int j = j0 + r * GPW + grp;
      if (sub == 0 && j < ns) sd[j] = acc[r];
    }
  }
  __syncthreads();
}

/** exact_distances_rows with the row layout chosen once per call: a runtime test of D inside the row loop made
 * the compiler wait for each row's load before issuing the next. */
template <int LX>
__device__ __forceinline__ void exact_distances(const int* sid, int ns, const __half* __restrict__ vectors, int D,
                                                const float* sq, float* sd)
{
  if ((D & 7) == 0)
    exact_distances_rows<LX, true>(sid, ns, vectors, D, sq, sd);
  else
    exact_distances_rows<LX, false>(sid, ns, vectors, D, sq, sd);
}

// ------------------------------------------------------------------ kept-list merges (search_kernels.cuh:345-508)

/** A (distance, id) pair as one 64-bit key ordered by (distance bits, id): distances are non-negative. */
__device__ __forceinline__ uint64_t dist_key(float d, long long id)
{
  return (static_cast<uint64_t>(__float_as_uint(d)) << 32) | static_cast<unsigned>(id);
}

/**
 * One compare-exchange step (size, stride) of a bitonic sorting network over keys held in registers: thread t
 * holds elements base + C t + j, j < C, of a sequence of C blockDim keys (base a multiple of it).  Each element
 * keeps the smaller or the larger of itself and its partner (index ^ stride), as its position in the
 * ascending / descending run of length `size` says.  Partners in the same thread are compared in registers,
 * partners in the same wavefront are exchanged by lane shuffles, partners in other wavefronts through LDS (xch,
 * C blockDim keys) between two barriers.
 */
template <int C>
__device__ __forceinline__ void bitonic_step(uint64_t (&k)[C], uint64_t* xch, int64_t base, int64_t size, int stride)
{
  const int t = threadIdx.x;
  auto keep_min = [&](int j) {
    const int64_t i = base + C * t + j;
    return ((i & stride) == 0) == ((i & size) == 0);
  };
  if (stride < C) {
#pragma unroll
    for (int j = 0; j < C; j++) {
      const int jp = j ^ stride;
      if (jp > j) {
        const uint64_t a = k[j], b = k[jp];
        const bool lo   = keep_min(j);
        k[j]            = lo ? min(a, b) : max(a, b);
        k[jp]           = lo ? max(a, b) : min(a, b);
      }
    }
  } else if (stride < 64 * C) {
#pragma unroll
    for (int j = 0; j < C; j++) {
      const uint64_t p = __shfl_xor(k[j], stride / C);
      k[j]             = keep_min(j) ? min(k[j], p) : max(k[j], p);
    }
  } else {
    __syncthreads();  // the previous exchange has been read
#pragma unroll
    for (int j = 0; j < C; j++)
      xch[C * t + j] = k[j];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < C; j++) {
      const uint64_t p = xch[(C * t + j) ^ stride];
      k[j]             = keep_min(j) ? min(k[j], p) : max(k[j], p);
    }
  }
}

/** Ascending sort of the C blockDim keys held in registers (thread t: keys C t .. C t + C - 1 of the result). */
template <int C>
__device__ __forceinline__ void block_sort(uint64_t (&k)[C], uint64_t* xch)
{
  const int total = C * static_cast<int>(blockDim.x);
  for (int size = 2; size <= total; size <<= 1)
    for (int stride = size >> 1; stride > 0; stride >>= 1)
      bitonic_step<C>(k, xch, 0, size, stride);
}

/** LDS of a kept-list merge of up to KEYS keys (C blockDim for the largest C a kernel uses). */
template <int KEYS>
struct merge_lds {
  uint64_t xch[KEYS];
  int wsum[16];
  uint64_t last[16];
};

/** Where a merge's LDS lives: the exchange of C blockDim keys, and 16 words of each per-wavefront scratch. */
struct merge_view {
  uint64_t* xch;
  int* wsum;
  uint64_t* last;
};

template <int KEYS>
__device__ __forceinline__ auto view(merge_lds<KEYS>& m) -> merge_view
{
  return {m.xch, m.wsum, m.last};
}

/** LDS bytes of merge_view over `keys` exchange keys (8-byte aligned). */
__host__ __device__ constexpr auto merge_bytes(int keys) -> size_t
{
  return static_cast<size_t>(keys) * 8 + 16 * 8 + 16 * 4;
}

/**
 * The kept list merged with new keys (search_kernels.cuh:379-415): the keys of the kept list (pb, pd: KO entries,
 * ignored when `fresh`, -1 entries empty) and the ns new (sdv[i], sid[i]) pairs, sorted together in registers,
 * and the first KO distinct keys written back to (pb, pd), padded with (-1, +inf).  Thread t loads elements
 * C t .. C t + C - 1 of the concatenation (kept first), so equal keys end next to each other after the sort; a
 * key is kept when it differs from its predecessor, and its place is the number of kept keys before it (a
 * workgroup prefix sum).  ns <= C blockDim - KO.  Every thread of the workgroup calls it.
 */
template <int C>
__device__ void merge_keep(long long* pb, float* pd, int KO, bool fresh, const int* sid, const float* sdv, int ns,
                           long long* ob, float* od, int KOout, merge_view sh)
{
  const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
  uint64_t k[C];
#pragma unroll
  for (int j = 0; j < C; j++) {
    const int i = C * t + j;
    uint64_t v  = kEmpty;
    if (i < KO) {
      const long long id = (!fresh && pb != nullptr) ? pb[i] : -1;
      if (id >= 0) v = dist_key(pd[i], id);
    } else if (i - KO < ns) {
      v = dist_key(sdv[i - KO], sid[i - KO]);
    }
    k[j] = v;
  }
  __syncthreads();  // the kept list is read before it is overwritten below
  block_sort<C>(k, sh.xch);
  // the predecessor of this thread's first key: the previous lane's last, or the previous wavefront's
  uint64_t prev = __shfl_up(k[C - 1], 1);
  if (lane == 63) sh.last[wid] = k[C - 1];
  __syncthreads();
  if (lane == 0) prev = wid > 0 ? sh.last[wid - 1] : kEmpty - 1;
  bool keep[C];
  int mine = 0;
#pragma unroll
  for (int j = 0; j < C; j++) {
    keep[j] = k[j] != kEmpty && k[j] != (j == 0 ? prev : k[j - 1]);
    mine += keep[j] ? 1 : 0;
  }
  int total = 0;
  int at    = block_exclusive_sum(mine, sh.wsum, &total);
#pragma unroll
  for (int j = 0; j < C; j++) {
    if (keep[j] && at < KOout) {
      ob[at] = static_cast<long long>(static_cast<unsigned>(k[j] & 0xffffffffULL));
      od[at] = __uint_as_float(static_cast<unsigned>(k[j] >> 32));
    }
    at += keep[j] ? 1 : 0;
  }
  for (int o = min(total, KOout) + t; o < KOout; o += blockDim.x) {
    ob[o] = -1;
    od[o] = INFINITY;
  }
}

/**
 * f(std::integral_constant<int, C>) with C the keys per thread that hold `keys` keys over `threads` threads, C a power
 * of two up to MAXC (the callers' limits keep keys <= MAXC threads).
 */
template <int MAXC = 4, typename F>
__device__ __forceinline__ void with_keys_per_thread(int keys, int threads, F&& f)
{
  if (keys <= threads)
    f(std::integral_constant<int, 1>{});
  else if (keys <= 2 * threads || MAXC <= 2)
    f(std::integral_constant<int, 2>{});
  else if (keys <= 4 * threads || MAXC <= 4)
    f(std::integral_constant<int, 4>{});
  else
    f(std::integral_constant<int, MAXC <= 8 ? MAXC : 8>{});
}

/** The keys per thread of a kept-list merge of `keys` keys over `threads` threads (with_keys_per_thread's C). */
__host__ __device__ constexpr auto keys_per_thread(int keys, int threads) -> int
{
  return keys <= threads ? 1 : keys <= 2 * threads ? 2 : keys <= 4 * threads ? 4 : 8;
}

constexpr int kRerankThreads = 128;         // rerank_keep_kernel's workgroup: one query
constexpr int64_t kWideRerank = int64_t{1} << 15;  // R D from which a query takes 256 threads
constexpr int kHistWindow    = 256;  // the most recent history entries a round skips (earlier ones are reranked again)

/** Slots of the set of a round's history window (hoff entries before it): a power of two at least twice the window,
 * 0 for a round without one. */
__host__ __device__ constexpr auto hist_slots(int hoff) -> int
{
  const int w = hoff < kHistWindow ? hoff : kHistWindow;
  int s       = 64;
  while (s < 2 * w)
    s <<= 1;
  return w > 0 ? s : 0;
}

/**
 * LDS of rerank_keep_kernel for R reranked keys, KO kept, D coordinates and a history set of `slots`, carved from its
 * dynamic LDS in this order: the region the selection and the merge use in turn (8-byte aligned), the selected ids,
 * their distances, the ids left to rerank, the query, the history set.  Sized per launch, so small R and KO leave room
 * for more workgroups per CU.
 */
__host__ __device__ constexpr auto rerank_region_bytes(int R, int KO, int threads) -> size_t
{
  const size_t merge = merge_bytes(keys_per_thread(KO + R, threads) * threads);
  return ((sizeof(bin_select_lds) > merge ? sizeof(bin_select_lds) : merge) + 7) / 8 * 8;
}
__host__ __device__ constexpr auto rerank_lds_bytes(int R, int KO, int D, int threads, int slots) -> size_t
{
  return rerank_region_bytes(R, KO, threads) + static_cast<size_t>(R) * 12 + static_cast<size_t>(D) * 4 +
         static_cast<size_t>(slots) * 4;
}

/** Slot of id v in the set hs of `slots` slots (a power of two; -1 empty, linear probing), inserting it when
 * `insert`; -1 when it is absent (a lookup) or the set is full. */
__device__ __forceinline__ int hist_slot(int* hs, int slots, int v, bool insert)
{
  unsigned h = (static_cast<unsigned>(v) * kIdHash) & static_cast<unsigned>(slots - 1);
  for (int p = 0; p < slots; p++) {
    const int e = insert ? atomicCAS(&hs[h], -1, v) : hs[h];
    if (e == v || (insert && e == -1)) return static_cast<int>(h);
    if (e == -1) return -1;
    h = (h + 1) & static_cast<unsigned>(slots - 1);
  }
  return -1;
}

/**
 * Exact rerank of the R sketch-nearest candidates of a query, merged into its kept list of the best
 * KO (search_kernels.cuh:421-467).  fresh: the kept list starts empty.  One workgroup of NT threads per query, C keys a
 * thread in the merge (the host's choice for KO + R).
 *
 * Rounds after the first skip what an earlier round reranked.  hist [m, H] holds every round's selected ids (each round
 * R entries, -1 padded): this round's go to hist[q, hoff .. hoff + R) when hstore, and unless fresh the ids at
 * hist[q, 0 .. hoff) (the last kHistWindow of them) are the earlier rounds'.  Whenever the kept list is merged, it
 * becomes the KO smallest distinct keys of every key merged so far, so an id an earlier round reranked has its exact key
 * either in the kept list already (merging it again changes nothing) or above all KO kept keys (it cannot enter):
 * dropping it leaves the merge's result unchanged.  It is neither read nor merged; nskip [m] (when not null) gets the
 * count.  The window's ids are loaded as the kernel starts and their set (hslots slots, at least twice the window)
 * cleared, so neither waits after the selection.
 */
// Eight waves a SIMD: the selection's 64-bit tie bounds took the kernel to about 100 SGPRs, which allow seven (the
// excess spills to VGPR lanes); measured at 10M rows, the first round's launch went from 94 to 84 us.  Merges of 8
// keys a thread (KO + R above 512 on 128 threads) need more than the 64 VGPRs of eight waves: seven.
template <int LX, int NT, int C>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(C <= 4 ? 8 : 7, C <= 4 ? 8 : 7))) void
rerank_keep_kernel(
  const int* __restrict__ cand, const float* __restrict__ dist, const int* __restrict__ nin, int W,
  const __half* __restrict__ vectors, int D, const float* __restrict__ Q, int R, int KO,
  long long* __restrict__ bi, float* __restrict__ bd, bool fresh, int* __restrict__ hist, int H, int hoff, bool hstore,
  int hslots, int* __restrict__ nskip)
{
  const int q = blockIdx.x;
  extern __shared__ uint64_t rk_lds[];
  __shared__ int nfresh;  // selected ids no earlier round reranked
  const size_t region = rerank_region_bytes(R, KO, NT);
  auto* base          = reinterpret_cast<unsigned char*>(rk_lds);
  auto& sel           = *reinterpret_cast<bin_select_lds*>(base);
  const int keys      = keys_per_thread(KO + R, NT) * NT;
  merge_view mv{reinterpret_cast<uint64_t*>(base), reinterpret_cast<int*>(base + static_cast<size_t>(keys) * 8 + 16 * 8),
                reinterpret_cast<uint64_t*>(base + static_cast<size_t>(keys) * 8)};
  int* sid  = reinterpret_cast<int*>(base + region);
  float* sd = reinterpret_cast<float*>(sid + R);
  int* rid  = reinterpret_cast<int*>(sd + R);  // the selected ids left to rerank (filtered rounds)
  float* sq = reinterpret_cast<float*>(rid + R);
  int* hs   = reinterpret_cast<int*>(sq + D);  // the history window's set
  int* hrow = hist != nullptr ? hist + static_cast<int64_t>(q) * H : nullptr;
  const bool filter = !fresh && hoff > 0;  // the host passes hist and hslots >= 2 min(hoff, kHistWindow) then
  constexpr int kPer = (kHistWindow + NT - 1) / NT;
  int hv[kPer];
  if (filter) {
    const int h0 = hoff > kHistWindow ? hoff - kHistWindow : 0;
#pragma unroll
    for (int e = 0; e < kPer; e++) {  // unconditional loads of clamped in-bounds entries, then a select
      const int i = h0 + threadIdx.x + e * NT;
      const int v = hrow[i < hoff ? i : hoff - 1];
      hv[e]       = i < hoff ? v : -1;
    }
    for (int i = threadIdx.x; i < hslots; i += NT)
      hs[i] = -1;
    if (threadIdx.x == 0) nfresh = 0;
  }
  const int n = min(nin[q], W);
  for (int i = threadIdx.x; i < D; i += blockDim.x)
    sq[i] = Q[static_cast<int64_t>(q) * D + i];
  // the selection's barriers order the set's clearing before its inserts below
  const int ns = select_by_bins(reinterpret_cast<const unsigned*>(dist + static_cast<int64_t>(q) * W),
                                cand + static_cast<int64_t>(q) * W, n, R, sid, nullptr, sel);
  if (hstore)
    for (int t = threadIdx.x; t < R; t += NT)
      hrow[hoff + t] = t < ns ? sid[t] : -1;
  int nr        = ns;  // the selected ids reranked here
  const int* rr = sid;
  if (filter) {
#pragma unroll
    for (int e = 0; e < kPer; e++)
      if (hv[e] >= 0) hist_slot(hs, hslots, hv[e], true);
    __syncthreads();
    for (int i0 = 0; i0 < ns; i0 += NT) {  // uniform trip count: the appends use ballots
      const int i     = i0 + threadIdx.x;
      const int v     = sid[i < ns ? i : 0];
      const bool keep = i < ns && hist_slot(hs, hslots, v, false) < 0;
      const int at    = wave_append(keep, &nfresh);
      if (keep) rid[at] = v;
    }
    __syncthreads();
    nr = nfresh;
    rr = rid;
  }
  if (nskip != nullptr && threadIdx.x == 0) nskip[q] = ns - nr;
  exact_distances<LX>(rr, nr, vectors, D, sq, sd);
  // exact_distances ended with a barrier: the region is free for the merge
  merge_keep<C>(bi + static_cast<int64_t>(q) * KO, bd + static_cast<int64_t>(q) * KO, KO, fresh, rr, sd, nr,
                bi + static_cast<int64_t>(q) * KO, bd + static_cast<int64_t>(q) * KO, KO, mv);
}

/** The KO sketch-nearest candidates merged into the kept list by sketch distance (:471-508). */
__global__ __launch_bounds__(512) void sketch_keep_kernel(const int* __restrict__ cand,
                                                          const float* __restrict__ dist,
                                                          const int* __restrict__ nin, int W, int KO,
                                                          long long* __restrict__ si,
                                                          float* __restrict__ sd, bool fresh)
{
  const int q = blockIdx.x;
  __shared__ union {
    bin_select_lds sel;
    merge_lds<2 * kMaxSketchKO> merge;
  } u;
  __shared__ int sid[kMaxSketchKO];
  __shared__ float sdv[kMaxSketchKO];
  const int n  = min(nin[q], W);
  const int ns = select_by_bins(reinterpret_cast<const unsigned*>(dist + static_cast<int64_t>(q) * W),
                                cand + static_cast<int64_t>(q) * W, n, KO, sid, sdv, u.sel);
  long long* pb = si + static_cast<int64_t>(q) * KO;
  float* pd     = sd + static_cast<int64_t>(q) * KO;
  with_keys_per_thread(KO + ns, blockDim.x, [&](auto c) {
    constexpr int C = decltype(c)::value;
    merge_keep<C>(pb, pd, KO, fresh, sid, sdv, ns, pb, pd, KO, view(u.merge));
  });
}

/**
 * A set of ids in LDS, in nb buckets of four slots (nb a power of two): an id lives in its home bucket (a
 * multiplicative hash) or, when that is full, in the next buckets.  A lookup reads a whole bucket with one 16-byte
 * load.  The set is sized per launch to at least twice the ids it takes (at most kPickHash slots).
 */
struct id_buckets {
  static constexpr int kSlots = 4;
  int4* b;
  int nb;

  [[nodiscard]] __device__ unsigned home(long long v) const
  {
    return ((static_cast<unsigned>(v) * kIdHash) >> 7) & static_cast<unsigned>(nb - 1);
  }
  __device__ void clear() const
  {
    for (int i = threadIdx.x; i < nb; i += blockDim.x)
      b[i] = make_int4(-1, -1, -1, -1);
  }
  __device__ void insert(int v) const
  {
    for (unsigned h = home(v), p = 0; p < static_cast<unsigned>(nb); p++, h = (h + 1) & (nb - 1)) {
      int* slot = reinterpret_cast<int*>(&b[h]);
      for (int j = 0; j < kSlots; j++) {
        const int prev = atomicCAS(&slot[j], -1, v);
        if (prev == -1 || prev == v) return;
      }
    }
  }
  [[nodiscard]] __device__ bool contains(int v) const
  {
    for (unsigned h = home(v), p = 0; p < static_cast<unsigned>(nb); p++, h = (h + 1) & (nb - 1)) {
      const int4 w = b[h];
      if (w.x == v || w.y == v || w.z == v || w.w == v) return true;
      if (w.w == -1) return false;  // a bucket with a free slot ends the run
    }
    return false;
  }
};

/** Buckets of pick_starts_kernel's set for `off` expanded ids: at least 2 off slots, at most kPickHash. */
__host__ __device__ constexpr auto pick_buckets(int off) -> int
{
  int nb = 4;
  while (nb * id_buckets::kSlots < 2 * off && nb * id_buckets::kSlots < kPickHash)
    nb <<= 1;
  return nb;
}

/**
 * Start points of a wave (search_kernels.cuh:571-631): the first S kept entries (best first) that no
 * earlier wave expanded (done[:, :off]), written to done[:, off:off + S] and to the gather segments
 * seg2 = (row, rowlen); (-1 / (0, 0)) when fewer remain.  The expanded ids go into an LDS bucket set, every
 * thread marks its kept entries fresh or not, and wavefront 0 takes the fresh ones in order by ballots.
 */
__global__ __launch_bounds__(256) void pick_starts_kernel(const long long* __restrict__ si, int KO,
                                                          long long* __restrict__ done, int E,
                                                          int off, int S, int rowlen,
                                                          int2* __restrict__ seg2, int nb)
{
  const int q = blockIdx.x;
  extern __shared__ int4 pick_lds[];  // the set's nb buckets (none when off is 0)
  const id_buckets seen{pick_lds, nb};
  __shared__ unsigned char fresh[kMaxSketchKO];
  const long long* ps = si + static_cast<int64_t>(q) * KO;
  long long* pd       = done + static_cast<int64_t>(q) * E;
  if (off > 0) {
    seen.clear();
    __syncthreads();
    for (int i = threadIdx.x; i < off; i += blockDim.x) {
      const long long v = pd[i];
      if (v >= 0) seen.insert(static_cast<int>(v));
    }
    __syncthreads();
  }
  for (int i = threadIdx.x; i < KO; i += blockDim.x) {
    const long long v = ps[i];
    fresh[i]          = v >= 0 && (off == 0 || !seen.contains(static_cast<int>(v)));
  }
  __syncthreads();
  if ((threadIdx.x >> 6) != 0) return;
  const int lane = threadIdx.x & 63;
  int at         = 0;
  for (int i0 = 0; i0 < KO && at < S; i0 += 64) {
    const int i     = i0 + lane;
    const bool take = i < KO && fresh[i];
    const unsigned long long mask = __ballot(take);
    const int o = at + __popcll(mask & ((1ULL << lane) - 1ULL));
    if (take && o < S) {
      long long v                            = ps[i];
      pd[off + o]                            = v;
      seg2[static_cast<int64_t>(q) * S + o] = make_int2(static_cast<int>(v), rowlen);
    }
    at += __popcll(mask);
  }
  for (int o = min(at, S) + lane; o < S; o += 64) {
    pd[off + o]                            = -1;
    seg2[static_cast<int64_t>(q) * S + o] = make_int2(0, 0);
  }
}

/**
 * Exact rerank of the first R kept entries (sketch-rank mode) into the best k (:634-669): the valid entries
 * (id >= 0) are numbered by a workgroup prefix count, their exact distances computed, and the (distance, id)
 * keys merged into an empty list of k.
 */
template <int LX>
__global__ __launch_bounds__(kKeepThreads) void final_rerank_kernel(
  const long long* __restrict__ si, int KO, int R, const __half* __restrict__ vectors, int D,
  const float* __restrict__ Q, int k, long long* __restrict__ bi, float* __restrict__ bd)
{
  const int q = blockIdx.x;
  extern __shared__ float sq[];
  __shared__ merge_lds<kMaxRerank> m2;
  __shared__ int sid[kMaxRerank];
  __shared__ float sd[kMaxRerank];
  __shared__ int nvalid;
  const long long* ps = si + static_cast<int64_t>(q) * KO;
  for (int i = threadIdx.x; i < D; i += blockDim.x)
    sq[i] = Q[static_cast<int64_t>(q) * D + i];
  // R <= 512 = 2 entries per thread, in order
  long long v[2];
  int mine = 0;
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int i = 2 * threadIdx.x + j;
    v[j]        = i < R ? ps[i] : -1;
    mine += v[j] >= 0 ? 1 : 0;
  }
  int total = 0;
  int at    = block_exclusive_sum(mine, m2.wsum, &total);
#pragma unroll
  for (int j = 0; j < 2; j++)
    if (v[j] >= 0) sid[at++] = static_cast<int>(v[j]);
  if (threadIdx.x == 0) nvalid = total;
  __syncthreads();
  const int ns = nvalid;
  exact_distances<LX>(sid, ns, vectors, D, sq, sd);
  with_keys_per_thread(ns, blockDim.x, [&](auto c) {
    constexpr int C = decltype(c)::value < 2 ? decltype(c)::value : 2;
    merge_keep<C>(nullptr, nullptr, 0, true, sid, sd, ns, bi + static_cast<int64_t>(q) * k,
                  bd + static_cast<int64_t>(q) * k, k, view(m2));
  });
}

// ------------------------------------------------------------------ unfused merge (fused_merge = false)
//
// The reference's ablation of the fused kernels (search.cu:213-291, search_kernels.cuh:798-954): candidate keys
// sorted in global memory, a pool of the kept list and the R best candidates, the pools sorted, and the first KO
// distinct keys kept; start points by a sorted list of the expanded ids.  Same results as the fused kernels.

/** ukey[q, j] = (dist, id) key of candidate j < n of query q, the empty key past n (W per query). */
__global__ void cand_keys_kernel(const int* __restrict__ cand, const float* __restrict__ dist,
                                 const int* __restrict__ nin, int W, uint64_t* __restrict__ ukey)
{
  const int q     = blockIdx.x;
  const int n     = min(nin[q], W);
  const int64_t o = static_cast<int64_t>(q) * W;
  for (int j = threadIdx.x; j < W; j += blockDim.x)
    ukey[o + j] = j < n ? dist_key(dist[o + j], cand[o + j]) : kEmpty;
}

/**
 * Every row of keys [rows, width] sorted ascending in place (width a power of two, one workgroup per row).
 * Tiles of C blockDim keys are sorted in registers; for rows wider than a tile the bitonic steps whose
 * partners lie in other tiles run over global memory, each followed by a barrier.
 */
template <int C>
__global__ __launch_bounds__(256) void sort_rows_kernel(uint64_t* __restrict__ keys, int width)
{
  __shared__ uint64_t xch[C * 256];
  uint64_t* row  = keys + static_cast<int64_t>(blockIdx.x) * width;
  const int tile = C * static_cast<int>(blockDim.x);
  const int t    = threadIdx.x;
  // every step of the sizes up to a tile stays inside the tile: one pass over the tiles
  for (int base = 0; base < width; base += tile) {
    uint64_t k[C];
#pragma unroll
    for (int j = 0; j < C; j++)
      k[j] = row[base + C * t + j];
    for (int size = 2; size <= tile; size <<= 1)
      for (int st = size >> 1; st > 0; st >>= 1)
        bitonic_step<C>(k, xch, base, size, st);
#pragma unroll
    for (int j = 0; j < C; j++)
      row[base + C * t + j] = k[j];
  }
  __syncthreads();
  for (int size = 2 * tile; size <= width; size <<= 1) {
    int stride = size >> 1;
    for (; stride >= tile; stride >>= 1) {  // partners in other tiles: through global memory
      for (int i = t; i < width; i += blockDim.x) {
        const int p = i ^ stride;
        if (p > i) {
          const uint64_t a = row[i], b = row[p];
          if ((a > b) == ((i & size) == 0)) {
            row[i] = b;
            row[p] = a;
          }
        }
      }
      __syncthreads();
    }
    for (int base = 0; base < width; base += tile) {  // the rest of this size inside each tile
      uint64_t k[C];
#pragma unroll
      for (int j = 0; j < C; j++)
        k[j] = row[base + C * t + j];
      for (int st = stride; st > 0; st >>= 1)
        bitonic_step<C>(k, xch, base, size, st);
#pragma unroll
      for (int j = 0; j < C; j++)
        row[base + C * t + j] = k[j];
    }
    __syncthreads();
  }
}

/**
 * The pool of each query [pool keys]: its kept list (none when fresh), then its first min(R, n) sorted
 * candidates, with exact distances (vectors non-null) or their sketch distances, the empty key after.
 */
template <int LX>
__global__ __launch_bounds__(kKeepThreads) void pool_keys_kernel(
  const uint64_t* __restrict__ sorted, const int* __restrict__ nin, int W, const __half* __restrict__ vectors, int D,
  const float* __restrict__ Q, int R, const long long* __restrict__ si, const float* __restrict__ sd, int KO,
  bool fresh, int pool, uint64_t* __restrict__ out)
{
  const int q = blockIdx.x;
  extern __shared__ float sq[];
  __shared__ int sid[kMaxSketchKO];
  __shared__ float sdist[kMaxSketchKO];
  const uint64_t* sk   = sorted + static_cast<int64_t>(q) * W;
  const int ns         = min(R, min(nin[q], W));
  const long long* pb  = si + static_cast<int64_t>(q) * KO;
  const float* pdv     = sd + static_cast<int64_t>(q) * KO;
  uint64_t* po         = out + static_cast<int64_t>(q) * pool;
  for (int i = threadIdx.x; i < pool; i += blockDim.x) {
    uint64_t v = kEmpty;
    if (i < KO) {
      if (!fresh && pb[i] >= 0) v = dist_key(pdv[i], pb[i]);
    } else if (i - KO < ns && vectors == nullptr) {
      v = sk[i - KO];
    }
    po[i] = v;
  }
  if (vectors == nullptr) return;
  for (int i = threadIdx.x; i < D; i += blockDim.x)
    sq[i] = Q[static_cast<int64_t>(q) * D + i];
  for (int i = threadIdx.x; i < ns; i += blockDim.x)
    sid[i] = static_cast<int>(sk[i] & 0xffffffffULL);
  __syncthreads();
  exact_distances<LX>(sid, ns, vectors, D, sq, sdist);
  for (int i = threadIdx.x; i < ns; i += blockDim.x)
    po[KO + i] = dist_key(sdist[i], sid[i]);
}

/** The first KO distinct keys of every sorted pool into the kept list, padded with (-1, +inf): one wavefront
 * per query, the distinct keys placed by ballot counts. */
__global__ __launch_bounds__(64) void keep_distinct_kernel(const uint64_t* __restrict__ pooled, int pool, int KO,
                                                          long long* __restrict__ si, float* __restrict__ sd)
{
  const int q = blockIdx.x, lane = threadIdx.x;
  const uint64_t* key = pooled + static_cast<int64_t>(q) * pool;
  long long* pb       = si + static_cast<int64_t>(q) * KO;
  float* pd           = sd + static_cast<int64_t>(q) * KO;
  int at              = 0;
  for (int i0 = 0; i0 < pool && at < KO; i0 += 64) {
    const int i      = i0 + lane;
    const uint64_t v = i < pool ? key[i] : kEmpty;
    const bool keep  = v != kEmpty && (i == 0 || key[i - 1] != v);
    const unsigned long long mask = __ballot(keep);
    const int o = at + __popcll(mask & ((1ULL << lane) - 1ULL));
    if (keep && o < KO) {
      pb[o] = static_cast<long long>(static_cast<unsigned>(v & 0xffffffffULL));
      pd[o] = __uint_as_float(static_cast<unsigned>(v >> 32));
    }
    at += __popcll(mask);
  }
  for (int o = min(at, KO) + lane; o < KO; o += 64) {
    pb[o] = -1;
    pd[o] = INFINITY;
  }
}

/** dsort[q, i] = done[q, i] + 1 for i < off (ids >= -1 as unsigned keys), the empty key up to Ep. */
__global__ void done_keys_kernel(const long long* __restrict__ done, int E, int off, int Ep,
                                 uint64_t* __restrict__ dsort)
{
  const int q = blockIdx.x;
  for (int i = threadIdx.x; i < Ep; i += blockDim.x)
    dsort[static_cast<int64_t>(q) * Ep + i] =
      i < off ? static_cast<uint64_t>(done[static_cast<int64_t>(q) * E + i] + 1) : kEmpty;
}

/** fresh[q, i]: kept entry i of query q is an id no earlier wave expanded (a binary search of the sorted ids). */
__global__ void mark_fresh_kernel(const long long* __restrict__ si, int KO, const uint64_t* __restrict__ dsort,
                                  int Ep, int off, int64_t total, unsigned char* __restrict__ fresh)
{
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= total) return;
  const long long v = si[t];
  bool f            = v >= 0;
  if (f && off > 0) {
    const uint64_t want = static_cast<uint64_t>(v + 1);
    const uint64_t* d   = dsort + (t / KO) * Ep;
    int lo = 0, hi = off;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (d[mid] < want)
        lo = mid + 1;
      else
        hi = mid;
    }
    f = !(lo < off && d[lo] == want);
  }
  fresh[t] = f;
}

/** The first S fresh kept entries of every query as its start points (one wavefront per query, by ballots), as
 * pick_starts_kernel writes them. */
__global__ __launch_bounds__(64) void take_starts_kernel(const long long* __restrict__ si,
                                                        const unsigned char* __restrict__ fresh, int KO,
                                                        long long* __restrict__ done, int E, int off, int S,
                                                        int rowlen, int2* __restrict__ seg2)
{
  const int q = blockIdx.x, lane = threadIdx.x;
  const long long* ps     = si + static_cast<int64_t>(q) * KO;
  const unsigned char* fr = fresh + static_cast<int64_t>(q) * KO;
  long long* pd           = done + static_cast<int64_t>(q) * E;
  int at                  = 0;
  for (int i0 = 0; i0 < KO && at < S; i0 += 64) {
    const int i     = i0 + lane;
    const bool take = i < KO && fr[i];
    const unsigned long long mask = __ballot(take);
    const int o = at + __popcll(mask & ((1ULL << lane) - 1ULL));
    if (take && o < S) {
      pd[off + o]                            = ps[i];
      seg2[static_cast<int64_t>(q) * S + o] = make_int2(static_cast<int>(ps[i]), rowlen);
    }
    at += __popcll(mask);
  }
  for (int o = min(at, S) + lane; o < S; o += 64) {
    pd[off + o]                            = -1;
    seg2[static_cast<int64_t>(q) * S + o] = make_int2(0, 0);
  }
}

__global__ void take_k_kernel(const long long* __restrict__ si, const float* __restrict__ sd, int KO,
                              int k, int m, long long* __restrict__ bi, float* __restrict__ bd)
{
  int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= static_cast<int64_t>(m) * k) return;
  int64_t q = t / k, j = t % k;
  bi[t]     = si[q * KO + j];
  bd[t]     = sd[q * KO + j];
}

/** out[r] = the `words` 32-bit words of src at word offset off[r] (one workgroup per range). */
__global__ void copy_ranges_kernel(const uint32_t* __restrict__ src, const int64_t* __restrict__ off, int64_t n,
                                   int words, uint32_t* __restrict__ out)
{
  for (int64_t r = blockIdx.x; r < n; r += gridDim.x)
    for (int i = threadIdx.x; i < words; i += blockDim.x)
      out[r * words + i] = src[off[r] + i];
}

}  // namespace

// ================================================================== launchers

namespace {

/** f(std::integral_constant<int, LX>) with LX = the exact-distance lanes per row for dimension D. */
template <typename F>
void with_lx(int D, F&& f)
{
  const int nch = (D + 7) / 8;
  int lx        = 1;
  while (lx < nch && lx < 32)
    lx <<= 1;
  switch (lx) {
    case 1: f(std::integral_constant<int, 1>{}); break;
    case 2: f(std::integral_constant<int, 2>{}); break;
    case 4: f(std::integral_constant<int, 4>{}); break;
    case 8: f(std::integral_constant<int, 8>{}); break;
    case 16: f(std::integral_constant<int, 16>{}); break;
    default: f(std::integral_constant<int, 32>{}); break;
  }
}

}  // namespace


void launch_center(const float* q, const float* mu, int64_t m, int D, float* qc, __half* qh,
                   hipStream_t s)
{
  const int64_t total = m * D;
  if (total == 0) return;
  center_kernel<<<grid_for(total, 256), 256, 0, s>>>(q, mu, total, D, qc, qh);
  OCTEX_HIP(hipGetLastError());
}

void launch_pad_rows(float* q, int from, int m, int D, hipStream_t s)
{
  const int64_t total = static_cast<int64_t>(m - from) * D;
  if (total <= 0) return;
  pad_rows_kernel<<<grid_for(total, 256), 256, 0, s>>>(q, from, m, D);
  OCTEX_HIP(hipGetLastError());
}

void launch_project(const __half* qh, const __half* ucatT, const __half* shift, int m, int K, int N,
                    __half* Y, hipStream_t s)
{
  if (m == 0 || N == 0) return;
  OCTEX_EXPECTS(K >= 1, "octex: projection needs a positive dimension");
  OCTEX_EXPECTS(N % 8 == 0, "octex: projection outputs must be a multiple of 8 (copies x 8 blocks)");
  dim3 grid(static_cast<unsigned>((m + 63) / 64), static_cast<unsigned>((N + 255) / 256));
  if (K % 16 == 0)
    project_kernel<true><<<grid, 256, 0, s>>>(qh, ucatT, shift, m, K, N, Y);
  else
    project_kernel<false><<<grid, 256, 0, s>>>(qh, ucatT, shift, m, K, N, Y);
  OCTEX_HIP(hipGetLastError());
}

void launch_sketch_query(const float* qc, const float* basis, int m, int D, int S, float* qs,
                         hipStream_t s)
{
  if (static_cast<int64_t>(m) * S == 0) return;
  OCTEX_EXPECTS(D >= 1 && 16 * static_cast<int64_t>(D) * sizeof(float) <= 64 * 1024,
                "octex: the sketch query stages 16 query rows of at most 4096 values in LDS");
  dim3 grid(static_cast<unsigned>((S + 63) / 64), static_cast<unsigned>((m + 15) / 16));
  sketch_query_kernel<<<grid, 256, 16 * D * sizeof(float), s>>>(qc, basis, m, D, S, qs);
  OCTEX_HIP(hipGetLastError());
}

void launch_e8(const float* y, int64_t n, int b, float inv_f, float* p, long long* h, hipStream_t s)
{
  if (n == 0) return;
  auto g = grid_for(n, 256);
  switch (b) {
    case 1: e8_kernel<1><<<g, 256, 0, s>>>(y, n, inv_f, p, h); break;
    case 2: e8_kernel<2><<<g, 256, 0, s>>>(y, n, inv_f, p, h); break;
    case 3: e8_kernel<3><<<g, 256, 0, s>>>(y, n, inv_f, p, h); break;
    case 4: e8_kernel<4><<<g, 256, 0, s>>>(y, n, inv_f, p, h); break;
    case 5: e8_kernel<5><<<g, 256, 0, s>>>(y, n, inv_f, p, h); break;
    case 6: e8_kernel<6><<<g, 256, 0, s>>>(y, n, inv_f, p, h); break;
    case 8: e8_kernel<8><<<g, 256, 0, s>>>(y, n, inv_f, p, h); break;
    default: fail("octex: blocks must be 1-6 or 8");
  }
  OCTEX_HIP(hipGetLastError());
}

void launch_bucket_lines(const int* off, int64_t T1, const long long* keys, int64_t Mmax, int64_t CL,
                         bucket_line* lines, hipStream_t s)
{
  OCTEX_EXPECTS(T1 >= 2 && CL >= 0, "octex: bucket lines of offsets rows of at least 2 entries");
  const int64_t total = CL * (T1 - 1);
  if (total == 0) return;
  bucket_lines_kernel<<<grid_for(total, 256), 256, 0, s>>>(off, T1, keys, Mmax, total, lines);
  OCTEX_HIP(hipGetLastError());
}

void launch_probe(const __half* Y, int m, int C, int L, int B, const float* inv_f, const int* off,
                  const bucket_line* lines, int64_t T1, const long long* keys, int64_t Mmax, const int* base, int l,
                  int lr, int logT, int2* seg, hipStream_t s)
{
  const int64_t tot = static_cast<int64_t>(m) * C;
  if (tot == 0) return;
  OCTEX_EXPECTS(T1 == (int64_t{1} << logT) + 1, "octex: offsets rows must hold 2^log_buckets + 1 entries");
  OCTEX_EXPECTS(L >= 1, "octex: at least one spacing");
  // items per wavefront: about 24 wavefronts per CU over the whole grid (6 per SIMD, what the registers allow; 16
  // and 32 measured slower), at least one item per lane
  static const int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    return n;
  }();
  const int64_t chunk = std::max<int64_t>(64, (tot + int64_t{24} * cus - 1) / (int64_t{24} * cus));
  const int64_t waves = (tot + chunk - 1) / chunk;
  auto g              = grid_for(waves * 64, 256);
#define OCTEX_PROBE(b)                                                                                          \
  (lines != nullptr ? probe_kernel<b, true><<<g, 256, 0, s>>>(Y, m, C, L, inv_f, off, lines, T1, keys, Mmax, base, \
                                                              l, lr, logT, chunk, seg)                             \
                    : probe_kernel<b, false><<<g, 256, 0, s>>>(Y, m, C, L, inv_f, off, lines, T1, keys, Mmax,      \
                                                               base, l, lr, logT, chunk, seg))
  switch (B) {
    case 1: OCTEX_PROBE(1); break;
    case 2: OCTEX_PROBE(2); break;
    case 3: OCTEX_PROBE(3); break;
    case 4: OCTEX_PROBE(4); break;
    case 5: OCTEX_PROBE(5); break;
    case 6: OCTEX_PROBE(6); break;
    case 8: OCTEX_PROBE(8); break;
    default: fail("octex: blocks must be 1-6 or 8");
  }
#undef OCTEX_PROBE
  OCTEX_HIP(hipGetLastError());
}

auto gather_cap(int W, int nseg, int max_len) -> int
{
  return static_cast<int>(std::min<int64_t>(W, static_cast<int64_t>(nseg) * std::max(max_len, 1)));
}

auto gather_smem(int W, int S, int nseg, int max_len, bool lds_slots) -> size_t
{
  return static_cast<size_t>(nseg) * sizeof(long long) + static_cast<size_t>(W + 2 * S + nseg + 1) * sizeof(int) +
         (lds_slots ? static_cast<size_t>(gather_cap(W, nseg, max_len)) * sizeof(unsigned short) : 0);
}

namespace {

constexpr size_t kGatherLds = 160 * 1024 - 256;  // the CU's LDS less the kernel's static LDS (its state)

template <bool kBalanced>
void gather_impl(bool rows, const int2* seg, int nseg, int max_len, int m, const long long* list_ptr,
                 const int* table, int table_len, int64_t n, const signed char* code, int pitch, const float* scale,
                 const float* qs, int S, int W, int logW, int* cand, float* dist, int* nout, earlier_rows er,
                 int* nknown, hipStream_t s)
{
  OCTEX_EXPECTS(pitch >= S && pitch % 16 == 0, "octex: sketch rows are at least S bytes apart, 16-byte aligned");
  if (m == 0) return;
  OCTEX_EXPECTS(nseg >= 1, "octex: a gather needs at least one segment per query");
  OCTEX_EXPECTS(max_len >= 0, "octex: segment lengths are non-negative");
  OCTEX_EXPECTS(W == (1 << logW) && W <= kMaxHash, "octex: hash set size");
  OCTEX_EXPECTS(S % 16 == 0 && S >= 16 && S <= 512, "octex: sketch width: a multiple of 16, <= 512");
  const bool lds_slots = gather_smem(W, S, nseg, max_len, true) <= kGatherLds;  // else the slots go to cand
  const size_t smem    = gather_smem(W, S, nseg, max_len, lds_slots);
  OCTEX_EXPECTS(smem <= kGatherLds, "octex: gather needs %zu bytes of LDS (max 160 KiB)", smem);
  const int cap = gather_cap(W, nseg, max_len);
  OCTEX_EXPECTS(er.count >= 0 && er.count <= 2 && (er.count == 0 || rows), "octex: earlier rows of a row gather");
  for (int r = 0; r < er.count; r++)
    OCTEX_EXPECTS(er.cand[r] != nullptr && er.dist[r] != nullptr && er.n[r] != nullptr && er.W[r] >= 1 &&
                    er.cand[r] != cand && er.dist[r] != dist,
                  "octex: an earlier row set is another batch row set");
  int Lr = 1;  // the reference's lanes per candidate: the next power of two >= S / 16, at most 32
  while (Lr < S / 16 && Lr < 32)
    Lr <<= 1;
  auto go = [&](auto rows_tag, auto lr_tag) {
    constexpr bool kRowsTag = decltype(rows_tag)::value;
    constexpr int LR        = decltype(lr_tag)::value;
    auto launch             = [&](auto kernel) {
      allow_lds(reinterpret_cast<const void*>(kernel), smem);
      kernel<<<m, kRowsTag ? kGatherRowThreads : kGatherListThreads, smem, s>>>(
        seg, nseg, list_ptr, table, table_len, n, code, scale, qs, S, pitch, W, logW, cap, cand, dist, nout, er,
        nknown);
    };
    if (lds_slots)
      launch(&gather_kernel<kRowsTag, LR, true, kBalanced>);
    else
      launch(&gather_kernel<kRowsTag, LR, false, kBalanced>);
  };
  auto by_lr = [&](auto rows_tag) {
    switch (Lr) {
      case 1: go(rows_tag, std::integral_constant<int, 1>{}); break;
      case 2: go(rows_tag, std::integral_constant<int, 2>{}); break;
      case 4: go(rows_tag, std::integral_constant<int, 4>{}); break;
      case 8: go(rows_tag, std::integral_constant<int, 8>{}); break;
      case 16: go(rows_tag, std::integral_constant<int, 16>{}); break;
      default: go(rows_tag, std::integral_constant<int, 32>{}); break;
    }
  };
  if (rows)
    by_lr(std::true_type{});
  else
    by_lr(std::false_type{});
  OCTEX_HIP(hipGetLastError());
}

/** sort_rows_kernel over rows of `width` keys (a power of two): up to 256 threads, up to 16 keys each. */
void sort_rows(uint64_t* keys, int rows, int width, hipStream_t s)
{
  if (rows == 0 || width <= 1) return;
  OCTEX_EXPECTS((width & (width - 1)) == 0, "octex: sorted rows hold a power of two keys");
  const int threads = std::min(256, width);
  const int c       = std::min(16, width / threads);
  switch (c) {
    case 1: sort_rows_kernel<1><<<rows, threads, 0, s>>>(keys, width); break;
    case 2: sort_rows_kernel<2><<<rows, threads, 0, s>>>(keys, width); break;
    case 4: sort_rows_kernel<4><<<rows, threads, 0, s>>>(keys, width); break;
    case 8: sort_rows_kernel<8><<<rows, threads, 0, s>>>(keys, width); break;
    default: sort_rows_kernel<16><<<rows, threads, 0, s>>>(keys, width); break;
  }
  OCTEX_HIP(hipGetLastError());
}

}  // namespace

void launch_gather(bool rows, const int2* seg, int nseg, int max_len, int m, const long long* list_ptr,
                   const int* table, int table_len, int64_t n, const signed char* code, int pitch,
                   const float* scale, const float* qs, int S, int W, int logW, int* cand, float* dist,
                   int* nout, hipStream_t s)
{
  gather_impl<true>(rows, seg, nseg, max_len, m, list_ptr, table, table_len, n, code, pitch, scale, qs, S, W, logW,
                    cand, dist, nout, earlier_rows{}, nullptr, s);
}

void launch_gather_reuse(const int2* seg, int nseg, int max_len, int m, const int* table, int table_len, int64_t n,
                         const signed char* code, int pitch, const float* scale, const float* qs, int S, int W,
                         int logW, int* cand, float* dist, int* nout, earlier_rows const& er, int* nknown,
                         bool balanced, hipStream_t s)
{
  (balanced ? gather_impl<true> : gather_impl<false>)(true, seg, nseg, max_len, m, nullptr, table, table_len, n, code,
                                                      pitch, scale, qs, S, W, logW, cand, dist, nout, er, nknown, s);
}

void launch_gather_segments(bool rows, const int2* seg, int nseg, int max_len, int m, const long long* list_ptr,
                            const int* table, int table_len, int64_t n, const signed char* code, int pitch,
                            const float* scale, const float* qs, int S, int W, int logW, int* cand, float* dist,
                            int* nout, hipStream_t s)
{
  gather_impl<false>(rows, seg, nseg, max_len, m, list_ptr, table, table_len, n, code, pitch, scale, qs, S, W, logW,
                     cand, dist, nout, earlier_rows{}, nullptr, s);
}

void launch_unfused_keep(const int* cand, const float* dist, const int* nin, int m, int W, const __half* vectors,
                         int D, const float* Q, int R, int KO, int pool, bool fresh, uint64_t* ukey, uint64_t* upool,
                         long long* si, float* sd, hipStream_t s)
{
  if (m == 0) return;
  OCTEX_EXPECTS(R >= 1 && R <= kMaxSketchKO && KO >= 1 && KO + R <= pool && (pool & (pool - 1)) == 0,
                "octex: unfused merge pools: kept + reranked keys in a power of two");
  OCTEX_EXPECTS(vectors == nullptr || R <= kMaxRerank, "octex: rerank in [1, 512] and max(starts, k) + rerank <= 1024");
  cand_keys_kernel<<<m, 256, 0, s>>>(cand, dist, nin, W, ukey);
  OCTEX_HIP(hipGetLastError());
  sort_rows(ukey, m, W, s);
  with_lx(D, [&](auto lx) {
    pool_keys_kernel<decltype(lx)::value><<<m, kKeepThreads, vectors != nullptr ? D * sizeof(float) : 0, s>>>(
      ukey, nin, W, vectors, D, Q, R, si, sd, KO, fresh, pool, upool);
  });
  OCTEX_HIP(hipGetLastError());
  sort_rows(upool, m, pool, s);
  keep_distinct_kernel<<<m, 64, 0, s>>>(upool, pool, KO, si, sd);
  OCTEX_HIP(hipGetLastError());
}

void launch_unfused_pick(const long long* si, int m, int KO, long long* done, int E, int off, int S, int rowlen,
                         uint64_t* dsort, int Ep, unsigned char* fresh, int2* seg2, hipStream_t s)
{
  if (m == 0) return;
  OCTEX_EXPECTS(KO <= kMaxSketchKO && off <= kMaxExpanded && off + S <= E && off <= Ep,
                "octex: starts * (waves - 1) <= 6144");
  if (off > 0) {
    done_keys_kernel<<<m, 256, 0, s>>>(done, E, off, Ep, dsort);
    OCTEX_HIP(hipGetLastError());
    sort_rows(dsort, m, Ep, s);
  }
  const int64_t total = int64_t{m} * KO;
  mark_fresh_kernel<<<grid_for(total, 256), 256, 0, s>>>(si, KO, dsort, Ep, off, total, fresh);
  OCTEX_HIP(hipGetLastError());
  take_starts_kernel<<<m, 64, 0, s>>>(si, fresh, KO, done, E, off, S, rowlen, seg2);
  OCTEX_HIP(hipGetLastError());
}

void launch_rerank_keep(const int* cand, const float* dist, const int* nin, int m, int W, const __half* vectors, int D,
                        const float* Q, int R, int KO, long long* si, float* sd, bool fresh, int* hist, int H, int hoff,
                        bool hstore, int* nskip, hipStream_t s)
{
  if (m == 0) return;
  OCTEX_EXPECTS(R >= 1 && R <= kMaxRerank && KO + R <= kMaxKeepSort && KO >= 1,
                "octex: rerank in [1, 512] and max(starts, k) + rerank <= 1024");
  OCTEX_EXPECTS(D % 2 == 0, "octex: the dimension must be even");
  OCTEX_EXPECTS(hoff >= 0 && (hist != nullptr || (hoff == 0 && !hstore)) && (!hstore || hoff + R <= H) && hoff <= H,
                "octex: the selected-id history must hold this round's offset and ids");
  // 128 threads a query (16 queries in flight per CU): measured at 100M rows with the history skip, the waves'
  // launches 0.155 / 0.125 ms on 256 threads, 0.141 / 0.096 ms on 128.  Rounds of many long rows (R D >= 2^15: 512
  // rows of 960 at gist1m) take 256, twice the rows in flight
  const int nt      = static_cast<int64_t>(R) * D >= kWideRerank ? 256 : kRerankThreads;
  const int hslots  = !fresh && hoff > 0 ? hist_slots(hoff) : 0;
  const size_t smem = rerank_lds_bytes(R, KO, D, nt, hslots);
  const int c       = keys_per_thread(KO + R, nt);
  with_lx(D, [&](auto lx) {
    constexpr int LX = decltype(lx)::value;
    auto go          = [&](auto kernel) {
      allow_lds(reinterpret_cast<const void*>(kernel), smem);
      kernel<<<m, nt, smem, s>>>(cand, dist, nin, W, vectors, D, Q, R, KO, si, sd, fresh, hist, H, hoff, hstore, hslots,
                                 nskip);
    };
    auto by_c = [&](auto nt_tag) {
      constexpr int NT = decltype(nt_tag)::value;
      switch (c) {
        case 1: go(&rerank_keep_kernel<LX, NT, 1>); break;
        case 2: go(&rerank_keep_kernel<LX, NT, 2>); break;
        case 4: go(&rerank_keep_kernel<LX, NT, 4>); break;
        default: go(&rerank_keep_kernel<LX, NT, 8>); break;
      }
    };
    if (nt == 256)
      by_c(std::integral_constant<int, 256>{});
    else
      by_c(std::integral_constant<int, kRerankThreads>{});
  });
  OCTEX_HIP(hipGetLastError());
}

void launch_sketch_keep(const int* cand, const float* dist, const int* nin, int m, int W, int KO,
                        long long* si, float* sd, bool fresh, hipStream_t s)
{
  if (m == 0) return;
  OCTEX_EXPECTS(KO >= 1 && KO <= kMaxSketchKO, "octex: max(starts, k) must be <= 1024 with sketch_rank");
  sketch_keep_kernel<<<m, 512, 0, s>>>(cand, dist, nin, W, KO, si, sd, fresh);
  OCTEX_HIP(hipGetLastError());
}

void launch_pick_starts(const long long* si, int m, int KO, long long* done, int E, int off, int S,
                        int rowlen, int2* seg2, hipStream_t s)
{
  if (m == 0) return;
  OCTEX_EXPECTS(KO <= kMaxSketchKO && off <= kMaxExpanded && off + S <= E,
                "octex: starts * (waves - 1) <= 6144");
  // the set of the off ids earlier waves expanded, sized to them (a wave's own LDS, so more workgroups per CU)
  const int nb      = pick_buckets(off);
  const size_t smem = off > 0 ? static_cast<size_t>(nb) * sizeof(int4) : 0;
  pick_starts_kernel<<<m, 256, smem, s>>>(si, KO, done, E, off, S, rowlen, seg2, nb);
  OCTEX_HIP(hipGetLastError());
}

void launch_final_rerank(const long long* si, int m, int KO, int R, const __half* vectors, int D,
                         const float* Q, int k, long long* bi, float* bd, hipStream_t s)
{
  if (m == 0) return;
  OCTEX_EXPECTS(R >= k && R <= kMaxRerank && R <= KO,
                "octex: final_rerank 0 (sketch order) or k <= final_rerank <= 512");
  with_lx(D, [&](auto lx) {
    final_rerank_kernel<decltype(lx)::value>
      <<<m, kKeepThreads, D * sizeof(float), s>>>(si, KO, R, vectors, D, Q, k, bi, bd);
  });
  OCTEX_HIP(hipGetLastError());
}

void launch_take_k(const long long* si, const float* sd, int m, int KO, int k, long long* bi,
                   float* bd, hipStream_t s)
{
  const int64_t total = static_cast<int64_t>(m) * k;
  if (total == 0) return;
  take_k_kernel<<<grid_for(total, 256), 256, 0, s>>>(si, sd, KO, k, m, bi, bd);
  OCTEX_HIP(hipGetLastError());
}

void launch_copy_ranges(const uint32_t* src, const int64_t* off, int64_t n, int words, uint32_t* out,
                        hipStream_t s)
{
  if (n == 0 || words == 0) return;
  copy_ranges_kernel<<<static_cast<unsigned>(std::min<int64_t>(n, 65536)), 64, 0, s>>>(src, off, n, words, out);
  OCTEX_HIP(hipGetLastError());
}

}  // namespace cuvs::neighbors::octex::detail
