// Stage entry points: one search kernel per call on caller-provided device buffers (for the parity
// tests; see octex_amd/octex_amd.h).  Each call checks its arguments, launches, and waits.

#include "common.hpp"
#include "kernels.hpp"

#include <cuvs/core/c_api.h>
#include <octex_amd/octex_amd.h>

#include <algorithm>
#include <exception>
#include <vector>

namespace {

using namespace cuvs::neighbors::octex::detail;

template <typename Fn>
auto run(void* stream, Fn fn) -> cuvsError_t
{
  try {
    auto s = static_cast<hipStream_t>(stream);
    fn(s);
    OCTEX_HIP(hipStreamSynchronize(s));
    cuvsSetLastErrorText(nullptr);
    return CUVS_SUCCESS;
  } catch (std::exception const& e) {
    cuvsSetLastErrorText(e.what());
  } catch (...) {
    cuvsSetLastErrorText("unknown exception");
  }
  return CUVS_ERROR;
}

void need(const void* p, const char* what)
{
  OCTEX_EXPECTS(p != nullptr, "octex: %s is NULL", what);
}

}  // namespace

extern "C" cuvsError_t octexStageCenter(const float* q, const float* mu, int64_t m, int32_t D, float* qc,
                                        void* qh, void* stream)
{
  return run(stream, [&](hipStream_t s) {
    need(q, "q"), need(mu, "mu"), need(qc, "qc"), need(qh, "qh");
    launch_center(q, mu, m, D, qc, static_cast<__half*>(qh), s);
  });
}

extern "C" cuvsError_t octexStageProject(const void* qh, const void* ucatT, const void* shift, int32_t m,
                                         int32_t K, int32_t N, void* Y, void* stream)
{
  return run(stream, [&](hipStream_t s) {
    need(qh, "qh"), need(ucatT, "ucatT"), need(shift, "shift"), need(Y, "Y");
    OCTEX_EXPECTS(m >= 0 && K >= 1 && N >= 0, "octex: projection shape");
    launch_project(static_cast<const __half*>(qh), static_cast<const __half*>(ucatT),
                   static_cast<const __half*>(shift), m, K, N, static_cast<__half*>(Y), s);
  });
}

extern "C" cuvsError_t octexStageSketchQuery(const float* qc, const float* basis, int32_t m, int32_t D,
                                             int32_t S, float* qs, void* stream)
{
  return run(stream, [&](hipStream_t s) {
    need(qc, "qc"), need(basis, "basis"), need(qs, "qs");
    launch_sketch_query(qc, basis, m, D, S, qs, s);
  });
}

extern "C" cuvsError_t octexStageE8(const float* y, int64_t n, int32_t b, float inv_f, float* p, int64_t* h,
                                    void* stream)
{
  return run(stream, [&](hipStream_t s) {
    need(y, "y"), need(p, "p"), need(h, "h");
    launch_e8(y, n, b, inv_f, p, reinterpret_cast<long long*>(h), s);
  });
}

extern "C" cuvsError_t octexStageProbe(const void* Y, int32_t m, int32_t C, int32_t L, int32_t B,
                                       const float* inv_f, const int32_t* off, int64_t T1, const int64_t* keys,
                                       int64_t Mmax, const int32_t* base, int32_t l, int32_t lr, int32_t logT,
                                       int32_t* seg, void* stream)
{
  return run(stream, [&](hipStream_t s) {
    need(Y, "Y"), need(inv_f, "inv_f"), need(off, "offsets"), need(keys, "keys"), need(base, "base");
    need(seg, "seg");
    OCTEX_EXPECTS(m >= 0 && C >= 1 && L >= 1 && logT >= 1 && logT <= 30, "octex: probe shape");
    launch_probe(static_cast<const __half*>(Y), m, C, L, B, inv_f, off, nullptr, T1,
                 reinterpret_cast<const long long*>(keys), Mmax, base, l, lr, logT, reinterpret_cast<int2*>(seg),
                 s);
  });
}

extern "C" cuvsError_t octexStageProbeLines(const void* Y, int32_t m, int32_t C, int32_t L, int32_t B,
                                            const float* inv_f, const int32_t* off, int64_t T1, const int64_t* keys,
                                            int64_t Mmax, const int32_t* base, int32_t l, int32_t lr, int32_t logT,
                                            int32_t* seg, void* stream)
{
  return run(stream, [&](hipStream_t s) {
    need(Y, "Y"), need(inv_f, "inv_f"), need(off, "offsets"), need(keys, "keys"), need(base, "base");
    need(seg, "seg");
    OCTEX_EXPECTS(m >= 0 && C >= 1 && L >= 1 && logT >= 1 && logT <= 30 && T1 == (int64_t{1} << logT) + 1,
                  "octex: probe shape");
    dbuf lines(static_cast<size_t>(C) * L * (T1 - 1) * sizeof(bucket_line));
    launch_bucket_lines(off, T1, reinterpret_cast<const long long*>(keys), Mmax, int64_t{C} * L,
                        lines.as<bucket_line>(), s);
    launch_probe(static_cast<const __half*>(Y), m, C, L, B, inv_f, off, lines.as<bucket_line>(), T1,
                 reinterpret_cast<const long long*>(keys), Mmax, base, l, lr, logT, reinterpret_cast<int2*>(seg),
                 s);
    OCTEX_HIP(hipStreamSynchronize(s));  // before the lines are freed
  });
}

extern "C" cuvsError_t octexStageGather(int32_t rows, const int32_t* seg, int32_t nseg, int32_t m,
                                        const int32_t* lists, int64_t stride, const int32_t* table,
                                        int32_t table_len, int64_t n, const int8_t* code, const float* scale, const float* qs,
                                        int32_t S, int32_t W, int32_t* cand, float* dist, int32_t* nout,
                                        void* stream)
{
  return run(stream, [&](hipStream_t s) {
    need(seg, "seg"), need(code, "code"), need(scale, "scale"), need(qs, "qs");
    need(cand, "cand"), need(dist, "dist"), need(nout, "nout");
    if (rows)
      need(table, "table");
    else
      need(lists, "lists");
    OCTEX_EXPECTS(W >= (1 << kMinLogHash) && (W & (W - 1)) == 0, "octex: W must be a power of two >= 2048");
    dbuf ptrs;
    if (!rows) {  // the pointer of every copy's lists: lists + c * stride
      std::vector<long long> hp(nseg);
      for (int c = 0; c < nseg; c++)
        hp[c] = reinterpret_cast<long long>(lists + static_cast<int64_t>(c) * stride);
      ptrs = dbuf(hp.size() * sizeof(long long));
      upload(ptrs.ptr, hp.data(), ptrs.size, s);
    }
    int max_len = 0;  // the longest segment (sizes the candidate list)
    {
      std::vector<int2> hs(static_cast<size_t>(m) * nseg);
      if (!hs.empty()) OCTEX_HIP(hipMemcpy(hs.data(), seg, hs.size() * sizeof(int2), hipMemcpyDefault));
      for (auto const& v : hs)
        max_len = std::max(max_len, v.y);
    }
    launch_gather(rows != 0, reinterpret_cast<const int2*>(seg), nseg, max_len, m, ptrs.as<long long>(), table, table_len,
                  n, reinterpret_cast<const signed char*>(code), S, scale, qs, S, W, log2_ceil(W), cand, dist,
                  nout, s);
    OCTEX_HIP(hipStreamSynchronize(s));
  });
}

extern "C" cuvsError_t octexStageGatherReuse(const int32_t* seg, int32_t nseg, int32_t m, const int32_t* table,
                                             int32_t table_len, int64_t n, const int8_t* code, const float* scale,
                                             const float* qs, int32_t S, int32_t W, int32_t* cand, float* dist,
                                             int32_t* nout, int32_t nold, const int32_t* const* old_cand,
                                             const float* const* old_dist, const int32_t* const* old_n,
                                             const int32_t* old_W, int32_t* nknown, void* stream)
{
  return run(stream, [&](hipStream_t s) {
    need(seg, "seg"), need(table, "table"), need(code, "code"), need(scale, "scale"), need(qs, "qs");
    need(cand, "cand"), need(dist, "dist"), need(nout, "nout");
    OCTEX_EXPECTS(W >= (1 << kMinLogHash) && (W & (W - 1)) == 0, "octex: W must be a power of two >= 2048");
    OCTEX_EXPECTS(nold >= 0 && nold <= 2 && (nold == 0 || (old_cand && old_dist && old_n && old_W)),
                  "octex: at most two earlier rows");
    earlier_rows er;
    for (int r = 0; r < nold; r++) {
      er.cand[r] = old_cand[r];
      er.dist[r] = old_dist[r];
      er.n[r]    = old_n[r];
      er.W[r]    = old_W[r];
    }
    er.count = nold;
    int max_len = 0;  // the longest segment (sizes the candidate list)
    {
      std::vector<int2> hs(static_cast<size_t>(m) * nseg);
      if (!hs.empty()) OCTEX_HIP(hipMemcpy(hs.data(), seg, hs.size() * sizeof(int2), hipMemcpyDefault));
      for (auto const& v : hs)
        max_len = std::max(max_len, v.y);
    }
    launch_gather_reuse(reinterpret_cast<const int2*>(seg), nseg, max_len, m, table, table_len, n,
                        reinterpret_cast<const signed char*>(code), S, scale, qs, S, W, log2_ceil(W), cand, dist,
                        nout, er, nknown, true, s);
    OCTEX_HIP(hipStreamSynchronize(s));
  });
}

extern "C" cuvsError_t octexStageRerankKeepHistory(const int32_t* cand, const float* dist, const int32_t* nin,
                                                   int32_t m, int32_t W, const void* vectors, int32_t D, const float* Q,
                                                   int32_t R, int32_t KO, int64_t* si, float* sd, int32_t fresh,
                                                   int32_t* hist, int32_t H, int32_t hoff, int32_t hstore,
                                                   int32_t* nskip, void* stream)
{
  return run(stream, [&](hipStream_t s) {
    need(cand, "cand"), need(dist, "dist"), need(nin, "nin"), need(vectors, "vectors"), need(Q, "Q");
    need(si, "si"), need(sd, "sd");
    launch_rerank_keep(cand, dist, nin, m, W, static_cast<const __half*>(vectors), D, Q, R, KO,
                       reinterpret_cast<long long*>(si), sd, fresh != 0, hist, H, hoff, hstore != 0, nskip, s);
  });
}

extern "C" cuvsError_t octexStageRerankKeep(const int32_t* cand, const float* dist, const int32_t* nin,
                                            int32_t m, int32_t W, const void* vectors, int32_t D, const float* Q,
                                            int32_t R, int32_t KO, int64_t* si, float* sd, int32_t fresh,
                                            void* stream)
{
  return octexStageRerankKeepHistory(cand, dist, nin, m, W, vectors, D, Q, R, KO, si, sd, fresh, nullptr, 0, 0, 0,
                                     nullptr, stream);
}

extern "C" cuvsError_t octexStageSketchKeep(const int32_t* cand, const float* dist, const int32_t* nin,
                                            int32_t m, int32_t W, int32_t KO, int64_t* si, float* sd,
                                            int32_t fresh, void* stream)
{
  return run(stream, [&](hipStream_t s) {
    need(cand, "cand"), need(dist, "dist"), need(nin, "nin"), need(si, "si"), need(sd, "sd");
    launch_sketch_keep(cand, dist, nin, m, W, KO, reinterpret_cast<long long*>(si), sd, fresh != 0, s);
  });
}

extern "C" cuvsError_t octexStagePickStarts(const int64_t* si, int32_t m, int32_t KO, int64_t* done, int32_t E,
                                            int32_t off, int32_t S, int32_t rowlen, int32_t* seg2, void* stream)
{
  return run(stream, [&](hipStream_t s) {
    need(si, "si"), need(done, "done"), need(seg2, "seg2");
    launch_pick_starts(reinterpret_cast<const long long*>(si), m, KO, reinterpret_cast<long long*>(done), E,
                       off, S, rowlen, reinterpret_cast<int2*>(seg2), s);
  });
}

extern "C" cuvsError_t octexStageFinalRerank(const int64_t* si, int32_t m, int32_t KO, int32_t R,
                                             const void* vectors, int32_t D, const float* Q, int32_t k,
                                             int64_t* bi, float* bd, void* stream)
{
  return run(stream, [&](hipStream_t s) {
    need(si, "si"), need(vectors, "vectors"), need(Q, "Q"), need(bi, "bi"), need(bd, "bd");
    launch_final_rerank(reinterpret_cast<const long long*>(si), m, KO, R, static_cast<const __half*>(vectors),
                        D, Q, k, reinterpret_cast<long long*>(bi), bd, s);
  });
}

extern "C" cuvsError_t octexStageTakeK(const int64_t* si, const float* sd, int32_t m, int32_t KO, int32_t k,
                                       int64_t* bi, float* bd, void* stream)
{
  return run(stream, [&](hipStream_t s) {
    need(si, "si"), need(sd, "sd"), need(bi, "bi"), need(bd, "bd");
    OCTEX_EXPECTS(k <= KO, "octex: k <= KO");
    launch_take_k(reinterpret_cast<const long long*>(si), sd, m, KO, k, reinterpret_cast<long long*>(bi), bd,
                  s);
  });
}
