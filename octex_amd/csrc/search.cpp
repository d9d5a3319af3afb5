// octex::search for one MI355X (the reference: search.cu:294-518 first_round / wave_round, :619-814
// plans, :816-961 the batch loop).  A plan holds the batch buffers of one (batch, k, search
// parameters) and one hipGraph of the whole batch: center, projection, sketch query, probe, gather,
// keep, then the waves (pick starts, gather rows, keep) and the best k.  Batches larger than the
// captured size are split; the last partial batch is padded with copies of its first query.

#include "search.hpp"

#include "common.hpp"
#include "index_impl.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <cmath>
#include <functional>
#include <cstring>
#include <string>

namespace cuvs::neighbors::octex {

namespace detail {

index_impl::~index_impl()
{
  plans.clear();
  if (stream != nullptr) {
    (void)hipSetDevice(device);
    (void)hipStreamSynchronize(stream);
    (void)hipStreamDestroy(stream);
  }
}

plan::~plan()
{
  // an evicted plan can be released by a search whose batch is still running on the index's stream: its
  // graph and buffers go only after that work
  if (stream != nullptr) (void)hipStreamSynchronize(stream);
  if (graph != nullptr) (void)hipGraphExecDestroy(graph);
  if (ev_in != nullptr) (void)hipEventDestroy(ev_in);
  if (ev_out != nullptr) (void)hipEventDestroy(ev_out);
}

namespace {

template <typename T>
auto alloc(int64_t count, int fill = -2) -> dbuf
{
  dbuf b(static_cast<size_t>(std::max<int64_t>(count, 1)) * sizeof(T));
  if (fill != -2) OCTEX_HIP(hipMemset(b.ptr, fill, b.size));
  return b;
}

/** One stage of a batch: its name (as profiled) and its launch on the index's stream. */
struct stage {
  std::string name;
  std::function<void()> launch;
};

/**
 * The launches of one batch in order (search.cu:294-518): the first round over all copies with the
 * best KO kept in si / sd, then the waves over the neighbor table, then the best k into bi / bd.
 */
auto batch_stages(index_impl const& ix, plan const& pl, hipStream_t s) -> std::vector<stage>
{
  const int D = static_cast<int>(ix.dim), S = ix.sketch_width, C = ix.copies, m = pl.m;
  std::vector<stage> out;
  auto add = [&](const char* n, std::function<void()> f) { out.push_back({n, std::move(f)}); };
  add("center", [&ix, &pl, s, m, D] {
    launch_center(pl.qbuf.as<float>(), ix.mean.as<float>(), m, D, pl.qc.as<float>(), pl.qh.as<__half>(), s);
  });
  add("project", [&ix, &pl, s, m, D, C] {
    launch_project(pl.qh.as<__half>(), ix.ucatT.as<__half>(), ix.shift.as<__half>(), m, D, C * 8 * ix.blocks,
                   pl.Y.as<__half>(), s);
  });
  add("sketch_query", [&ix, &pl, s, m, D, S] {
    launch_sketch_query(pl.qc.as<float>(), ix.basis.as<float>(), m, D, S, pl.qs.as<float>(), s);
  });
  add("probe", [&ix, &pl, s, m, C] {
    launch_probe(pl.Y.as<__half>(), m, C, ix.levels(), ix.blocks, ix.inv_f.as<float>(), ix.offsets.as<int>(), ix.T1,
                 ix.keys.as<long long>(), ix.mmax, ix.base.as<int>(), ix.list_len, pl.lr, ix.log_buckets,
                 pl.seg.as<int2>(), s);
  });
  add("gather_lists", [&ix, &pl, s, m, S, C] {
    launch_gather(false, pl.seg.as<int2>(), C, pl.lr, m, ix.list_ptr.as<long long>(), nullptr, 0, ix.n, ix.code(),
                  ix.sketch_pitch, ix.scale.as<float>(), pl.qs.as<float>(), S, pl.W, pl.logW, pl.cand.as<int>(),
                  pl.dist.as<float>(), pl.nin.as<int>(), s);
  });
  if (pl.sp.sketch_rank)
    add("sketch_keep", [&pl, s, m] {
      launch_sketch_keep(pl.cand.as<int>(), pl.dist.as<float>(), pl.nin.as<int>(), m, pl.W, pl.KO,
                         pl.si.as<long long>(), pl.sd.as<float>(), true, s);
    });
  else
    add("rerank_keep", [&ix, &pl, s, m, D] {
      launch_rerank_keep(pl.cand.as<int>(), pl.dist.as<float>(), pl.nin.as<int>(), m, pl.W, ix.vecs(), D,
                         pl.qbuf.as<float>(), pl.R1, pl.KO, pl.si.as<long long>(), pl.sd.as<float>(), true, s);
    });
  const int st = pl.sp.starts, nw = pl.sp.waves;
  for (int wv = 0; wv < nw; wv++) {
    add("pick_starts", [&ix, &pl, s, m, st, nw, wv] {
      launch_pick_starts(pl.si.as<long long>(), m, pl.KO, pl.done.as<long long>(), st * nw, wv * st, st,
                         ix.table_len, pl.seg2.as<int2>(), s);
    });
    add("gather_rows", [&ix, &pl, s, m, S, st] {
      launch_gather(true, pl.seg2.as<int2>(), st, ix.table_len, m, nullptr, ix.rows(), ix.table_len, ix.n, ix.code(),
                    ix.sketch_pitch, ix.scale.as<float>(), pl.qs.as<float>(), S, pl.W2, pl.logW2, pl.cand2.as<int>(),
                    pl.dist2.as<float>(), pl.n2.as<int>(), s);
    });
    if (pl.sp.sketch_rank)
      add("sketch_keep_wave", [&pl, s, m] {
        launch_sketch_keep(pl.cand2.as<int>(), pl.dist2.as<float>(), pl.n2.as<int>(), m, pl.W2, pl.KO,
                           pl.si.as<long long>(), pl.sd.as<float>(), false, s);
      });
    else
      add("rerank_keep_wave", [&ix, &pl, s, m, D] {
        launch_rerank_keep(pl.cand2.as<int>(), pl.dist2.as<float>(), pl.n2.as<int>(), m, pl.W2, ix.vecs(), D,
                           pl.qbuf.as<float>(), pl.R2, pl.KO, pl.si.as<long long>(), pl.sd.as<float>(), false, s);
      });
  }
  if (pl.sp.sketch_rank && pl.FR > 0)
    add("final_rerank", [&ix, &pl, s, m, D] {
      launch_final_rerank(pl.si.as<long long>(), m, pl.KO, pl.FR, ix.vecs(), D, pl.qbuf.as<float>(), pl.k,
                          pl.bi.as<long long>(), pl.bd.as<float>(), s);
    });
  else
    add("take_k", [&pl, s, m] {
      launch_take_k(pl.si.as<long long>(), pl.sd.as<float>(), m, pl.KO, pl.k, pl.bi.as<long long>(), pl.bd.as<float>(),
                    s);
    });
  return out;
}

void launch_batch(index_impl const& ix, plan const& pl, hipStream_t s)
{
  for (auto& st : batch_stages(ix, pl, s))
    st.launch();
}

auto make_plan(index_impl& ix, search_params const& sp, int m, int k) -> std::shared_ptr<plan>
{
  auto pl   = std::make_shared<plan>();
  pl->stream = ix.stream;
  pl->sp    = sp;
  pl->m     = m;
  pl->k     = k;
  pl->KO    = std::max(sp.starts, k);
  pl->lr    = std::min(sp.read, ix.list_len);
  pl->R1    = sp.rerank;
  pl->R2    = sp.wave_rerank;
  pl->FR    = std::min(sp.final_rerank, pl->KO);
  const int D = static_cast<int>(ix.dim), S = sp.starts, sw = ix.sketch_width, C = ix.copies;
  // parameter limits (search.cu:638-656, 681-692): the same checks and texts
  OCTEX_EXPECTS(sp.read >= 1 && sp.starts >= 1 && sp.waves >= 0, "octex: read, starts >= 1 and waves >= 0");
  OCTEX_EXPECTS(sp.waves == 0 || ix.table_len > 0, "octex: waves need the neighbor table");
  OCTEX_EXPECTS(pl->KO <= (sp.sketch_rank ? kMaxSketchKO : kMaxRerank),
                "octex: max(starts, k) must be <= 512 (1024 with sketch_rank)");
  OCTEX_EXPECTS(sp.sketch_rank || (sp.rerank >= 1 && sp.rerank <= kMaxRerank && pl->KO + sp.rerank <= kMaxKeepSort),
                "octex: rerank in [1, 512] and max(starts, k) + rerank <= 1024");
  OCTEX_EXPECTS(sp.sketch_rank || sp.waves == 0 ||
                  (sp.wave_rerank >= 1 && sp.wave_rerank <= kMaxRerank && pl->KO + sp.wave_rerank <= kMaxKeepSort),
                "octex: wave_rerank in [1, 512] and max(starts, k) + wave_rerank <= 1024");
  OCTEX_EXPECTS(!sp.sketch_rank || pl->FR == 0 || (k <= pl->FR && pl->FR <= kMaxRerank),
                "octex: final_rerank 0 (sketch order) or k <= final_rerank <= 512");
  OCTEX_EXPECTS(sp.waves <= 1 || S * (sp.waves - 1) <= kMaxExpanded, "octex: starts * (waves - 1) <= 6144");
  const int log_max = log2_ceil(kMaxHash);
  OCTEX_EXPECTS(int64_t{C} * pl->lr <= kMaxHash, "octex: copies x read too large for the shared-memory hash set");
  pl->logW = std::clamp(log2_ceil(static_cast<int64_t>(std::ceil(C * pl->lr * 1.5f))), kMinLogHash, log_max);
  pl->W    = 1 << pl->logW;
  if (sp.waves > 0) {
    OCTEX_EXPECTS(int64_t{S} * ix.table_len <= kMaxHash,
                  "octex: starts x table_len too large for the shared-memory hash set");
    pl->logW2 = std::clamp(log2_ceil(static_cast<int64_t>(std::ceil(S * ix.table_len * 1.5f))), kMinLogHash, log_max);
    pl->W2    = 1 << pl->logW2;
  }
  const int wdt = 8 * ix.blocks * C;
  pl->qbuf      = alloc<float>(int64_t{m} * D, 0);
  pl->qc        = alloc<float>(int64_t{m} * D);
  pl->qh        = alloc<__half>(int64_t{m} * D);
  pl->Y         = alloc<__half>(int64_t{m} * wdt);
  pl->qs        = alloc<float>(int64_t{m} * sw);
  pl->seg       = alloc<int2>(int64_t{m} * C);
  pl->cand      = alloc<int>(int64_t{m} * pl->W);
  pl->dist      = alloc<float>(int64_t{m} * pl->W);
  pl->nin       = alloc<int>(m);
  pl->si        = alloc<long long>(int64_t{m} * pl->KO, 0xff);
  pl->sd        = alloc<float>(int64_t{m} * pl->KO);
  if (sp.waves > 0) {
    pl->done  = alloc<long long>(int64_t{m} * S * sp.waves);
    pl->seg2  = alloc<int2>(int64_t{m} * S);
    pl->cand2 = alloc<int>(int64_t{m} * pl->W2);
    pl->dist2 = alloc<float>(int64_t{m} * pl->W2);
    pl->n2    = alloc<int>(m);
  }
  pl->bi = alloc<long long>(int64_t{m} * k);
  pl->bd = alloc<float>(int64_t{m} * k);
  for (dbuf const* b : {&pl->qbuf, &pl->qc, &pl->qh, &pl->Y, &pl->qs, &pl->seg, &pl->cand, &pl->dist,
                        &pl->nin, &pl->si, &pl->sd, &pl->done, &pl->seg2, &pl->cand2, &pl->dist2,
                        &pl->n2, &pl->bi, &pl->bd})
    pl->buffer_bytes += static_cast<int64_t>(b->size);
  OCTEX_HIP(hipEventCreateWithFlags(&pl->ev_in, hipEventDisableTiming));
  OCTEX_HIP(hipEventCreateWithFlags(&pl->ev_out, hipEventDisableTiming));
  // one eager run (code objects loaded, LDS limits set), then the capture of the whole batch
  hipStream_t s = ix.stream;
  OCTEX_HIP(hipDeviceSynchronize());
  launch_batch(ix, *pl, s);
  OCTEX_HIP(hipStreamSynchronize(s));
  if (sp.use_graph) {
    hipGraph_t graph = nullptr;
    OCTEX_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    try {
      launch_batch(ix, *pl, s);
    } catch (...) {
      hipGraph_t g2 = nullptr;
      (void)hipStreamEndCapture(s, &g2);
      if (g2 != nullptr) (void)hipGraphDestroy(g2);
      throw;
    }
    OCTEX_HIP(hipStreamEndCapture(s, &graph));
    OCTEX_HIP(hipGraphInstantiate(&pl->graph, graph, nullptr, nullptr, 0));
    OCTEX_HIP(hipGraphDestroy(graph));
  }
  return pl;
}

}  // namespace

auto plan_key(search_params const& sp, int m, int k) -> std::string
{
  return std::to_string(m) + "/" + std::to_string(k) + "/" + std::to_string(sp.read) + "/" +
         std::to_string(sp.starts) + "/" + std::to_string(sp.waves) + "/" + std::to_string(sp.rerank) +
         "/" + std::to_string(sp.wave_rerank) + "/" + std::to_string(sp.sketch_rank) + "/" +
         std::to_string(sp.final_rerank) + "/" + std::to_string(sp.balanced_gather) +
         std::to_string(sp.fused_merge) + std::to_string(sp.use_graph);
}

auto get_plan(index_impl& ix, search_params const& sp, int m, int k) -> std::shared_ptr<plan>
{
  const std::string key = plan_key(sp, m, k);
  std::lock_guard<std::mutex> lock(ix.mu);
  auto it = ix.plans.find(key);
  if (it != ix.plans.end()) return it->second;
  // one cached configuration: the previous plan's buffers go before the new ones are allocated
  ix.plans.clear();
  auto pl       = make_plan(ix, sp, m, k);
  ix.plans[key] = pl;
  return pl;
}

void run_batch(index_impl const& ix, plan const& pl, hipStream_t s)
{
  if (pl.graph != nullptr) {
    OCTEX_HIP(hipGraphLaunch(pl.graph, s));
  } else {
    launch_batch(ix, pl, s);
  }
}

void search_impl(raft::resources const& res, search_params const& sp, index const& idx, const float* queries,
                 int64_t nq, int64_t qdim, int64_t* neighbors, float* distances, int64_t k, bool host_out,
                 bool resident)
{
  auto& ix = idx.impl();
  OCTEX_EXPECTS(qdim == ix.dim, "octex: query dimension differs from the index");
  OCTEX_EXPECTS(k >= 1, "octex: k >= 1");
  if (nq == 0) return;
  int cur = 0;
  OCTEX_HIP(hipGetDevice(&cur));
  OCTEX_HIP(hipSetDevice(ix.device));
  const int m = static_cast<int>(std::min<int64_t>(std::max(sp.batch, 1), nq));
  std::unique_lock<std::mutex> run(ix.stream_mu);
  auto pl = get_plan(ix, sp, m, static_cast<int>(k));  // released before `run` on every path
  const int64_t D  = ix.dim;
  hipStream_t s    = ix.stream;
  hipStream_t call = raft::resource::get_cuda_stream(res);
  OCTEX_HIP(hipEventRecord(pl->ev_in, call));
  OCTEX_HIP(hipStreamWaitEvent(s, pl->ev_in, 0));
  for (int64_t b0 = 0; b0 < nq; b0 += m) {
    const int n = static_cast<int>(std::min<int64_t>(m, nq - b0));
    if (!resident) {
      OCTEX_HIP(hipMemcpyAsync(pl->qbuf.ptr, queries + b0 * D, sizeof(float) * n * D, hipMemcpyDefault, s));
      if (n < m) launch_pad_rows(pl->qbuf.as<float>(), n, m, static_cast<int>(D), s);
    }
    run_batch(ix, *pl, s);
    if (!resident) {
      OCTEX_HIP(hipMemcpyAsync(neighbors + b0 * k, pl->bi.ptr, sizeof(int64_t) * n * k, hipMemcpyDefault, s));
      OCTEX_HIP(hipMemcpyAsync(distances + b0 * k, pl->bd.ptr, sizeof(float) * n * k, hipMemcpyDefault, s));
    }
  }
  OCTEX_HIP(hipEventRecord(pl->ev_out, s));
  OCTEX_HIP(hipStreamWaitEvent(call, pl->ev_out, 0));
  pl.reset();  // an evicted plan goes here, with the stream lock held
  run.unlock();
  if (host_out) OCTEX_HIP(hipStreamSynchronize(call));
  OCTEX_HIP(hipSetDevice(cur));
}

/**
 * One batch of the plan launched kernel by kernel with HIP events around every launch on the index's
 * stream, `reps` times (the queries already in the plan's query buffer).  Returns the average
 * milliseconds per launch by stage name, in launch order, and the work counters of the batch.
 */
void profile_batch(index_impl& ix, plan& pl, int reps, std::vector<std::string>& names, std::vector<double>& ms,
                   profile_counters& cnt)
{
  hipStream_t s = ix.stream;
  const int C = ix.copies, m = pl.m, st = pl.sp.starts;
  auto steps    = batch_stages(ix, pl, s);
  std::vector<hipEvent_t> ev(steps.size() + 1);
  for (auto& e : ev)
    OCTEX_HIP(hipEventCreate(&e));
  names.clear();
  ms.assign(steps.size(), 0.0);
  for (auto& st2 : steps)
    names.push_back(st2.name);
  cnt = profile_counters{};
  std::vector<int> nin(m), n2(m);
  std::vector<int2> segh(static_cast<size_t>(m) * std::max(C, st));
  for (int r = 0; r < reps; r++) {
    const bool last = r + 1 == reps;
    int wv = -1;
    for (size_t i = 0; i < steps.size(); i++) {
      OCTEX_HIP(hipEventRecord(ev[i], s));
      steps[i].launch();
      OCTEX_HIP(hipEventRecord(ev[i + 1], s));
      OCTEX_HIP(hipEventSynchronize(ev[i + 1]));
      float t = 0;
      OCTEX_HIP(hipEventElapsedTime(&t, ev[i], ev[i + 1]));
      ms[i] += t / reps;
      if (!last) continue;
      // work counters of the last repetition, read between launches (outside the timed pairs)
      const std::string& nm = steps[i].name;
      if (nm == "probe") {
        OCTEX_HIP(hipMemcpy(segh.data(), pl.seg.ptr, sizeof(int2) * m * C, hipMemcpyDeviceToHost));
        const int L = ix.levels();
        std::vector<int> base(static_cast<size_t>(C) * L);
        OCTEX_HIP(hipMemcpy(base.data(), ix.base.ptr, sizeof(int) * base.size(), hipMemcpyDeviceToHost));
        for (int64_t j = 0; j < int64_t{m} * C; j++) {
          cnt.seg_hits += segh[j].y > 0;
          cnt.entries1 += segh[j].y;
          if (segh[j].y > 0) {  // the level whose rows hold the segment's cell
            const int* bc = base.data() + (j % C) * L;
            const int row = segh[j].x / ix.list_len;
            const int lv  = static_cast<int>(std::upper_bound(bc, bc + L, row) - bc) - 1;
            cnt.hit_level[std::clamp(lv, 0, 7)]++;
          }
        }
      } else if (nm == "gather_lists") {
        OCTEX_HIP(hipMemcpy(nin.data(), pl.nin.ptr, sizeof(int) * m, hipMemcpyDeviceToHost));
        for (int v : nin) {
          cnt.distinct1 += v;
          cnt.reranked1 += std::min(v, pl.sp.sketch_rank ? pl.KO : pl.R1);
        }
      } else if (nm == "pick_starts") {
        wv++;
        OCTEX_HIP(hipMemcpy(segh.data(), pl.seg2.ptr, sizeof(int2) * m * st, hipMemcpyDeviceToHost));
        for (int64_t j = 0; j < int64_t{m} * st; j++)
          cnt.starts2[wv] += segh[j].y > 0;
      } else if (nm == "gather_rows") {
        OCTEX_HIP(hipMemcpy(n2.data(), pl.n2.ptr, sizeof(int) * m, hipMemcpyDeviceToHost));
        for (int v : n2) {
          cnt.distinct2[wv] += v;
          cnt.reranked2[wv] += std::min(v, pl.sp.sketch_rank ? pl.KO : pl.R2);
        }
      }
    }
  }
  for (auto& e : ev)
    (void)hipEventDestroy(e);
}

}  // namespace detail

// ------------------------------------------------------------------ index and search (octex.hpp)

index::index(std::shared_ptr<detail::index_impl> impl) : impl_(std::move(impl)) {}
index::index(index&&) noexcept                    = default;
auto index::operator=(index&&) noexcept -> index& = default;
index::~index()                                   = default;

auto index::size() const noexcept -> int64_t { return impl_->n; }
auto index::dim() const noexcept -> int64_t { return impl_->dim; }
auto index::copies() const noexcept -> int { return impl_->copies; }
auto index::devices() const noexcept -> std::vector<int> const& { return impl_->devices; }
auto index::device_bytes() const -> std::vector<int64_t> { return {impl_->bytes}; }
auto index::impl() const noexcept -> detail::index_impl& { return *impl_; }

void search(raft::resources const& res, search_params const& params, index const& idx,
            raft::host_matrix_view<const float, int64_t, raft::row_major> queries,
            raft::host_matrix_view<int64_t, int64_t, raft::row_major> neighbors,
            raft::host_matrix_view<float, int64_t, raft::row_major> distances)
{
  OCTEX_EXPECTS(neighbors.extent(0) == queries.extent(0) && distances.extent(0) == queries.extent(0) &&
                  distances.extent(1) == neighbors.extent(1),
                "octex: output shapes");
  detail::search_impl(res, params, idx, queries.data_handle(), queries.extent(0), queries.extent(1),
                      neighbors.data_handle(), distances.data_handle(), neighbors.extent(1), true, false);
}

void search(raft::resources const& res, search_params const& params, index const& idx,
            raft::device_matrix_view<const float, int64_t, raft::row_major> queries,
            raft::device_matrix_view<int64_t, int64_t, raft::row_major> neighbors,
            raft::device_matrix_view<float, int64_t, raft::row_major> distances)
{
  OCTEX_EXPECTS(neighbors.extent(0) == queries.extent(0) && distances.extent(0) == queries.extent(0) &&
                  distances.extent(1) == neighbors.extent(1),
                "octex: output shapes");
  detail::search_impl(res, params, idx, queries.data_handle(), queries.extent(0), queries.extent(1),
                      neighbors.data_handle(), distances.data_handle(), neighbors.extent(1), false, false);
}

}  // namespace cuvs::neighbors::octex
