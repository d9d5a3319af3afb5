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
#include <cstdlib>
#include <cstring>
#include <functional>
#include <string>
#include <type_traits>

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

auto make_shape(index_impl const& ix, search_params const& sp, int m, int k) -> plan_shape
{
  plan_shape sh;
  sh.sp = sp;
  sh.m  = m;
  sh.k  = k;
  sh.KO = std::max(sp.starts, k);
  sh.lr = std::min(sp.read, ix.list_len);
  sh.R1 = sp.rerank;
  sh.R2 = sp.wave_rerank;
  sh.FR = std::min(sp.final_rerank, sh.KO);
  const int S = sp.starts, C = ix.copies;
  // parameter limits (search.cu:638-656, 681-692): the same checks and texts
  OCTEX_EXPECTS(m >= 1 && k >= 1, "octex: a batch of at least one query and k >= 1");
  OCTEX_EXPECTS(sp.read >= 1 && sp.starts >= 1 && sp.waves >= 0, "octex: read, starts >= 1 and waves >= 0");
  OCTEX_EXPECTS(sp.waves == 0 || ix.table_len > 0, "octex: waves need the neighbor table");
  OCTEX_EXPECTS(sh.KO <= (sp.sketch_rank ? kMaxSketchKO : kMaxRerank),
                "octex: max(starts, k) must be <= 512 (1024 with sketch_rank)");
  OCTEX_EXPECTS(sp.sketch_rank || (sp.rerank >= 1 && sp.rerank <= kMaxRerank && sh.KO + sp.rerank <= kMaxKeepSort),
                "octex: rerank in [1, 512] and max(starts, k) + rerank <= 1024");
  OCTEX_EXPECTS(sp.sketch_rank || sp.waves == 0 ||
                  (sp.wave_rerank >= 1 && sp.wave_rerank <= kMaxRerank && sh.KO + sp.wave_rerank <= kMaxKeepSort),
                "octex: wave_rerank in [1, 512] and max(starts, k) + wave_rerank <= 1024");
  OCTEX_EXPECTS(!sp.sketch_rank || sh.FR == 0 || (k <= sh.FR && sh.FR <= kMaxRerank),
                "octex: final_rerank 0 (sketch order) or k <= final_rerank <= 512");
  OCTEX_EXPECTS(sp.waves <= 1 || S * (sp.waves - 1) <= kMaxExpanded, "octex: starts * (waves - 1) <= 6144");
  const int log_max = log2_ceil(kMaxHash);
  OCTEX_EXPECTS(int64_t{C} * sh.lr <= kMaxHash, "octex: copies x read too large for the shared-memory hash set");
  sh.logW = std::clamp(log2_ceil(static_cast<int64_t>(std::ceil(C * sh.lr * 1.5f))), kMinLogHash, log_max);
  sh.W    = 1 << sh.logW;
  if (sp.waves > 0) {
    OCTEX_EXPECTS(int64_t{S} * ix.table_len <= kMaxHash,
                  "octex: starts x table_len too large for the shared-memory hash set");
    sh.logW2 = std::clamp(log2_ceil(static_cast<int64_t>(std::ceil(S * ix.table_len * 1.5f))), kMinLogHash, log_max);
    sh.W2    = 1 << sh.logW2;
    // the fused exact rerank keeps the ids every round but the last selects, to skip them when selected again
    if (sp.fused_merge && !sp.sketch_rank) sh.H = sh.R1 + sh.R2 * (sp.waves - 1);
    // the first wave's gather takes the scores of its candidates found in the first round's row.  OCTEX_GATHER_REUSE
    // (read when a plan is made): 0, no wave does; prev, every wave from the previous round's row; all, later waves
    // from the first round's and the previous wave's rows.  Measured at 100M rows (no graphs): the first wave
    // 0.737 -> 0.690 ms; the second, from the first wave's row, 0.474 -> 0.485 ms although 43 % of its candidates are
    // found there (the scan of 2,858 entries a query costs what the 729 rows it saves do)
    const char* e          = std::getenv("OCTEX_GATHER_REUSE");
    const std::string mode = e != nullptr ? e : "1";
    sh.reuse               = mode != "0";
    sh.reuse_later         = mode == "prev" || mode == "all";
    sh.reuse_first         = mode == "all";
    sh.ring                = sh.reuse_later && sp.waves > 1 ? 2 : 1;
  }
  if (!sp.fused_merge) {  // the pools of the unfused merge: the kept list and the R best candidates
    auto pool = [&](int R) { return 1 << log2_ceil(sh.KO + (sp.sketch_rank ? sh.KO : R)); };
    sh.pool1 = pool(sh.R1);
    sh.pool2 = sp.waves > 0 ? pool(sh.R2) : 0;
    sh.Ep    = sp.waves > 1 ? 1 << log2_ceil(int64_t{S} * (sp.waves - 1)) : 0;
  }
  return sh;
}

auto carve_buffers(index_impl const& ix, plan_shape const& sh, void* base, batch_buffers* out) -> size_t
{
  const int64_t m = sh.m, D = ix.dim, C = ix.copies, S = ix.sketch_width, st = sh.sp.starts;
  const int64_t wdt = int64_t{8} * ix.blocks * C;
  size_t at = 0;
  auto take = [&](auto*& p, int64_t count) {
    using T = std::remove_pointer_t<std::remove_reference_t<decltype(p)>>;
    at = (at + 255) / 256 * 256;
    p  = base != nullptr && count > 0 ? reinterpret_cast<T*>(static_cast<char*>(base) + at) : nullptr;
    at += static_cast<size_t>(std::max<int64_t>(count, 0)) * sizeof(T);
  };
  batch_buffers b;
  take(b.qbuf, m * D);
  take(b.qc, m * D);
  take(b.qh, m * D);
  take(b.Y, m * wdt);
  take(b.qs, m * S);
  take(b.seg, m * C);
  take(b.cand, m * sh.W);
  take(b.dist, m * sh.W);
  take(b.nin, m);
  take(b.si, m * sh.KO);
  take(b.sd, m * sh.KO);
  if (sh.sp.waves > 0) {
    take(b.done, m * st * sh.sp.waves);
    take(b.seg2, m * st);
    for (int r = 0; r < sh.ring; r++) {
      take(b.cand2[r], m * sh.W2);
      take(b.dist2[r], m * sh.W2);
      take(b.n2[r], m);
    }
    take(b.nknown, m);
    take(b.nskip, m);
    take(b.hist, m * sh.H);
  }
  take(b.bi, m * sh.k);
  take(b.bd, m * sh.k);
  if (!sh.sp.fused_merge) {
    take(b.ukey, m * std::max(sh.W, sh.W2));
    take(b.upool, m * std::max(sh.pool1, sh.pool2));
    take(b.dsort, m * sh.Ep);
    take(b.fresh, m * sh.KO);
  }
  if (out != nullptr) *out = b;
  return (at + 255) / 256 * 256;
}

auto named_buffer(index_impl const& ix, plan_shape const& sh, batch_buffers const& b, std::string const& n)
  -> std::pair<const void*, size_t>
{
  const size_t m = static_cast<size_t>(sh.m), D = static_cast<size_t>(ix.dim), C = static_cast<size_t>(ix.copies);
  const size_t S = static_cast<size_t>(ix.sketch_width), st = static_cast<size_t>(sh.sp.starts);
  const size_t wv = static_cast<size_t>(sh.sp.waves), W = static_cast<size_t>(sh.W), W2 = static_cast<size_t>(sh.W2);
  const size_t KO = static_cast<size_t>(sh.KO), k = static_cast<size_t>(sh.k);
  const int last   = wv > 0 ? static_cast<int>((wv - 1) % static_cast<size_t>(sh.ring)) : 0;  // the last wave's rows
  const size_t wdt = size_t{8} * static_cast<size_t>(ix.blocks) * C;
  const std::pair<const char*, std::pair<const void*, size_t>> all[] = {
    {"queries", {b.qbuf, m * D * 4}}, {"qc", {b.qc, m * D * 4}},     {"qh", {b.qh, m * D * 2}},
    {"Y", {b.Y, m * wdt * 2}},        {"qs", {b.qs, m * S * 4}},     {"seg", {b.seg, m * C * 8}},
    {"cand", {b.cand, m * W * 4}},    {"dist", {b.dist, m * W * 4}}, {"nin", {b.nin, m * 4}},
    {"si", {b.si, m * KO * 8}},       {"sd", {b.sd, m * KO * 4}},    {"done", {b.done, m * st * wv * 8}},
    {"seg2", {b.seg2, m * st * 8}},   {"cand2", {b.cand2[last], m * W2 * 4}}, {"dist2", {b.dist2[last], m * W2 * 4}},
    {"n2", {b.n2[last], wv > 0 ? m * 4 : 0}}, {"nknown", {b.nknown, wv > 0 ? m * 4 : 0}},
    {"nskip", {b.nskip, wv > 0 ? m * 4 : 0}},
    {"hist", {b.hist, m * static_cast<size_t>(sh.H) * 4}}, {"bi", {b.bi, m * k * 8}},  {"bd", {b.bd, m * k * 4}},
  };
  for (auto const& [name, where] : all)
    if (n == name) return where.first != nullptr ? where : std::pair<const void*, size_t>(nullptr, 0);
  fail("octex: unknown plan buffer %s", n.c_str());
}

namespace {

/** One stage of a batch: its name (as profiled) and its launch. */
struct stage {
  std::string name;
  std::function<void()> launch;
};

/**
 * The launches of one batch in order (search.cu:294-518): the first round over all copies with the
 * best KO kept in si / sd, then the waves over the neighbor table, then the best k into bi / bd.  The
 * reference's ablation switches pick other kernels with the same results: balanced_gather = false reads
 * every segment whole by one wavefront (gather_warp_kernel, search_kernels.cuh:687-792), fused_merge =
 * false keeps and picks start points through sorts in global memory (search.cu:213-291).
 */
auto batch_stages(index_impl const& ix, plan_shape const& sh, batch_buffers const& b, hipStream_t s)
  -> std::vector<stage>
{
  const int D = static_cast<int>(ix.dim), S = ix.sketch_width, C = ix.copies, m = sh.m;
  const bool balanced = sh.sp.balanced_gather, fused = sh.sp.fused_merge, sketch_rank = sh.sp.sketch_rank;
  std::vector<stage> out;
  auto add = [&](const char* n, std::function<void()> f) { out.push_back({n, std::move(f)}); };
  add("center", [&ix, b, s, m, D] { launch_center(b.qbuf, ix.mean.as<float>(), m, D, b.qc, b.qh, s); });
  add("project", [&ix, b, s, m, D, C] {
    launch_project(b.qh, ix.ucatT.as<__half>(), ix.shift.as<__half>(), m, D, C * 8 * ix.blocks, b.Y, s);
  });
  add("sketch_query", [&ix, b, s, m, D, S] { launch_sketch_query(b.qc, ix.basis.as<float>(), m, D, S, b.qs, s); });
  add("probe", [&ix, b, sh, s, m, C] {
    launch_probe(b.Y, m, C, ix.levels(), ix.blocks, ix.inv_f.as<float>(), ix.offsets.as<int>(),
                 ix.lines.as<bucket_line>(), ix.T1, ix.keys.as<long long>(), ix.mmax, ix.base.as<int>(), ix.list_len,
                 sh.lr, ix.log_buckets, b.seg, s);
  });
  // stage names as profiled: the ablation paths are marked, so a profile shows which kernels ran
  const std::string whole = balanced ? "" : "_whole", unfused = fused ? "" : "_unfused";
  auto gather = [&](std::string const& name, bool rows, const int2* seg, int nseg, int max_len, int W, int logW,
                    int* cand, float* dist, int* n) {
    add((name + whole).c_str(), [&ix, b, s, m, S, rows, seg, nseg, max_len, W, logW, cand, dist, n, balanced] {
      (balanced ? launch_gather : launch_gather_segments)(
        rows, seg, nseg, max_len, m, rows ? nullptr : ix.list_ptr.as<long long>(), rows ? ix.rows() : nullptr,
        ix.table_len, ix.n, ix.code(), ix.sketch_pitch, ix.scale.as<float>(), b.qs, S, W, logW, cand, dist, n, s);
    });
  };
  // the kept list merged with a round's candidates: fused (one kernel) or through global-memory sorts.  The fused
  // rerank of round r (0 the first) keeps its selected ids at hist[:, off(r) ..) for the later rounds, which skip them:
  // off(0) = 0, off(r) = rerank + (r - 1) wave_rerank
  auto keep = [&](std::string const& base_name, const int* cand, const float* dist, const int* n, int W, int R,
                  int pool, int round) {
    const bool fresh = round == 0;
    const int hoff   = round == 0 ? 0 : sh.R1 + (round - 1) * sh.R2;
    const bool store = sh.H > 0 && round < sh.sp.waves;
    const std::string nm = base_name + unfused;
    const char* name     = nm.c_str();
    if (fused && sketch_rank)
      add(name, [b, sh, s, m, cand, dist, n, W, fresh] {
        launch_sketch_keep(cand, dist, n, m, W, sh.KO, b.si, b.sd, fresh, s);
      });
    else if (fused)
      add(name, [&ix, b, sh, s, m, D, cand, dist, n, W, R, fresh, hoff, store] {
        launch_rerank_keep(cand, dist, n, m, W, ix.vecs(), D, b.qbuf, R, sh.KO, b.si, b.sd, fresh,
                           sh.H > 0 ? b.hist : nullptr, sh.H, sh.H > 0 ? hoff : 0, store, fresh ? nullptr : b.nskip, s);
      });
    else
      add(name, [&ix, b, sh, s, m, D, cand, dist, n, W, R, pool, fresh, sketch_rank] {
        launch_unfused_keep(cand, dist, n, m, W, sketch_rank ? nullptr : ix.vecs(), D, b.qbuf,
                            sketch_rank ? sh.KO : R, sh.KO, pool, fresh, b.ukey, b.upool, b.si, b.sd, s);
      });
  };
  gather("gather_lists", false, b.seg, C, sh.lr, sh.W, sh.logW, b.cand, b.dist, b.nin);
  keep(sketch_rank ? "sketch_keep" : "rerank_keep", b.cand, b.dist, b.nin, sh.W, sh.R1, sh.pool1, 0);
  const int st = sh.sp.starts, nw = sh.sp.waves;
  for (int wv = 0; wv < nw; wv++) {
    add(("pick_starts" + unfused).c_str(), [&ix, b, sh, s, m, st, nw, wv, fused] {
      if (fused)
        launch_pick_starts(b.si, m, sh.KO, b.done, st * nw, wv * st, st, ix.table_len, b.seg2, s);
      else
        launch_unfused_pick(b.si, m, sh.KO, b.done, st * nw, wv * st, st, ix.table_len, b.dsort, sh.Ep, b.fresh,
                            b.seg2, s);
    });
    const int r = wv % sh.ring;
    if (sh.reuse && (wv == 0 || sh.reuse_later)) {
      earlier_rows er;  // the first round's row, and the previous wave's
      auto add_row = [&er](const int* c, const float* d, const int* n, int W) {
        er.cand[er.count] = c;
        er.dist[er.count] = d;
        er.n[er.count]    = n;
        er.W[er.count]    = W;
        er.count++;
      };
      if (wv == 0 || sh.reuse_first) add_row(b.cand, b.dist, b.nin, sh.W);
      if (wv > 0) {
        const int rp = (wv - 1) % sh.ring;
        add_row(b.cand2[rp], b.dist2[rp], b.n2[rp], sh.W2);
      }
      add(("gather_rows" + whole).c_str(), [&ix, b, sh, s, m, S, st, r, er, balanced] {
        launch_gather_reuse(b.seg2, st, ix.table_len, m, ix.rows(), ix.table_len, ix.n, ix.code(), ix.sketch_pitch,
                            ix.scale.as<float>(), b.qs, S, sh.W2, sh.logW2, b.cand2[r], b.dist2[r], b.n2[r], er,
                            b.nknown, balanced, s);
      });
    } else {
      gather("gather_rows", true, b.seg2, st, ix.table_len, sh.W2, sh.logW2, b.cand2[r], b.dist2[r], b.n2[r]);
    }
    keep(sketch_rank ? "sketch_keep_wave" : "rerank_keep_wave", b.cand2[r], b.dist2[r], b.n2[r], sh.W2, sh.R2,
         sh.pool2, wv + 1);
  }
  if (sketch_rank && sh.FR > 0)
    add("final_rerank", [&ix, b, sh, s, m, D] {
      launch_final_rerank(b.si, m, sh.KO, sh.FR, ix.vecs(), D, b.qbuf, sh.k, b.bi, b.bd, s);
    });
  else
    add("take_k", [b, sh, s, m] { launch_take_k(b.si, b.sd, m, sh.KO, sh.k, b.bi, b.bd, s); });
  return out;
}

auto make_plan(index_impl& ix, search_params const& sp, int m, int k) -> std::shared_ptr<plan>
{
  auto pl    = std::make_shared<plan>();
  pl->stream = ix.stream;
  pl->shape  = make_shape(ix, sp, m, k);
  pl->block  = dbuf(carve_buffers(ix, pl->shape, nullptr, nullptr));
  carve_buffers(ix, pl->shape, pl->block.ptr, &pl->buf);
  OCTEX_HIP(hipEventCreateWithFlags(&pl->ev_in, hipEventDisableTiming));
  OCTEX_HIP(hipEventCreateWithFlags(&pl->ev_out, hipEventDisableTiming));
  // one eager run on zeroed buffers (code objects loaded, LDS limits set), then the capture of the whole batch.
  // Only the index's own stream is drained first: the index arrays were complete when its load or build returned,
  // and other streams (another index's searches) are not waited for
  hipStream_t s = ix.stream;
  OCTEX_HIP(hipStreamSynchronize(s));
  OCTEX_HIP(hipMemsetAsync(pl->block.ptr, 0, pl->block.size, s));
  launch_batch(ix, pl->shape, pl->buf, s);
  OCTEX_HIP(hipStreamSynchronize(s));
  if (sp.use_graph) {
    hipGraph_t graph = nullptr;
    OCTEX_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    try {
      launch_batch(ix, pl->shape, pl->buf, s);
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

void launch_batch(index_impl const& ix, plan_shape const& sh, batch_buffers const& b, hipStream_t s)
{
  for (auto& st : batch_stages(ix, sh, b, s))
    st.launch();
}

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
    launch_batch(ix, pl.shape, pl.buf, s);
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
  auto const& b    = pl->buf;
  const int64_t D  = ix.dim;
  hipStream_t s    = ix.stream;
  hipStream_t call = raft::resource::get_cuda_stream(res);
  OCTEX_HIP(hipEventRecord(pl->ev_in, call));
  OCTEX_HIP(hipStreamWaitEvent(s, pl->ev_in, 0));
  for (int64_t b0 = 0; b0 < nq; b0 += m) {
    const int n = static_cast<int>(std::min<int64_t>(m, nq - b0));
    if (!resident) {
      OCTEX_HIP(hipMemcpyAsync(b.qbuf, queries + b0 * D, sizeof(float) * n * D, hipMemcpyDefault, s));
      if (n < m) launch_pad_rows(b.qbuf, n, m, static_cast<int>(D), s);
    }
    run_batch(ix, *pl, s);
    if (!resident) {
      OCTEX_HIP(hipMemcpyAsync(neighbors + b0 * k, b.bi, sizeof(int64_t) * n * k, hipMemcpyDefault, s));
      OCTEX_HIP(hipMemcpyAsync(distances + b0 * k, b.bd, sizeof(float) * n * k, hipMemcpyDefault, s));
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
  auto const& sh = pl.shape;
  auto const& b  = pl.buf;
  const int C = ix.copies, m = sh.m, st = sh.sp.starts;
  auto steps    = batch_stages(ix, sh, b, s);
  std::vector<hipEvent_t> ev(steps.size() + 1);
  for (auto& e : ev)
    OCTEX_HIP(hipEventCreate(&e));
  names.clear();
  ms.assign(steps.size(), 0.0);
  for (auto& st2 : steps)
    names.push_back(st2.name);
  cnt = profile_counters{};
  std::vector<int> nin(m), n2(m), nk(m), prev2(m);  // prev2: the previous wave's counts
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
        OCTEX_HIP(hipMemcpy(segh.data(), b.seg, sizeof(int2) * m * C, hipMemcpyDeviceToHost));
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
        OCTEX_HIP(hipMemcpy(nin.data(), b.nin, sizeof(int) * m, hipMemcpyDeviceToHost));
        for (int v : nin) {
          cnt.distinct1 += v;
          cnt.reranked1 += std::min(v, sh.sp.sketch_rank ? sh.KO : sh.R1);
        }
      } else if (nm == "pick_starts") {
        wv++;
        OCTEX_HIP(hipMemcpy(segh.data(), b.seg2, sizeof(int2) * m * st, hipMemcpyDeviceToHost));
        for (int64_t j = 0; j < int64_t{m} * st; j++)
          cnt.starts2[wv] += segh[j].y > 0;
      } else if (nm == "gather_rows") {
        const int slot = wv % sh.ring;
        OCTEX_HIP(hipMemcpy(n2.data(), b.n2[slot], sizeof(int) * m, hipMemcpyDeviceToHost));
        OCTEX_HIP(hipMemcpy(nk.data(), b.nknown, sizeof(int) * m, hipMemcpyDeviceToHost));
        for (int q = 0; q < m; q++) {
          cnt.distinct2[wv] += n2[q];
          cnt.reranked2[wv] += std::min(n2[q], sh.sp.sketch_rank ? sh.KO : sh.R2);
          if (!sh.reuse || (wv > 0 && !sh.reuse_later)) continue;
          cnt.known2[wv] += nk[q];
          cnt.oldread2[wv] += (wv == 0 || sh.reuse_first ? std::min(nin[q], sh.W) : 0) +
                              (wv > 0 ? std::min(prev2[q], sh.W2) : 0);
        }
        prev2 = n2;
      } else if (nm == "rerank_keep_wave") {
        OCTEX_HIP(hipMemcpy(nk.data(), b.nskip, sizeof(int) * m, hipMemcpyDeviceToHost));
        for (int v : nk)
          cnt.skipped2[wv] += v;
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
