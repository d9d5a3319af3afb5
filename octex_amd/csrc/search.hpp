// Search plans of one MI355X: batch buffers and the hipGraph of one (batch, k, search parameters).
#pragma once

#include "common.hpp"

#include <cuvs/neighbors/octex.hpp>

#include <memory>
#include <mutex>
#include <string>
#include <vector>

namespace cuvs::neighbors::octex::detail {

struct index_impl;

struct plan {
  search_params sp;
  int m = 0, k = 0, KO = 0, lr = 0, R1 = 0, R2 = 0, FR = 0;
  int W = 0, logW = 0, W2 = 0, logW2 = 0;  // hash-set / candidate capacity per query
  // qbuf f32 [m, D] queries; qc f32 / qh f16 [m, D] centered; Y f16 [m, C 8b]; qs f32 [m, S];
  // seg int2 [m, C]; cand i32 / dist f32 [m, W], nin [m]; si i64 / sd f32 [m, KO] kept list;
  // done i64 [m, starts waves]; seg2 int2 [m, starts]; cand2 / dist2 [m, W2], n2 [m]; bi / bd [m, k]
  dbuf qbuf, qc, qh, Y, qs, seg, cand, dist, nin, si, sd, done, seg2, cand2, dist2, n2, bi, bd;
  hipGraphExec_t graph = nullptr;
  hipEvent_t ev_in = nullptr, ev_out = nullptr;
  hipStream_t stream = nullptr;  // the index's stream, where every batch of the plan runs
  int64_t buffer_bytes = 0;
  plan() = default;
  plan(plan const&) = delete;
  ~plan();
};

auto plan_key(search_params const& sp, int m, int k) -> std::string;
auto get_plan(index_impl& ix, search_params const& sp, int m, int k) -> std::shared_ptr<plan>;
/** One batch of the plan on stream s (graph replay, or direct launches without a graph). */
void run_batch(index_impl const& ix, plan const& pl, hipStream_t s);
/** Work counters of one profiled batch (summed over its m queries; per wave for the waves). */
struct profile_counters {
  int64_t seg_hits = 0, entries1 = 0, distinct1 = 0, reranked1 = 0;
  int64_t starts2[16] = {}, distinct2[16] = {}, reranked2[16] = {};
  int64_t hit_level[8] = {};  // probe hits by level (0 the finest); misses are m C - seg_hits
};
void profile_batch(index_impl& ix, plan& pl, int reps, std::vector<std::string>& names, std::vector<double>& ms,
                   profile_counters& cnt);
/**
 * The batch loop (search.cu:816-961).  resident: the queries of the previous call stay in place in
 * the plan's query buffer (one batch only) and nothing is copied in or out (the timing protocol).
 */
void search_impl(raft::resources const& res, search_params const& sp, index const& idx, const float* queries,
                 int64_t nq, int64_t qdim, int64_t* neighbors, float* distances, int64_t k, bool host_out,
                 bool resident);

}  // namespace cuvs::neighbors::octex::detail
