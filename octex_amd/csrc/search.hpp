// Search plans of one MI355X: the shape of one (batch, k, search parameters), its per-batch buffers and the
// hipGraph of one batch.
#pragma once

#include "common.hpp"

#include <cuvs/neighbors/octex.hpp>

#include <hip/hip_fp16.h>

#include <cstdint>
#include <memory>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

namespace cuvs::neighbors::octex::detail {

struct index_impl;

/** Batch size, k, parameters and the sizes derived from them (search.cu:619-655, 677-693). */
struct plan_shape {
  search_params sp;
  int m = 0, k = 0, KO = 0, lr = 0, R1 = 0, R2 = 0, FR = 0;
  int W = 0, logW = 0, W2 = 0, logW2 = 0;  // hash-set / candidate capacity per query
  int pool1 = 0, pool2 = 0;                // unfused merge (fused_merge = false): keys per query's pool
  int Ep = 0;                              // unfused start points: sorted expanded ids per query
  int H = 0;  // the fused rerank's history of selected ids per query: rerank + wave_rerank (waves - 1)
  // wave row sets: wave w writes set w % ring.  With reuse the first wave takes the scores its candidates have in the
  // first round's row; with reuse_later the later waves too, from set (w - 1) % ring (ring 2) and, with reuse_first,
  // from the first round's row
  int ring         = 1;
  bool reuse       = false;
  bool reuse_later = false;
  bool reuse_first = false;
};

/**
 * Where every per-batch array lies (device addresses): qbuf f32 [m, D] queries; qc f32 / qh f16 [m, D]
 * centred; Y f16 [m, C 8b]; qs f32 [m, S]; seg int2 [m, C]; cand i32 / dist f32 [m, W], nin [m]; si i64 /
 * sd f32 [m, KO] kept list; done i64 [m, starts waves]; seg2 int2 [m, starts]; cand2 / dist2 [m, W2], n2 [m], one
 * set per ring slot; nknown [m] (candidates of the last wave gather whose scores came from earlier rows); nskip [m]
 * (selected candidates the last wave's rerank did not rerank again); hist i32 [m, H] (the fused rerank's
 * selected ids of every round but the last); bi i64 / bd f32 [m, k]; with fused_merge = false also ukey u64
 * [m, max(W, W2)] candidate keys (sorted in place), upool u64 [m, max(pool1, pool2)] pools, dsort i64 [m, Ep] the ids
 * earlier waves expanded, sorted (Ep the power of two >= starts (waves - 1)), and fresh u8 [m, KO].
 */
constexpr int kRing = 2;  // wave row sets at most

struct batch_buffers {
  float *qbuf = nullptr, *qc = nullptr, *qs = nullptr, *dist = nullptr, *sd = nullptr, *bd = nullptr;
  float* dist2[kRing] = {};
  __half *qh = nullptr, *Y = nullptr;
  int2 *seg = nullptr, *seg2 = nullptr;
  int *cand = nullptr, *nin = nullptr, *nknown = nullptr, *nskip = nullptr, *hist = nullptr;
  int* cand2[kRing] = {};
  int* n2[kRing]    = {};
  long long *si = nullptr, *done = nullptr, *bi = nullptr;
  uint64_t *ukey = nullptr, *upool = nullptr, *dsort = nullptr;
  unsigned char* fresh = nullptr;
};

/** The shape of a plan, with the reference's parameter limits checked (the same texts). */
auto make_shape(index_impl const& ix, search_params const& sp, int m, int k) -> plan_shape;

/**
 * Lay the batch buffers of shape `sh` out in one block starting at `base` (each at a 256-byte boundary) and
 * return the block's size in bytes; with base null only the size is computed.  Every buffer is written by a
 * batch before it is read, so a block needs no clearing.
 */
auto carve_buffers(index_impl const& ix, plan_shape const& sh, void* base, batch_buffers* out) -> size_t;

/** A named batch buffer ("queries", "Y", "seg", "cand", ..., as octexIndexCopyPlanBuffer lists) and its bytes. */
auto named_buffer(index_impl const& ix, plan_shape const& sh, batch_buffers const& b, std::string const& name)
  -> std::pair<const void*, size_t>;

/** One plan: its shape, one block of batch buffers and the graph of a whole batch on the index's stream. */
struct plan {
  plan_shape shape;
  dbuf block;
  batch_buffers buf;
  hipGraphExec_t graph = nullptr;
  hipEvent_t ev_in = nullptr, ev_out = nullptr;
  hipStream_t stream = nullptr;  // the index's stream, where every batch of the plan runs
  plan() = default;
  plan(plan const&) = delete;
  ~plan();
};

auto plan_key(search_params const& sp, int m, int k) -> std::string;
auto get_plan(index_impl& ix, search_params const& sp, int m, int k) -> std::shared_ptr<plan>;
/** One batch of the plan on stream s (graph replay, or direct launches without a graph). */
void run_batch(index_impl const& ix, plan const& pl, hipStream_t s);
/** The launches of one batch over the buffers b on stream s, in order (direct launches, no graph). */
void launch_batch(index_impl const& ix, plan_shape const& sh, batch_buffers const& b, hipStream_t s);
/** Work counters of one profiled batch (summed over its m queries; per wave for the waves). */
struct profile_counters {
  int64_t seg_hits = 0, entries1 = 0, distinct1 = 0, reranked1 = 0;
  int64_t starts2[16] = {}, distinct2[16] = {}, reranked2[16] = {};
  int64_t known2[16] = {};    // wave candidates whose scores came from earlier rows
  int64_t oldread2[16] = {};  // entries of earlier rows each wave gather read
  int64_t skipped2[16] = {};  // selected wave candidates not reranked again (an earlier round reranked them)
  int64_t hit_level[8] = {};  // probe hits by level (0 the finest); misses are m C - seg_hits
};
void profile_batch(index_impl& ix, plan& pl, int reps, std::vector<std::string>& names, std::vector<double>& ms,
                   profile_counters& cnt);
/**
 * The search of device queries [nq, dim] into device neighbors / distances [nq, k] on stream s with every batch
 * buffer in the library's file-scope scratch array of the index's GPU (search_noalloc.cpp): no device allocation,
 * direct launches, no graph.  A batch whose buffers exceed the array is an error.
 */
void search_no_alloc(search_params const& sp, index const& idx, const float* queries, int64_t nq, int64_t dim,
                     int64_t k, int64_t* neighbors, float* distances, hipStream_t s);
/**
 * The batch loop (search.cu:816-961).  resident: the queries of the previous call stay in place in
 * the plan's query buffer (one batch only) and nothing is copied in or out (the timing protocol).
 */
void search_impl(raft::resources const& res, search_params const& sp, index const& idx, const float* queries,
                 int64_t nq, int64_t qdim, int64_t* neighbors, float* distances, int64_t k, bool host_out,
                 bool resident);

}  // namespace cuvs::neighbors::octex::detail
