// Launchers of the octex search kernels for gfx950 (kernels.hip).  Every launcher checks the shapes
// its grid assumes and throws an "octex: ..." error before a launch that would not fit.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace cuvs::neighbors::octex::detail {

// limits of the per-query LDS structures (search_kernels.cuh:20-29)
constexpr int kMinLogHash     = 11;     // smallest hash set: 2^11 slots
constexpr int kMaxHash        = 32768;  // largest hash set (LDS)
constexpr int kMaxRerank      = 512;    // exact rerank depth per round
constexpr int kMaxKeepSort    = 1024;   // kept + reranked keys sorted together
constexpr int kMaxSketchKO    = 1024;   // kept entries of the sketch merge
constexpr int kPickHash       = 8192;   // hash set of the expanded start points
constexpr int kMaxExpanded    = 6144;   // start points expanded by earlier waves
constexpr int kGatherListThreads = 256;  // gathers of cell lists (first round): small hash sets, many per CU
constexpr int kGatherRowThreads  = 512;  // gathers of neighbor-table rows (waves)
constexpr int kKeepThreads    = 256;

/** log2 of the hash set of a query reading `total` entries: ceil(log2(1.5 total)) in [11, log_cap]. */
inline auto hash_log_host(int total, int log_cap) -> int
{
  if (total <= 0) return kMinLogHash;
  int64_t want = (3 * int64_t{total} + 1) / 2;
  int e        = 0;
  while ((int64_t{1} << e) < want)
    e++;
  return e < kMinLogHash ? kMinLogHash : (e > log_cap ? log_cap : e);
}

void launch_center(const float* q, const float* mu, int64_t m, int D, float* qc, __half* qh,
                   hipStream_t s);
void launch_pad_rows(float* q, int from, int m, int D, hipStream_t s);
/** Y [m, N] = qh [m, K] @ ucatT [N, K]^T + shift [N] (fp16 MFMA, fp32 accumulate, fp16 out). */
void launch_project(const __half* qh, const __half* ucatT, const __half* shift, int m, int K, int N,
                    __half* Y, hipStream_t s);
/** qs [m, S] = qc [m, D] @ basis [D, S] (fp32, sequential fma over d). */
void launch_sketch_query(const float* qc, const float* basis, int m, int D, int S, float* qs,
                         hipStream_t s);
/** E8^b points and hashes of y [n, 8b] * inv_f (the E8 decode of the probe, for tests). */
void launch_e8(const float* y, int64_t n, int b, float inv_f, float* p, long long* h, hipStream_t s);
/**
 * One bucket of a (copy, level) cell table as the probe reads it: its first key and the range [p0, p1) of its keys in
 * the level's keys (the CSR offsets off[b], off[b + 1]).  A level's probe is then one 16-byte load, and a second read
 * of the keys only when the bucket holds more than one key and the first is not the cell's.
 */
struct alignas(16) bucket_line {
  long long key0;  // keys[p0] when p1 > p0
  int p0, p1;
};
/** lines [CL, T1 - 1] of the CSR offsets off [CL, T1] into keys [CL, Mmax]. */
void launch_bucket_lines(const int* off, int64_t T1, const long long* keys, int64_t Mmax, int64_t CL,
                         bucket_line* lines, hipStream_t s);
/**
 * Segments seg [m, C] of every (query, copy): the finest level whose bucket (h & (T1 - 2), T1 - 1 = 2^logT) holds the
 * cell id h of the query's E8 point, as (first list row, lr), or (0, 0) (search_kernels.cuh:84-127).  With lines (may
 * be null) the buckets are read from them, else from off.
 */
void launch_probe(const __half* Y, int m, int C, int L, int B, const float* inv_f, const int* off,
                  const bucket_line* lines, int64_t T1, const long long* keys, int64_t Mmax, const int* base, int l,
                  int lr, int logT, int2* seg, hipStream_t s);
/** LDS bytes of a gather over `nseg` segments per query with hash sets up to W slots; lds_slots: with the
 * candidates' 16-bit slot list in LDS too (else it is kept in the query's row of cand). */
auto gather_smem(int W, int S, int nseg, int max_len, bool lds_slots) -> size_t;
/**
 * The distinct ids of every query's segments with their sketch scores into cand / dist [m, W] (ids in any order,
 * count in nout [m]).
 * Ids at or above `n` (a corrupt list or table entry) are skipped like the -1 padding.
 * Lists: segment c of a query reads copy c's lists at list_ptr[c] (a device pointer per copy).
 * code [n, pitch]: the S sketch codes of row v start at code + v * pitch.
 * max_len: no segment is longer (a query keeps at most min(W, nseg * max_len) candidates).
 */
/**
 * Up to two earlier candidate rows of a batch: ids and sketch scores cand / dist [m, W[r]], counts n [m].  A query's
 * sketch score of an id is the same in every round, so a row gather takes the scores of the candidates found there
 * instead of reading their sketch rows again.
 */
struct earlier_rows {
  const int* cand[2]    = {};
  const float* dist[2]  = {};
  const int* n[2]       = {};
  int W[2]              = {};
  int count             = 0;
};
void launch_gather(bool rows, const int2* seg, int nseg, int max_len, int m, const long long* list_ptr,
                   const int* table, int table_len, int64_t n, const signed char* code, int pitch,
                   const float* scale, const float* qs, int S, int W, int logW, int* cand, float* dist,
                   int* nout, hipStream_t s);
/**
 * launch_gather over table rows (rows = true) taking the scores of candidates found in the earlier rows `er`: those
 * candidates come last in each query's row (positions nout - nknown .. nout - 1), copied, and the others are scored as
 * launch_gather scores them.  nknown [m] (may be null) gets their count.  The earlier rows are used only when the
 * candidates' slot list fits in LDS beside the hash set (else nknown is 0).
 */
void launch_gather_reuse(const int2* seg, int nseg, int max_len, int m, const int* table, int table_len, int64_t n,
                         const signed char* code, int pitch, const float* scale, const float* qs, int S, int W,
                         int logW, int* cand, float* dist, int* nout, earlier_rows const& er, int* nknown,
                         bool balanced, hipStream_t s);
/** launch_gather without the load balance (balanced_gather = false): a wavefront reads each segment whole
 * (search_kernels.cuh:687-792).  Same arguments and results. */
void launch_gather_segments(bool rows, const int2* seg, int nseg, int max_len, int m, const long long* list_ptr,
                            const int* table, int table_len, int64_t n, const signed char* code, int pitch,
                            const float* scale, const float* qs, int S, int W, int logW, int* cand, float* dist,
                            int* nout, hipStream_t s);
/**
 * The kept list merged with a round's candidates without the fused kernels (fused_merge = false,
 * search.cu:213-253): every candidate's key into ukey [m, W] and each row sorted, the pool of the kept list
 * (none when fresh) and the R first sorted candidates with exact distances (vectors non-null; their sketch
 * distances when null) into upool [m, pool] and sorted, the first KO distinct keys into si / sd.
 */
void launch_unfused_keep(const int* cand, const float* dist, const int* nin, int m, int W, const __half* vectors,
                         int D, const float* Q, int R, int KO, int pool, bool fresh, uint64_t* ukey, uint64_t* upool,
                         long long* si, float* sd, hipStream_t s);
/** Start points without the fused selection (search.cu:261-291): the ids earlier waves expanded sorted into
 * dsort [m, Ep], kept entries marked fresh by binary search, the first S fresh taken. */
void launch_unfused_pick(const long long* si, int m, int KO, long long* done, int E, int off, int S, int rowlen,
                         uint64_t* dsort, int Ep, unsigned char* fresh, int2* seg2, hipStream_t s);
/**
 * Exact rerank of each query's R sketch-nearest candidates (of its nin [m] in cand / dist [m, W]) merged into its kept
 * list si / sd [m, KO] (search_kernels.cuh:421-467).
 * hist [m, H] (may be null with hoff 0 and no store): the selected ids of a batch's rounds, R entries each, -1 padded;
 * with hstore this round's go to hist[q, hoff .. hoff + R).  Unless fresh, the ids of hist[q, 0 .. hoff) are those the
 * earlier rounds reranked into this kept list; those of its last 256 entries, selected again, are neither read nor
 * merged (the kept list of the KO smallest keys comes out the same), and nskip [m] (when not null) gets their count.
 */
void launch_rerank_keep(const int* cand, const float* dist, const int* nin, int m, int W, const __half* vectors, int D,
                        const float* Q, int R, int KO, long long* si, float* sd, bool fresh, int* hist, int H, int hoff,
                        bool hstore, int* nskip, hipStream_t s);
void launch_sketch_keep(const int* cand, const float* dist, const int* nin, int m, int W, int KO,
                        long long* si, float* sd, bool fresh, hipStream_t s);
void launch_pick_starts(const long long* si, int m, int KO, long long* done, int E, int off, int S,
                        int rowlen, int2* seg2, hipStream_t s);
void launch_final_rerank(const long long* si, int m, int KO, int R, const __half* vectors, int D,
                         const float* Q, int k, long long* bi, float* bd, hipStream_t s);
/** out [n, words] = the 32-bit words src[off[r], off[r] + words) of every range r (offsets on the device). */
void launch_copy_ranges(const uint32_t* src, const int64_t* off, int64_t n, int words, uint32_t* out,
                        hipStream_t s);
void launch_take_k(const long long* si, const float* sd, int m, int KO, int k, long long* bi,
                   float* bd, hipStream_t s);

}  // namespace cuvs::neighbors::octex::detail
