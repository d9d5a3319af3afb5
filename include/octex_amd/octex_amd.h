/*
 * liboctex_amd.so entry points beyond the reference's cuvsOctex* C ABI.  None of them has a
 * counterpart in the reference's C ABI:
 *   - introspection of a search (the reference exposes the same to its bench and tests through the
 *     C++-only detail::timed_batch / resident_search / memory_report, introspect.hpp:41-60);
 *   - the stage entry points: one HIP kernel each, on caller-provided device buffers, so that the
 *     parity tests call every kernel of the search path with controlled inputs (as the reference's
 *     cpp/tests/test_search.cu launches its kernels directly).
 * All return CUVS_SUCCESS / CUVS_ERROR with cuvsGetLastErrorText() set; `stream` is a hipStream_t
 * (NULL: the null stream); the stage calls wait for their kernel before returning.
 */
#pragma once

#include <cuvs/core/c_api.h>
#include <cuvs/neighbors/octex.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/** Copy a buffer of the index's cached search plan ("queries", "Y", "qs", "seg", "cand", "dist",
 * "nin", "si", "sd", "done", "seg2", "cand2", "dist2", "n2", "bi", "bd") to dst (host or device),
 * at most `bytes`; *size receives the buffer's size.  The buffers hold the last batch searched. */
cuvsError_t octexIndexCopyPlanBuffer(cuvsOctexIndex_t index, const char* name, void* dst, int64_t bytes,
                                     int64_t* size);

/**
 * Build the index of a float32 / float16 dataset [n, dim] in the HBM of the current GPU (or
 * params->devices[0]) and place it in the empty handle `index`, ready to search, without a round
 * trip through files; with `path` non-NULL the format-1 directory is written as well.  *seconds
 * (optional) receives the build time.  cuvsOctexBuild + cuvsOctexLoad in one step.
 */
cuvsError_t octexBuildInMemory(cuvsResources_t res, cuvsOctexIndexParams_t params, DLManagedTensor* dataset,
                               const char* path, cuvsOctexIndex_t index, double* seconds);

/**
 * Profile one batch of queries [m <= batch, dim] (float32, host or device): a normal search, then the
 * same batch launched kernel by kernel `reps` times with HIP events around every launch on the index's
 * stream.  names (64 x 32 chars) and ms receive the stages in launch order with their average
 * milliseconds, *nstages their count; counters (108 int64, optional): probe hits, list entries read,
 * distinct first-round candidates, first-round reranked, then per wave (16 each) valid start points,
 * distinct candidates and reranked entries, then probe hits by level (8, the finest first), then per wave (16 each)
 * the selected candidates not reranked again (an earlier round reranked them), the candidates whose scores came from
 * earlier rows, and the earlier rows' entries read; all summed over the batch's m rows.
 */
cuvsError_t octexIndexProfileBatch(cuvsOctexIndex_t index, cuvsOctexSearchParams_t params, DLManagedTensor* queries,
                                   int64_t k, int32_t reps, char* names, double* ms, int32_t* nstages,
                                   int64_t* counters);

/**
 * Copy an array of a loaded or built index to dst (host or device), at most `bytes`; *size receives
 * its size: "lists" (of copy `copy`), "keys", "offsets", "base", "ucatT", "shift", "inv_f", "mean",
 * "basis", "scale", "sketch" ([n, sketch_pitch]: rows padded in memory), "vectors", "table",
 * "spacings" (float32), and "meta" (12 int64: n, dim, copies, blocks, levels, list_len, log_buckets,
 * sketch_width, table_len, mmax, T1, sketch_pitch).
 */
cuvsError_t octexIndexCopyArray(cuvsOctexIndex_t index, const char* name, int32_t copy, void* dst, int64_t bytes,
                                int64_t* size);

/**
 * Copy bytes [offset, offset + bytes) of an array named as in octexIndexCopyArray (not "meta" or
 * "spacings") to dst; a range outside the array is an error.  Used to read a few list rows of a
 * large index without copying whole arrays.
 */
cuvsError_t octexIndexCopyArrayRange(cuvsOctexIndex_t index, const char* name, int32_t copy, int64_t offset,
                                     void* dst, int64_t bytes);

/**
 * Copy `count` ranges of `bytes` bytes (a multiple of 4) at byte offsets[r] (host, multiples of 4) of an
 * array named as in octexIndexCopyArray to dst [count, bytes] (host or device), gathered on the GPU in
 * one launch; a range outside the array is an error.
 */
cuvsError_t octexIndexCopyArrayRanges(cuvsOctexIndex_t index, const char* name, int32_t copy,
                                      const int64_t* offsets, int64_t count, int64_t bytes, void* dst);

/** The cached plan's shape: {m, k, KO, lr, W, W2, rerank, wave_rerank, final_rerank, graph?}. */
cuvsError_t octexIndexPlanInfo(cuvsOctexIndex_t index, int32_t* info);

/**
 * Move the fp16 vectors, the neighbor table and / or the sketch of an index (nonzero flags) from HBM to
 * pinned host memory, where the kernels read them over the host link: the placements vectors_on_host,
 * table_on_host and sketch = host of load_params (load.cu:159-185, 444-476) for an index built in
 * memory.  Cached search plans are dropped.  Searches of the index from other threads wait for it, and the
 * device copies are freed only after the work already on the index's stream.  No counterpart in the reference,
 * whose builder always writes a directory that load() then places.
 */
cuvsError_t octexIndexPlaceOnHost(cuvsOctexIndex_t index, int32_t vectors, int32_t table, int32_t sketch);

/**
 * Open and check an index directory on the host, as cuvsOctexLoad does before it touches a device:
 * meta.json parsed ("files" remapping honoured, unknown keys ignored), every array's dtype and full shape
 * compared with meta.json, the copies the load parameters select, and every level's cell table inside its
 * keys and lists.  info (10 int64, optional): n, dim, copies selected, copies in the directory, blocks,
 * levels, list_len, log_buckets, sketch_width, table_len.  Makes no HIP call, so it runs without a GPU.
 * No counterpart in the reference, whose load reads and places in one pass (load.cu:206-494).
 */
cuvsError_t octexIndexCheckDirectory(const char* path, cuvsOctexLoadParams_t params, int64_t* info);

/**
 * No counterpart in the reference: for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  cuvsOctexSearch for device queries [nq, dim] (float32,
 * row major) with every per-batch buffer in a file-scope device array of 256 MiB that each GPU holds until the
 * process ends, instead of a cached plan's allocations; the batch's kernels run directly on `stream` (a
 * hipStream_t, NULL the null stream; no graph) and write neighbors [nq, k] (int64) and distances [nq, k] (float32),
 * device memory, ordered on that stream.  The queries are split into batches of min(params->batch, nq); a batch
 * whose buffers exceed 256 MiB is an error that names the bytes it needs (lower params->batch).  No call allocates
 * or frees device memory.  Every call on one GPU shares that GPU's array: calls that overlap on one GPU (other
 * streams or threads) race, and the index must not change while one runs.
 */
cuvsError_t octexSearchNoAlloc(cuvsOctexSearchParams_t params, cuvsOctexIndex_t index, const float* queries,
                               int64_t nq, int64_t dim, int64_t k, int64_t* neighbors, float* distances, void* stream);

/**
 * No counterpart in the reference (measurement): the random-row read ceiling that the search gathers are held
 * against.  Reads n rows of row_bytes (a multiple of 16, at most 512) at uniformly random row numbers in
 * [0, rows) of base (rows * pitch bytes of device memory), one 16-byte load per lane, in_flight (1, 2, 4 or 8)
 * rows per lane group in flight, over `blocks` workgroups of 256 threads; out (device, blocks * 256 / G words,
 * G = the next power of two >= row_bytes / 16) gets an XOR of the words read.  Asynchronous on `stream`.
 */
cuvsError_t octexMeasureRowReads(const void* base, int64_t rows, int32_t pitch, int32_t row_bytes, int64_t n,
                                 int32_t in_flight, int32_t blocks, uint64_t seed, uint32_t* out, void* stream);

/* ---- stage entry points (fp16 arrays as raw 16-bit words) ---- */

/** qc = q - mu, qh = fp16(qc) (search_kernels.cuh:57-69). */
cuvsError_t octexStageCenter(const float* q, const float* mu, int64_t m, int32_t D, float* qc, void* qh,
                             void* stream);
/** Y [m, N] = qh [m, K] @ ucatT [N, K]^T + shift [N], fp16 (search.cu:305-320). */
cuvsError_t octexStageProject(const void* qh, const void* ucatT, const void* shift, int32_t m, int32_t K,
                              int32_t N, void* Y, void* stream);
/** qs [m, S] = qc [m, D] @ basis [D, S] (search.cu:323-341, fp32). */
cuvsError_t octexStageSketchQuery(const float* qc, const float* basis, int32_t m, int32_t D, int32_t S,
                                  float* qs, void* stream);
/** E8^b points p [n, 8b] and hashes h [n] of y [n, 8b] * inv_f (e8.cuh:44-85). */
cuvsError_t octexStageE8(const float* y, int64_t n, int32_t b, float inv_f, float* p, int64_t* h,
                         void* stream);
/** probe_kernel (search_kernels.cuh:84-127): seg [m, C, 2]. */
cuvsError_t octexStageProbe(const void* Y, int32_t m, int32_t C, int32_t L, int32_t B, const float* inv_f,
                            const int32_t* off, int64_t T1, const int64_t* keys, int64_t Mmax,
                            const int32_t* base, int32_t l, int32_t lr, int32_t logT, int32_t* seg,
                            void* stream);
/** octexStageProbe reading the buckets from bucket lines (first key and key range of every bucket, 16 bytes) built
 * from off and keys, as the search does when they fit in HBM; the same segments. */
cuvsError_t octexStageProbeLines(const void* Y, int32_t m, int32_t C, int32_t L, int32_t B, const float* inv_f,
                                 const int32_t* off, int64_t T1, const int64_t* keys, int64_t Mmax,
                                 const int32_t* base, int32_t l, int32_t lr, int32_t logT, int32_t* seg,
                                 void* stream);
/** gather_kernel (search_kernels.cuh:138-253): rows = 0 lists, 1 table rows; W a power of two; ids at or
 * above n are skipped like the -1 padding. */
cuvsError_t octexStageGather(int32_t rows, const int32_t* seg, int32_t nseg, int32_t m, const int32_t* lists,
                             int64_t stride, const int32_t* table, int32_t table_len, int64_t n, const int8_t* code,
                             const float* scale, const float* qs, int32_t S, int32_t W, int32_t* cand,
                             float* dist, int32_t* nout, void* stream);
/** octexStageGather over table rows taking the scores of candidates found in up to two earlier candidate rows
 * (old_cand / old_dist [m, old_W[r]], counts old_n [m]; host arrays of device pointers), as the search's wave
 * gathers do: those candidates come last in each row, copied, and nknown [m] (may be NULL) gets their count. */
cuvsError_t octexStageGatherReuse(const int32_t* seg, int32_t nseg, int32_t m, const int32_t* table,
                                  int32_t table_len, int64_t n, const int8_t* code, const float* scale,
                                  const float* qs, int32_t S, int32_t W, int32_t* cand, float* dist, int32_t* nout,
                                  int32_t nold, const int32_t* const* old_cand, const float* const* old_dist,
                                  const int32_t* const* old_n, const int32_t* old_W, int32_t* nknown, void* stream);
/** rerank_keep_kernel (search_kernels.cuh:421-467). */
cuvsError_t octexStageRerankKeep(const int32_t* cand, const float* dist, const int32_t* nin, int32_t m,
                                 int32_t W, const void* vectors, int32_t D, const float* Q, int32_t R,
                                 int32_t KO, int64_t* si, float* sd, int32_t fresh, void* stream);
/** octexStageRerankKeep with the history of a batch's selected ids, as the search's rounds run it: hist [m, H] holds
 * each round's R selected ids (-1 padded); with hstore this round's go to hist[q, hoff .. hoff + R); unless fresh, the
 * ids of hist[q, 0 .. hoff) were reranked into this kept list by earlier rounds, and those of its last 256 entries are
 * skipped when selected again (counted in nskip [m], may be NULL). */
cuvsError_t octexStageRerankKeepHistory(const int32_t* cand, const float* dist, const int32_t* nin, int32_t m,
                                        int32_t W, const void* vectors, int32_t D, const float* Q, int32_t R,
                                        int32_t KO, int64_t* si, float* sd, int32_t fresh, int32_t* hist, int32_t H,
                                        int32_t hoff, int32_t hstore, int32_t* nskip, void* stream);
/** sketch_keep_kernel (search_kernels.cuh:471-508). */
cuvsError_t octexStageSketchKeep(const int32_t* cand, const float* dist, const int32_t* nin, int32_t m,
                                 int32_t W, int32_t KO, int64_t* si, float* sd, int32_t fresh, void* stream);
/** pick_starts_kernel (search_kernels.cuh:571-631). */
cuvsError_t octexStagePickStarts(const int64_t* si, int32_t m, int32_t KO, int64_t* done, int32_t E,
                                 int32_t off, int32_t S, int32_t rowlen, int32_t* seg2, void* stream);
/** final_rerank_kernel (search_kernels.cuh:634-669). */
cuvsError_t octexStageFinalRerank(const int64_t* si, int32_t m, int32_t KO, int32_t R, const void* vectors,
                                  int32_t D, const float* Q, int32_t k, int64_t* bi, float* bd, void* stream);
/** take_k_kernel (search_kernels.cuh:672-685). */
cuvsError_t octexStageTakeK(const int64_t* si, const float* sd, int32_t m, int32_t KO, int32_t k, int64_t* bi,
                            float* bd, void* stream);

#ifdef __cplusplus
}
#endif
