/*
 * CPU oracle of the octex batched search path: TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * A plain C++ restatement of the reference's search arithmetic (cpp/src/neighbors/octex/detail/e8.cuh,
 * detail/search_kernels.cuh and search.cu) used only by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py, as the checker of the HIP library and as the CPU baseline (for the 100k-row
 * CPU workload also its host build, orc_build).  The product (octex_amd/) never links, loads or calls it.
 *
 * Arithmetic pins (both here and in the HIP kernels), where the reference leaves the order to nvcc:
 *   - E8 distances da/dc:   t = x - a; acc = fma(t, t, acc)                 (e8.cuh:56-57)
 *   - sketch score:         u = fma(code, scale, -qs); d = fma(u, u, d), Lr-lane chunks of 16 then
 *                           an xor butterfly over o = Lr/2 .. 1            (search_kernels.cuh:227-251)
 *   - exact distance:       LX lanes per row (the next power of two >= D / 8, at most 32), lane sub
 *                           takes the 8-element chunks sub, sub + LX, ... in order; t = x - q;
 *                           acc = fma(t, t, acc); xor butterfly over LX/2 .. 1
 *                           (search_kernels.cuh:325-342 with 16-byte chunks per lane)
 *   - selections:           the R smallest by (distance bits, id); the reference takes threshold ties in
 *                           atomicAdd order (search_kernels.cuh:307), here the smallest ids win.
 * Parity unpinned at bit level against the reference itself: the fp16 projection (cuBLASLt order), the
 * TF32 sketch-query GEMM, and nvcc's contraction choices (only an NVIDIA run could fix them).
 */
#pragma once

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/** The arrays of one loaded index (single device, replicate placement; load.cu:284-427). */
typedef struct {
  int64_t n, dim;
  int32_t copies, blocks, levels, list_len, log_buckets, sketch_width, table_len;
  const float* inv_f;      /* [L] float(1 / double(spacing)) (load.cu:397-399) */
  const int32_t* lists;    /* [C, stride] */
  int64_t stride;
  const int64_t* keys;     /* [C, L, mmax] */
  int64_t mmax;
  const int32_t* offsets;  /* [C, L, T1] */
  int64_t T1;
  const int32_t* base;     /* [C, L] */
  const uint16_t* ucat;    /* [D, C * 8b] fp16 (load.cu:385-396) */
  const uint16_t* shift;   /* [C * 8b] fp16 */
  const float* mean;       /* [D] */
  const float* basis;      /* [D, S] */
  const float* scale;      /* [S] */
  const int8_t* sketch;    /* [N, S] */
  const uint16_t* vectors; /* [N, D] fp16 */
  const int32_t* table;    /* [N, table_len] or NULL */
} orc_index;

typedef struct {
  int32_t read, starts, waves, rerank, wave_rerank, batch, sketch_rank, final_rerank;
} orc_search_params;

/** Optional per-query intermediates of orc_search (any pointer may be NULL). */
typedef struct {
  int32_t* seg;   /* [nq, C, 2] probe segments */
  int32_t* n1;    /* [nq] distinct first-round candidates */
  int64_t* si1;   /* [nq, KO] kept list after the first round */
  float* sd1;
  int32_t* n2;    /* [nq, waves] distinct candidates of every wave */
  int64_t* si;    /* [nq, KO] final kept list */
  float* sd;
} orc_trace;

/* fp16 <-> fp32, IEEE round to nearest even */
uint16_t orc_f2h(float f);
float orc_h2f(uint16_t h);
void orc_f2h_n(const float* x, int64_t n, uint16_t* out);
void orc_h2f_n(const uint16_t* x, int64_t n, float* out);

/* E8 (e8.cuh:24-85) */
void orc_e8_point(const float* x, float* p);
int64_t orc_e8b_hash64(const float* y, int b, float inv_f);
/** p[i] = E8^b point of y[i] * inv_f, h[i] = its hash (test_build.cu:57-70 shape). */
void orc_e8_batch(const float* y, int64_t n, int b, float inv_f, float* p, int64_t* h);

/* query preparation (search_kernels.cuh:57-69, search.cu:305-341) */
void orc_center(const float* q, const float* mu, int64_t m, int D, float* qc, uint16_t* qh);
/** Y = fp16(sum_d qh[q, d] ucat[d, j] + shift[j]) with an fp64 sum; Yd (optional) the fp64 values. */
void orc_project(const uint16_t* qh, int64_t m, int D, const uint16_t* ucat, int wdt,
                 const uint16_t* shift, uint16_t* Y, double* Yd);
void orc_sketch_query(const float* qc, int64_t m, int D, const float* basis, int S, float* qs);

/* per-stage functions */
void orc_probe(const orc_index* ix, const uint16_t* Y, int64_t m, int lr, int32_t* seg);
/** Distinct ids of the segments (rows = 0: lists, 1: table rows), ascending, with sketch scores. */
int orc_gather(const orc_index* ix, const int32_t* seg, int nseg, int rows, const float* qs,
               int32_t* cand, float* dist, int cap);
float orc_sketch_dist(const int8_t* code, const float* scale, const float* qs, int S);
float orc_exact_dist(const uint16_t* x, const float* q, int D);
/** The R smallest of n (dist, id) pairs by (distance bits, id), ascending. */
int orc_select(const int32_t* cand, const float* dist, int n, int R, int32_t* sid, float* sd);
/** Kept list merge (search_kernels.cuh:379-415): keys of the kept list (unless fresh) and the new
 * pairs sorted, the first KO distinct kept, padded with (-1, +inf). */
void orc_merge_keep(int64_t* si, float* sd, int KO, int fresh, const int32_t* nid, const float* nd,
                    int nn);
/** rerank_keep_kernel (search_kernels.cuh:421-467) for one query. */
void orc_rerank_keep(const orc_index* ix, const int32_t* cand, const float* dist, int n,
                     const float* q, int R, int KO, int fresh, int64_t* si, float* sd);
/** sketch_keep_kernel (search_kernels.cuh:471-508) for one query. */
void orc_sketch_keep(const int32_t* cand, const float* dist, int n, int KO, int fresh, int64_t* si,
                     float* sd);
/** pick_starts_kernel (search_kernels.cuh:571-631) for one query: returns the starts written. */
int orc_pick_starts(const int64_t* si, int KO, int64_t* done, int off, int S, int rowlen,
                    int32_t* seg2);
/** final_rerank_kernel (search_kernels.cuh:634-669) for one query. */
void orc_final_rerank(const orc_index* ix, const int64_t* si, int R, const float* q, int k,
                      int64_t* bi, float* bd);

/**
 * The whole search (search.cu:294-518, 816-961): every query independently (the batch split and the
 * padding of the last batch change no result).  Y [nq, C*8b] and qs [nq, S] override the
 * projections when given (parity given the GPU's own Y and qs); else orc_project / orc_sketch_query.
 * threads: host threads over queries.  Returns 0, or -1 with a message in orc_last_error().
 */
int orc_search(const orc_index* ix, const orc_search_params* sp, const float* q, int64_t nq, int k,
               const uint16_t* Y, const float* qs, int64_t* I, float* D, int threads,
               const orc_trace* trace);
const char* orc_last_error(void);

/* ---- small CPU builder (format 1; build.cu:104-426) for test indexes ---- */
typedef struct {
  int32_t copies, blocks, pca_dims;
  const float* spacings;
  int32_t n_spacings;
  int32_t list_len, min_cell, log_buckets, sketch_width, table_len;
  int32_t reverse_edges, exact_lists, member_lists;
  uint64_t seed;
  int32_t threads; /* host threads over copies and table rows (< 1: one); the files do not depend on it */
} orc_build_params;

/** Build an index of x [n, d] (fp32, rounded to fp16 first as build.cu:434-441) into `path`. */
int orc_build(const float* x, int64_t n, int64_t d, const orc_build_params* p, const char* path);

/** Exact k nearest neighbors of q [m, d] among x [n, d] (fp64 distances, ties by id). */
void orc_bruteforce(const float* x, int64_t n, const float* q, int64_t m, int64_t d, int k,
                    int64_t* I, float* D, int threads);

#ifdef __cplusplus
}
#endif
