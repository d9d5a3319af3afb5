/*
 * octex C ABI for MI355X: the cuvsOctex* entry points of the reference (c/include/cuvs/neighbors/octex.h),
 * with the same names, signatures, struct field order and enum values, so that a C caller or a
 * binding written against the reference links against liboctex_amd.so unchanged.
 *
 * Tensors are DLPack.  Device tensors are kDLROCM (HIP device memory) or kDLROCMHost (pinned host
 * memory); host tensors are kDLCPU or kDLROCMHost.  Errors: every call returns CUVS_SUCCESS or
 * CUVS_ERROR and sets the thread's last error text (cuvsGetLastErrorText).
 */
#pragma once

#include <cuvs/core/c_api.h>
#include <dlpack/dlpack.h>
#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/**
 * Index build parameters (cuvs::neighbors::octex::index_params); reference: octex.h:31-76.
 * `spacings` and `devices` are the caller's arrays, read only during cuvsOctexBuild; NULL (or a count
 * of 0) keeps the C++ default.
 */
struct cuvsOctexIndexParams {
  int32_t copies;            /* randomly projected copies */
  int32_t blocks;            /* E8 blocks per copy: 8 * blocks projected dimensions */
  int32_t pca_dims;          /* principal directions the projections rotate */
  const float* spacings;     /* cell spacings, fine to coarse (NULL: 2.0, 2.5, 3.2, 4.0, 5.0) */
  int32_t n_spacings;
  int32_t list_len;          /* vectors per populated cell, nearest first */
  int32_t min_cell;          /* lists only for cells of at least this many vectors (not the coarsest) */
  int32_t log_buckets;       /* log2 of the hash buckets per copy and spacing */
  int32_t sketch_width;      /* int8 sketch coordinates (0: dimension rounded down to 16, at most 128) */
  int32_t table_len;         /* neighbor-table row length (0: no table) */
  bool reverse_edges;        /* merge reverse edges into the table */
  bool exact_lists;          /* exact cell lists (brute force in the projection) */
  int32_t list_probes;       /* probes of the approximate list construction */
  bool member_lists;         /* cell lists from the members of each cell */
  int64_t exact_table_max;   /* up to this many vectors the table is exact */
  int32_t table_passes;      /* search passes of a searched table, 1 to 3 */
  bool table_sketch_order;   /* searched-table rows in sketch order */
  bool write_behind;         /* write arrays while the table is built */
  uint64_t seed;             /* seed of the projections and shifts */
  const int32_t* devices;    /* GPUs of the build (NULL: all visible) */
  int32_t n_devices;
};

typedef struct cuvsOctexIndexParams* cuvsOctexIndexParams_t;

/** Allocate index parameters with the C++ defaults (reference octex.h:81). */
cuvsError_t cuvsOctexIndexParamsCreate(cuvsOctexIndexParams_t* params);

/** Free index parameters (reference octex.h:84). */
cuvsError_t cuvsOctexIndexParamsDestroy(cuvsOctexIndexParams_t params);

/** Where the parts of an index live (reference octex.h:96-101). */
typedef enum {
  OCTEX_PLACEMENT_REPLICATE = 0, /* every GPU holds the whole index */
  OCTEX_PLACEMENT_SHARD     = 1  /* copies and table rows split over the GPUs */
} cuvsOctexPlacement;

/** Where the int8 sketch lives (reference octex.h:104-111). */
typedef enum {
  OCTEX_SKETCH_REPLICATE = 0, /* a full copy on every GPU */
  OCTEX_SKETCH_SHARD     = 1, /* row ranges over the GPUs */
  OCTEX_SKETCH_HOST      = 2  /* pinned host memory, read in place */
} cuvsOctexSketchPlacement;

/** Load parameters (cuvs::neighbors::octex::load_params); reference octex.h:117-140. */
struct cuvsOctexLoadParams {
  const int32_t* devices;  /* GPUs that hold the index (NULL: all visible) */
  int32_t n_devices;
  cuvsOctexPlacement placement;
  bool vectors_on_host;    /* fp16 vectors in pinned host memory */
  bool shard_vectors;      /* vectors split by rows over the GPUs */
  bool table_on_host;      /* neighbor table in pinned host memory */
  cuvsOctexSketchPlacement sketch;
  int32_t parts;           /* the copies were saved in this many parts (0: one) */
  int32_t copies_per_part; /* first copies of every part only (0: all) */
  int32_t copies_limit;    /* first copies only (0: all; one part) */
  int32_t list_limit;      /* first entries of every cell list only (0: all) */
};

typedef struct cuvsOctexLoadParams* cuvsOctexLoadParams_t;

/** Allocate load parameters with the C++ defaults (reference octex.h:146). */
cuvsError_t cuvsOctexLoadParamsCreate(cuvsOctexLoadParams_t* params);

/** Free load parameters (reference octex.h:149). */
cuvsError_t cuvsOctexLoadParamsDestroy(cuvsOctexLoadParams_t params);

/** Search parameters (cuvs::neighbors::octex::search_params); reference octex.h:161-184. */
struct cuvsOctexSearchParams {
  int32_t read;         /* list entries read per copy in the first round */
  int32_t starts;       /* best first-round hits kept as start points */
  int32_t waves;        /* waves over the neighbor table */
  int32_t rerank;       /* exact rerank depth of the first round */
  int32_t wave_rerank;  /* exact rerank depth of every wave */
  int32_t batch;        /* queries per captured batch */
  bool sketch_rank;     /* rank by the sketch, rerank exactly at the end */
  int32_t final_rerank; /* sketch-rank mode: kept entries reranked at the end */
  bool balanced_gather; /* ablation: load-balanced gather */
  bool fused_merge;     /* ablation: fused keep / pick-starts kernels */
  bool use_graph;       /* ablation: one hipGraph per batch */
};

typedef struct cuvsOctexSearchParams* cuvsOctexSearchParams_t;

/** Allocate search parameters with the C++ defaults (reference octex.h:189). */
cuvsError_t cuvsOctexSearchParamsCreate(cuvsOctexSearchParams_t* params);

/** Free search parameters (reference octex.h:192). */
cuvsError_t cuvsOctexSearchParamsDestroy(cuvsOctexSearchParams_t params);

/** An opaque index handle (reference octex.h:204-208). */
typedef struct {
  uintptr_t addr;
} cuvsOctexIndex;

typedef cuvsOctexIndex* cuvsOctexIndex_t;

/** Allocate an empty index handle (reference octex.h:211). */
cuvsError_t cuvsOctexIndexCreate(cuvsOctexIndex_t* index);

/** Free an index handle and its index, with all its device memory (reference octex.h:214). */
cuvsError_t cuvsOctexIndexDestroy(cuvsOctexIndex_t index);

/** Number of vectors (reference octex.h:217). */
cuvsError_t cuvsOctexIndexGetSize(cuvsOctexIndex_t index, int64_t* size);

/** Dimension (reference octex.h:220). */
cuvsError_t cuvsOctexIndexGetDim(cuvsOctexIndex_t index, int64_t* dim);

/** Copies loaded (reference octex.h:223). */
cuvsError_t cuvsOctexIndexGetCopies(cuvsOctexIndex_t index, int32_t* copies);

/** Number of GPUs holding the index (reference octex.h:226). */
cuvsError_t cuvsOctexIndexGetNumDevices(cuvsOctexIndex_t index, int32_t* n_devices);

/** The GPUs holding the index (reference octex.h:230). */
cuvsError_t cuvsOctexIndexGetDevices(cuvsOctexIndex_t index, int32_t* devices);

/** Device bytes per GPU (reference octex.h:234). */
cuvsError_t cuvsOctexIndexGetDeviceBytes(cuvsOctexIndex_t index, int64_t* bytes);

/**
 * Build an index of a float32 or float16 dataset [n_rows, dim] into the directory `path` (created);
 * reference octex.h:261-264.  A dataset in device memory is copied to the host first.
 */
cuvsError_t cuvsOctexBuild(cuvsResources_t res, cuvsOctexIndexParams_t params, DLManagedTensor* dataset,
                           const char* path);

/** Load an index directory into an empty handle (`params` NULL: defaults); reference octex.h:268-271. */
cuvsError_t cuvsOctexLoad(cuvsResources_t res, const char* path, cuvsOctexLoadParams_t params,
                          cuvsOctexIndex_t index);

/**
 * Approximate k nearest neighbors, k = neighbors' second extent (reference octex.h:290-295): queries
 * [n, dim] float32, neighbors [n, k] int64, distances [n, k] float32 (squared L2, nearest first), all
 * host or all device.  Host results are complete on return; device results are ordered on the
 * stream of `res`.
 */
cuvsError_t cuvsOctexSearch(cuvsResources_t res, cuvsOctexSearchParams_t params, cuvsOctexIndex_t index,
                            DLManagedTensor* queries, DLManagedTensor* neighbors, DLManagedTensor* distances);

#ifdef __cplusplus
}
#endif
