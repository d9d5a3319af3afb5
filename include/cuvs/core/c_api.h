/*
 * The subset of the cuVS core C API (cuvs/core/c_api.h) that the cuvsOctex* C ABI uses: error codes,
 * the resources handle, its stream, and the thread-local last error text.  Names and signatures follow
 * cuVS (octex.h:8 includes it; exceptions.hpp:17-33 and guide.md:86-125 use it); the numeric values of
 * cuvsError_t follow cuVS's enum order {CUVS_ERROR, CUVS_SUCCESS}.
 */
#pragma once

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum { CUVS_ERROR, CUVS_SUCCESS } cuvsError_t;

/** An opaque handle of a raft::resources: the device and stream that calls run on. */
typedef uintptr_t cuvsResources_t;

/** Create resources on the current device with the default (null) stream. */
cuvsError_t cuvsResourcesCreate(cuvsResources_t* res);

/** Destroy resources. */
cuvsError_t cuvsResourcesDestroy(cuvsResources_t res);

/** Set the HIP stream (a hipStream_t, passed as void*) that calls with these resources use. */
cuvsError_t cuvsStreamSet(cuvsResources_t res, void* stream);

/** The HIP stream of the resources. */
cuvsError_t cuvsStreamGet(cuvsResources_t res, void** stream);

/** Wait for the work queued on the stream of the resources. */
cuvsError_t cuvsStreamSync(cuvsResources_t res);

/** The text of the last error of this thread ("" after a success). */
const char* cuvsGetLastErrorText(void);

/** Set the last error text of this thread (NULL clears it). */
void cuvsSetLastErrorText(const char* error);

#ifdef __cplusplus
}
#endif
