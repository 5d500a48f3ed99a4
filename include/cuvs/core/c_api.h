/*
 * The part of the cuVS C core that the certex C API needs: resources, error codes and the
 * last-error text. Names and enumerator values follow the cuVS C API so that C callers written
 * against cuVS compile unchanged; the stream handle is a plain pointer (a hipStream_t).
 */
#pragma once

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CUVS_EXPORT __attribute__((visibility("default")))

/** Status of every call: CUVS_ERROR carries a message in cuvsGetLastErrorText(). */
typedef enum { CUVS_ERROR = 0, CUVS_SUCCESS = 1 } cuvsError_t;

/** Opaque handle of a device, a stream on it, and the scratch memory of the searches. */
typedef uintptr_t cuvsResources_t;

/** Create resources on the current device with a stream of their own (default priority). */
CUVS_EXPORT cuvsError_t cuvsResourcesCreate(cuvsResources_t* res);

/** Free resources; waits for the work queued on their stream. */
CUVS_EXPORT cuvsError_t cuvsResourcesDestroy(cuvsResources_t res);

/** Make the resources issue their work on `stream` (a hipStream_t; NULL: the null stream). */
CUVS_EXPORT cuvsError_t cuvsStreamSet(cuvsResources_t res, void* stream);

/** The stream of the resources (a hipStream_t). */
CUVS_EXPORT cuvsError_t cuvsStreamGet(cuvsResources_t res, void** stream);

/** Wait for every piece of work queued on the stream of the resources. */
CUVS_EXPORT cuvsError_t cuvsStreamSync(cuvsResources_t res);

/** Text of the last error of the calling thread, or NULL after a successful call. */
CUVS_EXPORT const char* cuvsGetLastErrorText(void);

/** Replace the last-error text of the calling thread (NULL clears it). */
CUVS_EXPORT void cuvsSetLastErrorText(const char* error);

#ifdef __cplusplus
}
#endif
