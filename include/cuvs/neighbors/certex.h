/*
 * C API of the exact k-NN index, MI355X build.
 *
 * The 15 cuvsCertex* entry points and the two parameter structs have the names, signatures,
 * field order and semantics of the reference C API (c/include/cuvs/neighbors/certex.h:30-221,
 * implementation c/src/neighbors/certex.cpp:162-371); each declaration cites the reference line it
 * replaces. Tensors are DLPack v1.0 (device tensors: kDLROCM, also accepted as kDLCUDA; host
 * tensors: kDLCPU, kDLCUDAHost, kDLROCMHost), dense and row major, and are borrowed: no deleter is
 * called. Every call returns CUVS_SUCCESS or CUVS_ERROR with a message in cuvsGetLastErrorText().
 * Work is queued on the stream of `res` and is not waited for (cuvsStreamSync waits).
 *
 * The entry points after the reference set (cuvsCertexIndexGet*, cuvsCertexReserve,
 * cuvsCertexStats*) expose what the reference's Python binding reads from its nanobind module
 * (python/src/core.cpp:571-691), so that the Python package runs over this C API alone.
 */
#pragma once

#include <cuvs/core/c_api.h>
#include <cuvs/distance/distance.h>
#include <cuvs/neighbors/common.h>
#include <dlpack/dlpack.h>
#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/** Index parameters (reference certex.h:30-49). */
struct cuvsCertexIndexParams {
  cuvsDistanceType metric;
  int32_t width;
  double variance;
  int32_t anchor_stride;
  int64_t pca_sample;
  bool host_vectors;
  int32_t n_lists;
  bool local_projections;
  bool int8_rows;
};
typedef struct cuvsCertexIndexParams* cuvsCertexIndexParams_t;

/** Defaults of the C++ API (reference certex.h:54, certex.cpp:162-176). */
CUVS_EXPORT cuvsError_t cuvsCertexIndexParamsCreate(cuvsCertexIndexParams_t* params);
/** Reference certex.h:57. */
CUVS_EXPORT cuvsError_t cuvsCertexIndexParamsDestroy(cuvsCertexIndexParams_t params);

/** Search parameters (reference certex.h:69-76). */
struct cuvsCertexSearchParams {
  int32_t anchors;
  int32_t batch_size;
  int32_t probe_lists;
};
typedef struct cuvsCertexSearchParams* cuvsCertexSearchParams_t;

/** Reference certex.h:81. */
CUVS_EXPORT cuvsError_t cuvsCertexSearchParamsCreate(cuvsCertexSearchParams_t* params);
/** Reference certex.h:84. */
CUVS_EXPORT cuvsError_t cuvsCertexSearchParamsDestroy(cuvsCertexSearchParams_t params);

/** Opaque index of float32, float16, int8 or uint8 vectors (reference certex.h:96-101). */
typedef struct {
  uintptr_t addr;
  DLDataType dtype;
} cuvsCertexIndex;
typedef cuvsCertexIndex* cuvsCertexIndex_t;

/** Empty handle (reference certex.h:106). */
CUVS_EXPORT cuvsError_t cuvsCertexIndexCreate(cuvsCertexIndex_t* index);
/** Free a handle and its index (reference certex.h:109). */
CUVS_EXPORT cuvsError_t cuvsCertexIndexDestroy(cuvsCertexIndex_t index);
/** Vectors added, removed ones included (reference certex.h:112). */
CUVS_EXPORT cuvsError_t cuvsCertexIndexGetSize(cuvsCertexIndex_t index, int64_t* size);
/** Dimension (reference certex.h:115). */
CUVS_EXPORT cuvsError_t cuvsCertexIndexGetDim(cuvsCertexIndex_t index, int64_t* dim);

/** Build from a dataset [n, dim] in device or host memory (reference certex.h:138-141). */
CUVS_EXPORT cuvsError_t cuvsCertexBuild(cuvsResources_t res,
                                        cuvsCertexIndexParams_t params,
                                        DLManagedTensor* dataset,
                                        cuvsCertexIndex_t index);

/** Append vectors with the next consecutive ids (reference certex.h:145-147). */
CUVS_EXPORT cuvsError_t cuvsCertexExtend(cuvsResources_t res,
                                         DLManagedTensor* new_vectors,
                                         cuvsCertexIndex_t index);

/** Remove vectors by id, an int64 device vector (reference certex.h:150-152). */
CUVS_EXPORT cuvsError_t cuvsCertexRemove(cuvsResources_t res,
                                         DLManagedTensor* ids,
                                         cuvsCertexIndex_t index);

/** Labels (int32 device vector) of vectors first, first + 1, ... (reference certex.h:156-159). */
CUVS_EXPORT cuvsError_t cuvsCertexSetLabels(cuvsResources_t res,
                                            DLManagedTensor* labels,
                                            int64_t first,
                                            cuvsCertexIndex_t index);

/** Label partition of the screening rows (reference certex.h:163); a speed option only. */
CUVS_EXPORT cuvsError_t cuvsCertexPartitionByLabels(cuvsResources_t res, cuvsCertexIndex_t index);

/**
 * Exact k nearest neighbours, k = the second extent of `neighbors` (reference certex.h:183-189):
 * queries [nq, dim] (device, index type), neighbors [nq, k] int64, distances [nq, k] float32.
 */
CUVS_EXPORT cuvsError_t cuvsCertexSearch(cuvsResources_t res,
                                         cuvsCertexSearchParams_t params,
                                         cuvsCertexIndex_t index,
                                         DLManagedTensor* queries,
                                         DLManagedTensor* neighbors,
                                         DLManagedTensor* distances,
                                         cuvsFilter filter);

/**
 * cuvsCertexSearch with no device or pinned host memory allocated during the call. It has no
 * counterpart in the reference; it is for callers that cannot allocate (tight serving loops,
 * harnesses that forbid hipMalloc). Same arguments, checks and results as cuvsCertexSearch. The
 * scratch is one fixed 128 MiB device array per GPU, held from the library's load on that GPU
 * until the process ends; larger batches are split into smaller ones, and a search that needs more
 * than 128 MiB for a single query returns CUVS_ERROR. Calls on one GPU share that array and take
 * turns: a call waits on the host for the previous call to return, and its stream waits on the GPU
 * (an event, no host sync) for the previous call's last kernel, whatever stream or resources that
 * call used. The array keeps the previous call's contents; each call clears what must start at 0.
 */
CUVS_EXPORT cuvsError_t cuvsCertexSearchNoAlloc(cuvsResources_t res,
                                                cuvsCertexSearchParams_t params,
                                                cuvsCertexIndex_t index,
                                                DLManagedTensor* queries,
                                                DLManagedTensor* neighbors,
                                                DLManagedTensor* distances,
                                                cuvsFilter filter);

/** Exact k nearest neighbours among the vectors of each query's label (certex.h:195-201). */
CUVS_EXPORT cuvsError_t cuvsCertexSearchWithLabels(cuvsResources_t res,
                                                   cuvsCertexSearchParams_t params,
                                                   cuvsCertexIndex_t index,
                                                   DLManagedTensor* queries,
                                                   DLManagedTensor* query_labels,
                                                   DLManagedTensor* neighbors,
                                                   DLManagedTensor* distances);

/** Save the index with its vectors (reference certex.h:213-215). */
CUVS_EXPORT cuvsError_t cuvsCertexSerialize(cuvsResources_t res,
                                            const char* filename,
                                            cuvsCertexIndex_t index);

/** Load into an empty handle; the vector type comes from the file (reference certex.h:219-221). */
CUVS_EXPORT cuvsError_t cuvsCertexDeserialize(cuvsResources_t res,
                                              const char* filename,
                                              cuvsCertexIndex_t index);

/* ---- read by the Python package (reference python/src/core.cpp:571-691) ---- */

/** Number of removed vectors (core.cpp n_removed). */
CUVS_EXPORT cuvsError_t cuvsCertexIndexGetRemoved(cuvsCertexIndex_t index, int64_t* n_removed);
/** Rows allocated (core.cpp reserve / capacity). */
CUVS_EXPORT cuvsError_t cuvsCertexIndexGetCapacity(cuvsCertexIndex_t index, int64_t* capacity);
/** Screening width m (core.cpp width). */
CUVS_EXPORT cuvsError_t cuvsCertexIndexGetWidth(cuvsCertexIndex_t index, int32_t* width);
/** Metric (core.cpp metric). */
CUVS_EXPORT cuvsError_t cuvsCertexIndexGetMetric(cuvsCertexIndex_t index,
                                                 cuvsDistanceType* metric);
/** Anchor stride (core.cpp anchor_stride). */
CUVS_EXPORT cuvsError_t cuvsCertexIndexGetAnchorStride(cuvsCertexIndex_t index, int32_t* stride);
/** Whether labels were set (core.cpp has_labels). */
CUVS_EXPORT cuvsError_t cuvsCertexIndexHasLabels(cuvsCertexIndex_t index, bool* has_labels);
/**
 * Whether the float vectors are kept in pinned host memory (core.cpp host_vectors, read by
 * certex/index.py:379 when an index is loaded).
 */
CUVS_EXPORT cuvsError_t cuvsCertexIndexGetHostVectors(cuvsCertexIndex_t index, bool* host_vectors);
/**
 * Vectors covered by the label partition (0 when none); the ones added later go through the
 * label filter (reference index::n_partitioned, certex.hpp:301-306).
 */
CUVS_EXPORT cuvsError_t cuvsCertexIndexGetPartitioned(cuvsCertexIndex_t index,
                                                      int64_t* n_partitioned);
/**
 * Number of k-means lists (0 when none), and the vectors they cover: those of the build, stored
 * in list order (reference index::n_lists / list_offsets, certex.hpp:321-334).
 */
CUVS_EXPORT cuvsError_t cuvsCertexIndexGetLists(cuvsCertexIndex_t index,
                                                int32_t* n_lists,
                                                int64_t* n_listed);
/**
 * Grow the capacity to at least `capacity` rows (core.cpp reserve). On a handle that holds no
 * index yet, the next cuvsCertexBuild allocates that capacity (this build's addition).
 */
CUVS_EXPORT cuvsError_t cuvsCertexReserve(cuvsResources_t res,
                                          int64_t capacity,
                                          cuvsCertexIndex_t index);
/**
 * The ids in the order of the stored rows of an index with lists (core.cpp list_order, reference
 * certex/index.py:353-359): `order` is an int32 device vector with one entry per vector added
 * (cuvsCertexIndexGetSize). Queries taken in this order share their nearest lists within a batch.
 * CUVS_ERROR when the index has no lists.
 */
CUVS_EXPORT cuvsError_t cuvsCertexIndexListOrder(cuvsResources_t res,
                                                 cuvsCertexIndex_t index,
                                                 DLManagedTensor* order);
/** Start counting the searches of the calling thread (core.cpp stats_begin). */
CUVS_EXPORT cuvsError_t cuvsCertexStatsBegin(void);
/** Stop counting: queries, certified survivors, exact distances (core.cpp stats_end). */
CUVS_EXPORT cuvsError_t cuvsCertexStatsEnd(int64_t* queries, int64_t* survivors,
                                           int64_t* verified);

/* ---- kernel timing (no counterpart in the reference; used by the benchmark) ---- */

/** Phases timed by cuvsCertexTimingEnd: anchor pass, threshold, screen, exact re-rank + top-k. */
enum cuvsCertexPhase {
  CERTEX_PHASE_ANCHORS   = 0,
  CERTEX_PHASE_THRESHOLD = 1,
  CERTEX_PHASE_SCREEN    = 2,
  CERTEX_PHASE_VERIFY    = 3,
  CERTEX_N_PHASES        = 4
};
/** Record HIP events around every kernel of the searches of the calling thread (adds no host
 *  wait to the searches). */
CUVS_EXPORT cuvsError_t cuvsCertexTimingBegin(void);
/** Stop recording; waits for the recorded events and returns per phase the summed kernel time in
 *  milliseconds and the number of launches (arrays of CERTEX_N_PHASES). */
CUVS_EXPORT cuvsError_t cuvsCertexTimingEnd(double* ms, int64_t* launches);
/** The average shader clock in MHz of the screen workgroups timed between the last
 *  cuvsCertexTimingBegin and cuvsCertexTimingEnd: each workgroup's life in shader clock cycles
 *  (s_memtime) over its life in real time (s_memrealtime, 100 MHz), summed over the workgroups;
 *  0 if no screen ran. The clock the card sustained on this work, next to its 2.4 GHz peak. */
CUVS_EXPORT cuvsError_t cuvsCertexTimingShaderClock(double* mhz);

/**
 * Free the scratch memory that searches on `res` have grown (device buffers and pinned host
 * staging), after waiting for its stream; later searches grow it again. The counterpart of the
 * reference's Python trim_pool (certex/index.py:165-169), which returns the unused memory of the
 * device's stream-ordered pool.
 */
CUVS_EXPORT cuvsError_t cuvsCertexTrimPool(cuvsResources_t res);

/**
 * Testing only, no counterpart in the reference: every scratch request of searches on `res` above
 * `bytes` fails as an allocation failure would, so that tests can exercise the batch halving
 * (reference certex.cu:1477-1502). 0 removes the cap.
 */
CUVS_EXPORT cuvsError_t cuvsCertexTestScratchCap(cuvsResources_t res, int64_t bytes);

/**
 * Testing only, no counterpart in the reference (it replaces the kernel-level harness of
 * cpp/tests/neighbors/certex_kernels.cu:62-180): the next search batch of the calling thread (an
 * unrouted search without a list probe) copies its intermediate arrays to host memory, taken from
 * its own launches: the encoded queries ("qrows"), the anchor group table ("gmax"), the
 * thresholds ("theta"), the buckets ("count", "rows", and "vals" for float indexes), for float
 * indexes the certified bound U of each query ("ub_q"), the query scalars ("qscal"), and the
 * certificate's lower and upper bound of every bucket entry ("lb", "ub"), plus the index's
 * screening rows ("codes", "rowc") and the batch's shape (int64 "B", "k", "cap", "n_groups",
 * "group_steps", "fine", "anchor_stride", "row_bytes", "size", "all_rows").
 */
CUVS_EXPORT cuvsError_t cuvsCertexTestCaptureBegin(void);
/** Testing only: the size in bytes of a captured array in *bytes, and a copy to `host` unless
 *  NULL; CUVS_ERROR for a name that the last capture does not hold. */
CUVS_EXPORT cuvsError_t cuvsCertexTestCaptureGet(const char* name, void* host, int64_t* bytes);

#ifdef __cplusplus
}
#endif
