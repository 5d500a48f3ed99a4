/*
 * C++ API of the exact k-NN index, MI355X build.
 *
 * Mirrors cuvs::neighbors::certex (reference cpp/include/cuvs/neighbors/certex.hpp:43-779): the
 * same namespace, parameter structs, index class and free functions build / extend / remove /
 * set_labels / search, over vectors of float, half, int8_t and uint8_t. RAFT mdspans are replaced
 * by plain pointer views and raft::resources by cuvs::resources (a device, a HIP stream and the
 * scratch memory of the searches); no HIP or torch type appears in this header.
 */
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace cuvs {

namespace distance {
/** Metric enumerators with the values of cuVS (cuvs/distance/distance.hpp). */
enum class DistanceType : int { L2Expanded = 0, CosineExpanded = 2, InnerProduct = 6 };
}  // namespace distance

namespace detail {
struct resources_state;
}

/** A device, a stream on it (hipStream_t as void*) and grow-only scratch memory of searches. */
class resources {
 public:
  /** Resources on the current device; stream nullptr: a new stream owned by the resources. */
  explicit resources(void* stream = nullptr);
  ~resources();
  resources(resources const&)            = delete;
  resources& operator=(resources const&) = delete;

  [[nodiscard]] auto stream() const -> void*;
  void set_stream(void* stream);
  [[nodiscard]] auto device() const -> int;
  void sync() const;
  /** Free the scratch memory that the searches on these resources have grown (device slots and
   *  pinned host staging), after waiting for the stream; later searches grow it again. The
   *  counterpart of the reference's trim_pool (certex/index.py:165-169). */
  void trim() const;
  /** Testing only (no counterpart in the reference): a scratch request above `bytes` fails as an
   *  allocation failure would, so that the search's batch halving can be exercised; 0 = no cap. */
  void set_scratch_cap(size_t bytes) const;
  [[nodiscard]] auto state() const -> detail::resources_state&;

 private:
  std::unique_ptr<detail::resources_state> s_;
};

}  // namespace cuvs

namespace cuvs::neighbors::certex {

/** Storage of a half-precision coordinate (IEEE binary16 bits). */
struct half_t {
  uint16_t bits;
};

/** Storage of a bfloat16 coordinate (the upper 16 bits of an IEEE binary32). An addition of this
 *  build: a float index of bfloat16 vectors keeps them exactly at 2 bytes per coordinate. */
struct bfloat16_t {
  uint16_t bits;
};

/** Parameters of an index (reference certex.hpp:43-89). */
struct index_params {
  cuvs::distance::DistanceType metric = cuvs::distance::DistanceType::L2Expanded;
  int width                          = 0;
  double variance                    = 0.95;
  int anchor_stride                  = 16;
  int64_t pca_sample                 = 1000000;
  bool host_vectors                  = false;
  int n_lists                        = 0;
  int64_t kmeans_sample              = 1000000;
  bool local_projections             = false;
  bool int8_rows                     = false;
  /** Rows allocated by the build (0: the dataset's); this build's addition. Later additions up
   * to it need no reallocation, which briefly holds two copies of the stored rows. */
  int64_t capacity = 0;
};

/**
 * Parameters of a search (reference certex.hpp:96-107). anchors: the reference scores exactly the
 * best anchor of each of max(anchors, 2k) top anchor groups and takes the k-th best score; this
 * build takes the k-th best over every anchor group, certified from screen values (8-bit vectors:
 * exact integer screen values; float vectors: the certificate's upper bound of the score), which
 * is the reference's choice with anchors at least the number of groups, so the value cannot
 * change the threshold; any value is accepted, as in the reference.
 */
struct search_params {
  int anchors     = 128;
  int batch_size  = 2048;
  int probe_lists = 2;
};

/** A dense row-major matrix in device or host memory. */
template <typename T>
struct matrix_view {
  T* data        = nullptr;
  int64_t rows   = 0;
  int64_t cols   = 0;
  bool on_device = true;
};

/** Filter of a search (reference Filter, detail/kernels.hpp:39-62). */
struct filter {
  enum class kind : int { none = 0, bitset = 1, bitmap = 2 };
  kind type             = kind::none;
  const uint32_t* words = nullptr;  // device words; bit j of word i is entry 32 i + j
};

/** Counters of the searches of the calling thread (reference detail/kernels.hpp:256-263). */
struct search_stats {
  int64_t queries   = 0;
  int64_t survivors = 0;
  int64_t verified  = 0;
};
/** Start counting the searches of the calling thread (syncs the search streams while on). */
void stats_begin();
/** Stop counting and return the counts since stats_begin(). */
auto stats_end() -> search_stats;

/** Kernel time of the searches of the calling thread, recorded with HIP events per phase. */
struct kernel_times {
  double ms[4]        = {0, 0, 0, 0};  // anchors, threshold, screen, verify + top-k
  int64_t launches[4] = {0, 0, 0, 0};
};
void timing_begin();
auto timing_end() -> kernel_times;
/** Testing only (no counterpart in the reference): copy the intermediate arrays of the calling
 *  thread's next search batch (an unrouted search without a list probe) and the index's screening
 *  rows; capture_get returns an array's bytes and copies it to `host` unless null. */
void capture_begin();
auto capture_get(std::string const& name, void* host) -> int64_t;
/** Average shader clock (MHz) of the screen workgroups timed between the last timing_begin() and
 *  timing_end(): their lives in shader clock cycles over their lives in real time; 0 if none. */
auto timing_shader_clock_mhz() -> double;

namespace detail {
struct index_state;
}

/**
 * Exact k-NN index. Every search returns the exact k nearest stored vectors of every query, ranked
 * by the total order (fp64 score, id), so that ties go to the lower id.
 */
template <typename T>
class index {
 public:
  explicit index(cuvs::resources const& res);
  index(index&&) noexcept;
  index& operator=(index&&) noexcept;
  ~index();

  [[nodiscard]] auto size() const noexcept -> int64_t;
  [[nodiscard]] auto dim() const noexcept -> int64_t;
  [[nodiscard]] auto capacity() const noexcept -> int64_t;
  [[nodiscard]] auto n_removed() const noexcept -> int64_t;
  [[nodiscard]] auto width() const noexcept -> int;
  [[nodiscard]] auto anchor_stride() const noexcept -> int;
  [[nodiscard]] auto metric() const noexcept -> cuvs::distance::DistanceType;
  [[nodiscard]] auto has_labels() const noexcept -> bool;
  /** Vectors covered by the label partition (0: none; later additions are not). */
  [[nodiscard]] auto n_partitioned() const noexcept -> int64_t;
  /**
   * k-means lists (index_params::n_lists; reference certex.hpp:321-334): the stored rows
   * [list_offsets()[j], list_offsets()[j + 1]) hold the vectors of list j, which covers the
   * vectors of the build; later vectors follow in insertion order. 0 lists: rows are ids.
   */
  [[nodiscard]] auto n_lists() const noexcept -> int;
  [[nodiscard]] auto list_offsets() const noexcept -> std::vector<int64_t> const&;
  [[nodiscard]] auto host_vectors() const noexcept -> bool;
  [[nodiscard]] auto state() const -> detail::index_state&;

 private:
  std::unique_ptr<detail::index_state> s_;
};

/** Build an index from a dataset [n, dim] (reference certex.hpp:481-529). */
template <typename T>
auto build(cuvs::resources const& res, index_params const& params, matrix_view<const T> dataset)
  -> index<T>;

/** Append vectors; they receive the next consecutive ids (reference certex.hpp:531-560). */
template <typename T>
void extend(cuvs::resources const& res, matrix_view<const T> new_vectors, index<T>* idx);

/** Grow the capacity to at least `capacity` rows without adding vectors. */
template <typename T>
void reserve(cuvs::resources const& res, int64_t capacity, index<T>* idx);

/** Remove vectors by id (device int64 ids); no later search returns them (certex.hpp:562-575). */
template <typename T>
void remove(cuvs::resources const& res, const int64_t* ids, int64_t n_ids, index<T>* idx);

/** Set the labels (device int32, >= 0) of the vectors first .. first + n - 1 (certex.hpp:577-600). */
template <typename T>
void set_labels(cuvs::resources const& res, const int32_t* labels, int64_t n, index<T>* idx,
                int64_t first = 0);

/**
 * Copy the screening rows into label order (reference certex.hpp:601-624, certex.cu:1542-1606),
 * a speed option of label search: each label's queries then screen only that label's rows, and
 * the rows added later go through the label filter. Needs labels; results do not change.
 */
template <typename T>
void partition_by_labels(cuvs::resources const& res, index<T>* idx);

/**
 * Exact k nearest neighbours of every query (reference certex.hpp:602-705): queries [nq, dim] in
 * device memory, neighbors [nq, k] int64 and distances [nq, k] float32 in device memory. Distances
 * follow cuVS brute force: squared L2, inner products, or cosine distances (1 - cos). Entries
 * beyond the vectors that the filter keeps get id -1 and distance +inf (-inf for inner products).
 */
template <typename T>
void search(cuvs::resources const& res, search_params const& params, index<T> const& idx,
            matrix_view<const T> queries, int64_t* neighbors, float* distances, int64_t k,
            filter f = {});

/**
 * The search above, with no device or pinned memory allocated during the call (no counterpart in
 * the reference; for callers that cannot allocate, such as tight serving loops). Its scratch is a
 * fixed array of no_alloc_scratch_bytes() (128 MiB) per GPU, held from the library's load on that
 * GPU until the process ends; batches that need more are split. Calls on one GPU take turns on
 * that array: on the host by a lock, and on the GPU by an event that each call's stream waits for
 * and records again after its last kernel. Throws when a single query needs more.
 */
template <typename T>
void search_without_allocation(cuvs::resources const& res, search_params const& params,
                               index<T> const& idx, matrix_view<const T> queries,
                               int64_t* neighbors, float* distances, int64_t k, filter f = {});
/** Bytes of the per-GPU scratch array of search_without_allocation. */
auto no_alloc_scratch_bytes() -> size_t;

/**
 * Exact k nearest neighbours of every query among the vectors of its label (int32 labels, one per
 * query). The labels are in device memory, or in host memory with labels_on_host: the search over
 * the label partition plans its launches from them on the host, and host labels spare it a copy
 * back and a wait for the stream.
 */
template <typename T>
void search(cuvs::resources const& res, search_params const& params, index<T> const& idx,
            matrix_view<const T> queries, const int32_t* query_labels, int64_t* neighbors,
            float* distances, int64_t k, bool labels_on_host = false);

/**
 * The ids in the order of the stored rows (reference Index.list_order, certex/index.py:353-359,
 * served by python/src/core.cpp list_order): out[row] = the id stored at row, for all size()
 * rows, written to device memory on the stream of `res`. Rows of the build are in list order;
 * rows added later are their own ids. An index without lists is an error.
 */
template <typename T>
void list_order(cuvs::resources const& res, index<T> const& idx, int32_t* out);

/**
 * Save the index, its vectors and every quantity a search reads (reference
 * certex_serialize.cu:42-150). The file starts with the NumPy descriptor of the vector type padded
 * to 4 bytes ("<f4", "<f2", "|i1", "|u1"), the magic 0x43455258 and the format version.
 */
template <typename T>
void serialize(cuvs::resources const& res, std::string const& filename, index<T> const& idx);

/** Load an index saved by serialize into `idx` (reference certex_serialize.cu:152-243). */
template <typename T>
void deserialize(cuvs::resources const& res, std::string const& filename, index<T>* idx);

}  // namespace cuvs::neighbors::certex
