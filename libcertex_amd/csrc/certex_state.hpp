// Internal state of the resources and of an index, shared by the C++ API and the C API.
#pragma once

#include <cuvs/neighbors/certex.hpp>

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <shared_mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "kernels.hpp"

#define CERTEX_HIP_TRY(call)                                                              \
  do {                                                                                    \
    const hipError_t e_ = (call);                                                         \
    if (e_ != hipSuccess) {                                                               \
      throw std::runtime_error(std::string("certex: HIP error: ") + hipGetErrorString(e_) + \
                               " at " #call);                                             \
    }                                                                                     \
  } while (0)

namespace cuvs::neighbors::certex {

/** Thrown when a batch needs more scratch memory than allowed; the search halves the batch. */
struct batch_too_large : std::runtime_error {
  batch_too_large() : std::runtime_error("certex: the batch does not fit the scratch memory") {}
};

inline void expects(bool ok, const char* message)
{
  if (!ok) { throw std::invalid_argument(message); }
}

}  // namespace cuvs::neighbors::certex

namespace cuvs::detail {

/**
 * Owned memory that kernels read: device memory, or (host = true) pinned host memory mapped into
 * the device's address space (hipHostMalloc), which kernels read over PCIe.
 */
struct device_buffer {
  void* p      = nullptr;
  size_t bytes = 0;
  bool host    = false;
  device_buffer() = default;
  explicit device_buffer(size_t n, bool in_host = false) : host(in_host) { resize_discard(n); }
  device_buffer(device_buffer const&)            = delete;
  device_buffer& operator=(device_buffer const&) = delete;
  device_buffer(device_buffer&& o) noexcept : p(o.p), bytes(o.bytes), host(o.host)
  {
    o.p     = nullptr;
    o.bytes = 0;
  }
  device_buffer& operator=(device_buffer&& o) noexcept
  {
    std::swap(p, o.p);
    std::swap(bytes, o.bytes);
    std::swap(host, o.host);
    return *this;
  }
  ~device_buffer() { release(); }
  void release()
  {
    if (p != nullptr) { (void)(host ? hipHostFree(p) : hipFree(p)); }
    p     = nullptr;
    bytes = 0;
  }
  /** Reallocate to n bytes (contents lost). */
  void resize_discard(size_t n)
  {
    release();
    if (n > 0) {
      const hipError_t e = host ? hipHostMalloc(&p, n, hipHostMallocMapped) : hipMalloc(&p, n);
      if (e != hipSuccess) {
        (void)hipGetLastError();
        p = nullptr;
        throw std::bad_alloc();
      }
      bytes = n;
    }
  }
  template <typename U>
  U* as() const
  {
    return static_cast<U*>(p);
  }
};

/** Slots of the scratch memory of a search. */
enum ws_slot : int {
  ws_qcodes = 0,
  ws_gmax,
  ws_theta,
  ws_count,
  ws_rows,
  ws_small,
  ws_staging,
  ws_qscal,
  ws_vals,
  ws_route,       // label routing of a batch: order, sorted labels, group tables
  ws_probe_dist,  // list probe: center distances of the batch's queries
  ws_probe,       // list probe: nearest lists, pair tables
  ws_probe_rows,  // list probe: the query row of every (query, list) pair
  ws_spill,       // screen spill pool: packed query and row of each entry (+ value, fp16 rows)
  ws_qpaired,     // the batch's fp16 query rows in the paired layout (the tiled screen)
  ws_qlabels,     // query labels given in host memory, copied for the label filter
  ws_n_slots
};

[[noreturn]] inline void throw_too_large() { throw cuvs::neighbors::certex::batch_too_large(); }

struct resources_state {
  int device          = 0;
  hipStream_t stream  = nullptr;
  bool owns_stream    = false;
  int64_t bucket_cap  = 1024;  // survivors per query kept by the last searches
  bool spill_pool     = false;  // a screen's LDS survivor lists overflowed: provide a spill pool
  device_buffer slots[ws_n_slots];
  void* host_small    = nullptr;  // pinned host words for counters read back by the host
  hipEvent_t read_back = nullptr;  // recorded behind a read-back into host_small
  void* host_stage    = nullptr;  // pinned host staging of the routing tables (grow-only)
  size_t host_stage_bytes = 0;
  hipEvent_t staged   = nullptr;  // recorded behind the last copy out of host_stage
  bool staged_pending = false;    // `staged` has been recorded
  // testing only: a slot request above this many bytes fails as an allocation failure would
  // (resources::set_scratch_cap, C cuvsCertexTestScratchCap; 0 = none)
  size_t slot_cap = 0;

  // Arena mode (searches that allocate nothing): while `arena` is set, get() carves the slots
  // out of [arena, arena + arena_bytes) instead of the owned buffers, and a request that does
  // not fit throws batch_too_large (the search then halves its batch and starts the arena over).
  // Work is stream-ordered, so a batch may reuse what the previous batch of the stream carved.
  char* arena        = nullptr;
  size_t arena_bytes = 0;
  size_t arena_used  = 0;
  void* carved[ws_n_slots]        = {};
  size_t carved_bytes[ws_n_slots] = {};

  /** Forget every carved slot: the next batch carves from the start of the arena. */
  void arena_reset()
  {
    arena_used = 0;
    for (int i = 0; i < ws_n_slots; ++i) {
      carved[i]       = nullptr;
      carved_bytes[i] = 0;
    }
  }

  /** Pinned host staging of at least `bytes` bytes (grow-only; waits for the stream first). The
   *  last copy out of it has completed when this returns. */
  void* stage(size_t bytes)
  {
    if (arena != nullptr) {
      throw std::logic_error("certex: a search without allocation cannot stage host memory");
    }
    if (staged_pending) {
      CERTEX_HIP_TRY(hipEventSynchronize(staged));
      staged_pending = false;
    }
    if (host_stage_bytes < bytes) {
      CERTEX_HIP_TRY(hipStreamSynchronize(stream));
      if (host_stage != nullptr) { CERTEX_HIP_TRY(hipHostFree(host_stage)); }
      host_stage       = nullptr;
      host_stage_bytes = 0;
      const size_t n   = bytes + bytes / 4;
      CERTEX_HIP_TRY(hipHostMalloc(&host_stage, n, hipHostMallocDefault));
      host_stage_bytes = n;
    }
    return host_stage;
  }

  /** Copies `bytes` of the staging to device memory `dst` on the stream, without waiting; the
   *  next stage() waits for the copy before it hands the staging out again. */
  void copy_staged(void* dst, size_t bytes)
  {
    CERTEX_HIP_TRY(hipMemcpyAsync(dst, host_stage, bytes, hipMemcpyHostToDevice, stream));
    CERTEX_HIP_TRY(hipEventRecord(staged, stream));
    staged_pending = true;
  }

  /** Scratch slot of at least `bytes` bytes (grow-only; waits for the stream before growing). */
  void* get(int slot, size_t bytes)
  {
    if (arena != nullptr) {
      if (carved_bytes[slot] >= bytes) { return carved[slot]; }
      const size_t n = (bytes + 255) / 256 * 256;
      if (n > arena_bytes - arena_used) { throw_too_large(); }
      carved[slot]       = arena + arena_used;
      carved_bytes[slot] = n;
      arena_used += n;
      return carved[slot];
    }
    if (slot_cap > 0 && bytes > slot_cap) { throw std::bad_alloc(); }
    device_buffer& b = slots[slot];
    if (b.bytes < bytes) {
      CERTEX_HIP_TRY(hipStreamSynchronize(stream));
      b.resize_discard(bytes + bytes / 4);
    }
    return b.p;
  }
};

}  // namespace cuvs::detail

namespace cuvs::neighbors::certex::detail {

enum class vtype : int { f32 = 0, f16 = 1, i8 = 2, u8 = 3, bf16 = 4 };

template <typename T>
constexpr vtype vtype_of();
template <>
constexpr vtype vtype_of<float>() { return vtype::f32; }
template <>
constexpr vtype vtype_of<half_t>() { return vtype::f16; }
template <>
constexpr vtype vtype_of<bfloat16_t>() { return vtype::bf16; }
template <>
constexpr vtype vtype_of<int8_t>() { return vtype::i8; }
template <>
constexpr vtype vtype_of<uint8_t>() { return vtype::u8; }

/**
 * A copy of the screening rows and row terms of the ids [0, n) ordered by a key (label or list):
 * ids[i] = id of partition row i, pos[id] = its partition row; the rows of key j are
 * [offsets[j], offsets[j + 1]).
 */
struct row_partition {
  int64_t n   = 0;
  bool paired = false;  // codes in the paired layout (rows of more than 256 bytes)
  cuvs::detail::device_buffer codes;
  cuvs::detail::device_buffer rowc;
  cuvs::detail::device_buffer ids;
  cuvs::detail::device_buffer pos;
  std::vector<int64_t> offsets;
  cuvs::detail::device_buffer offsets_dev;  // the same offsets on the device (int64)
};

struct index_state {
  int device                            = 0;
  vtype type                            = vtype::f32;
  cuvs::distance::DistanceType dmetric  = cuvs::distance::DistanceType::L2Expanded;
  certex_amd::metric_kind metric        = certex_amd::metric_kind::l2;
  int64_t dim                           = 0;
  int64_t size                          = 0;
  int64_t capacity                      = 0;
  int64_t n_removed                     = 0;
  int row_bytes                         = 0;
  int anchor_stride                     = 16;
  int width                             = 0;
  bool host_vectors                     = false;
  bool has_labels                       = false;
  index_params params{};
  // screening rows and their terms. Integer vectors: int8 codes (the vectors themselves, uint8
  // shifted by -128) and int32 terms. Float vectors: fp16 rows of (x - center) / alpha and fp32
  // terms; the vectors as given are kept in `vectors` for the exact scores.
  cuvs::detail::device_buffer codes;
  cuvs::detail::device_buffer rowc;
  cuvs::detail::device_buffer labels;
  cuvs::detail::device_buffer vectors;  // float vectors [capacity, dim]; pinned host memory when
                                        // host_vectors (the exact-score kernels read it over PCIe)
  // the anchor copy: anchor j holds the screening row and term of id j * anchor_stride, so that
  // the anchor pass reads consecutive rows whose groups mix rows from all over the index (the
  // stored rows may be in list order)
  cuvs::detail::device_buffer anchor_codes;
  cuvs::detail::device_buffer anchor_rowc;
  cuvs::detail::device_buffer center;   // double [dim]
  cuvs::detail::device_buffer maxima;   // double [2]: max |fp16(Z)|, max |Z - fp16(Z)|
  double alpha   = 1.0;
  double gamma   = 0.0;  // fp32 accumulation error factor of a screening product
  int halves     = 0;    // fp16 row length
  bool normalize = false;
  // label partition (a speed option of label search): a copy of the rows in label order
  row_partition label_part;
  // k-means lists (a speed option of every search: the rows of the nearest lists of a query bound
  // its threshold). The stored rows [0, n_listed) are in list order: list j holds the rows
  // [list_offsets[j], list_offsets[j + 1]); row_ids[row] = its id, id_rows[id] = its row. Rows
  // added later are their own ids.
  int n_lists      = 0;
  int64_t n_listed = 0;
  cuvs::detail::device_buffer row_ids;
  cuvs::detail::device_buffer id_rows;
  cuvs::detail::device_buffer centers;    // float [n_lists, list_width]
  cuvs::detail::device_buffer centers_q;  // the centers in the rows' type [pad_centers, row_bytes]
  cuvs::detail::device_buffer cterm;      // float [pad_centers]: |centers_q|^2 / 2
  std::vector<int64_t> list_offsets;
  cuvs::detail::device_buffer list_offsets_dev;  // the same offsets in device memory
  // cterm with +inf for the lists of fewer than kListAnchorMin anchors, and the count of the others:
  // the center terms of the list-anchor threshold, whose lists then all hold that many anchors
  cuvs::detail::device_buffer cterm_anchor;
  int n_anchor_lists = 0;
  int list_width = 0;  // elements of a screening row: row_bytes (int8) or halves (fp16)
  mutable std::shared_mutex rw;  // searches: shared per batch; publication of updates: exclusive
  std::mutex writer;             // one update at a time
  // the GPU work of the last published update: a writer records it on its stream before it
  // publishes, and every later search or update waits for it on its own stream (a wait on the
  // GPU, not on the host), so that an update needs no host synchronisation to be visible to
  // searches on other streams
  hipEvent_t updated = nullptr;

  index_state() { CERTEX_HIP_TRY(hipEventCreateWithFlags(&updated, hipEventDisableTiming)); }
  ~index_state()
  {
    if (updated != nullptr) { (void)hipEventDestroy(updated); }
  }
  index_state(index_state const&)            = delete;
  index_state& operator=(index_state const&) = delete;

  /** Orders `stream` after the last published update (searches, and writers before they write). */
  void await_updates(hipStream_t stream) const { CERTEX_HIP_TRY(hipStreamWaitEvent(stream, updated, 0)); }
  /** Marks the work queued so far on `stream` as the update about to be published. */
  void mark_update(hipStream_t stream) { CERTEX_HIP_TRY(hipEventRecord(updated, stream)); }
};

}  // namespace cuvs::neighbors::certex::detail
