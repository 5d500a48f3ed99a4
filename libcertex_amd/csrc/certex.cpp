// Host orchestration of the exact k-NN index (MI355X build).
//
// Reference: cpp/src/neighbors/certex/certex.cu (build_from 641-703, extend_from 705-732,
// remove 803-843, search_batch 885-1402, search_one_batch 1404-1443, search 1460-1508,
// set_labels 1815-1840, index ctor / reserve 1844-1936). The pipeline of one batch here:
//   encode queries -> anchor pass (int8 MFMA, best screen value per anchor group) -> threshold
//   (k-th best group) -> screen (int8 MFMA, survivors into per-query buckets) -> one host read of
//   the largest bucket (re-run with larger buckets on overflow, as the reference re-runs on
//   segment overflow) -> fp64 exact scores and top-k by (score, id) -> output conversion.

#include "certex_state.hpp"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <functional>
#include <map>
#include <memory>
#include <new>
#include <thread>

namespace cuvs {

resources::resources(void* stream) : s_(std::make_unique<detail::resources_state>())
{
  CERTEX_HIP_TRY(hipGetDevice(&s_->device));
  if (stream != nullptr) {
    s_->stream = static_cast<hipStream_t>(stream);
  } else {
    CERTEX_HIP_TRY(hipStreamCreateWithFlags(&s_->stream, hipStreamNonBlocking));
    s_->owns_stream = true;
  }
  CERTEX_HIP_TRY(hipHostMalloc(&s_->host_small, 64, hipHostMallocDefault));
  CERTEX_HIP_TRY(hipEventCreateWithFlags(&s_->read_back, hipEventDisableTiming));
  CERTEX_HIP_TRY(hipEventCreateWithFlags(&s_->staged, hipEventDisableTiming));
}

resources::~resources()
{
  if (s_) {
    (void)hipStreamSynchronize(s_->stream);
    for (auto& b : s_->slots) { b.release(); }
    if (s_->host_small) { (void)hipHostFree(s_->host_small); }
    if (s_->read_back) { (void)hipEventDestroy(s_->read_back); }
    if (s_->staged) { (void)hipEventDestroy(s_->staged); }
    if (s_->host_stage) { (void)hipHostFree(s_->host_stage); }
    if (s_->owns_stream) { (void)hipStreamDestroy(s_->stream); }
  }
}

auto resources::stream() const -> void* { return s_->stream; }

void resources::set_stream(void* stream)
{
  CERTEX_HIP_TRY(hipStreamSynchronize(s_->stream));
  if (s_->owns_stream) {
    CERTEX_HIP_TRY(hipStreamDestroy(s_->stream));
    s_->owns_stream = false;
  }
  s_->stream = static_cast<hipStream_t>(stream);
}

auto resources::device() const -> int { return s_->device; }

void resources::sync() const { CERTEX_HIP_TRY(hipStreamSynchronize(s_->stream)); }

void resources::trim() const
{
  if (s_->arena != nullptr) {
    throw std::logic_error("certex: trim during a search without allocation on these resources");
  }
  CERTEX_HIP_TRY(hipStreamSynchronize(s_->stream));
  for (auto& b : s_->slots) { b.release(); }
  if (s_->host_stage != nullptr) {
    CERTEX_HIP_TRY(hipHostFree(s_->host_stage));
    s_->host_stage       = nullptr;
    s_->host_stage_bytes = 0;
    s_->staged_pending   = false;
  }
}

void resources::set_scratch_cap(size_t bytes) const { s_->slot_cap = bytes; }

auto resources::state() const -> detail::resources_state& { return *s_; }

}  // namespace cuvs

namespace cuvs::neighbors::certex {

namespace {

thread_local bool t_stats_on = false;
thread_local search_stats t_stats{};

/** Event pairs around the kernels of the calling thread's searches while timing is on, and the
 *  shader clock counters of the timed screens (two device words, cycles and 100 MHz ticks). */
struct timing_state {
  bool on = false;
  unsigned long long* clock = nullptr;
  double clock_mhz          = 0;
  struct mark {
    int phase;
    hipEvent_t start, stop;
  };
  std::vector<mark> marks;
  std::vector<hipEvent_t> pool;
  auto event() -> hipEvent_t
  {
    if (!pool.empty()) {
      hipEvent_t e = pool.back();
      pool.pop_back();
      return e;
    }
    hipEvent_t e;
    CERTEX_HIP_TRY(hipEventCreate(&e));
    return e;
  }
};
thread_local timing_state t_timing;

/**
 * Testing only: copies of the intermediate arrays of the next search batch of the calling thread
 * (query rows, group table, thresholds, buckets, certificate bounds) and of the index's screening
 * rows, taken from the search's own launches, so that tests can check the screen and the
 * certificate against a brute force (capture_begin, capture_get).
 */
struct capture_state {
  bool on = false;
  std::map<std::string, std::vector<char>> arrays;
  void put(const char* name, const void* dev, size_t bytes, hipStream_t stream)
  {
    auto& v = arrays[name];
    v.resize(bytes);
    if (bytes > 0) { CERTEX_HIP_TRY(hipMemcpyAsync(v.data(), dev, bytes, hipMemcpyDefault, stream)); }
  }
  template <typename V>
  void value(const char* name, V x)
  {
    auto& v = arrays[name];
    v.resize(sizeof(V));
    std::memcpy(v.data(), &x, sizeof(V));
  }
};
thread_local capture_state t_capture;

/** A device array of n elements that lives for one capture (testing only). */
template <typename V>
struct capture_buffer {
  V* p = nullptr;
  explicit capture_buffer(size_t n) { CERTEX_HIP_TRY(hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(V))); }
  ~capture_buffer() { (void)hipFree(p); }
  capture_buffer(capture_buffer const&)            = delete;
  capture_buffer& operator=(capture_buffer const&) = delete;
};

/** Run `launch` between two events of `phase` when timing is on. */
template <typename F>
void timed(int phase, hipStream_t stream, F&& launch)
{
  if (!t_timing.on) {
    launch();
    return;
  }
  hipEvent_t a = t_timing.event(), b = t_timing.event();
  CERTEX_HIP_TRY(hipEventRecord(a, stream));
  launch();
  CERTEX_HIP_TRY(hipEventRecord(b, stream));
  t_timing.marks.push_back({phase, a, b});
}

using certex_amd::metric_kind;
using detail::index_state;
using detail::vtype;

auto to_kind(cuvs::distance::DistanceType m) -> metric_kind
{
  switch (m) {
    case cuvs::distance::DistanceType::L2Expanded: return metric_kind::l2;
    case cuvs::distance::DistanceType::InnerProduct: return metric_kind::inner;
    case cuvs::distance::DistanceType::CosineExpanded: return metric_kind::cosine;
  }
  throw std::invalid_argument("certex supports L2Expanded, InnerProduct, and CosineExpanded");
}

auto is_int(vtype t) -> bool { return t == vtype::i8 || t == vtype::u8; }
auto elem_of(vtype t) -> certex_amd::elem
{
  return t == vtype::f32 ? certex_amd::elem::f32
                         : (t == vtype::bf16 ? certex_amd::elem::bf16 : certex_amd::elem::f16);
}
auto elem_size(vtype t) -> size_t
{
  return t == vtype::f32 ? 4 : ((t == vtype::f16 || t == vtype::bf16) ? 2 : 1);
}

/** Grow every per-row array to `cap` rows (the caller holds the writer lock). */
void grow(cuvs::resources const& res, index_state& st, int64_t cap)
{
  if (cap <= st.capacity) { return; }
  hipStream_t stream = static_cast<hipStream_t>(res.stream());
  const size_t vbytes = is_int(st.type) ? 0 : size_t(st.dim) * elem_size(st.type);
  cuvs::detail::device_buffer codes(size_t(cap) * st.row_bytes);
  cuvs::detail::device_buffer rowc(size_t(cap) * 4);
  cuvs::detail::device_buffer vectors(size_t(cap) * vbytes, st.host_vectors);
  const int64_t s       = std::max(1, st.anchor_stride);
  const int64_t a_cap   = (cap + s - 1) / s;
  const int64_t a_size  = (st.size + s - 1) / s;
  cuvs::detail::device_buffer anchor_codes(size_t(a_cap) * st.row_bytes);
  cuvs::detail::device_buffer anchor_rowc(size_t(a_cap) * 4);
  cuvs::detail::device_buffer labels;
  auto copy = [&](cuvs::detail::device_buffer& dst, cuvs::detail::device_buffer const& src,
                  size_t bytes) {  // device or pinned host memory on either side
    if (bytes > 0) { CERTEX_HIP_TRY(hipMemcpyAsync(dst.p, src.p, bytes, hipMemcpyDefault, stream)); }
  };
  copy(codes, st.codes, size_t(st.size) * st.row_bytes);
  copy(rowc, st.rowc, size_t(st.size) * 4);
  copy(vectors, st.vectors, size_t(st.size) * vbytes);
  copy(anchor_codes, st.anchor_codes, size_t(a_size) * st.row_bytes);
  copy(anchor_rowc, st.anchor_rowc, size_t(a_size) * 4);
  if (st.has_labels) {
    labels.resize_discard(size_t(cap) * sizeof(int32_t));
    certex_amd::fill_i32(labels.as<int32_t>(), cap, -1, stream);
    copy(labels, st.labels, size_t(st.size) * sizeof(int32_t));
  }
  CERTEX_HIP_TRY(hipStreamSynchronize(stream));
  {
    // searches in flight on other streams may still read the old arrays
    std::unique_lock lk(st.rw);
    CERTEX_HIP_TRY(hipDeviceSynchronize());
    st.codes        = std::move(codes);
    st.rowc         = std::move(rowc);
    st.vectors      = std::move(vectors);
    st.anchor_codes = std::move(anchor_codes);
    st.anchor_rowc  = std::move(anchor_rowc);
    if (st.has_labels) { st.labels = std::move(labels); }
    st.capacity = cap;
  }
}

/** The anchor copy of the ids [first, end): anchors ceil(first / s) .. ceil(end / s) - 1. */
void refresh_anchors(cuvs::resources const& res, index_state& st, int64_t first, int64_t end)
{
  const int64_t s = std::max(1, st.anchor_stride);
  // anchor j is id j * s, read from its stored row: id_rows[id] for listed ids
  certex_amd::gather_anchors(st.codes.p, st.rowc.p, st.row_bytes, s, (first + s - 1) / s,
                             (end + s - 1) / s, st.id_rows.as<int32_t>(), st.n_listed,
                             st.anchor_codes.p, st.anchor_rowc.p,
                             static_cast<hipStream_t>(res.stream()));
}

/** Encode integer rows [0, n) of a device or host matrix into stored rows first, first + 1, ... */
void append_int(cuvs::resources const& res, index_state& st, const uint8_t* x, int64_t n,
                bool on_device, int64_t first)
{
  hipStream_t stream = static_cast<hipStream_t>(res.stream());
  const uint8_t flip = st.type == vtype::u8 ? 0x80 : 0;
  if (on_device) {
    certex_amd::encode_rows_i8(x, n, st.dim, st.row_bytes, flip, st.metric,
                               st.codes.as<int8_t>() + first * st.row_bytes,
                               st.rowc.as<int32_t>() + first, stream);
    return;
  }
  // host rows: staged through device memory in chunks of at most 64 MB
  const int64_t chunk = std::max<int64_t>(1, (int64_t(64) << 20) / std::max<int64_t>(1, st.dim));
  cuvs::detail::device_buffer staging(size_t(std::min(chunk, n)) * st.dim);
  for (int64_t r = 0; r < n; r += chunk) {
    const int64_t m = std::min(chunk, n - r);
    CERTEX_HIP_TRY(hipMemcpyAsync(staging.p, x + r * st.dim, size_t(m) * st.dim,
                                  hipMemcpyHostToDevice, stream));
    certex_amd::encode_rows_i8(staging.as<uint8_t>(), m, st.dim, st.row_bytes, flip, st.metric,
                               st.codes.as<int8_t>() + (first + r) * st.row_bytes,
                               st.rowc.as<int32_t>() + first + r, stream);
    CERTEX_HIP_TRY(hipStreamSynchronize(stream));
  }
}

/** Copy float rows [0, n) into the stored vectors first, ... and encode their screening rows. */
void append_float(cuvs::resources const& res, index_state& st, const void* x, int64_t n,
                  bool on_device, int64_t first)
{
  hipStream_t stream = static_cast<hipStream_t>(res.stream());
  const size_t rb    = size_t(st.dim) * elem_size(st.type);
  char* dst          = st.vectors.as<char>() + size_t(first) * rb;
  // the stored vectors are device or pinned host memory, the source device or host memory
  (void)on_device;
  CERTEX_HIP_TRY(hipMemcpyAsync(dst, x, size_t(n) * rb, hipMemcpyDefault, stream));
  certex_amd::encode_rows_f16(dst, elem_of(st.type), n, st.dim, st.halves, st.normalize,
                              st.center.as<double>(), 1.0 / st.alpha, st.metric, st.gamma,
                              st.codes.as<uint16_t>() + size_t(first) * st.halves,
                              st.rowc.as<float>() + first, st.maxima.as<double>(), stream);
}

/**
 * Anchor grouping: the anchor pass records one best value per group of group_steps * 64 anchors
 * (coarse), or per group of 4 anchors (fine) when k is large next to the anchor steps, so that
 * the k-th best group stays close to the k-th best anchor; the [nq_pad, n_groups] table stays
 * under 1 GB.
 */
struct anchor_plan {
  int stride;
  int64_t first = 0;  // plain passes: the first anchor of the anchor copy that the pass covers
  int64_t n_anchor, n_groups;
  int64_t group_steps;
  bool fine = false;
};
constexpr int64_t kTableBytes = int64_t(1) << 30;

/** Coarse groups when there are at least 64 k anchor steps; fine groups otherwise. */
void size_groups(anchor_plan& p, int64_t max_anchors, int64_t tail_anchors, int64_t nq_pad, int k,
                 int64_t* part_groups)
{
  const int64_t steps      = certex_amd::screen_steps(max_anchors);
  const int64_t tail_steps = certex_amd::screen_steps(tail_anchors);
  const int64_t q          = certex_amd::kFineGroup;
  const int64_t fine_cols  = (max_anchors + q - 1) / q + (tail_anchors + q - 1) / q;
  if (steps < 64 * int64_t(k) && nq_pad * fine_cols * 4 <= kTableBytes) {
    p.fine        = true;
    p.group_steps = 1;
    p.n_groups    = fine_cols;
    *part_groups  = (max_anchors + q - 1) / q;
    return;
  }
  int64_t g = std::max<int64_t>(1, steps / (64 * int64_t(k)));
  while (nq_pad * ((steps + g - 1) / g + (tail_steps + g - 1) / g) * 4 > kTableBytes) { g *= 2; }
  p.fine        = false;
  p.group_steps = g;
  *part_groups  = (steps + g - 1) / g;
  p.n_groups    = *part_groups + (tail_steps + g - 1) / g;
}

/** The anchors of the anchor copy from anchor `first` on. */
auto plan_anchors(index_state const& st, int64_t first, int64_t nq_pad, int k) -> anchor_plan
{
  anchor_plan p{};
  p.stride   = std::max(1, st.anchor_stride);
  p.first    = first;
  p.n_anchor = (st.size + p.stride - 1) / p.stride - first;
  int64_t part = 0;
  size_groups(p, p.n_anchor, 0, nq_pad, k, &part);
  return p;
}

/**
 * Routing of one label-sorted batch over the label partition (reference route_plan,
 * certex.cu:1669-1712): per label, its queries against its partition rows, as two group tables
 * (the anchor pass and the screen tile the groups differently); the rows added after the
 * partition (the tail) are screened with the label filter.
 */
struct route_plan {
  const certex_amd::screen_group* anchor_groups = nullptr;
  const certex_amd::screen_group* screen_groups = nullptr;
  int n_route          = 0;
  int64_t anchor_tiles = 0, screen_tiles = 0;
  int anchor_chunk     = 0;
  int screen_chunk     = 0;
  bool anchor_tiled    = false;  // the partition's anchor pass runs as tiles (anchors_f16_tile)
  int64_t part_groups  = 0;  // anchor group columns of the partition (the tail's follow)
  // every query of the batch is routed and every label's fine groups fill all part_groups
  // columns: the routed anchor pass then writes every column of the batch's table rows itself
  bool covers_table = false;
  anchor_plan ap{};
  // query i of the batch (in label order) is the caller's query rows[i], and its results go to the
  // caller's row rows[i] (null: the batch is in the caller's order)
  const int32_t* rows = nullptr;
};

constexpr int kScreenChunk = 128;      // most steps per screen workgroup
constexpr int kRoutedChunk = 32;       // most steps per workgroup of a routed screen
constexpr int64_t kMinTiles = 2048;    // workgroups a launch should have (8 per CU)

auto anchor_chunk_steps(bool wide, int64_t g) -> int
{
  return int(wide ? 8 * g * std::max<int64_t>(1, 4 / g) : 4 * g * std::max<int64_t>(1, 16 / g));
}

/**
 * Steps per workgroup: the largest of cap, cap / 2, ... (multiples of unit) that still gives the
 * launch kMinTiles workgroups; small batches and short scans split into smaller chunks so that
 * every CU gets work.
 */
template <typename F>
auto pick_chunk(int64_t unit, int64_t cap, F&& tiles) -> int
{
  int64_t c = std::max(unit, cap / unit * unit);
  while (c > unit && tiles(c) < kMinTiles) { c = std::max(unit, c / 2 / unit * unit); }
  return int(c);
}

/** Chunk of a plain (unrouted) pass over n_scan scan indices. */
auto plain_chunk(index_state const& st, int64_t nq, int64_t nq_pad, int64_t n_scan, int64_t unit,
                 int64_t cap) -> int
{
  const bool f16      = !is_int(st.type);
  const int64_t qb    = certex_amd::screen_query_block(f16, st.row_bytes, nq_pad);
  const int64_t n_qb  = (nq + qb - 1) / qb;
  const int64_t steps = certex_amd::screen_steps(n_scan);
  return pick_chunk(unit, cap, [&](int64_t c) { return n_qb * ((steps + c - 1) / c); });
}

auto waves_of(index_state const& st) -> int64_t
{
  return certex_amd::screen_waves(!is_int(st.type), st.row_bytes);
}

/** The screen pass of rows of more than 256 bytes (fp16 rows of more than 128 halves, int8 rows of
 *  more than 256 coordinates) runs the tiled kernel. */
auto uses_tile_screen(index_state const& st) -> bool { return st.row_bytes > 256; }

/**
 * Anchor pass: every anchor of the index, or the partition's (routed) and the tail's, into the
 * columns [0, ap.n_groups) of a group table of row_len columns.
 */
template <typename F>
void anchor_pass(index_state const& st, certex_amd::screen_args aa, anchor_plan const& ap,
                 int64_t row_len, route_plan const* route, F&& launch, hipStream_t stream)
{
  aa.row_stride  = ap.stride;
  aa.n_groups    = row_len;
  aa.group_steps = int(ap.group_steps);
  aa.fine        = ap.fine;
  const int64_t unit = waves_of(st) * ap.group_steps;
  const int64_t cap  = anchor_chunk_steps(waves_of(st) == 8, ap.group_steps);
  if (route == nullptr) {  // the anchor copy, consecutive rows
    aa.codes       = st.anchor_codes.as<int8_t>();
    aa.rowc        = st.anchor_rowc.p;
    aa.row_stride  = 1;
    aa.row_base    = ap.first;
    aa.id_scale    = ap.stride;
    aa.n_scan      = ap.n_anchor;
    aa.chunk_steps = plain_chunk(st, aa.nq, aa.nq_pad, aa.n_scan, unit, cap);
    launch(aa, stream);
    return;
  }
  // columns of labels with fewer groups, and the rows of queries in no group, stay at the lowest
  // value (no anchor); nothing to fill when the routed pass writes every column of every row
  if (!route->covers_table) {
    if (is_int(st.type)) {
      certex_amd::fill_i32(static_cast<int32_t*>(aa.gmax), aa.nq_pad * ap.n_groups, INT32_MIN,
                           stream);
    } else {
      certex_amd::fill_u32(static_cast<uint32_t*>(aa.gmax), aa.nq_pad * ap.n_groups, 0xff800000u,
                           stream);
    }
  }
  certex_amd::screen_args r = aa;
  r.codes                   = st.label_part.codes.as<int8_t>();
  r.rowc                    = st.label_part.rowc.p;
  r.rows_paired             = st.label_part.paired;
  r.anchor_pairs            = st.label_part.paired;
  r.tiled                   = route->anchor_tiled;
  r.groups                  = route->anchor_groups;
  r.n_route                 = route->n_route;
  r.n_tiles                 = route->anchor_tiles;
  r.chunk_steps             = route->anchor_chunk;
  r.filter.kind             = 0;  // every row of a group carries the group's label
  if (r.n_tiles > 0) { launch(r, stream); }
  const int64_t tail = st.size - st.label_part.n;
  if (tail > 0) {
    certex_amd::screen_args t = aa;
    t.row_base                = st.label_part.n;
    t.n_scan                  = (tail + ap.stride - 1) / ap.stride;
    t.grp_base                = route->part_groups;
    t.chunk_steps             = plain_chunk(st, t.nq, t.nq_pad, t.n_scan, unit, cap);
    launch(t, stream);
  }
}

/** Screen pass: every row, or the partition's (routed) and the tail's (label filter). */
template <typename F>
auto screen_pass(index_state const& st, route_plan const* route, F&& launch)
{
  // fp16 rows of more than 128 halves: the tiled screen, one tile of 256 rows per workgroup
  const bool tiled = uses_tile_screen(st);
  return [&st, route, launch, tiled](certex_amd::screen_args& sa, hipStream_t stream) {
    auto chunk = [&](certex_amd::screen_args const& x) {
      return tiled ? certex_amd::tile_chunk_steps()
                   : plain_chunk(st, x.nq, x.nq_pad, x.n_scan, waves_of(st), kScreenChunk);
    };
    if (route == nullptr) {
      sa.chunk_steps = chunk(sa);
      launch(sa, stream);
      return;
    }
    certex_amd::screen_args r = sa;
    r.codes                   = st.label_part.codes.as<int8_t>();
    r.rowc                    = st.label_part.rowc.p;
    r.rows_paired             = st.label_part.paired;
    r.groups                  = route->screen_groups;
    r.n_route                 = route->n_route;
    r.n_tiles                 = route->screen_tiles;
    r.chunk_steps             = route->screen_chunk;
    r.filter.kind             = 0;
    if (r.n_tiles > 0) { launch(r, stream); }
    const int64_t tail = st.size - st.label_part.n;
    if (tail > 0) {
      certex_amd::screen_args t = sa;
      t.row_base                = st.label_part.n;
      t.n_scan                  = tail;
      t.chunk_steps             = chunk(t);
      launch(t, stream);
    }
  };
}

/** No work launched behind the screen before its bucket check (see screen_into_buckets). */
struct no_speculation {
  void operator()() const {}
};

/**
 * Screen pass into per-query buckets, re-run with larger buckets while one overflows (the
 * reference re-runs on segment overflow, certex.cu:1208-1269). Returns false when some query
 * keeps so many rows that scoring every row is cheaper (all_rows).
 * `speculate` launches the work that reads the buckets (the exact re-rank) right behind the
 * screen, before the host has read back the largest bucket: the host then waits for that read-back
 * only (an event), not for the re-rank. When the check fails (a re-run, or all_rows) the
 * speculative work has read clipped buckets, and what the caller launches next overwrites its
 * results in stream order.
 */
template <typename F, typename V = no_speculation>
bool screen_into_buckets(cuvs::resources const& res, int64_t B, int64_t nq_pad, int64_t size,
                         certex_amd::screen_args& sa, F&& screen, uint32_t*& count,
                         uint32_t*& rows, int64_t& cap, float** vals = nullptr,
                         int64_t* worst_out = nullptr, V&& speculate = V{})
{
  auto& rs           = res.state();
  hipStream_t stream = rs.stream;
  auto* small        = static_cast<uint32_t*>(rs.get(cuvs::detail::ws_small, 64));
  count              = static_cast<uint32_t*>(rs.get(cuvs::detail::ws_count, size_t(nq_pad) * 4));
  cap                = rs.bucket_cap;
  const int64_t all_rows_above = std::max<int64_t>(1 << 16, size / 8);
  while (true) {
    if (size_t(nq_pad) * size_t(cap) * 4 > (size_t(1) << 32)) { throw batch_too_large(); }
    rows = static_cast<uint32_t*>(
      rs.get(cuvs::detail::ws_rows, size_t(nq_pad) * size_t(cap) * 4));
    if (vals != nullptr) {
      *vals = static_cast<float*>(
        rs.get(cuvs::detail::ws_vals, size_t(nq_pad) * size_t(cap) * 4));
      sa.cand_vals = *vals;
    }
    // survivors past the workgroups' LDS lists: a pool of the buckets' size, once a search of
    // these resources has overflowed them (the first such search took the slower atomic path)
    sa.spill = nullptr, sa.spill_pool = 0;
    if (rs.spill_pool) {
      const size_t e = size_t(nq_pad) * size_t(cap);
      const size_t w = size_t(certex_amd::spill_words(vals != nullptr));
      sa.spill       = static_cast<uint32_t*>(rs.get(cuvs::detail::ws_spill, e * 4 * w));
      sa.spill_pool  = int64_t(e);
    }
    certex_amd::fill_u32(count, nq_pad, 0, stream);
    certex_amd::fill_u32(small, 2, 0, stream);
    sa.spill_need  = small + 1;
    sa.n_scan      = size;
    sa.row_stride  = 1;
    sa.cand_count  = count;
    sa.cand_rows   = rows;
    sa.cap         = cap;
    sa.clock = t_timing.on ? t_timing.clock : nullptr;
    timed(2, stream, [&] { screen(sa, stream); });
    sa.clock = nullptr;
    certex_amd::max_u32(count, B, small, stream);
    CERTEX_HIP_TRY(hipMemcpyAsync(rs.host_small, small, 8, hipMemcpyDeviceToHost, stream));
    CERTEX_HIP_TRY(hipEventRecord(rs.read_back, stream));
    speculate();
    CERTEX_HIP_TRY(hipEventSynchronize(rs.read_back));
    const int64_t worst = static_cast<uint32_t*>(rs.host_small)[0];
    if (static_cast<uint32_t*>(rs.host_small)[1] > 0) { rs.spill_pool = true; }
    if (worst_out != nullptr) { *worst_out = worst; }
    if (worst <= cap) { return true; }
    if (worst > all_rows_above) { return false; }
    int64_t c = 1024;
    while (c < worst) { c *= 2; }
    cap           = c;
    rs.bucket_cap = c;
  }
}

/**
 * Adds the batch's queries and survivors to the thread's counts; `verified` too unless the verify
 * kernel counts the rows it scores itself (verified_by_kernel).
 */
void count_stats(cuvs::resources const& res, index_state const& st, int64_t B, bool all_rows,
                 const uint32_t* count, int64_t cap, bool verified_by_kernel = false)
{
  if (!t_stats_on) { return; }
  auto& rs           = res.state();
  hipStream_t stream = rs.stream;
  t_stats.queries += B;
  if (all_rows) {
    const int64_t live = st.size - st.n_removed;
    t_stats.survivors += B * live;
    if (!verified_by_kernel) { t_stats.verified += B * live; }
    return;
  }
  auto* small = static_cast<uint32_t*>(rs.get(cuvs::detail::ws_small, 64));
  auto* sums  = reinterpret_cast<unsigned long long*>(small + 4);
  certex_amd::fill_u32(small + 4, 4, 0, stream);
  certex_amd::sum_u32(count, B, int64_t(1) << 40, sums, stream);
  certex_amd::sum_u32(count, B, cap, sums + 1, stream);
  CERTEX_HIP_TRY(hipMemcpyAsync(rs.host_small, sums, 16, hipMemcpyDeviceToHost, stream));
  CERTEX_HIP_TRY(hipStreamSynchronize(stream));
  auto* h = static_cast<unsigned long long*>(rs.host_small);
  t_stats.survivors += int64_t(h[0]);
  if (!verified_by_kernel) { t_stats.verified += int64_t(h[1]); }
}

/**
 * The list probe of one batch (reference probe_lists, lists.cuh:351-460): the p nearest lists of
 * every query, and more of its nearest (up to kMaxProbe) while they hold fewer than kProbeRows * k
 * rows. Every (query, list) pair scans all rows of the list as fine anchor groups of 4, written to
 * the query's row of the group table; the pairs are grouped by list so that the rows of a list are
 * read once for all of its queries.
 */
struct probe_plan {
  int64_t n_pairs = 0;
  int64_t nq_pad  = 0;
  int64_t cols    = 0;     // table columns of the probe: those of the query with the most
  bool enough     = true;  // every query met kProbeRows * k rows
  std::vector<int32_t> pair_q, pair_col;  // per pair, in list order
  std::vector<certex_amd::screen_group> groups;
  int64_t group_steps = 0;  // 0: groups of 4 rows; else groups of group_steps steps
  int64_t tiles       = 0;
  int chunk           = 0;
};
constexpr int64_t kProbeRows       = 16;
constexpr int64_t kProbeTableBytes = int64_t(256) << 20;

/** Plans the probe from the encoded query rows; false when the index has no lists to probe. */
bool plan_probe(cuvs::resources const& res, index_state const& st, const void* qrows, int64_t B,
                int k, int p, probe_plan& pp)
{
  auto& rs           = res.state();
  hipStream_t stream = rs.stream;
  const bool f16     = !is_int(st.type);
  const int L        = st.n_lists;
  const int Lp       = certex_amd::pad_centers(L);
  const int pmax     = std::min(L, certex_amd::kMaxProbe);
  p                  = std::min(p, pmax);
  auto* dist  = static_cast<float*>(rs.get(cuvs::detail::ws_probe_dist, size_t(B) * Lp * 4));
  auto* lists = static_cast<int32_t*>(rs.get(cuvs::detail::ws_probe, size_t(B) * pmax * 4));
  certex_amd::center_distances(qrows, f16, B, st.row_bytes, st.centers_q.p, st.cterm.as<float>(),
                               Lp, dist, stream);
  certex_amd::nearest_lists(dist, B, L, Lp, pmax, lists, stream);
  std::vector<int32_t> h(size_t(B) * pmax);
  CERTEX_HIP_TRY(hipMemcpyAsync(h.data(), lists, h.size() * 4, hipMemcpyDeviceToHost, stream));
  CERTEX_HIP_TRY(hipStreamSynchronize(stream));
  const auto& off    = st.list_offsets;
  const int64_t want = kProbeRows * k;
  auto list_rows     = [&](int32_t j) { return off[size_t(j) + 1] - off[size_t(j)]; };
  std::vector<int32_t> taken(static_cast<size_t>(B));
  std::vector<int64_t> start(static_cast<size_t>(L) + 1, 0);
  for (int64_t q = 0; q < B; ++q) {
    int64_t rows = 0;
    int t        = 0;
    for (; t < pmax; ++t) {
      const int32_t j = h[size_t(q * pmax + t)];
      if (j < 0 || (t >= p && rows >= want)) { break; }
      rows += list_rows(j);
      ++start[size_t(j) + 1];
    }
    taken[size_t(q)] = t;
    pp.enough        = pp.enough && rows >= want;
  }
  // groups of 4 rows while the probe's table stays within kProbeTableBytes, else of g steps (64 g
  // rows), g a power of two; every query should keep 4 k groups
  auto list_cols = [&](int32_t j, int64_t g) {
    return g == 0 ? (list_rows(j) + certex_amd::kFineGroup - 1) / certex_amd::kFineGroup
                  : (certex_amd::screen_steps(list_rows(j)) + g - 1) / g;
  };
  auto widest = [&](int64_t g, int64_t* narrowest) {
    int64_t most = 0, least = INT64_MAX;
    for (int64_t q = 0; q < B; ++q) {
      int64_t c = 0;
      for (int t = 0; t < taken[size_t(q)]; ++t) { c += list_cols(h[size_t(q * pmax + t)], g); }
      most  = std::max(most, c);
      least = std::min(least, c);
    }
    *narrowest = least;
    return most;
  };
  const int64_t nq_pad = certex_amd::pad_queries(B);
  int64_t g = 0, least = 0;
  pp.cols   = widest(0, &least);
  while (nq_pad * pp.cols * 4 > kProbeTableBytes) {
    g       = g == 0 ? 1 : 2 * g;
    pp.cols = widest(g, &least);
  }
  pp.group_steps = g;
  pp.enough      = pp.enough && least >= 4 * int64_t(k);
  for (int j = 0; j < L; ++j) { start[size_t(j) + 1] += start[size_t(j)]; }
  pp.n_pairs = start[size_t(L)];
  pp.nq_pad  = certex_amd::pad_queries(pp.n_pairs);
  pp.pair_q.resize(size_t(pp.n_pairs));
  pp.pair_col.resize(size_t(pp.n_pairs));
  {
    std::vector<int64_t> fill(start.begin(), start.end() - 1);
    for (int64_t q = 0; q < B; ++q) {
      int64_t col = 0;
      for (int t = 0; t < taken[size_t(q)]; ++t) {
        const int32_t j   = h[size_t(q * pmax + t)];
        const int64_t s   = fill[size_t(j)]++;
        pp.pair_q[size_t(s)]   = int32_t(q);
        pp.pair_col[size_t(s)] = int32_t(col);
        col += list_cols(j, g);
      }
    }
  }
  for (int j = 0; j < L; ++j) {
    const int64_t nq = start[size_t(j) + 1] - start[size_t(j)];
    if (nq > 0 && list_rows(j) > 0) {
      pp.groups.push_back({start[size_t(j)], nq, off[size_t(j)], list_rows(j), 0});
    }
  }
  if (pp.groups.empty()) { return false; }
  const bool wide     = st.row_bytes > 256;
  const int qb        = certex_amd::screen_query_block(f16, st.row_bytes, pp.nq_pad);
  const int64_t waves = waves_of(st);
  const int64_t gs    = std::max<int64_t>(1, g);
  pp.chunk = pick_chunk(waves * gs, anchor_chunk_steps(wide, gs), [&](int64_t c) {
    int64_t t = 0;
    for (auto const& e : pp.groups) { t += certex_amd::screen_group_tiles(e.nq, e.nx, qb, int(c)); }
    return t;
  });
  for (auto& e : pp.groups) {
    e.tile0  = certex_amd::screen_group_tile0(pp.tiles, e.nq, qb);
    pp.tiles = e.tile0 + certex_amd::screen_group_tiles(e.nq, e.nx, qb, pp.chunk);
  }
  return true;
}

/** The probe's launch into the columns col0 + ... of a group table of row_len columns. */
template <typename F>
void probe_pass(cuvs::resources const& res, index_state const& st, certex_amd::screen_args aa,
                probe_plan const& pp, int64_t col0, int64_t row_len, F&& launch)
{
  auto& rs           = res.state();
  hipStream_t stream = rs.stream;
  // device tables: pair query, pair column, groups
  const size_t pair_bytes = (size_t(pp.n_pairs) * 4 + 15) / 16 * 16;
  const size_t grp_bytes  = pp.groups.size() * sizeof(certex_amd::screen_group);
  std::vector<char> host(2 * pair_bytes + grp_bytes);
  std::memcpy(host.data(), pp.pair_q.data(), size_t(pp.n_pairs) * 4);
  auto* hc = reinterpret_cast<int32_t*>(host.data() + pair_bytes);
  for (int64_t i = 0; i < pp.n_pairs; ++i) { hc[i] = int32_t(col0 + pp.pair_col[size_t(i)]); }
  std::memcpy(host.data() + 2 * pair_bytes, pp.groups.data(), grp_bytes);
  char* dev = static_cast<char*>(rs.get(cuvs::detail::ws_probe, host.size()));
  CERTEX_HIP_TRY(hipMemcpyAsync(dev, host.data(), host.size(), hipMemcpyHostToDevice, stream));
  const auto* d_q = reinterpret_cast<const int32_t*>(dev);
  auto* rows      = rs.get(cuvs::detail::ws_probe_rows, size_t(pp.nq_pad) * st.row_bytes);
  certex_amd::gather_rows(aa.qcodes, d_q, pp.n_pairs, st.row_bytes, rows, stream);
  certex_amd::screen_args r = aa;
  r.codes       = st.codes.as<int8_t>();
  r.rowc        = st.rowc.p;
  r.qcodes      = static_cast<const int8_t*>(rows);
  r.nq          = pp.n_pairs;
  r.nq_pad      = pp.nq_pad;
  r.groups      = reinterpret_cast<const certex_amd::screen_group*>(dev + 2 * pair_bytes);
  r.n_route     = int(pp.groups.size());
  r.n_tiles     = pp.tiles;
  r.chunk_steps = pp.chunk;
  r.row_stride  = 1;
  r.row_base    = 0;
  r.fine        = pp.group_steps == 0;
  r.group_steps = int(std::max<int64_t>(1, pp.group_steps));
  r.grp_base    = 0;
  r.n_groups    = row_len;
  r.out_row     = d_q;
  r.out_col     = reinterpret_cast<const int32_t*>(dev + pair_bytes);
  launch(r, stream);
  CERTEX_HIP_TRY(hipStreamSynchronize(stream));  // the host tables go out of scope
}

/**
 * The group table of a batch: the anchors' groups, or the list probe's groups over the listed rows
 * and the anchors' over the rows added after the lists (columns of the anchors first). No stored
 * row may sit in two groups: the k-th best group must stand for k distinct rows. Without enough
 * rows in some query's probed lists the batch uses the anchors alone.
 */
/** Fewest anchors of a list whose anchors may bound a threshold (8 such lists hold 4 k anchors
 *  for every k <= 64). */
constexpr int64_t kListAnchorMin = 32;

struct table_plan {
  anchor_plan ap{};
  bool anchors = true;
  probe_plan pp;
  int list_anchors = 0;  // > 0: the groups are the list anchors of this many nearest lists
  int64_t n_groups = 0;
};

/**
 * Stride of the list anchors: half the anchor stride. The nearest lists hold the rows near the
 * query, where twice the density of the anchors of every row halves the survivors (config 2: 163
 * -> 82 per query; the screen 1.7% faster at one clock, the re-rank 0.105 -> 0.063 ms, the
 * anchors 0.143 -> 0.190 ms). A quarter (41 survivors) cost more in the anchors (0.275 ms) than
 * it saved.
 */
auto list_anchor_stride(index_state const& st) -> int64_t { return std::max(1, st.anchor_stride / 2); }

/**
 * The list-anchor threshold's center terms: cterm, with +inf for every list of fewer than
 * kListAnchorMin anchors (rows list_offsets[j] + i list_anchor_stride), so that the nearest lists
 * of a query are lists of at least that many anchors. Set where the lists are set (build, load).
 */
void set_anchor_centers(cuvs::resources const& res, index_state& st)
{
  hipStream_t stream = static_cast<hipStream_t>(res.stream());
  const int L        = st.n_lists;
  const int Lp       = certex_amd::pad_centers(L);
  const int64_t s    = list_anchor_stride(st);
  std::vector<float> ct(static_cast<size_t>(Lp));
  CERTEX_HIP_TRY(hipMemcpyAsync(ct.data(), st.cterm.p, size_t(Lp) * 4, hipMemcpyDeviceToHost, stream));
  CERTEX_HIP_TRY(hipStreamSynchronize(stream));
  int big = 0;
  for (int j = 0; j < L; ++j) {
    const int64_t na = (st.list_offsets[size_t(j) + 1] - st.list_offsets[size_t(j)] + s - 1) / s;
    if (na < kListAnchorMin) {
      ct[size_t(j)] = INFINITY;
    } else {
      ++big;
    }
  }
  st.cterm_anchor.resize_discard(size_t(Lp) * 4);
  CERTEX_HIP_TRY(hipMemcpyAsync(st.cterm_anchor.p, ct.data(), size_t(Lp) * 4, hipMemcpyHostToDevice, stream));
  CERTEX_HIP_TRY(hipStreamSynchronize(stream));
  st.n_anchor_lists = big;
}

/**
 * Lists whose anchors bound the threshold of a search that probes no list: the p = min(lists, 8)
 * nearest lists of each query, or 0 where the anchors of every row serve instead. Any k distinct
 * rows bound the k-th best screen value from below, so the threshold is exact either way; the
 * lists only pick rows near the query, and the anchors of its 8 nearest lists (about 1,200 at
 * 10M rows in 4,096 lists) hold the anchors that set the threshold of the anchors of every row.
 * Integer rows of at most 256 bytes, no filter (the anchors would have to pass it), k <= 64, at
 * least half of the rows listed, and 8 lists of at least kListAnchorMin anchors to choose from
 * (the nearest lists are chosen among those: every query meets 8 kListAnchorMin >= 4 k anchors).
 */
int list_anchor_lists(index_state const& st, int k, search_params const& params,
                      certex_amd::filter_args const& fa)
{
  const int p = certex_amd::kMaxProbe;
  if (!is_int(st.type) || st.row_bytes > 256 || st.n_anchor_lists < p || params.probe_lists > 0 ||
      fa.kind != 0 || k > 64 || 2 * st.n_listed < st.size) {
    return 0;
  }
  return p;
}

auto plan_table(cuvs::resources const& res, index_state const& st, const void* qrows, int64_t B,
                int64_t nq_pad, int k, search_params const& params,
                certex_amd::filter_args const& fa, route_plan const* route) -> table_plan
{
  table_plan tp;
  if (route != nullptr) {
    tp.ap       = route->ap;
    tp.n_groups = tp.ap.n_groups;
    return tp;
  }
  tp.list_anchors = list_anchor_lists(st, k, params, fa);
  if (tp.list_anchors > 0) {
    tp.anchors  = false;
    tp.n_groups = 64 * int64_t(tp.list_anchors);
    return tp;
  }
  bool probe = st.n_lists > 0 && params.probe_lists > 0 && (fa.kind == 0 || fa.kind == 1) &&
               plan_probe(res, st, qrows, B, k, params.probe_lists, tp.pp) && tp.pp.enough;
  if (probe) {  // the anchors of the ids added after the lists (the first id >= n_listed on)
    const int64_t s     = std::max(1, st.anchor_stride);
    const int64_t first = (st.n_listed + s - 1) / s;
    tp.anchors          = first < (st.size + s - 1) / s;
    if (tp.anchors) { tp.ap = plan_anchors(st, first, nq_pad, k); }
    const int64_t acols = tp.anchors ? tp.ap.n_groups : 0;
    probe = nq_pad * (acols + tp.pp.cols) * 4 <= kTableBytes;
  }
  if (!probe) {  // anchors over every row
    tp.pp      = probe_plan{};
    tp.anchors = true;
    tp.ap      = plan_anchors(st, 0, nq_pad, k);
  }
  tp.n_groups = (tp.anchors ? tp.ap.n_groups : 0) + tp.pp.cols;
  return tp;
}

/** Fills the group table (lowest values) where the probe leaves columns unwritten, then the passes. */
template <typename F>
void table_pass(cuvs::resources const& res, index_state const& st, certex_amd::screen_args aa,
                table_plan const& tp, route_plan const* route, F&& launch)
{
  auto& rs           = res.state();
  hipStream_t stream = rs.stream;
  if (tp.list_anchors > 0) {
    // the nearest lists of every query, then the group table of their anchors (every column)
    const int p  = tp.list_anchors;
    const int Lp = certex_amd::pad_centers(st.n_lists);
    auto* lists  = static_cast<int32_t*>(rs.get(cuvs::detail::ws_probe, size_t(aa.nq) * p * 4));
    void* temp   = rs.get(cuvs::detail::ws_probe_dist,
                          certex_amd::list_anchor_temp_bytes(aa.nq, st.n_lists));
    certex_amd::nearest_lists_i8(aa.qcodes, st.row_bytes, aa.nq, st.centers_q.p,
                                 st.cterm_anchor.as<float>(), Lp, st.n_lists, lists, temp, stream);
    certex_amd::list_anchor_groups(st.codes.as<int8_t>(), st.rowc.as<int32_t>(), st.row_bytes,
                                   aa.qcodes, aa.nq, lists, st.list_offsets_dev.as<int64_t>(),
                                   st.n_lists, list_anchor_stride(st), temp,
                                   static_cast<int32_t*>(aa.gmax), stream);
    return;
  }
  if (tp.pp.n_pairs > 0) {
    if (is_int(st.type)) {
      certex_amd::fill_i32(static_cast<int32_t*>(aa.gmax), aa.nq_pad * tp.n_groups, INT32_MIN,
                           stream);
    } else {
      certex_amd::fill_u32(static_cast<uint32_t*>(aa.gmax), aa.nq_pad * tp.n_groups, 0xff800000u,
                           stream);
    }
  }
  if (tp.anchors) { anchor_pass(st, aa, tp.ap, tp.n_groups, route, launch, stream); }
  if (tp.pp.n_pairs > 0) {
    probe_pass(res, st, aa, tp.pp, tp.anchors ? tp.ap.n_groups : 0, tp.n_groups, launch);
  }
}

/** Testing only: the batch's shape, its table plan and the index's screening rows. */
void capture_common(index_state const& st, table_plan const& tp, int64_t B, int64_t nq_pad, int k,
                    bool all_rows, int64_t cap, route_plan const* route, hipStream_t stream)
{
  expects(route == nullptr && tp.pp.n_pairs == 0,
          "certex: a capture covers unrouted searches without a list probe");
  expects(B <= 65535, "certex: a capture covers batches of at most 65,535 queries");
  t_capture.value("B", int64_t(B));
  t_capture.value("nq_pad", int64_t(nq_pad));
  t_capture.value("k", int64_t(k));
  t_capture.value("all_rows", int64_t(all_rows));
  t_capture.value("cap", int64_t(all_rows ? 0 : cap));
  t_capture.value("n_groups", int64_t(tp.n_groups));
  t_capture.value("group_steps", int64_t(tp.ap.group_steps));
  t_capture.value("fine", int64_t(tp.ap.fine));
  t_capture.value("anchor_stride", int64_t(tp.ap.stride));
  t_capture.value("list_anchors", int64_t(tp.list_anchors));
  t_capture.value("list_anchor_stride", list_anchor_stride(st));
  t_capture.value("row_bytes", int64_t(st.row_bytes));
  t_capture.value("size", int64_t(st.size));
  t_capture.put("codes", st.codes.p, size_t(st.size) * st.row_bytes, stream);
  t_capture.put("rowc", st.rowc.p, size_t(st.size) * 4, stream);
}

/** One batch of queries of an integer index (the caller holds the shared lock). */
void search_batch_int(cuvs::resources const& res, index_state const& st, const void* queries,
                      int64_t B, int k, int64_t q0, int64_t* neighbors, float* distances,
                      certex_amd::filter_args fa, search_params const& params,
                      route_plan const* route)
{
  auto& rs             = res.state();
  hipStream_t stream   = rs.stream;
  const int64_t size   = st.size;
  const int64_t nq_pad = certex_amd::pad_queries(B);
  const uint8_t flip   = st.type == vtype::u8 ? 0x80 : 0;
  fa.q0                = q0;
  fa.row_ids           = st.row_ids.as<int32_t>();
  fa.n_listed          = st.n_listed;

  auto* qcodes =
    static_cast<int8_t*>(rs.get(cuvs::detail::ws_qcodes, size_t(nq_pad) * st.row_bytes));
  // rows of more than 256 bytes: the tiled screen reads the queries in the paired layout (a second
  // copy, written by the same kernel)
  const bool wide = uses_tile_screen(st);
  auto* qpaired   = wide ? static_cast<int8_t*>(rs.get(cuvs::detail::ws_qpaired,
                                                       size_t(nq_pad) * st.row_bytes))
                         : nullptr;
  const int32_t* qmap = route != nullptr ? route->rows : nullptr;
  certex_amd::encode_queries_i8(static_cast<const uint8_t*>(queries), B, nq_pad, st.dim,
                                st.row_bytes, flip, qcodes, stream, qpaired, qmap);

  // group table: the best screen value of every group of anchors (every anchor_stride-th stored
  // row) and of the probed lists' rows; the k-th best group is the threshold of the query
  const table_plan tp = plan_table(res, st, qcodes, B, nq_pad, k, params, fa, route);
  certex_amd::screen_args sa{};
  sa.codes     = st.codes.as<int8_t>();
  sa.rowc      = st.rowc.p;
  sa.row_bytes = st.row_bytes;
  sa.qcodes    = qcodes;
  sa.qpaired   = qpaired;
  sa.nq        = B;
  sa.nq_pad    = nq_pad;
  sa.filter    = fa;

  auto* theta   = static_cast<int32_t*>(rs.get(cuvs::detail::ws_theta, size_t(nq_pad) * 4));
  bool all_rows = tp.n_groups < k;
  if (!all_rows) {
    auto* gmax = static_cast<int32_t*>(
      rs.get(cuvs::detail::ws_gmax, size_t(nq_pad) * size_t(tp.n_groups) * 4));
    certex_amd::screen_args aa = sa;
    aa.gmax                    = gmax;
    timed(0, stream, [&] { table_pass(res, st, aa, tp, route, certex_amd::anchors_i8); });
    timed(1, stream,
          [&] { certex_amd::threshold_i8(gmax, tp.n_groups, B, nq_pad, k, theta, stream); });
  }

  uint32_t *count = nullptr, *rows = nullptr;
  int64_t cap = 0, worst = -1;
  if (!all_rows) {
    sa.theta = theta;
    all_rows = !screen_into_buckets(res, B, nq_pad, size, sa,
                                    screen_pass(st, route, certex_amd::screen_i8), count, rows,
                                    cap, nullptr, &worst);
  }
  count_stats(res, st, B, all_rows, count, cap);
  if (t_capture.on) {
    capture_common(st, tp, B, nq_pad, k, all_rows, cap, route, stream);
    t_capture.put("qrows", qcodes, size_t(B) * st.row_bytes, stream);
    t_capture.put("theta", theta, size_t(B) * 4, stream);
    if (tp.n_groups >= k) {
      t_capture.put("gmax", rs.get(cuvs::detail::ws_gmax, 1), size_t(B) * tp.n_groups * 4, stream);
    }
    if (tp.list_anchors > 0) {
      t_capture.put("lists", rs.get(cuvs::detail::ws_probe, 1), size_t(B) * tp.list_anchors * 4,
                    stream);
      t_capture.put("list_offsets", st.list_offsets_dev.p, size_t(st.n_lists + 1) * 8, stream);
    }
    if (!all_rows) {
      t_capture.put("count", count, size_t(B) * 4, stream);
      t_capture.put("rows", rows, size_t(B) * cap * 4, stream);
    }
    CERTEX_HIP_TRY(hipStreamSynchronize(stream));
    t_capture.on = false;
  }

  certex_amd::verify_args va{};
  va.cand_count = count;
  va.cand_rows  = rows;
  va.cap        = cap;
  va.all_rows   = all_rows;
  va.max_cand   = all_rows ? -1 : worst;
  va.n_rows     = size;
  va.codes      = st.codes.as<int8_t>();
  va.rowc       = st.rowc.as<int32_t>();
  va.row_bytes  = st.row_bytes;
  va.dim        = st.dim;
  va.flip       = flip;
  va.qcodes     = qcodes;
  va.metric     = st.metric;
  va.filter     = fa;
  va.nq         = B;
  va.k          = k;
  if (route != nullptr) {
    va.part_ids   = st.label_part.ids.as<int32_t>();
    va.n_part     = st.label_part.n;
    va.part_codes  = st.label_part.codes.as<int8_t>();
    va.part_paired = st.label_part.paired;
  }
  va.distances = distances;
  va.neighbors = neighbors;
  va.out_rows  = qmap;
  timed(3, stream, [&] { certex_amd::verify_topk_i8(va, stream); });
}

/** One batch of queries of a float index (the caller holds the shared lock). */
void search_batch_float(cuvs::resources const& res, index_state const& st, const void* queries,
                        int64_t B, int k, int64_t q0, int64_t* neighbors, float* distances,
                        certex_amd::filter_args fa, search_params const& params,
                        route_plan const* route)
{
  auto& rs             = res.state();
  hipStream_t stream   = rs.stream;
  const int64_t size   = st.size;
  const int64_t nq_pad = certex_amd::pad_queries(B);
  const auto t         = elem_of(st.type);
  const bool wide      = st.halves > 128;  // the K-loop screen
  fa.q0                = q0;
  fa.row_ids           = st.row_ids.as<int32_t>();
  fa.n_listed          = st.n_listed;

  auto* qrows =
    static_cast<uint16_t*>(rs.get(cuvs::detail::ws_qcodes, size_t(nq_pad) * st.row_bytes));
  auto* qscal = static_cast<double*>(rs.get(cuvs::detail::ws_qscal, size_t(nq_pad) * 3 * 8));
  // the tiled screen reads the queries in the paired layout (a second copy, written by the same
  // kernel; nq_pad is even)
  auto* qpaired = wide ? static_cast<uint16_t*>(rs.get(cuvs::detail::ws_qpaired,
                                                       size_t(nq_pad) * st.row_bytes))
                       : nullptr;
  const int32_t* qmap = route != nullptr ? route->rows : nullptr;
  certex_amd::encode_queries_f16(queries, t, B, nq_pad, st.dim, st.halves, st.normalize,
                                 st.center.as<double>(), 1.0 / st.alpha, qrows, qscal, stream,
                                 qpaired, qmap);

  const table_plan tp = plan_table(res, st, qrows, B, nq_pad, k, params, fa, route);
  certex_amd::screen_args sa{};
  sa.codes     = st.codes.as<int8_t>();
  sa.rowc      = st.rowc.p;
  sa.row_bytes = st.row_bytes;
  sa.qcodes    = reinterpret_cast<const int8_t*>(qrows);
  sa.qpaired   = reinterpret_cast<const int8_t*>(qpaired);
  sa.nq        = B;
  sa.nq_pad    = nq_pad;
  sa.filter    = fa;

  auto* theta   = static_cast<float*>(rs.get(cuvs::detail::ws_theta, size_t(nq_pad) * 4));
  bool all_rows = tp.n_groups < k;
  certex_amd::threshold_f_args ta{};
  std::unique_ptr<capture_buffer<double>> ub_q;  // testing: U per query
  if (!all_rows) {
    auto* gmax = static_cast<float*>(
      rs.get(cuvs::detail::ws_gmax, size_t(nq_pad) * size_t(tp.n_groups) * 4));
    certex_amd::screen_args aa = sa;
    aa.gmax                    = gmax;
    timed(0, stream, [&] {
      table_pass(res, st, aa, tp, route,
                 wide ? certex_amd::anchors_f16_wide : certex_amd::anchors_f16);
    });
    // theta certified from the k-th best group maximum (no exact anchor scores)
    ta.gmax     = gmax;
    ta.n_groups = tp.n_groups;
    ta.nq       = B;
    ta.nq_pad   = nq_pad;
    ta.k        = k;
    ta.metric   = st.metric;
    ta.qscal    = qscal;
    ta.maxima   = st.maxima.as<double>();
    ta.alpha2   = st.alpha * st.alpha;
    ta.gamma    = st.gamma;
    ta.theta    = theta;
    if (t_capture.on) {
      ub_q = std::make_unique<capture_buffer<double>>(size_t(nq_pad));
      ta.ub = ub_q->p;
    }
    timed(1, stream, [&] { certex_amd::threshold_f16(ta, stream); });
    ta.ub = nullptr;
  }

  uint32_t *count = nullptr, *rows = nullptr;
  float* vals = nullptr;
  int64_t cap = 0;
  unsigned long long* scored = nullptr;
  if (t_stats_on) {
    auto* small = static_cast<uint32_t*>(rs.get(cuvs::detail::ws_small, 64));
    scored      = reinterpret_cast<unsigned long long*>(small + 8);
  }
  certex_amd::verify_f_args va{};
  va.n_rows     = size;
  va.vectors    = st.vectors.p;
  va.qscal      = qscal;
  va.maxima     = st.maxima.as<double>();
  va.alpha2     = st.alpha * st.alpha;
  va.gamma      = st.gamma;
  va.rowc       = st.rowc.as<float>();
  va.queries    = queries;
  va.query_rows = qmap;
  va.t          = t;
  va.dim        = st.dim;
  va.metric     = st.metric;
  va.filter     = fa;
  va.nq         = B;
  va.k          = k;
  va.distances  = distances;
  va.neighbors  = neighbors;
  va.out_rows   = qmap;
  va.scored     = scored;
  if (route != nullptr) {
    va.part_ids = st.label_part.ids.as<int32_t>();
    va.n_part   = st.label_part.n;
  }
  // the exact re-rank over the buckets as they are, or over every row (all_rows)
  auto verify = [&](bool every_row) {
    va.cand_count = count;
    va.cand_rows  = rows;
    va.cand_vals  = vals;
    va.cap        = cap;
    va.all_rows   = every_row;
    if (scored != nullptr) { certex_amd::fill_u32(reinterpret_cast<uint32_t*>(scored), 2, 0, stream); }
    timed(3, stream, [&] { certex_amd::verify_topk_f(va, stream); });
  };
  bool verified = false;
  // a capture reads the buckets before the verification (which compacts them in place)
  const bool capture = t_capture.on;
  if (!all_rows) {
    sa.theta = theta;
    all_rows = !screen_into_buckets(
      res, B, nq_pad, size, sa,
      screen_pass(st, route, wide ? certex_amd::screen_f16_tile : certex_amd::screen_f16), count,
      rows, cap, &vals, nullptr, [&] {
        if (!capture) { verify(false); }
      });
    verified = !all_rows && !capture;
  }
  if (capture) {
    capture_common(st, tp, B, nq_pad, k, all_rows, cap, route, stream);
    t_capture.put("qrows", qrows, size_t(B) * st.row_bytes, stream);
    t_capture.put("qscal", qscal, size_t(B) * 3 * 8, stream);
    t_capture.put("theta", theta, size_t(B) * 4, stream);
    t_capture.put("maxima", st.maxima.p, 2 * sizeof(double), stream);
    t_capture.value("alpha2", st.alpha * st.alpha);
    t_capture.value("gamma", st.gamma);
    t_capture.value("halves", int64_t(st.halves));
    if (ub_q) {
      t_capture.put("gmax", ta.gmax, size_t(B) * tp.n_groups * 4, stream);
      t_capture.put("ub_q", ub_q->p, size_t(B) * 8, stream);
    }
    if (!all_rows) {
      t_capture.put("count", count, size_t(B) * 4, stream);
      t_capture.put("rows", rows, size_t(B) * cap * 4, stream);
      t_capture.put("vals", vals, size_t(B) * cap * 4, stream);
      certex_amd::threshold_f_args ca{};
      ca.nq = B, ca.nq_pad = nq_pad, ca.k = k, ca.metric = st.metric, ca.qscal = qscal;
      ca.maxima = st.maxima.as<double>(), ca.alpha2 = st.alpha * st.alpha, ca.gamma = st.gamma;
      capture_buffer<double> lb(size_t(B) * cap), ub(size_t(B) * cap);
      certex_amd::certificate_bounds(ca, count, vals, cap, lb.p, ub.p, stream);
      t_capture.put("lb", lb.p, size_t(B) * cap * 8, stream);
      t_capture.put("ub", ub.p, size_t(B) * cap * 8, stream);
      CERTEX_HIP_TRY(hipStreamSynchronize(stream));
    }
    CERTEX_HIP_TRY(hipStreamSynchronize(stream));
    t_capture.on = false;
    if (!all_rows) {
      verify(false);
      verified = true;
    }
  }
  if (!verified) { verify(true); }
  count_stats(res, st, B, all_rows, count, cap, true);
  if (scored != nullptr) {
    CERTEX_HIP_TRY(hipMemcpyAsync(rs.host_small, scored, 8, hipMemcpyDeviceToHost, stream));
    CERTEX_HIP_TRY(hipStreamSynchronize(stream));
    t_stats.verified += int64_t(*static_cast<unsigned long long*>(rs.host_small));
  }
}

using batch_fn = void (*)(cuvs::resources const&, index_state const&, const void*, int64_t, int,
                          int64_t, int64_t*, float*, certex_amd::filter_args,
                          search_params const&, route_plan const*);

/**
 * Label search of one batch over the label partition (reference search_by_labels,
 * certex.cu:1613-1735): the queries in label order (stable), one routed group per label that has
 * partition rows, the tail through the label filter, and the results back in query order.
 *
 * Query labels in host memory are sorted and grouped on the host (exact workgroup counts, no wait
 * for the GPU). Labels in device memory never come back: a stable radix sort of the batch's labels
 * and route_tables build the groups on the device, one per label of the partition, and each pass
 * is launched with an upper bound of its workgroups (route_tiles_bound), the ones past the last
 * group exiting at once.
 */
void routed_batch(cuvs::resources const& res, index_state const& st, batch_fn batch,
                  const char* queries, int64_t B, int k, const int32_t* qlabels,
                  const int32_t* hlabels, int64_t* neighbors, float* distances,
                  certex_amd::filter_args fa, search_params const& params)
{
  auto& rs             = res.state();
  hipStream_t stream   = rs.stream;
  const bool on_device = hlabels == nullptr;
  const auto& off      = st.label_part.offsets;
  const int64_t n_lab  = int64_t(off.size()) - 1;
  std::vector<int32_t> order, sorted;
  std::vector<certex_amd::screen_group> ga, gs;
  bool in_order = false;  // host labels in non-decreasing order: no gather or scatter
  if (!on_device) {
    // queries in label order, stable: a counting sort when the batch's labels span a small range
    // (one pass, no comparisons), else a comparison sort
    const int32_t* lab = hlabels;
    order.resize(size_t(B));
    sorted.resize(size_t(B));
    const auto [lo_it, hi_it] = std::minmax_element(lab, lab + B);
    const int64_t lo = B > 0 ? *lo_it : 0, span = B > 0 ? int64_t(*hi_it) - lo + 1 : 0;
    if (span <= 4 * B + 1024) {
      std::vector<int64_t> start(static_cast<size_t>(span) + 1, 0);
      for (int64_t i = 0; i < B; ++i) { ++start[size_t(lab[i] - lo) + 1]; }
      for (int64_t v = 0; v < span; ++v) { start[size_t(v) + 1] += start[size_t(v)]; }
      for (int64_t i = 0; i < B; ++i) { order[size_t(start[size_t(lab[i] - lo)]++)] = int32_t(i); }
    } else {
      for (int64_t i = 0; i < B; ++i) { order[size_t(i)] = int32_t(i); }
      std::stable_sort(order.begin(), order.end(), [&](int32_t a, int32_t b) { return lab[a] < lab[b]; });
    }
    in_order = std::is_sorted(lab, lab + B);
    for (int64_t i = 0; i < B;) {
      const int32_t l = lab[order[size_t(i)]];
      int64_t j       = i;
      while (j < B && lab[order[size_t(j)]] == l) { sorted[size_t(j++)] = l; }
      if (l >= 0 && int64_t(l) < n_lab && off[size_t(l) + 1] > off[size_t(l)]) {
        certex_amd::screen_group g{i, j - i, off[size_t(l)], off[size_t(l) + 1] - off[size_t(l)], 0};
        ga.push_back(g);
        gs.push_back(g);
      }
      i = j;
    }
  } else {
    // the groups the device will build, with queries spread over the labels as their rows are:
    // the plan (stride, group columns, chunks) then does not depend on the labels of the batch
    for (int64_t l = 0; l < n_lab; ++l) {
      const int64_t nx = off[size_t(l) + 1] - off[size_t(l)];
      if (nx == 0) { continue; }
      const int64_t nq = std::max<int64_t>(1, (B * nx + st.label_part.n - 1) / std::max<int64_t>(1, st.label_part.n));
      gs.push_back({0, nq, off[size_t(l)], nx, 0});
    }
    ga = gs;
  }
  int64_t max_nx = 0;
  for (auto const& e : ga) { max_nx = std::max(max_nx, e.nx); }

  const int64_t nq_pad = certex_amd::pad_queries(B);
  const bool f16       = !is_int(st.type);
  const bool wide      = st.row_bytes > 256;
  const int qb         = certex_amd::screen_query_block(f16, st.row_bytes, nq_pad);
  // the largest label's anchors should form at least 4 k fine groups: below the index's stride,
  // a denser one (a query whose label still has fewer than k groups keeps all of its rows)
  const int stride = int(std::max<int64_t>(
    1, std::min<int64_t>(std::max(1, st.anchor_stride),
                         max_nx / (4 * certex_amd::kFineGroup * int64_t(k)))));
  // anchor groups: per label as plan_anchors sizes them for the largest label; the tail's
  // columns follow the partition's
  // a label's anchors: one row every stride, or over a paired partition the row pairs every
  // 2 stride (the anchor pass then reads whole lines)
  const bool apairs = st.label_part.paired;
  auto anchors_of   = [&](certex_amd::screen_group const& e) {
    return apairs ? certex_amd::paired_anchor_count(e.x0, e.nx, stride) : (e.nx + stride - 1) / stride;
  };
  int64_t max_anchors = 0;
  for (auto const& e : ga) { max_anchors = std::max(max_anchors, anchors_of(e)); }
  route_plan route;
  route.ap.stride   = stride;
  route.ap.n_anchor = 0;
  size_groups(route.ap, max_anchors, (st.size - st.label_part.n + stride - 1) / stride, nq_pad, k,
              &route.part_groups);
  if (!on_device && route.ap.fine) {
    int64_t routed = 0;
    bool equal     = true;
    for (auto const& e : ga) {
      routed += e.nq;
      equal = equal && anchors_of(e) == max_anchors;
    }
    route.covers_table = routed == B && equal;
  }
  const int64_t waves = waves_of(st);
  // the screen's groups: the tiled screen's query blocks and 256-row chunks for wide rows;
  // so too the anchor pass over anchor pairs with fine groups (its tiles start at an even query)
  const bool tiled    = uses_tile_screen(st);
  route.anchor_tiled  = tiled && apairs && route.ap.fine;
  const int qba       = route.anchor_tiled ? certex_amd::tile_block_queries() : qb;
  const int64_t alead = route.anchor_tiled ? 1 : 0;  // odd first queries take one slot more
  route.anchor_chunk  = route.anchor_tiled
                          ? certex_amd::tile_chunk_steps()
                          : pick_chunk(waves * route.ap.group_steps,
                                       anchor_chunk_steps(wide, route.ap.group_steps), [&](int64_t c) {
                                         int64_t t = 0;
                                         for (auto const& e : ga) {
                                           t += certex_amd::screen_group_tiles(e.nq, anchors_of(e), qb, int(c));
                                         }
                                         return t;
                                       });
  const int qbs    = tiled ? certex_amd::tile_block_queries() : qb;
  route.screen_chunk =
    tiled ? certex_amd::tile_chunk_steps() : pick_chunk(waves, kRoutedChunk, [&](int64_t c) {
      int64_t t = 0;
      for (auto const& e : gs) { t += certex_amd::screen_group_tiles(e.nq, e.nx, qb, int(c)); }
      return t;
    });

  const size_t lab_bytes = (size_t(B) * 4 + 15) / 16 * 16;
  int32_t *d_order = nullptr, *d_sorted = nullptr;
  if (!on_device) {
    for (auto& e : ga) {
      const int64_t nq   = e.nq + (e.q0 & alead);
      e.tile0            = certex_amd::screen_group_tile0(route.anchor_tiles, nq, qba);
      route.anchor_tiles =
        e.tile0 + certex_amd::screen_group_tiles(nq, anchors_of(e), qba, route.anchor_chunk);
    }
    // the tiled screen aligns a group's query blocks (and, over paired rows, its tiles) to pairs
    for (auto& e : gs) {
      if (tiled) {
        e.tile0            = certex_amd::screen_group_tile0(route.screen_tiles, e.nq + (e.q0 & 1), qbs);
        route.screen_tiles = e.tile0 + certex_amd::paired_group_tiles(e, st.label_part.paired, qbs,
                                                                      route.screen_chunk);
      } else {
        e.tile0            = certex_amd::screen_group_tile0(route.screen_tiles, e.nq, qbs);
        route.screen_tiles = e.tile0 + certex_amd::screen_group_tiles(e.nq, e.nx, qbs, route.screen_chunk);
      }
    }
    route.n_route = int(gs.size());
    // device copies: order, sorted labels, the two group tables, packed as on the device in
    // pinned staging, then one copy
    const size_t tab_bytes = std::max<size_t>(1, gs.size()) * sizeof(certex_amd::screen_group);
    char* dev = static_cast<char*>(rs.get(cuvs::detail::ws_route, 2 * lab_bytes + 2 * tab_bytes));
    d_order  = reinterpret_cast<int32_t*>(dev);
    d_sorted = reinterpret_cast<int32_t*>(dev + lab_bytes);
    auto* d_ga = reinterpret_cast<certex_amd::screen_group*>(dev + 2 * lab_bytes);
    auto* d_gs = reinterpret_cast<certex_amd::screen_group*>(dev + 2 * lab_bytes + tab_bytes);
    const size_t all_bytes = 2 * lab_bytes + 2 * tab_bytes;
    char* hs               = static_cast<char*>(rs.stage(all_bytes));
    std::memcpy(hs, order.data(), size_t(B) * 4);
    std::memcpy(hs + lab_bytes, sorted.data(), size_t(B) * 4);
    if (!gs.empty()) {
      std::memcpy(hs + 2 * lab_bytes, ga.data(), ga.size() * sizeof(ga[0]));
      std::memcpy(hs + 2 * lab_bytes + tab_bytes, gs.data(), gs.size() * sizeof(gs[0]));
    }
    rs.copy_staged(dev, all_bytes);
    route.anchor_groups = d_ga;
    route.screen_groups = d_gs;
  } else {
    // workgroups of a pass, at most: a label with chunk count c and n_qb query blocks takes
    // 8 n_qb ceil(c / 8) (rounded up to 8), and n_qb <= 1 + (nq + 1) / qb summed over labels
    // stays below labels + (B + labels) / qb
    auto bound = [&](auto&& scans, int q_blk, int chunk) {
      int64_t sum = 0, cmax = 0, n = 0;
      for (auto const& e : gs) {
        const int64_t c = 8 * ((certex_amd::screen_group_tiles(1, scans(e), q_blk, chunk) + 7) / 8);
        sum += c;
        cmax = std::max(cmax, c);
        ++n;
      }
      return sum + cmax * ((B + 2 * n + q_blk - 1) / q_blk);
    };
    route.anchor_tiles = bound([&](auto const& e) { return anchors_of(e); }, qba, route.anchor_chunk);
    route.screen_tiles = bound([&](auto const& e) { return e.nx + 1; }, qbs, route.screen_chunk);
    route.n_route      = int(n_lab);
    const size_t tab_bytes  = size_t(std::max<int64_t>(1, n_lab)) * sizeof(certex_amd::screen_group);
    const size_t sort_bytes = (certex_amd::sort_by_label_temp_bytes(B) + 255) / 256 * 256;
    char* dev = static_cast<char*>(
      rs.get(cuvs::detail::ws_route, 3 * lab_bytes + 2 * tab_bytes + sort_bytes));
    d_order      = reinterpret_cast<int32_t*>(dev);
    d_sorted     = reinterpret_cast<int32_t*>(dev + lab_bytes);
    auto* d_iota = reinterpret_cast<int32_t*>(dev + 2 * lab_bytes);
    auto* d_ga   = reinterpret_cast<certex_amd::screen_group*>(dev + 3 * lab_bytes);
    auto* d_gs   = reinterpret_cast<certex_amd::screen_group*>(dev + 3 * lab_bytes + tab_bytes);
    void* temp   = dev + 3 * lab_bytes + 2 * tab_bytes;
    const bool small = certex_amd::route_small_fits(B, n_lab);
    if (!small) {
      CERTEX_HIP_TRY(certex_amd::sort_by_label(qlabels, B, d_iota, d_sorted, d_order, temp,
                                               sort_bytes, stream));
    }
    certex_amd::route_table_args ra{};
    ra.sorted        = d_sorted;
    ra.B             = B;
    ra.offsets       = st.label_part.offsets_dev.as<int64_t>();
    ra.n_labels      = n_lab;
    ra.anchor_stride = stride;
    ra.anchor_pairs  = apairs;
    ra.anchor_qb     = qba;
    ra.anchor_chunk  = route.anchor_chunk;
    ra.anchor_lead   = int(alead);
    ra.screen_tiled  = tiled;
    ra.rows_paired   = st.label_part.paired;
    ra.screen_qb     = qbs;
    ra.screen_chunk  = route.screen_chunk;
    ra.anchor_groups = d_ga;
    ra.screen_groups = d_gs;
    if (small) {  // few labels: the sort and the tables in one launch
      certex_amd::route_small(ra, qlabels, d_order, d_sorted, stream);
    } else {
      certex_amd::route_tables(ra, stream);
    }
    route.anchor_groups = d_ga;
    route.screen_groups = d_gs;
  }

  fa.query_labels = d_sorted;  // the label filter of the tail, in the sorted order
  // the batch in label order reads the caller's queries through d_order and writes the results
  // to their rows (host labels already in label order, a KeyCache's heads: the batch itself)
  route.rows = in_order ? nullptr : d_order;
  batch(res, st, queries, B, k, 0, neighbors, distances, fa, params, &route);
  // no wait here: the next use of the staging waits for this batch's copy of the tables
}

template <typename T>
void search_impl(cuvs::resources const& res, search_params const& params, index<T> const& idx,
                 matrix_view<const T> queries, int64_t* neighbors, float* distances, int64_t k,
                 certex_amd::filter_args fa, bool no_alloc = false,
                 const int32_t* host_labels = nullptr)
{
  index_state const& st = idx.state();
  expects(queries.on_device, "certex: the queries must be in device memory");
  expects(queries.cols == st.dim, "dimension mismatch");
  expects(k >= 1 && k <= 2048, "certex returns at most 2048 neighbors per query");
  expects(st.size >= k, "the index holds fewer than k vectors");
  const int64_t nq = queries.rows;
  if (nq == 0) { return; }
  if (t_stats_on) { res.sync(); }
  const int64_t bs   = std::max(1, params.batch_size);
  const size_t qrow  = size_t(st.dim) * sizeof(T);
  const batch_fn batch = is_int(st.type) ? search_batch_int : search_batch_float;
  // a search without allocation screens label queries through the label filter: routing a
  // batch over the label partition stages its tables in pinned host memory
  const bool route = fa.kind == 3 && st.label_part.n > 0 && !no_alloc;
  if (host_labels != nullptr && !route) {
    // the label filter reads the query labels on the GPU: one copy through pinned staging
    auto& rs  = res.state();
    auto* dev = static_cast<int32_t*>(rs.get(cuvs::detail::ws_qlabels, size_t(nq) * 4));
    std::memcpy(rs.stage(size_t(nq) * 4), host_labels, size_t(nq) * 4);
    rs.copy_staged(dev, size_t(nq) * 4);
    fa.query_labels = dev;
  }
  std::function<void(int64_t, int64_t)> run = [&](int64_t b0, int64_t B) {
    if (no_alloc) { res.state().arena_reset(); }
    try {
      const char* q = reinterpret_cast<const char*>(queries.data) + size_t(b0) * qrow;
      if (route) {
        routed_batch(res, st, batch, q, B, int(k),
                     host_labels != nullptr ? nullptr : fa.query_labels + b0,
                     host_labels != nullptr ? host_labels + b0 : nullptr, neighbors + b0 * k,
                     distances + b0 * k, fa, params);
      } else {
        batch(res, st, q, B, int(k), b0, neighbors + b0 * k, distances + b0 * k, fa, params,
              nullptr);
      }
    } catch (batch_too_large const&) {
      if (B < 2) { throw; }
      run(b0, B / 2);
      run(b0 + B / 2, B - B / 2);
    } catch (std::bad_alloc const&) {
      if (B < 2 || no_alloc) { throw; }
      res.sync();
      run(b0, B / 2);
      run(b0 + B / 2, B - B / 2);
    }
  };
  for (int64_t b0 = 0; b0 < nq; b0 += bs) {
    std::shared_lock batch_view(st.rw);  // the rows of this batch stay fixed during updates
    st.await_updates(res.state().stream);
    run(b0, std::min(bs, nq - b0));
  }
}

/**
 * Device scratch of the searches that allocate nothing (search_without_allocation): one array per
 * GPU, allocated when the library's code object is loaded on that GPU and held until the process
 * ends. Host code must not pass `scratch` itself (on the host it is a stand-in symbol, not a device
 * address): scratch_of() returns the device address of each GPU's copy.
 */
constexpr size_t kNoAllocScratchBytes = size_t(128) << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
char* g_scratch[kMaxDevices] = {};
/** Per GPU: held by the search that uses the scratch array, from its first launch to its last. */
std::mutex g_scratch_use[kMaxDevices];
/** Per GPU: recorded after the last launch of the latest search on the scratch array. */
hipEvent_t g_scratch_done[kMaxDevices] = {};

/** The device address of `device`'s scratch array, looked up once per device with it current
 * (the event that orders its users is created at the same time). */
auto scratch_of(int device) -> char*
{
  expects(device >= 0 && device < kMaxDevices, "certex: device ordinal out of range");
  std::lock_guard lk(g_scratch_mutex);
  if (g_scratch[device] == nullptr) {
    int current = 0;
    CERTEX_HIP_TRY(hipGetDevice(&current));
    if (current != device) { CERTEX_HIP_TRY(hipSetDevice(device)); }
    void* ptr            = nullptr;
    hipError_t err       = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    hipEvent_t done      = nullptr;
    if (err == hipSuccess) { err = hipEventCreateWithFlags(&done, hipEventDisableTiming); }
    if (current != device) { CERTEX_HIP_TRY(hipSetDevice(current)); }
    CERTEX_HIP_TRY(err);
    expects(ptr != nullptr, "certex: no device address for the scratch array");
    g_scratch_done[device] = done;
    g_scratch[device]      = static_cast<char*>(ptr);
  }
  return g_scratch[device];
}

/**
 * Exclusive use of one GPU's scratch array for one search. The host lock orders the calls; on the
 * GPU, the search's stream first waits for the event recorded after the previous search's last
 * launch (on whatever stream that ran), and the event is recorded again after this search's last
 * launch. So searches on different streams or resources never overlap on the array, even though
 * each call returns with its last kernels still queued.
 */
struct scratch_turn {
  int device;
  hipStream_t stream;
  std::unique_lock<std::mutex> lk;
  scratch_turn(int dev, hipStream_t s) : device(dev), stream(s), lk(g_scratch_use[dev])
  {
    CERTEX_HIP_TRY(hipStreamWaitEvent(stream, g_scratch_done[device], 0));
  }
  ~scratch_turn() { (void)hipEventRecord(g_scratch_done[device], stream); }
};

/** Arena mode of the resources for the duration of one call (restored on every exit). */
struct arena_scope {
  cuvs::detail::resources_state& rs;
  arena_scope(cuvs::detail::resources_state& r, char* base, size_t bytes) : rs(r)
  {
    expects(rs.arena == nullptr, "certex: a search without allocation is already running on these resources");
    rs.arena       = base;
    rs.arena_bytes = bytes;
    rs.arena_reset();
  }
  ~arena_scope()
  {
    rs.arena_reset();
    rs.arena       = nullptr;
    rs.arena_bytes = 0;
  }
};

}  // namespace

auto no_alloc_scratch_bytes() -> size_t { return kNoAllocScratchBytes; }

template <typename T>
void search_without_allocation(cuvs::resources const& res, search_params const& params,
                               index<T> const& idx, matrix_view<const T> queries,
                               int64_t* neighbors, float* distances, int64_t k, filter f)
{
  certex_amd::filter_args fa{};
  if (f.type != filter::kind::none) {
    expects(f.words != nullptr, "certex: a filter needs its words");
    fa.kind      = f.type == filter::kind::bitset ? 1 : 2;
    fa.words     = f.words;
    fa.bitmap_ld = idx.size();
  }
  expects(!t_capture.on, "certex: a capture covers the allocating search");
  char* base = scratch_of(res.device());
  scratch_turn turn(res.device(), static_cast<hipStream_t>(res.stream()));
  arena_scope scope(res.state(), base, kNoAllocScratchBytes);
  try {
    search_impl(res, params, idx, queries, neighbors, distances, k, fa, true);
  } catch (batch_too_large const&) {
    throw std::runtime_error(
      "certex: one query of this search needs more than the 128 MiB scratch of a search without "
      "allocation; use the allocating search");
  }
}

void capture_begin()
{
  t_capture.arrays.clear();
  t_capture.on = true;
}

auto capture_get(std::string const& name, void* host) -> int64_t
{
  auto it = t_capture.arrays.find(name);
  expects(it != t_capture.arrays.end(), "certex: the capture holds no array of that name");
  if (host != nullptr) { std::memcpy(host, it->second.data(), it->second.size()); }
  return int64_t(it->second.size());
}

void stats_begin()
{
  t_stats_on = true;
  t_stats    = {};
}

auto stats_end() -> search_stats
{
  t_stats_on = false;
  return t_stats;
}

void timing_begin()
{
  if (t_timing.clock == nullptr) {
    CERTEX_HIP_TRY(hipMalloc(&t_timing.clock, 2 * sizeof(unsigned long long)));
  }
  CERTEX_HIP_TRY(hipDeviceSynchronize());
  CERTEX_HIP_TRY(hipMemset(t_timing.clock, 0, 2 * sizeof(unsigned long long)));
  CERTEX_HIP_TRY(hipDeviceSynchronize());
  t_timing.clock_mhz = 0;
  t_timing.on = true;
  for (auto& m : t_timing.marks) {
    t_timing.pool.push_back(m.start);
    t_timing.pool.push_back(m.stop);
  }
  t_timing.marks.clear();
}

auto timing_end() -> kernel_times
{
  kernel_times out;
  t_timing.on = false;
  for (auto& m : t_timing.marks) {
    CERTEX_HIP_TRY(hipEventSynchronize(m.stop));
    float ms = 0;
    CERTEX_HIP_TRY(hipEventElapsedTime(&ms, m.start, m.stop));
    out.ms[m.phase] += ms;
    out.launches[m.phase] += 1;
    t_timing.pool.push_back(m.start);
    t_timing.pool.push_back(m.stop);
  }
  t_timing.marks.clear();
  if (t_timing.clock != nullptr) {
    CERTEX_HIP_TRY(hipDeviceSynchronize());
    unsigned long long c[2] = {};
    CERTEX_HIP_TRY(hipMemcpy(c, t_timing.clock, sizeof(c), hipMemcpyDeviceToHost));
    // s_memrealtime counts at a constant 100 MHz
    t_timing.clock_mhz = c[1] > 0 ? double(c[0]) / double(c[1]) * 100.0 : 0.0;
  }
  return out;
}

auto timing_shader_clock_mhz() -> double { return t_timing.clock_mhz; }

template <typename T>
index<T>::index(cuvs::resources const& res) : s_(std::make_unique<index_state>())
{
  s_->device = res.device();
  s_->type   = detail::vtype_of<T>();
}
template <typename T>
index<T>::index(index&&) noexcept = default;
template <typename T>
index<T>& index<T>::operator=(index&&) noexcept = default;
template <typename T>
index<T>::~index() = default;

template <typename T>
auto index<T>::size() const noexcept -> int64_t { return s_->size; }
template <typename T>
auto index<T>::dim() const noexcept -> int64_t { return s_->dim; }
template <typename T>
auto index<T>::capacity() const noexcept -> int64_t { return s_->capacity; }
template <typename T>
auto index<T>::n_removed() const noexcept -> int64_t { return s_->n_removed; }
template <typename T>
auto index<T>::width() const noexcept -> int { return s_->width; }
template <typename T>
auto index<T>::anchor_stride() const noexcept -> int { return s_->anchor_stride; }
template <typename T>
auto index<T>::metric() const noexcept -> cuvs::distance::DistanceType { return s_->dmetric; }
template <typename T>
auto index<T>::has_labels() const noexcept -> bool { return s_->has_labels; }
template <typename T>
auto index<T>::n_partitioned() const noexcept -> int64_t { return s_->label_part.n; }
template <typename T>
auto index<T>::n_lists() const noexcept -> int { return s_->n_lists; }
template <typename T>
auto index<T>::list_offsets() const noexcept -> std::vector<int64_t> const&
{
  return s_->list_offsets;
}
template <typename T>
auto index<T>::host_vectors() const noexcept -> bool { return s_->host_vectors; }
template <typename T>
auto index<T>::state() const -> detail::index_state& { return *s_; }

constexpr int kKmeansRounds = 10;

/**
 * k-means lists of the stored rows [0, n) (reference fit_lists, lists.cuh:137-210): centers from
 * an evenly strided sample of the screening rows (kKmeansRounds Lloyd rounds from sample rows
 * spread evenly over it), every row's nearest center, and a stable sort of the ids by list, which
 * gives row_ids, id_rows and the list offsets. The caller then stores the rows in that order.
 */
void fit_lists(cuvs::resources const& res, index_state& st, int64_t n)
{
  using cuvs::detail::device_buffer;
  hipStream_t stream = static_cast<hipStream_t>(res.stream());
  const int L        = st.params.n_lists;
  const bool f16     = !is_int(st.type);
  const int width    = f16 ? st.halves : st.row_bytes;
  const int Lp       = certex_amd::pad_centers(L);
  const int64_t s    = std::max<int64_t>(L, std::min<int64_t>(n, st.params.kmeans_sample));
  const int64_t step = std::max<int64_t>(1, n / s);
  const int64_t cnt  = std::min<int64_t>(s, (n + step - 1) / step);
  device_buffer centers(size_t(L) * width * 4), centers_q(size_t(Lp) * st.row_bytes),
    cterm(size_t(Lp) * 4), assign(size_t(n) * 4);
  {
    device_buffer sids(size_t(cnt) * 4), sample(size_t(cnt) * st.row_bytes);
    device_buffer sums(size_t(L) * width * 4), counts(size_t(L) * 4), init_d(size_t(L) * 4);
    certex_amd::strided_ids(sids.as<int32_t>(), cnt, step, stream);
    certex_amd::gather_rows(st.codes.p, sids.as<int32_t>(), cnt, st.row_bytes, sample.p, stream);
    std::vector<int32_t> init(static_cast<size_t>(L));
    for (int c = 0; c < L; ++c) { init[size_t(c)] = int32_t(int64_t(c) * cnt / L); }
    CERTEX_HIP_TRY(
      hipMemcpyAsync(init_d.p, init.data(), init.size() * 4, hipMemcpyHostToDevice, stream));
    certex_amd::rows_to_centers(sample.p, f16, init_d.as<int32_t>(), L, width,
                                centers.as<float>(), stream);
    certex_amd::finish_centers(nullptr, nullptr, L, Lp, width, f16, centers.as<float>(),
                               centers_q.p, cterm.as<float>(), stream);
    for (int it = 0; it < kKmeansRounds; ++it) {
      certex_amd::nearest_centers(sample.p, f16, cnt, st.row_bytes, centers_q.p,
                                  cterm.as<float>(), Lp, assign.as<int32_t>(), stream);
      certex_amd::fill_u32(sums.as<uint32_t>(), int64_t(L) * width, 0, stream);
      certex_amd::fill_u32(counts.as<uint32_t>(), L, 0, stream);
      certex_amd::center_sums(sample.p, f16, cnt, width, assign.as<int32_t>(), L,
                              sums.as<float>(), counts.as<unsigned int>(), stream);
      certex_amd::finish_centers(sums.as<float>(), counts.as<unsigned int>(), L, Lp, width, f16,
                                 centers.as<float>(), centers_q.p, cterm.as<float>(), stream);
    }
    CERTEX_HIP_TRY(hipStreamSynchronize(stream));
  }
  // the list of every row, then the ids in list order (stable: ascending ids within a list)
  certex_amd::nearest_centers(st.codes.p, f16, n, st.row_bytes, centers_q.p, cterm.as<float>(),
                              Lp, assign.as<int32_t>(), stream);
  device_buffer keys(size_t(n) * 4), ids_tmp(size_t(n) * 4), row_ids(size_t(n) * 4),
    id_rows(size_t(n) * 4), offs(size_t(L + 1) * 8);
  const size_t tb = certex_amd::sort_by_label_temp_bytes(n);
  {
    device_buffer temp(std::max<size_t>(tb, 16));
    CERTEX_HIP_TRY(certex_amd::sort_by_label(assign.as<int32_t>(), n, ids_tmp.as<int32_t>(),
                                             keys.as<int32_t>(), row_ids.as<int32_t>(), temp.p,
                                             tb, stream));
    certex_amd::label_offsets(keys.as<int32_t>(), n, L, offs.as<int64_t>(), stream);
    certex_amd::invert_ids(row_ids.as<int32_t>(), n, id_rows.as<int32_t>(), stream);
    st.list_offsets.assign(size_t(L) + 1, 0);
    CERTEX_HIP_TRY(hipMemcpyAsync(st.list_offsets.data(), offs.p, st.list_offsets.size() * 8,
                                  hipMemcpyDeviceToHost, stream));
    CERTEX_HIP_TRY(hipStreamSynchronize(stream));
  }
  st.n_lists          = L;
  st.list_width       = width;
  st.list_offsets_dev = std::move(offs);
  st.centers    = std::move(centers);
  st.centers_q  = std::move(centers_q);
  st.cterm      = std::move(cterm);
  st.row_ids    = std::move(row_ids);
  st.id_rows    = std::move(id_rows);
  set_anchor_centers(res, st);
}

/**
 * Stores the screening rows [0, n) in list order (reference permuted(), lists.cuh:88-100):
 * stored row r is encoded again from the vector of id row_ids[r], read from the stored vectors
 * (float) or from the integer source x (device or host).
 */
void store_in_lists(cuvs::resources const& res, index_state& st, int64_t n, const void* x,
                    bool on_device)
{
  hipStream_t stream  = static_cast<hipStream_t>(res.stream());
  const auto* row_ids = st.row_ids.as<int32_t>();
  if (!is_int(st.type)) {
    const size_t rb     = size_t(st.dim) * elem_size(st.type);
    const int64_t chunk = std::max<int64_t>(1, (int64_t(64) << 20) / int64_t(rb));
    cuvs::detail::device_buffer staging(size_t(std::min(chunk, n)) * rb);
    for (int64_t r = 0; r < n; r += chunk) {
      const int64_t m = std::min(chunk, n - r);
      certex_amd::gather_rows(st.vectors.p, row_ids + r, m, int64_t(rb), staging.p, stream);
      certex_amd::encode_rows_f16(staging.p, elem_of(st.type), m, st.dim, st.halves, st.normalize,
                                  st.center.as<double>(), 1.0 / st.alpha, st.metric, st.gamma,
                                  st.codes.as<uint16_t>() + size_t(r) * st.halves,
                                  st.rowc.as<float>() + r, st.maxima.as<double>(), stream);
    }
    CERTEX_HIP_TRY(hipStreamSynchronize(stream));
    st.n_listed = n;
    return;
  }
  const uint8_t flip  = st.type == vtype::u8 ? 0x80 : 0;
  const int64_t d     = st.dim;
  const int64_t chunk = std::max<int64_t>(1, (int64_t(64) << 20) / d);
  cuvs::detail::device_buffer staging(size_t(std::min(chunk, n)) * d);
  std::vector<int32_t> h_ids;
  std::vector<uint8_t> h_rows;
  if (!on_device) {
    h_ids.resize(size_t(n));
    h_rows.resize(size_t(std::min(chunk, n)) * d);
    CERTEX_HIP_TRY(
      hipMemcpyAsync(h_ids.data(), row_ids, size_t(n) * 4, hipMemcpyDeviceToHost, stream));
    CERTEX_HIP_TRY(hipStreamSynchronize(stream));
  }
  const auto* src = static_cast<const uint8_t*>(x);
  for (int64_t r = 0; r < n; r += chunk) {
    const int64_t m = std::min(chunk, n - r);
    if (on_device) {
      certex_amd::gather_rows(src, row_ids + r, m, d, staging.p, stream);
    } else {
      // host rows gathered by host threads, then one copy
      const int threads = int(std::max(1u, std::min(16u, std::thread::hardware_concurrency())));
      std::vector<std::thread> pool;
      for (int t = 0; t < threads; ++t) {
        pool.emplace_back([&, t] {
          for (int64_t i = t; i < m; i += threads) {
            std::memcpy(h_rows.data() + i * d, src + int64_t(h_ids[size_t(r + i)]) * d,
                        size_t(d));
          }
        });
      }
      for (auto& th : pool) { th.join(); }
      CERTEX_HIP_TRY(hipMemcpyAsync(staging.p, h_rows.data(), size_t(m) * d,
                                    hipMemcpyHostToDevice, stream));
    }
    certex_amd::encode_rows_i8(staging.as<uint8_t>(), m, d, st.row_bytes, flip, st.metric,
                               st.codes.as<int8_t>() + r * st.row_bytes,
                               st.rowc.as<int32_t>() + r, stream);
    CERTEX_HIP_TRY(hipStreamSynchronize(stream));
  }
  st.n_listed = n;
}

template <typename T>
auto build(cuvs::resources const& res, index_params const& params, matrix_view<const T> dataset)
  -> index<T>
{
  index<T> out(res);
  index_state& st = out.state();
  st.metric       = to_kind(params.metric);
  st.dmetric      = params.metric;
  expects(!(st.metric == metric_kind::cosine && is_int(st.type)),
          "certex: cosine distance needs float32 or float16 vectors");
  expects(dataset.rows >= 1 && dataset.cols >= 1, "certex: the dataset is empty");
  expects(params.anchor_stride >= 1, "certex: anchor_stride must be at least 1");
  expects(params.n_lists >= 0 && params.n_lists <= dataset.rows,
          "certex: n_lists must lie in [0, number of vectors]");
  expects(params.n_lists <= certex_amd::kMaxLists, "certex: at most 16384 lists");
  expects(params.n_lists == 0 || dataset.rows < (int64_t(1) << 31),
          "certex: at most 2^31 - 1 vectors in an index with lists");
  // options this build does not implement are refused rather than ignored. Every screen here
  // reads full-dimension rows (the exact int8 screen of 8-bit vectors; for float vectors the
  // certificate of full-dimension fp16 rows is folded into the row terms and thresholds), so the
  // width is always the dimension: width 0 (auto) or at least the dimension is accepted, a
  // projection below it is refused; variance and pca_sample only parametrize the auto rule
  expects(params.width <= 0 || params.width >= dataset.cols,
          "certex: a projection width below the dimension is not supported by this build (every "
          "screen reads full-dimension rows): use width 0 or at least the dimension");
  expects(params.variance > 0.0 && params.variance <= 1.0, "certex: variance must lie in (0, 1]");
  expects(params.pca_sample >= 1, "certex: pca_sample must be at least 1");
  expects(!params.local_projections,
          "certex: local_projections (a projection per list) is not supported by this build");
  expects(!params.int8_rows || is_int(st.type),
          "certex: int8_rows needs 8-bit vectors in this build (float vectors are screened as "
          "fp16 rows; 8-bit vectors always as exact int8 rows)");
  st.params        = params;
  st.dim           = dataset.cols;
  st.anchor_stride = params.anchor_stride;
  st.host_vectors  = params.host_vectors;
  std::lock_guard w(st.writer);
  if (is_int(st.type)) {
    expects(dataset.cols <= certex_amd::kMaxIntDim,
            "certex: integer vectors of more than 4096 coordinates are not supported by this build");
    st.row_bytes = certex_amd::int_row_bytes(st.dim);
    st.width     = int(st.dim);
    grow(res, st, std::max(dataset.rows, params.capacity));
    append_int(res, st, reinterpret_cast<const uint8_t*>(dataset.data), dataset.rows,
               dataset.on_device, 0);
    res.sync();
    if (params.n_lists > 0) {  // the rows in list order; ids stay the input order
      fit_lists(res, st, dataset.rows);
      store_in_lists(res, st, dataset.rows, dataset.data, dataset.on_device);
    }
    refresh_anchors(res, st, 0, dataset.rows);
    res.sync();
    st.size = dataset.rows;
    return out;
  }
  expects(dataset.cols <= certex_amd::kMaxF16Halves,
          "certex: float vectors of more than 4096 coordinates are not supported by this build");
  hipStream_t stream = static_cast<hipStream_t>(res.stream());
  st.halves          = certex_amd::f16_row_halves(st.dim);
  st.row_bytes       = 2 * st.halves;
  st.width           = int(st.dim);
  st.normalize       = st.metric == metric_kind::cosine;
  // fp32 accumulation of halves + 1 terms; a factor 2 covers truncating accumulation
  st.gamma = 2.0 * double(st.halves + 1) * std::ldexp(1.0, -24);
  grow(res, st, std::max(dataset.rows, params.capacity));
  const int64_t n = dataset.rows;
  const auto t    = elem_of(st.type);
  // the vectors, then the center (mean; none for inner products) and the scale alpha that puts
  // every screening row within norm 64
  const size_t rb = size_t(st.dim) * sizeof(T);
  CERTEX_HIP_TRY(hipMemcpyAsync(st.vectors.p, dataset.data, size_t(n) * rb, hipMemcpyDefault,
                                stream));
  st.center.resize_discard(size_t(st.dim) * sizeof(double));
  st.maxima.resize_discard(2 * sizeof(double));
  CERTEX_HIP_TRY(hipMemsetAsync(st.center.p, 0, size_t(st.dim) * sizeof(double), stream));
  CERTEX_HIP_TRY(hipMemsetAsync(st.maxima.p, 0, 2 * sizeof(double), stream));
  if (st.metric != metric_kind::inner) {
    certex_amd::column_sums(st.vectors.p, t, n, st.dim, st.normalize, st.center.as<double>(),
                            stream);
    std::vector<double> c(size_t(st.dim));
    CERTEX_HIP_TRY(hipMemcpyAsync(c.data(), st.center.p, c.size() * sizeof(double),
                                  hipMemcpyDeviceToHost, stream));
    CERTEX_HIP_TRY(hipStreamSynchronize(stream));
    for (auto& v : c) { v /= double(n); }
    CERTEX_HIP_TRY(hipMemcpyAsync(st.center.p, c.data(), c.size() * sizeof(double),
                                  hipMemcpyHostToDevice, stream));
  }
  double* scratch = st.maxima.as<double>();  // max |x - c| lands in maxima[0] first
  certex_amd::max_norm(st.vectors.p, t, n, st.dim, st.normalize, st.center.as<double>(), scratch,
                       stream);
  double max_norm = 0;
  CERTEX_HIP_TRY(hipMemcpyAsync(&max_norm, scratch, sizeof(double), hipMemcpyDeviceToHost, stream));
  CERTEX_HIP_TRY(hipStreamSynchronize(stream));
  st.alpha = max_norm > 0 ? max_norm / 64.0 : 1.0;
  CERTEX_HIP_TRY(hipMemsetAsync(st.maxima.p, 0, 2 * sizeof(double), stream));
  certex_amd::encode_rows_f16(st.vectors.p, t, n, st.dim, st.halves, st.normalize,
                              st.center.as<double>(), 1.0 / st.alpha, st.metric, st.gamma,
                              st.codes.as<uint16_t>(), st.rowc.as<float>(), st.maxima.as<double>(),
                              stream);
  res.sync();
  if (params.n_lists > 0) {  // the rows in list order; ids and stored vectors stay the input order
    fit_lists(res, st, n);
    store_in_lists(res, st, n, nullptr, true);
  }
  refresh_anchors(res, st, 0, n);
  res.sync();
  st.size = n;
  return out;
}

template <typename T>
void extend(cuvs::resources const& res, matrix_view<const T> new_vectors, index<T>* idx)
{
  index_state& st = idx->state();
  expects(new_vectors.cols == st.dim, "dimension mismatch");
  if (new_vectors.rows == 0) { return; }
  std::lock_guard w(st.writer);
  const hipStream_t stream = static_cast<hipStream_t>(res.stream());
  st.await_updates(stream);
  const int64_t need = st.size + new_vectors.rows;
  if (need > st.capacity) { grow(res, st, std::max(need, 2 * st.capacity)); }
  if (is_int(st.type)) {
    append_int(res, st, reinterpret_cast<const uint8_t*>(new_vectors.data), new_vectors.rows,
               new_vectors.on_device, st.size);
  } else {
    append_float(res, st, new_vectors.data, new_vectors.rows, new_vectors.on_device, st.size);
  }
  refresh_anchors(res, st, st.size, need);  // anchors of the new ids only: searches read the others
  // vectors from host memory are read by the copy: it completes before the call returns; device
  // vectors are read in stream order, and searches on other streams wait for the update's event
  if (!new_vectors.on_device) { res.sync(); }
  st.mark_update(stream);
  std::unique_lock publish(st.rw);
  st.size = need;
}

template <typename T>
void reserve(cuvs::resources const& res, int64_t capacity, index<T>* idx)
{
  index_state& st = idx->state();
  std::lock_guard w(st.writer);
  grow(res, st, capacity);
}

template <typename T>
void remove(cuvs::resources const& res, const int64_t* ids, int64_t n_ids, index<T>* idx)
{
  index_state& st = idx->state();
  if (n_ids == 0) { return; }
  std::lock_guard w(st.writer);
  auto& rs           = res.state();
  hipStream_t stream = rs.stream;
  auto* counter      = static_cast<unsigned long long*>(rs.get(cuvs::detail::ws_small, 64));
  std::unique_lock publish(st.rw);
  CERTEX_HIP_TRY(hipDeviceSynchronize());
  certex_amd::fill_u32(reinterpret_cast<uint32_t*>(counter), 2, 0, stream);
  certex_amd::row_places at;
  at.list_pos  = st.id_rows.as<int32_t>();
  at.n_listed  = st.n_listed;
  at.part_pos  = st.label_part.pos.as<int32_t>();
  at.n_part    = st.label_part.n;
  at.part_rowc = st.label_part.rowc.p;
  at.anchor_rowc   = st.anchor_rowc.p;
  at.anchor_stride = std::max(1, st.anchor_stride);
  at.n_anchor      = (st.size + at.anchor_stride - 1) / at.anchor_stride;
  if (is_int(st.type)) {
    certex_amd::remove_rows_i8(ids, n_ids, st.size, st.rowc.as<int32_t>(), counter, at, stream);
  } else {
    certex_amd::remove_rows_f16(ids, n_ids, st.size, st.rowc.as<float>(), counter, at, stream);
  }
  CERTEX_HIP_TRY(hipMemcpyAsync(rs.host_small, counter, 8, hipMemcpyDeviceToHost, stream));
  CERTEX_HIP_TRY(hipStreamSynchronize(stream));
  st.n_removed += int64_t(*static_cast<unsigned long long*>(rs.host_small));
}

template <typename T>
void list_order(cuvs::resources const& res, index<T> const& idx, int32_t* out)
{
  index_state const& st = idx.state();
  expects(st.n_lists > 0, "certex: the index has no lists");
  std::shared_lock view(st.rw);
  hipStream_t stream = static_cast<hipStream_t>(res.stream());
  st.await_updates(stream);
  if (st.n_listed > 0) {
    CERTEX_HIP_TRY(hipMemcpyAsync(out, st.row_ids.p, size_t(st.n_listed) * sizeof(int32_t),
                                  hipMemcpyDeviceToDevice, stream));
  }
  certex_amd::iota_i32(out + st.n_listed, st.size - st.n_listed, int32_t(st.n_listed), stream);
}

template <typename T>
void set_labels(cuvs::resources const& res, const int32_t* labels, int64_t n, index<T>* idx,
                int64_t first)
{
  index_state& st = idx->state();
  expects(first >= 0 && first + n <= st.size, "certex: labels beyond the vectors of the index");
  std::lock_guard w(st.writer);
  hipStream_t stream = static_cast<hipStream_t>(res.stream());
  st.await_updates(stream);
  std::unique_lock publish(st.rw);
  if (!st.has_labels) {
    CERTEX_HIP_TRY(hipDeviceSynchronize());
    st.labels.resize_discard(size_t(std::max<int64_t>(st.capacity, 1)) * sizeof(int32_t));
    certex_amd::fill_i32(st.labels.as<int32_t>(), st.capacity, -1, stream);
    st.has_labels = true;
  }
  if (n > 0) {
    CERTEX_HIP_TRY(hipMemcpyAsync(st.labels.as<int32_t>() + first, labels,
                                  size_t(n) * sizeof(int32_t), hipMemcpyDeviceToDevice, stream));
  }
  st.mark_update(stream);
  if (n > 0 && first < st.label_part.n) { st.label_part.n = 0; }  // the partition no longer matches
}

template <typename T>
void partition_by_labels(cuvs::resources const& res, index<T>* idx)
{
  index_state& st = idx->state();
  expects(st.has_labels, "certex: the index has no labels");
  std::lock_guard w(st.writer);
  const int64_t n = st.size;
  expects(n < (int64_t(1) << 31), "certex: at most 2^31 - 1 vectors per partition");
  hipStream_t stream = static_cast<hipStream_t>(res.stream());
  st.await_updates(stream);
  using cuvs::detail::device_buffer;
  // rows of more than 256 bytes: the copy is paired, so that the tiled screen copies whole
  // 128-byte lines per stage
  const bool paired = uses_tile_screen(st);
  device_buffer keys(size_t(n) * 4), ids_tmp(size_t(n) * 4), ids(size_t(n) * 4),
    pos(size_t(n) * 4),
    codes(size_t(paired ? certex_amd::paired_bytes(n, st.row_bytes) : n * int64_t(st.row_bytes))),
    rowc(size_t(n) * 4);
  std::vector<int64_t> offsets;
  device_buffer offsets_dev;
  if (n > 0) {
    const size_t tb = certex_amd::sort_by_label_temp_bytes(n);
    device_buffer temp(std::max<size_t>(tb, 16));
    CERTEX_HIP_TRY(certex_amd::sort_by_label(st.labels.as<int32_t>(), n, ids_tmp.as<int32_t>(),
                                             keys.as<int32_t>(), ids.as<int32_t>(), temp.p, tb,
                                             stream));
    int32_t max_label = -1;
    CERTEX_HIP_TRY(hipMemcpyAsync(&max_label, keys.as<int32_t>() + n - 1, 4,
                                  hipMemcpyDeviceToHost, stream));
    CERTEX_HIP_TRY(hipStreamSynchronize(stream));
    const int64_t n_labels = int64_t(max_label) + 1;  // unlabeled rows (-1) sort first
    device_buffer offs(size_t(n_labels + 1) * 8);
    certex_amd::label_offsets(keys.as<int32_t>(), n, n_labels, offs.as<int64_t>(), stream);
    offsets.resize(size_t(n_labels + 1));
    CERTEX_HIP_TRY(hipMemcpyAsync(offsets.data(), offs.p, offsets.size() * 8,
                                  hipMemcpyDeviceToHost, stream));
    offsets_dev = std::move(offs);
    // the stored row of every id (they differ in an index with lists)
    const int32_t* from = ids.as<int32_t>();
    if (st.n_listed > 0) {
      certex_amd::stored_rows(ids.as<int32_t>(), n, st.id_rows.as<int32_t>(), st.n_listed,
                              ids_tmp.as<int32_t>(), stream);
      from = ids_tmp.as<int32_t>();
    }
    if (paired) {
      certex_amd::gather_rows_paired(st.codes.p, from, n, st.row_bytes, codes.p, stream);
    } else {
      certex_amd::gather_rows(st.codes.p, from, n, st.row_bytes, codes.p, stream);
    }
    certex_amd::gather_rows(st.rowc.p, from, n, 4, rowc.p, stream);
    certex_amd::invert_ids(ids.as<int32_t>(), n, pos.as<int32_t>(), stream);
    CERTEX_HIP_TRY(hipStreamSynchronize(stream));
  }
  std::unique_lock publish(st.rw);
  CERTEX_HIP_TRY(hipDeviceSynchronize());  // searches on other streams may read the old copy
  st.label_part.codes   = std::move(codes);
  st.label_part.rowc    = std::move(rowc);
  st.label_part.ids     = std::move(ids);
  st.label_part.pos     = std::move(pos);
  st.label_part.offsets = std::move(offsets);
  st.label_part.offsets_dev = std::move(offsets_dev);
  st.label_part.paired  = paired;
  st.label_part.n       = n;
}

template <typename T>
void search(cuvs::resources const& res, search_params const& params, index<T> const& idx,
            matrix_view<const T> queries, int64_t* neighbors, float* distances, int64_t k,
            filter f)
{
  certex_amd::filter_args fa{};
  if (f.type != filter::kind::none) {
    expects(f.words != nullptr, "certex: a filter needs its words");
    fa.kind      = f.type == filter::kind::bitset ? 1 : 2;
    fa.words     = f.words;
    fa.bitmap_ld = idx.size();
  }
  search_impl(res, params, idx, queries, neighbors, distances, k, fa);
}

template <typename T>
void search(cuvs::resources const& res, search_params const& params, index<T> const& idx,
            matrix_view<const T> queries, const int32_t* query_labels, int64_t* neighbors,
            float* distances, int64_t k, bool labels_on_host)
{
  expects(idx.has_labels(), "certex: the index has no labels");
  certex_amd::filter_args fa{};
  fa.kind         = 3;
  fa.row_labels   = idx.state().labels.template as<int32_t>();
  fa.query_labels = labels_on_host ? nullptr : query_labels;
  search_impl(res, params, idx, queries, neighbors, distances, k, fa, false,
              labels_on_host ? query_labels : nullptr);
}


namespace {

constexpr uint32_t kMagic         = 0x43455258;  // "CERX"
constexpr uint32_t kFormatVersion = 101;         // this build's layout of the stored arrays

template <typename T>
auto dtype_prefix() -> std::string
{
  std::string s;
  if constexpr (std::is_same_v<T, float>) {
    s = "<f4";
  } else if constexpr (std::is_same_v<T, half_t>) {
    s = "<f2";
  } else if constexpr (std::is_same_v<T, bfloat16_t>) {
    s = "<b2";  // no NumPy descriptor: this build's own prefix for bfloat16 vectors
  } else if constexpr (std::is_same_v<T, int8_t>) {
    s = "|i1";
  } else {
    s = "|u1";
  }
  s.resize(4, '\0');
  return s;
}

template <typename V>
void put(std::ostream& os, V v)
{
  os.write(reinterpret_cast<const char*>(&v), sizeof(V));
}
template <typename V>
auto get(std::istream& is) -> V
{
  V v{};
  is.read(reinterpret_cast<char*>(&v), sizeof(V));
  expects(bool(is), "certex: the index file is truncated");
  return v;
}

/**
 * Two pinned host buffers of at most 64 MiB through which the arrays of an index move between the
 * device and a file, chunk by chunk: the copy of one chunk overlaps the file I/O of the other,
 * and host memory stays bounded whatever the size of the index (a 10^9-row index holds 128 GB
 * of rows).
 */
struct io_staging {
  static constexpr size_t kChunk = size_t(64) << 20;
  hipStream_t stream;
  size_t chunk     = 0;
  void* buf[2]     = {};
  hipEvent_t ev[2] = {};
  bool pending[2]  = {};
  io_staging(cuvs::resources const& res, size_t largest)
    : stream(static_cast<hipStream_t>(res.stream())), chunk(std::min(kChunk, std::max<size_t>(largest, size_t(1) << 20)))
  {
    for (int i = 0; i < 2; ++i) {
      CERTEX_HIP_TRY(hipHostMalloc(&buf[i], chunk, hipHostMallocDefault));
      CERTEX_HIP_TRY(hipEventCreateWithFlags(&ev[i], hipEventDisableTiming));
    }
  }
  ~io_staging()
  {
    (void)hipStreamSynchronize(stream);
    for (int i = 0; i < 2; ++i) {
      if (buf[i] != nullptr) { (void)hipHostFree(buf[i]); }
      if (ev[i] != nullptr) { (void)hipEventDestroy(ev[i]); }
    }
  }
  io_staging(io_staging const&)            = delete;
  io_staging& operator=(io_staging const&) = delete;
  void wait(int i)
  {
    if (pending[i]) { CERTEX_HIP_TRY(hipEventSynchronize(ev[i])); }
    pending[i] = false;
  }
  void copy(int i, void* dst, const void* src, size_t bytes)
  {
    CERTEX_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, stream));
    CERTEX_HIP_TRY(hipEventRecord(ev[i], stream));
    pending[i] = true;
  }

  /** Write `bytes` of device (or mapped host) memory at `p` to the file. */
  void put(std::ostream& os, const void* p, size_t bytes)
  {
    const char* src  = static_cast<const char*>(p);
    const size_t n   = (bytes + chunk - 1) / chunk;
    auto len         = [&](size_t c) { return std::min(chunk, bytes - c * chunk); };
    if (n > 0) { copy(0, buf[0], src, len(0)); }
    for (size_t c = 0; c < n; ++c) {
      const int b = int(c & 1);
      if (c + 1 < n) {
        wait(b ^ 1);  // its chunk went to the file in the previous iteration
        copy(b ^ 1, buf[b ^ 1], src + (c + 1) * chunk, len(c + 1));
      }
      wait(b);
      os.write(static_cast<const char*>(buf[b]), std::streamsize(len(c)));
    }
  }

  /** Read `bytes` from the file into device (or mapped host) memory at `p`; the stream is
   *  synchronised before this returns. */
  void get(std::istream& is, void* p, size_t bytes)
  {
    char* dst      = static_cast<char*>(p);
    const size_t n = (bytes + chunk - 1) / chunk;
    for (size_t c = 0; c < n; ++c) {
      const int b      = int(c & 1);
      const size_t len = std::min(chunk, bytes - c * chunk);
      wait(b);  // the copy of chunk c - 2 out of this buffer is done
      is.read(static_cast<char*>(buf[b]), std::streamsize(len));
      expects(bool(is), "certex: the index file is truncated");
      copy(b, dst + c * chunk, buf[b], len);
    }
    CERTEX_HIP_TRY(hipStreamSynchronize(stream));
    pending[0] = pending[1] = false;
  }
};

}  // namespace

template <typename T>
void serialize(cuvs::resources const& res, std::string const& filename, index<T> const& idx)
{
  index_state const& st = idx.state();
  std::shared_lock view(st.rw);
  st.await_updates(static_cast<hipStream_t>(res.stream()));
  std::ofstream os(filename, std::ios::binary);
  expects(os.good(), "certex: cannot open the index file for writing");
  os << dtype_prefix<T>();
  put(os, kMagic);
  put(os, kFormatVersion);
  put(os, int32_t(st.dmetric));
  put(os, int64_t(st.dim));
  put(os, int32_t(st.width));
  put(os, int32_t(st.anchor_stride));
  put(os, uint8_t(st.host_vectors));
  put(os, int64_t(st.size));
  put(os, int64_t(st.n_removed));
  put(os, uint8_t(st.has_labels));
  put(os, int32_t(st.row_bytes));
  put(os, st.alpha);
  put(os, st.gamma);
  put(os, int32_t(st.halves));
  put(os, uint8_t(st.normalize));
  const size_t n = size_t(st.size);
  io_staging io(res, n * std::max<size_t>(st.row_bytes, size_t(st.dim) * elem_size(st.type)));
  io.put(os, st.codes.p, n * st.row_bytes);
  io.put(os, st.rowc.p, n * 4);
  if (!is_int(st.type)) {
    io.put(os, st.vectors.p, n * size_t(st.dim) * elem_size(st.type));
    io.put(os, st.center.p, size_t(st.dim) * sizeof(double));
    io.put(os, st.maxima.p, 2 * sizeof(double));
  }
  if (st.has_labels) { io.put(os, st.labels.p, n * sizeof(int32_t)); }
  put(os, int32_t(st.n_lists));
  if (st.n_lists > 0) {
    put(os, int64_t(st.n_listed));
    put(os, int32_t(st.list_width));
    os.write(reinterpret_cast<const char*>(st.list_offsets.data()),
             std::streamsize(st.list_offsets.size() * 8));
    io.put(os, st.row_ids.p, size_t(st.n_listed) * 4);
    io.put(os, st.centers.p, size_t(st.n_lists) * st.list_width * 4);
  }
  expects(os.good(), "certex: writing the index file failed");
}

template <typename T>
void deserialize(cuvs::resources const& res, std::string const& filename, index<T>* idx)
{
  index_state& st = idx->state();
  std::ifstream is(filename, std::ios::binary);
  expects(is.good(), "certex: cannot open the index file");
  char prefix[4] = {};
  is.read(prefix, 4);
  expects(bool(is) && std::memcmp(prefix, dtype_prefix<T>().data(), 4) == 0,
          "certex: the file holds vectors of another type");
  expects(get<uint32_t>(is) == kMagic, "certex: not a CertEx index file");
  expects(get<uint32_t>(is) == kFormatVersion,
          "certex: the index file was written by another version of the library");
  std::lock_guard w(st.writer);
  st.dmetric       = static_cast<cuvs::distance::DistanceType>(get<int32_t>(is));
  st.metric        = to_kind(st.dmetric);
  st.dim           = get<int64_t>(is);
  st.width         = get<int32_t>(is);
  st.anchor_stride = get<int32_t>(is);
  st.host_vectors  = get<uint8_t>(is) != 0;
  const int64_t n  = get<int64_t>(is);
  st.n_removed     = get<int64_t>(is);
  const bool labels = get<uint8_t>(is) != 0;
  st.row_bytes     = get<int32_t>(is);
  st.alpha         = get<double>(is);
  st.gamma         = get<double>(is);
  st.halves        = get<int32_t>(is);
  st.normalize     = get<uint8_t>(is) != 0;
  expects(st.dim >= 1 && n >= 0 && st.row_bytes > 0, "certex: corrupt index file");
  st.size     = 0;
  st.capacity = 0;
  grow(res, st, std::max<int64_t>(n, 1));
  io_staging io(res, size_t(n) * std::max<size_t>(st.row_bytes, size_t(st.dim) * elem_size(st.type)));
  io.get(is, st.codes.p, size_t(n) * st.row_bytes);
  io.get(is, st.rowc.p, size_t(n) * 4);
  if (!is_int(st.type)) {
    st.center.resize_discard(size_t(st.dim) * sizeof(double));
    st.maxima.resize_discard(2 * sizeof(double));
    io.get(is, st.vectors.p, size_t(n) * size_t(st.dim) * elem_size(st.type));
    io.get(is, st.center.p, size_t(st.dim) * sizeof(double));
    io.get(is, st.maxima.p, 2 * sizeof(double));
  }
  if (labels) {
    st.labels.resize_discard(size_t(st.capacity) * sizeof(int32_t));
    io.get(is, st.labels.p, size_t(n) * sizeof(int32_t));
    st.has_labels = true;
  }
  const int32_t L = get<int32_t>(is);
  expects(L >= 0 && L <= certex_amd::kMaxLists, "certex: corrupt index file");
  if (L > 0) {
    st.n_listed   = get<int64_t>(is);
    st.list_width = get<int32_t>(is);
    expects(st.n_listed >= 0 && st.n_listed <= n && st.list_width > 0,
            "certex: corrupt index file");
    st.list_offsets.assign(size_t(L) + 1, 0);
    is.read(reinterpret_cast<char*>(st.list_offsets.data()), std::streamsize((L + 1) * 8));
    expects(bool(is), "certex: the index file is truncated");
    // the searches read the rows of a list at these offsets on the GPU
    expects(st.list_offsets.front() == 0 && st.list_offsets.back() == st.n_listed &&
              std::is_sorted(st.list_offsets.begin(), st.list_offsets.end()),
            "certex: corrupt index file");
    const int Lp = certex_amd::pad_centers(L);
    st.row_ids.resize_discard(size_t(std::max<int64_t>(st.n_listed, 1)) * 4);
    st.id_rows.resize_discard(size_t(std::max<int64_t>(st.n_listed, 1)) * 4);
    st.centers.resize_discard(size_t(L) * st.list_width * 4);
    st.centers_q.resize_discard(size_t(Lp) * st.row_bytes);
    st.cterm.resize_discard(size_t(Lp) * 4);
    io.get(is, st.row_ids.p, size_t(st.n_listed) * 4);
    io.get(is, st.centers.p, size_t(L) * st.list_width * 4);
    hipStream_t stream = static_cast<hipStream_t>(res.stream());
    certex_amd::invert_ids(st.row_ids.as<int32_t>(), st.n_listed, st.id_rows.as<int32_t>(), stream);
    certex_amd::finish_centers(nullptr, nullptr, L, Lp, st.list_width, !is_int(st.type),
                               st.centers.as<float>(), st.centers_q.p, st.cterm.as<float>(),
                               stream);
    st.list_offsets_dev.resize_discard(size_t(L + 1) * 8);
    CERTEX_HIP_TRY(hipMemcpyAsync(st.list_offsets_dev.p, st.list_offsets.data(), size_t(L + 1) * 8,
                                  hipMemcpyHostToDevice, stream));
    res.sync();
    st.n_lists = L;
    set_anchor_centers(res, st);
  }
  refresh_anchors(res, st, 0, n);
  res.sync();
  st.size = n;
}

#define CERTEX_INSTANTIATE(T)                                                                  \
  template class index<T>;                                                                     \
  template auto build<T>(cuvs::resources const&, index_params const&, matrix_view<const T>)    \
    -> index<T>;                                                                               \
  template void extend<T>(cuvs::resources const&, matrix_view<const T>, index<T>*);            \
  template void reserve<T>(cuvs::resources const&, int64_t, index<T>*);                        \
  template void remove<T>(cuvs::resources const&, const int64_t*, int64_t, index<T>*);         \
  template void set_labels<T>(cuvs::resources const&, const int32_t*, int64_t, index<T>*,      \
                              int64_t);                                                        \
  template void partition_by_labels<T>(cuvs::resources const&, index<T>*);                     \
  template void list_order<T>(cuvs::resources const&, index<T> const&, int32_t*);              \
  template void search_without_allocation<T>(cuvs::resources const&, search_params const&,     \
                                             index<T> const&, matrix_view<const T>, int64_t*,  \
                                             float*, int64_t, filter);                         \
  template void search<T>(cuvs::resources const&, search_params const&, index<T> const&,       \
                          matrix_view<const T>, int64_t*, float*, int64_t, filter);            \
  template void search<T>(cuvs::resources const&, search_params const&, index<T> const&,       \
                          matrix_view<const T>, const int32_t*, int64_t*, float*, int64_t,     \
                          bool);                                                               \
  template void serialize<T>(cuvs::resources const&, std::string const&, index<T> const&);     \
  template void deserialize<T>(cuvs::resources const&, std::string const&, index<T>*);

CERTEX_INSTANTIATE(float)
CERTEX_INSTANTIATE(half_t)
CERTEX_INSTANTIATE(bfloat16_t)
CERTEX_INSTANTIATE(int8_t)
CERTEX_INSTANTIATE(uint8_t)

}  // namespace cuvs::neighbors::certex
