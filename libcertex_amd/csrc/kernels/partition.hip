// Label partition of the screening rows and the per-batch routing moves (gfx950).
//
// Reference contract: partition_by_labels (certex.cu:1542-1606: a stable sort of the ids by
// label, the start of every label, the rows copied in label order) and the query permutation of
// search_by_labels (certex.cu:1613-1735: the batch in label order, results back in query order).
// The sort is hipCUB's radix sort over (label, id) pairs, stable, so the ids of one label stay
// ascending; unlabeled rows (-1) sort first and match no query.

#include "../kernels.hpp"

#include <hipcub/hipcub.hpp>
#include <stdexcept>

namespace certex_amd {
namespace {

inline unsigned blocks_for(int64_t n, int64_t cap = int64_t(1) << 20)
{
  const int64_t b = (n + 255) / 256;
  return unsigned(b < cap ? b : cap);
}

__global__ void iota_kernel(int32_t* p, int64_t n)
{
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * blockDim.x) {
    p[i] = int32_t(i);
  }
}

/** offsets[l] = the first sorted position whose label is >= l, for l = 0 .. n_labels. */
__global__ void label_offsets_kernel(const int32_t* keys, int64_t n, int64_t n_labels,
                                     int64_t* offsets)
{
  const int64_t l = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (l > n_labels) { return; }
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (keys[mid] < l) {
      lo = mid + 1;
    } else {
      hi = mid;
    }
  }
  offsets[l] = lo;
}

/** The first position in sorted[0, n) whose value is >= v. */
__device__ inline int64_t lower_pos(const int32_t* sorted, int64_t n, int64_t v)
{
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (int64_t(sorted[mid]) < v) {
      lo = mid + 1;
    } else {
      hi = mid;
    }
  }
  return lo;
}

constexpr int kRouteThreads = 1024;

/**
 * route_tables: one block; per round of kRouteThreads labels, each thread builds its label's two
 * groups and workgroup counts (rounded up to 8), an exclusive scan over the block places them
 * after the previous rounds' groups.
 */
/** Label l's group (its partition rows, its queries [q0, q0 + nq) of the sorted batch) and the
 *  workgroups of its anchor pass (ta) and screen (ts), each rounded up to 8 (an XCD octet). */
__device__ inline screen_group route_group(const route_table_args& a, int64_t l, int64_t q0,
                                           int64_t nq, int64_t& ta, int64_t& ts)
{
  screen_group g{0, 0, 0, 0, 0};
  ta = ts = 0;
  g.x0 = a.offsets[l];
  g.nx = a.offsets[l + 1] - g.x0;
  g.q0 = q0;
  g.nq = g.nx > 0 ? nq : 0;
  if (g.nq > 0) {
    const int64_t anchors = a.anchor_pairs ? paired_anchor_count(g.x0, g.nx, a.anchor_stride)
                                           : (g.nx + a.anchor_stride - 1) / a.anchor_stride;
    ta = screen_group_tiles(g.nq + (g.q0 & a.anchor_lead), anchors, a.anchor_qb, a.anchor_chunk);
    ts = a.screen_tiled ? paired_group_tiles(g, a.rows_paired, a.screen_qb, a.screen_chunk)
                        : screen_group_tiles(g.nq, g.nx, a.screen_qb, a.screen_chunk);
    ta = (ta + 7) / 8 * 8;
    ts = (ts + 7) / 8 * 8;
  }
  return g;
}

__global__ __launch_bounds__(kRouteThreads) void route_tables_kernel(route_table_args a)
{
  __shared__ int64_t sa[kRouteThreads], ss[kRouteThreads];
  __shared__ int64_t base_a, base_s;
  const int tid = threadIdx.x;
  if (tid == 0) { base_a = base_s = 0; }
  __syncthreads();
  for (int64_t l0 = 0; l0 < a.n_labels; l0 += kRouteThreads) {
    const int64_t l = l0 + tid;
    screen_group g{0, 0, 0, 0, 0};
    int64_t ta = 0, ts = 0;
    if (l < a.n_labels) {
      const int64_t q0 = lower_pos(a.sorted, a.B, l);
      g                = route_group(a, l, q0, lower_pos(a.sorted, a.B, l + 1) - q0, ta, ts);
    }
    // exclusive scan of the workgroup counts over the round (Hillis-Steele in LDS)
    sa[tid] = ta;
    ss[tid] = ts;
    __syncthreads();
    for (int off = 1; off < kRouteThreads; off <<= 1) {
      const int64_t va = tid >= off ? sa[tid - off] : 0;
      const int64_t vs = tid >= off ? ss[tid - off] : 0;
      __syncthreads();
      sa[tid] += va;
      ss[tid] += vs;
      __syncthreads();
    }
    if (l < a.n_labels) {
      screen_group ga = g, gs = g;
      ga.tile0 = base_a + sa[tid] - ta;
      gs.tile0 = base_s + ss[tid] - ts;
      a.anchor_groups[l] = ga;
      a.screen_groups[l] = gs;
    }
    __syncthreads();
    if (tid == kRouteThreads - 1) {
      base_a += sa[tid];
      base_s += ss[tid];
    }
    __syncthreads();
  }
}

/**
 * The routing of a batch of B query labels in one workgroup, for few labels (kSmallBuckets
 * buckets at most: labels below 0, each label of the partition, labels past it): a stable
 * counting sort of the batch by label into order / sorted, then the group tables of
 * route_tables_kernel, their queries read off the bucket counts. Chunks of 64 queries go to the
 * waves in turn; per chunk, seven ballots (one per bit of the bucket index) give every query the
 * lanes of its bucket, hence its rank within the chunk and the bucket's count. Replaces the radix sort (an index fill and five launches) and the separate
 * group-table launch. Labels below 0 and past the partition keep their relative order but not
 * their order by value: the groups only ask where each partition label starts and ends.
 */
constexpr int kSmallBuckets = 64;
constexpr int kSmallCounts  = 12288;  // LDS words for (chunk, bucket) counts: chunks x buckets

__global__ __launch_bounds__(kRouteThreads) void route_small_kernel(route_table_args a,
                                                                    const int32_t* labels,
                                                                    int32_t* order, int32_t* sorted)
{
  __shared__ int cnt[kSmallCounts];   // [chunk][bucket]: count, then its exclusive prefix over chunks
  __shared__ int tot[kSmallBuckets];  // queries per bucket
  __shared__ int start[kSmallBuckets + 1];
  __shared__ int64_t sa[kSmallBuckets], ss[kSmallBuckets];
  const int tid      = threadIdx.x;
  const int lane     = tid & 63;
  const int wave     = tid >> 6;
  constexpr int W    = kRouteThreads / 64;
  const int64_t B    = a.B;
  const int nb       = int(a.n_labels) + 2;
  const int n_chunks = int((B + 63) / 64);
  auto bucket_of     = [&](int32_t l) { return l < 0 ? 0 : (l < a.n_labels ? l + 1 : nb - 1); };
  // the labels of 4 chunks of a wave at a time, their loads in flight together (past B: none)
  constexpr int CB = 4;
  auto labels4     = [&](int c0, int32_t (&lb)[CB], bool (&in)[CB]) {
#pragma unroll
    for (int u = 0; u < CB; ++u) {
      const int64_t i = int64_t(c0 + u * W) * 64 + lane;
      in[u]           = i < B;
      lb[u]           = in[u] ? labels[i] : 0;
    }
  };
  // the lanes of the wave whose bucket equals this lane's (7 bits: -1, past B, sets bit 6, which no
  // bucket below 64 has); one ballot per bit instead of one per bucket
  auto same_bucket = [&](int b) {
    uint64_t m = ~uint64_t(0);
#pragma unroll
    for (int k = 0; k < 7; ++k) {
      const bool bit     = (b >> k) & 1;
      const uint64_t bal = __ballot(bit);
      m &= bit ? bal : ~bal;
    }
    return m;
  };
  for (int e = tid; e < n_chunks * nb; e += kRouteThreads) { cnt[e] = 0; }
  __syncthreads();
  // counts per (chunk, bucket): the lowest lane of each bucket present writes its count
  for (int c0 = wave; c0 < n_chunks; c0 += CB * W) {
    int32_t lb[CB];
    bool in[CB];
    labels4(c0, lb, in);
#pragma unroll
    for (int u = 0; u < CB; ++u) {
      const int c = c0 + u * W;
      if (c >= n_chunks) { break; }
      const int b      = in[u] ? bucket_of(lb[u]) : -1;
      const uint64_t m = same_bucket(b);
      const int below  = int(__builtin_amdgcn_mbcnt_hi(uint32_t(m >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(m), 0u)));
      if (b >= 0 && below == 0) { cnt[c * nb + b] = __builtin_popcountll(m); }
    }
  }
  __syncthreads();
  // per bucket, the exclusive prefix of its counts over the chunks (a wave per bucket)
  for (int v = wave; v < nb; v += W) {
    int carry = 0;
    for (int c0 = 0; c0 < n_chunks; c0 += 64) {
      const int c = c0 + lane;
      const int x = c < n_chunks ? cnt[c * nb + v] : 0;
      int incl    = x;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(incl, off);
        if (lane >= off) { incl += y; }
      }
      if (c < n_chunks) { cnt[c * nb + v] = carry + incl - x; }
      carry += __shfl(incl, 63);
    }
    if (lane == 0) { tot[v] = carry; }
  }
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int v = 0; v < nb; ++v) {
      start[v] = run;
      run += tot[v];
    }
    start[nb] = run;
  }
  __syncthreads();
  // the scatter: a query's place is its bucket's start, the bucket's count in earlier chunks and
  // its rank among the chunk's queries of the bucket
  for (int c0 = wave; c0 < n_chunks; c0 += CB * W) {
    int32_t lb[CB];
    bool in[CB];
    labels4(c0, lb, in);
#pragma unroll
    for (int u = 0; u < CB; ++u) {
      const int c = c0 + u * W;
      if (c >= n_chunks) { break; }
      const int64_t i  = int64_t(c) * 64 + lane;
      const int b      = in[u] ? bucket_of(lb[u]) : -1;
      const uint64_t m = same_bucket(b);
      const int rank   = int(__builtin_amdgcn_mbcnt_hi(uint32_t(m >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(m), 0u)));
      if (b >= 0) {
        const int pos = start[b] + cnt[c * nb + b] + rank;
        order[pos]    = int32_t(i);
        sorted[pos]   = lb[u];
      }
    }
  }
  // the group tables: label l is bucket l + 1; the workgroup counts' exclusive scan over the labels
  const int64_t l = tid;
  int64_t ta = 0, ts = 0;
  screen_group g{0, 0, 0, 0, 0};
  if (l < a.n_labels) { g = route_group(a, l, start[l + 1], tot[l + 1], ta, ts); }
  if (tid < kSmallBuckets) {
    sa[tid] = ta;
    ss[tid] = ts;
  }
  __syncthreads();
  if (l < a.n_labels) {
    int64_t pa = 0, ps = 0;
    for (int64_t j = 0; j < l; ++j) {
      pa += sa[j];
      ps += ss[j];
    }
    screen_group ga = g, gs = g;
    ga.tile0 = pa;
    gs.tile0 = ps;
    a.anchor_groups[l] = ga;
    a.screen_groups[l] = gs;
  }
}

/** dst row i = src row ids[i], rows of `units` 16-byte units. */
__global__ void gather_units_kernel(const int4* src, const int32_t* ids, int64_t n, int64_t units,
                                    int4* dst)
{
  const int64_t total = n * units;
  for (int64_t t = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; t < total;
       t += int64_t(gridDim.x) * blockDim.x) {
    const int64_t i = t / units, u = t % units;
    dst[t]          = src[int64_t(ids[i]) * units + u];
  }
}

/** dst row i = src row ids[i] in the paired layout: 16-byte unit u of row i at unit
 *  (i / 2) 2 units + (u / 4) 8 + (i % 2) 4 + u % 4 (units = row bytes / 16, a multiple of 8). */
__global__ void gather_paired_kernel(const int4* src, const int32_t* ids, int64_t n, int64_t units,
                                     int4* dst)
{
  const int64_t total = n * units;
  for (int64_t t = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; t < total;
       t += int64_t(gridDim.x) * blockDim.x) {
    const int64_t i = t / units, u = t % units;
    dst[(i >> 1) * 2 * units + (u >> 2) * 8 + (i & 1) * 4 + (u & 3)] = src[int64_t(ids[i]) * units + u];
  }
}

/** dst row i = src row ids[i], rows of `bytes` bytes (any length). */
__global__ void gather_bytes_kernel(const uint8_t* src, const int32_t* ids, int64_t n,
                                    int64_t bytes, uint8_t* dst)
{
  const int64_t total = n * bytes;
  for (int64_t t = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; t < total;
       t += int64_t(gridDim.x) * blockDim.x) {
    const int64_t i = t / bytes, b = t % bytes;
    dst[t]          = src[int64_t(ids[i]) * bytes + b];
  }
}

/** pos[ids[i]] = i. */
__global__ void invert_kernel(const int32_t* ids, int64_t n, int32_t* pos)
{
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * blockDim.x) {
    pos[ids[i]] = int32_t(i);
  }
}

/** Anchor j0 + t / units: one 16-byte unit of its codes (and its term with the first unit). */
__global__ void gather_anchors_kernel(const int4* codes, const uint32_t* rowc, int64_t units,
                                      int64_t stride, int64_t j0, int64_t n, const int32_t* id_rows,
                                      int64_t n_listed, int4* anchor_codes, uint32_t* anchor_rowc)
{
  for (int64_t t = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; t < n * units;
       t += int64_t(gridDim.x) * blockDim.x) {
    const int64_t j   = j0 + t / units, u = t % units;
    const int64_t id  = j * stride;
    const int64_t row = id < n_listed ? int64_t(id_rows[id]) : id;
    anchor_codes[j * units + u] = codes[row * units + u];
    if (u == 0) { anchor_rowc[j] = rowc[row]; }
  }
}

/** out[i] = i * step. */
__global__ void strided_kernel(int32_t* out, int64_t n, int64_t step)
{
  const int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (i < n) { out[i] = int32_t(i * step); }
}

/** out[i] = the stored row of id ids[i]: id_rows[id] below n_listed, else the id itself. */
__global__ void stored_rows_kernel(const int32_t* ids, int64_t n, const int32_t* id_rows,
                                   int64_t n_listed, int32_t* out)
{
  const int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (i >= n) { return; }
  const int32_t id = ids[i];
  out[i]           = id < n_listed ? id_rows[id] : id;
}

}  // namespace

void gather_anchors(const void* codes, const void* rowc, int row_bytes, int64_t stride, int64_t j0,
                    int64_t j1, const int32_t* id_rows, int64_t n_listed, void* anchor_codes,
                    void* anchor_rowc, hipStream_t stream)
{
  if (j1 <= j0) { return; }
  const int64_t units = row_bytes / 16;
  gather_anchors_kernel<<<blocks_for((j1 - j0) * units), 256, 0, stream>>>(
    static_cast<const int4*>(codes), static_cast<const uint32_t*>(rowc), units, stride, j0,
    j1 - j0, id_rows, n_listed, static_cast<int4*>(anchor_codes),
    static_cast<uint32_t*>(anchor_rowc));
}

void strided_ids(int32_t* out, int64_t n, int64_t step, hipStream_t stream)
{
  if (n == 0) { return; }
  strided_kernel<<<unsigned((n + 255) / 256), 256, 0, stream>>>(out, n, step);
}

void stored_rows(const int32_t* ids, int64_t n, const int32_t* id_rows, int64_t n_listed,
                 int32_t* out, hipStream_t stream)
{
  if (n == 0) { return; }
  stored_rows_kernel<<<unsigned((n + 255) / 256), 256, 0, stream>>>(ids, n, id_rows, n_listed,
                                                                    out);
}

size_t sort_by_label_temp_bytes(int64_t n)
{
  size_t bytes = 0;
  (void)hipcub::DeviceRadixSort::SortPairs(nullptr, bytes, static_cast<const int32_t*>(nullptr),
                                           static_cast<int32_t*>(nullptr),
                                           static_cast<const int32_t*>(nullptr),
                                           static_cast<int32_t*>(nullptr), int(n), 0, 32);
  return bytes;
}

hipError_t sort_by_label(const int32_t* labels, int64_t n, int32_t* ids_scratch, int32_t* keys_out,
                         int32_t* ids_out, void* temp, size_t temp_bytes, hipStream_t stream)
{
  if (n == 0) { return hipSuccess; }
  iota_kernel<<<blocks_for(n), 256, 0, stream>>>(ids_scratch, n);
  return hipcub::DeviceRadixSort::SortPairs(temp, temp_bytes, labels, keys_out, ids_scratch,
                                            ids_out, int(n), 0, 32, stream);
}

void route_tables(const route_table_args& a, hipStream_t stream)
{
  if (a.n_labels == 0) { return; }
  route_tables_kernel<<<1, kRouteThreads, 0, stream>>>(a);
}

bool route_small_fits(int64_t B, int64_t n_labels)
{
  const int64_t nb = n_labels + 2;
  return n_labels > 0 && nb <= kSmallBuckets && (B + 63) / 64 * nb <= kSmallCounts;
}

void route_small(const route_table_args& a, const int32_t* labels, int32_t* order, int32_t* sorted,
                 hipStream_t stream)
{
  if (!route_small_fits(a.B, a.n_labels)) {
    throw std::logic_error("certex: the one-workgroup routing takes at most 62 labels and 12,288 chunk counts");
  }
  route_small_kernel<<<1, kRouteThreads, 0, stream>>>(a, labels, order, sorted);
}

void label_offsets(const int32_t* keys_sorted, int64_t n, int64_t n_labels, int64_t* offsets,
                   hipStream_t stream)
{
  label_offsets_kernel<<<unsigned((n_labels + 1 + 255) / 256), 256, 0, stream>>>(
    keys_sorted, n, n_labels, offsets);
}

void gather_rows(const void* src, const int32_t* ids, int64_t n, int64_t row_bytes, void* dst,
                 hipStream_t stream)
{
  if (n == 0 || row_bytes == 0) { return; }
  if (row_bytes % 16 == 0) {
    gather_units_kernel<<<blocks_for(n * (row_bytes / 16)), 256, 0, stream>>>(
      static_cast<const int4*>(src), ids, n, row_bytes / 16, static_cast<int4*>(dst));
  } else {
    gather_bytes_kernel<<<blocks_for(n * row_bytes), 256, 0, stream>>>(
      static_cast<const uint8_t*>(src), ids, n, row_bytes, static_cast<uint8_t*>(dst));
  }
}

void gather_rows_paired(const void* src, const int32_t* ids, int64_t n, int64_t row_bytes,
                        void* dst, hipStream_t stream)
{
  if (n == 0) { return; }
  if (row_bytes % 128 != 0) { throw std::logic_error("certex: paired rows are whole 128-byte lines"); }
  gather_paired_kernel<<<blocks_for(n * (row_bytes / 16)), 256, 0, stream>>>(
    static_cast<const int4*>(src), ids, n, row_bytes / 16, static_cast<int4*>(dst));
}

void invert_ids(const int32_t* ids, int64_t n, int32_t* pos, hipStream_t stream)
{
  if (n == 0) { return; }
  invert_kernel<<<blocks_for(n), 256, 0, stream>>>(ids, n, pos);
}

}  // namespace certex_amd
