// Threshold selection, fp64 exact re-rank, per-query top-k and output conversion (gfx950).
//
// Reference contracts:
//   threshold  anchor_threshold (certex_kernels.cuh:310-370): the k-th best anchor bounds the k-th
//              neighbour; here the k-th largest of the per-group best screen values, found by an
//              LDS radix select over the 32-bit keys (4 passes of 8 bits).
//   re-rank    rounds_score / warp_score (detail/verify.cuh:186-218, certex_kernels.cuh:247-273):
//              the exact score of every survivor in fp64 from the stored vectors.
//   top-k      rounds_merge + segmented sort (detail/verify.cuh:240-364): here the survivors of a
//              query sit in LDS and are ordered by the total order (score, row), so ties go to the
//              lower id, which the reference does not guarantee.
//   finish     certex.cu:224-250.

#include "../kernels.hpp"

#include <cfloat>
#include <climits>
#include <cmath>

namespace certex_amd {
namespace {

constexpr int kThreads = 256;

/** Inclusive prefix sum over the 256 threads of a block (4 waves). */
__device__ inline int block_scan_incl(int v, int* wave_tot)
{
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int t = __shfl_up(incl, off);
    if (lane >= off) { incl += t; }
  }
  if (lane == 63) { wave_tot[wave] = incl; }
  __syncthreads();
  int add = 0;
  for (int w = 0; w < wave; ++w) { add += wave_tot[w]; }
  __syncthreads();
  return incl + add;
}

/** The largest of key[0, n) over the block (every thread gets it); scratch: 4 LDS words x 2. */
__device__ inline uint64_t block_max_key(const uint64_t* key, int n, uint64_t* wave_max)
{
  uint64_t m = 0;
  for (int e = threadIdx.x; e < n; e += kThreads) { m = key[e] > m ? key[e] : m; }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint64_t o = __shfl_xor(m, off);
    m                = o > m ? o : m;
  }
  if ((threadIdx.x & 63) == 0) { wave_max[threadIdx.x >> 6] = m; }
  __syncthreads();
  uint64_t r = wave_max[0];
  for (int w = 1; w < kThreads / 64; ++w) { r = wave_max[w] > r ? wave_max[w] : r; }
  __syncthreads();
  return r;
}

/**
 * Slot of this lane in an LDS list counted by *fill, for the lanes whose `take` is set: one LDS
 * atomic per wave (the taking lanes in lane order) instead of one per entry, which would all hit
 * the same word. Every lane of the wave calls it; the others get an unused value.
 */
__device__ inline int wave_append(bool take, int* fill)
{
  const uint64_t m = __ballot(take);
  if (m == 0) { return 0; }
  const int lane   = threadIdx.x & 63;
  const int leader = __builtin_ctzll(m);
  int base         = 0;
  if (lane == leader) { base = atomicAdd(fill, __builtin_popcountll(m)); }
  base = __builtin_amdgcn_readlane(base, leader);
  return base + int(__builtin_amdgcn_mbcnt_hi(uint32_t(m >> 32),
                                               __builtin_amdgcn_mbcnt_lo(uint32_t(m), 0u)));
}

/** Elements per thread whose global loads a scan issues together. */
constexpr int kBatch = 8;

/** Order-preserving map of a signed 32-bit value onto an unsigned key (descending value). */
__device__ inline uint32_t desc_key(int32_t v) { return ~(uint32_t(v) ^ 0x80000000u); }
__device__ inline int32_t desc_value(uint32_t key) { return int32_t(~key ^ 0x80000000u); }

template <typename F>
__device__ uint32_t radix_select(int64_t n, int rank, F key_of, uint32_t lo, uint32_t hi, int* hist,
                                 int* wave_tot, uint32_t* sel_digit, int* sel_rank);

template <typename F>
__device__ void key_range(int64_t n, F key_of, uint32_t& lo, uint32_t& hi, int& below,
                          uint32_t* red);

constexpr int kCollect = 2048;  // keys of the selected first digit copied into LDS, at most

template <typename F>
__device__ uint32_t radix_select_collect(int64_t n, int rank, F key_of, uint32_t lo, uint32_t hi,
                                         int* hist, int* wave_tot, uint32_t* sel_digit,
                                         int* sel_rank, uint32_t* list, int* n_list);

__global__ __launch_bounds__(kThreads) void threshold_kernel(
  const int32_t* gmax, int64_t n_groups, int64_t nq, int k, int32_t* theta)
{
  __shared__ int hist[257];
  __shared__ int wave_tot[4];
  __shared__ uint32_t red[48];
  __shared__ uint32_t sel_digit;
  __shared__ int sel_rank;
  const int64_t q = blockIdx.x;
  const int tid   = threadIdx.x;
  if (q >= nq) {
    if (tid == 0) { theta[q] = kKeepNone; }
    return;
  }
  if (n_groups < k) {
    if (tid == 0) { theta[q] = kKeepAll; }
    return;
  }
  const int32_t* v = gmax + q * n_groups;
  auto key_of      = [&](int64_t e) { return desc_key(v[e]); };
  uint32_t lo, hi;
  int below;
  key_range(n_groups, key_of, lo, hi, below, red);
  // the k-th largest value: the k-th smallest descending key (0xffffffff is the lowest value)
  __shared__ uint32_t list[kCollect];
  __shared__ int n_list;
  const uint32_t key = k > below ? 0xffffffffu
                                 : radix_select_collect(n_groups, k, key_of, lo, hi, hist, wave_tot,
                                                        &sel_digit, &sel_rank, list, &n_list);
  if (tid == 0) {
    const int32_t t = desc_value(key);
    theta[q]        = t > kKeepAll ? t : kKeepAll;
  }
}

__global__ void max_kernel(const uint32_t* c, int64_t n, uint32_t* out)
{
  uint32_t m = 0;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * blockDim.x) {
    m = max(m, c[i]);
  }
  for (int off = 32; off; off >>= 1) { m = max(m, uint32_t(__shfl_xor(int(m), off))); }
  if ((threadIdx.x & 63) == 0) { atomicMax(out, m); }
}

__global__ void sum_kernel(const uint32_t* c, int64_t n, int64_t cap, unsigned long long* out)
{
  unsigned long long s = 0;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * blockDim.x) {
    s += c[i] < cap ? c[i] : uint64_t(cap);
  }
  for (int off = 32; off; off >>= 1) {
    s += (unsigned long long)__shfl_xor((long long)s, off);
  }
  if ((threadIdx.x & 63) == 0) { atomicAdd(out, s); }
}

// ---- exact scores --------------------------------------------------------------------------

/** Order-preserving map of a double onto a 64-bit key (ascending); -0 maps as +0. */
__device__ inline uint64_t score_key(double s)
{
  const uint64_t b = __double_as_longlong(s + 0.0);
  return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}
__device__ inline double key_score(uint64_t k)
{
  const uint64_t b = (k >> 63) ? (k & 0x7fffffffffffffffull) : ~k;
  return __longlong_as_double((long long)b);
}

/**
 * Result t (query q, place j: t = q k + j) as the caller receives it, the output conversion of
 * certex.cu:224-250 (finish): the distance of fp64 score s (smaller is better) as float32 (l2:
 * s; inner product: -s = <q, x>; cosine: 1 + s = 1 - cos) and the id; id < 0: a missing entry,
 * +inf (-inf for the inner product) and -1.
 */
template <typename A>
__device__ inline void put_result(const A& a, int64_t q, int j, double s, int64_t id)
{
  const int64_t t = (a.out_rows != nullptr ? int64_t(a.out_rows[q]) : q) * a.k + j;
  float d;
  if (id < 0) {
    d = a.metric == metric_kind::inner ? -INFINITY : INFINITY;
  } else if (a.metric == metric_kind::inner) {
    d = float(-s);
  } else if (a.metric == metric_kind::cosine) {
    d = float(1.0 + s);
  } else {
    d = float(s);
  }
  a.distances[t] = d;
  a.neighbors[t] = id < 0 ? -1 : id;
}

__device__ inline bool keeps(const filter_args& f, int64_t q, uint32_t row)
{
  if (f.kind == 0) { return true; }
  row = listed_id(f, row);
  switch (f.kind) {
    case 1: return (f.words[row >> 5] >> (row & 31)) & 1u;
    case 2: {
      const int64_t bit = (f.q0 + q) * f.bitmap_ld + row;
      return (f.words[bit >> 5] >> (bit & 31)) & 1u;
    }
    case 3: return f.row_labels[row] == f.query_labels[f.q0 + q];
    default: return true;
  }
}

typedef int v4i_t __attribute__((ext_vector_type(4)));

/**
 * Exact score of stored integer row `xrow` (row_bytes bytes, 16-byte aligned) against the query
 * codes in LDS, in int32. The codes are int8 (uint8 coordinates shifted by -128, bias = 128) and
 * zero past dim in both. For 8-bit data every fp64 partial sum of the oracle is an exact integer,
 * so this exact integer converts to the same double:
 *   l2:    sum (q - x)^2 = |q|^2 + |x|^2 - 2 <q, x>            (at most 255^2 * 256 < 2^31)
 *   inner: -sum (q + bias)(x + bias) = -(<q, x> + bias (sum q + sum x) + bias^2 dim)
 * qq = |q|^2 and qs = sum q of the query codes. Each 16-byte load feeds twelve v_dot4_i32_i8.
 */
__device__ inline double int_score(const int8_t* qv, const int8_t* base, int64_t r, bool paired,
                                   int row_bytes, int64_t dim, int bias, int qq, int qs,
                                   metric_kind metric)
{
  int qx = 0, xx = 0, xs = 0;
  // row r of `base`: contiguous, or in the paired layout (a wide label partition), where each
  // 16-byte chunk lies whole inside one 64-byte piece
  const int8_t* xrow = base + (paired ? (r >> 1) * 2 * int64_t(row_bytes) + (r & 1) * 64 : r * int64_t(row_bytes));
  for (int j = 0; j < row_bytes; j += 16) {
    const int jo   = paired ? (j >> 6) * 128 + (j & 63) : j;
    const v4i_t x  = *reinterpret_cast<const v4i_t*>(xrow + jo);
    const v4i_t qw = *reinterpret_cast<const v4i_t*>(qv + j);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      qx = __builtin_amdgcn_sdot4(qw[b], x[b], qx, false);
      xx = __builtin_amdgcn_sdot4(x[b], x[b], xx, false);
      xs = __builtin_amdgcn_sdot4(x[b], 0x01010101, xs, false);
    }
  }
  if (metric == metric_kind::l2) { return double(qq + xx - 2 * qx); }
  return -double(int64_t(qx) + int64_t(bias) * (qs + xs) + int64_t(bias) * bias * dim);
}

/** |q|^2 and sum q of the query codes in LDS (row_bytes bytes, zero past dim). */
__device__ inline void query_sums(const int8_t* qv, int row_bytes, int& qq, int& qs)
{
  qq = 0;
  qs = 0;
  for (int j = 0; j < row_bytes; j += 16) {
    const v4i_t qw = *reinterpret_cast<const v4i_t*>(qv + j);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      qq = __builtin_amdgcn_sdot4(qw[b], qw[b], qq, false);
      qs = __builtin_amdgcn_sdot4(qw[b], 0x01010101, qs, false);
    }
  }
}

constexpr int kBuf = 4096;  // LDS candidates per query (keys 32 KB + rows 16 KB)

/** Bitonic sort of key/row pairs [0, P) in LDS by (key, row); P a power of two. */
__device__ inline void bitonic_sort(uint64_t* key, uint32_t* row, int P)
{
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < (P >> 1); i += kThreads) {
        const int lo  = 2 * i - (i & (stride - 1));
        const int hi  = lo + stride;
        const bool up = (lo & size) == 0;
        const uint64_t ka = key[lo], kb = key[hi];
        const uint32_t ra = row[lo], rb = row[hi];
        const bool greater = ka > kb || (ka == kb && ra > rb);
        if (greater == up) {
          key[lo] = kb;
          key[hi] = ka;
          row[lo] = rb;
          row[hi] = ra;
        }
      }
      __syncthreads();
    }
  }
}

/** (ka, ra) comes before (kb, rb): ascending key, then ascending row. */
__device__ __forceinline__ bool pair_less(uint64_t ka, uint32_t ra, uint64_t kb, uint32_t rb)
{
  return ka < kb || (ka == kb && ra < rb);
}

/**
 * One compare-exchange stage (SIZE, STRIDE) of bitonic_sort over kThreads E pairs held E per
 * thread in registers, thread t holding positions t E .. t E + E - 1: within the thread for
 * STRIDE < E, by a cross-lane exchange for partners in the same wave (STRIDE < 64 E), else
 * through LDS (key / row, two barriers).
 */
template <int E, int SIZE, int STRIDE>
__device__ __forceinline__ void bitonic_stage_regs(uint64_t (&k)[E], uint32_t (&r)[E],
                                                   uint64_t* key, uint32_t* row)
{
  const int t = threadIdx.x;
  if constexpr (STRIDE < E) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      if ((e & STRIDE) == 0) {
        const int p     = e + STRIDE;
        const bool up   = ((t * E + e) & SIZE) == 0;
        const bool swap = up ? pair_less(k[p], r[p], k[e], r[e]) : pair_less(k[e], r[e], k[p], r[p]);
        const uint64_t ke = k[e], kp = k[p];
        const uint32_t re = r[e], rp = r[p];
        k[e] = swap ? kp : ke;
        k[p] = swap ? ke : kp;
        r[e] = swap ? rp : re;
        r[p] = swap ? re : rp;
      }
    }
  } else if constexpr (STRIDE < 64 * E) {
    constexpr int D  = STRIDE / E;  // partner lane distance
    const bool lower = (t & D) == 0;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const uint64_t ok  = __shfl_xor(k[e], D);
      const uint32_t orr = __shfl_xor(r[e], D);
      const bool up      = ((t * E + e) & SIZE) == 0;
      if (pair_less(k[e], r[e], ok, orr) != (lower == up)) {  // the lower one keeps the minimum
        k[e] = ok;                                             // going up
        r[e] = orr;
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      key[t * E + e] = k[e];
      row[t * E + e] = r[e];
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int g        = t * E + e;
      const uint64_t ok  = key[g ^ STRIDE];
      const uint32_t orr = row[g ^ STRIDE];
      const bool up      = (g & SIZE) == 0;
      if (pair_less(k[e], r[e], ok, orr) != (((g & STRIDE) == 0) == up)) {
        k[e] = ok;
        r[e] = orr;
      }
    }
    __syncthreads();
  }
}

template <int E, int SIZE, int STRIDE>
__device__ __forceinline__ void bitonic_strides_regs(uint64_t (&k)[E], uint32_t (&r)[E],
                                                     uint64_t* key, uint32_t* row)
{
  bitonic_stage_regs<E, SIZE, STRIDE>(k, r, key, row);
  if constexpr (STRIDE > 1) { bitonic_strides_regs<E, SIZE, STRIDE / 2>(k, r, key, row); }
}

template <int E, int SIZE>
__device__ __forceinline__ void bitonic_sizes_regs(uint64_t (&k)[E], uint32_t (&r)[E],
                                                   uint64_t* key, uint32_t* row)
{
  bitonic_strides_regs<E, SIZE, SIZE / 2>(k, r, key, row);
  if constexpr (SIZE < kThreads * E) { bitonic_sizes_regs<E, 2 * SIZE>(k, r, key, row); }
}

/**
 * bitonic_sort of exactly kThreads E pairs (the same network, the same result), the pairs held E
 * per thread in registers: of the 66 stages of 2,048 pairs only the 3 whose partners sit in
 * another wave go through LDS and barriers (every stage of the LDS sort takes a barrier).
 */
template <int E>
__device__ void bitonic_sort_regs(uint64_t* key, uint32_t* row)
{
  const int t = threadIdx.x;
  uint64_t k[E];
  uint32_t r[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    k[e] = key[t * E + e];
    r[e] = row[t * E + e];
  }
  __syncthreads();  // every pair is read before the cross-wave stages write
  bitonic_sizes_regs<E, 2>(k, r, key, row);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    key[t * E + e] = k[e];
    row[t * E + e] = r[e];
  }
  __syncthreads();
}

/** bitonic_sort; with REGS, the register form for 1,024 and 2,048 pairs (it takes about 130
 *  VGPRs, which a kernel pays at every phase). */
template <bool REGS>
__device__ inline void sort_pairs(uint64_t* key, uint32_t* row, int P)
{
  if constexpr (REGS) {
    if (P == 8 * kThreads) {
      bitonic_sort_regs<8>(key, row);
      return;
    }
    if (P == 4 * kThreads) {
      bitonic_sort_regs<4>(key, row);
      return;
    }
  }
  bitonic_sort(key, row, P);
}

__device__ inline int pow2_at_least(int v)
{
  int p = 1;
  while (p < v) { p <<= 1; }
  return p;
}

/**
 * The rank-th smallest (1-based, rank <= n) (key, row) pair of key/row[0, n) in LDS, the pairs
 * being distinct: an LDS radix select over the eight 8-bit digits of the key and, when several
 * pairs share the selected key and `with_row`, over the four digits of the row among them. Every
 * thread of the block calls it and gets the same pair. Scratch: hist[256], wave_tot[4], and three
 * LDS words.
 */
__device__ inline void select_pair(const uint64_t* key, const uint32_t* row, int n, int rank,
                                   bool with_row, int* hist, int* wave_tot, uint32_t* sel_digit,
                                   int* sel_rank, int* sel_count, uint64_t* out_key,
                                   uint32_t* out_row)
{
  const int tid = threadIdx.x;
  // the keys' range: the bits that the smallest and the largest share are shared by every key (the
  // best scores of a query lie close together) and need no pass, whose counts would all go to one
  // histogram bin; the select runs 8 bits at a time from the first differing bit down
  __shared__ uint64_t rng[2 * (kThreads / 64)];
  uint64_t lo = ~0ull, hi = 0;
  for (int e = tid; e < n; e += kThreads) {
    const uint64_t kk = key[e];
    lo                = kk < lo ? kk : lo;
    hi                = kk > hi ? kk : hi;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint64_t l = __shfl_xor(lo, off), h = __shfl_xor(hi, off);
    lo               = l < lo ? l : lo;
    hi               = h > hi ? h : hi;
  }
  if ((tid & 63) == 0) {
    rng[tid >> 6]                 = lo;
    rng[kThreads / 64 + (tid >> 6)] = hi;
  }
  __syncthreads();
  lo = rng[0];
  hi = rng[kThreads / 64];
  for (int w = 1; w < kThreads / 64; ++w) {
    lo = rng[w] < lo ? rng[w] : lo;
    hi = rng[kThreads / 64 + w] > hi ? rng[kThreads / 64 + w] : hi;
  }
  __syncthreads();
  int r           = lo == hi ? 0 : 64 - __builtin_clzll(lo ^ hi);  // bits below the common prefix
  uint64_t mask   = r == 64 ? 0ull : ~((uint64_t(1) << r) - 1);
  uint64_t prefix = lo & mask;
  if (r == 0 && tid == 0) { *sel_count = n; }  // every key is the selected one
  while (r > 0) {
    const int w       = r < 8 ? r : 8;
    const int shift   = r - w;
    const uint64_t dm = (uint64_t(1) << w) - 1;
    hist[tid] = 0;
    __syncthreads();
    for (int e = tid; e < n; e += kThreads) {
      const uint64_t kk = key[e];
      if ((kk & mask) == prefix) { atomicAdd(&hist[int((kk >> shift) & dm)], 1); }
    }
    __syncthreads();
    const int c    = hist[tid];
    const int incl = block_scan_incl(c, wave_tot);
    if (incl - c < rank && rank <= incl) {
      *sel_digit = uint32_t(tid);
      *sel_rank  = rank - (incl - c);
      *sel_count = c;
    }
    __syncthreads();
    prefix |= uint64_t(*sel_digit) << shift;
    mask |= dm << shift;
    rank = *sel_rank;
    r -= w;
    __syncthreads();
  }
  __syncthreads();
  *out_key = prefix;
  if (!with_row) { return; }
  const int same = *sel_count;  // pairs whose key is the selected one
  uint32_t rp = 0, rm = 0;
  if (same == 1) {
    for (int e = tid; e < n; e += kThreads) {
      if (key[e] == prefix) { *sel_digit = row[e]; }
    }
    __syncthreads();
    rp = *sel_digit;
    __syncthreads();
  } else {
    for (int shift = 24; shift >= 0; shift -= 8) {
      hist[tid] = 0;
      __syncthreads();
      for (int e = tid; e < n; e += kThreads) {
        const uint32_t rr = row[e];
        if (key[e] == prefix && (rr & rm) == rp) { atomicAdd(&hist[(rr >> shift) & 255], 1); }
      }
      __syncthreads();
      const int c    = hist[tid];
      const int incl = block_scan_incl(c, wave_tot);
      if (incl - c < rank && rank <= incl) {
        *sel_digit = uint32_t(tid);
        *sel_rank  = rank - (incl - c);
      }
      __syncthreads();
      rp |= *sel_digit << shift;
      rm |= 255u << shift;
      rank = *sel_rank;
      __syncthreads();
    }
  }
  *out_row = rp;
}

/** Pair counts up to which a bitonic sort replaces the radix select (fewer barriers). */
constexpr int kSortBelow = 512;

/**
 * Keeps the k best (key, row) pairs of [0, n), k <= n <= kBuf, in [0, k) of the same arrays (in
 * order after a sort of few pairs, else in no particular order), and returns the k-th smallest
 * key (which bounds the k-th score). With the select, the kept pairs are compacted in place, 4
 * pairs per thread at a time (all pairs of a thread in registers had taken 48 VGPRs, which bounded
 * the verify kernels' occupancy).
 */
__device__ inline uint64_t keep_k_best(uint64_t* key, uint32_t* row, int n, int k, int* hist,
                                       int* wave_tot, uint32_t* sel_digit, int* sel_rank,
                                       int* sel_count, int* fill)
{
  if (n <= kSortBelow) {  // few pairs: one bitonic sort costs fewer barriers than the select
    const int P = pow2_at_least(n);
    for (int j = n + threadIdx.x; j < P; j += kThreads) {
      key[j] = ~0ull;
      row[j] = ~0u;
    }
    __syncthreads();
    bitonic_sort(key, row, P);
    return key[k - 1];
  }
  __shared__ uint64_t kth_key;
  __shared__ uint32_t kth_row;
  select_pair(key, row, n, k, n > k, hist, wave_tot, sel_digit, sel_rank, sel_count, &kth_key,
              &kth_row);
  const uint64_t K = kth_key;
  if (n == k) { return K; }
  const uint32_t R = kth_row;
  // in place, in chunks of kPer entries per thread: a chunk is read whole (barrier) before any of
  // its kept entries is written, and the kept count never passes the entries read so far
  constexpr int kPer = 4;
  if (threadIdx.x == 0) { *fill = 0; }
  __syncthreads();
  for (int c0 = 0; c0 < n; c0 += kThreads * kPer) {
    uint64_t kk[kPer];
    uint32_t rr[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int e = c0 + threadIdx.x + i * kThreads;
      kk[i]       = e < n ? key[e] : ~0ull;
      rr[i]       = e < n ? row[e] : ~0u;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int e   = c0 + threadIdx.x + i * kThreads;
      const bool in = e < n && (kk[i] < K || (kk[i] == K && rr[i] <= R));
      const int s   = wave_append(in, fill);
      if (in) {
        key[s] = kk[i];
        row[s] = rr[i];
      }
    }
    __syncthreads();
  }
  return K;
}

__global__ __launch_bounds__(kThreads) void verify_topk_i8_kernel(verify_args a, int cap)
{
  extern __shared__ __attribute__((aligned(16))) unsigned char dyn[];
  auto* key = reinterpret_cast<uint64_t*>(dyn);                    // [cap]
  auto* rid = reinterpret_cast<uint32_t*>(dyn + size_t(cap) * 8);  // [cap]
  auto* qv  = reinterpret_cast<int8_t*>(dyn + size_t(cap) * 12);   // [row_bytes]
  __shared__ int fill;
  __shared__ int hist[256];
  __shared__ int wave_tot[4];
  __shared__ uint32_t sel_digit;
  __shared__ int sel_rank, sel_count, kept;

  const int64_t q = blockIdx.x;
  const int tid   = threadIdx.x;
  const int k     = a.k;
  for (int j = tid; j < a.row_bytes; j += kThreads) { qv[j] = a.qcodes[q * a.row_bytes + j]; }
  const int bias = a.flip ? 128 : 0;
  __syncthreads();  // the query codes are in LDS
  int qq, qs;
  query_sums(qv, a.row_bytes, qq, qs);

  const int64_t n_cand =
    a.all_rows ? a.n_rows : (a.cand_count[q] < a.cap ? int64_t(a.cand_count[q]) : a.cap);
  if (!a.all_rows && n_cand <= a.small_max) { return; }  // the one-wave kernel's query
  const uint32_t* cand = a.cand_rows + q * a.cap;

  int have = 0;  // entries [0, have) of the buffer hold the best candidates so far
  if (tid == 0) { fill = 0; }
  __syncthreads();
  for (int64_t c0 = 0; c0 < n_cand;) {
    // fill the buffer beyond `have` with the next candidates (compacted by an LDS counter)
    const int room  = cap - have;
    const int64_t m = n_cand - c0 < room ? n_cand - c0 : room;
    for (int64_t e = tid; e < m; e += kThreads) {
      // the candidate's stored row (or partition row), then its id
      uint32_t r;
      bool live;
      const int8_t* base = a.codes;
      if (a.all_rows) {
        r    = uint32_t(c0 + e);
        live = a.rowc[r] != kDeadRow && keeps(a.filter, q, r);
      } else {
        r    = cand[c0 + e];
        live = true;
      }
      uint32_t id;
      bool paired = false;
      if (!a.all_rows && a.part_ids != nullptr && r < a.n_part) {
        base   = a.part_codes;
        paired = a.part_paired;
        id     = uint32_t(a.part_ids[r]);
      } else {
        id = listed_id(a.filter, r);
      }
      if (live) {
        const double s =
          int_score(qv, base, r, paired, a.row_bytes, a.dim, bias, qq, qs, a.metric);
        const int slot = have + atomicAdd(&fill, 1);
        key[slot]      = score_key(s);
        rid[slot]      = id;
      }
    }
    c0 += m;
    __syncthreads();
    have += fill;
    __syncthreads();
    if (tid == 0) { fill = 0; }
    if (c0 < n_cand && have > k) {  // keep the k best, drop the rest
      (void)keep_k_best(key, rid, have, k, hist, wave_tot, &sel_digit, &sel_rank, &sel_count,
                        &kept);
      have = k;
    }
    __syncthreads();
  }
  if (have > k) {
    (void)keep_k_best(key, rid, have, k, hist, wave_tot, &sel_digit, &sel_rank, &sel_count, &kept);
    have = k;
  }
  const int P = pow2_at_least(have > 1 ? have : 1);
  for (int j = have + tid; j < P; j += kThreads) {
    key[j] = ~0ull;
    rid[j] = ~0u;
  }
  __syncthreads();
  sort_pairs<false>(key, rid, P);
  for (int j = tid; j < k; j += kThreads) {
    put_result(a, q, j, j < have ? key_score(key[j]) : 0.0, j < have ? int64_t(rid[j]) : -1);
  }
}


/** Candidates per query up to which the integer re-rank runs one wave per query. */
constexpr int kSmallBucket = 512;

/**
 * The integer re-rank for small buckets (at most kSmallBucket candidates, k <= 64): one wave per
 * query. Each lane scores up to kSmallBucket / 64 candidates into registers; then k rounds of a
 * wave minimum over (score key, id) emit the k best in order, with no LDS buffer and no barrier.
 * The output is the block kernel's: the k smallest (key, id) pairs, ascending, then +inf / -1.
 * Queries with larger buckets are left to the block kernel.
 */
__global__ __launch_bounds__(kThreads) void verify_topk_i8_small_kernel(verify_args a)
{
  // dynamic LDS: the query codes of the block's waves [kThreads / 64][row_bytes]
  extern __shared__ __attribute__((aligned(16))) int8_t qlds[];
  const int lane    = threadIdx.x & 63;
  const int wave    = threadIdx.x >> 6;
  const int64_t q   = int64_t(blockIdx.x) * (kThreads / 64) + wave;
  const bool live_q = q < a.nq;
  int8_t* qv        = qlds + wave * a.row_bytes;
  if (live_q) {
    for (int j = lane; j < a.row_bytes; j += 64) { qv[j] = a.qcodes[q * a.row_bytes + j]; }
  }
  __syncthreads();  // the query codes are in LDS (the block's only barrier)
  if (!live_q) { return; }
  int qq, qs;
  query_sums(qv, a.row_bytes, qq, qs);
  const int bias       = a.flip ? 128 : 0;
  const int64_t n_cand = a.cand_count[q] < a.cap ? int64_t(a.cand_count[q]) : a.cap;
  if (n_cand > kSmallBucket) { return; }
  const uint32_t* cand = a.cand_rows + q * a.cap;
  constexpr int NPL    = kSmallBucket / 64;  // candidates per lane
  uint64_t key[NPL];
  uint32_t rid[NPL];
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int64_t e = lane + 64 * i;
    key[i]          = ~0ull;
    rid[i]          = ~0u;
    if (e < n_cand) {
      const uint32_t r   = cand[e];
      const int8_t* base = a.codes;
      uint32_t id;
      bool paired = false;
      if (a.part_ids != nullptr && r < a.n_part) {
        base   = a.part_codes;
        paired = a.part_paired;
        id     = uint32_t(a.part_ids[r]);
      } else {
        id = listed_id(a.filter, r);
      }
      key[i] = score_key(int_score(qv, base, r, paired, a.row_bytes, a.dim, bias,
                                   qq, qs, a.metric));
      rid[i] = id;
    }
  }
  double my_s   = INFINITY;
  int64_t my_r  = -1;
  for (int j = 0; j < a.k; ++j) {
    uint64_t bk = key[0];
    uint32_t br = rid[0];
#pragma unroll
    for (int i = 1; i < NPL; ++i) {
      if (key[i] < bk || (key[i] == bk && rid[i] < br)) {
        bk = key[i];
        br = rid[i];
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const uint32_t lo = uint32_t(__shfl_xor(int(uint32_t(bk)), off));
      const uint32_t hi = uint32_t(__shfl_xor(int(uint32_t(bk >> 32)), off));
      const uint64_t ok = (uint64_t(hi) << 32) | lo;
      const uint32_t orr = uint32_t(__shfl_xor(int(br), off));
      if (ok < bk || (ok == bk && orr < br)) {
        bk = ok;
        br = orr;
      }
    }
    if (bk == ~0ull) { break; }  // every lane holds the same pair: fewer than k candidates
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      if (key[i] == bk && rid[i] == br) {
        key[i] = ~0ull;
        rid[i] = ~0u;
      }
    }
    if (lane == j) {
      my_s = key_score(bk);
      my_r = int64_t(br);
    }
  }
  if (lane < a.k) { put_result(a, q, lane, my_s, my_r); }
}

// ---- float vectors ---------------------------------------------------------------------------

__device__ inline double fcoord(const void* p, elem t, int64_t i)
{
  if (t == elem::bf16) { return double(static_cast<const __bf16*>(p)[i]); }
  return t == elem::f32 ? double(static_cast<const float*>(p)[i])
                        : double(static_cast<const _Float16*>(p)[i]);
}

/**
 * Coordinates j .. j + P - 1 of a stored row as doubles (zero past dim): one vector load when
 * `aligned` (dim a multiple of P, so that j is too), else one coordinate at a time.
 */
/**
 * Coordinates j .. j + P - 1 of stored row `row` as doubles, zero at and past dim. ALIGNED (dim a
 * multiple of P, so that j is too): one vector load, from a clamped position when j >= dim; else
 * one coordinate at a time, each from a clamped position. The loads are unconditional, so that a
 * row's loads are issued together rather than each behind a branch.
 */
template <typename T, int P, bool ALIGNED>
__device__ __forceinline__ void load_coords(const T* x, int64_t row, int64_t dim, int64_t j, double (&b)[P])
{
  if constexpr (ALIGNED) {
    const bool ok    = j < dim;
    const T* src     = x + row * dim + (ok ? j : dim - P);
    if constexpr (P == 1) {
      const double v = double(src[0]);
      b[0]           = ok ? v : 0.0;
    } else {
      typedef T tp __attribute__((ext_vector_type(P)));
      const tp v = *reinterpret_cast<const tp*>(src);
#pragma unroll
      for (int u = 0; u < P; ++u) { b[u] = ok ? double(v[u]) : 0.0; }
    }
  } else {
#pragma unroll
    for (int u = 0; u < P; ++u) {
      const bool ok  = j + u < dim;
      const double v = double(x[row * dim + (ok ? j + u : dim - 1)]);
      b[u]           = ok ? v : 0.0;
    }
  }
}

/**
 * Exact fp64 scores of stored rows against the query whose coordinates sit in LDS as doubles, in
 * the oracle's canonical order: 64 partial sums, partial p accumulating coordinates p, p + 64, ...
 * in increasing order with fused multiply-adds, combined by the xor butterfly (for off = 32 .. 1:
 * p[i] + p[i ^ off]). A row is scored by L lanes of a wave (a slot): lane g of the slot keeps the
 * P = 64 / L consecutive partials P g .. P g + P - 1, read with one vector load per 64
 * coordinates; the butterfly levels off >= P pair lane g with lane g ^ (off / P) and the levels
 * below P combine partials inside a lane, so every lane of the slot ends with the same bits. With
 * L < 64 a wave scores 64 / L rows at once, NR rows per slot, U 64-coordinate blocks per
 * iteration. l2: sum (q - x)^2; inner: -sum q x; cosine: -sum q x / sqrt(sum q^2 sum x^2).
 * The element type, the metric and the alignment are template parameters: the loop holds no
 * branch, and the loads of an iteration go out together.
 */
template <int L, int NR, typename T, metric_kind M, bool ALIGNED>
__device__ __forceinline__ void slot_scores(const double* qv, const T* x, const int64_t (&rows)[NR],
                                   int64_t dim, int g, double (&out)[NR])
{
  constexpr int P = 64 / L;            // partials per lane
  constexpr int U = 64 / L >= 2 ? 2 : 4;  // 64-coordinate blocks per iteration
  double acc[NR][P], xx[NR][P], qq[P];
#pragma unroll
  for (int u = 0; u < P; ++u) {
    qq[u] = 0;
#pragma unroll
    for (int r = 0; r < NR; ++r) { acc[r][u] = xx[r][u] = 0; }
  }
  for (int64_t j0 = int64_t(P) * g; j0 < dim; j0 += 64 * U) {
    double b[NR][U][P];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
#pragma unroll
      for (int v = 0; v < U; ++v) { load_coords<T, P, ALIGNED>(x, rows[r], dim, j0 + 64 * v, b[r][v]); }
    }
#pragma unroll
    for (int v = 0; v < U; ++v) {
#pragma unroll
      for (int u = 0; u < P; ++u) {
        const int64_t j = j0 + 64 * v + u;
        if (j < dim) {
          const double a = qv[j];
          if constexpr (M == metric_kind::cosine) { qq[u] = fma(a, a, qq[u]); }
#pragma unroll
          for (int r = 0; r < NR; ++r) {
            const double xv = b[r][v][u];
            if constexpr (M == metric_kind::l2) {
              const double d = a - xv;
              acc[r][u]      = fma(d, d, acc[r][u]);
            } else {
              acc[r][u] = fma(a, xv, acc[r][u]);
              if constexpr (M == metric_kind::cosine) { xx[r][u] = fma(xv, xv, xx[r][u]); }
            }
          }
        }
      }
    }
  }
  // butterfly levels off = 32 .. P across the lanes of the slot: partner lane g ^ (off / P)
#pragma unroll
  for (int lx = 32 / P; lx >= 1; lx >>= 1) {
#pragma unroll
    for (int u = 0; u < P; ++u) {
      if constexpr (M == metric_kind::cosine) { qq[u] += __shfl_xor(qq[u], lx); }
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        acc[r][u] += __shfl_xor(acc[r][u], lx);
        if constexpr (M == metric_kind::cosine) { xx[r][u] += __shfl_xor(xx[r][u], lx); }
      }
    }
  }
  // levels off < P inside the lane: partial u pairs with u ^ off
#pragma unroll
  for (int h = P / 2; h >= 1; h >>= 1) {
#pragma unroll
    for (int u = 0; u < P; ++u) {
      if (u & h) { continue; }
      qq[u] += qq[u | h];
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        acc[r][u] += acc[r][u | h];
        xx[r][u] += xx[r][u | h];
      }
    }
  }
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    if constexpr (M == metric_kind::l2) {
      out[r] = acc[r][0];
    } else if constexpr (M == metric_kind::inner) {
      out[r] = -acc[r][0];
    } else {
      out[r] = -acc[r][0] / sqrt(qq[0] * xx[r][0]);
    }
  }
}

/** score_rows_l for one element type, metric and alignment. */
template <int L, typename T, metric_kind M, bool ALIGNED>
__device__ __forceinline__ void score_rows_t(const double* qv, const T* x, int64_t dim, const uint32_t* rid,
                                    uint64_t* key, int from, int to)
{
  constexpr int NR   = 2;  // rows per slot (1, 3 and 4 measured slower at configs 3 and 4)
  constexpr int PER  = (64 / L) * NR;  // rows per wave at a time
  const int lane     = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g        = lane % L;
  const int slot     = lane / L;
  for (int e0 = from + wave * PER; e0 < to; e0 += PER * (kThreads / 64)) {
    int64_t rows[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int e = e0 + slot * NR + r;
      rows[r]     = int64_t(rid[e < to ? e : to - 1]);
    }
    double sc[NR];
    slot_scores<L, NR, T, M, ALIGNED>(qv, x, rows, dim, g, sc);
    if (g == 0) {
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const int e = e0 + slot * NR + r;
        if (e < to) { key[e] = score_key(sc[r]); }
      }
    }
  }
}

template <int L, typename T>
__device__ __forceinline__ void score_rows_m(const double* qv, const T* x, int64_t dim, metric_kind metric,
                                    const uint32_t* rid, uint64_t* key, int from, int to)
{
  constexpr int P    = 64 / L;
  const bool aligned = dim % P == 0;
  switch (metric) {
    case metric_kind::l2:
      aligned ? score_rows_t<L, T, metric_kind::l2, true>(qv, x, dim, rid, key, from, to)
              : score_rows_t<L, T, metric_kind::l2, false>(qv, x, dim, rid, key, from, to);
      break;
    case metric_kind::inner:
      aligned ? score_rows_t<L, T, metric_kind::inner, true>(qv, x, dim, rid, key, from, to)
              : score_rows_t<L, T, metric_kind::inner, false>(qv, x, dim, rid, key, from, to);
      break;
    default:
      aligned ? score_rows_t<L, T, metric_kind::cosine, true>(qv, x, dim, rid, key, from, to)
              : score_rows_t<L, T, metric_kind::cosine, false>(qv, x, dim, rid, key, from, to);
      break;
  }
}

/** Scores rid[from, to) into key[] (ordered keys) with slots of L lanes, NR rows per slot. */
template <int L>
__device__ __forceinline__ void score_rows_l(const double* qv, const void* vectors, elem t, int64_t dim,
                                    metric_kind metric, const uint32_t* rid, uint64_t* key,
                                    int from, int to)
{
  if (t == elem::f32) {
    score_rows_m<L>(qv, static_cast<const float*>(vectors), dim, metric, rid, key, from, to);
  } else if (t == elem::bf16) {
    score_rows_m<L>(qv, static_cast<const __bf16*>(vectors), dim, metric, rid, key, from, to);
  } else {
    score_rows_m<L>(qv, static_cast<const _Float16*>(vectors), dim, metric, rid, key, from, to);
  }
}

/**
 * Lanes per scored row for vectors of `dim` coordinates: 16 up to 128 coordinates, 32 up to 256,
 * whole waves above (the kernels that score rows are instantiated per width, so that each keeps
 * the registers and occupancy of its own width).
 */
inline int score_lanes(int64_t dim) { return dim <= 128 ? 16 : (dim <= 256 ? 32 : 64); }

/** The smallest power of two >= v (host side). */
inline int pow2_ge(int v)
{
  int p = 1;
  while (p < v) { p <<= 1; }
  return p;
}

/** LDS entries of the candidate buffers: a power of two between lo and kBuf covering want. */
inline int buffer_entries(int want, int lo)
{
  int p = lo;
  while (p < want && p < kBuf) { p <<= 1; }
  return p;
}

/** Order-preserving map of a float onto an unsigned key (ascending). */
__device__ inline uint32_t fkey(float f)
{
  const uint32_t b = __float_as_uint(f + 0.0f);
  return (b >> 31) ? ~b : (b | 0x80000000u);
}

constexpr int kMaxFloatDim = kMaxF16Halves;  // widest float vector

/** The float of an ascending key of fkey. */
__device__ inline float key_value(uint32_t k)
{
  return __uint_as_float((k >> 31) ? (k & 0x7fffffffu) : ~k);
}

/**
 * The certificate's per-query error terms of the fp16 screen: C = the operand rounding of every
 * pair (cross) plus the fp32 accumulation of its products (accum), from the query's |fp16(W)|,
 * |W - fp16(W)| (qscal) and the index's largest |fp16(Z)|, |Z - fp16(Z)| (maxima).
 */
__device__ inline double screen_error(const threshold_f_args& a, int64_t q)
{
  const double nw = a.qscal[3 * q + 1], ew = a.qscal[3 * q + 2];
  const double nz = a.maxima[0], ez = a.maxima[1];
  const double cross = ew * nz + nw * ez + ew * ez;  // operand rounding, all pairs
  const double accum = a.gamma * nw * nz;            // fp32 accumulation of the products
  return cross + accum;
}

/**
 * The screen threshold of a score bound U: every pair of query q whose exact score is <= U has a
 * screen value >= the returned float (rounded down), which is never below -FLT_MAX. With
 * C = screen_error: inner products t(U) = -U / alpha2 - C; l2 t(U) = (|W|^2 - U / alpha2) / 2 - C
 * (cosine: l2 on the unit vectors with U_l2 = 2 + 2 U); both less 1e-10 of their scale.
 */
__device__ inline float theta_of(double U, const threshold_f_args& a, int64_t q)
{
  const double aq = a.qscal[3 * q];
  double th, scale;
  if (a.metric == metric_kind::inner) {
    th    = -U / a.alpha2;
    scale = fabs(th);
  } else {
    const double u  = a.metric == metric_kind::cosine ? (2.0 + 2.0 * U) : U;
    const double ua = u / a.alpha2;
    th              = (aq - ua) / 2.0;
    scale           = fabs(aq) + fabs(ua);
  }
  const double t = th - screen_error(a, q) - 1e-10 * scale - 1e-30;
  float f        = float(t);
  if (double(f) > t) { f = nextafterf(f, -INFINITY); }
  return f > -FLT_MAX ? f : -FLT_MAX;
}

/**
 * An upper bound of the exact score of a pair of query q whose fp16 screen value is v (finite).
 * The fp32 accumulation and the operand rounding bound the screen value from above as they bound
 * it from below: acc <= <W, Z> + C + (row term), for inner products acc <= <W, Z> + C, so the
 * score -alpha2 <W, Z> <= alpha2 (C - v). For l2 the row term, -|Z|^2 / 2 scaled by (1 - 2 gamma
 * - 1e-10) and rounded up to fp32, exceeds -|Z|^2 / 2 by at most D = |Z|max^2 (1.5 gamma + 1e-7)
 * (with its own accumulation error), |Z|max <= max |fp16(Z)| + max |Z - fp16(Z)|; then
 * score / alpha2 = |W|^2 - 2 (<W, Z> - |Z|^2 / 2) <= |W|^2 - 2 (v - C - D). |W|^2 is stored
 * lowered by 1e-13 and rounded in its sum; the results carry a margin of 1e-12 of their scale for
 * the fp64 rounding of these expressions. Cosine: l2 on the unit vectors, U = (U_l2 - 2) / 2.
 */
__device__ inline double screen_upper_bound(float vf, const threshold_f_args& a, int64_t q)
{
  const double v = double(vf);
  const double C = screen_error(a, q);
  if (a.metric == metric_kind::inner) {
    return a.alpha2 * (C - v) + 1e-12 * a.alpha2 * (fabs(v) + C) + 1e-300;
  }
  const double zmax = a.maxima[0] + a.maxima[1];
  const double D    = zmax * zmax * (1.5 * a.gamma + 1e-7);
  const double aq   = a.qscal[3 * q] * (1.0 + 1e-11);
  const double y    = aq - 2.0 * v + 2.0 * (C + D);
  const double ub   = a.alpha2 * y + 1e-12 * a.alpha2 * (aq + 2.0 * fabs(v) + 2.0 * (C + D)) + 1e-300;
  if (a.metric == metric_kind::cosine) { return (ub - 2.0) / 2.0 + 1e-12 * (fabs(ub) + 2.0); }
  return ub;
}


/**
 * theta[q] for the fp16 screen, certified from screen values alone: the k-th largest finite
 * group maximum v_k of the anchor pass belongs to k distinct live rows, each with a screen value
 * >= v_k, and the certificate bounds the score of a pair with screen value v from above by
 * screen_upper_bound(v); so U = screen_upper_bound(v_k) bounds the k-th neighbour's score, and
 * theta = theta_of(U). Groups whose maximum is -inf (no live anchor) or +inf (a row beyond the
 * fp16 range, whose score has no bound) are not counted. -FLT_MAX (keep every live row) with fewer
 * than k counted groups; +inf for padding queries.
 */
__global__ __launch_bounds__(kThreads) void threshold_f16_cert_kernel(threshold_f_args a)
{
  __shared__ int hist[257];
  __shared__ int wave_tot[4];
  __shared__ uint32_t red[48];
  __shared__ uint32_t sel_digit;
  __shared__ int sel_rank;
  const int64_t q = blockIdx.x;
  const int tid   = threadIdx.x;
  if (q >= a.nq) {
    if (tid == 0) { a.theta[q] = INFINITY; }
    return;
  }
  const float* v = a.gmax + q * a.n_groups;
  // the k-th largest finite value: the k-th smallest of the descending keys ~fkey, the others
  // (0xffffffff) last; the range pass counts the finite ones
  auto key_of = [&](int64_t e) {
    const float x = v[e];
    return isfinite(x) ? ~fkey(x) : 0xffffffffu;
  };
  uint32_t lo, hi;
  int finite;
  key_range(a.n_groups, key_of, lo, hi, finite, red);
  if (finite < a.k) {
    // keep every live row: removed rows (screen value -inf) still fail
    if (tid == 0) {
      a.theta[q] = -FLT_MAX;
      if (a.ub != nullptr) { a.ub[q] = INFINITY; }
    }
    return;
  }
  __shared__ uint32_t list[kCollect];
  __shared__ int n_list;
  const uint32_t key = radix_select_collect(a.n_groups, a.k, key_of, lo, hi, hist, wave_tot,
                                            &sel_digit, &sel_rank, list, &n_list);
  if (tid == 0) {
    const double U = screen_upper_bound(key_value(~key), a, q);
    a.theta[q]     = theta_of(U, a, q);
    if (a.ub != nullptr) { a.ub[q] = U; }
  }
}


/**
 * A lower bound of the exact score of a pair whose fp16 screen value is v: the inverse of the
 * threshold map theta_of (a pair with score s has v >= t(s), where t(U) is the
 * threshold before rounding), with 20 times its relative slack and a margin for the fp64 rounding
 * of this expression. C = the query's cross and accumulation terms; aq = |W|^2 (lower bound).
 */
__device__ inline double screen_lower_bound(float v, double aq, double C, double alpha2,
                                            metric_kind metric)
{
  const double R = double(v) + C + 1e-30;
  if (metric == metric_kind::inner) {
    // t(U) = -U / alpha2 - C - 1e-10 |U / alpha2| - 1e-30
    return -alpha2 * (R + 2e-9 * fabs(R)) - 1e-12 * alpha2 * (fabs(R) + 1e-300);
  }
  // l2 on the (unit) vectors: t(U) = (aq - U / alpha2) / 2 - C - 1e-10 (aq + U / alpha2) - 1e-30
  const double y  = (aq * (1.0 - 2e-9) - 2.0 * R) / (1.0 + 2e-9);
  const double lb = alpha2 * y - 1e-12 * alpha2 * (fabs(aq) + 2.0 * fabs(R) + 1e-300);
  if (metric == metric_kind::cosine) { return (lb - 2.0) / 2.0 - 1e-12 * (fabs(lb) + 2.0); }
  return lb;
}

/** Testing only: the certificate's two bounds of every bucket entry (certificate_bounds). */
__global__ void certificate_bounds_kernel(threshold_f_args a, const uint32_t* count,
                                          const float* vals, int64_t cap, double* lb, double* ub)
{
  const int64_t q = blockIdx.y;
  if (q >= a.nq) { return; }
  const int64_t n = count[q] < uint64_t(cap) ? int64_t(count[q]) : cap;
  const double aq = a.qscal[3 * q];
  const double C  = screen_error(a, q);
  for (int64_t slot = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; slot < n;
       slot += int64_t(gridDim.x) * blockDim.x) {
    const float v       = vals[q * cap + slot];
    lb[q * cap + slot] = screen_lower_bound(v, aq, C, a.alpha2, a.metric);
    ub[q * cap + slot] = screen_upper_bound(v, a, q);
  }
}

/** Inclusive prefix sum over the T threads of a block of T = 64 (one wave), kThreads or 1024. */
template <int T>
__device__ inline int scan_incl_t(int v, int* wave_tot)
{
  static_assert(T == 64 || T == kThreads || T == 1024, "block shapes of the selects");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int t = __shfl_up(incl, off);
    if (lane >= off) { incl += t; }
  }
  if constexpr (T == 64) {
    return incl;
  } else {
    if (lane == 63) { wave_tot[wave] = incl; }
    __syncthreads();
    int add = 0;
    for (int w = 0; w < wave; ++w) { add += wave_tot[w]; }
    __syncthreads();
    return incl + add;
  }
}

/** The minimum, the maximum and the sum of (lo, hi, n) over the T threads of a block; every
 *  thread gets them. red: 3 * 16 LDS words. */
template <int T>
__device__ inline void block_min_max_sum(uint32_t& lo, uint32_t& hi, int& n, uint32_t* red)
{
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint32_t l = __shfl_xor(lo, off), h = __shfl_xor(hi, off);
    const int c      = __shfl_xor(n, off);
    lo               = l < lo ? l : lo;
    hi               = h > hi ? h : hi;
    n += c;
  }
  if constexpr (T > 64) {
    constexpr int W = T / 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
      red[wave]      = lo;
      red[16 + wave] = hi;
      red[32 + wave] = uint32_t(n);
    }
    __syncthreads();
    lo = red[0];
    hi = red[16];
    n  = int(red[32]);
    for (int w = 1; w < W; ++w) {
      lo = red[w] < lo ? red[w] : lo;
      hi = red[16 + w] > hi ? red[16 + w] : hi;
      n += int(red[32 + w]);
    }
    __syncthreads();
  }
}

/**
 * The smallest key lo, the largest key hi below 0xffffffff and the number of keys below
 * 0xffffffff among key_of(e), e < n, over the block (every thread gets them); red: 48 LDS words.
 */
template <typename F>
__device__ void key_range(int64_t n, F key_of, uint32_t& lo, uint32_t& hi, int& below, uint32_t* red)
{
  lo    = 0xffffffffu;
  hi    = 0;
  below = 0;
  for (int64_t e0 = 0; e0 < n; e0 += int64_t(kThreads) * kBatch) {
    uint32_t kk[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int64_t e = e0 + i * kThreads + threadIdx.x;
      kk[i]           = key_of(e < n ? e : n - 1);
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      if (e0 + i * kThreads + threadIdx.x < n) {
        lo = kk[i] < lo ? kk[i] : lo;
        if (kk[i] != 0xffffffffu) {
          hi = kk[i] > hi ? kk[i] : hi;
          ++below;
        }
      }
    }
  }
  block_min_max_sum<kThreads>(lo, hi, below, red);
}

/** The state of an LDS radix select: the bits fixed so far (prefix under mask), the bits below
 *  them (r), and the rank still sought among the keys that share the prefix. */
struct radix_state {
  uint32_t prefix, mask;
  int r, rank;
};

/** The select's start: every key in [lo, hi] shares the bits above the first one where lo and hi
 *  differ. */
__device__ inline radix_state radix_start(uint32_t lo, uint32_t hi, int rank)
{
  radix_state st;
  st.r      = lo == hi ? 0 : 32 - __builtin_clz(lo ^ hi);
  st.mask   = st.r == 32 ? 0u : ~((1u << st.r) - 1u);
  st.prefix = lo & st.mask;
  st.rank   = rank;
  return st;
}

/**
 * One digit of the select (the top 8 of the r bits left, or all of them): an LDS histogram of
 * that digit over the keys key_of(e), e < n, that share the prefix, and the digit that holds the
 * rank. Returns how many keys share the longer prefix. Every thread of the block calls it.
 */
template <typename F>
__device__ int radix_pass(int64_t n, F key_of, radix_state& st, int* hist, int* wave_tot,
                          uint32_t* sel_digit, int* sel_rank)
{
  const int tid     = threadIdx.x;
  const int w       = st.r < 8 ? st.r : 8;
  const int shift   = st.r - w;
  const uint32_t dm = (1u << w) - 1u;
  hist[tid]         = 0;
  __syncthreads();
  int cur = -1, run_n = 0;  // a run of keys in one bin adds up before one atomic
  for (int64_t e0 = 0; e0 < n; e0 += int64_t(kThreads) * kBatch) {
    uint32_t kk[kBatch];  // loads first (from clamped positions), then the counts
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int64_t e = e0 + i * kThreads + tid;
      kk[i]           = key_of(e < n ? e : n - 1);
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      if (e0 + i * kThreads + tid < n && (kk[i] & st.mask) == st.prefix) {
        const int d = int((kk[i] >> shift) & dm);
        if (d == cur) {
          ++run_n;
        } else {
          if (run_n > 0) { atomicAdd(&hist[cur], run_n); }
          cur   = d;
          run_n = 1;
        }
      }
    }
  }
  if (run_n > 0) { atomicAdd(&hist[cur], run_n); }
  __syncthreads();
  const int c    = hist[tid];
  const int incl = block_scan_incl(c, wave_tot);
  if (incl - c < st.rank && st.rank <= incl) {
    *sel_digit = uint32_t(tid);
    *sel_rank  = st.rank - (incl - c);
    hist[256]  = c;  // the digit's count (one word past the histogram)
  }
  __syncthreads();
  st.prefix |= *sel_digit << shift;
  st.mask |= dm << shift;
  st.rank = *sel_rank;
  st.r -= w;
  const int count = hist[256];
  __syncthreads();
  return count;
}

/**
 * The rank-th smallest (1-based) of the 32-bit keys key_of(e), e < n, given their range: lo the
 * smallest key, hi the largest below 0xffffffff, and rank at most the number of keys below
 * 0xffffffff. An LDS radix select, 8 bits at a time from the top of the bits below the common
 * prefix of lo and hi (every key in between shares that prefix; a key 0xffffffff that shares it
 * sorts last and leaves the rank-th unchanged). Every thread of the block calls it and gets the
 * same key. hist holds 257 words.
 */
template <typename F>
__device__ uint32_t radix_select(int64_t n, int rank, F key_of, uint32_t lo, uint32_t hi, int* hist,
                                 int* wave_tot, uint32_t* sel_digit, int* sel_rank)
{
  radix_state st = radix_start(lo, hi, rank);
  while (st.r > 0) { (void)radix_pass(n, key_of, st, hist, wave_tot, sel_digit, sel_rank); }
  return st.prefix;
}

/**
 * radix_select for large n (a long row of a table in memory): after the first digit that leaves
 * at most kCollect keys sharing the prefix, one more pass copies them into list (LDS) and the
 * other digits read them there instead of all n keys, which saves the row's reads of the digits
 * after it. The same key as radix_select.
 */
template <typename F>
__device__ uint32_t radix_select_collect(int64_t n, int rank, F key_of, uint32_t lo, uint32_t hi,
                                         int* hist, int* wave_tot, uint32_t* sel_digit,
                                         int* sel_rank, uint32_t* list, int* n_list)
{
  radix_state st = radix_start(lo, hi, rank);
  if (st.r == 0) { return st.prefix; }
  int count = radix_pass(n, key_of, st, hist, wave_tot, sel_digit, sel_rank);
  while (st.r > 0 && count > kCollect) {
    count = radix_pass(n, key_of, st, hist, wave_tot, sel_digit, sel_rank);
  }
  if (st.r > 0) {
    const int tid = threadIdx.x;
    if (tid == 0) { *n_list = 0; }
    __syncthreads();
    for (int64_t e0 = 0; e0 < n; e0 += int64_t(kThreads) * kBatch) {
      uint32_t kk[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int64_t e = e0 + i * kThreads + tid;
        kk[i]           = key_of(e < n ? e : n - 1);
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const bool take = e0 + i * kThreads + tid < n && (kk[i] & st.mask) == st.prefix;
        const int slot  = wave_append(take, n_list);
        if (take) { list[slot] = kk[i]; }
      }
    }
    __syncthreads();
    const int nl = *n_list;  // = count
    auto key_at  = [&](int64_t e) { return list[e]; };
    while (st.r > 0) { (void)radix_pass(nl, key_at, st, hist, wave_tot, sel_digit, sel_rank); }
  }
  return st.prefix;
}

/**
 * The rank-th smallest (1-based) of the keys that the T threads of a block hold in registers,
 * VPT each (0xffffffff past the table, which sorts last and leaves every rank up to the number of
 * smaller keys unchanged): the LDS radix select of radix_select, reading the keys once from global
 * memory instead of once per digit. The bits that the smallest key and the largest key below
 * 0xffffffff share are shared by every key in between and are skipped: a query's group maxima lie
 * close together, and a first digit among those bits sends every count to one histogram bin.
 * The rest is selected 8 bits at a time from the top. Every thread gets the key.
 */
template <int T, int VPT>
__device__ uint32_t radix_select_regs(const uint32_t (&kk)[VPT], int rank, int* hist, int* wave_tot,
                                      uint32_t* red, uint32_t* sel_digit, int* sel_rank)
{
  constexpr int BPT = 256 / T > 0 ? 256 / T : 1;  // histogram bins per thread in the scan
  const int tid     = threadIdx.x;
  uint32_t lo = 0xffffffffu, hi = 0;
  int below = 0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    lo = kk[i] < lo ? kk[i] : lo;
    if (kk[i] != 0xffffffffu) {
      hi = kk[i] > hi ? kk[i] : hi;
      ++below;
    }
  }
  block_min_max_sum<T>(lo, hi, below, red);
  if (rank > below) { return 0xffffffffu; }
  if (lo == hi) { return lo; }
  int r           = 32 - __builtin_clz(lo ^ hi);  // bits below the common prefix
  uint32_t mask   = r == 32 ? 0u : ~((1u << r) - 1u);
  uint32_t prefix = lo & mask;
  while (r > 0) {
    const int w       = r < 8 ? r : 8;
    const int shift   = r - w;
    const uint32_t dm = (1u << w) - 1u;
    if (tid * BPT < 256) {
#pragma unroll
      for (int j = 0; j < BPT; ++j) { hist[tid * BPT + j] = 0; }
    }
    __syncthreads();
    // a thread's keys that fall into the bin of its previous key add up before one atomic: the
    // group maxima of a query crowd into few bins, where every key's own atomic serialised
    int cur = -1, run_n = 0;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      if ((kk[i] & mask) == prefix) {
        const int d = int((kk[i] >> shift) & dm);
        if (d == cur) {
          ++run_n;
        } else {
          if (run_n > 0) { atomicAdd(&hist[cur], run_n); }
          cur   = d;
          run_n = 1;
        }
      }
    }
    if (run_n > 0) { atomicAdd(&hist[cur], run_n); }
    __syncthreads();
    int c[BPT], sum = 0;
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
      c[j] = tid * BPT < 256 ? hist[tid * BPT + j] : 0;
      sum += c[j];
    }
    int run = scan_incl_t<T>(sum, wave_tot) - sum;
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
      if (run < rank && rank <= run + c[j]) {
        *sel_digit = uint32_t(tid * BPT + j);
        *sel_rank  = rank - run;
      }
      run += c[j];
    }
    __syncthreads();
    prefix |= *sel_digit << shift;
    mask |= dm << shift;
    rank = *sel_rank;
    r -= w;
    __syncthreads();
  }
  return prefix;
}

/** threshold_kernel with the query's group maxima read once into registers (n_groups <= T VPT). */
template <int T, int VPT>
__global__ __launch_bounds__(T) void threshold_regs_kernel(const int32_t* gmax, int64_t n_groups,
                                                           int64_t nq, int k, int32_t* theta)
{
  __shared__ int hist[256];
  __shared__ int wave_tot[16];
  __shared__ uint32_t red[48];
  __shared__ uint32_t sel_digit;
  __shared__ int sel_rank;
  const int64_t q = blockIdx.x;
  const int tid   = threadIdx.x;
  if (q >= nq) {
    if (tid == 0) { theta[q] = kKeepNone; }
    return;
  }
  if (n_groups < k) {
    if (tid == 0) { theta[q] = kKeepAll; }
    return;
  }
  const int32_t* v = gmax + q * n_groups;
  uint32_t kk[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int64_t e = int64_t(i) * T + tid;
    kk[i]           = e < n_groups ? desc_key(v[e]) : 0xffffffffu;
  }
  const uint32_t key = radix_select_regs<T, VPT>(kk, k, hist, wave_tot, red, &sel_digit, &sel_rank);
  if (tid == 0) {
    const int32_t t = desc_value(key);
    theta[q]        = t > kKeepAll ? t : kKeepAll;
  }
}

/** threshold_f16_cert_kernel with the query's group maxima read once into registers
 *  (n_groups <= T VPT); the count of finite groups comes from the same registers. */
template <int T, int VPT>
__global__ __launch_bounds__(T) void threshold_f16_cert_regs_kernel(threshold_f_args a)
{
  __shared__ int hist[256];
  __shared__ int wave_tot[16];
  __shared__ uint32_t red[48];
  __shared__ uint32_t sel_digit;
  __shared__ int sel_rank;
  const int64_t q = blockIdx.x;
  const int tid   = threadIdx.x;
  if (q >= a.nq) {
    if (tid == 0) { a.theta[q] = INFINITY; }
    return;
  }
  const float* v = a.gmax + q * a.n_groups;
  uint32_t kk[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int64_t e = int64_t(i) * T + tid;
    const float x   = e < a.n_groups ? v[e] : INFINITY;
    kk[i]           = isfinite(x) ? ~fkey(x) : 0xffffffffu;
  }
  // non-finite groups map to 0xffffffff: the select returns it when fewer than k are finite
  const uint32_t key = radix_select_regs<T, VPT>(kk, a.k, hist, wave_tot, red, &sel_digit, &sel_rank);
  if (tid != 0) { return; }
  if (key == 0xffffffffu) {
    a.theta[q] = -FLT_MAX;  // keep every live row: removed rows (screen value -inf) still fail
    if (a.ub != nullptr) { a.ub[q] = INFINITY; }
  } else {
    const double U = screen_upper_bound(key_value(~key), a, q);
    a.theta[q]     = theta_of(U, a, q);
    if (a.ub != nullptr) { a.ub[q] = U; }
  }
}

/** Launches K<T, VPT> for the smallest register shape holding n keys per query, one block per
 *  query; false when n exceeds the largest shape (the streaming kernel then runs). */
template <template <int, int> class L, typename... Args>
bool launch_select_regs(int64_t n, unsigned blocks, hipStream_t stream, Args... args)
{
  if (n <= 64 * 8) { L<64, 8>::go(blocks, stream, args...); return true; }
  if (n <= 64 * 16) { L<64, 16>::go(blocks, stream, args...); return true; }
  if (n <= kThreads * 8) { L<kThreads, 8>::go(blocks, stream, args...); return true; }
  if (n <= kThreads * 16) { L<kThreads, 16>::go(blocks, stream, args...); return true; }
  if (n <= kThreads * 72) { L<kThreads, 72>::go(blocks, stream, args...); return true; }
  return false;  // larger tables: the streaming kernels
}

template <int T, int VPT>
struct threshold_regs_launch {
  static void go(unsigned blocks, hipStream_t stream, const int32_t* gmax, int64_t n_groups,
                 int64_t nq, int k, int32_t* theta)
  {
    threshold_regs_kernel<T, VPT><<<blocks, T, 0, stream>>>(gmax, n_groups, nq, k, theta);
  }
};

template <int T, int VPT>
struct threshold_f_regs_launch {
  static void go(unsigned blocks, hipStream_t stream, const threshold_f_args& a)
  {
    threshold_f16_cert_regs_kernel<T, VPT><<<blocks, T, 0, stream>>>(a);
  }
};

/**
 * Exact re-rank of one query's survivors, one block per query. With screen values (fp16 rows),
 * the verification is ordered (the reference's verify_rounds, detail/verify.cuh:371-487): first
 * the k survivors with the largest screen values are scored, which bounds the k-th neighbour's
 * score by U; then only the survivors whose screen lower bound does not exceed U are scored
 * (U tightens as better rows arrive). Scores use one wave per row; the best k by (score, row)
 * stay in LDS. With 64-lane slots (d above 256) eight waves per SIMD, as many blocks as the LDS of a
 * CU holds at config 3 (18 spilled registers; against six waves per SIMD, verify 0.82 -> 0.79 ms).
 */
template <int L>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(L == 64 ? 8 : 4)))
void verify_topk_f_kernel(verify_f_args a, int cap)
{
  extern __shared__ __attribute__((aligned(16))) unsigned char dyn[];
  auto* key = reinterpret_cast<uint64_t*>(dyn);                 // [cap]
  auto* rid = reinterpret_cast<uint32_t*>(dyn + size_t(cap) * 8);  // [cap]
  auto* qv  = reinterpret_cast<double*>(dyn + size_t(cap) * 12);  // [dim]
  __shared__ int hist[257];
  __shared__ int wave_tot[4];
  __shared__ uint32_t red[48];
  __shared__ uint32_t sel_digit;
  __shared__ int sel_rank;
  __shared__ int sel_count;
  __shared__ int fill;
  // survivors whose screen values phase A selects in registers, 24 per thread; not with 64-lane
  // slots (d above 256), whose waves leave no registers to spare (16 per thread at six waves per
  // SIMD measured 4% slower than the streaming select, config 3)
  constexpr bool REGS = L != 64;
  constexpr int RV    = 24;

  const int64_t q = blockIdx.x;
  const int tid   = threadIdx.x;
  const int k     = a.k;
  const int64_t qr = a.query_rows != nullptr ? int64_t(a.query_rows[q]) : q;
  for (int64_t j = tid; j < a.dim; j += kThreads) { qv[j] = fcoord(a.queries, a.t, qr * a.dim + j); }

  const int64_t n_cand =
    a.all_rows ? a.n_rows : (a.cand_count[q] < a.cap ? int64_t(a.cand_count[q]) : a.cap);
  const uint32_t* cand = a.cand_rows + q * a.cap;
  const float* vals    = (a.all_rows || a.cand_vals == nullptr) ? nullptr : a.cand_vals + q * a.cap;

  auto to_id = [&](uint32_t r) {
    return (a.part_ids != nullptr && r < a.n_part) ? uint32_t(a.part_ids[r])
                                                   : listed_id(a.filter, r);
  };
  int64_t n_scored = 0;
  auto score       = [&](int from, int to) {
    n_scored += to - from;
    score_rows_l<L>(qv, a.vectors, a.t, a.dim, a.metric, rid, key, from, to);
  };
  int have = 0;  // entries [0, have) of key / rid are scored
  // the k best so far move to [0, k) (unordered); the k-th key bounds the k-th score. With
  // exactly k entries the k-th key is their largest, and nothing moves
  __shared__ uint64_t wave_max[kThreads / 64];
  uint64_t kth = ~0ull;
  auto keep_best = [&]() {
    if (have < k) { return; }
    kth  = have == k ? block_max_key(key, k, wave_max)
                     : keep_k_best(key, rid, have, k, hist, wave_tot, &sel_digit, &sel_rank,
                                   &sel_count, &fill);
    have = k;
  };

  // phase A: the survivors whose screen value is at least the k-th largest (descending keys)
  bool ordered = vals != nullptr && n_cand > k;
  uint32_t tk  = 0;
  double U = INFINITY, aq = 0, C = 0;
  if (REGS && ordered && n_cand <= int64_t(kThreads) * RV) {
    // the survivors' screen values read once into registers (RV per thread; 0xffffffff past the
    // bucket sorts last), selected there, and the k best collected from the same registers
    uint32_t kk[RV];
#pragma unroll
    for (int i = 0; i < RV; ++i) {
      const int64_t e = int64_t(i) * kThreads + tid;
      kk[i]           = e < n_cand ? ~fkey(vals[e]) : 0xffffffffu;
    }
    tk = radix_select_regs<kThreads, RV>(kk, k, hist, wave_tot, red, &sel_digit, &sel_rank);
    if (tid == 0) { fill = 0; }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < RV; ++i) {
      const int64_t e = int64_t(i) * kThreads + tid;
      const bool take = e < n_cand && kk[i] <= tk;
      const int slot  = wave_append(take, &fill);
      if (take && slot < cap) { rid[slot] = to_id(cand[e]); }
    }
    __syncthreads();
  } else if (ordered) {
    // the survivors' screen values lie close together above theta: the select starts below the
    // bits they share (all finite or +inf, so every key is below 0xffffffff)
    auto key_of = [&](int64_t e) { return ~fkey(vals[e]); };
    uint32_t lo, hi;
    int below;
    key_range(n_cand, key_of, lo, hi, below, reinterpret_cast<uint32_t*>(hist));
    tk = k <= below ? radix_select(n_cand, k, key_of, lo, hi, hist, wave_tot, &sel_digit, &sel_rank)
                    : radix_select(n_cand, k, key_of, 0u, 0xfffffffeu, hist, wave_tot, &sel_digit, &sel_rank);
    if (tid == 0) { fill = 0; }
    __syncthreads();
    for (int64_t e0 = 0; e0 < n_cand; e0 += int64_t(kThreads) * kBatch) {
      float v[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int64_t e = e0 + i * kThreads + tid;
        v[i]            = vals[e < n_cand ? e : n_cand - 1];
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int64_t e = e0 + i * kThreads + tid;
        const bool take = e < n_cand && ~fkey(v[i]) <= tk;
        const int slot  = wave_append(take, &fill);
        if (take && slot < cap) { rid[slot] = to_id(cand[e]); }
      }
    }
    __syncthreads();
  }
  if (ordered) {
    const int c = fill;
    __syncthreads();
    if (c <= cap) {
      have = c;
      score(0, c);
      __syncthreads();
      keep_best();
      U                = key_score(kth);  // k distinct live rows: bounds the k-th score
      const double nw  = a.qscal[3 * q + 1], ew = a.qscal[3 * q + 2];
      const double nz  = a.maxima[0], ez = a.maxima[1];
      aq               = a.qscal[3 * q];
      C                = a.gamma * nw * nz + ew * nz + nw * ez + ew * ez;
    } else {
      ordered = false;  // more ties at the k-th screen value than the buffer holds: score all
    }
  }

  // phase B: the rest (everything when not ordered), in chunks of at most the buffer's free
  // room. A cut back to the k best (which also tightens U) is a select over the whole buffer: it
  // runs once the rows scored past the k best come to k / 8 (U then moves enough to save
  // scores), or when the free room falls below a quarter of the buffer. The ordered scan keeps
  // few candidates (those whose lower bound reaches U), so its chunk spans the whole rest of
  // them: a chunk no longer than the room would cost one round of barriers and loads per room's
  // worth of candidates (1,024 at k = 2,048). When it keeps more than the room holds, that chunk
  // is scanned again at the room's size, and so is every chunk after it.
  int pending = have;  // entries [pending, have) are appended and not scored yet
  bool wide   = ordered;
  for (int64_t c0 = 0; c0 < n_cand;) {
    const int room  = cap - have;
    const int64_t m = wide || n_cand - c0 < room ? n_cand - c0 : room;
    if (tid == 0) { fill = 0; }
    __syncthreads();
    for (int64_t e0 = 0; e0 < m; e0 += int64_t(kThreads) * kBatch) {
      bool take[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int64_t e   = e0 + i * kThreads + tid;
        const int64_t idx = c0 + (e < m ? e : m - 1);  // loads from clamped positions
        if (a.all_rows) {
          take[i] = a.rowc[idx] != -INFINITY && keeps(a.filter, q, uint32_t(idx));
        } else if (ordered) {
          const float v = vals[idx];
          take[i] = ~fkey(v) > tk && screen_lower_bound(v, aq, C, a.alpha2, a.metric) <= U;
        } else {
          take[i] = true;
        }
        take[i] = take[i] && e < m;
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int slot = wave_append(take[i], &fill);
        if (take[i] && slot < room) {
          const int64_t idx = c0 + e0 + i * kThreads + tid;
          rid[have + slot]  = a.all_rows ? listed_id(a.filter, uint32_t(idx)) : to_id(cand[idx]);
        }
      }
    }
    __syncthreads();
    const int added = fill;
    __syncthreads();  // every thread has read fill before the next chunk resets it
    if (added > room) {  // more kept than the room holds: this chunk again, at the room's size
      wide = false;
      continue;
    }
    have += added;
    c0 += m;
    // a scoring round costs a memory latency even for one row: score once the buffer runs short
    // of room or the scan ends (U tightens only through scored rows)
    if (c0 >= n_cand || cap - have < cap / 4) {
      score(pending, have);
      pending = have;
      __syncthreads();
      if (have > k && c0 < n_cand && (8 * (have - k) >= k || cap - have < cap / 4)) {
        keep_best();
        pending = have;
        if (ordered) { U = key_score(kth); }
      }
    }
  }
  {  // the final k in (score, row) order: one sort of all entries when they are few (the best
     // k come first), else a cut back to the k best and a sort of those
    if (have > kSortBelow) { keep_best(); }
    const int P = pow2_at_least(have > 1 ? have : 1);
    for (int j = have + tid; j < P; j += kThreads) {
      key[j] = ~0ull;
      rid[j] = ~0u;
    }
    __syncthreads();
    sort_pairs<L == 16>(key, rid, P);
    have = have < k ? have : k;
  }
  for (int j = tid; j < k; j += kThreads) {
    put_result(a, q, j, j < have ? key_score(key[j]) : 0.0, j < have ? int64_t(rid[j]) : -1);
  }
  if (a.scored != nullptr && tid == 0) { atomicAdd(a.scored, (unsigned long long)n_scored); }
}


}  // namespace

void threshold_i8(const int32_t* gmax, int64_t n_groups, int64_t nq, int64_t nq_pad, int k,
                  int32_t* theta, hipStream_t stream)
{
  if (nq_pad == 0) { return; }
  if (launch_select_regs<threshold_regs_launch>(n_groups, unsigned(nq_pad), stream, gmax, n_groups,
                                                nq, k, theta)) {
    return;
  }
  threshold_kernel<<<unsigned(nq_pad), kThreads, 0, stream>>>(gmax, n_groups, nq, k, theta);
}

void max_u32(const uint32_t* count, int64_t n, uint32_t* out, hipStream_t stream)
{
  const int64_t blocks = (n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024;
  if (blocks > 0) { max_kernel<<<unsigned(blocks), 256, 0, stream>>>(count, n, out); }
}

void sum_u32(const uint32_t* count, int64_t n, int64_t cap, unsigned long long* out,
             hipStream_t stream)
{
  const int64_t blocks = (n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024;
  if (blocks > 0) { sum_kernel<<<unsigned(blocks), 256, 0, stream>>>(count, n, cap, out); }
}

void verify_topk_i8(const verify_args& a, hipStream_t stream)
{
  if (a.nq == 0) { return; }
  verify_args b = a;
  b.small_max   = -1;
  if (!a.all_rows && a.k <= 64) {
    // buckets of up to kSmallBucket candidates: one wave per query; the block kernel then takes
    // only the larger buckets (launched when the host saw one)
    verify_topk_i8_small_kernel<<<unsigned((a.nq + 3) / 4), kThreads,
                                  size_t(kThreads / 64) * size_t(a.row_bytes), stream>>>(a);
    if (a.max_cand >= 0 && a.max_cand <= kSmallBucket) { return; }
    b.small_max = kSmallBucket;
  }
  // room for 2 k candidates (at least 1,024): small k keeps the block's LDS small, so that many
  // blocks share a CU
  int cap = pow2_ge(2 * a.k);
  cap     = cap > 1024 ? (cap < kBuf ? cap : kBuf) : 1024;
  const size_t bytes = size_t(cap) * 12 + size_t(a.row_bytes);
  verify_topk_i8_kernel<<<unsigned(a.nq), kThreads, bytes, stream>>>(b, cap);
}

/** Launches a kernel with `bytes` of dynamic LDS (raising the kernel's limit when needed). */
template <typename K, typename... Args>
void launch_dyn(K kernel, unsigned blocks, size_t bytes, hipStream_t stream, Args... args)
{
  if (bytes > 65536 && hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           int(bytes)) != hipSuccess) {
    (void)hipGetLastError();
  }
  kernel<<<blocks, kThreads, bytes, stream>>>(args...);
}

void threshold_f16(const threshold_f_args& a, hipStream_t stream)
{
  if (a.nq_pad == 0) { return; }
  if (launch_select_regs<threshold_f_regs_launch>(a.n_groups, unsigned(a.nq_pad), stream, a)) {
    return;
  }
  threshold_f16_cert_kernel<<<unsigned(a.nq_pad), kThreads, 0, stream>>>(a);
}

void certificate_bounds(const threshold_f_args& a, const uint32_t* count, const float* vals,
                        int64_t cap, double* lb, double* ub, hipStream_t stream)
{
  if (a.nq == 0 || cap == 0) { return; }
  const dim3 grid(unsigned((cap + 255) / 256 < 64 ? (cap + 255) / 256 : 64), unsigned(a.nq));
  certificate_bounds_kernel<<<grid, 256, 0, stream>>>(a, count, vals, cap, lb, ub);
}

void verify_topk_f(const verify_f_args& a, hipStream_t stream)
{
  if (a.nq == 0) { return; }
  // room for k scored rows plus a chunk of k / 2 more (at least the final sort's power of two):
  // less LDS per block than 4 k, so more blocks share a CU
  int cap = (3 * a.k / 2 + 255) / 256 * 256;
  cap     = cap > pow2_ge(a.k) ? cap : pow2_ge(a.k);
  cap     = cap > 1024 ? (cap < kBuf ? cap : kBuf) : 1024;
  const size_t bytes  = size_t(cap) * 12 + size_t(a.dim) * 8;
  const unsigned grid = unsigned(a.nq);
  switch (score_lanes(a.dim)) {
    case 16: launch_dyn(verify_topk_f_kernel<16>, grid, bytes, stream, a, cap); break;
    case 32: launch_dyn(verify_topk_f_kernel<32>, grid, bytes, stream, a, cap); break;
    default: launch_dyn(verify_topk_f_kernel<64>, grid, bytes, stream, a, cap); break;
  }
}

}  // namespace certex_amd
