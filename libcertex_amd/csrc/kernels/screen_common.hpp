// Pieces shared by the MFMA screens (screen.hip: rows of up to 256 bytes with the queries of a
// workgroup resident in LDS; screen_wide.hip: fp16 rows of more than 128 halves, K loop).
//
// MFMA tile: operand A holds 16 stored rows and operand B 16 queries, so lane l owns query l % 16
// and rows 4 (l / 16) + r, r = 0..3, of the tile. A step is 4 or 8 row tiles (bt); bit
// bt * 4 + r of a lane's survivor mask marks row row0 + bt * 16 + r, with row0 = the step's first
// row + 4 (l / 16).
#pragma once

#include "../kernels.hpp"

#include <climits>
#include <cmath>

namespace certex_amd::screen_detail {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

/** Survivors a workgroup gathers in LDS before it flushes them to the per-query buckets. */
constexpr int kHitCap = 1024;

struct int8_rows {
  using acc_t  = v4i;
  using frag_t = v4i;
  using val_t  = int;
  static constexpr bool kValues = false;  // survivors carry no screen value (verify scores all)
  __device__ static acc_t mfma(frag_t a, frag_t b, acc_t c)
  {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
  }
  __device__ static val_t lowest() { return INT_MIN; }
  __device__ static val_t dead() { return kDeadRow; }
  __device__ static val_t keep_none() { return kKeepNone; }  // no screen value reaches it
  __device__ static val_t vmax(val_t a, val_t b) { return max(a, b); }
};

struct f16_rows {
  using acc_t  = v4f;
  using frag_t = v8h;
  using val_t  = float;
  static constexpr bool kValues = true;  // survivors carry their screen value (ordered verify)
  __device__ static acc_t mfma(frag_t a, frag_t b, acc_t c)
  {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  __device__ static val_t lowest() { return -INFINITY; }
  __device__ static val_t dead() { return -INFINITY; }
  __device__ static val_t keep_none() { return __builtin_nanf(""); }  // no value compares >= NaN
  __device__ static val_t vmax(val_t a, val_t b) { return fmaxf(a, b); }
};

/** The share of one workgroup of a screen launch. */
struct screen_work {
  int64_t q0;       // first query of the block
  int64_t q_end;    // queries [q_first, q_end) are live (others in the block are padding)
  int64_t q_first;  // first live query of the group (q0 or later)
  int64_t chunk;    // row chunk: scan steps [chunk * chunk_steps, (chunk + 1) * chunk_steps)
  int64_t n_scan;   // scan indices of the pass
  int64_t base;     // stored row of scan index i: base + i * row_stride (anchor pairs:
                    // base + (i / 2) 2 row_stride + i % 2)
  int rlead;        // scan indices below rlead are not live (pair alignment)
  bool valid;
};

/** x / d for x >= 0 and d > 0, in 32-bit arithmetic when x fits (the usual case). */
__device__ inline int64_t div_small(int64_t x, int64_t d)
{
  if ((uint64_t(x) >> 32) == 0 && (uint64_t(d) >> 32) == 0) { return int64_t(uint32_t(x) / uint32_t(d)); }
  return x / d;
}

/**
 * Work of block b. Plain launches: block b runs on XCD b % 8 and the query blocks of one row
 * chunk are consecutive on one XCD (chunk = (b / 8 / n_qb) * 8 + b % 8). Routed launches: the
 * group whose tiles hold b (a ballot over the first tiles of up to 64 groups, else a binary
 * search over them), then query block and chunk within it, in the same XCD order when the group
 * has several query blocks (its tile0 is then a multiple of 8, screen_group_tile0). Blocks past a
 * group's chunks (octet padding, alignment gaps) are invalid. Every lane of the block calls it.
 * PAIRS (the tiled screen over paired queries and, with rows_paired, paired rows): a routed
 * group's query blocks start at an even query and its tiles at an even row, one slot before the
 * group when its first query or row is odd (that slot is not live); screen_group_tiles counts
 * such a group with nq + (q0 & 1) queries and nx + (x0 & 1) rows (paired_group_tiles).
 */
template <int QB, bool PAIRS = false>
__device__ inline screen_work work_of(const screen_args& a, uint32_t b)
{
  screen_work w;
  w.q_first = 0;
  w.rlead   = 0;
  if (a.groups == nullptr) {
    const int64_t n_steps  = screen_steps(a.n_scan);
    const int64_t n_chunks = (n_steps + a.chunk_steps - 1) / a.chunk_steps;
    const uint32_t n_qb    = uint32_t((a.nq + QB - 1) / QB);
    const uint32_t i       = b >> 3;
    w.q0                   = int64_t(i % n_qb) * QB;
    w.q_end                = a.nq;
    w.chunk                = int64_t(i / n_qb) * 8 + (b & 7);
    w.n_scan               = a.n_scan;
    w.base                 = a.row_base;
    w.valid                = w.chunk < n_chunks;
    return w;
  }
  // the group: one vector load of up to 64 groups' first tiles and a ballot, else a binary search
  int lo = 0;
  if (a.n_route <= 64) {
    const int lane   = threadIdx.x & 63;
    const int64_t t0 = lane < a.n_route ? a.groups[lane].tile0 : INT64_MAX;
    const int c      = __popcll(__ballot(t0 <= int64_t(b)));
    lo               = __builtin_amdgcn_readfirstlane(c > 0 ? c - 1 : 0);
  } else {
    int hi = a.n_route - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (a.groups[mid].tile0 <= int64_t(b)) {
        lo = mid;
      } else {
        hi = mid - 1;
      }
    }
  }
  const screen_group g = a.groups[lo];
  const int64_t t      = int64_t(b) - g.tile0;
  const int qlead      = PAIRS ? int(g.q0 & 1) : 0;
  const int rlead      = PAIRS && a.rows_paired && !a.anchor_pairs ? int(g.x0 & 1) : 0;
  const uint32_t n_qb  = uint32_t(div_small(g.nq + qlead + QB - 1, QB));
  const uint32_t i     = uint32_t(t) >> 3;
  w.q0                 = g.q0 - qlead + int64_t(n_qb > 1 ? i % n_qb : 0) * QB;
  w.q_end              = g.q0 + g.nq;
  w.q_first            = g.q0;
  w.chunk              = n_qb > 1 ? int64_t(i / n_qb) * 8 + (t & 7) : t;
  w.n_scan             = a.anchor_pairs      ? paired_anchor_count(g.x0, g.nx, a.row_stride)
                         : a.row_stride == 1 ? g.nx + rlead
                                             : div_small(g.nx + a.row_stride - 1, a.row_stride);
  w.base               = a.anchor_pairs ? g.x0 + (g.x0 & 1) : g.x0 - rlead;
  w.rlead              = rlead;
  const int64_t steps  = screen_steps(w.n_scan);
  // a group without queries (a label search's table has one group per label) runs nothing
  w.valid              = g.nq > 0 && t >= 0 && w.chunk < div_small(steps + a.chunk_steps - 1, a.chunk_steps);
  return w;
}

/**
 * Copies the query rows [q0, q0 + n) of qcodes (ROWB bytes each) into LDS, 16-byte chunk c of row
 * r at slot(r, c); rows at or past q_end are zero. NT threads (the workgroup) take part. Each thread issues a batch of 8 loads before
 * their LDS stores, so a batch costs one memory latency (a load-store loop would wait once per
 * chunk).
 */
template <int NT, typename Slot>
__device__ __forceinline__ void stage_queries(const int8_t* qcodes, int ROWB, int64_t q0,
                                              int64_t q_end, int n, uint8_t* lds, Slot slot)
{
  constexpr int BATCH = 8;
  const int CPR       = ROWB / 16;  // chunks per row
  const int total     = n * CPR;
  for (int e0 = 0; e0 < total; e0 += NT * BATCH) {
    v4i v[BATCH];
#pragma unroll
    for (int i = 0; i < BATCH; ++i) {
      const int e = e0 + i * NT + int(threadIdx.x);
      const int r = e / CPR, c = e % CPR;
      v[i]        = v4i{0, 0, 0, 0};
      if (e < total && q0 + r < q_end) {
        v[i] = *reinterpret_cast<const v4i*>(qcodes + (q0 + r) * ROWB + 16 * c);
      }
    }
#pragma unroll
    for (int i = 0; i < BATCH; ++i) {
      const int e = e0 + i * NT + int(threadIdx.x);
      const int r = e / CPR, c = e % CPR;
      if (e < total) { *reinterpret_cast<v4i*>(lds + r * ROWB + 16 * slot(r, c)) = v[i]; }
    }
  }
}

/**
 * Group table entry of group `col` of the pass for launch query q: row q from column grp_base, or
 * (list probe) row out_row[q] from column out_col[q].
 */
__device__ inline int64_t table_entry(const screen_args& a, int64_t q, int64_t col)
{
  const int64_t row  = a.out_row != nullptr ? int64_t(a.out_row[q]) : q;
  const int64_t base = a.out_col != nullptr ? int64_t(a.out_col[q]) : a.grp_base;
  return row * a.n_groups + base + col;
}

/** Filter test of a pair (query q of the batch, id). */
__device__ inline bool keeps_id(const filter_args& f, int64_t q, uint32_t id)
{
  switch (f.kind) {
    case 1: return (f.words[id >> 5] >> (id & 31)) & 1u;
    case 2: {
      const int64_t bit = (f.q0 + q) * f.bitmap_ld + id;
      return (f.words[bit >> 5] >> (bit & 31)) & 1u;
    }
    case 3: return f.row_labels[id] == f.query_labels[f.q0 + q];
    default: return true;
  }
}

/** Filter test of a pair (query q of the batch, stored row). */
__device__ inline bool keeps(const filter_args& f, int64_t q, uint32_t row)
{
  if (f.kind == 0) { return true; }
  return keeps_id(f, q, listed_id(f, row));
}

/** Filter test of a pair (query q, row of the pass): anchors of the anchor copy carry their id. */
__device__ inline bool keeps_row(const screen_args& a, int64_t q, uint32_t row)
{
  if (a.filter.kind == 0) { return true; }
  return a.id_scale > 0 ? keeps_id(a.filter, q, uint32_t(row * a.id_scale))
                        : keeps(a.filter, q, row);
}

/**
 * Label filter of the anchor pass, row side: the labels of the lane's 16 rows of a step (entry
 * bt * 4 + r: scan index row0 + bt * 16 + r; 0xffffffff past the scan), read once per step. Each
 * query tile then compares them with one query label instead of reading two labels per pair.
 */
struct step_labels {
  bool on = false;  // a label filter (kind 3)
  uint32_t v[16];
};

__device__ inline void load_step_labels(const screen_args& a, const screen_work& w, int64_t row0,
                                        step_labels& L)
{
  L.on = a.filter.kind == 3;
  if (!L.on) { return; }
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int64_t idx = row0 + (j >> 2) * 16 + (j & 3);
    const bool in     = idx < w.n_scan;
    const uint32_t row = uint32_t(w.base + (in ? idx : 0) * a.row_stride);
    const uint32_t id  = a.id_scale > 0 ? uint32_t(row * a.id_scale) : listed_id(a.filter, row);
    const uint32_t lab = a.filter.row_labels[id];
    L.v[j]             = in ? lab : 0xffffffffu;
  }
}

/**
 * The filter's verdicts for query q (q < q_end) on the lane's 16 rows of the step (bit
 * bt * 4 + r; rows past the scan are cleared): one compare per row against the row labels of
 * the step for a label filter, else one test per row in a rolled loop (which keeps the anchor
 * pass's code small enough to stay inlined).
 */
__device__ __forceinline__ uint32_t filter_mask(const screen_args& a, const screen_work& w,
                                                const step_labels& L, int64_t q, int64_t row0)
{
  if (L.on) {
    const uint32_t qlab = uint32_t(a.filter.query_labels[a.filter.q0 + q]);
    uint32_t keep       = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) { keep |= uint32_t(L.v[j] == qlab) << j; }
    return keep;
  }
  uint32_t keep = 0;
#pragma unroll 1
  for (int j = 0; j < 16; ++j) {
    const int64_t idx = row0 + (j >> 2) * 16 + (j & 3);
    if (idx < w.n_scan && keeps_row(a, q, uint32_t(w.base + idx * a.row_stride))) {
      keep |= 1u << j;
    }
  }
  return keep;
}

/** Writes spill pool entry e (an index into the launch's pool): query qloc of the workgroup, row
 *  roff past the workgroup's first row (below 2^kSpillRowBits), and the screen value for fp16 rows
 *  (one 8-byte store). */
template <bool VALS>
__device__ __forceinline__ void spill_put(const screen_args& a, int64_t e, uint32_t qloc, uint32_t roff,
                                          float val)
{
  const uint32_t w0 = (qloc << kSpillRowBits) | roff;
  if constexpr (VALS) {
    reinterpret_cast<uint2*>(a.spill)[e] = make_uint2(w0, __float_as_uint(val));
  } else {
    a.spill[e] = w0;
  }
}

/**
 * LDS survivor list of a workgroup: hit_q / hit_row / hit_val (the screen values, when the rows
 * carry them) of `cap` entries (kHitCap, or what the K-loop screen's LDS leaves) and the count
 * n_hits, passed as separate pointers (a struct of LDS addresses can end up as a constant
 * initializer, which the backend rejects).
 */

/**
 * Appends the survivors of one 16-query tile of a step to the workgroup's list: `bits` is this
 * lane's survivor mask over NB = 16 or 32 rows (4 or 8 row tiles), `qloc` its query within the
 * workgroup, row0 the stored row of its bit 0, rbase the workgroup's first row (spill entries hold
 * rows as offsets from it), v the screen values of bits 0..15 (used when VALS, NB = 16), spill_n
 * (LDS, per query of the workgroup) the count of each query's entries in the spill region. The
 * wave reserves all of its survivors with one LDS atomic: each lane's offset is the exclusive
 * prefix of the survivor counts, summed from one ballot per bit of the count. The lanes then write
 * their survivors in as many rounds as the busiest lane has survivors, with no vote or atomic per
 * round. Every lane of the wave must call it.
 */
template <int NB, bool FILT, bool VALS, typename V>
__device__ __forceinline__ void push_hits(uint32_t bits, uint32_t qloc, int64_t row0, int64_t rbase,
                                          int64_t q0, const screen_args& a, uint32_t* hit_q,
                                          uint32_t* hit_row, float* hit_val, uint32_t* n_hits,
                                          uint32_t* spill_n, uint32_t cap, const V (&v)[16])
{
  static_assert(NB == 16 || NB == 32, "16 or 32 rows per lane");
  static_assert(!VALS || NB == 16, "screen values come with 4 row tiles");
  if constexpr (FILT) {
    uint32_t scan = bits;
    while (scan) {
      const int j = __builtin_ctz(scan);
      scan &= scan - 1;
      if (!keeps(a.filter, q0 + qloc, uint32_t(row0 + (j >> 2) * 16 + (j & 3)))) {
        bits &= ~(1u << j);
      }
    }
  }
  const uint32_t cnt = uint32_t(__builtin_popcount(bits));
  uint32_t excl = 0, total = 0;
#pragma unroll
  for (int b = 0; (1 << b) <= NB; ++b) {
    const uint64_t m = __ballot((cnt >> b) & 1u);
    excl += __builtin_amdgcn_mbcnt_hi(uint32_t(m >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(m), 0u))
            << b;
    total += uint32_t(__builtin_popcountll(m)) << b;
  }
  if (total == 0) { return; }
  const int lane   = threadIdx.x & 63;
  const int leader = __builtin_ctzll(__ballot(1));
  uint32_t base    = 0;
  if (lane == leader) { base = atomicAdd(n_hits, total); }
  const uint32_t first = uint32_t(__builtin_amdgcn_readlane(int(base), leader));
  uint32_t pos         = first + excl;
  // the screen values pass through an empty asm statement, and no select below reads an array:
  // selects between array elements are otherwise folded into one load at a computed index, which
  // puts the values in scratch memory
  const auto L = [](float f) {
    if constexpr (VALS) { asm("" : "+v"(f)); }
    return f;
  };
  const float x0 = L(float(v[0])), x1 = L(float(v[1])), x2 = L(float(v[2])), x3 = L(float(v[3]));
  const float x4 = L(float(v[4])), x5 = L(float(v[5])), x6 = L(float(v[6])), x7 = L(float(v[7]));
  const float x8 = L(float(v[8])), x9 = L(float(v[9])), x10 = L(float(v[10])), x11 = L(float(v[11]));
  const float x12 = L(float(v[12])), x13 = L(float(v[13])), x14 = L(float(v[14])), x15 = L(float(v[15]));
  // each lane writes its survivors at pos, pos + 1, ...: the list, then the workgroup's spill
  // region (plain stores, moved to the buckets by the flush), then, when both are full (or no pool
  // was provided), straight into the global bucket with one atomic each. A wave whose survivors all
  // go to the list, or all to the region, takes a loop without the per-survivor choice
  const auto each = [&](auto put) {
    while (bits != 0) {
      const int j = __builtin_ctz(bits);
      bits &= bits - 1;
      float val   = 0.0f;
      if constexpr (VALS) {
        // value j of the lane's 16: a select tree on the 4 bits of j (15 selects on 4 masks)
        const bool b0 = (j & 1) != 0, b1 = (j & 2) != 0, b2 = (j & 4) != 0, b3 = (j & 8) != 0;
        const float a0 = b0 ? x1 : x0, a1 = b0 ? x3 : x2, a2 = b0 ? x5 : x4, a3 = b0 ? x7 : x6;
        const float a4 = b0 ? x9 : x8, a5 = b0 ? x11 : x10, a6 = b0 ? x13 : x12, a7 = b0 ? x15 : x14;
        const float c0 = b1 ? a1 : a0, c1 = b1 ? a3 : a2, c2 = b1 ? a5 : a4, c3 = b1 ? a7 : a6;
        const float d0 = b2 ? c1 : c0, d1 = b2 ? c3 : c2;
        val            = b3 ? d1 : d0;
      }
      put(uint32_t((j >> 2) * 16 + (j & 3)), val);
      ++pos;
    }
  };
  const uint32_t roff0 = uint32_t(row0 - rbase);
  if (first + total <= cap) {
    each([&](uint32_t d, float val) {
      hit_q[pos]   = qloc;
      hit_row[pos] = uint32_t(row0) + d;
      if constexpr (VALS) { hit_val[pos] = val; }
    });
    return;
  }
  const int64_t e0 = int64_t(blockIdx.x) * a.spill_cap - int64_t(cap);
  if (first >= cap && int64_t(first - cap) + total <= a.spill_cap) {
    if (cnt != 0) { atomicAdd(&spill_n[qloc], cnt); }
    each([&](uint32_t d, float val) { spill_put<VALS>(a, e0 + pos, qloc, roff0 + d, val); });
    return;
  }
  each([&](uint32_t d, float val) {
    if (pos < cap) {
      hit_q[pos]   = qloc;
      hit_row[pos] = uint32_t(row0) + d;
      if constexpr (VALS) { hit_val[pos] = val; }
    } else if (int64_t(pos - cap) < a.spill_cap) {
      atomicAdd(&spill_n[qloc], 1u);
      spill_put<VALS>(a, e0 + pos, qloc, roff0 + d, val);
    } else {
      const int64_t q   = q0 + qloc;
      const uint32_t at = atomicAdd(a.cand_count + q, 1u);
      if (at < a.cap) {
        a.cand_rows[q * a.cap + at] = uint32_t(row0) + d;
        if constexpr (VALS) { a.cand_vals[q * a.cap + at] = val; }
      }
    }
  });
}

/**
 * Flushes the workgroup's survivors to the per-query buckets (after a barrier, once the queries in
 * LDS are no longer read): the LDS list (the first `cap` of n_hits) and the entries of its spill
 * region past it. Each LDS entry's rank among its query's survivors comes from an LDS counter
 * (cnt), the region's entries follow the query's LDS entries (cursor cur); then one global atomic
 * per query reserves the query's slots. `scratch` holds 2 qb + cap words of LDS (the query rows'
 * space); rbase is the workgroup's first row (spill_put); spill_n, when given, the count of each
 * query's region entries (push_hits), so that the region is read once. Records the workgroup's
 * count past the LDS list in spill_need.
 */
template <bool VALS>
__device__ inline void flush_hits(int64_t q0, int64_t rbase, int qb, const screen_args& a, const uint32_t* hit_q,
                                  const uint32_t* hit_row, const float* hit_val,
                                  const uint32_t* n_hits, uint32_t cap, uint32_t* scratch,
                                  const uint32_t* spill_n = nullptr)
{
  uint32_t* cnt        = scratch;           // [qb] survivors per query, then their first slot
  uint32_t* cur        = scratch + qb;      // [qb] the next rank of a region entry per query
  uint32_t* rank       = scratch + 2 * qb;  // [cap]
  const uint32_t total = *n_hits;
  const uint32_t nh    = total < cap ? total : cap;
  const uint32_t past  = total - nh;
  const uint32_t ns    = past < uint32_t(a.spill_cap) ? past : uint32_t(a.spill_cap);
  const int64_t region = int64_t(blockIdx.x) * a.spill_cap;
  if (threadIdx.x == 0 && past > 0 && a.spill_need != nullptr) { atomicMax(a.spill_need, past); }
  for (int e = threadIdx.x; e < qb; e += blockDim.x) { cnt[e] = 0; }
  __syncthreads();
  for (uint32_t e = threadIdx.x; e < nh; e += blockDim.x) { rank[e] = atomicAdd(&cnt[hit_q[e]], 1u); }
  __syncthreads();
  for (int e = threadIdx.x; e < qb; e += blockDim.x) {
    cur[e] = cnt[e];
    if (spill_n != nullptr) { cnt[e] += spill_n[e]; }
  }
  __syncthreads();
  const uint32_t* sp   = a.spill + region * spill_words(VALS);
  // the region's entries, SB per thread and round: their loads are in flight together
  constexpr int SB      = 8;
  const auto region_rounds = [&](auto f) {
    for (uint32_t e0 = threadIdx.x; e0 < ns; e0 += SB * blockDim.x) {
      uint32_t w0[SB], w1[SB];
#pragma unroll
      for (int i = 0; i < SB; ++i) {
        const uint32_t e = e0 + uint32_t(i) * blockDim.x;
        w0[i] = 0, w1[i] = 0;
        if (e < ns) {
          if constexpr (VALS) {
            const uint2 v = reinterpret_cast<const uint2*>(sp)[e];
            w0[i] = v.x, w1[i] = v.y;
          } else {
            w0[i] = sp[e];
          }
        }
      }
#pragma unroll
      for (int i = 0; i < SB; ++i) {
        if (e0 + uint32_t(i) * blockDim.x < ns) { f(w0[i], w1[i]); }
      }
    }
  };
  if (spill_n == nullptr) {
    region_rounds([&](uint32_t w0, uint32_t) { atomicAdd(&cnt[w0 >> kSpillRowBits], 1u); });
    __syncthreads();
  }
  for (int e = threadIdx.x; e < qb; e += blockDim.x) {
    if (cnt[e] != 0) { cnt[e] = atomicAdd(a.cand_count + q0 + e, cnt[e]); }
  }
  __syncthreads();
  for (uint32_t e = threadIdx.x; e < nh; e += blockDim.x) {
    const uint32_t ql    = hit_q[e];
    const uint32_t bslot = cnt[ql] + rank[e];
    if (bslot < a.cap) {
      const int64_t q                = q0 + ql;
      a.cand_rows[q * a.cap + bslot] = hit_row[e];
      if constexpr (VALS) { a.cand_vals[q * a.cap + bslot] = hit_val[e]; }
    }
  }
  region_rounds([&](uint32_t w0, uint32_t w1) {
    const uint32_t ql    = w0 >> kSpillRowBits;
    const uint32_t bslot = cnt[ql] + atomicAdd(&cur[ql], 1u);
    if (bslot < a.cap) {
      const int64_t q                = q0 + ql;
      a.cand_rows[q * a.cap + bslot] = uint32_t(rbase + (w0 & ((1u << kSpillRowBits) - 1)));
      if constexpr (VALS) { a.cand_vals[q * a.cap + bslot] = __uint_as_float(w1); }
    }
  });
}

/** A workgroup's life by the shader clock and by the constant 100 MHz counter, added to
 *  a.clock[0] and a.clock[1] at stop() when the launch is timed (a.clock non-null). */
struct wg_clock {
  uint64_t t0 = 0, r0 = 0;
  __device__ __forceinline__ void start(const screen_args& a)
  {
    if (a.clock != nullptr) {
      t0 = __builtin_amdgcn_s_memtime();
      r0 = __builtin_amdgcn_s_memrealtime();
    }
  }
  __device__ __forceinline__ void stop(const screen_args& a) const
  {
    if (a.clock != nullptr && threadIdx.x == 0) {
      const uint64_t t1 = __builtin_amdgcn_s_memtime();
      const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
      atomicAdd(a.clock, static_cast<unsigned long long>(t1 - t0));
      atomicAdd(a.clock + 1, static_cast<unsigned long long>(r1 - r0));
    }
  }
};

/**
 * Anchor pass, one 16-query tile of a 64-row step: folds the best screen value of this lane's
 * query over the step into the wave's running group maximum gml[e] (e = the query's slot).
 * `col[bt]` holds the tile's accumulators of row tile bt. With a filter, bit bt * 4 + r of `keep`
 * says whether the lane's row bt * 16 + r of the step passes it.
 */
template <typename R, bool FILT>
__device__ __forceinline__ void anchor_tile(const typename R::acc_t (&col)[4], int e,
                                            typename R::val_t* gml, uint32_t keep)
{
  using val_t    = typename R::val_t;
  const int lane = threadIdx.x & 63;
  val_t m        = R::lowest();
#pragma unroll
  for (int bt = 0; bt < 4; ++bt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      val_t v = col[bt][r];
      if constexpr (FILT) {
        if (!((keep >> (bt * 4 + r)) & 1u)) { v = R::lowest(); }
      }
      m = R::vmax(m, v);
    }
  }
  m = R::vmax(m, __shfl_xor(m, 16));
  m = R::vmax(m, __shfl_xor(m, 32));
  if (lane < 16) { gml[e] = R::vmax(gml[e], m); }
}

/**
 * Anchor pass with fine groups, one 16-query tile of a 64-row step: the best screen value of each
 * lane's 4 consecutive anchors of each of its 4 row tiles is one group, column grp_base + (scan
 * index of the first of the 4) / 4 of the query's row of the group table. row0 is the scan index
 * of the lane's bit 0; q the lane's query (written only when live).
 *
 * With a wave's LDS block tr (256 values), the 16 x 16 (query, group) values of the tile go
 * through tr so that each store instruction writes 4 queries x 16 consecutive groups (64 bytes of
 * each of 4 table rows); stored straight from the accumulators, each store instruction wrote 4
 * bytes to each of 16 rows. Without tr the lanes store their values directly.
 */
template <typename R, bool FILT>
__device__ __forceinline__ void anchor_tile_fine(const typename R::acc_t (&col)[4], int64_t row0,
                                                 int64_t q, bool live, const screen_args& a,
                                                 const screen_work& w, typename R::val_t* gmax,
                                                 uint32_t keep, typename R::val_t* tr = nullptr)
{
  using val_t    = typename R::val_t;
  const int lane = threadIdx.x & 63;
  val_t m[4];
#pragma unroll
  for (int bt = 0; bt < 4; ++bt) {
    m[bt] = R::lowest();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      val_t v = col[bt][r];
      if constexpr (FILT) {
        if (!((keep >> (bt * 4 + r)) & 1u)) { v = R::lowest(); }
      }
      m[bt] = R::vmax(m[bt], v);
    }
  }
  if (tr == nullptr) {
#pragma unroll
    for (int bt = 0; bt < 4; ++bt) {
      const int64_t first = row0 + bt * 16;  // scan index of the group's first anchor
      if (live && first < w.n_scan) { gmax[table_entry(a, q, first / kFineGroup)] = m[bt]; }
    }
    return;
  }
  // lane (query ql, sub) holds groups 4 bt + sub of the step: into tr[query][group of the step]
  const int ql  = lane & 15;
  const int sub = lane >> 4;
#pragma unroll
  for (int bt = 0; bt < 4; ++bt) { tr[ql * 16 + bt * 4 + sub] = m[bt]; }
  // LDS operations of a wave complete in order; the fence keeps the compiler from moving the
  // reads above the other lanes' writes
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  // store c: lane (sub, gi) takes group gi of query 4 c + sub of the tile
  const int gi          = lane & 15;
  const int64_t first   = row0 - 4 * sub + 4 * gi;  // the step's first row (a multiple of 64), + 4 gi
  const int64_t q_tile  = q - ql;
  const bool has_group  = first < w.n_scan;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int qi    = 4 * c + sub;
    const val_t v   = tr[qi * 16 + gi];
    const int64_t x = q_tile + qi;
    if (has_group && x < w.q_end) { gmax[table_entry(a, x, first / kFineGroup)] = v; }
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");  // every read before the next tile's writes
}

}  // namespace certex_amd::screen_detail
