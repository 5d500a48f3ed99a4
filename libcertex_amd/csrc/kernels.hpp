// Launchers of the gfx950 kernels of the exact k-NN search path. Every launcher takes plain device
// pointers, sizes and the stream to queue on; none allocates or synchronises.
//
// The role of each launcher in the reference pipeline (cpp/src/neighbors/certex/certex.cu:885-1402):
//   encode_rows_i8       encode_int8_rows / encode_rows        (detail/int8.cuh:30-77)
//   encode_queries_i8    encode_int8_queries / encode_queries  (detail/int8.cuh:84-136)
//   screen_i8 (anchors)  anchor_groups + select_k              (detail/kernels.hpp:125-135)
//   threshold_i8         anchor_scores + anchor_threshold      (certex_kernels.cuh:276-370)
//   screen_i8 (screen)   screen_int8 + survivor segments       (detail/screen_int8.cu:99-292)
//   verify_topk          survivor_keys + sort + verify_rounds  (certex_kernels.cuh:458-515,
//                                                               detail/verify.cuh:371-487)
//   finish               finish<S>                             (certex.cu:224-250)
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace certex_amd {

/** Row term of a removed or padding row: its screen value can never reach a threshold. */
constexpr int32_t kDeadRow = -(1 << 30);
/** Lowest threshold: keeps every live row (a live row's screen value exceeds -2^26). */
constexpr int32_t kKeepAll = -(1 << 29);
/** Threshold of a padding query: keeps nothing. */
constexpr int32_t kKeepNone = 0x7fffffff;

/** Rows of one screen step. */
constexpr int kStepRows  = 64;
/** Spill pool entries: the low kSpillRowBits bits of an entry's first word hold its row's offset
 *  from the workgroup's first row, the bits above its query within the workgroup. */
constexpr int kSpillRowBits = 20;
/** Words of a spill entry: the packed query and row, then the screen value for fp16 rows. */
constexpr int spill_words(bool values) { return values ? 2 : 1; }
/** Widest integer row (bytes) that the MFMA screen instantiates. */
constexpr int kMaxIntDim = 4096;

/** Queries per screen workgroup for a batch of nq queries (512, or 128 for small batches). */
__host__ __device__ inline int query_block(int64_t nq) { return nq > 128 ? 512 : 128; }
/** Padded query count of a batch: a multiple of its query block. */
__host__ __device__ inline int64_t pad_queries(int64_t nq)
{
  const int qb = query_block(nq);
  return (nq + qb - 1) / qb * qb;
}
/** Query block of a padded batch (the kernels' view of query_block). */
__host__ __device__ inline int screen_block_queries(int64_t nq_pad) { return nq_pad % 512 == 0 ? 512 : 128; }
/**
 * Query block of the narrow screens: screen_block_queries, except fp16 rows of 128 halves, which
 * take 128 queries (32 KB of LDS, several workgroups per CU, where 512 took 128 KB and left one);
 * their survivors, thousands per query in a KV-cache search, then overlap other workgroups' MFMAs.
 */
__host__ __device__ inline int narrow_block_queries(bool f16, int row_bytes, int64_t nq_pad)
{
  return f16 && row_bytes == 256 ? 128 : screen_block_queries(nq_pad);
}

enum class metric_kind : int { l2 = 0, inner = 1, cosine = 2 };

/**
 * Paired row layout of fp16 rows (row_bytes a multiple of 128): rows 2p and 2p + 1 share 2
 * row_bytes bytes, and their 64-byte pieces c alternate, so that one 128-byte line holds piece c
 * of both rows: byte b of row r sits at (r / 2) 2 row_bytes + (b / 64) 128 + (r % 2) 64 + b % 64.
 * The tiled screen copies a stage (one 64-byte piece of every row of a tile) as whole lines.
 */
__host__ __device__ inline int64_t paired_offset(int64_t r, int64_t b, int64_t row_bytes)
{
  return (r >> 1) * 2 * row_bytes + (b >> 6) * 128 + (r & 1) * 64 + (b & 63);
}
/** Bytes of n rows in the paired layout (a whole number of pairs). */
__host__ __device__ inline int64_t paired_bytes(int64_t n, int64_t row_bytes) { return (n + 1) / 2 * 2 * row_bytes; }
/**
 * Anchors of a routed group of rows [x0, x0 + nx) of a paired partition, taken in pairs: both rows
 * of the row pairs that start at x0e + 2 s j (x0e: x0 rounded up to even), while they lie in the
 * group. Scan index i is stored row x0e + (i / 2) 2 s + i % 2, so that the anchor pass reads whole
 * 128-byte lines (both rows of a line) where single rows every s would take half lines. About nx / s
 * anchors, as with one row every s.
 */
__host__ __device__ inline int64_t paired_anchor_count(int64_t x0, int64_t nx, int64_t s)
{
  const int64_t avail = nx - (x0 & 1);
  if (avail <= 0) { return 0; }
  const int64_t pairs = (avail + 2 * s - 1) / (2 * s);
  return 2 * pairs - (2 * s * (pairs - 1) + 1 >= avail ? 1 : 0);
}

/** Bytes of a stored integer screening row of `dim` coordinates (zero padded): 128, 256, or
 *  above 256 coordinates a multiple of 256 (the tiled screen and the K-loop anchor pass). */
__host__ __device__ inline int int_row_bytes(int64_t dim)
{
  return dim <= 128 ? 128 : int((dim + 255) / 256 * 256);
}

// --- encoding -------------------------------------------------------------------------------

/**
 * codes[i, :] = x[i, :] ^ flip (flip = 0x80 turns uint8 into the int8 code x - 128, 0 keeps int8),
 * zero padded to row_bytes; rowc[i] = the row term of the screen (l2: -floor(|x'|^2 / 2); inner:
 * 128 * sum(x') for uint8, 0 for int8). Rows first .. first + n - 1 of the stored arrays.
 */
void encode_rows_i8(const uint8_t* x, int64_t n, int64_t dim, int row_bytes, uint8_t flip,
                    metric_kind metric, int8_t* codes, int32_t* rowc, hipStream_t stream);

/** qcodes[i] = q[rows[i]] ^ flip (q[i] when rows is null), zero padded, for i < nq; padding
 *  queries [nq, nq_pad) are zero; the same codes again in the paired layout into qpaired unless
 *  null (the tiled screen's queries). */
void encode_queries_i8(const uint8_t* q, int64_t nq, int64_t nq_pad, int64_t dim, int row_bytes,
                       uint8_t flip, int8_t* qcodes, hipStream_t stream, int8_t* qpaired = nullptr,
                       const int32_t* rows = nullptr);

/**
 * Tombstones of ids and where their rows are stored: with lists the ids below n_listed live in
 * stored row list_pos[id]; with a label partition the ids below n_part also have the copy
 * part_rowc[part_pos[id]].
 */
struct row_places {
  const int32_t* list_pos = nullptr;
  int64_t n_listed        = 0;
  const int32_t* part_pos = nullptr;
  int64_t n_part          = 0;
  void* part_rowc         = nullptr;
  // the anchor copy: the ids j * anchor_stride (j < n_anchor) also have the term anchor_rowc[j]
  void* anchor_rowc     = nullptr;
  int64_t anchor_stride = 0;
  int64_t n_anchor      = 0;
};

/**
 * Tombstone rows by id: the row term of the id's stored row becomes kDeadRow for 0 <= id < size;
 * counts the ids that were live into *newly_removed (ids out of range or repeated count once at
 * most).
 */
void remove_rows_i8(const int64_t* ids, int64_t n, int64_t size, int32_t* rowc,
                    unsigned long long* newly_removed, const row_places& at, hipStream_t stream);

void fill_u32(uint32_t* p, int64_t n, uint32_t v, hipStream_t stream);
void fill_i32(int32_t* p, int64_t n, int32_t v, hipStream_t stream);
/** p[i] = first + i for i < n. */
void iota_i32(int32_t* p, int64_t n, int32_t first, hipStream_t stream);

// --- screen -------------------------------------------------------------------------------

struct filter_args {
  int kind = 0;                     // 0 none, 1 bitset over rows, 2 bitmap per query, 3 labels
  const uint32_t* words = nullptr;  // bitset / bitmap words
  int64_t bitmap_ld = 0;            // bits per bitmap row (= index size when built)
  int64_t q0 = 0;                   // first query of the batch (bitmap row, label offset)
  const int32_t* row_labels = nullptr;
  const int32_t* query_labels = nullptr;  // of all queries of the search
  // an index with lists stores the rows [0, n_listed) in list order: stored row r < n_listed holds
  // the id row_ids[r], later rows are their own ids. Filters test ids; the exact-score kernels
  // report ids.
  const int32_t* row_ids = nullptr;
  int64_t n_listed       = 0;
};

/** The id held by stored row `row`. */
__host__ __device__ inline uint32_t listed_id(const filter_args& f, uint32_t row)
{
  return row < f.n_listed ? uint32_t(f.row_ids[row]) : row;
}

/**
 * One routed pairing of a label-partitioned search: the queries [q0, q0 + nq) of the (label
 * sorted) batch against the stored rows [x0, x0 + nx) of the partition; its workgroups are
 * tile0 .. tile0 + ceil(nq / QB) * chunks - 1 of the launch.
 */
struct screen_group {
  int64_t q0, nq;
  int64_t x0, nx;
  int64_t tile0;
};

struct screen_args {
  const int8_t* codes;   // stored rows [*, row_bytes]: int8 codes or fp16 values
  const void* rowc;      // row terms: int32 (int8 rows) or float (fp16 rows)
  int64_t n_scan;        // scanned rows: scan index i reads stored row row_base + i * row_stride
  int64_t row_base = 0;  // first stored row of the pass
  int row_stride;        // 1 for the screen, the anchor stride for the anchor pass
  // routed pass (label partition): the workgroups follow the group table (n_scan and row_base
  // come from each group). Survivors and anchors are recorded as stored rows: a routed pass over
  // the partition records partition rows (below n_part), the tail pass records ids (n_part and
  // above); the exact-score kernels map partition rows to ids (part_ids)
  const screen_group* groups = nullptr;
  int n_route                = 0;
  int64_t n_tiles            = 0;  // workgroups of a routed launch
  int row_bytes;         // 64 KS
  const int8_t* qcodes;  // [nq_pad, row_bytes]
  const void* theta;     // [nq_pad] int32 or float (screen only)
  int64_t nq;            // live queries
  int64_t nq_pad;        // pad_queries(nq)
  // the queries again in the paired layout (fp16 rows read by the tiled screen), and whether the
  // stored rows are paired (the label partition of fp16 rows of more than 128 halves)
  const int8_t* qpaired = nullptr;
  bool rows_paired      = false;
  // routed anchor pass over a paired partition: the anchors of a group are row pairs
  // (paired_anchor_count), row_stride the pairs' half spacing; with tiled, the pass runs as tiles
  // of the tiled screen (fine groups, paired queries, chunk_steps = tile_chunk_steps())
  bool anchor_pairs = false;
  bool tiled        = false;
  int chunk_steps;       // steps of kStepRows rows per workgroup: 4 waves x a whole number of
                         // anchor groups
  filter_args filter;
  // screen: candidate buckets
  uint32_t* cand_count = nullptr;  // [nq_pad]
  uint32_t* cand_rows  = nullptr;  // [nq_pad, cap]
  float* cand_vals     = nullptr;  // [nq_pad, cap] screen values (fp16 rows only)
  int64_t cap          = 0;
  // screen: survivors past a workgroup's LDS list go to the workgroup's own region of a pool of
  // spill_pool entries, with plain stores; the launcher splits the pool evenly among its
  // workgroups (spill_cap each), and the workgroup's flush moves its region into the buckets.
  // An entry is one word, (query within the block) << kSpillRowBits | (row - the workgroup's first
  // row), followed for fp16 rows by the screen value's bits (kSpillWords). Survivors past the
  // region take a global atomic each. spill_need (device word) gets the largest count past the
  // LDS list of any workgroup, so that the host knows whether to provide a pool.
  uint32_t* spill     = nullptr;
  int64_t spill_pool  = 0;
  int64_t spill_cap   = 0;  // set by the launcher
  uint32_t* spill_need = nullptr;
  // shader clock of the screen's workgroups (timing mode only, else null): every workgroup adds
  // its life in shader clock cycles (s_memtime) to clock[0] and in ticks of the constant 100 MHz
  // counter (s_memrealtime) to clock[1]
  unsigned long long* clock = nullptr;
  // anchors: group maxima [nq_pad, n_groups] (int32 or float), a group = group_steps steps
  void* gmax       = nullptr;
  int64_t n_groups = 0;
  int64_t grp_base = 0;  // first group column of the pass
  int group_steps  = 1;
  // fine groups: a group is 4 consecutive anchors (column grp_base + scan index / 4) instead of
  // group_steps steps, for searches whose k is large next to the number of anchor steps
  bool fine = false;
  // a pass over the anchor copy: stored row r of the pass is anchor r, the vector of id
  // r * id_scale (0: the rows are stored rows of the index)
  int64_t id_scale = 0;
  // list probe: query q of the launch writes its groups to row out_row[q] of the table, from column
  // out_col[q] on (null: row q, column grp_base)
  const int32_t* out_row = nullptr;
  const int32_t* out_col = nullptr;
};

/** Anchors per fine group. */
constexpr int kFineGroup = 4;

/** Queries per workgroup of the screen kernels for a batch padded to nq_pad. */
int screen_query_block(bool f16, int row_bytes, int64_t nq_pad);
/**
 * Workgroups of one routed group: query blocks x row chunks. A group of several query blocks
 * takes its chunks in octets (8 n_qb workgroups per octet, the last octet padded with workgroups
 * that exit at once), so that the query blocks of one chunk run on one XCD, as in plain launches.
 */
__host__ __device__ inline int64_t screen_group_tiles(int64_t nq, int64_t n_scan, int qb, int chunk_steps)
{
  const int64_t steps    = (n_scan + kStepRows - 1) / kStepRows;
  const int64_t n_chunks = (steps + chunk_steps - 1) / chunk_steps;
  const int64_t n_qb     = (nq + qb - 1) / qb;
  return n_qb > 1 ? 8 * n_qb * ((n_chunks + 7) / 8) : n_chunks;
}
/**
 * The same for the tiled screen over paired queries (and rows, rows_paired): a group whose first
 * query (row) is odd starts one slot earlier, at the pair's first query (row).
 */
__host__ __device__ inline int64_t paired_group_tiles(const screen_group& g, bool rows_paired, int qb, int chunk_steps)
{
  return screen_group_tiles(g.nq + (g.q0 & 1), g.nx + (rows_paired ? (g.x0 & 1) : 0), qb, chunk_steps);
}
/**
 * First workgroup of a routed group that follows `tiles` workgroups: a multiple of 8 for a group
 * of several query blocks (workgroup b runs on XCD b % 8), else `tiles`.
 */
__host__ __device__ inline int64_t screen_group_tile0(int64_t tiles, int64_t nq, int qb)
{
  return (nq + qb - 1) / qb > 1 ? (tiles + 7) / 8 * 8 : tiles;
}

/** Steps of kStepRows rows that cover n_scan rows. */
__host__ __device__ inline int64_t screen_steps(int64_t n_scan) { return (n_scan + kStepRows - 1) / kStepRows; }

/** Int8 MFMA pass that keeps (query, row) pairs whose screen value reaches the query threshold
 *  (rows of more than 256 bytes: screen_i8_tile). */
void screen_i8(const screen_args& a, hipStream_t stream);

/** Int8 MFMA pass that records the best screen value of every group of anchors for every query
 *  (rows of more than 256 bytes: anchors_i8_wide). */
void anchors_i8(const screen_args& a, hipStream_t stream);

/** The same two passes over fp16 rows (f32 accumulation, certified threshold). */
void screen_f16(const screen_args& a, hipStream_t stream);
void anchors_f16(const screen_args& a, hipStream_t stream);
/**
 * The fp16 anchor pass for rows of more than 128 halves (a multiple of 128, at most
 * kMaxF16Halves): a K loop, workgroups of 8 waves; chunk_steps is a multiple of 8 group_steps.
 */
void anchors_f16_wide(const screen_args& a, hipStream_t stream);
/** The same K-loop anchor pass over int8 rows of more than 256 bytes (a multiple of 256). */
void anchors_i8_wide(const screen_args& a, hipStream_t stream);
/**
 * The fp16 screen for rows of more than 128 halves as LDS-staged tiles: a workgroup multiplies
 * 256 rows (chunk_steps = tile_chunk_steps()) with tile_block_queries() queries; row_stride 1.
 */
void screen_f16_tile(const screen_args& a, hipStream_t stream);
/**
 * The routed fp16 anchor pass over a paired partition with anchor pairs and fine groups, as tiles
 * of the same kernel (256 anchors x tile_block_queries() queries): each lane writes the best
 * screen value of its 4 consecutive anchors of every row tile and query tile to the group table.
 * anchors_f16_wide runs it for a pass with `tiled`.
 */
void anchors_f16_tile(const screen_args& a, hipStream_t stream);
/** The tiled screen and tiled anchor pass over int8 rows of more than 256 bytes (exact int32
 *  screen values; survivors carry no value). */
void screen_i8_tile(const screen_args& a, hipStream_t stream);
void anchors_i8_tile(const screen_args& a, hipStream_t stream);
int tile_chunk_steps();
int tile_block_queries();

/**
 * theta[q] = the k-th largest of gmax[q, 0 .. n_groups) (kKeepAll when n_groups < k, and never
 * below kKeepAll); padding queries q >= nq get kKeepNone.
 */
void threshold_i8(const int32_t* gmax, int64_t n_groups, int64_t nq, int64_t nq_pad, int k,
                  int32_t* theta, hipStream_t stream);

/** *out = max(count[0 .. n)). */
void max_u32(const uint32_t* count, int64_t n, uint32_t* out, hipStream_t stream);
/** *out += sum(min(count[i], cap)) over i < n (64-bit). */
void sum_u32(const uint32_t* count, int64_t n, int64_t cap, unsigned long long* out,
             hipStream_t stream);

// --- exact re-rank and top-k -----------------------------------------------------------------

struct verify_args {
  // candidates: the bucket of each query, or every row when all_rows
  const uint32_t* cand_count;
  const uint32_t* cand_rows;
  int64_t cap;
  bool all_rows;
  int64_t max_cand  = -1;  // the largest bucket count when the host knows it (else -1)
  int64_t small_max = -1;  // set by the launcher: buckets up to this size take the one-wave path
  int64_t n_rows;         // rows of the index (all_rows)
  // vectors: integer codes (int path)
  const int8_t* codes;
  const int32_t* rowc;  // liveness (kDeadRow) for all_rows
  int row_bytes;
  int64_t dim;
  uint8_t flip;
  const int8_t* qcodes;
  metric_kind metric;
  filter_args filter;  // applied to all_rows candidates
  int64_t nq;
  int k;
  // routed searches: candidate rows below n_part are partition rows, id = part_ids[row], codes in
  // part_codes; the other rows are stored rows (filter.row_ids maps them to ids)
  const int32_t* part_ids  = nullptr;
  int64_t n_part           = 0;
  const int8_t* part_codes = nullptr;
  bool part_paired         = false;  // part_codes in the paired layout (rows of more than 256 bytes)
  // the results as the caller receives them, in (score, id) order: distances [nq, k] in the
  // metric's form (+inf, -inf for the inner product, where missing), ids [nq, k] (-1 where missing);
  // query q's row of both is out_rows[q] (a routed batch in label order), or q when out_rows is null
  float* distances;
  int64_t* neighbors;
  const int32_t* out_rows = nullptr;
};

/** fp64 exact scores of the candidates of every query and their k best by (score, row). */
void verify_topk_i8(const verify_args& a, hipStream_t stream);

// --- float vectors (float32 / float16) ------------------------------------------------------

enum class elem : int { f32 = 0, f16 = 1, bf16 = 2 };

/** Widest fp16 screening row (halves) of the screens. */
constexpr int kMaxF16Halves = 4096;
/**
 * Row length (halves) of the fp16 screening rows for dimension dim: 64, 128, or dim rounded up
 * to a multiple of 128 (rows of more than 128 halves use the K-loop screen).
 */
__host__ __device__ inline int f16_row_halves(int64_t dim)
{
  return dim <= 64 ? 64 : int((dim + 127) / 128 * 128);
}
/** Waves of a screen workgroup: 8 for the K-loop anchor pass of rows of more than 256 bytes (fp16
 *  or int8), 4 otherwise. */
__host__ __device__ inline int screen_waves(bool f16, int row_bytes)
{
  (void)f16;
  return row_bytes > 256 ? 8 : 4;
}

/**
 * sums[j] += sum over rows of x[i, j] (x normalised to unit length when `normalize`), in fp64;
 * the center of the screening rows is sums / n.
 */
void column_sums(const void* x, elem t, int64_t n, int64_t dim, bool normalize, double* sums,
                 hipStream_t stream);
/** *out = max(*out, max over rows of |x_i - center|) (x normalised when `normalize`). */
void max_norm(const void* x, elem t, int64_t n, int64_t dim, bool normalize, const double* center,
              double* out, hipStream_t stream);

/**
 * fp16 screening rows: Z = (x - center) / alpha (x normalised when `normalize`), rows[i] =
 * fp16(Z) with subnormal results set to 0, zero padded to `halves`; rowc[i] = the row term
 * rounded up (l2 / cosine: -(|Z|^2 / 2)(1 - 2 gamma - slack); inner: 0); maxima[0] and [1] are
 * raised to the row's |fp16(Z)| and |Z - fp16(Z)| (upper bounds). Rows whose |Z| exceeds the
 * fp16-safe bound get zeros and rowc = +inf (always a candidate).
 */
void encode_rows_f16(const void* x, elem t, int64_t n, int64_t dim, int halves, bool normalize,
                     const double* center, double inv_alpha, metric_kind metric, double gamma,
                     uint16_t* rows, float* rowc, double* maxima, hipStream_t stream);

/**
 * Query rows the same way (row i from the caller's row rows[i], or i when rows is null);
 * qscal[3 i + 0..2] = |W|^2, |fp16(W)| and |W - fp16(W)| (upper bounds, |W|^2 a lower bound) for
 * i < nq; padding queries are zero.
 */
void encode_queries_f16(const void* q, elem t, int64_t nq, int64_t nq_pad, int64_t dim,
                        int halves, bool normalize, const double* center, double inv_alpha,
                        uint16_t* qrows, double* qscal, hipStream_t stream,
                        uint16_t* qpaired = nullptr, const int32_t* rows = nullptr);

/** Float tombstones (row term -inf) of ids, as remove_rows_i8. */
void remove_rows_f16(const int64_t* ids, int64_t n, int64_t size, float* rowc,
                     unsigned long long* newly_removed, const row_places& at, hipStream_t stream);

struct threshold_f_args {
  const float* gmax;     // [nq_pad, n_groups] best screen value per anchor group
  int64_t n_groups;
  int64_t nq, nq_pad;
  int k;
  metric_kind metric;
  const double* qscal;   // [nq_pad, 3]
  const double* maxima;  // [2]
  double alpha2;         // alpha^2
  double gamma;
  float* theta;          // [nq_pad]
  // testing only (null in searches): U per live query, the certified bound of its k-th
  // neighbour's score that theta is derived from (+inf when fewer than k groups count)
  double* ub = nullptr;
};
/**
 * theta[q] for fp16 rows, certified from the anchor pass alone: the k-th largest finite group
 * maximum belongs to k distinct live rows; the certificate's upper bound of the score of a pair
 * with that screen value bounds the k-th neighbour's score by U, and theta is the screen value
 * below which no pair can have a score <= U (rounded down). -FLT_MAX (keep every live row) with
 * fewer than k such groups; +inf for padding queries.
 */
void threshold_f16(const threshold_f_args& a, hipStream_t stream);

/**
 * Testing only: the certificate's bounds of the exact score of every bucket entry of the live
 * queries, from its screen value v: lb[q, slot] = the lower bound that the ordered verification
 * uses, ub[q, slot] = the upper bound that the threshold uses (both for slot < min(count[q], cap)).
 */
void certificate_bounds(const threshold_f_args& a, const uint32_t* count, const float* vals,
                        int64_t cap, double* lb, double* ub, hipStream_t stream);

struct verify_f_args {
  const uint32_t* cand_count;
  const uint32_t* cand_rows;
  const float* cand_vals;  // screen values of the candidates (ordered verification), or null
  int64_t cap;
  bool all_rows;
  int64_t n_rows;
  const void* vectors;  // original vectors [*, dim]
  const float* rowc;    // liveness (-inf) for all_rows
  const void* queries;  // original queries: query q of the batch is row query_rows[q] (or q)
  const int32_t* query_rows = nullptr;
  elem t;
  int64_t dim;
  metric_kind metric;
  filter_args filter;
  int64_t nq;
  int k;
  // the certificate of the screen (lower bounds from screen values): as in threshold_f_args
  const double* qscal;
  const double* maxima;
  double alpha2;
  double gamma;
  unsigned long long* scored;  // optional: += the rows scored exactly (the stats' verified count)
  const int32_t* part_ids = nullptr;  // routed: candidate rows below n_part are partition rows
  int64_t n_part          = 0;
  float* distances;    // as in verify_args
  int64_t* neighbors;
  const int32_t* out_rows = nullptr;  // as in verify_args
};
/**
 * fp64 exact scores (the canonical order of the oracle) and top-k by (score, row); with screen
 * values, only the candidates whose certified lower bound can reach the top k are scored.
 */
void verify_topk_f(const verify_f_args& a, hipStream_t stream);

// --- label partition and routing ------------------------------------------------------------

/** Temporary bytes of sort_by_label for n rows. */
size_t sort_by_label_temp_bytes(int64_t n);
/**
 * Stable sort of the ids 0 .. n-1 by label (unlabeled -1 first): keys_out = sorted labels,
 * ids_out = ids in label order (ascending within a label). n < 2^31.
 */
hipError_t sort_by_label(const int32_t* labels, int64_t n, int32_t* ids_scratch, int32_t* keys_out,
                         int32_t* ids_out, void* temp, size_t temp_bytes, hipStream_t stream);
/** offsets[l] = first position of label >= l in keys_sorted, l = 0 .. n_labels. */
void label_offsets(const int32_t* keys_sorted, int64_t n, int64_t n_labels, int64_t* offsets,
                   hipStream_t stream);

/**
 * The routing tables of a label search over the label partition, built on the device from the
 * batch's labels sorted ascending (sorted[B]) and the partition's label offsets (offsets[n_labels
 * + 1]): one group per label l of the partition, in both tables, with the queries [q0, q0 + nq) of
 * label l (none when the label has no rows) and its rows [offsets[l], offsets[l + 1]). Each
 * group's workgroups follow the previous group's, their count rounded up to a multiple of 8 (so a
 * group's first workgroup is a multiple of 8). The anchor table counts the group's anchors (row
 * pairs with anchor_pairs, else one row every anchor_stride), the screen table its rows. The host
 * launches each pass with route_tiles_bound workgroups; those past the last group exit.
 */
struct route_table_args {
  const int32_t* sorted;
  int64_t B;
  const int64_t* offsets;
  int64_t n_labels;
  int anchor_stride;
  bool anchor_pairs;
  int anchor_qb;
  int anchor_chunk;
  int anchor_lead;  // 1: a group whose first query is odd starts one query early (paired queries)
  bool screen_tiled;
  bool rows_paired;
  int screen_qb;
  int screen_chunk;
  screen_group* anchor_groups;
  screen_group* screen_groups;
};
void route_tables(const route_table_args& a, hipStream_t stream);
/** Whether route_small takes a batch of B labels over n_labels partition labels. */
bool route_small_fits(int64_t B, int64_t n_labels);
/** The routing of a batch in one launch for few labels: order / sorted of the batch's labels (a
 *  stable sort by label, as sort_by_label; a.sorted = sorted) and the group tables of
 *  route_tables. */
void route_small(const route_table_args& a, const int32_t* labels, int32_t* order, int32_t* sorted,
                 hipStream_t stream);
/** dst row i = src row ids[i] (rows of row_bytes bytes). */
void gather_rows(const void* src, const int32_t* ids, int64_t n, int64_t row_bytes, void* dst,
                 hipStream_t stream);
/** The same into the paired layout of dst (row_bytes a multiple of 128, paired_bytes(n) bytes). */
void gather_rows_paired(const void* src, const int32_t* ids, int64_t n, int64_t row_bytes,
                        void* dst, hipStream_t stream);
/** pos[ids[i]] = i. */
void invert_ids(const int32_t* ids, int64_t n, int32_t* pos, hipStream_t stream);

/** out[i] = i * step for i < n. */
void strided_ids(int32_t* out, int64_t n, int64_t step, hipStream_t stream);
/**
 * The anchor copy: anchors j0 .. j1 - 1 (the ids j * stride) get the codes and row term of their
 * stored rows (id_rows[id] below n_listed, else the id itself).
 */
void gather_anchors(const void* codes, const void* rowc, int row_bytes, int64_t stride, int64_t j0,
                    int64_t j1, const int32_t* id_rows, int64_t n_listed, void* anchor_codes,
                    void* anchor_rowc, hipStream_t stream);
/** out[i] = the stored row of id ids[i] (id_rows[id] for id < n_listed, else id). */
void stored_rows(const int32_t* ids, int64_t n, const int32_t* id_rows, int64_t n_listed,
                 int32_t* out, hipStream_t stream);

// --- k-means lists (screening coordinates, squared L2) --------------------------------------

/** Most lists an index may have, and most lists a query probes. */
constexpr int kMaxLists = 16384;
constexpr int kMaxProbe = 8;
/** Centers are stored padded to a multiple of 64 (padding: zero rows, cterm = +inf). */
__host__ __device__ inline int pad_centers(int n) { return (n + 63) / 64 * 64; }
/**
 * out[i] = the center nearest to screening row i (int8 codes or fp16 rows of row_bytes bytes);
 * centers_q = the centers in the rows' type [n_centers_pad, row_bytes], cterm = |center|^2 / 2.
 */
void nearest_centers(const void* rows, bool f16, int64_t n, int row_bytes, const void* centers_q,
                     const float* cterm, int n_centers_pad, int32_t* out, hipStream_t stream);
/** dist[i, c] = cterm[c] - <row i, center c> for all padded centers (row stride n_centers_pad). */
void center_distances(const void* rows, bool f16, int64_t n, int row_bytes,
                      const void* centers_q, const float* cterm, int n_centers_pad, float* dist,
                      hipStream_t stream);
/** lists[q, 0 .. p) = the p nearest of the n_lists centers of dist row q (ld floats), p <= 8. */
void nearest_lists(const float* dist, int64_t nq, int n_lists, int ld, int p, int32_t* lists,
                   hipStream_t stream);
/**
 * lists[q, 0 .. 8) = 8 nearest lists of int8 query q (codes of 128 or 256 bytes) by
 * cterm[c] - <q', center c>, ascending, ties to the lower list: the best two lists of each of 32
 * fixed parts of the centers, then the 8 best of those (a list may stand in for a nearer one of
 * the same part as two nearer still); centers
 * of cterm +inf are never taken (-1 where fewer than 8 are finite). No distance matrix. Also
 * counts the queries of every list into temp (list_anchor_temp_bytes), for list_anchor_groups.
 */
void nearest_lists_i8(const int8_t* qcodes, int row_bytes, int64_t nq, const void* centers_q,
                      const float* cterm, int n_centers_pad, int n_lists, int32_t* lists,
                      void* temp, hipStream_t stream);
/** Bytes of the temporary memory of nearest_lists_i8 and list_anchor_groups. */
size_t list_anchor_temp_bytes(int64_t nq, int n_lists);
/**
 * The group table of the list anchors, a threshold source of integer rows of 128 or 256 bytes:
 * for query q < nq and its t-th nearest list j = lists[q 8 + t] (t < 8; -1: none), anchor i of
 * j is the stored row offsets[j] + i stride (i < ceil(rows of j / stride)), and column
 * t 64 + i % 64 of the query's row of gmax (512 columns) gets the largest screen value
 * <q', x'> + rowc[x] of its anchors (INT32_MIN for a column without one). Every column holds
 * distinct rows, so the k-th largest column bounds the k-th best screen value from below. The
 * pairs (q, t) are grouped by list in temp (counted there by nearest_lists_i8 on the same lists),
 * so that one workgroup copies the anchors of a list into LDS once for up to 32 of its queries.
 */
void list_anchor_groups(const int8_t* codes, const int32_t* rowc, int row_bytes,
                        const int8_t* qcodes, int64_t nq, const int32_t* lists,
                        const int64_t* offsets, int n_lists, int64_t stride, void* temp,
                        int32_t* gmax, hipStream_t stream);
/** sums[assign[i]] += row i; counts[assign[i]] += 1 (float atomics; width elements per row). */
void center_sums(const void* rows, bool f16, int64_t n, int width, const int32_t* assign,
                 int n_centers, float* sums, unsigned int* counts, hipStream_t stream);
/**
 * centers = sums / counts where counts > 0 (counts may be null: keep the centers); then their copy
 * in the rows' type (centers_q) and cterm, for the n_centers_pad padded centers.
 */
void finish_centers(const float* sums, const unsigned int* counts, int n_centers,
                    int n_centers_pad, int width, bool f16, float* centers, void* centers_q,
                    float* cterm, hipStream_t stream);
/** centers[c] = rows[ids[c]] as floats. */
void rows_to_centers(const void* rows, bool f16, const int32_t* ids, int n_centers, int width,
                     float* centers, hipStream_t stream);

}  // namespace certex_amd
