// Screen for rows of more than 256 bytes (gfx950): fp16 rows of more than 128 halves (certified)
// and int8 rows of more than 256 coordinates (exact); LDS-staged tiles of rows and queries, both
// fed to the MFMA from LDS, two workgroups resident per CU.
//
// Reference contract: detail/screen_sm80.cu:117-379 and detail/screen_sm90.cu:594-785 (fp16 MMA,
// fp32 accumulation, keep a pair iff its screen value reaches the query threshold; the reference
// stages 128 x 128 x 64 tiles). The certificate is the one of screen.hip: the row term enters as
// the accumulator's initial value and the host folds every rounding error into the row term and
// the threshold, so the test needs no per-pair arithmetic.
//
// Work decomposition:
// - a workgroup of 4 waves computes one tile of 256 stored rows x 128 queries, all of the row's
//   bytes, in stages of 64 bytes of every row and query (one MFMA k-step: 32 halves or 64 int8);
// - two workgroups share a CU (73.5 KB of LDS and 4 waves each, 2 waves per SIMD), so that one
//   workgroup's barriers, copies' latency, survivor epilogue and flush overlap the other's MFMAs;
// - a stage of both operands is copied into LDS by global_load_lds_dwordx4 (no VGPRs): a copy
//   moves 16 rows x 64 bytes, lane i on row i / 4. Row r's 64 bytes are half of a 128-byte LDS
//   line (the line of rows r & ~1), and its 16-byte chunk c lands in slot c ^ ((r >> 1) & 3) of
//   that half, so lane i reads chunk (i & 3) ^ ((i >> 3) & 3) of its row. The ds_read_b128 of a
//   16-row MFMA fragment (lanes on 16 rows, one chunk) then serves 8 lanes per pass from 8
//   distinct 16-byte slots of a 128-byte line: no bank conflicts;
// - the queries, and the rows of a routed pass (the label partition), are stored in the paired
//   layout (paired_offset): piece s of rows 2p and 2p + 1 share one 128-byte line, so a copy asks
//   for 8 whole lines. The memory pipeline serves whole lines about twice as fast as half lines
//   (measured: 33 against 15 TB/s of LDS-DMA from L2). A tile starts at an even row and query;
//   a group whose first row (query) is odd starts one slot early, and that slot is not live;
// - three stage buffers: the copies of stage s + 2 fly while the MFMAs run on stage s; at the top
//   of stage s a wave waits for its own copies of stage s only (those of s + 1 stay in flight),
//   then one barrier publishes stage s and frees the buffer of stage s - 1;
// - the waves form a 2 x 2 grid: wave (wr, wq) multiplies tile rows 128 wr .. 128 wr + 127 (8 row
//   tiles) with tile queries 64 wq .. 64 wq + 63 (4 query tiles), v_mfma_f32_16x16x32_f16 (fp16)
//   or v_mfma_i32_16x16x64_i8 (int8), the row tiles as operand A: 128 accumulator registers per
//   lane. Chunk lane / 16 of a stage's 64 bytes is the k-slice of a lane in both operands;
// - the row terms and the query thresholds are copied into LDS with the first stages;
// - after the last stage the staging LDS holds the survivor list. Per query tile a lane has 32
//   rows; the wave reserves its survivors with one LDS atomic (exclusive prefix of the lanes'
//   counts from one ballot + mbcnt per bit of the count), the lanes park their 32 screen values in
//   LDS and write each survivor with its value read back by bit index (a per-survivor select over
//   registers cost twice as much; int8 rows carry no value), then one flush per workgroup moves the
//   list into the per-query buckets (flush_hits of screen_common.hpp).
// Workgroup b runs on XCD b % 8; the query blocks of one row tile run on one XCD (work_of), so a
// row tile is fetched from HBM about once.
//
// The same kernel (ANCH) runs the routed anchor pass over a paired partition with fine groups: a
// tile's 256 rows are anchors taken in row pairs (scan index i is stored row base + (i / 2) 2 s +
// i % 2), and instead of survivors each lane writes the maximum of its 4 accumulators of every row
// tile and query tile, the screen value of one fine group of 4 anchors, to the group table.

#include "screen_common.hpp"

#include <algorithm>
#include <stdexcept>
#include <type_traits>
#include <utility>

namespace certex_amd {
namespace {

using namespace screen_detail;

constexpr int kTileWaves = 4;
constexpr int kTileRows  = 256;              // stored rows of a tile (4 steps of 64)
constexpr int kStageB    = 64;               // bytes of a row per stage (32 halves)
constexpr int kBufs      = 3;                // stage buffers
constexpr int kTileSteps = kTileRows / kStepRows;
static_assert(kTileRows <= (1 << kSpillRowBits), "spill entries address a tile's rows");

typedef const __attribute__((address_space(1))) void* gptr;
typedef __attribute__((address_space(3))) void* lptr;

/** s_waitcnt vmcnt(N) (expcnt and lgkmcnt left at their maxima): at most N of this wave's global
 *  loads, LDS-DMA copies included, are still in flight (they complete in issue order). */
template <int N>
__device__ __forceinline__ void wait_copies()
{
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0f70);
}

/** LDS-DMA copy of 16 (B = 16) or 4 (B = 4) bytes per lane from g to LDS byte m0 + B * lane, issued
 *  as inline assembly: the compiler then neither counts it among the loads it waits for nor orders
 *  LDS reads against it (it models such copies as LDS stores of unknown address and would wait for
 *  every LDS read before each copy). The kernel orders the copies itself: a stage's copies target
 *  a buffer that no wave reads, and s_waitcnt vmcnt plus a barrier publish them. An LDS-DMA
 *  instruction needs one wait state after the write of M0. */
template <int B>
__device__ __forceinline__ void lds_copy(const void* g, uint32_t m0)
{
  if constexpr (B == 16) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(m0) : "m0");
  } else {
    static_assert(B == 4, "4 or 16 bytes per lane");
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(m0) : "m0");
  }
}

/** The LDS byte address of p (a pointer into the workgroup's LDS). */
__device__ __forceinline__ uint32_t lds_addr(const void* p)
{
  return uint32_t(reinterpret_cast<uintptr_t>((lptr)(const_cast<void*>(p))));
}

/** Staging LDS of a workgroup of TQ queries: three stage buffers of (256 + TQ) rows x 64 bytes. */
constexpr int tile_lds(int tq) { return kBufs * (kTileRows + tq) * kStageB; }

/** All LDS of a workgroup: the staging, then the TQ query thresholds and the 256 row terms. */
constexpr int tile_lds_total(int tq) { return tile_lds(tq) + 4 * tq + 4 * kTileRows; }

/** Survivor list entries that fit the staging LDS: 12 bytes each plus the flush's rank word,
 *  after the flush's 2 TQ counters and the waves' 8 KB of parked screen values. */
constexpr int tile_hit_cap(int tq) { return (tile_lds(tq) - kTileWaves * 8192 - 8 * tq) / 16 / 64 * 64; }

/** f(std::integral_constant<int, i>{}) for i = 0 .. N - 1, unrolled at compile time. */
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>)
{
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f)
{
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

/**
 * The tile of a workgroup: RT row tiles (16 rows each) and QT query tiles per wave; 256 / (16 RT)
 * waves along the rows and the rest of the 4 along the queries, TQ = 16 QT x that many queries.
 */
template <int RT, int QT>
struct tile_shape {
  static constexpr int WR = kTileRows / (16 * RT);
  static constexpr int WQ = kTileWaves / WR;
  static constexpr int TQ = 16 * QT * WQ;
  static_assert(WR * WQ == kTileWaves && WR * 16 * RT == kTileRows, "4 waves cover the tile");
};

template <typename R, int RT, int QT, bool FILT, bool ANCH>
__global__ __launch_bounds__(64 * kTileWaves, 2) void screen_tile_kernel(screen_args a)
{
  using acc_t       = typename R::acc_t;
  using frag_t      = typename R::frag_t;
  using val_t       = typename R::val_t;
  using S           = tile_shape<RT, QT>;
  static_assert(sizeof(frag_t) == 16 && sizeof(val_t) == 4, "16-byte operands, 4-byte values");
  constexpr int TQ  = S::TQ;
  static_assert(TQ <= (1 << (32 - kSpillRowBits)), "a spill entry holds the query within the tile");
  constexpr int CA  = kTileRows / 16 / kTileWaves;  // row copies per wave and stage
  constexpr int CB  = TQ / 16 / kTileWaves;         // query copies per wave and stage
  constexpr int NC  = CA + CB;                      // copies per wave and stage
  static_assert(CA * 16 * kTileWaves == kTileRows && CB * 16 * kTileWaves == TQ,
                "every wave issues the same copies (the stage waits count them)");
  constexpr int CPT = (NC + RT - 1) / RT;           // copies per row tile
  constexpr int BUF = (kTileRows + TQ) * kStageB;   // one stage buffer: rows, then queries
  constexpr int CAP = tile_hit_cap(TQ);
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  __shared__ uint32_t n_hits;

  const int tid  = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wr   = wave / S::WQ;  // row part of the tile
  const int wq   = wave % S::WQ;  // query part of the tile

  const screen_work w = work_of<TQ, true>(a, blockIdx.x);
  if (!w.valid) { return; }
  wg_clock clk;
  if constexpr (!ANCH) { clk.start(a); }
  const int RB          = a.row_bytes;  // bytes per row: a multiple of 128
  const int n_stages    = RB / kStageB;
  const int64_t scan0   = w.chunk * kTileRows;  // scan index of tile row 0 (an even stored row
                                                // with paired rows, as the first query is even)
  // live tile rows [r_lo, n_rows) and tile queries [q_lo, n_q): a group whose first row (query)
  // is odd starts its tiles one paired row (query) early
  const int64_t n_rows  = w.n_scan - scan0 < kTileRows ? w.n_scan - scan0 : kTileRows;
  const int r_lo        = scan0 == 0 ? w.rlead : 0;
  const int64_t n_q     = w.q_end - w.q0 < TQ ? w.q_end - w.q0 : TQ;
  const int q_lo        = w.q_first > w.q0 ? int(w.q_first - w.q0) : 0;
  // stored row of tile row r: consecutive rows, or (ANCH, anchor pairs) both rows of a pair
  // every 2 row_stride rows from the tile's first pair (scan index i = stored row
  // base + (i / 2) 2 row_stride + i % 2; scan0 is even)
  const int64_t s2     = ANCH ? 2 * int64_t(a.row_stride) : 2;
  const int64_t row_t0 = ANCH ? w.base + (scan0 >> 1) * s2 : w.base + scan0;
  auto tile_rel        = [&](int64_t r) { return ANCH ? (r >> 1) * s2 + (r & 1) : r; };

  if (tid == 0) { n_hits = 0; }

  // the query thresholds and the row terms into LDS past the staging (waited for with stage 0);
  // indices past the live queries and rows repeat the last live one (the slot before a group's
  // first live one reads its neighbour, in the same allocation)
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  val_t* th_lds    = reinterpret_cast<val_t*>(lds + tile_lds(TQ));
  val_t* rc_lds    = th_lds + TQ;
  {
    const int64_t r = wave_u * 64 + lane;
    lds_copy<4>(static_cast<const val_t*>(a.rowc) + row_t0 + tile_rel(r < n_rows ? r : n_rows - 1),
                lds_addr(rc_lds + wave_u * 64));
    if (!ANCH && wave_u * 64 < TQ) {
      const int64_t q = wave_u * 64 + lane;
      lds_copy<4>(static_cast<const val_t*>(a.theta) + w.q0 + (q < n_q ? q : n_q - 1),
                  lds_addr(th_lds + wave_u * 64));
    }
  }

  // this lane's copy offsets: rows of copies j < CA (tile rows (CA wave + j) * 16 + lane / 4), and
  // queries of copies j < CB (tile queries (CB wave + j) * 16 + lane / 4); rows and queries past
  // the tile's live ones repeat its last live one (their results are never kept). The queries are
  // paired, and so are the rows with rows_paired: the 8 lanes of a row pair then read one whole
  // 128-byte line per copy, and a stage advances 128 bytes (64 unpaired). A paired tile starts at
  // an even row and query, where the pair starts.
  const bool rp     = a.rows_paired;
  const int rstep   = rp ? 128 : kStageB;
  const int crow    = lane >> 2;
  const int cchunk  = (lane & 3) ^ ((lane >> 3) & 3);
  const char* rbase = reinterpret_cast<const char*>(a.codes) + row_t0 * int64_t(RB) + cchunk * 16;
  const char* qbase = reinterpret_cast<const char*>(a.qpaired) + w.q0 * int64_t(RB) + cchunk * 16;
  uint32_t roff[CA], qoff[CB];
#pragma unroll
  for (int j = 0; j < CA; ++j) {
    int64_t r = (wave * CA + j) * 16 + crow;
    r         = tile_rel(r < n_rows ? r : n_rows - 1);
    roff[j]   = uint32_t(rp ? (r & ~int64_t(1)) * RB + (r & 1) * 64 : r * RB);
  }
#pragma unroll
  for (int j = 0; j < CB; ++j) {
    int64_t q = (wave * CB + j) * 16 + crow;
    q         = q < n_q ? q : n_q - 1;
    qoff[j]   = uint32_t((q & ~int64_t(1)) * RB + (q & 1) * 64);
  }
  // copy j (0 .. NC - 1) of stage s: rows for j < CA, queries after; the LDS destination is
  // wave-uniform (scalar: M0)
  auto copy = [&](int s, int j) {
    uint8_t* buf = lds + (s % kBufs) * BUF;
    if (j < CA) {
      lds_copy<16>(rbase + s * rstep + roff[j], lds_addr(buf + ((wave_u * CA + j) * 16) * kStageB));
    } else {
      lds_copy<16>(qbase + s * 128 + qoff[j - CA],
                   lds_addr(buf + (kTileRows + (wave_u * CB + j - CA) * 16) * kStageB));
    }
  };
  auto issue = [&](int s) {
#pragma unroll
    for (int j = 0; j < NC; ++j) { copy(s, j); }
  };

  // fragment addresses within a stage buffer: row tile bt, query tile qt, chunk lane / 16
  const int frow = lane & 15;
  const int fch  = lane >> 4;
  auto a_frag    = [&](const uint8_t* buf, int bt) {
    const int r = wr * 16 * RT + bt * 16 + frow;
    return *reinterpret_cast<const frag_t*>(buf + r * kStageB + ((fch ^ ((r >> 1) & 3)) << 4));
  };
  auto b_frag = [&](const uint8_t* buf, int qt) {
    const int t = wq * 16 * QT + qt * 16 + frow;
    return *reinterpret_cast<const frag_t*>(buf + (kTileRows + t) * kStageB + ((fch ^ ((t >> 1) & 3)) << 4));
  };

  acc_t acc[RT][QT];

  // one stage: wait for this wave's copies of stage s (with COPY, those of stage s + 1 stay in
  // flight), publish the stage, read its fragments and run its MFMAs; with COPY the copies of stage
  // s + 2 go between the row tiles, pinned with sched_group_barrier (DS read 0x100, VMEM read
  // 0x020, MFMA 0x008), so that their issue hides behind MFMAs
  auto stage = [&](int s, auto more, auto copy_next) {
    constexpr bool MORE = decltype(more)::value;       // stage s + 1 is in flight
    constexpr bool COPY = decltype(copy_next)::value;  // issue stage s + 2
    if constexpr (MORE) {
      wait_copies<NC>();
    } else {
      wait_copies<0>();
    }
    __syncthreads();
    const uint8_t* buf = lds + (s % kBufs) * BUF;
    frag_t ar[RT], bq[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) { bq[qt] = b_frag(buf, qt); }
#pragma unroll
    for (int bt = 0; bt < RT; ++bt) { ar[bt] = a_frag(buf, bt); }
    __builtin_amdgcn_sched_group_barrier(0x100, QT + RT, 0);
    __builtin_amdgcn_s_setprio(1);
    static_for<RT>([&](auto BT) {
      constexpr int bt = decltype(BT)::value;
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) { acc[bt][qt] = R::mfma(ar[bt], bq[qt], acc[bt][qt]); }
      __builtin_amdgcn_sched_group_barrier(0x008, QT, 0);
      if constexpr (COPY) {
        constexpr int c0 = bt * CPT;
        constexpr int c1 = c0 + CPT < NC ? c0 + CPT : NC;
        if constexpr (c1 > c0) {
#pragma unroll
          for (int j = c0; j < c1; ++j) { copy(s + 2, j); }
          __builtin_amdgcn_sched_group_barrier(0x020, c1 - c0, 0);
        }
      }
    });
    __builtin_amdgcn_s_setprio(0);
  };

  issue(0);
  issue(1);
  // stage 0 also publishes the row terms: the accumulators start at them (dead past the live rows)
  wait_copies<NC>();
  __syncthreads();
#pragma unroll
  for (int bt = 0; bt < RT; ++bt) {
    const int r0 = wr * 16 * RT + bt * 16 + (lane >> 4) * 4;
    acc_t c      = *reinterpret_cast<const acc_t*>(rc_lds + r0);
#pragma unroll
    for (int j = 0; j < 4; ++j) { c[j] = r0 + j >= r_lo && r0 + j < n_rows ? c[j] : R::dead(); }
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) { acc[bt][qt] = c; }
  }
  int s = 0;
  for (; s + 2 < n_stages; ++s) { stage(s, std::true_type{}, std::true_type{}); }
  stage(s, std::true_type{}, std::false_type{});
  stage(s + 1, std::false_type{}, std::false_type{});

  if constexpr (ANCH) {
    // fine groups: the 4 consecutive anchors of a lane's row tile are one group of the table.
    // Lane (query frow, fch) holds group 4 bt + fch of the wave's 16 RT / 4 consecutive groups
    // for each row tile bt; the values go through the staging LDS (free after the last stage),
    // transposed to the wave's queries x groups, so that each store instruction writes whole
    // 128-byte runs of 2 table rows instead of 16 bytes of each of 16 rows
    constexpr int NGW = 4 * RT;       // groups of the wave per query tile
    constexpr int TS  = NGW + 1;      // LDS words per query (one more: fewer bank conflicts)
    constexpr int QPS = 64 / NGW;     // queries per store instruction
    static_assert(64 % NGW == 0 && 16 % QPS == 0, "a store instruction covers whole query rows");
    static_assert(kTileWaves * QT * 16 * TS * 4 <= tile_lds(TQ), "the transpose fits the staging");
    __syncthreads();  // every wave is done with the stage buffers
    val_t* gmax       = static_cast<val_t*>(a.gmax);
    val_t* tr         = reinterpret_cast<val_t*>(lds) + (wave * QT) * 16 * TS;
    const int64_t g0  = (scan0 + wr * 16 * RT) / kFineGroup;  // the wave's first group
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
      for (int bt = 0; bt < RT; ++bt) {
        const acc_t v = acc[bt][qt];
        tr[qt * 16 * TS + frow * TS + bt * 4 + fch] = R::vmax(R::vmax(v[0], v[1]), R::vmax(v[2], v[3]));
      }
    }
    // LDS operations of a wave complete in order; the fence keeps the compiler from moving the
    // reads above the other lanes' writes
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    const int j          = lane % NGW;  // the lane's group of the wave
    const bool has_group = (g0 + j) * kFineGroup < w.n_scan;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
      for (int c = 0; c < 16 / QPS; ++c) {
        const int qi    = c * QPS + lane / NGW;  // query of the tile
        const int qloc  = wq * 16 * QT + qt * 16 + qi;
        const val_t m   = tr[qt * 16 * TS + qi * TS + j];
        if (has_group && qloc >= q_lo && qloc < n_q) { gmax[table_entry(a, w.q0 + qloc, g0 + j)] = m; }
      }
    }
    return;
  }
  __syncthreads();  // the staging LDS becomes the survivor list

  uint32_t* hit_q    = reinterpret_cast<uint32_t*>(lds);
  uint32_t* hit_row  = hit_q + CAP;
  float* hit_val     = reinterpret_cast<float*>(hit_row + CAP);  // fp16 rows only
  uint32_t* scratch  = reinterpret_cast<uint32_t*>(hit_val + CAP);  // 2 TQ + CAP words
  // per wave 8 KB: a lane's 4 RT screen values of one query tile, 16-byte slot bt ^ (lane & 7) of
  // its 128 bytes, so that the survivor loop reads a value by its bit index
  uint8_t* vals      = lds + tile_lds(TQ) - kTileWaves * 8192 + wave * 8192 + lane * 128;
  const int64_t row_t = w.base + scan0;  // the tile's first row: spill entries are offsets from it
  const int64_t row0  = row_t + wr * 16 * RT + (lane >> 4) * 4;  // stored row of bit 0
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qloc = wq * 16 * QT + qt * 16 + frow;
    // a padding query keeps nothing (fp16: no value compares >= NaN; int8: none reaches the max)
    const val_t th = qloc >= q_lo && qloc < n_q ? th_lds[qloc] : R::keep_none();
    uint32_t bits  = 0;  // bit bt * 4 + r: row row0 + 16 bt + r
#pragma unroll
    for (int bt = 0; bt < RT; ++bt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) { bits |= uint32_t(acc[bt][qt][r] >= th) << (bt * 4 + r); }
    }
    if (!__any(bits != 0)) { continue; }
    if constexpr (FILT) {
      uint32_t scan = bits;
      while (scan) {
        const int j = __builtin_ctz(scan);
        scan &= scan - 1;
        if (!keeps(a.filter, w.q0 + qloc, uint32_t(row0 + (j >> 2) * 16 + (j & 3)))) {
          bits &= ~(1u << j);
        }
      }
    }
    if constexpr (R::kValues) {
#pragma unroll
      for (int bt = 0; bt < RT; ++bt) {
        *reinterpret_cast<acc_t*>(vals + ((bt ^ (lane & 7)) << 4)) = acc[bt][qt];
      }
    }
    const uint32_t cnt = uint32_t(__builtin_popcount(bits));
    uint32_t excl = 0, total = 0;
#pragma unroll
    for (int b = 0; (1 << b) <= 4 * RT; ++b) {
      const uint64_t m = __ballot((cnt >> b) & 1u);
      excl += __builtin_amdgcn_mbcnt_hi(uint32_t(m >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(m), 0u)) << b;
      total += uint32_t(__builtin_popcountll(m)) << b;
    }
    if (total == 0) { continue; }
    const int leader = __builtin_ctzll(__ballot(1));
    uint32_t base    = 0;
    if (lane == leader) { base = atomicAdd(&n_hits, total); }
    const uint32_t first = uint32_t(__builtin_amdgcn_readlane(int(base), leader));
    uint32_t pos         = first + excl;
    // each survivor with its value (read back from the parked values by bit index); a wave whose
    // survivors all fit the list takes a loop without the choice between list, region and bucket
    const auto each = [&](auto put) {
      while (bits != 0) {
        const int j = __builtin_ctz(bits);
        bits &= bits - 1;
        float val   = 0;
        if constexpr (R::kValues) {
          val = *reinterpret_cast<const float*>(vals + ((((j >> 2) ^ (lane & 7)) << 4) | ((j & 3) << 2)));
        }
        put(uint32_t((j >> 2) * 16 + (j & 3)), val);
        ++pos;
      }
    };
    if (first + total <= uint32_t(CAP)) {
      each([&](uint32_t d, float val) {
        hit_q[pos]   = uint32_t(qloc);
        hit_row[pos] = uint32_t(row0) + d;
        if constexpr (R::kValues) { hit_val[pos] = val; }
      });
      continue;
    }
    each([&](uint32_t d, float val) {
      const uint32_t row = uint32_t(row0) + d;
      if (pos < uint32_t(CAP)) {
        hit_q[pos]   = uint32_t(qloc);
        hit_row[pos] = row;
        if constexpr (R::kValues) { hit_val[pos] = val; }
      } else if (int64_t(pos - CAP) < a.spill_cap) {
        spill_put<R::kValues>(a, int64_t(blockIdx.x) * a.spill_cap + int64_t(pos - CAP), uint32_t(qloc),
                              uint32_t(row0 - row_t) + d, val);
      } else {
        const int64_t q   = w.q0 + qloc;
        const uint32_t at = atomicAdd(a.cand_count + q, 1u);
        if (at < a.cap) {
          a.cand_rows[q * a.cap + at] = row;
          if constexpr (R::kValues) { a.cand_vals[q * a.cap + at] = val; }
        }
      }
    });
  }
  __syncthreads();
  flush_hits<R::kValues>(w.q0, row_t, TQ, a, hit_q, hit_row, hit_val, &n_hits, uint32_t(CAP), scratch);
  clk.stop(a);
}

template <typename R, int RT, int QT, bool FILT, bool ANCH>
void launch_shape(const screen_args& a, hipStream_t stream)
{
  constexpr int TQ = tile_shape<RT, QT>::TQ;
  int64_t blocks   = 0;
  if (a.groups != nullptr) {
    blocks = a.n_tiles;
  } else {
    const int64_t n_steps  = screen_steps(a.n_scan);
    const int64_t n_chunks = (n_steps + kTileSteps - 1) / kTileSteps;
    const int64_t n_qb     = (a.nq + TQ - 1) / TQ;
    blocks                 = n_steps == 0 ? 0 : 8 * n_qb * ((n_chunks + 7) / 8);
  }
  if (blocks == 0) { return; }
  const bool shape = ANCH ? a.groups != nullptr && a.anchor_pairs && a.rows_paired && a.fine &&
                             a.filter.kind == 0 && a.gmax != nullptr
                           : a.row_stride == 1 && !(a.rows_paired && a.groups == nullptr);
  if (!shape || a.chunk_steps != kTileSteps || a.row_bytes % 128 != 0 || a.qpaired == nullptr) {
    throw std::logic_error(
      "certex: the tiled screen needs chunks of 4 steps over rows of 128-byte multiples, paired "
      "queries, and paired rows only in routed passes (anchor passes: routed over anchor pairs, "
      "fine groups, no filter)");
  }
  screen_args b = a;
  b.spill_cap   = !ANCH && a.spill != nullptr ? a.spill_pool / blocks : 0;
  auto* k       = &screen_tile_kernel<R, RT, QT, FILT, ANCH>;
  const int lds = tile_lds_total(TQ);
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                          hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess) {
    (void)hipGetLastError();
    throw std::runtime_error("certex: the tiled screen cannot reserve its LDS");
  }
  k<<<dim3(unsigned(blocks)), 64 * kTileWaves, lds, stream>>>(b);
}

}  // namespace

int tile_chunk_steps() { return kTileSteps; }

int tile_block_queries() { return tile_shape<8, 4>::TQ; }

void screen_f16_tile(const screen_args& a, hipStream_t stream)
{
  if (a.filter.kind != 0) {
    launch_shape<f16_rows, 8, 4, true, false>(a, stream);
  } else {
    launch_shape<f16_rows, 8, 4, false, false>(a, stream);
  }
}

void anchors_f16_tile(const screen_args& a, hipStream_t stream)
{
  launch_shape<f16_rows, 8, 4, false, true>(a, stream);
}

void screen_i8_tile(const screen_args& a, hipStream_t stream)
{
  if (a.filter.kind != 0) {
    launch_shape<int8_rows, 8, 4, true, false>(a, stream);
  } else {
    launch_shape<int8_rows, 8, 4, false, false>(a, stream);
  }
}

void anchors_i8_tile(const screen_args& a, hipStream_t stream)
{
  launch_shape<int8_rows, 8, 4, false, true>(a, stream);
}

}  // namespace certex_amd
