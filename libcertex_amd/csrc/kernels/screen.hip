// MFMA screens of the exact k-NN path (gfx950): int8 rows (exact) and fp16 rows (certified).
//
// Reference contract: detail/screen_int8.cu:99-292 and detail/screen_sm80.cu:117-379 (screen a
// batch of queries against every stored row, keep the pairs that pass the query's threshold) and
// the anchor-group pass of detail/kernels.hpp:125-135.
//
// int8 rows. The stored int8 code of a uint8 coordinate is x - 128 (x ^ 0x80), so the int32
// accumulator holds the exact value
//     acc(q, x) = <q', x'> + rowc(x),   rowc = -floor(|x'|^2 / 2)   (l2)
//                                      rowc = 128 sum(x')          (inner product of uint8)
// and the squared distance is |q'|^2 - 2 acc + (|x'|^2 mod 2): a larger acc is a closer row and
// the test acc >= theta(q) is exact.
// fp16 rows. Rows hold fp16(Z) for Z = (x - c) / alpha; the fp32 accumulator holds
// <fp16(W), fp16(Z)> + rowc(x) with rowc ~ -|Z|^2 / 2 (l2, cosine) or 0 (inner product). The host
// folds the rounding error of both operands and of the fp32 accumulation into theta(q) and rowc,
// so that acc >= theta(q) holds for every pair whose exact score passes the threshold.
//
// MFMA tile: operand A holds 16 stored rows, operand B holds 16 queries (one 16-byte fragment per
// lane per 64-byte K step: v_mfma_i32_16x16x64_i8 or v_mfma_f32_16x16x32_f16), so lane l owns
// query (l % 16) and rows 4 (l / 16) + r, r = 0..3. The row term enters as the C operand (four
// consecutive rows = one 16-byte load); the per-query test is a max over the lane's 16
// accumulators of a 64-row step and one compare per query tile.
//
// Work decomposition:
// - a step is BT row tiles (16 BT rows) and a query group QT query tiles (16 QT queries): the
//   int8 screen runs BT = 8 against QT = 2, so that each query fragment read from LDS feeds 8 row
//   tiles (4 in the other passes, BT = QT = 4), which halves the LDS reads per MFMA;
// - a workgroup holds QB queries (512, or 128 for small batches) in LDS for its whole life, rows
//   stored with their 16-byte chunks XOR-swizzled by the row so that the ds_read_b128 of a query
//   tile is free of bank conflicts;
// - each of its 4 waves streams its own contiguous quarter of a chunk of stored rows straight
//   from HBM/L2 into registers, 64 rows (one step) at a time, and runs the step against all QB
//   queries in groups of 64, reading the next group's query fragments from LDS while the current
//   group's MFMAs run; no barrier in the main loop;
// - block b runs on XCD b % 8 and the chunk index is derived so that the query blocks of one chunk
//   run on one XCD together: a chunk is read from HBM about once per pass into that XCD's L2.
// Survivors are compacted with a ballot + mbcnt rank and one LDS reservation per round into a
// per-workgroup list, flushed to the per-query buckets at the end.

#include "screen_common.hpp"

#include <stdexcept>
#include <type_traits>

namespace certex_amd {
namespace {

using namespace screen_detail;

/** 16-byte chunk slot of chunk c of row r (conflict-free ds_read_b128 of 16 rows x 1 chunk). */
template <int KS>
__device__ __forceinline__ int slot(int r, int c)
{
  return KS == 2 ? (c ^ (r & 7)) : (c ^ (r & 15));
}

/** f(integral_constant<int, I>) for I = B .. E - 1, unrolled at compile time. */
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f)
{
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

template <typename R, int KS, int QB, bool ANCHORS, bool FILT, int BT, int QT, bool FINE = false>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(QT == 1 && QB == 128 && (!ANCHORS || (FINE && !FILT)) ? 3 : 2)))
void screen_kernel(screen_args a)
{
  using acc_t  = typename R::acc_t;
  using frag_t = typename R::frag_t;
  using val_t  = typename R::val_t;
  constexpr int ROWB   = 64 * KS;
  constexpr int GQ     = 16 * QT;        // queries of a group
  constexpr int NG     = QB / GQ;        // groups of the workgroup
  constexpr int TR     = 16 * BT;        // rows of a step
  constexpr int SPT    = TR / kStepRows; // chunk steps (kStepRows rows) per step
  // coarse anchor groups without argmax or filter: each lane folds its values into a register per
  // (query group, query tile) every step; the lanes of a query reduce and write once per group
  constexpr bool RUNREG = ANCHORS && !FILT && !FINE;
  // FINE (anchor passes with fine groups of 4 anchors, a.fine) and coarse anchor passes are
  // separate kernels: each carries only its own group code, and its registers
  static_assert(ANCHORS || !FINE, "fine groups are an anchor pass's");
  static_assert(NG % 2 == 0, "query groups are processed in pairs");
  static_assert(BT * 4 <= 32, "a lane's survivor mask of one query tile is 32 bits");
  static_assert(!ANCHORS || BT == 4, "the anchor pass runs 64-row steps");
  static_assert(!R::kValues || BT == 4, "screen values travel for 16 rows per query tile");
  static_assert(QB <= (1 << (32 - kSpillRowBits)), "a spill entry holds the query within the block");
  __shared__ __attribute__((aligned(16))) uint8_t qlds[QB * ROWB];
  __shared__ val_t thl[ANCHORS ? 1 : QB];
  __shared__ val_t gml[ANCHORS ? 4 * QB : 1];
  __shared__ val_t ftr[ANCHORS ? 4 * 256 : 1];  // fine groups: each wave's 16 x 16 transpose
  __shared__ uint32_t hit_q[ANCHORS ? 1 : kHitCap];
  __shared__ uint32_t hit_row[ANCHORS ? 1 : kHitCap];
  __shared__ float hit_val[ANCHORS || !R::kValues ? 1 : kHitCap];
  __shared__ uint32_t n_hits;
  __shared__ uint32_t spill_n[ANCHORS ? 1 : QB];  // entries of each query in the spill region

  const val_t* rowc  = static_cast<const val_t*>(a.rowc);
  const val_t* theta = static_cast<const val_t*>(a.theta);
  val_t* gmax        = static_cast<val_t*>(a.gmax);

  const int tid  = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  const screen_work w = work_of<QB>(a, blockIdx.x);
  if (!w.valid) { return; }
  wg_clock clk;
  if constexpr (!ANCHORS) { clk.start(a); }
  const int64_t n_steps = screen_steps(w.n_scan);  // chunk steps
  const int64_t q0      = w.q0;
  // groups holding a live query, rounded up to a pair (the last query block of a batch or of a
  // routed group is partly padding)
  const int64_t live = w.q_end - q0;
  const int ng       = live >= QB ? NG : int(((live + GQ - 1) / GQ + 1) & ~int64_t(1));
  // this wave's chunk steps: a contiguous quarter of the chunk (a whole number of anchor groups,
  // and of steps: the launcher picks BT > 4 only for chunks of whole steps per wave)
  const int64_t quarter = a.chunk_steps / 4;
  const int64_t w0      = w.chunk * a.chunk_steps + wave * quarter;
  const int64_t w1      = w0 + quarter < n_steps ? w0 + quarter : n_steps;
  // the workgroup's first row: its spill entries hold rows as offsets from it
  const int64_t rbase   = w.base + w.chunk * a.chunk_steps * kStepRows;
  // coarse anchor groups of one group per wave: each wave's group maxima wait in LDS, and the
  // workgroup writes each query's 4 consecutive columns together at its end (one 16-byte run per
  // query instead of four 4-byte stores to four lines of the table)
  const bool staged = RUNREG && quarter == a.group_steps;

  if (tid == 0) { n_hits = 0; }
  // only the groups that run are staged (a routed group's block is often mostly padding)
  const int qlive = ng * GQ;
  stage_queries<256>(a.qcodes, ROWB, q0, w.q_end, qlive, qlds,
                     [](int r, int c) { return slot<KS>(r, c); });
  if constexpr (ANCHORS) {
    for (int e = tid; e < 4 * QB; e += 256) {
      if (e % QB >= qlive) { continue; }
      gml[e] = R::lowest();
    }
  } else {
    for (int e = tid; e < qlive; e += 256) {
      thl[e] = q0 + e < w.q_end ? theta[q0 + e] : R::keep_none();
    }
    for (int e = tid; e < QB; e += 256) { spill_n[e] = 0; }
  }
  __syncthreads();

  frag_t av[BT][KS];
  acc_t cc[BT];
  // the screen reads consecutive rows (stride 1), the anchor pass every row_stride-th
  const int64_t stride = ANCHORS ? a.row_stride : 1;
  // a step whose rows all exist: straight-line loads, so that the steady-state loop has one
  // path for the compiler's wait counts
  auto load_rows = [&](int64_t s) {
#pragma unroll
    for (int bt = 0; bt < BT; ++bt) {
      const int64_t r   = s * TR + bt * 16 + (lane & 15);
      const int8_t* src = a.codes + (w.base + r * stride) * ROWB + (lane >> 4) * 16;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        av[bt][ks] = *reinterpret_cast<const frag_t*>(src + 64 * ks);
      }
      const int64_t r4 = s * TR + bt * 16 + (lane >> 4) * 4;
      if constexpr (ANCHORS) {
#pragma unroll
        for (int j = 0; j < 4; ++j) { cc[bt][j] = rowc[w.base + (r4 + j) * stride]; }
      } else {
        cc[bt] = *reinterpret_cast<const acc_t*>(rowc + w.base + r4);
      }
    }
  };
  // the last step of a scan whose length is not a multiple of TR
  auto load_rows_tail = [&](int64_t s) {
#pragma unroll
    for (int bt = 0; bt < BT; ++bt) {
      int64_t r = s * TR + bt * 16 + (lane & 15);
      r         = r < w.n_scan ? r : 0;  // rows past the end read row 0; their term kills them
      const int8_t* src = a.codes + (w.base + r * stride) * ROWB + (lane >> 4) * 16;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        av[bt][ks] = *reinterpret_cast<const frag_t*>(src + 64 * ks);
      }
      const int64_t r4 = s * TR + bt * 16 + (lane >> 4) * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        cc[bt][j] = r4 + j < w.n_scan ? rowc[w.base + (r4 + j) * stride] : R::dead();
      }
    }
  };
  auto read_queries = [&](int g, frag_t (&bf)[QT][KS], val_t (&th)[QT]) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int r = g * GQ + qt * 16 + (lane & 15);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        bf[qt][ks] = *reinterpret_cast<const frag_t*>(qlds + r * ROWB +
                                                      16 * slot<KS>(r, (lane >> 4) + 4 * ks));
      }
      th[qt] = ANCHORS ? val_t(0) : thl[r];
    }
  };

  int64_t row0 = 0;  // scan index of (bt = 0, r = 0) of this lane in the current step
  step_labels SL;    // the label filter's row labels of the step (anchor pass with a filter)
  auto mfmas = [&](const frag_t (&bf)[QT][KS], acc_t (&acc)[BT][QT]) {
    __builtin_amdgcn_s_setprio(1);
    // K-slice outermost: consecutive MFMAs share their row fragment (operand A) across the query
    // tiles, so fewer operand bits switch from one MFMA to the next on this power-limited part
    // (measured against the slices of one tile back to back: 0.8% faster, and 2% faster than
    // holding the query fragment across the row tiles)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int bt = 0; bt < BT; ++bt) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          acc[bt][qt] = R::mfma(av[bt][ks], bf[qt][ks], ks == 0 ? cc[bt] : acc[bt][qt]);
        }
      }
    }
    __builtin_amdgcn_s_setprio(0);
  };
  auto group = [&](int g, const frag_t (&bf)[QT][KS], const val_t (&th)[QT])
                   __attribute__((always_inline)) {
    acc_t acc[BT][QT];
    mfmas(bf, acc);

    if constexpr (ANCHORS) {
      if constexpr (FINE) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const acc_t col[4] = {acc[0][qt], acc[1][qt], acc[2][qt], acc[3][qt]};
          const int64_t q    = q0 + g * GQ + qt * 16 + (lane & 15);
          const int64_t qc   = q < w.q_end ? q : w.q_end - 1;  // padding: any live query's
          const uint32_t kp  = FILT ? filter_mask(a, w, SL, qc, row0) : 0u;
          anchor_tile_fine<R, FILT>(col, row0, q, q < w.q_end, a, w, gmax, kp, ftr + wave * 256);
        }
      } else {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const acc_t col[4] = {acc[0][qt], acc[1][qt], acc[2][qt], acc[3][qt]};
          const int64_t q    = q0 + g * GQ + qt * 16 + (lane & 15);
          const int64_t qc   = q < w.q_end ? q : w.q_end - 1;  // padding: any live query's
          const uint32_t kp  = FILT ? filter_mask(a, w, SL, qc, row0) : 0u;
          anchor_tile<R, FILT>(col, wave * QB + g * GQ + qt * 16 + lane, gml, kp);
        }
      }
    } else {
      val_t mq[QT];
      bool hit = false;
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        val_t m = acc[0][qt][0];
#pragma unroll
        for (int bt = 0; bt < BT; ++bt) {
#pragma unroll
          for (int r = 0; r < 4; ++r) { m = R::vmax(m, acc[bt][qt][r]); }
        }
        mq[qt] = m;
        hit |= m >= th[qt];
      }
      if (__builtin_expect(__any(hit), 0)) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          if (!__any(mq[qt] >= th[qt])) { continue; }
          uint32_t bits = 0;
#pragma unroll
          for (int bt = 0; bt < BT; ++bt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              bits |= uint32_t(acc[bt][qt][r] >= th[qt]) << (bt * 4 + r);
            }
          }
          const uint32_t qloc = uint32_t(g * GQ + qt * 16 + (lane & 15));
          val_t v16[16]       = {};
          if constexpr (R::kValues) {
#pragma unroll
            for (int bt = 0; bt < 4; ++bt) {
#pragma unroll
              for (int r = 0; r < 4; ++r) { v16[bt * 4 + r] = acc[bt][qt][r]; }
            }
          }
          push_hits<BT * 4, FILT, R::kValues>(bits, qloc, w.base + row0, rbase, q0, a, hit_q, hit_row,
                                              hit_val, &n_hits, spill_n, uint32_t(kHitCap), v16);
        }
      }
    }
  };

  frag_t b0[QT][KS], b1[QT][KS];
  val_t t0[QT], t1[QT];
  read_queries(0, b0, t0);
  val_t run[RUNREG ? NG : 1][QT];
#pragma unroll
  for (int g = 0; g < (RUNREG ? NG : 1); ++g) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) { run[g][qt] = R::lowest(); }
  }
  auto step = [&](int64_t s) {
    row0 = s * TR + (lane >> 4) * 4;
    if constexpr (ANCHORS && FILT) { load_step_labels(a, w, row0, SL); }
    if constexpr (RUNREG) {
      {
        // the groups at compile time, so that run[][] stays in registers
        auto group_run = [&](auto gc, const frag_t (&bf)[QT][KS]) {
          constexpr int g = decltype(gc)::value;
          acc_t acc[BT][QT];
          mfmas(bf, acc);
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) {
            val_t m = run[g][qt];
#pragma unroll
            for (int bt = 0; bt < BT; ++bt) {
#pragma unroll
              for (int r = 0; r < 4; ++r) { m = R::vmax(m, acc[bt][qt][r]); }
            }
            run[g][qt] = m;
          }
        };
        static_for<0, NG / 2>([&](auto pc) {
          constexpr int g = 2 * decltype(pc)::value;
          // keep each pair of groups in place: hoisting every group's query reads to the top of
          // the unrolled loop would exceed the registers
          __builtin_amdgcn_sched_barrier(0);
          if (g < ng) {
            read_queries(g + 1, b1, t1);
            group_run(std::integral_constant<int, g>{}, b0);
            read_queries(g + 2 < ng ? g + 2 : 0, b0, t0);
            group_run(std::integral_constant<int, g + 1>{}, b1);
          }
        });
        // end of an anchor group (group_steps steps, aligned to the wave's range): the maxima of
        // the 4 lanes of each query (l, l ^ 16, l ^ 32, l ^ 48) go to the table
        if ((s + 1) % a.group_steps == 0 || s + 1 == n_steps) {
          static_for<0, NG>([&](auto gc) {
            constexpr int g = decltype(gc)::value;
            if (g < ng) {
#pragma unroll
              for (int qt = 0; qt < QT; ++qt) {
                val_t m         = run[g][qt];
                m               = R::vmax(m, __shfl_xor(m, 16));
                m               = R::vmax(m, __shfl_xor(m, 32));
                const int64_t q = q0 + g * GQ + qt * 16 + (lane & 15);
                if (staged) {
                  if (lane < 16) { gml[wave * QB + g * GQ + qt * 16 + lane] = m; }
                } else if (lane < 16 && q < w.q_end) {
                  gmax[table_entry(a, q, s / a.group_steps)] = m;
                }
                run[g][qt] = R::lowest();
              }
            }
          });
        }
        return;
      }
    }
#pragma unroll 1
    for (int g = 0; g < ng; g += 2) {
      read_queries(g + 1, b1, t1);
      group(g, b0, t0);
      read_queries(g + 2 < ng ? g + 2 : 0, b0, t0);
      group(g + 1, b1, t1);
    }
    if constexpr (ANCHORS) {
      // end of an anchor group (group_steps steps, aligned to the wave's range)
      if (!FINE && ((s + 1) % a.group_steps == 0 || s + 1 == n_steps)) {
        for (int e = lane; e < QB; e += 64) {
          if (q0 + e < w.q_end) { gmax[table_entry(a, q0 + e, s / a.group_steps)] = gml[wave * QB + e]; }
          gml[wave * QB + e] = R::lowest();
        }
      }
    }
  };
  // this wave's steps [s0, s1): its chunk steps hold whole steps
  const int64_t s0   = w0 / SPT;
  const int64_t s1   = (w1 + SPT - 1) / SPT;
  const int64_t full = w.n_scan / TR;  // steps whose rows all exist
  const int64_t s1f  = s1 < full ? s1 : full;
  for (int64_t s = s0; s < s1f; ++s) {
    load_rows(s);
    step(s);
  }
  if (s0 <= full && full < s1) {  // the scan's last, partial step, when it is this wave's
    load_rows_tail(full);
    step(full);
  }

  if constexpr (RUNREG) {
    if (staged) {
      // wave v's group is column 4 chunk + v (its quarter is that one group); a wave of the last
      // chunk past the scan has no group
      __syncthreads();
      const int64_t col0 = w.chunk * 4;
      for (int i = tid; i < 4 * qlive; i += 256) {
        const int e = i >> 2, v = i & 3;
        const bool has = w.chunk * a.chunk_steps + v * quarter < n_steps;
        if (has && q0 + e < w.q_end) { gmax[table_entry(a, q0 + e, col0 + v)] = gml[v * QB + e]; }
      }
    }
  }
  if constexpr (!ANCHORS) {
    __syncthreads();
    flush_hits<R::kValues>(q0, rbase, QB, a, hit_q, hit_row, hit_val, &n_hits, uint32_t(kHitCap),
                           reinterpret_cast<uint32_t*>(qlds), spill_n);
    clk.stop(a);
  }
}

template <typename R, bool ANCHORS, bool FILT, bool FINE>
void launch_other(const screen_args& b, dim3 grid, int ks, int qb_size, hipStream_t stream);

template <typename R, bool ANCHORS, bool FILT>
void launch(const screen_args& a, hipStream_t stream)
{
  const int qb_size = narrow_block_queries(R::kValues, a.row_bytes, a.nq_pad);
  int64_t blocks    = 0;
  if (a.groups != nullptr) {
    blocks = a.n_tiles;
  } else {
    const int64_t n_steps  = screen_steps(a.n_scan);
    const int64_t n_chunks = (n_steps + a.chunk_steps - 1) / a.chunk_steps;
    const int64_t n_qb     = (a.nq + qb_size - 1) / qb_size;
    blocks                 = n_steps == 0 ? 0 : 8 * n_qb * ((n_chunks + 7) / 8);
  }
  if (blocks == 0) { return; }
  const dim3 grid{unsigned(blocks)};
  const int ks  = a.row_bytes / 64;
  screen_args b = a;
  b.spill_cap   = !ANCHORS && a.spill != nullptr ? a.spill_pool / blocks : 0;
  if (b.spill_cap > 0 && b.chunk_steps * kStepRows > (int64_t(1) << kSpillRowBits)) {
    throw std::logic_error("certex: a screen chunk has more rows than a spill entry can address");
  }
  if constexpr (ANCHORS) {
    if (a.fine) {
      launch_other<R, ANCHORS, FILT, true>(b, grid, ks, qb_size, stream);
      return;
    }
  }
  if constexpr (ANCHORS && !FILT) {
    // coarse groups keep their running maxima in registers: groups of 32 queries (2 tiles)
    // leave room for them; 16 (one tile) for 256-byte rows in 128-query blocks, as below
    if (ks == 2 && qb_size == 512) {
      screen_kernel<R, 2, 512, ANCHORS, FILT, 4, 2><<<grid, 256, 0, stream>>>(b);
    } else if (ks == 2) {
      screen_kernel<R, 2, 128, ANCHORS, FILT, 4, 2><<<grid, 256, 0, stream>>>(b);
    } else if (ks == 4 && qb_size == 512) {
      screen_kernel<R, 4, 512, ANCHORS, FILT, 4, 2><<<grid, 256, 0, stream>>>(b);
    } else if (ks == 4) {
      screen_kernel<R, 4, 128, ANCHORS, FILT, 4, 1><<<grid, 256, 0, stream>>>(b);
    }
  } else {
    launch_other<R, ANCHORS, FILT, false>(b, grid, ks, qb_size, stream);
  }
}

/** The launches other than the register-maxima anchor pass (FINE: anchor passes with fine
 *  groups). */
template <typename R, bool ANCHORS, bool FILT, bool FINE>
void launch_other(const screen_args& b, dim3 grid, int ks, int qb_size, hipStream_t stream)
{
  if constexpr (!ANCHORS && !R::kValues) {
    // steps of 128 rows when every wave's share of a chunk is whole steps
    if (ks == 2 && qb_size == 512 && (b.chunk_steps / 4) % 2 == 0) {
      screen_kernel<R, 2, 512, ANCHORS, FILT, 8, 2><<<grid, 256, 0, stream>>>(b);
      return;
    }
  }
  // groups of 32 queries: with 64, the fragments of 256-byte rows took more than the registers of
  // two waves per SIMD, and the compiler made the group's code a function call. 256-byte rows in
  // 128-query blocks take groups of 16 (one query tile): 166 VGPRs, three waves per SIMD, whose
  // row loads (each feeding a quarter of the MFMAs of a 512-query block) then overlap more
  if (ks == 2 && qb_size == 512) {
    screen_kernel<R, 2, 512, ANCHORS, FILT, 4, 2, FINE><<<grid, 256, 0, stream>>>(b);
  } else if (ks == 2) {
    screen_kernel<R, 2, 128, ANCHORS, FILT, 4, 2, FINE><<<grid, 256, 0, stream>>>(b);
  } else if (ks == 4 && qb_size == 512) {
    screen_kernel<R, 4, 512, ANCHORS, FILT, 4, 2, FINE><<<grid, 256, 0, stream>>>(b);
  } else if (ks == 4) {
    screen_kernel<R, 4, 128, ANCHORS, FILT, 4, 1, FINE><<<grid, 256, 0, stream>>>(b);
  }
  // other row widths are rejected by the host before any launch
}

}  // namespace

int wide_block_queries(int row_bytes);  // screen_wide.hip

int screen_query_block(bool f16, int row_bytes, int64_t nq_pad)
{
  // rows of more than 256 bytes (fp16 or int8) take the K-loop anchor pass's blocks
  return row_bytes > 256 ? wide_block_queries(row_bytes) : narrow_block_queries(f16, row_bytes, nq_pad);
}

void screen_i8(const screen_args& a, hipStream_t stream)
{
  if (a.row_bytes > 256) {  // int8 rows of more than 256 coordinates: the tiled screen
    screen_i8_tile(a, stream);
  } else if (a.filter.kind != 0) {
    launch<int8_rows, false, true>(a, stream);
  } else {
    launch<int8_rows, false, false>(a, stream);
  }
}

void anchors_i8(const screen_args& a, hipStream_t stream)
{
  if (a.row_bytes > 256) {  // the K-loop anchor pass (or its tiled form over anchor pairs)
    anchors_i8_wide(a, stream);
  } else if (a.filter.kind != 0) {
    launch<int8_rows, true, true>(a, stream);
  } else {
    launch<int8_rows, true, false>(a, stream);
  }
}

void screen_f16(const screen_args& a, hipStream_t stream)
{
  if (a.filter.kind != 0) {
    launch<f16_rows, false, true>(a, stream);
  } else {
    launch<f16_rows, false, false>(a, stream);
  }
}

void anchors_f16(const screen_args& a, hipStream_t stream)
{
  if (a.filter.kind != 0) {
    launch<f16_rows, true, true>(a, stream);
  } else {
    launch<f16_rows, true, false>(a, stream);
  }
}

}  // namespace certex_amd
