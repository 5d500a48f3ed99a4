// Anchor pass for rows of more than 256 bytes (gfx950): fp16 rows of more than 128 halves and
// int8 rows of more than 256 coordinates, a K loop over the row's bytes.
//
// Reference contract: the anchor groups of detail/kernels.hpp:125-135 and detail/screen_sm80.cu:
// 304-372 (fp16 MMA, fp32 accumulation, the best screen value of every group of anchors for every
// query) and, for int8 rows, the exact int32 screen values of screen.hip. The screen pass of such
// rows is screen_tile.hip. The row term enters as the accumulator's initial value.
//
// Work decomposition:
// - a workgroup of 8 waves holds QB = 16 QT queries (all their bytes) in LDS for its whole life,
//   16-byte chunks XOR-swizzled by the query (chunk c of query r sits in slot c ^ (r & 15)), so
//   the ds_read_b128 of a 16-query fragment is free of bank conflicts;
// - each wave streams its own contiguous eighth of a chunk of stored rows, 64 rows per step, and
//   runs the K loop in chunks of 128 bytes; the next chunk's row fragments are loaded into a
//   second register set while the MFMAs of the current chunk run. No barrier in the main loop.
// - within a 128-byte chunk, lane group g = lane / 16 supplies bytes 32 g .. 32 g + 15 to the
//   first MFMA (v_mfma_f32_16x16x32_f16: 8 halves; v_mfma_i32_16x16x64_i8: 16 int8) and 32 g + 16
//   .. 32 g + 31 to the second, in both operands (a permutation of the summation order), so a
//   row's fragments are 32 contiguous bytes per lane group. The rows are loaded with the 4 lanes of a quad on one row's 128-byte line (the memory
//   pipeline serves a quad that shares a line at once, and 16 lanes on 16 rows one line at a
//   time), and 4 ds_bpermute per 16 bytes move them to the MFMA's lanes;
// - block b runs on XCD b % 8; the query blocks of one row chunk run on one XCD together.
// Group maxima go to the group table, per coarse group of anchor steps or per fine group of 4
// anchors.

#include "screen_common.hpp"

#include <algorithm>
#include <stdexcept>

namespace certex_amd {
namespace {

using namespace screen_detail;

constexpr int kWideWaves = 8;

/** Pointers into global memory, so that loads through them stay global (never flat) loads. */
typedef const __attribute__((address_space(1))) int8_t* gbytes;

template <typename F>
__device__ __forceinline__ F gload(gbytes p)
{
  return *reinterpret_cast<const __attribute__((address_space(1))) F*>(p);
}

template <typename R, int QT, bool FILT>
__global__ __launch_bounds__(64 * kWideWaves, 1) void screen_wide_kernel(screen_args a)
{
  using acc_t  = typename R::acc_t;
  using frag_t = typename R::frag_t;
  using val_t  = typename R::val_t;
  static_assert(sizeof(frag_t) == 16, "a lane's MFMA operand is 16 bytes");
  constexpr int QB = 16 * QT;
  // dynamic LDS: the queries [QB][row_bytes] (swizzled)
  extern __shared__ __attribute__((aligned(16))) uint8_t qlds[];
  __shared__ val_t gml[kWideWaves * QB];

  const val_t* rowc = static_cast<const val_t*>(a.rowc);
  val_t* gmax       = static_cast<val_t*>(a.gmax);

  const int tid   = threadIdx.x;
  const int lane  = tid & 63;
  const int wave  = tid >> 6;
  const int RB    = a.row_bytes;      // bytes per row (stored rows and LDS query rows), a multiple of 256
  const int NC    = RB / 128;         // K chunks of 128 bytes, even

  const screen_work w = work_of<QB>(a, blockIdx.x);
  if (!w.valid) { return; }
  const int64_t n_steps = screen_steps(w.n_scan);
  const int64_t q0      = w.q0;
  const int64_t eighth  = a.chunk_steps / kWideWaves;  // whole anchor groups
  const int64_t w0      = w.chunk * a.chunk_steps + wave * eighth;
  const int64_t w1      = w0 + eighth < n_steps ? w0 + eighth : n_steps;

  stage_queries<64 * kWideWaves>(a.qcodes, RB, q0, w.q_end, QB, qlds,
                                 [](int r, int c) { return c ^ (r & 15); });
  for (int e = tid; e < kWideWaves * QB; e += 64 * kWideWaves) { gml[e] = R::lowest(); }
  __syncthreads();

  frag_t av[2][4][2];  // [buffer][row tile][first / second MFMA of the chunk]
  acc_t cc[4];
  // Row addresses: the rows of step s start at the uniform address step_base(s); lane l reads
  // row bt * 16 + l / 4 of the step (clamped to the pass's last row, whose term is dead past the
  // end) at a 32-bit offset O[bt]: the 4 lanes of a quad read one row's 128-byte line, which the
  // memory pipeline serves about 3.3 times as fast as 4 lines (measured), and compute() moves the
  // pieces to the MFMA's lanes. The loads then take the scalar-base + vector-offset form
  // and a lane keeps 4 offsets per step instead of 4 pointers (64-bit pointers for this and the
  // next step pushed the kernel past 256 VGPRs). Every load of the main loop is unconditional,
  // so that the compiler's wait counts see one straight path and the prefetches stay in flight.
  // Paired rows (rows_paired): byte b of stored row R at paired_offset(R, b); a 128-byte chunk of a
  // row is then two 64-byte pieces 128 bytes apart, lanes 0-1 of a quad on the first and 2-3 on
  // the second, and chunk c starts 256 c bytes into the pair.
  const gbytes codes     = (gbytes)a.codes;
  const bool rp          = a.rows_paired;
  const int64_t cstep    = rp ? 256 : 128;  // bytes between consecutive 128-byte chunks of a row
  auto row_at = [&](int64_t sr) { return rp ? (sr & ~int64_t(1)) * RB + (sr & 1) * 64 : sr * RB; };
  // stored row of scan index i: one row every row_stride, or with anchor pairs both rows of a
  // pair every 2 row_stride from an even base (the two quads of a pair then read one whole line)
  const bool apairs = a.anchor_pairs;
  auto row_of = [&](int64_t i) {
    return apairs ? w.base + (i >> 1) * (2 * int64_t(a.row_stride)) + (i & 1) : w.base + i * a.row_stride;
  };
  auto step_base = [&](int64_t s) {
    return codes + row_at(row_of(s * kStepRows) & ~int64_t(rp ? 1 : 0));
  };
  auto offsets   = [&](int64_t s, uint32_t (&O)[4]) {
    const int64_t R0 = row_of(s * kStepRows) & ~int64_t(rp ? 1 : 0);
    const int q      = lane & 3;
#pragma unroll
    for (int bt = 0; bt < 4; ++bt) {
      int64_t r = s * kStepRows + bt * 16 + (lane >> 2);
      r         = r < w.n_scan ? r : w.n_scan - 1;
      O[bt]     = uint32_t(row_at(row_of(r)) - row_at(R0) +
                           (rp ? (q >> 1) * 128 + (q & 1) * 32 : q * 32));
    }
  };
  auto load_chunk = [&](gbytes base, const uint32_t (&O)[4], int64_t off,
                        frag_t (&A)[4][2]) {
#pragma unroll
    for (int bt = 0; bt < 4; ++bt) {
      A[bt][0] = gload<frag_t>(base + off + O[bt]);
      A[bt][1] = gload<frag_t>(base + off + 16 + O[bt]);
    }
  };
  auto load_terms = [&](int64_t s) {
#pragma unroll
    for (int bt = 0; bt < 4; ++bt) {
      const int64_t r4 = s * kStepRows + bt * 16 + (lane >> 4) * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool ok  = r4 + j < w.n_scan;
        const val_t v  = rowc[row_of(ok ? r4 + j : 0)];
        cc[bt][j]      = ok ? v : R::dead();
      }
    }
  };

  acc_t acc[4][QT];
  // lane 4 rr + g loaded row rr's pieces for lane group g; the MFMA takes them in lane 16 g + rr
  const int perm_src = 4 * (4 * (lane & 15) + (lane >> 4));
  auto to_mfma_lanes = [&](frag_t& x) {
    v4i v = __builtin_bit_cast(v4i, x);
#pragma unroll
    for (int i = 0; i < 4; ++i) { v[i] = __builtin_amdgcn_ds_bpermute(perm_src, v[i]); }
    x = __builtin_bit_cast(frag_t, v);
  };
  auto compute = [&](int c, frag_t (&A)[4][2]) {
#pragma unroll
    for (int bt = 0; bt < 4; ++bt) {
      to_mfma_lanes(A[bt][0]);
      to_mfma_lanes(A[bt][1]);
    }
    const uint8_t* qbase = qlds + (lane & 15) * RB;
    const int c0         = c * 8 + (lane >> 4) * 2;  // this lane's first 16-byte chunk
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int r         = qt * 16 + (lane & 15);
      const uint8_t* qrow = qbase + qt * 16 * RB;
      const frag_t b0     = *reinterpret_cast<const frag_t*>(qrow + 16 * ((c0) ^ (r & 15)));
      const frag_t b1     = *reinterpret_cast<const frag_t*>(qrow + 16 * ((c0 + 1) ^ (r & 15)));
#pragma unroll
      for (int bt = 0; bt < 4; ++bt) {
        acc[bt][qt] = R::mfma(A[bt][0], b0, acc[bt][qt]);
        acc[bt][qt] = R::mfma(A[bt][1], b1, acc[bt][qt]);
      }
    }
    __builtin_amdgcn_s_setprio(0);
  };

  // offsets(s) needs a step that exists (s * 64 < n_scan): a wave whose share of the last chunk
  // is empty (w0 >= n_steps) loads nothing
  gbytes B = step_base(w0);
  uint32_t O[4] = {0, 0, 0, 0};
  if (w0 < w1) {
    offsets(w0, O);
    load_chunk(B, O, 0, av[0]);
    load_terms(w0);
  }
  for (int64_t s = w0; s < w1; ++s) {
#pragma unroll
    for (int bt = 0; bt < 4; ++bt) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) { acc[bt][qt] = cc[bt]; }
    }
#pragma unroll 1
    for (int c = 0; c < NC - 2; c += 2) {
      load_chunk(B, O, int64_t(c + 1) * cstep, av[1]);
      compute(c, av[0]);
      load_chunk(B, O, int64_t(c + 2) * cstep, av[0]);
      compute(c + 1, av[1]);
    }
    // the last two chunks; the next step's terms and first chunk are loaded meanwhile (the last
    // step reloads its own); loaded this late, they hold no registers during the K loop
    const int64_t sn = s + 1 < w1 ? s + 1 : s;
    const gbytes BN  = step_base(sn);
    uint32_t ON[4];
    offsets(sn, ON);
    load_terms(sn);
    load_chunk(B, O, int64_t(NC - 1) * cstep, av[1]);
    compute(NC - 2, av[0]);
    load_chunk(BN, ON, 0, av[0]);
    compute(NC - 1, av[1]);
    B = BN;
#pragma unroll
    for (int bt = 0; bt < 4; ++bt) { O[bt] = ON[bt]; }

    const int64_t row0 = s * kStepRows + (lane >> 4) * 4;
    step_labels SL;  // the label filter's row labels of the step
    if constexpr (FILT) { load_step_labels(a, w, row0, SL); }
    if (a.fine) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        const acc_t col[4] = {acc[0][qt], acc[1][qt], acc[2][qt], acc[3][qt]};
        const int64_t q    = q0 + qt * 16 + (lane & 15);
        const int64_t qc   = q < w.q_end ? q : w.q_end - 1;  // padding: any live query's
        const uint32_t kp  = FILT ? filter_mask(a, w, SL, qc, row0) : 0u;
        anchor_tile_fine<R, FILT>(col, row0, q, q < w.q_end, a, w, gmax, kp);
      }
    } else {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        const acc_t col[4] = {acc[0][qt], acc[1][qt], acc[2][qt], acc[3][qt]};
        const int64_t q    = q0 + qt * 16 + (lane & 15);
        const int64_t qc   = q < w.q_end ? q : w.q_end - 1;  // padding: any live query's
        const uint32_t kp  = FILT ? filter_mask(a, w, SL, qc, row0) : 0u;
        anchor_tile<R, FILT>(col, wave * QB + qt * 16 + lane, gml, kp);
      }
    }
    // end of an anchor group (group_steps steps, aligned to the wave's range)
    if (!a.fine && ((s + 1) % a.group_steps == 0 || s + 1 == n_steps)) {
      for (int e = lane; e < QB; e += 64) {
        if (q0 + e < w.q_end) { gmax[table_entry(a, q0 + e, s / a.group_steps)] = gml[wave * QB + e]; }
        gml[wave * QB + e] = R::lowest();
      }
    }
  }
}

template <typename R, int QT, bool FILT>
void launch_qt(const screen_args& a, dim3 grid, size_t lds, hipStream_t stream)
{
  auto* k = &screen_wide_kernel<R, QT, FILT>;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                          hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)) != hipSuccess) {
    (void)hipGetLastError();
    throw std::runtime_error("certex: the wide anchor pass cannot reserve its LDS");
  }
  k<<<grid, 64 * kWideWaves, lds, stream>>>(a);
}

/** LDS bytes a workgroup may use. */
int max_lds()
{
  static const int v = [] {
    int dev = 0, r = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&r, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess) {
      (void)hipGetLastError();
      return 65536;
    }
    return r;
  }();
  return v;
}

/**
 * Query tiles of a workgroup for rows of `row_bytes`: the largest of 6, 4, 2, 1 whose queries and
 * the group table (gml: 4 bytes per query per wave, counted as 8) fit the LDS (0: none fits). More queries
 * per workgroup means more work per row fetched.
 */
int wide_query_tiles(int row_bytes)
{
  for (int qt : {6, 4, 2, 1}) {
    if (16 * qt * (row_bytes + 8 * kWideWaves) <= max_lds()) { return qt; }
  }
  return 0;
}

template <typename R, bool FILT>
void launch(const screen_args& a, hipStream_t stream)
{
  const int qt = wide_query_tiles(a.row_bytes);
  const int qb = 16 * qt;
  if (qt == 0) { throw std::invalid_argument("certex: the rows are too wide for the LDS"); }
  if (a.row_bytes % 256 != 0) {
    throw std::logic_error("certex: the K-loop anchor pass takes rows of whole 256-byte pairs of chunks");
  }
  int64_t blocks = 0;
  if (a.groups != nullptr) {
    blocks = a.n_tiles;
  } else {
    const int64_t n_steps  = screen_steps(a.n_scan);
    const int64_t n_chunks = (n_steps + a.chunk_steps - 1) / a.chunk_steps;
    const int64_t n_qb     = (a.nq + qb - 1) / qb;
    blocks                 = n_steps == 0 ? 0 : 8 * n_qb * ((n_chunks + 7) / 8);
  }
  if (blocks == 0) { return; }
  if (a.anchor_pairs && (a.groups == nullptr || !a.rows_paired || a.filter.kind != 0)) {
    throw std::logic_error("certex: anchor pairs need a routed pass over paired rows without a filter");
  }
  const dim3 grid{unsigned(blocks)};
  const size_t lds = size_t(qb) * size_t(a.row_bytes);
  switch (qt) {
    case 6: launch_qt<R, 6, FILT>(a, grid, lds, stream); break;
    case 4: launch_qt<R, 4, FILT>(a, grid, lds, stream); break;
    case 2: launch_qt<R, 2, FILT>(a, grid, lds, stream); break;
    default: launch_qt<R, 1, FILT>(a, grid, lds, stream); break;
  }
}

}  // namespace

int wide_block_queries(int row_bytes) { return 16 * wide_query_tiles(row_bytes); }

void anchors_f16_wide(const screen_args& a, hipStream_t stream)
{
  if (a.tiled) {
    anchors_f16_tile(a, stream);
  } else if (a.filter.kind != 0) {
    launch<f16_rows, true>(a, stream);
  } else {
    launch<f16_rows, false>(a, stream);
  }
}

void anchors_i8_wide(const screen_args& a, hipStream_t stream)
{
  if (a.tiled) {
    anchors_i8_tile(a, stream);
  } else if (a.filter.kind != 0) {
    launch<int8_rows, true>(a, stream);
  } else {
    launch<int8_rows, false>(a, stream);
  }
}

}  // namespace certex_amd
