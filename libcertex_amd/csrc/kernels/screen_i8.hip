// Int8 MFMA screen of the exact k-NN path for integer vectors (gfx950).
//
// Reference contract: detail/screen_int8.cu:99-292 (int8 codes, int32 accumulation, fp32
// Cauchy-Schwarz epilogue) and the anchor-group pass of detail/kernels.hpp:125-135. This kernel
// is built differently: the stored int8 code of a uint8 coordinate is x - 128 (x ^ 0x80), so the
// int32 MFMA accumulator holds the exact value
//     acc(q, x) = <q', x'> + rowc(x),   rowc = -floor(|x'|^2 / 2)   (l2)
//                                      rowc = 128 sum(x')          (inner product of uint8)
// and the squared distance is |q'|^2 - 2 acc + (|x'|^2 mod 2). A larger acc is a closer row, no
// rounding-error term exists, and the certified test of the reference degenerates to the exact
// integer comparison acc >= theta(q).
//
// Layout of one MFMA tile (v_mfma_i32_16x16x64_i8): operand A holds 16 stored rows, operand B
// holds 16 queries, so lane l owns query (l % 16) and rows 4 (l / 16) + r, r = 0..3, of the tile.
// The row term enters as the C operand (four consecutive rows = one 16-byte LDS read), and the
// per-query test is a max over the lane's 16 accumulators of a step and one compare.
//
// Work decomposition: a workgroup (4 waves) keeps 256 queries resident in registers (64 per
// wave) and streams a chunk of stored rows through double-buffered LDS, 64 rows per step. Block
// b runs on XCD b % 8; the chunk index is derived so that all query blocks of one chunk run on one
// XCD at about the same time, and the chunk is read from HBM once per pass into that XCD's L2.

#include "../kernels.hpp"

#include <climits>

namespace certex_amd {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kWaves  = 4;
constexpr int kQT     = 4;  // 16-query tiles per wave
constexpr int kBT     = 4;  // 16-row tiles per step
constexpr int kHitCap = 1024;

template <int KS>
struct lds_layout {
  static constexpr int kRowBytes  = 64 * KS;
  // 16 bytes of padding per row: the 16 lanes of a ds_read_b128 quarter-wave that read rows
  // 0..15 at one column start in 16 distinct 4-bank groups.
  static constexpr int kPitch     = kRowBytes + 16;
  static constexpr int kRowsBytes = kStepRows * kPitch;
  static constexpr int kBufBytes  = kRowsBytes + kStepRows * 4;
};

__device__ inline bool keeps(const filter_args& f, int64_t q, uint32_t row)
{
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

template <int KS, bool ANCHORS, bool FILT>
__global__ __launch_bounds__(256, 2) void screen_kernel(screen_args a)
{
  using L = lds_layout<KS>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * L::kBufBytes];
  __shared__ uint32_t hit_q[ANCHORS ? 1 : kHitCap];
  __shared__ uint32_t hit_row[ANCHORS ? 1 : kHitCap];
  __shared__ uint32_t n_hits;

  const int tid  = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  const int64_t n_steps  = screen_steps(a.n_scan);
  const int64_t n_chunks = (n_steps + a.chunk_steps - 1) / a.chunk_steps;
  const int n_qb         = int(a.nq_pad / kBlockQ);
  const uint32_t b       = blockIdx.x;
  const uint32_t i       = b >> 3;
  const int qb           = int(i % uint32_t(n_qb));
  const int64_t chunk    = int64_t(i / uint32_t(n_qb)) * 8 + (b & 7);
  if (chunk >= n_chunks) { return; }
  const int64_t s0 = chunk * a.chunk_steps;
  const int64_t s1 = s0 + a.chunk_steps < n_steps ? s0 + a.chunk_steps : n_steps;

  if (tid == 0) { n_hits = 0; }

  // resident queries (B operands) and their thresholds
  const int64_t qw = int64_t(qb) * kBlockQ + wave * 64;
  v4i qf[kQT][KS];
  int th[kQT];
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt) {
    const int64_t q   = qw + qt * 16 + (lane & 15);
    const int8_t* src = a.qcodes + q * L::kRowBytes + (lane >> 4) * 16;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) { qf[qt][ks] = *reinterpret_cast<const v4i*>(src + ks * 64); }
    th[qt] = ANCHORS ? 0 : a.theta[q];
  }

  // global -> LDS staging: thread t moves 16 KS bytes of row t / 4 and, for t % 4 == 0, its term
  v4i pre[KS];
  int prc = 0;
  auto load_step = [&](int64_t s) {
    const int64_t r = s * kStepRows + (tid >> 2);
    if (r < a.n_scan) {
      const int64_t row = r * a.row_stride;
      const int8_t* src = a.codes + row * L::kRowBytes + (tid & 3) * 16 * KS;
#pragma unroll
      for (int c = 0; c < KS; ++c) { pre[c] = *reinterpret_cast<const v4i*>(src + 16 * c); }
      prc = (tid & 3) == 0 ? a.rowc[row] : 0;
    } else {
#pragma unroll
      for (int c = 0; c < KS; ++c) { pre[c] = v4i{0, 0, 0, 0}; }
      prc = kDeadRow;
    }
  };
  auto store_step = [&](int buf) {
    uint8_t* base = smem + buf * L::kBufBytes;
    uint8_t* dst  = base + (tid >> 2) * L::kPitch + (tid & 3) * 16 * KS;
#pragma unroll
    for (int c = 0; c < KS; ++c) { *reinterpret_cast<v4i*>(dst + 16 * c) = pre[c]; }
    if ((tid & 3) == 0) { reinterpret_cast<int32_t*>(base + L::kRowsBytes)[tid >> 2] = prc; }
  };

  load_step(s0);
  store_step(0);
  __syncthreads();

  int gm[kQT];
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt) { gm[qt] = INT_MIN; }

  for (int64_t s = s0; s < s1; ++s) {
    const int buf   = int(s - s0) & 1;
    const bool more = s + 1 < s1;
    if (more) { load_step(s + 1); }

    const uint8_t* base = smem + buf * L::kBufBytes;
    v4i acc[kBT][kQT];
#pragma unroll
    for (int bt = 0; bt < kBT; ++bt) {
      const uint8_t* rp = base + (bt * 16 + (lane & 15)) * L::kPitch + (lane >> 4) * 16;
      v4i av[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) { av[ks] = *reinterpret_cast<const v4i*>(rp + ks * 64); }
      const v4i c = *reinterpret_cast<const v4i*>(base + L::kRowsBytes +
                                                   (bt * 16 + (lane >> 4) * 4) * 4);
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt) {
        v4i t = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[0], qf[qt][0], c, 0, 0, 0);
#pragma unroll
        for (int ks = 1; ks < KS; ++ks) {
          t = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[ks], qf[qt][ks], t, 0, 0, 0);
        }
        acc[bt][qt] = t;
      }
    }

    const int64_t row0 = s * kStepRows + (lane >> 4) * 4;  // scan index of (bt = 0, r = 0)
    if constexpr (!ANCHORS) {
      bool hit = false;
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt) {
        int m = acc[0][qt][0];
#pragma unroll
        for (int bt = 0; bt < kBT; ++bt) {
#pragma unroll
          for (int r = 0; r < 4; ++r) { m = max(m, acc[bt][qt][r]); }
        }
        hit |= m >= th[qt];
      }
      if (__any(hit)) {
        // compaction: per-lane hit masks, a wave prefix sum of their popcounts, one LDS
        // reservation per wave and query tile
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
          const int qloc = wave * 64 + qt * 16 + (lane & 15);
          uint32_t bits  = 0;
#pragma unroll
          for (int bt = 0; bt < kBT; ++bt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              bits |= uint32_t(acc[bt][qt][r] >= th[qt]) << (bt * 4 + r);
            }
          }
          if constexpr (FILT) {
            uint32_t scan = bits;
            while (scan) {
              const int j = __builtin_ctz(scan);
              scan &= scan - 1;
              const uint32_t row = uint32_t(row0 + (j >> 2) * 16 + (j & 3));
              if (!keeps(a.filter, int64_t(qb) * kBlockQ + qloc, row)) { bits &= ~(1u << j); }
            }
          }
          const int cnt = __builtin_popcount(bits);
          int incl      = cnt;
#pragma unroll
          for (int off = 1; off < 64; off <<= 1) {
            const int t = __shfl_up(incl, off);
            if (lane >= off) { incl += t; }
          }
          const int total = __shfl(incl, 63);
          if (total == 0) { continue; }
          uint32_t pos = 0;
          if (lane == 0) { pos = atomicAdd(&n_hits, uint32_t(total)); }
          pos = uint32_t(__shfl(int(pos), 0)) + uint32_t(incl - cnt);
          while (bits) {
            const int j = __builtin_ctz(bits);
            bits &= bits - 1;
            const uint32_t row = uint32_t(row0 + (j >> 2) * 16 + (j & 3));
            if (pos < kHitCap) {
              hit_q[pos]   = uint32_t(qloc);
              hit_row[pos] = row;
            } else {  // LDS list full: straight to the global bucket
              const int64_t q     = int64_t(qb) * kBlockQ + qloc;
              const uint32_t slot = atomicAdd(a.cand_count + q, 1u);
              if (slot < a.cap) { a.cand_rows[q * a.cap + slot] = row; }
            }
            ++pos;
          }
        }
      }
    } else {
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt) {
        int m = INT_MIN;
#pragma unroll
        for (int bt = 0; bt < kBT; ++bt) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            int v = acc[bt][qt][r];
            if constexpr (FILT) {
              const int64_t idx = row0 + bt * 16 + r;
              if (idx < a.n_scan &&
                  !keeps(a.filter, qw + qt * 16 + (lane & 15), uint32_t(idx * a.row_stride))) {
                v = INT_MIN;
              }
            }
            m = max(m, v);
          }
        }
        m      = max(m, __shfl_xor(m, 16));
        m      = max(m, __shfl_xor(m, 32));
        gm[qt] = max(gm[qt], m);
      }
      if ((s + 1) % a.group_steps == 0 || s + 1 == n_steps) {
        const int64_t g = s / a.group_steps;
        if (lane < 16) {
#pragma unroll
          for (int qt = 0; qt < kQT; ++qt) {
            a.gmax[(qw + qt * 16 + lane) * a.n_groups + g] = gm[qt];
          }
        }
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) { gm[qt] = INT_MIN; }
      }
    }

    if (more) { store_step(buf ^ 1); }
    __syncthreads();
  }

  if constexpr (!ANCHORS) {
    const uint32_t nh = n_hits < uint32_t(kHitCap) ? n_hits : uint32_t(kHitCap);
    for (uint32_t e = tid; e < nh; e += 256) {
      const int64_t q     = int64_t(qb) * kBlockQ + hit_q[e];
      const uint32_t slot = atomicAdd(a.cand_count + q, 1u);
      if (slot < a.cap) { a.cand_rows[q * a.cap + slot] = hit_row[e]; }
    }
  }
}

template <bool ANCHORS, bool FILT>
void launch(const screen_args& a, hipStream_t stream)
{
  const int64_t n_steps  = screen_steps(a.n_scan);
  const int64_t n_chunks = (n_steps + a.chunk_steps - 1) / a.chunk_steps;
  const int64_t n_qb     = a.nq_pad / kBlockQ;
  const int64_t blocks   = 8 * n_qb * ((n_chunks + 7) / 8);
  if (n_steps == 0 || n_qb == 0) { return; }
  const dim3 grid{unsigned(blocks)};
  switch (a.row_bytes / 64) {
    case 1: screen_kernel<1, ANCHORS, FILT><<<grid, 256, 0, stream>>>(a); break;
    case 2: screen_kernel<2, ANCHORS, FILT><<<grid, 256, 0, stream>>>(a); break;
    case 3: screen_kernel<3, ANCHORS, FILT><<<grid, 256, 0, stream>>>(a); break;
    case 4: screen_kernel<4, ANCHORS, FILT><<<grid, 256, 0, stream>>>(a); break;
    default: break;  // the host rejects wider rows before any launch
  }
}

}  // namespace

void screen_i8(const screen_args& a, hipStream_t stream)
{
  if (a.filter.kind != 0) {
    launch<false, true>(a, stream);
  } else {
    launch<false, false>(a, stream);
  }
}

void anchors_i8(const screen_args& a, hipStream_t stream)
{
  if (a.filter.kind != 0) {
    launch<true, true>(a, stream);
  } else {
    launch<true, false>(a, stream);
  }
}

}  // namespace certex_amd
